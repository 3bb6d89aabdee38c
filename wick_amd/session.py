"""Session semantics on the device-resident cache (src/engine.rs:101-145).

A DeviceSession owns one KV cache on the GPU and the tokens it holds.  prefill()
keeps the longest common prefix of the cached tokens and the new prompt
(truncating the cache by setting its length, as Session::prefill does at
src/engine.rs:127-132), recomputes at least the prompt's last token so its
logits are available, and runs the rest in chunks of 256 tokens
(src/engine.rs:107, :134).  step() feeds one token (:141-145).  generate() is
Session::generate (:156-213) without the text side: the prompt's uncached part
and the sampling loop run on the device (the tokenizer and stop strings are not
part of this library; stop ids are).
"""
from dataclasses import dataclass, field

import numpy as np

from .device_model import DeviceModel
from .sampler import SamplerConfig

CHUNK = 256  # Session's CHUNK (src/engine.rs:107)


@dataclass
class GenResult:
    """GenResult (src/engine.rs:71-80) without the text."""
    tokens: list = field(default_factory=list)
    prompt_tokens: int = 0
    reused_tokens: int = 0
    finish: str = "length"


class DeviceSession:
    def __init__(self, model: DeviceModel, context):
        self.model = model
        self.cache = model.new_cache(context)
        self.tokens = []

    def close(self):
        self.cache.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def context(self):
        return self.cache.capacity

    def prefill(self, prompt):
        """Make the cache hold exactly `prompt`; returns (logits after its last token,
        number of tokens reused from the cache)."""
        prompt = [int(t) for t in prompt]
        if not prompt:
            raise ValueError("empty prompt")
        if len(prompt) > self.context():
            raise ValueError(f"prompt is {len(prompt)} tokens, context is {self.context()}")
        keep = 0
        for a, b in zip(self.tokens, prompt):
            if a != b:
                break
            keep += 1
        if keep == len(prompt):
            keep -= 1  # the last token's logits are still needed
        self.tokens = self.tokens[:keep]
        self.cache.len = keep
        logits = None
        for off in range(keep, len(prompt), CHUNK):
            chunk = prompt[off:off + CHUNK]
            logits = self.model.forward(self.cache, chunk)
            self.tokens.extend(chunk)
        return logits, keep

    def generate(self, prompt, max_tokens=256, sampler=None, stops=()):
        """Session::generate: a fresh Sampler per call (src/engine.rs:171), max_tokens
        clamped to the room left (:167-169), a stop id ends the reply (:181-184)."""
        prompt = [int(t) for t in prompt]
        if not prompt:
            raise ValueError("empty prompt")
        if len(prompt) > self.context():
            raise ValueError(f"prompt is {len(prompt)} tokens, context is {self.context()}")
        keep = 0
        for a, b in zip(self.tokens, prompt):
            if a != b:
                break
            keep += 1
        keep = min(keep, len(prompt) - 1)
        self.cache.len = keep
        s = self.model.new_sampler(sampler if sampler is not None else SamplerConfig())
        try:
            out = self.model.generate(self.cache, s, prompt, max_tokens, stops)
        finally:
            s.close()
        self.tokens = (prompt + out)[:self.cache.len]
        room = self.context() - len(prompt)
        finish = "stop" if len(out) < min(max_tokens, room) else "length"
        return GenResult(tokens=out, prompt_tokens=len(prompt), reused_tokens=keep, finish=finish)

    def step(self, token):
        """Feed one token, returning the logits for the next."""
        self.tokens.append(int(token))
        return self.model.forward(self.cache, [int(token)])

    def __len__(self):
        return len(self.tokens)


def greedy(session, prompt, n):
    """prefill + n greedy steps with sampler::argmax on the host (src/sampler.rs:129-137)."""
    logits, keep = session.prefill(prompt)
    out = []
    for _ in range(n):
        tok = int(np.argmax(logits[0]))  # first index of the maximum, as wick's argmax
        out.append(tok)
        logits = session.step(tok)
    return out, keep
