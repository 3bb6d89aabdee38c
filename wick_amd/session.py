"""Session semantics on the device-resident cache (src/engine.rs:101-145).

A DeviceSession owns one KV cache on the GPU and the tokens it holds.  prefill()
keeps the longest common prefix of the cached tokens and the new prompt
(truncating the cache by setting its length, as Session::prefill does at
src/engine.rs:127-132), recomputes at least the prompt's last token so its
logits are available, and runs the rest in chunks of 256 tokens
(src/engine.rs:107, :134).  step() feeds one token (:141-145).
"""
import numpy as np

from .device_model import DeviceModel

CHUNK = 256  # Session's CHUNK (src/engine.rs:107)


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
