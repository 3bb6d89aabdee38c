"""Model configuration and weight loading for the host side.

Config mirrors /root/reference/src/config.rs (Config::from_json :55-133,
q_dim/kv_dim :153-159, rope_inv_freq :162-185); load_safetensors mirrors the
header checks of /root/reference/src/safetensors.rs:81-118 and the bf16/f16
widening of /root/reference/src/quant.rs.  Only f32 compute is supported, as
in the configs this path is measured on.
"""
import json
import math
import os
import struct
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np


@dataclass
class RopeScaling:
    factor: float
    low_freq_factor: float
    high_freq_factor: float
    original_max_position: int


@dataclass
class Config:
    arch: str
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    max_position: int = 4096
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_scaling: Optional[RopeScaling] = None
    tie_embeddings: bool = False
    attn_bias: bool = False
    qk_norm: bool = False
    eos_tokens: List[int] = field(default_factory=list)

    @staticmethod
    def from_json(j):
        name = (j.get("architectures") or [None])[0] or j.get("model_type")
        arch = {"LlamaForCausalLM": "llama", "MistralForCausalLM": "llama", "llama": "llama", "mistral": "llama",
                "Qwen2ForCausalLM": "qwen2", "qwen2": "qwen2", "Qwen3ForCausalLM": "qwen3", "qwen3": "qwen3"}.get(name)
        if arch is None:
            raise ValueError(f"unsupported architecture {name}")
        def need(k):
            v = j.get(k)
            if not isinstance(v, int) or isinstance(v, bool) or v < 0:
                raise ValueError(f"config.json: missing {k}")
            return v
        hidden = need("hidden_size")
        heads = need("num_attention_heads")
        kv_heads = j.get("num_key_value_heads") or heads
        head_dim = j.get("head_dim") or hidden // heads
        act = j.get("hidden_act")
        if isinstance(act, str) and act != "silu":
            # src/config.rs:74-78: only SwiGLU (silu) FFNs are implemented
            raise ValueError(f"unsupported activation {act}")
        # transformers 5 writes rope_parameters (rope_theta inside); older configs
        # have top-level rope_theta and rope_scaling.  Only a missing or null
        # rope_scaling falls back to rope_parameters (src/config.rs:81-89).
        rp = j.get("rope_parameters")
        theta = j.get("rope_theta")
        if not isinstance(theta, (int, float)) or isinstance(theta, bool):
            theta = rp.get("rope_theta") if isinstance(rp, dict) else None
            if not isinstance(theta, (int, float)) or isinstance(theta, bool):
                theta = None
        rs = j.get("rope_scaling")
        if rs is None:
            rs = rp
        scaling = None
        if rs is not None:
            kind = None
            if isinstance(rs, dict):
                kind = rs["rope_type"] if "rope_type" in rs else rs.get("type")
            if not isinstance(kind, str):
                kind = "default"
            if kind == "llama3":
                def f(k):
                    v = rs.get(k)
                    if not isinstance(v, (int, float)) or isinstance(v, bool):
                        raise ValueError(f"rope_scaling: missing {k}")
                    return v
                scaling = RopeScaling(float(np.float32(f("factor"))), float(np.float32(f("low_freq_factor"))),
                                      float(np.float32(f("high_freq_factor"))),
                                      int(f("original_max_position_embeddings")))
            elif kind != "default":
                raise ValueError(f"unsupported rope_scaling type {kind!r}")
        eos = j.get("eos_token_id")
        eps = j.get("rms_norm_eps")
        cfg = Config(arch=arch, hidden=hidden, intermediate=need("intermediate_size"), layers=need("num_hidden_layers"),
                     heads=heads, kv_heads=kv_heads, head_dim=head_dim, vocab=need("vocab_size"),
                     max_position=j.get("max_position_embeddings") or 4096,
                     rms_eps=float(np.float32(eps if isinstance(eps, (int, float)) and not isinstance(eps, bool)
                                              else 1e-6)),
                     rope_theta=float(np.float32(theta if theta is not None else 10000.0)),
                     rope_scaling=scaling, tie_embeddings=bool(j.get("tie_word_embeddings", False)),
                     attn_bias=arch == "qwen2" or bool(j.get("attention_bias", False)), qk_norm=arch == "qwen3",
                     eos_tokens=list(eos) if isinstance(eos, list) else ([eos] if eos is not None else []))
        if cfg.heads % cfg.kv_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        if cfg.head_dim % 2:
            raise ValueError("head_dim must be even for rotary embeddings")
        return cfg

    @staticmethod
    def load(d):
        with open(os.path.join(d, "config.json")) as f:
            return Config.from_json(json.load(f))

    @property
    def q_dim(self):
        return self.heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim

    def rope_inv_freq(self):
        """f64 arithmetic rounded to f32, as src/config.rs:162-185."""
        d = self.head_dim
        theta = float(np.float32(self.rope_theta))
        out = np.empty(d // 2, np.float32)
        for i in range(d // 2):
            inv = 1.0 / math.pow(theta, 2.0 * i / d)
            rs = self.rope_scaling
            if rs is not None:
                omp = float(rs.original_max_position)
                low_w = omp / rs.low_freq_factor
                high_w = omp / rs.high_freq_factor
                wavelen = 2.0 * math.pi / inv
                if wavelen < high_w:
                    pass
                elif wavelen > low_w:
                    inv = inv / rs.factor
                else:
                    smooth = (omp / wavelen - rs.low_freq_factor) / (rs.high_freq_factor - rs.low_freq_factor)
                    inv = (1.0 - smooth) * inv / rs.factor + smooth * inv
            out[i] = np.float32(inv)
        return out


def load_safetensors(path):
    """name -> float32 ndarray, read through a memory map (src/safetensors.rs:56-118 maps
    the file too).  F32 tensors are views of the mapped pages, so handing them to
    wick_hip_model_create copies them from the page cache straight into HBM without
    a host copy; bf16 and f16 are widened exactly into new arrays."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    if mm.size < 8:
        raise ValueError("file too short")
    hlen = int(np.frombuffer(mm[:8].tobytes(), "<u8")[0])
    if hlen > mm.size - 8:
        raise ValueError("bad header length")
    header = json.loads(mm[8:8 + hlen].tobytes().decode("utf-8"))
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        b, e = info["data_offsets"]
        shape = tuple(info["shape"])
        n = int(np.prod(shape)) if shape else 1
        dt = info["dtype"]
        size = {"F32": 4, "BF16": 2, "F16": 2}.get(dt)
        if size is None:
            raise ValueError(f"{name}: unsupported dtype {dt}")
        if e < b or base + e > mm.size or e - b != n * size:
            raise ValueError(f"{name}: data range does not match its shape")
        buf = mm[base + b:base + e]
        if dt == "F32":
            a = buf.view("<f4") if (base + b) % 4 == 0 else np.frombuffer(buf.tobytes(), "<f4")
        elif dt == "BF16":
            a = (buf.view("<u2").astype(np.uint32) << 16).view(np.float32)
        else:
            a = buf.view("<f2").astype(np.float32)
        out[name] = a.reshape(shape)
    return out


def load_safetensors_dir(d):
    """Every tensor of a model directory: model.safetensors, or each shard that
    model.safetensors.index.json's weight_map names, merged into one dict
    (SafeTensors::open_dir, src/safetensors.rs:56-75: shards in sorted order,
    each opened once, a later shard's tensor replacing an earlier one's)."""
    index = os.path.join(d, "model.safetensors.index.json")
    if not os.path.exists(index):
        return load_safetensors(os.path.join(d, "model.safetensors"))
    with open(index) as f:
        j = json.load(f)
    wm = j.get("weight_map") if isinstance(j, dict) else None
    if not isinstance(wm, dict):
        raise ValueError(f"{index}: index has no weight_map")
    out = {}
    for shard in sorted({v for v in wm.values() if isinstance(v, str)}):
        out.update(load_safetensors(os.path.join(d, shard)))
    return out


LAYER_TENSORS = ("attn_norm", "wq", "wk", "wv", "wo", "bq", "bk", "bv", "q_norm", "k_norm", "ffn_norm", "w_gate",
                 "w_up", "w_down")
_HF = {"attn_norm": "input_layernorm.weight", "wq": "self_attn.q_proj.weight", "wk": "self_attn.k_proj.weight",
       "wv": "self_attn.v_proj.weight", "wo": "self_attn.o_proj.weight", "bq": "self_attn.q_proj.bias",
       "bk": "self_attn.k_proj.bias", "bv": "self_attn.v_proj.bias", "q_norm": "self_attn.q_norm.weight",
       "k_norm": "self_attn.k_norm.weight", "ffn_norm": "post_attention_layernorm.weight",
       "w_gate": "mlp.gate_proj.weight", "w_up": "mlp.up_proj.weight", "w_down": "mlp.down_proj.weight"}


def load_weights(d, cfg):
    """f32 weights in wick's naming (Model::from_tensors, src/model.rs:178-235), with shape checks."""
    st = load_safetensors_dir(d)
    h, q, kv, ff = cfg.hidden, cfg.q_dim, cfg.kv_dim, cfg.intermediate
    shapes = {"attn_norm": (h,), "wq": (q, h), "wk": (kv, h), "wv": (kv, h), "wo": (h, q), "bq": (q,), "bk": (kv,),
              "bv": (kv,), "q_norm": (cfg.head_dim,), "k_norm": (cfg.head_dim,), "ffn_norm": (h,),
              "w_gate": (ff, h), "w_up": (ff, h), "w_down": (h, ff)}
    optional = {"bq", "bk", "bv", "q_norm", "k_norm"}

    def get(name, shape):
        if name not in st:
            raise ValueError(f"missing tensor {name}")
        a = st[name]
        if a.size != int(np.prod(shape)) or (len(shape) == 2 and a.shape != shape):
            raise ValueError(f"{name}: expected shape {list(shape)}, found {list(a.shape)}")
        return np.ascontiguousarray(a.reshape(shape))

    w = {"embed": get("model.embed_tokens.weight", (cfg.vocab, h)), "norm": get("model.norm.weight", (h,))}
    tied = cfg.tie_embeddings or "lm_head.weight" not in st
    w["lm_head"] = None if tied else get("lm_head.weight", (cfg.vocab, h))
    layers = []
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        lw = {}
        for k in LAYER_TENSORS:
            name = p + _HF[k]
            lw[k] = get(name, shapes[k]) if (k not in optional or name in st) else None
        if cfg.attn_bias and (lw["bq"] is None or lw["bk"] is None or lw["bv"] is None):
            raise ValueError(f"{p}: missing attention biases")
        if cfg.arch == "qwen3" and (lw["q_norm"] is None or lw["k_norm"] is None):
            raise ValueError(f"{p}: missing q_norm/k_norm")
        layers.append(lw)
    w["layers"] = layers
    return w
