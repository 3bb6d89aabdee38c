"""Host-side loading: config.json parsing and safetensors (single file and sharded).

Restates the reference's loader contract: Config::from_json
(/root/reference/src/config.rs:55-133), SafeTensors::open_dir with a sharded
index (/root/reference/src/safetensors.rs:56-75), and the test
rejects_mismatched_weights (/root/reference/tests/tiny_models.rs:134-147).
CPU only.
"""
import json
import os
import shutil

import numpy as np
import pytest

from wick_amd.model import Config, load_safetensors, load_safetensors_dir, load_weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "tiny")
MODELS = ["llama3-scaled-f32", "qwen2-bias-bf16", "qwen3-qknorm-f32"]


def _raw_tensors(path):
    """name -> (dtype, shape, raw bytes) straight from a safetensors file."""
    with open(path, "rb") as f:
        data = f.read()
    hlen = int.from_bytes(data[:8], "little")
    header = json.loads(data[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        b, e = info["data_offsets"]
        out[name] = (info["dtype"], info["shape"], data[base + b:base + e])
    return out


def _write_safetensors(path, tensors):
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, raw) in tensors.items():
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


@pytest.mark.parametrize("name", MODELS)
def test_sharded_checkpoint_loads_the_same_weights(name, tmp_path):
    src = os.path.join(GOLDEN, name)
    raw = _raw_tensors(os.path.join(src, "model.safetensors"))
    names = sorted(raw)
    # two shards, tensors interleaved between them; the index lists them in
    # reverse so the loader's own (sorted) shard order is what counts
    shards = {"model-00002-of-00002.safetensors": names[1::2], "model-00001-of-00002.safetensors": names[0::2]}
    weight_map = {}
    for shard, members in shards.items():
        _write_safetensors(os.path.join(tmp_path, shard), {n: raw[n] for n in members})
        weight_map.update({n: shard for n in members})
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": dict(reversed(list(weight_map.items())))}, f)
    shutil.copy(os.path.join(src, "config.json"), tmp_path)

    single = load_safetensors(os.path.join(src, "model.safetensors"))
    merged = load_safetensors_dir(str(tmp_path))
    assert sorted(merged) == sorted(single)
    for n in single:
        assert merged[n].dtype == single[n].dtype and merged[n].shape == single[n].shape
        assert np.array_equal(merged[n].view(np.uint32), single[n].view(np.uint32)), n

    cfg = Config.load(src)
    w1, w2 = load_weights(src, cfg), load_weights(str(tmp_path), cfg)
    assert np.array_equal(w1["embed"], w2["embed"])
    for l1, l2 in zip(w1["layers"], w2["layers"]):
        for k in l1:
            assert (l1[k] is None) == (l2[k] is None), k
            if l1[k] is not None:
                assert np.array_equal(l1[k], l2[k]), k


def test_index_without_weight_map_is_an_error(tmp_path):
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}}, f)
    with pytest.raises(ValueError, match="weight_map"):
        load_safetensors_dir(str(tmp_path))


def test_rejects_mismatched_weights(tmp_path):
    """tests/tiny_models.rs:134-147: a config that disagrees with the tensors
    (hidden_size 64 -> 96) fails cleanly with an "expected shape" message."""
    src = os.path.join(GOLDEN, "qwen2-bias-bf16")
    shutil.copy(os.path.join(src, "model.safetensors"), tmp_path)
    with open(os.path.join(src, "config.json")) as f:
        text = f.read()
    assert '"hidden_size": 64' in text
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        f.write(text.replace('"hidden_size": 64', '"hidden_size": 96'))
    cfg = Config.load(str(tmp_path))
    with pytest.raises(ValueError, match="expected shape"):
        load_weights(str(tmp_path), cfg)


def _base_config():
    with open(os.path.join(GOLDEN, "llama3-scaled-f32", "config.json")) as f:
        return json.load(f)


def test_unsupported_activation_is_rejected():
    """src/config.rs:74-78: an FFN other than SwiGLU must not load silently."""
    j = _base_config()
    j["hidden_act"] = "gelu"
    with pytest.raises(ValueError, match="unsupported activation gelu"):
        Config.from_json(j)
    j["hidden_act"] = "silu"
    Config.from_json(j)
    del j["hidden_act"]
    Config.from_json(j)


def test_rope_scaling_fallback_only_when_missing_or_null():
    """src/config.rs:81-106: rope_scaling is used when present and not null --
    even an empty object, which means the default rotation -- and only a
    missing or null rope_scaling falls back to rope_parameters."""
    j = _base_config()
    llama3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
              "original_max_position_embeddings": 64}
    for k in ("rope_scaling", "rope_parameters"):
        j.pop(k, None)
    j["rope_theta"] = 10000.0
    j["rope_parameters"] = dict(llama3, rope_theta=10000.0)
    assert Config.from_json(j).rope_scaling is not None          # missing -> rope_parameters
    j["rope_scaling"] = None
    assert Config.from_json(j).rope_scaling is not None          # null -> rope_parameters
    j["rope_scaling"] = {}
    assert Config.from_json(j).rope_scaling is None              # {} -> default rotation
    j["rope_scaling"] = {"type": "default"}
    assert Config.from_json(j).rope_scaling is None
    j["rope_scaling"] = {"rope_type": "yarn", "factor": 4.0}
    with pytest.raises(ValueError, match="unsupported rope_scaling"):
        Config.from_json(j)
    j["rope_scaling"] = dict(llama3)
    del j["rope_scaling"]["low_freq_factor"]
    with pytest.raises(ValueError, match="missing low_freq_factor"):
        Config.from_json(j)


def test_theta_and_eps_defaults():
    j = _base_config()
    for k in ("rope_theta", "rope_parameters", "rope_scaling"):
        j.pop(k, None)
    j["rms_norm_eps"] = None
    cfg = Config.from_json(j)
    assert cfg.rope_theta == 10000.0 and cfg.rms_eps == float(np.float32(1e-6))
    j["rope_parameters"] = {"rope_theta": 500000.0, "rope_type": "default"}
    assert Config.from_json(j).rope_theta == 500000.0
    j["rope_theta"] = 1e6
    assert Config.from_json(j).rope_theta == 1e6


def test_missing_required_key_is_a_clean_error():
    j = _base_config()
    del j["intermediate_size"]
    with pytest.raises(ValueError, match="missing intermediate_size"):
        Config.from_json(j)
