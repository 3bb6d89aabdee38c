"""Parity on the configurations' own inputs: the tensors bench.py times, drawn
with wick's generator on the device (xoshiro256** seeded through splitmix64,
/root/reference/src/sampler.rs:28-55; one seed per configuration), through the
C ABI against the CPU oracle on host copies of the same tensors.  Per element
|gpu - cpu| <= 2e-5 + 1e-4 |cpu| (the north star's bound).  configs[0] on its
own inputs is tests/test_e2e_gpu.py::test_smollm2_135m_on_the_configs_own_inputs."""
import pytest

import bench
import oracle_lib as ol
from wick_amd import DeviceKvCache

pytestmark = pytest.mark.gpu
THREADS = ol.threads_default()


def _torch():
    import torch
    return torch, torch.device("cuda:0")


def test_config2_decode_all_layers_on_its_own_inputs():
    """Qwen2.5 shape, 24 layers x 32768 positions (seed 2), every
    layer's decode at cache lengths 512, 4096 and 32768."""
    torch, dev = _torch()
    kv, q, att = bench.setup_decode(torch, DeviceKvCache, dev)
    c = bench.DEC
    hd = c["heads"] * c["d"]
    outs = {}
    try:
        for L in (512, 4096, c["L"]):
            for layer in range(c["layers"]):
                kv.attention_device(layer, c["heads"], q.data_ptr() + 4 * hd * layer, 1, L - 1,
                                    att.data_ptr() + 4 * hd * layer)
            torch.cuda.synchronize()
            outs[L] = att.cpu().numpy()
        rec = bench.parity_decode(bench.read_decode_layers(kv), q.cpu().numpy(), outs, THREADS)
    finally:
        kv.close()
    for L in (512, 4096, c["L"]):
        print(f"L={L}: {rec[f'L{L}']}")
    assert rec["ok"], rec


@pytest.mark.parametrize("T", [512, 2048])
def test_config3_prefill_on_its_own_inputs(T):
    """Qwen3 shape, QK-norm then RoPE applied to the seed-3 inputs, empty cache."""
    torch, dev = _torch()
    p = bench.PRE
    _, _, rec = bench.measure_prefill(torch, DeviceKvCache, dev, p["heads"], p["kv_heads"], p["d"], T, 0,
                                      p["theta"], p["seed"], qk_norm=True, steps=1, check_threads=THREADS)
    print(f"T={T}: {rec}")
    assert rec["ok"], rec


def test_config4_chunked_prefill_on_its_own_inputs():
    """TinyLlama shape, 512 tokens onto 1536 cached positions (seed 4)."""
    torch, dev = _torch()
    c = bench.CHUNKED
    _, _, rec = bench.measure_prefill(torch, DeviceKvCache, dev, c["heads"], c["kv_heads"], c["d"], c["t"],
                                      c["start"], c["theta"], c["seed"], qk_norm=False, steps=1,
                                      check_threads=THREADS)
    print(rec)
    assert rec["ok"], rec


def test_config5_layer0_on_its_own_inputs():
    """Llama-3-8B shape, layer 0 of the seed-5 cache (65536 positions),
    decode over the whole cache and over its first 32768 positions."""
    torch, dev = _torch()
    c = bench.LONG
    k, v, q = bench.long_decode_layer_inputs(torch, dev, layer=0)
    att = torch.empty_like(q)
    recs = {}
    with DeviceKvCache(1, c["L"], c["kv_heads"], c["d"]) as kv:
        kv.set_stream(torch.cuda.current_stream().cuda_stream)
        kv.append_device(0, 0, c["L"], k.data_ptr(), v.data_ptr())
        kh, vh, qh = k.cpu().numpy(), v.cpu().numpy(), q.cpu().numpy()
        for L in (c["L"], 32768):
            kv.attention_device(0, c["heads"], q.data_ptr(), 1, L - 1, att.data_ptr())
            torch.cuda.synchronize()
            recs[L] = bench.parity_attention(qh, kh[:L], vh[:L], 1, L - 1, c["heads"], c["kv_heads"], c["d"],
                                             att.cpu().numpy(), THREADS)
    for L, rec in recs.items():
        print(f"L={L}: {rec}")
        assert rec["ok"], (L, rec)
