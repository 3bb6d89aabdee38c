"""The C ABI library loads and exports every symbol include/*.h declares.

CPU-only: argument checks that fail before any device work are exercised; no
compute call is made without a GPU.
"""
import ctypes
import os
import re

import pytest

from wick_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in sorted(os.listdir(inc)):
        if fn.endswith(".h"):
            with open(os.path.join(inc, fn)) as f:
                names |= set(re.findall(r"\b(wick_hip_\w+)\s*\(", f.read()))
    return names


def test_header_and_binding_agree():
    assert header_symbols() == set(_native.SIGNATURES)


def test_header_constants_and_binding_agree():
    """Status codes and option numbers: the header's #defines and the Python binding's."""
    with open(os.path.join(ROOT, "include", "wick_hip.h")) as f:
        defs = dict(re.findall(r"#define WICK_HIP_(\w+)\s+\(?(-?\d+)\)?", f.read()))
    assert {k: int(v) for k, v in defs.items()} == {
        "OK": _native.OK, "EINVAL": _native.EINVAL, "EHIP": _native.EHIP, "ENOMEM": _native.ENOMEM,
        "EDEVICE": _native.EDEVICE, "OPT_DECODE_CHUNK": _native.OPT_DECODE_CHUNK,
        "OPT_DECODE_ORDER": _native.OPT_DECODE_ORDER}


def test_library_exports_every_symbol():
    lib = _native.load()
    for name in header_symbols():
        assert hasattr(lib, name), name


def test_integration_build_rs_lists_every_source():
    """The build.rs that INTEGRATION.md gives the Rust side compiles exactly the
    sources wick_amd/build.py builds libwick_hip.so from."""
    from wick_amd import build
    with open(os.path.join(ROOT, "INTEGRATION.md")) as f:
        text = f.read()
    block = re.search(r"## 1\. `build\.rs`.*?```rust\n(.*?)```", text, re.S)
    assert block, "INTEGRATION.md has no build.rs block"
    listed = re.findall(r'"(wick_amd/csrc/[\w.]+)"', block.group(1))
    assert len(listed) == len(set(listed)), listed
    assert sorted(listed) == sorted(build.HIP_SOURCES)
    for src in build.HIP_SOURCES:
        assert os.path.exists(os.path.join(ROOT, src)), src


def test_library_leaves_no_internal_symbol_undefined():
    """Every wick_hip_* and wick:: symbol the library uses is defined in it: a
    source missing from the build list shows up here (as it would at link time)."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--undefined-only", _native.HIP_LIB], check=True,
                         stdout=subprocess.PIPE, text=True).stdout
    missing = [l.split()[-1] for l in out.splitlines() if "wick_hip_" in l or "4wick" in l]
    assert not missing, missing


def test_argument_errors_without_device_work():
    lib = _native.load()
    h = ctypes.c_void_p()
    assert lib.wick_hip_kv_create(1, 16, 2, 48, ctypes.byref(h)) == _native.EINVAL
    assert b"head_dim" in lib.wick_hip_last_error()
    assert lib.wick_hip_kv_create(0, 16, 2, 64, ctypes.byref(h)) == _native.EINVAL
    assert lib.wick_hip_kv_create(1, 16, 2, 64, None) == _native.EINVAL
    lib.wick_hip_kv_destroy(None)
    assert lib.wick_hip_kv_set_option(None, 1, 64) == _native.EINVAL
    assert lib.wick_hip_attention(None, 0, 4, None, 1, 0, None) == _native.EINVAL
    assert lib.wick_hip_attention_device_noalloc(None, 0, 4, None, 1, 0, None) == _native.EINVAL
    assert lib.wick_hip_kv_last_grid(None) == 0
    assert lib.wick_hip_kv_set_rope(None, None) == _native.EINVAL
    assert lib.wick_hip_kv_set_prep(None, 0, 4, None, None, None, None, None, ctypes.c_float(1e-6)) == _native.EINVAL
    assert lib.wick_hip_attend(None, 0, 4, None, None, None, 1, 0, None) == _native.EINVAL
    assert lib.wick_hip_attend_device(None, 0, 4, None, None, None, 1, 0, None) == _native.EINVAL
    assert b"null" in lib.wick_hip_last_error()
    m = ctypes.c_void_p()
    assert lib.wick_hip_model_create(None, None, None, None, None, None, ctypes.byref(m)) == _native.EINVAL
    assert lib.wick_hip_model_create(None, None, None, None, None, None, None) == _native.EINVAL
    lib.wick_hip_model_destroy(None)
    assert lib.wick_hip_model_new_cache(None, 16, ctypes.byref(m)) == _native.EINVAL
    assert lib.wick_hip_model_forward(None, None, None, 1, 0, 0, None) == _native.EINVAL
    assert lib.wick_hip_model_prefill(None, None, None, 1, 0, None) == _native.EINVAL
    assert lib.wick_hip_model_decode(None, None, 0, 0, 1, None) == _native.EINVAL
    assert lib.wick_hip_model_new_sampler(None, None, ctypes.byref(m)) == _native.EINVAL
    n = ctypes.c_int()
    assert lib.wick_hip_model_generate(None, None, None, None, 1, 0, 1, None, 0, None, ctypes.byref(n),
                                       ctypes.byref(n)) == _native.EINVAL
    from wick_amd.sampler import SamplerConfig, c_config
    cfg = c_config(SamplerConfig())
    assert lib.wick_hip_sampler_create(None, 10, None, ctypes.byref(m)) == _native.EINVAL
    assert lib.wick_hip_sampler_create(ctypes.byref(cfg), 0, None, ctypes.byref(m)) == _native.EINVAL
    assert b"vocab" in lib.wick_hip_last_error()
    assert lib.wick_hip_sampler_create(ctypes.byref(cfg), 10, None, None) == _native.EINVAL
    lib.wick_hip_sampler_destroy(None)
    assert lib.wick_hip_sampler_sample(None, None, None, 0, None) == _native.EINVAL
    assert lib.wick_hip_sampler_sample_device(None, None, None, 0, None) == _native.EINVAL
    assert lib.wick_hip_sampler_rng_state(None, None) == _native.EINVAL
    assert lib.wick_hip_sampler_last_candidates(None, None, None, None, None, 0) == _native.EINVAL


def test_no_device_is_an_error_not_a_fallback():
    try:
        import torch
        if torch.cuda.device_count() > 0:
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    lib = _native.load()
    h = ctypes.c_void_p()
    rc = lib.wick_hip_kv_create(1, 16, 2, 64, ctypes.byref(h))
    assert rc == _native.EDEVICE, rc
    assert not h.value
    from wick_amd.sampler import SamplerConfig, c_config
    cfg = c_config(SamplerConfig())
    assert lib.wick_hip_sampler_create(ctypes.byref(cfg), 100, None, ctypes.byref(h)) == _native.EDEVICE
    assert not h.value


def test_host_mirror_loads_and_reports_errors():
    import numpy as np
    from wick_amd import host
    from wick_amd.model import Config
    lib = host.load()
    assert lib.wick_host_model_create(None, None, None, None, None, None, 1) is None
    assert b"null" in lib.wick_host_last_error()
    # a model can be built on the CPU; a device cache cannot be made without a GPU
    cfg = Config("llama", 32, 64, 1, 4, 2, 16, 8, rms_eps=1e-5)
    rng = np.random.default_rng(0)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    w = {"embed": f(8, 32), "norm": np.ones(32, np.float32), "lm_head": None,
         "layers": [{"attn_norm": np.ones(32, np.float32), "wq": f(64, 32), "wk": f(32, 32), "wv": f(32, 32),
                     "wo": f(32, 64), "bq": None, "bk": None, "bv": None, "q_norm": None, "k_norm": None,
                     "ffn_norm": np.ones(32, np.float32), "w_gate": f(64, 32), "w_up": f(64, 32),
                     "w_down": f(32, 64)}]}
    m = host.HostModel(cfg, w, threads=2)
    try:
        import torch
        if torch.cuda.device_count() > 0:
            return
    except ImportError:
        pass
    with pytest.raises(RuntimeError, match="no HIP device|wick_hip_kv_create"):
        m.new_state(16)


def test_c_program_links_every_declared_function(tmp_path):
    """The headers compile as strict C99 on their own, and a C program that takes the
    address of every function they declare links against libwick_hip.so and runs
    (it makes no call, so no device is needed): the declarations and the exported
    definitions agree for a C linker, not only for ctypes."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    headers = sorted(fn for fn in os.listdir(os.path.join(ROOT, "include")) if fn.endswith(".h"))
    names = sorted(header_symbols())
    src = tmp_path / "link_all.c"
    src.write_text(
        "".join(f'#include "{h}"\n' for h in headers)
        + "#include <stdio.h>\n"
        + "typedef void (*fn_t)(void);\n"
        + "static const fn_t table[] = {\n"
        + "".join(f"    (fn_t)&{n},\n" for n in names)
        + "};\n"
        + "int main(void) {\n"
        + "    size_t i, n = sizeof table / sizeof table[0];\n"
        + "    for (i = 0; i < n; i++)\n"
        + "        if (!table[i]) return 1;\n"
        + '    printf("%u\\n", (unsigned)n);\n'
        + "    return 0;\n"
        + "}\n")
    exe = tmp_path / "link_all"
    libdir = os.path.dirname(_native.HIP_LIB)
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
                    "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe),
                    "-L", libdir, "-l:" + os.path.basename(_native.HIP_LIB), "-Wl,-rpath," + libdir,
                    "-Wl,--no-as-needed"], check=True)
    out = subprocess.run([str(exe)], check=True, stdout=subprocess.PIPE, text=True).stdout
    assert int(out) == len(names)
