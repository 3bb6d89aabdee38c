"""A C host program over include/wick_hip.h (tests/c_host/decode_demo.c): the
boundary exercised the way a non-Python caller -- wick's Rust side -- would,
with no Python or torch between the caller and the library."""
import os
import shutil
import subprocess

import pytest

from wick_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c_host", "decode_demo.c")


def build(out):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    libdir = os.path.dirname(_native.HIP_LIB)
    subprocess.run([gcc, "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"), SRC,
                    "-o", out, "-L", libdir, "-l:" + os.path.basename(_native.HIP_LIB), "-Wl,-rpath," + libdir,
                    "-lm"], check=True)
    return out


def test_c_host_builds(tmp_path):
    assert os.path.exists(build(str(tmp_path / "decode_demo")))


@pytest.mark.gpu
def test_c_host_decode_and_prefill(tmp_path):
    exe = build(str(tmp_path / "decode_demo"))
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip().endswith("all ok")
