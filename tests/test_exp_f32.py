"""The device sampler's exp (wick_amd/csrc/exp_f32.h) against the C library's
expf, which is what wick's f32::exp calls (the softmax of Sampler::sample,
/root/reference/src/sampler.rs:97): the same bits for every one of the 2^32
f32 inputs.  The header's function is compiled for the host (hipcc) and run
over all inputs; the expected values are the host's expf, i.e. glibc's build
for CPUs with FMA (the variant glibc selects on x86-64 CPUs that have it).
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "wick_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _cpu_has_fma():
    try:
        with open("/proc/cpuinfo") as f:
            return any(line.startswith("flags") and " fma " in line + " " for line in f)
    except OSError:
        return False


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not found")
@pytest.mark.skipif(not _cpu_has_fma(), reason="the host's expf is glibc's build for CPUs without FMA")
def test_exp_f32_matches_host_expf_on_every_input(tmp_path):
    exe = str(tmp_path / "exp_f32_check")
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-I", CSRC, os.path.join(HERE, "exp_f32_check.cpp"), "-o", exe],
                   check=True, timeout=300)
    threads = str(max(1, min(8, os.cpu_count() or 1)))
    r = subprocess.run([exe, threads], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
