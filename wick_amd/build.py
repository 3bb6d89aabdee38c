"""Build the native libraries in-tree (hipcc cross-compiles gfx950; no GPU needed).

    python -m wick_amd.build
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOSTSRC = os.path.join(HERE, "host")
INCLUDE = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (the host pass warns that it
# does not know the feature; that is expected).
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


# Every source of libwick_hip.so, relative to the repository root.  A Rust
# build.rs that compiles the library lists exactly these files.
HIP_SOURCES = (
    "wick_amd/csrc/attention.hip",
    "wick_amd/csrc/prep.hip",
    "wick_amd/csrc/model.hip",
    "wick_amd/csrc/sampler.hip",
    "wick_amd/csrc/api.cpp",
    "wick_amd/csrc/model_api.cpp",
    "wick_amd/csrc/sampler_api.cpp",
)


def build_hip():
    out = os.path.join(HERE, "libwick_hip.so")
    srcs = [os.path.join(ROOT, f) for f in HIP_SOURCES]
    _run([HIPCC, *HIP_FLAGS, "-shared", f"-I{INCLUDE}", f"-I{CSRC}", *srcs, "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_host():
    """The C++ host mirror of wick's Model::forward over the C ABI."""
    srcs = sorted(os.path.join(HOSTSRC, f) for f in os.listdir(HOSTSRC) if f.endswith(".cpp")) \
        if os.path.isdir(HOSTSRC) else []
    if not srcs:
        return None
    out = os.path.join(HERE, "libwick_host.so")
    cmd = ["g++", "-O2", "-mavx2", "-mfma", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-std=c++17",
           "-shared", "-pthread", f"-I{INCLUDE}", *srcs, "-o", out + ".tmp",
           f"-L{HERE}", "-lwick_hip", "-Wl,-rpath,$ORIGIN"]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


PROBE_SOURCES = ("roofline_probe.hip", "synth.hip")


def build_probe():
    """Measurement helpers for bench.py (read ceiling, launch floor, synthetic
    inputs from wick's generator); not part of the attention path."""
    out = os.path.join(HERE, "libwick_probe.so")
    _run([HIPCC, *HIP_FLAGS, "-shared", *(os.path.join(CSRC, f) for f in PROBE_SOURCES), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_all():
    build_hip()
    build_host()
    build_probe()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
