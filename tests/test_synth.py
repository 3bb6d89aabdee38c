"""bench.py's synthetic inputs come from wick's generator (xoshiro256** seeded
through splitmix64, /root/reference/src/sampler.rs:28-55): the Python form
(wick_amd/synthetic.py, token ids) against the oracle's pinned generator, and the
jump polynomials libwick_probe.so's wick_synth_normal uses to cut a seed's stream
into per-row substreams, against the powers of the generator's own transition
matrix over GF(2): jump = 2^128 draws, long jump = 2^192 draws."""
import ctypes
import os
import re

import numpy as np

import oracle_lib as ol
from wick_amd.synthetic import WickRng, wick_prompt

HERE = os.path.dirname(os.path.abspath(__file__))
SYNTH = os.path.join(os.path.dirname(HERE), "wick_amd", "csrc", "synth.hip")
M64 = (1 << 64) - 1


def step(s):
    """The state update of xoshiro256** (linear over GF(2))."""
    t = (s[1] << 17) & M64
    s[2] ^= s[0]
    s[3] ^= s[1]
    s[1] ^= s[2]
    s[0] ^= s[3]
    s[2] ^= t
    s[3] = ((s[3] << 45) | (s[3] >> 19)) & M64


def poly_jump(s, poly):
    """The published jump algorithm: XOR of the states at the polynomial's set bits."""
    s, a = list(s), [0, 0, 0, 0]
    for w in poly:
        for b in range(64):
            if (w >> b) & 1:
                a = [a[i] ^ s[i] for i in range(4)]
            step(s)
    return a


def to_bits(s):
    return np.array([(s[i // 64] >> (i % 64)) & 1 for i in range(256)], dtype=np.float64)


def from_bits(v):
    s = [0, 0, 0, 0]
    for i in range(256):
        if int(v[i]) & 1:
            s[i // 64] |= 1 << (i % 64)
    return s


def transition_power(log2_n):
    """M^(2^log2_n) over GF(2), M the one-draw transition."""
    m = np.zeros((256, 256))
    for i in range(256):
        s = from_bits(np.eye(256)[i])
        step(s)
        m[:, i] = to_bits(s)
    for _ in range(log2_n):
        m = np.mod(m @ m, 2.0)
    return m


def constants():
    src = open(SYNTH).read()
    out = {}
    for name in ("kJump", "kLongJump"):
        body = re.search(name + r"\[4\] = \{([^}]*)\}", src).group(1)
        out[name] = [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]+)ULL", body)]
        assert len(out[name]) == 4
    return out


def test_python_generator_matches_the_oracle():
    for seed in (0, 1, 2, 0xDEADBEEF, M64):
        a, b = WickRng(seed), ol.OracleRng(seed)
        assert [a.next_u64() for _ in range(200)] == [b.next_u64() for _ in range(200)]


def test_prompt_ids_are_the_generator_modulo_the_vocabulary():
    rng = ol.OracleRng(1)
    assert wick_prompt(1, 128, 49152).tolist() == [rng.next_u64() % 49152 for _ in range(128)]


def test_jump_polynomials_advance_2_to_128_and_2_to_192_draws():
    c = constants()
    m128 = transition_power(128)
    m192 = m128.copy()
    for _ in range(64):
        m192 = np.mod(m192 @ m192, 2.0)
    rng = np.random.default_rng(0)
    for _ in range(3):
        s = [int(x) for x in rng.integers(0, 1 << 63, 4)]
        assert poly_jump(s, c["kJump"]) == from_bits(np.mod(m128 @ to_bits(s), 2.0))
        assert poly_jump(s, c["kLongJump"]) == from_bits(np.mod(m192 @ to_bits(s), 2.0))
    # a dropped or flipped bit of a polynomial would not pass
    bad = list(c["kJump"])
    bad[2] ^= 1 << 17
    s = [1, 2, 3, 4]
    assert poly_jump(s, bad) != from_bits(np.mod(m128 @ to_bits(s), 2.0))


def test_synth_rejects_bad_shapes_before_touching_the_device():
    lib = ctypes.CDLL(os.path.join(os.path.dirname(HERE), "wick_amd", "libwick_probe.so"))
    lib.wick_synth_normal.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_int,
                                      ctypes.c_ulonglong, ctypes.c_float, ctypes.c_void_p]
    assert lib.wick_synth_normal(None, 0, 1, 2, 0, 1.0, None) != 0  # no output
    assert lib.wick_synth_normal(ctypes.c_void_p(256), 0, 1, 3, 0, 1.0, None) != 0  # odd row
    assert lib.wick_synth_normal(ctypes.c_void_p(256), -1, 1, 2, 0, 1.0, None) != 0  # negative tensor
    assert lib.wick_synth_normal(ctypes.c_void_p(256), 0, 0, 2, 0, 1.0, None) != 0  # no rows
