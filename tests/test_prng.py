"""PRNG pins: the init generator (mulberry32 + Box-Muller, src/module.ts:72-90) and the
in-kernel hashes (test/_eval.ts:544-603), checked against independent formulations."""
import math

import numpy as np

import pyoracle
from tensorgrad_amd.module import Mulberry32, box_muller_block


def _mulberry32_scalar(seed, n):
    """One draw at a time, straight from the generator's recurrence on Python ints."""
    s = seed & 0xFFFFFFFF
    out = []
    for _ in range(n):
        s = (s + 0x6D2B79F5) & 0xFFFFFFFF
        t = s
        t = ((t ^ (t >> 15)) * (t | 1)) & 0xFFFFFFFF
        t = (t ^ ((t + (((t ^ (t >> 7)) * (t | 61)) & 0xFFFFFFFF)) & 0xFFFFFFFF)) & 0xFFFFFFFF
        out.append(((t ^ (t >> 14)) & 0xFFFFFFFF) / 4294967296)
    return out


def test_mulberry32_vectorised_equals_recurrence():
    for seed in (0, 1, 42, 12345, 0xFFFFFFFF, 1001):
        r = Mulberry32(seed)
        got = list(r.take(300)) + list(r.take(7))
        assert got == _mulberry32_scalar(seed, 307)


def test_mulberry32_uniformity():
    u = Mulberry32(7).take(200000)
    assert u.min() >= 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 3e-3 and abs(u.var() - 1 / 12) < 2e-3


def test_box_muller_pairs_and_moments():
    rng = Mulberry32(42)
    z = box_muller_block(rng, 5)
    u = _mulberry32_scalar(42, 10)
    want = [math.sqrt(-2 * math.log(max(1e-10, u[2 * i]))) * math.cos(2 * math.pi * u[2 * i + 1]) for i in range(5)]
    assert list(z) == want
    big = box_muller_block(Mulberry32(3), 100000)
    assert abs(big.mean()) < 0.02 and abs(big.std() - 1) < 0.02


def _pcg_imul_py(seed, sc, i):
    h = (seed ^ sc ^ i) & 0xFFFFFFFF
    h = (h * 747796405 + 2891336453) & 0xFFFFFFFF
    h = (((h ^ (h >> ((h >> 28) + 4))) & 0xFFFFFFFF) * 277803737) & 0xFFFFFFFF
    return (h ^ (h >> 22)) & 0xFFFFFFFF


def _pcg_f64_py(seed, sc, i):
    """JS semantics: each `*` and `+` is one correctly rounded IEEE double operation
    (Python floats are IEEE doubles), then ToUint32 of the integral result."""
    h = (seed ^ sc ^ i) & 0xFFFFFFFF
    h = int(float(h) * 747796405.0 + 2891336453.0) % 2 ** 32
    x = (h ^ (h >> ((h >> 28) + 4))) & 0xFFFFFFFF
    h = int(float(x) * 277803737.0) % 2 ** 32
    return (h ^ (h >> 22)) & 0xFFFFFFFF


def test_pcg_hashes_match_independent_formulations():
    rng = np.random.default_rng(0)
    for seed, sc, i in rng.integers(0, 2 ** 32, size=(2000, 3), dtype=np.uint64).tolist():
        assert pyoracle.pcg_f64(seed, sc, i) == _pcg_f64_py(seed, sc, i)
        h1, h2 = pyoracle.pcg_imul2(seed, sc, i)
        assert h1 == _pcg_imul_py(seed, sc, i)
        assert h2 == _pcg_imul_py(h1, 0, 0)
    # the f64 hash really differs from the wrapping one (rounded products above 2^53)
    diffs = sum(pyoracle.pcg_f64(s, 0, 0) != _pcg_imul_py(s, 0, 0) for s in range(1 << 20, (1 << 20) + 2000))
    assert diffs > 1000


def test_salt_constant():
    for salt in (0, 1, 2, 23, 1000):
        assert pyoracle.salt_const(salt) == (salt * 0x9E3779B1) & 0xFFFFFFFF
