"""Test data generators.

``RefTestRng`` restates the reference unit-test generator (tests/test_main.cpp:26-48):
a global xorshift32 seeded 0x12345678, ``make_bf16`` and ``clustered``. C++ leaves
the evaluation order of ``make_bf16(exp, rnd() & 0x7F, rnd() & 1)`` unspecified;
this helper draws the mantissa first, then the sign. The reference tests only check
invariants on this data (round trip, raw == xkv bits), so the draw order changes
which values are tested, not what a test asserts.
"""
from __future__ import annotations

import numpy as np


def make_bf16(exp: int, mant: int, sign: int) -> int:
    return (0x8000 if sign else 0) | ((exp & 0xFF) << 7) | (mant & 0x7F)


class RefTestRng:
    def __init__(self, seed: int = 0x12345678):
        self.s = seed & 0xFFFFFFFF

    def rnd(self) -> int:
        s = self.s
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        self.s = s
        return s

    def clustered(self, n: int, base: int, spread: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint16)
        for i in range(n):
            exp = base + self.rnd() % spread
            if self.rnd() % 200 == 0:
                exp = (base + 80) & 0xFF
            mant = self.rnd() & 0x7F
            sign = self.rnd() & 1
            out[i] = make_bf16(exp, mant, sign)
        return out

    def queries(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint16)
        for i in range(n):
            mant = self.rnd() & 0x7F
            sign = self.rnd() & 1
            out[i] = make_bf16(120, mant, sign)
        return out


# The reference's test_bitexact cases (tests/test_main.cpp:165-172):
# (dim, n_q, seq, block, threads).
REF_BITEXACT_CASES = [
    (64, 1, 1, 128, 1),
    (64, 7, 17, 128, 1),
    (64, 7, 128, 128, 1),
    (64, 3, 200, 64, 1),
    (64, 7, 300, 64, 4),
    (32, 2, 90, 32, 1),
    (16, 1, 40, 16, 1),
    (64, 7, 256, 128, 4),
]


def ref_test_stream():
    """Replays the reference test binary's draw sequence (test_main.cpp:161-172):
    yields ("roundtrip", block, kv), ("size", kv), then ("bitexact", case, q, k, v)."""
    rng = RefTestRng()
    for block in (16, 32, 64, 128):
        kv = rng.clustered(300 * 64, 110, 6)
        kv[0] = 0
        kv[1] = 0x8000
        kv[2] = 0x0001
        kv[3] = 0x7F80
        kv[4] = 0x7FC1
        yield ("roundtrip", block, kv)
    yield ("size", rng.clustered(128 * 64, 100, 3))
    for case in REF_BITEXACT_CASES:
        dim, n_q, seq, block, threads = case
        k = rng.clustered(seq * dim, 108, 8)
        v = rng.clustered(seq * dim, 112, 5)
        q = rng.queries(n_q * dim)
        yield ("bitexact", case, q, k, v)


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """FP32 -> BF16 bits, round to nearest even (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def random_kv(rng: np.random.Generator, seq: int, dim: int, *, spread_lo=-4.0, spread_hi=2.0,
              sigma=1.0, outliers=0, specials=False, wide=False) -> np.ndarray:
    """Gaussian K/V with a per-channel log-uniform scale, rounded to BF16."""
    scale = np.exp2(rng.uniform(spread_lo, spread_hi, size=dim)).astype(np.float32)
    if outliers:
        scale[rng.choice(dim, outliers, replace=False)] *= 32.0
    x = (rng.standard_normal((seq, dim)).astype(np.float32) * sigma) * scale
    if wide:
        x *= np.exp2(rng.integers(-30, 30, size=(seq, dim))).astype(np.float32)
    b = bf16_from_f32(x.reshape(-1))
    if specials:
        n = b.size
        idx = rng.choice(n, max(8, n // 500), replace=False)
        pool = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x7F80, 0xFF80, 0x7FC1, 0x0040],
                        dtype=np.uint16)
        b[idx] = pool[rng.integers(0, pool.size, size=idx.size)]
    return b
