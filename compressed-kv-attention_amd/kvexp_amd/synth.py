"""Seeded synthetic K/V/Q for the BASELINE configurations (numpy, BF16 bits as uint16).

Every tensor is drawn from numpy's PCG64 with a seed derived from the config
seed and the (sequence, layer, head) position, so a head can be regenerated on
its own. Values are FP32 rounded to BF16 (nearest even).

  C1  dim 64, seq 8192, 1 query. K, V = N(0,1) * 2^U(-4,2) per channel; about
      0.3% of elements get their exponent moved 20 binades down (escapes).
  C2  Qwen2.5-0.5B step: 24 layers x 2 KV heads x 7 queries, dim 64, seq 32768.
      K = N(0,1) * 2^U(-6,4) per channel, 2 outlier channels x32; ~6% of K
      blocks drawn from a 3-binade band (they encode as 2-bit). V = N(0, 0.5^2)
      with ~0.3% of its elements moved 20 binades down (escapes; K's own
      escape rate is ~0.3%). Q = N(0,1).
  C3  C2 with 32 sequences of lengths round(exp(U(ln 1024, ln 32768))).
  C4  Llama-3-8B step: 32 layers x 8 KV heads x 4 queries, dim 128, seq 131072.
      K = N(0,1) * 2^U(-5,3), V = N(0, 0.5^2).
  C5  dim 256, block 255, seq 100003, 8 KV heads x 8 queries, batch 4; K with a
      wide exponent spread, blocks that encode raw / 2-bit / 4-bit, and
      denormals, +-0 and +-Inf planted.
"""
from __future__ import annotations

import numpy as np

CONFIGS = {
    "c1": dict(layers=1, kv_heads=1, group=1, dim=64, seq=8192, block=128, batch=1, seed=1),
    "c2": dict(layers=24, kv_heads=2, group=7, dim=64, seq=32768, block=128, batch=1, seed=2),
    "c3": dict(layers=24, kv_heads=2, group=7, dim=64, seq=None, block=128, batch=32, seed=3),
    "c4": dict(layers=32, kv_heads=8, group=4, dim=128, seq=131072, block=128, batch=1, seed=4),
    "c5": dict(layers=1, kv_heads=8, group=8, dim=256, seq=100003, block=255, batch=4, seed=5),
}


def bf16(x: np.ndarray) -> np.ndarray:
    """FP32 -> BF16 bits, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def rng_for(seed: int, *pos: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, *pos])))


def c3_lengths(seed: int = 3, n: int = 32) -> list[int]:
    r = rng_for(seed, 999)
    return [int(round(np.exp(r.uniform(np.log(1024), np.log(32768))))) for _ in range(n)]


def head_kv(cfg: str, seq: int, b: int = 0, layer: int = 0, head: int = 0):
    """(k, v) as uint16 [seq * dim] for one KV head of a configuration."""
    c = CONFIGS[cfg]
    dim, block = c["dim"], c["block"]
    r = rng_for(c["seed"], b, layer, head)
    if cfg == "c1":
        scale = np.exp2(r.uniform(-4, 2, dim)).astype(np.float32)
        k = r.standard_normal((seq, dim), dtype=np.float32) * scale
        v = r.standard_normal((seq, dim), dtype=np.float32) * np.exp2(r.uniform(-4, 2, dim)).astype(np.float32)
        kb, vb = bf16(k.reshape(-1)), bf16(v.reshape(-1))
        for arr in (kb, vb):
            sel = r.random(arr.size) < 0.003
            e = (arr[sel] >> 7) & 0xFF
            e = np.where(e > 20, e - 20, e + 20)
            arr[sel] = (arr[sel] & 0x807F) | (e.astype(np.uint16) << 7)
        return kb, vb
    if cfg in ("c2", "c3"):
        scale = np.exp2(r.uniform(-6, 4, dim)).astype(np.float32)
        scale[r.choice(dim, 2, replace=False)] *= 32.0
        k = r.standard_normal((seq, dim), dtype=np.float32) * scale
        nblk = (seq + block - 1) // block
        narrow = np.nonzero(r.random(nblk) < 0.06)[0]
        for bi in narrow:
            t0, t1 = bi * block, min(seq, (bi + 1) * block)
            band = r.uniform(1.0, 7.99, (t1 - t0, dim)).astype(np.float32)
            sign = np.where(r.random((t1 - t0, dim)) < 0.5, -1.0, 1.0).astype(np.float32)
            k[t0:t1] = band * sign * scale
        v = r.standard_normal((seq, dim), dtype=np.float32) * np.float32(0.5)
        vb = bf16(v.reshape(-1))
        # ~0.3 % of V elements moved 20 binades down (near-zero values that
        # leave every 4-bit window): with K's own escapes (its 2-bit blocks
        # and distribution tails, ~0.3 %) the step's escape rate is ~0.3 %
        sel = np.nonzero(r.random(vb.size) < 0.003)[0]
        e = (vb[sel] >> 7) & 0xFF
        vb[sel] = (vb[sel] & 0x807F) | (np.where(e > 20, e - 20, e + 20).astype(np.uint16) << 7)
        return bf16(k.reshape(-1)), vb
    if cfg == "c4":
        scale = np.exp2(r.uniform(-5, 3, dim)).astype(np.float32)
        k = r.standard_normal((seq, dim), dtype=np.float32) * scale
        v = r.standard_normal((seq, dim), dtype=np.float32) * np.float32(0.5)
        return bf16(k.reshape(-1)), bf16(v.reshape(-1))
    if cfg == "c5":
        nblk = (seq + block - 1) // block
        kind = r.integers(0, 10, nblk)  # 0: raw-like spread, 1-2: 2-bit band, else 4-bit with ~8% escapes
        k = np.empty((seq, dim), dtype=np.float32)
        for bi in range(nblk):
            t0, t1 = bi * block, min(seq, (bi + 1) * block)
            n = t1 - t0
            if kind[bi] == 0:
                k[t0:t1] = r.standard_normal((n, dim), dtype=np.float32) * np.exp2(
                    r.integers(-60, 60, (n, dim))).astype(np.float32)
            elif kind[bi] <= 2:
                k[t0:t1] = r.uniform(1.0, 7.99, (n, dim)).astype(np.float32) * np.where(
                    r.random((n, dim)) < .5, -1, 1).astype(np.float32)
            else:
                x = r.standard_normal((n, dim), dtype=np.float32)
                wide = r.random((n, dim)) < 0.08
                x[wide] *= np.exp2(r.integers(-40, 40, wide.sum())).astype(np.float32)
                k[t0:t1] = x
        kb = bf16(k.reshape(-1))
        specials = np.array([0x0000, 0x8000, 0x0001, 0x8003, 0x007F, 0x7F80, 0xFF80], dtype=np.uint16)
        idx = r.choice(kb.size, kb.size // 1000, replace=False)
        kb[idx] = specials[r.integers(0, specials.size, idx.size)]
        v = r.standard_normal((seq, dim), dtype=np.float32) * np.float32(0.5)
        vb = bf16(v.reshape(-1))
        idx = r.choice(vb.size, vb.size // 5000, replace=False)
        vb[idx] = specials[r.integers(0, 5, idx.size)]  # V: zeros and denormals only
        return kb, vb
    raise KeyError(cfg)


def queries(cfg: str, n_heads: int, b: int = 0) -> np.ndarray:
    """Q for n_heads KV heads x group queries: uint16 [n_heads * group * dim]."""
    c = CONFIGS[cfg]
    r = rng_for(c["seed"], b, 10_000)
    x = r.standard_normal(n_heads * c["group"] * c["dim"], dtype=np.float32)
    return bf16(x)
