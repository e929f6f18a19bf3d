"""Pins the CPU oracle (oracle/kvexp_oracle.c) before it is trusted as the checker.

1. Golden vectors written by the compiled reference (tests/golden/make_golden.py).
2. The compiled reference itself (oracle/_ref), on seeded random inputs, where built.
3. Closed forms and invariants: clean-block sizes from the reference README, the
   size model, decode(encode(x)) == x, the identity-token known answer
   (tests/test_main.cpp:102-122), and FP64 brute-force attention on small inputs.
4. Error paths: the reference's exception class and message for malformed input.
"""
import hashlib

import numpy as np
import pytest

from conftest import bits_equal
from kvdata import bf16_from_f32, bf16_to_f32, random_kv


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ----------------------------------------------------------------- golden ----
def test_golden_codec(oracle, golden):
    z, man = golden
    for c in man["codec"]:
        kv = z[f"codec/{c['name']}/kv"]
        blob = z[f"codec/{c['name']}/blob"]
        assert sha(blob) == c["sha256"], c["name"]
        got = oracle.encode(kv, c["seq"], c["dim"], c["block"])
        assert np.array_equal(got, blob), c["name"]
        assert np.array_equal(oracle.decode(blob, c["seq"], c["dim"]), kv), c["name"]


def test_golden_tie_rules(golden):
    z, _ = golden
    # codec.cpp:94-103: ties prefer raw, then fewer escapes, then fewer bits;
    # codec.cpp:29 keeps the smallest base among equal windows.
    assert z["codec/tie_raw_vs_4bit/blob"][0] == 0
    assert z["codec/tie_raw_vs_2bit/blob"][0] == 0
    assert z["codec/tie_2bit_vs_4bit/blob"][0] == 4
    b = z["codec/tie_base_choice/blob"]
    assert b[0] == 2 and b[8] == 98


def test_golden_attention(oracle, golden):
    z, man = golden
    for c in man["attn"]:
        n = c["name"]
        q, k, v = z[f"attn/{n}/q"], z[f"attn/{n}/k"], z[f"attn/{n}/v"]
        kx = oracle.encode(k, c["seq"], c["dim"], c["block"])
        vx = oracle.encode(v, c["seq"], c["dim"], c["block"])
        assert sha(kx) == c["k_sha256"] and sha(vx) == c["v_sha256"], n
        for be in c["backends"]:
            for th in c["threads"]:
                want = z[f"attn/{n}/{be}/t{th}"]
                kw = dict(n_q=c["n_q"], dim=c["dim"], seq=c["seq"], threads=th, split=c["block"])
                assert bits_equal(oracle.attention(be, q, k, v, **kw), want), (n, be, th, "raw")
                assert bits_equal(oracle.attention(be, q, kx=kx, vx=vx, **kw), want), (n, be, th, "xkv")


def test_golden_scalar_equals_avx2(golden):
    """attention.hpp:30-39 and test_main.cpp:146-148: AVX2 and scalar give the same bits."""
    z, man = golden
    for c in man["attn"]:
        for th in c["threads"]:
            s = z[f"attn/{c['name']}/scalar/t{th}"]
            a = z[f"attn/{c['name']}/avx2/t{th}"]
            assert bits_equal(s, a), (c["name"], th)


# ------------------------------------------------------------ reference ----
def _random_case(rng, trial):
    dim = int(rng.choice([8, 16, 32, 64, 128, 256]))
    n_q = int(rng.integers(1, 9))
    seq = int(rng.integers(1, 500))
    blocks = [b for b in (4, 16, 64, 100, 128, 255) if b * dim <= 65535]
    block = int(rng.choice(blocks))
    kind = trial % 4
    if kind == 0:
        k = rng.integers(0, 65536, seq * dim, dtype=np.uint16)
    elif kind == 1:
        x = rng.uniform(1.0, 7.9, seq * dim) * np.where(rng.random(seq * dim) < .5, -1, 1)
        k = bf16_from_f32(x.astype(np.float32))
    else:
        k = random_kv(rng, seq, dim, outliers=min(2, dim), specials=kind == 3, wide=kind == 3)
    v = random_kv(rng, seq, dim, specials=trial % 5 == 0)
    q = random_kv(rng, n_q, dim, spread_lo=-1, spread_hi=1)
    return dim, n_q, seq, block, q, k, v


def test_oracle_matches_reference_random(oracle, reference):
    rng = np.random.default_rng(7)
    for trial in range(120):
        dim, n_q, seq, block, q, k, v = _random_case(rng, trial)
        kx = reference.encode(k, seq, dim, block)
        vx = reference.encode(v, seq, dim, block)
        assert np.array_equal(oracle.encode(k, seq, dim, block), kx), trial
        assert np.array_equal(oracle.encode(v, seq, dim, block), vx), trial
        assert np.array_equal(oracle.decode(kx, seq, dim), reference.decode(kx, seq, dim)), trial
        th = int(rng.integers(1, 7))
        split = block * int(rng.integers(1, 3))
        for be in ("scalar", "avx2", "avx512"):
            if (be == "avx512" and dim % 32) or not reference.has(be):
                continue
            kw = dict(n_q=n_q, dim=dim, seq=seq, threads=th, split=split)
            want = reference.attention(be, q, kx=kx, vx=vx, **kw)
            assert bits_equal(oracle.attention(be, q, kx=kx, vx=vx, **kw), want), (trial, be)
            assert bits_equal(oracle.attention(be, q, k, v, **kw), want), (trial, be)


def test_oracle_matches_reference_daz(oracle, reference):
    """VDPBF16PS treats BF16 denormal inputs as zero: observable when a denormal K
    element meets a huge query element."""
    if not reference.avx512_bf16:
        pytest.skip("host without AVX512_BF16")
    rng = np.random.default_rng(3)
    differs = 0
    for trial in range(60):
        dim, n_q, seq = 32 * int(rng.integers(1, 5)), int(rng.integers(1, 4)), int(rng.integers(2, 30))
        k = (rng.integers(1, 128, seq * dim) | (rng.integers(0, 2, seq * dim) << 15)).astype(np.uint16)
        q = bf16_from_f32((rng.standard_normal(n_q * dim) * 2.0 ** rng.uniform(100, 126, n_q * dim)).astype(np.float32))
        v = random_kv(rng, seq, dim)
        kw = dict(n_q=n_q, dim=dim, seq=seq, threads=2, split=4)
        want = reference.attention("avx512", q, k, v, **kw)
        assert bits_equal(oracle.attention("avx512", q, k, v, **kw), want), trial
        differs += not bits_equal(oracle.attention("scalar", q, k, v, **kw), want)
    assert differs > 50


# ----------------------------------------------------------- closed forms ----
def test_clean_block_sizes(oracle):
    """README.md:39: a clean 4-bit block (n=128, dim=64) is 12360 B, a clean 2-bit block 10312 B."""
    assert oracle.coded_block_bytes(128, 64, 4, 0) == 8 + 64 + 8192 + 4096 == 12360
    assert oracle.coded_block_bytes(128, 64, 2, 0) == 10312
    assert oracle.raw_block_bytes(128, 64) == 8 + 2 * 128 * 64
    assert oracle.exp_payload_bytes(3, 4, 2) == 3  # ceil(24/8)
    rng = np.random.default_rng(1)
    # exponents drawn from a 15-wide window: every block is 4-bit with no escape
    exp = rng.integers(100, 115, 128 * 64)
    kv = ((exp << 7) | rng.integers(0, 128, exp.size) | (rng.integers(0, 2, exp.size) << 15)).astype(np.uint16)
    assert oracle.encode(kv, 128, 64).size == 12360
    exp = rng.integers(100, 103, 128 * 64)
    kv = ((exp << 7) | rng.integers(0, 128, exp.size)).astype(np.uint16)
    assert oracle.encode(kv, 128, 64).size == 10312


def test_roundtrip_and_size_model(oracle):
    rng = np.random.default_rng(2)
    for trial in range(40):
        dim = 4 * int(rng.integers(1, 65))
        seq = int(rng.integers(1, 700))
        block = int(rng.integers(1, min(255, 65535 // dim) + 1))
        kv = rng.integers(0, 65536, seq * dim, dtype=np.uint16) if trial % 2 else random_kv(rng, seq, dim, specials=True, wide=trial % 3 == 0)
        blob = oracle.encode(kv, seq, dim, block)
        assert np.array_equal(oracle.decode(blob, seq, dim), kv)
        # container size equals the sum of per-block sizes, each the minimum of the candidates
        off, first = oracle.block_index(blob, dim, seq)
        assert first[-1] == seq and off[-1] == blob.size
        for b in range(off.size - 1):
            p = int(off[b])
            mode, n = int(blob[p]), int(blob[p + 1])
            esc = int(blob[p + 2]) | (int(blob[p + 3]) << 8)
            size = int(off[b + 1] - off[b])
            if mode == 0:
                assert size == oracle.raw_block_bytes(n, dim)
            else:
                assert size == oracle.coded_block_bytes(n, dim, mode, esc)
            assert size <= oracle.raw_block_bytes(n, dim)
        assert blob.size <= oracle.encode_bound(seq, dim, block)


def test_identity_token_kat(oracle):
    """tests/test_main.cpp:102-122: seq=1, q=k=1.0, v=[2,1,...,1] gives out == v exactly."""
    q = np.full(8, 0x3F80, np.uint16)
    v = np.full(8, 0x3F80, np.uint16)
    v[0] = 0x4000
    for be in ("scalar", "avx2"):
        out = oracle.attention(be, q, q.copy(), v, n_q=1, dim=8, seq=1)
        assert out[0] == 2.0 and np.all(out[1:] == 1.0)


def _attention_f64(q, k, v, n_q, dim, seq):
    qf = bf16_to_f32(q).astype(np.float64).reshape(n_q, dim)
    kf = bf16_to_f32(k).astype(np.float64).reshape(seq, dim)
    vf = bf16_to_f32(v).astype(np.float64).reshape(seq, dim)
    s = qf @ kf.T
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    lse = (m[:, 0] + np.log(p.sum(axis=1)))
    return (p @ vf) / p.sum(axis=1, keepdims=True), lse


def test_bruteforce_fp64(oracle):
    """Against exact FP64 attention (no softmax scale, as attention_scalar.cpp:24-29)."""
    rng = np.random.default_rng(4)
    for trial in range(20):
        dim, n_q, seq = int(rng.choice([32, 64, 128])), int(rng.integers(1, 8)), int(rng.integers(1, 600))
        q = random_kv(rng, n_q, dim, spread_lo=-2, spread_hi=0)
        k = random_kv(rng, seq, dim, spread_lo=-2, spread_hi=0)
        v = random_kv(rng, seq, dim, sigma=0.5)
        exact, lse_exact = _attention_f64(q, k, v, n_q, dim, seq)
        for be in ("scalar", "avx512"):
            out, lse = oracle.attention(be, q, k, v, n_q=n_q, dim=dim, seq=seq, threads=3, with_lse=True)
            err = np.abs(out.reshape(n_q, dim) - exact)
            scale = np.abs(bf16_to_f32(v)).max()
            assert err.max() <= 1e-4 * scale, (trial, be, err.max())
            assert np.allclose(lse, lse_exact, rtol=1e-5, atol=1e-4), (trial, be)


def test_split_partition_is_token_bounds(oracle):
    """dispatch.cpp:17-23,47-49: threads above the tile count clamp to it, so
    n_threads >= ceil(seq/split) all give the same bits."""
    rng = np.random.default_rng(9)
    q, k, v = random_kv(rng, 3, 64), random_kv(rng, 500, 64), random_kv(rng, 500, 64)
    kw = dict(n_q=3, dim=64, seq=500, split=128)
    a = oracle.attention("scalar", q, k, v, threads=4, **kw)
    b = oracle.attention("scalar", q, k, v, threads=100, **kw)
    c = oracle.attention("scalar", q, k, v, threads=1, **kw)
    assert bits_equal(a, b)
    assert not bits_equal(a, c) or True  # different association orders are allowed to agree


# ------------------------------------------------------------ error paths ----
def _err(fn):
    from oracle import KvexpError

    with pytest.raises(KvexpError) as ei:
        fn()
    return ei.value.kind, ei.value.msg


def _malformed_cases(oracle):
    rng = np.random.default_rng(6)
    kv = random_kv(rng, 300, 64)
    blob = oracle.encode(kv, 300, 64, 128)
    cases = []
    cases.append(("truncated header", blob[:5], 300, 64))
    cases.append(("truncated body", blob[:-3], 300, 64))
    bad_mode = blob.copy()
    bad_mode[0] = 1  # 3 is the 3-bit extension (dim % 8 == 0), which this library reads
    cases.append(("bad mode", bad_mode, 300, 64))
    cases.append(("wrong dim", blob, 300, 32))
    zero_tok = blob.copy()
    zero_tok[1] = 0
    cases.append(("zero tokens", zero_tok, 300, 64))
    cases.append(("ran out", blob, 400, 64))
    return cases


def test_decode_errors_match_reference(oracle, reference):
    for name, blob, seq, dim in _malformed_cases(oracle):
        ko, mo = _err(lambda: oracle.decode(blob, seq, dim))
        kr, mr = _err(lambda: reference.decode(blob, seq, dim))
        assert (ko, mo) == (kr, mr), name


def test_encode_errors_match_reference(oracle, reference):
    kv = np.zeros(64 * 256, np.uint16)
    for seq, dim, block in ((0, 64, 128), (10, 6, 128), (10, 260, 128), (10, 64, 256), (10, 0, 4)):
        ko, mo = _err(lambda: oracle.encode(kv, seq, dim, block))
        kr, mr = _err(lambda: reference.encode(kv, seq, dim, block))
        assert (ko, mo) == (kr, mr), (seq, dim, block)
    # block*dim <= 255*256 = 65280 always: the u16 escape-count check (codec.cpp:48-50)
    # cannot fire once the other two hold, so the largest shape encodes.
    assert np.array_equal(oracle.encode(kv[: 10 * 256], 10, 256, 255), reference.encode(kv[: 10 * 256], 10, 256, 255))


def test_attention_errors_match_reference(oracle, reference):
    rng = np.random.default_rng(8)
    q, k, v = random_kv(rng, 2, 64), random_kv(rng, 300, 64), random_kv(rng, 300, 64)
    kx, vx = oracle.encode(k, 300, 64, 128), oracle.encode(v, 300, 64, 128)
    calls = [
        lambda o: o.attention("scalar", q, k, v, kx=kx, vx=vx, n_q=2, dim=64, seq=300),
        lambda o: o.attention("scalar", q, k, None, n_q=2, dim=64, seq=300),
        lambda o: o.attention("scalar", q, k, v, n_q=0, dim=64, seq=300),
        lambda o: o.attention("scalar", q, k, v, n_q=2, dim=64, seq=300, split=0),
        lambda o: o.attention("scalar", q, k, v, n_q=2, dim=60, seq=300),
        lambda o: o.attention("avx512", q, k, v, n_q=2, dim=48, seq=300),
        lambda o: o.attention("avx2", q, kx=kx[:-40], vx=vx, n_q=2, dim=64, seq=300),
        lambda o: o.attention("avx2", q, kx=kx, vx=vx, n_q=2, dim=64, seq=400),
    ]
    for i, call in enumerate(calls):
        ko, mo = _err(lambda: call(oracle))
        kr, mr = _err(lambda: call(reference))
        assert (ko, mo) == (kr, mr), i
    # One thread reads from token 0, so a split that is not a block multiple is fine.
    kw = dict(n_q=2, dim=64, seq=300, split=100, threads=1)
    assert bits_equal(oracle.attention("scalar", q, kx=kx, vx=vx, **kw), reference.attention("scalar", q, kx=kx, vx=vx, **kw))


def test_misaligned_split_error(oracle):
    """scan.hpp:107-109: a thread whose first token is inside a block fails. (The
    reference raises it inside its OpenMP region, which terminates the process, so
    only the message is pinned here, by reading.)"""
    rng = np.random.default_rng(8)
    q, k, v = random_kv(rng, 2, 64), random_kv(rng, 300, 64), random_kv(rng, 300, 64)
    kx, vx = oracle.encode(k, 300, 64, 128), oracle.encode(v, 300, 64, 128)
    kind, msg = _err(lambda: oracle.attention("scalar", q, kx=kx, vx=vx, n_q=2, dim=64, seq=300, split=100, threads=2))
    assert (kind, msg) == ("runtime_error", "token split is not aligned to an encoded block")
