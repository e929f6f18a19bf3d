"""GPU fused decode attention (kvexp_hip_attention_run and the Backend::Hip host
entry) against the reference.

Parity, as stated for this path:
  (2) XKV and raw GPU results are bit-identical (same kernel order).
  (3) FP32 outputs match the reference scalar/AVX2 path (KVEXP_HIP_ORDER_SCALAR)
      and AVX-512 path (KVEXP_HIP_ORDER_DPBF16) within max relative error
      1e-5 per element. The kernels repeat the reference's operations one for
      one, so for the same split these tests assert bit equality, which
      implies the 1e-5 bound (asserted separately as well).
Expected values come from the reference's golden outputs (tests/golden) and
from the oracle, which is pinned to the compiled reference.
"""
import numpy as np
import pytest

from conftest import bits_equal, say, to_dev
from kvdata import bf16_from_f32, random_kv

pytestmark = pytest.mark.gpu

ORDER = {"scalar": 0, "avx2": 0, "avx512": 1}
REL_TOL = 1e-5


def max_rel_err(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    both_nan = np.isnan(got) & np.isnan(want)
    same_inf = np.isinf(got) & np.isinf(want) & (np.sign(got) == np.sign(want))
    ok = both_nan | same_inf
    d = np.abs(got - want)
    denom = np.maximum(np.abs(want), np.finfo(np.float32).tiny)
    rel = np.where(ok, 0.0, d / denom)
    rel = np.where(np.isnan(rel), np.inf, rel)
    return float(rel.max()) if rel.size else 0.0


def run_gpu(ctx, order, q, heads_np, n_q, dim, split, xkv, with_lse=False):
    """heads_np: list of dicts (k, v uint16, seq, splits); returns out (and lse)."""
    import torch

    block = split
    heads = []
    for h in heads_np:
        if xkv:
            kx = ctx.encode(to_dev(h["k"], torch.int16), h["seq"], dim, h.get("block", block))
            vx = ctx.encode(to_dev(h["v"], torch.int16), h["seq"], dim, h.get("block", block))
            heads.append(dict(kx=kx, vx=vx, seq=h["seq"], splits=h["splits"]))
        else:
            heads.append(dict(k=to_dev(h["k"], torch.int16), v=to_dev(h["v"], torch.int16), seq=h["seq"],
                              splits=h["splits"]))
    plan = ctx.plan(heads, n_q, dim, split, order)
    dq = to_dev(q, torch.int16)
    lse = torch.empty(len(heads) * n_q, dtype=torch.float32, device="cuda:0") if with_lse else None
    out = plan.run(dq, lse=lse, check_errors=True)
    res = out.cpu().numpy()
    plan.close()
    return (res, lse.cpu().numpy()) if with_lse else res


def test_golden_outputs(ctx, golden):
    """Every reference golden output (scalar, AVX2, AVX-512; thread counts as
    splits), from raw and from XKV inputs."""
    z, man = golden
    for c in man["attn"]:
        n = c["name"]
        q, k, v = z[f"attn/{n}/q"], z[f"attn/{n}/k"], z[f"attn/{n}/v"]
        for be in c["backends"]:
            for th in c["threads"]:
                say("golden attention", n, be, th)
                want = z[f"attn/{n}/{be}/t{th}"]
                heads = [dict(k=k, v=v, seq=c["seq"], splits=th)]
                for xkv in (False, True):
                    got = run_gpu(ctx, ORDER[be], q, heads, c["n_q"], c["dim"], c["block"], xkv)
                    assert bits_equal(got, want), (n, be, th, xkv)
                    assert max_rel_err(got, want) <= REL_TOL


def _case(rng, trial):
    dim = int(rng.choice([8, 16, 32, 64, 96, 128, 192, 256]))
    n_q = int(rng.choice([1, 2, 4, 7, 8, 11, 16]))
    seq = int(rng.integers(1, 1400))
    blocks = [b for b in (16, 64, 100, 128, 255) if b * dim <= 65535]
    block = int(rng.choice(blocks))
    kind = trial % 4
    if kind == 0:
        k = random_kv(rng, seq, dim, spread_lo=-6, spread_hi=4, outliers=min(2, dim))
    elif kind == 1:
        x = rng.uniform(1.0, 7.9, seq * dim) * np.where(rng.random(seq * dim) < .5, -1, 1)
        k = bf16_from_f32(x.astype(np.float32) * 0.25)
    elif kind == 2:
        k = rng.integers(0, 65536, seq * dim, dtype=np.uint16)
        k[(k & 0x7F80) == 0x7F80] &= 0x3FFF
        k = bf16_from_f32(np.clip(np.nan_to_num((k.astype(np.uint32) << 16).view(np.float32)), -8, 8))
    else:
        k = random_kv(rng, seq, dim, specials=True, wide=True)
    v = random_kv(rng, seq, dim, sigma=0.5, specials=trial % 5 == 0)
    q = random_kv(rng, n_q, dim, spread_lo=-1, spread_hi=1)
    splits = int(rng.integers(1, 9))
    return dim, n_q, seq, block, q, k, v, splits


def test_random_against_oracle(ctx, oracle):
    rng = np.random.default_rng(2024)
    for trial in range(48):
        dim, n_q, seq, block, q, k, v, splits = _case(rng, trial)
        for be in ("scalar", "avx512"):
            if be == "avx512" and dim % 32:
                continue
            say("random attention", trial, be, dict(dim=dim, n_q=n_q, seq=seq, block=block, splits=splits))
            want = oracle.attention(be, q, k, v, n_q=n_q, dim=dim, seq=seq, threads=splits, split=block)
            heads = [dict(k=k, v=v, seq=seq, splits=splits)]
            raw = run_gpu(ctx, ORDER[be], q, heads, n_q, dim, block, False)
            xkv = run_gpu(ctx, ORDER[be], q, heads, n_q, dim, block, True)
            assert bits_equal(raw, xkv), (trial, be)
            assert bits_equal(raw, want), (trial, be, max_rel_err(raw, want))


def test_many_heads_variable_length(ctx, oracle):
    """A batched plan over heads of different lengths and split counts (the
    shape of BASELINE config 3, shortened), with LSE."""
    rng = np.random.default_rng(77)
    dim, n_q, block = 64, 7, 128
    heads = []
    for h in range(20):
        seq = int(round(np.exp(rng.uniform(np.log(40), np.log(3000)))))
        heads.append(dict(k=random_kv(rng, seq, dim, spread_lo=-6, spread_hi=4, outliers=2),
                          v=random_kv(rng, seq, dim, sigma=0.5), seq=seq, splits=int(rng.integers(1, 12))))
    q = random_kv(rng, len(heads) * n_q, dim)
    say("variable-length plan", len(heads))
    want, lse_want = oracle.attention_heads("scalar", q, [dict(k=h["k"], v=h["v"], seq=h["seq"], threads=h["splits"])
                                                          for h in heads], n_q=n_q, dim=dim, split=block,
                                            with_lse=True)
    raw, lse_raw = run_gpu(ctx, 0, q, heads, n_q, dim, block, False, with_lse=True)
    xkv, lse_x = run_gpu(ctx, 0, q, heads, n_q, dim, block, True, with_lse=True)
    assert bits_equal(raw, xkv) and bits_equal(lse_raw, lse_x)
    assert bits_equal(raw, want)
    # LSE = m + log(l): no reference output; device log vs glibc logf within 2 ulp-ish
    assert np.allclose(lse_raw, lse_want, rtol=1e-6, atol=1e-6)


def test_wave_launch_shapes(ctx, oracle):
    """Plans of at most as many split waves as the GPU has CUs (one wave per
    workgroup), of up to twice as many (two) and of more (the kernel's four
    at head_dim 64): the same bits as the oracle in each."""
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rng = np.random.default_rng(91)
    dim, n_q, block, seq, splits = 64, 7, 128, 512, 4
    for n_items in (cus // 2, cus + 4 * 8, 2 * cus + 4 * 8):
        n_heads = n_items // splits
        heads = [dict(k=random_kv(rng, seq, dim, spread_lo=-6, spread_hi=4, outliers=2),
                      v=random_kv(rng, seq, dim, sigma=0.5), seq=seq, splits=splits) for _ in range(n_heads)]
        q = random_kv(rng, n_heads * n_q, dim)
        say("launch shape", dict(items=n_heads * splits, cus=cus))
        want = oracle.attention_heads("scalar", q, [dict(k=h["k"], v=h["v"], seq=seq, threads=splits) for h in heads],
                                      n_q=n_q, dim=dim, split=block)
        raw = run_gpu(ctx, 0, q, heads, n_q, dim, block, False)
        xkv = run_gpu(ctx, 0, q, heads, n_q, dim, block, True)
        assert bits_equal(raw, xkv)
        assert bits_equal(xkv, want)


def _escape_heavy_kv(rng, seq, dim, frac, narrow=False):
    """K with a fraction `frac` of elements pushed 2^8..2^14 away from their
    channel's exponent window, so that coded blocks carry many escapes
    (`narrow`: values within three binades, so blocks pick 2-bit codes)."""
    if narrow:
        x = (rng.uniform(1.0, 7.9, (seq, dim)) * rng.choice([-0.25, 0.25], (seq, dim))).astype(np.float32)
        k = bf16_from_f32(x.reshape(-1))
    else:
        k = random_kv(rng, seq, dim, spread_lo=-3, spread_hi=3)
    x = (k.astype(np.uint32) << 16).view(np.float32).reshape(seq, dim).copy()
    hit = rng.random((seq, dim)) < frac
    x[hit] *= np.exp2(rng.integers(8, 15, size=int(hit.sum())) * rng.choice([-1, 1], size=int(hit.sum())))
    return bf16_from_f32(x.reshape(-1))


def _max_block_escapes(oracle, blob, dim, seq):
    offs, first = oracle.block_index(blob, dim, seq)
    hdr = np.asarray(blob)[np.asarray(offs[:-1])[:, None] + np.arange(4)[None, :]].astype(np.int64)
    coded = hdr[:, 0] != 0
    esc = hdr[:, 2] | (hdr[:, 3] << 8)
    return int(esc[coded].max()) if coded.any() else 0


@pytest.mark.parametrize("backend", ["scalar", "avx512"])
@pytest.mark.parametrize("dim", [64, 128, 256])
def test_wave_kernel_groups_and_escapes(ctx, oracle, dim, backend):
    """The one-wave kernel (head_dim 64, 128 and 256, both score orders) for every
    query-row count G it is instantiated for, on containers whose blocks
    carry from 0 to several hundred escapes (blocks with more than 64 read
    the escape index in windows), block sizes that do and do not split into
    64-token chunks, ragged lengths and several splits per head."""
    rng = np.random.default_rng(4242 + dim)
    seen_big = False
    cases = [(1, 128, 0.05, False), (2, 255, 0.02, False), (3, 100, 0.0, False), (7, 128, 0.3, False),
             (8, 64, 0.01, False), (5, 128, 0.002, True), (7, 255, 0.1, True), (11, 128, 0.05, False),
             (4, 128, 0.6, False), (6, 128, 0.0, True)]
    for trial, (n_q, block, frac, narrow) in enumerate(cases):
        heads = []
        for h in range(3):
            seq = int(rng.integers(1, 1500))
            k = _escape_heavy_kv(rng, seq, dim, frac, narrow)
            v = _escape_heavy_kv(rng, seq, dim, frac / 2, narrow)
            heads.append(dict(k=k, v=v, seq=seq, splits=int(rng.integers(1, 7)), block=block))
            if frac:
                seen_big |= _max_block_escapes(oracle, oracle.encode(k, seq, dim, block), dim, seq) > 64
        q = random_kv(rng, len(heads) * n_q, dim, spread_lo=-1, spread_hi=1)
        say("wave kernel", backend, dim, trial,
            dict(n_q=n_q, block=block, frac=frac, narrow=narrow, seqs=[h["seq"] for h in heads]))
        want = oracle.attention_heads(backend, q, [dict(k=h["k"], v=h["v"], seq=h["seq"], threads=h["splits"])
                                                   for h in heads], n_q=n_q, dim=dim, split=block)
        raw = run_gpu(ctx, ORDER[backend], q, heads, n_q, dim, block, False)
        xkv = run_gpu(ctx, ORDER[backend], q, heads, n_q, dim, block, True)
        assert bits_equal(raw, xkv), trial
        assert bits_equal(raw, want), (trial, max_rel_err(raw, want))
    assert seen_big


# Tokens (from a split's first token) whose scores set a new running maximum:
# for query rows 0-3 (UP) and rows 4-7 (DOWN). Every position of a quad of
# four tokens, two and four moves in one quad, a move in each group of 16
# tokens of the second chunk, the first chunk's last token.
MOVES_UP = [1, 2, 3, 4, 9, 10, 16, 17, 18, 19, 35, 63, 69, 85, 101, 117]
MOVES_DOWN = [0, 6, 7, 13, 22, 31, 47, 62, 100, 127]


@pytest.mark.parametrize("backend", ["scalar", "avx512"])
@pytest.mark.parametrize("dim", [64, 128, 256])
def test_wave_fold_chosen_moves(ctx, oracle, dim, backend):
    """Running maxima that move at chosen tokens of each split's first two
    chunks (MOVES_UP for query rows 0-3, MOVES_DOWN for rows 4-7: K rows of
    growing magnitude and one sign among small random ones, queries of one
    sign per row group), so that the fold's path for tokens that move a
    maximum (at head_dim 256 the loop over quads of four tokens) meets moves
    at every position of a quad, several in one quad and none in others;
    XKV == raw == oracle in both score orders."""
    rng = np.random.default_rng(9 + dim)
    n_q, block, seq, splits = 8, 128, 640, 2
    x = rng.standard_normal((seq, dim)).astype(np.float32) * np.float32(0.05)
    chosen = sorted([(t, 1.0) for t in MOVES_UP] + [(t, -1.0) for t in MOVES_DOWN])
    k_th = 0
    for s0 in (0, 256):  # the two splits' first tokens (5 blocks over 2 splits)
        for t, sign in chosen:
            x[s0 + t] = np.float32(sign * (1.0 + 0.05 * k_th))
            k_th += 1
    k = bf16_from_f32(x.reshape(-1))
    v = random_kv(rng, seq, dim)
    qf = np.abs(rng.standard_normal((n_q, dim)).astype(np.float32)) * np.float32(0.5) + np.float32(0.25)
    qf[4:] *= -1.0
    q = bf16_from_f32(qf.reshape(-1))
    heads = [dict(k=k, v=v, seq=seq, splits=splits, block=block)]
    say("wave fold, chosen moves", backend, dict(dim=dim, seq=seq, splits=splits))
    want = oracle.attention_heads(backend, q, [dict(k=k, v=v, seq=seq, threads=splits)], n_q=n_q, dim=dim,
                                  split=block)
    raw = run_gpu(ctx, ORDER[backend], q, heads, n_q, dim, block, False)
    xkv = run_gpu(ctx, ORDER[backend], q, heads, n_q, dim, block, True)
    assert not np.isnan(want).any()
    assert bits_equal(raw, xkv)
    assert bits_equal(raw, want), max_rel_err(raw, want)


def _mixed_block_kv(rng, seq, dim, block, kinds):
    """Tokens whose blocks cycle through `kinds`: "raw" (values spread over 60
    binades: the encoder stores the block raw), "coded" (4-bit codes, a few
    escapes) and "narrow" (2-bit codes)."""
    parts = []
    for b0 in range(0, seq, block):
        n = min(block, seq - b0)
        kind = kinds[(b0 // block) % len(kinds)]
        if kind == "raw":
            parts.append(random_kv(rng, n, dim, wide=True))
        else:
            parts.append(_escape_heavy_kv(rng, n, dim, 0.01, narrow=kind == "narrow"))
    return np.concatenate(parts)


def _block_modes(oracle, blob, dim, seq):
    offs, _ = oracle.block_index(blob, dim, seq)
    return set(int(m) for m in np.asarray(blob)[np.asarray(offs[:-1])])


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_wave_kernel_mixed_raw_and_coded_blocks(ctx, oracle, dim):
    """Raw, 4-bit and 2-bit blocks interleaved in K and, in another order, in
    V, so that a chunk ends where either tensor's block ends, raw chunks are
    cut at 48 rows, and block sizes of 100 and 255 tokens leave partial
    chunks; blocks start at every even byte offset of the container (the
    piece loads at head_dim 128 and 256 clamp to the last piece of a cut
    chunk). XKV equals raw and the oracle bit for bit."""
    rng = np.random.default_rng(707 + dim)
    for trial, (n_q, block) in enumerate([(4, 100), (7, 255), (1, 128), (8, 100)]):
        heads = []
        for h in range(3):
            seq = int(rng.integers(200, 1400))
            k = _mixed_block_kv(rng, seq, dim, block, ["raw", "coded", "narrow", "coded"])
            v = _mixed_block_kv(rng, seq, dim, block, ["coded", "raw", "raw", "narrow"])
            heads.append(dict(k=k, v=v, seq=seq, splits=int(rng.integers(1, 5)), block=block))
            if h == 0:
                modes = _block_modes(oracle, oracle.encode(k, seq, dim, block), dim, seq)
                assert {0, 4}.issubset(modes), modes
        q = random_kv(rng, len(heads) * n_q, dim, spread_lo=-1, spread_hi=1)
        say("mixed blocks", dim, trial, dict(n_q=n_q, block=block, seqs=[h["seq"] for h in heads]))
        want = oracle.attention_heads("scalar", q, [dict(k=h["k"], v=h["v"], seq=h["seq"], threads=h["splits"])
                                                    for h in heads], n_q=n_q, dim=dim, split=block)
        raw = run_gpu(ctx, ORDER["scalar"], q, heads, n_q, dim, block, False)
        xkv = run_gpu(ctx, ORDER["scalar"], q, heads, n_q, dim, block, True)
        assert bits_equal(raw, xkv), trial
        assert bits_equal(raw, want), (trial, max_rel_err(raw, want))


def _scaled_blocks(rng, x, block, shifts, special_blocks=0.3):
    """x [seq, dim] float32 with each block of `block` rows scaled by 2^s, s
    drawn from `shifts` per block; a fraction `special_blocks` of the blocks
    also gets a few zeros and BF16 denormals."""
    seq, dim = x.shape
    nb = (seq + block - 1) // block
    s = np.repeat(rng.choice(shifts, size=nb), block)[:seq]
    b = bf16_from_f32((x * np.exp2(s)[:, None]).astype(np.float32).reshape(-1)).reshape(seq, dim)
    pool = np.array([0x0000, 0x8000, 0x0001, 0x8003, 0x0050], np.uint16)
    for i in np.flatnonzero(rng.random(nb) < special_blocks):
        rows = b[i * block:(i + 1) * block].reshape(-1)
        idx = rng.choice(rows.size, max(1, rows.size // 1000), replace=False)
        rows[idx] = rng.choice(pool, idx.size)
        b[i * block:(i + 1) * block] = rows.reshape(-1, dim)
    return b.reshape(-1)


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_wave_dpbf16_flush_guard(ctx, oracle, dim):
    """AVX-512 BF16 order on the one-wave kernel where VDPBF16PS's flushes
    matter: K blocks scaled by 2^0 .. 2^-90 and query rows by 2^0 .. 2^-50,
    so that some chunks meet the exponent bound of the matrix-core path
    (E_k + E_q >= 142) and others take the flushing path, with products
    below 2^-126 (flushed to zero), denormal K and q elements (read as zero)
    and escapes among them; XKV and raw inputs, every G class."""
    rng = np.random.default_rng(777 + dim)
    block = 128
    for trial, n_q in enumerate([1, 4, 5, 7, 8]):
        heads = []
        for h in range(3):
            seq = int(rng.integers(1, 1200))
            kx = (random_kv(rng, seq, dim, spread_lo=-3, spread_hi=3).astype(np.uint32) << 16).view(np.float32)
            vx = (random_kv(rng, seq, dim, sigma=0.5).astype(np.uint32) << 16).view(np.float32)
            k = _scaled_blocks(rng, kx.reshape(seq, dim), block, [0, -40, -60, -75, -90])
            v = _scaled_blocks(rng, vx.reshape(seq, dim), block, [0, 0, -20])
            heads.append(dict(k=k, v=v, seq=seq, splits=int(rng.integers(1, 6)), block=block))
        qx = (random_kv(rng, len(heads) * n_q, dim, spread_lo=-1, spread_hi=1).astype(np.uint32) << 16)
        q = _scaled_blocks(rng, qx.view(np.float32).reshape(-1, dim), 1, [0, -30, -50])
        say("dpbf16 flush guard", dim, trial, dict(n_q=n_q, seqs=[h["seq"] for h in heads]))
        want = oracle.attention_heads("avx512", q, [dict(k=h["k"], v=h["v"], seq=h["seq"], threads=h["splits"])
                                                    for h in heads], n_q=n_q, dim=dim, split=block)
        raw = run_gpu(ctx, 1, q, heads, n_q, dim, block, False)
        xkv = run_gpu(ctx, 1, q, heads, n_q, dim, block, True)
        assert bits_equal(raw, xkv), trial
        assert bits_equal(raw, want), (trial, max_rel_err(raw, want))


def test_host_entry_backend_hip(ctx, oracle, golden):
    """kvexp_hip_attention_decode_host: the attention_decode argument list with
    host pointers (the Backend::Hip case of dispatch.cpp)."""
    z, man = golden
    c = next(c for c in man["attn"] if c["name"].startswith("qwen_like"))
    n = c["name"]
    q, k, v = z[f"attn/{n}/q"], z[f"attn/{n}/k"], z[f"attn/{n}/v"]
    kx = oracle.encode(k, c["seq"], c["dim"], c["block"])
    vx = oracle.encode(v, c["seq"], c["dim"], c["block"])
    for be in ("scalar", "avx512"):
        for th in c["threads"]:
            say("host entry", be, th)
            kw = dict(n_q=c["n_q"], dim=c["dim"], seq=c["seq"], threads=th, split=c["block"])
            want = z[f"attn/{n}/{be}/t{th}"]
            assert bits_equal(ctx.attention_decode_host(ORDER[be], q, k, v, **kw), want)
            assert bits_equal(ctx.attention_decode_host(ORDER[be], q, kx=kx, vx=vx, **kw), want)


def test_split_and_argument_errors(ctx, oracle):
    import kvexp_amd

    rng = np.random.default_rng(8)
    q, k, v = random_kv(rng, 2, 64), random_kv(rng, 300, 64), random_kv(rng, 300, 64)
    kx, vx = oracle.encode(k, 300, 64, 128), oracle.encode(v, 300, 64, 128)

    def err(fn):
        with pytest.raises(kvexp_amd.KvexpHipError) as ei:
            fn()
        return ei.value.kind, ei.value.msg

    H = ctx.attention_decode_host
    say("error paths")
    assert err(lambda: H(0, q, kx=kx, vx=vx, n_q=2, dim=64, seq=300, split=100, threads=2)) == (
        "runtime_error", "token split is not aligned to an encoded block")
    assert err(lambda: H(0, q, kx=kx, vx=vx, n_q=2, dim=64, seq=400)) == ("runtime_error", "xkv ran out of tokens")
    assert err(lambda: H(0, q, k, v, kx=kx, vx=vx, n_q=2, dim=64, seq=300)) == (
        "invalid_argument", "attention_decode: pass raw K and V or xkv K and V, not both")
    assert err(lambda: H(0, q, k, v, n_q=2, dim=60, seq=300)) == ("invalid_argument", "scalar attention: bad shape")
    assert err(lambda: H(1, q, k, v, n_q=2, dim=48, seq=300)) == (
        "invalid_argument", "avx512 attention: head_dim must be a multiple of 32")
    assert err(lambda: H(0, q, k, v, n_q=0, dim=64, seq=300)) == ("invalid_argument", "attention_decode: bad argument")
    assert err(lambda: H(0, q, kx=kx[:-40], vx=vx, n_q=2, dim=64, seq=300)) == (
        "runtime_error", "truncated coded xkv block")
    # one thread reads from token 0: any split works
    out = H(0, q, kx=kx, vx=vx, n_q=2, dim=64, seq=300, split=100, threads=1)
    assert bits_equal(out, oracle.attention("scalar", q, k, v, n_q=2, dim=64, seq=300, split=100, threads=1))


def test_plan_reused_with_new_queries(ctx, oracle):
    """One plan run several times with different queries (as a decode loop
    does): every run must read its own queries, never a previous run's copy."""
    import torch

    rng = np.random.default_rng(909)
    dim, n_q, block, seq = 64, 7, 128, 1500
    heads_np = [dict(k=random_kv(rng, seq, dim, spread_lo=-6, spread_hi=4, outliers=2),
                     v=random_kv(rng, seq, dim, sigma=0.5), seq=seq, splits=s) for s in (1, 5, 12)]
    for xkv in (False, True):
        hs = []
        for h in heads_np:
            if xkv:
                hs.append(dict(kx=ctx.encode(to_dev(h["k"], torch.int16), seq, dim, block),
                               vx=ctx.encode(to_dev(h["v"], torch.int16), seq, dim, block), seq=seq,
                               splits=h["splits"]))
            else:
                hs.append(dict(k=to_dev(h["k"], torch.int16), v=to_dev(h["v"], torch.int16), seq=seq,
                               splits=h["splits"]))
        plan = ctx.plan(hs, n_q, dim, block, 0)
        for run in range(4):
            q = random_kv(rng, len(heads_np) * n_q, dim)
            say("plan reuse", dict(xkv=xkv, run=run))
            got = plan.run(to_dev(q, torch.int16), check_errors=True).cpu().numpy()
            want = oracle.attention_heads("scalar", q, [dict(k=h["k"], v=h["v"], seq=seq, threads=h["splits"])
                                                        for h in heads_np], n_q=n_q, dim=dim, split=block)
            assert bits_equal(got, want), (xkv, run)
        plan.close()
