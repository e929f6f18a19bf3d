"""The 3-bit format extension on the GPU: the encoder (whole and by appends)
against the oracle's 3-bit encoder byte for byte, decode and the host index
walk of 3-bit containers, and attention over them (one-wave kernel at
head_dim 64 and 128, the general kernel at 256; both score orders): XKV
equal to raw and to the oracle, bit for bit."""
import numpy as np
import pytest

from conftest import bits_equal, say, to_dev
from kvdata import bf16_from_f32, random_kv
from test_gpu_attention import ORDER, _scaled_blocks, max_rel_err, run_gpu
from test_gpu_codec import _encode, _kinds

pytestmark = pytest.mark.gpu

M3 = 0x1C  # raw, 2-, 3- and 4-bit
MREF = 0x14


@pytest.fixture
def ctx3(ctx):
    ctx.set_encoder_modes(M3)
    try:
        yield ctx
    finally:
        ctx.set_encoder_modes(MREF)


def _kv3(rng, seq, dim, frac=0.0, sigma=1.0):
    """Values whose exponents mostly fit a 7-wide window per channel, with a
    fraction `frac` pushed 2^8..2^14 away (escapes)."""
    k = random_kv(rng, seq, dim, spread_lo=-1, spread_hi=1, sigma=sigma)
    if not frac:
        return k
    x = (k.astype(np.uint32) << 16).view(np.float32).reshape(seq, dim).copy()
    hit = rng.random((seq, dim)) < frac
    x[hit] *= np.exp2(rng.integers(8, 15, size=int(hit.sum())) * rng.choice([-1, 1], size=int(hit.sum())))
    return bf16_from_f32(x.reshape(-1))


def test_3bit_containers(ctx3, oracle):
    assert ctx3.encoder_modes == M3
    rng = np.random.default_rng(303)
    seen = np.zeros(5, np.int64)
    for trial in range(30):
        dim = 8 * int(rng.integers(1, 33)) if trial % 5 else 4 * int(rng.integers(1, 65))
        block = int(rng.integers(1, min(255, 65535 // dim) + 1))
        seq = int(rng.integers(1, 1500))
        kind = trial % 6
        kv = _kinds(rng, seq, dim, kind) if kind < 4 else _kv3(rng, seq, dim, 0.01 * (kind - 4))
        say("3-bit codec", trial, dict(dim=dim, block=block, seq=seq, kind=kind))
        enc, blob = _encode(ctx3, kv, seq, dim, block)
        want = oracle.encode(kv, seq, dim, block, modes=M3)
        assert np.array_equal(blob, want), trial
        off, first = oracle.block_index(want, dim, seq)
        assert np.array_equal(enc.offsets.cpu().numpy(), off), trial
        assert np.array_equal(enc.first.cpu().numpy(), first), trial
        assert np.array_equal(ctx3.decode(enc).cpu().numpy().view(np.uint16), kv), trial
        up = ctx3.upload(want, dim, seq, block)  # host index walk
        assert np.array_equal(ctx3.decode(up).cpu().numpy().view(np.uint16), kv), trial
        seen += oracle.mode_counts(want, dim)
    assert seen[3] > 0 and seen[2] > 0 and seen[4] > 0 and seen[0] > 0, seen


def test_3bit_setting_is_per_context(ctx3, oracle):
    """The default setting gives encode_bf16's containers again."""
    import torch

    rng = np.random.default_rng(304)
    kv = _kv3(rng, 500, 64)
    _, b3 = _encode(ctx3, kv, 500, 64, 128)
    assert oracle.mode_counts(b3, 64)[3] > 0
    ctx3.set_encoder_modes(MREF)
    _, bref = _encode(ctx3, kv, 500, 64, 128)
    assert np.array_equal(bref, oracle.encode(kv, 500, 64, 128))
    from kvexp_amd import KvexpHipError

    with pytest.raises(KvexpHipError):
        ctx3.set_encoder_modes(0x21)
    torch.cuda.synchronize()


@pytest.mark.parametrize("backend", ["scalar", "avx512"])
@pytest.mark.parametrize("dim", [64, 128, 256])
def test_3bit_attention(ctx3, oracle, dim, backend):
    rng = np.random.default_rng(5150 + dim)
    n3 = 0
    cases = [(1, 128, 0.0), (4, 128, 0.05), (7, 255, 0.3), (8, 64, 0.01), (5, 100, 0.002), (11, 128, 0.02)]
    for trial, (n_q, block, frac) in enumerate(cases):
        heads = []
        for h in range(3):
            seq = int(rng.integers(1, 1300))
            k = _kv3(rng, seq, dim, frac)
            v = _kv3(rng, seq, dim, frac / 2, sigma=0.5)
            heads.append(dict(k=k, v=v, seq=seq, splits=int(rng.integers(1, 7)), block=block))
            n3 += oracle.mode_counts(oracle.encode(k, seq, dim, block, modes=M3), dim)[3]
        q = random_kv(rng, len(heads) * n_q, dim, spread_lo=-1, spread_hi=1)
        say("3-bit attention", backend, dim, trial, dict(n_q=n_q, block=block, frac=frac,
                                                         seqs=[h["seq"] for h in heads]))
        want = oracle.attention_heads(backend, q, [dict(k=h["k"], v=h["v"], seq=h["seq"], threads=h["splits"])
                                                   for h in heads], n_q=n_q, dim=dim, split=block)
        raw = run_gpu(ctx3, ORDER[backend], q, heads, n_q, dim, block, False)
        xkv = run_gpu(ctx3, ORDER[backend], q, heads, n_q, dim, block, True)
        assert bits_equal(raw, xkv), trial
        assert bits_equal(raw, want), (trial, max_rel_err(raw, want))
    assert n3 > 0


@pytest.mark.parametrize("dim", [64, 128])
def test_3bit_dpbf16_flush_guard(ctx3, oracle, dim):
    """AVX-512 order over 3-bit blocks scaled by 2^0 .. 2^-90 (chunks on both
    sides of the matrix-core path's exponent bound)."""
    rng = np.random.default_rng(8080 + dim)
    block = 128
    for trial, n_q in enumerate([1, 5, 7, 8]):
        heads = []
        for h in range(3):
            seq = int(rng.integers(1, 1200))
            kx = (_kv3(rng, seq, dim, 0.01).astype(np.uint32) << 16).view(np.float32)
            vx = (_kv3(rng, seq, dim, sigma=0.5).astype(np.uint32) << 16).view(np.float32)
            k = _scaled_blocks(rng, kx.reshape(seq, dim), block, [0, -40, -60, -75, -90])
            v = _scaled_blocks(rng, vx.reshape(seq, dim), block, [0, 0, -20])
            heads.append(dict(k=k, v=v, seq=seq, splits=int(rng.integers(1, 6)), block=block))
        qx = (random_kv(rng, len(heads) * n_q, dim, spread_lo=-1, spread_hi=1).astype(np.uint32) << 16)
        q = _scaled_blocks(rng, qx.view(np.float32).reshape(-1, dim), 1, [0, -30, -50])
        say("3-bit dpbf16 flush guard", dim, trial, dict(n_q=n_q, seqs=[h["seq"] for h in heads]))
        want = oracle.attention_heads("avx512", q, [dict(k=h["k"], v=h["v"], seq=h["seq"], threads=h["splits"])
                                                    for h in heads], n_q=n_q, dim=dim, split=block)
        raw = run_gpu(ctx3, 1, q, heads, n_q, dim, block, False)
        xkv = run_gpu(ctx3, 1, q, heads, n_q, dim, block, True)
        assert bits_equal(raw, xkv), trial
        assert bits_equal(raw, want), (trial, max_rel_err(raw, want))


@pytest.mark.parametrize("dim,block", [(64, 128), (128, 128), (256, 255), (8, 3)])
def test_3bit_append(ctx3, oracle, dim, block):
    """A container grown by appends with the 3-bit extension allowed equals
    the oracle's 3-bit encode of the tokens so far, bytes and index."""
    import torch

    rng = np.random.default_rng(dim * 7 + block)
    total = 3 * block + 29
    kv = np.concatenate([_kv3(rng, total // 2, dim, 0.01), _kinds(rng, total - total // 2, dim, 3)])
    cache = ctx3.cache(dim, total, block)
    sizes = [1, 2, block - 1, block, 1, 2 * block + 3, 5]
    pos = step = 0
    while pos < total:
        n = min(sizes[step % len(sizes)], total - pos)
        step += 1
        cache.append(to_dev(kv[pos * dim:(pos + n) * dim], torch.int16), n)
        pos += n
        want = oracle.encode(kv[: pos * dim], pos, dim, block, modes=M3)
        enc = cache.view()
        say("3-bit append", dim, block, step, dict(n=n, tokens=pos, bytes=enc.nbytes))
        assert enc.nbytes == want.size
        assert np.array_equal(enc.blob[: enc.nbytes].cpu().numpy(), want), (step, pos)
        off, first = oracle.block_index(want, dim, pos)
        assert np.array_equal(enc.offsets.cpu().numpy(), off), (step, pos)
    assert oracle.mode_counts(want, dim)[3] > 0
