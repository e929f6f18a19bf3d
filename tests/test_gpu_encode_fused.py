"""The one-pass encoder (encode_fused_kernel; head_dim % 8 == 0, at most
16,384 elements per block, 16-byte aligned sources) against the oracle's
encode_bf16 (codec.cpp:39-164) and against the three-launch encoder, which
runs for the same tokens from a source that is not 16-byte aligned: shapes
at the edges of its register tile (1, 2, 4 and 8 chunks of 16 bytes per
thread), partial last blocks, blocks of one token, raw-only data, the 3-bit
modes; containers of thousands of blocks and batched appends from empty and
from partial trailing blocks (its look-back over many earlier blocks, 64 at
a time, and the containers' own offsets); and the wrap of its look-back
epoch after 65,535 launches on one context."""
import ctypes as C

import numpy as np
import pytest

from conftest import say, to_dev
from kvdata import random_kv

pytestmark = pytest.mark.gpu

SHAPES = [  # (dim, block, seq): chunk rows per thread 1, 2, 4, 8 and odd shapes
    (8, 1, 37), (8, 255, 1000), (16, 128, 777), (24, 100, 5000), (40, 200, 999), (64, 128, 32773),
    (64, 255, 3000), (80, 128, 4000), (96, 170, 3001), (128, 128, 20000), (128, 64, 100), (256, 64, 5000),
    (136, 120, 1234), (256, 1, 9),
]


def _data(rng, seq, dim, kind):
    if kind == "wide":
        return random_kv(rng, seq, dim, outliers=min(2, dim), specials=True, wide=True)
    return random_kv(rng, seq, dim, outliers=min(2, dim), specials=kind == "specials")


def _encode_unaligned(ctx, kv, seq, dim, block):
    """The same tokens from a source 2 bytes past a 16-byte boundary: the
    three-launch encoder."""
    import torch

    buf = torch.zeros(kv.size + 8, dtype=torch.int16, device="cuda:0")
    buf[1:1 + kv.size] = to_dev(kv, torch.int16)
    src = buf[1:1 + kv.size]
    assert src.data_ptr() % 16 != 0
    enc = ctx.encode(src, seq, dim, block)
    return enc.blob[: enc.nbytes].cpu().numpy(), enc.offsets.cpu().numpy(), enc.first.cpu().numpy()


@pytest.mark.parametrize("modes", ["reference", "3bit"])
def test_fused_encode_shapes(ctx, oracle, modes):
    import torch

    import kvexp_amd

    rng = np.random.default_rng(31)
    extra = kvexp_amd.MODE_3BIT if modes == "3bit" else 0
    ctx.set_encoder_modes(kvexp_amd.MODES_REFERENCE | extra)
    try:
        for i, (dim, block, seq) in enumerate(SHAPES):
            kind = ("outliers", "specials", "wide")[i % 3]
            say("fused encode", modes, dict(dim=dim, block=block, seq=seq, kind=kind))
            kv = _data(rng, seq, dim, kind)
            dev = to_dev(kv, torch.int16)
            assert dev.data_ptr() % 16 == 0
            enc = ctx.encode(dev, seq, dim, block)
            blob = enc.blob[: enc.nbytes].cpu().numpy()
            want = oracle.encode(kv, seq, dim, block, modes=0x14 | (0x08 if extra else 0))
            assert blob.size == want.size, (dim, block, seq)
            assert np.array_equal(blob, want), (dim, block, seq)
            off, first = oracle.block_index(want, dim, seq)
            assert np.array_equal(enc.offsets.cpu().numpy(), off), (dim, block, seq)
            assert np.array_equal(enc.first.cpu().numpy(), first), (dim, block, seq)
            ublob, uoff, ufirst = _encode_unaligned(ctx, kv, seq, dim, block)
            assert np.array_equal(ublob, want) and np.array_equal(uoff, off) and np.array_equal(ufirst, first)
            dec = ctx.decode(enc).cpu().numpy().view(np.uint16)
            assert np.array_equal(dec, kv), (dim, block, seq)
    finally:
        ctx.set_encoder_modes(kvexp_amd.MODES_REFERENCE)


def test_fused_append_prefill(ctx, oracle):
    """One kvexp_hip_append_batch call over 10 containers (empty, partial
    trailing blocks, block-aligned) adding thousands of tokens each: every
    container equals encode_bf16 of its tokens."""
    import torch

    rng = np.random.default_rng(8)
    dim, block = 64, 128
    start = [0, 1, 127, 128, 129, 0, 1000, 5, 256, 0]
    add = [9000, 8000, 1, 7000, 129, 0, 12345, 300, 3, 6400]
    data = [_data(rng, s + a + 1, dim, ("outliers", "specials", "wide")[i % 3])
            for i, (s, a) in enumerate(zip(start, add))]
    caches = [ctx.cache(dim, s + a + 1, block) for s, a in zip(start, add)]
    for c, d, s in zip(caches, data, start):
        if s:
            c.append(to_dev(d[: s * dim], torch.int16), s)
    toks = [to_dev(d[s * dim:(s + a) * dim] if a else d[:dim], torch.int16) for d, s, a in zip(data, start, add)]
    say("fused append prefill", dict(containers=len(caches), tokens=sum(add)))
    ctx.append_batch(caches, toks, add, check_errors=True)
    for i, (c, d, s, a) in enumerate(zip(caches, data, start, add)):
        n_tok = s + a
        if n_tok == 0:
            assert c.size() == 0
            continue
        want = oracle.encode(d[: n_tok * dim], n_tok, dim, block)
        n = c.size()
        assert n == want.size, i
        assert np.array_equal(c.blob[:n].cpu().numpy(), want), i
        off, first = oracle.block_index(want, dim, n_tok)
        assert np.array_equal(c.view().offsets.cpu().numpy(), off), i
        assert np.array_equal(c.view().first.cpu().numpy(), first), i


def test_fused_looping_workgroups(ctx, oracle):
    """Jobs with more blocks than workgroups stay resident (a workgroup then
    encodes several blocks, by ticket, and loads the next block's tokens
    while it finishes the current one): single encodes at 1, 4 and 8 chunk
    rows per thread with 1,094 to 1,875 blocks (MI355X keeps at most 1,024
    workgroups of the head_dim 128 and 256 shapes resident, 1,536 of head_dim
    64), and one batched append from empty of three head_dim-128 containers
    of 391 blocks each."""
    import torch

    rng = np.random.default_rng(12)
    for dim, block, seq in [(128, 128, 140000), (256, 64, 70010), (64, 128, 240000), (8, 255, 600000)]:
        kind = "wide" if dim == 256 else "outliers"
        say("fused encode, looping workgroups", dict(dim=dim, block=block, seq=seq, kind=kind))
        kv = _data(rng, seq, dim, kind)
        enc = ctx.encode(to_dev(kv, torch.int16), seq, dim, block)
        want = oracle.encode(kv, seq, dim, block)
        assert enc.nbytes == want.size, (dim, block, seq)
        assert np.array_equal(enc.blob[: enc.nbytes].cpu().numpy(), want), (dim, block, seq)
        off, first = oracle.block_index(want, dim, seq)
        assert np.array_equal(enc.offsets.cpu().numpy(), off), (dim, block, seq)
        assert np.array_equal(enc.first.cpu().numpy(), first), (dim, block, seq)

    dim, block, add = 128, 128, 50000
    data = [_data(rng, add, dim, kind) for kind in ("outliers", "specials", "wide")]
    caches = [ctx.cache(dim, add, block) for _ in data]
    say("fused append, looping workgroups", dict(containers=len(caches), dim=dim, tokens=add))
    ctx.append_batch(caches, [to_dev(d, torch.int16) for d in data], [add] * len(data), check_errors=True)
    for i, (c, d) in enumerate(zip(caches, data)):
        want = oracle.encode(d, add, dim, block)
        n = c.size()
        assert n == want.size, i
        assert np.array_equal(c.blob[:n].cpu().numpy(), want), i
        off, first = oracle.block_index(want, dim, add)
        assert np.array_equal(c.view().offsets.cpu().numpy(), off), i
        assert np.array_equal(c.view().first.cpu().numpy(), first), i


def test_fused_epoch_wrap(oracle):
    """A container of 313 blocks, then 65,534 one-block encodes, then another
    container of 313 blocks with other tokens on the same context: the last
    launch has the first one's epoch again (the epochs run 1..65535), so it
    is right only if the look-back words were cleared when the epoch wrapped."""
    import torch

    import kvexp_amd

    ctx = kvexp_amd.Context(0)
    rng = np.random.default_rng(4)
    dim, block, seq = 64, 128, 40000
    a = random_kv(rng, seq, dim, outliers=2)
    b = random_kv(rng, seq, dim, outliers=2, wide=True)
    say("fused epoch wrap: first container")
    enc_a = ctx.encode(to_dev(a, torch.int16), seq, dim, block)
    assert np.array_equal(enc_a.blob[: enc_a.nbytes].cpu().numpy(), oracle.encode(a, seq, dim, block))
    L = kvexp_amd.lib()
    one = to_dev(random_kv(rng, 1, 8), torch.int16)
    cap = kvexp_amd.encode_bound(1, 8, 1)
    out = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    offs = torch.empty(2, dtype=torch.int64, device="cuda:0")
    first = torch.empty(2, dtype=torch.int32, device="cuda:0")
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    say("fused epoch wrap: 65534 one-block encodes")
    for i in range(65534):
        rc = L.kvexp_hip_encode(ctx.h, C.c_void_p(one.data_ptr()), 1, 8, 1, C.c_void_p(out.data_ptr()), cap,
                                C.c_void_p(offs.data_ptr()), C.c_void_p(first.data_ptr()), None, stream)
        assert rc == 0
        if i % 8192 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    say("fused epoch wrap: second container")
    enc_b = ctx.encode(to_dev(b, torch.int16), seq, dim, block)
    want = oracle.encode(b, seq, dim, block)
    assert np.array_equal(enc_b.blob[: enc_b.nbytes].cpu().numpy(), want)
    off, fst = oracle.block_index(want, dim, seq)
    assert np.array_equal(enc_b.offsets.cpu().numpy(), off)
    assert np.array_equal(enc_b.first.cpu().numpy(), fst)
