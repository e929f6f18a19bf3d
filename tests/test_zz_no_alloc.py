"""kvexp_hip_encode_noalloc (the encoder entry point that allocates nothing:
its scratch is the library's static per-GPU device array) called through the
C ABI, checked byte for byte against kvexp_hip_encode on the same inputs:
the container, its block index and the status word, on calls in a row whose
later inputs are smaller (the scratch keeps the previous call's contents), on
one-pass calls after a three-launch call, on
the 3-bit encoder modes, and the oracle's encode_bf16 for the first call;
and captured once in a graph, replayed over inputs of different block sizes.
Inputs too large for the scratch are refused before any GPU work."""
import ctypes as C

import numpy as np
import pytest

from conftest import say, to_dev
from kvdata import random_kv

pytestmark = pytest.mark.gpu

CAPACITY = 6  # KVEXP_HIP_CAPACITY


def _noalloc(ctx, kv_dev, seq, dim, block, with_status):
    import torch

    import kvexp_amd

    L = kvexp_amd.lib()
    cap = kvexp_amd.encode_bound(seq, dim, block)
    nb = L.kvexp_hip_block_count(seq, block)
    dev = kv_dev.device
    # outputs filled with a pattern, so bytes left unwritten would show
    blob = torch.full((cap,), 0xA5, dtype=torch.uint8, device=dev)
    offs = torch.full((nb + 1,), -7, dtype=torch.int64, device=dev)
    first = torch.full((nb + 1,), -7, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev) if with_status else None
    stream = torch.cuda.current_stream()
    rc = L.kvexp_hip_encode_noalloc(ctx.h, C.c_void_p(kv_dev.data_ptr()), seq, dim, block,
                                    C.c_void_p(blob.data_ptr()), cap, C.c_void_p(offs.data_ptr()),
                                    C.c_void_p(first.data_ptr()),
                                    C.c_void_p(status.data_ptr()) if status is not None else None,
                                    C.c_void_p(stream.cuda_stream))
    kvexp_amd.check(rc)
    torch.cuda.synchronize()
    n = int(offs[nb].item())
    return (blob[:n].cpu().numpy(), offs.cpu().numpy(), first.cpu().numpy(),
            int(status.item()) if status is not None else 0)


def _encode(ctx, kv_dev, seq, dim, block):
    enc = ctx.encode(kv_dev, seq, dim, block)
    return enc.blob[: enc.nbytes].cpu().numpy(), enc.offsets.cpu().numpy(), enc.first.cpu().numpy()


@pytest.mark.parametrize("modes", ["reference", "3bit"])
def test_noalloc_encode_equals_encode(ctx, oracle, modes):
    import torch

    import kvexp_amd

    rng = np.random.default_rng(77)
    ctx.set_encoder_modes(kvexp_amd.MODES_REFERENCE | (kvexp_amd.MODE_3BIT if modes == "3bit" else 0))
    try:
        # larger first, then smaller: the second call runs on the first's leftovers;
        # the last call is one pass again after a three-launch call (head_dim 256,
        # 255-token blocks) wrote its metadata over the one-pass look-back words
        cases = [(20000, 64, 128, True), (1234, 64, 128, False), (3001, 128, 100, True), (5, 256, 255, False),
                 (700, 64, 128, True)]
        for i, (seq, dim, block, with_status) in enumerate(cases):
            say("encode_noalloc", modes, seq, dim, block)
            kv = random_kv(rng, seq, dim)
            kv_dev = to_dev(kv, torch.int16)
            blob, offs, first, st = _noalloc(ctx, kv_dev, seq, dim, block, with_status)
            want_blob, want_offs, want_first = _encode(ctx, kv_dev, seq, dim, block)
            assert st == 0
            assert np.array_equal(blob, want_blob), (seq, dim, block)
            assert np.array_equal(offs, want_offs), (seq, dim, block)
            assert np.array_equal(first, want_first), (seq, dim, block)
            if i == 0 and modes == "reference":
                assert np.array_equal(blob, oracle.encode(kv, seq, dim, block))
    finally:
        ctx.set_encoder_modes(kvexp_amd.MODES_REFERENCE)


def test_noalloc_refuses_inputs_beyond_its_scratch(ctx):
    import torch

    import kvexp_amd

    L = kvexp_amd.lib()
    tiny = torch.zeros(16, dtype=torch.uint8, device="cuda:0")
    # 6,000 blocks of head_dim 256 need about 4.7 MB of scratch: refused
    # during the argument checks, before any launch (the buffers are never read)
    seq, dim, block = 6000 * 128, 256, 128
    rc = L.kvexp_hip_encode_noalloc(ctx.h, C.c_void_p(tiny.data_ptr()), seq, dim, block,
                                    C.c_void_p(tiny.data_ptr()), kvexp_amd.encode_bound(seq, dim, block),
                                    C.c_void_p(tiny.data_ptr()), C.c_void_p(tiny.data_ptr()), None, None)
    assert rc == CAPACITY
    assert "scratch" in L.kvexp_hip_last_error().decode()
    # a null block index is refused too (the index is an output here)
    rc = L.kvexp_hip_encode_noalloc(ctx.h, C.c_void_p(tiny.data_ptr()), 4, 4, 128, C.c_void_p(tiny.data_ptr()),
                                    kvexp_amd.encode_bound(4, 4, 128), None, None, None, None)
    assert rc != 0


def test_noalloc_encode_graph_replays(ctx):
    """kvexp_hip_encode_noalloc captured once in a graph, replayed over inputs
    whose blocks differ in size (so a look-back entry left by an earlier replay
    would place blocks wrongly): every replay's container and index equal
    kvexp_hip_encode's on the same input, with eager encodes between replays."""
    import torch

    import kvexp_amd

    L = kvexp_amd.lib()
    seq, dim, block = 20000, 64, 128
    cap = kvexp_amd.encode_bound(seq, dim, block)
    nb = L.kvexp_hip_block_count(seq, block)
    rng = np.random.default_rng(91)
    # inputs with different block modes and escape counts: plain random data,
    # data with a wide exponent spread (raw and 2-bit blocks), data with zeros
    inputs = [random_kv(rng, seq, dim), random_kv(rng, seq, dim, wide=True), random_kv(rng, seq, dim)]
    inputs[2][::7] = 0
    kv_static = to_dev(inputs[0], torch.int16)
    blob = torch.full((cap,), 0xA5, dtype=torch.uint8, device="cuda:0")
    offs = torch.full((nb + 1,), -7, dtype=torch.int64, device="cuda:0")
    first = torch.full((nb + 1,), -7, dtype=torch.int32, device="cuda:0")
    status = torch.zeros(1, dtype=torch.int32, device="cuda:0")

    def call(stream):
        kvexp_amd.check(L.kvexp_hip_encode_noalloc(
            ctx.h, C.c_void_p(kv_static.data_ptr()), seq, dim, block, C.c_void_p(blob.data_ptr()), cap,
            C.c_void_p(offs.data_ptr()), C.c_void_p(first.data_ptr()), C.c_void_p(status.data_ptr()),
            C.c_void_p(stream.cuda_stream)))

    say("encode_noalloc graph: eager warm-up")
    call(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            call(torch.cuda.current_stream())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep, i in enumerate([1, 0, 2, 2, 1]):
        say("encode_noalloc graph: replay", rep, "input", i)
        kv_static.copy_(to_dev(inputs[i], torch.int16))
        blob.fill_(0xA5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        n = int(offs[nb].item())
        got = (blob[:n].cpu().numpy(), offs.cpu().numpy(), first.cpu().numpy())
        want_blob, want_offs, want_first = _encode(ctx, kv_static, seq, dim, block)
        assert int(status.item()) == 0
        assert np.array_equal(got[1], want_offs), (rep, i)
        assert np.array_equal(got[2], want_first), (rep, i)
        assert np.array_equal(got[0], want_blob), (rep, i)
