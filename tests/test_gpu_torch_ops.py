"""torch.ops.kvexp.decode_attention / decode_attention_raw on the GPU: bit-equal
to the oracle (the reference's attention_decode with n_threads = n_splits) in
both score orders, XKV equal to raw, plan reuse, torch.compile."""
import numpy as np
import pytest

from conftest import bits_equal, say, to_dev
from kvdata import random_kv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("order,backend", [(0, "scalar"), (1, "avx512")])
def test_decode_attention_ops(ctx, oracle, order, backend):
    import torch

    import kvexp_amd.torch_ops as ops

    rng = np.random.default_rng(31 + order)
    dim, n_q, block, splits = 64, 7, 128, 3
    seqs = [700, 700, 700]
    ks = [random_kv(rng, s, dim, spread_lo=-6, spread_hi=4, outliers=2) for s in seqs]
    vs = [random_kv(rng, s, dim, sigma=0.5) for s in seqs]
    q = random_kv(rng, len(seqs) * n_q, dim)
    want = oracle.attention_heads(backend, q, [dict(k=k, v=v, seq=s, threads=splits) for k, v, s in zip(ks, vs, seqs)],
                                  n_q=n_q, dim=dim, split=block)
    dq = to_dev(q, torch.int16).view(torch.bfloat16).view(len(seqs), n_q, dim)
    kx = [ctx.encode(to_dev(k, torch.int16), s, dim, block) for k, s in zip(ks, seqs)]
    vx = [ctx.encode(to_dev(v, torch.int16), s, dim, block) for v, s in zip(vs, seqs)]
    say("torch op xkv", backend)
    out = ops.decode_attention_containers(dq, kx, vx, seqs, splits, block, order)
    assert out.shape == (3, n_q, dim)
    assert bits_equal(out.cpu().numpy().reshape(-1), want)
    say("torch op raw", backend)
    kr = torch.stack([to_dev(k, torch.int16).view(torch.bfloat16).view(s, dim) for k, s in zip(ks, seqs)])
    vr = torch.stack([to_dev(v, torch.int16).view(torch.bfloat16).view(s, dim) for v, s in zip(vs, seqs)])
    raw = torch.ops.kvexp.decode_attention_raw(dq, kr, vr, splits, block, order, False)
    assert bits_equal(raw.cpu().numpy().reshape(-1), want)
    # plan reuse: the same containers twice, same bits
    a = ops.decode_attention_containers(dq, kx, vx, seqs, splits, block, order, reuse_plan=True)
    b = ops.decode_attention_containers(dq, kx, vx, seqs, splits, block, order, reuse_plan=True)
    assert bits_equal(a.cpu().numpy(), b.cpu().numpy()) and bits_equal(a.cpu().numpy().reshape(-1), want)
    ops.clear_plan_cache()


def test_decode_attention_compiled(ctx, oracle):
    """The op inside a torch.compile'd function (traced through its fake
    implementation) gives the eager bits."""
    import torch

    import kvexp_amd.torch_ops  # noqa: F401

    rng = np.random.default_rng(77)
    dim, n_q, seq, block = 64, 4, 300, 128
    k = to_dev(random_kv(rng, 2 * seq, dim), torch.int16).view(torch.bfloat16).view(2, seq, dim)
    v = to_dev(random_kv(rng, 2 * seq, dim, sigma=0.5), torch.int16).view(torch.bfloat16).view(2, seq, dim)
    q = to_dev(random_kv(rng, 2 * n_q, dim), torch.int16).view(torch.bfloat16).view(2, n_q, dim)

    def step(q, k, v):
        return torch.ops.kvexp.decode_attention_raw(q, k, v, 2, block, 0, False) * 1.0

    eager = step(q, k, v)
    say("torch.compile op")
    compiled = torch.compile(step, backend="eager", fullgraph=True)(q, k, v)
    assert bits_equal(eager.cpu().numpy(), compiled.cpu().numpy())


@pytest.mark.parametrize("order", [0, 1])
def test_decode_loop_ops(ctx, oracle, order):
    """The ops in a decode loop with reuse_plan=True: containers grown by one
    token per step (crossing a block boundary), the plan re-targeted by
    kvexp_hip_plan_update; every step equal to a freshly built plan, the
    last steps to the oracle. The raw op the same over views of a
    preallocated [n_heads, max_seq, dim] buffer, and decode_attention_kv
    over the same caches registered once."""
    import torch

    import kvexp_amd
    import kvexp_amd.torch_ops as ops

    rng = np.random.default_rng(91 + order)
    dim, n_q, block, splits, n_heads = 64, 7, 128, 2, 3
    start, steps = 250, 12
    max_seq = start + steps
    ks = [random_kv(rng, max_seq, dim, spread_lo=-6, spread_hi=4, outliers=2) for _ in range(n_heads)]
    vs = [random_kv(rng, max_seq, dim, sigma=0.5) for _ in range(n_heads)]
    q = random_kv(rng, n_heads * n_q, dim)
    dq = to_dev(q, torch.int16).view(torch.bfloat16).view(n_heads, n_q, dim)
    dk = [to_dev(k, torch.int16) for k in ks]
    dv = [to_dev(v, torch.int16) for v in vs]
    kc = [kvexp_amd.Cache(ctx, dim, max_seq, block) for _ in range(n_heads)]
    vc = [kvexp_amd.Cache(ctx, dim, max_seq, block) for _ in range(n_heads)]
    for i in range(n_heads):
        kc[i].append(dk[i][: start * dim], start, sync_size=False)
        vc[i].append(dv[i][: start * dim], start, sync_size=False)
    kbuf = torch.stack([d.view(torch.bfloat16).view(max_seq, dim) for d in dk])
    vbuf = torch.stack([d.view(torch.bfloat16).view(max_seq, dim) for d in dv])
    handle = ops.register_kv(kc, vc, n_q, dim, splits, block, order)
    seq = start
    for step in range(steps):
        for i in range(n_heads):
            kc[i].append(dk[i][seq * dim:(seq + 1) * dim], 1, sync_size=False)
            vc[i].append(dv[i][seq * dim:(seq + 1) * dim], 1, sync_size=False)
        seq += 1
        say("decode loop op", order, seq)
        kv, vv = [c.view() for c in kc], [c.view() for c in vc]
        got = ops.decode_attention_containers(dq, kv, vv, [seq] * n_heads, splits, block, order, reuse_plan=True)
        fresh = ops.decode_attention_containers(dq, kv, vv, [seq] * n_heads, splits, block, order)
        assert bits_equal(got.cpu().numpy(), fresh.cpu().numpy()), seq
        raw = torch.ops.kvexp.decode_attention_raw(dq, kbuf[:, :seq], vbuf[:, :seq], splits, block, order, True)
        assert bits_equal(raw.cpu().numpy(), fresh.cpu().numpy()), seq
        by_handle = torch.ops.kvexp.decode_attention_kv(dq, handle, [seq] * n_heads)
        assert bits_equal(by_handle.cpu().numpy(), fresh.cpu().numpy()), seq
        if step >= steps - 2:
            backend = "scalar" if order == 0 else "avx512"
            want = oracle.attention_heads(
                backend, q, [dict(k=k[: seq * dim], v=v[: seq * dim], seq=seq, threads=splits) for k, v in zip(ks, vs)],
                n_q=n_q, dim=dim, split=block)
            assert bits_equal(got.cpu().numpy().reshape(-1), want), seq
    ops.unregister_kv(handle)
    ops.clear_plan_cache()
