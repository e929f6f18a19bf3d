"""Whole configurations at full size on the GPU, checked through properties
that do not need the oracle (which would take hours at these sizes):

* every KV head of the step: XKV attention == raw BF16 attention bit for bit
  (the reference bench's memcmp gate, bench.cpp:644-646, 688-690);
* every container: GPU decode == the tokens it was encoded from.

Inputs are drawn on the device with the configuration's distributions
(torch RNG, seeded): c4 (256 KV heads x 131072 tokens, head_dim 128, 12.96 GB
of containers) and c3 (32 ragged sequences x 48 KV heads, with ~6 % narrow
K blocks that take 2-bit codes). The per-head oracle comparisons at these
lengths are in test_gpu_configs.py."""
import pytest

from conftest import say

pytestmark = pytest.mark.gpu


def _kv(torch, g, dev, seq, dim, block, narrow, spread, outliers):
    scale = torch.exp2(torch.rand(dim, generator=g, device=dev) * (spread[1] - spread[0]) + spread[0])
    if outliers:
        scale[torch.randperm(dim, generator=g, device=dev)[:outliers]] *= 32.0
    k = torch.randn(seq, dim, generator=g, device=dev) * scale
    if narrow:
        nb = (seq + block - 1) // block
        pick = torch.rand(nb, generator=g, device=dev) < narrow
        rows = pick.repeat_interleave(block)[:seq]
        band = (torch.rand(seq, dim, generator=g, device=dev) * 6.99 + 1.0) * \
            torch.where(torch.rand(seq, dim, generator=g, device=dev) < 0.5, -1.0, 1.0) * scale
        k = torch.where(rows[:, None], band, k)
    v = torch.randn(seq, dim, generator=g, device=dev) * 0.5
    return (k.to(torch.bfloat16).view(torch.int16).reshape(-1), v.to(torch.bfloat16).view(torch.int16).reshape(-1))


def _step(ctx, heads_raw, seqs, n_q, dim, block, splits, order, q):
    import torch

    xs = [dict(kx=ctx.encode(k, s, dim, block), vx=ctx.encode(v, s, dim, block), seq=s, splits=sp)
          for (k, v), s, sp in zip(heads_raw, seqs, splits)]
    for (k, v), h in zip(heads_raw, xs):  # every container decodes to its tokens
        assert torch.equal(ctx.decode(h["kx"]), k) and torch.equal(ctx.decode(h["vx"]), v)
    px = ctx.plan(xs, n_q, dim, block, order)
    pr = ctx.plan([dict(k=k, v=v, seq=s, splits=sp) for (k, v), s, sp in zip(heads_raw, seqs, splits)], n_q, dim,
                  block, order)
    ox = px.run(q, check_errors=True)
    orw = pr.run(q, check_errors=True)
    torch.cuda.synchronize()
    px.close()
    pr.close()
    return torch.equal(ox.view(torch.int32), orw.view(torch.int32)), sum(h["kx"].nbytes + h["vx"].nbytes for h in xs)


def test_c4_full_step(ctx):
    import torch

    dev = torch.device("cuda", ctx.device)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    H, S, D, G, BT = 256, 131072, 128, 4, 128
    heads = [_kv(torch, g, dev, S, D, BT, 0.0, (-5, 3), 0) for _ in range(H)]
    q = torch.randn(H * G * D, generator=g, device=dev).to(torch.bfloat16).view(torch.int16)
    splits = ctx.suggest_splits(H, S, BT, dim=D, n_q=G)
    assert splits == 8  # one round of resident waves at head_dim 128 (two per SIMD)
    assert ctx.suggest_splits(48, 32768, 128, dim=64, n_q=7) == 64 == ctx.suggest_splits(48, 32768, 128)
    for order in (0, 1):
        say("c4 full step", dict(heads=H, seq=S, order=order, splits=splits))
        same, container = _step(ctx, heads, [S] * H, G, D, BT, [splits] * H, order, q)
        assert same, order
        assert 0.70 < container / (4 * S * D * H) < 0.80


def test_c3_full_batch(ctx):
    import torch

    from kvexp_amd import synth

    dev = torch.device("cuda", ctx.device)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    c = synth.CONFIGS["c3"]
    lens = synth.c3_lengths(c["seed"], c["batch"])
    seqs, heads = [], []
    for seq in lens:
        for _ in range(c["layers"] * c["kv_heads"]):
            heads.append(_kv(torch, g, dev, seq, c["dim"], c["block"], 0.06, (-6, 4), 2))
            seqs.append(seq)
    # longest split of the uniform count no longer than the mean split of one
    # round of resident waves (3 per SIMD at head_dim 64, 7 query rows)
    uniform = ctx.suggest_splits_batch(seqs, c["block"], c["dim"], c["group"])
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert uniform == max(seqs) * 12 * cus // sum(seqs)
    assert ctx.suggest_splits_batch([32768] * 48, 128) == ctx.suggest_splits(48, 32768, 128)
    splits = [max(1, min(64, s // 512)) for s in seqs]
    q = torch.randn(len(heads) * c["group"] * c["dim"], generator=g, device=dev).to(torch.bfloat16).view(torch.int16)
    say("c3 full batch", dict(heads=len(heads), tokens=sum(seqs)))
    same, _ = _step(ctx, heads, seqs, c["group"], c["dim"], c["block"], splits, 0, q)
    assert same
