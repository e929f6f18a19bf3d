"""GPU encoder and block decoder (kvexp_hip_encode / kvexp_hip_decode) against the
oracle and the reference's golden containers: containers byte-identical to
encode_bf16 (codec.cpp:39-164), decode bit-identical to decode_bf16
(codec.cpp:166-174), block index equal to the header walk, and the reference's
format errors reported for damaged containers. Appends (kvexp_hip_append)
must leave the container byte-identical to encode_bf16 of the whole sequence
after every call."""
import numpy as np
import pytest

from conftest import bits_equal, say, to_dev
from kvdata import bf16_from_f32, random_kv

pytestmark = pytest.mark.gpu


def _encode(ctx, kv, seq, dim, block):
    import torch

    enc = ctx.encode(to_dev(kv, torch.int16), seq, dim, block)
    blob = enc.blob[: enc.nbytes].cpu().numpy()
    return enc, blob


def test_golden_containers(ctx, oracle, golden):
    import torch

    z, man = golden
    for c in man["codec"]:
        say("golden codec", c["name"])
        kv = z[f"codec/{c['name']}/kv"]
        want = z[f"codec/{c['name']}/blob"]
        enc, blob = _encode(ctx, kv, c["seq"], c["dim"], c["block"])
        assert np.array_equal(blob, want), c["name"]
        off, first = oracle.block_index(want, c["dim"], c["seq"])
        assert np.array_equal(enc.offsets.cpu().numpy(), off), c["name"]
        assert np.array_equal(enc.first.cpu().numpy(), first), c["name"]
        dec = ctx.decode(enc).cpu().numpy().view(np.uint16)
        assert np.array_equal(dec, kv), c["name"]
        up = ctx.upload(want, c["dim"], c["seq"], c["block"])
        dec2 = ctx.decode(up).cpu().numpy().view(np.uint16)
        assert np.array_equal(dec2, kv), c["name"]
        torch.cuda.synchronize()


def _kinds(rng, seq, dim, kind):
    n = seq * dim
    if kind == 0:
        return rng.integers(0, 65536, n, dtype=np.uint16)
    if kind == 1:
        x = rng.uniform(1.0, 7.9, n) * np.where(rng.random(n) < .5, -1, 1)
        return bf16_from_f32(x.astype(np.float32))
    if kind == 2:
        return random_kv(rng, seq, dim, outliers=min(2, dim), specials=True, wide=True)
    return random_kv(rng, seq, dim, outliers=min(2, dim))


def test_random_containers(ctx, oracle):
    rng = np.random.default_rng(123)
    for trial in range(60):
        dim = 4 * int(rng.integers(1, 65))
        block = int(rng.integers(1, min(255, 65535 // dim) + 1))
        seq = int(rng.integers(1, 1500))
        kind = trial % 4
        say("random codec", trial, dict(dim=dim, block=block, seq=seq, kind=kind))
        kv = _kinds(rng, seq, dim, kind)
        enc, blob = _encode(ctx, kv, seq, dim, block)
        want = oracle.encode(kv, seq, dim, block)
        assert np.array_equal(blob, want), trial
        dec = ctx.decode(enc).cpu().numpy().view(np.uint16)
        assert np.array_equal(dec, kv), trial
        if seq > 1:
            part = seq // 2
            dec = ctx.decode(enc, seq=part).cpu().numpy().view(np.uint16)
            assert np.array_equal(dec, kv[: part * dim]), trial


def test_full_size_roundtrips(ctx, oracle):
    """BASELINE sizes: C2 (dim 64, seq 32768) and C5 (dim 256, block 255,
    seq 100003: 392 full blocks + a 43-token tail) encode byte-identically and
    decode back to the input."""
    from kvexp_amd import synth

    for cfg, seq in (("c2", 32768), ("c5", 100003), ("c1", 8192)):
        c = synth.CONFIGS[cfg]
        k, v = synth.head_kv(cfg, seq)
        for name, kv in (("k", k), ("v", v)):
            say("full-size codec", cfg, name, seq)
            enc, blob = _encode(ctx, kv, seq, c["dim"], c["block"])
            assert np.array_equal(blob, oracle.encode(kv, seq, c["dim"], c["block"])), (cfg, name)
            assert np.array_equal(ctx.decode(enc).cpu().numpy().view(np.uint16), kv), (cfg, name)
            st = oracle.container_stats(blob, c["dim"])
            say("  mode mix", st)


def _damaged(ctx, oracle, mutate):
    import torch

    import kvexp_amd

    rng = np.random.default_rng(5)
    kv = random_kv(rng, 300, 64)
    kv[rng.choice(kv.size, 200, replace=False)] = 0x7000  # out-of-window exponents: escapes in 4-bit blocks
    blob = oracle.encode(kv, 300, 64, 128)
    assert all(oracle.container_stats(blob, 64)[m] == 0 for m in ("raw", "bits2"))
    up = ctx.upload(blob, 64, 300, 128)
    host = up.blob.cpu().numpy()
    mutate(host, up)
    up.blob.copy_(torch.from_numpy(host))
    with pytest.raises(kvexp_amd.KvexpHipError) as ei:
        ctx.decode(up)
    return ei.value


def test_damaged_container_errors(ctx, oracle):
    def bad_mode(h, up):
        h[int(up.offsets[1])] = 5  # (3 is the 3-bit extension, read at dim 64)

    def bad_dim(h, up):
        h[int(up.offsets[0]) + 4] = 32

    def fewer_escapes(h, up):
        o = int(up.offsets[1])
        n = int(h[o + 2]) | (int(h[o + 3]) << 8)
        assert n > 0
        h[o + 2], h[o + 3] = (n - 1) & 0xFF, (n - 1) >> 8

    say("damaged: mode")
    e = _damaged(ctx, oracle, bad_mode)
    assert e.kind == "runtime_error" and e.msg == "unknown xkv block mode"
    say("damaged: dim")
    e = _damaged(ctx, oracle, bad_dim)
    assert e.kind == "runtime_error" and e.msg == "xkv block dimension or length mismatch"
    say("damaged: escapes")
    e = _damaged(ctx, oracle, fewer_escapes)
    assert e.kind == "runtime_error" and e.msg == "xkv escape stream overrun"


def test_decode_ran_out(ctx, oracle):
    import kvexp_amd

    rng = np.random.default_rng(9)
    kv = random_kv(rng, 200, 32)
    enc, _ = _encode(ctx, kv, 200, 32, 64)
    with pytest.raises(kvexp_amd.KvexpHipError) as ei:
        ctx.decode(enc, seq=201)
    assert ei.value.msg == "xkv decode ran out of blocks"


def test_encode_argument_errors(ctx, reference):
    import torch

    import kvexp_amd

    kv = torch.zeros(64 * 256, dtype=torch.int16, device="cuda:0")
    for seq, dim, block in ((0, 64, 128), (10, 6, 128), (10, 260, 128), (10, 64, 256)):
        with pytest.raises(kvexp_amd.KvexpHipError) as ei:
            ctx.encode(kv, seq, dim, block)
        from oracle import KvexpError

        with pytest.raises(KvexpError) as er:
            reference.encode(np.zeros(64 * 256, np.uint16), seq, dim, block)
        assert (ei.value.kind, ei.value.msg) == (er.value.kind, er.value.msg)


@pytest.mark.parametrize("dim,block", [(64, 128), (128, 128), (256, 255), (36, 100), (8, 1)])
def test_append_equals_whole_encode(ctx, oracle, dim, block):
    """A container grown by appends of assorted sizes (single tokens,
    partial blocks, exact blocks, several blocks at once, none) equals
    encode_bf16 of the tokens so far after every append: bytes, block index,
    decode; data with raw, 2-bit and 4-bit blocks, escapes and specials."""
    import torch

    rng = np.random.default_rng(dim * 1000 + block)
    total = 3 * block + 37 if block > 1 else 300
    kv = np.concatenate([_kinds(rng, total, dim, kind)[: (total // 4) * dim] for kind in (0, 1, 2, 3)])
    total = kv.size // dim
    cache = ctx.cache(dim, total + 5, block)
    sizes = [1, 0, 2, block - 1 if block > 1 else 1, block, 1, 2 * block + 3, 5]
    pos = 0
    step = 0
    while pos < total:
        n = min(sizes[step % len(sizes)], total - pos)
        step += 1
        cache.append(to_dev(kv[pos * dim:(pos + n) * dim], torch.int16), n)
        pos += n
        if n == 0:
            continue
        want = oracle.encode(kv[: pos * dim], pos, dim, block)
        enc = cache.view()
        say("append", dim, block, step, dict(n=n, tokens=pos, bytes=enc.nbytes))
        assert enc.nbytes == want.size
        assert np.array_equal(enc.blob[: enc.nbytes].cpu().numpy(), want), (step, pos)
        off, first = oracle.block_index(want, dim, pos)
        assert np.array_equal(enc.offsets.cpu().numpy(), off), (step, pos)
        assert np.array_equal(enc.first.cpu().numpy(), first), (step, pos)
        if step % 3 == 0 or pos == total:
            dec = ctx.decode(enc).cpu().numpy().view(np.uint16)
            assert np.array_equal(dec, kv[: pos * dim]), (step, pos)
    from kvexp_amd import KvexpHipError

    with pytest.raises(KvexpHipError) as e:
        cache.append(to_dev(kv[: 6 * dim], torch.int16), 6)
    assert e.value.kind == "capacity"


def test_append_attention_after_encode(ctx, oracle):
    """A container made by kvexp_hip_encode and continued by appends (the tail
    filled from the caller's tokens) gives the same attention bits as a
    container encoded whole."""
    import torch

    rng = np.random.default_rng(99)
    dim, block, n_q = 64, 128, 7
    seq0, seq = 1000, 1300
    k = random_kv(rng, seq, dim, spread_lo=-6, spread_hi=4, outliers=2)
    v = random_kv(rng, seq, dim, sigma=0.5)
    q = random_kv(rng, n_q, dim)
    caches = []
    for x in (k, v):
        c = ctx.cache(dim, seq, block)
        enc0 = ctx.encode(to_dev(x[: seq0 * dim], torch.int16), seq0, dim, block)
        c.blob[: enc0.nbytes] = enc0.blob[: enc0.nbytes]
        c.offsets[: enc0.n_blocks + 1] = enc0.offsets
        c.first[: enc0.n_blocks + 1] = enc0.first
        tail = seq0 % block
        c.tail[: tail * dim] = to_dev(x[(seq0 - tail) * dim: seq0 * dim], torch.int16)
        c.seq, c.nbytes = seq0, enc0.nbytes
        for t in range(seq0, seq, 60):
            n = min(60, seq - t)
            c.append(to_dev(x[t * dim:(t + n) * dim], torch.int16), n)
        caches.append(c)
    splits = 3
    kx, vx = caches[0].view(), caches[1].view()
    assert np.array_equal(kx.blob[: kx.nbytes].cpu().numpy(), oracle.encode(k, seq, dim, block))
    plan = ctx.plan([dict(kx=kx, vx=vx, seq=seq, splits=splits)], n_q, dim, block)
    out = torch.empty(n_q * dim, dtype=torch.float32, device=torch.device("cuda", ctx.device))
    plan.run(to_dev(q, torch.int16), out)
    want = oracle.attention_heads("scalar", q, [dict(k=k, v=v, seq=seq, threads=splits)], n_q=n_q, dim=dim,
                                  split=block)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), np.asarray(want, np.float32).view(np.uint32))


def test_append_batch(ctx, oracle):
    """kvexp_hip_append_batch over containers in different states (empty,
    partial trailing block, block-aligned) with different append sizes (0, 1,
    a partial block, several blocks) in one call; repeated rounds, each
    container equal to encode_bf16 of its tokens so far after every round."""
    import torch

    rng = np.random.default_rng(2024)
    dim, block, n_c = 64, 128, 12
    total = 1200
    data = [_kinds(rng, total, dim, i % 4) for i in range(n_c)]
    caches = [ctx.cache(dim, total, block) for _ in range(n_c)]
    start = [0, 1, 127, 128, 129, 300, 0, 5, 256, 511, 64, 1000]
    for c, d, st in zip(caches, data, start):  # bring each container to its starting length
        if st:
            c.append(to_dev(d[: st * dim], torch.int16), st)
    pos = list(start)
    for rnd, sizes in enumerate([[1] * n_c, [0, 3, 1, 127, 128, 129, 0, 250, 1, 1, 64, 2],
                                 [1] * n_c, [5, 0, 300, 2, 1, 77, 128, 1, 0, 130, 7, 100]]):
        ns = [min(k, total - p) for k, p in zip(sizes, pos)]
        toks = [to_dev(d[p * dim:(p + k) * dim] if k else d[:dim], torch.int16) for d, p, k in zip(data, pos, ns)]
        ctx.append_batch(caches, toks, ns, check_errors=True)
        for i, (c, d) in enumerate(zip(caches, data)):
            pos[i] += ns[i]
            if pos[i] == 0:
                continue
            want = oracle.encode(d[: pos[i] * dim], pos[i], dim, block)
            n = c.size()
            say("append batch", rnd, i, dict(tokens=pos[i], bytes=n))
            assert n == want.size, (rnd, i)
            assert np.array_equal(c.blob[:n].cpu().numpy(), want), (rnd, i)
            off, first = oracle.block_index(want, dim, pos[i])
            assert np.array_equal(c.view().offsets.cpu().numpy(), off), (rnd, i)
            assert np.array_equal(c.view().first.cpu().numpy(), first), (rnd, i)


def test_append_set_steps(ctx, oracle):
    """AppendSet (the job table kept between steps) over 24 decode steps of
    one token per container plus one multi-token step, against encode_bf16."""
    import torch

    rng = np.random.default_rng(5)
    dim, block, n_c, seq0, steps = 64, 128, 6, 250, 24
    data = [_kinds(rng, seq0 + steps + 40, dim, i % 4).reshape(-1, dim) for i in range(n_c)]
    caches = [ctx.cache(dim, seq0 + steps + 40, block) for _ in range(n_c)]
    for c, d in zip(caches, data):
        c.append(to_dev(d[:seq0].reshape(-1), torch.int16), seq0)
    aset = ctx.append_set(caches)
    pos = seq0
    for step in list(range(steps)) + [-1]:
        n = 1 if step >= 0 else 40
        toks = to_dev(np.stack([d[pos:pos + n] for d in data]).reshape(-1), torch.int16)
        aset.append(toks, n, check_errors=(step % 8 == 0))
        pos += n
    for i, (c, d) in enumerate(zip(caches, data)):
        want = oracle.encode(d[:pos].reshape(-1), pos, dim, block)
        nb = c.size()
        say("append set", i, dict(tokens=pos, bytes=nb))
        assert c.seq == pos and nb == want.size
        assert np.array_equal(c.blob[:nb].cpu().numpy(), want), i


@pytest.mark.parametrize("dim,n_q,order", [(64, 7, 0), (128, 4, 1), (64, 9, 0)])
def test_decode_loop_plan_update(ctx, oracle, dim, n_q, order):
    """A decode loop: every step appends one token to each K/V container
    (AppendSet), re-targets one plan with kvexp_hip_plan_update (fast path
    inside a block, full rebuild when a block starts) and runs it; every
    step's output is bit-equal to a new plan over fresh encodes of the same
    tokens, and to the oracle at the first and last steps."""
    import torch

    rng = np.random.default_rng(dim + n_q)
    block, heads_n, splits = 128, 3, 3
    seq0, steps = 250, 12  # crosses the block boundary at 256
    ks = [random_kv(rng, seq0 + steps, dim, spread_lo=-6, spread_hi=4, outliers=2).reshape(-1, dim)
          for _ in range(heads_n)]
    vs = [random_kv(rng, seq0 + steps, dim, sigma=0.5).reshape(-1, dim) for _ in range(heads_n)]
    q = to_dev(random_kv(rng, heads_n * n_q, dim), torch.int16)
    caches = []
    for h in range(heads_n):
        for x in (ks[h], vs[h]):
            c = ctx.cache(dim, seq0 + steps, block)
            c.append(to_dev(x[:seq0].reshape(-1), torch.int16), seq0)
            caches.append(c)
    aset = ctx.append_set(caches)

    def heads_of(seq, views):
        return [dict(kx=views[2 * h], vx=views[2 * h + 1], seq=seq, splits=splits) for h in range(heads_n)]

    def views():
        out = []
        for c in caches:
            e = c.view()
            e.nbytes = -1  # the capacity stands in for the size
            out.append(e)
        return out

    plan = ctx.plan(heads_of(seq0, views()), n_q, dim, block, order)
    backend = "scalar" if order == 0 else "avx512"
    for step in range(steps):
        seq = seq0 + step + 1
        toks = torch.stack([to_dev(x[seq - 1:seq].reshape(-1), torch.int16)
                            for h in range(heads_n) for x in (ks[h], vs[h])]).contiguous()
        aset.append(toks, 1)
        plan.update(heads_of(seq, views()))
        got = plan.run(q, check_errors=True).cpu().numpy()
        fresh = [ctx.encode(to_dev(x[:seq].reshape(-1), torch.int16), seq, dim, block)
                 for h in range(heads_n) for x in (ks[h], vs[h])]
        ref_plan = ctx.plan(heads_of(seq, fresh), n_q, dim, block, order)
        want = ref_plan.run(q).cpu().numpy()
        say("decode loop", dim, n_q, order, step, dict(seq=seq))
        assert bits_equal(got, want), step
        if step in (0, steps - 1):
            ref = oracle.attention_heads(backend, q.cpu().numpy().view(np.uint16),
                                         [dict(k=ks[h][:seq].reshape(-1), v=vs[h][:seq].reshape(-1), seq=seq,
                                               threads=splits) for h in range(heads_n)],
                                         n_q=n_q, dim=dim, split=block)
            assert bits_equal(got, ref), step


def test_plan_update_raw_heads(ctx, oracle):
    """kvexp_hip_plan_update on a plan over raw BF16 heads (buffers sized for
    the final length): each step's output equals a new plan's, inside a split
    tile and across one."""
    import torch

    rng = np.random.default_rng(8)
    dim, n_q, block, heads_n, splits = 64, 7, 128, 2, 3
    seq0, steps = 380, 8  # crosses the tile boundary at 384
    ks = [to_dev(random_kv(rng, seq0 + steps, dim), torch.int16) for _ in range(heads_n)]
    vs = [to_dev(random_kv(rng, seq0 + steps, dim, sigma=0.5), torch.int16) for _ in range(heads_n)]
    q = to_dev(random_kv(rng, heads_n * n_q, dim), torch.int16)

    def heads_at(seq):
        return [dict(k=ks[h], v=vs[h], seq=seq, splits=splits) for h in range(heads_n)]

    plan = ctx.plan(heads_at(seq0), n_q, dim, block)
    for step in range(steps):
        seq = seq0 + step + 1
        plan.update(heads_at(seq))
        got = plan.run(q, check_errors=True).cpu().numpy()
        want = ctx.plan(heads_at(seq), n_q, dim, block).run(q).cpu().numpy()
        say("raw plan update", step, dict(seq=seq))
        assert bits_equal(got, want), step


def test_plan_update_failure_leaves_plan_refusing_runs(ctx, oracle):
    """A plan update whose rebuild fails (a damaged block header found by the
    rebuild's checks) keeps the plan's memory valid and makes every later run
    fail without launching a kernel, until an update succeeds; the run after
    that equals a new plan's."""
    import torch

    import kvexp_amd

    rng = np.random.default_rng(31)
    dim, n_q, block, splits = 64, 7, 128, 2
    seq0, seq1 = 250, 260  # the append starts a block: the update rebuilds
    k = random_kv(rng, seq1, dim, spread_lo=-6, spread_hi=4, outliers=2).reshape(-1, dim)
    v = random_kv(rng, seq1, dim, sigma=0.5).reshape(-1, dim)
    q = to_dev(random_kv(rng, n_q, dim), torch.int16)
    caches = []
    for x in (k, v):
        c = ctx.cache(dim, seq1, block)
        c.append(to_dev(x[:seq0].reshape(-1), torch.int16), seq0)
        caches.append(c)

    def heads(seq):
        views = []
        for c in caches:
            e = c.view()
            e.nbytes = -1
            views.append(e)
        return [dict(kx=views[0], vx=views[1], seq=seq, splits=splits)]

    plan = ctx.plan(heads(seq0), n_q, dim, block)
    for i, x in enumerate((k, v)):
        caches[i].append(to_dev(x[seq0:seq1].reshape(-1), torch.int16), seq1 - seq0)
    torch.cuda.synchronize()
    saved = int(caches[0].blob[0].item())
    caches[0].blob[0] = 5  # block 0 of K: mode byte 5 is no mode of the format
    say("plan update failure: damaged update")
    with pytest.raises(kvexp_amd.KvexpHipError) as ei:
        plan.update(heads(seq1))
    assert ei.value.kind == "runtime_error" and ei.value.msg == "unknown xkv block mode"
    out = torch.full((n_q * dim,), 7.0, dtype=torch.float32, device="cuda:0")
    say("plan update failure: run refused")
    with pytest.raises(kvexp_amd.KvexpHipError) as ei:
        plan.run(q, out=out)
    assert ei.value.kind == "runtime_error" and "stale" in ei.value.msg
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused run wrote its output"
    caches[0].blob[0] = saved
    say("plan update failure: repaired update")
    plan.update(heads(seq1))
    got = plan.run(q, check_errors=True).cpu().numpy()
    fresh = [ctx.encode(to_dev(x.reshape(-1), torch.int16), seq1, dim, block) for x in (k, v)]
    want = ctx.plan([dict(kx=fresh[0], vx=fresh[1], seq=seq1, splits=splits)], n_q, dim, block).run(q).cpu().numpy()
    assert bits_equal(got, want)
    ref = oracle.attention("scalar", q.cpu().numpy().view(np.uint16), k.reshape(-1), v.reshape(-1), n_q=n_q, dim=dim,
                           seq=seq1, threads=splits, split=block)
    assert bits_equal(got, ref)
