"""GPU encoder and block decoder (kvexp_hip_encode / kvexp_hip_decode) against the
oracle and the reference's golden containers: containers byte-identical to
encode_bf16 (codec.cpp:39-164), decode bit-identical to decode_bf16
(codec.cpp:166-174), block index equal to the header walk, and the reference's
format errors reported for damaged containers."""
import numpy as np
import pytest

from conftest import say, to_dev
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
        h[int(up.offsets[1])] = 3

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
