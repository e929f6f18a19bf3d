"""The reference bench's model scope on a KVD1/QSN1 pair (kvexp_amd.dumps.model_scope):
a synthetic dump in dump_kv.py's layout, every layer and KV head on the GPU,
XKV bit-equal to raw and to the oracle (the reference's attention_decode)."""
import numpy as np
import pytest

from conftest import bits_equal, say
from kvdata import random_kv

pytestmark = pytest.mark.gpu


def test_model_scope_on_a_dump(ctx, oracle, tmp_path):
    from kvexp_amd import dumps

    rng = np.random.default_rng(12)
    layers, kv, group, dim, seq = 2, 2, 7, 64, 700
    nq = kv * group
    k = np.stack([np.stack([random_kv(rng, seq, dim, spread_lo=-6, spread_hi=4, outliers=2).reshape(seq, dim)
                            for _ in range(kv)]) for _ in range(layers)])
    v = np.stack([np.stack([random_kv(rng, seq, dim, sigma=0.5).reshape(seq, dim) for _ in range(kv)])
                  for _ in range(layers)])
    pos = [300, 700]
    qs = random_kv(rng, len(pos) * layers * nq, dim).reshape(len(pos), layers, nq, dim)
    kp, qp = str(tmp_path / "s.kvd"), str(tmp_path / "s.qsnap")
    dumps.write_dump(kp, k, v, qs[-1])
    dumps.write_qsnap(qp, pos, qs)
    d, s = dumps.parse_dump(kp), dumps.load_qsnap(qp)
    for L in pos:
        splits = 3
        say("dump model scope", L)
        plan, dq, keep = dumps.model_scope(ctx, d, s, L, splits=splits)
        got = plan.run(dq, check_errors=True).cpu().numpy()
        plan_r, dq_r, keep_r = dumps.model_scope(ctx, d, s, L, splits=splits, raw=True)
        assert bits_equal(got, plan_r.run(dq_r).cpu().numpy())
        si = dumps.snap_index(s, L)
        want = oracle.attention_heads(
            "scalar", np.ascontiguousarray(s.q[si]).reshape(-1),
            [dict(k=np.ascontiguousarray(k[ly, h, :L]).reshape(-1), v=np.ascontiguousarray(v[ly, h, :L]).reshape(-1),
                  seq=L, threads=splits) for ly in range(layers) for h in range(kv)],
            n_q=group, dim=dim, split=128)
        assert bits_equal(got, want)
