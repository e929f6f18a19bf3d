"""KVD1 / QSN1 files (kvexp_amd.dumps): the layout dump_kv.py writes, read back
as the reference bench reads it, and the reference's messages for damaged
files (src/bench.cpp:87-164)."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "compressed-kv-attention_amd"))
from kvexp_amd import dumps  # noqa: E402


def _files(tmp_path, layers=2, kv=2, nq=6, dim=16, seq=40, pos=(10, 40)):
    rng = np.random.default_rng(1)
    k = rng.integers(0, 65536, (layers, kv, seq, dim), dtype=np.uint16)
    v = rng.integers(0, 65536, (layers, kv, seq, dim), dtype=np.uint16)
    q_last = rng.integers(0, 65536, (layers, nq, dim), dtype=np.uint16)
    qs = rng.integers(0, 65536, (len(pos), layers, nq, dim), dtype=np.uint16)
    kp, qp = str(tmp_path / "m.kvd"), str(tmp_path / "m.qsnap")
    dumps.write_dump(kp, k, v, q_last)
    dumps.write_qsnap(qp, list(pos), qs)
    return kp, qp, k, v, q_last, qs


def test_round_trip_and_layout(tmp_path):
    kp, qp, k, v, q_last, qs = _files(tmp_path)
    raw = open(kp, "rb").read()
    assert raw[:4] == b"KVD1" and np.frombuffer(raw[4:32], "<u4").tolist() == [1, 2, 2, 6, 16, 40, 0]
    assert len(raw) == 32 + 2 * k.nbytes + q_last.nbytes
    d = dumps.parse_dump(kp)
    assert (d.layers, d.kv, d.nq, d.dim, d.seq) == (2, 2, 6, 16, 40)
    kk, vv = d.head(1, 0, 25)
    assert np.array_equal(kk, k[1, 0, :25]) and np.array_equal(vv, v[1, 0, :25])
    s = dumps.load_qsnap(qp)
    assert s.pos == [10, 40] and (s.layers, s.nq, s.dim) == (2, 6, 16)
    assert dumps.snap_index(s, 40) == 1
    assert np.array_equal(s.query(1, 1, 3, 3), qs[1, 1, 3:6])
    with pytest.raises(RuntimeError, match="no query snapshot for this length"):
        dumps.snap_index(s, 11)


def test_damaged_files(tmp_path):
    kp, qp, *_ = _files(tmp_path)
    raw = open(kp, "rb").read()
    bad = tmp_path / "bad.kvd"
    bad.write_bytes(raw[:31])
    with pytest.raises(RuntimeError, match="dump too small"):
        dumps.parse_dump(str(bad))
    bad.write_bytes(b"KVD2" + raw[4:])
    with pytest.raises(RuntimeError, match="not a KVD1 v1 dump"):
        dumps.parse_dump(str(bad))
    bad.write_bytes(raw[:4] + np.array([2], "<u4").tobytes() + raw[8:])
    with pytest.raises(RuntimeError, match="not a KVD1 v1 dump"):
        dumps.parse_dump(str(bad))
    bad.write_bytes(raw[: 32 + 2 * 2 * 2 * 40 * 16 * 2 - 1])
    with pytest.raises(RuntimeError, match="dump truncated"):
        dumps.parse_dump(str(bad))
    rq = open(qp, "rb").read()
    badq = tmp_path / "bad.qsnap"
    badq.write_bytes(b"QSN2" + rq[4:])
    with pytest.raises(RuntimeError, match="bad qsnap magic"):
        dumps.load_qsnap(str(badq))
    badq.write_bytes(rq[:10])
    with pytest.raises(RuntimeError, match="bad qsnap magic"):
        dumps.load_qsnap(str(badq))
    badq.write_bytes(rq[:-1])
    with pytest.raises(RuntimeError, match="truncated qsnap"):
        dumps.load_qsnap(str(badq))
    with pytest.raises(RuntimeError, match="open qsnap failed"):
        dumps.load_qsnap(str(tmp_path / "missing.qsnap"))
