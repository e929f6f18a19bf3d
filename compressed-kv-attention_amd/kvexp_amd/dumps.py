"""KVD1 KV dumps and QSN1 query snapshots (the reference bench's real-data inputs).

Readers follow the reference bench (src/bench.cpp:76-163: parse_dump,
load_qsnap, head_ptr, query_ptr, snap_index), with the same checks and
messages (raised as RuntimeError, the reference's std::runtime_error). The
writers produce the files python/dump_kv.py writes (write_dump at
dump_kv.py:157-177, the .qsnap block at dump_kv.py:302-312), for tests and for
synthetic dumps; a real dump needs a model download and is not made here.

KVD1: 32-byte header of little-endian u32 (magic "KVD1", version 1, layers,
kv heads, q heads, head_dim, seq, 0), then K [layers, kv, seq, dim] BF16, then
V of the same shape (then the last-position Q, which the bench does not read).
QSN1: u32 magic "QSN1", n_snap, layers, q heads; n_snap u32 positions; u32
head_dim; Q [n_snap, layers, q heads, dim] BF16.

``model_scope`` runs the reference bench's model scope (every layer and KV
head at one snapshot length, src/bench.cpp:668-684) on the GPU: containers
encoded on the device, one plan over all heads.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np

KVD1_MAGIC = b"KVD1"
QSN1_MAGIC = b"QSN1"


@dataclass
class KVDump:
    layers: int
    kv: int
    nq: int
    dim: int
    seq: int
    k: np.ndarray  # [layers, kv, seq, dim] uint16 (memory-mapped)
    v: np.ndarray

    def head(self, layer: int, h: int, seq: int | None = None):
        """K and V of (layer, kv head) over the first `seq` tokens (head_ptr)."""
        n = self.seq if seq is None else seq
        return self.k[layer, h, :n], self.v[layer, h, :n]


@dataclass
class QSnap:
    pos: list
    layers: int
    nq: int
    dim: int
    q: np.ndarray  # [n_snap, layers, nq, dim] uint16

    def query(self, snap: int, layer: int, q0: int, n: int):
        """n query rows from q0 (query_ptr)."""
        return self.q[snap, layer, q0:q0 + n]


def parse_dump(path: str) -> KVDump:
    """parse_dump (src/bench.cpp:87-108) over a memory map of the file."""
    size = os.path.getsize(path)
    if size < 32:
        raise RuntimeError("dump too small")
    hdr = np.fromfile(path, dtype="<u4", count=8)
    if hdr[:1].tobytes() != KVD1_MAGIC or int(hdr[1]) != 1:
        raise RuntimeError("not a KVD1 v1 dump")
    layers, kv, nq, dim, seq = (int(x) for x in hdr[2:7])
    plane = layers * kv * seq * dim
    if size < 32 + plane * 4:
        raise RuntimeError("dump truncated")
    m = np.memmap(path, dtype="<u2", mode="r", offset=32, shape=(2 * plane,))
    k = m[:plane].reshape(layers, kv, seq, dim)
    v = m[plane:].reshape(layers, kv, seq, dim)
    return KVDump(layers, kv, nq, dim, seq, k, v)


def load_qsnap(path: str) -> QSnap:
    """load_qsnap (src/bench.cpp:118-143)."""
    try:
        f = open(path, "rb")
    except OSError:
        raise RuntimeError("open qsnap failed") from None
    with f:
        head = f.read(16)
        if len(head) < 16 or head[:4] != QSN1_MAGIC:
            raise RuntimeError("bad qsnap magic")
        nsnap, layers, nq = (int(x) for x in np.frombuffer(head[4:], dtype="<u4"))
        pb = f.read(4 * nsnap)
        d = f.read(4)
        dim = int(np.frombuffer(d, dtype="<u4")[0]) if len(d) == 4 else 0
        n = nsnap * layers * nq * dim
        qb = f.read(2 * n)
        if len(pb) != 4 * nsnap or len(d) != 4 or len(qb) != 2 * n:
            raise RuntimeError("truncated qsnap")
    pos = np.frombuffer(pb, dtype="<i4")
    q = np.frombuffer(qb, dtype="<u2")
    return QSnap([int(x) for x in pos], layers, nq, dim, q.reshape(nsnap, layers, nq, dim))


def snap_index(s: QSnap, seq: int) -> int:
    """snap_index (src/bench.cpp:157-164)."""
    for i, p in enumerate(s.pos):
        if p == seq:
            return i
    raise RuntimeError("no query snapshot for this length")


def write_dump(path: str, k: np.ndarray, v: np.ndarray, q: np.ndarray) -> None:
    """k, v [layers, kv, seq, dim], q [layers, q heads, dim] uint16, laid out as
    dump_kv.py's write_dump."""
    hdr = np.zeros(8, dtype="<u4")
    hdr[0] = np.frombuffer(KVD1_MAGIC, dtype="<u4")[0]
    hdr[1] = 1
    hdr[2], hdr[3], hdr[4], hdr[5], hdr[6] = k.shape[0], k.shape[1], q.shape[1], k.shape[3], k.shape[2]
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.ascontiguousarray(k, dtype="<u2").tobytes())
        f.write(np.ascontiguousarray(v, dtype="<u2").tobytes())
        f.write(np.ascontiguousarray(q, dtype="<u2").tobytes())


def write_qsnap(path: str, positions: list, q: np.ndarray) -> None:
    """q [n_snap, layers, q heads, dim] uint16, laid out as dump_kv.py's .qsnap."""
    hdr = np.zeros(4, dtype="<u4")
    hdr[0] = np.frombuffer(QSN1_MAGIC, dtype="<u4")[0]
    hdr[1], hdr[2], hdr[3] = len(positions), q.shape[1], q.shape[2]
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.asarray(positions, dtype="<u4").tobytes())
        f.write(np.asarray([q.shape[3]], dtype="<u4").tobytes())
        f.write(np.ascontiguousarray(q, dtype="<u2").tobytes())


def model_scope(ctx, dump: KVDump, qs: QSnap, seq: int, splits: int = 0, order: int = 0, block: int = 128,
                raw: bool = False):
    """Every layer and KV head of the dump at snapshot length `seq`
    (src/bench.cpp:668-684): returns (plan, q, containers) with q
    [layers * kv, group, dim] BF16 bits on the device, ready for plan.run().
    The K/V of each head are encoded on the device (kvexp_hip_encode), or
    passed raw with raw=True; splits = 0 takes the library's suggestion."""
    import torch

    if dump.nq % dump.kv or qs.nq != dump.nq or qs.layers != dump.layers or qs.dim != dump.dim:
        raise RuntimeError("dump and query snapshot shapes differ")
    if seq > dump.seq:
        raise RuntimeError("snapshot length beyond the dump")
    si = snap_index(qs, seq)
    group = dump.nq // dump.kv
    dev = torch.device("cuda", ctx.device)
    n = dump.layers * dump.kv
    splits = splits or ctx.suggest_splits(n, seq, block)
    heads, keep = [], []
    for layer in range(dump.layers):
        for h in range(dump.kv):
            k, v = dump.head(layer, h, seq)
            dk = torch.from_numpy(np.array(k).view(np.int16).reshape(-1)).to(dev)  # copies out of the map
            dv = torch.from_numpy(np.array(v).view(np.int16).reshape(-1)).to(dev)
            if raw:
                heads.append(dict(k=dk, v=dv, seq=seq, splits=splits))
            else:
                heads.append(dict(kx=ctx.encode(dk, seq, dump.dim, block), vx=ctx.encode(dv, seq, dump.dim, block),
                                  seq=seq, splits=splits))
            keep += [dk, dv]
    q = np.stack([qs.query(si, layer, h * group, group) for layer in range(dump.layers) for h in range(dump.kv)])
    dq = torch.from_numpy(np.array(q).view(np.int16).reshape(-1)).to(dev)
    plan = ctx.plan(heads, group, dump.dim, block, order)
    return plan, dq, (heads, keep)
