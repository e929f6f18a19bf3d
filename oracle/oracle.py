"""TEST INFRASTRUCTURE ONLY — numpy bindings of the CPU oracle and of the compiled reference.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module, and only as the checker. The product path never does.

* :class:`Oracle` wraps ``oracle/_build/libkvexp_oracle.so`` (the plain-C
  restatement in ``oracle/kvexp_oracle.c``).
* :class:`Reference` wraps ``oracle/_ref/libkvexp_ref.so``: the reference
  library compiled from its own sources by ``oracle/Makefile`` plus the
  ``oracle/ref_shim.cpp`` C shim. It exists only where it was built (this
  container, and GPU boxes that received the prebuilt file).

Errors come back as :class:`KvexpError` carrying the reference's exception
class name (``invalid_argument`` / ``runtime_error`` / ``logic_error``) and
its ``what()`` text.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libkvexp_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libkvexp_ref.so")

BACKENDS = {"scalar": 0, "avx2": 1, "avx512": 2}
_KIND = {1: "invalid_argument", 2: "runtime_error", 3: "logic_error", 4: "exception", 5: "capacity"}


class KvexpError(Exception):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_KIND.get(code, code)}: {msg}")
        self.code = code
        self.kind = _KIND.get(code, str(code))
        self.msg = msg


def build(with_reference: bool = True) -> None:
    """Runs oracle/Makefile (the reference part only where its sources exist)."""
    target = "all" if with_reference else "oracle"
    subprocess.run(["make", "-s", "-C", HERE, target], check=True)


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def _u8(a) -> np.ndarray:
    if isinstance(a, (bytes, bytearray)):
        return np.frombuffer(bytes(a), dtype=np.uint8)
    return np.ascontiguousarray(a, dtype=np.uint8)


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build(with_reference=False)
        L = C.CDLL(path)
        vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
        L.oracle_last_error.restype = C.c_char_p
        L.oracle_encode_bound.restype = sz
        L.oracle_encode_bound.argtypes = [i32, i32, i32]
        L.oracle_encode.argtypes = [vp, i32, i32, i32, vp, sz, C.POINTER(sz)]
        L.oracle_encode_modes.argtypes = [vp, i32, i32, i32, C.c_uint, vp, sz, C.POINTER(sz)]
        L.oracle_container_mode_counts.argtypes = [vp, sz, i32, vp]
        L.oracle_decode.argtypes = [vp, sz, i32, i32, vp]
        L.oracle_block_index.argtypes = [vp, sz, i32, i32, vp, vp, i32, C.POINTER(i32)]
        L.oracle_container_stats.argtypes = [vp, sz, i32] + [C.POINTER(C.c_int64)] * 4
        L.oracle_attention.argtypes = [i32, vp, vp, vp, vp, sz, vp, sz, vp, vp, i32, i32, i32, i32, i32]
        L.oracle_attention_heads.argtypes = [i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32,
                                             vp, vp, i32, vp]
        L.oracle_score_scalar.restype = C.c_float
        L.oracle_score_scalar.argtypes = [vp, vp, i32]
        L.oracle_score_dpbf16.restype = C.c_float
        L.oracle_score_dpbf16.argtypes = [vp, vp, i32]
        L.oracle_expf_array.argtypes = [vp, vp, sz]
        L.oracle_expf_compare.restype = sz
        L.oracle_expf_compare.argtypes = [vp, vp, sz, C.POINTER(C.c_int64)]
        L.oracle_expf_compare_range.restype = sz
        L.oracle_expf_compare_range.argtypes = [C.c_uint32, C.c_uint32, vp, C.POINTER(C.c_int64)]
        for f in ("oracle_exp_payload_bytes", "oracle_coded_block_bytes", "oracle_raw_block_bytes"):
            getattr(L, f).restype = i32
        self.L = L

    def _check(self, rc: int) -> None:
        if rc:
            raise KvexpError(rc, self.L.oracle_last_error().decode())

    # size model -----------------------------------------------------------
    def exp_payload_bytes(self, n, dim, bits):
        return self.L.oracle_exp_payload_bytes(n, dim, bits)

    def coded_block_bytes(self, n, dim, bits, esc):
        return self.L.oracle_coded_block_bytes(n, dim, bits, esc)

    def raw_block_bytes(self, n, dim):
        return self.L.oracle_raw_block_bytes(n, dim)

    def encode_bound(self, seq, dim, block):
        return int(self.L.oracle_encode_bound(seq, dim, block))

    # codec ----------------------------------------------------------------
    def encode(self, kv, seq: int, dim: int, block: int = 128, modes: int | None = None) -> np.ndarray:
        """encode_bf16; with `modes` (bit m: coded mode m may be chosen), the
        encoder with that choice of modes (0x14 = encode_bf16, 0x1c adds the
        3-bit extension)."""
        kv = _u16(kv)
        cap = max(self.encode_bound(seq, dim, block), 1)
        out = np.zeros(cap, dtype=np.uint8)
        n = C.c_size_t(0)
        src = _p(kv) if kv.size else None
        if modes is None:
            self._check(self.L.oracle_encode(src, seq, dim, block, _p(out), cap, C.byref(n)))
        else:
            self._check(self.L.oracle_encode_modes(src, seq, dim, block, modes, _p(out), cap, C.byref(n)))
        return out[: n.value].copy()

    def mode_counts(self, blob, dim: int) -> list:
        """Blocks per mode byte 0..4."""
        blob = _u8(blob)
        c = np.zeros(5, dtype=np.int64)
        self._check(self.L.oracle_container_mode_counts(_p(blob), blob.size, dim, _p(c)))
        return [int(x) for x in c]

    def decode(self, blob, seq: int, dim: int) -> np.ndarray:
        blob = _u8(blob)
        out = np.zeros(max(seq * dim, 1), dtype=np.uint16)
        self._check(self.L.oracle_decode(_p(blob), blob.size, seq, dim, _p(out)))
        return out[: seq * dim]

    def block_index(self, blob, dim: int, seq: int):
        blob = _u8(blob)
        cap = blob.size // 8 + 2
        off = np.zeros(cap + 1, dtype=np.int64)
        first = np.zeros(cap + 1, dtype=np.int32)
        nb = C.c_int(0)
        self._check(self.L.oracle_block_index(_p(blob), blob.size, dim, seq, _p(off), _p(first), cap,
                                              C.byref(nb)))
        return off[: nb.value + 1].copy(), first[: nb.value + 1].copy()

    def container_stats(self, blob, dim: int) -> dict:
        blob = _u8(blob)
        v = [C.c_int64(0) for _ in range(4)]
        self._check(self.L.oracle_container_stats(_p(blob), blob.size, dim, *[C.byref(x) for x in v]))
        return dict(raw=v[0].value, bits2=v[1].value, bits4=v[2].value, escapes=v[3].value)

    # attention ------------------------------------------------------------
    def attention(self, backend, q, k=None, v=None, kx=None, vx=None, *, n_q: int, dim: int, seq: int,
                  threads: int = 1, split: int = 128, with_lse: bool = False):
        be = BACKENDS[backend] if isinstance(backend, str) else int(backend)
        q = _u16(q)
        k = None if k is None else _u16(k)
        v = None if v is None else _u16(v)
        kx = None if kx is None else _u8(kx)
        vx = None if vx is None else _u8(vx)
        out = np.zeros(max(n_q * dim, 1), dtype=np.float32)
        lse = np.zeros(max(n_q, 1), dtype=np.float32) if with_lse else None
        self._check(self.L.oracle_attention(
            be, _p(q), _p(k), _p(v), _p(kx), 0 if kx is None else kx.size, _p(vx),
            0 if vx is None else vx.size, _p(out), _p(lse), n_q, dim, seq, threads, split))
        out = out[: n_q * dim]
        return (out, lse[:n_q]) if with_lse else out

    def attention_heads(self, backend, q, heads, *, n_q: int, dim: int, split: int = 128,
                        with_lse: bool = False):
        """heads: list of dicts with keys seq, threads and either k/v (u16) or kx/vx (u8)."""
        be = BACKENDS[backend] if isinstance(backend, str) else int(backend)
        H = len(heads)
        q = _u16(q)
        xkv = "kx" in heads[0]
        keep = []
        if xkv:
            ks = [_u8(h["kx"]) for h in heads]
            vs = [_u8(h["vx"]) for h in heads]
        else:
            ks = [_u16(h["k"]) for h in heads]
            vs = [_u16(h["v"]) for h in heads]
        keep += ks + vs
        kp = (C.c_void_p * H)(*[a.ctypes.data for a in ks])
        vpp = (C.c_void_p * H)(*[a.ctypes.data for a in vs])
        kb = np.array([a.size for a in ks], dtype=np.uint64)
        vb = np.array([a.size for a in vs], dtype=np.uint64)
        seq = np.array([h["seq"] for h in heads], dtype=np.int32)
        thr = np.array([h.get("threads", 1) for h in heads], dtype=np.int32)
        out = np.zeros(H * n_q * dim, dtype=np.float32)
        lse = np.zeros(H * n_q, dtype=np.float32) if with_lse else None
        st = np.zeros(H, dtype=np.int32)
        args = [be, H, _p(q)]
        if xkv:
            args += [None, None, C.cast(kp, C.c_void_p), _p(kb), C.cast(vpp, C.c_void_p), _p(vb)]
        else:
            args += [C.cast(kp, C.c_void_p), C.cast(vpp, C.c_void_p), None, None, None, None]
        args += [_p(out), _p(lse), n_q, dim, _p(seq), _p(thr), split, _p(st)]
        self._check(self.L.oracle_attention_heads(*args))
        return (out, lse) if with_lse else out

    def score(self, q, k, dim: int, order: str = "scalar") -> float:
        q, k = _u16(q), _u16(k)
        f = self.L.oracle_score_scalar if order == "scalar" else self.L.oracle_score_dpbf16
        return float(f(_p(q), _p(k), dim))

    # expf -------------------------------------------------------------------
    def expf(self, x) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        self.L.oracle_expf_array(_p(x), _p(y), x.size)
        return y

    def expf_compare_range(self, lo: int, hi: int, y: np.ndarray):
        first = C.c_int64(-1)
        y = np.ascontiguousarray(y, dtype=np.float32)
        bad = self.L.oracle_expf_compare_range(lo, hi, _p(y), C.byref(first))
        return int(bad), int(first.value)


class Reference:
    """The compiled reference library (oracle/_ref). Raises FileNotFoundError when absent."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = C.CDLL(path)
        vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
        L.kvexp_ref_last_error.restype = C.c_char_p
        L.kvexp_ref_detect_cpu.argtypes = [C.POINTER(i32), C.POINTER(i32)]
        L.kvexp_ref_encode.argtypes = [vp, i32, i32, i32, vp, sz, C.POINTER(sz)]
        L.kvexp_ref_decode.argtypes = [vp, sz, i32, i32, vp]
        L.kvexp_ref_attention.argtypes = [i32, vp, vp, vp, vp, sz, vp, sz, vp, i32, i32, i32, i32, i32]
        self.L = L
        a, b = C.c_int(0), C.c_int(0)
        L.kvexp_ref_detect_cpu(C.byref(a), C.byref(b))
        self.avx2, self.avx512_bf16 = bool(a.value), bool(b.value)

    def has(self, backend: str) -> bool:
        return {"scalar": True, "avx2": self.avx2, "avx512": self.avx512_bf16}[backend]

    def _check(self, rc: int) -> None:
        if rc:
            raise KvexpError(rc, self.L.kvexp_ref_last_error().decode())

    def encode(self, kv, seq: int, dim: int, block: int = 128) -> np.ndarray:
        kv = _u16(kv)
        cap = max(seq, 1) * max(dim, 1) * 2 + (max(seq, 1) // max(block, 1) + 2) * 8
        out = np.zeros(cap, dtype=np.uint8)
        n = C.c_size_t(0)
        self._check(self.L.kvexp_ref_encode(_p(kv) if kv.size else None, seq, dim, block, _p(out), cap,
                                            C.byref(n)))
        return out[: n.value].copy()

    def decode(self, blob, seq: int, dim: int) -> np.ndarray:
        blob = _u8(blob)
        out = np.zeros(max(seq * dim, 1), dtype=np.uint16)
        self._check(self.L.kvexp_ref_decode(_p(blob), blob.size, seq, dim, _p(out)))
        return out[: seq * dim]

    def attention(self, backend, q, k=None, v=None, kx=None, vx=None, *, n_q: int, dim: int, seq: int,
                  threads: int = 1, split: int = 128):
        be = BACKENDS[backend] if isinstance(backend, str) else int(backend)
        q = _u16(q)
        k = None if k is None else _u16(k)
        v = None if v is None else _u16(v)
        kx = None if kx is None else _u8(kx)
        vx = None if vx is None else _u8(vx)
        out = np.zeros(max(n_q * dim, 1), dtype=np.float32)
        self._check(self.L.kvexp_ref_attention(
            be, _p(q), _p(k), _p(v), _p(kx), 0 if kx is None else kx.size, _p(vx),
            0 if vx is None else vx.size, _p(out), n_q, dim, seq, threads, split))
        return out[: n_q * dim]

    def attention_heads(self, backend, q, ks, vs, *, xkv: bool, n_q: int, dim: int, seq: int, split: int = 128,
                        omp_threads: int = 1, out=None):
        """The reference bench's model_heads scope: OpenMP over heads, one thread per head.
        ks/vs: lists of uint16 arrays (raw) or uint8 containers (xkv). Returns out."""
        be = BACKENDS[backend] if isinstance(backend, str) else int(backend)
        L = self.L
        if not hasattr(L, "_heads_typed"):
            vp, i32 = C.c_void_p, C.c_int
            L.kvexp_ref_attention_heads.argtypes = [i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32,
                                                    i32]
            L._heads_typed = True
        H = len(ks)
        kp = (C.c_void_p * H)(*[a.ctypes.data for a in ks])
        vpp = (C.c_void_p * H)(*[a.ctypes.data for a in vs])
        q = _u16(q)
        if out is None:
            out = np.zeros(H * n_q * dim, dtype=np.float32)
        if xkv:
            kb = np.array([a.size for a in ks], dtype=np.uint64)
            vb = np.array([a.size for a in vs], dtype=np.uint64)
            args = [None, None, C.cast(kp, C.c_void_p), _p(kb), C.cast(vpp, C.c_void_p), _p(vb)]
        else:
            args = [C.cast(kp, C.c_void_p), C.cast(vpp, C.c_void_p), None, None, None, None]
        self._check(L.kvexp_ref_attention_heads(be, H, omp_threads, _p(q), *args, _p(out), n_q, dim, seq, split))
        return out


def reference_or_none():
    try:
        return Reference()
    except (FileNotFoundError, OSError):
        return None
