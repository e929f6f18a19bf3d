"""Python access to the kvexp-amd C ABI (include/kvexp_hip.h) over torch device memory.

The library ``lib/libkvexp_hip.so`` is built in-tree by ``build.py``; importing
this module does not build it, and every entry point raises if it is missing
(there is no CPU fallback). Tensors are torch CUDA(ROCm) tensors; BF16 data is
carried as ``torch.int16`` / ``torch.bfloat16`` bits.

Errors are :class:`KvexpHipError` with the C ABI status and the reference-style
message (``invalid_argument`` / ``runtime_error`` / ``logic_error`` kinds).
"""
from __future__ import annotations

import ctypes as C
import os
import re
from dataclasses import dataclass

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "lib", "libkvexp_hip.so")
HEADER = os.path.join(ROOT, "include", "kvexp_hip.h")

ORDER_SCALAR = 0
ORDER_DPBF16 = 1
# coded block modes the encoders may choose (kvexp_hip_set_encoder_modes)
MODE_2BIT, MODE_3BIT, MODE_4BIT = 4, 8, 16
MODES_REFERENCE = MODE_2BIT | MODE_4BIT

_KIND = {1: "invalid_argument", 2: "runtime_error", 3: "logic_error", 4: "unsupported", 5: "device_error",
         6: "capacity"}

_lib = None


class KvexpHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_KIND.get(code, code)}: {msg}")
        self.code = code
        self.kind = _KIND.get(code, str(code))
        self.msg = msg


class _AppendJob(C.Structure):
    _fields_ = [
        ("d_new", C.c_void_p), ("n_new", C.c_int32), ("n_tokens", C.c_int32),
        ("d_tail", C.c_void_p), ("d_blob", C.c_void_p), ("capacity", C.c_uint64),
        ("d_offsets", C.c_void_p), ("d_first_token", C.c_void_p),
        ("index_capacity", C.c_int32), ("reserved", C.c_int32),
    ]

    @classmethod
    def _fields_offsets(cls):
        return [(name, getattr(cls, name).offset) for name, _ in cls._fields_]


class _Head(C.Structure):
    _fields_ = [
        ("k_xkv", C.c_void_p), ("v_xkv", C.c_void_p),
        ("k_bytes", C.c_uint64), ("v_bytes", C.c_uint64),
        ("k_offsets", C.c_void_p), ("v_offsets", C.c_void_p),
        ("k_first_token", C.c_void_p), ("v_first_token", C.c_void_p),
        ("k_n_blocks", C.c_int32), ("v_n_blocks", C.c_int32),
        ("k_raw", C.c_void_p), ("v_raw", C.c_void_p),
        ("seq", C.c_int32), ("n_splits", C.c_int32),
    ]


def declared_symbols() -> list[str]:
    """Names of the functions include/kvexp_hip.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvexp_hip_\w+)\s*\(", text)))


def lib() -> C.CDLL:
    """Loads the library (raises FileNotFoundError when it was not built).

    KVEXP_HIP_LIBRARY, when set, names another build of the same library.
    """
    global _lib
    if _lib is not None:
        return _lib
    path = os.environ.get("KVEXP_HIP_LIBRARY", LIB_PATH)
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: run compressed-kv-attention_amd/build.py")
    L = C.CDLL(path)
    vp, sz, i32, i64 = C.c_void_p, C.c_size_t, C.c_int, C.c_int64
    L.kvexp_hip_status_string.restype = C.c_char_p
    L.kvexp_hip_status_string.argtypes = [i32]
    L.kvexp_hip_last_error.restype = C.c_char_p
    L.kvexp_hip_version.restype = C.c_char_p
    L.kvexp_hip_ctx_create.argtypes = [i32, C.POINTER(vp)]
    L.kvexp_hip_ctx_destroy.argtypes = [vp]
    for f in ("kvexp_hip_exp_payload_bytes", "kvexp_hip_coded_block_bytes", "kvexp_hip_raw_block_bytes",
              "kvexp_hip_block_count"):
        getattr(L, f).restype = i32
    L.kvexp_hip_encode_bound.restype = i64
    L.kvexp_hip_encode_bound.argtypes = [i32, i32, i32]
    L.kvexp_hip_build_index.argtypes = [vp, sz, i32, i32, vp, vp, i32, C.POINTER(i32)]
    L.kvexp_hip_encode.argtypes = [vp, vp, i32, i32, i32, vp, sz, vp, vp, C.POINTER(sz), vp]
    L.kvexp_hip_encode_noalloc.argtypes = [vp, vp, i32, i32, i32, vp, sz, vp, vp, vp, vp]
    L.kvexp_hip_decode.argtypes = [vp, vp, sz, vp, vp, i32, i32, i32, vp, i32, vp]
    L.kvexp_hip_append.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp, sz, vp, vp, i32, C.POINTER(sz), vp]
    L.kvexp_hip_append_batch.argtypes = [vp, C.POINTER(_AppendJob), i32, i32, i32, i32, vp]
    L.kvexp_hip_plan_create.argtypes = [vp, C.POINTER(_Head), i32, i32, i32, i32, i32, vp, C.POINTER(vp)]
    L.kvexp_hip_plan_destroy.argtypes = [vp]
    L.kvexp_hip_plan_update.argtypes = [vp, C.POINTER(_Head), i32, vp]
    L.kvexp_hip_suggest_splits.argtypes = [vp, i32, i32, i32]
    L.kvexp_hip_suggest_splits_for.argtypes = [vp, i32, i32, i32, i32, i32, i32]
    L.kvexp_hip_suggest_splits_batch.argtypes = [vp, i32, vp, i32, i32, i32, i32]
    L.kvexp_hip_set_encoder_modes.argtypes = [vp, C.c_uint]
    L.kvexp_hip_get_encoder_modes.argtypes = [vp]
    L.kvexp_hip_attention_run.argtypes = [vp, vp, vp, vp, i32, vp]
    L.kvexp_hip_plan_status.argtypes = [vp, vp]
    L.kvexp_hip_plan_timing.argtypes = [vp, i32]
    L.kvexp_hip_plan_kernel_time.argtypes = [vp, C.POINTER(C.c_double), C.POINTER(C.c_int)]
    L.kvexp_hip_attention_decode_host.argtypes = [vp, i32, vp, vp, vp, vp, sz, vp, sz, vp, i32, i32, i32, i32, i32]
    L.kvexp_hip_expf.argtypes = [vp, vp, vp, sz, vp]
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        raise KvexpHipError(rc, lib().kvexp_hip_last_error().decode())


def _ptr(t) -> int | None:
    if t is None:
        return None
    return int(t.data_ptr())


def _stream(stream):
    import torch

    if stream is None:
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return C.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


# ----------------------------------------------------------------- host-only --
def encode_bound(seq: int, dim: int, block: int = 128) -> int:
    return int(lib().kvexp_hip_encode_bound(seq, dim, block))


def build_index(blob, dim: int, seq: int):
    """Host walk of a host container (numpy uint8) -> (offsets int64, first int32) numpy arrays."""
    import numpy as np

    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    cap = blob.size // 8 + 2
    off = np.zeros(cap + 1, dtype=np.int64)
    first = np.zeros(cap + 1, dtype=np.int32)
    nb = C.c_int(0)
    check(lib().kvexp_hip_build_index(blob.ctypes.data_as(C.c_void_p), blob.size, dim, seq,
                                      off.ctypes.data_as(C.c_void_p), first.ctypes.data_as(C.c_void_p), cap,
                                      C.byref(nb)))
    return off[: nb.value + 1].copy(), first[: nb.value + 1].copy()


# ------------------------------------------------------------------- device --
@dataclass
class Encoded:
    """A device container and its block index."""
    blob: "object"     # torch.uint8 [capacity]
    nbytes: int
    offsets: "object"  # torch.int64 [n_blocks + 1]
    first: "object"    # torch.int32 [n_blocks + 1]
    seq: int
    dim: int
    block: int

    @property
    def n_blocks(self) -> int:
        return int(self.offsets.numel()) - 1


class Cache:
    """A device container grown by appends (kvexp_hip_append): the buffers for
    max_tokens tokens, the block index and the raw trailing partial block."""

    def __init__(self, ctx: "Context", dim: int, max_tokens: int, block: int = 128):
        import torch

        dev = torch.device("cuda", ctx.device)
        self.ctx, self.dim, self.block, self.max_tokens = ctx, dim, block, max_tokens
        self.capacity = max(encode_bound(max_tokens, dim, block), 1)
        self.index_capacity = max(lib().kvexp_hip_block_count(max_tokens, block), 0) + 1
        self.blob = torch.empty(self.capacity, dtype=torch.uint8, device=dev)
        self.offsets = torch.empty(self.index_capacity, dtype=torch.int64, device=dev)
        self.first = torch.empty(self.index_capacity, dtype=torch.int32, device=dev)
        self.tail = torch.empty(block * dim, dtype=torch.int16, device=dev)
        self.seq = 0
        self.nbytes = 0
        self.append(None, 0)

    def append(self, tokens, n: int | None = None, stream=None, sync_size: bool = True) -> None:
        """tokens: device tensor holding [n, dim] BF16 bits (or None with n = 0)."""
        n = int(tokens.numel() // self.dim) if n is None else int(n)
        out = C.c_size_t(0)
        check(lib().kvexp_hip_append(self.ctx.h, _ptr(tokens), n, self.seq, self.dim, self.block, _ptr(self.tail),
                                     _ptr(self.blob), self.capacity, _ptr(self.offsets), _ptr(self.first),
                                     self.index_capacity, C.byref(out) if sync_size else None, _stream(stream)))
        self.seq += n
        self.nbytes = int(out.value) if sync_size else -1

    def _job(self, tokens, n: int) -> _AppendJob:
        j = _AppendJob()
        j.d_new, j.n_new, j.n_tokens = _ptr(tokens), n, self.seq
        j.d_tail, j.d_blob, j.capacity = _ptr(self.tail), _ptr(self.blob), self.capacity
        j.d_offsets, j.d_first_token, j.index_capacity = _ptr(self.offsets), _ptr(self.first), self.index_capacity
        return j

    def size(self, stream=None) -> int:
        """Container bytes (reads the index's terminal entry; synchronises)."""
        nb = max(lib().kvexp_hip_block_count(self.seq, self.block), 0)
        self.nbytes = int(self.offsets[nb].item())
        return self.nbytes

    def view(self) -> Encoded:
        """The container as an Encoded (shares this cache's memory)."""
        nb = max(lib().kvexp_hip_block_count(self.seq, self.block), 0)
        return Encoded(self.blob, self.nbytes, self.offsets[: nb + 1], self.first[: nb + 1], self.seq, self.dim,
                       self.block)


class AppendSet:
    """A fixed list of caches (one dim and block size) appended together each
    step, as a decode loop does: the kvexp_hip_append_job table is kept as a
    numpy structured array with the C layout and updated in place, and the
    new tokens come as one [n_caches, n, dim] BF16 device tensor."""

    def __init__(self, ctx: "Context", caches: list):
        import numpy as np

        self.ctx, self.caches = ctx, list(caches)
        c0 = self.caches[0]
        self.dim, self.block = c0.dim, c0.block
        dt = np.dtype({"names": ["d_new", "n_new", "n_tokens", "d_tail", "d_blob", "capacity", "d_offsets",
                                 "d_first_token", "index_capacity", "reserved"],
                       "formats": ["<u8", "<i4", "<i4", "<u8", "<u8", "<u8", "<u8", "<u8", "<i4", "<i4"],
                       "offsets": [o for _, o in _AppendJob._fields_offsets()],
                       "itemsize": C.sizeof(_AppendJob)})
        j = np.zeros(len(self.caches), dtype=dt)
        for i, c in enumerate(self.caches):
            if c.dim != self.dim or c.block != self.block:
                raise ValueError("AppendSet: caches of one dim and block size")
            j[i] = (0, 0, c.seq, _ptr(c.tail), _ptr(c.blob), c.capacity, _ptr(c.offsets), _ptr(c.first),
                    c.index_capacity, 0)
        self.jobs = j
        self._stride = np.arange(len(self.caches), dtype=np.uint64)

    def append(self, tokens, n: int, check_errors: bool = False, stream=None) -> None:
        """tokens: contiguous device tensor [n_caches, n, dim] of BF16 bits."""
        import numpy as np

        j = self.jobs
        j["d_new"] = np.uint64(_ptr(tokens)) + self._stride * np.uint64(n * self.dim * 2)
        j["n_new"] = n
        check(lib().kvexp_hip_append_batch(self.ctx.h, C.cast(j.ctypes.data, C.POINTER(_AppendJob)), len(j),
                                           self.dim, self.block, 1 if check_errors else 0, _stream(stream)))
        j["n_tokens"] += n
        for c in self.caches:
            c.seq += n
            c.nbytes = -1


class Context:
    """One device context (workspace + status word)."""

    def __init__(self, device: int = 0):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("kvexp_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
        self.device = device
        h = C.c_void_p()
        check(lib().kvexp_hip_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().kvexp_hip_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # codec ------------------------------------------------------------------
    def set_encoder_modes(self, modes: int) -> None:
        """Coded modes this context's encoders may choose: MODES_REFERENCE
        (encode_bf16's containers, the default) or MODES_REFERENCE | MODE_3BIT
        (the 3-bit format extension)."""
        check(lib().kvexp_hip_set_encoder_modes(self.h, modes))

    @property
    def encoder_modes(self) -> int:
        return int(lib().kvexp_hip_get_encoder_modes(self.h))

    def encode(self, kv, seq: int, dim: int, block: int = 128, stream=None, sync_size: bool = True) -> Encoded:
        """kv: device tensor holding [seq, dim] BF16 bits (int16/bfloat16)."""
        import torch

        dev = torch.device("cuda", self.device)
        cap = max(encode_bound(seq, dim, block), 1)
        nb = max(lib().kvexp_hip_block_count(seq, block), 0)
        blob = torch.empty(cap, dtype=torch.uint8, device=dev)
        offs = torch.empty(nb + 1, dtype=torch.int64, device=dev)
        first = torch.empty(nb + 1, dtype=torch.int32, device=dev)
        n = C.c_size_t(0)
        check(lib().kvexp_hip_encode(self.h, _ptr(kv), seq, dim, block, _ptr(blob), cap, _ptr(offs), _ptr(first),
                                     C.byref(n) if sync_size else None, _stream(stream)))
        return Encoded(blob, int(n.value) if sync_size else -1, offs, first, seq, dim, block)

    def cache(self, dim: int, max_tokens: int, block: int = 128) -> "Cache":
        """An empty appendable container for up to max_tokens tokens."""
        return Cache(self, dim, max_tokens, block)

    def append_set(self, caches: list) -> "AppendSet":
        return AppendSet(self, caches)

    def append_batch(self, caches: list, tokens: list, n: int | list, check_errors: bool = False,
                     stream=None) -> None:
        """Appends tokens[i] ([n_i, dim] BF16 device tensors) to caches[i] in one
        kvexp_hip_append_batch call (all caches of one dim and block size).
        Container sizes are not read back (Cache.size() does that)."""
        ns = [int(n)] * len(caches) if isinstance(n, int) else [int(x) for x in n]
        arr = (_AppendJob * len(caches))()
        for i, (c, t) in enumerate(zip(caches, tokens)):
            arr[i] = c._job(t, ns[i])
        c0 = caches[0]
        check(lib().kvexp_hip_append_batch(self.h, arr, len(caches), c0.dim, c0.block, 1 if check_errors else 0,
                                           _stream(stream)))
        for c, k in zip(caches, ns):
            c.seq += k
            c.nbytes = -1

    def upload(self, blob_np, dim: int, seq: int, block: int = 128) -> Encoded:
        """A host container (numpy uint8) to the device, with its host-built index."""
        import torch

        off, first = build_index(blob_np, dim, seq)
        dev = torch.device("cuda", self.device)
        b = torch.from_numpy(blob_np.copy()).to(dev) if blob_np.size else torch.zeros(4, dtype=torch.uint8, device=dev)
        return Encoded(b, int(blob_np.size), torch.from_numpy(off).to(dev), torch.from_numpy(first).to(dev), seq, dim,
                       block)

    def decode(self, enc: Encoded, seq: int | None = None, out=None, check_errors: bool = True, stream=None):
        import torch

        seq = enc.seq if seq is None else seq
        if out is None:
            out = torch.empty(max(seq * enc.dim, 1), dtype=torch.int16, device=torch.device("cuda", self.device))
        check(lib().kvexp_hip_decode(self.h, _ptr(enc.blob), enc.nbytes, _ptr(enc.offsets), _ptr(enc.first),
                                     enc.n_blocks, seq, enc.dim, _ptr(out), 1 if check_errors else 0,
                                     _stream(stream)))
        return out[: seq * enc.dim]

    # attention --------------------------------------------------------------
    def plan(self, heads: list, n_q: int, dim: int, split: int = 128, order: int = ORDER_SCALAR,
             stream=None) -> "Plan":
        """heads: dicts with 'seq', 'splits' and either 'k'/'v' (raw device tensors) or
        'kx'/'vx' (Encoded; a Cache.view() whose size was not read back passes
        its capacity as the byte count). The build is ordered on `stream`
        (default: torch's current stream), after the work that wrote the
        containers."""
        arr, keep = _heads_array(heads)
        p = C.c_void_p()
        check(lib().kvexp_hip_plan_create(self.h, arr, len(heads), n_q, dim, split, order, _stream(stream),
                                          C.byref(p)))
        plan = Plan(self, p, len(heads), n_q, dim, keep)
        plan._arr = arr
        plan._caps = [(h["kx"].blob.numel(), h["vx"].blob.numel()) if "kx" in h else (0, 0) for h in heads]
        return plan

    def expf(self, x, out=None, stream=None):
        import torch

        if out is None:
            out = torch.empty_like(x)
        check(lib().kvexp_hip_expf(self.h, _ptr(x), _ptr(out), x.numel(), _stream(stream)))
        return out

    def suggest_splits(self, n_heads: int, seq: int, split: int = 128, dim: int | None = None, n_q: int = 7,
                       order: int = ORDER_SCALAR) -> int:
        if dim is None:
            return int(lib().kvexp_hip_suggest_splits(self.h, n_heads, seq, split))
        return int(lib().kvexp_hip_suggest_splits_for(self.h, n_heads, seq, split, dim, n_q, order))

    def suggest_splits_batch(self, seqs, split: int = 128, dim: int = 64, n_q: int = 7,
                             order: int = ORDER_SCALAR) -> int:
        """One split count for heads of the given (ragged) lengths."""
        import numpy as np

        arr = np.ascontiguousarray(np.asarray(seqs, dtype=np.int32))
        return int(lib().kvexp_hip_suggest_splits_batch(self.h, len(arr), arr.ctypes.data, split, dim, n_q, order))

    def attention_decode_host(self, order, q, k=None, v=None, kx=None, vx=None, *, n_q, dim, seq, threads=1,
                              split=128):
        """The Backend::Hip entry with host numpy buffers (reference argument list)."""
        import numpy as np

        def np_ptr(a):
            return None if a is None else a.ctypes.data_as(C.c_void_p)

        q = np.ascontiguousarray(q, dtype=np.uint16)
        k = None if k is None else np.ascontiguousarray(k, dtype=np.uint16)
        v = None if v is None else np.ascontiguousarray(v, dtype=np.uint16)
        kx = None if kx is None else np.ascontiguousarray(kx, dtype=np.uint8)
        vx = None if vx is None else np.ascontiguousarray(vx, dtype=np.uint8)
        out = np.zeros(max(n_q * dim, 1), dtype=np.float32)
        check(lib().kvexp_hip_attention_decode_host(
            self.h, order, np_ptr(q), np_ptr(k), np_ptr(v), np_ptr(kx), 0 if kx is None else kx.size, np_ptr(vx),
            0 if vx is None else vx.size, np_ptr(out), n_q, dim, seq, threads, split))
        return out[: n_q * dim]


def _heads_array(heads: list):
    arr = (_Head * len(heads))()
    keep = []
    for i, h in enumerate(heads):
        H = arr[i]
        H.seq = int(h["seq"])
        H.n_splits = int(h.get("splits", 1))
        if "kx" in h:
            kx, vx = h["kx"], h["vx"]
            keep += [kx, vx]
            H.k_xkv, H.v_xkv = _ptr(kx.blob), _ptr(vx.blob)
            H.k_bytes = kx.nbytes if kx.nbytes >= 0 else kx.blob.numel()
            H.v_bytes = vx.nbytes if vx.nbytes >= 0 else vx.blob.numel()
            H.k_offsets, H.v_offsets = _ptr(kx.offsets), _ptr(vx.offsets)
            H.k_first_token, H.v_first_token = _ptr(kx.first), _ptr(vx.first)
            H.k_n_blocks, H.v_n_blocks = kx.n_blocks, vx.n_blocks
        else:
            keep += [h["k"], h["v"]]
            H.k_raw, H.v_raw = _ptr(h["k"]), _ptr(h["v"])
    return arr, keep


_HEAD_DTYPE = None


def _head_dtype():
    """numpy view of kvexp_hip_head (edits a head table in place)."""
    global _HEAD_DTYPE
    if _HEAD_DTYPE is None:
        import numpy as np

        _HEAD_DTYPE = np.dtype({"names": [f for f, _ in _Head._fields_],
                                "formats": ["<u8" if t in (C.c_void_p, C.c_uint64) else "<i4"
                                            for _, t in _Head._fields_],
                                "offsets": [getattr(_Head, f).offset for f, _ in _Head._fields_],
                                "itemsize": C.sizeof(_Head)})
    return _HEAD_DTYPE


class Plan:
    def __init__(self, ctx: Context, h, n_heads: int, n_q: int, dim: int, keep):
        self.ctx, self.h, self.n_heads, self.n_q, self.dim, self._keep = ctx, h, n_heads, n_q, dim, keep

    def update(self, heads: list, stream=None) -> None:
        """kvexp_hip_plan_update: the plan's heads (same dicts as for Context.plan)
        with new lengths after appends."""
        arr, keep = _heads_array(heads)
        check(lib().kvexp_hip_plan_update(self.h, arr, len(heads), _stream(stream)))
        self._keep, self._arr = keep, arr
        self._caps = [(h["kx"].blob.numel(), h["vx"].blob.numel()) if "kx" in h else (0, 0) for h in heads]

    def update_lengths(self, seq, block: int = 128, stream=None) -> None:
        """kvexp_hip_plan_update for regular containers grown by appends: every
        head (or head i, for a list) now holds `seq` tokens in `block`-token
        blocks; the head table of the last create/update is edited in place
        (byte counts become the buffers' capacities)."""
        import numpy as np

        n = self.n_heads
        v = np.frombuffer(self._arr, dtype=_head_dtype(), count=n)
        seqs = np.full(n, int(seq), np.int64) if np.isscalar(seq) else np.asarray(seq, np.int64)
        nb = (seqs + block - 1) // block
        v["seq"] = seqs
        if self._caps and self._caps[0][0]:
            caps = np.asarray(self._caps, dtype=np.uint64)
            v["k_bytes"], v["v_bytes"] = caps[:, 0], caps[:, 1]
            v["k_n_blocks"], v["v_n_blocks"] = nb, nb
        check(lib().kvexp_hip_plan_update(self.h, self._arr, n, _stream(stream)))

    def update_heads(self, seqs, k_bytes=None, v_bytes=None, k_blocks=None, v_blocks=None, stream=None) -> None:
        """kvexp_hip_plan_update with per-head lengths (and, for XKV heads, byte
        and block counts; a negative byte count stands for the buffer's
        capacity), edited in place in the head table of the last create or
        update: the same buffers, grown by appends."""
        import numpy as np

        n = self.n_heads
        v = np.frombuffer(self._arr, dtype=_head_dtype(), count=n)
        v["seq"] = np.asarray(seqs, np.int64)
        if k_bytes is not None:
            caps = np.asarray(self._caps, dtype=np.int64)
            kb, vb = np.asarray(k_bytes, np.int64), np.asarray(v_bytes, np.int64)
            v["k_bytes"] = np.where(kb < 0, caps[:, 0], kb)
            v["v_bytes"] = np.where(vb < 0, caps[:, 1], vb)
            v["k_n_blocks"], v["v_n_blocks"] = np.asarray(k_blocks, np.int64), np.asarray(v_blocks, np.int64)
        check(lib().kvexp_hip_plan_update(self.h, self._arr, n, _stream(stream)))

    def run(self, q, out=None, lse=None, check_errors: bool = False, stream=None):
        import torch

        if out is None:
            out = torch.empty(self.n_heads * self.n_q * self.dim, dtype=torch.float32, device=q.device)
        check(lib().kvexp_hip_attention_run(self.h, _ptr(q), _ptr(out), _ptr(lse), 1 if check_errors else 0,
                                            _stream(stream)))
        return out

    def status(self, stream=None) -> None:
        check(lib().kvexp_hip_plan_status(self.h, _stream(stream)))

    def timing(self, enable: bool = True) -> None:
        """Records a HIP event pair around the split kernels of every later run."""
        check(lib().kvexp_hip_plan_timing(self.h, 1 if enable else 0))

    def kernel_time(self) -> tuple[float, int]:
        """(summed split-kernel ms, runs) since timing was enabled or last read; clears the record."""
        ms, runs = C.c_double(0.0), C.c_int(0)
        check(lib().kvexp_hip_plan_kernel_time(self.h, C.byref(ms), C.byref(runs)))
        return ms.value, runs.value

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().kvexp_hip_plan_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
