"""PyTorch operators over the kvexp-amd C ABI (torch.library custom ops).

``torch.ops.kvexp.decode_attention`` is kvexp::attention_decode
(reference include/kvexp/attention.hpp:58-61, src/dispatch.cpp:27-104) for a
batch of KV heads held as XKV containers on the device; ``decode_attention_raw``
is the same call over raw BF16 K/V ([n_heads, seq, dim]). The argument
meaning follows the reference: ``n_splits`` is attention_decode's n_threads
(token_bounds over ``split_tokens``-token tiles, splits merged left to
right), ``order`` picks the score order (0: scalar/AVX2, 1: AVX-512 BF16),
and the output is FP32 [n_heads, n_q, dim], bit-identical to the reference
backend of that order run with the same n_threads.

Both run on torch's current stream. Each call builds a plan (the device
descriptors of the heads: block descriptors, escape records, work items),
which reads the block indexes and costs far more than the attention itself,
and synchronises the stream before releasing it. With ``reuse_plan=True`` the
plan is kept per set of buffers (the same tensors and split count) and a
call with new lengths re-targets it with kvexp_hip_plan_update instead: the
decode loop, where every container grows by appends between calls. Inside a
block that update is a launch on the stream (no synchronisation, no
allocation); when a head gains a block the plan is rebuilt. Reuse is the
caller's choice: it is for buffers whose contents only grow by appends
(kvexp_hip_append) while the plan lives; a container rewritten in place
otherwise would meet a stale plan.
The fake implementations give the output's shape and dtype, so the ops
trace under torch.compile / FakeTensorMode without a GPU.
"""
from __future__ import annotations

from collections import OrderedDict

import torch
from torch import Tensor

from . import ORDER_SCALAR, Context, Encoded

_contexts: dict[int, Context] = {}
_plans: "OrderedDict[tuple, object]" = OrderedDict()
_MAX_PLANS = 16


def _context(device: torch.device) -> Context:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _contexts:
        _contexts[idx] = Context(idx)
    return _contexts[idx]


def _cached_plan(key: tuple, lens: tuple, build, update):
    """The plan kept for `key` (built on first use), re-targeted with
    `update(plan)` when the lengths differ from its last call's."""
    entry = _plans.get(key)
    if entry is None:
        entry = [build(), lens]
        _plans[key] = entry
        while len(_plans) > _MAX_PLANS:
            _plans.popitem(last=False)[1][0].close()
    else:
        _plans.move_to_end(key)
        if entry[1] != lens:
            update(entry[0])
            entry[1] = lens
    return entry[0]


def clear_plan_cache() -> None:
    while _plans:
        _plans.popitem()[1][0].close()


def _check_q(q: Tensor, n_heads: int) -> tuple[int, int]:
    if q.device.type != "cuda":
        raise ValueError("kvexp.decode_attention: q must be a ROCm device tensor")
    if q.dim() != 3 or q.shape[0] != n_heads:
        raise ValueError("kvexp.decode_attention: q must be [n_heads, n_q, dim]")
    if q.dtype not in (torch.bfloat16, torch.int16):
        raise ValueError("kvexp.decode_attention: q must hold BF16 (bfloat16 or int16 bits)")
    return int(q.shape[1]), int(q.shape[2])


@torch.library.custom_op("kvexp::decode_attention", mutates_args=())
def decode_attention(q: Tensor, k_blobs: list[Tensor], k_offsets: list[Tensor], k_first: list[Tensor],
                     v_blobs: list[Tensor], v_offsets: list[Tensor], v_first: list[Tensor], k_bytes: list[int],
                     v_bytes: list[int], seqs: list[int], n_splits: int, split_tokens: int = 128,
                     order: int = ORDER_SCALAR, reuse_plan: bool = False) -> Tensor:
    n_heads = len(seqs)
    n_q, dim = _check_q(q, n_heads)
    lists = (k_blobs, k_offsets, k_first, v_blobs, v_offsets, v_first, k_bytes, v_bytes)
    if any(len(x) != n_heads for x in lists):
        raise ValueError("kvexp.decode_attention: one container, index and length per head")
    ctx = _context(q.device)
    # the plan follows the buffers; lengths, byte and block counts are what an update changes
    key = ("xkv", q.device.index, n_q, dim, int(n_splits), int(split_tokens), int(order),
           tuple(int(t.data_ptr()) for t in k_blobs + v_blobs + k_offsets + v_offsets + k_first + v_first))
    k_blocks = [int(t.numel()) - 1 for t in k_offsets]
    v_blocks = [int(t.numel()) - 1 for t in v_offsets]
    lens = (tuple(int(x) for x in seqs), tuple(int(b) for b in k_bytes), tuple(int(b) for b in v_bytes),
            tuple(k_blocks), tuple(v_blocks))

    def build():
        heads = []
        for i in range(n_heads):
            kx = Encoded(k_blobs[i], int(k_bytes[i]), k_offsets[i], k_first[i], int(seqs[i]), dim, split_tokens)
            vx = Encoded(v_blobs[i], int(v_bytes[i]), v_offsets[i], v_first[i], int(seqs[i]), dim, split_tokens)
            heads.append(dict(kx=kx, vx=vx, seq=int(seqs[i]), splits=int(n_splits)))
        return ctx.plan(heads, n_q, dim, int(split_tokens), int(order))

    def update(plan):
        plan.update_heads(lens[0], lens[1], lens[2], k_blocks, v_blocks, stream=torch.cuda.current_stream(q.device))

    return _run(q, key, lens, build, update, reuse_plan, n_heads, n_q, dim)


def _run(q: Tensor, key: tuple, lens: tuple, build, update, reuse: bool, n_heads: int, n_q: int,
         dim: int) -> Tensor:
    plan = _cached_plan(key, lens, build, update) if reuse else build()
    out = torch.empty((n_heads, n_q, dim), dtype=torch.float32, device=q.device)
    try:
        plan.run(q.contiguous(), out, stream=torch.cuda.current_stream(q.device))
    finally:
        if not reuse:
            torch.cuda.current_stream(q.device).synchronize()  # the plan's buffers outlive the launch
            plan.close()
    return out


@decode_attention.register_fake
def _(q, k_blobs, k_offsets, k_first, v_blobs, v_offsets, v_first, k_bytes, v_bytes, seqs, n_splits,
      split_tokens=128, order=ORDER_SCALAR, reuse_plan=False):
    return q.new_empty(q.shape, dtype=torch.float32)


@torch.library.custom_op("kvexp::decode_attention_raw", mutates_args=())
def decode_attention_raw(q: Tensor, k: Tensor, v: Tensor, n_splits: int, split_tokens: int = 128,
                         order: int = ORDER_SCALAR, reuse_plan: bool = False) -> Tensor:
    if k.dim() != 3 or v.shape != k.shape:
        raise ValueError("kvexp.decode_attention_raw: k and v must be [n_heads, seq, dim]")
    n_heads, seq, _ = k.shape
    n_q, dim = _check_q(q, n_heads)
    if k.shape[2] != dim or k.dtype not in (torch.bfloat16, torch.int16) or v.dtype != k.dtype:
        raise ValueError("kvexp.decode_attention_raw: K/V must hold BF16 [n_heads, seq, dim]")
    # each head's rows must be contiguous; heads may sit apart (a view of a
    # larger buffer that a decode loop fills), which keeps the buffer's address
    if k.stride(2) != 1 or k.stride(1) != dim:
        k = k.contiguous()
    if v.stride(2) != 1 or v.stride(1) != dim:
        v = v.contiguous()
    ctx = _context(q.device)
    # heads are rows of k / v: the buffers are the base pointers and the head stride
    key = ("raw", q.device.index, n_q, dim, int(n_splits), int(split_tokens), int(order), int(k.data_ptr()),
           int(v.data_ptr()), n_heads, int(k.stride(0)), int(v.stride(0)))
    lens = (seq,)

    def build():
        heads = [dict(k=k[i], v=v[i], seq=seq, splits=int(n_splits)) for i in range(n_heads)]
        return ctx.plan(heads, n_q, dim, int(split_tokens), int(order))

    def update(plan):
        plan.update_heads([seq] * n_heads, stream=torch.cuda.current_stream(q.device))

    return _run(q, key, lens, build, update, reuse_plan, n_heads, n_q, dim)


@decode_attention_raw.register_fake
def _(q, k, v, n_splits, split_tokens=128, order=ORDER_SCALAR, reuse_plan=False):
    return q.new_empty(q.shape, dtype=torch.float32)


# ---- decode loops over registered containers ----------------------------
# A decode loop calls attention every step over the same containers, grown by
# appends. Passing every container's tensors through the op each step costs
# host time (per-tensor checks and keys for 6 lists); registering the
# containers once and passing only a handle and the lengths keeps the step
# to the op's dispatch, one head-table edit and two library calls.
_kv_sets: dict[int, dict] = {}


def register_kv(ks: list, vs: list, n_q: int, dim: int, n_splits: int, split_tokens: int = 128,
                order: int = ORDER_SCALAR) -> int:
    """Registers per-head K and V caches (kvexp_amd.Cache, or Encoded views of
    caches) for torch.ops.kvexp.decode_attention_kv; returns the handle. The
    caches must grow only by appends while registered (their block index
    then follows from the length: `split_tokens`-token blocks)."""
    if len(ks) != len(vs) or not ks:
        raise ValueError("kvexp.register_kv: one K and one V cache per head")
    for c in list(ks) + list(vs):
        # the block index of a cache is derived from its length in
        # split_tokens-token blocks, so every cache must use that block size
        if int(getattr(c, "block", split_tokens)) != int(split_tokens):
            raise ValueError(f"kvexp.register_kv: a cache of {c.block}-token blocks with split_tokens "
                             f"{split_tokens} (they must be equal)")
        if int(getattr(c, "dim", dim)) != int(dim):
            raise ValueError(f"kvexp.register_kv: a cache of head_dim {c.dim}, registered as {dim}")
    h = 1 + max(_kv_sets, default=0)
    _kv_sets[h] = dict(ks=list(ks), vs=list(vs), n_q=int(n_q), dim=int(dim), n_splits=int(n_splits),
                       split=int(split_tokens), order=int(order), plan=None, seqs=None, stream=None)
    return h


def unregister_kv(handle: int) -> None:
    e = _kv_sets.pop(int(handle), None)
    if e is not None and e["plan"] is not None:
        # the plan's buffers outlive its queued runs: wait for the stream of
        # its last update or run (and the current one)
        if e["stream"] is not None:
            e["stream"].synchronize()
        torch.cuda.current_stream().synchronize()
        e["plan"].close()


@torch.library.custom_op("kvexp::decode_attention_kv", mutates_args=())
def decode_attention_kv(q: Tensor, kv: int, seqs: list[int]) -> Tensor:
    """attention_decode over the caches registered as `kv` at lengths `seqs`
    (one per head), on torch's current stream: the first call builds the plan,
    later calls with new lengths re-target it (kvexp_hip_plan_update)."""
    e = _kv_sets.get(int(kv))
    if e is None:
        raise ValueError("kvexp.decode_attention_kv: unknown handle (register_kv)")
    n_heads = len(e["ks"])
    n_q, dim = _check_q(q, n_heads)
    if n_q != e["n_q"] or dim != e["dim"] or len(seqs) != n_heads:
        raise ValueError("kvexp.decode_attention_kv: q [n_heads, n_q, dim] and one length per head, as registered")
    stream = torch.cuda.current_stream(q.device)
    seqs = [int(x) for x in seqs]
    if e["plan"] is None:
        ctx = _context(q.device)
        heads = []
        for k, v, s in zip(e["ks"], e["vs"], seqs):
            kx, vx = _cap_view(k, s, e["split"]), _cap_view(v, s, e["split"])
            heads.append(dict(kx=kx, vx=vx, seq=s, splits=e["n_splits"]))
        e["plan"] = ctx.plan(heads, n_q, dim, e["split"], e["order"], stream=stream)
        e["seqs"] = seqs
    elif seqs != e["seqs"]:
        bt = e["split"]
        nb = [(s + bt - 1) // bt for s in seqs]
        neg = [-1] * n_heads
        e["plan"].update_heads(seqs, neg, neg, nb, nb, stream=stream)
        e["seqs"] = seqs
    out = torch.empty((n_heads, n_q, dim), dtype=torch.float32, device=q.device)
    e["plan"].run(q.contiguous(), out, stream=stream)
    e["stream"] = stream
    return out


@decode_attention_kv.register_fake
def _(q, kv, seqs):
    return q.new_empty(q.shape, dtype=torch.float32)


def _cap_view(c, seq: int, block: int) -> Encoded:
    """A cache (or a view of one) at `seq` tokens, its capacity as the byte count."""
    n_blocks = (seq + block - 1) // block
    return Encoded(c.blob, -1, c.offsets[: n_blocks + 1], c.first[: n_blocks + 1], seq, c.dim, block)


def decode_attention_containers(q: Tensor, ks: list, vs: list, seqs: list[int], n_splits: int,
                                split_tokens: int = 128, order: int = ORDER_SCALAR,
                                reuse_plan: bool = False) -> Tensor:
    """decode_attention over lists of Encoded (or Cache views)."""
    return torch.ops.kvexp.decode_attention(
        q, [e.blob for e in ks], [e.offsets for e in ks], [e.first for e in ks], [e.blob for e in vs],
        [e.offsets for e in vs], [e.first for e in vs], [int(e.nbytes) for e in ks], [int(e.nbytes) for e in vs],
        [int(s) for s in seqs], int(n_splits), int(split_tokens), int(order), bool(reuse_plan))
