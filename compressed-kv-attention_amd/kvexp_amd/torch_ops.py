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
descriptors of the heads: block descriptors, escape index, work items), which
reads the block indexes and costs far more than the attention itself; with
``reuse_plan=True`` the plan is kept and reused while the same tensors,
lengths and split count come back. Reuse is for containers that do not
change while they are used (a container rewritten in place at the same
address would meet a stale plan), so it is the caller's choice.
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


def _cached_plan(key: tuple, build):
    p = _plans.get(key)
    if p is None:
        p = build()
        _plans[key] = p
        while len(_plans) > _MAX_PLANS:
            _plans.popitem(last=False)[1].close()
    else:
        _plans.move_to_end(key)
    return p


def clear_plan_cache() -> None:
    while _plans:
        _plans.popitem()[1].close()


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
    key = ("xkv", q.device.index, n_q, dim, int(n_splits), int(split_tokens), int(order),
           tuple(int(t.data_ptr()) for t in k_blobs + v_blobs + k_offsets + v_offsets + k_first + v_first),
           tuple(int(b) for b in k_bytes + v_bytes), tuple(int(s) for s in seqs))

    def build():
        heads = []
        for i in range(n_heads):
            kx = Encoded(k_blobs[i], int(k_bytes[i]), k_offsets[i], k_first[i], int(seqs[i]), dim, split_tokens)
            vx = Encoded(v_blobs[i], int(v_bytes[i]), v_offsets[i], v_first[i], int(seqs[i]), dim, split_tokens)
            heads.append(dict(kx=kx, vx=vx, seq=int(seqs[i]), splits=int(n_splits)))
        return ctx.plan(heads, n_q, dim, int(split_tokens), int(order))

    return _run(q, key, build, reuse_plan, n_heads, n_q, dim)


def _run(q: Tensor, key: tuple, build, reuse: bool, n_heads: int, n_q: int, dim: int) -> Tensor:
    plan = _cached_plan(key, build) if reuse else build()
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
    k, v = k.contiguous(), v.contiguous()
    ctx = _context(q.device)
    key = ("raw", q.device.index, n_q, dim, int(n_splits), int(split_tokens), int(order), int(k.data_ptr()),
           int(v.data_ptr()), n_heads, seq)

    def build():
        heads = [dict(k=k[i], v=v[i], seq=seq, splits=int(n_splits)) for i in range(n_heads)]
        return ctx.plan(heads, n_q, dim, int(split_tokens), int(order))

    return _run(q, key, build, reuse_plan, n_heads, n_q, dim)


@decode_attention_raw.register_fake
def _(q, k, v, n_splits, split_tokens=128, order=ORDER_SCALAR, reuse_plan=False):
    return q.new_empty(q.shape, dtype=torch.float32)


def decode_attention_containers(q: Tensor, ks: list, vs: list, seqs: list[int], n_splits: int,
                                split_tokens: int = 128, order: int = ORDER_SCALAR,
                                reuse_plan: bool = False) -> Tensor:
    """decode_attention over lists of Encoded (or Cache views)."""
    return torch.ops.kvexp.decode_attention(
        q, [e.blob for e in ks], [e.offsets for e in ks], [e.first for e in ks], [e.blob for e in vs],
        [e.offsets for e in vs], [e.first for e in vs], [int(e.nbytes) for e in ks], [int(e.nbytes) for e in vs],
        [int(s) for s in seqs], int(n_splits), int(split_tokens), int(order), bool(reuse_plan))
