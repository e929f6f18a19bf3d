"""The torch.library operators (kvexp_amd.torch_ops): registration and shape
inference on the CPU (FakeTensorMode, no GPU); the GPU results are checked
in test_gpu_torch_ops.py."""
import os
import sys

import pytest

torch = pytest.importorskip("torch")

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "compressed-kv-attention_amd"))


def test_ops_registered_and_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    import kvexp_amd.torch_ops  # noqa: F401  (registers the ops)

    assert hasattr(torch.ops.kvexp, "decode_attention")
    assert hasattr(torch.ops.kvexp, "decode_attention_raw")
    with FakeTensorMode():
        q = torch.empty(3, 7, 64, dtype=torch.bfloat16)
        k = torch.empty(3, 1000, 64, dtype=torch.bfloat16)
        out = torch.ops.kvexp.decode_attention_raw(q, k, k, 4, 128, 0, False)
        assert out.shape == (3, 7, 64) and out.dtype == torch.float32
        blobs = [torch.empty(100, dtype=torch.uint8) for _ in range(3)]
        offs = [torch.empty(9, dtype=torch.int64) for _ in range(3)]
        first = [torch.empty(9, dtype=torch.int32) for _ in range(3)]
        out = torch.ops.kvexp.decode_attention(q, blobs, offs, first, blobs, offs, first, [100] * 3, [100] * 3,
                                               [1000] * 3, 4, 128, 1, True)
        assert out.shape == (3, 7, 64) and out.dtype == torch.float32


def test_ops_reject_cpu_tensors():
    import kvexp_amd.torch_ops  # noqa: F401

    q = torch.zeros(1, 1, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 10, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device tensor"):
        torch.ops.kvexp.decode_attention_raw(q, k, k, 1, 128, 0, False)


def test_register_kv_rejects_other_block_sizes():
    """register_kv derives each cache's block index from its length in
    split_tokens-token blocks, so caches of another block size (or head_dim)
    are refused when registered, not misread later."""
    from types import SimpleNamespace

    from kvexp_amd import torch_ops

    good = SimpleNamespace(block=128, dim=64)
    odd = SimpleNamespace(block=64, dim=64)
    with pytest.raises(ValueError, match="64-token blocks with split_tokens 128"):
        torch_ops.register_kv([good, odd], [good, good], 7, 64, 4, 128)
    with pytest.raises(ValueError, match="head_dim 64, registered as 128"):
        torch_ops.register_kv([good], [good], 7, 128, 4, 128)
    h = torch_ops.register_kv([good], [good], 7, 64, 4, 128)
    torch_ops.unregister_kv(h)  # no plan was built: nothing to wait for
