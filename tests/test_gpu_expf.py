"""The GPU build of the kernels' exp against the host libm expf (the function the
reference calls). The host build of the same source is compared exhaustively in
test_expf.py; here the device build is compared on dense ranges where results
are denormal or near the special-case thresholds, on [-1, 0], and on a stride of
all non-positive floats (softmax arguments are never positive)."""
import numpy as np
import pytest

from conftest import say, to_dev

pytestmark = pytest.mark.gpu


def _bits_range(lo: float, hi: float) -> np.ndarray:
    a = np.array([lo, hi], dtype=np.float32).view(np.uint32)
    lo_b, hi_b = int(min(a)), int(max(a))
    return np.arange(lo_b, hi_b + 1, dtype=np.uint32)


def test_device_expf_equals_libm(ctx, oracle):
    import torch

    parts = [
        _bits_range(-105.0, -86.0),            # denormal results, underflow threshold
        _bits_range(-1.0, -0.0),               # all of [-1, 0]
        np.arange(0x80000000, 0xFFFFFFFF, 61, dtype=np.uint32),  # stride over all negatives (incl. NaN)
        np.array([0x00000000, 0x80000000, 0xFF800000, 0x7F800000, 0x7FC00000, 0xFFC00001, 0x42B17218,
                  0x42B17217, 0xC2CFF1B4, 0xC2CFF1B5, 0x3F800000], dtype=np.uint32),
    ]
    for i, bits in enumerate(parts):
        say("expf part", i, bits.size)
        x = bits.view(np.float32)
        y = ctx.expf(to_dev(x)).cpu().numpy()
        torch.cuda.synchronize()
        bad = oracle.L.oracle_expf_compare(x.ctypes.data, y.ctypes.data, x.size,
                                           __import__("ctypes").byref(__import__("ctypes").c_int64(-1)))
        assert bad == 0, f"part {i}: {bad} mismatches"
