import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests"),
          os.path.join(ROOT, "compressed-kv-attention_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running (full BASELINE-size) case")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle import reference_or_none

    r = reference_or_none()
    if r is None:
        pytest.skip("compiled reference (oracle/_ref) not built on this host")
    return r


@pytest.fixture(scope="session")
def golden():
    path = os.path.join(ROOT, "tests", "golden", "ref_vectors.npz")
    import json

    with open(os.path.join(ROOT, "tests", "golden", "ref_vectors.json")) as f:
        manifest = json.load(f)
    return np.load(path, allow_pickle=False), manifest


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise equality of float arrays, any NaN matching any NaN."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


@pytest.fixture(scope="session")
def ctx():
    """A kvexp_amd context on cuda:0 (GPU tests only)."""
    import torch

    import kvexp_amd

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = kvexp_amd.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def say(*a):
    """Progress line that names the case before a GPU step (flushed)."""
    print("[gpu-case]", *a, flush=True)


def to_dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to("cuda:0")
