"""The reference's C++ API (include/kvexp/attention.hpp, codec.hpp) called
from C++: lib/cxx_api_threads, a g++/OpenMP program linked against
libkvexp_hip_cxx.so, runs attention_decode (Backend::Hip and
Backend::HipDpbf16, raw and XKV inputs) and encode_bf16 / decode_bf16 as the
jobs of an OpenMP parallel for over 8 host threads, as the reference's bench
calls attention_decode (src/bench.cpp:715-728). Every result is compared bit
for bit with the reference's golden outputs and containers, and every thread
checks the exception classes and messages of bad calls.

KVEXP_CXX_CASES_DIR, when set, names a directory the fixture files are
written to (and kept), so that the same program can be run again over them,
e.g. under rocprofv3 --hip-trace to count the device allocations per call."""
import os
import subprocess

import numpy as np
import pytest

from conftest import say

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(os.path.dirname(HERE), "compressed-kv-attention_amd", "lib", "cxx_api_threads")
BACKEND = {"scalar": 0, "avx2": 0, "avx512": 1}


def write_cases(d, oracle, golden) -> int:
    """Golden attention cases as the program's fixture files; returns their count."""
    z, man = golden
    lines = []
    for c in man["attn"]:
        n = c["name"]
        q, k, v = z[f"attn/{n}/q"], z[f"attn/{n}/k"], z[f"attn/{n}/v"]
        kx = oracle.encode(k, c["seq"], c["dim"], c["block"])
        vx = oracle.encode(v, c["seq"], c["dim"], c["block"])
        for be in c["backends"]:
            for th in c["threads"]:
                name = f"{n}_{be}_t{th}"
                want = z[f"attn/{n}/{be}/t{th}"].astype(np.float32)
                for ext, arr in (("q", q.astype(np.uint16)), ("k", k.astype(np.uint16)), ("v", v.astype(np.uint16)),
                                 ("kx", kx), ("vx", vx), ("want", want)):
                    arr.tofile(os.path.join(d, f"{name}.{ext}"))
                lines.append(f"{name} {BACKEND[be]} {c['n_q']} {c['dim']} {c['seq']} {th} {c['block']} "
                             f"{kx.size} {vx.size}")
    with open(os.path.join(d, "cases.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return len(lines)


def test_cxx_api_from_eight_threads(tmp_path, oracle, golden):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: run compressed-kv-attention_amd/build.py")
    d = os.environ.get("KVEXP_CXX_CASES_DIR") or str(tmp_path)
    os.makedirs(d, exist_ok=True)
    n = write_cases(d, oracle, golden)
    say("cxx api: cases", n)
    r = subprocess.run([BIN, d, "8", "2"], capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "8 threads (8 ran jobs)" in r.stdout and " 0 failures" in r.stdout
