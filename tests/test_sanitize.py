"""The library's host container walk (compressed-kv-attention_amd/csrc/host/
host_walk.hpp: parse_block, scan.hpp:28-66; the block index of a reader,
scan.hpp:144-151, 176-189; token_bounds, dispatch.cpp:17-23) and the C oracle,
built with AddressSanitizer and UndefinedBehaviorSanitizer by gcc/g++ and run
over intact, cut and edited containers (tests/csrc/sanitize_walk.cpp,
`make -C oracle sanitize`). CPU only: no GPU code is built or run."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("make") is None, reason="needs g++ and make")
def test_host_walk_and_oracle_under_asan_ubsan():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"],
                       capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    line = [s for s in r.stdout.splitlines() if s.startswith("sanitize_walk:")]
    assert line and line[-1].endswith(": ok"), out[-4000:]
    # the run covered every part: containers, cuts, edits that the walk
    # refused, and attention runs
    words = line[-1].split()
    assert int(words[1]) >= 200 and int(words[3]) >= 10000 and int(words[5]) >= 5000
    assert int(words[9]) >= 15
