"""Pins the kernels' exp (compressed-kv-attention_amd/csrc/hip/kvexp_expf.h).

The reference's softmax uses std::exp(float), i.e. glibc's expf. The header
restates glibc 2.35's algorithm; here the same source is compiled for the host
and compared with the host libm over all 2^32 float bit patterns (the GPU
build is checked against the host libm on the device in test_gpu_expf.py).
"""
import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "csrc", "expf_exhaustive.c")
INC = os.path.join(ROOT, "compressed-kv-attention_amd", "csrc", "hip")


def test_expf_restatement_equals_libm_on_all_floats():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "expf_exhaustive")
        subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", f"-I{INC}", SRC, "-o", exe,
                        "-lm"], check=True)
        out = subprocess.run([exe, "0", str(1 << 32)], check=True, capture_output=True, text=True).stdout.split()
    mismatches, first = int(out[0]), int(out[1])
    assert mismatches == 0, f"{mismatches} mismatches, first at bits 0x{first:08x}"
