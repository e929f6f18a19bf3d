"""Builds the libraries in-tree, under lib/:

  libkvexp_hip.so      the C ABI (include/kvexp_hip.h) and the gfx950 kernels;
                       exports C symbols only
  libkvexp_hip_cxx.so  the reference's C++ API (include/kvexp/*.hpp) over it,
                       for programs that use this library instead of the
                       reference's (a separate library, so the C ABI links
                       beside the reference's own kvexp:: symbols)
  cxx_api_threads      the C++ caller used by tests/test_gpu_cxx_api.py,
                       built with g++ and OpenMP as the reference's own code

    python compressed-kv-attention_amd/build.py [--jobs N] [--asm] [--trace]

(N defaults to the host's CPU count, at most 8.)

Every source is compiled with hipcc for gfx950 only, with the numeric flags
the reference uses for its own code (-ffp-contract=off, no fast math), and
with packed FP32 instructions disabled (-packed-fp32-ops target feature).
``--asm`` also writes the device assembly of each kernel file to
``_build/asm/`` for inspection. ``--trace`` builds, instead of the library
above, lib/trace/libkvexp_hip_trace.so: the same sources compiled with
KVEXP_PHASE_TRACE, whose split kernel (scalar order, XKV) and one-pass
encoder record per-wave / per-block cycle counts by phase, read back with
kvexp_hip_phase_trace_read / kvexp_hip_encode_trace_read
(``bench.py --phase-trace``). It is a measurement build, never loaded unless
KVEXP_HIP_LIBRARY names it.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libkvexp_hip.so")
LIB_CXX = os.path.join(LIB_DIR, "libkvexp_hip_cxx.so")
CXX_TEST = os.path.join(LIB_DIR, "cxx_api_threads")
CXX_TEST_SRC = os.path.join(ROOT, "tests", "csrc", "cxx_api_threads.cpp")
OBJ_DIR = os.path.join(HERE, "_build", "obj")
TRACE_OBJ_DIR = os.path.join(HERE, "_build", "obj_trace")
TRACE_LIB = os.path.join(LIB_DIR, "trace", "libkvexp_hip_trace.so")
ASM_DIR = os.path.join(HERE, "_build", "asm")

ARCH = "gfx950"
# the split kernel's instantiation units first (the longest compiles), so
# that a parallel build starts them at once
SOURCES = [
    "csrc/hip/attention_wave_d256_o1.hip",
    "csrc/hip/attention_wave_d256_o0.hip",
    "csrc/hip/attention_wave_d128_o1.hip",
    "csrc/hip/attention_wave_d128_o0.hip",
    "csrc/hip/attention_wave_d64_o1.hip",
    "csrc/hip/attention_wave_d64_o0.hip",
    "csrc/hip/attention_wave.hip",
    "csrc/hip/codec_kernels.hip",
    "csrc/hip/attention_kernels.hip",
    "csrc/host/kvexp_hip_api.cpp",
]
CXX_SOURCES = ["csrc/host/kvexp_cpp_api.cpp"]
HEADERS = [
    "csrc/hip/attention_wave.h",
    "csrc/hip/kvexp_device.h",
    "csrc/hip/kvexp_expf.h",
    "csrc/hip/kvexp_types.h",
    "csrc/host/host_walk.hpp",
    "../include/kvexp_hip.h",
    "../include/kvexp/attention.hpp",
    "../include/kvexp/codec.hpp",
    "../include/kvexp/bf16.hpp",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm 7.x expected under /opt/rocm)")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-fno-fast-math",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
        f"-I{os.path.join(ROOT, 'include')}",
        f"-I{os.path.join(HERE, 'csrc', 'hip')}",
    ]


def _newest(paths) -> float:
    return max(os.path.getmtime(os.path.join(HERE, p)) for p in paths)


def _compile(src: str, force: bool, trace: bool = False) -> str:
    obj = os.path.join(TRACE_OBJ_DIR if trace else OBJ_DIR, os.path.basename(src) + ".o")
    dep_time = max(_newest([src]), _newest(HEADERS), os.path.getmtime(__file__))
    if not force and os.path.exists(obj) and os.path.getmtime(obj) >= dep_time:
        return obj
    if src.endswith(".hip"):
        cmd = [hipcc()] + common_flags() + ["-x", "hip"]
    else:  # host-only translation unit: plain C++ against the HIP runtime headers
        cmd = [hipcc()] + [f for f in common_flags() if not f.startswith("--offload-arch")] + ["-x", "c++"]
        cmd = [c for c in cmd if c not in ("-Xclang", "-target-feature", "-packed-fp32-ops")]
        cmd += ["-D__HIP_PLATFORM_AMD__=1", "-I/opt/rocm/include"]
    if trace:
        cmd += ["-DKVEXP_PHASE_TRACE"]
    cmd += ["-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def _asm(src: str) -> None:
    os.makedirs(ASM_DIR, exist_ok=True)
    out = os.path.join(ASM_DIR, os.path.basename(src) + ".s")
    cmd = [hipcc()] + common_flags() + ["-x", "hip", "--cuda-device-only", "-S",
                                         os.path.join(HERE, src), "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, text=True)


def default_jobs() -> int:
    return max(1, min(8, os.cpu_count() or 1))


def build(force: bool = True, jobs: int = 0, asm: bool = False) -> str:
    """Compiles every source (``force``: even when up to date) and links the library."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    jobs = jobs if jobs > 0 else default_jobs()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), SOURCES + CXX_SOURCES))
        if asm:
            list(ex.map(_asm, [s for s in SOURCES if s.endswith(".hip")]))
    _link([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC"] + objs[: len(SOURCES)], LIB)
    _link([hipcc(), "-shared", "-fPIC"] + objs[len(SOURCES):] +
          [f"-L{LIB_DIR}", "-lkvexp_hip", "-Wl,-rpath,$ORIGIN"], LIB_CXX)
    # the C++ caller: plain g++ with OpenMP against the public headers only
    _link(["g++", "-O2", "-std=c++17", "-fopenmp", "-pthread", f"-I{os.path.join(ROOT, 'include')}", CXX_TEST_SRC,
           f"-L{LIB_DIR}", "-lkvexp_hip_cxx", "-lkvexp_hip", "-Wl,-rpath,$ORIGIN"], CXX_TEST)
    return LIB


def build_trace(jobs: int = 0) -> str:
    """Compiles every kernel source with KVEXP_PHASE_TRACE into the trace library."""
    os.makedirs(TRACE_OBJ_DIR, exist_ok=True)
    os.makedirs(os.path.dirname(TRACE_LIB), exist_ok=True)
    jobs = jobs if jobs > 0 else default_jobs()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, True, trace=True), SOURCES))
    _link([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC"] + objs, TRACE_LIB)
    return TRACE_LIB


def _link(cmd: list[str], out: str) -> None:
    tmp = out + ".tmp"
    cmd = cmd + ["-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=0)
    ap.add_argument("--asm", action="store_true")
    ap.add_argument("--incremental", action="store_true", help="skip up-to-date objects")
    ap.add_argument("--trace", action="store_true", help="build the phase-trace library instead")
    a = ap.parse_args()
    if a.trace:
        print(build_trace(jobs=a.jobs))
        return 0
    print(build(force=not a.incremental, jobs=a.jobs, asm=a.asm))
    return 0


if __name__ == "__main__":
    sys.exit(main())
