"""kvexp::detect_cpu of the C++ drop-in (libkvexp_hip_cxx.so) against the
reference's own detect_cpu (src/cpu.cpp:35-61, compiled into oracle/_ref) on
this host, and against the kernel's CPU flags (/proc/cpuinfo lists avx2 and
the AVX-512 sets only where the OS saves their state)."""
import ctypes as C
import os

import pytest

import kvexp_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref", "libkvexp_ref.so")


class CpuFeatures(C.Structure):
    # include/kvexp/attention.hpp: struct CpuFeatures { bool avx2; bool avx512_bf16; }
    _fields_ = [("avx2", C.c_bool), ("avx512_bf16", C.c_bool)]


def _ours():
    kvexp_amd.lib()  # loads libkvexp_hip.so, which the C++ library links
    cxx = C.CDLL(os.path.join(os.path.dirname(kvexp_amd.LIB_PATH), "libkvexp_hip_cxx.so"))
    fn = getattr(cxx, "_ZN5kvexp10detect_cpuEv")
    fn.restype = CpuFeatures
    f = fn()
    return bool(f.avx2), bool(f.avx512_bf16)


def _cpuinfo_flags():
    with open("/proc/cpuinfo") as fh:
        for line in fh:
            if line.startswith("flags"):
                return set(line.split(":", 1)[1].split())
    return set()


@pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref not built")
def test_detect_cpu_equals_reference():
    ref = C.CDLL(REF)
    a, b = C.c_int(-1), C.c_int(-1)
    assert ref.kvexp_ref_detect_cpu(C.byref(a), C.byref(b)) == 0
    assert _ours() == (bool(a.value), bool(b.value))


@pytest.mark.skipif(not os.path.exists("/proc/cpuinfo"), reason="no /proc/cpuinfo")
def test_detect_cpu_matches_kernel_flags():
    fl = _cpuinfo_flags()
    want = ("avx2" in fl, {"avx512f", "avx512bw", "avx512vl", "avx512_bf16"} <= fl)
    assert _ours() == want
