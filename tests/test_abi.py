"""CPU checks of the C ABI library (no GPU needed): it loads, exports every
symbol include/kvexp_hip.h declares, and its host-side logic (size model,
block walk and its error messages) agrees with the oracle and the reference."""
import ctypes as C
import os

import numpy as np
import pytest

from kvdata import random_kv

amd = pytest.importorskip("kvexp_amd")


def test_library_exports_every_declared_symbol():
    L = amd.lib()
    names = amd.declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_cpp_api_symbols_exported():
    """The C++ API lives in libkvexp_hip_cxx.so; libkvexp_hip.so exports C
    symbols only, so it links beside the reference library (whose kvexp::
    symbols the C++ API mirrors) without a clash."""
    cxx = os.path.join(os.path.dirname(amd.LIB_PATH), "libkvexp_hip_cxx.so")
    out = os.popen(f"nm -D --defined-only {cxx}").read()
    for sym in ("_ZN5kvexp16attention_decode", "_ZN5kvexp11encode_bf16", "_ZN5kvexp11decode_bf16",
                "_ZN5kvexp10detect_cpuEv", "_ZN5kvexp10set_device"):
        assert sym in out, sym
    c_only = os.popen(f"nm -D --defined-only {amd.LIB_PATH}").read()
    assert "_ZN5kvexp" not in c_only
    assert "kvexp_hip_attention_decode_host" in c_only


def test_status_strings():
    L = amd.lib()
    for code in range(7):
        assert L.kvexp_hip_status_string(code)
    assert b"gfx950" in L.kvexp_hip_version()


def test_size_model_matches_oracle(oracle):
    L = amd.lib()
    rng = np.random.default_rng(0)
    for _ in range(200):
        n, dim = int(rng.integers(1, 256)), 4 * int(rng.integers(1, 65))
        bits, esc = int(rng.choice([2, 4])), int(rng.integers(0, 100))
        assert L.kvexp_hip_exp_payload_bytes(n, dim, bits) == oracle.exp_payload_bytes(n, dim, bits)
        assert L.kvexp_hip_coded_block_bytes(n, dim, bits, esc) == oracle.coded_block_bytes(n, dim, bits, esc)
        assert L.kvexp_hip_raw_block_bytes(n, dim) == oracle.raw_block_bytes(n, dim)
        seq, block = int(rng.integers(1, 10000)), int(rng.integers(1, 256))
        assert amd.encode_bound(seq, dim, block) == oracle.encode_bound(seq, dim, block)


def test_build_index_matches_oracle(oracle, golden):
    z, man = golden
    for c in man["codec"]:
        blob = z[f"codec/{c['name']}/blob"]
        for seq in (c["seq"], max(1, c["seq"] // 2)):
            off, first = amd.build_index(blob, c["dim"], seq)
            o2, f2 = oracle.block_index(blob, c["dim"], seq)
            assert np.array_equal(off, o2) and np.array_equal(first, f2), c["name"]


def test_build_index_errors_match_reference_messages(oracle):
    rng = np.random.default_rng(6)
    kv = random_kv(rng, 300, 64)
    blob = oracle.encode(kv, 300, 64, 128)
    bad_mode = blob.copy()
    bad_mode[0] = 1  # 3 is the 3-bit extension (dim % 8 == 0), which this library reads
    zero_tok = blob.copy()
    zero_tok[1] = 0
    cases = [(blob[:5], 64, "truncated xkv block header"), (blob[:-3], 64, "truncated coded xkv block"),
             (bad_mode, 64, "unknown xkv block mode"), (blob, 32, "xkv block dimension or length mismatch"),
             (zero_tok, 64, "xkv block dimension or length mismatch")]
    for b, dim, msg in cases:
        with pytest.raises(amd.KvexpHipError) as ei:
            amd.build_index(b, dim, 300)
        assert ei.value.kind == "runtime_error" and ei.value.msg == msg
        # the oracle (restating scan.hpp) reports the same for a decode of the same bytes
        from oracle import KvexpError

        with pytest.raises(KvexpError) as e2:
            oracle.decode(b, 300, dim)
        assert e2.value.msg == msg


def test_context_without_gpu_fails_cleanly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = amd.lib()
    h = C.c_void_p()
    rc = L.kvexp_hip_ctx_create(0, C.byref(h))
    assert rc != 0 and not h.value
    assert L.kvexp_hip_last_error()


def test_null_arguments_rejected():
    L = amd.lib()
    nb = C.c_int(0)
    assert L.kvexp_hip_build_index(None, 10, 64, 10, None, None, 4, C.byref(nb)) == 1
    p = C.c_void_p()
    assert L.kvexp_hip_plan_create(None, None, 0, 1, 64, 128, 0, None, C.byref(p)) == 1
    assert b"bad argument" in L.kvexp_hip_last_error()
    n = C.c_size_t(0)
    assert L.kvexp_hip_append(None, None, 1, 0, 64, 128, None, None, 0, None, None, 0, C.byref(n), None) == 1
    assert b"null context" in L.kvexp_hip_last_error()
