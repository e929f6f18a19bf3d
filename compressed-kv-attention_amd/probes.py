"""Measurement probes behind the compute-bound evidence of the split kernel.

    python compressed-kv-attention_amd/probes.py build          # on the CPU, after build.py
    python compressed-kv-attention_amd/probes.py coexec         # GPU
    python compressed-kv-attention_amd/probes.py bf16-exact     # GPU
    python compressed-kv-attention_amd/probes.py phase-trace    # GPU (c2; phase-trace-c4: c4)
    python compressed-kv-attention_amd/probes.py encode-trace   # GPU

build        compiles csrc/probes/*.hip into lib/probes/ and a phase-traced
             copy of the library (attention_wave.hip and codec_kernels.hip with
             KVEXP_PHASE_TRACE, the other objects from build.py) as
             lib/probes/libkvexp_hip_trace.so.
coexec       cycles per wave-iteration of MFMA and vector-ALU instruction mixes
             at 2 and 4 waves per SIMD (mfma_valu_coexec.hip).
bf16-exact   whether a BF16 4x4x4 MFMA with one live K slot equals fmaf on
             the widened inputs, by input class (bf16_mfma_exact.hip).
phase-trace  c2 (48 KV heads x 7 queries, head_dim 64, 32K tokens, 64
             splits) through the traced library: cycles per wave in each
             phase of the chunk loop; phase-trace-c4 the same for c4 (256
             KV heads x 4 queries, head_dim 128, 128K tokens, 8 splits).
encode-trace the c2 prefill through the traced library: cycles per block in
             each phase of the one-pass encoder.
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE_DIR = os.path.join(HERE, "lib", "probes")
TRACE_LIB = os.path.join(PROBE_DIR, "libkvexp_hip_trace.so")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-Xclang",
         "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build() -> None:
    sys.path.insert(0, HERE)
    import build as lib_build

    hipcc = lib_build.hipcc()
    os.makedirs(PROBE_DIR, exist_ok=True)
    for name in ("mfma_valu_coexec", "bf16_mfma_exact"):
        _run([hipcc, *FLAGS, os.path.join(HERE, "csrc", "probes", name + ".hip"), "-o",
              os.path.join(PROBE_DIR, name)])
    inc = ["-I" + os.path.join(os.path.dirname(HERE), "include"), "-I" + os.path.join(HERE, "csrc", "hip")]
    traced = []
    for name in ("attention_wave", "codec_kernels"):
        obj = os.path.join(PROBE_DIR, name + "_trace.o")
        _run([hipcc, *FLAGS, "-fPIC", "-DKVEXP_PHASE_TRACE", *inc, "-x", "hip", "-c",
              os.path.join(HERE, "csrc", "hip", name + ".hip"), "-o", obj])
        traced.append(obj)
    others = [os.path.join(lib_build.OBJ_DIR, n + ".o")
              for n in ("attention_kernels.hip", "attention_wave256.hip", "kvexp_hip_api.cpp")]
    for o in others:
        if not os.path.exists(o):
            raise SystemExit(f"{o} missing: run compressed-kv-attention_amd/build.py first")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", TRACE_LIB, *others, *traced])


def coexec() -> None:
    _run([os.path.join(PROBE_DIR, "mfma_valu_coexec")])


# ---------------------------------------------------------------- bf16-exact --
CLASSES = ["normal", "cancel", "tie", "den_in", "den_prod", "den_c", "zeros", "huge", "wide_c"]
N_WAVES = 4096


def _bf16_inputs(slot: int, seed: int = 100):
    """A [waves, 64, 4] BF16 (live slot `slot`, other slots 0), B [waves, 64, 4]
    BF16 (other slots finite), C [waves, 256] FP32 laid out as the MFMA's
    accumulator (lane 4b + j, register i); one class of values per wave."""
    import numpy as np

    sys.path.insert(0, HERE)
    from kvexp_amd.synth import bf16

    def f(u16):
        return (u16.astype(np.uint32) << 16).view(np.float32)

    rng0 = np.random.default_rng(7)
    A = np.zeros((N_WAVES, 64, 4), np.uint16)
    B = bf16((rng0.standard_normal(N_WAVES * 256) * np.exp2(rng0.uniform(-4, 4, N_WAVES * 256))).astype(np.float32))
    B = B.reshape(N_WAVES, 64, 4)
    C = np.zeros((N_WAVES, 64, 4), np.float32)
    r = np.random.default_rng(seed)
    with np.errstate(over="ignore"):
        for w in range(N_WAVES):
            cl = CLASSES[w % len(CLASSES)]
            a = bf16((r.standard_normal(64) * np.exp2(r.uniform(-8, 8, 64))).astype(np.float32))
            b = bf16((r.standard_normal(64) * np.exp2(r.uniform(-8, 8, 64))).astype(np.float32))
            c = (r.standard_normal((64, 4)) * np.exp2(r.uniform(-12, 12, (64, 4)))).astype(np.float32)
            if cl == "den_in":
                m = r.random(64) < 0.5
                b[m] = r.integers(1, 128, m.sum()).astype(np.uint16) | (r.integers(0, 2, m.sum()).astype(np.uint16) << 15)
                m2 = r.random(64) < 0.3
                a[m2] = r.integers(1, 128, m2.sum()).astype(np.uint16)
                c = (c * np.float32(2.0 ** -30)).astype(np.float32)
            elif cl == "den_prod":
                a = bf16((r.standard_normal(64) * np.exp2(r.uniform(-70, -55, 64))).astype(np.float32))
                b = bf16((r.standard_normal(64) * np.exp2(r.uniform(-75, -60, 64))).astype(np.float32))
                c = np.where(r.random((64, 4)) < 0.5, 0.0, c * np.float32(2.0 ** -130)).astype(np.float32)
            elif cl == "den_c":
                c = (r.standard_normal((64, 4)) * np.float32(2.0 ** -130)).astype(np.float32)
                a = bf16((r.standard_normal(64) * np.exp2(r.uniform(-70, -60, 64))).astype(np.float32))
            elif cl == "zeros":
                a[r.random(64) < 0.3] = 0x8000
                b[r.random(64) < 0.3] = 0x0000
                a[r.random(64) < 0.2] = 0x0000
                b[r.random(64) < 0.2] = 0x8000
                z = r.random((64, 4))
                c[z < 0.3] = 0.0
                c[(z >= 0.3) & (z < 0.6)] = -0.0
            elif cl == "huge":
                a = bf16((r.standard_normal(64) * np.exp2(r.uniform(60, 70, 64))).astype(np.float32))
                b = bf16((r.standard_normal(64) * np.exp2(r.uniform(55, 66, 64))).astype(np.float32))
                c = (r.standard_normal((64, 4)) * np.float32(2.0 ** 127)).astype(np.float32)
            elif cl == "wide_c":
                c = (r.standard_normal((64, 4)) * np.exp2(r.uniform(-40, 40, (64, 4)))).astype(np.float32)
            A[w, :, slot] = a
            B[w, :, slot] = b
            if cl in ("cancel", "tie"):
                for bk in range(16):
                    for j in range(4):
                        for i in range(4):
                            p = float(f(a[4 * bk + i:4 * bk + i + 1])[0]) * float(f(b[4 * bk + j:4 * bk + j + 1])[0])
                            if cl == "cancel":
                                cc = np.float32(-p) + np.float32(r.integers(-3, 4)) * np.spacing(np.float32(abs(p)))
                            elif p == 0:
                                cc = np.float32(1.0)
                            else:  # ulp(c) = 2 |p|: c + p is a tie
                                e = np.floor(np.log2(abs(p))) + 24
                                cc = np.float32((1 + r.integers(0, 2 ** 20) * 2.0 ** -23) * 2.0 ** e)
                                cc = cc * np.float32(np.sign(r.standard_normal()))
                            C[w, 4 * bk + j, i] = cc
            else:
                C[w] = c
    return A, B, C.reshape(N_WAVES, 256)


def bf16_exact() -> None:
    import numpy as np

    exe = os.path.join(PROBE_DIR, "bf16_mfma_exact")
    with tempfile.TemporaryDirectory() as d:
        for slot in range(4):
            A, B, C = _bf16_inputs(slot)
            A.tofile(os.path.join(d, "a.bin"))
            B.tofile(os.path.join(d, "b.bin"))
            C.tofile(os.path.join(d, "c.bin"))
            _run([exe, d, str(N_WAVES), str(slot)])
            m = np.fromfile(os.path.join(d, "mfma.bin"), np.uint32).reshape(N_WAVES, 256)
            r = np.fromfile(os.path.join(d, "ref.bin"), np.uint32).reshape(N_WAVES, 256)
            for k, cl in enumerate(CLASSES):
                ws = np.arange(k, N_WAVES, len(CLASSES))
                fm, fr = m[ws].view(np.float32), r[ws].view(np.float32)
                bad = (m[ws] != r[ws]) & ~(np.isnan(fm) & np.isnan(fr))
                line = f"slot {slot} {cl:9s}: {int(bad.sum()):6d} of {bad.size} results differ from fmaf"
                if bad.any():
                    wi, e = np.argwhere(bad)[0]
                    line += f" (e.g. mfma {m[ws][wi, e]:08x}, fmaf {r[ws][wi, e]:08x})"
                print(line, flush=True)


def phase_trace(config: str = "c2") -> None:
    import ctypes as C

    import numpy as np

    os.environ["KVEXP_HIP_LIBRARY"] = TRACE_LIB
    sys.path.insert(0, HERE)
    import torch

    import kvexp_amd
    from kvexp_amd import synth

    L = kvexp_amd.lib()
    cfg = synth.CONFIGS[config]
    S, D, G, BT = cfg["seq"], cfg["dim"], cfg["group"], cfg["block"]
    ctx = kvexp_amd.Context(0)
    dev = torch.device("cuda:0")
    heads = []
    if config == "c2":
        splits = 64
        for layer in range(24):
            for h in range(2):
                k, v = synth.head_kv("c2", S, 0, layer, h)
                kx = ctx.encode(torch.from_numpy(k.view(np.int16)).to(dev), S, D, BT)
                vx = ctx.encode(torch.from_numpy(v.view(np.int16)).to(dev), S, D, BT)
                heads.append(dict(kx=kx, vx=vx, seq=S, splits=splits))
    else:  # c4: K and V from torch's generator on the GPU, as bench.py --config c4
        splits = 8
        g = torch.Generator(device=dev)
        g.manual_seed(cfg["seed"])
        for _ in range(cfg["layers"] * cfg["kv_heads"]):
            scale = torch.exp2(torch.rand(D, generator=g, device=dev) * 8 - 5)
            k = (torch.randn(S, D, generator=g, device=dev) * scale).to(torch.bfloat16).view(torch.int16).reshape(-1)
            v = (torch.randn(S, D, generator=g, device=dev) * 0.5).to(torch.bfloat16).view(torch.int16).reshape(-1)
            heads.append(dict(kx=ctx.encode(k, S, D, BT), vx=ctx.encode(v, S, D, BT), seq=S, splits=splits))
    n_heads = len(heads)
    q = torch.randn(n_heads * G * D, device=dev).to(torch.bfloat16).view(torch.int16)
    plan = ctx.plan(heads, G, D, BT)
    for _ in range(100 if config == "c2" else 10):
        plan.run(q)
    torch.cuda.synchronize()
    nph = 12
    buf = np.zeros(8192 * (nph + 3), dtype=np.uint64)
    L.kvexp_hip_phase_trace_read.argtypes = [C.c_void_p, C.c_size_t]
    kvexp_amd.check(L.kvexp_hip_phase_trace_read(buf.ctypes.data_as(C.c_void_p), buf.size))
    t = buf.reshape(8192, nph + 3)[: n_heads * splits].astype(np.int64)
    life = t[:, 1] - t[:, 0]
    ph = t[:, 2:2 + nph]
    names = ["K rows wait", "K decode + escapes", "scores", "softmax coefficients", "V rows wait", "V decode",
             "V escapes", "next K block entered", "next K rows requested", "next V block entered",
             "next V rows requested", "fold"]
    chunks = S // splits // 64  # chunks per wave
    print(f"{config}, {splits} splits: {len(t)} waves of {chunks} chunks; wave life: mean {life.mean():.0f} cycles "
          f"(min {life.min()}, max {life.max()})")
    for i, n in enumerate(names):
        print(f"  {n:32s} {ph[:, i].mean():9.0f} cycles/wave ({100 * ph[:, i].mean() / life.mean():5.1f} %), "
              f"{ph[:, i].mean() / chunks:6.0f} per chunk")
    print(f"  {'outside the chunk loop':32s} {(life - ph.sum(1)).mean():9.0f} cycles/wave")


def encode_trace() -> None:
    """The c2 prefill (96 containers from empty to 32,768 tokens in one
    kvexp_hip_append_batch call: 24,576 blocks) through the traced library:
    cycles per block in each phase of the one-pass encoder."""
    import ctypes as C

    import numpy as np

    os.environ["KVEXP_HIP_LIBRARY"] = TRACE_LIB
    sys.path.insert(0, HERE)
    import torch

    import kvexp_amd
    from kvexp_amd import synth

    L = kvexp_amd.lib()
    cfg = synth.CONFIGS["c2"]
    S, D, BT = cfg["seq"], cfg["dim"], cfg["block"]
    ctx = kvexp_amd.Context(0)
    dev = torch.device("cuda:0")
    src = []
    for layer in range(cfg["layers"]):
        for h in range(cfg["kv_heads"]):
            for x in synth.head_kv("c2", S, 0, layer, h):
                src.append(torch.from_numpy(x.view(np.int16)).to(dev))
    caches = [ctx.cache(D, S, BT) for _ in src]
    for _ in range(5):
        for c in caches:
            c.seq = 0
        ctx.append_batch(caches, src, S)
    torch.cuda.synchronize()
    nb = len(src) * (S // BT)
    buf = np.zeros(32768 * 12, dtype=np.uint64)
    L.kvexp_hip_encode_trace_read.argtypes = [C.c_void_p, C.c_size_t]
    kvexp_amd.check(L.kvexp_hip_encode_trace_read(buf.ctypes.data_as(C.c_void_p), buf.size))
    t = buf.reshape(32768, 12)[:nb].astype(np.int64)
    life = t[:, 8] - t[:, 0]
    names = ["job + ticket", "(none)", "tokens arrive", "histograms", "window bases + mode", "codes + escape ranks",
             "look-back", "stores issued"]
    print(f"c2 prefill: {nb} blocks; block life mean {life.mean():.0f} cycles "
          f"(min {life.min()}, max {life.max()})")
    for i, n in enumerate(names):
        d = t[:, i + 1] - t[:, i]
        print(f"  {n:22s} {d.mean():8.0f} cycles/block ({100 * d.mean() / life.mean():5.1f} %), "
              f"p50 {np.percentile(d, 50):7.0f}, p99 {np.percentile(d, 99):7.0f}")
    polls = t[:, 9]
    print(f"  look-back waits: {np.mean(polls > 0) * 100:.1f} % of blocks polled again; mean {polls.mean():.2f}, "
          f"max {polls.max()}")
    blocks_per_job = S // BT
    b = np.arange(nb) % blocks_per_job
    same = np.mean(t[:, 11] == b)
    near = np.mean(np.abs(t[:, 11] - b) <= 8)
    print(f"  ticket equals blockIdx.x for {same * 100:.1f} % of blocks ({near * 100:.1f} % within 8)")


if __name__ == "__main__":
    cmds = {"build": build, "coexec": coexec, "bf16-exact": bf16_exact, "phase-trace": phase_trace,
            "phase-trace-c4": lambda: phase_trace("c4"), "encode-trace": encode_trace}
    if len(sys.argv) != 2 or sys.argv[1] not in cmds:
        raise SystemExit(__doc__)
    cmds[sys.argv[1]]()
