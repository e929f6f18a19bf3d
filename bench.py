"""Benchmark of the fused compressed-KV decode step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c2] [--gpus 1]
    python bench.py --workload append [--steps K] [--warmup W]
    python bench.py --workload dump --kvd FILE.kvd --qsnap FILE.qsnap [--lengths 4096,32768]

Workload ("c2"): a full Qwen2.5-0.5B decode step at a
32K context: 24 layers x 2 KV heads, 7 queries per KV head (GQA), head_dim 64,
seq 32768, XKV containers with 128-token blocks, seeded synthetic K/V/Q
(kvexp_amd/synth.py). One step = the fused attention over all 48 KV heads
(split kernel + ordered merge), inputs resident in HBM.

Before timing, the XKV step's output is compared bit for bit with the raw
BF16 step's (same kernel order), as the reference bench memcmps raw vs XKV.
Each timed step reads a different copy of the containers (--copies, default 4,
1.2 GB in total) so consecutive steps cannot be served from the 256 MB
Infinity Cache.

Prints one JSON line. value = container bytes per step / seconds per step
(GB/s, 1e9), the step being all kernels of one run (q widening, split
kernel, merge). roofline.achieved = algorithmic bytes of one split-kernel
launch (all K/V container bytes + Q + output) / that kernel's average
duration, measured with HIP events the library records around the split
kernel on the run's stream (kvexp_hip_plan_timing). roofline.traffic = HBM
bytes per launch from the committed counter summary
profiles/attn_wave_c2_traffic.md (null when absent). cpu_baseline = the
reference library (oracle/_ref, compiled from the reference sources) running
its model_heads scope (OpenMP over KV heads, AVX-512 BF16 when the host has
it, else AVX2) on a bounded sample of the same step.

--workload append measures the producer side on the same c2 shape: the
96 K/V containers (48 KV heads) grown on the device by kvexp_hip_append_batch.
value = decode-step append time (one new token per container, one batched
call) in µs; the line also carries the prefill rate (32768 tokens into every
container in one call, GB/s of BF16 input) with its HBM roofline, and the
reference's encode_bf16 on the host as the CPU baseline. Containers are
checked byte for byte against kvexp_hip_encode of the same tokens.

--config c1 | c3 | c4 | c5 measures the other configurations of BASELINE.json
(parity cases, not the quoted line), one JSON line each: c1 (one KV head,
seq 8192, one query; L2-resident, reported in µs), c3 (the ragged batch:
32 sequences x 48 KV heads, split count from kvexp_hip_suggest_splits_batch),
c4 (256 KV heads x seq 131072, head_dim 128, 4 queries; K and V generated
on the GPU with the config's distributions, torch's RNG, since the host
generator would take minutes) and c5 (batch 4 x 8 KV heads x seq 100003,
head_dim 256, 255-token blocks, 8 queries). c1, c3 and c5 use the host
generator (kvexp_amd/synth.py). XKV is checked bit for bit against raw
before timing; each line carries the split kernel's HBM roofline.

--phase-trace (after `build.py --trace`) loads the trace build of the
library and prints, instead of a bench line, where the split kernel's waves
spend their cycles (c2 or --config c4: cycles per wave in each phase of the
chunk loop) or, with --workload append, where the one-pass encoder's blocks
spend theirs during the c2 prefill. Its kernels record clock stamps, so its
times are not the library's.

--workload dump runs the reference bench's model scope on a real KV dump
(KVD1 + QSN1 files written by the reference's python/dump_kv.py): every
layer and KV head at each snapshot length, XKV checked bit for bit against
raw BF16 before timing; one JSON line with a row per length.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "compressed-kv-attention_amd"))

HBM_PEAK_GBPS = 8000.0
METRIC = "decode-step µs + achieved HBM GB/s (% peak), Qwen2.5-0.5B shape, 32K ctx"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def measured_traffic(profile: str = "attn_wave_c2_traffic.md"):
    """HBM bytes per launch of a kernel from its committed counter summary
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by a plain copy kernel of
    known size): the split kernel's by default. None when there is none."""
    path = os.path.join(ROOT, "profiles", profile)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def copy_probe(torch, dev):
    """Three device-to-device copies of 256 MiB: the known-size kernel the
    FETCH_SIZE / WRITE_SIZE counters are scaled by."""
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy probe: 3 copies of {n} bytes")


def bench_append(a, torch, np, kvexp_amd, synth) -> int:
    cfg = synth.CONFIGS["c2"]
    L, KV, D, S, BT = cfg["layers"], cfg["kv_heads"], cfg["dim"], cfg["seq"], cfg["block"]
    T = 2 * L * KV  # K and V containers
    dev = torch.device("cuda:0")
    ctx = kvexp_amd.Context(0)
    if a.copy_probe:
        copy_probe(torch, dev)
    steps, warmup = a.steps, a.warmup
    extra = 4 * steps + warmup + 1  # warmup + timed append steps, then the three decode loops
    t0 = time.time()
    src, host = [], []
    for l in range(L):
        for h in range(KV):
            k, v = synth.head_kv("c2", S + extra, 0, l, h)
            for x in (k, v):
                src.append(torch.from_numpy(x.view(np.int16)).to(dev))
                if len(host) < 16:
                    host.append(x)
    caches = [ctx.cache(D, S + extra, BT) for _ in range(T)]
    torch.cuda.synchronize()
    log(f"append inputs ready in {time.time() - t0:.1f}s: {T} containers")

    # prefill: every container from empty to S tokens in one call (the
    # calls rewrite the same buffers: each starts from n_tokens = 0)
    pre = [t[: S * D] for t in src]

    def prefill():
        for c in caches:
            c.seq = 0
        ctx.append_batch(caches, pre, S)

    for _ in range(2):
        prefill()
    torch.cuda.synchronize()
    # calls back to back between two HIP events on the stream
    n_pre = max(3, min(20, steps // 10))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n_pre):
        prefill()
    e1.record()
    torch.cuda.synchronize()
    pre_ms = e0.elapsed_time(e1) / n_pre
    container = sum(c.size() for c in caches)
    raw_bytes = 2 * S * D * T
    pre_gbps = raw_bytes / (pre_ms * 1e-3) / 1e9
    algo = raw_bytes + container  # read the tokens once, write the containers
    log(f"prefill {pre_ms * 1e3:.1f} us for {T} x {S} tokens: {pre_gbps:.1f} GB/s of input, "
        f"containers {container} B")

    # decode steps: one token per container per call, the step's tokens as
    # one [containers, 1, dim] tensor (as a model's K/V projections give them)
    one = torch.stack([t.view(-1, D)[S:S + extra] for t in src], dim=1).contiguous()  # [extra, T, D]
    aset = ctx.append_set(caches)
    for i in range(warmup):
        aset.append(one[i], 1)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    e0.record()
    for i in range(warmup, warmup + steps):
        aset.append(one[i], 1)
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t_start) * 1e3 / steps
    step_ms = e0.elapsed_time(e1) / steps
    n_tok = S + warmup + steps
    # parity: every container equals the GPU encoder's output for the same tokens
    same = True
    for c, t in zip(caches, src):
        enc = ctx.encode(t[: n_tok * D], n_tok, D, BT)
        n = c.size()
        same &= n == enc.nbytes and bool(torch.equal(c.blob[:n], enc.blob[:n]))
    log(f"decode-step append {step_ms * 1e3:.1f} us (wall {wall_ms * 1e3:.1f}), containers equal encode: {same}")
    # attention over the grown containers: a plan is built per step in a
    # decode loop; its creation time, and the output against a plan over
    # freshly encoded copies of the same tokens
    G = cfg["group"]
    H = L * KV
    q = torch.from_numpy(synth.queries("c2", H).view(np.int16)).to(dev)
    splits = ctx.suggest_splits(H, n_tok, BT)
    views = [c.view() for c in caches]
    torch.cuda.synchronize()
    t_plan = time.perf_counter()
    plan = ctx.plan([dict(kx=views[2 * i], vx=views[2 * i + 1], seq=n_tok, splits=splits) for i in range(H)], G, D,
                    BT)
    plan_ms = (time.perf_counter() - t_plan) * 1e3
    encs = [ctx.encode(t[: n_tok * D], n_tok, D, BT) for t in src]
    plan2 = ctx.plan([dict(kx=encs[2 * i], vx=encs[2 * i + 1], seq=n_tok, splits=splits) for i in range(H)], G, D,
                     BT)
    o1 = plan.run(q, check_errors=True)
    o2 = plan2.run(q, check_errors=True)
    torch.cuda.synchronize()
    attn_same = bool(torch.equal(o1.view(torch.int32), o2.view(torch.int32)))
    log(f"plan over appended containers: created in {plan_ms:.2f} ms; attention equals fresh encode: {attn_same}")

    # decode loop: append one token to every container, re-target the plan,
    # run the attention (the plan update is the fast path inside a block and
    # a rebuild when a block starts)
    def heads_at(seq):
        out = []
        for i in range(H):
            kx, vx = caches[2 * i].view(), caches[2 * i + 1].view()
            kx.nbytes = vx.nbytes = -1  # capacity stands in for the size
            out.append(dict(kx=kx, vx=vx, seq=seq, splits=splits))
        return out

    loop_steps = min(steps, extra - warmup - steps - 1)
    out = torch.empty(H * G * D, dtype=torch.float32, device=dev)
    base = warmup + steps
    plan.update(heads_at(S + base))  # byte counts become the capacities; then lengths only
    torch.cuda.synchronize()
    t_loop = time.perf_counter()
    e0.record()
    for i in range(base, base + loop_steps):
        aset.append(one[i], 1)
        plan.update_lengths(S + i + 1, BT)
        plan.run(q, out)
    e1.record()
    torch.cuda.synchronize()
    loop_ms = e0.elapsed_time(e1) / max(1, loop_steps)
    loop_wall = (time.perf_counter() - t_loop) * 1e3 / max(1, loop_steps)
    n_end = S + base + loop_steps
    fresh = [ctx.encode(t[: n_end * D], n_end, D, BT) for t in src]
    plan3 = ctx.plan([dict(kx=fresh[2 * i], vx=fresh[2 * i + 1], seq=n_end, splits=splits) for i in range(H)], G, D,
                     BT)
    o3 = plan3.run(q, check_errors=True)
    plan.status()
    torch.cuda.synchronize()
    loop_same = bool(torch.equal(out.view(torch.int32), o3.view(torch.int32)))
    log(f"decode loop (append + plan update + attention): {loop_ms * 1e3:.1f} us per step (wall "
        f"{loop_wall * 1e3:.1f}) over {loop_steps} steps; last output equals fresh plan: {loop_same}")

    # the same loop through the PyTorch operator (torch.ops.kvexp.decode_attention,
    # reuse_plan=True: the op keeps the plan for these buffers and re-targets it)
    import kvexp_amd.torch_ops as ops

    dq3 = q.view(torch.bfloat16).view(H, G, D)
    base2 = base + loop_steps
    op_steps = loop_steps
    seq_now = S + base2
    kviews = [caches[2 * i].view() for i in range(H)]
    vviews = [caches[2 * i + 1].view() for i in range(H)]
    for e in kviews + vviews:
        e.nbytes = -1
    o_op = ops.decode_attention_containers(dq3, kviews, vviews, [seq_now] * H, splits, BT, 0, reuse_plan=True)
    torch.cuda.synchronize()
    t_op = time.perf_counter()
    e0.record()
    for i in range(base2, base2 + op_steps):
        aset.append(one[i], 1)
        seq_now = S + i + 1
        kviews = [caches[2 * j].view() for j in range(H)]
        vviews = [caches[2 * j + 1].view() for j in range(H)]
        for e in kviews + vviews:
            e.nbytes = -1
        o_op = ops.decode_attention_containers(dq3, kviews, vviews, [seq_now] * H, splits, BT, 0, reuse_plan=True)
    e1.record()
    torch.cuda.synchronize()
    op_ms = e0.elapsed_time(e1) / max(1, op_steps)
    op_wall = (time.perf_counter() - t_op) * 1e3 / max(1, op_steps)
    fresh2 = [ctx.encode(t[: seq_now * D], seq_now, D, BT) for t in src]
    plan4 = ctx.plan([dict(kx=fresh2[2 * i], vx=fresh2[2 * i + 1], seq=seq_now, splits=splits) for i in range(H)],
                     G, D, BT)
    o4 = plan4.run(q, check_errors=True)
    torch.cuda.synchronize()
    op_same = bool(torch.equal(o_op.reshape(-1).view(torch.int32), o4.view(torch.int32)))
    ops.clear_plan_cache()
    # and through decode_attention_kv over the caches registered once (only the
    # lengths cross the op each step)
    handle = ops.register_kv([caches[2 * i] for i in range(H)], [caches[2 * i + 1] for i in range(H)], G, D, splits,
                             BT, 0)
    base3 = base2 + op_steps
    seq_now = S + base3
    o_kv = torch.ops.kvexp.decode_attention_kv(dq3, handle, [seq_now] * H)
    torch.cuda.synchronize()
    t_kv = time.perf_counter()
    e0.record()
    for i in range(base3, base3 + op_steps):
        aset.append(one[i], 1)
        seq_now = S + i + 1
        o_kv = torch.ops.kvexp.decode_attention_kv(dq3, handle, [seq_now] * H)
    e1.record()
    torch.cuda.synchronize()
    kv_ms = e0.elapsed_time(e1) / max(1, op_steps)
    kv_wall = (time.perf_counter() - t_kv) * 1e3 / max(1, op_steps)
    fresh3 = [ctx.encode(t[: seq_now * D], seq_now, D, BT) for t in src]
    plan5 = ctx.plan([dict(kx=fresh3[2 * i], vx=fresh3[2 * i + 1], seq=seq_now, splits=splits) for i in range(H)],
                     G, D, BT)
    o5 = plan5.run(q, check_errors=True)
    torch.cuda.synchronize()
    kv_same = bool(torch.equal(o_kv.reshape(-1).view(torch.int32), o5.view(torch.int32)))
    ops.unregister_kv(handle)
    log(f"decode loop through torch.ops.kvexp.decode_attention (append + op): {op_ms * 1e3:.1f} us per step "
        f"(wall {op_wall * 1e3:.1f}) over {op_steps} steps; last output equals fresh plan: {op_same}")
    log(f"decode loop through torch.ops.kvexp.decode_attention_kv (append + op on registered caches): "
        f"{kv_ms * 1e3:.1f} us per step (wall {kv_wall * 1e3:.1f}); last output equals fresh plan: {kv_same}")

    cpu = None
    if not a.no_cpu_baseline:
        try:
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            from oracle import Reference

            R = Reference()
            times = []
            budget = time.perf_counter()
            while len(times) < 2 or (time.perf_counter() - budget < 15.0 and len(times) < 10):
                t1 = time.perf_counter()
                for x in host:
                    R.encode(x[: S * D], S, D, BT)
                times.append(time.perf_counter() - t1)
            med = float(np.median(times))
            cpu = {"value": round(len(host) * 2 * S * D / med / 1e9, 4), "unit": "GB/s", "cores": 1,
                   "kind": "reference",
                   "sample": f"encode_bf16 of {len(host)} of the {T} c2 tensors ({S} tokens each), one thread, "
                             f"median of {len(times)} runs ({med * 1e3:.1f} ms)"}
            log("cpu baseline", cpu)
        except FileNotFoundError:
            cpu = {"value": None, "unit": "GB/s", "cores": 0, "kind": "reference",
                   "sample": "oracle/_ref/libkvexp_ref.so not present on this host"}
    line = {
        "metric": "decode-step append µs (one token into each of 96 K/V containers), Qwen2.5-0.5B shape, 32K ctx",
        "value": round(step_ms * 1e3, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded, kvexp_amd/synth.py config c2)",
        "config": {"workload": "append: 48 KV heads x (K, V), head_dim 64, 128-token blocks, containers at 32K "
                               "tokens", "containers": T, "dim": D, "block": BT, "seq": S},
        "wall_us_per_step": round(wall_ms * 1e3, 2),
        "prefill": {"us": round(pre_ms * 1e3, 2), "tokens_per_container": S, "input_GBps": round(pre_gbps, 2)},
        "containers_equal_encode": same,
        "plan_create_ms": round(plan_ms, 3),
        "decode_loop_us_per_step": round(loop_ms * 1e3, 2),
        "decode_loop_wall_us_per_step": round(loop_wall * 1e3, 2),
        "decode_loop_equal_fresh_plan": loop_same,
        "op_decode_loop_us_per_step": round(op_ms * 1e3, 2),
        "op_decode_loop_wall_us_per_step": round(op_wall * 1e3, 2),
        "op_decode_loop_equal_fresh_plan": op_same,
        "op_kv_decode_loop_us_per_step": round(kv_ms * 1e3, 2),
        "op_kv_decode_loop_wall_us_per_step": round(kv_wall * 1e3, 2),
        "op_kv_decode_loop_equal_fresh_plan": kv_same,
        "attention_equal_fresh_encode": attn_same,
        "roofline": {"bound": "hbm", "achieved": round(algo / (pre_ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(algo / (pre_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic("encode_fused_c2_prefill.md"),
                     "kernel": "prefill append (job-table copy + one-pass encoder + tail launches)",
                     "algorithmic_bytes": algo},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def host_info() -> dict:
    """Logical CPUs, sockets, physical cores, the AVX512_BF16 flag and the
    last-level cache of this host (Linux /proc and /sys)."""
    info = {"nproc": os.cpu_count() or 1, "sockets": None, "physical_cores": None, "avx512_bf16": None,
            "avx2": None, "model": None, "llc_bytes": None}
    try:
        cores, sockets, flags = set(), set(), ""
        phys = core = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "physical id":
                phys = v
                sockets.add(v)
            elif k == "core id":
                core = v
            elif k == "flags" and not flags:
                flags = v
            elif k == "model name" and info["model"] is None:
                info["model"] = v
            elif not k and phys is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None:
            cores.add((phys, core))
        info["sockets"] = len(sockets) or None
        info["physical_cores"] = len(cores) or None
        fl = set(flags.split())
        info["avx512_bf16"], info["avx2"] = "avx512_bf16" in fl, "avx2" in fl
    except OSError:
        pass
    try:  # sum of the distinct level-3 caches
        seen, total = set(), 0
        base = "/sys/devices/system/cpu"
        for cpu in os.listdir(base):
            d = os.path.join(base, cpu, "cache", "index3")
            if not cpu.startswith("cpu") or not os.path.isdir(d):
                continue
            shared = open(os.path.join(d, "shared_cpu_list")).read().strip()
            if shared in seen:
                continue
            seen.add(shared)
            size = open(os.path.join(d, "size")).read().strip().upper()
            mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(size[-1], 1)
            total += int(size.rstrip("KMG")) * mult
        info["llc_bytes"] = total or None
    except OSError:
        pass
    return info


def cpu_baseline_c2(R, np, a, q, ks, vs, kxs, vxs, G, D, S, BT) -> dict:
    """The reference's own library (oracle/_ref) on this host, as its bench times
    it (bench.cpp:189-218, 644-646, 711-728): every ISA the host has (AVX-512
    BF16, AVX2), two scopes (model_heads: OpenMP over all KV heads of the step,
    one thread each; head: KV head 0, sequence-parallel over the threads), raw
    and XKV inputs whose outputs are compared bit for bit first, 2 untimed
    calls, then the median of >= 5 samples, each after a sweep of a host buffer
    of >= 2x the last-level cache (cold)."""
    host = host_info()
    phys = host["physical_cores"] or host["nproc"]
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)  # the box's CPU share, when set
    threads = a.cpu_threads or (min(phys, share) if share > 0 else phys)
    sweep_bytes = max(2 * (host["llc_bytes"] or 0), 1 << 30)
    sweep = np.zeros(sweep_bytes // 8, dtype=np.uint64)

    def cold():
        np.add(sweep, 1, out=sweep)

    def timed_cold(fn, n=5):
        fn()
        fn()
        ts = []
        for _ in range(n):
            cold()
            t1 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t1)
        return float(np.median(ts))

    H = len(ks)
    container = sum(x.size for x in kxs) + sum(x.size for x in vxs)
    tight = sum(x.size * 2 for x in ks) + sum(x.size * 2 for x in vs)
    head_c = kxs[0].size + vxs[0].size
    lines = []
    isas = [i for i in ("avx512", "avx2") if R.has(i)] or ["scalar"]
    for isa in isas:
        ox = R.attention_heads(isa, q, kxs, vxs, xkv=True, n_q=G, dim=D, seq=S, split=BT, omp_threads=threads)
        orw = R.attention_heads(isa, q, ks, vs, xkv=False, n_q=G, dim=D, seq=S, split=BT, omp_threads=threads)
        same = bool(np.array_equal(ox.view(np.uint32), orw.view(np.uint32)))
        tx = timed_cold(lambda: R.attention_heads(isa, q, kxs, vxs, xkv=True, n_q=G, dim=D, seq=S, split=BT,
                                                  omp_threads=threads))
        tr = timed_cold(lambda: R.attention_heads(isa, q, ks, vs, xkv=False, n_q=G, dim=D, seq=S, split=BT,
                                                  omp_threads=threads))
        lines.append({"isa": isa, "scope": "model_heads", "threads": threads, "heads": H,
                      "xkv_ms": round(tx * 1e3, 3), "raw_ms": round(tr * 1e3, 3),
                      "xkv_GBps": round(container / tx / 1e9, 3), "raw_GBps_tight": round(tight / tr / 1e9, 3),
                      "xkv_over_raw": round(tx / tr, 4), "raw_equal_xkv": same})
        q0 = q[: G * D]
        hx = R.attention(isa, q0, kx=kxs[0], vx=vxs[0], n_q=G, dim=D, seq=S, threads=threads, split=BT)
        hr = R.attention(isa, q0, k=ks[0], v=vs[0], n_q=G, dim=D, seq=S, threads=threads, split=BT)
        hsame = bool(np.array_equal(hx.view(np.uint32), hr.view(np.uint32)))
        thx = timed_cold(lambda: R.attention(isa, q0, kx=kxs[0], vx=vxs[0], n_q=G, dim=D, seq=S, threads=threads,
                                             split=BT))
        thr = timed_cold(lambda: R.attention(isa, q0, k=ks[0], v=vs[0], n_q=G, dim=D, seq=S, threads=threads,
                                             split=BT))
        lines.append({"isa": isa, "scope": "head", "threads": threads, "heads": 1,
                      "xkv_ms": round(thx * 1e3, 3), "raw_ms": round(thr * 1e3, 3),
                      "xkv_GBps": round(head_c / thx / 1e9, 3), "xkv_over_raw": round(thx / thr, 4),
                      "raw_equal_xkv": hsame})
    main = lines[0]
    return {"value": main["xkv_GBps"], "unit": "GB/s", "cores": threads, "kind": "reference",
            "sample": f"the whole c2 step on the host: all {H} KV heads x {G} queries, seq {S}, XKV, "
                      f"{main['isa']} backend, OpenMP over heads with one thread each (bench.cpp model_heads), "
                      f"{threads} threads; cold median of 5 after 2 untimed calls, a {sweep_bytes >> 20} MiB "
                      f"host sweep before each sample; {main['xkv_ms']:.1f} ms per step "
                      f"(raw {main['raw_ms']:.1f} ms, raw == XKV: {main['raw_equal_xkv']})",
            "host": host, "threads_note": ("the box's CPU share (OMP_NUM_THREADS)" if share > 0 and share < phys
                                           else "all physical cores"),
            "lines": lines}


# The split kernel's other bound: SIMD instruction issue. Per chunk of 64
# tokens at head_dim 64 and 7 query rows a wave issues 256 FP32 matrix-core
# products (128 score, 128 fold) and, on c2's containers, about a thousand
# other vector-ALU instructions; both counts are read from the committed SQ
# counter summary (SQ_INSTS_MFMA and SQ_INSTS_VALU - SQ_INSTS_MFMA per
# chunk). A product keeps the matrix pipe busy 8 cycles
# (SQ_VALU_MFMA_BUSY_CYCLES / SQ_INSTS_MFMA in the same summary), and a
# vector instruction takes at least 2.8 cycles of the SIMD's issue at three
# waves per SIMD (the fast class of a per-instruction throughput probe on
# gfx950; others take 4.2-4.4); the two kinds do not overlap. Chunks are
# spread over the 1,024 SIMDs at the 2.4 GHz clock the counters show, so
# ideal_us is a floor: the time the SIMDs would take issuing back to back.
ISSUE_MFMA_CYC, ISSUE_VALU_CYC = 8.0, 2.8
SIMDS, CLOCK_GHZ = 1024, 2.4
SQ_PROFILE = "attn_wave_c2_sq_counters.md"


def profile_value(profile: str, key: str):
    """A `key: value` line of a committed profile summary (None if absent)."""
    try:
        for line in open(os.path.join(ROOT, "profiles", profile)):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def issue_roofline(tokens: int, kernel_us: float, three_bit: bool):
    if three_bit:
        return None  # the vector instruction count was measured on encode_bf16's containers
    mfma = profile_value(SQ_PROFILE, "mfma_per_chunk")
    valu = profile_value(SQ_PROFILE, "valu_per_chunk")
    if mfma is None or valu is None:
        return None
    chunks = tokens / 64
    cycles = chunks / SIMDS * (mfma * ISSUE_MFMA_CYC + valu * ISSUE_VALU_CYC)
    ideal_us = cycles / (CLOCK_GHZ * 1e3)
    return {"bound": "simd-issue", "ideal_us": round(ideal_us, 2), "achieved_us": round(kernel_us, 2),
            "frac": round(ideal_us / kernel_us, 4), "mfma_per_chunk": mfma, "valu_per_chunk": valu,
            "mfma_cycles": ISSUE_MFMA_CYC, "valu_cycles": ISSUE_VALU_CYC, "source": "profiles/" + SQ_PROFILE}


def bench_config(a, torch, np, kvexp_amd, synth) -> int:
    """--config c1 / c3 / c4 / c5 (see the module docstring)."""
    name = a.config
    cfg = synth.CONFIGS[name]
    G, D, BT = cfg["group"], cfg["dim"], cfg["block"]
    dev = torch.device("cuda:0")
    ctx = kvexp_amd.Context(0)
    t0 = time.time()
    kx, vx, kr, vr, seqs = [], [], [], [], []
    if name == "c4":
        g = torch.Generator(device=dev)
        g.manual_seed(cfg["seed"])
        n_heads, lens = cfg["layers"] * cfg["kv_heads"], None
    else:
        lens = synth.c3_lengths(cfg["seed"], cfg["batch"]) if name == "c3" else [cfg["seq"]] * cfg["batch"]
        n_heads = len(lens) * cfg["layers"] * cfg["kv_heads"]
    for i in range(n_heads):
        if name == "c4":
            S = cfg["seq"]
            scale = torch.exp2(torch.rand(D, generator=g, device=dev) * 8 - 5)
            k = (torch.randn(S, D, generator=g, device=dev) * scale).to(torch.bfloat16).view(torch.int16).reshape(-1)
            v = (torch.randn(S, D, generator=g, device=dev) * 0.5).to(torch.bfloat16).view(torch.int16).reshape(-1)
        else:
            per = cfg["layers"] * cfg["kv_heads"]
            b, lh = divmod(i, per)
            S = lens[b]
            hk, hv = synth.head_kv(name, S, b, lh // cfg["kv_heads"], lh % cfg["kv_heads"])
            k = torch.from_numpy(hk.view(np.int16)).to(dev)
            v = torch.from_numpy(hv.view(np.int16)).to(dev)
        kx.append(ctx.encode(k, S, D, BT, sync_size=False))
        vx.append(ctx.encode(v, S, D, BT, sync_size=False))
        kr.append(k)
        vr.append(v)
        seqs.append(S)
        if (i + 1) % 256 == 0:
            log(f"{name}: {i + 1} of {n_heads} heads generated and encoded ({time.time() - t0:.0f} s)")
    torch.cuda.synchronize()
    for e in kx + vx:
        e.nbytes = int(e.offsets[-1])
    container = sum(e.nbytes for e in kx + vx)
    tight = 4 * D * sum(seqs)
    splits = a.splits or (ctx.suggest_splits_batch(seqs, BT, D, G) if name == "c3"
                          else ctx.suggest_splits(n_heads, seqs[0], BT, dim=D, n_q=G))
    q = torch.randn(n_heads * G * D, device=dev).to(torch.bfloat16).view(torch.int16)
    px = ctx.plan([dict(kx=kx[i], vx=vx[i], seq=seqs[i], splits=splits) for i in range(n_heads)], G, D, BT)
    pr = ctx.plan([dict(k=kr[i], v=vr[i], seq=seqs[i], splits=splits) for i in range(n_heads)], G, D, BT)
    ox = px.run(q, check_errors=True).clone()
    orw = pr.run(q, check_errors=True).clone()
    torch.cuda.synchronize()
    same = bool(torch.equal(ox.view(torch.int32), orw.view(torch.int32)))
    log(f"{name}: {n_heads} heads, {sum(seqs)} tokens, container {container} B (ratio {container / tight:.6f}), "
        f"splits {splits}, XKV == raw: {same} ({time.time() - t0:.0f} s)")
    out = torch.empty(n_heads * G * D, dtype=torch.float32, device=dev)

    def timed(p):
        for _ in range(a.warmup):
            p.run(q, out)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(a.steps):
            p.run(q, out)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / a.steps

    ms_x, ms_r = timed(px), timed(pr)
    # the split kernel alone (HIP events on its stream around each launch)
    px.timing(True)
    timed(px)
    kern_ms, kern_runs = px.kernel_time()
    px.timing(False)
    kern_avg_ms = kern_ms / max(1, kern_runs)
    px.close()
    pr.close()
    gbps = container / (ms_x * 1e-3) / 1e9
    # algorithmic bytes of one split-kernel launch: every container byte, Q
    # (BF16) and the output (FP32) once
    algo = container + n_heads * G * D * 2 + n_heads * G * D * 4
    achieved = algo / (kern_avg_ms * 1e-3) / 1e9
    log(f"{name}: xkv {ms_x * 1e3:.1f} us/step ({gbps:.0f} GB/s of containers; split kernel "
        f"{kern_avg_ms * 1e3:.1f} us = {achieved:.0f} GB/s), raw {ms_r * 1e3:.1f} us/step")
    print(json.dumps({
        "metric": f"decode-step µs + achieved HBM GB/s, BASELINE config {name} (parity case, not the quoted line)",
        "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "us_per_step": round(ms_x * 1e3, 2), "higher_is_better": True, "dtype": "f32",
        "data": "synthetic (GPU-generated, config distributions)" if name == "c4"
                else f"synthetic (seeded, kvexp_amd/synth.py config {name})",
        "config": {"workload": name, "kv_heads": n_heads, "group": G, "dim": D, "block": BT,
                   "tokens": sum(seqs), "max_seq": max(seqs), "splits_per_head": splits},
        "pct_hbm_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2), "container_bytes": container,
        "tight_bytes": tight, "raw_us_per_step": round(ms_r * 1e3, 2), "xkv_over_raw": round(ms_x / ms_r, 4),
        "xkv_bit_equal_raw": same,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": f"attn_wave_kernel<{G}, {D}, true, 0>", "kernel_us": round(kern_avg_ms * 1e3, 2),
                     "algorithmic_bytes": algo},
    }), flush=True)
    return 0 if same else 1


def bench_dump(a, torch, np, kvexp_amd) -> int:
    from kvexp_amd import dumps

    if not a.kvd or not a.qsnap:
        raise SystemExit("--workload dump needs --kvd and --qsnap (files written by the reference's dump_kv.py)")
    d, qs = dumps.parse_dump(a.kvd), dumps.load_qsnap(a.qsnap)
    lengths = [int(x) for x in a.lengths.split(",")] if a.lengths else [p for p in qs.pos if p <= d.seq]
    ctx = kvexp_amd.Context(0)
    rows = []
    for L in lengths:
        plan, dq, keep = dumps.model_scope(ctx, d, qs, L, splits=a.splits)
        plan_r, dq_r, keep_r = dumps.model_scope(ctx, d, qs, L, splits=a.splits, raw=True)
        ox, orw = plan.run(dq, check_errors=True), plan_r.run(dq_r, check_errors=True)
        torch.cuda.synchronize()
        same = bool(torch.equal(ox.view(torch.int32), orw.view(torch.int32)))
        container = sum(h["kx"].nbytes + h["vx"].nbytes for h in keep[0])
        tight = 4 * L * d.dim * d.layers * d.kv
        res = []
        for p, q in ((plan, dq), (plan_r, dq_r)):
            for _ in range(a.warmup):
                p.run(q, ox)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(a.steps):
                p.run(q, ox)
            e1.record()
            torch.cuda.synchronize()
            res.append(e0.elapsed_time(e1) / a.steps)
        row = {"seq": L, "xkv_us": round(res[0] * 1e3, 2), "raw_us": round(res[1] * 1e3, 2),
               "container_bytes": container, "tight_bytes": tight, "kv_ratio": round(container / tight, 6),
               "xkv_GBps_container": round(container / (res[0] * 1e-3) / 1e9, 2),
               "xkv_bit_equal_raw": same}
        log("dump", row)
        rows.append(row)
    print(json.dumps({"metric": "model-scope decode step µs on a real KV dump", "unit": "us",
                      "value": rows[-1]["xkv_us"] if rows else None, "n_gpus": 1, "steps": a.steps,
                      "warmup": a.warmup, "higher_is_better": False, "data": os.path.basename(a.kvd),
                      "config": {"workload": "dump model scope", "layers": d.layers, "kv_heads": d.kv,
                                 "q_heads": d.nq, "dim": d.dim, "dump_seq": d.seq},
                      "rows": rows}), flush=True)
    return 0


TRACE_LIB = os.path.join(ROOT, "compressed-kv-attention_amd", "lib", "trace", "libkvexp_hip_trace.so")


def phase_trace(a) -> int:
    """Cycles per wave in each phase of the split kernel's chunk loop (c2 or
    c4), or per block in each phase of the one-pass encoder (--workload
    append: the c2 prefill), from the trace build of the library."""
    import ctypes as C

    if not os.path.exists(TRACE_LIB):
        raise SystemExit(f"{TRACE_LIB} missing: run compressed-kv-attention_amd/build.py --trace")
    os.environ["KVEXP_HIP_LIBRARY"] = TRACE_LIB
    import numpy as np
    import torch

    import kvexp_amd
    from kvexp_amd import synth

    L = kvexp_amd.lib()
    ctx = kvexp_amd.Context(0)
    dev = torch.device("cuda:0")
    if a.workload == "append":
        cfg = synth.CONFIGS["c2"]
        S, D, BT = cfg["seq"], cfg["dim"], cfg["block"]
        src = [torch.from_numpy(x.view(np.int16)).to(dev)
               for layer in range(cfg["layers"]) for h in range(cfg["kv_heads"])
               for x in synth.head_kv("c2", S, 0, layer, h)]
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
        names = ["histograms cleared", "(none)", "tokens arrive", "histograms", "window bases + mode",
                 "codes + escape ranks", "look-back", "stores issued"]
        print(f"c2 prefill: {nb} blocks; block life mean {life.mean():.0f} cycles (min {life.min()}, max {life.max()})")
        for i, n in enumerate(names):
            d = t[:, i + 1] - t[:, i]
            print(f"  {n:22s} {d.mean():8.0f} cycles/block ({100 * d.mean() / life.mean():5.1f} %), "
                  f"p50 {np.percentile(d, 50):7.0f}, p99 {np.percentile(d, 99):7.0f}")
        polls = t[:, 9]
        print(f"  look-back waits: {np.mean(polls > 0) * 100:.1f} % of blocks polled again; "
              f"mean {polls.mean():.2f}, max {polls.max()}")
        # the persistent workgroups: blocks per workgroup and how much of the
        # launch each spends inside its blocks
        # (a workgroup's blocks run on one CU, whose clock they share)
        job = np.arange(nb) // (S // BT)
        wg = job * 65536 + t[:, 11]
        first, last, busy, count = {}, {}, {}, {}
        for k, t0, t1, lf in zip(wg, t[:, 0], t[:, 8], life):
            first[k] = min(first.get(k, t0), t0)
            last[k] = max(last.get(k, t1), t1)
            busy[k] = busy.get(k, 0) + lf
            count[k] = count.get(k, 0) + 1
        keys = list(busy)
        span = np.array([last[k] - first[k] for k in keys])
        frac = np.array([busy[k] for k in keys]) / span
        cnt = np.array([count[k] for k in keys])
        print(f"  {int(t[:, 11].max()) + 1} workgroups per job, {len(keys)} in all; blocks per workgroup "
              f"{cnt.mean():.1f} (min {cnt.min()}, max {cnt.max()}); a workgroup's first-to-last-block span "
              f"{span.mean():.0f} cycles, {frac.mean() * 100:.1f} % of it inside its blocks")
        return 0
    config = a.config
    if config not in ("c2", "c4"):
        raise SystemExit("--phase-trace takes --config c2 or c4")
    cfg = synth.CONFIGS[config]
    S, D, G, BT = cfg["seq"], cfg["dim"], cfg["group"], cfg["block"]
    heads = []
    if config == "c2":
        splits = 64
        for layer in range(cfg["layers"]):
            for h in range(cfg["kv_heads"]):
                k, v = synth.head_kv("c2", S, 0, layer, h)
                kx = ctx.encode(torch.from_numpy(k.view(np.int16)).to(dev), S, D, BT)
                vx = ctx.encode(torch.from_numpy(v.view(np.int16)).to(dev), S, D, BT)
                heads.append(dict(kx=kx, vx=vx, seq=S, splits=splits))
    else:  # K and V from torch's generator on the GPU, as --config c4
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
    L.kvexp_hip_phase_trace_read.argtypes = [C.c_void_p, C.c_size_t, C.c_int]
    kvexp_amd.check(L.kvexp_hip_phase_trace_read(buf.ctypes.data_as(C.c_void_p), buf.size, D))
    t = buf.reshape(8192, nph + 3)[: n_heads * splits].astype(np.int64)
    life = t[:, 1] - t[:, 0]
    ph = t[:, 2:2 + nph]
    names = ["K rows wait", "K decode + escapes", "scores", "softmax coefficients", "V rows wait", "V decode",
             "V escapes", "next K block entered", "next K rows requested", "next V block entered",
             "next V rows requested", "fold"]
    chunks = S // splits // 64
    print(f"{config}, {splits} splits: {len(t)} waves of {chunks} chunks; wave life: mean {life.mean():.0f} cycles "
          f"(min {life.min()}, max {life.max()})")
    for i, n in enumerate(names):
        print(f"  {n:32s} {ph[:, i].mean():9.0f} cycles/wave ({100 * ph[:, i].mean() / life.mean():5.1f} %), "
              f"{ph[:, i].mean() / chunks:6.0f} per chunk")
    print(f"  {'outside the chunk loop':32s} {(life - ph.sum(1)).mean():9.0f} cycles/wave")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed steps first (the GPU clock takes a few ms to ramp up after the setup)")
    ap.add_argument("--config", default="c2")
    ap.add_argument("--copies", type=int, default=4)
    ap.add_argument("--splits", type=int, default=0, help="splits per KV head (0 = library suggestion)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--workload", default="attention", choices=["attention", "append", "dump"])
    ap.add_argument("--kvd", default="", help="KVD1 dump (--workload dump)")
    ap.add_argument("--qsnap", default="", help="QSN1 query snapshots (--workload dump)")
    ap.add_argument("--lengths", default="", help="comma-separated snapshot lengths (--workload dump)")
    ap.add_argument("--three-bit", action="store_true",
                    help="encode with the 3-bit format extension allowed (not the reference's containers; "
                         "a side measurement, not the quoted line)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a 256 MiB device copy (counter calibration under rocprofv3 --pmc)")
    ap.add_argument("--phase-trace", action="store_true",
                    help="with the trace build (build.py --trace): cycles by phase of the split kernel's chunk "
                         "loop (c2, --config c4) or of the one-pass encoder (--workload append)")
    a = ap.parse_args()
    if a.phase_trace:
        return phase_trace(a)
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not a measured path)"}))
        return 2

    import numpy as np
    import torch

    import kvexp_amd
    from kvexp_amd import synth

    if a.workload == "append":
        return bench_append(a, torch, np, kvexp_amd, synth)
    if a.workload == "dump":
        return bench_dump(a, torch, np, kvexp_amd)
    if a.config in ("c1", "c3", "c4", "c5"):
        return bench_config(a, torch, np, kvexp_amd, synth)
    if a.config != "c2":
        raise SystemExit("--config takes c1, c2 (the quoted line), c3, c4 or c5")
    cfg = synth.CONFIGS["c2"]
    L, KV, G, D, S, BT = cfg["layers"], cfg["kv_heads"], cfg["group"], cfg["dim"], cfg["seq"], cfg["block"]
    H = L * KV
    dev = torch.device("cuda:0")
    ctx = kvexp_amd.Context(0)
    if a.three_bit:
        ctx.set_encoder_modes(kvexp_amd.MODES_REFERENCE | kvexp_amd.MODE_3BIT)

    # ---- inputs: generate per head, upload raw, encode on the GPU ---------------
    t0 = time.time()
    raw_k, raw_v, enc_k, enc_v = [], [], [], []
    host_kx, host_vx = [], []
    for l in range(L):
        for h in range(KV):
            k, v = synth.head_kv("c2", S, 0, l, h)
            dk = torch.from_numpy(k.view(np.int16)).to(dev)
            dv = torch.from_numpy(v.view(np.int16)).to(dev)
            raw_k.append(dk)
            raw_v.append(dv)
            enc_k.append(ctx.encode(dk, S, D, BT))
            enc_v.append(ctx.encode(dv, S, D, BT))
    q = torch.from_numpy(synth.queries("c2", H).view(np.int16)).to(dev)
    torch.cuda.synchronize()
    container = sum(e.nbytes for e in enc_k) + sum(e.nbytes for e in enc_v)
    tight = 4 * S * D * H
    log(f"inputs ready in {time.time() - t0:.1f}s: container {container} B, tight {tight} B, "
        f"ratio {container / tight:.6f}")

    # block mode mix from the headers
    stats = dict(raw=0, bits2=0, bits3=0, bits4=0, escapes=0)
    for e in enc_k + enc_v:
        off = e.offsets.cpu().numpy()
        blob = e.blob[: e.nbytes].cpu().numpy()
        hdr = blob[off[:-1, None] + np.arange(4)[None, :]]
        modes = hdr[:, 0]
        stats["raw"] += int((modes == 0).sum())
        stats["bits2"] += int((modes == 2).sum())
        stats["bits3"] += int((modes == 3).sum())
        stats["bits4"] += int((modes == 4).sum())
        stats["escapes"] += int((hdr[:, 2].astype(np.int64) | (hdr[:, 3].astype(np.int64) << 8)).sum())

    splits = a.splits or ctx.suggest_splits(H, S, BT)
    copies = max(1, a.copies)

    def clone_enc(e):
        return kvexp_amd.Encoded(e.blob.clone(), e.nbytes, e.offsets, e.first, e.seq, e.dim, e.block)

    xkv_plans, raw_plans, enc_copies = [], [], []
    for c in range(copies):
        ek = enc_k if c == 0 else [clone_enc(e) for e in enc_k]
        ev = enc_v if c == 0 else [clone_enc(e) for e in enc_v]
        enc_copies.append((ek, ev))
        xkv_plans.append(ctx.plan([dict(kx=ek[i], vx=ev[i], seq=S, splits=splits) for i in range(H)], G, D, BT))
        rk = raw_k if c == 0 else [t.clone() for t in raw_k]
        rv = raw_v if c == 0 else [t.clone() for t in raw_v]
        raw_plans.append(ctx.plan([dict(k=rk[i], v=rv[i], seq=S, splits=splits) for i in range(H)], G, D, BT))
    out_x = torch.empty(H * G * D, dtype=torch.float32, device=dev)
    out_r = torch.empty_like(out_x)

    # ---- correctness gate: XKV == raw, bit for bit -------------------------------
    xkv_plans[0].run(q, out_x, check_errors=True)
    raw_plans[0].run(q, out_r, check_errors=True)
    torch.cuda.synchronize()
    ox, orw = out_x.cpu().numpy(), out_r.cpu().numpy()
    bit_equal = bool(np.array_equal(np.isnan(ox), np.isnan(orw)) and
                     np.array_equal(ox[~np.isnan(ox)].view(np.uint32), orw[~np.isnan(orw)].view(np.uint32)))
    if not bit_equal:
        log("XKV and raw outputs differ")
    stream = torch.cuda.current_stream()

    def timed(plans, out, steps, warmup):
        """K steps back to back, bracketed by synchronisations; returns
        (wall ms per step, event ms per step). No per-step events: an event
        record between steps adds time of its own."""
        for i in range(warmup):
            plans[i % len(plans)].run(q, out)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t_start = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            plans[i % len(plans)].run(q, out)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t_start
        return wall / steps * 1e3, e0.elapsed_time(e1) / steps

    # The GPU's clock ramps up under load for some 100 ms (and drops again
    # while the host builds plans): a settle period of untimed steps (about
    # 300 ms) comes before each timed pass that follows idle time, so that a
    # short --warmup does not time a cold clock.
    def settle(plan_sets, outs):
        t_settle, n_settle = time.perf_counter(), 0
        while time.perf_counter() - t_settle < 0.3:
            for plans, out in zip(plan_sets, outs):
                for p in plans:
                    p.run(q, out)
                n_settle += len(plans)
            torch.cuda.synchronize()
        return n_settle, (time.perf_counter() - t_settle) * 1e3

    n_settle, t_settle = settle([xkv_plans, raw_plans], [out_x, out_r])
    log(f"clock settle: {n_settle} untimed steps in {t_settle:.0f} ms")

    ms_x, ev_x = timed(xkv_plans, out_x, a.steps, a.warmup)
    # the split kernel alone, in a separate pass: the library's event pair
    # around it adds a little time between the launches of a step
    for p in xkv_plans:
        p.timing(True)
    timed(xkv_plans, out_x, max(20, a.steps // 2), 0)
    kern_ms, kern_runs = 0.0, 0
    for p in xkv_plans:
        t_ms, t_runs = p.kernel_time()
        p.timing(False)
        kern_ms += t_ms
        kern_runs += t_runs
    kern_avg_ms = kern_ms / max(1, kern_runs)
    ms_r, ev_r = timed(raw_plans, out_r, max(10, a.steps // 2), a.warmup)
    log(f"xkv {ms_x * 1e3:.1f} us/step (events {ev_x * 1e3:.1f}, split kernel "
        f"{kern_avg_ms * 1e3:.1f} over {kern_runs} runs), raw {ms_r * 1e3:.1f} us/step")

    # side figures: one copy every step (partly served by the 256 MB
    # Infinity Cache), the median of 25 singly timed steps (the reference
    # bench's statistic), and the AVX-512 BF16 score order (Backend::HipDpbf16)
    ms_hot, _ = timed(xkv_plans[:1], out_x, max(20, a.steps // 2), 20)
    samples = []
    for i in range(25):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        xkv_plans[i % copies].run(q, out_x)
        e1.record(stream)
        torch.cuda.synchronize()
        samples.append(e0.elapsed_time(e1))
    med_ms = float(np.median(samples))
    # the AVX-512 order's own split count (its kernel may run fewer waves per SIMD)
    dp_splits = a.splits or ctx.suggest_splits(H, S, BT, dim=D, n_q=G, order=1)
    dp_plans = [ctx.plan([dict(kx=ek[i], vx=ev[i], seq=S, splits=dp_splits) for i in range(H)], G, D, BT, order=1)
                for ek, ev in enc_copies]
    dp_raw = ctx.plan([dict(k=raw_k[i], v=raw_v[i], seq=S, splits=dp_splits) for i in range(H)], G, D, BT,
                      order=1)
    odp = dp_plans[0].run(q, check_errors=True).clone()
    odr = dp_raw.run(q, check_errors=True).clone()
    torch.cuda.synchronize()
    dp_equal = bool(torch.equal(odp.view(torch.int32), odr.view(torch.int32)))
    settle([dp_plans], [out_x])  # the plan builds left the GPU idle
    ms_dp, _ = timed(dp_plans, out_x, max(20, a.steps // 2), max(a.warmup, 8 * copies))
    for p in dp_plans + [dp_raw]:
        p.close()
    log(f"hot (one copy) {ms_hot * 1e3:.1f} us/step, median of 25 single steps {med_ms * 1e3:.1f} us; "
        f"AVX-512 BF16 order {ms_dp * 1e3:.1f} us/step at {dp_splits} splits (XKV == raw: {dp_equal})")

    q_bytes = H * G * D * 2
    out_bytes = H * G * D * 4
    algo_bytes = container + q_bytes + out_bytes
    achieved = algo_bytes / (kern_avg_ms * 1e-3) / 1e9
    traffic = None if a.three_bit else measured_traffic()  # the counters were read on encode_bf16's containers
    value = container / (ms_x * 1e-3) / 1e9

    if a.copy_probe:
        copy_probe(torch, dev)

    # ---- CPU baseline: the compiled reference, both scopes, cold samples ----------
    cpu = None
    if not a.no_cpu_baseline:
        try:
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            from oracle import Reference

            R = Reference()
            cpu = cpu_baseline_c2(
                R, np, a, q.cpu().numpy().view(np.uint16),
                [t.cpu().numpy().view(np.uint16) for t in raw_k], [t.cpu().numpy().view(np.uint16) for t in raw_v],
                [e.blob[: e.nbytes].cpu().numpy() for e in enc_k], [e.blob[: e.nbytes].cpu().numpy() for e in enc_v],
                G, D, S, BT)
            log("cpu baseline", json.dumps(cpu))
        except FileNotFoundError:
            cpu = {"value": None, "unit": "GB/s", "cores": 0, "kind": "reference",
                   "sample": "oracle/_ref/libkvexp_ref.so not present on this host"}

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_x, 5),
        "us_per_step": round(ms_x * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, kvexp_amd/synth.py config c2)",
        "config": {"workload": "c2: full 24-layer Qwen2.5-0.5B decode step, 48 KV heads x 7 queries, head_dim 64, "
                               "seq 32768, XKV 128-token blocks", "kv_heads": H, "group": G, "dim": D, "seq": S,
                   "block": BT, "splits_per_head": splits, "copies": copies,
                   "format": "XKV + 3-bit extension" if a.three_bit else "XKV (encode_bf16)"},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "container_bytes": container,
        "tight_bytes": tight,
        "uncompressed_equiv_GBps": round(tight / (ms_x * 1e-3) / 1e9, 2),
        "raw_us_per_step": round(ms_r * 1e3, 2),
        "raw_GBps_tight": round(tight / (ms_r * 1e-3) / 1e9, 2),
        "xkv_over_raw": round(ms_x / ms_r, 4),
        "xkv_bit_equal_raw": bit_equal,
        "hot_us_per_step": round(ms_hot * 1e3, 2),
        "median_us_single_step": round(med_ms * 1e3, 2),
        "dpbf16_us_per_step": round(ms_dp * 1e3, 2),
        "dpbf16_splits_per_head": dp_splits,
        "dpbf16_xkv_bit_equal_raw": dp_equal,
        "block_modes": stats,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": "attn_wave_kernel<7, 64, true, 0>", "kernel_us": round(kern_avg_ms * 1e3, 2),
                     "algorithmic_bytes": algo_bytes},
        "issue": issue_roofline(H * S, kern_avg_ms * 1e3, a.three_bit),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
