#!/usr/bin/env python3
"""Fused RoPE + GQA decode layer-step on one MI355X: KV-stream HBM GB/s and us/layer.

Default workload = BASELINE.json configs[1] ("c2"): 32 query heads, 8 KV
heads, head dim 128, fp32 token-major KV cache holding 16384 positions, one
new token at pos 16384 (n = 16385 after the append), RoPE theta 500000,
scale 1/sqrt(128), batch 1, q/K/V ~ N(0,1) from the repo's seeded generator.

One step = one layer-step of the hot path through the C ABI
(molot_hip_decode_step): RoPE of q and k, append of k/v into the cache,
split-K attention (attn_kernel) and its log-sum-exp combine
(combine_kernel), two launches on one stream.  Steps cycle over enough layers' KV caches
(>= 1 GiB in total) that the 256 MB Infinity Cache cannot serve the stream:
every step reads its layer's KV from HBM, as consecutive layers of a real
decode do.  The K timed steps run as one HIP graph replay bracketed by
events, inputs already resident in HBM.

value = unique KV bytes per step / time per step ("KV-stream GB/s").
roofline = the dominant kernel, attn_kernel (RoPE, append and the split-K
KV stream): its average launch duration comes from start/stop HIP events
that HIP stamps from the kernel's own dispatch (the library launches with
hipExtLaunchKernelGGL while molot_hip_profile_* is on; eager launches on
the bench stream after the timed region); achieved = the step's algorithmic
bytes (all of which that kernel moves) / that duration; traffic =
calibrated rocprofv3 FETCH_SIZE + WRITE_SIZE per launch
(profiles/traffic.json).
cpu_baseline = the reference's own attn.h decode step (oracle/_ref, built
from the reference headers) on the host cores, same workload, bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
METRIC = ("KV-stream HBM GB/s (% of peak) + µs/layer, 32q/8kv/d128 @16k ctx, 1 GPU")

CONFIGS = {
    # name: (nq, nkv, d, pos, theta, window, kv_dtype, sigma_kv)
    "c1": (32, 8, 128, 4096, 500000.0, 0, 0, 1.0),
    "c2": (32, 8, 128, 16384, 500000.0, 0, 0, 1.0),
    "c3": (8, 4, 256, 32768, 10000.0, 1024, 0, 1.0),
    "c5": (64, 8, 128, 131072, 500000.0, 0, 1, 0.5),
}
DESCR = {
    "c1": "fused RoPE+GQA decode layer-step, 32q/8kv/d128 fp32 KV, pos 4096 (n=4097), batch 1",
    "c2": "fused RoPE+GQA decode layer-step, 32q/8kv/d128 fp32 KV, ctx 16384 (n=16385), batch 1",
    "c3": "sliding-window GQA decode layer-step, 8q/4kv/d256 fp32 KV, pos 32768, window 1024",
    "c5": "long-context GQA decode layer-step, 64q/8kv/d128 bf16 KV, pos 131072 (n=131073)",
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=0, help="KV caches to cycle (0 = auto, >=1 GiB)")
    ap.add_argument("--kernel-launches", type=int, default=200,
                    help="individually timed attention launches for the roofline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="budget of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = min(16, cores available)")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead")
    ap.add_argument("--split-chunk", type=int, default=0, help="tokens per chunk (0 = auto)")
    ap.add_argument("--wgs-per-cu", type=int, default=0, help="workgroups per CU (0 = auto)")
    ap.add_argument("--variant", type=int, default=0, help="kernel mapping variant (0 = default)")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="rocprofv3 PMC traffic summary (FETCH_SIZE/WRITE_SIZE per launch)")
    ap.add_argument("--pmc-run", action="store_true",
                    help="counter-collection pass: 20 eager steps + 3 copy-probe launches of 1 GiB, "
                         "no timing (run under rocprofv3 --pmc)")
    ap.add_argument("--quiet", action="store_true")
    return ap.parse_args()


def log(args, *a):
    if not args.quiet:
        print("[bench]", *a, file=sys.stderr, flush=True)


def algorithmic_bytes(nq, nkv, d, n_att, s_kv):
    """Bytes one layer-step must move (decode-attention roofline):
    KV stream 2*nkv*n_att*d*s_kv, q read + O write 2*nq*d*4, new k/v read as
    fp32 and written at s_kv, the RoPE table d/2*4."""
    kv = 2 * nkv * n_att * d * s_kv
    other = 2 * nq * d * 4 + 2 * nkv * d * (4 + s_kv) + (d // 2) * 4
    return kv, kv + other


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path shards by KV head across GPUs with no exchange (see DESIGN.md), "
              "but nothing here launches on more than one device.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from molot_amd import attn
    from molot_amd import lib as L
    from molot_amd.synth import Stream, f32_to_bf16

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    lib = L.load()
    torch.cuda.set_device(0)
    if args.split_chunk:
        attn.set_split_chunk(args.split_chunk)
    if args.wgs_per_cu or args.variant:
        lib.molot_hip_set_tuning(args.wgs_per_cu, args.variant)

    nq, nkv, d, pos, theta, window, kvd, sigma = CONFIGS[args.config]
    s_kv = 4 if kvd == 0 else 2
    n = pos + 1
    t0 = max(0, pos - window + 1) if window > 0 else 0
    n_att = n - t0
    kv_bytes, step_bytes = algorithmic_bytes(nq, nkv, d, n_att, s_kv)
    cache_bytes = 2 * n * nkv * d * s_kv
    layers = args.layers or max(2, math.ceil((1 << 30) / cache_bytes))
    scale = 1.0 / math.sqrt(d)

    # ---- inputs (seeded; one host draw, replicated per layer on the device) ----
    t_setup = time.time()
    st = Stream(1234)
    q_h = st.normal((nq, d))
    k_h = st.normal((nkv, d))
    v_h = st.normal((nkv, d))
    K_h = np.zeros((n, nkv * d), np.float32)
    V_h = np.zeros_like(K_h)
    K_h[:pos] = st.normal((pos, nkv * d), sigma)
    V_h[:pos] = st.normal((pos, nkv * d), sigma)
    dt = torch.float32 if kvd == 0 else torch.bfloat16

    def to_dev(a):
        if kvd == 0:
            return torch.from_numpy(a).cuda()
        return torch.from_numpy(f32_to_bf16(a).view(np.int16)).cuda().view(torch.bfloat16)

    K0, V0 = to_dev(K_h), to_dev(V_h)
    Ks = [K0] + [torch.empty_like(K0) for _ in range(layers - 1)]
    Vs = [V0] + [torch.empty_like(V0) for _ in range(layers - 1)]
    for i in range(1, layers):
        Ks[i].copy_(K0)
        Vs[i].copy_(V0)
    q = torch.from_numpy(q_h).cuda()
    k_new = torch.from_numpy(k_h).cuda()
    v_new = torch.from_numpy(v_h).cuda()
    inv = attn.rope_inv_freq(theta, d).cuda()
    O = torch.empty((nq, d), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    del K_h, V_h
    log(args, f"setup {time.time() - t_setup:.1f}s: {args.config} layers={layers} "
        f"cache={cache_bytes / 2**20:.0f} MiB/layer dtype={dt}")

    P = ctypes.c_void_p
    qp, kp, vp, ip, op = (P(t.data_ptr()) for t in (q, k_new, v_new, inv, O))
    Kp = [P(t.data_ptr()) for t in Ks]
    Vp = [P(t.data_ptr()) for t in Vs]

    def cur_stream():
        return P(torch.cuda.current_stream().cuda_stream)

    def step(i, stream):
        l = i % layers
        rc = lib.molot_hip_decode_step(qp, kp, vp, Kp[l], Vp[l], op, nq, nkv, d, pos, pos, ip,
                                       scale, window, kvd, stream)
        if rc:
            raise L.MolotHipError(rc, "decode_step")

    def attention(i, stream):
        l = i % layers
        rc = lib.molot_hip_attn_decode_gqa_cache(qp, Kp[l], Vp[l], op, nq, nkv, n, d, scale, pos,
                                                 window, kvd, stream)
        if rc:
            raise L.MolotHipError(rc, "attn_decode_gqa_cache")

    nch = ctypes.c_int()
    chk = ctypes.c_int()
    # the fused step tiles the cached rows; the new token joins the last chunk
    lib.molot_hip_split_plan(nkv, n_att - 1, d, kvd, ctypes.byref(nch), ctypes.byref(chk))

    if args.pmc_run:
        # eager launches only (one counter record per dispatch), then a copy of
        # known size whose FETCH_SIZE / WRITE_SIZE calibrate the counters
        for i in range(args.warmup):
            step(i, cur_stream())
        for i in range(20):
            step(i, cur_stream())
        torch.cuda.synchronize()
        cb = 1 << 30
        src = torch.ones(cb // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            L.check(lib.molot_probe_copy(P(dst.data_ptr()), P(src.data_ptr()), cb, cur_stream()),
                    "probe_copy")
        torch.cuda.synchronize()
        print(json.dumps({"pmc_run": args.config, "steps": 20, "copy_bytes": cb,
                          "step_algorithmic_bytes": step_bytes, "kv_bytes": kv_bytes}))
        return 0

    # ---- warmup + timed steps ----
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        sp = cur_stream()
        for i in range(args.warmup):
            step(i, sp)
    torch.cuda.synchronize()

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    mode = "eager" if args.no_graph else "graph"
    if args.no_graph:
        with torch.cuda.stream(s):
            torch.cuda.synchronize()
            start.record(s)
            for i in range(args.steps):
                step(i, sp)
            end.record(s)
        torch.cuda.synchronize()
    else:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            spc = cur_stream()
            for i in range(args.steps):
                step(i, spc)
        with torch.cuda.stream(s):
            g.replay()  # upload + one untimed pass
            torch.cuda.synchronize()
            start.record(s)
            g.replay()
            end.record(s)
        torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    us_step = ms_per_step * 1e3
    value = kv_bytes / (ms_per_step * 1e-3) / 1e9
    log(args, f"{mode}: {args.steps} steps in {total_ms:.3f} ms -> {us_step:.2f} us/step, "
        f"KV-stream {value:.0f} GB/s ({100 * value / HBM_PEAK_GBPS:.1f}% of 8 TB/s)")

    # ---- per-kernel durations: while profiling is on, the library launches
    # each kernel with start/stop HIP events stamped by its dispatch (eager
    # launches on the bench stream, after the timed region) ----
    def kernel_times(fn, J):
        with torch.cuda.stream(s):
            for i in range(20):
                fn(i, sp)
            torch.cuda.synchronize()
            L.check(lib.molot_hip_profile_begin(J), "profile_begin")
            for i in range(J):
                fn(i, sp)
        am, cm = ctypes.c_float(), ctypes.c_float()
        na, nc = ctypes.c_int(), ctypes.c_int()
        L.check(lib.molot_hip_profile_end(ctypes.byref(am), ctypes.byref(cm), ctypes.byref(na),
                                          ctypes.byref(nc)), "profile_end")
        k1 = am.value / max(1, na.value) * 1e3
        k2 = cm.value / nc.value * 1e3 if nc.value else 0.0
        return k1, k2

    J = max(10, args.kernel_launches)
    k1_us, k2_us = kernel_times(step, J)
    a1_us, a2_us = kernel_times(attention, J)
    achieved = step_bytes / (k1_us * 1e-6) / 1e9
    log(args, f"attn_kernel {k1_us:.2f} us/launch -> {achieved:.0f} GB/s "
        f"(chunks {nch.value} x {chk.value} tokens); combine_kernel {k2_us:.2f} us; "
        f"attention-only entry: {a1_us:.2f} + {a2_us:.2f} us")

    # ---- achievable streaming-read peak on this box (probe kernel, 4 GiB) ----
    probe_bytes = 4 << 30
    buf = torch.empty(probe_bytes // 4, dtype=torch.float32, device="cuda")
    buf.fill_(1.0)
    sink = torch.empty(1 << 16, dtype=torch.float32, device="cuda")
    with torch.cuda.stream(s):
        for _ in range(3):
            lib.molot_probe_read(P(buf.data_ptr()), probe_bytes, P(sink.data_ptr()), sink.numel(),
                                 sp)
        torch.cuda.synchronize()
        start.record(s)
        for _ in range(10):
            lib.molot_probe_read(P(buf.data_ptr()), probe_bytes, P(sink.data_ptr()), sink.numel(),
                                 sp)
        end.record(s)
    torch.cuda.synchronize()
    read_peak = 10 * probe_bytes / (start.elapsed_time(end) * 1e-3) / 1e9
    del buf
    log(args, f"streaming-read probe: {read_peak:.0f} GB/s")

    # ---- traffic measured by rocprofv3 PMC runs (committed summary), if present ----
    traffic = None
    try:
        with open(args.traffic) as f:
            tr = json.load(f)
        if tr.get("config") == args.config:
            traffic = tr.get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        pass

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if kvd == 0 else "bf16-kv/f32-acc",
        "data": "synthetic (seeded N(0,1) q/K/V, splitmix64+Box-Muller, seed 1234)",
        "config": {"workload": DESCR[args.config], "config": args.config, "nq": nq, "nkv": nkv,
                   "head_dim": d, "pos": pos, "n": n, "window": window, "rope_theta": theta,
                   "batch": 1, "kv_layers_cycled": layers, "timing": mode,
                   "split_chunks": nch.value, "chunk_tokens": chk.value},
        "us_per_layer_step": round(us_step, 3),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "pct_of_measured_read_peak": round(100 * value / read_peak, 2),
        "measured_read_peak_gbps": round(read_peak, 1),
        "kv_bytes_per_step": kv_bytes,
        "algorithmic_bytes_per_step": step_bytes,
        "total_gbps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "head_traffic_gbps": round(2 * nq * n_att * d * s_kv / (ms_per_step * 1e-3) / 1e9, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": f"attn_kernel<{d},{min(8, nq // nkv)},{'float' if kvd == 0 else 'bf16'},"
                      "paged=false,rope=true> (then combine_kernel: split-K merge)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "launch_us": round(k1_us, 3),
            "algorithmic_bytes_per_launch": step_bytes,
            "combine_launch_us": round(k2_us, 3),
            "step_gbps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        },
    }

    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline(args, q_h, k_h, v_h, nq, nkv, d, pos, theta, window,
                                           kvd, sigma, scale, kv_bytes)
    print(json.dumps(out), flush=True)
    return 0


def cpu_baseline(args, q_h, k_h, v_h, nq, nkv, d, pos, theta, window, kvd, sigma, scale,
                 kv_bytes):
    """The reference's decode step on the host cores (bounded sample).

    kind "reference": include/molot/attn.h + forward.h's rope/append sequence,
    compiled from the reference headers into oracle/_ref (ThreadPool with
    `cores` threads).  Falls back to the oracle's C restatement ("port") when
    that library is absent or the host lacks AVX512F.  bf16 configs have no
    reference counterpart: the reference runs on the widened values."""
    import numpy as np

    import oracle
    from molot_amd.synth import Stream, bf16_to_f32, f32_to_bf16

    cores = args.cpu_threads or min(16, len(os.sched_getaffinity(0)))
    n = pos + 1
    st = Stream(4321)
    S = nkv * d
    # rotate copies so the KV stream is DRAM-cold w.r.t. the host LLC
    per_copy = 2 * n * S * 4
    copies = max(2, math.ceil(256 * 2**20 / per_copy))
    Ks, Vs = [], []
    for _ in range(copies):
        K = np.zeros((n, S), np.float32)
        V = np.zeros_like(K)
        K[:pos] = st.normal((pos, S), sigma)
        V[:pos] = st.normal((pos, S), sigma)
        if kvd:
            K[:pos] = bf16_to_f32(f32_to_bf16(K[:pos]))
            V[:pos] = bf16_to_f32(f32_to_bf16(V[:pos]))
        Ks.append(K)
        Vs.append(V)
    inv = oracle.rope_inv_freq(theta, d)
    O = np.empty((nq, d), np.float32)
    P = oracle._p
    kind = "reference" if oracle.ref_available() else "port"
    pool = oracle.RefPool(cores) if kind == "reference" else None

    def one(i):
        q = q_h.copy()
        k = k_h.copy()
        c = i % copies
        if kind == "reference":
            rc = oracle.ref().ref_decode_step(P(q), P(k), P(v_h), P(Ks[c]), P(Vs[c]), P(O), nq,
                                              nkv, d, pos, n, pos, P(inv), scale, window, pool.h)
            assert rc == 0
        else:
            oracle.lib().orc_decode_step(P(q), P(k), P(v_h), P(Ks[c]), P(Vs[c]), P(O), nq, nkv,
                                         d, pos, pos, P(inv), scale, window, 0, cores)

    for i in range(2):  # warmup 2 (bench/bench.cc:45-52)
        one(i)
    t0 = time.perf_counter()
    steps = 0
    while True:
        one(steps)
        steps += 1
        el = time.perf_counter() - t0
        if (el >= args.cpu_seconds and steps >= 3) or steps >= 100000:
            break
    if pool:
        pool.close()
    ms = el / steps * 1e3
    gbps = kv_bytes / (ms * 1e-3) / 1e9
    log(args, f"cpu baseline ({kind}, {cores} threads): {ms:.3f} ms/step -> {gbps:.1f} GB/s")
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": kind,
        "ms_per_step": round(ms, 4),
        "sample": (f"{steps} layer-steps of {args.config} (rope q/k + append + "
                   f"attn_decode_gqa_cache, n={n}) cycling {copies} KV copies of "
                   f"{per_copy / 2**20:.0f} MiB, {el:.1f} s; "
                   + ("reference headers via oracle/_ref, ThreadPool" if kind == "reference"
                      else "oracle C restatement, OpenMP static over heads")
                   + ("; bf16 values widened to fp32 (no reference bf16 path)" if kvd else "")),
    }


if __name__ == "__main__":
    sys.exit(main())
