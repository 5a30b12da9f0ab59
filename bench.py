#!/usr/bin/env python3
"""Fused RoPE + GQA decode layer-step on one MI355X: KV-stream HBM GB/s and us/layer.

Default workload = BASELINE.json configs[1] ("c2"): 32 query heads, 8 KV
heads, head dim 128, fp32 token-major KV cache holding 16384 positions, one
new token at pos 16384 (n = 16385 after the append), RoPE theta 500000,
scale 1/sqrt(128), batch 1, q/K/V ~ N(0,1) from the repo's seeded generator.
`--config c1|c3|c4|c5` measures the other BASELINE configs the same way
(c4: 64 sequences over a paged bf16 cache, molot_hip_decode_step_paged);
c2q8|c4q8|c5q8 run c2, c4 and c5 over Q8 caches (int8 codes + an fp32 scale
per KV head row); p1|p2|p3 time the layer prefill (p3: d = 256, windowed).

One step = one layer-step of the hot path through the C ABI
(molot_hip_decode_step): RoPE of q and k, append of k/v into the cache,
split-K attention (attn_kernel) and, when the context spans more than one
chunk, its log-sum-exp merge: inside the same launch for long fp32 contexts
(the workgroup that completes a KV head's chunks merges them), else a
second launch on the stream (combine_kernel).
Steps cycle over enough layers' KV caches (>= 1 GiB of attended KV in
total) that the 256 MB Infinity Cache cannot serve the stream: every step
reads its layer's KV from HBM, as consecutive layers of a real decode do.
The K timed steps run as one HIP graph replay bracketed by events, inputs
already resident in HBM.

value = unique KV bytes per step / time per step ("KV-stream GB/s").
roofline = the dominant kernel, attn_kernel (RoPE, append and the split-K
KV stream): its average launch duration comes from start/stop HIP events
that HIP stamps from the kernel's own dispatch (the library launches with
hipExtLaunchKernelGGL while molot_hip_profile_* is on; eager launches on
the bench stream after the timed region); achieved = the step's algorithmic
bytes (all of which that kernel moves) / that duration; traffic =
calibrated rocprofv3 FETCH_SIZE + WRITE_SIZE per launch
(profiles/traffic.json, per config, written by molot_amd.rocprof; null when
that record was measured on another version of the kernel source).
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
from types import SimpleNamespace

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
BOX_CPU_SHARE = 16  # host cores a one-GPU job is allotted on the GPU boxes


def metric_name(cfg):
    """BASELINE.json's metric, naming the configuration measured."""
    kv = {0: "", 1: " bf16", 2: " Q8"}[cfg["kvd"]]  # fp32 KV: BASELINE.json's own wording
    shape = f"{cfg['nq']}q/{cfg['nkv']}kv/d{cfg['d']}{kv}"
    if "batch" in cfg:
        where = f"{cfg['batch']} paged seqs of ctx U[{cfg['lmin']},{cfg['lmax']}]"
    else:
        ctx = cfg["pos"]
        where = f"@{ctx // 1024}k ctx" if ctx % 1024 == 0 else f"@{ctx} ctx"
        if cfg["window"]:
            where += f", window {cfg['window']}"
    return f"KV-stream HBM GB/s (% of peak) + µs/layer, {shape} {where}, 1 GPU"


def host_cpu():
    """The host cores the CPU baseline runs on, and what the machine reports.

    The reference's ThreadPool defaults to every hardware thread
    (include/molot/thread_pool.h:19-23).  Here the pool takes every core this
    process may run on (its affinity set, bounded by a cgroup CPU quota if
    one is set), at most the BOX_CPU_SHARE cores a one-GPU job is allotted on
    the GPU boxes."""
    nproc = os.cpu_count() or 1
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
            if q != "max":
                quota = int(q) / int(per)
    except (OSError, ValueError):
        pass
    threads = aff if quota is None else max(1, min(aff, int(quota)))
    threads = min(threads, BOX_CPU_SHARE)
    model, llc = "unknown", "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    for idx in (3, 2):
        try:
            with open(f"/sys/devices/system/cpu/cpu0/cache/index{idx}/size") as f:
                llc = f"L{idx} {f.read().strip()}"
            break
        except OSError:
            continue
    info = {"nproc": nproc, "affinity_cores": aff, "cgroup_cpu_quota": quota,
            "threads": threads, "cpu_model": model, "llc": llc,
            "thread_rule": f"every core in the process's affinity set and CPU quota, at most "
                           f"{BOX_CPU_SHARE} (a one-GPU job's share of the GPU box)"}
    return threads, info
COLD_BYTES = 1 << 30  # attended KV cycled per timed pass (> 256 MB Infinity Cache)

CONFIGS = {
    # contiguous token-major cache, batch 1
    "c1": dict(nq=32, nkv=8, d=128, pos=4096, theta=500000.0, window=0, kvd=0, sigma=1.0),
    "c2": dict(nq=32, nkv=8, d=128, pos=16384, theta=500000.0, window=0, kvd=0, sigma=1.0),
    "c3": dict(nq=8, nkv=4, d=256, pos=32768, theta=10000.0, window=1024, kvd=0, sigma=1.0),
    "c5": dict(nq=64, nkv=8, d=128, pos=131072, theta=500000.0, window=0, kvd=1, sigma=0.5),
    # paged bf16 cache, 64 sequences of context U[512, 8192], shuffled 16-row pages
    "c4": dict(nq=32, nkv=8, d=128, theta=500000.0, window=0, kvd=1, sigma=1.0, batch=64,
               lmin=512, lmax=8192, page=16),
    # the same workloads over Q8 caches (int8 codes + an fp32 scale per KV head row)
    "c2q8": dict(nq=32, nkv=8, d=128, pos=16384, theta=500000.0, window=0, kvd=2, sigma=1.0),
    "c5q8": dict(nq=64, nkv=8, d=128, pos=131072, theta=500000.0, window=0, kvd=2, sigma=0.5),
    "c3q8": dict(nq=8, nkv=4, d=256, pos=32768, theta=10000.0, window=1024, kvd=2, sigma=1.0),
    # a gemma4 global layer (model.h:562-564): head dim 512, 8q/2kv, 32k context
    "c6": dict(nq=8, nkv=2, d=512, pos=32768, theta=1000000.0, window=0, kvd=0, sigma=1.0),
    "c6q8": dict(nq=8, nkv=2, d=512, pos=32768, theta=1000000.0, window=0, kvd=2, sigma=1.0),
    # gemma4's two layer kinds over bf16 caches (a 256-wide sliding-window layer, a 512-wide
    # global one)
    "c3bf16": dict(nq=8, nkv=4, d=256, pos=32768, theta=10000.0, window=1024, kvd=1, sigma=1.0),
    "c6bf16": dict(nq=8, nkv=2, d=512, pos=32768, theta=1000000.0, window=0, kvd=1, sigma=1.0),
    "c4q8": dict(nq=32, nkv=8, d=128, theta=500000.0, window=0, kvd=2, sigma=1.0, batch=64,
                 lmin=512, lmax=8192, page=16),
    # prefill (gemm.h:409-446, forward.h:367-399): M prompt tokens after n0 cached
    "p1": dict(nq=32, nkv=8, d=128, theta=500000.0, window=0, kvd=0, sigma=1.0, prompt=2048,
               n0=0),
    "p2": dict(nq=32, nkv=8, d=128, theta=500000.0, window=0, kvd=0, sigma=1.0, prompt=512,
               n0=16384),
    "p3": dict(nq=8, nkv=4, d=256, theta=10000.0, window=1024, kvd=0, sigma=1.0, prompt=2048,
               n0=0),
}
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix, published
# the prefill's fp32-exact products on the dense fp16 matrix cores (fp32
# and Q8 caches): a score term and a PV term each as three fp16 piece
# products (two row-scaled fp16 pieces of q and K, of P and V)
PIECE_PRODUCTS = 3.0
PIECE_PEAK_TFLOPS = BF16_MFMA_PEAK_TFLOPS / PIECE_PRODUCTS
SIX_PRODUCT_PEAK_TFLOPS = BF16_MFMA_PEAK_TFLOPS / 6  # six bf16 products per term, both halves
DESCR = {
    "c1": "fused RoPE+GQA decode layer-step, 32q/8kv/d128 fp32 KV, pos 4096 (n=4097), batch 1",
    "c2": "fused RoPE+GQA decode layer-step, 32q/8kv/d128 fp32 KV, ctx 16384 (n=16385), batch 1",
    "c3": "sliding-window GQA decode layer-step, 8q/4kv/d256 fp32 KV, pos 32768, window 1024",
    "c4": "continuous-batching decode step, 64 sequences of ctx U[512,8192], 32q/8kv/d128, "
          "bf16 KV in shuffled 16-token pages",
    "c5": "long-context GQA decode layer-step, 64q/8kv/d128 bf16 KV, pos 131072 (n=131073)",
    "c2q8": "fused RoPE+GQA decode layer-step, 32q/8kv/d128 Q8 KV, ctx 16384 (n=16385), batch 1",
    "c5q8": "long-context GQA decode layer-step, 64q/8kv/d128 Q8 KV, pos 131072 (n=131073)",
    "c3q8": "sliding-window GQA decode layer-step, 8q/4kv/d256 Q8 KV, pos 32768, window 1024",
    "c6": "gemma4 global-layer decode step, 8q/2kv/d512 fp32 KV, ctx 32768 (n=32769), batch 1",
    "c6q8": "gemma4 global-layer decode step, 8q/2kv/d512 Q8 KV, ctx 32768 (n=32769), batch 1",
    "c3bf16": "sliding-window GQA decode layer-step, 8q/4kv/d256 bf16 KV, pos 32768, window 1024",
    "c6bf16": "gemma4 global-layer decode step, 8q/2kv/d512 bf16 KV, ctx 32768 (n=32769), "
              "batch 1",
    "c4q8": "continuous-batching decode step, 64 sequences of ctx U[512,8192], 32q/8kv/d128, "
            "Q8 KV in shuffled 16-token pages",
    "p1": "layer prefill (RoPE + append + causal attention), 2048-token prompt, 32q/8kv/d128 "
          "fp32 KV",
    "p2": "layer prefill, 512-token prompt after 16384 cached tokens, 32q/8kv/d128 fp32 KV",
    "p3": "layer prefill, 2048-token prompt, Gemma-style 8q/4kv/d256, window 1024, fp32 KV",
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=0,
                    help="KV caches to cycle (0 = auto, >= 1 GiB of attended KV)")
    ap.add_argument("--kernel-launches", type=int, default=200,
                    help="individually timed attention launches for the roofline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="budget of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0 = every core the process may use, at most the box's 16-core share")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead")
    ap.add_argument("--split-chunk", type=int, default=0, help="tokens per chunk (0 = auto)")
    ap.add_argument("--wgs-per-cu", type=int, default=0, help="workgroups per CU (0 = auto)")
    ap.add_argument("--merge", type=int, default=-1,
                    help="1 = split-K partials merged inside the attention launch where possible, "
                         "0 = by the combine kernel, -1 = the library's choice (default)")
    ap.add_argument("--prefill-presplit", type=int, default=1,
                    help="prefill: 1 = keys split into pieces once per launch, 0 = per tile")
    ap.add_argument("--norms", action="store_true",
                    help="the step with the layer's q/k/v RMS norms fused in (forward.h:554-563)")
    ap.add_argument("--block-order", type=int, default=1,
                    help="1 = waves claim K/V blocks dynamically (default), 0 = fixed order")
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


def row_bytes(kvd, d):
    """Bytes of one cached KV head row: fp32, bf16, or Q8 (d codes + an fp32 scale)."""
    return 4 * d if kvd == 0 else 2 * d if kvd == 1 else d + 4


def algorithmic_bytes(nq, nkv, d, n_att, rb):
    """Bytes one sequence's layer-step must move (decode-attention roofline):
    KV stream 2*nkv*n_att*rb (rb = bytes per cached head row), q read + O
    write 2*nq*d*4, new k/v read as fp32 and written as rows.  The RoPE table
    (d/2*4) is added once per step."""
    kv = 2 * nkv * n_att * rb
    other = 2 * nq * d * 4 + 2 * nkv * (4 * d + rb)
    return kv, kv + other


def kernel_label(d, nq, nkv, kvd, paged, nchunks, combined):
    G = nq // nkv
    pg = "true" if paged else "false"
    if kvd and d in (64, 128):  # the matrix-core kernel (bf16 and Q8 caches)
        gh = 16 if G % 16 == 0 else 8 if G % 8 == 0 else 4 if G % 4 == 0 else 2 if G % 2 == 0 else 1
        s = (f"attn_mfma_kernel<{d},{gh},paged={pg},rope=true,"
             f"q8={'true' if kvd == 2 else 'false'}>")
    else:
        gh = 8 if G % 8 == 0 else 4 if G % 4 == 0 else 2 if G % 2 == 0 else 1
        gh = min(gh, 4) if d > 256 else gh  # at most 4 q heads a workgroup at d = 512
        t = {0: "float", 1: "bf16", 2: "q8"}[kvd]
        s = f"attn_kernel<{d},{gh},{t},paged={pg},rope=true>"
    if nchunks <= 1:
        return s + " (single chunk)"
    return s + (" (then combine_kernel: split-K merge)" if combined else
                " (split-K chunks merged in the same launch)")


def synthetic_q8(st, rows, nkv, d, sigma, np):
    """Q8 rows of the format (codes, then per-head fp32 scales): codes
    rint(32 N(0,1)) clipped to +-127, scale sigma/32 (values ~ N(0, sigma^2))."""
    codes = np.clip(np.rint(st.normal((rows, nkv * d)) * 32.0), -127, 127).astype(np.int8)
    scales = np.full((rows, nkv), sigma / 32.0, np.float32)
    return codes, scales


# ---------------------------------------------------------------------------
# workloads: inputs resident on the device, one step / attention-only launch,
# byte counts and the CPU-baseline sample

def contiguous_workload(args, cfg, lib, L, torch, np):
    from molot_amd import attn
    from molot_amd.synth import Stream, f32_to_bf16

    nq, nkv, d, pos = cfg["nq"], cfg["nkv"], cfg["d"], cfg["pos"]
    theta, window, kvd, sigma = cfg["theta"], cfg["window"], cfg["kvd"], cfg["sigma"]
    rb = row_bytes(kvd, d)
    n = pos + 1
    t0 = max(0, pos - window + 1) if window > 0 else 0
    n_att = n - t0
    kv_bytes, step_bytes = algorithmic_bytes(nq, nkv, d, n_att, rb)
    step_bytes += (d // 2) * 4
    R = lib.molot_hip_q8_row_bytes(nkv, d) if kvd == 2 else nkv * rb  # bytes per token
    cache_bytes = 2 * n * R
    layers = args.layers or max(2, math.ceil(COLD_BYTES / kv_bytes))
    scale = 1.0 / math.sqrt(d)

    st = Stream(1234)
    q_h = st.normal((nq, d))
    k_h = st.normal((nkv, d))
    v_h = st.normal((nkv, d))
    if kvd == 2:
        # token-major Q8 rows [n][R]: codes [nkv][d], then the nkv scales
        K_h = np.zeros((n, R), np.uint8)
        V_h = np.zeros_like(K_h)
        for X in (K_h, V_h):
            codes, scales = synthetic_q8(st, pos - t0, nkv, d, sigma, np)
            X[t0:pos, :nkv * d] = codes.view(np.uint8)
            X[t0:pos, nkv * d:nkv * d + 4 * nkv] = scales.view(np.uint8)
    else:
        K_h = np.zeros((n, nkv * d), np.float32)
        V_h = np.zeros_like(K_h)
        # only the attended rows are drawn (a window's earlier rows are never read)
        K_h[t0:pos] = st.normal((pos - t0, nkv * d), sigma)
        V_h[t0:pos] = st.normal((pos - t0, nkv * d), sigma)
    dt = {0: torch.float32, 1: torch.bfloat16, 2: torch.uint8}[kvd]

    def to_dev(a):
        if kvd != 1:
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
    wts = torch.from_numpy((1 + st.normal((2, d), 0.2)).astype(np.float32)).cuda()
    torch.cuda.synchronize()
    del K_h, V_h

    P = ctypes.c_void_p
    qp, kp, vp, ip, op = (P(t.data_ptr()) for t in (q, k_new, v_new, inv, O))
    qnp, knp = P(wts[0].data_ptr()), P(wts[1].data_ptr())
    Kp = [P(t.data_ptr()) for t in Ks]
    Vp = [P(t.data_ptr()) for t in Vs]

    def step(i, stream):
        l = i % layers
        if args.norms:
            rc = lib.molot_hip_decode_step_norm(qp, kp, vp, Kp[l], Vp[l], op, nq, nkv, d, pos, pos,
                                                qnp, knp, 1, 1e-6, ip, scale, window, kvd, stream)
        else:
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

    def cpu(args_):
        return cpu_baseline_contiguous(args_, q_h, k_h, v_h, nq, nkv, d, pos, theta, window, kvd,
                                       sigma, scale, kv_bytes)

    return SimpleNamespace(
        step=step, attention=attention, kv_bytes=kv_bytes, step_bytes=step_bytes, layers=layers,
        cache_desc=f"cache={cache_bytes / 2**20:.0f} MiB/layer dtype={dt}", paged=False,
        head_traffic=2 * nq * n_att * rb, cpu=cpu,
        config={"nq": nq, "nkv": nkv, "head_dim": d, "pos": pos, "n": n, "window": window,
                "rope_theta": theta, "batch": 1, "qkv_norms": bool(args.norms)},
        keep=(Ks, Vs, q, k_new, v_new, inv, O))


def paged_workload(args, cfg, lib, L, torch, np):
    """c4: B sequences with context U[lmin, lmax] from the seeded stream, one
    new token each; bf16 K/V pages [block][nkv][page][d] behind a shuffled
    block table (the tests' make_paged draws, same order and seed)."""
    from molot_amd import attn
    from molot_amd.synth import Stream, f32_to_bf16

    nq, nkv, d, B, page = cfg["nq"], cfg["nkv"], cfg["d"], cfg["batch"], cfg["page"]
    theta, window, kvd, sigma = cfg["theta"], cfg["window"], cfg["kvd"], cfg["sigma"]
    assert kvd in (1, 2) and window == 0
    rb = row_bytes(kvd, d)
    st = Stream(1234)
    q_h = st.normal((B, nq, d))
    k_h = st.normal((B, nkv, d))
    v_h = st.normal((B, nkv, d))
    Lc = st.uniform_int(cfg["lmin"], cfg["lmax"], B).astype(np.int32)  # context before the token
    n = Lc + 1
    blocks = (n + page - 1) // page
    nblk = int(blocks.sum()) + 7
    perm = st.permutation(nblk)
    max_blocks = int(blocks.max())
    bt = np.zeros((B, max_blocks), np.int32)
    o = 0
    for b in range(B):
        bt[b, :blocks[b]] = perm[o:o + blocks[b]]
        o += blocks[b]
    if kvd == 2:
        # Q8 blocks: codes [nkv][page][d], then scales [nkv][page]
        pools = []
        for _ in range(2):
            codes, scales = synthetic_q8(st, nblk * page, nkv, d, sigma, np)
            codes = codes.reshape(nblk, page, nkv, d).transpose(0, 2, 1, 3).reshape(nblk, -1)
            scales = scales.reshape(nblk, page, nkv).transpose(0, 2, 1).reshape(nblk, -1)
            pools.append(np.ascontiguousarray(np.concatenate(
                [codes.view(np.uint8), scales.view(np.uint8)], axis=1)))
        Kp_h, Vp_h = pools
    else:
        Kp_h = f32_to_bf16(st.normal((nblk, nkv, page, d), sigma))
        Vp_h = f32_to_bf16(st.normal((nblk, nkv, page, d), sigma))

    kv_bytes = 0
    step_bytes = (d // 2) * 4 + int(blocks.sum()) * 4  # RoPE table + block-table entries
    for b in range(B):
        kv, tot = algorithmic_bytes(nq, nkv, d, int(n[b]), rb)
        kv_bytes += kv
        step_bytes += tot + 4  # + its seq_lens entry
    cache_bytes = 2 * nblk * nkv * page * rb
    layers = args.layers or max(2, math.ceil(COLD_BYTES / kv_bytes))
    scale = 1.0 / math.sqrt(d)

    def to_dev_bf16(a):
        if kvd == 2:
            return torch.from_numpy(a).cuda()
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)

    K0, V0 = to_dev_bf16(Kp_h), to_dev_bf16(Vp_h)
    Ks = [K0] + [torch.empty_like(K0) for _ in range(layers - 1)]
    Vs = [V0] + [torch.empty_like(V0) for _ in range(layers - 1)]
    for i in range(1, layers):
        Ks[i].copy_(K0)
        Vs[i].copy_(V0)
    q = torch.from_numpy(q_h).cuda()
    k_new = torch.from_numpy(k_h).cuda()
    v_new = torch.from_numpy(v_h).cuda()
    bt_d = torch.from_numpy(bt.reshape(-1)).cuda()
    sl_d = torch.from_numpy(n.astype(np.int32)).cuda()
    inv = attn.rope_inv_freq(theta, d).cuda()
    O = torch.empty((B, nq, d), dtype=torch.float32, device="cuda")
    wts = torch.from_numpy((1 + st.normal((2, d), 0.2)).astype(np.float32)).cuda()
    torch.cuda.synchronize()
    max_len = int(n.max())

    P = ctypes.c_void_p
    qp, kp, vp, ip, op, btp, slp = (P(t.data_ptr())
                                    for t in (q, k_new, v_new, inv, O, bt_d, sl_d))
    qnp, knp = P(wts[0].data_ptr()), P(wts[1].data_ptr())
    Kp = [P(t.data_ptr()) for t in Ks]
    Vp = [P(t.data_ptr()) for t in Vs]

    def step(i, stream):
        l = i % layers
        if args.norms:
            rc = lib.molot_hip_decode_step_paged_norm(qp, kp, vp, Kp[l], Vp[l], op, btp, slp, None,
                                                      B, max_blocks, max_len, nq, nkv, d, page,
                                                      qnp, knp, 1, 1e-6, ip, scale, window, kvd,
                                                      stream)
        else:
            rc = lib.molot_hip_decode_step_paged(qp, kp, vp, Kp[l], Vp[l], op, btp, slp, None, B,
                                                 max_blocks, max_len, nq, nkv, d, page, ip, scale,
                                                 window, kvd, stream)
        if rc:
            raise L.MolotHipError(rc, "decode_step_paged")

    def attention(i, stream):
        l = i % layers
        rc = lib.molot_hip_attn_decode_paged(qp, Kp[l], Vp[l], op, btp, slp, None, B, max_blocks,
                                             max_len, nq, nkv, d, page, scale, window, kvd,
                                             stream)
        if rc:
            raise L.MolotHipError(rc, "attn_decode_paged")

    def cpu(args_):
        return cpu_baseline_paged(args_, q_h, k_h, v_h, Kp_h, Vp_h, bt, n, nq, nkv, d, page,
                                  theta, scale, kv_bytes, kvd)

    return SimpleNamespace(
        step=step, attention=attention, kv_bytes=kv_bytes, step_bytes=step_bytes, layers=layers,
        cache_desc=(f"{B} seqs, ctx {int(Lc.min())}..{int(Lc.max())} (sum {int(n.sum())}), "
                    f"{nblk} pages, cache={cache_bytes / 2**20:.0f} MiB/layer "
                    f"{'Q8' if kvd == 2 else 'bf16'}"),
        paged=True, head_traffic=2 * nq * int(n.sum()) * rb, cpu=cpu,
        config={"nq": nq, "nkv": nkv, "head_dim": d, "batch": B, "page": page,
                "ctx_min": int(Lc.min()), "ctx_max": int(Lc.max()), "tokens": int(n.sum()),
                "window": window, "rope_theta": theta, "qkv_norms": bool(args.norms)},
        keep=(Ks, Vs, q, k_new, v_new, bt_d, sl_d, inv, O))


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path would shard by KV head across GPUs with no exchange, "
              "but nothing here launches on more than one device.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from molot_amd import attn
    from molot_amd import lib as L

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    lib = L.load()
    torch.cuda.set_device(0)
    if args.split_chunk:
        attn.set_split_chunk(args.split_chunk)
    if args.wgs_per_cu:
        lib.molot_hip_set_tuning(args.wgs_per_cu)
    lib.molot_hip_set_merge(args.merge)
    lib.molot_hip_set_prefill_presplit(args.prefill_presplit)
    lib.molot_hip_set_block_order(args.block_order)

    cfg = CONFIGS[args.config]
    if "prompt" in cfg:
        return run_prefill(args, cfg, lib, L, torch, np)
    t_setup = time.time()
    make = paged_workload if "batch" in cfg else contiguous_workload
    wl = make(args, cfg, lib, L, torch, np)
    kvd = cfg["kvd"]
    log(args, f"setup {time.time() - t_setup:.1f}s: {args.config} layers={wl.layers} "
        f"{wl.cache_desc}")

    P = ctypes.c_void_p

    def cur_stream():
        return P(torch.cuda.current_stream().cuda_stream)

    step, attention = wl.step, wl.attention
    kv_bytes, step_bytes = wl.kv_bytes, wl.step_bytes

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
        probe = L.load_probe()
        for _ in range(3):
            L.check(probe.molot_probe_copy(P(dst.data_ptr()), P(src.data_ptr()), cb, cur_stream()),
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
    nch, chk = attn.last_plan()

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
    kname = "attn_mfma_kernel" if kvd and cfg["d"] in (64, 128) else "attn_kernel"
    log(args, f"{kname} {k1_us:.2f} us/launch -> {achieved:.0f} GB/s "
        f"(chunks {nch} x {chk} rows); combine {k2_us:.2f} us; "
        f"attention-only entry: {a1_us:.2f} + {a2_us:.2f} us")

    # ---- achievable streaming-read peak on this box (probe kernel, 4 GiB) ----
    probe_bytes = 4 << 30
    buf = torch.empty(probe_bytes // 4, dtype=torch.float32, device="cuda")
    buf.fill_(1.0)
    sink = torch.empty(1 << 16, dtype=torch.float32, device="cuda")
    probe = L.load_probe()
    with torch.cuda.stream(s):
        for _ in range(3):
            probe.molot_probe_read(P(buf.data_ptr()), probe_bytes, P(sink.data_ptr()), sink.numel(),
                                   sp)
        torch.cuda.synchronize()
        start.record(s)
        for _ in range(10):
            probe.molot_probe_read(P(buf.data_ptr()), probe_bytes, P(sink.data_ptr()), sink.numel(),
                                   sp)
        end.record(s)
    torch.cuda.synchronize()
    read_peak = 10 * probe_bytes / (start.elapsed_time(end) * 1e-3) / 1e9
    del buf
    log(args, f"streaming-read probe: {read_peak:.0f} GB/s")

    # ---- traffic measured by rocprofv3 PMC runs (committed summary), if it was
    # measured on this kernel source (molot_amd.rocprof stamps each entry) ----
    traffic, traffic_note = None, "no rocprofv3 PMC record for this config"
    try:
        from molot_amd.rocprof import source_hash
        with open(args.traffic) as f:
            ent = json.load(f).get(args.config, {})
        if ent and ent.get("source_sha256") == source_hash():
            traffic = ent.get("traffic_bytes_per_launch")
            traffic_note = "FETCH_SIZE + WRITE_SIZE (profiles/traffic.json, this kernel source)"
        elif ent:
            traffic_note = "profiles/traffic.json was measured on another kernel source"
    except (OSError, ValueError, AttributeError):
        pass

    # The boundary with host buffers (never `value`): the C++ drop-in's
    # decode call (DeviceKV::decode) given the reference's host vectors, which
    # it stages through a pinned mirror (q, k_new, v_new in one copy, q and o
    # back in one) and synchronizes, timed by tests/cpp/host_io_time against
    # the same call with device vectors (fp32 caches; built by build()).  Full
    # runs only (with the CPU baseline): under a profiler (--cpu-seconds 0)
    # its launches would join the trace.
    host_io = None
    timer = os.path.join(ROOT, "tests", "cpp", "host_io_time")
    if (not wl.paged and kvd == 0 and not args.norms and args.cpu_seconds > 0
            and os.path.exists(timer)):
        import subprocess
        cmd = [timer, str(cfg["nq"]), str(cfg["nkv"]), str(cfg["d"]), str(cfg["pos"]),
               str(cfg["window"]), "200", str(wl.layers)]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        vals = dict(kv.split("=") for kv in r.stdout.split()) if r.returncode == 0 else {}
        if "host_us" in vals:
            us_io, us_dev = float(vals["host_us"]), float(vals["device_us"])
            host_io = {"us_per_step": round(us_io, 2),
                       "kv_gbps": round(kv_bytes / (us_io * 1e-6) / 1e9, 1),
                       "device_vectors_us_per_step": round(us_dev, 2),
                       "timing": "200 synchronous DeviceKV::decode calls, host wall clock, "
                                 f"{wl.layers} layer caches cycled (tests/cpp/host_io_time)",
                       "buffers": "the reference's host q, k_new, v_new, ao, staged by the "
                                  "C++ drop-in through a pinned mirror"}
            log(args, f"C++ drop-in with host vectors: {us_io:.1f} us/call "
                f"({us_dev:.1f} with device vectors, synchronous calls)")

    config = {"workload": DESCR[args.config], "config": args.config}
    config.update(wl.config)
    config.update({"kv_layers_cycled": wl.layers, "timing": mode, "split_chunks": nch,
                   "chunk_rows": chk})
    out = {
        "metric": metric_name(cfg),
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {0: "f32", 1: "bf16-kv/f32-acc", 2: "q8-kv/f32-acc"}[kvd],
        "data": (f"synthetic (seeded N(0,{cfg['sigma']:g}) K/V"
                 + (" as Q8 codes rint(32 N(0,1)) with scale sigma/32" if kvd == 2 else "")
                 + ", N(0,1) q/k/v, splitmix64+Box-Muller, seed 1234)"),
        "config": config,
        "us_per_layer_step": round(us_step, 3),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "pct_of_measured_read_peak": round(100 * value / read_peak, 2),
        "measured_read_peak_gbps": round(read_peak, 1),
        "kv_bytes_per_step": kv_bytes,
        "algorithmic_bytes_per_step": step_bytes,
        "total_gbps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "head_traffic_gbps": round(wl.head_traffic / (ms_per_step * 1e-3) / 1e9, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_label(cfg["d"], cfg["nq"], cfg["nkv"], kvd, wl.paged, nch, k2_us > 0),
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "launch_us": round(k1_us, 3),
            "algorithmic_bytes_per_launch": step_bytes,
            "combine_launch_us": round(k2_us, 3),
            "step_gbps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        },
    }

    if host_io is not None:
        out["host_io"] = host_io
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = wl.cpu(args)
    print(json.dumps(out), flush=True)
    return 0


def run_prefill(args, cfg, lib, L, torch, np):
    """Prefill configs: one step = molot_hip_prefill_step for one layer (RoPE
    of the prompt's q and k, append of its M rows, causal attention); value =
    attention TFLOP/s, 4*d flops per (q head, query, attended key)."""
    from molot_amd import attn
    from molot_amd.synth import Stream

    nq, nkv, d, M, n0 = cfg["nq"], cfg["nkv"], cfg["d"], cfg["prompt"], cfg["n0"]
    theta, window = cfg["theta"], cfg["window"]
    N = n0 + M
    scale = 1.0 / math.sqrt(d)
    t0s = [max(0, n0 + m - window + 1) if window > 0 else 0 for m in range(M)]
    keys = sum(min(n0 + m + 1, N) - t0s[m] for m in range(M))
    flops = 4 * d * nq * keys
    t_setup = time.time()
    st = Stream(1234)
    q_h = st.normal((M, nq, d))
    k_h = st.normal((M, nkv, d))
    v_h = st.normal((M, nkv, d))
    K_h = np.zeros((N, nkv * d), np.float32)
    V_h = np.zeros_like(K_h)
    K_h[:n0] = st.normal((n0, nkv * d))
    V_h[:n0] = st.normal((n0, nkv * d))
    q, kn, vn = (torch.from_numpy(x).cuda() for x in (q_h, k_h, v_h))
    K, V = torch.from_numpy(K_h).cuda(), torch.from_numpy(V_h).cuda()
    inv = attn.rope_inv_freq(theta, d).cuda()
    O = torch.empty((M, nq, d), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    log(args, f"setup {time.time() - t_setup:.1f}s: {args.config} M={M} after {n0}, "
        f"{keys} (query, key) pairs per head, {flops / 1e9:.1f} GFLOP/step")
    P = ctypes.c_void_p
    qp, kp, vp, Kp, Vp, ip, op = (P(t.data_ptr()) for t in (q, kn, vn, K, V, inv, O))

    def step(i, stream):
        rc = lib.molot_hip_prefill_step(qp, kp, vp, Kp, Vp, op, nq, nkv, d, M, n0, n0, None, None,
                                        0, 1e-6, ip, scale, window, 0, stream)
        if rc:
            raise L.MolotHipError(rc, "prefill_step")

    def cur_stream():
        return P(torch.cuda.current_stream().cuda_stream)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    steps = max(1, args.steps // 25)  # each step is ~100x a decode step
    with torch.cuda.stream(s):
        sp = cur_stream()
        for i in range(max(2, args.warmup // 10)):
            step(i, sp)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(s)
        for i in range(steps):
            step(i, sp)
        end.record(s)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    value = flops / (ms * 1e-3) / 1e12
    log(args, f"eager: {steps} steps, {ms * 1e3:.1f} us/step -> {value:.1f} TFLOP/s "
        f"({100 * value / PIECE_PEAK_TFLOPS:.1f}% of the 3-product matrix ceiling, "
        f"{100 * value / FP32_MFMA_PEAK_TFLOPS:.1f}% of the fp32 MFMA peak)")
    with torch.cuda.stream(s):
        L.check(lib.molot_hip_profile_begin(steps), "profile_begin")
        for i in range(steps):
            step(i, sp)
    am, cm = ctypes.c_float(), ctypes.c_float()
    na, nc = ctypes.c_int(), ctypes.c_int()
    L.check(lib.molot_hip_profile_end(ctypes.byref(am), ctypes.byref(cm), ctypes.byref(na),
                                      ctypes.byref(nc)), "profile_end")
    k_us = am.value / max(1, na.value) * 1e3
    achieved = flops / (k_us * 1e-6) / 1e12
    kname = "prefill_mfma16_kernel"
    log(args, f"{kname} {k_us:.1f} us/launch -> {achieved:.1f} TFLOP/s")
    out = {
        "metric": "prefill attention TFLOP/s (causal, 4*d flops per head x query x key)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": max(2, args.warmup // 10),
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) q/k/v and cache, splitmix64+Box-Muller, seed 1234)",
        "config": {"workload": DESCR[args.config], "config": args.config, "nq": nq, "nkv": nkv,
                   "head_dim": d, "prompt": M, "cached": n0, "window": window,
                   "rope_theta": theta, "timing": "eager"},
        "flops_per_step": flops,
        # peak: the ceiling of the instructions the kernel issues.  It takes
        # a score term and a PV term each as three fp16 piece products on the
        # 2500 TFLOP/s dense matrix cores, so 2500 / 3 fp32-equivalent
        # TFLOP/s; beside it the ceiling of six bf16 products for both (the
        # kernel before its fp16 pieces) and the fp32 matrix peak (the
        # precision the products keep).
        "roofline": {"bound": "mfma", "kernel": "%s<%d,float>" % (kname, d),
                     "achieved": round(achieved, 2), "peak": round(PIECE_PEAK_TFLOPS, 1),
                     "unit": "TFLOP/s", "frac": round(achieved / PIECE_PEAK_TFLOPS, 4),
                     "traffic": None, "launch_us": round(k_us, 2),
                     "peak_basis": "dense fp16 MFMA 2500 TFLOP/s / 3 piece products "
                                   "(scores and PV: 3 fp16 each)",
                     "six_product_peak": round(SIX_PRODUCT_PEAK_TFLOPS, 1),
                     "frac_of_six_product_peak": round(achieved / SIX_PRODUCT_PEAK_TFLOPS, 4),
                     "fp32_mfma_peak": FP32_MFMA_PEAK_TFLOPS,
                     "frac_of_fp32_mfma_peak": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4)},
    }
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline_prefill(args, q_h, K_h, V_h, nq, nkv, d, M, N, n0,
                                                   scale, window, flops)
    print(json.dumps(out), flush=True)
    return 0


def cpu_baseline_prefill(args, q_h, K_h, V_h, nq, nkv, d, M, N, n0, scale, window, flops):
    """The reference's attn_prefill_gqa (gemm.h:409-446, oracle/_ref) on the
    host cores over the same cache (the new rows left as drawn: timing
    only), whole calls within the time budget."""
    import numpy as np

    import oracle
    cores, host = host_cpu()
    cores = args.cpu_threads or cores
    O = np.empty_like(q_h)
    P = oracle._p
    kind = "reference" if oracle.ref_available() else "port"
    pool = oracle.RefPool(cores) if kind == "reference" else None

    def one(i):
        if kind == "reference":
            oracle.ref().ref_attn_prefill_gqa(P(q_h), P(K_h), P(V_h), P(O), nq, nkv, M, N, d,
                                              scale, n0, window, pool.h)
        else:
            oracle.lib().orc_attn_prefill(P(q_h), P(K_h), P(V_h), P(O), nq, nkv, M, N, d, scale,
                                          n0, window, 0, cores)

    steps, el = _cpu_loop(args, one)
    if pool:
        pool.close()
    ms = el / steps * 1e3
    tf = flops / (ms * 1e-3) / 1e12
    log(args, f"cpu baseline ({kind}, {cores} threads): {ms:.1f} ms/step -> {tf * 1e3:.1f} GFLOP/s")
    return {"value": round(tf, 5), "unit": "TFLOP/s", "cores": cores, "kind": kind,
            "ms_per_step": round(ms, 3), "host": host,
            "sample": f"{steps} calls of attn_prefill_gqa on the {args.config} workload, "
                      f"{el:.1f} s, ThreadPool" if kind == "reference" else
                      f"{steps} calls of the oracle's prefill, {el:.1f} s, OpenMP"}


def _cpu_loop(args, one):
    for i in range(2):  # warmup 2 (bench/bench.cc:45-52)
        one(i)
    t0 = time.perf_counter()
    steps = 0
    while True:
        one(steps)
        steps += 1
        el = time.perf_counter() - t0
        if (el >= args.cpu_seconds and steps >= 3) or steps >= 100000:
            return steps, el


def cpu_baseline_contiguous(args, q_h, k_h, v_h, nq, nkv, d, pos, theta, window, kvd, sigma,
                            scale, kv_bytes):
    """The reference's decode step on the host cores (bounded sample).

    kind "reference": include/molot/attn.h + forward.h's rope/append sequence,
    compiled from the reference headers into oracle/_ref (ThreadPool with
    `cores` threads).  Falls back to the oracle's C restatement ("port") when
    that library is absent or the host lacks AVX512F.  bf16 configs have no
    reference counterpart: the reference runs on the widened values."""
    import numpy as np

    import oracle
    from molot_amd.synth import Stream, bf16_to_f32, f32_to_bf16

    cores, host = host_cpu()
    cores = args.cpu_threads or cores
    n = pos + 1
    t0 = max(0, pos - window + 1) if window > 0 else 0
    st = Stream(4321)
    S = nkv * d
    # rotate copies so the attended KV exceeds the host LLC (DRAM-cold); rows
    # before a window are never touched, so np.zeros leaves them unbacked
    per_copy = 2 * (n - t0) * S * 4
    copies = max(2, math.ceil(512 * 2**20 / per_copy))
    rows = st.normal((pos - t0, S), sigma)
    rows_v = st.normal((pos - t0, S), sigma)
    if kvd == 1:
        rows = bf16_to_f32(f32_to_bf16(rows))
        rows_v = bf16_to_f32(f32_to_bf16(rows_v))
    Ks, Vs = [], []
    for _ in range(copies):
        K = np.zeros((n, S), np.float32)
        V = np.zeros_like(K)
        K[t0:pos] = rows
        V[t0:pos] = rows_v
        Ks.append(K)
        Vs.append(V)
    del rows, rows_v
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

    steps, el = _cpu_loop(args, one)
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
        "host": host,
        "sample": (f"{steps} layer-steps of {args.config} (rope q/k + append + "
                   f"attn_decode_gqa_cache, n={n}, rows {t0}..{n - 1}) cycling {copies} KV "
                   f"copies of {per_copy / 2**20:.0f} MiB attended, {el:.1f} s; "
                   + ("reference headers via oracle/_ref, ThreadPool" if kind == "reference"
                      else "oracle C restatement, OpenMP static over heads")
                   + ("; bf16 values widened to fp32 (no reference bf16 path)" if kvd == 1
                      else "; fp32 rows of the same shape (no reference Q8 cache)" if kvd == 2
                      else "")),
    }


def cpu_baseline_paged(args, q_h, k_h, v_h, Kp_h, Vp_h, bt, n, nq, nkv, d, page, theta, scale,
                       kv_bytes, kvd=1):
    """c4 on the host cores: the reference's decode step (rope q/k, append,
    attn_decode_gqa_cache) once per sequence, over per-sequence contiguous
    fp32 caches gathered from the pages and widened from bf16 (or
    dequantized from Q8).  The reference has neither a paged nor a bf16 or
    Q8 cache, so this is the reference algorithm on the same values, not a
    reference run of the same format; the contiguous fp32 copies are 2x
    (bf16) or ~4x (Q8) the GPU's bytes, and the GB/s reported is the GPU
    workload's KV bytes over the CPU time."""
    import numpy as np

    import oracle
    from molot_amd.synth import bf16_to_f32

    cores, host = host_cpu()
    cores = args.cpu_threads or cores
    B = len(n)
    S = nkv * d
    Kc, Vc = [], []
    def widen(pages):  # [blocks][nkv][page][d] fp32 values of bf16 or Q8 pages
        if kvd == 1:
            return bf16_to_f32(pages)
        m = pages.shape[0]
        codes = pages[:, :nkv * page * d].view(np.int8).astype(np.float32)
        sc = np.ascontiguousarray(pages[:, nkv * page * d:]).view(np.float32)
        return codes.reshape(m, nkv, page, d) * sc.reshape(m, nkv, page, 1)

    for b in range(B):
        nb = int(n[b])
        blk = bt[b, :(nb + page - 1) // page]
        for src, dst in ((Kp_h, Kc), (Vp_h, Vc)):
            x = widen(src[blk]).transpose(0, 2, 1, 3).reshape(-1, S)[:nb]
            dst.append(np.ascontiguousarray(x))
    inv = oracle.rope_inv_freq(theta, d)
    O = np.empty((nq, d), np.float32)
    P = oracle._p
    kind = "reference" if oracle.ref_available() else "port"
    pool = oracle.RefPool(cores) if kind == "reference" else None

    def one(i):
        for b in range(B):
            nb = int(n[b])
            q = q_h[b].copy()
            k = k_h[b].copy()
            v = v_h[b].copy()
            if kind == "reference":
                rc = oracle.ref().ref_decode_step(P(q), P(k), P(v), P(Kc[b]), P(Vc[b]), P(O), nq,
                                                  nkv, d, nb - 1, nb, nb - 1, P(inv), scale, 0,
                                                  pool.h)
                assert rc == 0
            else:
                oracle.lib().orc_decode_step(P(q), P(k), P(v), P(Kc[b]), P(Vc[b]), P(O), nq,
                                             nkv, d, nb - 1, nb - 1, P(inv), scale, 0, 0, cores)

    steps, el = _cpu_loop(args, one)
    if pool:
        pool.close()
    ms = el / steps * 1e3
    gbps = kv_bytes / (ms * 1e-3) / 1e9
    log(args, f"cpu baseline ({kind}, {cores} threads): {ms:.3f} ms/step -> {gbps:.1f} GB/s")
    fp32_mib = sum(x.nbytes for x in Kc + Vc) / 2**20
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": kind,
        "ms_per_step": round(ms, 4),
        "host": host,
        "sample": (f"{steps} batch-steps of {args.config} ({B} sequences, each rope q/k + append + "
                   f"attn_decode_gqa_cache over its contiguous fp32 cache, {fp32_mib:.0f} MiB in "
                   f"all), {el:.1f} s; "
                   + ("reference headers via oracle/_ref, ThreadPool" if kind == "reference"
                      else "oracle C restatement, OpenMP static over heads")
                   + ("; Q8 pages gathered and dequantized to fp32 (the reference has no "
                      "paged or Q8 cache)" if kvd == 2 else
                      "; bf16 pages gathered and widened to fp32 (the reference has no paged "
                      "or bf16 cache)")),
    }


if __name__ == "__main__":
    sys.exit(main())
