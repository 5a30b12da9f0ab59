"""Parity of the HIP prefill attention (include/molot/gemm.h:409-446) and of
one layer's fused prefill (forward.h:367-399) with the oracle (MI355X only).

Every call goes through the C ABI.  Bar: normwise max|gpu-ref|/max|ref|
<= 1e-5 against the oracle on the same values (fp32 caches, and bf16 caches
widened: the kernel itself is fp32-accurate on those values); RoPE outputs
and the appended rows within fp32 rounding of the oracle's.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import normwise_err
from gpu_util import dev, dev_bf16, host
from molot_amd import attn
from molot_amd.synth import Stream, bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

TOL = 1e-5
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def announce(msg):
    print(f"[case] {msg}", flush=True)


def cache(st, N, nkv, d, bf16):
    K = st.normal((N, nkv * d))
    V = st.normal((N, nkv * d))
    if bf16:
        return f32_to_bf16(K), f32_to_bf16(V)
    return K, V


def on_dev(x):
    return dev_bf16(x) if x.dtype == np.uint16 else dev(x)


@pytest.mark.parametrize("name", ["prefill_g4_d64", "prefill_norm_win_d128"])
def test_golden_prefill_step(gpu, name):
    """Against the compiled reference's forward.h prefill sequence."""
    g = golden(name)
    nq, nkv, d, M, pos0 = (int(g[k]) for k in ("nq", "nkv", "d", "M", "pos0"))
    norms = int(g["norms"])
    K = np.zeros((pos0 + M, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos0], V[:pos0] = g["K"], g["V"]
    q, Kd, Vd = dev(g["q"]), dev(K), dev(V)
    O = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(q, dev(g["k_new"]), dev(g["v_new"]), Kd, Vd, O, nq, nkv, d, M, pos0, pos0,
                      dev(g["inv_freq"]), float(g["scale"]), int(g["window"]),
                      q_norm=dev(g["q_norm"]) if norms else None,
                      k_norm=dev(g["k_norm"]) if norms else None, v_norm=bool(norms),
                      eps=float(g["eps"]))
    np.testing.assert_allclose(host(q), g["q_rot"], rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(host(Kd)[pos0:], g["K_after"], rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(host(Vd)[pos0:], g["V_after"], rtol=1e-6, atol=1e-7)
    assert normwise_err(host(O), g["O"]) < TOL


@pytest.mark.parametrize("nq,nkv,d,M,N,pos0,window,bf16", [
    (32, 8, 128, 100, 100, 0, 0, False),     # fresh prompt
    (32, 8, 128, 77, 1077, 1000, 0, False),  # appended to a context
    (8, 4, 256, 50, 3050, 3000, 1024, False),  # gemma-style window, d256
    (8, 4, 256, 70, 170, 100, 33, True),
    (64, 8, 128, 33, 533, 500, 0, True),     # G = 8
    (32, 2, 64, 21, 71, 50, 0, False),       # G = 16
    (16, 16, 64, 65, 65, 0, 0, True),        # G = 1
    (12, 4, 128, 30, 60, 30, 7, False),      # G = 3
    (8, 2, 64, 12, 30, 25, 0, False),        # pos0 + M > N: causal end clipped at N
    (8, 2, 128, 1, 500, 499, 0, False),      # a single query
])
def test_prefill_vs_oracle(gpu, nq, nkv, d, M, N, pos0, window, bf16):
    announce(f"prefill {nq}/{nkv}/{d} M={M} N={N} pos0={pos0} win={window} bf16={bf16}")
    st = Stream(M + N + d + nq)
    Q = st.normal((M, nq, d))
    K, V = cache(st, N, nkv, d, bf16)
    O = torch.empty((M, nq, d), device="cuda")
    scale = 1 / math.sqrt(d)
    attn.attn_prefill_gqa(dev(Q), on_dev(K), on_dev(V), O, nq, nkv, M, N, d, scale, pos0, window)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, scale, pos0, window)
    err = normwise_err(host(O), R)
    print(f"prefill normwise err {err:.3e}", flush=True)
    assert err < TOL


def test_prefill_empty_cases(gpu):
    """Queries whose window holds no slot get O = 0; an empty cache gives 0."""
    st = Stream(70)
    nq, nkv, d = 8, 2, 64
    Q = st.normal((4, nq, d))
    K, V = cache(st, 10, nkv, d, False)
    O = torch.full((4, nq, d), 5.0, device="cuda")
    # positions 40..43 with window 5 over a 10-slot cache: nothing attended
    attn.attn_prefill_gqa(dev(Q), dev(K), dev(V), O, nq, nkv, 4, 10, d, 0.125, 40, 5)
    assert np.all(host(O) == 0)
    O.fill_(5.0)
    attn.attn_prefill_gqa(dev(Q), dev(K), dev(V), O, nq, nkv, 4, 0, d, 0.125, 0, 0)
    assert np.all(host(O) == 0)


def test_prefill_single_query_matches_decode_kernel(gpu):
    """M = 1 through the prefill kernel equals the decode kernel's attention."""
    st = Stream(71)
    nq, nkv, d, N = 32, 8, 128, 4097
    Q = st.normal((1, nq, d))
    K, V = cache(st, N, nkv, d, False)
    Op = torch.empty((1, nq, d), device="cuda")
    Od = torch.empty((nq, d), device="cuda")
    attn.attn_prefill_gqa(dev(Q), dev(K), dev(V), Op, nq, nkv, 1, N, d, 0.088, N - 1, 0)
    attn.attn_decode_gqa_cache(dev(Q[0]), dev(K), dev(V), Od, nq, nkv, N, d, 0.088, N - 1, 0)
    assert normwise_err(host(Op)[0], host(Od)) < 2e-6


@pytest.mark.parametrize("bf16", [False, True])
def test_prefill_step_vs_oracle(gpu, bf16):
    """One layer's prefill with norms: 200 prompt tokens after 300 cached."""
    announce(f"prefill step 32q/8kv/d128 M=200 after 300 bf16={bf16}")
    st = Stream(72 + bf16)
    nq, nkv, d, M, n0 = 32, 8, 128, 200, 300
    q = st.normal((M, nq, d), 2.0)
    k = st.normal((M, nkv, d), 2.0)
    v = st.normal((M, nkv, d), 2.0)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K, V = cache(st, n0 + M, nkv, d, bf16)
    K[n0:] = 0
    V[n0:] = 0
    inv = oracle.rope_inv_freq(500000.0, d)
    qd, Kd, Vd = dev(q), on_dev(K), on_dev(V)
    O = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, M, n0, n0, dev(inv), 0.088, 0,
                      q_norm=dev(qn), k_norm=dev(kn), v_norm=True, eps=1e-6)
    Kc, Vc = K.copy(), V.copy()
    oq, oO = oracle.prefill_step(q, k, v, Kc, Vc, nq, nkv, d, M, n0, n0, qn, kn, 1, 1e-6, inv,
                                 0.088, 0)
    np.testing.assert_allclose(host(qd), oq, rtol=2e-6, atol=4e-6)
    if bf16:  # the normed rows may differ by an fp32 ulp before their bf16 rounding
        Kh = bf16_to_f32(host(Kd.view(torch.int16)).view(np.uint16))
        Vh = bf16_to_f32(host(Vd.view(torch.int16)).view(np.uint16))
        assert np.max(np.abs(Kh - bf16_to_f32(Kc))) <= 8e-3 * np.max(np.abs(bf16_to_f32(Kc)))
        assert np.max(np.abs(Vh - bf16_to_f32(Vc))) <= 8e-3 * np.max(np.abs(bf16_to_f32(Vc)))
        # the attention itself against the oracle on the GPU's own cache rows
        R = oracle.attn_prefill(host(qd), host(Kd.view(torch.int16)).view(np.uint16),
                                host(Vd.view(torch.int16)).view(np.uint16), nq, nkv, M, n0 + M,
                                d, 0.088, n0, 0)
        assert normwise_err(host(O), R) < TOL
        assert normwise_err(host(O), oO) < 2e-2
    else:
        np.testing.assert_allclose(host(Kd), Kc, rtol=2e-6, atol=4e-6)
        np.testing.assert_allclose(host(Vd), Vc, rtol=1e-6, atol=1e-7)
        assert normwise_err(host(O), oO) < TOL


@pytest.mark.parametrize("nq,nkv,d,bf16", [(32, 8, 128, False), (32, 8, 128, True),
                                           (8, 2, 64, False), (8, 4, 256, False),
                                           (8, 4, 256, True)])
def test_prefill_step_paged_matches_contiguous(gpu, nq, nkv, d, bf16):
    """The paged prefill step (shuffled 16-row pages, spare blocks) on the
    same logical rows as the contiguous one: the same kernel arithmetic, so
    O, the rotated q and the appended rows agree bit for bit; O also against
    the oracle on the contiguous cache."""
    announce(f"paged prefill step {nq}/{nkv}/{d} bf16={bf16}")
    st = Stream(91 + d + bf16)
    M, n0, page, spare = 77, 300, 16, 5
    cap = n0 + M
    q = st.normal((M, nq, d))
    k = st.normal((M, nkv, d))
    v = st.normal((M, nkv, d))
    K, V = cache(st, cap, nkv, d, bf16)
    K[n0:] = 0
    V[n0:] = 0
    nb = (cap + page - 1) // page
    nblk = nb + spare
    row = st.permutation(nblk)[:nb].astype(np.int32)
    Kp = np.zeros((nblk, nkv, page, d), K.dtype)
    Vp = np.zeros((nblk, nkv, page, d), V.dtype)
    for t in range(n0):
        Kp[row[t // page], :, t % page] = K[t].reshape(nkv, d)
        Vp[row[t // page], :, t % page] = V[t].reshape(nkv, d)
    inv = dev(oracle.rope_inv_freq(500000.0, d))
    s = 1 / math.sqrt(d)
    qc, qp = dev(q), dev(q)
    Kc, Vc = on_dev(K), on_dev(V)
    Kpd, Vpd = on_dev(Kp.reshape(nblk, -1)), on_dev(Vp.reshape(nblk, -1))
    Oc = torch.empty((M, nq, d), device="cuda")
    Op = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(qc, dev(k), dev(v), Kc, Vc, Oc, nq, nkv, d, M, n0, n0, inv, s, 0)
    attn.prefill_step_paged(qp, dev(k), dev(v), Kpd, Vpd, Op, torch.from_numpy(row).cuda(), nb,
                            page, nq, nkv, d, M, n0, n0, inv, s, 0)
    torch.cuda.synchronize()
    assert torch.equal(qp, qc)
    assert torch.equal(Op, Oc)
    Kph = host(Kpd.view(torch.int16) if bf16 else Kpd).reshape(nblk, nkv, page, d)
    Kch = host(Kc.view(torch.int16) if bf16 else Kc)
    for t in range(n0, cap):
        assert np.array_equal(Kph[row[t // page], :, t % page].reshape(-1), Kch[t]), t
    R = oracle.attn_prefill(host(qc), host(Kc.view(torch.int16)).view(np.uint16) if bf16 else
                            host(Kc), host(Vc.view(torch.int16)).view(np.uint16) if bf16 else
                            host(Vc), nq, nkv, M, cap, d, s, n0, 0)
    assert normwise_err(host(Oc), R) < TOL


def _prefill_both(run):
    """run() with the keys split once per launch (the default) and per
    staged tile; returns both outputs."""
    try:
        attn.set_prefill_presplit(True)
        o1 = run()
        attn.set_prefill_presplit(False)
        o0 = run()
    finally:
        attn.set_prefill_presplit(True)
    return o1, o0


@pytest.mark.parametrize("nq,nkv,d,M,N,pos0,window,kv", [
    (32, 8, 128, 300, 1300, 1000, 0, "f32"),    # 8 waves, two tile buffers
    (8, 4, 256, 70, 3070, 3000, 1024, "f32"),   # fp32 d256: two K buffers and one V, window
    (32, 2, 64, 40, 90, 50, 0, "f32"),          # d64
    (8, 2, 128, 5, 40, 35, 0, "f32"),           # few rows: the 4-wave grid
    (8, 4, 256, 33, 233, 200, 37, "f32"),       # window cutting inside a tile
    (32, 8, 128, 77, 1077, 1000, 0, "q8"),
    (8, 2, 64, 50, 3050, 3000, 1024, "q8"),
])
def test_prefill_presplit_matches_per_tile(gpu, nq, nkv, d, M, N, pos0, window, kv):
    """fp32 and Q8 caches: the keys split into bf16 pieces once per launch
    (pf_split_kernel) and copied into LDS by direct loads give the bits of
    the per-tile split (the same pieces, the same products), and the
    oracle's result."""
    announce(f"presplit {nq}/{nkv}/{d} M={M} N={N} pos0={pos0} win={window} {kv}")
    st = Stream(M + N + 3 * d + nq)
    Q = st.normal((M, nq, d))
    if kv == "q8":
        K, V = (oracle.q8_cache(st.normal((N, nkv * d)), nkv, d) for _ in range(2))
        Kd, Vd = (torch.from_numpy(np.ascontiguousarray(x, dtype=np.uint8)).cuda() for x in (K, V))
    else:
        K, V = cache(st, N, nkv, d, False)
        Kd, Vd = dev(K), dev(V)
    s = 1 / math.sqrt(d)
    Qd = dev(Q)

    def run():
        O = torch.full((M, nq, d), float("nan"), device="cuda")
        attn.attn_prefill_gqa(Qd, Kd, Vd, O, nq, nkv, M, N, d, s, pos0, window)
        return host(O)

    o1, o0 = _prefill_both(run)
    assert np.array_equal(o1, o0)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, window)
    err = normwise_err(o1, R)
    print(f"presplit normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("d,q8", [(128, False), (256, False), (64, True)])
def test_prefill_presplit_paged(gpu, d, q8):
    """The paged prefill over shuffled pages: pieces gathered through the
    block table once per launch, the same bits as the per-tile split."""
    announce(f"presplit paged d={d} q8={q8}")
    st = Stream(300 + d + q8)
    nq, nkv, M, n0, page, spare = 16, 4, 60, 400, 16, 3
    N = n0 + M
    nb = (N + page - 1) // page
    nblk = nb + spare
    row = st.permutation(nblk)[:nb].astype(np.int32)
    Q = st.normal((M, nq, d))
    if q8:
        rb = oracle.q8_block_bytes(nkv, d, page)
        Kp = np.zeros((nblk, rb), np.uint8)
        Vp = np.zeros((nblk, rb), np.uint8)
        for X in (Kp, Vp):
            codes = np.clip(np.rint(st.normal((nblk, nkv, page, d)) * 32), -127, 127).astype(np.int8)
            scales = (np.abs(st.normal((nblk, nkv, page))) * 0.03 + 0.01).astype(np.float32)
            X[:, :nkv * page * d] = codes.reshape(nblk, -1).view(np.uint8)
            X[:, nkv * page * d:nkv * page * d + 4 * nkv * page] = scales.reshape(nblk, -1).view(np.uint8)
        Kd, Vd = (torch.from_numpy(x).cuda() for x in (Kp, Vp))
    else:
        Kp = st.normal((nblk, nkv * page * d))
        Vp = st.normal((nblk, nkv * page * d))
        Kd, Vd = dev(Kp), dev(Vp)
    bt = torch.from_numpy(row).cuda()
    s = 1 / math.sqrt(d)
    Qd = dev(Q)

    def run():
        O = torch.full((M, nq, d), float("nan"), device="cuda")
        attn.attn_prefill_paged(Qd, Kd, Vd, O, bt, nb, page, nq, nkv, M, N, d, s, n0, 0)
        return host(O)

    o1, o0 = _prefill_both(run)
    assert np.isfinite(o1).all()
    assert np.array_equal(o1, o0)


def _key_splits(M, N, nq, nkv, pos0, cus):
    """The launch's key split count for an unwindowed prefill on 8-wave
    workgroups of 128 query rows: the query blocks' workgroups below the
    CU count take ceil(cus / workgroups) splits, at most 16 and at least 4
    key tiles of 32 each."""
    nqb = -(-M * (nq // nkv) // 128)
    if nqb * nkv >= cus:
        return 1
    tiles = (min(pos0 + M, N) + 31) // 32
    return max(1, min(16, -(-cus // (nqb * nkv)), tiles // 4))


@pytest.mark.parametrize("d,M,splits", [(64, 256, 8), (128, 352, 6), (256, 256, 8),
                                        (96, 352, 6), (40, 256, 8), (128, 512, 4),
                                        (256, 512, 4), (64, 512, 4)])
def test_prefill_split_merge_widths(gpu, d, M, splits):
    """The merge of a prompt's key splits (combine_rows_kernel) at each lane
    width (4 outputs a lane at d = 256, 2 at 128, 1 at 64), over up to 4 and
    up to 8 splits, and at padded head dims (96 in 128, 40 in 64): 16q/4kv
    after 1000 cached rows against the oracle."""
    nq, nkv, pos0 = 16, 4, 1000
    N = pos0 + M
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if _key_splits(M, N, nq, nkv, pos0, cus) != splits:
        pytest.skip(f"{cus} CUs: this shape takes another split count")
    announce(f"prefill split merge d={d} M={M} splits={splits}")
    st = Stream(900 + d + M)
    Q = st.normal((M, nq, d))
    K, V = cache(st, N, nkv, d, False)
    s = 1 / math.sqrt(d)
    O = torch.empty((M, nq, d), device="cuda")
    attn.attn_prefill_gqa(dev(Q), dev(K), dev(V), O, nq, nkv, M, N, d, s, pos0, 0)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, 0)
    err = normwise_err(host(O), R)
    print(f"split merge normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("kv", ["f32", "q8"])
@pytest.mark.parametrize("presplit", [True, False])
def test_prefill_row_scales(gpu, kv, presplit):
    """The scores over fp32 and Q8 values take q and K rows as two fp16
    pieces of the row scaled by a power of two.  K rows 2^-30 .. 2^30 apart
    and q rows with three channels 1000x the rest, scaled so that the
    largest scores stay near 5 and the softmax mixes rows of every scale,
    on both splits of the keys, against the oracle."""
    announce(f"prefill row scales kv={kv} presplit={presplit}")
    nq, nkv, d, M, N, pos0 = 16, 4, 128, 64, 1064, 1000
    st = Stream(950 + (kv == "q8") + 2 * presplit)
    e = np.random.default_rng(951).integers(-30, 31, size=N)
    K = (st.normal((N, nkv * d)) * np.exp2(e)[:, None]).astype(np.float32)
    V = st.normal((N, nkv * d))
    Q = st.normal((M, nq, d))
    Q[:, :, [5, 40, 99]] *= 1000.0
    Q = (Q * 2.0 ** -30 / 30).astype(np.float32)
    if kv == "q8":
        K, V = oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
        Kd = torch.from_numpy(np.ascontiguousarray(K, dtype=np.uint8)).cuda()
        Vd = torch.from_numpy(np.ascontiguousarray(V, dtype=np.uint8)).cuda()
    else:
        Kd, Vd = dev(K), dev(V)
    s = 1 / math.sqrt(d)
    O = torch.empty((M, nq, d), device="cuda")
    attn.set_prefill_presplit(presplit)
    try:
        attn.attn_prefill_gqa(dev(Q), Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)
    finally:
        attn.set_prefill_presplit(True)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, 0)
    err = normwise_err(host(O), R)
    print(f"row scales normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("kv", ["f32", "q8"])
@pytest.mark.parametrize("presplit", [True, False])
def test_prefill_v_row_scales(gpu, kv, presplit):
    """PV over fp32 and Q8 values takes V rows as two fp16 pieces of the row
    scaled by a power of two, the rows' units folded into P, keys more than
    2^7 below a tile's largest unit in further bands.  V rows 2^-20 .. 2^20
    apart, with each key's score lowered by its row's exponent (q channel 0
    times K channel 0 adds -e ln 2), so that every scale contributes to O
    alike and a band dropped or misweighted shows; against the oracle."""
    announce(f"prefill V row scales kv={kv} presplit={presplit}")
    nq, nkv, d, M, N, pos0 = 16, 4, 128, 64, 1064, 1000
    st = Stream(960 + (kv == "q8") + 2 * presplit)
    e = np.random.default_rng(961).integers(-20, 21, size=N)
    s = 1 / math.sqrt(d)
    c = 8.0
    V = (st.normal((N, nkv * d)) * np.exp2(e)[:, None]).astype(np.float32)
    K = st.normal((N, nkv * d))
    for h in range(nkv):
        K[:, h * d] = -e * math.log(2) / (c * s)
    K = K.astype(np.float32)
    Q = st.normal((M, nq, d))
    Q[:, :, 0] = c
    Q = Q.astype(np.float32)
    if kv == "q8":
        K, V = oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
        Kd = torch.from_numpy(np.ascontiguousarray(K, dtype=np.uint8)).cuda()
        Vd = torch.from_numpy(np.ascontiguousarray(V, dtype=np.uint8)).cuda()
    else:
        Kd, Vd = dev(K), dev(V)
    O = torch.empty((M, nq, d), device="cuda")
    attn.set_prefill_presplit(presplit)
    try:
        attn.attn_prefill_gqa(dev(Q), Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)
    finally:
        attn.set_prefill_presplit(True)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, 0)
    err = normwise_err(host(O), R)
    print(f"V row scales normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("kv", ["f32", "q8"])
@pytest.mark.parametrize("presplit", [True, False])
def test_prefill_ramp_scales(gpu, kv, presplit):
    """Scores that rise along the keys by 40 (log2 units) while the V rows
    fall by 2^-40, so that p * v stays alike: the running max keeps moving,
    and each query row's PV unit has to follow o down with it (a unit kept
    at the early keys' scale would hold the late keys' terms to 2^-40 of
    it).  Prompt rows see the whole ramp; against the oracle."""
    announce(f"prefill ramp scales kv={kv} presplit={presplit}")
    nq, nkv, d, M, N, pos0 = 16, 4, 128, 64, 1064, 1000
    st = Stream(970 + (kv == "q8") + 2 * presplit)
    e = np.round(np.arange(N) * 40.0 / N) - 20.0
    s = 1 / math.sqrt(d)
    c = 8.0
    V = (st.normal((N, nkv * d)) * np.exp2(-e)[:, None]).astype(np.float32)
    K = st.normal((N, nkv * d))
    for h in range(nkv):
        K[:, h * d] = e * math.log(2) / (c * s)
    K = K.astype(np.float32)
    Q = st.normal((M, nq, d))
    Q[:, :, 0] = c
    Q = Q.astype(np.float32)
    if kv == "q8":
        K, V = oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
        Kd = torch.from_numpy(np.ascontiguousarray(K, dtype=np.uint8)).cuda()
        Vd = torch.from_numpy(np.ascontiguousarray(V, dtype=np.uint8)).cuda()
    else:
        Kd, Vd = dev(K), dev(V)
    O = torch.empty((M, nq, d), device="cuda")
    attn.set_prefill_presplit(presplit)
    try:
        attn.attn_prefill_gqa(dev(Q), Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)
    finally:
        attn.set_prefill_presplit(True)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, 0)
    err = normwise_err(host(O), R)
    print(f"ramp scales normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kv", ["f32", "q8"])
@pytest.mark.parametrize("window", [0, 200])
def test_prefill_random_row_scales(gpu, d, kv, window):
    """K and V rows each scaled by their own 2^U(-12, 12), q rows by
    2^U(-6, 6), at every head dim the matrix-core prefill tiles, with and
    without a window: the row units of the scores and of PV, and the query
    rows' PV shifts, over scales that move from row to row; against the
    oracle."""
    announce(f"prefill random row scales d={d} kv={kv} window={window}")
    nq, nkv, M, N, pos0 = 8, 2, 70, 600, 530
    rng = np.random.default_rng(980 + d + (kv == "q8") + window)
    st = Stream(981 + d + (kv == "q8") + window)
    K = (st.normal((N, nkv * d)) * np.exp2(rng.uniform(-12, 12, size=N))[:, None]).astype(np.float32)
    V = (st.normal((N, nkv * d)) * np.exp2(rng.uniform(-12, 12, size=N))[:, None]).astype(np.float32)
    Q = (st.normal((M, nq, d)) * np.exp2(rng.uniform(-6, 6, size=(M, nq)))[:, :, None])
    Q = Q.astype(np.float32)
    if kv == "q8":
        K, V = oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
        Kd = torch.from_numpy(np.ascontiguousarray(K, dtype=np.uint8)).cuda()
        Vd = torch.from_numpy(np.ascontiguousarray(V, dtype=np.uint8)).cuda()
    else:
        Kd, Vd = dev(K), dev(V)
    s = 2.0 ** -12 / math.sqrt(d)
    O = torch.empty((M, nq, d), device="cuda")
    attn.attn_prefill_gqa(dev(Q), Kd, Vd, O, nq, nkv, M, N, d, s, pos0, window)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, window)
    err = normwise_err(host(O), R)
    print(f"random row scales normwise err {err:.3e}", flush=True)
    assert err < TOL


def test_prefill_2k_prompt(gpu):
    """A 2048-token prompt at the headline head shape (the bench workload)."""
    announce("prefill 32q/8kv/d128 M=2048 fresh")
    st = Stream(74)
    nq, nkv, d, M = 32, 8, 128, 2048
    Q = st.normal((M, nq, d))
    K, V = cache(st, M, nkv, d, False)
    O = torch.empty((M, nq, d), device="cuda")
    attn.attn_prefill_gqa(dev(Q), dev(K), dev(V), O, nq, nkv, M, M, d, 0.088, 0, 0)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, M, d, 0.088, 0, 0)
    err = normwise_err(host(O), R)
    print(f"prefill 2k normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("d,bf16", [(128, False), (96, False), (80, True)])
def test_prefill_graph_replays_match_eager(gpu, d, bf16):
    """The prefill attention captured in a HIP graph: 40 queries after 3000
    cached rows (the key-split grid and its combine kernel; fp32 with the
    once-per-launch key split, bf16 staged per tile, 96 and 80 padded).
    The stream's workspaces are sized by one launch before the capture and
    reused by every replay; each replay, with eager work and
    synchronisations between them, equals the eager result bit for bit."""
    announce(f"prefill graph d={d} bf16={bf16}")
    nq, nkv, M, N, pos0 = 16, 4, 40, 3040, 3000
    st = Stream(400 + d + bf16)
    Q = st.normal((M, nq, d))
    K, V = cache(st, N, nkv, d, bf16)
    Qd, Kd, Vd = dev(Q), on_dev(K), on_dev(V)
    s = 1 / math.sqrt(d)
    O = torch.empty((M, nq, d), device="cuda")
    attn.attn_prefill_gqa(Qd, Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)
    eager = host(O)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        attn.attn_prefill_gqa(Qd, Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        attn.attn_prefill_gqa(Qd, Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)
    O2 = torch.empty((8, nq, d), device="cuda")
    for r in range(4):
        O.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(O), eager), f"replay {r}"
        # eager work in between replays: another prefill on the current stream
        attn.attn_prefill_gqa(Qd[:8].contiguous(), Kd, Vd, O2, nq, nkv, 8, 2008, d, s, 2000, 0)
        torch.cuda.synchronize()
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, 0)
    assert normwise_err(eager, R) < TOL
