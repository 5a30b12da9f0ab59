"""Head dims other than 64, 128 and 256 on the decode and prefill paths
(MI355X only).

The reference takes any head dim (include/molot/attn.h:99, :174 and
gemm.h:26 run scalar tails; model.h:518 derives qhd from the weights).  The
vector-ALU decode kernels are built for D = 64, 128 and 256; an even head
dim d runs padded in the next of them: q is zero-padded to D, the K/V rows
are read at their stored length d, and every output is written at d.  These
tests hold every decode entry at such dims to the oracle (1e-5 normwise for
fp32, and for bf16 on the same bf16 values), covering d % 4 == 2, single and
split chunks, the in-launch merge and the combine kernel, windows, norms,
the paged cache and the head-major layout.  The prefill kernels take a
multiple of 8 below 256 (fp32 or bf16 caches) padded the same way, through
the bf16 pieces of the keys; those tests hold the prefill attention, the
fused prefill step and its paged form to the oracle at the same bar.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import normwise_err
from gpu_util import dev, dev_bf16, host, make_decode, make_paged, oracle_decode, oracle_paged
from molot_amd import attn
from molot_amd.synth import Stream, bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5


def announce(msg):
    print(f"[case] {msg}", flush=True)


def run_step(p, qn=None, kn=None, v_norm=False):
    q = dev(p.q)
    K = dev_bf16(p.K) if p.kv_dtype else dev(p.K)
    V = dev_bf16(p.V) if p.kv_dtype else dev(p.V)
    O = torch.full((p.nq, p.d), float("nan"), device="cuda")
    attn.decode_step(q, dev(p.k_new), dev(p.v_new), K, V, O, p.nq, p.nkv, p.d, p.pos, p.pos,
                     dev(p.inv_freq), p.scale, p.window,
                     q_norm=None if qn is None else dev(qn), k_norm=None if kn is None else dev(kn),
                     v_norm=v_norm, eps=1e-6)
    bits = (lambda t: host(t.view(torch.int16)).view(np.uint16)) if p.kv_dtype else host
    return host(q), bits(K), bits(V), host(O)


def check_rows(p, Kh, Vh, oK, oV):
    """The appended row as the oracle stores it; no other row touched."""
    np.testing.assert_array_equal(Kh[:p.pos], p.K[:p.pos])
    np.testing.assert_array_equal(Vh[:p.pos], p.V[:p.pos])
    if p.kv_dtype:
        for X, R in ((Kh, oK), (Vh, oV)):
            dx = np.abs(bf16_to_f32(X[p.pos]) - bf16_to_f32(R[p.pos]))
            assert np.max(dx) <= 8e-3 * max(1.0, float(np.max(np.abs(bf16_to_f32(R[p.pos])))))
    else:
        np.testing.assert_allclose(Kh[p.pos], oK[p.pos], atol=4e-6, rtol=2e-6)
        np.testing.assert_allclose(Vh[p.pos], oV[p.pos], atol=1e-6, rtol=1e-6)


# (nq, nkv, d, pos, window, bf16): slot counts of 8 at pos >= 8192 merge in
# the launch, others use the combine kernel; pos 10 is one chunk
STEPS = [
    (32, 8, 80, 3000, 0, False),
    (32, 8, 96, 9000, 0, False),     # in-launch merge
    (32, 8, 112, 2500, 0, False),
    (16, 4, 160, 2000, 0, False),
    (8, 4, 192, 5000, 1024, False),  # Gemma-like window
    (8, 2, 192, 10, 0, False),       # one chunk
    (32, 8, 66, 9000, 0, False),     # d % 4 == 2, in-launch merge
    (12, 4, 250, 1500, 300, False),  # d % 4 == 2, D = 256
    (8, 8, 2, 700, 0, False),        # the smallest even head dim
    (32, 8, 80, 3000, 0, True),      # bf16 caches of these dims take the vector-ALU kernel
    (64, 8, 96, 2000, 0, True),
    (8, 4, 200, 1200, 0, True),
    (16, 4, 34, 900, 0, True),       # bf16 with d % 8 == 2
]


@pytest.mark.parametrize("shape", STEPS, ids=[f"{s[0]}q{s[1]}kv_d{s[2]}_n{s[3]}"
                                              f"{'_w' + str(s[4]) if s[4] else ''}"
                                              f"{'_bf16' if s[5] else ''}" for s in STEPS])
def test_decode_step_head_dims(gpu, shape):
    nq, nkv, d, pos, window, bf16 = shape
    announce(f"decode step {shape}")
    p = make_decode(nq, nkv, d, pos, window=window, seed=pos + 3 * d, bf16=bf16)
    q, Kh, Vh, O = run_step(p)
    oq, _, oO, oK, oV = oracle_decode(p)
    np.testing.assert_allclose(q, oq, atol=4e-6, rtol=2e-6)
    check_rows(p, Kh, Vh, oK, oV)
    assert np.isfinite(O).all()
    err = normwise_err(O, oO)
    # the oracle beside the float64 brute force on the GPU's own cache and q
    Kw, Vw = (bf16_to_f32(Kh), bf16_to_f32(Vh)) if p.kv_dtype else (Kh, Vh)
    R64 = oracle.attn_decode_f64(q, Kw, Vw, nq, nkv, pos + 1, d, p.scale, pos, window, nkv * d, d)
    e64 = normwise_err(oO, R64)
    print(f"d={d}: normwise err {err:.3e} (oracle vs f64 {e64:.3e})", flush=True)
    assert err < FP32_TOL
    assert e64 < FP32_TOL
    assert normwise_err(O, R64) < FP32_TOL


@pytest.mark.parametrize("d,bf16", [(80, False), (96, True), (250, False)])
def test_decode_step_norms_head_dims(gpu, d, bf16):
    """The layer's norms at the stored head dim (means over d, not D)."""
    announce(f"decode step with norms d={d} bf16={bf16}")
    p = make_decode(16, 4, d, 1500, seed=d + 5, bf16=bf16)
    st = Stream(d)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    q, Kh, Vh, O = run_step(p, qn, kn, True)
    Kc, Vc = p.K.copy(), p.V.copy()
    oq, _, oO = oracle.decode_step_norm(p.q, p.k_new, p.v_new, Kc, Vc, p.nq, p.nkv, d, p.pos,
                                        p.pos, qn, kn, True, 1e-6, p.inv_freq, p.scale, 0)
    np.testing.assert_allclose(q, oq, atol=4e-6, rtol=2e-6)
    check_rows(p, Kh, Vh, Kc, Vc)
    assert normwise_err(O, oO) < FP32_TOL


@pytest.mark.parametrize("d", [72, 112, 66, 34])
def test_attention_entries_head_dims(gpu, d):
    """attn_decode_gqa_cache (token-major) and attn_decode_gqa (head-major)."""
    announce(f"attention-only entries d={d}")
    st = Stream(40 + d)
    nq, nkv, n = 16, 4, 2345
    Q = st.normal((nq, d))
    K = st.normal((n, nkv * d))
    V = st.normal((n, nkv * d))
    s = 1.0 / math.sqrt(d)
    O = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), dev(K), dev(V), O, nq, nkv, n, d, s, n - 1, 0)
    ref = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, s, n - 1, 0)
    assert normwise_err(host(O), ref) < FP32_TOL
    Kh = np.ascontiguousarray(K.reshape(n, nkv, d).transpose(1, 0, 2))
    Vh = np.ascontiguousarray(V.reshape(n, nkv, d).transpose(1, 0, 2))
    O2 = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa(dev(Q), dev(Kh), dev(Vh), O2, nq, nkv, n, d, s)
    assert normwise_err(host(O2), ref) < FP32_TOL


@pytest.mark.parametrize("d", [34, 66, 96])
def test_attention_entries_head_dims_bf16(gpu, d):
    """The attention-only entries over bf16 caches at padded head dims,
    d % 4 == 2 included (4-byte rows of two elements): against the oracle on
    the bf16 values, token-major and head-major."""
    announce(f"attention-only entries bf16 d={d}")
    st = Stream(60 + d)
    nq, nkv, n = 8, 2, 1500
    Q = st.normal((nq, d))
    Kb = f32_to_bf16(st.normal((n, nkv * d)))
    Vb = f32_to_bf16(st.normal((n, nkv * d)))
    K, V = bf16_to_f32(Kb), bf16_to_f32(Vb)
    s = 1.0 / math.sqrt(d)
    ref = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, s, n - 1, 300)
    O = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), dev_bf16(Kb), dev_bf16(Vb), O, nq, nkv, n, d, s, n - 1, 300)
    assert normwise_err(host(O), ref) < FP32_TOL
    Kh = np.ascontiguousarray(Kb.reshape(n, nkv, d).transpose(1, 0, 2))
    Vh = np.ascontiguousarray(Vb.reshape(n, nkv, d).transpose(1, 0, 2))
    O2 = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_win(dev(Q), dev_bf16(Kh), dev_bf16(Vh), O2, nq, nkv, n, d, s, n - 1, 300)
    assert normwise_err(host(O2), ref) < FP32_TOL


@pytest.mark.parametrize("d,bf16", [(96, True), (80, False), (130, True)])
def test_paged_head_dims(gpu, d, bf16):
    """A shuffled paged batch at the stored head dim."""
    announce(f"paged d={d} bf16={bf16}")
    P = make_paged(7, 16, 4, d, 0, 900, seed=d + 11, bf16=bf16)
    inv = oracle.rope_inv_freq(10000.0, d)
    s = 1.0 / math.sqrt(d)
    B, nq, nkv, page = P["B"], P["nq"], P["nkv"], P["page"]
    K = dev_bf16(P["Kp"]) if bf16 else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf16 else dev(P["Vp"])
    q = dev(P["q"])
    O = torch.empty((B, nq, d), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O, dev(P["bt"].reshape(-1)),
                           dev(P["n"]), None, B, P["max_blocks"], nq, nkv, d, page, dev(inv), s, 0)
    oq, oK, oV, oO = oracle_paged(P, inv, s)
    np.testing.assert_allclose(host(q), oq, atol=4e-6, rtol=2e-6)
    assert normwise_err(host(O), oO) < FP32_TOL


# Prefill at padded head dims: the prefill kernels are built for D = 64, 128
# and 256; a multiple of 8 below 256 (fp32 or bf16 cache) runs padded to the
# next D through the bf16 pieces (the split zero-fills each row past d).
def prefill_cache(st, N, nkv, d, bf16):
    K = st.normal((N, nkv * d))
    V = st.normal((N, nkv * d))
    if bf16:
        return f32_to_bf16(K), f32_to_bf16(V)
    return K, V


def on_dev(x):
    return dev_bf16(x) if x.dtype == np.uint16 else dev(x)


@pytest.mark.parametrize("nq,nkv,d,M,N,pos0,window,bf16", [
    (16, 4, 96, 100, 100, 0, 0, False),      # fresh prompt
    (16, 4, 80, 60, 1060, 1000, 0, True),    # appended to a context
    (8, 2, 112, 50, 3050, 3000, 1024, False),  # window, split key tiles
    (8, 4, 192, 70, 170, 100, 33, True),     # D = 256
    (32, 8, 72, 33, 533, 500, 0, False),     # G = 4
    (8, 8, 200, 1, 700, 699, 0, True),       # a single query
    (8, 2, 40, 12, 30, 25, 0, False),        # D = 64, causal end clipped at N
])
def test_prefill_head_dims(gpu, nq, nkv, d, M, N, pos0, window, bf16):
    announce(f"prefill {nq}/{nkv}/d{d} M={M} N={N} pos0={pos0} win={window} bf16={bf16}")
    st = Stream(M + N + d + nq + 5)
    Q = st.normal((M, nq, d))
    K, V = prefill_cache(st, N, nkv, d, bf16)
    O = torch.full((M, nq, d), float("nan"), device="cuda")
    scale = 1 / math.sqrt(d)
    attn.attn_prefill_gqa(dev(Q), on_dev(K), on_dev(V), O, nq, nkv, M, N, d, scale, pos0, window)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, scale, pos0, window)
    err = normwise_err(host(O), R)
    print(f"prefill normwise err {err:.3e}", flush=True)
    assert err < FP32_TOL


@pytest.mark.parametrize("d,bf16", [(96, False), (120, True), (208, False)])
def test_prefill_step_head_dims(gpu, d, bf16):
    """One layer's prefill with norms at a padded head dim: 90 prompt tokens
    after 150 cached, against the oracle's forward.h:367-399 sequence."""
    announce(f"prefill step 16q/4kv/d{d} M=90 after 150 bf16={bf16}")
    st = Stream(170 + d + bf16)
    nq, nkv, M, n0 = 16, 4, 90, 150
    q = st.normal((M, nq, d), 2.0)
    k = st.normal((M, nkv, d), 2.0)
    v = st.normal((M, nkv, d), 2.0)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K, V = prefill_cache(st, n0 + M, nkv, d, bf16)
    K[n0:] = 0
    V[n0:] = 0
    inv = oracle.rope_inv_freq(1000000.0, d)
    s = 1 / math.sqrt(d)
    qd, Kd, Vd = dev(q), on_dev(K), on_dev(V)
    O = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, M, n0, n0, dev(inv), s, 0,
                      q_norm=dev(qn), k_norm=dev(kn), v_norm=True, eps=1e-6)
    Kc, Vc = K.copy(), V.copy()
    oq, oO = oracle.prefill_step(q, k, v, Kc, Vc, nq, nkv, d, M, n0, n0, qn, kn, 1, 1e-6, inv, s,
                                 0)
    np.testing.assert_allclose(host(qd), oq, rtol=2e-6, atol=4e-6)
    if bf16:  # the attention on the GPU's own bf16 rows (normed rows may differ by an ulp)
        bits = lambda t: host(t.view(torch.int16)).view(np.uint16)
        R = oracle.attn_prefill(host(qd), bits(Kd), bits(Vd), nq, nkv, M, n0 + M, d, s, n0, 0)
        assert normwise_err(host(O), R) < FP32_TOL
        assert normwise_err(host(O), oO) < 2e-2
    else:
        np.testing.assert_allclose(host(Kd), Kc, rtol=2e-6, atol=4e-6)
        np.testing.assert_allclose(host(Vd), Vc, rtol=1e-6, atol=1e-7)
        assert normwise_err(host(O), oO) < FP32_TOL


@pytest.mark.parametrize("d,bf16", [(96, True), (160, False)])
def test_prefill_step_paged_head_dims(gpu, d, bf16):
    """The paged prefill step (shuffled 16-row pages) at a padded head dim
    equals the contiguous one bit for bit."""
    announce(f"paged prefill step 8/2/d{d} bf16={bf16}")
    st = Stream(191 + d + bf16)
    nq, nkv, M, n0, page, spare = 8, 2, 45, 200, 16, 3
    cap = n0 + M
    q = st.normal((M, nq, d))
    k = st.normal((M, nkv, d))
    v = st.normal((M, nkv, d))
    K, V = prefill_cache(st, cap, nkv, d, bf16)
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
    inv = dev(oracle.rope_inv_freq(10000.0, d))
    s = 1 / math.sqrt(d)
    qc, qp = dev(q), dev(q)
    Kc, Vc = on_dev(K), on_dev(V)
    Kpd, Vpd = on_dev(Kp.reshape(nblk, -1)), on_dev(Vp.reshape(nblk, -1))
    Oc = torch.empty((M, nq, d), device="cuda")
    Op = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(qc, dev(k), dev(v), Kc, Vc, Oc, nq, nkv, d, M, n0, n0, inv, s, 0)
    attn.prefill_step_paged(qp, dev(k), dev(v), Kpd, Vpd, Op, torch.from_numpy(row).cuda(), nb,
                            page, nq, nkv, d, M, n0, n0, inv, s, 0)
    assert torch.equal(Oc, Op)
    assert torch.equal(qc, qp)
    R = oracle.attn_prefill(host(qc), host(Kc.view(torch.int16)).view(np.uint16) if bf16
                            else host(Kc), host(Vc.view(torch.int16)).view(np.uint16) if bf16
                            else host(Vc), nq, nkv, M, cap, d, s, n0, 0)
    assert normwise_err(host(Oc), R) < FP32_TOL


@pytest.mark.parametrize("nq,nkv,d,M,N,pos0,window", [
    (16, 4, 96, 70, 1070, 1000, 0), (8, 4, 200, 40, 540, 500, 100), (8, 2, 56, 33, 33, 0, 0)])
def test_prefill_head_dims_per_tile_split(gpu, nq, nkv, d, M, N, pos0, window):
    """An fp32 cache at a padded head dim: the keys split once per launch and
    split per staged tile (the path under stream capture and past the pieces
    workspace's limit) give the same bits, and the oracle's result."""
    announce(f"prefill per-tile split {nq}/{nkv}/d{d} M={M} N={N} win={window}")
    st = Stream(300 + d)
    Q = st.normal((M, nq, d))
    K, V = prefill_cache(st, N, nkv, d, False)
    s = 1 / math.sqrt(d)
    outs = []
    try:
        for pre in (True, False):
            attn.set_prefill_presplit(pre)
            O = torch.full((M, nq, d), float("nan"), device="cuda")
            attn.attn_prefill_gqa(dev(Q), dev(K), dev(V), O, nq, nkv, M, N, d, s, pos0, window)
            outs.append(host(O))
    finally:
        attn.set_prefill_presplit(True)
    assert np.array_equal(outs[0], outs[1])
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, s, pos0, window)
    assert normwise_err(outs[1], R) < FP32_TOL
