"""Parity of the HIP decode-attention path with the oracle (MI355X only).

Every call goes through the C ABI (molot_amd.attn -> libmolot_amd.so).
Bars: normwise max|gpu-ref|/max|ref| <= 1e-5 for fp32
KV; for bf16 KV <= 1e-5 against the oracle run on the same bf16 values and
<= 2e-2 against the fp32 originals.  RoPE outputs within a few ulp; the KV
append is bit-exact.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import normwise_err
from gpu_util import (dev, dev_bf16, host, make_decode, make_paged, oracle_decode,
                      oracle_paged, widen)
from molot_amd import attn
from molot_amd.synth import Stream, bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def announce(msg):
    print(f"[case] {msg}", flush=True)


def run_decode_gpu(p):
    """rope+append+attention on the GPU; returns (q_rot, K_after, V_after, O)."""
    q = dev(p.q)
    K = dev_bf16(p.K) if p.kv_dtype else dev(p.K)
    V = dev_bf16(p.V) if p.kv_dtype else dev(p.V)
    O = torch.empty((p.nq, p.d), dtype=torch.float32, device="cuda")
    attn.decode_step(q, dev(p.k_new), dev(p.v_new), K, V, O, p.nq, p.nkv, p.d, p.pos, p.pos,
                     dev(p.inv_freq), p.scale, p.window)
    if p.kv_dtype:
        Kh = host(K.view(torch.int16)).view(np.uint16)
        Vh = host(V.view(torch.int16)).view(np.uint16)
    else:
        Kh, Vh = host(K), host(V)
    return host(q), Kh, Vh, host(O)


# ---------------------------------------------------------------------------
# golden fixtures written from the compiled reference

@pytest.mark.parametrize("name", ["decode_step_g4_d128", "decode_step_win_d256",
                                  "decode_step_g8_d64_scale1"])
def test_golden_decode_step(gpu, name):
    announce(name)
    g = golden(name)
    nq, nkv, d, pos = int(g["nq"]), int(g["nkv"]), int(g["d"]), int(g["pos"])
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos], V[:pos] = g["K"], g["V"]
    q, Kd, Vd = dev(g["q"]), dev(K), dev(V)
    O = torch.empty((nq, d), dtype=torch.float32, device="cuda")
    attn.decode_step(q, dev(g["k_new"]), dev(g["v_new"]), Kd, Vd, O, nq, nkv, d, pos, pos,
                     dev(g["inv_freq"]), float(g["scale"]), int(g["window"]))
    np.testing.assert_allclose(host(q), g["q_rot"], atol=2e-6)
    Kh, Vh = host(Kd), host(Vd)
    np.testing.assert_allclose(Kh[pos], g["k_rot"].reshape(-1), atol=2e-6)
    np.testing.assert_array_equal(Vh[pos], g["v_new"].reshape(-1))
    np.testing.assert_array_equal(Kh[:pos], g["K"])  # nothing else written
    assert normwise_err(host(O), g["O"]) < FP32_TOL


def test_golden_head(gpu):
    g = golden("head_bench_check")
    n, d = int(g["n"]), int(g["d"])
    O = torch.empty(d, dtype=torch.float32, device="cuda")
    attn.attn_decode_head(dev(g["Q"]), dev(g["K"]), dev(g["V"]), O, n, d, float(g["scale"]))
    o = host(O)
    assert np.max(np.abs(o - g["O"])) < 1e-3  # bench/bench.cc:216 bar
    assert normwise_err(o, g["O"]) < FP32_TOL


@pytest.mark.parametrize("name", ["gqa_headmajor_d64", "gqa_win_headmajor_d64"])
def test_golden_headmajor(gpu, name):
    g = golden(name)
    nq, nkv, n, d = (int(g[k]) for k in ("nq", "nkv", "n", "d"))
    O = torch.empty((nq, d), dtype=torch.float32, device="cuda")
    if int(g["window"]) > 0:
        attn.attn_decode_gqa_win(dev(g["Q"]), dev(g["K"]), dev(g["V"]), O, nq, nkv, n, d,
                                 float(g["scale"]), int(g["pos_cur"]), int(g["window"]))
    else:
        attn.attn_decode_gqa(dev(g["Q"]), dev(g["K"]), dev(g["V"]), O, nq, nkv, n, d,
                             float(g["scale"]))
    assert normwise_err(host(O), g["O"]) < FP32_TOL


def test_golden_bf16_cache(gpu):
    g = golden("bf16_cache_g8_d128")
    nq, nkv, n, d = (int(g[k]) for k in ("nq", "nkv", "n", "d"))
    O = torch.empty((nq, d), dtype=torch.float32, device="cuda")
    attn.attn_decode_gqa_cache(dev(g["Q"]), dev_bf16(g["K_bf16"]), dev_bf16(g["V_bf16"]), O, nq,
                               nkv, n, d, float(g["scale"]), n - 1, 0)
    assert normwise_err(host(O), g["O"]) < FP32_TOL


@pytest.mark.parametrize("name", ["rope_d128_theta5e5", "rope_d256_theta1e4"])
def test_golden_rope(gpu, name):
    g = golden(name)
    inv = dev(g["inv_freq"])
    for i, pos in enumerate(g["positions"]):
        x = dev(g["X"][i])
        attn.rope_apply(x, int(pos), inv)
        y = host(x)
        assert np.max(np.abs(y - g["Y"][i])) <= 4e-7 * max(1.0, float(np.max(np.abs(g["Y"][i]))))


def test_vexp_known_answers(gpu):
    """bench/bench.cc:220-234 on the GPU softmax exp: relerr < 1e-5."""
    kat = np.array([-87., -20., -10., -5., -3., -2., -1.5, -1., -0.75, -0.5, -0.25, -0.1, -0.01,
                    0., 1., 50.], np.float32)
    y = host(attn.vexp(dev(kat)))
    ref = np.exp(kat.astype(np.float64))
    assert np.max(np.abs(y - ref) / ref) < 1e-5
    g = golden("vexp_points")
    yg = host(attn.vexp(dev(g["X"])))
    x = g["X"].astype(np.float64)
    inside = (x >= -87.3) & (x <= 88.0)  # both sides representable as normal floats
    np.testing.assert_allclose(yg[inside], np.exp(x[inside]), rtol=1e-5)


def test_prob_exp_known_answers(gpu):
    """The probabilities' exp (2^(x*log2 e), one v_exp_f32, as every decode
    and prefill kernel takes it) at the bench/bench.cc:220-234 points and
    the golden points (reference: norm.h:35-47's exp_avx512_ps), relerr
    < 1e-5; and across |s - m| up to the range the kernels feed it: scores
    sit at most 8 base-2 units above the running max (the lazy max), down to
    where e^x leaves the normal floats."""
    kat = np.array([-87., -20., -10., -5., -3., -2., -1.5, -1., -0.75, -0.5, -0.25, -0.1, -0.01,
                    0., 1., 50.], np.float32)
    y = host(attn.prob_exp(dev(kat)))
    ref = np.exp(kat.astype(np.float64))
    assert np.max(np.abs(y - ref) / ref) < 1e-5
    g = golden("vexp_points")
    yg = host(attn.prob_exp(dev(g["X"])))
    x = g["X"].astype(np.float64)
    inside = (x >= -87.3) & (x <= 88.0)  # both sides representable as normal floats
    np.testing.assert_allclose(yg[inside], np.exp(x[inside]), rtol=1e-5)
    # the kernels' own range, densely: x = s - m in [-87, 8 ln 2]
    st = Stream(71)
    u = (st.words(1 << 16) >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    xs = (-87.0 + (87.0 + 8 * math.log(2)) * u).astype(np.float32)
    ys = host(attn.prob_exp(dev(xs))).astype(np.float64)
    rel = np.abs(ys - np.exp(xs.astype(np.float64))) / np.exp(xs.astype(np.float64))
    # the rounding of x*log2(e) bounds the error by ~|x| * 2^-24 (plus the
    # instruction's own ~1 ulp): a planted natural-units exp2 (no log2 e)
    # would miss by orders of magnitude
    assert np.max(rel) < 1e-5
    assert np.all(rel <= 2.0 ** -22 + np.abs(xs.astype(np.float64)) * 2.0 ** -23)


def test_inv_freq_host_table(gpu):
    for base, d in ((500000.0, 128), (10000.0, 256)):
        got = attn.rope_inv_freq(base, d).numpy()
        np.testing.assert_array_equal(got, oracle.rope_inv_freq(base, d))


# ---------------------------------------------------------------------------
# BASELINE configs at full size against the oracle

def check_decode(p, tol=FP32_TOL, label="", f64_tol=None):
    q_rot, K_after, V_after, O = run_decode_gpu(p)
    oq, ok, oO, oK, oV = oracle_decode(p)
    np.testing.assert_allclose(q_rot, oq, atol=4e-6, rtol=2e-6)
    np.testing.assert_array_equal(V_after[p.pos], oV[p.pos])
    if p.kv_dtype == 0:
        np.testing.assert_allclose(K_after[p.pos], oK[p.pos], atol=4e-6, rtol=2e-6)
    else:  # bf16 rounding of a value that may differ by an ulp before rounding
        kd = np.abs(bf16_to_f32(K_after[p.pos]) - bf16_to_f32(oK[p.pos]))
        assert np.max(kd) <= 8e-3 * max(1.0, float(np.max(np.abs(bf16_to_f32(oK[p.pos])))))
    np.testing.assert_array_equal(K_after[:p.pos], p.K[:p.pos])
    err = normwise_err(O, oO)
    # float64 brute force on the same (rotated, appended) inputs: separates the
    # kernel's rounding from the fp32 oracle's own sequential-sum rounding
    f64 = oracle.attn_decode_f64(oq, oK, oV, p.nq, p.nkv, p.pos + 1, p.d, p.scale, p.pos,
                                 p.window, p.nkv * p.d, p.d)
    e_gpu, e_orc = normwise_err(O, f64), normwise_err(oO, f64)
    print(f"{label} normwise err vs oracle {err:.3e}; vs f64: gpu {e_gpu:.3e} oracle {e_orc:.3e}",
          flush=True)
    if p.kv_dtype == 0:
        assert err < tol
    else:
        assert err < BF16_TOL  # north_star bar for bf16 KV
        assert e_gpu < FP32_TOL  # and the kernel itself is fp32-accurate on those values
    if f64_tol is not None:
        assert e_gpu < f64_tol
    return O


def test_c1_llama8b_ctx4096(gpu):
    announce("c1 32q/8kv/d128 pos 4096 fp32")
    check_decode(make_decode(32, 8, 128, 4096, base=500000.0), label="c1")


def test_c2_llama8b_ctx16384(gpu):
    announce("c2 32q/8kv/d128 pos 16384 fp32")
    check_decode(make_decode(32, 8, 128, 16384, base=500000.0), label="c2")


def test_c3_sliding_window(gpu):
    announce("c3 8q/4kv/d256 pos 32768 window 1024 fp32")
    check_decode(make_decode(8, 4, 256, 32768, base=10000.0, window=1024), label="c3")


def test_c5_70b_ctx131072_bf16(gpu):
    announce("c5 64q/8kv/d128 pos 131072 bf16 sigma 0.5")
    p = make_decode(64, 8, 128, 131072, base=500000.0, sigma_kv=0.5, bf16=True)
    O = check_decode(p, label="c5 vs oracle on bf16 values")
    # against fp32 originals: regenerate them from the same stream positions
    st = Stream(1234)
    st.normal((64, 128)), st.normal((8, 128)), st.normal((8, 128))
    Kf = np.zeros((p.pos + 1, 8 * 128), np.float32)
    Vf = np.zeros_like(Kf)
    Kf[:p.pos] = st.normal((p.pos, 1024), 0.5)
    Vf[:p.pos] = st.normal((p.pos, 1024), 0.5)
    _, _, Of = oracle.decode_step(p.q, p.k_new, p.v_new, Kf, Vf, 64, 8, 128, p.pos, p.pos,
                                  p.inv_freq, p.scale, 0)
    assert normwise_err(O, Of) < BF16_TOL


# ---------------------------------------------------------------------------
# shapes, windows, ragged lengths, chunking

@pytest.mark.parametrize("nq,nkv,d", [(32, 8, 128), (8, 4, 256), (64, 8, 128), (16, 16, 64),
                                      (24, 8, 128), (16, 1, 128), (32, 2, 64), (12, 4, 256),
                                      (16, 2, 256)])
@pytest.mark.parametrize("pos", [0, 1, 15, 16, 63, 64, 65, 1000, 2049])
def test_shapes_and_ragged_lengths(gpu, nq, nkv, d, pos):
    announce(f"shape {nq}/{nkv}/{d} pos {pos}")
    check_decode(make_decode(nq, nkv, d, pos, seed=pos + 7 * nq + d), label="shape")


@pytest.mark.parametrize("window", [1, 2, 17, 64, 1000, 5000])
def test_windows(gpu, window):
    announce(f"window {window}")
    check_decode(make_decode(8, 4, 256, 3000, base=10000.0, window=window, seed=window),
                 label="window")


@pytest.mark.parametrize("chunk", [16, 64, 256, 1024])
def test_forced_chunk_sizes(gpu, chunk):
    announce(f"chunk {chunk}")
    attn.set_split_chunk(chunk)
    try:
        check_decode(make_decode(32, 8, 128, 5000, seed=chunk), label=f"chunk{chunk}")
        check_decode(make_decode(64, 8, 128, 700, seed=chunk + 1, bf16=True), label="bf16")
    finally:
        attn.set_split_chunk(0)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("factor", [100.0, 1000.0])
def test_outlier_q_channels(gpu, bf16, factor):
    """q with a few channels factor x the rest (LLM activations have such
    outliers) through the fused step: RoPE, append and attention against the
    oracle to the usual bars (fp32 and bf16 caches; the matrix-core kernel's
    q pieces are per element)."""
    announce(f"outlier q channels x{factor:g} bf16={bf16}")
    p = make_decode(32, 8, 128, 2000, seed=int(factor) + bf16, bf16=bf16)
    p.q[:, [3, 40, 77, 100]] *= factor
    # scores of several hundred: the fp32 oracle's own sequential sums then
    # err by ~1.5e-5 against a float64 brute force (the kernel by ~4e-6), so
    # the kernel is held to 1e-5 of float64 and to 3e-5 of the fp32 oracle
    check_decode(p, tol=3e-5, label=f"outlier{factor:g}", f64_tol=FP32_TOL)


@pytest.mark.parametrize("nq,nkv,d,pos", [(32, 8, 128, 3000), (8, 1, 64, 999), (8, 4, 256, 555),
                                          (4, 4, 128, 1)])
def test_bf16_cache_shapes(gpu, nq, nkv, d, pos):
    announce(f"bf16 {nq}/{nkv}/{d} pos {pos}")
    check_decode(make_decode(nq, nkv, d, pos, seed=pos, bf16=True), label="bf16")


@pytest.mark.parametrize("nq,nkv,d", [(32, 8, 128), (64, 8, 128), (32, 2, 128), (16, 16, 64),
                                      (32, 2, 64), (24, 8, 128), (12, 4, 64)])
@pytest.mark.parametrize("pos", [0, 1, 31, 32, 33, 100, 2049])
def test_bf16_mfma_shapes_and_ragged_lengths(gpu, nq, nkv, d, pos):
    """bf16 KV on the matrix-core kernel: groups of 4, 8, 16, 1 and 3 q heads
    per KV head (16 share one MFMA tile; 3 run as three 1-head groups), both
    head dims it serves, and lengths on either side of its 32-row tiles."""
    announce(f"bf16 mfma {nq}/{nkv}/{d} pos {pos}")
    check_decode(make_decode(nq, nkv, d, pos, seed=pos + 3 * nq + d, bf16=True),
                 label="bf16 mfma")


@pytest.mark.parametrize("window", [1, 31, 33, 1000])
def test_bf16_windows(gpu, window):
    announce(f"bf16 window {window}")
    check_decode(make_decode(32, 8, 128, 3000, window=window, seed=40 + window, bf16=True),
                 label="bf16 window")


def test_bf16_mfma_matches_valu_path(gpu):
    """The matrix-core and the vector-ALU kernel agree on one bf16 cache (both
    fp32-accurate on those values; they differ in summation order only)."""
    from molot_amd import lib as L
    announce("bf16 mfma vs valu 64q/8kv/d128 n=20000")
    p = make_decode(64, 8, 128, 20000, seed=31, sigma_kv=0.5, bf16=True)
    Q = dev(oracle.rope_apply(p.q, p.pos, p.inv_freq))
    K, V = dev_bf16(p.K), dev_bf16(p.V)
    outs = []
    try:
        for path in (1, 0):
            L.load().molot_hip_set_bf16_path(path)
            O = torch.empty((64, 128), device="cuda")
            attn.attn_decode_gqa_cache(Q, K, V, O, 64, 8, p.pos, 128, p.scale, p.pos - 1, 0)
            outs.append(host(O))
    finally:
        L.load().molot_hip_set_bf16_path(1)
    assert normwise_err(outs[0], outs[1]) < 2e-6


def test_bf16_properties(gpu):
    """Exact-answer cases on the matrix-core kernel (values exact in bf16):
    constant V gives that constant; V of KV head j equal to j+1 gives
    O[h] = h // G + 1 (the GQA mapping); a dominant key returns its V row."""
    announce("bf16 properties 64q/8kv/d128 n=9001")
    st = Stream(41)
    nq, nkv, d, n = 64, 8, 128, 9001
    Q = st.normal((nq, d))
    K = f32_to_bf16(st.normal((n, nkv * d), 0.5))
    O = torch.empty((nq, d), device="cuda")
    Vc = f32_to_bf16(np.full((n, nkv * d), -1.25, np.float32))
    attn.attn_decode_gqa_cache(dev(Q), dev_bf16(K), dev_bf16(Vc), O, nq, nkv, n, d, 0.088, n - 1,
                               0)
    np.testing.assert_allclose(host(O), -1.25, rtol=1e-6)
    Vj = f32_to_bf16(np.repeat(np.arange(1, nkv + 1, dtype=np.float32), d)[None, :].repeat(n, 0))
    attn.attn_decode_gqa_cache(dev(Q), dev_bf16(K), dev_bf16(Vj), O, nq, nkv, n, d, 0.088, n - 1,
                               0)
    np.testing.assert_allclose(host(O), (np.arange(nq) // 8 + 1)[:, None].repeat(d, 1),
                               rtol=1e-6)
    # key 4321 of every head aligned with q (score ~ 60 above the rest)
    Kd = bf16_to_f32(K).copy()
    for h in range(nkv):
        Kd[4321, h * d:(h + 1) * d] = 40.0 * np.sign(Q[h * 8])
    V = st.normal((n, nkv * d))
    Vb = f32_to_bf16(V)
    attn.attn_decode_gqa_cache(dev(Q), dev_bf16(f32_to_bf16(Kd)), dev_bf16(Vb), O, nq, nkv, n, d,
                               0.088, n - 1, 0)
    np.testing.assert_allclose(host(O)[0::8], bf16_to_f32(Vb)[4321].reshape(nkv, d), rtol=1e-5,
                               atol=1e-6)


# ---------------------------------------------------------------------------
# the layer's norms fused into the step (forward.h:554, 562-563)

def _norm_weights(d, seed):
    st = Stream(seed)
    return ((1 + st.normal((d,), 0.2)).astype(np.float32),
            (1 + st.normal((d,), 0.2)).astype(np.float32))


@pytest.mark.parametrize("name", ["decode_step_norm_g4_d128", "decode_step_norm_win_d256"])
def test_golden_decode_step_norm(gpu, name):
    """Against the compiled reference's forward.h sequence with norms."""
    g = golden(name)
    nq, nkv, d, pos = int(g["nq"]), int(g["nkv"]), int(g["d"]), int(g["pos"])
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos], V[:pos] = g["K"], g["V"]
    q, Kd, Vd = dev(g["q"]), dev(K), dev(V)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step(q, dev(g["k_new"]), dev(g["v_new"]), Kd, Vd, O, nq, nkv, d, pos, pos,
                     dev(g["inv_freq"]), float(g["scale"]), int(g["window"]),
                     q_norm=dev(g["q_norm"]), k_norm=dev(g["k_norm"]), v_norm=bool(g["v_norm"]),
                     eps=float(g["eps"]))
    np.testing.assert_allclose(host(q), g["q_rot"], rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(host(Kd)[pos], g["k_rot"].reshape(-1), rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(host(Vd)[pos], g["v_normed"].reshape(-1), rtol=1e-6, atol=1e-7)
    assert normwise_err(host(O), g["O"]) < FP32_TOL


def _check_step_norm(p, qn, kn, v_norm, label):
    q = dev(p.q)
    K = dev_bf16(p.K) if p.kv_dtype else dev(p.K)
    V = dev_bf16(p.V) if p.kv_dtype else dev(p.V)
    O = torch.empty((p.nq, p.d), device="cuda")
    attn.decode_step(q, dev(p.k_new), dev(p.v_new), K, V, O, p.nq, p.nkv, p.d, p.pos, p.pos,
                     dev(p.inv_freq), p.scale, p.window, q_norm=None if qn is None else dev(qn),
                     k_norm=None if kn is None else dev(kn), v_norm=v_norm, eps=1e-6)
    Kc, Vc = p.K.copy(), p.V.copy()
    oq, ok, oO = oracle.decode_step_norm(p.q, p.k_new, p.v_new, Kc, Vc, p.nq, p.nkv, p.d, p.pos,
                                         p.pos, qn, kn, v_norm, 1e-6, p.inv_freq, p.scale,
                                         p.window)
    np.testing.assert_allclose(host(q), oq, rtol=2e-6, atol=4e-6)
    if p.kv_dtype:
        Vh = host(V.view(torch.int16)).view(np.uint16)
        kd = np.abs(bf16_to_f32(host(K.view(torch.int16)).view(np.uint16)[p.pos]) -
                    bf16_to_f32(Kc[p.pos]))
        assert np.max(kd) <= 8e-3 * max(1.0, float(np.max(np.abs(bf16_to_f32(Kc[p.pos])))))
        vd = np.abs(bf16_to_f32(Vh[p.pos]) - bf16_to_f32(Vc[p.pos]))
        assert np.max(vd) <= 8e-3 * max(1.0, float(np.max(np.abs(bf16_to_f32(Vc[p.pos])))))
        tol = BF16_TOL
    else:
        np.testing.assert_allclose(host(K)[p.pos], Kc[p.pos], rtol=2e-6, atol=4e-6)
        np.testing.assert_allclose(host(V)[p.pos], Vc[p.pos], rtol=1e-6, atol=1e-7)
        tol = FP32_TOL
    err = normwise_err(host(O), oO)
    print(f"{label} normwise err vs oracle {err:.3e}", flush=True)
    assert err < tol


def test_step_norms_c3_gemma_shape(gpu):
    """Gemma-style layer at the c3 shape: q/k norm weights, v norm, scale 1."""
    announce("norms c3 8q/4kv/d256 pos 32768 window 1024 scale 1")
    p = make_decode(8, 4, 256, 32768, base=10000.0, window=1024, scale=1.0, seed=51)
    qn, kn = _norm_weights(256, 52)
    _check_step_norm(p, qn, kn, True, "norms c3")


@pytest.mark.parametrize("which", ["q", "k", "v", "qkv"])
def test_step_norms_each_alone(gpu, which):
    announce(f"norms {which} 32q/8kv/d128 pos 3000")
    p = make_decode(32, 8, 128, 3000, seed=53)
    qn, kn = _norm_weights(128, 54)
    _check_step_norm(p, qn if "q" in which else None, kn if "k" in which else None,
                     "v" in which, f"norms {which}")


def test_step_norms_bf16_matrix_core(gpu):
    announce("norms bf16 64q/8kv/d128 pos 20000")
    p = make_decode(64, 8, 128, 20000, seed=55, sigma_kv=0.5, bf16=True)
    qn, kn = _norm_weights(128, 56)
    _check_step_norm(p, qn, kn, True, "norms bf16")


def test_step_norms_new_token_outside_window(gpu):
    """slot 10 at pos 100 with window 5: nothing attended (O = 0), the normed
    rotated k and the normed v still land in the slot (unfused kernel)."""
    p = make_decode(8, 2, 64, 10, seed=57)
    qn, kn = _norm_weights(64, 58)
    q = dev(p.q)
    K, V = dev(p.K), dev(p.V)
    O = torch.full((8, 64), 3.0, device="cuda")
    attn.decode_step(q, dev(p.k_new), dev(p.v_new), K, V, O, 8, 2, 64, 10, 100, dev(p.inv_freq),
                     p.scale, 5, q_norm=dev(qn), k_norm=dev(kn), v_norm=True, eps=1e-6)
    Kc, Vc = p.K.copy(), p.V.copy()
    oq, ok, _ = oracle.decode_step_norm(p.q, p.k_new, p.v_new, Kc, Vc, 8, 2, 64, 10, 100, qn, kn,
                                        1, 1e-6, p.inv_freq, p.scale, 5)
    assert np.all(host(O) == 0)
    np.testing.assert_allclose(host(q), oq, rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(host(K)[10], Kc[10], rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(host(V)[10], Vc[10], rtol=1e-6, atol=1e-7)


def test_empty_window_gives_zero(gpu):
    st = Stream(3)
    Q = dev(st.normal((4, 128)))
    K = dev(st.normal((50, 2 * 128)))
    O = torch.full((4, 128), 7.0, device="cuda")
    attn.attn_decode_gqa_cache(Q, K, K, O, 4, 2, 50, 128, 0.1, 500, 10)  # t0 = 491 > n
    assert np.all(host(O) == 0)


def test_headmajor_equals_token_major(gpu):
    st = Stream(4)
    nq, nkv, d, n = 32, 8, 128, 3333
    Q = st.normal((nq, d))
    K = st.normal((n, nkv * d))
    V = st.normal((n, nkv * d))
    O1 = torch.empty((nq, d), device="cuda")
    O2 = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), dev(K), dev(V), O1, nq, nkv, n, d, 0.088, n - 1, 0)
    Kh = np.ascontiguousarray(K.reshape(n, nkv, d).transpose(1, 0, 2))
    Vh = np.ascontiguousarray(V.reshape(n, nkv, d).transpose(1, 0, 2))
    attn.attn_decode_gqa(dev(Q), dev(Kh), dev(Vh), O2, nq, nkv, n, d, 0.088)
    o1, o2 = host(O1), host(O2)
    assert normwise_err(o2, o1) < 1e-6
    R = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.088, n - 1, 0)
    assert normwise_err(o1, R) < FP32_TOL


@pytest.mark.parametrize("kind", ["up", "down", "saw"])
@pytest.mark.parametrize("n,bf16", [(16385, False), (3000, False), (5000, True)])
def test_running_max_ramps(gpu, kind, n, bf16):
    """Scores that climb through the context move the running max block after
    block (the kernels rescale only when a score passes the max by more than
    2^8 in base 2); falling and sawtooth scores keep it put or move it in
    jumps.  All q heads share one direction u and every cached key is
    noise + lam_t * u, so the score of row t is lam_t*|q|*scale plus noise,
    spanning ~60 (natural units).  Against the float64 brute force on the
    same (bf16-rounded) values."""
    announce(f"running-max ramp {kind} n={n} bf16={bf16}")
    nq, nkv, d = 32, 8, 128
    st = Stream(91 + n + bf16 + len(kind))
    q0 = st.normal((d,))
    Q = np.repeat(q0[None, :], nq, 0).astype(np.float32)
    scale = 1.0 / math.sqrt(d)
    u = q0 / np.linalg.norm(q0)
    t = np.arange(n, dtype=np.float64)
    span = 60.0 / (np.linalg.norm(q0) * scale)
    lam = {"up": span * t / n, "down": span * (1 - t / n),
           "saw": span * ((t % 700) / 700) * (0.5 + 0.5 * t / n)}[kind]
    K = (0.1 * st.normal((n, nkv * d))).astype(np.float64)
    K += np.tile(lam[:, None] * u[None, :], (1, nkv))
    K = K.astype(np.float32)
    V = st.normal((n, nkv * d))
    if bf16:
        Kb, Vb = f32_to_bf16(K), f32_to_bf16(V)
        Kd, Vd = dev_bf16(Kb), dev_bf16(Vb)
        K, V = bf16_to_f32(Kb), bf16_to_f32(Vb)
    else:
        Kd, Vd = dev(K), dev(V)
    O = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), Kd, Vd, O, nq, nkv, n, d, scale, n - 1, 0)
    ref = oracle.attn_decode_f64(Q, K, V, nq, nkv, n, d, scale, n - 1, 0, nkv * d, d)
    err = normwise_err(host(O), ref)
    print(f"ramp {kind} n={n} bf16={bf16}: normwise err vs f64 {err:.3e}", flush=True)
    assert err < FP32_TOL


# ---------------------------------------------------------------------------
# size-independent properties at the headline size

def test_properties_at_16k(gpu):
    announce("properties at n=16385")
    st = Stream(5)
    nq, nkv, d, n = 32, 8, 128, 16385
    Q = st.normal((nq, d))
    K = st.normal((n, nkv * d))
    V = np.full((n, nkv * d), -1.25, np.float32)
    O = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), dev(K), dev(V), O, nq, nkv, n, d, 0.088, n - 1, 0)
    np.testing.assert_allclose(host(O), -1.25, rtol=1e-6)  # constant V
    # GQA mapping: V of kv head j is j+1 everywhere -> O[h] = h//4 + 1
    Vj = np.repeat(np.arange(1, nkv + 1, dtype=np.float32), d)[None, :].repeat(n, 0)
    attn.attn_decode_gqa_cache(dev(Q), dev(K), dev(Vj), O, nq, nkv, n, d, 0.088, n - 1, 0)
    np.testing.assert_allclose(host(O), (np.arange(nq) // 4 + 1)[:, None].repeat(d, 1),
                               rtol=1e-6)
    # permutation of (K_t, V_t) pairs
    V = st.normal((n, nkv * d))
    perm = st.permutation(n)
    O2 = torch.empty_like(O)
    attn.attn_decode_gqa_cache(dev(Q), dev(K), dev(V), O, nq, nkv, n, d, 0.088, n - 1, 0)
    attn.attn_decode_gqa_cache(dev(Q), dev(K[perm]), dev(V[perm]), O2, nq, nkv, n, d, 0.088,
                               n - 1, 0)
    assert normwise_err(host(O2), host(O)) < 2e-6
    # window == slicing
    w = 1000
    attn.attn_decode_gqa_cache(dev(Q), dev(K), dev(V), O, nq, nkv, n, d, 0.088, n - 1, w)
    attn.attn_decode_gqa_cache(dev(Q), dev(K[n - w:]), dev(V[n - w:]), O2, nq, nkv, w, d, 0.088,
                               w - 1, 0)
    assert normwise_err(host(O), host(O2)) < 2e-6


def test_fresh_stream_workspace(gpu):
    """First launches on a brand-new stream: its workspace is created by the
    first launch, then grown by a larger one (the old buffer is retired, not
    freed); every launch must match the oracle."""
    s = torch.cuda.Stream()
    for pos, seed in ((3000, 21), (16384, 22), (16384, 23)):
        p = make_decode(32, 8, 128, pos, seed=seed)
        with torch.cuda.stream(s):
            _, _, _, O = run_decode_gpu(p)
        _, _, oO, _, _ = oracle_decode(p)
        assert normwise_err(O, oO) < FP32_TOL, pos


def test_capture_without_warmup_is_refused(gpu):
    """Capturing a shape whose workspace does not exist yet on the capturing
    stream is refused on the host (MOLOT_ENOWS) before anything is launched."""
    from molot_amd.lib import ENOWS, MolotHipError
    # 64 KV heads: more split-K slots than any earlier launch on a pooled stream
    p = make_decode(64, 64, 64, 5000, base=10000.0, seed=24)
    q, kn, vn = dev(p.q), dev(p.k_new), dev(p.v_new)
    K, V, inv = dev(p.K), dev(p.V), dev(p.inv_freq)
    O = torch.empty((64, 64), device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(MolotHipError) as e:
        with torch.cuda.graph(g, stream=s):
            attn.decode_step(q, kn, vn, K, V, O, 64, 64, 64, p.pos, p.pos, inv, p.scale, 0)
    assert e.value.status == ENOWS
    torch.cuda.synchronize()


def test_non_default_stream(gpu):
    s = torch.cuda.Stream()
    p = make_decode(32, 8, 128, 2000, seed=9)
    with torch.cuda.stream(s):
        q_rot, _, _, O = run_decode_gpu(p)
    _, _, oO, _, _ = oracle_decode(p)
    assert normwise_err(O, oO) < FP32_TOL


def test_repeated_calls_are_deterministic(gpu):
    """Fixed block order: bit-identical runs.  Dynamic order (the default):
    runs agree to fp32 rounding of a different summation order."""
    from molot_amd import lib as L
    p = make_decode(32, 8, 128, 16384, seed=10)
    Q = dev(oracle.rope_apply(p.q, p.pos, p.inv_freq))
    K, V = dev(p.K), dev(p.V)

    def runs():
        outs = []
        for _ in range(3):
            O = torch.empty((32, 128), device="cuda")
            attn.attn_decode_gqa_cache(Q, K, V, O, 32, 8, p.pos, 128, p.scale, p.pos - 1, 0)
            outs.append(host(O))
        return outs

    L.load().molot_hip_set_block_order(0)
    try:
        fixed = runs()
    finally:
        L.load().molot_hip_set_block_order(1)
    assert np.array_equal(fixed[0], fixed[1]) and np.array_equal(fixed[1], fixed[2])
    for o in runs():
        assert normwise_err(o, fixed[0]) < 1e-6


# ---------------------------------------------------------------------------
# paged, batched (config 4 and smaller)

def run_paged(P, inv, scale, window=0, pos=None):
    bf = P["Kp"].dtype == np.uint16
    K = dev_bf16(P["Kp"]) if bf else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf else dev(P["Vp"])
    q = dev(P["q"])
    bt, sl = dev(P["bt"].reshape(-1)), dev(P["n"])
    pd = None if pos is None else dev(pos)
    attn.rope_append_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, bt, sl, pd, P["B"],
                           P["max_blocks"], P["nq"], P["nkv"], P["d"], P["page"], dev(inv))
    O = torch.empty((P["B"], P["nq"], P["d"]), device="cuda")
    attn.attn_decode_paged(q, K, V, O, bt, sl, pd, P["B"], P["max_blocks"], P["nq"], P["nkv"],
                           P["d"], P["page"], scale, window)
    if bf:
        Kh = host(K.view(torch.int16)).view(np.uint16)
        Vh = host(V.view(torch.int16)).view(np.uint16)
    else:
        Kh, Vh = host(K), host(V)
    return host(q), Kh, Vh, host(O)


def test_c4_continuous_batching_paged_bf16(gpu):
    announce("c4 64 seqs U[512,8192] paged16 shuffled bf16")
    P = make_paged(64, 32, 8, 128, 512, 8192)
    inv = oracle.rope_inv_freq(500000.0, 128)
    s = 1 / math.sqrt(128)
    q, Kh, Vh, O = run_paged(P, inv, s)
    oq, oK, oV, oO = oracle_paged(P, inv, s)
    np.testing.assert_allclose(q, oq, atol=4e-6, rtol=2e-6)
    np.testing.assert_array_equal(Vh, oV)
    err = normwise_err(O, oO)
    print(f"c4 normwise err {err:.3e}", flush=True)
    assert err < FP32_TOL
    # against the fp32 originals (the same draws, not rounded to bf16): the
    # quantization band of the north star, 2e-2
    Pf = make_paged(64, 32, 8, 128, 512, 8192, bf16=False)
    _, _, _, Of = oracle_paged(Pf, inv, s)
    errf = normwise_err(O, Of)
    print(f"c4 vs fp32 originals {errf:.3e}", flush=True)
    assert errf < BF16_TOL


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("window", [0, 40])
def test_paged_small_ragged(gpu, bf16, window):
    P = make_paged(9, 8, 2, 64, 0, 300, seed=77 + window, bf16=bf16)
    inv = oracle.rope_inv_freq(10000.0, 64)
    q, Kh, Vh, O = run_paged(P, inv, 0.125, window)
    oq, oK, oV, oO = oracle_paged(P, inv, 0.125, window)
    assert normwise_err(O, oO) < FP32_TOL


def run_paged_fused(P, inv, scale, window=0):
    bf = P["Kp"].dtype == np.uint16
    K = dev_bf16(P["Kp"]) if bf else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf else dev(P["Vp"])
    q = dev(P["q"])
    O = torch.empty((P["B"], P["nq"], P["d"]), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O,
                           dev(P["bt"].reshape(-1)), dev(P["n"]), None, P["B"], P["max_blocks"],
                           P["nq"], P["nkv"], P["d"], P["page"], dev(inv), scale, window)
    if bf:
        Kh = host(K.view(torch.int16)).view(np.uint16)
        Vh = host(V.view(torch.int16)).view(np.uint16)
    else:
        Kh, Vh = host(K), host(V)
    return host(q), Kh, Vh, host(O)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("window", [0, 100])
@pytest.mark.parametrize("shape", [(32, 8, 128), (8, 4, 256)], ids=["d128", "d256"])
def test_paged_fused_step(gpu, bf16, window, shape):
    """molot_hip_decode_step_paged (one launch) == oracle rope + append + attention."""
    nq, nkv, d = shape
    announce(f"paged fused {nq}/{nkv}/{d} bf16={bf16} window={window}")
    P = make_paged(17, nq, nkv, d, 0, 2000, seed=5 + window + d, bf16=bf16)
    inv = oracle.rope_inv_freq(500000.0, d)
    s = 1 / math.sqrt(d)
    q, Kh, Vh, O = run_paged_fused(P, inv, s, window)
    oq, oK, oV, oO = oracle_paged(P, inv, s, window)
    np.testing.assert_allclose(q, oq, atol=4e-6, rtol=2e-6)
    np.testing.assert_array_equal(Vh, oV)
    assert normwise_err(O, oO) < FP32_TOL


def test_c4_fused_step(gpu):
    announce("c4 fused decode_step_paged")
    P = make_paged(64, 32, 8, 128, 512, 8192)
    inv = oracle.rope_inv_freq(500000.0, 128)
    s = 1 / math.sqrt(128)
    q, Kh, Vh, O = run_paged_fused(P, inv, s)
    oq, oK, oV, oO = oracle_paged(P, inv, s)
    np.testing.assert_array_equal(Vh, oV)
    assert normwise_err(O, oO) < FP32_TOL
    _, _, _, Of = oracle_paged(make_paged(64, 32, 8, 128, 512, 8192, bf16=False), inv, s)
    assert normwise_err(O, Of) < BF16_TOL  # against the fp32 originals


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("explicit_pos", [False, True])
def test_paged_step_norms(gpu, bf16, explicit_pos):
    """Paged batch with the layer's norms, per sequence; explicit positions
    take the unfused RoPE/append kernel, which applies the same norms."""
    announce(f"paged norms bf16={bf16} explicit_pos={explicit_pos}")
    P = make_paged(13, 32, 8, 128, 0, 1500, seed=61 + bf16, bf16=bf16)
    inv = oracle.rope_inv_freq(500000.0, 128)
    qn, kn = _norm_weights(128, 62)
    pos = (P["n"] - 1 + 7).astype(np.int32) if explicit_pos else None
    bf = P["Kp"].dtype == np.uint16
    K = dev_bf16(P["Kp"]) if bf else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf else dev(P["Vp"])
    q = dev(P["q"])
    O = torch.empty((P["B"], 32, 128), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O,
                           dev(P["bt"].reshape(-1)), dev(P["n"]),
                           None if pos is None else dev(pos), P["B"], P["max_blocks"], 32, 8, 128,
                           16, dev(inv), 0.088, 0, q_norm=dev(qn), k_norm=dev(kn), v_norm=True,
                           eps=1e-6)
    Pn = dict(P)
    Pn["q"] = oracle.rmsnorm(P["q"], qn, 1e-6)
    Pn["k_new"] = oracle.rmsnorm(P["k_new"], kn, 1e-6)
    Pn["v_new"] = oracle.rmsnorm(P["v_new"].reshape(P["B"], -1), None, 1e-6).reshape(
        P["v_new"].shape)
    oq, oK, oV, oO = oracle_paged(Pn, inv, 0.088, 0, pos)
    np.testing.assert_allclose(host(q), oq, rtol=2e-6, atol=4e-6)
    err = normwise_err(host(O), oO)
    print(f"paged norms normwise err {err:.3e}", flush=True)
    if bf:  # the normed v may differ by an fp32 ulp before its bf16 rounding
        Vh = host(V.view(torch.int16)).view(np.uint16)
        for b in range(P["B"]):
            slot = int(P["n"][b]) - 1
            blk = P["bt"][b, slot // 16]
            ref = bf16_to_f32(oV[blk, :, slot % 16])
            assert np.max(np.abs(bf16_to_f32(Vh[blk, :, slot % 16]) - ref)) <= \
                8e-3 * max(1.0, float(np.max(np.abs(ref))))
        assert err < BF16_TOL
    else:
        np.testing.assert_allclose(host(V), oV, rtol=1e-6, atol=1e-7)
        assert err < FP32_TOL


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("dynamic", [0, 1])
def test_graph_replays_match_eager(gpu, dynamic, bf16):
    """The fused step captured in a HIP graph: every replay (with eager work and
    synchronisations between replays) equals the eager result -- bit for bit
    with the fixed block order, to fp32 rounding with the dynamic one.  fp32
    KV runs the vector-ALU kernel, bf16 the matrix-core one; both reuse the
    stream's split-K workspace across replays."""
    from molot_amd import lib as L
    L.load().molot_hip_set_block_order(dynamic)
    try:
        p = make_decode(32, 8, 128, 6000, seed=12, bf16=bf16)
        q0 = dev(p.q)
        K, V = (dev_bf16(p.K), dev_bf16(p.V)) if bf16 else (dev(p.K), dev(p.V))
        kn, vn, inv = dev(p.k_new), dev(p.v_new), dev(p.inv_freq)
        O = torch.empty((32, 128), device="cuda")
        q = q0.clone()
        attn.decode_step(q, kn, vn, K, V, O, 32, 8, 128, p.pos, p.pos, inv, p.scale, 0)
        eager = host(O)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            q.copy_(q0)
            attn.decode_step(q, kn, vn, K, V, O, 32, 8, 128, p.pos, p.pos, inv, p.scale, 0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        qg = q0.clone()
        with torch.cuda.graph(g, stream=s):
            attn.decode_step(qg, kn, vn, K, V, O, 32, 8, 128, p.pos, p.pos, inv, p.scale, 0)
        for r in range(5):
            qg.copy_(q0)
            O.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = host(O)
            if dynamic:
                assert normwise_err(got, eager) < 1e-6, f"replay {r}"
            else:
                assert np.array_equal(got, eager), f"replay {r}"
            # eager work in between replays
            attn.attn_decode_gqa_cache(q, K, V, O, 32, 8, p.pos + 1, 128, p.scale, p.pos, 0)
            torch.cuda.synchronize()
    finally:
        L.load().molot_hip_set_block_order(1)


def test_paged_matches_contiguous(gpu):
    """The same logical cache through a shuffled block table or contiguous."""
    st = Stream(6)
    nq, nkv, d, n, page = 32, 8, 128, 1234, 16
    Q = st.normal((nq, d))
    K = st.normal((n, nkv * d))
    V = st.normal((n, nkv * d))
    nblk = (n + page - 1) // page
    perm = st.permutation(nblk)
    Kp = np.zeros((nblk, nkv, page, d), np.float32)
    Vp = np.zeros_like(Kp)
    for i in range(nblk):
        rows = slice(i * page, min(n, (i + 1) * page))
        m = rows.stop - rows.start
        Kp[perm[i], :, :m] = K[rows].reshape(m, nkv, d).transpose(1, 0, 2)
        Vp[perm[i], :, :m] = V[rows].reshape(m, nkv, d).transpose(1, 0, 2)
    O1 = torch.empty((nq, d), device="cuda")
    O2 = torch.empty((1, nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), dev(K), dev(V), O1, nq, nkv, n, d, 0.088, n - 1, 0)
    attn.attn_decode_paged(dev(Q), dev(Kp), dev(Vp), O2, dev(perm), dev(np.array([n], np.int32)),
                           None, 1, nblk, nq, nkv, d, page, 0.088)
    assert normwise_err(host(O2)[0], host(O1)) < 1e-6


# ---------------------------------------------------------------------------
# errors reported through the ABI, never a launch

def test_error_codes(gpu):
    from molot_amd.lib import MolotHipError
    st = Stream(8)
    Q = dev(st.normal((6, 96)))
    K = dev(st.normal((10, 4 * 96)))
    O = torch.empty((6, 96), device="cuda")
    with pytest.raises(MolotHipError) as e:  # nq % nkv != 0
        attn.attn_decode_gqa_cache(Q, K, K, O, 6, 4, 10, 96, 0.1, 9, 0)
    assert e.value.status == -22
    Q2 = dev(st.normal((4, 96)))
    with pytest.raises(MolotHipError) as e:  # an odd head dim: no kernel takes it
        attn.attn_decode_gqa_cache(Q2, K, K, O, 4, 4, 10, 95, 0.1, 9, 0)
    assert e.value.status == -95
    cache = attn.KVCache(2, 2, 64)
    inv = dev(oracle.rope_inv_freq(10000.0, 64))
    q = dev(st.normal((4, 64)))
    kn = dev(st.normal((2, 64)))
    cache.append(q, kn, kn, 4, 0, inv)
    cache.append(q, kn, kn, 4, 1, inv)
    with pytest.raises(RuntimeError, match="KV cache full"):  # forward.h:570
        cache.append(q, kn, kn, 4, 2, inv)
