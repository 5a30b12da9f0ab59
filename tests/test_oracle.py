"""Pin the CPU oracle before it is trusted to judge the GPU path.

Each oracle function is checked against something other than its own
formula: the reference's known-answer points and attention check
(bench/bench.cc:186-234), the reference's outputs (golden fixtures written
from the compiled reference headers, and the compiled reference itself where
it is available), a float64 brute force, and closed-form invariants chosen so
that a plausible mistake (wrong RoPE pairing, sign, GQA index, dropped
window, missing normalisation) fails one of them.
"""
import glob
import math
import os

import numpy as np
import pytest

import oracle
from conftest import normwise_err
from molot_amd.synth import Stream, bf16_to_f32, f32_to_bf16

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def kv_token_major(st, n, nkv, d, sigma=1.0):
    return st.normal((n, nkv * d), sigma), st.normal((n, nkv * d), sigma)


# ---------------------------------------------------------------------------
# a5 vexp: bench/bench.cc:220-234 known-answer points, relerr < 1e-5

KAT = np.array([-87., -20., -10., -5., -3., -2., -1.5, -1., -0.75, -0.5, -0.25, -0.1, -0.01, 0.,
                1., 50.], np.float32)


def test_vexp_known_answers():
    y = oracle.vexp(KAT)
    ref = np.exp(KAT.astype(np.float64))
    rel = np.max(np.abs(y - ref) / (ref + 1e-30))
    assert rel < 1e-5, rel


def test_vexp_golden_points():
    g = golden("vexp_points")
    y = oracle.vexp(g["X"])
    # restated Taylor-5 vs the reference's compiled exp_avx512_ps; the reference
    # is built with -ffast-math, which flushes denormal results to zero, so
    # results below FLT_MIN may differ by a denormal
    np.testing.assert_allclose(y, g["Y"], rtol=2e-7, atol=1.2e-38)


def test_vexp_clamps_like_reference():
    y = oracle.vexp(np.array([-1000., 1000.], np.float32))
    assert y[0] == pytest.approx(math.exp(-88), rel=1e-5)
    assert y[1] == pytest.approx(math.exp(88), rel=1e-5)


# ---------------------------------------------------------------------------
# a4 dot

def test_dot_matches_double():
    st = Stream(5)
    for n in (1, 15, 16, 17, 128, 131, 256):
        a, b = st.normal(n), st.normal(n)
        ref = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        assert oracle.dot(a, b) == pytest.approx(ref, rel=1e-5, abs=1e-5)


# ---------------------------------------------------------------------------
# a1/a2 RoPE

def test_inv_freq_closed_form():
    for base, d in ((500000.0, 128), (10000.0, 256), (10000.0, 64)):
        got = oracle.rope_inv_freq(base, d)
        ref = 1.0 / np.power(float(base), 2.0 * np.arange(d // 2) / d)
        np.testing.assert_allclose(got, ref, rtol=3e-7)
        assert got[0] == 1.0


def rope_f64(x, pos, inv):
    """NEOX half-split rotation in float64 with the fp32 angle pos*inv_freq."""
    d = x.shape[-1]
    h = d // 2
    ang = (np.float32(pos) * inv.astype(np.float32)).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x = x.astype(np.float64)
    y = np.empty_like(x)
    y[..., :h] = x[..., :h] * c - x[..., h:] * s
    y[..., h:] = x[..., :h] * s + x[..., h:] * c
    return y


def rope_adjacent_f64(x, pos, inv):
    """The (2i, 2i+1) pairing of the dead qk_dot_rope (attn.h:37-52) -- a planted
    mistake: the checks below must tell it apart from rope_apply."""
    ang = (np.float32(pos) * inv.astype(np.float32)).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x = x.astype(np.float64)
    y = np.empty_like(x)
    y[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    y[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
    return y


@pytest.mark.parametrize("name", ["rope_d128_theta5e5", "rope_d256_theta1e4", "rope_d512_theta1e6"])
def test_rope_golden_and_closed_form(name):
    g = golden(name)
    inv = g["inv_freq"]
    for i, pos in enumerate(g["positions"]):
        got = oracle.rope_apply(g["X"][i], int(pos), inv)
        # reference output (compiled rope_apply): within 2 ulp-scale of the data
        assert np.max(np.abs(got - g["Y"][i])) <= 4e-7 * max(1.0, np.max(np.abs(g["Y"][i])))
        # closed form in float64 on the same fp32 angle
        f64 = rope_f64(g["X"][i], int(pos), inv)
        assert np.max(np.abs(got - f64)) < 2e-6
        if pos > 0:
            wrong = rope_adjacent_f64(g["X"][i], int(pos), inv)
            assert np.max(np.abs(wrong - g["Y"][i])) > 1e-2  # the planted mistake is caught


def test_inv_freq_golden_ulps():
    """The reference table is built under -ffast-math, where GCC may lower
    pow(base, e) through exp/log; its bits then differ from a correctly
    rounded powf by an ulp.  The path takes the table as an input, so the
    drop-in passes the caller's bits through unchanged; the formula only has
    to agree to ~2 ulp."""
    for name, base, d in (("rope_d128_theta5e5", 500000.0, 128), ("rope_d256_theta1e4", 10000.0,
                                                                    256)):
        g = golden(name)
        np.testing.assert_allclose(oracle.rope_inv_freq(base, d), g["inv_freq"], rtol=2.5e-7,
                                   atol=0)


def test_rope_invariants():
    st = Stream(7)
    d = 128
    inv = oracle.rope_inv_freq(500000.0, d)
    x = st.normal((4, d))
    # pos 0 is the identity, bit for bit
    assert np.array_equal(oracle.rope_apply(x, 0, inv), x)
    # each pair's norm is preserved
    y = oracle.rope_apply(x, 12345, inv)
    n0 = x[:, :64] ** 2 + x[:, 64:] ** 2
    n1 = y[:, :64].astype(np.float64) ** 2 + y[:, 64:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=2e-6, atol=1e-6)
    # <R_p q, R_p' k> depends only on p - p'
    q, k = st.normal(d), st.normal(d)
    a = float(np.dot(oracle.rope_apply(q, 100, inv).astype(np.float64),
                     oracle.rope_apply(k, 37, inv)))
    b = float(np.dot(oracle.rope_apply(q, 63, inv).astype(np.float64), k))
    assert a == pytest.approx(b, rel=1e-4, abs=1e-4)
    # composition R_a R_b = R_{a+b}
    ab = oracle.rope_apply(oracle.rope_apply(x, 20, inv), 22, inv)
    np.testing.assert_allclose(ab, oracle.rope_apply(x, 42, inv), atol=2e-5)


# ---------------------------------------------------------------------------
# bf16 rounding (quant.h:192-198)

def test_bf16_rne_points():
    bits = np.array([0x3F800000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F808001, 0xBF808000],
                    np.uint32)
    want = np.array([0x3F80, 0x3F80, 0x3F82, 0x3F81, 0x3F81, 0xBF80], np.uint16)
    x = bits.view(np.float32)
    assert np.array_equal(oracle.f32_to_bf16(x), want)
    assert np.array_equal(f32_to_bf16(x), want)
    assert np.array_equal(bf16_to_f32(want), (want.astype(np.uint32) << 16).view(np.float32))


def test_bf16_golden_rounding():
    g = golden("bf16_cache_g8_d128")
    assert np.array_equal(oracle.f32_to_bf16(g["K_f32"]), g["K_bf16"])
    assert np.array_equal(f32_to_bf16(g["V_f32"]), g["V_bf16"])


# ---------------------------------------------------------------------------
# a6-a10 attention

def test_attention_bench_check():
    """bench/bench.cc:186-218: single head, n=512, d=128, N(0,1)*0.2, max-abs < 1e-3
    against the double-precision formulation (here ~1e-7 is reached)."""
    st = Stream(1234)
    n, d = 512, 128
    Q = st.normal(d, 0.2)
    K = st.normal((n, d), 0.2)
    V = st.normal((n, d), 0.2)
    s = 1 / math.sqrt(d)
    O = oracle.attn_decode(Q, K, V, 1, 1, n, d, s, n, 0, d, n * d)
    R = oracle.attn_decode_f64(Q, K, V, 1, 1, n, d, s, n, 0, d, n * d)
    assert np.max(np.abs(O - R)) < 1e-3
    assert normwise_err(O, R) < 1e-5


@pytest.mark.parametrize("name", ["decode_step_g4_d128", "decode_step_win_d256",
                                  "decode_step_g8_d64_scale1"])
def test_decode_step_golden(name):
    g = golden(name)
    nq, nkv, d, pos = int(g["nq"]), int(g["nkv"]), int(g["d"]), int(g["pos"])
    Kc = np.zeros((pos + 1, nkv * d), np.float32)
    Vc = np.zeros_like(Kc)
    Kc[:pos] = g["K"]
    Vc[:pos] = g["V"]
    q_rot, k_rot, O = oracle.decode_step(g["q"], g["k_new"], g["v_new"], Kc, Vc, nq, nkv, d, pos,
                                         pos, g["inv_freq"], float(g["scale"]), int(g["window"]))
    np.testing.assert_allclose(q_rot, g["q_rot"], atol=2e-6)
    np.testing.assert_allclose(k_rot, g["k_rot"], atol=2e-6)
    np.testing.assert_array_equal(Kc[pos], k_rot.reshape(-1))
    np.testing.assert_array_equal(Vc[pos], g["v_new"].reshape(-1))
    assert normwise_err(O, g["O"]) < 2e-6


# ---------------------------------------------------------------------------
# rmsnorm (norm.h:9-28), rmsnorm_plain (norm.h:82-96) and the step with the
# layer's norms (forward.h:554-563)

def _rms_f64(x, w, eps):
    x64 = x.astype(np.float64)
    y = x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    return y if w is None else y * w.astype(np.float64)


def test_rmsnorm_golden_and_closed_form():
    """Against the compiled reference's outputs and the float64 formula, on
    row lengths with and without a scalar tail; the "tiny" rows have
    mean(x^2) ~ eps, so a dropped or misplaced eps fails."""
    g = golden("rmsnorm_cases")
    eps = float(g["eps"])
    for n in g["sizes"]:
        for tag in ("unit", "tiny"):
            x, w = g[f"x_{tag}_{n}"], g[f"w_{tag}_{n}"]
            y, yp = oracle.rmsnorm(x, w, eps), oracle.rmsnorm(x, None, eps)
            np.testing.assert_allclose(y, g[f"y_{tag}_{n}"], rtol=5e-7, atol=0)
            np.testing.assert_allclose(yp, g[f"yplain_{tag}_{n}"], rtol=5e-7, atol=0)
            np.testing.assert_allclose(y, _rms_f64(x, w, eps), rtol=1e-6)
            np.testing.assert_allclose(yp, _rms_f64(x, None, eps), rtol=1e-6)


def test_rmsnorm_invariants():
    st = Stream(32)
    x = st.normal((6, 128))
    w = (1 + st.normal((128,), 0.3)).astype(np.float32)
    # with eps = 0, scaling by 4 is exact through every step: same bits
    np.testing.assert_array_equal(oracle.rmsnorm(4 * x, w, 0.0), oracle.rmsnorm(x, w, 0.0))
    # plain: unit RMS; weighted: the plain result times w, elementwise
    yp = oracle.rmsnorm(x, None, 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(yp.astype(np.float64) ** 2, axis=1)), 1.0,
                               rtol=1e-6)
    np.testing.assert_array_equal(oracle.rmsnorm(x, w, 1e-6), oracle.rmsnorm(x, None, 1e-6) * w)


def _step_norm_from_golden(g):
    nq, nkv, d, pos = int(g["nq"]), int(g["nkv"]), int(g["d"]), int(g["pos"])
    Kc = np.zeros((pos + 1, nkv * d), np.float32)
    Vc = np.zeros_like(Kc)
    Kc[:pos] = g["K"]
    Vc[:pos] = g["V"]
    q_rot, k_rot, O = oracle.decode_step_norm(g["q"], g["k_new"], g["v_new"], Kc, Vc, nq, nkv, d,
                                              pos, pos, g["q_norm"], g["k_norm"],
                                              int(g["v_norm"]), float(g["eps"]), g["inv_freq"],
                                              float(g["scale"]), int(g["window"]))
    return q_rot, k_rot, O, Kc, Vc


@pytest.mark.parametrize("name", ["decode_step_norm_g4_d128", "decode_step_norm_win_d256",
                                  "decode_step_norm_g4_d512_scale1"])
def test_decode_step_norm_golden(name):
    g = golden(name)
    pos = int(g["pos"])
    q_rot, k_rot, O, Kc, Vc = _step_norm_from_golden(g)
    np.testing.assert_allclose(q_rot, g["q_rot"], rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(k_rot, g["k_rot"], rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(Kc[pos], k_rot.reshape(-1))
    np.testing.assert_allclose(Vc[pos], g["v_normed"].reshape(-1), rtol=5e-7, atol=0)
    assert normwise_err(O, g["O"]) < 2e-6


def test_v_norm_is_over_all_kv_heads():
    """forward.h:563 normalises v over all nkv*d values at once; a per-head
    normalisation (a plausible misreading) misses the reference's cache row."""
    g = golden("decode_step_norm_g4_d128")
    nkv, d, eps = int(g["nkv"]), int(g["d"]), float(g["eps"])
    joint = oracle.rmsnorm(g["v_new"].reshape(-1), None, eps)
    per_head = oracle.rmsnorm(g["v_new"].reshape(nkv, d), None, eps).reshape(-1)
    np.testing.assert_allclose(joint, g["v_normed"].reshape(-1), rtol=5e-7, atol=0)
    assert np.max(np.abs(per_head - g["v_normed"].reshape(-1))) > 1e-3


# ---------------------------------------------------------------------------
# Layers without RoPE (an empty L.freq: forward.h:556, :566, :373, :381 skip
# rope_apply) and layers reading another layer's KV (forward.h:578-591,
# :394-398), against fixtures written from the compiled forward.h sequences

def test_decode_step_nope_golden():
    g = golden("decode_step_nope_g4_d128")
    nq, nkv, d, pos = int(g["nq"]), int(g["nkv"]), int(g["d"]), int(g["pos"])
    Kc = np.zeros((pos + 1, nkv * d), np.float32)
    Vc = np.zeros_like(Kc)
    Kc[:pos], Vc[:pos] = g["K"], g["V"]
    q_out, k_out, O = oracle.decode_step_norm(g["q"], g["k_new"], g["v_new"], Kc, Vc, nq, nkv, d,
                                              pos, pos, g["q_norm"], g["k_norm"], 1,
                                              float(g["eps"]), None, float(g["scale"]),
                                              int(g["window"]))
    np.testing.assert_allclose(q_out, g["q_out"], rtol=5e-7, atol=1e-7)  # normed, unrotated
    np.testing.assert_allclose(k_out, g["k_out"], rtol=5e-7, atol=1e-7)
    np.testing.assert_array_equal(Kc[pos], k_out.reshape(-1))
    np.testing.assert_allclose(Vc[pos], g["v_normed"].reshape(-1), rtol=5e-7, atol=0)
    assert normwise_err(O, g["O"]) < 2e-6


def test_planted_rope_on_nope_layer_is_caught():
    """Rotating a NoPE layer's q and k (with any table, here the model's
    usual one) misses the reference's step, which leaves them unrotated."""
    g = golden("decode_step_nope_g4_d128")
    nq, nkv, d, pos = int(g["nq"]), int(g["nkv"]), int(g["d"]), int(g["pos"])
    Kc = np.zeros((pos + 1, nkv * d), np.float32)
    Vc = np.zeros_like(Kc)
    Kc[:pos], Vc[:pos] = g["K"], g["V"]
    q_out, _, O = oracle.decode_step_norm(g["q"], g["k_new"], g["v_new"], Kc, Vc, nq, nkv, d, pos,
                                          pos, g["q_norm"], g["k_norm"], 1, float(g["eps"]),
                                          oracle.rope_inv_freq(500000.0, d), float(g["scale"]),
                                          int(g["window"]))
    assert np.max(np.abs(q_out - g["q_out"])) > 1e-2
    assert normwise_err(O, g["O"]) > 1e-4


@pytest.mark.parametrize("name", ["decode_step_shared_g4_d128", "decode_step_shared_nope_win_d256",
                                  "decode_step_shared_d512"])
def test_decode_step_shared_golden(name):
    g = golden(name)
    nq, nkv, d, n, pos = (int(g[k]) for k in ("nq", "nkv", "d", "n", "pos"))
    inv = g["inv_freq"] if int(g["rope"]) else None
    K, V = g["K"].copy(), g["V"].copy()
    q_out, O = oracle.decode_step_shared(g["q"], K, V, nq, nkv, d, n, pos, g["q_norm"],
                                         float(g["eps"]), inv, float(g["scale"]), int(g["window"]))
    np.testing.assert_allclose(q_out, g["q_out"], rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(K, g["K"])  # nothing appended
    # d = 512 at scale 1 with a normed q and unnormed keys: scores ~ N(0, d),
    # |s - max| up to ~60, where one fp32 ulp of a score moves its weight by
    # ~4e-6 relative; the path's 1e-5 normwise parity bar applies there
    assert normwise_err(O, g["O"]) < (2e-6 if d <= 256 else 1e-5)


def test_shared_step_equals_owning_step():
    """A layer reading a cache that already holds this token's row (the
    source layer appended it earlier in the step) gets the owning layer's
    output and rotated q: the shared step is the decode step minus its
    append."""
    st = Stream(41)
    nq, nkv, d, pos, window = 8, 2, 128, 300, 0
    q, k, v = st.normal((nq, d)), st.normal((nkv, d)), st.normal((nkv, d))
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos], V[:pos] = kv_token_major(st, pos, nkv, d)
    inv = oracle.rope_inv_freq(500000.0, d)
    q1, _, O1 = oracle.decode_step_norm(q, k, v, K, V, nq, nkv, d, pos, pos, qn, None, 0, 1e-6,
                                        inv, 0.1, window)
    q2, O2 = oracle.decode_step_shared(q, K, V, nq, nkv, d, pos + 1, pos, qn, 1e-6, inv, 0.1,
                                       window)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(O1, O2)


def test_prefill_nope_golden():
    g = golden("prefill_nope_d128")
    nq, nkv, d, M, pos0 = (int(g[k]) for k in ("nq", "nkv", "d", "M", "pos0"))
    Kc = np.zeros((pos0 + M, nkv * d), np.float32)
    Vc = np.zeros_like(Kc)
    Kc[:pos0], Vc[:pos0] = g["K"], g["V"]
    q_out, O = oracle.prefill_step(g["q"], g["k_new"], g["v_new"], Kc, Vc, nq, nkv, d, M, pos0,
                                   pos0, g["q_norm"], g["k_norm"], 1, float(g["eps"]), None,
                                   float(g["scale"]), int(g["window"]))
    np.testing.assert_allclose(q_out, g["q_out"], rtol=5e-7, atol=1e-7)
    np.testing.assert_allclose(Kc[pos0:], g["K_after"], rtol=5e-7, atol=1e-7)
    np.testing.assert_allclose(Vc[pos0:], g["V_after"], rtol=1e-6, atol=1e-7)
    assert normwise_err(O, g["O"]) < 2e-6


def test_prefill_shared_golden():
    g = golden("prefill_shared_win_d128")
    nq, nkv, d, M, N, pos0 = (int(g[k]) for k in ("nq", "nkv", "d", "M", "N", "pos0"))
    q_out = oracle.prefill_q(g["q"], nq, d, M, pos0, g["q_norm"], float(g["eps"]), g["inv_freq"])
    O = oracle.attn_prefill(q_out, g["K"], g["V"], nq, nkv, M, N, d, float(g["scale"]), pos0,
                            int(g["window"]))
    np.testing.assert_allclose(q_out, g["q_out"], rtol=2e-6, atol=4e-6)
    assert normwise_err(O, g["O"]) < 2e-6


# ---------------------------------------------------------------------------
# prefill attention (gemm.h:409-446) and the layer's prefill (forward.h:367-399)

def _prefill_f64(Q, K, V, nq, nkv, M, N, d, scale, pos0, window):
    G = nq // nkv
    O = np.zeros((M, nq, d))
    for m in range(M):
        pos = pos0 + m
        t0 = min(max(0, pos - window + 1) if window > 0 else 0, N)
        nn = min(pos + 1, N)
        if nn <= t0:
            continue
        for h in range(nq):
            kv = h // G
            Kh = K[t0:nn, kv * d:(kv + 1) * d].astype(np.float64)
            Vh = V[t0:nn, kv * d:(kv + 1) * d].astype(np.float64)
            s = Kh @ Q[m, h].astype(np.float64) * scale
            e = np.exp(s - s.max())
            O[m, h] = (e / e.sum()) @ Vh
    return O


@pytest.mark.parametrize("name", ["prefill_g4_d64", "prefill_norm_win_d128", "prefill_norm_d512"])
def test_prefill_golden(name):
    g = golden(name)
    nq, nkv, d, M, pos0 = (int(g[k]) for k in ("nq", "nkv", "d", "M", "pos0"))
    Kc = np.zeros((pos0 + M, nkv * d), np.float32)
    Vc = np.zeros_like(Kc)
    Kc[:pos0], Vc[:pos0] = g["K"], g["V"]
    norms = int(g["norms"])
    q_rot, O = oracle.prefill_step(g["q"], g["k_new"], g["v_new"], Kc, Vc, nq, nkv, d, M, pos0,
                                   pos0, g["q_norm"] if norms else None,
                                   g["k_norm"] if norms else None, norms, float(g["eps"]),
                                   g["inv_freq"], float(g["scale"]), int(g["window"]))
    np.testing.assert_allclose(q_rot, g["q_rot"], rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(Kc[pos0:], g["K_after"], rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(Vc[pos0:], g["V_after"], rtol=1e-6, atol=1e-7)
    assert normwise_err(O, g["O"]) < 2e-6


@pytest.mark.parametrize("nq,nkv,d,M,N,pos0,window", [(8, 2, 64, 40, 90, 50, 0),
                                                      (4, 4, 128, 33, 33, 0, 0),
                                                      (16, 1, 64, 20, 70, 50, 16),
                                                      (6, 2, 256, 9, 200, 191, 0),
                                                      (8, 2, 64, 12, 30, 25, 0),
                                                      (8, 4, 96, 20, 120, 100, 33),
                                                      (8, 2, 40, 12, 30, 25, 0),
                                                      (4, 2, 512, 10, 60, 50, 0),
                                                      (4, 1, 512, 7, 40, 33, 9),
                                                      (6, 2, 36, 15, 40, 25, 0),
                                                      (4, 2, 100, 9, 50, 41, 20),
                                                      (4, 1, 250, 8, 30, 22, 0)])
def test_prefill_vs_f64(nq, nkv, d, M, N, pos0, window):
    """Causal masking, windows, a cache longer than the prompt's positions
    (pos0 + M > N clips at N) and every GQA grouping, against float64."""
    st = Stream(M + N + d)
    Q = st.normal((M, nq, d))
    K, V = kv_token_major(st, N, nkv, d)
    O = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, 1 / math.sqrt(d), pos0, window)
    R = _prefill_f64(Q, K, V, nq, nkv, M, N, d, 1 / math.sqrt(d), pos0, window)
    assert normwise_err(O, R) < 1e-6


def test_prefill_single_query_is_decode_attention():
    """M = 1 at pos0 = N - 1 is the decode attention of attn.h:125-177 (which
    uses the vector exp: the two differ by its 1.5e-6 relative error)."""
    st = Stream(34)
    nq, nkv, d, N = 32, 8, 128, 777
    Q = st.normal((1, nq, d))
    K, V = kv_token_major(st, N, nkv, d)
    for window in (0, 100):
        O = oracle.attn_prefill(Q, K, V, nq, nkv, 1, N, d, 0.088, N - 1, window)
        R = oracle.attn_decode_gqa_cache(Q[0], K, V, nq, nkv, N, d, 0.088, N - 1, window)
        assert normwise_err(O[0], R) < 5e-6


def test_prefill_first_token_sees_only_itself():
    st = Stream(35)
    nq, nkv, d, M = 8, 2, 64, 5
    Q = st.normal((M, nq, d))
    K, V = kv_token_major(st, M, nkv, d)
    O = oracle.attn_prefill(Q, K, V, nq, nkv, M, M, d, 0.125, 0, 0)
    for h in range(nq):
        np.testing.assert_array_equal(O[0, h], V[0, (h // 4) * d:(h // 4 + 1) * d])


def test_planted_non_causal_prefill_is_caught():
    """Attending the whole cache instead of the causal prefix fails float64."""
    st = Stream(36)
    nq, nkv, d, M, N = 4, 1, 64, 16, 16
    Q = st.normal((M, nq, d))
    K, V = kv_token_major(st, N, nkv, d)
    R = _prefill_f64(Q, K, V, nq, nkv, M, N, d, 0.125, 0, 0)
    full = np.stack([oracle.attn_decode_gqa_cache(Q[m], K, V, nq, nkv, N, d, 0.125, N - 1, 0)
                     for m in range(M)])
    assert normwise_err(full, R) > 1e-2


# ---------------------------------------------------------------------------
# Q8 KV cache: quantize_q8_row (quant.h:34-50) per KV head row

@pytest.mark.parametrize("name", ["q8_rows_d128", "q8_rows_d512"])
def test_q8_quantizer_golden(name):
    """Bit-exact against the compiled reference on its edge cases (zero row,
    exact half-step ties, tiny values, the absmax element at +-127)."""
    g = golden(name)
    for i in range(g["X"].shape[0]):
        s, q = oracle.quantize_q8_row(g["X"][i])
        assert s == g["S"][i], i
        np.testing.assert_array_equal(q, g["Q"][i])


def test_q8_quantizer_bounds():
    st = Stream(38)
    for sigma in (1.0, 5.0, 1e-4):
        x = st.normal((128,), sigma)
        s, q = oracle.quantize_q8_row(x)
        assert s == np.float32(np.abs(x).max()) / np.float32(127.0)
        assert np.abs(q.astype(np.int32)).max() == 127
        # round-off at most half a step (division and product rounding aside)
        assert np.max(np.abs(x - q.astype(np.float32) * np.float32(s))) <= 0.5 * s * (1 + 1e-5)
    # values already on the grid come back exactly
    k = np.arange(-127, 129, 2, dtype=np.float32)[:128]
    s, q = oracle.quantize_q8_row(k * np.float32(0.25))
    assert s == 0.25
    np.testing.assert_array_equal(q, k.astype(np.int8))


@pytest.mark.parametrize("nkv,d", [(4, 128), (4, 100), (3, 36)])
def test_q8_attention_is_attention_on_dequantized_rows(nkv, d):
    """The Q8 cache read through its byte layout (rows, then per-head scales)
    gives bit for bit the attention over its dequantized fp32 rows: pins the
    scale addressing, which a wrong offset would break, also at head dims
    whose rows end off a 16-byte boundary (nkv = 3, d = 36: 108 codes, 12
    scale bytes, 8 bytes of padding)."""
    st = Stream(39 + d)
    nq, n = 4 * nkv, 301
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d, 2.0)
    Kq, Vq = oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
    assert Kq.shape == (n, nkv * d + (4 * nkv + 15) // 16 * 16)  # codes, then padded scales
    Kd, Vd = oracle.q8_dequant(Kq, nkv, d), oracle.q8_dequant(Vq, nkv, d)
    for window in (0, 77):
        a = oracle.attn_decode_gqa_cache(Q, Kq, Vq, nq, nkv, n, d, 0.088, n - 1, window)
        b = oracle.attn_decode_gqa_cache(Q, Kd, Vd, nq, nkv, n, d, 0.088, n - 1, window)
        np.testing.assert_array_equal(a, b)
    # and the quantization error of the cache is the 8-bit one
    assert np.max(np.abs(Kd - K)) <= np.abs(K).max() / 127 * 0.51


@pytest.mark.parametrize("nkv,d", [(4, 256), (8, 128), (2, 64), (2, 100), (1, 300)])
def test_q8_prefill_is_prefill_on_dequantized_rows(nkv, d):
    """The prefill over a Q8 cache gives bit for bit the prefill over its
    dequantized fp32 rows, at the matrix-core head dims (d = 256: 1040-byte
    rows at nkv = 4) and at padded ones: pins the prefill's Q8 row and scale
    addressing."""
    st = Stream(41 + d)
    nq, M, N, pos0 = 2 * nkv, 17, 240, 223
    Q = st.normal((M, nq, d))
    K, V = kv_token_major(st, N, nkv, d, 2.0)
    Kq, Vq = oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
    Kd, Vd = oracle.q8_dequant(Kq, nkv, d), oracle.q8_dequant(Vq, nkv, d)
    for window in (0, 50):
        a = oracle.attn_prefill(Q, Kq, Vq, nq, nkv, M, N, d, 0.0625, pos0, window)
        b = oracle.attn_prefill(Q, Kd, Vd, nq, nkv, M, N, d, 0.0625, pos0, window)
        np.testing.assert_array_equal(a, b)
        assert normwise_err(a, _prefill_f64(Q, Kd, Vd, nq, nkv, M, N, d, 0.0625, pos0,
                                            window)) < 1e-6


def test_q8_decode_step_appends_quantized_row():
    st = Stream(40)
    nq, nkv, d, pos = 8, 2, 64, 90
    q, k, v = st.normal((nq, d)), st.normal((nkv, d)), st.normal((nkv, d))
    K, V = kv_token_major(st, pos + 1, nkv, d)
    Kq, Vq = oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
    inv = oracle.rope_inv_freq(10000.0, d)
    _, k_rot, O = oracle.decode_step(q, k, v, Kq, Vq, nq, nkv, d, pos, pos, inv, 0.125, 0)
    np.testing.assert_array_equal(Kq[pos], oracle.q8_cache(k_rot.reshape(1, -1), nkv, d)[0])
    np.testing.assert_array_equal(Vq[pos], oracle.q8_cache(v.reshape(1, -1), nkv, d)[0])


@pytest.mark.parametrize("d", [64, 100])
def test_q8_paged_is_token_major_through_a_block_table(d):
    """Paged Q8 blocks ([nkv][page][d] codes, then [nkv][page] scales) read
    through a shuffled block table give bit for bit the token-major Q8
    attention on the same rows: pins the paged scale addressing."""
    st = Stream(41 + d)
    nq, nkv, n, page = 16, 4, 203, 16
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d, 2.0)
    nblk = (n + page - 1) // page
    perm = st.permutation(nblk + 3)[:nblk].astype(np.int32)
    Kp = np.zeros((nblk + 3, nkv, page, d), np.float32)
    Vp = np.zeros_like(Kp)
    for i in range(nblk):
        rows = slice(i * page, min(n, (i + 1) * page))
        m = rows.stop - rows.start
        Kp[perm[i], :, :m] = K[rows].reshape(m, nkv, d).transpose(1, 0, 2)
        Vp[perm[i], :, :m] = V[rows].reshape(m, nkv, d).transpose(1, 0, 2)
    Pk, Pv = oracle.q8_pages(Kp), oracle.q8_pages(Vp)
    assert Pk.shape == (nblk + 3, nkv * page * (d + 4))
    # the pages dequantize to the token-major cache's rows
    Kd = oracle.q8_dequant(oracle.q8_cache(K, nkv, d), nkv, d)
    Pd = oracle.q8_pages_dequant(Pk, nkv, d, page)
    for i in range(nblk):
        m = min(n, (i + 1) * page) - i * page
        np.testing.assert_array_equal(Pd[perm[i], :, :m],
                                      Kd[i * page:i * page + m].reshape(m, nkv, d).transpose(1, 0, 2))
    for window in (0, 50):
        a = oracle.attn_decode_paged(Q[None], Pk, Pv, perm[None], np.array([n], np.int32), None, 1,
                                     nblk, nq, nkv, d, page, 0.1, window)[0]
        b = oracle.attn_decode_gqa_cache(Q, oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d),
                                         nq, nkv, n, d, 0.1, n - 1, window)
        np.testing.assert_array_equal(a, b)
    # one slot rewritten in place equals re-quantizing the pages with it
    x = st.normal((nkv, d))
    P2 = Pk.copy()
    oracle.q8_page_store(P2, int(perm[3]), 5, x, nkv, d, page)
    Kp[perm[3], :, 5] = x
    np.testing.assert_array_equal(P2, oracle.q8_pages(Kp))


def test_head_golden():
    g = golden("head_bench_check")
    n, d = int(g["n"]), int(g["d"])
    O = oracle.attn_decode(g["Q"], g["K"], g["V"], 1, 1, n, d, float(g["scale"]), n, 0, d, n * d)
    assert normwise_err(O[0], g["O"]) < 2e-6


@pytest.mark.parametrize("name", ["gqa_headmajor_d64", "gqa_win_headmajor_d64"])
def test_headmajor_golden(name):
    g = golden(name)
    nq, nkv, n, d = (int(g[k]) for k in ("nq", "nkv", "n", "d"))
    O = oracle.attn_decode(g["Q"], g["K"], g["V"], nq, nkv, n, d, float(g["scale"]),
                           int(g["pos_cur"]), int(g["window"]), d, n * d)
    assert normwise_err(O, g["O"]) < 2e-6


def test_bf16_golden_attention():
    g = golden("bf16_cache_g8_d128")
    nq, nkv, n, d = (int(g[k]) for k in ("nq", "nkv", "n", "d"))
    O = oracle.attn_decode(g["Q"], g["K_bf16"], g["V_bf16"], nq, nkv, n, d, float(g["scale"]),
                           n - 1, 0, nkv * d, d)
    assert normwise_err(O, g["O"]) < 2e-6


@pytest.mark.parametrize("nq,nkv,d,n,window", [(32, 8, 128, 4097, 0), (8, 4, 256, 3000, 1024),
                                               (64, 8, 128, 2500, 0), (4, 4, 64, 333, 7),
                                               # head dims the GPU runs padded, and d = 512
                                               (8, 2, 34, 900, 0), (16, 4, 80, 1200, 300),
                                               (8, 4, 250, 700, 0), (8, 2, 512, 1500, 0),
                                               (16, 2, 512, 800, 256), (4, 4, 300, 400, 0),
                                               (8, 8, 2, 700, 0)])
def test_restatement_vs_f64(nq, nkv, d, n, window):
    st = Stream(nq * 1000 + n)
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d)
    s = 1 / math.sqrt(d)
    O = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, s, n - 1, window)
    R = oracle.attn_decode_f64(Q, K, V, nq, nkv, n, d, s, n - 1, window, nkv * d, d)
    assert normwise_err(O, R) < 1e-5


# closed-form attention properties -------------------------------------------

def test_constant_v_gives_constant_output():
    st = Stream(21)
    nq, nkv, d, n = 8, 2, 128, 300
    Q = st.normal((nq, d))
    K = st.normal((n, nkv * d))
    V = np.full((n, nkv * d), 0.375, np.float32)
    O = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.1, n - 1, 0)
    np.testing.assert_allclose(O, 0.375, rtol=2e-6)


def test_equal_keys_give_mean_of_window():
    st = Stream(22)
    nq, nkv, d, n, w = 4, 1, 64, 200, 50
    Q = st.normal((nq, d))
    K = np.tile(st.normal((1, d)), (n, 1))
    V = st.normal((n, d))
    O = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.3, n - 1, w)
    want = V[n - w:].astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(O, np.tile(want, (nq, 1)), atol=2e-6)


def test_dominant_key_selects_its_value():
    st = Stream(23)
    nq, nkv, d, n = 2, 1, 64, 100
    Q = st.normal((nq, d))
    K = st.normal((n, d)) * 0.01
    K[37] = Q[0] * 50  # score ~ 50*|q|^2*scale >> others for head 0
    V = st.normal((n, d))
    O = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 1.0, n - 1, 0)
    np.testing.assert_allclose(O[0], V[37], atol=1e-5)


def test_gqa_head_mapping():
    """query head h reads KV head h // (nq/nkv) (attn.h:131)."""
    st = Stream(24)
    nq, nkv, d, n = 12, 3, 64, 50
    Q = st.normal((nq, d))
    K = st.normal((n, nkv * d))
    V = np.zeros((n, nkv, d), np.float32)
    for j in range(nkv):
        V[:, j, :] = j + 1
    O = oracle.attn_decode_gqa_cache(Q, K, V.reshape(n, -1), nq, nkv, n, d, 0.2, n - 1, 0)
    for h in range(nq):
        np.testing.assert_allclose(O[h], h // (nq // nkv) + 1, rtol=2e-6)


def test_window_equals_sliced_full_attention():
    st = Stream(25)
    nq, nkv, d, n, w = 8, 4, 256, 500, 64
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d)
    full_w = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.06, n - 1, w)
    sliced = oracle.attn_decode_gqa_cache(Q, K[n - w:], V[n - w:], nq, nkv, w, d, 0.06, w - 1, 0)
    np.testing.assert_array_equal(full_w, sliced)
    # window >= n and window <= 0 are the full prefix
    a = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.06, n - 1, 0)
    b = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.06, n - 1, n + 5)
    np.testing.assert_array_equal(a, b)


def test_empty_range_gives_zero():
    st = Stream(26)
    Q = st.normal((2, 64))
    K = st.normal((10, 64))
    O = oracle.attn_decode_gqa_cache(Q, K, K, 2, 1, 10, 64, 0.1, 100, 5)  # t0 = 96 > n
    assert np.all(O == 0)


def test_permutation_invariance():
    st = Stream(27)
    nq, nkv, d, n = 8, 2, 128, 700
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d)
    perm = st.permutation(n)
    a = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.09, n - 1, 0)
    b = oracle.attn_decode_gqa_cache(Q, K[perm], V[perm], nq, nkv, n, d, 0.09, n - 1, 0)
    assert normwise_err(b, a) < 2e-6


def test_layouts_agree():
    """token-major [n][nkv*d], head-major [nkv][n][d] and paged are one computation."""
    st = Stream(28)
    nq, nkv, d, n, page = 8, 2, 64, 333, 16
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d)
    tm = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.1, n - 1, 0)
    Kh = np.ascontiguousarray(K.reshape(n, nkv, d).transpose(1, 0, 2))
    Vh = np.ascontiguousarray(V.reshape(n, nkv, d).transpose(1, 0, 2))
    hm = oracle.attn_decode(Q, Kh, Vh, nq, nkv, n, d, 0.1, n - 1, 0, d, n * d)
    np.testing.assert_array_equal(tm, hm)
    nblk = (n + page - 1) // page
    perm = st.permutation(nblk + 5)[:nblk]
    Kp = np.zeros((nblk + 5, nkv, page, d), np.float32)
    Vp = np.zeros_like(Kp)
    for i in range(nblk):
        rows = slice(i * page, min(n, (i + 1) * page))
        m = rows.stop - rows.start
        Kp[perm[i], :, :m] = K[rows].reshape(m, nkv, d).transpose(1, 0, 2)
        Vp[perm[i], :, :m] = V[rows].reshape(m, nkv, d).transpose(1, 0, 2)
    pg = oracle.attn_decode_paged(Q, Kp, Vp, perm.reshape(1, -1), np.array([n]), None, 1, nblk,
                                  nq, nkv, d, page, 0.1)
    np.testing.assert_array_equal(pg[0], tm)


def test_thread_count_invariance():
    st = Stream(29)
    nq, nkv, d, n = 32, 8, 128, 1000
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d)
    a = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.08, n - 1, 0, nthreads=1)
    b = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, 0.08, n - 1, 0, nthreads=5)
    np.testing.assert_array_equal(a, b)


def test_planted_missing_normalisation_is_caught():
    """A variant that skips 1/den must fail the f64 comparison the GPU is held to."""
    st = Stream(30)
    nq, nkv, d, n = 4, 1, 64, 64
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d)
    R = oracle.attn_decode_f64(Q, K, V, nq, nkv, n, d, 0.125, n - 1, 0, nkv * d, d)
    s = (Q.astype(np.float64) @ K.astype(np.float64).T) * 0.125
    e = np.exp(s - s.max(axis=1, keepdims=True))
    unnormalised = e @ V.astype(np.float64)
    assert normwise_err(unnormalised, R) > 1e-2


def test_golden_fixture_set_present():
    names = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))
    assert len(names) >= 10, names


# ---------------------------------------------------------------------------
# against the compiled reference, where it is available on this host

needs_ref = pytest.mark.skipif(not oracle.ref_available(),
                               reason="compiled reference not available on this host")


@needs_ref
def test_ref_pool_coverage():
    """bench/bench.cc:59-66: parallel_for touches every index exactly once."""
    with oracle.RefPool(4) as pool:
        seen = np.zeros(100000, np.int32)
        oracle.ref().ref_pool_cover(pool.h, seen.size, oracle._p(seen))
        assert np.all(seen == 1)


@needs_ref
@pytest.mark.parametrize("nq,nkv,d,n,window,pos_cur", [(32, 8, 128, 4097, 0, 4096),
                                                       (8, 4, 256, 2100, 1024, 2099),
                                                       (8, 8, 64, 17, 0, 16),
                                                       (16, 2, 128, 1, 0, 0),
                                                       (8, 2, 34, 300, 0, 299),
                                                       (16, 4, 80, 500, 100, 499),
                                                       (8, 4, 250, 400, 0, 399),
                                                       (8, 2, 512, 600, 0, 599),
                                                       (16, 2, 512, 300, 128, 299)])
def test_restatement_vs_reference(nq, nkv, d, n, window, pos_cur):
    st = Stream(n + d)
    Q = st.normal((nq, d))
    K, V = kv_token_major(st, n, nkv, d)
    s = 1 / math.sqrt(d)
    O = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, s, pos_cur, window)
    R = np.empty_like(O)
    with oracle.RefPool(4) as pool:
        oracle.ref().ref_attn_decode_gqa_cache(oracle._p(Q), oracle._p(K), oracle._p(V),
                                               oracle._p(R), nq, nkv, n, d, s, pos_cur, window,
                                               pool.h)
    assert normwise_err(O, R) < 2e-6


@needs_ref
def test_decode_step_norm_vs_reference():
    """The restated step with norms against the compiled forward.h sequence
    at the headline head shape (q/k norm weights, joint v norm, window)."""
    st = Stream(33)
    nq, nkv, d, pos, window = 32, 8, 128, 1500, 700
    q, k, v = st.normal((nq, d), 2.0), st.normal((nkv, d), 2.0), st.normal((nkv, d), 2.0)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos], V[:pos] = kv_token_major(st, pos, nkv, d)
    inv = oracle.rope_inv_freq(500000.0, d)
    Ko, Vo = K.copy(), V.copy()
    q_rot, k_rot, O = oracle.decode_step_norm(q, k, v, Ko, Vo, nq, nkv, d, pos, pos, qn, kn, 1,
                                              1e-6, inv, 1.0, window)
    qr, kr, vr = q.copy(), k.copy(), v.copy()
    Kr, Vr = K.copy(), V.copy()
    R = np.empty((nq, d), np.float32)
    P = oracle._p
    with oracle.RefPool(4) as pool:
        rc = oracle.ref().ref_decode_step_norm(P(qr), P(kr), P(vr), P(Kr), P(Vr), P(R), nq, nkv, d,
                                               pos, pos + 1, pos, P(qn), P(kn), 1, 1e-6, P(inv),
                                               1.0, window, pool.h)
    assert rc == 0
    np.testing.assert_allclose(q_rot, qr, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(Vo[pos], Vr[pos], rtol=5e-7, atol=0)
    assert normwise_err(O, R) < 2e-6


@needs_ref
def test_prefill_vs_reference():
    st = Stream(37)
    nq, nkv, d, M, N, pos0 = 32, 8, 128, 70, 300, 230
    Q = st.normal((M, nq, d))
    K, V = kv_token_major(st, N, nkv, d)
    for window in (0, 64):
        O = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, 0.088, pos0, window)
        R = np.empty_like(O)
        with oracle.RefPool(4) as pool:
            oracle.ref().ref_attn_prefill_gqa(oracle._p(Q), oracle._p(K), oracle._p(V),
                                              oracle._p(R), nq, nkv, M, N, d, 0.088, pos0, window,
                                              pool.h)
        assert normwise_err(O, R) < 1e-6


@needs_ref
def test_vexp_vs_reference_random():
    st = Stream(31)
    x = (st.normal(4096) * 20).clip(-100, 100).astype(np.float32)
    y = oracle.vexp(x)
    r = np.empty_like(x)
    for i in range(0, x.size, 16):
        oracle.ref().ref_exp16(oracle._p(x[i:i + 16]), oracle._p(r[i:i + 16]))
    np.testing.assert_allclose(y, r, rtol=2e-7, atol=1.2e-38)  # reference flushes denormals


@needs_ref
def test_nope_and_shared_steps_vs_reference():
    """The restated NoPE step and shared-KV step against the compiled
    forward.h sequences at the headline head shape, with a window."""
    st = Stream(43)
    nq, nkv, d, pos, window = 32, 8, 128, 1200, 500
    q, k, v = st.normal((nq, d), 2.0), st.normal((nkv, d), 2.0), st.normal((nkv, d), 2.0)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos], V[:pos] = kv_token_major(st, pos, nkv, d)
    P = oracle._p
    Ko, Vo = K.copy(), V.copy()
    q1, _, O1 = oracle.decode_step_norm(q, k, v, Ko, Vo, nq, nkv, d, pos, pos, qn, kn, 1, 1e-6,
                                        None, 1.0, window)
    qr, kr, vr, Kr, Vr = q.copy(), k.copy(), v.copy(), K.copy(), V.copy()
    R1 = np.empty((nq, d), np.float32)
    inv = oracle.rope_inv_freq(10000.0, d)
    q2, O2 = oracle.decode_step_shared(q, Ko, Vo, nq, nkv, d, pos + 1, pos, qn, 1e-6, inv, 1.0,
                                       window)
    qs_ = q.copy()
    R2 = np.empty((nq, d), np.float32)
    with oracle.RefPool(4) as pool:
        rc = oracle.ref().ref_decode_step_norm(P(qr), P(kr), P(vr), P(Kr), P(Vr), P(R1), nq, nkv,
                                               d, pos, pos + 1, pos, P(qn), P(kn), 1, 1e-6, None,
                                               1.0, window, pool.h)
        assert rc == 0
        rc = oracle.ref().ref_decode_step_shared(P(qs_), P(Kr), P(Vr), P(R2), nq, nkv, d, pos + 1,
                                                 pos, P(qn), 1e-6, P(inv), 1.0, window, pool.h)
        assert rc == 0
    np.testing.assert_allclose(q1, qr, rtol=5e-7, atol=1e-7)
    np.testing.assert_allclose(Vo[pos], Vr[pos], rtol=5e-7, atol=0)
    assert normwise_err(O1, R1) < 2e-6
    np.testing.assert_allclose(q2, qs_, rtol=2e-6, atol=2e-6)
    assert normwise_err(O2, R2) < 2e-6
