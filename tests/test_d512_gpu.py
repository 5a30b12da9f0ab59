"""Head dim 512 (and every even head dim up to it) on every decode, shared-KV
and prefill entry (MI355X only).

The reference's verified gemma4 models alternate 256-dim sliding-window
layers with 512-dim global layers (include/molot/model.h:562-564; qhd comes
from the weights, model.h:518), attend at scale 1 (model.h:39,
forward.h:170-173) after the q/k norms, and give their shared-KV tail's
global layers the 512-dim source (model.h:566-583).  attn.h:125-177 and
gemm.h:409-446 loop over any head dim.

Here the vector-ALU decode kernel runs D = 512 (fp32 V rows as two 16-byte
vectors a lane, a q row's norm summed through LDS, up to 4 q heads a
workgroup); d in (256, 512) runs padded to it.  The prefill at d = 512, and
at any even d that is not a multiple of 8, runs as prefill rows: each query
row a sequence of its own over the one cache.  Bars: 1e-5 normwise against
the oracle (fp32 caches; bf16 and Q8 on the same cache values), and the
oracle itself beside a float64 brute force.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import normwise_err
from gpu_util import dev, dev_bf16, host, make_decode, make_paged, oracle_decode, oracle_paged
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


def on_dev(a):
    return dev_bf16(a) if a.dtype == np.uint16 else dev(a)


def bits(t, like):
    if like.dtype == np.uint16:
        return host(t.view(torch.int16)).view(np.uint16)
    if like.dtype == np.uint8:
        return host(t).view(np.uint8)
    return host(t)


def caches(st, n, nkv, d, kind, sigma=1.0):
    K = st.normal((n, nkv * d), sigma)
    V = st.normal((n, nkv * d), sigma)
    if kind == "bf16":
        return f32_to_bf16(K), f32_to_bf16(V)
    if kind == "q8":
        return oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
    return K, V


def f64_beside(q_rot, K, V, nq, nkv, n, d, scale, pos, window):
    """The float64 brute force (bench/bench.cc:195-213) on the GPU's inputs:
    the oracle is held to it at the same time as the GPU to the oracle."""
    if K.dtype == np.uint8:
        K, V = oracle.q8_dequant(K, nkv, d), oracle.q8_dequant(V, nkv, d)
    elif K.dtype == np.uint16:
        K, V = bf16_to_f32(K), bf16_to_f32(V)
    return oracle.attn_decode_f64(q_rot, K, V, nq, nkv, n, d, scale, pos, window, nkv * d, d)


# ---------------------------------------------------------------------------
# the fused decode step

# (nq, nkv, d, pos, window, kind): G = nq / nkv in {1, 2, 4, 8}
STEPS = [
    (8, 8, 512, 3000, 0, "f32"),      # G = 1
    (8, 4, 512, 5000, 1024, "f32"),   # G = 2, window
    (8, 2, 512, 9000, 0, "f32"),      # G = 4: 2 slots, merged in the launch (1-D XCD map)
    (16, 2, 512, 4000, 0, "f32"),     # G = 8: two subgroups of 4 q heads
    (32, 8, 512, 2000, 0, "f32"),     # 8 slots
    (8, 2, 512, 10, 0, "f32"),        # one chunk
    (8, 2, 512, 6000, 0, "bf16"),
    (16, 2, 512, 3000, 512, "bf16"),  # G = 8, window
    (8, 1, 512, 2500, 0, "bf16"),     # G = 8, one KV head
    (8, 2, 300, 2000, 0, "f32"),      # padded to D = 512
    (8, 4, 384, 1500, 256, "f32"),
    (4, 2, 450, 900, 0, "bf16"),
    (8, 2, 510, 700, 0, "f32"),       # d % 4 == 2
]


def step_ids(s):
    return f"{s[0]}q{s[1]}kv_d{s[2]}_p{s[3]}{'_w' + str(s[4]) if s[4] else ''}_{s[5]}"


@pytest.mark.parametrize("shape", STEPS, ids=[step_ids(s) for s in STEPS])
def test_decode_step_d512(gpu, shape):
    nq, nkv, d, pos, window, kind = shape
    announce(f"decode step {step_ids(shape)}")
    p = make_decode(nq, nkv, d, pos, base=1000000.0, window=window, seed=pos + d + nq,
                    bf16=kind == "bf16")
    q = dev(p.q)
    K, V = on_dev(p.K), on_dev(p.V)
    O = torch.full((nq, d), float("nan"), device="cuda")
    attn.decode_step(q, dev(p.k_new), dev(p.v_new), K, V, O, nq, nkv, d, pos, pos,
                     dev(p.inv_freq), p.scale, window)
    oq, _, oO, oK, oV = oracle_decode(p)
    qh, Kh, Vh, Oh = host(q), bits(K, p.K), bits(V, p.V), host(O)
    np.testing.assert_allclose(qh, oq, atol=4e-6, rtol=2e-6)
    np.testing.assert_array_equal(Kh[:pos], p.K[:pos])
    if kind == "f32":
        np.testing.assert_allclose(Kh[pos], oK[pos], atol=4e-6, rtol=2e-6)
        np.testing.assert_array_equal(Vh[pos], oV[pos])
    else:
        dk = np.abs(bf16_to_f32(Kh[pos]) - bf16_to_f32(oK[pos]))
        assert np.max(dk) <= 8e-3 * max(1.0, float(np.max(np.abs(bf16_to_f32(oK[pos])))))
        np.testing.assert_array_equal(Vh[pos], oV[pos])
    assert np.isfinite(Oh).all()
    err = normwise_err(Oh, oO)
    # the oracle beside float64 on the GPU's own appended cache and q
    R64 = f64_beside(qh, Kh, Vh, nq, nkv, pos + 1, d, p.scale, pos, window)
    e64 = normwise_err(oO, R64)
    print(f"d={d}: normwise err {err:.3e} (oracle vs f64 {e64:.3e})", flush=True)
    assert err < TOL
    assert e64 < TOL
    assert normwise_err(Oh, R64) < TOL


@pytest.mark.parametrize("kind,window", [("f32", 0), ("bf16", 700), ("q8", 0)])
def test_decode_step_norms_scale1_d512(gpu, kind, window):
    """gemma4's global layer: q/k norms, joint v norm, scale 1."""
    announce(f"decode step with norms, scale 1, d=512 {kind} window={window}")
    nq, nkv, d, pos = 8, 2, 512, 2500
    st = Stream(512 + pos + window)
    q = st.normal((nq, d), 2.0)
    k = st.normal((nkv, d), 2.0)
    v = st.normal((nkv, d), 2.0)
    K, V = caches(st, pos + 1, nkv, d, kind)
    K[pos] = 0
    V[pos] = 0
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    inv = oracle.rope_inv_freq(1000000.0, d)
    qd, Kd, Vd = dev(q), on_dev(K), on_dev(V)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, pos, pos, dev(inv), 1.0, window,
                     q_norm=dev(qn), k_norm=dev(kn), v_norm=True, eps=1e-6)
    Kc, Vc = K.copy(), V.copy()
    oq, _, oO = oracle.decode_step_norm(q, k, v, Kc, Vc, nq, nkv, d, pos, pos, qn, kn, 1, 1e-6,
                                        inv, 1.0, window)
    np.testing.assert_allclose(host(qd), oq, atol=4e-6, rtol=2e-6)
    Kh, Vh = bits(Kd, K), bits(Vd, V)
    # the attention against the oracle on the GPU's own rows (a Q8 code of
    # the appended row may sit one off the oracle's when its input differs
    # by an ulp)
    R = oracle.attn_decode_gqa_cache(host(qd), Kh, Vh, nq, nkv, pos + 1, d, 1.0, pos, window)
    err = normwise_err(host(O), R)
    print(f"normwise err {err:.3e} (vs oracle step {normwise_err(host(O), oO):.3e})", flush=True)
    assert err < TOL
    if kind != "q8":
        assert normwise_err(host(O), oO) < TOL


def test_golden_decode_step_norm_d512(gpu):
    """Against the fixture written from the compiled forward.h sequence."""
    announce("golden decode_step_norm_g4_d512_scale1")
    g = golden("decode_step_norm_g4_d512_scale1")
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
    assert normwise_err(host(O), g["O"]) < TOL


def test_decode_step_nope_d512(gpu):
    """A layer without RoPE (inv_freq NULL) at d = 512, with its norms."""
    announce("decode step NoPE d=512")
    nq, nkv, d, pos = 8, 2, 512, 1800
    st = Stream(77)
    q, k, v = st.normal((nq, d), 2.0), st.normal((nkv, d), 2.0), st.normal((nkv, d), 2.0)
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos], V[:pos] = st.normal((pos, nkv * d)), st.normal((pos, nkv * d))
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    qd, Kd, Vd = dev(q), dev(K), dev(V)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, pos, pos, None, 1.0, 0,
                     q_norm=dev(qn), k_norm=dev(kn), v_norm=True, eps=1e-6)
    Kc, Vc = K.copy(), V.copy()
    oq, _, oO = oracle.decode_step_norm(q, k, v, Kc, Vc, nq, nkv, d, pos, pos, qn, kn, 1, 1e-6,
                                        None, 1.0, 0)
    np.testing.assert_allclose(host(qd), oq, atol=4e-6, rtol=2e-6)
    np.testing.assert_allclose(host(Kd)[pos], Kc[pos], atol=4e-6, rtol=2e-6)
    assert normwise_err(host(O), oO) < TOL


# ---------------------------------------------------------------------------
# attention-only entries, paged batches, Q8

@pytest.mark.parametrize("nq,nkv,n,window,kind", [
    (8, 2, 7000, 0, "f32"), (8, 4, 3000, 1000, "f32"), (16, 2, 5000, 0, "q8"),
    (8, 8, 400, 0, "q8"), (8, 2, 33, 0, "bf16")])
def test_attention_entries_d512(gpu, nq, nkv, n, window, kind):
    """attn_decode_gqa_cache (token-major) and, for fp32, attn_decode_gqa
    (head-major) at d = 512."""
    announce(f"attention d=512 {nq}/{nkv} n={n} w={window} {kind}")
    d = 512
    st = Stream(n + nq + 9)
    Q = st.normal((nq, d))
    K, V = caches(st, n, nkv, d, kind)
    s = 1 / math.sqrt(d)
    O = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), on_dev(K), on_dev(V), O, nq, nkv, n, d, s, n - 1, window)
    ref = oracle.attn_decode_gqa_cache(Q, K, V, nq, nkv, n, d, s, n - 1, window)
    assert normwise_err(host(O), ref) < TOL
    assert normwise_err(ref, f64_beside(Q, K, V, nq, nkv, n, d, s, n - 1, window)) < TOL
    if kind == "f32" and window == 0:
        Kh = np.ascontiguousarray(K.reshape(n, nkv, d).transpose(1, 0, 2))
        Vh = np.ascontiguousarray(V.reshape(n, nkv, d).transpose(1, 0, 2))
        O2 = torch.empty((nq, d), device="cuda")
        attn.attn_decode_gqa(dev(Q), dev(Kh), dev(Vh), O2, nq, nkv, n, d, s)
        assert normwise_err(host(O2), ref) < TOL


@pytest.mark.parametrize("d,bf16", [(512, True), (512, False), (420, True)])
def test_paged_decode_step_d512(gpu, d, bf16):
    """A shuffled paged batch of 9 sequences at d = 512 (and a padded d)."""
    announce(f"paged decode step d={d} bf16={bf16}")
    P = make_paged(9, 8, 2, d, 0, 2500, seed=d + 31 + bf16, bf16=bf16)
    inv = oracle.rope_inv_freq(1000000.0, d)
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
    assert normwise_err(host(O), oO) < TOL


def test_q8_decode_step_d512(gpu):
    """The fused step over a Q8 cache at d = 512: the kernel quantizes the
    new rows (quant.h:34-50); at position 0 RoPE is the identity, so the
    appended bytes are the oracle's bit for bit."""
    nq, nkv, d = 8, 2, 512
    for pos in (0, 4000):
        announce(f"q8 decode step d=512 pos={pos}")
        st = Stream(pos + 3)
        q, k, v = st.normal((nq, d), 2.0), st.normal((nkv, d), 2.0), st.normal((nkv, d), 2.0)
        K, V = caches(st, pos + 1, nkv, d, "q8")
        K[pos] = 0
        V[pos] = 0
        inv = oracle.rope_inv_freq(1000000.0, d)
        s = 1 / math.sqrt(d)
        qd, Kd, Vd = dev(q), dev(K), dev(V)
        O = torch.empty((nq, d), device="cuda")
        attn.decode_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, pos, pos, dev(inv), s, 0)
        Kc, Vc = K.copy(), V.copy()
        oq, _, oO = oracle.decode_step(q, k, v, Kc, Vc, nq, nkv, d, pos, pos, inv, s, 0)
        np.testing.assert_allclose(host(qd), oq, rtol=2e-6, atol=4e-6)
        Kh, Vh = bits(Kd, K), bits(Vd, V)
        np.testing.assert_array_equal(Vh[pos], Vc[pos])
        if pos == 0:
            np.testing.assert_array_equal(Kh[pos], Kc[pos])
        R = oracle.attn_decode_gqa_cache(host(qd), Kh, Vh, nq, nkv, pos + 1, d, s, pos, 0)
        assert normwise_err(host(O), R) < TOL


# ---------------------------------------------------------------------------
# layers reading another layer's KV

@pytest.mark.parametrize("kind,window,rope", [("f32", 0, True), ("bf16", 300, True),
                                              ("q8", 0, True), ("f32", 0, False)])
def test_shared_decode_d512(gpu, kind, window, rope):
    announce(f"shared decode d=512 {kind} w={window} rope={rope}")
    nq, nkv, d, n = 8, 2, 512, 3000
    st = Stream(n + window + rope)
    q = st.normal((nq, d))
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K, V = caches(st, n, nkv, d, kind)
    inv = oracle.rope_inv_freq(1000000.0, d) if rope else None
    qd = dev(q)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step_shared(qd, on_dev(K), on_dev(V), O, nq, nkv, d, n, n - 1,
                            None if inv is None else dev(inv), 1.0, window, q_norm=dev(qn),
                            eps=1e-6)
    q_ref, O_ref = oracle.decode_step_shared(q, K, V, nq, nkv, d, n, n - 1, qn, 1e-6, inv, 1.0,
                                             window)
    np.testing.assert_allclose(host(qd), q_ref, rtol=2e-6, atol=4e-6)
    assert normwise_err(host(O), O_ref) < TOL


def test_golden_decode_step_shared_d512(gpu):
    announce("golden decode_step_shared_d512")
    g = golden("decode_step_shared_d512")
    nq, nkv, d, n, pos = (int(g[k]) for k in ("nq", "nkv", "d", "n", "pos"))
    q, Kd, Vd = dev(g["q"]), dev(g["K"]), dev(g["V"])
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step_shared(q, Kd, Vd, O, nq, nkv, d, n, pos, dev(g["inv_freq"]),
                            float(g["scale"]), int(g["window"]), q_norm=dev(g["q_norm"]),
                            eps=float(g["eps"]))
    np.testing.assert_allclose(host(q), g["q_out"], rtol=2e-6, atol=4e-6)
    assert normwise_err(host(O), g["O"]) < TOL


@pytest.mark.parametrize("bf16", [False, True])
def test_shared_paged_decode_d512(gpu, bf16):
    announce(f"shared paged decode d=512 bf16={bf16}")
    P = make_paged(7, 8, 2, 512, 40, 2000, seed=61 + bf16, bf16=bf16)
    B, nq, nkv, d, page = P["B"], 8, 2, 512, 16
    st = Stream(62)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    inv = oracle.rope_inv_freq(1000000.0, d)
    K = dev_bf16(P["Kp"]) if bf16 else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf16 else dev(P["Vp"])
    q = dev(P["q"])
    O = torch.empty((B, nq, d), device="cuda")
    attn.decode_step_paged_shared(q, K, V, O, dev(P["bt"].reshape(-1)), dev(P["n"]), None, B,
                                  P["max_blocks"], nq, nkv, d, page, dev(inv), 1.0, 0,
                                  q_norm=dev(qn), eps=1e-6)
    qh, Oh = host(q), host(O)
    for b in range(B):
        n = int(P["n"][b])
        blk = P["bt"][b, :(n + page - 1) // page]
        Kc = P["Kp"][blk].transpose(0, 2, 1, 3).reshape(-1, nkv * d)[:n]
        Vc = P["Vp"][blk].transpose(0, 2, 1, 3).reshape(-1, nkv * d)[:n]
        q_ref, O_ref = oracle.decode_step_shared(P["q"][b], Kc, Vc, nq, nkv, d, n, n - 1, qn, 1e-6,
                                                 inv, 1.0, 0)
        np.testing.assert_allclose(qh[b], q_ref, rtol=2e-6, atol=4e-6)
        assert normwise_err(Oh[b], O_ref) < TOL, b


# ---------------------------------------------------------------------------
# prefill: d = 512 and even head dims that are not multiples of 8 (prefill rows)

PREFILLS = [
    # (nq, nkv, d, M, N, pos0, window, kind)
    (8, 2, 512, 64, 64, 0, 0, "f32"),        # fresh prompt
    (8, 2, 512, 40, 1040, 1000, 0, "bf16"),  # appended to a context
    (8, 4, 512, 50, 3050, 3000, 1024, "f32"),  # window
    (16, 2, 512, 20, 520, 500, 0, "q8"),     # G = 8, Q8
    (8, 8, 512, 1, 700, 699, 0, "f32"),      # a single query
    (8, 2, 512, 12, 30, 25, 0, "f32"),       # causal end clipped at N
    (8, 2, 36, 70, 170, 100, 0, "f32"),      # d % 8 != 0
    (16, 4, 100, 33, 533, 500, 64, "bf16"),
    (8, 2, 250, 25, 225, 200, 0, "f32"),
    (8, 2, 300, 30, 130, 100, 0, "f32"),     # padded to D = 512
]


@pytest.mark.parametrize("shape", PREFILLS,
                         ids=[f"{s[0]}q{s[1]}kv_d{s[2]}_M{s[3]}_N{s[4]}_w{s[6]}_{s[7]}"
                              for s in PREFILLS])
def test_prefill_d512(gpu, shape):
    nq, nkv, d, M, N, pos0, window, kind = shape
    announce(f"prefill {shape}")
    st = Stream(M + N + d + nq + 7)
    Q = st.normal((M, nq, d))
    K, V = caches(st, N, nkv, d, kind)
    O = torch.full((M, nq, d), float("nan"), device="cuda")
    scale = 1 / math.sqrt(d)
    attn.attn_prefill_gqa(dev(Q), on_dev(K), on_dev(V), O, nq, nkv, M, N, d, scale, pos0, window)
    R = oracle.attn_prefill(Q, K, V, nq, nkv, M, N, d, scale, pos0, window)
    err = normwise_err(host(O), R)
    print(f"prefill normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("d,kind", [(512, "f32"), (512, "bf16"), (512, "q8"), (36, "f32")])
def test_prefill_step_d512(gpu, d, kind):
    """One layer's prefill with norms (forward.h:367-399): 60 prompt tokens
    after 100 cached, at scale 1."""
    announce(f"prefill step 8q/2kv/d{d} M=60 after 100 {kind}")
    st = Stream(170 + d + len(kind))
    nq, nkv, M, n0 = 8, 2, 60, 100
    q = st.normal((M, nq, d), 2.0)
    k = st.normal((M, nkv, d), 2.0)
    v = st.normal((M, nkv, d), 2.0)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K0, V0 = caches(st, n0 + M, nkv, d, kind)
    K0[n0:] = 0
    V0[n0:] = 0
    inv = oracle.rope_inv_freq(1000000.0, d)
    qd, Kd, Vd = dev(q), on_dev(K0), on_dev(V0)
    O = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, M, n0, n0, dev(inv), 1.0, 0,
                      q_norm=dev(qn), k_norm=dev(kn), v_norm=True, eps=1e-6)
    Kc, Vc = K0.copy(), V0.copy()
    q_ref, O_ref = oracle.prefill_step(q, k, v, Kc, Vc, nq, nkv, d, M, n0, n0, qn, kn, 1, 1e-6,
                                       inv, 1.0, 0)
    np.testing.assert_allclose(host(qd), q_ref, rtol=2e-6, atol=4e-6)
    # attention against the oracle on the GPU's own appended rows
    Kh, Vh = bits(Kd, K0), bits(Vd, V0)
    R = oracle.attn_prefill(host(qd), Kh, Vh, nq, nkv, M, n0 + M, d, 1.0, n0, 0)
    err = normwise_err(host(O), R)
    print(f"prefill step normwise err {err:.3e} (vs oracle step "
          f"{normwise_err(host(O), O_ref):.3e})", flush=True)
    assert err < TOL
    if kind == "f32":
        assert normwise_err(host(O), O_ref) < TOL


def test_golden_prefill_d512(gpu):
    announce("golden prefill_norm_d512")
    g = golden("prefill_norm_d512")
    nq, nkv, d, M, pos0 = (int(g[k]) for k in ("nq", "nkv", "d", "M", "pos0"))
    K = np.zeros((pos0 + M, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos0], V[:pos0] = g["K"], g["V"]
    q, Kd, Vd = dev(g["q"]), dev(K), dev(V)
    O = torch.empty((M, nq, d), device="cuda")
    norms = int(g["norms"])
    attn.prefill_step(q, dev(g["k_new"]), dev(g["v_new"]), Kd, Vd, O, nq, nkv, d, M, pos0, pos0,
                      dev(g["inv_freq"]), float(g["scale"]), int(g["window"]),
                      q_norm=dev(g["q_norm"]) if norms else None,
                      k_norm=dev(g["k_norm"]) if norms else None, v_norm=bool(norms),
                      eps=float(g["eps"]))
    np.testing.assert_allclose(host(q), g["q_rot"], rtol=2e-6, atol=4e-6)
    np.testing.assert_allclose(host(Kd)[pos0:], g["K_after"], rtol=2e-6, atol=4e-6)
    assert normwise_err(host(O), g["O"]) < TOL


def test_prefill_paged_d512(gpu):
    """The prefill step through a shuffled block-table row equals the
    contiguous one (to the rounding of the waves' dynamic block claims,
    which order each row's sums differently from run to run), and the
    shared-KV prefill (prefill_q + paged attention) the oracle."""
    announce("paged prefill d=512")
    st = Stream(93)
    nq, nkv, d, M, n0, page = 8, 2, 512, 37, 213, 16
    N = n0 + M
    q = st.normal((M, nq, d))
    k = st.normal((M, nkv, d))
    v = st.normal((M, nkv, d))
    K0, V0 = caches(st, N, nkv, d, "f32")
    K0[n0:] = 0
    V0[n0:] = 0
    nb = (N + page - 1) // page
    row = st.permutation(nb + 3)[:nb].astype(np.int32)
    Kp = np.zeros((nb + 3, nkv, page, d), np.float32)
    Vp = np.zeros_like(Kp)
    for t in range(N):
        Kp[row[t // page], :, t % page] = K0[t].reshape(nkv, d)
        Vp[row[t // page], :, t % page] = V0[t].reshape(nkv, d)
    inv = dev(oracle.rope_inv_freq(1000000.0, d))
    qc, qp = dev(q), dev(q)
    Kc, Vc = dev(K0), dev(V0)
    Kpd, Vpd = dev(Kp.reshape(nb + 3, -1)), dev(Vp.reshape(nb + 3, -1))
    Oc = torch.empty((M, nq, d), device="cuda")
    Op = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(qc, dev(k), dev(v), Kc, Vc, Oc, nq, nkv, d, M, n0, n0, inv, 0.05, 0)
    attn.prefill_step_paged(qp, dev(k), dev(v), Kpd, Vpd, Op, torch.from_numpy(row).cuda(), nb,
                            page, nq, nkv, d, M, n0, n0, inv, 0.05, 0)
    torch.cuda.synchronize()
    assert torch.equal(qp, qc)
    assert normwise_err(host(Op), host(Oc)) < 1e-6
    Kh = host(Kc)
    R = oracle.attn_prefill(host(qc), Kh, host(Vc), nq, nkv, M, N, d, 0.05, n0, 0)
    assert normwise_err(host(Oc), R) < TOL
    # a shared-KV layer's prefill over the same pages
    q2 = dev(q)
    O2 = torch.empty((M, nq, d), device="cuda")
    attn.prefill_q(q2, nq, d, M, n0, inv)
    attn.attn_prefill_paged(q2, Kpd, Vpd, O2, torch.from_numpy(row).cuda(), nb, page, nq, nkv, M, N,
                            d, 0.05, n0)
    R2 = oracle.attn_prefill(host(q2), Kh, host(Vc), nq, nkv, M, N, d, 0.05, n0, 0)
    assert normwise_err(host(O2), R2) < TOL
