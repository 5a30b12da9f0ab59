"""Layers without RoPE and layers reading another layer's KV (MI355X only).

forward.h rotates q and k only when the layer has a frequency table
(forward.h:373, :381, :556, :566: `if (!L.freq.empty())`; rope_swa_only
models give their global layers none, model.h:535-536).  A layer without
its own KV (L.has_kv false, the shared-KV tail of model.h:562-583) norms
and rotates q, appends nothing and attends the source layer's cache over
its n slots (forward.h:578-591 for decode, :370-375 and :394-398 for
prefill).  The entries: inv_freq = NULL on every fused entry;
molot_hip_decode_step_shared, molot_hip_decode_step_paged_shared,
molot_hip_prefill_q and molot_hip_attn_prefill_paged.  Checked against
fixtures written from the compiled forward.h sequences and against the
oracle at 1e-5 normwise (fp32 caches; bf16 and Q8 against the oracle run
on the same cache bytes).
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
from molot_amd.synth import Stream, f32_to_bf16

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def announce(msg):
    print(f"[case] {msg}", flush=True)


def on_dev(a):
    """A host cache as a device tensor of its type (fp32, bf16 bits, Q8 bytes)."""
    if a.dtype == np.uint16:
        return dev_bf16(a)
    return dev(a)


def cache_host(t, like):
    if like.dtype == np.uint16:
        return host(t.view(torch.int16)).view(np.uint16)
    return host(t)


def kv_cache(st, n, nkv, d, kind):
    """[n][row] caches of N(0,1) rows: fp32, bf16 bits or Q8 bytes."""
    K = st.normal((n, nkv * d))
    V = st.normal((n, nkv * d))
    if kind == "bf16":
        return f32_to_bf16(K), f32_to_bf16(V)
    if kind == "q8":
        return oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)
    return K, V


# ---------------------------------------------------------------------------
# layers without RoPE

def test_golden_decode_step_nope(gpu):
    announce("golden decode_step_nope_g4_d128")
    g = golden("decode_step_nope_g4_d128")
    nq, nkv, d, pos = int(g["nq"]), int(g["nkv"]), int(g["d"]), int(g["pos"])
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos], V[:pos] = g["K"], g["V"]
    q, Kd, Vd = dev(g["q"]), dev(K), dev(V)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step(q, dev(g["k_new"]), dev(g["v_new"]), Kd, Vd, O, nq, nkv, d, pos, pos, None,
                     float(g["scale"]), int(g["window"]), q_norm=dev(g["q_norm"]),
                     k_norm=dev(g["k_norm"]), v_norm=True, eps=float(g["eps"]))
    np.testing.assert_allclose(host(q), g["q_out"], rtol=2e-6, atol=2e-6)  # normed, unrotated
    Kh, Vh = host(Kd), host(Vd)
    np.testing.assert_allclose(Kh[pos], g["k_out"].reshape(-1), rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(Vh[pos], g["v_normed"].reshape(-1), rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(Kh[:pos], g["K"])
    assert normwise_err(host(O), g["O"]) < FP32_TOL


@pytest.mark.parametrize("nq,nkv,d,pos,window,kind", [(32, 8, 128, 5000, 0, "f32"),
                                                      (8, 4, 256, 3000, 300, "f32"),
                                                      (64, 8, 128, 9000, 0, "bf16"),
                                                      (32, 8, 128, 4000, 0, "q8")])
def test_nope_decode_step_vs_oracle(gpu, nq, nkv, d, pos, window, kind):
    """The fused step with inv_freq = NULL: q left unrotated (bit for bit),
    k appended unrotated, O as the oracle's NoPE step."""
    announce(f"nope step {nq}/{nkv}/{d} pos {pos} w {window} {kind}")
    st = Stream(pos + d)
    q, k, v = st.normal((nq, d)), st.normal((nkv, d)), st.normal((nkv, d))
    K, V = kv_cache(st, pos + 1, nkv, d, kind)
    K[pos] = 0
    V[pos] = 0
    Kd, Vd = on_dev(K), on_dev(V)
    qd = dev(q)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, pos, pos, None, 0.09, window)
    np.testing.assert_array_equal(host(qd), q)
    Kc, Vc = K.copy(), V.copy()
    _, k_out, O_ref = oracle.decode_step(q, k, v, Kc, Vc, nq, nkv, d, pos, pos, None, 0.09, window)
    np.testing.assert_array_equal(k_out, k)
    np.testing.assert_array_equal(cache_host(Vd, V)[pos], Vc[pos])
    np.testing.assert_array_equal(cache_host(Kd, K)[pos], Kc[pos])
    assert normwise_err(host(O), O_ref) < FP32_TOL


@pytest.mark.parametrize("bf16", [False, True])
def test_nope_paged_step(gpu, bf16):
    announce(f"nope paged step bf16={bf16}")
    P = make_paged(9, 32, 8, 128, 100, 2500, seed=71 + bf16, bf16=bf16)
    K = dev_bf16(P["Kp"]) if bf16 else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf16 else dev(P["Vp"])
    q = dev(P["q"])
    O = torch.empty((P["B"], 32, 128), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O, dev(P["bt"].reshape(-1)),
                           dev(P["n"]), None, P["B"], P["max_blocks"], 32, 8, 128, 16, None, 0.088,
                           0)
    np.testing.assert_array_equal(host(q), P["q"])
    _, _, oV, oO = oracle_paged(P, None, 0.088)
    np.testing.assert_array_equal(cache_host(V, P["Vp"]), oV)
    assert normwise_err(host(O), oO) < FP32_TOL


def test_golden_prefill_nope(gpu):
    announce("golden prefill_nope_d128")
    g = golden("prefill_nope_d128")
    nq, nkv, d, M, pos0 = (int(g[k]) for k in ("nq", "nkv", "d", "M", "pos0"))
    K = np.zeros((pos0 + M, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos0], V[:pos0] = g["K"], g["V"]
    q, Kd, Vd = dev(g["q"]), dev(K), dev(V)
    O = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(q, dev(g["k_new"]), dev(g["v_new"]), Kd, Vd, O, nq, nkv, d, M, pos0, pos0,
                      None, float(g["scale"]), int(g["window"]), q_norm=dev(g["q_norm"]),
                      k_norm=dev(g["k_norm"]), v_norm=True, eps=float(g["eps"]))
    np.testing.assert_allclose(host(q), g["q_out"], rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(host(Kd)[pos0:], g["K_after"], rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(host(Vd)[pos0:], g["V_after"], rtol=2e-6, atol=2e-6)
    assert normwise_err(host(O), g["O"]) < FP32_TOL


# ---------------------------------------------------------------------------
# layers reading another layer's KV

@pytest.mark.parametrize("name", ["decode_step_shared_g4_d128", "decode_step_shared_nope_win_d256"])
def test_golden_decode_step_shared(gpu, name):
    announce(f"golden {name}")
    g = golden(name)
    nq, nkv, d, n, pos = (int(g[k]) for k in ("nq", "nkv", "d", "n", "pos"))
    inv = dev(g["inv_freq"]) if int(g["rope"]) else None
    q, Kd, Vd = dev(g["q"]), dev(g["K"]), dev(g["V"])
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step_shared(q, Kd, Vd, O, nq, nkv, d, n, pos, inv, float(g["scale"]),
                            int(g["window"]), q_norm=dev(g["q_norm"]), eps=float(g["eps"]))
    np.testing.assert_allclose(host(q), g["q_out"], rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(host(Kd), g["K"])  # nothing appended
    np.testing.assert_array_equal(host(Vd), g["V"])
    assert normwise_err(host(O), g["O"]) < FP32_TOL


@pytest.mark.parametrize("nq,nkv,d,n,window,kind,rope", [
    (32, 8, 128, 16385, 0, "f32", True),     # c2's cache, split and merged
    (32, 8, 128, 300, 0, "f32", False),
    (8, 4, 256, 5000, 1000, "f32", True),
    (64, 8, 128, 20000, 0, "bf16", True),    # matrix-core kernel
    (32, 8, 128, 3000, 0, "q8", True),
    (32, 8, 64, 1, 0, "f32", True),           # one slot
])
def test_shared_decode_vs_oracle(gpu, nq, nkv, d, n, window, kind, rope):
    announce(f"shared decode {nq}/{nkv}/{d} n {n} w {window} {kind} rope={rope}")
    st = Stream(n + 3 * d)
    q = st.normal((nq, d))
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K, V = kv_cache(st, n, nkv, d, kind)
    inv = oracle.rope_inv_freq(500000.0, d) if rope else None
    pos = n - 1
    qd = dev(q)
    Kd, Vd = on_dev(K), on_dev(V)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step_shared(qd, Kd, Vd, O, nq, nkv, d, n, pos, None if inv is None else dev(inv),
                            0.088, window, q_norm=dev(qn), eps=1e-6)
    q_ref, O_ref = oracle.decode_step_shared(q, K, V, nq, nkv, d, n, pos, qn, 1e-6, inv, 0.088,
                                             window)
    np.testing.assert_allclose(host(qd), q_ref, rtol=2e-6, atol=4e-6)
    assert normwise_err(host(O), O_ref) < FP32_TOL
    np.testing.assert_array_equal(cache_host(Kd, K), K)


@pytest.mark.parametrize("bf16", [False, True])
def test_shared_paged_decode(gpu, bf16):
    """A batch attending another layer's pages: each sequence equals the
    oracle's shared step on its own rows gathered from the pages."""
    announce(f"shared paged decode bf16={bf16}")
    P = make_paged(11, 32, 8, 128, 50, 3000, seed=81 + bf16, bf16=bf16)
    B, nq, nkv, d, page = P["B"], 32, 8, 128, 16
    st = Stream(82)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    inv = oracle.rope_inv_freq(500000.0, d)
    K = dev_bf16(P["Kp"]) if bf16 else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf16 else dev(P["Vp"])
    q = dev(P["q"])
    O = torch.empty((B, nq, d), device="cuda")
    attn.decode_step_paged_shared(q, K, V, O, dev(P["bt"].reshape(-1)), dev(P["n"]), None, B,
                                  P["max_blocks"], nq, nkv, d, page, dev(inv), 0.088, 0,
                                  q_norm=dev(qn), eps=1e-6)
    qh, Oh = host(q), host(O)
    for b in range(B):
        n = int(P["n"][b])
        blk = P["bt"][b, :(n + page - 1) // page]
        Kc = P["Kp"][blk].transpose(0, 2, 1, 3).reshape(-1, nkv * d)[:n]
        Vc = P["Vp"][blk].transpose(0, 2, 1, 3).reshape(-1, nkv * d)[:n]
        q_ref, O_ref = oracle.decode_step_shared(P["q"][b], Kc, Vc, nq, nkv, d, n, n - 1, qn, 1e-6,
                                                 inv, 0.088, 0)
        np.testing.assert_allclose(qh[b], q_ref, rtol=2e-6, atol=4e-6)
        assert normwise_err(Oh[b], O_ref) < FP32_TOL, b


@pytest.mark.parametrize("bf16", [False, True])
def test_shared_paged_decode_empty_window(gpu, bf16):
    """A shared-KV batch with positions given: sequences whose window starts
    past their cache (pos - window + 1 >= n) attend nothing, so o = 0, yet
    their q still leaves normed and rotated (forward.h:554-558 runs before
    every attention call); the others equal the oracle's shared step."""
    announce(f"shared paged decode, emptied windows, bf16={bf16}")
    P = make_paged(9, 32, 8, 128, 50, 900, seed=85 + bf16, bf16=bf16)
    B, nq, nkv, d, page, window = P["B"], 32, 8, 128, 16, 64
    st = Stream(86)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    inv = oracle.rope_inv_freq(500000.0, d)
    # positions: some at the cache end, some far past it (window emptied)
    pos = np.array([int(P["n"][b]) - 1 + (0 if b % 3 else 5000) for b in range(B)], np.int32)
    K = dev_bf16(P["Kp"]) if bf16 else dev(P["Kp"])
    V = dev_bf16(P["Vp"]) if bf16 else dev(P["Vp"])
    q = dev(P["q"])
    O = torch.full((B, nq, d), float("nan"), device="cuda")
    attn.decode_step_paged_shared(q, K, V, O, dev(P["bt"].reshape(-1)), dev(P["n"]), dev(pos), B,
                                  P["max_blocks"], nq, nkv, d, page, dev(inv), 0.088, window,
                                  q_norm=dev(qn), eps=1e-6)
    qh, Oh = host(q), host(O)
    for b in range(B):
        n = int(P["n"][b])
        blk = P["bt"][b, :(n + page - 1) // page]
        Kc = P["Kp"][blk].transpose(0, 2, 1, 3).reshape(-1, nkv * d)[:n]
        Vc = P["Vp"][blk].transpose(0, 2, 1, 3).reshape(-1, nkv * d)[:n]
        q_ref, O_ref = oracle.decode_step_shared(P["q"][b], Kc, Vc, nq, nkv, d, n, int(pos[b]), qn,
                                                 1e-6, inv, 0.088, window)
        np.testing.assert_allclose(qh[b], q_ref, rtol=2e-6, atol=4e-6, err_msg=f"seq {b}")
        if b % 3 == 0:
            assert np.all(Oh[b] == 0.0), b
        else:
            assert normwise_err(Oh[b], O_ref) < FP32_TOL, b


def test_golden_prefill_shared(gpu):
    announce("golden prefill_shared_win_d128")
    g = golden("prefill_shared_win_d128")
    nq, nkv, d, M, N, pos0 = (int(g[k]) for k in ("nq", "nkv", "d", "M", "N", "pos0"))
    q, Kd, Vd = dev(g["q"]), dev(g["K"]), dev(g["V"])
    O = torch.empty((M, nq, d), device="cuda")
    attn.prefill_q(q, nq, d, M, pos0, dev(g["inv_freq"]), q_norm=dev(g["q_norm"]),
                   eps=float(g["eps"]))
    attn.attn_prefill_gqa(q, Kd, Vd, O, nq, nkv, M, N, d, float(g["scale"]), pos0,
                          int(g["window"]))
    np.testing.assert_allclose(host(q), g["q_out"], rtol=2e-6, atol=4e-6)
    assert normwise_err(host(O), g["O"]) < FP32_TOL


@pytest.mark.parametrize("rope", [True, False])
def test_shared_prefill_paged_matches_contiguous(gpu, rope):
    """The shared-KV prefill through a shuffled block-table row equals the
    contiguous one bit for bit, and the oracle's."""
    announce(f"shared paged prefill rope={rope}")
    st = Stream(91)
    nq, nkv, d, M, N, pos0, page = 16, 4, 128, 37, 250, 213, 16
    q = st.normal((M, nq, d))
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    K, V = kv_cache(st, N, nkv, d, "f32")
    nb = (N + page - 1) // page
    row = st.permutation(nb + 3)[:nb].astype(np.int32)
    Kp = np.zeros((nb + 3, nkv, page, d), np.float32)
    Vp = np.zeros_like(Kp)
    for t in range(N):
        Kp[row[t // page], :, t % page] = K[t].reshape(nkv, d)
        Vp[row[t // page], :, t % page] = V[t].reshape(nkv, d)
    inv = oracle.rope_inv_freq(500000.0, d) if rope else None
    invd = None if inv is None else dev(inv)
    qc, qp = dev(q), dev(q)
    Oc = torch.empty((M, nq, d), device="cuda")
    Op = torch.empty((M, nq, d), device="cuda")
    attn.prefill_q(qc, nq, d, M, pos0, invd, q_norm=dev(qn))
    attn.attn_prefill_gqa(qc, dev(K), dev(V), Oc, nq, nkv, M, N, d, 0.088, pos0, 0)
    attn.prefill_q(qp, nq, d, M, pos0, invd, q_norm=dev(qn))
    attn.attn_prefill_paged(qp, dev(Kp.reshape(nb + 3, -1)), dev(Vp.reshape(nb + 3, -1)), Op,
                            torch.from_numpy(row).cuda(), nb, page, nq, nkv, M, N, d, 0.088, pos0)
    torch.cuda.synchronize()
    assert torch.equal(qp, qc)
    assert torch.equal(Op, Oc)
    q_ref = oracle.prefill_q(q, nq, d, M, pos0, qn, 1e-6, inv)
    np.testing.assert_allclose(host(qc), q_ref, rtol=2e-6, atol=4e-6)
    R = oracle.attn_prefill(q_ref, K, V, nq, nkv, M, N, d, 0.088, pos0, 0)
    assert normwise_err(host(Oc), R) < FP32_TOL


@pytest.mark.parametrize("d,norm,rope", [(512, True, True), (2048, True, False),
                                         (300, False, True), (192, True, True), (64, True, True)])
def test_prefill_q_head_dims(gpu, d, norm, rope):
    """molot_hip_prefill_q at any even d up to 2048 (one 4-wave workgroup per
    token; lane l of a head's wave takes pairs l, l + 64, ...; instances for
    up to 64, 128 and 1024 pairs), with and without the norm and the
    rotation, against the oracle."""
    announce(f"prefill_q d={d} norm={norm} rope={rope}")
    st = Stream(500 + d)
    nq, M, pos0 = 4, 37, 1000
    q = st.normal((M, nq, d))
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32) if norm else None
    inv = oracle.rope_inv_freq(10000.0, d) if rope else None
    qd = dev(q)
    attn.prefill_q(qd, nq, d, M, pos0, None if inv is None else dev(inv),
                   q_norm=None if qn is None else dev(qn))
    q_ref = oracle.prefill_q(q, nq, d, M, pos0, qn, 1e-6, inv)
    np.testing.assert_allclose(host(qd), q_ref, rtol=2e-6, atol=4e-6)


def test_shared_step_equals_owning_step(gpu):
    """After the owning layer's fused step appended this token, a layer
    sharing its cache (same q, norm and table) gets the owning layer's O
    and rotated q."""
    announce("shared step == owning step")
    p = make_decode(32, 8, 128, 7000, seed=93)
    qn = dev((1 + Stream(94).normal((128,), 0.2)).astype(np.float32))
    inv = dev(p.inv_freq)
    K, V = dev(p.K), dev(p.V)
    q1, q2 = dev(p.q), dev(p.q)
    O1 = torch.empty((32, 128), device="cuda")
    O2 = torch.empty((32, 128), device="cuda")
    attn.decode_step(q1, dev(p.k_new), dev(p.v_new), K, V, O1, 32, 8, 128, p.pos, p.pos, inv,
                     p.scale, 0, q_norm=qn)
    attn.decode_step_shared(q2, K, V, O2, 32, 8, 128, p.pos + 1, p.pos, inv, p.scale, 0, q_norm=qn)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert normwise_err(host(O2), host(O1)) < 1e-6
