"""Parity of the Q8 KV cache paths with the oracle (MI355X only).

Q8 rows are the reference's Q8_0 row quantizer (include/molot/quant.h:34-50)
per KV head row; the layouts are this library's (include/molot_amd/attn_hip.h,
oracle/attn_oracle.c).  Every call goes through the C ABI.

Bars:
  * attention over the same Q8 bytes: normwise max|gpu-ref|/max|ref| <= 1e-5
    against the oracle, which dequantizes each row as code * s in fp32 (the
    kernels widen codes to bf16 exactly and carry q and p in three bf16
    pieces, so they are fp32-accurate on those values);
  * rows the kernels quantize: bit-exact codes and scales where their fp32
    input is the oracle's bit for bit (v without its norm; k at position 0,
    where RoPE is the identity); elsewhere the rotated or normed input may
    differ by an fp32 ulp, so a code may differ by one and a scale by an ulp.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import normwise_err
from gpu_util import dev, host, make_paged
from molot_amd import attn
from molot_amd.lib import EINVAL, ENOTSUP, MolotHipError
from molot_amd.synth import Stream

pytestmark = pytest.mark.gpu

TOL = 1e-5


def announce(msg):
    print(f"[case] {msg}", flush=True)


def dev_u8(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def host_u8(t: torch.Tensor) -> np.ndarray:
    return host(t).view(np.uint8)


def q8_caches(st, N, nkv, d, sigma=1.0):
    K = st.normal((N, nkv * d), sigma)
    V = st.normal((N, nkv * d), sigma)
    return oracle.q8_cache(K, nkv, d), oracle.q8_cache(V, nkv, d)


def split_row(C, nkv, d):
    """(codes [nkv][d] int8, scales [nkv] fp32) of one token-major Q8 row."""
    codes = C[:nkv * d].view(np.int8).reshape(nkv, d)
    scales = np.ascontiguousarray(C[nkv * d:nkv * d + 4 * nkv]).view(np.float32)
    return codes, scales


def assert_rows_close(got, ref, nkv, d):
    """Quantized rows of fp32 inputs that may differ by an ulp: scales within
    a few ulps, codes within one."""
    gc, gs = split_row(got, nkv, d)
    rc, rs = split_row(ref, nkv, d)
    np.testing.assert_allclose(gs, rs, rtol=4e-7 * 8)
    assert np.max(np.abs(gc.astype(np.int32) - rc.astype(np.int32))) <= 1


# ---------------------------------------------------------------------------
# attention over a Q8 cache

@pytest.mark.parametrize("nq,nkv,d,n,pos,window", [
    (32, 8, 128, 4097, 4096, 0),     # headline head shape
    (32, 8, 64, 1000, 999, 0),
    (64, 8, 128, 3001, 3000, 0),     # G = 8
    (16, 16, 64, 777, 776, 0),       # G = 1
    (12, 4, 128, 500, 499, 100),     # G = 3, window
    (32, 2, 64, 50, 49, 0),          # G = 16, one short chunk
    (32, 8, 128, 20000, 19999, 4096),
    (8, 2, 128, 1, 0, 0),            # a single row
    (8, 4, 256, 32769, 32768, 1024),  # Gemma-shaped c3 layer: d = 256 on the vector-ALU kernel
    (16, 2, 256, 3000, 2999, 0),     # d = 256, G = 8
    (8, 8, 256, 40, 39, 0),          # d = 256, one chunk
])
def test_q8_decode_vs_oracle(gpu, nq, nkv, d, n, pos, window):
    announce(f"q8 decode {nq}/{nkv}/{d} n={n} window={window}")
    st = Stream(n + nq + d)
    Q = st.normal((nq, d))
    Kq, Vq = q8_caches(st, n, nkv, d)
    O = torch.empty((nq, d), device="cuda")
    s = 1 / math.sqrt(d)
    attn.attn_decode_gqa_cache(dev(Q), dev_u8(Kq), dev_u8(Vq), O, nq, nkv, n, d, s, pos, window)
    R = oracle.attn_decode_gqa_cache(Q, Kq, Vq, nq, nkv, n, d, s, pos, window)
    err = normwise_err(host(O), R)
    print(f"q8 normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("factor", [100.0, 1000.0])
def test_q8_decode_outlier_q_channels(gpu, factor):
    """q with a few channels factor x the rest (LLM activations have such
    outliers), at the usual 1/sqrt(d) scale: the scores' int8 pieces share
    one scale per head, so this is where their resolution would show."""
    announce(f"q8 decode with {factor:g}x outlier q channels")
    st = Stream(int(factor) + 5)
    nq, nkv, d, n = 32, 8, 128, 3000
    Q = st.normal((nq, d))
    Q[:, [3, 40, 77, 100]] *= factor
    Kq, Vq = q8_caches(st, n, nkv, d)
    O = torch.empty((nq, d), device="cuda")
    s = 1 / math.sqrt(d)
    attn.attn_decode_gqa_cache(dev(Q), dev_u8(Kq), dev_u8(Vq), O, nq, nkv, n, d, s, n - 1, 0)
    R = oracle.attn_decode_gqa_cache(Q, Kq, Vq, nq, nkv, n, d, s, n - 1, 0)
    err = normwise_err(host(O), R)
    print(f"q8 outlier normwise err {err:.3e}", flush=True)
    assert err < TOL


def test_q8_equals_fp32_on_dequantized_rows(gpu):
    """Q8 attention == fp32-cache attention on the dequantized rows (the
    fp32 vector-ALU kernel), to fp32 rounding."""
    st = Stream(11)
    nq, nkv, d, n = 32, 8, 128, 5000
    Q = st.normal((nq, d))
    Kq, Vq = q8_caches(st, n, nkv, d, 3.0)
    O8 = torch.empty((nq, d), device="cuda")
    O32 = torch.empty((nq, d), device="cuda")
    attn.attn_decode_gqa_cache(dev(Q), dev_u8(Kq), dev_u8(Vq), O8, nq, nkv, n, d, 0.088, n - 1, 0)
    attn.attn_decode_gqa_cache(dev(Q), dev(oracle.q8_dequant(Kq, nkv, d)),
                               dev(oracle.q8_dequant(Vq, nkv, d)), O32, nq, nkv, n, d, 0.088,
                               n - 1, 0)
    assert normwise_err(host(O8), host(O32)) < TOL


def test_q8_split_plans_agree(gpu):
    """The same Q8 problem cut into different chunk counts."""
    st = Stream(12)
    nq, nkv, d, n = 32, 8, 128, 9000
    Q = st.normal((nq, d))
    Kq, Vq = q8_caches(st, n, nkv, d)
    R = oracle.attn_decode_gqa_cache(Q, Kq, Vq, nq, nkv, n, d, 0.088, n - 1, 0)
    Qd, Kd, Vd = dev(Q), dev_u8(Kq), dev_u8(Vq)
    try:
        for chunk in (0, 64, 512, 2048):
            attn.set_split_chunk(chunk)
            O = torch.empty((nq, d), device="cuda")
            attn.attn_decode_gqa_cache(Qd, Kd, Vd, O, nq, nkv, n, d, 0.088, n - 1, 0)
            assert normwise_err(host(O), R) < TOL, f"chunk {chunk}"
    finally:
        attn.set_split_chunk(0)


# ---------------------------------------------------------------------------
# the fused step: RoPE, append (quantized in the kernel), attention

@pytest.mark.parametrize("d,pos,window,norms", [
    (128, 0, 0, False),      # RoPE is the identity: every byte exact
    (128, 3000, 0, False),
    (64, 1500, 0, True),
    (128, 5000, 1024, True),
    (128, 2000, 1, False),   # the window holds the new token only
])
def test_q8_decode_step_vs_oracle(gpu, d, pos, window, norms, nq=32, nkv=8):
    announce(f"q8 decode_step {nq}/{nkv}/{d} pos={pos} window={window} norms={norms}")
    st = Stream(pos + d + window)
    q = st.normal((nq, d), 2.0)
    k = st.normal((nkv, d), 2.0)
    v = st.normal((nkv, d), 2.0)
    Kq, Vq = q8_caches(st, pos + 1, nkv, d)
    Kq[pos] = 0
    Vq[pos] = 0
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32) if norms else None
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32) if norms else None
    inv = oracle.rope_inv_freq(500000.0, d)
    s = 1 / math.sqrt(d)
    qd, Kd, Vd = dev(q), dev_u8(Kq), dev_u8(Vq)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, pos, pos, dev(inv), s, window,
                     q_norm=None if qn is None else dev(qn),
                     k_norm=None if kn is None else dev(kn), v_norm=norms, eps=1e-6)
    Kc, Vc = Kq.copy(), Vq.copy()
    oq, _, oO = oracle.decode_step_norm(q, k, v, Kc, Vc, nq, nkv, d, pos, pos, qn, kn,
                                        int(norms), 1e-6, inv, s, window)
    np.testing.assert_allclose(host(qd), oq, rtol=2e-6, atol=4e-6)
    Kh, Vh = host_u8(Kd), host_u8(Vd)
    np.testing.assert_array_equal(Kh[:pos], Kq[:pos])  # the cache before the slot untouched
    if pos == 0 and not norms:
        np.testing.assert_array_equal(Kh[pos], Kc[pos])
    else:
        assert_rows_close(Kh[pos], Kc[pos], nkv, d)
    if not norms:
        np.testing.assert_array_equal(Vh[pos], Vc[pos])
    else:
        assert_rows_close(Vh[pos], Vc[pos], nkv, d)
    # the attention against the oracle on the GPU's own rows
    R = oracle.attn_decode_gqa_cache(host(qd), Kh, Vh, nq, nkv, pos + 1, d, s, pos, window)
    err = normwise_err(host(O), R)
    print(f"q8 step normwise err {err:.3e} (vs oracle step {normwise_err(host(O), oO):.3e})",
          flush=True)
    assert err < TOL
    assert normwise_err(host(O), oO) < 1e-3  # a code off by one moves o by ~1e-5 of its scale


@pytest.mark.parametrize("nq,nkv,pos,window,norms", [
    (8, 4, 0, 0, False),        # RoPE is the identity: every byte exact
    (8, 4, 32768, 1024, False),  # the Gemma-shaped c3 layer over a Q8 cache
    (16, 4, 3000, 0, True),
])
def test_q8_decode_step_d256_vs_oracle(gpu, nq, nkv, pos, window, norms):
    """d = 256 Q8 caches (the vector-ALU kernel quantizes the new row)."""
    test_q8_decode_step_vs_oracle(gpu, 256, pos, window, norms, nq=nq, nkv=nkv)


def test_q8_rope_append_vs_oracle(gpu):
    """The unfused append kernel writes the oracle's bytes (v always, k at
    position 0) and rotates q as the oracle."""
    nq, nkv, d = 16, 4, 64
    st = Stream(13)
    for pos in (0, 777):
        q = st.normal((nq, d))
        k = st.normal((nkv, d))
        v = st.normal((nkv, d), 5.0)
        inv = oracle.rope_inv_freq(10000.0, d)
        R = oracle.q8_row_bytes(nkv, d)
        Kd = torch.zeros((pos + 1) * R, dtype=torch.uint8, device="cuda")
        Vd = torch.zeros_like(Kd)
        qd = dev(q)
        attn.rope_append(qd, dev(k), dev(v), Kd, Vd, nq, nkv, d, pos, pos, dev(inv))
        kr = oracle.rope_apply(k, pos, inv)
        Kr = np.zeros((1, R), np.uint8)
        Vr = np.zeros((1, R), np.uint8)
        oracle.q8_store_token(Kr, 0, kr, nkv, d)
        oracle.q8_store_token(Vr, 0, v, nkv, d)
        Kh = host_u8(Kd).reshape(pos + 1, R)
        Vh = host_u8(Vd).reshape(pos + 1, R)
        np.testing.assert_array_equal(Vh[pos], Vr[0])
        if pos == 0:
            np.testing.assert_array_equal(Kh[pos], Kr[0])
        else:
            assert_rows_close(Kh[pos], Kr[0], nkv, d)
        np.testing.assert_allclose(host(qd), oracle.rope_apply(q, pos, inv), rtol=2e-6,
                                   atol=4e-6)


def test_q8_quantizer_edge_rows(gpu):
    """Rows of zeros (scale 1, codes 0), a single spike, and values on the
    rounding midpoints, appended at position 0 (RoPE the identity)."""
    nq, nkv, d = 8, 4, 128
    k = np.zeros((nkv, d), np.float32)
    k[1, 5] = -3.0                                             # one spike: code -127
    k[2] = (np.arange(d, dtype=np.float32) - 64) * (1 / 127)   # steps of s/2 around codes
    k[3] = 1e-30                                               # tiny, not > 0 after /127? still > 0
    v = k[::-1].copy()
    q = np.ones((nq, d), np.float32)
    inv = oracle.rope_inv_freq(10000.0, d)
    R = oracle.q8_row_bytes(nkv, d)
    Kd = torch.zeros(R, dtype=torch.uint8, device="cuda")
    Vd = torch.zeros_like(Kd)
    O = torch.empty((nq, d), device="cuda")
    attn.decode_step(dev(q), dev(k), dev(v), Kd, Vd, O, nq, nkv, d, 0, 0, dev(inv), 0.1, 0)
    Kr = np.zeros((1, R), np.uint8)
    Vr = np.zeros((1, R), np.uint8)
    oracle.q8_store_token(Kr, 0, k, nkv, d)
    oracle.q8_store_token(Vr, 0, v, nkv, d)
    np.testing.assert_array_equal(host_u8(Kd), Kr[0])
    np.testing.assert_array_equal(host_u8(Vd), Vr[0])
    # one row: o is that row's dequantized v
    np.testing.assert_allclose(host(O), np.repeat(oracle.q8_dequant(Vr, nkv, d).reshape(
        nkv, d), nq // nkv, axis=0), rtol=1e-6, atol=1e-30)


# ---------------------------------------------------------------------------
# paged Q8

def q8_paged_problem(B, nq, nkv, d, lmin, lmax, seed, page=16):
    P = make_paged(B, nq, nkv, d, lmin, lmax, page=page, seed=seed, bf16=False)
    P["Kp"] = oracle.q8_pages(P["Kp"])
    P["Vp"] = oracle.q8_pages(P["Vp"])
    return P


def oracle_paged_q8(P, inv, scale, window=0, qn=None, kn=None, v_norm=False):
    """RoPE (and norms) of each sequence's new token, its quantized append
    into slot n-1, then paged attention on the oracle."""
    Kp, Vp = P["Kp"].copy(), P["Vp"].copy()
    B, nq, nkv, d, page = P["B"], P["nq"], P["nkv"], P["d"], P["page"]
    q = np.empty_like(P["q"])
    for b in range(B):
        n = int(P["n"][b])
        qb, kb, vb = P["q"][b], P["k_new"][b], P["v_new"][b]
        if qn is not None:
            qb = oracle.rmsnorm(qb, qn, 1e-6)
        if kn is not None:
            kb = oracle.rmsnorm(kb, kn, 1e-6)
        if v_norm:
            vb = oracle.rmsnorm(vb.reshape(-1), None, 1e-6).reshape(nkv, d)
        q[b] = oracle.rope_apply(qb, n - 1, inv)
        k = oracle.rope_apply(kb, n - 1, inv)
        blk = P["bt"][b, (n - 1) // page]
        oracle.q8_page_store(Kp, blk, (n - 1) % page, k, nkv, d, page)
        oracle.q8_page_store(Vp, blk, (n - 1) % page, vb, nkv, d, page)
    O = oracle.attn_decode_paged(q, Kp, Vp, P["bt"], P["n"], None, B, P["max_blocks"], nq, nkv,
                                 d, page, scale, window)
    return q, Kp, Vp, O


@pytest.mark.parametrize("d,window", [(128, 0), (64, 0), (128, 300), (256, 0), (256, 300)])
def test_q8_paged_attention_vs_oracle(gpu, d, window):
    announce(f"q8 paged attention d={d} window={window}")
    P = q8_paged_problem(11, 32, 8, d, 0, 2500, seed=20 + d + window)
    s = 1 / math.sqrt(d)
    O = torch.empty((P["B"], 32, d), device="cuda")
    attn.attn_decode_paged(dev(P["q"]), dev_u8(P["Kp"]), dev_u8(P["Vp"]), O,
                           dev(P["bt"].reshape(-1)), dev(P["n"]), None, P["B"], P["max_blocks"],
                           32, 8, d, 16, s, window)
    R = oracle.attn_decode_paged(P["q"], P["Kp"], P["Vp"], P["bt"], P["n"], None, P["B"],
                                 P["max_blocks"], 32, 8, d, 16, s, window)
    err = normwise_err(host(O), R)
    print(f"q8 paged normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("norms", [False, True])
def test_q8_paged_fused_step_vs_oracle(gpu, norms):
    announce(f"q8 paged fused step norms={norms}")
    P = q8_paged_problem(17, 32, 8, 128, 0, 2000, seed=31 + norms)
    inv = oracle.rope_inv_freq(500000.0, 128)
    s = 1 / math.sqrt(128)
    st = Stream(33)
    qn = (1 + st.normal((128,), 0.2)).astype(np.float32) if norms else None
    kn = (1 + st.normal((128,), 0.2)).astype(np.float32) if norms else None
    q, K, V = dev(P["q"]), dev_u8(P["Kp"]), dev_u8(P["Vp"])
    O = torch.empty((P["B"], 32, 128), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O,
                           dev(P["bt"].reshape(-1)), dev(P["n"]), None, P["B"], P["max_blocks"],
                           32, 8, 128, 16, dev(inv), s, 0,
                           q_norm=None if qn is None else dev(qn),
                           k_norm=None if kn is None else dev(kn), v_norm=norms, eps=1e-6)
    oq, oK, oV, oO = oracle_paged_q8(P, inv, s, 0, qn, kn, norms)
    np.testing.assert_allclose(host(q), oq, rtol=2e-6, atol=4e-6)
    Kh, Vh = host_u8(K).reshape(oK.shape), host_u8(V).reshape(oV.shape)
    if not norms:
        np.testing.assert_array_equal(Vh, oV)
    R = oracle.attn_decode_paged(host(q), Kh, Vh, P["bt"], P["n"], None, P["B"],
                                 P["max_blocks"], 32, 8, 128, 16, s, 0)
    err = normwise_err(host(O), R)
    print(f"q8 paged step normwise err {err:.3e}", flush=True)
    assert err < TOL
    assert normwise_err(host(O), oO) < 1e-3


def test_q8_paged_explicit_positions(gpu):
    """pos[] given: the unfused append kernel, then paged attention."""
    P = q8_paged_problem(9, 16, 4, 64, 10, 900, seed=41)
    inv = oracle.rope_inv_freq(10000.0, 64)
    pos = (P["n"] - 1).astype(np.int32)  # the default positions, passed explicitly
    q, K, V = dev(P["q"]), dev_u8(P["Kp"]), dev_u8(P["Vp"])
    O = torch.empty((P["B"], 16, 64), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O,
                           dev(P["bt"].reshape(-1)), dev(P["n"]), dev(pos), P["B"],
                           P["max_blocks"], 16, 4, 64, 16, dev(inv), 0.125, 0)
    oq, oK, oV, oO = oracle_paged_q8(P, inv, 0.125)
    np.testing.assert_array_equal(host_u8(V).reshape(oV.shape), oV)
    Kh, Vh = host_u8(K).reshape(oK.shape), host_u8(V).reshape(oV.shape)
    R = oracle.attn_decode_paged(host(q), Kh, Vh, P["bt"], P["n"], None, P["B"],
                                 P["max_blocks"], 16, 4, 64, 16, 0.125, 0)
    assert normwise_err(host(O), R) < TOL


def test_q8_paged_matches_contiguous(gpu):
    """The same logical Q8 cache through a shuffled block table or token-major."""
    st = Stream(42)
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
    attn.attn_decode_gqa_cache(dev(Q), dev_u8(oracle.q8_cache(K, nkv, d)),
                               dev_u8(oracle.q8_cache(V, nkv, d)), O1, nq, nkv, n, d, 0.088,
                               n - 1, 0)
    attn.attn_decode_paged(dev(Q), dev_u8(oracle.q8_pages(Kp)), dev_u8(oracle.q8_pages(Vp)), O2,
                           dev(perm), dev(np.array([n], np.int32)), None, 1, nblk, nq, nkv, d,
                           page, 0.088)
    assert normwise_err(host(O2)[0], host(O1)) < 2e-6


def test_q8_c4_continuous_batching(gpu):
    """The c4 batch (64 sequences, U[512, 8192) tokens, shuffled 16-token
    pages) on a Q8 pool, fused step."""
    announce("q8 c4 64 seqs U[512,8192] paged16")
    P = q8_paged_problem(64, 32, 8, 128, 512, 8192, seed=1234)
    inv = oracle.rope_inv_freq(500000.0, 128)
    s = 1 / math.sqrt(128)
    q, K, V = dev(P["q"]), dev_u8(P["Kp"]), dev_u8(P["Vp"])
    O = torch.empty((P["B"], 32, 128), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O,
                           dev(P["bt"].reshape(-1)), dev(P["n"]), None, P["B"], P["max_blocks"],
                           32, 8, 128, 16, dev(inv), s, 0)
    oq, oK, oV, oO = oracle_paged_q8(P, inv, s)
    np.testing.assert_array_equal(host_u8(V).reshape(oV.shape), oV)
    Kh = host_u8(K).reshape(oK.shape)
    R = oracle.attn_decode_paged(host(q), Kh, oV, P["bt"], P["n"], None, P["B"], P["max_blocks"],
                                 32, 8, 128, 16, s, 0)
    err = normwise_err(host(O), R)
    print(f"q8 c4 normwise err {err:.3e}", flush=True)
    assert err < TOL


# ---------------------------------------------------------------------------
# prefill over a Q8 cache

@pytest.mark.parametrize("nq,nkv,d,M,N,pos0,window", [
    (32, 8, 128, 100, 100, 0, 0),
    (32, 8, 128, 77, 1077, 1000, 0),
    (8, 2, 64, 50, 3050, 3000, 1024),
    (16, 16, 64, 65, 65, 0, 0),      # G = 1
    (12, 4, 128, 30, 60, 30, 7),     # G = 3
    (8, 4, 256, 70, 3070, 3000, 1024),  # d = 256 (pieces only), window, split keys
    (8, 4, 256, 100, 100, 0, 0),
    (8, 4, 256, 4, 10, 40, 5),       # no query attends a key: O = 0
])
def test_q8_prefill_vs_oracle(gpu, nq, nkv, d, M, N, pos0, window):
    announce(f"q8 prefill {nq}/{nkv}/{d} M={M} N={N} pos0={pos0} win={window}")
    st = Stream(M + N + d)
    Q = st.normal((M, nq, d))
    Kq, Vq = q8_caches(st, N, nkv, d)
    O = torch.empty((M, nq, d), device="cuda")
    s = 1 / math.sqrt(d)
    attn.attn_prefill_gqa(dev(Q), dev_u8(Kq), dev_u8(Vq), O, nq, nkv, M, N, d, s, pos0, window)
    R = oracle.attn_prefill(Q, Kq, Vq, nq, nkv, M, N, d, s, pos0, window)
    err = normwise_err(host(O), R)
    print(f"q8 prefill normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("nq,nkv,d,M,n0", [(32, 8, 128, 200, 300), (8, 4, 256, 90, 150)])
def test_q8_prefill_step_vs_oracle(gpu, nq, nkv, d, M, n0):
    """One layer's prefill with norms on a Q8 cache: M tokens after n0."""
    announce(f"q8 prefill step {nq}q/{nkv}kv/d{d} M={M} after {n0}")
    st = Stream(50 + d)
    q = st.normal((M, nq, d), 2.0)
    k = st.normal((M, nkv, d), 2.0)
    v = st.normal((M, nkv, d), 2.0)
    qn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    kn = (1 + st.normal((d,), 0.2)).astype(np.float32)
    Kq, Vq = q8_caches(st, n0 + M, nkv, d)
    Kq[n0:] = 0
    Vq[n0:] = 0
    inv = oracle.rope_inv_freq(500000.0, d)
    qd, Kd, Vd = dev(q), dev_u8(Kq), dev_u8(Vq)
    O = torch.empty((M, nq, d), device="cuda")
    attn.prefill_step(qd, dev(k), dev(v), Kd, Vd, O, nq, nkv, d, M, n0, n0, dev(inv), 0.088, 0,
                      q_norm=dev(qn), k_norm=dev(kn), v_norm=True, eps=1e-6)
    Kc, Vc = Kq.copy(), Vq.copy()
    oq, oO = oracle.prefill_step(q, k, v, Kc, Vc, nq, nkv, d, M, n0, n0, qn, kn, 1, 1e-6, inv,
                                 0.088, 0)
    np.testing.assert_allclose(host(qd), oq, rtol=2e-6, atol=4e-6)
    Kh = host_u8(Kd).reshape(Kq.shape)
    Vh = host_u8(Vd).reshape(Vq.shape)
    np.testing.assert_array_equal(Kh[:n0], Kq[:n0])
    for t in range(n0, n0 + M):
        assert_rows_close(Kh[t], Kc[t], nkv, d)
        assert_rows_close(Vh[t], Vc[t], nkv, d)
    R = oracle.attn_prefill(host(qd), Kh, Vh, nq, nkv, M, n0 + M, d, 0.088, n0, 0)
    assert normwise_err(host(O), R) < TOL
    assert normwise_err(host(O), oO) < 1e-3


def test_q8_prefill_d256_paged_matches_contiguous(gpu):
    """A Q8 cache at d = 256 in shuffled 16-row pages: the same rows as the
    contiguous cache, the same pieces and products, the same bits."""
    announce("q8 prefill paged d256")
    st = Stream(58)
    nq, nkv, d, M, n0, page, spare = 8, 4, 256, 50, 400, 16, 3
    N = n0 + M
    Q = st.normal((M, nq, d))
    Kq, Vq = q8_caches(st, N, nkv, d)
    nb = (N + page - 1) // page
    nblk = nb + spare
    row = st.permutation(nblk)[:nb].astype(np.int32)
    rb = oracle.q8_block_bytes(nkv, d, page)
    pools = []
    for C in (Kq, Vq):
        codes = np.zeros((nblk, nkv, page, d), np.int8)
        scales = np.zeros((nblk, nkv, page), np.float32)
        for t in range(N):
            c, sc = split_row(C[t], nkv, d)
            codes[row[t // page], :, t % page] = c
            scales[row[t // page], :, t % page] = sc
        X = np.zeros((nblk, rb), np.uint8)
        X[:, :nkv * page * d] = codes.reshape(nblk, -1).view(np.uint8)
        X[:, nkv * page * d:nkv * page * d + 4 * nkv * page] = scales.reshape(nblk, -1).view(np.uint8)
        pools.append(X)
    s = 1 / math.sqrt(d)
    Oc = torch.full((M, nq, d), float("nan"), device="cuda")
    Op = torch.full((M, nq, d), float("nan"), device="cuda")
    attn.attn_prefill_gqa(dev(Q), dev_u8(Kq), dev_u8(Vq), Oc, nq, nkv, M, N, d, s, n0, 0)
    attn.attn_prefill_paged(dev(Q), dev_u8(pools[0]), dev_u8(pools[1]), Op,
                            torch.from_numpy(row).cuda(), nb, page, nq, nkv, M, N, d, s, n0, 0)
    assert torch.equal(Oc, Op)
    R = oracle.attn_prefill(Q, Kq, Vq, nq, nkv, M, N, d, s, n0, 0)
    assert normwise_err(host(Oc), R) < TOL


def test_q8_d256_prefill_without_pieces_in_a_graph(gpu):
    """A Q8 prefill at d = 256 reads its keys as bf16 pieces split once per
    launch (its matrix-core kernel has no per-tile split).  Captured on a
    stream whose pieces workspace is too small (it cannot grow under
    capture), it runs on the vector-ALU kernel instead, each query row a
    sequence of its own; every replay equals the oracle, and the eager
    pieces path, to the 1e-5 bar."""
    announce("q8 d256 prefill captured without its pieces")
    nq, nkv, d, M, N, pos0 = 8, 4, 256, 40, 3040, 3000
    st = Stream(66)
    Q = st.normal((M, nq, d))
    Kq, Vq = q8_caches(st, N, nkv, d)
    Qd, Kd, Vd = dev(Q), dev_u8(Kq), dev_u8(Vq)
    s = 1 / math.sqrt(d)
    O = torch.empty((M, nq, d), device="cuda")
    attn.attn_prefill_gqa(Qd, Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)  # pieces, eager
    eager = host(O)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # sizes the side stream's workspaces for a shorter cache
        attn.attn_prefill_gqa(Qd, Kd, Vd, O, nq, nkv, M, 1040, d, s, 1000, 0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        attn.attn_prefill_gqa(Qd, Kd, Vd, O, nq, nkv, M, N, d, s, pos0, 0)
    R = oracle.attn_prefill(Q, Kq, Vq, nq, nkv, M, N, d, s, pos0, 0)
    for r in range(3):
        O.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = host(O)
        assert normwise_err(got, R) < TOL, f"replay {r}"
        assert normwise_err(got, eager) < TOL, f"replay {r}"
    assert normwise_err(eager, R) < TOL


# ---------------------------------------------------------------------------
# Q8 caches at head dims other than 64, 128, 256 and 512: the vector-ALU
# kernel for the next of them, each row read at its d codes in 4-code pieces

@pytest.mark.parametrize("nq,nkv,d,n,window", [
    (16, 4, 48, 900, 0),       # D = 64
    (32, 8, 96, 3000, 0),      # D = 128
    (16, 2, 100, 2000, 300),   # d % 8 == 4, window
    (8, 4, 200, 1500, 0),      # D = 256
    (8, 2, 300, 2500, 0),      # D = 512
    (8, 8, 500, 40, 0),        # one chunk
    (12, 3, 36, 1000, 0),      # 124-byte token rows: off 16-byte boundaries
])
def test_q8_padded_decode_vs_oracle(gpu, nq, nkv, d, n, window):
    announce(f"q8 padded decode {nq}/{nkv}/{d} n={n} window={window}")
    st = Stream(n + d + 17)
    Q = st.normal((nq, d))
    Kq, Vq = q8_caches(st, n, nkv, d)
    O = torch.empty((nq, d), device="cuda")
    s = 1 / math.sqrt(d)
    attn.attn_decode_gqa_cache(dev(Q), dev_u8(Kq), dev_u8(Vq), O, nq, nkv, n, d, s, n - 1, window)
    R = oracle.attn_decode_gqa_cache(Q, Kq, Vq, nq, nkv, n, d, s, n - 1, window)
    err = normwise_err(host(O), R)
    print(f"q8 padded normwise err {err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("d,pos,norms,nkv", [(96, 0, False, 4), (96, 2000, True, 4),
                                              (300, 1200, False, 4), (36, 700, True, 4),
                                              (20, 900, False, 3)])
def test_q8_padded_decode_step_vs_oracle(gpu, d, pos, norms, nkv):
    """The fused step at a padded head dim: the kernel quantizes the new
    rows over their d values (bit-exact bytes at position 0) and stores d
    codes a head, never the padding.  nkv = 3, d = 20: 60 codes and 16 scale
    bytes, so token rows start off 16-byte boundaries."""
    test_q8_decode_step_vs_oracle(gpu, d, pos, 0, norms, nq=4 * nkv, nkv=nkv)


def test_q8_padded_paged_and_prefill(gpu):
    """Paged Q8 pages and the prefill (query rows on the vector-ALU kernel)
    at d = 100, against the oracle on the same bytes."""
    nq, nkv, d, page = 8, 4, 100, 16
    announce("q8 padded paged decode d=100")
    P = q8_paged_problem(5, nq, nkv, d, 50, 900, seed=77)
    inv = oracle.rope_inv_freq(10000.0, d)
    s = 1 / math.sqrt(d)
    B = P["B"]
    q, K, V = dev(P["q"]), dev_u8(P["Kp"]), dev_u8(P["Vp"])
    O = torch.empty((B, nq, d), device="cuda")
    attn.decode_step_paged(q, dev(P["k_new"]), dev(P["v_new"]), K, V, O,
                           dev(P["bt"].reshape(-1)), dev(P["n"]), None, B, P["max_blocks"], nq,
                           nkv, d, page, dev(inv), s, 0)
    oq, oK, oV, oO = oracle_paged_q8(P, inv, s)
    np.testing.assert_allclose(host(q), oq, rtol=2e-6, atol=4e-6)
    Kh, Vh = host_u8(K).reshape(oK.shape), host_u8(V).reshape(oV.shape)
    np.testing.assert_array_equal(Vh, oV)  # v's codes and scales, and no byte past d
    R = oracle.attn_decode_paged(host(q), Kh, Vh, P["bt"], P["n"], None, B, P["max_blocks"], nq,
                                 nkv, d, page, s, 0)
    assert normwise_err(host(O), R) < TOL
    assert normwise_err(host(O), oO) < 1e-3  # appended k may differ by a code (see above)
    announce("q8 padded prefill d=100")
    st = Stream(78)
    M, N, pos0 = 30, 430, 400
    Qm = st.normal((M, nq, d))
    Kq, Vq = q8_caches(st, N, nkv, d)
    Om = torch.full((M, nq, d), float("nan"), device="cuda")
    attn.attn_prefill_gqa(dev(Qm), dev_u8(Kq), dev_u8(Vq), Om, nq, nkv, M, N, d, s, pos0, 64)
    R = oracle.attn_prefill(Qm, Kq, Vq, nq, nkv, M, N, d, s, pos0, 64)
    assert normwise_err(host(Om), R) < TOL


# ---------------------------------------------------------------------------
# shapes the Q8 paths do not take: errors through the ABI, never a launch

def test_q8_errors(gpu):
    st = Stream(60)
    Q = dev(st.normal((8, 90)))
    O = torch.empty((8, 90), device="cuda")
    C = torch.zeros(10 * oracle.q8_row_bytes(2, 90), dtype=torch.uint8, device="cuda")
    with pytest.raises(MolotHipError) as e:  # Q8 caches: multiples of 4 only
        attn.attn_decode_gqa_cache(Q, C, C, O, 8, 2, 10, 90, 0.1, 9, 0)
    assert e.value.status == ENOTSUP
    Q = dev(st.normal((8, 64)))
    O = torch.empty((8, 64), device="cuda")
    C = torch.zeros(10 * oracle.q8_row_bytes(2, 64), dtype=torch.uint8, device="cuda")
    with pytest.raises(MolotHipError) as e:  # head-major layout: not a Q8 layout
        attn.attn_decode_gqa(Q, C, C, O, 8, 2, 10, 64, 0.1)
    assert e.value.status == EINVAL
    # paged Q8 blocks must stay 16-byte aligned: nkv * page a multiple of 4
    Qp = dev(st.normal((1, 8, 64)))
    Op = torch.empty((1, 8, 64), device="cuda")
    pool = torch.zeros(4 * oracle.q8_block_bytes(1, 64, 2), dtype=torch.uint8, device="cuda")
    with pytest.raises(MolotHipError) as e:
        attn.attn_decode_paged(Qp, pool, pool, Op, dev(np.array([0, 1], np.int32)),
                               dev(np.array([3], np.int32)), None, 1, 2, 8, 1, 64, 2, 0.1)
    assert e.value.status == EINVAL
