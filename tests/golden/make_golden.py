"""Write the golden fixtures under tests/golden/ from the reference itself.

Runs in the build container only, where the reference tree is present: the
expected outputs come from the reference's own header-only C++ (compiled
where it lies by oracle/Makefile into oracle/_ref/libmolot_ref.so), called
through oracle.ref().  Each fixture stores its inputs and the reference's
outputs as plain arrays (np.savez, no pickles), so tests need neither the
reference nor the generator to reproduce them.

Usage:  make -C oracle && python tests/golden/make_golden.py [fixture ...]
        (no names: write every fixture)
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from molot_amd.synth import Stream  # noqa: E402

P = oracle._p


def _save(name: str, **arrays) -> None:
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **{k: np.asarray(v) for k, v in arrays.items()})
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def ref_inv_freq(base, d):
    out = np.empty(d // 2, np.float32)
    oracle.ref().ref_rope_inv_freq(float(base), d, P(out))
    return out


def gen_decode_step(name, nq, nkv, d, n0, base, window, scale, seed, pool):
    """forward.h:556-591 through the reference: rope q/k, append, attention."""
    R = oracle.ref()
    st = Stream(seed)
    q = st.normal((nq, d))
    k = st.normal((nkv, d))
    v = st.normal((nkv, d))
    cap = n0 + 1
    Kc = np.zeros((cap, nkv * d), np.float32)
    Vc = np.zeros((cap, nkv * d), np.float32)
    Kc[:n0] = st.normal((n0, nkv * d))
    Vc[:n0] = st.normal((n0, nkv * d))
    inv = ref_inv_freq(base, d)
    q_rot, k_rot = q.copy(), k.copy()
    Kout, Vout = Kc.copy(), Vc.copy()
    O = np.empty((nq, d), np.float32)
    rc = R.ref_decode_step(P(q_rot), P(k_rot), P(v), P(Kout), P(Vout), P(O), nq, nkv, d, n0, cap,
                           n0, P(inv), float(scale), int(window), pool.h)
    assert rc == 0
    _save(name, q=q, k_new=k, v_new=v, K=Kc[:n0], V=Vc[:n0], inv_freq=inv, q_rot=q_rot,
          k_rot=k_rot, O=O, nq=nq, nkv=nkv, d=d, pos=n0, base=base, window=window, scale=scale,
          seed=seed)


def gen_decode_step_norm(name, nq, nkv, d, n0, base, window, scale, eps, v_norm, seed, pool):
    """forward.h:554-591 with the layer's norms, through the reference:
    rmsnorm of q and k heads (weights), rmsnorm_plain of v, rope, append,
    attention.  Weights are drawn around 1 like trained norm gains."""
    R = oracle.ref()
    st = Stream(seed)
    q = st.normal((nq, d), 3.0)
    k = st.normal((nkv, d), 3.0)
    v = st.normal((nkv, d), 3.0)
    q_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    k_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    cap = n0 + 1
    Kc = np.zeros((cap, nkv * d), np.float32)
    Vc = np.zeros((cap, nkv * d), np.float32)
    Kc[:n0] = st.normal((n0, nkv * d))
    Vc[:n0] = st.normal((n0, nkv * d))
    inv = ref_inv_freq(base, d)
    q_rot, k_rot, v_out = q.copy(), k.copy(), v.copy()
    Kout, Vout = Kc.copy(), Vc.copy()
    O = np.empty((nq, d), np.float32)
    rc = R.ref_decode_step_norm(P(q_rot), P(k_rot), P(v_out), P(Kout), P(Vout), P(O), nq, nkv, d,
                                n0, cap, n0, P(q_norm), P(k_norm), int(v_norm), float(eps), P(inv),
                                float(scale), int(window), pool.h)
    assert rc == 0
    _save(name, q=q, k_new=k, v_new=v, K=Kc[:n0], V=Vc[:n0], inv_freq=inv, q_norm=q_norm,
          k_norm=k_norm, q_rot=q_rot, k_rot=k_rot, v_normed=v_out, O=O, nq=nq, nkv=nkv, d=d,
          pos=n0, base=base, window=window, scale=scale, eps=eps, v_norm=v_norm, seed=seed)


def gen_rmsnorm(name, sizes, seed):
    """rmsnorm / rmsnorm_plain (norm.h:9-28, :82-96) on rows of several
    lengths (vector body and scalar tail) and magnitudes where eps matters."""
    R = oracle.ref()
    st = Stream(seed)
    out = {}
    for n in sizes:
        for tag, sig in (("unit", 1.0), ("tiny", 1e-3)):
            x = st.normal((n,), sig)
            w = (1.0 + st.normal((n,), 0.3)).astype(np.float32)
            y = np.empty(n, np.float32)
            yp = np.empty(n, np.float32)
            R.ref_rmsnorm(P(x), P(w), P(y), n, 1e-6)
            R.ref_rmsnorm_plain(P(x), P(yp), n, 1e-6)
            out[f"x_{tag}_{n}"], out[f"w_{tag}_{n}"] = x, w
            out[f"y_{tag}_{n}"], out[f"yplain_{tag}_{n}"] = y, yp
    _save(name, sizes=np.array(sizes), eps=1e-6, seed=seed, **out)


def gen_prefill(name, nq, nkv, d, M, n0, base, window, scale, eps, norms, seed, pool):
    """forward.h:367-399 for one layer through the reference: per-token norms
    (when `norms`) and RoPE, append of M rows after n0 cached ones, then
    attn_prefill_gqa (gemm.h:409-446) over N = n0 + M at pos0 = n0."""
    R = oracle.ref()
    st = Stream(seed)
    q = st.normal((M, nq, d), 2.0)
    k = st.normal((M, nkv, d), 2.0)
    v = st.normal((M, nkv, d), 2.0)
    q_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    k_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    cap = n0 + M
    Kc = np.zeros((cap, nkv * d), np.float32)
    Vc = np.zeros((cap, nkv * d), np.float32)
    Kc[:n0] = st.normal((n0, nkv * d))
    Vc[:n0] = st.normal((n0, nkv * d))
    inv = ref_inv_freq(base, d)
    q_rot, k_rot, v_out = q.copy(), k.copy(), v.copy()
    Kout, Vout = Kc.copy(), Vc.copy()
    O = np.empty((M, nq, d), np.float32)
    rc = R.ref_prefill_step(P(q_rot), P(k_rot), P(v_out), P(Kout), P(Vout), P(O), nq, nkv, d, M,
                            n0, cap, n0, P(q_norm) if norms else None,
                            P(k_norm) if norms else None, int(norms), float(eps), P(inv),
                            float(scale), int(window), pool.h)
    assert rc == 0
    _save(name, q=q, k_new=k, v_new=v, K=Kc[:n0], V=Vc[:n0], inv_freq=inv, q_norm=q_norm,
          k_norm=k_norm, norms=int(norms), q_rot=q_rot, K_after=Kout[n0:], V_after=Vout[n0:],
          O=O, nq=nq, nkv=nkv, d=d, M=M, pos0=n0, base=base, window=window, scale=scale, eps=eps,
          seed=seed)


def gen_decode_step_nope(name, nq, nkv, d, n0, window, scale, eps, seed, pool):
    """forward.h:554-591 for a layer without RoPE (an empty L.freq:
    rope_swa_only models' global layers, model.h:535-536), through the
    reference with the norms: q/k rmsnorm, v rmsnorm_plain, no rope_apply
    (forward.h:556, :566 skip it), append, attention."""
    R = oracle.ref()
    st = Stream(seed)
    q = st.normal((nq, d), 2.0)
    k = st.normal((nkv, d), 2.0)
    v = st.normal((nkv, d), 2.0)
    q_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    k_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    cap = n0 + 1
    Kc = np.zeros((cap, nkv * d), np.float32)
    Vc = np.zeros((cap, nkv * d), np.float32)
    Kc[:n0] = st.normal((n0, nkv * d))
    Vc[:n0] = st.normal((n0, nkv * d))
    q_out, k_out, v_out = q.copy(), k.copy(), v.copy()
    Kout, Vout = Kc.copy(), Vc.copy()
    O = np.empty((nq, d), np.float32)
    rc = R.ref_decode_step_norm(P(q_out), P(k_out), P(v_out), P(Kout), P(Vout), P(O), nq, nkv,
                                d, n0, cap, n0, P(q_norm), P(k_norm), 1, float(eps), None,
                                float(scale), int(window), pool.h)
    assert rc == 0
    _save(name, q=q, k_new=k, v_new=v, K=Kc[:n0], V=Vc[:n0], q_norm=q_norm, k_norm=k_norm,
          q_out=q_out, k_out=k_out, v_normed=v_out, O=O, nq=nq, nkv=nkv, d=d, pos=n0,
          window=window, scale=scale, eps=eps, seed=seed)


def gen_decode_step_shared(name, nq, nkv, d, n, pos, base, window, scale, eps, rope, seed,
                           pool):
    """forward.h:554-558, 578-591 for a layer reading another layer's cache
    (L.has_kv false) through the reference: q rmsnorm, rope_apply when the
    layer has a table, attn_decode_gqa_cache over the source's n slots."""
    R = oracle.ref()
    st = Stream(seed)
    q = st.normal((nq, d), 2.0)
    q_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    Kc = st.normal((n, nkv * d))
    Vc = st.normal((n, nkv * d))
    inv = ref_inv_freq(base, d) if rope else None
    q_out = q.copy()
    O = np.empty((nq, d), np.float32)
    rc = R.ref_decode_step_shared(P(q_out), P(Kc), P(Vc), P(O), nq, nkv, d, n, pos, P(q_norm),
                                  float(eps), P(inv) if rope else None, float(scale),
                                  int(window), pool.h)
    assert rc == 0
    extra = {"inv_freq": inv} if rope else {}
    _save(name, q=q, K=Kc, V=Vc, q_norm=q_norm, q_out=q_out, O=O, nq=nq, nkv=nkv, d=d, n=n,
          pos=pos, window=window, scale=scale, eps=eps, rope=int(rope), seed=seed, **extra)


def gen_prefill_nope(name, nq, nkv, d, M, n0, window, scale, eps, seed, pool):
    """forward.h:367-399 for a layer without RoPE through the reference:
    per-token norms, no rotation (forward.h:373, :381), append, causal
    attention."""
    R = oracle.ref()
    st = Stream(seed)
    q = st.normal((M, nq, d), 2.0)
    k = st.normal((M, nkv, d), 2.0)
    v = st.normal((M, nkv, d), 2.0)
    q_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    k_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    cap = n0 + M
    Kc = np.zeros((cap, nkv * d), np.float32)
    Vc = np.zeros((cap, nkv * d), np.float32)
    Kc[:n0] = st.normal((n0, nkv * d))
    Vc[:n0] = st.normal((n0, nkv * d))
    q_out, k_out, v_out = q.copy(), k.copy(), v.copy()
    Kout, Vout = Kc.copy(), Vc.copy()
    O = np.empty((M, nq, d), np.float32)
    rc = R.ref_prefill_step(P(q_out), P(k_out), P(v_out), P(Kout), P(Vout), P(O), nq, nkv, d, M,
                            n0, cap, n0, P(q_norm), P(k_norm), 1, float(eps), None, float(scale),
                            int(window), pool.h)
    assert rc == 0
    _save(name, q=q, k_new=k, v_new=v, K=Kc[:n0], V=Vc[:n0], q_norm=q_norm, k_norm=k_norm,
          q_out=q_out, K_after=Kout[n0:], V_after=Vout[n0:], O=O, nq=nq, nkv=nkv, d=d, M=M,
          pos0=n0, window=window, scale=scale, eps=eps, seed=seed)


def gen_prefill_shared(name, nq, nkv, d, M, N, pos0, base, window, scale, eps, seed, pool):
    """forward.h:367-399 for a layer without its own KV through the
    reference: per-token q rmsnorm and rope_apply, no append, then
    attn_prefill_gqa over the source cache's N slots at pos0."""
    R = oracle.ref()
    st = Stream(seed)
    q = st.normal((M, nq, d), 2.0)
    q_norm = (1.0 + st.normal((d,), 0.2)).astype(np.float32)
    Kc = st.normal((N, nkv * d))
    Vc = st.normal((N, nkv * d))
    inv = ref_inv_freq(base, d)
    q_out = q.copy()
    O = np.empty((M, nq, d), np.float32)
    R.ref_prefill_shared(P(q_out), P(Kc), P(Vc), P(O), nq, nkv, d, M, N, pos0, P(q_norm),
                         float(eps), P(inv), float(scale), int(window), pool.h)
    _save(name, q=q, K=Kc, V=Vc, q_norm=q_norm, inv_freq=inv, q_out=q_out, O=O, nq=nq, nkv=nkv,
          d=d, M=M, N=N, pos0=pos0, window=window, scale=scale, eps=eps, seed=seed)


def gen_q8_rows(name, d, seed):
    """quantize_q8_row (quant.h:34-50) through the reference on rows that
    probe its edges: Gaussian rows of two scales, an all-zero row (scale 1),
    rows of exact half-steps (ties of nearbyint), tiny values, and a row
    whose absmax element sits at +-127 exactly."""
    R = oracle.ref()
    st = Stream(seed)
    rows = [st.normal((d,), 1.0), st.normal((d,), 3.0), np.zeros(d, np.float32)]
    s = np.float32(0.5)
    ties = (np.arange(d, dtype=np.float32) - d / 2 + np.float32(0.5)) * s
    ties[0] = np.float32(127.0) * s  # fixes the scale at 0.5: every x/s is k + 0.5
    rows += [ties, -ties, st.normal((d,), 1e-30), st.normal((d,), 1e-3)]
    X = np.stack([r.astype(np.float32) for r in rows])
    S = np.empty(len(rows), np.float32)
    Q = np.empty((len(rows), d), np.int8)
    for i in range(len(rows)):
        R.ref_quantize_q8_row(P(X[i]), d, P(S[i:i + 1]), P(Q[i]))
    _save(name, X=X, S=S, Q=Q, d=d, seed=seed)


def gen_head(name, n, d, sigma, seed):
    """attn_decode_head (attn.h:104-107), the bench/bench.cc:186-218 check shape."""
    R = oracle.ref()
    st = Stream(seed)
    Q = st.normal((d,), sigma)
    K = st.normal((n, d), sigma)
    V = st.normal((n, d), sigma)
    O = np.empty(d, np.float32)
    scale = 1.0 / math.sqrt(d)
    R.ref_attn_decode_head(P(Q), P(K), P(V), P(O), n, d, scale)
    _save(name, Q=Q, K=K, V=V, O=O, n=n, d=d, scale=scale, sigma=sigma, seed=seed)


def gen_gqa_headmajor(name, nq, nkv, n, d, pos_cur, window, seed, pool):
    """attn_decode_gqa (window 0) / attn_decode_gqa_win over [nkv][n][d]."""
    R = oracle.ref()
    st = Stream(seed)
    Q = st.normal((nq, d))
    K = st.normal((nkv, n, d))
    V = st.normal((nkv, n, d))
    O = np.empty((nq, d), np.float32)
    scale = 1.0 / math.sqrt(d)
    if window > 0:
        R.ref_attn_decode_gqa_win(P(Q), P(K), P(V), P(O), nq, nkv, n, d, scale, pos_cur, window,
                                  pool.h)
    else:
        R.ref_attn_decode_gqa(P(Q), P(K), P(V), P(O), nq, nkv, n, d, scale, pool.h)
    _save(name, Q=Q, K=K, V=V, O=O, nq=nq, nkv=nkv, n=n, d=d, scale=scale, pos_cur=pos_cur,
          window=window, seed=seed)


def gen_bf16_cache(name, nq, nkv, n, d, sigma, seed, pool):
    """bf16 KV: values rounded with the reference's fp32_to_bf16 (quant.h:192-198),
    attention by the reference over the widened values (the reference has no
    bf16 attention; this pins rounding + widening + the fp32 math)."""
    R = oracle.ref()
    st = Stream(seed)
    Q = st.normal((nq, d))
    Kf = st.normal((n, nkv * d), sigma)
    Vf = st.normal((n, nkv * d), sigma)
    to_bf = np.vectorize(lambda x: R.ref_fp32_to_bf16(float(x)), otypes=[np.uint16])
    Kb = to_bf(Kf)
    Vb = to_bf(Vf)
    widen = np.vectorize(lambda b: R.ref_bf16_to_fp32(int(b)), otypes=[np.float32])
    Kw = widen(Kb)
    Vw = widen(Vb)
    O = np.empty((nq, d), np.float32)
    scale = 1.0 / math.sqrt(d)
    R.ref_attn_decode_gqa_cache(P(Q), P(Kw), P(Vw), P(O), nq, nkv, n, d, scale, n - 1, 0, pool.h)
    _save(name, Q=Q, K_f32=Kf, V_f32=Vf, K_bf16=Kb, V_bf16=Vb, O=O, nq=nq, nkv=nkv, n=n, d=d,
          scale=scale, sigma=sigma, seed=seed)


def gen_rope(name, d, base, positions, seed):
    R = oracle.ref()
    st = Stream(seed)
    inv = ref_inv_freq(base, d)
    X = st.normal((len(positions), 4, d))
    Y = X.copy()
    for i, p in enumerate(positions):
        for h in range(4):
            row = np.ascontiguousarray(Y[i, h])
            R.ref_rope_apply(P(row), d, int(p), P(inv))
            Y[i, h] = row
    _save(name, X=X, Y=Y, inv_freq=inv, positions=np.asarray(positions, np.int32), d=d, base=base,
          seed=seed)


def gen_vexp(name, seed):
    R = oracle.ref()
    kat = np.array([-87., -20., -10., -5., -3., -2., -1.5, -1., -0.75, -0.5, -0.25, -0.1, -0.01,
                    0., 1., 50.], np.float32)  # bench/bench.cc:222-223
    st = Stream(seed)
    u = (st.words(48) >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    rnd = (-88.0 * u).astype(np.float32)
    X = np.concatenate([kat, rnd, np.array([-100., -88.5, 88., 89., 100., -1e-6, 1e-6, 10., 20.,
                                            -30., -60., -80., 0.5, 2., 5., 40.], np.float32)])
    Y = np.empty_like(X)
    for i in range(0, X.size, 16):
        R.ref_exp16(P(X[i:i + 16]), P(Y[i:i + 16]))
    _save(name, X=X, Y=Y, seed=seed)


def main() -> None:
    if not oracle.ref_available():
        sys.exit("reference library not available: build it with `make -C oracle` here")
    only = set(sys.argv[1:])  # fixture names to (re)write; all when empty

    def want(name):
        return not only or name in only

    with oracle.RefPool(4) as pool:
        if want("decode_step_g4_d128"):
            gen_decode_step("decode_step_g4_d128", nq=8, nkv=2, d=128, n0=100, base=500000.0,
                            window=0, scale=1.0 / math.sqrt(128), seed=11, pool=pool)
        if want("decode_step_win_d256"):
            gen_decode_step("decode_step_win_d256", nq=4, nkv=2, d=256, n0=60, base=10000.0,
                            window=16, scale=1.0 / math.sqrt(256), seed=12, pool=pool)
        if want("decode_step_g8_d64_scale1"):
            gen_decode_step("decode_step_g8_d64_scale1", nq=8, nkv=1, d=64, n0=150,
                            base=500000.0, window=0, scale=1.0, seed=13, pool=pool)
        if want("decode_step_norm_g4_d128"):
            gen_decode_step_norm("decode_step_norm_g4_d128", nq=8, nkv=2, d=128, n0=90,
                                 base=500000.0, window=0, scale=1.0, eps=1e-6, v_norm=1,
                                 seed=20, pool=pool)
        if want("decode_step_norm_win_d256"):
            gen_decode_step_norm("decode_step_norm_win_d256", nq=4, nkv=2, d=256, n0=60,
                                 base=10000.0, window=16, scale=1.0, eps=1e-6, v_norm=0,
                                 seed=21, pool=pool)
        if want("prefill_g4_d64"):
            gen_prefill("prefill_g4_d64", nq=4, nkv=1, d=64, M=21, n0=30, base=500000.0,
                        window=0, scale=1.0 / math.sqrt(64), eps=1e-6, norms=False, seed=23,
                        pool=pool)
        if want("prefill_norm_win_d128"):
            gen_prefill("prefill_norm_win_d128", nq=4, nkv=2, d=128, M=12, n0=20, base=10000.0,
                        window=8, scale=1.0, eps=1e-6, norms=True, seed=24, pool=pool)
        if want("decode_step_nope_g4_d128"):
            gen_decode_step_nope("decode_step_nope_g4_d128", nq=8, nkv=2, d=128, n0=77,
                                 window=0, scale=1.0, eps=1e-6, seed=26, pool=pool)
        if want("decode_step_shared_g4_d128"):
            gen_decode_step_shared("decode_step_shared_g4_d128", nq=8, nkv=2, d=128, n=120,
                                   pos=119, base=500000.0, window=0, scale=1.0, eps=1e-6,
                                   rope=True, seed=27, pool=pool)
        if want("decode_step_shared_nope_win_d256"):
            gen_decode_step_shared("decode_step_shared_nope_win_d256", nq=4, nkv=2, d=256, n=70,
                                   pos=69, base=10000.0, window=20, scale=1.0, eps=1e-6,
                                   rope=False, seed=28, pool=pool)
        if want("prefill_nope_d128"):
            gen_prefill_nope("prefill_nope_d128", nq=4, nkv=2, d=128, M=13, n0=25, window=0,
                             scale=1.0, eps=1e-6, seed=29, pool=pool)
        if want("prefill_shared_win_d128"):
            gen_prefill_shared("prefill_shared_win_d128", nq=4, nkv=2, d=128, M=10, N=40,
                               pos0=30, base=10000.0, window=12, scale=1.0, eps=1e-6, seed=30,
                               pool=pool)
        if want("head_bench_check"):
            gen_head("head_bench_check", n=160, d=128, sigma=0.2, seed=1234)
        if want("gqa_headmajor_d64"):
            gen_gqa_headmajor("gqa_headmajor_d64", nq=4, nkv=1, n=97, d=64, pos_cur=97,
                              window=0, seed=14, pool=pool)
        if want("gqa_win_headmajor_d64"):
            gen_gqa_headmajor("gqa_win_headmajor_d64", nq=4, nkv=2, n=90, d=64, pos_cur=89,
                              window=20, seed=15, pool=pool)
        # head dim 512: the global layers of the reference's gemma4 models
        # (model.h:562-564), attention scale 1 (model.h:39, forward.h:170-173)
        if want("decode_step_norm_g4_d512_scale1"):
            gen_decode_step_norm("decode_step_norm_g4_d512_scale1", nq=8, nkv=2, d=512, n0=24,
                                 base=1000000.0, window=0, scale=1.0, eps=1e-6, v_norm=1,
                                 seed=31, pool=pool)
        if want("prefill_norm_d512"):
            gen_prefill("prefill_norm_d512", nq=4, nkv=1, d=512, M=6, n0=10, base=1000000.0,
                        window=0, scale=1.0, eps=1e-6, norms=True, seed=32, pool=pool)
        if want("decode_step_shared_d512"):
            gen_decode_step_shared("decode_step_shared_d512", nq=4, nkv=1, d=512, n=30, pos=29,
                                   base=1000000.0, window=0, scale=1.0, eps=1e-6, rope=True,
                                   seed=33, pool=pool)
        if want("bf16_cache_g8_d128"):
            gen_bf16_cache("bf16_cache_g8_d128", nq=8, nkv=1, n=70, d=128, sigma=1.0, seed=16,
                           pool=pool)
    if want("rope_d128_theta5e5"):
        gen_rope("rope_d128_theta5e5", 128, 500000.0, [0, 1, 7, 4096, 16384, 131072], seed=17)
    if want("rope_d256_theta1e4"):
        gen_rope("rope_d256_theta1e4", 256, 10000.0, [0, 3, 1023, 32768], seed=18)
    if want("rope_d512_theta1e6"):
        gen_rope("rope_d512_theta1e6", 512, 1000000.0, [0, 5, 4096, 131072], seed=34)
    if want("q8_rows_d512"):
        gen_q8_rows("q8_rows_d512", 512, seed=35)
    if want("vexp_points"):
        gen_vexp("vexp_points", seed=19)
    if want("q8_rows_d128"):
        gen_q8_rows("q8_rows_d128", 128, seed=25)
    if want("rmsnorm_cases"):
        gen_rmsnorm("rmsnorm_cases", [7, 16, 100, 128, 256, 1024], seed=22)


if __name__ == "__main__":
    main()
