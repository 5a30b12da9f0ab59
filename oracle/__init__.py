"""CPU oracle for the decode-attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or as the timed CPU baseline);
the product path (molot_amd) never calls it.

Two native libraries, built by oracle/Makefile:
  liboracle.so          restatement of the reference algorithm in plain C
                        (attn_oracle.c, each function citing the reference
                        file:line it follows) + a float64 brute force
  _ref/libmolot_ref.so  the reference's own headers compiled where they lie
                        (ref_shim.cc); optional -- present only where the
                        reference tree was available at build time, and
                        usable only on an AVX512F host
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_HERE, "liboracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libmolot_ref.so")

KV_F32 = 0
KV_BF16 = 1
KV_Q8 = 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double
_I64 = ctypes.c_int64

_lib = None
_ref = None


def _p(a):
    return ctypes.c_void_p(0 if a is None else a.ctypes.data)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle not built: {ORACLE_SO} (make -C oracle)")
        L = ctypes.CDLL(ORACLE_SO)
        sig = {
            "orc_rope_inv_freq": (None, [_F, _I, _P]),
            "orc_rope_apply": (None, [_P, _I, _I, _P]),
            "orc_rope_apply_heads": (None, [_P, _I, _I, _I, _P]),
            "orc_vexp16": (None, [_P, _P]),
            "orc_vexp": (None, [_P, _P, _I64]),
            "orc_dot": (_F, [_P, _P, _I]),
            "orc_f32_to_bf16_array": (None, [_P, _P, _I64]),
            "orc_attn_decode": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _I64, _I64,
                                       _I64, _P, _I, _I]),
            "orc_attn_decode_gqa_cache": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I]),
            "orc_attn_decode_paged": (None, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                             _F, _I, _I, _I]),
            "orc_decode_step": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _I, _I,
                                       _I]),
            "orc_attn_decode_f64": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _D, _I, _I, _I, _I64,
                                           _I64, _I64, _P, _I, _I]),
            "orc_rmsnorm": (None, [_P, _P, _P, _I, _F]),
            "orc_q8_row_bytes": (_I, [_I, _I]),
            "orc_q8_block_bytes": (_I64, [_I, _I, _I]),
            "orc_quantize_q8_row": (None, [_P, _I, _P, _P]),
            "orc_q8_store_token": (None, [_P, _I64, _P, _I, _I]),
            "orc_q8_store_tokens": (None, [_P, _I64, _P, _I, _I]),
            "orc_attn_prefill": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _I, _I]),
            "orc_decode_step_norm": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P,
                                            _I, _F, _P, _F, _I, _I, _I]),
            "orc_prefill_q": (None, [_P, _I, _I, _I, _I, _P, _F, _P]),
            "orc_decode_step_shared": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _P, _F,
                                              _I, _I, _I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def host_has_avx512f() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            return " avx512f" in f.read()
    except OSError:
        return False


def ref_available() -> bool:
    return os.path.exists(REF_SO) and host_has_avx512f()


def ref() -> ctypes.CDLL:
    """The compiled reference headers (raises if unavailable on this host)."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError("reference library unavailable (not built, or host lacks AVX512F)")
        R = ctypes.CDLL(REF_SO)
        sig = {
            "ref_pool_create": (_P, [_I]),
            "ref_pool_destroy": (None, [_P]),
            "ref_pool_size": (_I, [_P]),
            "ref_pool_cover": (None, [_P, _I64, _P]),
            "ref_rope_inv_freq": (None, [_F, _I, _P]),
            "ref_rope_apply": (None, [_P, _I, _I, _P]),
            "ref_exp16": (None, [_P, _P]),
            "ref_dot": (_F, [_P, _P, _I]),
            "ref_fp32_to_bf16": (ctypes.c_uint16, [_F]),
            "ref_bf16_to_fp32": (_F, [ctypes.c_uint16]),
            "ref_attn_decode_head_win": (None, [_P, _P, _P, _P, _I, _I, _F, _I, _I]),
            "ref_attn_decode_head": (None, [_P, _P, _P, _P, _I, _I, _F]),
            "ref_attn_decode_gqa": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P]),
            "ref_attn_decode_gqa_cache": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P]),
            "ref_attn_decode_gqa_win": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P]),
            "ref_decode_step": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _F, _I,
                                     _P]),
            "ref_attn_prefill_gqa": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I,
                                            _P]),
            "ref_prefill_step": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P,
                                      _I, _F, _P, _F, _I, _P]),
            "ref_quantize_q8_row": (None, [_P, _I, _P, _P]),
            "ref_rmsnorm": (None, [_P, _P, _P, _I, _F]),
            "ref_rmsnorm_plain": (None, [_P, _P, _I, _F]),
            "ref_decode_step_norm": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P,
                                          _I, _F, _P, _F, _I, _P]),
            "ref_decode_step_shared": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _P, _F,
                                            _I, _P]),
            "ref_prefill_shared": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _F, _P, _F,
                                          _I, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(R, name)
            fn.restype = res
            fn.argtypes = args
        _ref = R
    return _ref


class RefPool:
    """The reference's ThreadPool (thread_pool.h:17-126) with n threads."""

    def __init__(self, nthreads: int = 0):
        self.h = ref().ref_pool_create(int(nthreads))

    def size(self) -> int:
        return ref().ref_pool_size(self.h)

    def close(self) -> None:
        if self.h:
            ref().ref_pool_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


# ---------------------------------------------------------------------------
# restatement (liboracle.so)

def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def rope_inv_freq(base: float, d: int) -> np.ndarray:
    out = np.empty(d // 2, dtype=np.float32)
    lib().orc_rope_inv_freq(float(base), int(d), _p(out))
    return out


def rope_apply(x: np.ndarray, pos: int, inv_freq: np.ndarray) -> np.ndarray:
    """Returns a rotated copy of x[..., d] (every head)."""
    y = _f32(x).copy()
    d = y.shape[-1]
    lib().orc_rope_apply_heads(_p(y), y.size // d, d, int(pos), _p(_f32(inv_freq)))
    return y


def vexp(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_vexp(_p(x), _p(y), x.size)
    return y


def dot(a: np.ndarray, b: np.ndarray) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().orc_dot(_p(a), _p(b), a.size))


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def _kv_code(K: np.ndarray) -> int:
    if K.dtype == np.float32:
        return KV_F32
    if K.dtype == np.uint16:
        return KV_BF16
    if K.dtype == np.uint8:
        return KV_Q8
    raise TypeError(f"KV dtype {K.dtype}: float32, uint16 (bf16 bits) or uint8 (Q8 bytes)")


def attn_decode(Q, K, V, nq, nkv, n, d, scale, pos_cur, window, tok_stride, head_stride,
                block_stride=0, block_table=None, page=0, nthreads=0) -> np.ndarray:
    """fp32 restatement of attn.h:125-177 over a strided / paged K,V."""
    Q = _f32(Q)
    K = np.ascontiguousarray(K)
    V = np.ascontiguousarray(V)
    bt = None if block_table is None else np.ascontiguousarray(block_table, dtype=np.int32)
    O = np.empty((nq, d), dtype=np.float32)
    lib().orc_attn_decode(_p(Q), _p(K), _p(V), _p(O), nq, nkv, int(n), d, float(scale),
                          int(pos_cur), int(window), _kv_code(K), int(tok_stride),
                          int(head_stride), int(block_stride), _p(bt), int(page), int(nthreads))
    return O


def attn_decode_gqa_cache(Q, K, V, nq, nkv, n, qhd, scale, pos_cur, window, nthreads=0):
    return attn_decode(Q, K, V, nq, nkv, n, qhd, scale, pos_cur, window, nkv * qhd, qhd,
                       nthreads=nthreads)


def attn_decode_f64(Q, K, V, nq, nkv, n, d, scale, pos_cur, window, tok_stride, head_stride,
                    block_stride=0, block_table=None, page=0, nthreads=0) -> np.ndarray:
    """float64 brute force (formulation of bench/bench.cc:195-213)."""
    Q = _f32(Q)
    K = np.ascontiguousarray(K)
    V = np.ascontiguousarray(V)
    bt = None if block_table is None else np.ascontiguousarray(block_table, dtype=np.int32)
    O = np.empty((nq, d), dtype=np.float64)
    lib().orc_attn_decode_f64(_p(Q), _p(K), _p(V), _p(O), nq, nkv, int(n), d, float(scale),
                              int(pos_cur), int(window), _kv_code(K), int(tok_stride),
                              int(head_stride), int(block_stride), _p(bt), int(page),
                              int(nthreads))
    return O


def attn_decode_paged(Q, Kp, Vp, block_table, seq_lens, pos, B, max_blocks, nq, nkv, d, page,
                      scale, window=0, nthreads=0) -> np.ndarray:
    Q = _f32(Q)
    Kp = np.ascontiguousarray(Kp)
    Vp = np.ascontiguousarray(Vp)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    ps = None if pos is None else np.ascontiguousarray(pos, dtype=np.int32)
    O = np.empty((B, nq, d), dtype=np.float32)
    lib().orc_attn_decode_paged(_p(Q), _p(Kp), _p(Vp), _p(O), _p(bt), _p(sl), _p(ps), B,
                                max_blocks, nq, nkv, d, page, float(scale), int(window),
                                _kv_code(Kp), int(nthreads))
    return O


def _table(inv_freq):
    """A RoPE table, or None for a layer without RoPE (an empty L.freq)."""
    return None if inv_freq is None else _f32(inv_freq)


def decode_step(q, k_new, v_new, Kc, Vc, nq, nkv, d, slot, pos, inv_freq, scale, window,
                nthreads=0):
    """forward.h:556-591: returns (q_rot, k_rot, O); Kc/Vc are updated in place.
    inv_freq None: no RoPE (forward.h:556, :566)."""
    q = _f32(q).copy()
    k = _f32(k_new).copy()
    v = _f32(v_new)
    O = np.empty((nq, d), dtype=np.float32)
    lib().orc_decode_step(_p(q), _p(k), _p(v), _p(Kc), _p(Vc), _p(O), nq, nkv, d, int(slot),
                          int(pos), _p(_table(inv_freq)), float(scale), int(window), _kv_code(Kc),
                          int(nthreads))
    return q, k, O


def rmsnorm(x: np.ndarray, w=None, eps: float = 1e-6) -> np.ndarray:
    """norm.h:9-28 over the last axis (w None: rmsnorm_plain, norm.h:82-96)."""
    x = _f32(x)
    n = x.shape[-1]
    y = np.empty_like(x)
    wp = None if w is None else _f32(w)
    xs, ys = x.reshape(-1, n), y.reshape(-1, n)
    for i in range(xs.shape[0]):
        lib().orc_rmsnorm(_p(xs[i]), _p(wp), _p(ys[i]), n, float(eps))
    return y


def decode_step_norm(q, k_new, v_new, Kc, Vc, nq, nkv, d, slot, pos, q_norm, k_norm, v_norm,
                     eps, inv_freq, scale, window, nthreads=0):
    """forward.h:554-591 with the layer's norms: returns (q_rot, k_rot, O);
    Kc/Vc are updated in place."""
    q = _f32(q).copy()
    k = _f32(k_new).copy()
    v = _f32(v_new)
    O = np.empty((nq, d), dtype=np.float32)
    qn = None if q_norm is None else _f32(q_norm)
    kn = None if k_norm is None else _f32(k_norm)
    lib().orc_decode_step_norm(_p(q), _p(k), _p(v), _p(Kc), _p(Vc), _p(O), nq, nkv, d, int(slot),
                               int(pos), _p(qn), _p(kn), int(v_norm), float(eps),
                               _p(_table(inv_freq)), float(scale), int(window), _kv_code(Kc),
                               int(nthreads))
    return q, k, O


def attn_prefill(Qm, K, V, nq, nkv, M, N, d, scale, pos0, window, nthreads=0) -> np.ndarray:
    """gemm.h:409-446: causal prefill of M queries [M][nq][d] over the
    token-major cache [N][nkv*d] (float32 or bf16 bits)."""
    Qm = _f32(Qm)
    K = np.ascontiguousarray(K)
    V = np.ascontiguousarray(V)
    O = np.empty((M, nq, d), dtype=np.float32)
    lib().orc_attn_prefill(_p(Qm), _p(K), _p(V), _p(O), nq, nkv, int(M), int(N), d, float(scale),
                           int(pos0), int(window), _kv_code(K), int(nthreads))
    return O


def prefill_step(q, k_new, v_new, Kc, Vc, nq, nkv, d, M, slot0, pos0, q_norm, k_norm, v_norm,
                 eps, inv_freq, scale, window, nthreads=0):
    """forward.h:367-399 for one layer from the restated parts: per token m
    the norms (NULL weights / v_norm 0 skip them) and RoPE at pos0 + m of q
    [M][nq][d] and k_new [M][nkv][d], append at slot slot0 + m (bf16 caches
    rounded), then attn_prefill over N = slot0 + M.  Returns (q_rot, O);
    Kc/Vc are updated in place."""
    q = _f32(q).copy().reshape(M, nq, d)
    k = _f32(k_new).copy().reshape(M, nkv, d)
    v = _f32(v_new).copy().reshape(M, nkv, d)
    inv = _table(inv_freq)
    for m in range(M):
        if q_norm is not None:
            q[m] = rmsnorm(q[m], q_norm, eps)
        if inv is not None:  # forward.h:373
            q[m] = rope_apply(q[m], pos0 + m, inv)
        if k_norm is not None:
            k[m] = rmsnorm(k[m], k_norm, eps)
        if v_norm:
            v[m] = rmsnorm(v[m].reshape(-1), None, eps).reshape(nkv, d)
        if inv is not None:  # forward.h:381
            k[m] = rope_apply(k[m], pos0 + m, inv)
        if Kc.dtype == np.uint16:
            Kc[slot0 + m] = f32_to_bf16(k[m].reshape(-1))
            Vc[slot0 + m] = f32_to_bf16(v[m].reshape(-1))
        elif Kc.dtype == np.uint8:
            q8_store_token(Kc, slot0 + m, k[m], nkv, d)
            q8_store_token(Vc, slot0 + m, v[m], nkv, d)
        else:
            Kc[slot0 + m] = k[m].reshape(-1)
            Vc[slot0 + m] = v[m].reshape(-1)
    O = attn_prefill(q, Kc, Vc, nq, nkv, M, slot0 + M, d, scale, pos0, window, nthreads)
    return q, O


def prefill_q(q, nq, d, M, pos0, q_norm, eps, inv_freq):
    """The query prologue of a layer without its own KV (forward.h:370-375):
    rows [M][nq][d] normed (q_norm None: no norm) and rotated at pos0 + m
    (inv_freq None: no RoPE).  Returns the new rows."""
    q = _f32(q).copy().reshape(M, nq, d)
    lib().orc_prefill_q(_p(q), nq, d, int(M), int(pos0), _p(None if q_norm is None else
                                                            _f32(q_norm)), float(eps),
                        _p(_table(inv_freq)))
    return q


def decode_step_shared(q, Kc, Vc, nq, nkv, d, n, pos, q_norm, eps, inv_freq, scale, window,
                       nthreads=0):
    """forward.h:554-558, 578-591 for a layer reading another layer's cache
    Kc/Vc (token-major; n valid slots): returns (q_rot, O), appends nothing."""
    q = _f32(q).copy()
    O = np.empty((nq, d), dtype=np.float32)
    Kc = np.ascontiguousarray(Kc)
    Vc = np.ascontiguousarray(Vc)
    lib().orc_decode_step_shared(_p(q), _p(Kc), _p(Vc), _p(O), nq, nkv, d, int(n), int(pos),
                                 _p(None if q_norm is None else _f32(q_norm)), float(eps),
                                 _p(_table(inv_freq)), float(scale), int(window), _kv_code(Kc),
                                 int(nthreads))
    return q, O


# ---------------------------------------------------------------------------
# Q8 KV cache (this build's format; see attn_oracle.c): token-major rows of
# [nkv][d] int8 then nkv fp32 scales padded to 16 bytes, as uint8 arrays.

def q8_row_bytes(nkv: int, d: int) -> int:
    return int(lib().orc_q8_row_bytes(nkv, d))


def quantize_q8_row(x: np.ndarray):
    """quantize_q8_row (quant.h:34-50) of one row: (scale, int8 values)."""
    x = _f32(x)
    q = np.empty(x.size, np.int8)
    s = np.empty(1, np.float32)
    lib().orc_quantize_q8_row(_p(x), x.size, _p(q), _p(s))
    return float(s[0]), q


def q8_cache(X: np.ndarray, nkv: int, d: int) -> np.ndarray:
    """A token-major Q8 cache [N][row bytes] from fp32 rows X [N][nkv*d]."""
    X = np.ascontiguousarray(_f32(X).reshape(-1, nkv * d))
    N = X.shape[0]
    out = np.zeros((N, q8_row_bytes(nkv, d)), np.uint8)
    lib().orc_q8_store_tokens(_p(out), N, _p(X), nkv, d)
    return out


def q8_store_token(C: np.ndarray, t: int, x: np.ndarray, nkv: int, d: int) -> None:
    """Quantize rows x [nkv][d] into token t of the token-major Q8 cache C."""
    assert C.dtype == np.uint8 and C.flags.c_contiguous and C.shape[1] == q8_row_bytes(nkv, d)
    lib().orc_q8_store_token(_p(C), int(t), _p(_f32(x).reshape(-1)), nkv, d)


# Paged Q8: block = [nkv][page][d] int8 codes, then [nkv][page] fp32 scales
# (q8_block_bytes(nkv, d, page) bytes), as uint8 arrays [nblk][block bytes].

def q8_block_bytes(nkv: int, d: int, page: int) -> int:
    return int(lib().orc_q8_block_bytes(nkv, d, page))


def q8_pages(Xp: np.ndarray) -> np.ndarray:
    """Quantize fp32 pages Xp [nblk][nkv][page][d] row by row into Q8 blocks."""
    nblk, nkv, page, d = Xp.shape
    tok = np.ascontiguousarray(_f32(Xp).transpose(0, 2, 1, 3)).reshape(nblk * page, nkv * d)
    C = q8_cache(tok, nkv, d)
    codes = C[:, :nkv * d].reshape(nblk, page, nkv, d).transpose(0, 2, 1, 3)
    scales = C[:, nkv * d:nkv * d + 4 * nkv].reshape(nblk, page, nkv, 4).transpose(0, 2, 1, 3)
    out = np.concatenate([codes.reshape(nblk, -1), scales.reshape(nblk, -1)], axis=1)
    assert out.shape[1] == q8_block_bytes(nkv, d, page)
    return np.ascontiguousarray(out)


def q8_pages_dequant(P: np.ndarray, nkv: int, d: int, page: int) -> np.ndarray:
    """fp32 [nblk][nkv][page][d] of Q8 blocks."""
    nblk = P.shape[0]
    q = P[:, :nkv * page * d].view(np.int8).astype(np.float32).reshape(nblk, nkv, page, d)
    s = np.ascontiguousarray(P[:, nkv * page * d:]).view(np.float32).reshape(nblk, nkv, page, 1)
    return q * s


def q8_page_store(P: np.ndarray, blk: int, sl: int, x: np.ndarray, nkv: int, d: int,
                  page: int) -> None:
    """Quantize rows x [nkv][d] into slot sl of Q8 block blk."""
    x = _f32(x).reshape(nkv, d)
    for h in range(nkv):
        s, q = quantize_q8_row(x[h])
        o = (h * page + sl) * d
        P[blk, o:o + d] = q.view(np.uint8)
        so = nkv * page * d + 4 * (h * page + sl)
        P[blk, so:so + 4] = np.array([s], np.float32).view(np.uint8)


def q8_dequant(C: np.ndarray, nkv: int, d: int) -> np.ndarray:
    """fp32 [N][nkv*d] of a token-major Q8 cache."""
    q = C[:, :nkv * d].view(np.int8).astype(np.float32).reshape(C.shape[0], nkv, d)
    s = C[:, nkv * d:nkv * d + 4 * nkv].copy().view(np.float32).reshape(C.shape[0], nkv, 1)
    return (q * s).reshape(C.shape[0], nkv * d)
