"""Python host interface of the decode-attention path, over the C ABI.

Names, argument order and meaning follow the reference's C++ interface
(include/molot/attn.h, include/molot/forward.h) so tests read like the
reference's own checks; tensors are torch device tensors (torch supplies
device memory and the current HIP stream, nothing else).  Every call is
asynchronous on the current stream, like the C ABI.

Shapes are validated here before any pointer crosses the ABI, so a kernel
never sees a buffer smaller than the shape it is told.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import lib as _lib
from .lib import KV_BF16, KV_F32, KV_Q8, check

__all__ = [
    "KV_F32", "KV_BF16", "KV_Q8", "q8_row_bytes", "q8_block_bytes", "rope_inv_freq", "rope_apply", "rope_append", "attn_decode_gqa_cache",
    "attn_decode_gqa", "attn_decode_gqa_win", "attn_decode_head", "attn_decode_head_win",
    "attn_decode_strided", "decode_step", "attn_decode_paged", "decode_step_paged",
    "rope_append_paged", "vexp", "decode_step_shared", "decode_step_paged_shared", "prefill_q",
    "attn_prefill_paged", "set_merge", "set_prefill_presplit",
    "last_plan", "set_split_chunk", "attn_prefill_gqa", "prefill_step", "KVCache", "kv_dtype_of",
]


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _need(t: torch.Tensor, name: str, dtype=None, min_numel: int = 0) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a device tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise TypeError(f"{name}: dtype {t.dtype} not supported")
    if t.numel() < min_numel:
        raise ValueError(f"{name}: holds {t.numel()} elements, shape needs {min_numel}")


def kv_dtype_of(t: torch.Tensor) -> int:
    """KV element code of a cache tensor: fp32, bf16 (as bf16/int16 bits), or
    Q8 (uint8/int8 bytes of the Q8 layouts, include/molot_amd/attn_hip.h)."""
    if t.dtype == torch.float32:
        return KV_F32
    if t.dtype in (torch.bfloat16, torch.int16, torch.uint16):
        return KV_BF16
    if t.dtype in (torch.uint8, torch.int8):
        return KV_Q8
    raise TypeError(f"KV cache dtype {t.dtype} not supported (float32, bfloat16 or Q8 bytes)")


_KV_DTYPES = (torch.float32, torch.bfloat16, torch.int16, torch.uint16, torch.uint8, torch.int8)


def q8_row_bytes(nkv: int, d: int) -> int:
    """Bytes per token of a token-major Q8 cache (codes, then padded scales)."""
    return int(_lib.load().molot_hip_q8_row_bytes(int(nkv), int(d)))


def q8_block_bytes(nkv: int, d: int, page: int) -> int:
    """Bytes per block of a paged Q8 cache."""
    return int(_lib.load().molot_hip_q8_block_bytes(int(nkv), int(d), int(page)))


def _row_units(kvd: int, nkv: int, d: int) -> int:
    """Tensor elements per token of a token-major cache."""
    return q8_row_bytes(nkv, d) if kvd == KV_Q8 else nkv * d


def _block_units(kvd: int, nkv: int, d: int, page: int) -> int:
    """Tensor elements per block of a paged cache."""
    return q8_block_bytes(nkv, d, page) if kvd == KV_Q8 else nkv * page * d


def rope_inv_freq(base: float, d: int) -> torch.Tensor:
    """Host fp32 table 1/base^(2i/d), i < d/2 (include/molot/attn.h:31-33)."""
    out = (ctypes.c_float * (d // 2))()
    _lib.load().molot_rope_inv_freq(float(base), int(d), out)
    return torch.tensor(list(out), dtype=torch.float32)


def rope_apply(x: torch.Tensor, pos: int, inv_freq: torch.Tensor) -> torch.Tensor:
    """In-place NEOX RoPE of every head of x[..., d] (include/molot/attn.h:19-28)."""
    d = x.shape[-1]
    _need(x, "x", torch.float32)
    _need(inv_freq, "inv_freq", torch.float32, d // 2)
    nheads = x.numel() // d
    check(_lib.load().molot_hip_rope_apply(_ptr(x), nheads, d, int(pos), _ptr(inv_freq),
                                           _stream()), "rope_apply")
    return x


def rope_append(q, k_new, v_new, K, V, nq, nkv, d, slot, pos, inv_freq, cap=None):
    """RoPE q (in place) and k_new, append k/v at `slot` (forward.h:556-575)."""
    kvd = kv_dtype_of(K)
    row = _row_units(kvd, nkv, d)
    cap = K.numel() // row if cap is None else cap
    if slot < 0 or slot >= cap:
        raise RuntimeError("fwd: KV cache full")  # forward.h:570
    _need(q, "q", torch.float32, nq * d)
    _need(k_new, "k_new", torch.float32, nkv * d)
    _need(v_new, "v_new", torch.float32, nkv * d)
    _need(K, "K", _KV_DTYPES, (slot + 1) * row)
    _need(V, "V", K.dtype, (slot + 1) * row)
    _need_table(inv_freq, d)
    check(_lib.load().molot_hip_rope_append(_ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V),
                                            nq, nkv, d, int(slot), int(pos), _ptr(inv_freq), kvd,
                                            _stream()), "rope_append")


def attn_decode_strided(Q, K, V, O, nq, nkv, n, d, tok_stride, head_stride, scale, pos_cur,
                        window):
    """Attention with row t of KV head h at t*tok_stride + h*head_stride
    (Q8: the token-major byte layout, tok_stride = q8_row_bytes(nkv, d))."""
    kvd = kv_dtype_of(K)
    _need(Q, "Q", torch.float32, nq * d)
    _need(O, "O", torch.float32, nq * d)
    if n > 0:
        span = (n - 1) * tok_stride + (nkv - 1) * head_stride + d
        if kvd == KV_Q8:
            span = n * tok_stride  # the row's scales end it
        _need(K, "K", _KV_DTYPES, span)
        _need(V, "V", K.dtype, span)
    check(_lib.load().molot_hip_attn_decode_strided(
        _ptr(Q), _ptr(K), _ptr(V), _ptr(O), nq, nkv, int(n), d, int(tok_stride), int(head_stride),
        float(scale), int(pos_cur), int(window), kvd, _stream()), "attn_decode")
    return O


def attn_decode_gqa_cache(Q, K, V, O, nq, nkv, n, qhd, scale, pos_cur, window):
    """GQA decode over the token-major cache [n][nkv*qhd] (attn.h:125-177)."""
    row = _row_units(kv_dtype_of(K), nkv, qhd)
    return attn_decode_strided(Q, K, V, O, nq, nkv, n, qhd, row, qhd, scale, pos_cur, window)


def attn_decode_gqa(Q, K, V, O, nq, nkv, n, d, scale):
    """GQA decode over the head-major layout [nkv][n][d] (attn.h:111-120)."""
    return attn_decode_strided(Q, K, V, O, nq, nkv, n, d, d, n * d, scale, n, 0)


def attn_decode_gqa_win(Q, K, V, O, nq, nkv, n, d, scale, pos_cur, window):
    """Head-major GQA decode with a sliding window (attn.h:178-187)."""
    return attn_decode_strided(Q, K, V, O, nq, nkv, n, d, d, n * d, scale, pos_cur, window)


def attn_decode_head_win(Q, K, V, out, n, d, scale, pos_cur, window):
    """One head over contiguous K/V [n][d] (attn.h:57-101)."""
    return attn_decode_strided(Q, K, V, out, 1, 1, n, d, d, n * d, scale, pos_cur, window)


def attn_decode_head(Q, K, V, out, n, d, scale):
    """One head, full prefix (attn.h:104-107)."""
    return attn_decode_head_win(Q, K, V, out, n, d, scale, n if n > 0 else 0, 0)


def decode_step(q, k_new, v_new, K, V, O, nq, nkv, d, slot, pos, inv_freq, scale, window,
                q_norm=None, k_norm=None, v_norm=False, eps=1e-6):
    """forward.h:556-591 for one layer in one fused launch: RoPE of q (in place)
    and k_new, append of k/v at `slot`, attention over slot+1 at pos_cur=pos.

    With the layer's norms (forward.h:554, 562-563): q and k RMS-normed per
    head with weights q_norm / k_norm ([d] device tensors), v over all its
    nkv*d values when v_norm, before RoPE and the append."""
    kvd = kv_dtype_of(K)
    row = _row_units(kvd, nkv, d)
    cap = K.numel() // row
    if slot < 0 or slot >= cap:
        raise RuntimeError("fwd: KV cache full")  # forward.h:570
    _need(q, "q", torch.float32, nq * d)
    _need(k_new, "k_new", torch.float32, nkv * d)
    _need(v_new, "v_new", torch.float32, nkv * d)
    _need(K, "K", _KV_DTYPES, (slot + 1) * row)
    _need(V, "V", K.dtype, (slot + 1) * row)
    _need(O, "O", torch.float32, nq * d)
    _need_table(inv_freq, d)
    if q_norm is None and k_norm is None and not v_norm:
        check(_lib.load().molot_hip_decode_step(
            _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V), _ptr(O), nq, nkv, d, int(slot),
            int(pos), _ptr(inv_freq), float(scale), int(window), kvd, _stream()), "decode_step")
        return O
    _need_norms(q_norm, k_norm, d)
    check(_lib.load().molot_hip_decode_step_norm(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V), _ptr(O), nq, nkv, d, int(slot),
        int(pos), _ptr(q_norm), _ptr(k_norm), int(bool(v_norm)), float(eps), _ptr(inv_freq),
        float(scale), int(window), kvd, _stream()), "decode_step_norm")
    return O


def _need_table(inv_freq, d):
    """A RoPE table of d/2 floats, or None: a layer without RoPE (an empty
    L.freq, model.h:535-536), whose q and k forward.h leaves unrotated."""
    if inv_freq is not None:
        _need(inv_freq, "inv_freq", torch.float32, d // 2)


def _need_norms(q_norm, k_norm, d):
    if q_norm is not None:
        _need(q_norm, "q_norm", torch.float32, d)
    if k_norm is not None:
        _need(k_norm, "k_norm", torch.float32, d)


def _check_paged(block_table, seq_lens, pos, B, max_blocks, nkv, d, page, K, V):
    _need(block_table, "block_table", torch.int32, B * max_blocks)
    _need(seq_lens, "seq_lens", torch.int32, B)
    if pos is not None:
        _need(pos, "pos", torch.int32, B)
    bu = _block_units(kv_dtype_of(K), nkv, d, page)
    nblocks = K.numel() // bu
    _need(K, "K", _KV_DTYPES, nblocks * bu)
    _need(V, "V", K.dtype, nblocks * bu)
    # host-side bounds check of every block id a kernel can reach
    lens = seq_lens.cpu()
    if int(lens.min()) < 0 or int(lens.max()) > max_blocks * page:
        raise ValueError("seq_lens outside [0, max_blocks*page]")
    bt = block_table.view(B, max_blocks).cpu()
    for b in range(B):
        used = (int(lens[b]) + page - 1) // page
        if used and (int(bt[b, :used].min()) < 0 or int(bt[b, :used].max()) >= nblocks):
            raise ValueError(f"block_table row {b} names a block outside the pool")
    return int(lens.max()) if B else 0


def attn_decode_paged(Q, K, V, O, block_table, seq_lens, pos, B, max_blocks, nq, nkv, d, page,
                      scale, window=0):
    """Batched decode over a paged cache [blocks][nkv][page][d] (no reference counterpart)."""
    kvd = kv_dtype_of(K)
    _need(Q, "Q", torch.float32, B * nq * d)
    _need(O, "O", torch.float32, B * nq * d)
    max_len = _check_paged(block_table, seq_lens, pos, B, max_blocks, nkv, d, page, K, V)
    check(_lib.load().molot_hip_attn_decode_paged(
        _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(block_table), _ptr(seq_lens), _ptr(pos), B,
        max_blocks, max_len, nq, nkv, d, page, float(scale), int(window), kvd, _stream()),
        "attn_decode_paged")
    return O


def decode_step_paged(q, k_new, v_new, K, V, O, block_table, seq_lens, pos, B, max_blocks, nq,
                      nkv, d, page, inv_freq, scale, window=0, q_norm=None, k_norm=None,
                      v_norm=False, eps=1e-6):
    """Fused RoPE + append + attention for B sequences over a paged cache.

    seq_lens[b] counts the new token, which lands in slot seq_lens[b]-1.
    Norms as decode_step, per sequence."""
    kvd = kv_dtype_of(K)
    _need(q, "q", torch.float32, B * nq * d)
    _need(O, "O", torch.float32, B * nq * d)
    _need(k_new, "k_new", torch.float32, B * nkv * d)
    _need(v_new, "v_new", torch.float32, B * nkv * d)
    _need_table(inv_freq, d)
    max_len = _check_paged(block_table, seq_lens, pos, B, max_blocks, nkv, d, page, K, V)
    if B and int(seq_lens.min()) < 1:
        raise ValueError("decode_step_paged: every sequence needs seq_lens >= 1")
    if q_norm is None and k_norm is None and not v_norm:
        check(_lib.load().molot_hip_decode_step_paged(
            _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V), _ptr(O), _ptr(block_table),
            _ptr(seq_lens), _ptr(pos), B, max_blocks, max_len, nq, nkv, d, page, _ptr(inv_freq),
            float(scale), int(window), kvd, _stream()), "decode_step_paged")
        return O
    _need_norms(q_norm, k_norm, d)
    check(_lib.load().molot_hip_decode_step_paged_norm(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V), _ptr(O), _ptr(block_table),
        _ptr(seq_lens), _ptr(pos), B, max_blocks, max_len, nq, nkv, d, page, _ptr(q_norm),
        _ptr(k_norm), int(bool(v_norm)), float(eps), _ptr(inv_freq), float(scale), int(window),
        kvd, _stream()), "decode_step_paged_norm")
    return O


def attn_prefill_gqa(Qm, K, V, Om, nq, nkv, M, N, d, scale, pos0, window=0):
    """gemm.h:409-446: causal prefill attention of M queries [M][nq][d]
    (positions pos0..) over the token-major cache [N][nkv*d]."""
    kvd = kv_dtype_of(K)
    row = _row_units(kvd, nkv, d)
    _need(Qm, "Qm", torch.float32, M * nq * d)
    _need(Om, "Om", torch.float32, M * nq * d)
    _need(K, "K", _KV_DTYPES, N * row)
    _need(V, "V", K.dtype, N * row)
    check(_lib.load().molot_hip_attn_prefill_gqa(
        _ptr(Qm), _ptr(K), _ptr(V), _ptr(Om), nq, nkv, int(M), int(N), d, float(scale),
        int(pos0), int(window), kvd, _stream()), "attn_prefill_gqa")
    return Om


def prefill_step(q, k_new, v_new, K, V, O, nq, nkv, d, M, slot0, pos0, inv_freq, scale,
                 window=0, q_norm=None, k_norm=None, v_norm=False, eps=1e-6):
    """forward.h:367-399 for one layer: norms (optional) and RoPE of the M
    prompt tokens' q (in place) and k, append at slots slot0.., then causal
    prefill attention over slot0 + M."""
    kvd = kv_dtype_of(K)
    row = _row_units(kvd, nkv, d)
    cap = K.numel() // row
    if slot0 + M > cap:
        raise RuntimeError("fwd: KV cache full")  # forward.h:380
    _need(q, "q", torch.float32, M * nq * d)
    _need(k_new, "k_new", torch.float32, M * nkv * d)
    _need(v_new, "v_new", torch.float32, M * nkv * d)
    _need(O, "O", torch.float32, M * nq * d)
    _need(K, "K", _KV_DTYPES, cap * row)
    _need(V, "V", K.dtype, cap * row)
    _need_table(inv_freq, d)
    _need_norms(q_norm, k_norm, d)
    check(_lib.load().molot_hip_prefill_step(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V), _ptr(O), nq, nkv, d, int(M),
        int(slot0), int(pos0), _ptr(q_norm), _ptr(k_norm), int(bool(v_norm)), float(eps),
        _ptr(inv_freq), float(scale), int(window), kvd, _stream()), "prefill_step")
    return O


def prefill_step_paged(q, k_new, v_new, K, V, O, block_row, max_blocks, page, nq, nkv, d, M,
                       slot0, pos0, inv_freq, scale, window=0, q_norm=None, k_norm=None,
                       v_norm=False, eps=1e-6):
    """prefill_step for one sequence of a paged cache [blocks][nkv][page][d]
    (Q8: the paged block layout): block_row [max_blocks] int32 is that
    sequence's row of the block table; the prompt's rows land in slots
    slot0 .. slot0+M-1 (no reference counterpart: the paged manager's
    per-sequence prefill)."""
    kvd = kv_dtype_of(K)
    if slot0 < 0 or slot0 + M > max_blocks * page:
        raise RuntimeError("fwd: KV cache full")
    _need(q, "q", torch.float32, M * nq * d)
    _need(k_new, "k_new", torch.float32, M * nkv * d)
    _need(v_new, "v_new", torch.float32, M * nkv * d)
    _need(O, "O", torch.float32, M * nq * d)
    _need_table(inv_freq, d)
    _need(block_row, "block_row", torch.int32, max_blocks)
    bu = _block_units(kvd, nkv, d, page)
    nblocks = K.numel() // bu
    _need(K, "K", _KV_DTYPES, nblocks * bu)
    _need(V, "V", K.dtype, nblocks * bu)
    used = (slot0 + M + page - 1) // page
    row = block_row.cpu()
    if used and (int(row[:used].min()) < 0 or int(row[:used].max()) >= nblocks):
        raise ValueError("block_row names a block outside the pool")
    _need_norms(q_norm, k_norm, d)
    check(_lib.load().molot_hip_prefill_step_paged(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V), _ptr(O), _ptr(block_row),
        int(max_blocks), int(page), nq, nkv, d, int(M), int(slot0), int(pos0), _ptr(q_norm),
        _ptr(k_norm), int(bool(v_norm)), float(eps), _ptr(inv_freq), float(scale), int(window),
        kvd, _stream()), "prefill_step_paged")
    return O


def decode_step_shared(q, K, V, O, nq, nkv, d, n, pos, inv_freq, scale, window=0, q_norm=None,
                       eps=1e-6):
    """forward.h:554-558, 578-591 for a layer reading another layer's cache
    K/V (token-major, n >= 1 valid slots): q normed (q_norm) and rotated
    (inv_freq; None: no RoPE) in place, attention into O; nothing appended."""
    kvd = kv_dtype_of(K)
    row = _row_units(kvd, nkv, d)
    if n < 1:
        raise RuntimeError("fwd: shared KV empty")  # forward.h:580
    _need(q, "q", torch.float32, nq * d)
    _need(O, "O", torch.float32, nq * d)
    _need(K, "K", _KV_DTYPES, n * row)
    _need(V, "V", K.dtype, n * row)
    _need_table(inv_freq, d)
    _need_norms(q_norm, None, d)
    check(_lib.load().molot_hip_decode_step_shared(
        _ptr(q), _ptr(K), _ptr(V), _ptr(O), nq, nkv, d, int(n), int(pos), _ptr(q_norm), float(eps),
        _ptr(inv_freq), float(scale), int(window), kvd, _stream()), "decode_step_shared")
    return O


def decode_step_paged_shared(q, K, V, O, block_table, seq_lens, pos, B, max_blocks, nq, nkv, d,
                             page, inv_freq, scale, window=0, q_norm=None, eps=1e-6):
    """decode_step_shared per sequence of a batch over the source layer's
    pages: sequence b attends its seq_lens[b] >= 1 rows."""
    kvd = kv_dtype_of(K)
    _need(q, "q", torch.float32, B * nq * d)
    _need(O, "O", torch.float32, B * nq * d)
    _need_table(inv_freq, d)
    _need_norms(q_norm, None, d)
    max_len = _check_paged(block_table, seq_lens, pos, B, max_blocks, nkv, d, page, K, V)
    if B and int(seq_lens.min()) < 1:
        raise RuntimeError("fwd: shared KV empty")
    check(_lib.load().molot_hip_decode_step_paged_shared(
        _ptr(q), _ptr(K), _ptr(V), _ptr(O), _ptr(block_table), _ptr(seq_lens), _ptr(pos), B,
        max_blocks, max_len, nq, nkv, d, page, _ptr(q_norm), float(eps), _ptr(inv_freq),
        float(scale), int(window), kvd, _stream()), "decode_step_paged_shared")
    return O


def prefill_q(q, nq, d, M, pos0, inv_freq, q_norm=None, eps=1e-6):
    """forward.h:370-375 for a layer without its own KV: the q heads of M
    prompt tokens [M][nq][d] normed and rotated at pos0 + m, in place."""
    _need(q, "q", torch.float32, M * nq * d)
    _need_table(inv_freq, d)
    _need_norms(q_norm, None, d)
    check(_lib.load().molot_hip_prefill_q(_ptr(q), nq, d, int(M), int(pos0), _ptr(q_norm),
                                          float(eps), _ptr(inv_freq), _stream()), "prefill_q")
    return q


def attn_prefill_paged(Qm, K, V, Om, block_row, max_blocks, page, nq, nkv, M, N, d, scale, pos0,
                       window=0):
    """attn_prefill_gqa over one sequence's pages (no reference counterpart)."""
    kvd = kv_dtype_of(K)
    _need(Qm, "Qm", torch.float32, M * nq * d)
    _need(Om, "Om", torch.float32, M * nq * d)
    _need(block_row, "block_row", torch.int32, max_blocks)
    bu = _block_units(kvd, nkv, d, page)
    nblocks = K.numel() // bu
    _need(K, "K", _KV_DTYPES, nblocks * bu)
    _need(V, "V", K.dtype, nblocks * bu)
    if N < 0 or N > max_blocks * page:
        raise ValueError("N outside [0, max_blocks*page]")
    used = (N + page - 1) // page
    row = block_row.cpu()
    if used and (int(row[:used].min()) < 0 or int(row[:used].max()) >= nblocks):
        raise ValueError("block_row names a block outside the pool")
    check(_lib.load().molot_hip_attn_prefill_paged(
        _ptr(Qm), _ptr(K), _ptr(V), _ptr(Om), _ptr(block_row), int(max_blocks), int(page), nq,
        nkv, int(M), int(N), d, float(scale), int(pos0), int(window), kvd, _stream()),
        "attn_prefill_paged")
    return Om


def rope_append_paged(q, k_new, v_new, K, V, block_table, seq_lens, pos, B, max_blocks, nq, nkv,
                      d, page, inv_freq):
    """RoPE + append of one token per sequence into its page slot seq_lens[b]-1."""
    kvd = kv_dtype_of(K)
    _need(q, "q", torch.float32, B * nq * d)
    _need(k_new, "k_new", torch.float32, B * nkv * d)
    _need(v_new, "v_new", torch.float32, B * nkv * d)
    _need_table(inv_freq, d)
    _check_paged(block_table, seq_lens, pos, B, max_blocks, nkv, d, page, K, V)
    if B and int(seq_lens.min()) < 1:
        raise ValueError("rope_append_paged: every sequence needs seq_lens >= 1")
    check(_lib.load().molot_hip_rope_append_paged(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(K), _ptr(V), _ptr(block_table), _ptr(seq_lens),
        _ptr(pos), B, max_blocks, nq, nkv, d, page, _ptr(inv_freq), kvd, _stream()),
        "rope_append_paged")


def vexp(x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    """The split-K merges' exp (device expf), elementwise (counterpart of
    norm.h:35-47)."""
    _need(x, "x", torch.float32)
    y = torch.empty_like(x) if y is None else y
    _need(y, "y", torch.float32, x.numel())
    check(_lib.load().molot_hip_vexp(_ptr(x), _ptr(y), x.numel(), _stream()), "vexp")
    return y


def prob_exp(x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    """The attention probabilities' exp as the kernels take it: 2^(x*log2 e)
    with one v_exp_f32 (counterpart of norm.h:35-47)."""
    _need(x, "x", torch.float32)
    y = torch.empty_like(x) if y is None else y
    _need(y, "y", torch.float32, x.numel())
    check(_lib.load().molot_hip_prob_exp(_ptr(x), _ptr(y), x.numel(), _stream()), "prob_exp")
    return y


def last_plan():
    """(chunks per (sequence, KV head), rows per chunk) of this thread's last
    attention launch."""
    nch, ch = ctypes.c_int(), ctypes.c_int()
    check(_lib.load().molot_hip_last_plan(ctypes.byref(nch), ctypes.byref(ch)), "last_plan")
    return nch.value, ch.value


def set_split_chunk(tokens: int) -> None:
    _lib.load().molot_hip_set_split_chunk(int(tokens))


def set_merge(in_launch) -> None:
    """Split-K chunks merged inside the attention launch (True), by the
    combine kernel (False), or as the library chooses (None, the default);
    see molot_hip_set_merge."""
    _lib.load().molot_hip_set_merge(-1 if in_launch is None else (1 if in_launch else 0))


def set_prefill_presplit(on: bool) -> None:
    """Prefill over fp32/Q8 caches from keys split into pieces once per
    launch (True, the default) or split per staged tile (False); see
    molot_hip_set_prefill_presplit.  Both give the same bits."""
    _lib.load().molot_hip_set_prefill_presplit(1 if on else 0)


def profile(fn, launches: int = 64):
    """Run fn() with launch profiling on; returns (attention launches,
    launches that needed the combine kernel) among them."""
    L = _lib.load()
    _lib.check(L.molot_hip_profile_begin(launches), "profile_begin")
    fn()
    am, cm = ctypes.c_float(), ctypes.c_float()
    na, nc = ctypes.c_int(), ctypes.c_int()
    _lib.check(L.molot_hip_profile_end(ctypes.byref(am), ctypes.byref(cm), ctypes.byref(na),
                                       ctypes.byref(nc)), "profile_end")
    return na.value, nc.value


class KVCache:
    """Device KV cache of one layer: [cap][nkv*hd] (forward.h:48-51, 104-110).

    ``append`` mirrors forward.h:566-575 (rope k, copy k/v into slot n, n++),
    fused with the RoPE of q; ``attend`` is forward.h:589-590.
    """

    def __init__(self, cap: int, nkv: int, hd: int, kv_dtype: int = KV_F32, device="cuda"):
        dt = {KV_F32: torch.float32, KV_BF16: torch.bfloat16, KV_Q8: torch.uint8}[kv_dtype]
        self.cap, self.nkv, self.hd, self.n = cap, nkv, hd, 0
        size = cap * _row_units(kv_dtype, nkv, hd)
        self.k = torch.zeros(size, dtype=dt, device=device)
        self.v = torch.zeros(size, dtype=dt, device=device)

    def reset(self) -> None:
        self.n = 0  # molot_chat.cc /reset: n = 0

    def append(self, q, k_new, v_new, nq, pos, inv_freq) -> None:
        if self.n >= self.cap:
            raise RuntimeError("fwd: KV cache full")
        rope_append(q, k_new, v_new, self.k, self.v, nq, self.nkv, self.hd, self.n, pos,
                    inv_freq, cap=self.cap)
        self.n += 1

    def attend(self, q, O, nq, scale, pos_cur, window=0):
        if self.n == 0:
            raise RuntimeError("fwd: shared KV empty")  # forward.h:580
        return attn_decode_gqa_cache(q, self.k, self.v, O, nq, self.nkv, self.n, self.hd, scale,
                                     pos_cur, window)


def default_scale(d: int) -> float:
    """1/sqrt(head_dim) (forward.h:170-173 when attn_scale_one is off)."""
    return 1.0 / math.sqrt(d)
