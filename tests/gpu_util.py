"""Helpers shared by the GPU tests: seeded problems, device transfer, oracle runs."""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

import oracle
from molot_amd.synth import Stream, bf16_to_f32, f32_to_bf16


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@dataclass
class Decode:
    """One decode step at `pos` on a token-major cache pre-filled at slots [0, pos)."""
    nq: int
    nkv: int
    d: int
    pos: int
    base: float
    window: int
    scale: float
    q: np.ndarray
    k_new: np.ndarray
    v_new: np.ndarray
    K: np.ndarray  # [pos+1][nkv*d] (slot pos zero until the append)
    V: np.ndarray
    inv_freq: np.ndarray
    kv_dtype: int = 0  # 0 fp32, 1 bf16 (K/V hold the bf16 bits)


def make_decode(nq, nkv, d, pos, base=500000.0, window=0, scale=None, seed=1234, sigma_kv=1.0,
                bf16=False) -> Decode:
    """Draw order: q, k_new, v_new, K cache, V cache (molot_amd.synth)."""
    st = Stream(seed)
    q = st.normal((nq, d))
    k = st.normal((nkv, d))
    v = st.normal((nkv, d))
    K = np.zeros((pos + 1, nkv * d), np.float32)
    V = np.zeros_like(K)
    K[:pos] = st.normal((pos, nkv * d), sigma_kv)
    V[:pos] = st.normal((pos, nkv * d), sigma_kv)
    inv = oracle.rope_inv_freq(base, d)
    s = 1.0 / math.sqrt(d) if scale is None else scale
    if bf16:
        K, V = f32_to_bf16(K), f32_to_bf16(V)
    return Decode(nq, nkv, d, pos, base, window, s, q, k, v, K, V, inv, 1 if bf16 else 0)


def oracle_decode(p: Decode, nthreads=0):
    """(q_rot, k_rot, O, K_after, V_after) from the CPU oracle."""
    Kc, Vc = p.K.copy(), p.V.copy()
    q_rot, k_rot, O = oracle.decode_step(p.q, p.k_new, p.v_new, Kc, Vc, p.nq, p.nkv, p.d, p.pos,
                                         p.pos, p.inv_freq, p.scale, p.window, nthreads)
    return q_rot, k_rot, O, Kc, Vc


def widen(K: np.ndarray) -> np.ndarray:
    return bf16_to_f32(K) if K.dtype == np.uint16 else K


def make_paged(B, nq, nkv, d, lmin, lmax, page=16, seed=1234, bf16=True, spare_blocks=7):
    """B sequences of U[lmin, lmax) cached tokens plus a new one, in shuffled
    pages of a pool with spare blocks (fp32, or bf16 bits)."""
    st = Stream(seed)
    q = st.normal((B, nq, d))
    k_new = st.normal((B, nkv, d))
    v_new = st.normal((B, nkv, d))
    L = st.uniform_int(lmin, lmax, B).astype(np.int32)  # context before the new token
    n = L + 1
    blocks = (n + page - 1) // page
    nblk = int(blocks.sum()) + spare_blocks
    perm = st.permutation(nblk)
    max_blocks = int(blocks.max())
    bt = np.zeros((B, max_blocks), np.int32)
    o = 0
    for b in range(B):
        bt[b, :blocks[b]] = perm[o:o + blocks[b]]
        o += blocks[b]
    Kp = st.normal((nblk, nkv, page, d))
    Vp = st.normal((nblk, nkv, page, d))
    if bf16:
        Kp, Vp = f32_to_bf16(Kp), f32_to_bf16(Vp)
    return dict(q=q, k_new=k_new, v_new=v_new, n=n, bt=bt, Kp=Kp, Vp=Vp, page=page,
                max_blocks=max_blocks, B=B, nq=nq, nkv=nkv, d=d)


def oracle_paged(P, inv, scale, window=0, pos=None):
    """The oracle's fused step per sequence of a make_paged batch: (q_rot, K pages, V pages, O)."""
    Kp, Vp = P["Kp"].copy(), P["Vp"].copy()
    B, nq, nkv, d, page = P["B"], P["nq"], P["nkv"], P["d"], P["page"]
    q = np.empty_like(P["q"])
    for b in range(B):
        n = int(P["n"][b])
        p = n - 1 if pos is None else int(pos[b])
        q[b] = P["q"][b] if inv is None else oracle.rope_apply(P["q"][b], p, inv)
        k = P["k_new"][b] if inv is None else oracle.rope_apply(P["k_new"][b], p, inv)
        slot = n - 1
        blk = P["bt"][b, slot // page]
        if Kp.dtype == np.uint16:
            Kp[blk, :, slot % page] = oracle.f32_to_bf16(k)
            Vp[blk, :, slot % page] = oracle.f32_to_bf16(P["v_new"][b])
        else:
            Kp[blk, :, slot % page] = k
            Vp[blk, :, slot % page] = P["v_new"][b]
    O = oracle.attn_decode_paged(q, Kp, Vp, P["bt"], P["n"], pos, B, P["max_blocks"], nq, nkv, d,
                                 page, scale, window)
    return q, Kp, Vp, O
