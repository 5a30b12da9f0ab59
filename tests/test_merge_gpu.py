"""The split-K merge inside the attention launch (MI355X only).

A split context's chunk partials are merged either by the combine kernel
launched after the attention kernel, or by the workgroup that completes a
slot, inside the attention launch (where the device dispatches workgroup i
to XCD i % 8 and a slot's chunks can share an XCD).  molot_hip_set_merge
forces either; by default a contiguous cache whose slots are a multiple of 8
merges in the launch and everything else uses the combine kernel.  Both must give the
oracle's result; they differ only in the summation order of the merge.
The arrival counters the in-launch merge uses must be back at zero after
every launch, whatever shapes follow one another on a stream.
"""
import numpy as np
import pytest
import torch

from conftest import normwise_err
from gpu_util import dev, dev_bf16, host, make_decode, make_paged, oracle_decode, oracle_paged
from molot_amd import attn

import oracle

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5


def announce(msg):
    print(f"[case] {msg}", flush=True)


def step(p, merge, window=None):
    """One fused decode step of problem p; returns (O, launches, combines)."""
    attn.set_merge(merge)
    try:
        q = dev(p.q)
        K = dev_bf16(p.K) if p.kv_dtype else dev(p.K)
        V = dev_bf16(p.V) if p.kv_dtype else dev(p.V)
        O = torch.empty((p.nq, p.d), dtype=torch.float32, device="cuda")
        w = p.window if window is None else window
        na, nc = attn.profile(lambda: attn.decode_step(q, dev(p.k_new), dev(p.v_new), K, V, O, p.nq,
                                                       p.nkv, p.d, p.pos, p.pos, dev(p.inv_freq),
                                                       p.scale, w))
        return host(O), host(q), na, nc
    finally:
        attn.set_merge(None)  # the library's default


# (nq, nkv, d, pos, window, bf16): slots = nkv * subgroups; 8 | slots keeps
# the 3-D grid, fewer than 8 take the 1-D XCD map, others the combine kernel
SHAPES = [
    (32, 8, 128, 6000, 0, False),    # c1/c2 shape: 8 slots, 32 chunks
    (8, 4, 256, 5000, 100, False),   # c3 shape: 4 slots (1-D map)
    (4, 1, 64, 3000, 0, False),      # one slot (1-D map)
    (16, 2, 128, 4000, 0, False),    # 2 slots of 8 heads
    (64, 16, 64, 2500, 0, False),    # 16 slots
    (24, 12, 128, 3000, 0, False),   # 12 slots: combine kernel
    (8, 8, 128, 3000, 0, False),     # one q head per slot (odd GH in the merge)
    (64, 8, 128, 20000, 0, True),    # c5 shape, bf16 on the matrix cores
    (32, 8, 64, 900, 0, True),       # bf16, few chunks
]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}q{s[1]}kv_d{s[2]}_n{s[3]}"
                                               f"{'_w' + str(s[4]) if s[4] else ''}"
                                               f"{'_bf16' if s[5] else ''}" for s in SHAPES])
def test_merge_in_launch_matches_combine(gpu, shape):
    nq, nkv, d, pos, window, bf16 = shape
    announce(f"merge {shape}")
    p = make_decode(nq, nkv, d, pos, window=window, seed=pos + d, bf16=bf16)
    o1, q1, na1, nc1 = step(p, True)
    o0, q0, na0, nc0 = step(p, False)
    slots = nkv  # one subgroup per KV head at these group sizes
    assert na1 == 1 and na0 == 1
    assert nc0 == 1, "a split context without the in-launch merge launches the combine kernel"
    if slots % 8 == 0 or slots < 8:
        assert nc1 == 0, "expected the merge inside the attention launch"
    else:
        assert nc1 == 1
    np.testing.assert_array_equal(q1, q0)  # the rotated q, written by either merge
    assert normwise_err(o1, o0) < 1e-6
    q_rot, _, O_ref, _, _ = oracle_decode(p)
    assert normwise_err(o1, O_ref) < FP32_TOL
    np.testing.assert_allclose(q1, q_rot, atol=2e-6)


@pytest.mark.parametrize("shape,in_launch", [((32, 8, 128, 9000, 0, False), True),
                                              ((64, 16, 64, 8500, 0, False), True),
                                              ((32, 8, 128, 6000, 0, False), False),
                                              ((8, 4, 256, 9000, 0, False), False),
                                              ((24, 12, 128, 9000, 0, False), False),
                                              ((64, 8, 128, 9000, 0, True), False)],
                         ids=["8slots", "16slots", "8slots_short", "4slots", "12slots",
                              "8slots_bf16"])
def test_merge_default_choice(gpu, shape, in_launch):
    """The library's default: an fp32 contiguous cache whose slots are a
    multiple of 8 and whose context spans at least 8192 rows merges in the
    launch (no combine launch); shorter contexts, other slot counts and the
    matrix-core kernel use the combine kernel; all match the oracle."""
    nq, nkv, d, pos, window, bf16 = shape
    announce(f"default merge {shape}")
    p = make_decode(nq, nkv, d, pos, window=window, seed=pos + 1, bf16=bf16)
    o, q, na, nc = step(p, None)
    assert na == 1
    assert nc == (0 if in_launch else 1)
    q_rot, _, O_ref, _, _ = oracle_decode(p)
    assert normwise_err(o, O_ref) < FP32_TOL
    np.testing.assert_allclose(q, q_rot, atol=2e-6)


def test_merge_counters_across_shapes(gpu):
    """Shapes of different chunk and slot counts in turn on one stream, each
    repeated: every repeat equals its first run, so no launch leaves an
    arrival counter behind for the next."""
    probs = [make_decode(32, 8, 128, 6000, seed=3), make_decode(8, 4, 256, 2000, window=700, seed=4),
             make_decode(4, 1, 64, 5000, seed=5), make_decode(32, 8, 128, 900, seed=6)]
    attn.set_split_chunk(0)
    first = []
    for r in range(3):
        for i, p in enumerate(probs):
            announce(f"counters round {r} problem {i}")
            o, _, _, nc = step(p, True)
            assert nc == 0
            if r == 0:
                first.append(o)
                _, _, O_ref, _, _ = oracle_decode(p)
                assert normwise_err(o, O_ref) < FP32_TOL
            else:
                assert normwise_err(o, first[i]) < 1e-6, f"round {r} problem {i}"


def test_merge_forced_chunk_counts(gpu):
    """Chunk counts from 2 to the merge's limit through forced chunk sizes."""
    p = make_decode(8, 8, 128, 4000, seed=11)
    _, _, O_ref, _, _ = oracle_decode(p)
    try:
        for chunk in (2048, 512, 64, 32):
            attn.set_split_chunk(chunk)
            announce(f"forced chunk {chunk}")
            o, _, _, nc = step(p, True)
            assert normwise_err(o, O_ref) < FP32_TOL, chunk
    finally:
        attn.set_split_chunk(0)


def test_merge_paged_batch(gpu):
    """A paged bf16 batch (64 slots: sequences of different chunk counts)
    merged in the launch equals the combine kernel's result and the oracle."""
    pg = make_paged(8, 32, 8, 128, 300, 3000, seed=21)
    B, nq, nkv, d, page = pg["B"], pg["nq"], pg["nkv"], pg["d"], pg["page"]
    inv = oracle.rope_inv_freq(500000.0, d)
    scale = 1.0 / np.sqrt(d)
    outs = []
    for merge in (True, False):
        attn.set_merge(merge)
        try:
            announce(f"paged batch merge={merge}")
            q = dev(pg["q"])
            K, V = dev_bf16(pg["Kp"]), dev_bf16(pg["Vp"])
            O = torch.empty((B, nq, d), dtype=torch.float32, device="cuda")
            attn.set_split_chunk(256)  # several chunks per sequence
            attn.decode_step_paged(q, dev(pg["k_new"]), dev(pg["v_new"]), K, V, O,
                                   dev(pg["bt"].reshape(-1)), dev(pg["n"]), None, B,
                                   pg["max_blocks"], nq, nkv, d, page, dev(inv), scale, 0)
            outs.append(host(O))
        finally:
            attn.set_split_chunk(0)
            attn.set_merge(None)
    assert normwise_err(outs[0], outs[1]) < 1e-6
    _, _, _, O_ref = oracle_paged(pg, inv, scale)
    assert normwise_err(outs[0], O_ref) < FP32_TOL
