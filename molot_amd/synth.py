"""Seeded synthetic inputs for the decode-attention path.

A repo-owned generator so inputs are reproducible without depending on
libstdc++'s ``normal_distribution``: splitmix64 produces a stream of 64-bit
words (word i of seed s is a pure function of (s, i), so long draws
vectorise), and Box-Muller turns consecutive word pairs into two standard
normals in float64, which are then scaled and rounded to float32.

Draw order for one decode step (fixed, so fixtures are reproducible):
q, k_new, v_new, then the K cache, then the V cache, then any block-table
permutation.  The default seed 1234 is the reference benchmark's
(bench/bench.cc:28).
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22  # normals per vectorised block (bounds float64 temporaries)


def splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    """Words start .. start+count-1 of the splitmix64 stream of ``seed``."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _box_muller(words: np.ndarray) -> np.ndarray:
    a = words[0::2]
    b = words[1::2]
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (b >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    ang = 2.0 * np.pi * u2
    out = np.empty(words.size, dtype=np.float64)
    out[0::2] = r * np.cos(ang)
    out[1::2] = r * np.sin(ang)
    return out


class Stream:
    """A position in the seeded word stream; every draw advances it."""

    def __init__(self, seed: int = 1234):
        self.seed = int(seed)
        self.pos = 0

    def words(self, count: int) -> np.ndarray:
        w = splitmix64(self.seed, self.pos, count)
        self.pos += count
        return w

    def normal(self, shape, sigma: float = 1.0) -> np.ndarray:
        """float32 N(0, sigma^2) of the given shape (sigma scales a unit normal).

        Blocks of _CHUNK normals are independent slices of the word stream, so
        long draws are filled by a few threads (numpy releases the GIL)."""
        count = int(np.prod(shape))
        out = np.empty(count, dtype=np.float32)
        base = self.pos
        starts = list(range(0, count, _CHUNK))

        def fill(start: int) -> None:
            m = min(_CHUNK, count - start)
            z = _box_muller(splitmix64(self.seed, base + start, m + (m & 1)))[:m]
            out[start:start + m] = (z * sigma).astype(np.float32)

        if len(starts) > 1:
            workers = max(1, min(8, os.cpu_count() or 1, len(starts)))
            with ThreadPoolExecutor(workers) as ex:
                list(ex.map(fill, starts))
        elif starts:
            fill(0)
        # every block consumed an even number of words (_CHUNK is even)
        self.pos = base + count + (count & 1)
        return out.reshape(shape)

    def uniform_int(self, lo: int, hi: int, count: int) -> np.ndarray:
        """Integers uniform in [lo, hi] (inclusive), via the top 53 bits."""
        u = (self.words(count) >> np.uint64(11)).astype(np.float64) / 9007199254740992.0
        return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)

    def permutation(self, n: int) -> np.ndarray:
        """Fisher-Yates shuffle of 0..n-1 driven by the stream."""
        perm = np.arange(n, dtype=np.int64)
        if n <= 1:
            return perm.astype(np.int32)
        w = self.words(n - 1)
        for k, i in enumerate(range(n - 1, 0, -1)):
            j = int(w[k] % np.uint64(i + 1))
            perm[i], perm[j] = perm[j], perm[i]
        return perm.astype(np.int32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (include/molot/quant.h:192-198)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    return (u >> np.uint64(16)).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp32 (include/molot/quant.h:186-191)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)

