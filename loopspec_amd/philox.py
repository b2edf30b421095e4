"""Philox4x32-10 counter-based generator (Salmon, Moraes, Dror, Shaw, SC'11).

Used to produce the uniforms that the verify/sample entry points consume, so
that the HIP kernels and the CPU oracle see identical draws. Block i of a
stream uses counter (i, 0, 0, 0) and key (seed_lo, seed_hi); each block yields
four 32-bit words, and word x becomes the binary32 uniform (x >> 8) * 2^-24 in
[0, 1).
"""

from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32(counter: np.ndarray, key: np.ndarray, rounds: int = 10) -> np.ndarray:
    """Apply Philox4x32-`rounds` to counters [N, 4] (uint32) with key [2] (uint32)."""
    c = np.asarray(counter, dtype=np.uint32).reshape(-1, 4).astype(np.uint64)
    k0 = np.uint32(key[0])
    k1 = np.uint32(key[1])
    c0, c1, c2, c3 = c[:, 0], c[:, 1], c[:, 2], c[:, 3]
    for r in range(rounds):
        if r:
            k0 = np.uint32((int(k0) + int(W0)) & 0xFFFFFFFF)
            k1 = np.uint32((int(k1) + int(W1)) & 0xFFFFFFFF)
        p0 = M0 * c0
        p1 = M1 * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK32
        c0, c1, c2, c3 = (hi1 ^ c1 ^ np.uint64(k0)), lo1, (hi0 ^ c3 ^ np.uint64(k1)), lo0
    return np.stack([c0, c1, c2, c3], axis=1).astype(np.uint32)


def random_words(n: int, seed: int, offset: int = 0) -> np.ndarray:
    """n uint32 words of the stream `seed`, starting at word `offset`."""
    first = offset // 4
    blocks = (offset + n + 3) // 4 - first
    ctr = np.zeros((blocks, 4), dtype=np.uint32)
    ctr[:, 0] = (np.arange(first, first + blocks, dtype=np.uint64) & MASK32).astype(np.uint32)
    ctr[:, 1] = ((np.arange(first, first + blocks, dtype=np.uint64) >> np.uint64(32)) & MASK32).astype(np.uint32)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)
    words = philox4x32(ctr, key).reshape(-1)
    start = offset - first * 4
    return words[start:start + n]


def uniforms(shape, seed: int, offset: int = 0) -> np.ndarray:
    """Binary32 uniforms in [0, 1): (word >> 8) * 2^-24."""
    n = int(np.prod(shape))
    w = random_words(n, seed, offset)
    return ((w >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)).reshape(shape)
