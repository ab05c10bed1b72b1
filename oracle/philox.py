"""Philox4x32-10 uniforms on the CPU (numpy) -- test infrastructure, never shipped.

Restates the counter-based generator the HIP kernels draw stochastic-rounding
uniforms from (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
as 1, 2, 3", SC'11; multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments
0x9E3779B9 / 0xBB67AE85, 10 rounds).  Stream positions of key ``seed`` are
grouped by 128: position ``P = 128*B + 32*q + 4*j + t`` (q, t in 0..3, j in
0..7) is the 24-bit field ``4*q + t`` of the 384-bit little-endian string
``out(24*B + 3*j) || out(24*B + 3*j + 1) || out(24*B + 3*j + 2)``, ``out(c)``
being the four words of Philox(counter = c as a 128-bit integer, key = seed),
mapped to [0, 1) as ``field * 2**-24``.  The reference has no such generator
(it draws from torch's CPU mt19937 / CUDA Philox streams); this module only
checks the device implementation and lets the CPU oracle replay the draws the
device consumed.  Pinned by the Random123 known-answer vectors and the
bit-reassembly check in ``tests/test_philox.py``.
"""

from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(counter: np.ndarray, key: tuple) -> np.ndarray:
    """counter: (N, 4) uint32 -> (N, 4) uint32 outputs for key (k0, k1)."""
    c = counter.astype(np.uint64)
    c0, c1, c2, c3 = c[:, 0], c[:, 1], c[:, 2], c[:, 3]
    k0, k1 = int(key[0]), int(key[1])
    for _ in range(10):
        p0 = M0 * c0
        p1 = M1 * c2
        n0 = (p1 >> np.uint64(32)) ^ c1 ^ np.uint64(k0)
        n2 = (p0 >> np.uint64(32)) ^ c3 ^ np.uint64(k1)
        c1 = p1 & MASK
        c3 = p0 & MASK
        c0, c2 = n0 & MASK, n2 & MASK
        k0 = (k0 + W0) & 0xFFFFFFFF
        k1 = (k1 + W1) & 0xFFFFFFFF
    return np.stack([c0, c1, c2, c3], axis=1).astype(np.uint32)


def lane_words(seed: int, groups: np.ndarray) -> np.ndarray:
    """The 12 Philox words of each lane of each position group: shape (len(groups), 8, 12)."""
    groups = np.asarray(groups, dtype=np.uint64)
    ctr = (groups[:, None, None] * np.uint64(24) + np.arange(8, dtype=np.uint64)[None, :, None] * np.uint64(3)
           + np.arange(3, dtype=np.uint64)[None, None, :]).reshape(-1)
    counter = np.zeros((ctr.size, 4), dtype=np.uint32)
    counter[:, 0] = (ctr & MASK).astype(np.uint32)
    counter[:, 1] = (ctr >> np.uint64(32)).astype(np.uint32)
    out = philox4x32_10(counter, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))
    return out.reshape(len(groups), 8, 12)


def uniforms(seed: int, offset: int, n: int) -> np.ndarray:
    """The n float32 uniforms at stream positions offset .. offset+n-1."""
    if n == 0:
        return np.zeros(0, dtype=np.float32)
    pos = np.uint64(offset) + np.arange(n, dtype=np.uint64)
    g0 = offset // 128
    words = lane_words(seed, np.arange(g0, (offset + n - 1) // 128 + 1, dtype=np.uint64))
    # 13th word of zeros so every 24-bit field reads two consecutive words
    words = np.concatenate([words, np.zeros(words.shape[:2] + (1,), dtype=np.uint32)], axis=2).astype(np.uint64)
    g = (pos // np.uint64(128) - np.uint64(g0)).astype(np.int64)
    p = (pos % np.uint64(128)).astype(np.int64)
    j, field = (p // 4) % 8, 4 * (p // 32) + p % 4
    bit = 24 * field
    k, sh = bit // 32, (bit % 32).astype(np.uint64)
    pair = words[g, j, k] | (words[g, j, k + 1] << np.uint64(32))
    value = (pair >> sh) & np.uint64(0xFFFFFF)
    return (value.astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)
