"""Philox4x32-10 uniforms on the CPU (numpy) -- test infrastructure, never shipped.

Restates the counter-based generator the HIP kernels draw stochastic-rounding
uniforms from (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
as 1, 2, 3", SC'11; multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments
0x9E3779B9 / 0xBB67AE85, 10 rounds).  Stream position k of key ``seed`` is
word ``k % 4`` of Philox(counter = k // 4 as a 128-bit integer, key = seed),
mapped to [0, 1) as ``(word >> 8) * 2**-24``.  The reference has no such
generator (it draws from torch's CPU mt19937 / CUDA Philox streams); this
module only checks the device implementation and lets the CPU oracle replay
the draws the device consumed.  Pinned by the Random123 known-answer vectors
in ``tests/test_philox.py``.
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


def uniforms(seed: int, offset: int, n: int) -> np.ndarray:
    """The n float32 uniforms at stream positions offset .. offset+n-1 (offset % 4 == 0)."""
    assert offset % 4 == 0
    blocks = (n + 3) // 4
    ctr = np.arange(blocks, dtype=np.uint64) + np.uint64(offset // 4)
    counter = np.zeros((blocks, 4), dtype=np.uint32)
    counter[:, 0] = (ctr & MASK).astype(np.uint32)
    counter[:, 1] = (ctr >> np.uint64(32)).astype(np.uint32)
    words = philox4x32_10(counter, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)).reshape(-1)[:n]
    return ((words >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)
