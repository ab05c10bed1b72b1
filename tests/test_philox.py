"""Pins of the CPU Philox4x32-10 restatement (oracle/philox.py) that the device draws are
checked against: the Random123 known-answer vectors, the stream-position mapping and the
24-bit uniform conversion."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import philox

# Random123 kat_vectors, philox4x32 with 10 rounds: (counter, key, output).
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,expect", KAT)
def test_random123_known_answers(counter, key, expect):
    out = philox.philox4x32_10(np.array([counter], dtype=np.uint32), key)[0]
    assert out.tolist() == list(expect)


def test_stream_positions_and_uniform_mapping():
    """Each lane of a position group reads its 16 fields from three Philox outputs: joining the
    fields back in order must give exactly the 384 output bits (no bit dropped, repeated or
    moved), for a group whose counters use both 32-bit counter words."""
    seed = 0x0123456789ABCDEF
    key = (seed & 0xFFFFFFFF, seed >> 32)
    group = (1 << 33) + 5  # counters 24 * group + ... exceed 2**32
    u = philox.uniforms(seed, 128 * group, 128)
    assert u.dtype == np.float32 and (u >= 0).all() and (u < 1).all()
    fields = (u.astype(np.float64) * 2.0 ** 24).astype(np.uint64)
    assert np.array_equal(fields.astype(np.float64) * 2.0 ** -24, u.astype(np.float64))  # 24-bit grid
    for j in range(8):
        bits = 0
        for q in range(4):
            for t in range(4):
                bits |= int(fields[32 * q + 4 * j + t]) << (24 * (4 * q + t))
        expect = 0
        for r in range(3):
            ctr = 24 * group + 3 * j + r
            words = philox.philox4x32_10(np.array([[ctr & 0xFFFFFFFF, ctr >> 32, 0, 0]], dtype=np.uint32), key)[0]
            for w in range(4):
                expect |= int(words[w]) << (32 * (4 * r + w))
        assert bits == expect, j
    # a write that starts inside a group reads the same positions
    assert np.array_equal(philox.uniforms(seed, 128 * group + 40, 50), u[40:90])


def test_uniforms_concatenate_across_writes():
    """Consecutive writes of one stream see one sequence (offsets advance by the draws taken)."""
    whole = philox.uniforms(7, 0, 64)
    parts = np.concatenate([philox.uniforms(7, 0, 24), philox.uniforms(7, 24, 40)])
    assert np.array_equal(whole, parts)


def test_uniforms_moments():
    u = philox.uniforms(11, 0, 1 << 16).astype(np.float64)
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005
