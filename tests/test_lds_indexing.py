"""Bounds of every data-dependent LDS index of the encode, restated on the host.

The step kernels index their LDS tables with values computed from the data: the lookup-table
bucket of x = m / s (from its bit pattern), the number of levels below x (`idx`, from the bucket's
entry), the level neighbours of idx, the update-SR entry of idx, the decode entry of a code byte.
Each restatement below follows the device code line for line (aw4_codec.h: lut_field,
lut_bucket_unsigned / lut_bucket_signed, encode_block, update_sr_tables, encode_block_la; decode4)
and the tables the library itself builds (aw4_encode_tables), and checks the index against the
size of the LDS array it reads, for every fp32 bit pattern class and for adversarial blocks
(all zero, NaN and infinite values, huge and subnormal values, values on the levels).
"""

import numpy as np
import pytest

from adamw4bit_amd import _lib
from adamw4bit_amd import quantization as q

EXP0, HALF, ENTRIES = _lib.LUT_EXP0, _lib.LUT_HALF, _lib.LUT_ENTRIES
N_LEVELS, N_PAIRS, N_DEC, N_STAGE = 16, 17, 256, 32
# lookup-table ids (aw4_codec.h): round-to-nearest per codebook, dyn4 with the zero floor, level counts
LUT_RTN = {cb: cb for cb in range(5)}
LUT_RTN_DYN4_FLOOR = 5
LUT_LEVELS = {cb: 6 + cb for cb in range(5)}


def lut_field(u):
    """min(max(ubfe(u, 20, 11), EXP0 - 1), EXP0 - 2 + HALF)."""
    return np.minimum(np.maximum((u >> np.uint32(20)) & np.uint32(0x7FF), EXP0 - 1), EXP0 - 2 + HALF).astype(np.int64)


def bucket_unsigned(x):
    return lut_field(x.view(np.uint32)) - (EXP0 - 1)


def bucket_signed(x):
    u = x.view(np.uint32)
    return lut_field(u) - (EXP0 - 1) + (u >> np.uint32(31)).astype(np.int64) * HALF


def every_bit_class():
    """One float per value of bits 20..31 (all a bucket reads), with the low 20 bits 0 and all ones."""
    top = np.arange(1 << 12, dtype=np.uint32) << np.uint32(20)
    return np.concatenate([top, top | np.uint32(0xFFFFF)]).view(np.float32)


@pytest.fixture(scope="module")
def luts():
    return _lib.encode_tables()  # (NUM_LUTS, ENTRIES, 4) words: thr bits, base, level lo, level hi


def idx_of(luts, lut_id, x, signed):
    """The kernel's code or level count of x: base + (x >= thr) of x's bucket entry."""
    b = bucket_signed(x) if signed else bucket_unsigned(x)
    assert b.min() >= 0 and b.max() < ENTRIES, (b.min(), b.max())
    entry = luts[lut_id][b]
    thr = entry[:, 0].copy().view(np.float32)
    return entry[:, 1].astype(np.int64) + (x >= thr)


def test_buckets_stay_in_the_table_for_every_bit_pattern():
    x = every_bit_class()
    for b in (bucket_unsigned(x), bucket_signed(x)):
        assert b.min() >= 0 and b.max() < ENTRIES
    # the unsigned form (second moments, x >= -0 or NaN) stays in the magnitude half
    assert bucket_unsigned(x).max() < HALF


def test_planted_unclamped_bucket_leaves_the_table():
    """Without the clamp (a plausible slip) the same patterns index far outside the table."""
    u = every_bit_class().view(np.uint32)
    raw = ((u >> np.uint32(20)) & np.uint32(0x7FF)).astype(np.int64) - (EXP0 - 1)
    assert raw.min() < 0 and raw.max() >= ENTRIES


def test_level_counts_and_codes_index_the_level_tables(luts):
    """Level count idx in [0, 16] (pairs / update-SR entries: 17), its neighbours lo = max(idx - 1, 0)
    and hi = min(idx, 15) in [0, 15], round-to-nearest codes in [0, 15], for every bit class."""
    x = every_bit_class()
    for cb in range(5):
        for signed in (False, True):
            idx = idx_of(luts, LUT_LEVELS[cb], x, signed)
            assert idx.min() >= 0 and idx.max() <= N_PAIRS - 1, (cb, idx.min(), idx.max())
            lo, hi = np.maximum(idx - 1, 0), np.minimum(idx, 15)
            assert lo.max() < N_LEVELS and hi.max() < N_LEVELS
            for lut in ([LUT_RTN[cb]] + ([LUT_RTN_DYN4_FLOOR] if cb == _lib.CB_DYN4 else [])):
                code = idx_of(luts, lut, x, signed)
                assert code.min() >= 0 and code.max() < N_LEVELS, (cb, lut, code.max())


def test_every_table_entry_keeps_its_indices_in_range(luts):
    """Entry by entry: base + 1 within the level count's range wherever the threshold is finite."""
    for lut_id in range(_lib.NUM_LUTS):
        base = luts[lut_id][:, 1].astype(np.int64)
        thr = luts[lut_id][:, 0].copy().view(np.float32)
        top = N_PAIRS - 1 if lut_id >= 6 else N_LEVELS - 1
        assert base.min() >= 0
        assert (base + np.isfinite(thr)).max() <= top, lut_id


def kernel_x(m):
    """x = m / s of one 128-value block as the encode forms it: s = max(NaN-propagating max |m|,
    1e-12); a NaN x (only where s is not finite) becomes the positive quiet NaN."""
    m = m.astype(np.float32)
    a = np.abs(m)
    amax = np.float32(np.nan) if np.isnan(a).any() else a.max()
    s = np.float32(np.nan) if np.isnan(amax) else max(amax, np.float32(1e-12))
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        x = (m / s).astype(np.float32)
    x[np.isnan(x)] = np.float32(np.nan)
    return x


def adversarial_blocks():
    rng = np.random.default_rng(0)
    levels = np.array(q.CODEBOOK_VALUES[q.CB_DYN4], dtype=np.float32)
    yield np.zeros(128, np.float32)
    yield np.full(128, np.nan, np.float32)
    yield np.full(128, np.inf, np.float32)
    b = rng.standard_normal(128).astype(np.float32)
    b[::7] = np.nan
    yield b
    b = rng.standard_normal(128).astype(np.float32)
    b[3] = -np.inf
    yield b
    yield np.full(128, np.float32(3e38))
    yield np.full(128, np.float32(1e-45))          # the smallest subnormal: s = 1e-12, x underflows
    yield np.tile(levels, 8)                       # every level exactly, scale 1 (idx 0 .. 15)
    yield np.tile(levels, 8) * np.float32(2.0 ** -100)
    yield np.concatenate([np.ones(1, np.float32), np.full(127, np.float32(1 - 2 ** -24))])


@pytest.mark.parametrize("k", range(10))
def test_adversarial_blocks_index_in_range(luts, k):
    m = list(adversarial_blocks())[k]
    for signed, blocks in ((False, [np.abs(m), np.maximum(m, 0)]), (True, [m, -m])):
        for v in blocks:
            x = kernel_x(v)
            for cb in range(5):
                idx = idx_of(luts, LUT_LEVELS[cb], x, signed)
                assert idx.min() >= 0 and idx.max() <= N_PAIRS - 1
                code = idx_of(luts, LUT_RTN[cb], x, signed)
                assert code.min() >= 0 and code.max() < N_LEVELS
            # the lookahead encode clamps x to [0, 1] (NaN kept) before its bucket
            xl = np.where(np.isnan(x), x, np.clip(x, 0, 1)).astype(np.float32)
            idx = idx_of(luts, LUT_LEVELS[_lib.CB_DYN4], xl, False)
            assert idx.max() <= N_PAIRS - 1
            assert np.maximum(idx - 1, 0).max() < N_LEVELS


def test_fixed_lane_indices_stay_in_their_arrays():
    """Indices that depend on the lane only (update_sr_tables, the code stage, decode4)."""
    j = np.arange(8)
    h = np.arange(2)[:, None]
    pre = j + 8 * h                     # usr_level_preconds: the 16 levels, two per lane
    entry = 1 + j + 8 * h               # update-SR entries 1..16, two per lane (entry 0: lane 0)
    assert pre.min() == 0 and pre.max() == N_LEVELS - 1 and len(np.unique(pre)) == N_LEVELS
    assert entry.min() == 1 and entry.max() == N_PAIRS - 1 and len(np.unique(entry)) == N_PAIRS - 1
    qq = np.arange(4)[:, None]
    word = 8 * qq + j                   # a lane's code word of quarter q
    assert word.min() == 0 and word.max() == N_STAGE - 1 and len(np.unique(word)) == N_STAGE
    assert (4 * j + 3).max() == N_STAGE - 1   # lane j stores words 4j .. 4j + 3 as one 8-byte piece
    w = np.arange(1 << 16, dtype=np.uint32)     # a 16-bit code word: two decode-table bytes
    assert (w & 0xFF).max() < N_DEC and ((w >> 8) & 0xFF).max() < N_DEC
    # searchsorted pairs as the library builds them: lo = max(i - 1, 0), hi = min(i, 15)
    i = np.arange(N_PAIRS)
    assert np.maximum(i - 1, 0).max() < N_LEVELS and np.minimum(i, 15).max() < N_LEVELS
