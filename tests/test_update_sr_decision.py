"""The kernel's update-SR decision rule against the reference's arithmetic (no GPU).

Update-SR (``_compiled_quantization.py:74-109``) picks the lower level with probability
P = (f(x) - f(b)) / (f(a) - f(b)), f(l) = 1 / (sqrt((s * l) / bias) + eps), every step rounded
in fp32.  The kernel decides most values with a rounded form of the exact identity
u < P  <=>  Q = (sqrt(b) - sqrt(x)) - u * g * E(x) > 0,  E(l) = c * sqrt(l) + eps,
c = sqrt(s / bias), g = (sqrt(b) - sqrt(a)) / E(a), and sends every value with |Q| inside its
band 2^-18 * sqrt(b) + 2^-19 * eps / c to the reference's own operations.  This test restates
that quick test in numpy fp32 -- with the hardware's faithful square roots and reciprocals
taken one ulp off in either direction -- and checks on random blocks, intervals, values and
draws that wherever it is sure, its decision equals the reference's, whether the host's
square root is correctly rounded or one ulp low (ATen's CPU sqrt is one or the other).
Half the draws sit within 4096 units of 2^-24 of the reference's own probability, where a
band 16 times narrower decides wrongly (planted below)."""

from __future__ import annotations

import numpy as np
import pytest

from adamw4bit_amd import quantization as q

F32 = np.float32


def ulp_shift(v, k):
    """v moved by k ulps (k in {-1, 0, 1}, elementwise) where v is positive and finite."""
    k = np.where(np.isfinite(v) & (v > 0), k, 0)
    return (v.view(np.int32) + k.astype(np.int32)).view(F32)


def fma32(a, b, c):
    """fp32 fused multiply-add via float64 (exact products; double rounding is vanishingly rare)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(F32)


def sqrt_cr(v):
    return np.sqrt(v.astype(np.float64)).astype(F32)


def reference_lower(s, bias, eps, a, b, x, u, host_low):
    """The reference's valid flag and its decision u < P, with the host's sqrt correctly rounded
    or (host_low) one ulp below where the root is not exact."""
    valid, p = reference_probability(s, bias, eps, a, b, x, host_low)
    return valid, u < p


def reference_probability(s, bias, eps, a, b, x, host_low):
    def f(l):
        v = np.maximum((s * l) / bias, F32(0))
        r = sqrt_cr(v)
        exact = r.astype(np.float64) ** 2 == v.astype(np.float64)
        r = np.where(host_low & ~exact & (r > 0), ulp_shift(r, -np.ones_like(r.view(np.int32))), r)
        return F32(1) / (r + eps)
    fa, fb, fx = f(a), f(b), f(x)
    den = fa - fb
    valid = (b > a) & (den > 0)
    return valid, (fx - fb) / np.maximum(den, F32(1e-30))


def quick(s, bias, eps, a_idx, b_idx, x, U, cb, rng, band_scale=1.0):
    """The kernel's quick test with random one-ulp errors in its faithful operations; returns
    (lower, sure, certain)."""
    n = len(x)
    jit = lambda: rng.integers(-1, 2, n)  # noqa: E731
    sq = np.where(cb > 0, np.sqrt(np.maximum(cb, 0).astype(np.float64)), 0).astype(F32)
    gap = (np.sqrt(cb[b_idx].astype(np.float64)) - np.sqrt(cb[a_idx].astype(np.float64))).astype(F32)
    bias_rcp = (F32(1) / bias).astype(F32)
    c = ulp_shift(sqrt_cr(s * bias_rcp), jit())
    c_rcp = ulp_shift((F32(1) / c).astype(F32), jit())
    e_lo = fma32(c, sq[a_idx], eps)
    e_hi = fma32(c, sq[b_idx], eps)
    g = np.where(e_lo > 0, (gap * F32(2.0 ** -24)) * ulp_shift((F32(1) / e_lo).astype(F32), jit()),
                 np.inf).astype(F32)
    w = ulp_shift(sqrt_cr(x), jit() * (x > 0))
    ex = fma32(c, w, eps)
    qv = fma32(-U, (g * ex).astype(F32), (sq[b_idx] - w).astype(F32))
    # the value's band: 2^-18 sqrt(b) + 2^-19 eps / c (the kernel's per-value form)
    band0 = (F32(2.0 ** -19 * band_scale) * (eps * c_rcp).astype(F32)).astype(F32)
    band = fma32(sq[b_idx], np.full(n, 2.0 ** -18 * band_scale, F32), band0)
    # a NaN Q counts as sure: a zero draw where g = +inf (E(a) = 0), whose P is 0
    # the block's intervals are all certain when c * gap > 2^-20 * E(b) for each; here the
    # value's own interval stands in (a block where any is uncertain decides exactly anyway)
    certain = (c * gap).astype(F32) > (F32(2.0 ** -20) * e_hi).astype(F32)
    return qv > 0, ~(np.abs(qv) <= band), certain


def sample(rng, n, codebook):
    cb = np.array(codebook, dtype=F32)
    idx = rng.integers(1, 16, n)  # searchsorted index: a = cb[idx - 1] < x <= b = cb[idx]
    a, b = cb[idx - 1], cb[idx]
    # values near either level, near the middle, and uniform over the interval
    t = rng.random(n)
    mode = rng.integers(0, 4, n)
    t = np.where(mode == 0, 1 - rng.random(n) * 1e-4, np.where(mode == 1, rng.random(n) * 1e-4, t))
    x = (a.astype(np.float64) + t * (b - a).astype(np.float64)).astype(F32)
    x = np.clip(x, np.nextafter(a, F32(2)), b).astype(F32)
    s = (10.0 ** rng.uniform(-12, 3, n)).astype(F32)
    bias = rng.choice(np.array([1.0, 0.0975, 0.5, 0.9, 1e-12, 0.2649], dtype=F32), n)
    eps = rng.choice(np.array([1e-8, 1e-6, 1e-12, 0.0, 1e-3], dtype=F32), n)
    # draws on both sides of the reference's own probability, where a band too narrow would
    # decide wrongly (half of them), and uniform draws (the other half)
    with np.errstate(all="ignore"):
        _, p = reference_probability(s, bias, eps, a, b, x, False)
    near = np.clip(np.round(np.nan_to_num(p, nan=0.5) * 2.0 ** 24) + rng.integers(-4096, 4097, n), 0, (1 << 24) - 1)
    uniform = rng.random(n) < 0.5
    U = np.where(uniform, rng.integers(0, 1 << 24, n), near).astype(F32)
    return cb, idx - 1, idx, a, b, x, s, bias, eps, U, uniform


@pytest.mark.parametrize("codebook", ["dyn4", "lin4"])
def test_quick_decision_is_the_reference_decision_wherever_it_is_sure(codebook):
    rng = np.random.default_rng(11 if codebook == "dyn4" else 12)
    cb_values = q.CODEBOOK_VALUES[q.CB_DYN4 if codebook == "dyn4" else q.CB_LIN4]
    unsure = total = 0
    for _ in range(6):
        with np.errstate(all="ignore"):
            cb, a_idx, b_idx, a, b, x, s, bias, eps, U, uniform = sample(rng, 400_000, cb_values)
        u = (U * F32(2.0 ** -24)).astype(F32)
        with np.errstate(all="ignore"):
            lower, sure, certain = quick(s, bias, eps, a_idx, b_idx, x, U, cb, rng)
        for host_low in (False, True):
            with np.errstate(all="ignore"):
                valid, ref_lower = reference_lower(s, bias, eps, a, b, x, u, host_low)
            decided = sure & certain & valid
            bad = decided & (lower != ref_lower)
            assert not bad.any(), (codebook, host_low, int(bad.sum()), x[bad][:4], s[bad][:4], U[bad][:4])
            # certain intervals are valid for the reference
            assert not (certain & ~valid).any(), (codebook, host_low)
        unsure += int((~sure & certain & uniform).sum())
        total += int(uniform.sum())
    # with uniform draws the band leaves few values to the exact path (these samples still crowd
    # the levels, where the band is widest in draw units)
    assert unsure / total < 2e-3, unsure / total


def test_a_narrower_band_would_be_wrong():
    """Planted mistake: the same check with the band 16 times narrower finds disagreements, so
    the check has the power to see a band that is too small."""
    rng = np.random.default_rng(13)
    bad_total = 0
    for _ in range(4):
        with np.errstate(all="ignore"):
            cb, a_idx, b_idx, a, b, x, s, bias, eps, U, uniform = sample(rng, 400_000, q.CODEBOOK_VALUES[q.CB_DYN4])
            u = (U * F32(2.0 ** -24)).astype(F32)
            lower, sure, certain = quick(s, bias, eps, a_idx, b_idx, x, U, cb, rng, band_scale=1 / 16)
            valid, ref_lower = reference_lower(s, bias, eps, a, b, x, u, True)
        bad_total += int((sure & certain & valid & (lower != ref_lower)).sum())
    assert bad_total > 0


@pytest.mark.parametrize("codebook", ["dyn4", "lin4"])
def test_a_value_at_its_upper_level_is_never_decided_lower(codebook):
    """Where every value of a quarter is sure, the kernel forms code = idx - lower without the
    guards: x at its upper level b must then come out upper (the guard x >= b, and P = 0 there),
    whatever the draw and the one-ulp errors of the faithful operations."""
    rng = np.random.default_rng(14 if codebook == "dyn4" else 15)
    cb_values = q.CODEBOOK_VALUES[q.CB_DYN4 if codebook == "dyn4" else q.CB_LIN4]
    for _ in range(4):
        with np.errstate(all="ignore"):
            cb, a_idx, b_idx, a, b, x, s, bias, eps, U, uniform = sample(rng, 400_000, cb_values)
            U = np.where(rng.random(len(x)) < 0.1, F32(0), U).astype(F32)  # zero draws too
            lower, sure, certain = quick(s, bias, eps, a_idx, b_idx, b.copy(), U, cb, rng)
        assert not (sure & certain & lower).any(), codebook


def test_certainty_products_stay_normal_for_every_codebook():
    """The update-SR table build compares c * gap * 2^-24 with 2^-44 * E(b) instead of c * gap with
    2^-20 * E(b).  Scaling both sides by 2^-24 leaves the comparison exact only while neither
    product is subnormal: for every codebook's real intervals (b > a >= 0) and the smallest block
    factor c = sqrt(1e-12 / bias) >= 1e-6, both stay normal."""
    tiny = np.finfo(F32).tiny
    c = F32(1e-6)
    for cbid in q.CODEBOOK_VALUES:
        cb = np.array(q.CODEBOOK_VALUES[cbid], dtype=F32)
        a, b = cb[:-1], cb[1:]
        real = (a >= 0) & (b > a)
        if not real.any():
            continue
        gap = (np.sqrt(b[real].astype(np.float64)) - np.sqrt(a[real].astype(np.float64))).astype(F32)
        gap_s = (gap * F32(2.0 ** -24)).astype(F32)
        assert (gap_s.astype(np.float64) == gap.astype(np.float64) * 2.0 ** -24).all(), cbid  # exact scaling
        assert (c * gap_s >= tiny).all(), cbid
        e_hi = (c * np.sqrt(b[real].astype(np.float64)).astype(F32)).astype(F32)  # E(b) >= c * sqrt(b) (eps >= 0)
        assert ((F32(2.0 ** -44) * e_hi).astype(F32) >= tiny).all(), cbid
