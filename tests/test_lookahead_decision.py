"""The kernel's quick lookahead update-SR decision against the reference's float64 rule (no GPU).

The lookahead rule (``quantize_dyn4_la_upd_sr``, ``quantization.py:779-895``) picks the lower
level with probability P, computed in float64 from the pending value z, its level pair
q_lo = s*a, q_hi = s*b and the next step's second moments n(q) = beta2*q + fresh:
P = (p(z) - p(q_hi)) / (p(q_lo) - p(q_hi)), p = 1 / (sqrt(n / bias) + eps), with a value-linear
fallback where the interval is flat.  With r = sqrt(n) and E = r / sqrt(bias) + eps the same P
is, exactly, N / D with N = (q_hi - z) (r_hi + r_lo) E_lo and D = (q_hi - q_lo) (r_hi + r_z) E_z:
positive factors without cancellation.  The kernel evaluates N and D in fp32 and, without a
division, decides by the sign of T = u D - N where |T| exceeds the band
2^-16 max(N, D) + 2^-46 M D (that is, |u - P| > 2^-16 max(1, P) + 2^-46 M, with
M = max(p_lo, 1) / (p_lo - p_hi), whose product with D needs no division either: the reference's
own float64 rounding grows with M), and sends every other value, and every value with
M >= 2^36 (near the reference's flat switch at 1e12) or n_lo below 2^-100 (where fp32 loses small
terms, and p_lo = +inf makes the reference's flat test true), to the float64 rule.  This test
restates the quick form in numpy fp32 -- the fresh term as the kernel forms it,
fp32(1 - beta2) * g * g, with gradients whose square underflows in fp32, its faithful operations
one ulp off either way, 1/sqrt(bias) three ulps off and sqrt(bias)/beta2 four -- and checks that
wherever it is sure it agrees with the float64 rule; draws sit on both sides of the reference's
probability, within 4096 units of 2^-24, where a band 64 times narrower disagrees (planted
below)."""

from __future__ import annotations

import numpy as np
import pytest

from adamw4bit_amd import quantization as q

F32 = np.float32
F64 = np.float64


def jitter(v, k):
    """v (fp32) moved by k ulps where finite and positive."""
    k = np.where(np.isfinite(v) & (v > 0), k, 0)
    return (v.view(np.int32) + k.astype(np.int32)).view(F32)


def fma32(a, b, c):
    return (a.astype(F64) * b.astype(F64) + c.astype(F64)).astype(F32)


def reference_prob_lo(z, a, b, s, fresh, beta2, bias, eps):
    """quantization.py:866-893 in float64 (numpy's float64 operations are IEEE, as ATen's)."""
    s64, z64 = s.astype(F64), z.astype(F64)
    q_lo, q_hi = s64 * a.astype(F64), s64 * b.astype(F64)
    n_lo = np.maximum(beta2 * q_lo + fresh, 0.0)
    n_ref = np.maximum(beta2 * z64 + fresh, 0.0)
    n_hi = np.maximum(beta2 * q_hi + fresh, 0.0)
    p_lo = 1.0 / (np.sqrt(n_lo / bias) + eps)
    p_ref = 1.0 / (np.sqrt(n_ref / bias) + eps)
    p_hi = 1.0 / (np.sqrt(n_hi / bias) + eps)
    denom, width = p_lo - p_hi, q_hi - q_lo
    raw = (p_ref - p_hi) / np.maximum(denom, 1e-300)
    fallback = 1.0 - np.clip((z64 - q_lo) / np.maximum(width, 1e-300), 0.0, 1.0)
    degenerate = width <= 0.0
    flat = (~degenerate) & (np.abs(denom) <= 1e-12 * np.maximum(np.maximum(np.abs(p_lo), np.abs(p_hi)), 1.0))
    p = np.where(flat, fallback, raw)
    p = np.where(degenerate, 1.0, p)
    return np.clip(p, 0.0, 1.0)


def quick(z, a, b, s, g, beta2, bias, eps, U, rng, band_scale=1.0):
    """The kernel's fp32 form with its rounding perturbed; returns (lower, sure)."""
    n = len(z)
    jit = lambda: rng.integers(-1, 2, n)  # noqa: E731
    fresh32 = ((F32(1.0 - beta2) * g).astype(F32) * g).astype(F32)  # fp32(1 - beta2) * g * g
    beta32 = np.full(n, beta2, F32)
    rb = jitter(np.full(n, 1.0 / np.sqrt(bias), F32), rng.integers(-3, 4, n))
    eps32 = np.full(n, eps, F32)
    q_lo, q_hi = (s * a).astype(F32), (s * b).astype(F32)
    n_lo, n_hi, n_z = fma32(beta32, q_lo, fresh32), fma32(beta32, q_hi, fresh32), fma32(beta32, z, fresh32)
    r_lo, r_hi, r_z = (jitter(np.sqrt(v.astype(F64)).astype(F32), jit()) for v in (n_lo, n_hi, n_z))
    e_lo, e_hi, e_z = fma32(r_lo, rb, eps32), fma32(r_hi, rb, eps32), fma32(r_z, rb, eps32)
    d_hi = fma32(s, b, -z)
    w = (s * (b - a).astype(F32)).astype(F32)
    s_lo = (r_hi + r_lo).astype(F32)
    sz_ez = ((r_hi + r_z).astype(F32) * e_z).astype(F32)
    num = ((d_hi * s_lo).astype(F32) * e_lo).astype(F32)
    den = (w * sz_ez).astype(F32)
    # M D = (r_hi + r_lo) E_hi max(1, E_lo) (r_hi + r_z) E_z sqrt(bias) / beta2 (the width cancels)
    sb = jitter(np.full(n, np.sqrt(bias) / beta2, F32), rng.integers(-4, 5, n))
    md = ((((s_lo * e_hi).astype(F32) * np.maximum(e_lo, F32(1))).astype(F32) * sz_ez).astype(F32) * sb).astype(F32)
    u = (U * F32(2.0 ** -24)).astype(F32)
    t = fma32(u, den, -num)
    band = fma32(np.full(n, 2.0 ** -16 * band_scale, F32), np.maximum(num, den), (F32(2.0 ** -46) * md).astype(F32))
    # n_lo below 2^-100 (fp32 loses small terms; p_lo = +inf when it is 0 with eps = 0, which
    # makes the reference's flat test true): the float64 rule
    sure = (np.abs(t) > band) & (md < (F32(2.0 ** 36) * den).astype(F32)) & (n_lo >= F32(2.0 ** -100))
    return t < 0, sure


def sample(rng, n):
    cb = np.array(q.CODEBOOK_VALUES[q.CB_DYN4], dtype=F32)
    idx = rng.integers(1, 16, n)
    a, b = cb[idx - 1], cb[idx]
    s = (10.0 ** rng.uniform(-10, 0, n)).astype(F32)
    t = rng.random(n)
    mode = rng.integers(0, 4, n)
    t = np.where(mode == 0, 1 - rng.random(n) * 1e-4, np.where(mode == 1, rng.random(n) * 1e-4, t))
    x = np.clip((a.astype(F64) + t * (b - a).astype(F64)).astype(F32), np.nextafter(a, F32(2)), b)
    z = (x.astype(F64) * s).astype(F32)
    beta2 = float(rng.choice([0.95, 0.999, 0.9, 0.45]))
    bias = float(rng.choice([1.0, 0.0975, 0.5, 1e-3, 0.999]))
    eps = float(rng.choice([1e-8, 1e-6, 0.0, 1e-12]))
    # the fresh term spans orders of magnitude around beta2 * q (where it decides P's shape)
    g = (np.sqrt(s.astype(F64)) * 10.0 ** rng.uniform(-4, 2, n)).astype(F32)
    g = np.where(rng.random(n) < 0.05, F32(0), g)
    g = np.where(rng.random(n) < 0.01, (g.astype(F64) * 1e-20).astype(F32), g)  # fp32 g*g underflows
    return z, a, b, s, g, beta2, bias, eps


def fresh64(g, beta2):
    """The reference's fresh term (1 - beta2) * g^2 in float64."""
    return (1.0 - beta2) * g.astype(F64) ** 2


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_quick_lookahead_decision_is_the_reference_decision_wherever_it_is_sure(seed):
    rng = np.random.default_rng(seed)
    unsure = total = 0
    for _ in range(4):
        z, a, b, s, g, beta2, bias, eps = sample(rng, 200_000)
        with np.errstate(all="ignore"):
            p = reference_prob_lo(z, a, b, s, fresh64(g, beta2), beta2, bias, eps)
            near = np.clip(np.round(p * 2.0 ** 24) + rng.integers(-4096, 4097, len(z)), 0, (1 << 24) - 1)
            uniform = rng.random(len(z)) < 0.5
            U = np.where(uniform, rng.integers(0, 1 << 24, len(z)), near).astype(F32)
            lower, sure = quick(z, a, b, s, g, beta2, bias, eps, U, rng)
        ref_lower = (U.astype(F64) * 2.0 ** -24) < p
        bad = sure & (lower != ref_lower)
        assert not bad.any(), (seed, int(bad.sum()), beta2, bias, eps)
        # the rate with uniform draws, away from the zero level (where zero and underflowing
        # gradients, drawn on purpose here, leave n_lo below 2^-100)
        regular = uniform & (a > 0)
        unsure += int((~sure & regular).sum())
        total += int(regular.sum())
    assert unsure / total < 2e-3, unsure / total


def test_a_narrower_lookahead_band_would_be_wrong():
    """Planted mistake: the band 64 times narrower disagrees with the reference somewhere."""
    rng = np.random.default_rng(9)
    bad_total = 0
    for _ in range(4):
        z, a, b, s, g, beta2, bias, eps = sample(rng, 200_000)
        with np.errstate(all="ignore"):
            p = reference_prob_lo(z, a, b, s, fresh64(g, beta2), beta2, bias, eps)
            U = np.clip(np.round(p * 2.0 ** 24) + rng.integers(-64, 65, len(z)), 0, (1 << 24) - 1).astype(F32)
            lower, sure = quick(z, a, b, s, g, beta2, bias, eps, U, rng, band_scale=1 / 64)
        bad_total += int((sure & (lower != ((U.astype(F64) * 2.0 ** -24) < p))).sum())
    assert bad_total > 0
