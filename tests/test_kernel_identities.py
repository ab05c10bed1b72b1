"""Arithmetic shortcuts of the step kernel, checked exhaustively on the CPU (no GPU).

The decayed parameter of a 16-bit parameter is p * fp32(1 - lr*wd) computed in fp32 and rounded
to the parameter's dtype (ATen's ``p.mul_(1 - lr*wd)`` on a bf16 / fp16 tensor,
``_optimized.py:215``).  The kernel skips that product and its rounding when
1 - 2^-9 < decay <= 1 (bf16) or 1 - 2^-12 < decay <= 1 (fp16): every 16-bit value then rounds
back to itself.  Checked here over every finite bf16 / fp16 bit pattern, at the decays next to
the bounds, with torch's own conversions; the bounds are tight (one step past them changes a
value)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

F32 = np.float32

BOUNDS = {torch.bfloat16: 1.0 - 2.0 ** -9, torch.float16: 1.0 - 2.0 ** -12}


def all_finite(dtype):
    """Every finite value of a 16-bit dtype, as that dtype."""
    v = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(dtype)
    return v[torch.isfinite(v.float())]


def decayed(p, decay):
    """fp32(p * decay) rounded to p's dtype, as ATen computes p.mul_(decay) for a 16-bit p."""
    return (p.float() * torch.tensor(decay, dtype=torch.float32)).to(p.dtype)


def decays_above(bound, n=64):
    """The n fp32 decays just above the bound, 1.0 itself and a few in between."""
    lo = np.nextafter(F32(bound), F32(2))
    ups = [lo]
    for _ in range(n - 1):
        ups.append(np.nextafter(ups[-1], F32(2)))
    mid = np.linspace(bound, 1.0, 50)[1:].astype(F32)
    return [float(d) for d in ups] + [float(d) for d in mid] + [1.0]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decay_within_the_bound_leaves_every_16_bit_parameter_unchanged(dtype):
    p = all_finite(dtype)
    for d in decays_above(BOUNDS[dtype]):
        assert float(F32(d)) > BOUNDS[dtype] and d <= 1.0
        out = decayed(p, d)
        same = out.view(torch.int16) == p.view(torch.int16)
        # -0 * decay and +0 * decay keep their signs; every other value too
        assert bool(same.all()), (dtype, d, p[~same][:4], out[~same][:4])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_the_decay_bound_is_tight(dtype):
    """Planted: at the bound itself half-way cases appear, and one fp32 step below it a value
    that is a power of two rounds down, so a looser bound would change parameters."""
    p = all_finite(dtype)
    below = float(np.nextafter(F32(BOUNDS[dtype]), F32(0)))
    out = decayed(p, below)
    assert bool((out.view(torch.int16) != p.view(torch.int16)).any())
