"""The per-step fp32 constants of a launch-table row (``_StepConstants``), restated with numpy's
float32 rounding: the reference computes them in float64 and ATen rounds each to fp32 where the
kernels use it (``_optimized.py:168-173``, ``_optimized_quantization.py:66-67``); the float64
decay and step coefficient of float64 parameters are the float64 values themselves.  The
hyperparameter part is cached per group setting; a tensor-valued learning rate is not cached."""

import math

import numpy as np
import pytest
import torch

from adamw4bit_amd import _lib
from adamw4bit_amd.adamw import _HYPER_CACHE, _StepConstants

F32 = np.float32


def expected(lr, betas, eps, wd, step, next_bias):
    b1, b2 = betas
    bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
    storage = 1 - b2 ** (step + 1) if next_bias else bc2
    w1, w2 = F32(1 - b1), F32(1 - b2)
    flags = 0
    if not abs(w1) < 0.5:
        flags |= _lib.TENSOR_LERP1_LARGE
        w1 = F32(w1 - F32(1))
    if not abs(w2) < 0.5:
        flags |= _lib.TENSOR_LERP2_LARGE
        w2 = F32(w2 - F32(1))
    bc2_sqrt = F32(math.sqrt(bc2))
    sr_bias = F32(max(storage, 1e-12))
    return dict(lerp_flags=flags, w1=float(w1), w2=float(w2), decay=float(F32(1 - lr * wd)),
                step_coef=float(F32(-lr / bc1)), bc2_sqrt=float(bc2_sqrt),
                bc2_sqrt_rcp=float(F32(1.0 / float(bc2_sqrt))), eps=float(F32(eps)),
                decay_f64=1 - lr * wd, step_coef_f64=-lr / bc1,
                m2=(float(sr_bias), float(F32(1.0 / float(sr_bias))), float(F32(eps))))


@pytest.mark.parametrize("betas", [(0.9, 0.95), (0.9, 0.999), (0.3, 0.45), (0.5, 0.6)])
@pytest.mark.parametrize("lr,wd,eps", [(1e-3, 0.1, 1e-8), (3e-4, 0.0, 1e-6), (0.1, 0.01, 0.0)])
def test_step_constants_are_the_reference_roundings(betas, lr, wd, eps):
    group = dict(betas=betas, lr=lr, weight_decay=wd, eps=eps)
    for step in (1, 2, 7, 100, 10_000):
        for scheme, next_bias in (("dyn4_nz", False), ("dyn4_upd_sr_fp32read_nextbc", True)):
            for _ in range(2):  # computed, then from the hyperparameter cache
                c = _StepConstants(group, step, scheme)
                want = expected(lr, betas, eps, wd, step, next_bias)
                got = {k: getattr(c, k) for k in want if k != "m2"}
                got["m2"] = c.m2_sr_values()
                assert got == want, (betas, lr, step, scheme)
    assert (betas[0], betas[1], lr, wd, eps) in _HYPER_CACHE


def test_tensor_learning_rate_is_not_cached():
    lr = torch.tensor(1e-3, dtype=torch.float64)
    group = dict(betas=(0.9, 0.95), lr=lr, weight_decay=0.1, eps=1e-8)
    before = len(_HYPER_CACHE)
    a = _StepConstants(group, 3, "dyn4_nz")
    lr.fill_(2e-3)  # a scheduler changing the tensor in place
    b = _StepConstants(group, 3, "dyn4_nz")
    assert len(_HYPER_CACHE) == before
    assert a.decay == float(F32(1 - 1e-3 * 0.1)) and b.decay == float(F32(1 - 2e-3 * 0.1))
    assert b.step_coef_f64 == -2e-3 / (1 - 0.9 ** 3)
