"""Shared helpers for the GPU tests: build the drop-in optimizer from a fixture
configuration, replay draws, compare states with the oracle."""

from __future__ import annotations

import json
import os

import numpy as np
import torch

import adamw4bit_amd as aw
from adamw4bit_amd import _lib
from oracle import philox
from oracle import reference_step as ref

DEVICE = "cuda"
PARAM_RTOL = 1e-6


def heavy_tailed(shape, gen, row_mu=-7.0, row_sigma=1.0):
    """Student-t(3) values times per-row log-normal magnitudes (fixed generator)."""
    z = torch.randn(shape, generator=gen)
    chi2 = (torch.randn((3,) + tuple(shape), generator=gen) ** 2).sum(0)
    t = z / torch.sqrt(chi2 / 3.0)
    rows = shape[0] if len(shape) > 1 else 1
    scale = torch.exp(row_mu + row_sigma * torch.randn(rows, generator=gen))
    return t * (scale.view(-1, *([1] * (len(shape) - 1))) if len(shape) > 1 else scale)


def build_optimizer(cfg, params):
    """The drop-in optimizer configured like a golden-fixture run."""
    hp = cfg["hyper"]
    kw = dict(lr=hp["lr"], betas=tuple(hp["betas"]), eps=hp["eps"], weight_decay=hp["weight_decay"],
              optimized=cfg["optimized"], quant_rng_seed=cfg["seed"])
    name = cfg["optimizer"]
    if name == "ZEEDENAdamW4Bit":
        opt = aw.ZEEDENAdamW4Bit(params, **kw)
    elif name == "ZIPSRAdamW4Bit":
        opt = aw.ZIPSRAdamW4Bit(params, **kw)
    else:
        groups = [dict(params=[p], m1_quant_scheme=e["m1"], m2_quant_scheme=e["m2"], use_eden_m2=e["eden"])
                  for p, e in zip(params, cfg["per_param"])]
        opt = aw.QuantizedAdamW(groups, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz", **kw)
    if cfg["optimized"]:
        for g in opt.param_groups:
            g["max_chunk_numel"] = cfg["chunk"]
    if cfg.get("m1_override"):
        idx, scheme = cfg["m1_override"]
        opt.set_m1_quant_scheme_for_parameters([params[j] for j in idx], scheme)
    return opt


class LoggedDraws:
    """Draw provider replaying the uniforms an oracle run recorded, write by write."""

    def __init__(self, oracle: ref.Oracle, params):
        # The oracle draws chunk by chunk; the device draws a whole write at once.
        per_write = {}
        for entry in oracle.draw_log:
            per_write.setdefault((entry.param, entry.moment, entry.step), []).append(entry.draws)
        self.queues = {}
        for (param, moment, step) in sorted(per_write):
            self.queues.setdefault((param, moment), []).append(torch.cat(per_write[(param, moment, step)]))
        self.index = {id(p): i for i, p in enumerate(params)}

    def __call__(self, p, moment, n, device):
        draws = self.queues[(self.index[id(p)], moment)].pop(0)
        assert draws.numel() == n
        return draws.to(device)


class PhiloxMirror:
    """Oracle draw_fn replaying the device's Philox streams (same seeds, same positions)."""

    def __init__(self, optimizer: aw.QuantizedAdamW, device):
        self.opt = optimizer
        self.device = torch.device(device)
        self.offsets = {"m1": 0, "m2": 0}

    def __call__(self, moment, n):
        seed = self.opt._stream(moment, self.device).seed
        off = self.offsets[moment]
        self.offsets[moment] = off + (n + 127) // 128 * 128
        return torch.from_numpy(philox.uniforms(seed, off, n))


def state_of(opt, p):
    st = opt.state[p]
    out = {"step": st["step"]}
    for m in ("m1", "m2"):
        if m == "m2" and "lookahead_pending_exp_avg_sq" in st:
            out["m2_pending"] = st["lookahead_pending_exp_avg_sq"].cpu()
        elif f"{m}_code" in st:
            out[f"{m}_code"] = st[f"{m}_code"].cpu()
            out[f"{m}_scale"] = st[f"{m}_quant_state"].absmax.cpu()
        else:
            out[f"{m}_fp32"] = st[m].cpu()
    return out


def oracle_state(ms_pair):
    st = {}
    for name, ms in zip(("m1", "m2"), ms_pair):
        if ms.scheme == "fp32":
            st[f"{name}_fp32"] = ms.values.clone()
        elif ms.scheme in ref.PENDING_LOOKAHEAD_SCHEMES:
            st[f"{name}_pending"] = ms.values.clone()
        else:
            st[f"{name}_code"] = ms.codes.clone()
            st[f"{name}_scale"] = ms.scales.clone()
    return st


def bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().cpu().contiguous()
    return t.view({8: torch.int64, 4: torch.int32, 2: torch.int16, 1: torch.uint8}[t.element_size()])


# Parameter bars.  The kernel's parameter update is faithful (hardware square root and reciprocal)
# and the reference's CPU square root is faithful too, so an update term may differ from the
# oracle's by a few of its own ulps, and a parameter by one rounding of the sum.  Measured over
# every comparison of the GPU suite (2,242 tensors) before these bars were set:
# * 16-bit parameters: every value within one storage ulp per step of the oracle's (the ulp
#   distance of the bit patterns), or within one storage ulp of the tensor's rms magnitude: where
#   the update nearly cancels a parameter, or the value is small enough for fine ulps, a few ulps
#   of the update term are many ulps of the result (measured: at most 5.6e-4 * rms, for fp16,
#   whose ulp at the rms is 9.8e-4 * rms).  At most F16_NOT_EXACT per step (plus one) of them
#   not bit-exact (measured at most 9.8e-4 per step; 0 in most tensors);
# * fp32 parameters: every value within FP32_SCALE_RTOL of the parameter scale, |got - expect| <=
#   5e-7 * (|expect| + rms(expect)) (measured at most 4.02e-7), and at most FP32_BEYOND_REL (plus
#   three) of them beyond a pure 1e-6 relative error |got - expect| <= 1e-6 |expect| (values near
#   zero, where the update term's last bits are a larger share; measured at most 5.5%, median
#   0.24%, more where the step size is large against the parameters).
# * float64 parameters: the update term is computed in float64 from the same fp32 moments, and
#   differs from the oracle's only through the fp32 denominator's faithful square root (ATen's and
#   the hardware's round differently on a few percent of inputs); every value within
#   FP64_SCALE_RTOL of the parameter scale.
F16_NOT_EXACT = 2e-3
FP32_SCALE_RTOL = 5e-7
FP32_BEYOND_REL = 0.05
FP64_SCALE_RTOL = 5e-7
# Relative size of one storage ulp of 16-bit values (7 / 10 explicit mantissa bits).
ULP16 = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def ulp_distance16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units in the last place between two 16-bit tensors of one dtype (+0 == -0)."""
    def ordered(t):
        v = bits(t).to(torch.int32)  # sign-extended bit patterns
        return torch.where(v < 0, -(v & 0x7FFF), v)
    return (ordered(a) - ordered(b)).abs()


# AW4_PARAM_STATS=path appends each comparison's statistics to path (JSON lines); with
# AW4_PARAM_STATS_COLLECT=1 as well, only the per-value bars are asserted (a run that measures the
# budgets' statistics over every test).
_COLLECT = bool(os.environ.get("AW4_PARAM_STATS_COLLECT"))


def _record(what: str, stats: dict) -> None:
    path = os.environ.get("AW4_PARAM_STATS")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"what": what, **stats}) + "\n")


def assert_params_close(got: torch.Tensor, expect: torch.Tensor, what: str, rtol: float = PARAM_RTOL,
                        steps: int = 1, exclude: torch.Tensor = None) -> float:
    """Parameters within the bars above after `steps` steps.  `exclude` (bool, one per value) drops
    values whose stochastic codes took the other level at some step (their trajectories
    legitimately part).  Returns the bit-exact fraction."""
    got = got.detach().cpu().reshape(-1)
    expect = expect.detach().cpu().reshape(-1)
    keep = torch.ones(expect.numel(), dtype=torch.bool) if exclude is None else ~exclude.reshape(-1)
    n = int(keep.sum())
    exact_mask = bits(got) == bits(expect)
    exact = float(exact_mask.double().mean())
    stats = {"dtype": str(got.dtype), "n": n, "steps": steps, "exact": exact}
    if got.dtype in (torch.bfloat16, torch.float16):
        d = ulp_distance16(got, expect)[keep]
        stats.update(max_ulps=int(d.max()) if n else 0, not_exact=int((d > 0).sum()))
        far = d > steps
        if bool(far.any()):
            e = expect.double()[keep]
            err = (got.double()[keep] - e).abs()
            rms = float(e.pow(2).mean().sqrt())
            stats.update(far=int(far.sum()), far_err_rms=float(err[far].max()) / rms,
                         far_abs_rms=float(e[far].abs().max()) / rms,
                         far_d_le8=int((d[far] <= 8).sum()))
        _record(what, stats)
        if _COLLECT:
            return exact
        if n:
            e = expect.double()[keep]
            err = (got.double()[keep] - e).abs()
            bad = (d > steps) & (err > ULP16[got.dtype] * float(e.pow(2).mean().sqrt()))
            assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {n} values more than {steps} ulp(s) and one "
                                         f"storage ulp of the rms from the oracle (worst {int(d.max())} ulps)")
        assert stats["not_exact"] <= F16_NOT_EXACT * steps * n + 1, (
            f"{what}: {stats['not_exact']} of {n} values not bit-exact (budget {F16_NOT_EXACT} per step)")
        return exact
    g = got.double()
    e = expect.double()
    err = (g - e).abs()
    scale = e.abs() + e.pow(2).mean().sqrt()
    if got.dtype == torch.float64:
        bad = (err > FP64_SCALE_RTOL * scale) & keep
        stats.update(worst_scale=float((err / scale)[keep].max()) if n else 0.0)
        _record(what, stats)
        assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {n} values beyond {FP64_SCALE_RTOL} of the scale; "
                                     f"worst {stats['worst_scale']:.3g} of it; bit-exact {exact:.6f}")
        return exact
    bad = (err > FP32_SCALE_RTOL * scale) & keep
    beyond = int(((err > rtol * e.abs()) & keep).sum())
    stats.update(beyond_rel=beyond, worst_scale=float((err / (rtol * scale))[keep].max()) if n else 0.0)
    _record(what, stats)
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {n} values beyond {FP32_SCALE_RTOL} of the scale; "
                                 f"worst {stats['worst_scale']:.3g} x 1e-6 of it; bit-exact {exact:.6f}")
    if _COLLECT:
        return exact
    assert beyond <= FP32_BEYOND_REL * n + 3, (f"{what}: {beyond} of {n} values beyond a 1e-6 relative error "
                                               f"(budget {FP32_BEYOND_REL}); bit-exact {exact:.6f}")
    return exact


def code_diff_mask(a: torch.Tensor, b: torch.Tensor, numel: int) -> torch.Tensor:
    """Per value: whether two packed code tensors hold different 4-bit codes."""
    a = a.cpu()
    b = b.cpu()
    lo = (a & 0x0F) != (b & 0x0F)
    hi = (a >> 4) != (b >> 4)
    return torch.stack([lo, hi], dim=-1).reshape(-1)[:numel]


def code_mismatch(a: torch.Tensor, b: torch.Tensor) -> int:
    """Number of differing 4-bit codes between two packed code tensors."""
    a = a.cpu()
    b = b.cpu()
    lo = ((a & 0x0F) != (b & 0x0F)).sum()
    hi = ((a >> 4) != (b >> 4)).sum()
    return int(lo + hi)


def uniforms_gpu(seed: int, offset: int, n: int) -> torch.Tensor:
    out = torch.empty(n, dtype=torch.float32, device=DEVICE)
    _lib.uniforms(seed, offset, n, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return out
