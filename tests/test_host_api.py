"""The optimizer's host API without a GPU: constructor validation with the reference's own
messages (``adamw.py:127-239``), the scheme set the fused step covers, and the errors for
the parts it does not (the reference's tests ``tests/quantization/test_upd_sr_store_eden.py``,
``test_dyn4_la_upd_sr.py`` and ``test_upd_sr_full4bit.py`` exercise the same paths)."""

from __future__ import annotations

import pytest
import torch

import adamw4bit_amd as aw
from adamw4bit_amd import quantization as q


def params():
    return [torch.nn.Parameter(torch.zeros(4096))]


def make(**kw):
    base = dict(m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz")
    base.update(kw)
    return aw.QuantizedAdamW(params(), **base)


@pytest.mark.parametrize("kw,message", [
    (dict(lr=-1.0), "Invalid learning rate"),
    (dict(eps=-1.0), "Invalid epsilon value"),
    (dict(betas=(1.0, 0.95)), "Invalid beta parameter at index 0"),
    (dict(betas=(0.9, -0.1)), "Invalid beta parameter at index 1"),
    (dict(weight_decay=-0.1), "Invalid weight_decay value"),
    (dict(quant_rng_seed=-3), "quant_rng_seed must be a non-negative integer"),
    (dict(m2_quant_scheme="dyn5"), "m2_quant_scheme must be one of"),
    (dict(m2_quant_scheme="dyn4_sr", use_eden_m2=True), "Vanilla stochastic-rounding m2 schemes"),
])
def test_constructor_rejects_bad_arguments(kw, message):
    with pytest.raises(ValueError, match=message):
        make(**kw)


@pytest.mark.parametrize("mode", ["lin4_upd_sr_store_eden", "dyn4_upd_sr_store_eden"])
def test_store_eden_rejects_use_eden_m2(mode):
    # test_upd_sr_store_eden.py:69-82
    with pytest.raises(ValueError, match="EDEN is built into the store path"):
        make(m1_quant_scheme="fp32", m2_quant_scheme=mode, use_eden_m2=True)


@pytest.mark.parametrize("scheme", ["dyn4_la_upd_sr", "dyn4_proxy_la_upd_sr", "dyn4_vproxy_la_upd_sr"])
def test_lookahead_rejects_extra_corrections(scheme):
    # test_dyn4_la_upd_sr.py:322-330: validated before anything else
    with pytest.raises(ValueError, match="supports m1_quant_scheme"):
        make(m1_quant_scheme="sdyn4", m2_quant_scheme=scheme)
    with pytest.raises(ValueError, match="use_eden_m2"):
        make(m1_quant_scheme="fp32", m2_quant_scheme=scheme, use_eden_m2=True)
    with pytest.raises(ValueError, match="update clipping"):
        make(m1_quant_scheme="fp32", m2_quant_scheme=scheme, update_norm_clip=1.0)


@pytest.mark.parametrize("m2", ["dyn4_upd_sr", "lin4_upd_sr", "dyn4_upd_sr_store_eden", "lin4_upd_sr_store_eden",
                                "dyn4_upd_sr_fp32read", "lin4_upd_sr_fp32read", "dyn4_lookahead_sr",
                                "dyn4_upd_sr_fp32read_nextbc", "dyn4_nz", "lin4_nz", "dyn4", "lin4", "dyn4_sr",
                                "lin4_sr", "fp32", "dyn4_la_upd_sr", "dyn4_proxy_la_upd_sr",
                                "dyn4_vproxy_la_upd_sr"])
@pytest.mark.parametrize("m1", ["nf4", "nf4_sr", "sdyn4", "sdyn4_sr", "fp32"])
def test_schemes_of_the_fused_step_construct(m1, m2):
    if "_la_" in m2 and m1 not in ("fp32", "nf4"):
        pytest.skip("lookahead update-SR takes an fp32 or nf4 m1 (adamw.py:198-208)")
    opt = make(m1_quant_scheme=m1, m2_quant_scheme=m2)
    group = opt.param_groups[0]
    assert group["m1_quant_scheme"] == m1 and group["m2_quant_scheme"] == m2
    for s in (m1, m2):
        if s != "fp32":
            assert q.default_block_size(s) == 128 and s in q.SCHEMES


@pytest.mark.parametrize("kw", [
    dict(m1_quant_scheme="linear"), dict(m2_quant_scheme="dynamic"),
    dict(update_sign_clip=0.5), dict(record_update_direction_every=2), dict(block_size=256),
])
def test_parts_outside_the_fused_step_raise(kw):
    with pytest.raises(NotImplementedError):
        make(**kw)


def test_step_needs_a_hip_device():
    opt = make()
    opt.param_groups[0]["params"][0].grad = torch.ones(4096)
    with pytest.raises(NotImplementedError, match="HIP devices"):
        opt.step()


@pytest.mark.parametrize("scheme", ["dyn4_la_upd_sr", "dyn4_proxy_la_upd_sr", "dyn4_vproxy_la_upd_sr"])
def test_lookahead_state_layout(scheme):
    # test_dyn4_la_upd_sr.py:106-114, 300-307: the pending form keeps fp32 state under
    # "lookahead_pending_exp_avg_sq" and no codes; the proxies keep codes.  Initial state only
    # (the step itself needs a HIP device).
    from adamw4bit_amd.quantization import PENDING_LOOKAHEAD_SCHEMES, SCHEMES, initial_code_and_scale
    assert SCHEMES[scheme][0] == q.CB_DYN4 and SCHEMES[scheme][1] == q.ROUND_LOOKAHEAD_SR
    if scheme not in PENDING_LOOKAHEAD_SCHEMES:
        assert initial_code_and_scale(scheme, False) == initial_code_and_scale("dyn4", False)


def test_clip_grad_norm_host_checks():
    # the fused clip covers the 2-norm of gradients on one HIP device (torch's other norms and CPU
    # tensors raise); no gradients gives torch's tensor(0.)
    opt = make()
    assert float(opt.clip_grad_norm_(1.0)) == 0.0 and opt._grad_clip is None
    opt.param_groups[0]["params"][0].grad = torch.ones(4096)
    with pytest.raises(NotImplementedError, match="2-norm"):
        opt.clip_grad_norm_(1.0, norm_type=float("inf"))
    with pytest.raises(NotImplementedError, match="one HIP device"):
        opt.clip_grad_norm_(1.0)


class _CountingOptimizer(torch.optim.Optimizer):
    """A one-parameter optimizer whose step is wrapped like ``QuantizedAdamW.step``."""

    def __init__(self, params):
        super().__init__(params, {})
        self.calls = []

    @aw.adamw._lean_step
    def step(self, closure=None, scale=1.0):
        self.calls.append(scale)
        return scale


@pytest.mark.filterwarnings("ignore:Warning. Profiler clears events:UserWarning")
def test_lean_step_keeps_torch_hooks_and_profiler_range():
    from torch.optim.optimizer import register_optimizer_step_post_hook, register_optimizer_step_pre_hook
    assert aw.QuantizedAdamW.step.hooked and aw.ZIPSRAdamW4Bit.step is aw.QuantizedAdamW.step
    opt = _CountingOptimizer([torch.nn.Parameter(torch.zeros(1))])
    assert type(opt).step.__wrapped__.__name__ == "step"  # not wrapped again by torch
    assert opt.step() == 1.0 and opt.calls == [1.0]
    seen = []
    pre = opt.register_step_pre_hook(lambda o, args, kwargs: (args, {**kwargs, "scale": 2.0}))
    post = opt.register_step_post_hook(lambda o, args, kwargs: seen.append(("post", kwargs["scale"])))
    gpre = register_optimizer_step_pre_hook(lambda o, args, kwargs: seen.append(("gpre", o is opt)))
    gpost = register_optimizer_step_post_hook(lambda o, args, kwargs: seen.append(("gpost", o is opt)))
    try:
        assert opt.step() == 2.0
        assert seen == [("gpre", True), ("post", 2.0), ("gpost", True)]
    finally:
        for h in (pre, post, gpre, gpost):
            h.remove()
    assert opt.step() == 1.0 and opt.calls == [1.0, 2.0, 1.0]
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        opt.step()
    names = {e.name for e in prof.events()}
    assert "Optimizer.step#_CountingOptimizer.step" in names


# ---------------------------------------------------------------------------
# The optimized backend's preflight gates (_optimized.py:85-136), decided on the host
# ---------------------------------------------------------------------------

def _gate(opt, p, state=None):
    group = opt.param_groups[0]
    requested = (opt._m1_scheme_for(p, group["m1_quant_scheme"]), group["m2_quant_scheme"])
    sizes = (128, 128)
    schemes = tuple(opt._effective_scheme(p, m, s) for m, s in zip(requested, sizes))
    return opt._plan_accepts(p, p.grad, group, requested, sizes, schemes, opt.state[p] if state is None else state)


def _quantized_state(p, packed=True):
    n = p.numel()
    codes = torch.zeros((n + 1) // 2 if packed else n, dtype=torch.uint8)
    st = {"step": 1}
    for m in ("m1", "m2"):
        st[f"{m}_code"] = codes.clone()
        st[f"{m}_quant_state"] = q.QuantState(absmax=torch.zeros(n // 128), shape=p.shape, dtype=torch.float32,
                                              blocksize=128, packed=packed)
    return st


def test_preflight_gates_follow_the_optimized_backend():
    """Each gate of _plan that sends a parameter to the reference step: overlapping gradient,
    strided parameter or gradient, incompatible state, a persisted fallback mark, a non-int step
    count, a bad chunk limit; everything else takes the optimized semantics."""
    p = torch.nn.Parameter(torch.zeros(64, 128))
    opt = aw.ZIPSRAdamW4Bit([p], optimized=True, quant_rng_seed=0)
    p.grad = torch.zeros_like(p)
    assert _gate(opt, p)
    assert _gate(opt, p, _quantized_state(p))
    assert _gate(opt, p, _quantized_state(p, packed=False))  # legacy unpacked codes are compatible
    p.grad = p.detach()  # shares the parameter's storage
    assert not _gate(opt, p)
    p.grad = torch.zeros(128, 64).t()
    assert not _gate(opt, p)
    p.grad = torch.zeros_like(p)
    st = _quantized_state(p)
    st["m1_code"] = st["m1_code"][::1].view(-1)[:-1]  # too short
    assert not _gate(opt, p, st)
    st = _quantized_state(p)
    st["m2_quant_state"].absmax = torch.zeros(2 * p.numel() // 128)[::2]  # strided scales
    assert not _gate(opt, p, st)
    st = _quantized_state(p)
    st["m2_code"] = st["m1_code"]  # two moments on one buffer
    assert not _gate(opt, p, st)
    st = _quantized_state(p)
    st["m1_code"] = p.grad.view(torch.uint8)[: p.numel() // 2]  # state on the gradient's storage
    assert not _gate(opt, p, st)
    st = _quantized_state(p)
    st["_optimized_full_fallback"] = True
    assert not _gate(opt, p, st)
    st = _quantized_state(p)
    st["step"] = torch.tensor(1.0)
    assert not _gate(opt, p, st)
    opt.param_groups[0]["max_chunk_numel"] = 64  # below the block alignment
    assert not _gate(opt, p)
    opt.param_groups[0]["max_chunk_numel"] = 128
    assert _gate(opt, p)
    strided = torch.nn.Parameter(torch.zeros(128, 64).t())
    strided.grad = torch.zeros(64, 128)
    o2 = aw.ZEEDENAdamW4Bit([strided], optimized=True)
    assert not _gate(o2, strided)
    assert not _gate(aw.ZEEDENAdamW4Bit([p], optimized=False), p)  # optimized=False: always the reference


def test_aliased_state_load_marks_both_parameters_and_persists():
    """Moment buffers that share storage after a load mark every owner for the reference step
    (_optimized.py:53-83); the mark travels in the state dict."""
    ps = [torch.nn.Parameter(torch.zeros(64, 128)) for _ in range(3)]
    opt = aw.ZIPSRAdamW4Bit(ps, optimized=True, quant_rng_seed=0)
    sd = opt.state_dict()
    states = [_quantized_state(p) for p in ps]
    states[1]["m2_code"] = states[0]["m2_code"]
    sd["state"] = {i: {k: (vars(v).copy() if isinstance(v, q.QuantState) else v) for k, v in st.items()}
                   for i, st in enumerate(states)}
    opt.load_state_dict(sd)
    marks = [opt.state[p].get("_optimized_full_fallback", False) for p in ps]
    assert marks == [True, True, False]
    o2 = aw.ZIPSRAdamW4Bit(ps, optimized=True, quant_rng_seed=0)
    sd2 = opt.state_dict()
    for i in (0, 1):  # un-alias: the mark alone must keep them on the reference step
        sd2["state"][i] = {k: (v.clone() if torch.is_tensor(v) else dict(v, absmax=v["absmax"].clone())
                               if isinstance(v, dict) else v) for k, v in sd2["state"][i].items()}
    o2.load_state_dict(sd2)
    assert [o2.state[p].get("_optimized_full_fallback", False) for p in ps] == [True, True, False]


def test_range_set_answers_as_the_pairwise_overlap_test():
    """The launch's record of written byte ranges (an interval union per device) answers every
    query as testing ``_overlaps`` against each recorded range would, empty ranges included."""
    import random

    from adamw4bit_amd.adamw import _overlaps, _RangeSet

    rng = random.Random(5)
    for trial in range(200):
        rs, kept = _RangeSet(), []
        for _ in range(rng.randint(1, 40)):
            key = rng.choice(["cuda:0", "cuda:1"])
            a = rng.randint(0, 200)
            r = (key, a, a + rng.choice([0, 1, 2, 5, 17, 40]))
            expect = any(_overlaps(r, q) for q in kept)
            assert rs.overlaps(r) == expect, (trial, r, kept)
            if rng.random() < 0.7:
                rs.add(r)
                kept.append(r)
