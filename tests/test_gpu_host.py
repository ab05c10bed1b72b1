"""GPU tests of the host side of the step: which semantics each parameter gets (the optimized
backend's preflight gates, _optimized.py:85-136), the cached launch plan's validity, atomic
steps, strided and misaligned parameters, and the compiled path through the torch operator.

Where a gate sends a parameter to the reference step, the check is against a twin optimizer
with ``optimized=False`` on plain contiguous copies: the same kernel with the reference step's
stochastic-rounding rules and initial draw count, which the golden trajectories pin."""

from __future__ import annotations

import pytest
import torch

import adamw4bit_amd as aw
from adamw4bit_amd import _lib
from oracle import reference_step as ref

from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

ARGS = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def log(msg):
    print(msg, flush=True)


def same_state(oa, pa, ob, pb, what):
    """Bit-identical parameters and moment state."""
    assert torch.equal(H.bits(pa.detach().contiguous()), H.bits(pb.detach().contiguous())), what
    sa, sb = H.state_of(oa, pa), H.state_of(ob, pb)
    assert sa.keys() == sb.keys() and sa["step"] == sb["step"], (what, sorted(sa), sorted(sb))
    for key in sa:
        if key != "step":
            assert torch.equal(H.bits(sa[key]), H.bits(sb[key])), (what, key)


def _deep_clone(value):
    if torch.is_tensor(value):
        return value.clone()
    if isinstance(value, dict):
        return {k: _deep_clone(v) for k, v in value.items()}
    return value


def grads_like(shapes, gen, dtype=torch.float32):
    return [H.heavy_tailed(s, gen).to(dtype).to(H.DEVICE) for s in shapes]


# ---------------------------------------------------------------------------
# The launch plan follows the parameters' storage
# ---------------------------------------------------------------------------

def test_plan_follows_swapped_parameter_storage():
    """``p.data`` can change without changing the Parameter object (vector_to_parameters,
    ``module.to(dtype)``, a manual ``p.data = ...``).  A step after such a swap must update the
    new storage exactly as a step that rebuilds its tables does; a plan that kept the old
    addresses would write into freed memory."""
    log("plan after p.data swaps")
    shapes = [(256, 512), (768,), (64, 1024)]
    gen = torch.Generator().manual_seed(31)
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=3, **ARGS)
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=3, **ARGS)
    for k in range(6):
        if k == 2:
            # vector_to_parameters: every parameter becomes a view of one new flat buffer
            for ps in (pa, pb):
                flat = torch.nn.utils.parameters_to_vector(ps).clone()
                torch.nn.utils.vector_to_parameters(flat, ps)
        if k == 4:
            for ps in (pa, pb):  # a dtype change, as module.to(torch.bfloat16) makes it
                for p in ps:
                    p.data = p.data.to(torch.bfloat16)
        dtype = pa[0].dtype
        for a, b, g in zip(pa, pb, grads_like(shapes, gen, dtype)):
            a.grad, b.grad = g.clone(), g.clone()
        oa.step()
        ob._launch_plan = None  # always the full path
        ob.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            same_state(oa, a, ob, b, (k, i))


# ---------------------------------------------------------------------------
# Parameters that do not allow vector access, strided parameters
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("recipe,dtype,offset", [("zeeden", torch.float32, 1), ("zipsr", torch.float32, 1),
                                                  ("zeeden", torch.bfloat16, 4), ("zipsr", torch.bfloat16, 4)])
def test_parameter_at_odd_offset_matches_oracle(recipe, dtype, offset):
    """A parameter (and gradient) a few elements into a flat buffer: fp32 one element in, whose
    rows cannot take 16-byte vector accesses; bf16 four elements (8 bytes) in, whose rows allow the
    4-value accesses but not the 16-byte parameter stores of the specialised bf16 kernels.  Both run
    the generic kernel; results equal the oracle's and the buffer's other elements stay as they were."""
    log(f"parameter at element offset {offset} ({recipe}, {dtype})")
    gen = torch.Generator().manual_seed(8)
    shape = (96, 256)
    n = shape[0] * shape[1]
    init = (torch.randn(shape, generator=gen) * 0.02).to(dtype)
    buf = torch.zeros(n + offset + 4, device=H.DEVICE, dtype=dtype)
    buf[offset:offset + n] = init.reshape(-1).to(H.DEVICE)
    p = torch.nn.Parameter(buf[offset:offset + n].view(shape))  # contiguous, off a 16-byte boundary
    assert p.is_contiguous() and p.data_ptr() % 16 == offset * p.element_size()
    kw = dict(optimized=True, quant_rng_seed=9 if recipe == "zipsr" else None, **ARGS)
    opt = aw.ZIPSRAdamW4Bit([p], **kw) if recipe == "zipsr" else aw.ZEEDENAdamW4Bit([p], **kw)
    m2 = "dyn4_upd_sr_fp32read" if recipe == "zipsr" else "dyn4_nz"
    cpu = [init.clone()]
    oracle = ref.Oracle(cpu, ref.Hyper(), ["nf4"], [m2], [recipe == "zeeden"], seed=kw["quant_rng_seed"],
                        draw_fn=H.PhiloxMirror(opt, H.DEVICE), usr_sqrt="cr")
    goff = 3 if dtype == torch.float32 else 4  # bf16: 8 bytes in, so the 4-value accesses stay allowed
    gbuf = torch.zeros(n + goff + 4, device=H.DEVICE, dtype=dtype)
    for _ in range(3):
        g = H.heavy_tailed(shape, gen).to(dtype)
        gbuf[goff:goff + n] = g.reshape(-1).to(H.DEVICE)
        p.grad = gbuf[goff:goff + n].view(shape)
        opt.step()
        oracle.step([g])
    torch.cuda.synchronize()
    st, ost = H.state_of(opt, p), H.oracle_state((oracle.states[0].m1, oracle.states[0].m2))
    for key in ost:
        flips = H.code_mismatch(st[key], ost[key]) if key.endswith("_code") else None
        if flips is not None:
            log(f"  {key}: {flips} codes differ")
            assert flips == 0, key
        else:
            assert torch.equal(H.bits(st[key]), H.bits(ost[key])), key
    H.assert_params_close(p, cpu[0], "odd offset", steps=3)
    assert bool((buf[:offset] == 0).all()) and bool((buf[offset + n:] == 0).all())  # neighbours untouched


def test_strided_parameter_takes_reference_step():
    """A non-contiguous parameter (a transposed view) is not the optimized backend's
    (_optimized.py:98): it follows the reference step, which updates it in logical order."""
    log("strided parameter")
    gen = torch.Generator().manual_seed(12)
    base = torch.randn(384, 256, generator=gen) * 0.02
    pa = torch.nn.Parameter(base.clone().to(H.DEVICE).t())       # (256, 384), strided
    pb = torch.nn.Parameter(base.clone().t().contiguous().to(H.DEVICE))
    assert not pa.is_contiguous()
    oa = aw.ZIPSRAdamW4Bit([pa], optimized=True, quant_rng_seed=6, **ARGS)
    ob = aw.ZIPSRAdamW4Bit([pb], optimized=False, quant_rng_seed=6, **ARGS)
    for k in range(3):
        g = H.heavy_tailed((256, 384), gen).to(H.DEVICE)
        pa.grad, pb.grad = g.clone(), g.clone()
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        assert not pa.is_contiguous()
        same_state(oa, pa, ob, pb, k)
    assert oa._launch_plan is None  # the staged copy is per step


# ---------------------------------------------------------------------------
# The optimized backend's gates: which parameters take the reference step
# ---------------------------------------------------------------------------

def test_gradient_overlapping_parameter_takes_reference_step():
    """A gradient that shares storage with its parameter sends the parameter to the reference
    step (_optimized.py:110-112), including its initial draw count: n draws for the zero state
    instead of one 128-value tile."""
    log("gradient aliasing its parameter")
    gen = torch.Generator().manual_seed(13)
    shape = (128, 512)
    n = shape[0] * shape[1]
    init = torch.randn(shape, generator=gen) * 1e-3
    pa = torch.nn.Parameter(init.clone().to(H.DEVICE))
    pb = torch.nn.Parameter(init.clone().to(H.DEVICE))
    oa = aw.ZIPSRAdamW4Bit([pa], optimized=True, quant_rng_seed=2, **ARGS)
    ob = aw.ZIPSRAdamW4Bit([pb], optimized=False, quant_rng_seed=2, **ARGS)
    for k in range(2):
        pa.grad = pa.detach()          # the gradient is the parameter's own storage
        pb.grad = pb.detach().clone()
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        same_state(oa, pa, ob, pb, k)
        if k == 0:
            # reference step: the zero state draws n, the step n (optimized: 128 + n)
            assert oa._stream("m2", pa.device).offset == 2 * n
            assert oa._launch_plan is None


def test_noncontiguous_gradient_takes_reference_step():
    log("non-contiguous gradient")
    gen = torch.Generator().manual_seed(14)
    shape = (192, 256)
    init = torch.randn(shape, generator=gen) * 0.02
    pa = torch.nn.Parameter(init.clone().to(H.DEVICE))
    pb = torch.nn.Parameter(init.clone().to(H.DEVICE))
    oa = aw.ZIPSRAdamW4Bit([pa], optimized=True, quant_rng_seed=7, **ARGS)
    ob = aw.ZIPSRAdamW4Bit([pb], optimized=False, quant_rng_seed=7, **ARGS)
    for k in range(2):
        g = H.heavy_tailed((shape[1], shape[0]), gen).to(H.DEVICE)
        pa.grad = g.t()                # strided view with the parameter's shape
        pb.grad = g.t().contiguous()
        assert not pa.grad.is_contiguous()
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        same_state(oa, pa, ob, pb, k)


def test_aliased_state_after_load_takes_reference_step(tmp_path):
    """Moment state that aliases another parameter's after a checkpoint load marks both
    parameters for the reference step for good (_optimized.py:53-83): the mark is saved and
    survives a resume, and the steps match an optimized=False twin."""
    log("aliased state after load")
    gen = torch.Generator().manual_seed(15)
    shapes = [(128, 256), (128, 256)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=4, **ARGS)
    for p, g in zip(pa, grads_like(shapes, gen)):
        p.grad = g
    oa.step()
    sd = oa.state_dict()
    # both parameters' m1 codes now share one tensor
    sd["state"][1]["m1_code"] = sd["state"][0]["m1_code"]
    pb = [torch.nn.Parameter(p.detach().clone()) for p in pa]
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=4, **ARGS)
    ob.load_state_dict(sd)
    assert all(ob.state[p].get("_optimized_full_fallback") is True for p in pb)
    torch.save(ob.state_dict(), tmp_path / "aliased.pt")
    pc = [torch.nn.Parameter(p.detach().clone()) for p in pb]
    oc = aw.ZIPSRAdamW4Bit(pc, optimized=True, quant_rng_seed=4, **ARGS)
    oc.load_state_dict(torch.load(tmp_path / "aliased.pt", weights_only=True))
    assert all(oc.state[p].get("_optimized_full_fallback") is True for p in pc)  # persisted
    # twin on the reference step, from the same (unaliased) starting state
    pd = [torch.nn.Parameter(p.detach().clone()) for p in pc]
    od = aw.ZIPSRAdamW4Bit(pd, optimized=False, quant_rng_seed=4, **ARGS)
    sd2 = oc.state_dict()
    for i in (0, 1):  # private copies: load_state_dict keeps same-device tensors, as torch's does
        sd2["state"][i] = {k: _deep_clone(v) for k, v in sd2["state"][i].items() if k != "_optimized_full_fallback"}
    od.load_state_dict(sd2)
    for k in range(2):
        for c, d, g in zip(pc, pd, grads_like(shapes, gen)):
            c.grad, d.grad = g.clone(), g.clone()
        oc.step()
        od.step()
        torch.cuda.synchronize()
        for i in (0, 1):
            assert oc.state[pc[i]]["_optimized_full_fallback"] is True
            # the reference step wrote fresh codes: the two parameters no longer share them
            same_state(oc, pc[i], od, pd[i], (k, i))
    assert oc.state[pc[0]]["m1_code"].data_ptr() != oc.state[pc[1]]["m1_code"].data_ptr()


# ---------------------------------------------------------------------------
# Atomic steps
# ---------------------------------------------------------------------------

def test_rejected_parameter_leaves_every_state_untouched():
    """A parameter the step cannot take (complex64), listed after one it can, raises before any
    state changes: the first parameter is not initialised, no stream moved."""
    log("rejected parameter: no state change")
    good = torch.nn.Parameter(torch.randn(64, 128, device=H.DEVICE) * 0.02)
    bad = torch.nn.Parameter(torch.randn(64, 128, device=H.DEVICE, dtype=torch.complex64))
    opt = aw.ZIPSRAdamW4Bit([good, bad], optimized=True, quant_rng_seed=1, **ARGS)
    good.grad = torch.randn_like(good) * 1e-3
    bad.grad = torch.randn_like(bad) * 1e-3
    before = good.detach().clone()
    with pytest.raises(NotImplementedError, match="complex64"):
        opt.step()
    torch.cuda.synchronize()
    assert len(opt.state[good]) == 0
    assert all(s.offset == 0 for s in opt._all_streams())
    assert torch.equal(good.detach(), before)
    # the same parameter stepped alone afterwards matches a fresh optimizer
    bad.grad = None
    twin = torch.nn.Parameter(before.clone())
    ot = aw.ZIPSRAdamW4Bit([twin], optimized=True, quant_rng_seed=1, **ARGS)
    twin.grad = good.grad.clone()
    opt.step()
    ot.step()
    torch.cuda.synchronize()
    same_state(opt, good, ot, twin, "after the rejected step")


def test_step_failing_after_enqueued_kernels_refuses_further_steps():
    """A step whose launches fail after some of its step kernels were enqueued cannot be undone
    (its tensors may be partly updated).  Injected in the library: the step of an fp32 and a bf16
    parameter is two launches; the first is made, the second fails without being attempted
    (AW4_ELAUNCHED).  The step raises HipLaunchIncomplete, the optimizer refuses further steps, and
    after the parameters and a checkpoint from before the failure are loaded it continues bit for bit
    like an optimizer that never failed.  With the failure at the first launch nothing was enqueued
    and the step is undone as before."""
    log("failure after enqueued kernels: refused until a checkpoint is loaded")
    gen = torch.Generator().manual_seed(23)
    shapes = [(128, 256), (64, 256)]
    dtypes = [torch.float32, torch.bfloat16]
    init = [(torch.randn(s, generator=gen) * 0.02).to(dt) for s, dt in zip(shapes, dtypes)]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=5, **ARGS)
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=5, **ARGS)
    for k in range(5):
        gs = [H.heavy_tailed(s, gen).to(dt).to(H.DEVICE) for s, dt in zip(shapes, dtypes)]
        for a, b, g in zip(pa, pb, gs):
            a.grad, b.grad = g.clone(), g.clone()
        if k in (1, 3):  # k == 1: the full path; k == 3: the cached plan
            saved_params = [a.detach().clone() for a in pa]
            saved_state = _deep_clone(oa.state_dict())
            # nothing enqueued: an ordinary failure, undone
            _lib.inject_launch_failure(0)
            with pytest.raises(_lib.HipLibraryError, match="injected") as info:
                oa.step()
            assert not isinstance(info.value, _lib.HipLaunchIncomplete)
            # one launch enqueued, then the failure
            _lib.inject_launch_failure(1)
            with pytest.raises(_lib.HipLaunchIncomplete, match="injected"):
                oa.step()
            with pytest.raises(RuntimeError, match="partly updated"):
                oa.step()
            torch.cuda.synchronize()
            with torch.no_grad():
                for a, saved in zip(pa, saved_params):
                    a.copy_(saved)
            oa.load_state_dict(saved_state)
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            same_state(oa, a, ob, b, (k, i))
    _lib.inject_launch_failure(-1)


def test_failed_launch_is_undone(monkeypatch):
    """A launch that fails leaves step counts, moment state and stream positions as they were,
    through the full path and through the cached plan."""
    log("failed launch: undone")
    gen = torch.Generator().manual_seed(17)
    shapes = [(128, 256), (768,)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=5, **ARGS)
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=5, **ARGS)
    real = _lib.fused_step

    def failing(table, stream):
        raise _lib.HipLibraryError("injected launch failure")

    for k in range(5):
        gs = grads_like(shapes, gen)
        if k in (0, 3):  # k == 0: full path (fresh state); k == 3: the cached plan
            for a, g in zip(pa, gs):
                a.grad = g.clone()
            snapshot = [dict(oa.state[a]) for a in pa]
            offsets = {id(s): s.offset for s in oa._all_streams()}
            monkeypatch.setattr(_lib, "fused_step", failing)
            with pytest.raises(_lib.HipLibraryError, match="injected"):
                oa.step()
            monkeypatch.setattr(_lib, "fused_step", real)
            for a, snap in zip(pa, snapshot):
                st = oa.state[a]
                assert st.keys() == snap.keys() and all(st[key] is snap[key] for key in st), k
            # streams opened by the failed step's checks start at 0; the others did not move
            assert all(s.offset == offsets.get(id(s), 0) for s in oa._all_streams()), k
        for a, b, g in zip(pa, pb, gs):
            a.grad, b.grad = g.clone(), g.clone()
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            same_state(oa, a, ob, b, (k, i))


# ---------------------------------------------------------------------------
# quant_rng_seed=None: draws come from torch's generator of the device
# ---------------------------------------------------------------------------

def test_unseeded_draws_follow_torch_generator(monkeypatch):
    """With ``quant_rng_seed=None`` the reference's stochastic writes draw from torch's default
    generator (``_optimized_quantization.py:37-43``): reseeding torch reproduces a run, another
    seed or another torch draw between steps changes it, and the cached plan takes the
    generator's current seed and position at every step."""
    log("unseeded streams follow torch's generator")
    gen = torch.Generator().manual_seed(23)
    shapes = [(64, 256), (512,)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    grads = [grads_like(shapes, gen) for _ in range(3)]
    real = _lib.fused_step
    tables = []

    def recording(table, stream):
        tables.append(table.copy())
        real(table, stream)

    monkeypatch.setattr(_lib, "fused_step", recording)

    def run(seeds, between=None):
        params = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
        opt = aw.ZIPSRAdamW4Bit(params, optimized=True, quant_rng_seed=None, **ARGS)
        for k, gs in enumerate(grads):
            if seeds[k] is not None:
                torch.manual_seed(seeds[k])
            if between is not None and k == 1:
                between()
            for p, g in zip(params, gs):
                p.grad = g.clone()
            opt.step()
        torch.cuda.synchronize()
        return opt, params

    def codes(opt, params):
        return [H.bits(opt.state[p]["m2_code"]) for p in params if "m2_code" in opt.state[p]]

    oa, pa = run([3, None, None])
    ob, pb = run([3, None, None])
    for i, (a, b) in enumerate(zip(pa, pb)):
        same_state(oa, a, ob, b, ("same seed", i))
    oc, pc = run([4, None, None])
    assert any(not torch.equal(x, y) for x, y in zip(codes(oa, pa), codes(oc, pc)))
    # a torch draw on the device between steps moves the stream
    od, pd = run([3, None, None], between=lambda: torch.rand(1000, device=H.DEVICE))
    assert any(not torch.equal(x, y) for x, y in zip(codes(oa, pa), codes(od, pd)))
    # reseeding before the third step: the cached plan's rows take the new key and position
    from adamw4bit_amd.adamw import _LaunchPlan
    prepare, planned = _LaunchPlan.prepare, []

    def counting(self, opt, records=True):
        out = prepare(self, opt, records)
        planned.append(out is not None)
        return out

    monkeypatch.setattr(_LaunchPlan, "prepare", counting)
    tables.clear()
    oe, pe = run([3, None, 9])
    assert planned == [True, True]  # steps 2 and 3 reuse the plan
    mix = aw.QuantizedAdamW._QUANT_RNG_OFFSETS["m2"] * 0x9E3779B97F4A7C15 & (2 ** 64 - 1)
    last = tables[-1]
    quantized = last["m2"]["rounding"] != _lib.ROUND_FP32
    assert quantized.any()
    assert set(last["m2"]["rng_seed"][quantized].tolist()) == {9 ^ mix}
    assert last["m2"]["rng_offset"][quantized].min() == 0


# ---------------------------------------------------------------------------
# torch.amp.GradScaler drives the optimizer unchanged
# ---------------------------------------------------------------------------

def test_grad_scaler_unscales_and_skips_steps():
    """A trainer with loss scaling: ``scaler.unscale_(opt)`` divides the gradients in place and
    records non-finite values, the fused clip reads the unscaled gradients, and
    ``scaler.step(opt)`` skips the step of an overflowed iteration.  States and parameters equal
    a twin optimizer stepped on the unscaled gradients of the iterations that were not skipped
    (scaling by a power of two is exact)."""
    log("GradScaler + fused clip")
    gen = torch.Generator().manual_seed(41)
    shapes = [(128, 256), (512,)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=2, **ARGS)
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=2, **ARGS)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 12, growth_interval=1000)
    for k in range(4):
        gs = grads_like(shapes, gen)
        scaler.scale(torch.ones((), device=H.DEVICE))  # the loss a trainer would scale
        scale = scaler.get_scale()
        for a, g in zip(pa, gs):
            a.grad = g * scale
        if k == 2:  # an overflowed iteration
            pa[0].grad.view(-1)[7] = float("inf")
        scaler.unscale_(oa)
        oa.clip_grad_norm_(1.0)
        scaler.step(oa)
        scaler.update()
        if k == 2:
            assert scaler.get_scale() == scale / 2  # the step was skipped
            assert all(oa.state[a]["step"] == 2 for a in pa)
            oa.zero_grad()  # drops the clip whose step was skipped
            continue
        for b, g in zip(pb, gs):
            b.grad = g.clone()
        ob.clip_grad_norm_(1.0)
        ob.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            same_state(oa, a, ob, b, (k, i))
    assert all(oa.state[a]["step"] == 3 for a in pa)


def _scaled_grads(params, gs, scale, k):
    for p, g in zip(params, gs):
        p.grad = (g * scale).to(p.dtype).to(H.DEVICE)
    if k == 2:  # an overflowed iteration
        params[0].grad.view(-1)[7] = float("inf")
    if k == 3:  # a NaN
        params[-1].grad.view(-1)[5] = float("nan")


@pytest.mark.parametrize("clip", [True, False])
def test_fused_unscale_matches_grad_scaler_unscale(clip):
    """The loss-scale unscaling fused into the clip's read of the gradients
    (``clip_grad_norm_(max_norm, grad_scaler=...)``, or ``unscale_grads_`` without a clip) against
    torch's ``scaler.unscale_(opt)`` writing the unscaled gradients, then the same clip and
    ``scaler.step`` / ``scaler.update``: the total norm, found_inf, the scale's trajectory, and
    parameters and moment state after every step bit-identical, over five iterations with a
    scale that is not a power of two (so unscaling rounds) and an overflowed (inf) and a NaN
    iteration, whose steps both skip.  The fused path leaves the gradients scaled in memory.
    (torch's unscale_ takes fp32 gradients only on this device: it refuses fp16, and its kernel
    has no bf16 instance; bf16 is the next test.)"""
    log(f"fused GradScaler unscale ({'with' if clip else 'without'} clip)")
    gen = torch.Generator().manual_seed(43)
    shapes = [(128, 256), (512,), (64, 256)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=4, **ARGS)
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=4, **ARGS)
    sa = torch.amp.GradScaler("cuda", init_scale=3.0 * 2 ** 10, growth_interval=2)
    sb = torch.amp.GradScaler("cuda", init_scale=3.0 * 2 ** 10, growth_interval=2)
    skipped = 0
    for k in range(5):
        gs = [H.heavy_tailed(s, gen) for s in shapes]
        sa.scale(torch.ones((), device=H.DEVICE))  # the loss a trainer would scale
        sb.scale(torch.ones((), device=H.DEVICE))
        scale = sa.get_scale()
        assert scale == sb.get_scale()
        _scaled_grads(pa, gs, scale, k)
        _scaled_grads(pb, gs, scale, k)
        scaled = [a.grad.clone() for a in pa]
        if clip:
            ta = oa.clip_grad_norm_(1.0, grad_scaler=sa)
            sb.unscale_(ob)
            tb = ob.clip_grad_norm_(1.0)
            assert ta.dtype == tb.dtype
            assert torch.equal(H.bits(ta), H.bits(tb)) or (bool(ta.isnan()) and bool(tb.isnan())), (k, ta, tb)
        else:
            oa.unscale_grads_(sa)
            sb.unscale_(ob)
        fa = sum(float(v) for v in sa._per_optimizer_states[id(oa)]["found_inf_per_device"].values())
        fb = sum(float(v) for v in sb._per_optimizer_states[id(ob)]["found_inf_per_device"].values())
        assert fa == fb == (1.0 if k in (2, 3) else 0.0), (k, fa, fb)
        with pytest.raises(RuntimeError, match="already been called"):
            sa.unscale_(oa)
        sa.step(oa)
        sb.step(ob)
        sa.update()
        sb.update()
        assert sa.get_scale() == sb.get_scale()
        for a, g in zip(pa, scaled):
            assert torch.equal(H.bits(a.grad), H.bits(g)), k  # still scaled in memory
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            same_state(oa, a, ob, b, (k, i))
        skipped += int(k in (2, 3))
        oa.zero_grad()  # drops the pending unscale/clip of a skipped step
        ob.zero_grad()
    assert all(oa.state[a]["step"] == 5 - skipped for a in pa)
    # torch's unscale_ refuses fp16 gradients, and so does the fused one
    ph = torch.nn.Parameter(torch.zeros(4096, dtype=torch.float16, device=H.DEVICE))
    oh = aw.ZIPSRAdamW4Bit([ph], optimized=True, quant_rng_seed=4, **ARGS)
    ph.grad = torch.ones_like(ph)
    sh = torch.amp.GradScaler("cuda")
    sh.scale(torch.ones((), device=H.DEVICE))
    with pytest.raises(ValueError, match="FP16"):
        oh.clip_grad_norm_(1.0, grad_scaler=sh)


def test_fused_unscale_of_bf16_gradients():
    """bf16 gradients, which torch's unscale_ kernel does not take here: the fused unscale reads
    each value as bf16(fp32(g) * inv_scale), the functor torch applies to its dtypes, so the
    result equals torch ops that unscale in place the same way (found_inf: any value not finite,
    the step skipped), followed by the fused clip and the step, bit for bit."""
    log("fused GradScaler unscale, bf16 gradients")
    gen = torch.Generator().manual_seed(47)
    shapes = [(128, 256), (64, 256)]
    init = [(torch.randn(s, generator=gen) * 0.02).to(torch.bfloat16) for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=6, **ARGS)
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=6, **ARGS)
    sa = torch.amp.GradScaler("cuda", init_scale=3.0 * 2 ** 10, growth_interval=2)
    for k in range(5):
        gs = [H.heavy_tailed(s, gen) for s in shapes]
        sa.scale(torch.ones((), device=H.DEVICE))
        scale = sa.get_scale()
        _scaled_grads(pa, gs, scale, k)
        _scaled_grads(pb, gs, scale, k)
        inv = sa._scale.double().reciprocal().float()
        found = any(not bool(torch.isfinite(b.grad).all()) for b in pb)
        for b in pb:
            b.grad = (b.grad.float() * inv).to(torch.bfloat16)
        ta = oa.clip_grad_norm_(1.0, grad_scaler=sa)
        tb = ob.clip_grad_norm_(1.0)
        assert torch.equal(H.bits(ta), H.bits(tb)) or (bool(ta.isnan()) and bool(tb.isnan())), (k, ta, tb)
        fa = sum(float(v) for v in sa._per_optimizer_states[id(oa)]["found_inf_per_device"].values())
        assert fa == float(found) == (1.0 if k in (2, 3) else 0.0), k
        sa.step(oa)
        sa.update()
        if not found:
            ob.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            same_state(oa, a, ob, b, (k, i))
        oa.zero_grad()
        ob.zero_grad()


def test_fused_clip_refuses_float64_gradients():
    """The fused clip and unscale read fp32/bf16/fp16 gradients; with a float64 gradient they
    raise before any device work, nothing is left pending, and the step still takes the float64
    parameter (unclipped)."""
    log("fused clip with a float64 gradient")
    p = torch.nn.Parameter(torch.randn(64, 256, device=H.DEVICE, dtype=torch.float64) * 0.02)
    q = torch.nn.Parameter(torch.randn(64, 256, device=H.DEVICE) * 0.02)
    opt = aw.ZIPSRAdamW4Bit([p, q], optimized=True, quant_rng_seed=2, **ARGS)
    p.grad = torch.randn_like(p) * 1e-3
    q.grad = torch.randn_like(q) * 1e-3
    scaler = torch.amp.GradScaler("cuda", init_scale=4.0)
    scaler.scale(torch.ones((), device=H.DEVICE))
    for call in (lambda: opt.clip_grad_norm_(1.0), lambda: opt.clip_grad_norm_(1.0, grad_scaler=scaler),
                 lambda: opt.unscale_grads_(scaler)):
        with pytest.raises(NotImplementedError, match="float32/bfloat16/float16 gradients"):
            call()
        assert opt._grad_clip is None
    before = p.detach().clone()
    opt.step()
    torch.cuda.synchronize()
    assert opt.state[p]["step"] == 1 and not torch.equal(p.detach(), before)


# ---------------------------------------------------------------------------
# torch.compile: the launch is the custom operator
# ---------------------------------------------------------------------------

def test_compiled_step_goes_through_the_operator_and_matches_eager():
    """``torch.compile`` of a function that calls ``opt.step()``: the host work runs eagerly
    (compiler-disabled), the launch is traced as ``adamw4bit_hip::fused_step_`` -- which takes
    its addresses from the tensors it receives, so functionalization copies are the ones
    written -- and parameters and states are bit-identical to eager steps, with version
    counters bumped."""
    log("compiled step through adamw4bit_hip::fused_step_")
    import torch._dynamo
    from torch._dynamo.testing import CompileCounterWithBackend

    torch._dynamo.reset()
    gen = torch.Generator().manual_seed(19)
    shapes = [(256, 128), (768,), (64, 512)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = aw.ZIPSRAdamW4Bit(pa, optimized=True, quant_rng_seed=11, **ARGS)
    ob = aw.ZIPSRAdamW4Bit(pb, optimized=True, quant_rng_seed=11, **ARGS)
    counter = CompileCounterWithBackend("inductor")

    @torch.compile(backend=counter)
    def compiled_step():
        oa.step()

    for k in range(3):
        for a, b, g in zip(pa, pb, grads_like(shapes, gen)):
            a.grad, b.grad = g.clone(), g.clone()
        versions = [a._version for a in pa]
        compiled_step()
        ob.step()
        torch.cuda.synchronize()
        assert all(a._version > v for a, v in zip(pa, versions)), k
        for i, (a, b) in enumerate(zip(pa, pb)):
            same_state(oa, a, ob, b, (k, i))
    targets = {str(node.target) for gm in counter.graphs for node in gm.graph.nodes if node.op == "call_function"}
    log(f"  {counter.frame_count} frames compiled; call targets {sorted(targets)}")
    assert any("adamw4bit_hip.fused_step_" in t for t in targets), targets


def test_concurrent_steps_on_two_streams_match_sequential():
    """Two host threads, each stepping its own optimizer on its own stream (16 tensors per step,
    so the tables go through the library's shared staging slots, and one single-tensor optimizer
    whose table travels in the launch arguments), interleave their library calls; every result
    is bit-identical to the same steps run one optimizer after the other."""
    import threading

    log("two threads, two streams")
    gen = torch.Generator().manual_seed(17)
    shapes_a = [(128, 64)] * 15 + [(768,)]
    shapes_b = [(256, 128)]
    init = {k: [torch.randn(s, generator=gen) * 0.02 for s in sh] for k, sh in (("a", shapes_a), ("b", shapes_b))}
    grads = {k: [[H.heavy_tailed(s, gen) for s in sh] for _ in range(12)] for k, sh in (("a", shapes_a), ("b", shapes_b))}
    make = {"a": lambda ps: aw.ZIPSRAdamW4Bit(ps, quant_rng_seed=5, optimized=True, **ARGS),
            "b": lambda ps: aw.ZEEDENAdamW4Bit(ps, optimized=True, **ARGS)}

    def build(k):
        ps = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init[k]]
        gs = [[g.to(H.DEVICE) for g in step] for step in grads[k]]
        return ps, make[k](ps), gs

    def run(ps, opt, gs, stream):
        with torch.cuda.stream(stream):
            for step in gs:
                for p, g in zip(ps, step):
                    p.grad = g
                opt.step()
        stream.synchronize()

    # sequential reference, each on the default stream
    seq = {k: build(k) for k in ("a", "b")}
    torch.cuda.synchronize()
    for k in ("a", "b"):
        run(*seq[k], torch.cuda.current_stream())
    # concurrent: one thread and one stream each (default priority)
    con = {k: build(k) for k in ("a", "b")}
    torch.cuda.synchronize()
    streams = {k: torch.cuda.Stream() for k in ("a", "b")}
    errors = []

    def worker(k):
        try:
            run(*con[k], streams[k])
        except BaseException as e:  # surfaced in the main thread
            errors.append((k, e))

    threads = [threading.Thread(target=worker, args=(k,)) for k in ("a", "b")]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a stepping thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for k in ("a", "b"):
        (pa, oa, _), (pb, ob, _) = seq[k], con[k]
        for i, (x, y) in enumerate(zip(pa, pb)):
            same_state(oa, x, ob, y, f"{k} tensor {i}")
    log("  both threads bit-identical to the sequential runs")
