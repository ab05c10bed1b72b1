"""``HipOptimizedBackend`` on the GPU, driven by the reference optimizer's step loop
(``adamw.py:497-502``, through the stand-in of tests/reference_like.py): every parameter the
reference's preflight takes is stepped in place (``True``), with the reference optimizer's state
layout and its per-moment generators as the random stream; parameters, moment state and the
stream positions are bit-identical to this package's own QuantizedAdamW with the same seed, one
launch per parameter or one per step (``deferred=True`` and ``flush``), and a checkpoint of the
reference optimizer's state and generators resumes exactly.  A declined parameter changes
nothing and consumes no draws."""

from __future__ import annotations

import copy

import pytest
import torch

import adamw4bit_amd as aw
from adamw4bit_amd.backend import HipOptimizedBackend
from adamw4bit_amd.quantization import QuantState

from tests import gpu_helpers as H
from tests.reference_like import ReferenceLikeOptimizer
from tests.test_backend_host import StubReferenceBackend

pytestmark = pytest.mark.gpu

HYPER = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
SHAPES = [(256, 512), (768,), (64, 4096), (1000,), (128, 256)]
DTYPES = [torch.float32, torch.float64, torch.bfloat16, torch.float32, torch.float64]


def same(oa, pa, ob, pb, what):
    assert torch.equal(H.bits(pa.detach()), H.bits(pb.detach())), what
    sa, sb = H.state_of(oa, pa), H.state_of(ob, pb)
    assert sa.keys() == sb.keys() and sa["step"] == sb["step"], (what, sorted(sa), sorted(sb))
    for key in sa:
        if key != "step":
            assert torch.equal(H.bits(sa[key]), H.bits(sb[key])), (what, key)


def make_pair(gen, deferred, seed):
    init = [(torch.randn(s, generator=gen) * 0.02).to(dt) for s, dt in zip(SHAPES, DTYPES)]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    ref = ReferenceLikeOptimizer(pa, backend=HipOptimizedBackend, deferred=deferred,
                                 reference_backend=StubReferenceBackend(False), quant_state_type=QuantState,
                                 quant_rng_seed=seed, **HYPER)
    own = aw.QuantizedAdamW(pb, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_upd_sr_fp32read", use_eden_m2=False,
                            optimized=True, quant_rng_seed=seed, **HYPER)
    return ref, pa, own, pb


def set_grads(params, grads):
    for p, g in zip(params, grads):
        p.grad = g.to(p.dtype).to(H.DEVICE)


@pytest.mark.parametrize("deferred", [False, True])
def test_reference_optimizer_steps_like_the_package_optimizer(deferred):
    print(f"reference optimizer through HipOptimizedBackend (deferred={deferred})", flush=True)
    gen = torch.Generator().manual_seed(61)
    ref, pa, own, pb = make_pair(gen, deferred, seed=7)
    for k in range(3):
        grads = [H.heavy_tailed(s, gen) for s in SHAPES]
        set_grads(pa, grads)
        set_grads(pb, grads)
        ref.step()
        own.step()
        torch.cuda.synchronize()
        assert ref.declined == []
        for i, (a, b) in enumerate(zip(pa, pb)):
            same(ref, a, own, b, (k, i))
        assert all(isinstance(ref.state[a]["m1_quant_state"], QuantState) for a in pa if a.numel() >= 4096)
    # the generators' offsets are the streams' positions: a checkpoint of state and generators
    # resumes exactly
    saved = copy.deepcopy(ref.state_dict())
    saved_generators = {m: {d: s.clone() for d, s in g.items()} for m, g in ref.generator_states().items()}
    saved_params = [a.detach().clone() for a in pa]
    pc = [torch.nn.Parameter(t.clone()) for t in saved_params]
    resumed = ReferenceLikeOptimizer(pc, backend=HipOptimizedBackend, deferred=deferred,
                                     reference_backend=StubReferenceBackend(False), quant_state_type=QuantState,
                                     quant_rng_seed=7, **HYPER)
    resumed.load_state_dict(saved)
    resumed.set_generator_states(saved_generators)
    for k in range(2):
        grads = [H.heavy_tailed(s, gen) for s in SHAPES]
        for ps in (pa, pb, pc):
            set_grads(ps, grads)
        ref.step()
        own.step()
        resumed.step()
        torch.cuda.synchronize()
        assert resumed.declined == []
        for i, (a, b, c) in enumerate(zip(pa, pb, pc)):
            same(ref, a, own, b, ("continued", k, i))
            same(ref, a, resumed, c, ("resumed", k, i))
    print("  5 steps bit-identical; checkpoint resumed exactly", flush=True)


def test_declined_parameter_changes_nothing_and_draws_nothing():
    """A parameter the reference's preflight declines (here: a gradient that overlaps its parameter)
    is left to the reference's step; nothing of it changes and its moment's generator does not move."""
    gen = torch.Generator().manual_seed(67)
    p = torch.nn.Parameter((torch.randn(64, 4096, generator=gen) * 0.02).to(H.DEVICE))
    q = torch.nn.Parameter((torch.randn(64, 4096, generator=gen) * 0.02).to(H.DEVICE))
    ref = ReferenceLikeOptimizer([p, q], backend=HipOptimizedBackend, reference_backend=StubReferenceBackend(False),
                                 quant_state_type=QuantState, quant_rng_seed=3, **HYPER)
    q.grad = (torch.randn(64, 4096, generator=gen) * 1e-3).to(H.DEVICE)
    p.grad = p.detach()  # the gradient is the parameter's own storage: _plan declines it
    before = p.detach().clone()
    ref.step()
    torch.cuda.synchronize()
    assert ref.declined == [p] and p not in ref.state
    assert torch.equal(p.detach(), before)
    m2 = ref._quant_generator("m2", p.device)
    taken = m2.get_offset()
    # q alone consumed draws: its m2 initialisation (the whole tensor: one chunk) and one write,
    # each 128 positions per 4 units of the generator's offset
    assert taken == 2 * q.numel() // 128 * 4
