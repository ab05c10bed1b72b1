"""``aw4_fused_step_noalloc`` (no device allocation) against ``aw4_fused_step``: the same rows
give bit-identical parameters and moment state, on two calls in a row, the second with fewer
and smaller tensors (the fixed table area keeps the last call's contents)."""

from __future__ import annotations

import pytest
import torch

import adamw4bit_amd as aw
from adamw4bit_amd import _lib

from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu


def _same(oa, pa, ob, pb, what):
    assert torch.equal(H.bits(pa), H.bits(pb)), what
    sa, sb = H.state_of(oa, pa), H.state_of(ob, pb)
    assert sa.keys() == sb.keys() and sa["step"] == sb["step"], what
    for key in sa:
        if key != "step":
            assert torch.equal(H.bits(sa[key]), H.bits(sb[key])), (what, key)


@pytest.mark.parametrize("recipe", ["zeeden", "zipsr"])
def test_noalloc_step_matches_fused_step(monkeypatch, recipe):
    print(f"noalloc vs fused step ({recipe})", flush=True)
    gen = torch.Generator().manual_seed(23)
    shapes = [(1024, 1024), (768,), (256, 384), (1000,), (64, 512)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    make = aw.ZIPSRAdamW4Bit if recipe == "zipsr" else aw.ZEEDENAdamW4Bit
    kw = dict(optimized=True, quant_rng_seed=12 if recipe == "zipsr" else None)
    oa, ob = make(pa, **kw), make(pb, **kw)
    regular = _lib.fused_step
    calls = []

    def noalloc(table, stream):
        calls.append(len(table))
        _lib.fused_step_noalloc(table, stream)

    # call 1: every tensor; call 2: only the three small ones (fewer rows, fewer tiles)
    for k, with_grad in enumerate(([0, 1, 2, 3, 4], [1, 3, 4])):
        for i, (a, b, s) in enumerate(zip(pa, pb, shapes)):
            g = H.heavy_tailed(s, gen).to(H.DEVICE) if i in with_grad else None
            a.grad = None if g is None else g.clone()
            b.grad = None if g is None else g.clone()
        oa.step()
        monkeypatch.setattr(_lib, "fused_step", noalloc)
        ob.step()
        monkeypatch.setattr(_lib, "fused_step", regular)
        torch.cuda.synchronize()
        for i in with_grad:
            _same(oa, pa[i], ob, pb[i], (k, i))
    assert calls == [5, 3]
