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


def test_noalloc_step_replays_from_a_hip_graph():
    """The no-allocation step captured in a graph (torch.cuda.graph over the library call on the
    capturing stream) and replayed three times, with other eager work and synchronizations
    between the replays: each replay leaves the parameters and moment state bit-identical to
    the same launch table called eagerly the same number of times from the same start."""
    print("noalloc step under graph capture", flush=True)
    gen = torch.Generator().manual_seed(31)
    shapes = [(128, 64), (256, 128), (768,)]
    params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(H.DEVICE)) for s in shapes]
    opt = aw.ZIPSRAdamW4Bit(params, quant_rng_seed=8, optimized=True)
    captured = []
    regular = _lib.fused_step
    for k in range(2):
        for p, s in zip(params, shapes):
            p.grad = H.heavy_tailed(s, gen).to(H.DEVICE)
        if k == 1:
            _lib.fused_step = lambda t, st: (captured.append(t.copy()), regular(t, st))
        try:
            opt.step()
        finally:
            _lib.fused_step = regular
    table = captured[-1]
    # everything the table's launch writes, to restore between the eager and the graph runs
    written = []
    for p in params:
        written.append(p.data)
        for key in ("m1_code", "m2_code", "m1", "m2"):
            if isinstance(opt.state[p].get(key), torch.Tensor):
                written.append(opt.state[p][key])
        for key in ("m1_quant_state", "m2_quant_state"):
            if opt.state[p].get(key) is not None:
                written.append(opt.state[p][key].absmax)
    torch.cuda.synchronize()
    start = [t.clone() for t in written]

    def snapshot():
        torch.cuda.synchronize()
        return [H.bits(t) for t in written]

    stream = torch.cuda.current_stream()
    eager = []
    for _ in range(3):
        _lib.fused_step_noalloc(table, stream.cuda_stream)
        eager.append(snapshot())
    for t, s in zip(written, start):
        t.copy_(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.fused_step_noalloc(table, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for t, s in zip(written, start):  # capture runs nothing; restore anyway
        t.copy_(s)
    other = torch.randn(1 << 20, device=H.DEVICE)
    for k in range(3):
        graph.replay()
        got = snapshot()
        for i, (a, b) in enumerate(zip(got, eager[k])):
            assert torch.equal(a, b), (k, i)
        other.mul_(1.0001)
        torch.cuda.synchronize()
    print("  3 replays bit-identical to the eager calls", flush=True)


def test_noalloc_step_allocates_no_device_memory():
    """The entry point's contract itself: after the first call on the device, calls with a launch
    table near the 1 MiB limit (3,000 tensors) leave the device's free memory unchanged, and one is
    captured in a graph under torch's global capture mode, which refuses calls that are unsafe
    during capture, then replayed."""
    print("noalloc step: no device allocation", flush=True)
    gen = torch.Generator().manual_seed(41)
    count = 3000
    params = [torch.nn.Parameter((torch.randn(4096, generator=gen) * 0.02).to(H.DEVICE)) for _ in range(count)]
    opt = aw.ZIPSRAdamW4Bit(params, quant_rng_seed=3, optimized=True)
    for p in params:
        p.grad = (torch.randn(4096, generator=gen) * 1e-3).to(H.DEVICE)
    captured = []
    regular = _lib.fused_step
    _lib.fused_step = lambda t, st: (captured.append(t.copy()), regular(t, st))
    try:
        opt.step()
    finally:
        _lib.fused_step = regular
    (table,) = captured
    assert len(table) == count
    nbytes = 64 + count * _lib.TENSOR.itemsize + (count + 1) * 8
    assert 0.8 * _lib.NOALLOC_TABLE_BYTES < nbytes < _lib.NOALLOC_TABLE_BYTES
    stream = torch.cuda.current_stream()
    _lib.fused_step_noalloc(table, stream.cuda_stream)  # warm-up: the device's first call
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(5):
        _lib.fused_step_noalloc(table, stream.cuda_stream)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="global"):
        _lib.fused_step_noalloc(table, torch.cuda.current_stream().cuda_stream)
    graph.replay()
    torch.cuda.synchronize()
    print(f"  free device memory {free0} -> {free1} over 5 calls; graph captured and replayed", flush=True)
