"""Seeded random configurations of the drop-in optimizer, stepped on the GPU and by the oracle
with the same inputs and draws (the bars of ``test_gpu_step``: round-to-nearest codes, block
scales and fp32 state bit-exact, no stochastic code parted, parameters within tolerance).

Each case draws its own mix: 1-3 parameter groups of 1-2 tensors, each group with an m1/m2
scheme pair the reference accepts (every m2 family: round-to-nearest with and without EDEN,
state-SR, update-SR with fp32 read-back, sampled read-back, store-EDEN, next-step bias, the
three lookahead forms, fp32), an optional nf4_sr retarget, the reference step or the optimized
one, fp32 / bf16 / fp16 parameters, tensors on the 4-bit path and on the fp32-state path
(fewer than 4,096 values or not a multiple of 128), betas on both sides of ATen's lerp switch,
weight decay on and off, the optimized step's chunk size (its draw accounting), and gradients
from heavy-tailed to tiny, with and without all-zero blocks.  Three steps each, so the second and
third reuse the first step's launch plan.  Eight more cases draw tensors of up to 33.6M values,
whose launches take 2, 3 or 4 tiles per wave, and 16 more (8 of the resume cases) draw the same
mixes with float64 parameters.  The configuration is printed before the case runs."""

from __future__ import annotations

import random

import pytest
import torch

import adamw4bit_amd as aw
from tests import gpu_helpers as H
from tests.test_gpu_step import compare_pair, log, run_pair

pytestmark = pytest.mark.gpu

M1 = ["nf4", "nf4_sr", "sdyn4", "sdyn4_sr", "fp32"]
# (m2 scheme, EDEN allowed)
M2 = [("dyn4_nz", True), ("dyn4", True), ("lin4_nz", True), ("lin4", True), ("lin4_sr", False),
      ("dyn4_sr", False), ("dyn4_upd_sr_fp32read", True), ("lin4_upd_sr_fp32read", True), ("fp32", False),
      ("dyn4_lookahead_sr", True), ("dyn4_upd_sr", True), ("lin4_upd_sr", True),
      ("dyn4_upd_sr_store_eden", False), ("lin4_upd_sr_store_eden", False),
      ("dyn4_upd_sr_fp32read_nextbc", True), ("dyn4_la_upd_sr", False), ("dyn4_proxy_la_upd_sr", False),
      ("dyn4_vproxy_la_upd_sr", False)]
LOOKAHEAD = {"dyn4_la_upd_sr", "dyn4_proxy_la_upd_sr", "dyn4_vproxy_la_upd_sr"}
SHAPES = [(4096,), (8192,), (128, 64), (256, 96), (300, 128), (64, 768), (40, 256),  # 4-bit path
          (4097,), (1000,), (768,), (5, 7), (129,), (128,)]                          # fp32 state
GRADS = {
    "heavy": None,  # Student-t(3) x per-row log-normal(-7, 1): run_pair's default
    "normal": lambda s, g: torch.randn(s, generator=g) * 1e-3,
    "tiny": lambda s, g: torch.randn(s, generator=g) * 1e-9,
    "unit": lambda s, g: torch.randn(s, generator=g),
}


# Larger tensors, whose launches take 2, 3 or 4 tiles per wave (the pool above stays at one)
LARGE_SHAPES = [(4096, 4096), (8192, 4096), (2048, 2048), (1024, 1024), (768,), (4097,), (128, 64)]


def draw_case(seed: int, shapes=SHAPES) -> dict:
    rng = random.Random(seed)
    dtype = rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    groups = []
    for _ in range(rng.randint(1, 3)):
        m2, eden_ok = rng.choice(M2)
        m1 = rng.choice(["fp32", "nf4"] if m2 in LOOKAHEAD else M1)
        eden = eden_ok and rng.random() < 0.5
        groups.append(dict(m1=m1, m2=m2, eden=eden, shapes=[rng.choice(shapes) for _ in range(rng.randint(1, 2))]))
    grads = rng.choice(list(GRADS))
    return dict(
        seed=seed, dtype=dtype, groups=groups, grads=grads,
        optimized=rng.random() < 0.6,
        lr=rng.choice([1e-4, 1e-3, 3e-2]),
        betas=rng.choice([(0.9, 0.95), (0.9, 0.999), (0.4, 0.45)]),
        eps=rng.choice([1e-8, 1e-6]),
        weight_decay=rng.choice([0.0, 0.1]),
        zero_blocks=rng.choice([0.0, 0.05]),
        retarget=rng.random() < 0.3,
        quant_rng_seed=rng.randrange(1 << 20),
        chunk=rng.choice([None, None, 1024, 4096]),  # the optimized step's chunk (its draw accounting)
    )


@pytest.mark.parametrize("seed", range(96))
def test_random_configuration_matches_oracle(seed):
    _check_against_oracle(seed, draw_case(seed))


@pytest.mark.parametrize("seed", range(7000, 7016))
def test_random_float64_configuration_matches_oracle(seed):
    """Configurations drawn the same way with float64 parameters, which the generic kernel updates
    in float64 (gradients read as fp32, fp32 moments and denominator)."""
    _check_against_oracle(seed, dict(draw_case(seed), dtype=torch.float64))


@pytest.mark.parametrize("seed", range(5005, 5013))
def test_large_random_configuration_matches_oracle(seed):
    """The same with tensors of up to 33.6M values (launches of 2-4 tiles per wave)."""
    _check_against_oracle(seed, draw_case(seed, LARGE_SHAPES))


def _check_against_oracle(seed: int, case: dict) -> None:
    log(f"random case {seed}: {case}")
    shapes, pairs = [], []
    for g in case["groups"]:
        for s in g["shapes"]:
            shapes.append(s)
            pairs.append((g["m1"], g["m2"], g["eden"]))
    retarget = None
    if case["retarget"]:
        cand = [i for i, (m1, m2, _) in enumerate(pairs) if m1 in ("nf4", "nf4_sr") and m2 not in LOOKAHEAD]
        if cand:
            retarget = ([cand[0]], "nf4_sr" if pairs[cand[0]][0] == "nf4" else "nf4")

    def make(ps):
        groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b, use_eden_m2=e) for p, (a, b, e) in zip(ps, pairs)]
        opt = aw.QuantizedAdamW(groups, lr=case["lr"], betas=case["betas"], eps=case["eps"],
                                weight_decay=case["weight_decay"], m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz",
                                quant_rng_seed=case["quant_rng_seed"], optimized=case["optimized"])
        if case["optimized"] and case["chunk"]:
            for group in opt.param_groups:
                group["max_chunk_numel"] = case["chunk"]
        return opt

    out = run_pair(make, shapes, case["dtype"], 3, seed=case["quant_rng_seed"], grad_seed=1000 + seed,
                   m1_override=retarget, zero_block_frac=case["zero_blocks"], grad_fn=GRADS[case["grads"]])
    compare_pair(*out, f"random case {seed}", steps=3)


def _flat_state(opt, p) -> dict:
    """Every entry of a parameter's optimizer state, tensors as bit patterns on the host."""
    from adamw4bit_amd.quantization import QuantState
    out = {}
    for key, value in opt.state[p].items():
        if isinstance(value, torch.Tensor):
            out[key] = H.bits(value)
        elif isinstance(value, QuantState):
            out[key] = (H.bits(value.absmax), tuple(value.shape) if value.shape is not None else None,
                        value.dtype, value.blocksize, value.packed)
        else:
            out[key] = value
    return out


@pytest.mark.parametrize("seed", range(24))
def test_random_configuration_resumes_exactly(seed, tmp_path):
    """Seeded random configurations (other draws than the oracle cases): two steps, a checkpoint
    written and read back with ``weights_only=True``, three more steps on fresh parameter objects
    is bit-identical to five uninterrupted steps: parameters and every state entry (codes, block
    scales, fp32 and pending lookahead state, the store-EDEN denominators, step counts), which
    also pins the random streams' positions across the checkpoint."""
    _check_resume(seed, draw_case(1000 + seed), tmp_path)


@pytest.mark.parametrize("seed", range(8))
def test_random_float64_configuration_resumes_exactly(seed, tmp_path):
    """The same with float64 parameters."""
    _check_resume(seed, dict(draw_case(1100 + seed), dtype=torch.float64), tmp_path)


def _check_resume(seed: int, case: dict, tmp_path) -> None:
    log(f"resume case {seed}: {case}")
    shapes, pairs = [], []
    for g in case["groups"]:
        for s in g["shapes"]:
            shapes.append(s)
            pairs.append((g["m1"], g["m2"], g["eden"]))
    dtype = case["dtype"]
    gen = torch.Generator().manual_seed(2000 + seed)
    grad_fn = GRADS[case["grads"]] or H.heavy_tailed
    init = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in shapes]
    grads = [[grad_fn(s, gen).to(dtype) for s in shapes] for _ in range(5)]
    cand = [i for i, (m1, m2, _) in enumerate(pairs) if m1 in ("nf4", "nf4_sr") and m2 not in LOOKAHEAD]
    retarget = cand[:1] if case["retarget"] else []

    def make(ps):
        groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b, use_eden_m2=e) for p, (a, b, e) in zip(ps, pairs)]
        opt = aw.QuantizedAdamW(groups, lr=case["lr"], betas=case["betas"], eps=case["eps"],
                                weight_decay=case["weight_decay"], m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz",
                                quant_rng_seed=case["quant_rng_seed"], optimized=case["optimized"])
        if case["optimized"] and case["chunk"]:
            for group in opt.param_groups:
                group["max_chunk_numel"] = case["chunk"]
        if retarget:
            opt.set_m1_quant_scheme_for_parameters([ps[i] for i in retarget],
                                                   "nf4_sr" if pairs[retarget[0]][0] == "nf4" else "nf4")
        return opt

    def run(opt, ps, steps):
        for k in steps:
            for p, g in zip(ps, grads[k]):
                p.grad = g.to(H.DEVICE)
            opt.step()

    a = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = make(a)
    run(oa, a, range(5))
    b = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    ob = make(b)
    run(ob, b, range(2))
    torch.save(ob.state_dict(), tmp_path / "ckpt.pt")
    sd = torch.load(tmp_path / "ckpt.pt", weights_only=True)
    c = [torch.nn.Parameter(p.detach().clone()) for p in b]
    oc = make(c)
    oc.load_state_dict(sd)
    run(oc, c, range(2, 5))
    torch.cuda.synchronize()
    for i, (pa, pc) in enumerate(zip(a, c)):
        assert torch.equal(H.bits(pa), H.bits(pc)), (seed, i, "parameter")
        sa, sc = _flat_state(oa, pa), _flat_state(oc, pc)
        assert set(sa) == set(sc), (seed, i, sorted(sa), sorted(sc))
        for key in sa:
            va, vc = sa[key], sc[key]
            if isinstance(va, torch.Tensor):
                assert torch.equal(va, vc), (seed, i, key)
            elif isinstance(va, tuple):
                assert torch.equal(va[0], vc[0]) and va[1:] == vc[1:], (seed, i, key)
            else:
                assert va == vc, (seed, i, key)
    log(f"  {len(a)} parameters bit-identical after resume")
