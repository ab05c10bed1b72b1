"""The benchmark workloads at full size on the GPU: the Llama-3-8B parameter set (291 tensors,
8,030,261,248 values) in fp32 under ZE-EDEN and ZIP-SR, and in bf16 under the mixed-scheme
stress case (ZIP-SR everywhere, the LM head's first moment nf4_sr, every tenth tensor an
fp32-m2 or EDEN-m2 ablation, 1% zero gradient blocks); and the fp32 set under the reference
step's research m2 schemes (read-back, store-EDEN, lookahead proxy and pending lookahead).  Each
step is one launch over all tensors, as the benchmark runs it.

Checked two ways, every step:
* every tensor, at full size, against what the step guarantees whatever the inputs: finite
  parameters, finite scales, raw scales at or above the 1e-12 floor (EDEN scales: positive,
  or 0 for an all-zero block), no code 0 in a zero-floored (dyn4_nz) moment, the step count;
* a sample -- the embedding, all nine tensors of the first layer, the final norm, the LM head,
  and for the mixed case the ablation tensors -- against the oracle on the CPU, fed the
  uniforms of the device's Philox stream at the positions the launch table gave each tensor
  (a tensor's result does not depend on the other rows of its launch), with the update-SR
  preconditioner's square root correctly rounded.  Codes, scales and fp32 states bit-exact,
  stochastic codes included (no value may part), parameters within tolerance.

About 75 GB of device memory and 15 GB of host memory; about a minute per test."""

from __future__ import annotations

import math

import pytest
import torch

import adamw4bit_amd as aw
import bench
from adamw4bit_amd import _lib
from oracle import reference_step as ref
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

STEPS = 3
LAYER0 = list(range(1, 10))   # q, k, v, o, gate, up, down, two RMSNorm vectors
FINAL_NORM, HEAD = 289, 290


def log(msg):
    print(msg, flush=True)


class TableDraws:
    """Oracle ``draw_fn`` for one tensor of a bigger launch: the write of step k draws from the
    stream position its row had in that step's launch table; at step 1 the zero-state encode
    asks first, and its draws never change a code (every value is an exact level)."""

    def __init__(self, seeds):
        self.seeds = seeds
        self.cursor = {}
        self.first = {}

    def start(self, offsets, first):
        self.cursor = dict(offsets)
        self.first = {m: first for m in offsets}

    def __call__(self, moment, n):
        if self.first.get(moment):
            self.first[moment] = False
            return torch.zeros(n)
        offset = self.cursor[moment]
        self.cursor[moment] = offset + (n + 127) // 128 * 128
        return H.uniforms_gpu(self.seeds[moment], offset, n).cpu()


def capture_tables(monkeypatch):
    tables = []
    real = _lib.fused_step

    def record(table, stream):
        tables.append(table.copy())
        real(table, stream)

    monkeypatch.setattr(_lib, "fused_step", record)
    return tables


def make_grads(shapes, seed, dtype, zero_blocks):
    gen = torch.Generator(device=H.DEVICE).manual_seed(seed + 1)
    grads = bench.make_grads(shapes, torch.device(H.DEVICE), seed=seed)
    out = []
    for g in grads:
        if zero_blocks and g.numel() % 128 == 0:
            nb = g.numel() // 128
            g.view(nb, 128)[torch.rand(nb, generator=gen, device=H.DEVICE) < zero_blocks] = 0.0
        out.append(g.to(dtype))
    return out


def check_invariants(opt, params, schemes, step):
    """Full-size checks of every tensor after a step."""
    bad = []
    for i, (p, (m1, m2, eden)) in enumerate(zip(params, schemes)):
        st = opt.state[p]
        assert st["step"] == step, (i, st["step"])
        if not bool(torch.isfinite(p).all()):
            bad.append((i, "param not finite"))
        for m, scheme, is_eden in (("m1", m1, False), ("m2", m2, eden)):
            if m == "m2" and "lookahead_pending_exp_avg_sq" in st:  # pending lookahead: fp32 state
                assert bool(torch.isfinite(st["lookahead_pending_exp_avg_sq"]).all()), (i, m)
                continue
            if f"{m}_code" not in st:
                assert bool(torch.isfinite(st[m]).all()), (i, m)
                continue
            s = st[f"{m}_quant_state"].absmax
            if not bool(torch.isfinite(s).all()):
                bad.append((i, f"{m} scale not finite"))
            if is_eden:
                if not bool((s >= 0).all()):
                    bad.append((i, f"{m} EDEN scale negative"))
            elif not bool((s >= 1e-12).all()):
                bad.append((i, f"{m} scale below the floor"))
            if scheme == "dyn4_nz":
                c = st[f"{m}_code"]
                if bool(((c & 0x0F) == 0).any()) or bool(((c >> 4) == 0).any()):
                    bad.append((i, f"{m} zero-floored moment holds code 0"))
    assert not bad, bad[:10]


def compare(opt, p, oracle, cpu_param, parted, what, dtype):
    """One sampled tensor against its oracle; returns (parted values, stochastic codes)."""
    st = H.state_of(opt, p)
    ost = H.oracle_state((oracle.states[0].m1, oracle.states[0].m2))
    assert set(st) - {"step"} == set(ost), (what, sorted(st), sorted(ost))
    stochastic = 0
    for m, ms in (("m1", oracle.states[0].m1), ("m2", oracle.states[0].m2)):
        if f"{m}_code" in ost:
            flips = H.code_mismatch(st[f"{m}_code"], ost[f"{m}_code"])
            if ref.is_stochastic(ms.scheme):
                stochastic += p.numel()
                log(f"  {what} {m} ({ms.scheme}): {flips} codes differ at the last step")
            else:
                assert flips == 0, f"{what} {m} ({ms.scheme}): {flips} flips"
                assert torch.equal(H.bits(st[f"{m}_scale"]), H.bits(ost[f"{m}_scale"])), (what, m)
        elif f"{m}_pending" in ost:  # a pending lookahead m2: its sampled fp32 state, bit-exact
            same = torch.equal(H.bits(st[f"{m}_pending"].reshape(-1)), H.bits(ost[f"{m}_pending"].reshape(-1)))
            assert same, (what, m)
            log(f"  {what} {m} ({ms.scheme}): pending state bit-exact")
        else:
            assert torch.equal(H.bits(st[f"{m}_fp32"].reshape(-1)), H.bits(ost[f"{m}_fp32"])), (what, m)
    exact = H.assert_params_close(p, cpu_param, what, steps=STEPS if dtype != torch.float32 else 1,
                                  exclude=parted)
    n_parted = int(parted.sum())
    log(f"  {what} {tuple(p.shape)}: parameters bit-exact {exact:.6f}; values parted {n_parted}")
    return n_parted, stochastic


def run_full(monkeypatch, make_opt, schemes, dtype, zero_blocks, sampled, seed, init_draws=True):
    """init_draws: the first step's zero-state encode of a stochastic moment asks for draws (the
    lookahead schemes store their zero state without any)."""
    shapes = bench.llama3_8b_shapes()
    assert sum(math.prod(s) for s in shapes) == 8_030_261_248 and len(shapes) == 291
    gen = torch.Generator(device=H.DEVICE).manual_seed(seed)
    params = [torch.nn.Parameter((torch.randn(s, generator=gen, device=H.DEVICE) * 0.02).to(dtype))
              for s in shapes]
    opt = make_opt(params)
    cpu = {i: params[i].detach().cpu().clone() for i in sampled}
    hp = opt.param_groups[0]
    hyper = ref.Hyper(hp["lr"], tuple(hp["betas"]), hp["eps"], hp["weight_decay"])
    seeds = {m: opt._stream(m, params[0].device).seed for m in ("m1", "m2")}
    draws = {i: TableDraws(seeds) for i in sampled}
    oracles = {i: ref.Oracle([cpu[i]], hyper, [schemes[i][0]], [schemes[i][1]], [schemes[i][2]],
                             seed=0, optimized=True, draw_fn=draws[i], usr_sqrt="cr") for i in sampled}
    parted = {i: torch.zeros(params[i].numel(), dtype=torch.bool) for i in sampled}
    tables = capture_tables(monkeypatch)
    for k in range(STEPS):
        grads = make_grads(shapes, seed + 10 * (k + 1), dtype, zero_blocks)
        for p, g in zip(params, grads):
            p.grad = g
        del grads
        opt.step()
        torch.cuda.synchronize()
        assert len(tables) == k + 1 and len(tables[k]) == 291
        log(f"step {k + 1}: launched; invariants over all 291 tensors")
        check_invariants(opt, params, schemes, k + 1)
        for i in sampled:
            row = tables[k][i]
            offsets = {m: int(row[m]["rng_offset"]) for m, s in (("m1", schemes[i][0]), ("m2", schemes[i][1]))
                       if s != "fp32" and ref.is_stochastic(s)}
            draws[i].start(offsets, first=(k == 0 and init_draws))
            oracles[i].step([params[i].grad.cpu()])
            st = H.state_of(opt, params[i])
            for m, ms in (("m1", oracles[i].states[0].m1), ("m2", oracles[i].states[0].m2)):
                if ref.is_stochastic(ms.scheme) and f"{m}_code" in st:
                    parted[i] |= H.code_diff_mask(st[f"{m}_code"], ms.codes, params[i].numel())
        log(f"step {k + 1}: oracle on {len(sampled)} sampled tensors done")
    total_parted = total_codes = 0
    for i in sampled:
        n_parted, n_codes = compare(opt, params[i], oracles[i], cpu[i], parted[i], f"tensor {i}", dtype)
        total_parted += n_parted
        total_codes += n_codes
    log(f"parted values {total_parted} of {total_codes} stochastic codes")
    assert total_parted == 0, (total_parted, total_codes)
    del params, opt, oracles
    torch.cuda.empty_cache()


@pytest.mark.parametrize("recipe", ["zeeden", "zipsr"])
def test_llama3_8b_fp32_full_size(monkeypatch, recipe):
    log(f"Llama-3-8B fp32 at full size, {recipe}, {STEPS} steps")
    if recipe == "zeeden":
        make = lambda ps: aw.ZEEDENAdamW4Bit(ps, optimized=True, quant_rng_seed=0)  # noqa: E731
        per = ("nf4", "dyn4_nz", True)
    else:
        make = lambda ps: aw.ZIPSRAdamW4Bit(ps, optimized=True, quant_rng_seed=0)  # noqa: E731
        per = ("nf4", "dyn4_upd_sr_fp32read", False)
    schemes = [per] * 291
    sampled = [0] + LAYER0 + [FINAL_NORM, HEAD]
    run_full(monkeypatch, make, schemes, torch.float32, 0.0, sampled, seed=41)


def test_llama3_8b_bf16_mixed_full_size(monkeypatch):
    log(f"Llama-3-8B bf16 mixed-scheme stress case at full size, {STEPS} steps")
    shapes = bench.llama3_8b_shapes()
    groups, per = bench.mixed_bf16_groups([torch.empty(0)] * len(shapes))
    schemes = [(m1, m2, g["use_eden_m2"]) for (m1, m2), g in zip(per, groups)]

    def make(ps):
        groups, _ = bench.mixed_bf16_groups(ps)
        opt = aw.QuantizedAdamW(groups, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_upd_sr_fp32read",
                                optimized=True, quant_rng_seed=0)
        opt.set_m1_quant_scheme_for_parameters([ps[HEAD]], "nf4_sr")
        return opt

    assert schemes[5][1] == "fp32" and schemes[15][2] and schemes[HEAD][0] == "nf4_sr"
    sampled = [0] + LAYER0 + [15, FINAL_NORM, HEAD]  # 5: fp32-m2 ablation, 15: EDEN-m2 ablation
    run_full(monkeypatch, make, schemes, torch.bfloat16, 0.01, sampled, seed=43)


@pytest.mark.parametrize("m2", ["dyn4_upd_sr", "dyn4_upd_sr_store_eden", "dyn4_proxy_la_upd_sr", "dyn4_la_upd_sr"])
def test_llama3_8b_research_m2_full_size(monkeypatch, m2):
    """The reference step's research m2 schemes over the whole Llama-3-8B fp32 set (one launch of
    their specialised kernel, twelve tiles per wave at this size), NF4 m1: invariants on every
    tensor, and the oracle on the first layer's small tensors and the norms (codes, scales and the
    pending lookahead state bit-exact; store-EDEN's kept 1 / denominator is checked at smaller
    sizes by test_gpu_step.py)."""
    log(f"Llama-3-8B fp32 at full size, nf4 + {m2}, {STEPS} steps")
    make = lambda ps: aw.QuantizedAdamW(ps, m1_quant_scheme="nf4", m2_quant_scheme=m2,  # noqa: E731
                                        optimized=True, quant_rng_seed=0)
    schemes = [("nf4", m2, False)] * 291
    sampled = [2, 3, 8, 9, FINAL_NORM]  # k and v projections (1024x4096), the layer's RMSNorm vectors
    run_full(monkeypatch, make, schemes, torch.float32, 0.0, sampled, seed=47, init_draws="la" not in m2)
