"""Parity of the fused HIP step with the CPU oracle and the reference's golden fixtures.

Bars (stated per comparison):
* codes and block scales of round-to-nearest moments: bit-exact;
* codes of stochastic moments fed the same uniforms: bit-exact against the oracle with the
  update-SR preconditioner's square root correctly rounded (``usr_sqrt="cr"``): no value may
  part.  Against fixtures the reference wrote, whose host square root is within one ulp of
  the correctly rounded one, update-SR codes may differ where that root does (budget 1e-5 of
  the codes; the count is logged);
* fp32-state moments: bit-exact;
* parameters: within 1e-6 relative (fp32) / one storage ulp (bf16, fp16), because the
  reference's CPU square root is up to 1 ulp below the correctly rounded one and the
  kernel's update term is faithful (within 3 ulps).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import adamw4bit_amd as aw
from adamw4bit_amd import _lib
from adamw4bit_amd import quantization as q
from oracle import philox
from oracle import reference_step as ref
from tests import gpu_helpers as H
from tests._fixtures import load, tensor, trajectory_names

pytestmark = pytest.mark.gpu
SR_BUDGET = 1e-5


def stream():
    return torch.cuda.current_stream().cuda_stream


def log(msg):
    print(msg, flush=True)


def test_host_sqrt_rounding_report():
    """Record how often this host's ATen CPU sqrt (the oracle's) differs from the correctly
    rounded square root the kernel computes; parameter comparisons depend on it."""
    x = torch.rand(1 << 20, generator=torch.Generator().manual_seed(0)) * 1e-3
    cr = np.sqrt(x.numpy().astype(np.float64)).astype(np.float32)
    ulps = x.sqrt().numpy().view(np.int32).astype(np.int64) - cr.view(np.int32)
    log(f"host {torch.backends.cpu.get_cpu_capability()}: ATen sqrt differs from correctly rounded on "
        f"{np.mean(ulps != 0):.4%} of values (ulp offsets {sorted(set(np.unique(ulps).tolist()))})")
    assert np.abs(ulps).max() <= 1


# ---------------------------------------------------------------------------
# Random draws
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("seed,offset,n", [(0, 0, 4096), (0x1A2B3C4D, 128, 1000), ((1 << 63) - 5, 1 << 34, 8192),
                                           (1584363401, 4 * 12345, 333), (99, (1 << 40) + 100, 700)])
def test_uniforms_match_cpu_philox(seed, offset, n):
    log(f"uniforms seed={seed} offset={offset} n={n}")
    got = H.uniforms_gpu(seed, offset, n).cpu().numpy()
    assert np.array_equal(got, philox.uniforms(seed, offset, n))
    assert got.min() >= 0.0 and got.max() < 1.0


# ---------------------------------------------------------------------------
# Codec (aw4_quantize / aw4_dequantize) against the reference's chunk codec vectors
# ---------------------------------------------------------------------------

def moment_desc(mode, eden, guards, codes, scales, draws=None, bias=1.0, eps=1e-8):
    cb, rounding, floor_zero = q.SCHEMES[mode]
    m = np.zeros((), dtype=_lib.MOMENT)
    m["codes"], m["scales"] = codes.data_ptr(), scales.data_ptr()
    m["codebook"], m["rounding"] = cb, rounding
    flags = (_lib.MOMENT_ZERO_FLOOR if floor_zero else 0) | (_lib.MOMENT_EDEN if eden else 0)
    flags |= _lib.MOMENT_GUARDS if guards else 0
    if draws is not None:
        m["draws"] = draws.data_ptr()
        flags |= _lib.MOMENT_EXT_DRAWS
    m["flags"] = flags
    b = np.float32(max(bias, 1e-12))
    m["sr_bias"], m["sr_bias_rcp"], m["sr_eps"] = b, np.float32(1) / b, np.float32(eps)
    return m


def gpu_encode(values, mode, eden, guards, draws=None, bias=1.0, eps=1e-8):
    n = values.numel()
    v = values.to(H.DEVICE).contiguous()
    codes = torch.empty(n // 2, dtype=torch.uint8, device=H.DEVICE)
    scales = torch.empty(n // 128, dtype=torch.float32, device=H.DEVICE)
    d = draws.reshape(-1).to(H.DEVICE).contiguous() if draws is not None else None
    m = moment_desc(mode, eden, guards, codes, scales, d, bias, eps)
    _lib.quantize(v.data_ptr(), n, m, stream())
    torch.cuda.synchronize()
    return codes.cpu(), scales.cpu()


def test_codec_vectors():
    entries, arrays = load("codec_vectors.npz")
    for e in entries:
        k = e["key"]
        log(f"codec vector {k}")
        values = torch.from_numpy(arrays[f"{k}_values"])
        draws = torch.from_numpy(arrays[f"{k}_draws"]) if e["stochastic"] else None
        codes, scales = gpu_encode(values, e["mode"], e["eden"], True, draws, e["bias"], e["eps"])
        expect_codes = torch.from_numpy(arrays[f"{k}_codes"])
        got = q.unpack_4bit_codes(codes, numel=values.numel())
        flips = int((got != expect_codes).sum())
        if e["stochastic"] and "upd" in e["mode"] or "lookahead" in e["mode"]:
            log(f"  {flips} codes differ from the reference's")
            assert flips <= max(0, int(SR_BUDGET * values.numel())), (k, flips)
        else:
            assert flips == 0, (k, flips)
        if flips == 0:
            assert torch.equal(H.bits(scales), H.bits(torch.from_numpy(arrays[f"{k}_scales"]))), k
        if "lookahead" not in e["mode"]:
            # the oracle with the correctly rounded root: bit-exact
            exp_codes, exp_scales = ref.encode(values, e["mode"], eden=e["eden"], draws=draws, bias=e["bias"],
                                               eps=e["eps"], usr_sqrt="cr")
            assert torch.equal(got, exp_codes), (k, int((got != exp_codes).sum()))
            assert torch.equal(H.bits(scales), H.bits(exp_scales)), k


@pytest.mark.parametrize("mode", ["nf4", "nf4_sr", "sdyn4_sr", "dyn4_sr", "lin4_sr", "dyn4_upd_sr_fp32read",
                                  "lin4_upd_sr_fp32read"])
def test_codec_without_guards_matches_reference_step_rules(mode):
    """The reference step's rounding (no exact-level guards, quantization.py:279-377)."""
    gen = torch.Generator().manual_seed(11)
    cb = ref.codebook(mode)
    signed = bool(cb[0] < 0)
    x = torch.rand(128 * 64, generator=gen) ** 3 * (1e-3 if not signed else 1.0)
    if signed:
        x = x * torch.sign(torch.randn(x.numel(), generator=gen))
    x.view(-1, 128)[:, :16] = cb * x.view(-1, 128)[:, :1].abs().clamp_min(1e-6)  # exact levels hit the guards
    draws = torch.rand(x.numel() // 128, 128, generator=gen)
    stochastic = ref.is_stochastic(mode)
    codes, scales = gpu_encode(x, mode, False, False, draws if stochastic else None, 0.0975, 1e-8)
    exp_codes, exp_scales = ref.encode(x, mode, draws=draws if stochastic else None, bias=0.0975, eps=1e-8,
                                       guards=False, usr_sqrt="cr")
    flips = int((q.unpack_4bit_codes(codes, numel=x.numel()) != exp_codes).sum())
    assert flips == 0, flips
    assert torch.equal(H.bits(scales), H.bits(exp_scales))


@pytest.mark.parametrize("mode", ["nf4", "sdyn4", "dyn4", "lin4", "lin4_nz"])
def test_dequantize_matches_oracle(mode):
    gen = torch.Generator().manual_seed(5)
    n = 128 * 300
    codes = torch.randint(0, 256, (n // 2,), dtype=torch.uint8, generator=gen)
    scales = torch.rand(n // 128, generator=gen) * 1e-2
    m = moment_desc(mode, False, False, codes.to(H.DEVICE), scales.to(H.DEVICE))
    c_dev, s_dev = codes.to(H.DEVICE), scales.to(H.DEVICE)
    m["codes"], m["scales"] = c_dev.data_ptr(), s_dev.data_ptr()
    out = torch.empty(n, dtype=torch.float32, device=H.DEVICE)
    _lib.dequantize(m, n, out.data_ptr(), stream())
    assert torch.equal(H.bits(out), H.bits(ref.decode(codes, scales, mode, n)))


# ---------------------------------------------------------------------------
# Golden trajectories produced by the reference itself
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", trajectory_names())
def test_golden_trajectory(name):
    cfg, arrays = load(name)
    log(f"trajectory {name}")
    from tests.test_oracle_golden import run_oracle
    oracle, _ = run_oracle(cfg, arrays, record_draws=True)
    n_params = len(cfg["shapes"])
    params = [torch.nn.Parameter(tensor(arrays[f"init_p{i}"], cfg["dtype"]).clone()
                                 .reshape(cfg["shapes"][i]).to(H.DEVICE)) for i in range(n_params)]
    opt = H.build_optimizer(cfg, params)
    opt._draw_provider = H.LoggedDraws(oracle, params)
    for k in range(cfg["steps"]):
        for i, p in enumerate(params):
            p.grad = tensor(arrays[f"grad_s{k}_p{i}"], cfg["dtype"]).reshape(cfg["shapes"][i]).to(H.DEVICE)
        opt.step()
        if (k + 1) not in cfg["snap_steps"]:
            continue
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            pre = f"after{k + 1}_p{i}"
            st = H.state_of(opt, p)
            assert st["step"] == int(arrays[f"{pre}_step"])
            for m in ("m1", "m2"):
                if f"{pre}_{m}_code" in arrays:
                    expect = torch.from_numpy(arrays[f"{pre}_{m}_code"])
                    flips = H.code_mismatch(st[f"{m}_code"], expect)
                    budget = int(SR_BUDGET * p.numel()) if cfg["seed"] is not None else 0
                    if budget:
                        log(f"  p{i} {m}: {flips} codes differ from the reference's")
                    assert flips <= budget, f"{name} {pre} {m}: {flips} code flips"
                    if flips == 0:
                        assert torch.equal(H.bits(st[f"{m}_scale"]),
                                           H.bits(torch.from_numpy(arrays[f"{pre}_{m}_scale"]))), (name, pre, m)
                else:
                    kind = "pending" if f"{pre}_{m}_pending" in arrays else "fp32"
                    assert torch.equal(H.bits(st[f"{m}_{kind}"].reshape(-1)),
                                       H.bits(torch.from_numpy(arrays[f"{pre}_{m}_{kind}"]).reshape(-1))), (name, m)
            # 1 / denominator of the store-EDEN schemes: within the square root's ulp
            if f"{pre}_m2_pre" in arrays:
                got = opt.state[p]["m2_read_preconditioner"].cpu().reshape(-1)
                torch.testing.assert_close(got, torch.from_numpy(arrays[f"{pre}_m2_pre"]).reshape(-1),
                                           rtol=1e-6, atol=0.0)
            else:
                assert "m2_read_preconditioner" not in opt.state[p]
            exact = H.assert_params_close(p, tensor(arrays[pre], cfg["dtype"]).reshape(p.shape),
                                          f"{name} step {k+1} p{i}", steps=k + 1)
            log(f"  p{i}: parameters bit-exact {exact:.6f}")


# ---------------------------------------------------------------------------
# Fresh inputs, on-device Philox draws replayed into the oracle
# ---------------------------------------------------------------------------

def run_pair(make_opt, shapes, dtype, steps, *, seed=0, grad_seed=1, m1_override=None, oracle_kwargs=None,
             zero_block_frac=0.0, grad_fn=None):
    """Step the drop-in optimizer on the GPU and the oracle on the CPU with identical inputs/draws
    (gradients: ``grad_fn(shape, generator)``, heavy-tailed by default; ``dtype``: one for every
    tensor, or a list of one per tensor)."""
    grad_fn = grad_fn or H.heavy_tailed
    gen = torch.Generator().manual_seed(grad_seed)
    dtypes = list(dtype) if isinstance(dtype, (list, tuple)) else [dtype] * len(shapes)  # one per tensor
    init = [(torch.randn(s, generator=gen) * 0.02).to(dt) for s, dt in zip(shapes, dtypes)]
    params = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    opt = make_opt(params)
    if m1_override:
        opt.set_m1_quant_scheme_for_parameters([params[j] for j in m1_override[0]], m1_override[1])
    per = []
    for group in opt.param_groups:
        for p in group["params"]:
            per.append((opt._m1_scheme_for(p, group["m1_quant_scheme"]), group["m2_quant_scheme"],
                        group["use_eden_m2"]))
    hp = opt.param_groups[0]
    cpu_params = [t.clone() for t in init]
    oracle = ref.Oracle(cpu_params, ref.Hyper(hp["lr"], tuple(hp["betas"]), hp["eps"], hp["weight_decay"]),
                        [e[0] for e in per], [e[1] for e in per], [e[2] for e in per],
                        seed=seed, optimized=opt._optimized,
                        chunk=hp.get("max_chunk_numel", ref.CHUNK_NUMEL),
                        draw_fn=H.PhiloxMirror(opt, H.DEVICE), **{"usr_sqrt": "cr", **(oracle_kwargs or {})})
    # Values whose stochastic codes took the other level at some step; their later states and
    # parameters part ways.  Against this oracle none may part.
    parted = [torch.zeros(p.numel(), dtype=torch.bool) for p in params]
    for _ in range(steps):
        grads = []
        for s, dt in zip(shapes, dtypes):
            g = grad_fn(s, gen)
            if zero_block_frac and g.numel() % 128 == 0:
                nb = g.numel() // 128
                g.view(nb, 128)[torch.rand(nb, generator=gen) < zero_block_frac] = 0.0
            grads.append(g.to(dt))
        for p, g in zip(params, grads):
            p.grad = g.to(H.DEVICE)
        opt.step()
        oracle.step(grads)
        for i, p in enumerate(params):
            st = H.state_of(opt, p)
            for m, ms in (("m1", oracle.states[i].m1), ("m2", oracle.states[i].m2)):
                if ref.is_stochastic(ms.scheme) and f"{m}_code" in st:
                    parted[i] |= H.code_diff_mask(st[f"{m}_code"], ms.codes, p.numel())
    torch.cuda.synchronize()
    return opt, params, oracle, cpu_params, parted


def compare_pair(opt, params, oracle, cpu_params, parted, what, steps=1):
    """Round-to-nearest moments and fp32 state bit-exact; stochastic moments bit-exact at every
    step (no value parted); parameters within tolerance."""
    total_parted = 0
    total_codes = 0
    for i, (p, cp) in enumerate(zip(params, cpu_params)):
        st = H.state_of(opt, p)
        ost = H.oracle_state((oracle.states[i].m1, oracle.states[i].m2))
        assert set(st) - {"step"} == set(ost), (what, i, sorted(st), sorted(ost))
        for m, ms in (("m1", oracle.states[i].m1), ("m2", oracle.states[i].m2)):
            if f"{m}_code" in ost:
                flips = H.code_mismatch(st[f"{m}_code"], ost[f"{m}_code"])
                if ref.is_stochastic(ms.scheme):
                    total_codes += p.numel()
                    if flips:
                        log(f"  p{i} {m} ({ms.scheme}): {flips} codes differ at the last step")
                else:
                    # the two moments evolve independently: a parted stochastic moment leaves this one exact
                    assert flips == 0, f"{what} p{i} {m} ({ms.scheme}): {flips} flips"
                    assert torch.equal(H.bits(st[f"{m}_scale"]), H.bits(ost[f"{m}_scale"])), (what, i, m)
            else:
                kind = "pending" if f"{m}_pending" in ost else "fp32"
                assert torch.equal(H.bits(st[f"{m}_{kind}"].reshape(-1)), H.bits(ost[f"{m}_{kind}"])), (what, i, m)
        n_parted = int(parted[i].sum())
        total_parted += n_parted
        exact = H.assert_params_close(p, cp, f"{what} p{i}", steps=steps, exclude=parted[i])
        log(f"  p{i} {tuple(p.shape)}: parameters bit-exact {exact:.6f}; values parted by a stochastic code {n_parted}")
    log(f"  parted values {total_parted} of {total_codes} stochastic codes")
    assert total_parted == 0, f"{what}: {total_parted} of {total_codes} stochastic codes parted"
    return total_parted


@pytest.mark.parametrize("grads", ["normal", "heavy"])
def test_zeeden_1024x1024_matches_oracle(grads):
    """One fp32 1024x1024 parameter under ZE-EDEN for 12 steps: the benchmark's small case with
    its seeded N(0, 1e-3) gradients (10 warmup steps and more), and with heavy-tailed ones."""
    log(f"zeeden 1024x1024 x 12 steps, {grads} gradients")
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True)
    normal = lambda shape, gen: torch.randn(shape, generator=gen) * 1e-3  # noqa: E731
    out = run_pair(lambda ps: aw.ZEEDENAdamW4Bit(ps, **args), [(1024, 1024)], torch.float32, 12, seed=None,
                   grad_fn=normal if grads == "normal" else None)
    compare_pair(*out, "zeeden 1024^2")


@pytest.mark.parametrize("recipe", ["zeeden", "zipsr"])
def test_float64_parameters_match_oracle(recipe):
    """float64 parameters, which the reference's optimized backend takes (_optimized.py:99): the
    gradient read as fp32(g), fp32 moments and denominator, the parameter decayed and updated in
    float64 (_optimized.py:215-222), by the generic kernel; quantized tensors and an fp32-state
    tensor, the full step and then the cached launch plan, next to an fp32 parameter."""
    log(f"float64 parameters, {recipe} x 4 steps")
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True)
    make = ((lambda ps: aw.ZEEDENAdamW4Bit(ps, **args)) if recipe == "zeeden"
            else (lambda ps: aw.ZIPSRAdamW4Bit(ps, quant_rng_seed=4, **args)))
    out = run_pair(make, [(256, 512), (1000,), (64, 4096), (128, 256)],
                   [torch.float64, torch.float64, torch.float64, torch.float32], 4,
                   seed=None if recipe == "zeeden" else 4, zero_block_frac=0.02)
    compare_pair(*out, f"float64 {recipe}", steps=4)


def test_zipsr_philox_matches_oracle():
    log("zipsr 512x1024 philox x 6 steps, nf4_sr head")
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=0)
    out = run_pair(lambda ps: aw.ZIPSRAdamW4Bit(ps, **args), [(512, 1024), (256, 128)], torch.float32, 6, seed=0,
                   m1_override=([1], "nf4_sr"))
    compare_pair(*out, "zipsr philox")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_sampled_read_schemes_match_oracle(dtype):
    """m2 read back after its encode (reference step, adamw.py:615-656): dyn4_upd_sr / lin4_upd_sr
    take the denominator from the stored sample, *_upd_sr_store_eden from the sample at the scale
    before EDEN and keep 1 / denominator as state; on-device Philox replayed into the oracle."""
    log(f"sampled-read schemes {dtype} x 4 steps")
    spec = [("nf4", "dyn4_upd_sr", False), ("nf4_sr", "lin4_upd_sr", True), ("fp32", "dyn4_upd_sr_store_eden", False),
            ("sdyn4", "lin4_upd_sr_store_eden", False), ("nf4", "dyn4_nz", True)]

    def make(ps):
        groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b, use_eden_m2=e) for p, (a, b, e) in zip(ps, spec)]
        return aw.QuantizedAdamW(groups, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True,
                                 quant_rng_seed=3, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz")
    out = run_pair(make, [(512, 1024), (256, 512), (384, 128), (1024, 256), (128, 256)], dtype, 4, seed=3,
                   zero_block_frac=0.02)
    compare_pair(*out, f"sampled read {dtype}", steps=4)
    opt, params, oracle, _, parted = out
    for i, p in enumerate(params):
        expect = oracle.states[i].read_preconditioner
        if expect is None:
            assert "m2_read_preconditioner" not in opt.state[p], i
            continue
        got = opt.state[p]["m2_read_preconditioner"].cpu().reshape(-1)
        keep = ~parted[i]
        torch.testing.assert_close(got[keep], expect.reshape(-1)[keep], rtol=1e-6, atol=0.0)
        assert got.shape[0] == p.numel() and "m2" not in opt.state[p]


@pytest.mark.parametrize("dtype,betas", [(torch.float32, (0.9, 0.95)), (torch.bfloat16, (0.9, 0.95)),
                                         (torch.float32, (0.3, 0.45)), (torch.float64, (0.9, 0.95))])
def test_lookahead_schemes_match_oracle(dtype, betas):
    """Lookahead update-SR m2 (reference step, adamw.py:566-614): the pending form samples its fp32
    state before the update, the proxies store codes sampled for the next step; float64
    probabilities, on-device Philox replayed into the oracle.  Codes, scales and the pending
    state bit-exact (no parted values).  Betas at most 0.5 take ATen's other lerp form (the
    row's LERP flags)."""
    log(f"lookahead schemes {dtype} betas {betas} x 4 steps")
    spec = [("nf4", "dyn4_la_upd_sr"), ("fp32", "dyn4_proxy_la_upd_sr"), ("nf4", "dyn4_vproxy_la_upd_sr"),
            ("fp32", "dyn4_la_upd_sr"), ("nf4", "dyn4_nz")]

    def make(ps):
        groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b) for p, (a, b) in zip(ps, spec)]
        return aw.QuantizedAdamW(groups, lr=1e-3, betas=betas, eps=1e-8, weight_decay=0.1, optimized=True,
                                 quant_rng_seed=5, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz")
    out = run_pair(make, [(512, 1024), (256, 512), (384, 128), (1024, 256), (128, 256)], dtype, 4, seed=5,
                   zero_block_frac=0.02)
    parted = compare_pair(*out, f"lookahead {dtype}", steps=4)
    assert parted == 0
    opt, params, _, _, _ = out
    for p, (_, m2) in zip(params, spec):
        st = opt.state[p]
        assert ("lookahead_pending_exp_avg_sq" in st) == (m2 == "dyn4_la_upd_sr")
        assert "m2_read_preconditioner" not in st


@pytest.mark.parametrize("kind", ["f32", "bf16", "mixed", "research_f16"])
def test_fused_clip_matches_torch_clip(kind):
    """clip_grad_norm_ fused into the step (examples/train_gpt_small.py:214's max_grad_norm): the
    total norm agrees with torch.nn.utils.clip_grad_norm_ on the CPU (float64 sums here, torch's own
    order there), the coefficient is torch's arithmetic on that norm bit for bit, and the step
    reads the gradients torch's in-place multiply would leave (oracle fed the same scaled
    gradients; bit-exact states, parameters within the usual tolerance).  Three steps: the first
    runs the full path, the next ones the cached launch plan; max_norm alternates between clipping
    and not (coefficient 1)."""
    log(f"fused clip {kind} x 3 steps")
    shapes = [(256, 512), (1000,), (4097,), (384, 128), (3, 5)]
    dtypes = {"f32": [torch.float32] * 5, "bf16": [torch.bfloat16] * 5, "research_f16": [torch.float16] * 5,
              "mixed": [torch.bfloat16, torch.float32, torch.bfloat16, torch.bfloat16, torch.float32]}[kind]
    # fp16 and the research m2 schemes run the generic kernels (lookahead: the gradients of
    # tile_grads; read-back: the deferred update), the rest the specialised ZIP-SR kernels
    schemes = ([("nf4", "dyn4_la_upd_sr"), ("fp32", "dyn4_proxy_la_upd_sr"), ("nf4", "dyn4_upd_sr"),
                ("nf4", "dyn4_vproxy_la_upd_sr"), ("nf4", "dyn4_nz")] if kind == "research_f16"
               else [("nf4", "dyn4_upd_sr_fp32read")] * 5)
    if kind == "research_f16":
        shapes = [(256, 512), (64, 128), (4097,), (384, 128), (3, 5)]
    gen = torch.Generator().manual_seed(21)
    init = [(torch.randn(s, generator=gen) * 0.02).to(dt) for s, dt in zip(shapes, dtypes)]
    params = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b) for p, (a, b) in zip(params, schemes)]
    opt = aw.QuantizedAdamW(groups, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True,
                            quant_rng_seed=4, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz")
    cpu_params = [t.clone() for t in init]
    oracle = ref.Oracle(cpu_params, ref.Hyper(1e-3, (0.9, 0.95), 1e-8, 0.1), [a for a, _ in schemes],
                        [b for _, b in schemes], [False] * 5, seed=4, draw_fn=H.PhiloxMirror(opt, H.DEVICE),
                        usr_sqrt="cr")
    parted = [torch.zeros(p.numel(), dtype=torch.bool) for p in params]
    for step, max_norm in enumerate((1e-3, 1e3, 2e-3)):
        grads = [H.heavy_tailed(s, gen).to(dt) for s, dt in zip(shapes, dtypes)]
        for p, g in zip(params, grads):
            p.grad = g.to(H.DEVICE)
        total = opt.clip_grad_norm_(max_norm)
        coef = opt._grad_clip[1][1].cpu().reshape(())
        with pytest.raises(RuntimeError, match="already pending"):
            opt.clip_grad_norm_(max_norm)
        if step == 0:  # a skipped step: zero_grad() drops the pending clip with the gradients
            opt.zero_grad()
            assert opt._grad_clip is None and all(p.grad is None for p in params)
            for p, g in zip(params, grads):
                p.grad = g.to(H.DEVICE)
            total = opt.clip_grad_norm_(max_norm)
            coef = opt._grad_clip[1][1].cpu().reshape(())
        expect_total, _ = ref.clip_grad_norm_f64(grads, max_norm)
        torch_total, _ = ref.clip_grad_norm(grads, max_norm)
        assert total.dtype == expect_total.dtype == torch_total.dtype and total.shape == ()
        # the float64 restatement: equal up to one ulp of the result dtype (the order of the
        # float64 sums differs); torch's own CPU clip: within its fp32 accumulation error
        ulp = H.ULP16.get(total.dtype, 2.0 ** -23)
        got, want, tt = float(total), float(expect_total), float(torch_total)
        assert abs(got - want) <= ulp * abs(want), (got, want)
        assert abs(got - tt) <= max(2e-5, 2 * ulp) * abs(tt), (got, tt)
        # torch's coefficient arithmetic on this norm, in its dtype
        t_cpu = total.cpu()
        assert torch.equal(coef.to(t_cpu.dtype), torch.clamp(max_norm / (t_cpu + 1e-6), max=1.0)), (float(coef), step)
        assert (float(coef) < 1.0) == (step != 1)
        opt.step()
        assert opt._grad_clip is None
        for g, pg in zip(grads, (p.grad.cpu() for p in params)):
            assert torch.equal(H.bits(g), H.bits(pg))  # the gradients stay unscaled in memory
        oracle.step(ref.scale_grads(grads, coef.to(t_cpu.dtype)))
        for i, p in enumerate(params):
            st = H.state_of(opt, p)
            ms = oracle.states[i].m2
            if ref.is_stochastic(ms.scheme) and "m2_code" in st:
                parted[i] |= H.code_diff_mask(st["m2_code"], ms.codes, p.numel())
    torch.cuda.synchronize()
    compare_pair(opt, params, oracle, cpu_params, parted, f"clip {kind}", steps=3)


def _same_or_both_nan(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.detach().cpu().reshape(-1), b.detach().cpu().reshape(-1)
    nan = torch.isnan(a.float())
    return bool(torch.equal(nan, torch.isnan(b.float()))) and torch.equal(H.bits(a[~nan]), H.bits(b[~nan]))


@pytest.mark.parametrize("recipe", ["zeeden", "zipsr", "research", "zipsr_float64"])
def test_non_finite_gradients_match_oracle(recipe):
    """NaN, +Inf and -Inf gradient values (in quantized tensors and an fp32-state tensor) follow
    the reference: the NaN / Inf block scales, the codes of a block whose scale is not finite
    (the kernel's IEEE forms), and the propagation into moments and parameters on the next
    steps.  Codes, fp32 states and scales equal the oracle's (NaN == NaN); parameters have the
    same NaNs and their finite values are within the usual tolerance.  fp32 parameters, and
    float64 ones under ZIP-SR (the generic kernel's float64 update)."""
    log(f"non-finite gradients, {recipe} x 3 steps")
    shapes = [(64, 128), (4096,), (1000,)]
    gen = torch.Generator().manual_seed(13)
    dtype = torch.float64 if recipe.endswith("_float64") else torch.float32
    recipe = recipe.replace("_float64", "")
    init = [(torch.randn(sh, generator=gen) * 0.02).to(dtype) for sh in shapes]
    params = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True)
    m1s = ["nf4"] * 3
    if recipe == "zeeden":
        opt = aw.ZEEDENAdamW4Bit(params, **args)
        m2s, eden = ["dyn4_nz"] * 3, True
    elif recipe == "zipsr":
        opt = aw.ZIPSRAdamW4Bit(params, quant_rng_seed=6, **args)
        m2s, eden = ["dyn4_upd_sr_fp32read"] * 3, False
    else:  # the research kernel: lookahead (float64 probabilities) and read-back m2
        m1s, m2s, eden = ["nf4", "fp32", "nf4"], ["dyn4_la_upd_sr", "dyn4_vproxy_la_upd_sr", "dyn4_upd_sr"], False
        groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b) for p, a, b in zip(params, m1s, m2s)]
        opt = aw.QuantizedAdamW(groups, quant_rng_seed=6, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz", **args)
    cpu = [t.clone() for t in init]
    oracle = ref.Oracle(cpu, ref.Hyper(1e-3, (0.9, 0.95), 1e-8, 0.1), m1s, m2s, [eden] * 3,
                        seed=None if recipe == "zeeden" else 6, draw_fn=H.PhiloxMirror(opt, H.DEVICE),
                        usr_sqrt="cr")
    for step in range(3):
        grads = [H.heavy_tailed(sh, gen) for sh in shapes]
        if step == 1:
            g0 = grads[0].view(-1)
            g0[3 * 128 + 5] = float("nan")      # one NaN in block 3
            g0[7 * 128 + 100] = float("inf")    # +Inf in block 7
            g0[9 * 128 + 1] = float("-inf")     # -Inf in block 9
            grads[1][2 * 128 + 64] = float("inf")
            grads[2][5] = float("nan")          # fp32-state tensor
        for p, g in zip(params, grads):
            p.grad = g.to(dtype).to(H.DEVICE)
        opt.step()
        oracle.step(grads)
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            st = H.state_of(opt, p)
            ost = H.oracle_state((oracle.states[i].m1, oracle.states[i].m2))
            for key, val in ost.items():
                if key.endswith("_code"):
                    assert torch.equal(st[key].cpu(), val), (recipe, step, i, key, H.code_mismatch(st[key], val))
                else:
                    assert _same_or_both_nan(st[key], val), (recipe, step, i, key)
            # parameters: the same NaNs, and the finite values within the usual tolerance
            got = p.detach().cpu().reshape(-1)
            want = cpu[i].reshape(-1)
            nan = torch.isnan(want)
            assert torch.equal(torch.isnan(got), nan), (recipe, step, i)
            H.assert_params_close(got[~nan], want[~nan], f"non-finite {recipe} step {step} p{i}", steps=step + 1)
    assert any(bool(torch.isnan(p.detach()).any()) for p in params)  # the NaN reached the parameters


def test_eager_step_bumps_version_counters():
    """The eager launch calls the library directly (not through the custom operator's dispatch)
    and bumps the version counters of everything it writes in place, as the operator does: an
    autograd graph that saved a parameter before the step refuses to backpropagate after it."""
    log("version counters after an eager step")
    p = torch.nn.Parameter(torch.randn(64, 128, device=H.DEVICE) * 0.02)
    small = torch.nn.Parameter(torch.randn(100, device=H.DEVICE))
    opt = aw.ZIPSRAdamW4Bit([p, small], lr=1e-3, optimized=True, quant_rng_seed=0)
    for step in range(2):  # the full path, then the cached launch plan
        p.grad, small.grad = torch.randn_like(p) * 1e-3, torch.randn_like(small)
        loss = (p * p).sum()  # saves p for backward
        before = (p._version, small._version, opt.state[p].get("m1_code", p)._version if step else 0)
        opt.step()
        assert p._version > before[0] and small._version > before[1], step
        if step:
            assert opt.state[p]["m1_code"]._version > before[2]
        with pytest.raises(RuntimeError, match="modified by an inplace operation"):
            loss.backward()


def test_tensor_beyond_2_31_values():
    """One fp32 parameter of 2^31 + 4096 values (64-bit element, code and scale offsets): the 4096
    values straddling element 2^31 are stepped exactly as a separate 4096-value parameter holding
    them, fed the uniforms at the same Philox positions of the big tensor's streams (ZIP-SR, two
    steps; bit-exact parameters, codes and scales).  Needs about 28 GB of device memory."""
    n = (1 << 31) + 4096
    lo, hi = (1 << 31) - 2048, (1 << 31) + 2048
    log(f"ZIP-SR, one tensor of {n} values, window [{lo}, {hi})")
    dev = torch.device(H.DEVICE)
    gen = torch.Generator(device=dev).manual_seed(31)
    big = torch.nn.Parameter(torch.randn(n, generator=gen, device=dev) * 0.02)
    probe = torch.nn.Parameter(big.detach()[lo:hi].clone())
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=0)
    opt_big, opt_probe = aw.ZIPSRAdamW4Bit([big], **args), aw.ZIPSRAdamW4Bit([probe], **args)
    for step in range(2):
        g = torch.randn(n, generator=gen, device=dev) * 1e-3
        big.grad, probe.grad = g, g[lo:hi].clone()
        opt_big.step()
        # the m2 write is the step's last draw from the big tensor's m2 stream: n positions,
        # rounded up to 128, ending at the stream's position now
        stream = opt_big._stream("m2", big.device)  # streams are keyed by the parameter's device
        seed, offset = stream.seed, stream.offset - (n + 127) // 128 * 128
        opt_probe._draw_provider = lambda p, moment, k, d: H.uniforms_gpu(seed, offset + lo, k)
        opt_probe.step()
        torch.cuda.synchronize()
        assert torch.equal(H.bits(big.detach()[lo:hi]), H.bits(probe.detach())), step
        sb, sp = opt_big.state[big], opt_probe.state[probe]
        for m in ("m1", "m2"):
            assert torch.equal(sb[f"{m}_code"][lo // 2:hi // 2].cpu(), sp[f"{m}_code"].cpu()), (step, m)
            assert torch.equal(H.bits(sb[f"{m}_quant_state"].absmax[lo // 128:hi // 128]),
                               H.bits(sp[f"{m}_quant_state"].absmax)), (step, m)
        del g
    log("  window bit-exact over 2 steps")


def test_zipsr_4096x4096_matches_oracle():
    """The benchmark's single-tensor ZIP-SR case at full size: one fp32 4096x4096 parameter,
    heavy-tailed gradients, quant_rng_seed=0, past its 10 warmup steps."""
    log("zipsr 4096x4096 x 11 steps (full size)")
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=0)
    out = run_pair(lambda ps: aw.ZIPSRAdamW4Bit(ps, **args), [(4096, 4096)], torch.float32, 11, seed=0)
    compare_pair(*out, "zipsr 4096^2", steps=11)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mixed_list_16bit(dtype):
    """Many tensors of ragged sizes, fp32-state ones included, one launch; 16-bit params and grads."""
    log(f"mixed list {dtype}")
    shapes = [(768,), (4096,), (4097,), (1,), (3,), (129,), (128,), (50, 256), (3072, 768), (4096, 3), (1000,)]
    args = dict(lr=2e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=3)
    out = run_pair(lambda ps: aw.ZIPSRAdamW4Bit(ps, **args), shapes, dtype, 4, seed=3, m1_override=([8], "nf4_sr"),
                   zero_block_frac=0.05)
    compare_pair(*out, f"mixed {dtype}", steps=4)


def test_scheme_groups_reference_step():
    """optimized=False (the reference step) over every scheme family, one group per scheme pair."""
    log("scheme groups, reference step")
    pairs = [("nf4", "dyn4_nz", True), ("sdyn4_sr", "lin4_sr", False), ("fp32", "dyn4", True),
             ("nf4", "lin4_nz", True), ("nf4", "dyn4_lookahead_sr", True), ("nf4", "fp32", False),
             ("nf4_sr", "dyn4_upd_sr_fp32read", True), ("sdyn4", "dyn4_sr", False),
             ("nf4", "lin4_upd_sr_fp32read", False), ("nf4", "lin4", False)]

    def make(ps):
        groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b, use_eden_m2=e) for p, (a, b, e) in zip(ps, pairs)]
        return aw.QuantizedAdamW(groups, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                                 m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz", quant_rng_seed=9, optimized=False)
    out = run_pair(make, [(8192,)] * len(pairs), torch.float32, 3, seed=9, zero_block_frac=0.02)
    compare_pair(*out, "scheme groups")


def test_gpt2_small_shaped_list_zeeden():
    """The GPT-2-small parameter list at full size (50257x768 embedding, 1024x768 positions, all 12
    layers: 148 tensors, 124,439,808 values): matrices take the 4-bit path and the 768/2304/3072
    LayerNorm and bias vectors (121,344 values) the fp32-state path, in one launch."""
    log("gpt2-small list, ZE-EDEN x 3 steps")
    d = 768
    layer = [(d,), (d,), (d, 3 * d), (3 * d,), (d, d), (d,), (d,), (d,), (d, 4 * d), (4 * d,), (4 * d, d), (d,)]
    shapes = [(50257, d), (1024, d)] + layer * 12 + [(d,), (d,)]
    assert len(shapes) == 148 and sum(math.prod(s) for s in shapes) == 124_439_808
    args = dict(lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True)
    out = run_pair(lambda ps: aw.ZEEDENAdamW4Bit(ps, **args), shapes, torch.float32, 3, seed=None)
    compare_pair(*out, "gpt2-small shapes", steps=3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mixed_recipes_split_launches(dtype):
    """One optimizer whose tensors need different kernels (ZE-EDEN and ZIP-SR recipe schemes, an
    nf4_sr head, an fp32 second moment, fp32-state vectors): the step splits into one launch per
    specialised kernel plus one generic launch, and every tensor still matches the oracle."""
    log(f"mixed recipes, split launches, {dtype}")
    pairs = [("nf4", "dyn4_nz", True), ("nf4", "dyn4_upd_sr_fp32read", False), ("nf4", "dyn4_nz", True),
             ("nf4", "dyn4_upd_sr_fp32read", False), ("nf4", "fp32", False), ("nf4", "dyn4_nz", True),
             ("nf4", "dyn4_upd_sr_fp32read", False), ("nf4", "dyn4_upd_sr_fp32read", True)]
    shapes = [(256, 512), (384, 256), (768,), (1000,), (128, 256), (64, 1024), (96, 512), (160, 256)]

    def make(ps):
        groups = [dict(params=[p], m1_quant_scheme=a, m2_quant_scheme=b, use_eden_m2=e)
                  for p, (a, b, e) in zip(ps, pairs)]
        return aw.QuantizedAdamW(groups, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                                 m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz", quant_rng_seed=5, optimized=True)
    out = run_pair(make, shapes, dtype, 4, seed=5, m1_override=([6], "nf4_sr"), zero_block_frac=0.02)
    compare_pair(*out, f"mixed recipes {dtype}", steps=4)


def test_mixed_parameter_dtypes_in_one_step():
    """fp32, bf16 and fp16 parameters in one optimizer step (one launch per dtype's specialised
    kernel, the fp32-state vectors with their dtype's launch), ZIP-SR with an nf4_sr retarget,
    three steps against the oracle."""
    log("mixed parameter dtypes")
    shapes = [(256, 128), (256, 128), (256, 128), (768,), (768,), (768,), (64, 512), (4096,), (1000,)]
    dtypes = [torch.float32, torch.bfloat16, torch.float16] * 3
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=29)
    out = run_pair(lambda ps: aw.ZIPSRAdamW4Bit(ps, **args), shapes, dtypes, 3, seed=29, m1_override=([1, 6], "nf4_sr"),
                   zero_block_frac=0.03)
    compare_pair(*out, "mixed dtypes", steps=3)


def test_thousands_of_tensors_in_one_launch():
    """1,536 tensors in one step (a 442 KB launch table staged through a grown slot): 4-bit ones
    of one to eight tiles and fp32-state ones in between, so that a wave's tiles are found by
    the binary search over a long tile-start list.  ZIP-SR, two steps, against the oracle."""
    log("1536 tensors, one launch")
    cycle = [(32, 128), (100,), (4096,), (7,), (64, 1024), (300,), (8192,), (129,)]
    shapes = [cycle[k % len(cycle)] for k in range(1536)]
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=13)
    out = run_pair(lambda ps: aw.ZIPSRAdamW4Bit(ps, **args), shapes, torch.float32, 2, seed=13)
    compare_pair(*out, "1536 tensors", steps=2)


@pytest.mark.parametrize("n", [11, 12])
def test_inline_table_limit(n):
    """A launch of eleven tensors takes its table in the kernel's arguments (3,392 of 3,584
    bytes: a 40-byte header, 296 bytes per tensor, 8 per tile start); twelve (3,696 bytes)
    stage it through device memory.  Both match the oracle, ZIP-SR over two steps."""
    log(f"inline table limit: {n} tensors")
    shapes = [(64, 128 * (1 + k % 3)) for k in range(n)]
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=11)
    out = run_pair(lambda ps: aw.ZIPSRAdamW4Bit(ps, **args), shapes, torch.float32, 2, seed=11)
    compare_pair(*out, f"{n} tensors", steps=2)


@pytest.mark.parametrize("m2_scheme,many", [(None, False), (None, True), ("dyn4_upd_sr_fp32read_nextbc", False),
                                            ("dyn4_la_upd_sr", False), ("dyn4_proxy_la_upd_sr", False),
                                            ("dyn4_vproxy_la_upd_sr", False)])
def test_launch_plan_reuse_matches_full_path(m2_scheme, many):
    """Steps reusing the previous step's launch tables are bit-identical to steps that rebuild
    them, through a learning-rate change, a parameter without gradient, an m1 retarget, and
    state tensors replaced by equal copies (a code or pending-state tensor, a QuantState's
    absmax), which the plan must not keep writing through its old addresses.  With the
    next-step storage bias the group's first tensor is an fp32-state one, whose m2 scheme (fp32)
    has the other bias: the step constants must not be shared across the two.  The lookahead
    schemes' rows carry a bias correction of the step (or the next) that the plan rewrites.
    `many`: 21 tensors, past the plan's small-plan limit (16 rows, checked and refreshed in
    Python) and past the launch-argument table (12 rows), so the plan's numpy path and the staged
    table run."""
    log(f"launch plan reuse vs full path ({m2_scheme or 'ZIP-SR'}{', 21 tensors' if many else ''})")
    shapes = [(256, 512), (768,), (64, 1024), (1000,), (128, 384)] + ([(128, 64)] * 16 if many else [])
    q0 = 0
    if m2_scheme is not None:
        shapes[0], shapes[1] = shapes[1], shapes[0]
        q0 = 1  # the first parameter with quantized state
    gen = torch.Generator().manual_seed(21)
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    args = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, optimized=True, quant_rng_seed=4)
    if m2_scheme is None:
        oa, ob = aw.ZIPSRAdamW4Bit(pa, **args), aw.ZIPSRAdamW4Bit(pb, **args)
    else:
        args.update(m1_quant_scheme="nf4", m2_quant_scheme=m2_scheme)
        oa, ob = aw.QuantizedAdamW(pa, **args), aw.QuantizedAdamW(pb, **args)
    reused = 0
    for k in range(7):
        for a, b, s in zip(pa, pb, shapes):
            g = H.heavy_tailed(s, gen).to(H.DEVICE)
            a.grad, b.grad = g.clone(), g.clone()
        if k == 3:
            pa[2].grad = pb[2].grad = None
        if k == 4:
            for o in (oa, ob):
                o.param_groups[0]["lr"] = 5e-4
        if k == 5:
            oa.set_m1_quant_scheme_for_parameters([pa[q0]], "nf4_sr")
            ob.set_m1_quant_scheme_for_parameters([pb[q0]], "nf4_sr")
        if k == 6:
            for o, ps in ((oa, pa), (ob, pb)):
                key = "m2_code" if "m2_code" in o.state[ps[q0]] else "lookahead_pending_exp_avg_sq"
                o.state[ps[q0]][key] = o.state[ps[q0]][key].clone()
                q = o.state[ps[4]]["m1_quant_state"]
                q.absmax = q.absmax.clone()
        before = oa._launch_plan
        oa.step()
        reused += int(before is not None and oa._launch_plan is before)
        ob._launch_plan = None  # always the full path
        ob.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            assert torch.equal(H.bits(a), H.bits(b)), (k, i)
            sa, sb = H.state_of(oa, a), H.state_of(ob, b)
            assert sa.keys() == sb.keys() and sa["step"] == sb["step"], (k, i)
            for key in sa:
                if key != "step":
                    assert torch.equal(H.bits(sa[key]), H.bits(sb[key])), (k, i, key)
    log(f"  plan reused on {reused} of 7 steps")
    assert reused >= 2  # steps 1 and 2; every later step changes the structure


def test_lerp_large_weight_betas():
    """betas with 1-beta >= 0.5 use ATen's other lerp formula."""
    log("large lerp weights")
    args = dict(lr=1e-3, betas=(0.3, 0.45), eps=1e-6, weight_decay=0.0, optimized=True)
    out = run_pair(lambda ps: aw.ZEEDENAdamW4Bit(ps, **args), [(64, 128), (700,)], torch.float32, 3, seed=None)
    compare_pair(*out, "large lerp")


# ---------------------------------------------------------------------------
# Checkpoints
# ---------------------------------------------------------------------------

def test_state_dict_resume_is_exact(tmp_path):
    log("state_dict resume")
    gen = torch.Generator().manual_seed(4)
    shapes = [(256, 128), (768,)]
    init = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    grads = [[H.heavy_tailed(s, gen) for s in shapes] for _ in range(6)]

    def make(ps):
        opt = aw.ZIPSRAdamW4Bit(ps, quant_rng_seed=21, optimized=True)
        opt.set_m1_quant_scheme_for_parameters([ps[0]], "nf4_sr")
        return opt

    a = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    oa = make(a)
    for k in range(6):
        for p, g in zip(a, grads[k]):
            p.grad = g.to(H.DEVICE)
        oa.step()

    b = [torch.nn.Parameter(t.clone().to(H.DEVICE)) for t in init]
    ob = make(b)
    for k in range(3):
        for p, g in zip(b, grads[k]):
            p.grad = g.to(H.DEVICE)
        ob.step()
    torch.save(ob.state_dict(), tmp_path / "ckpt.pt")
    sd = torch.load(tmp_path / "ckpt.pt", weights_only=True)
    assert sd["_quant_rng_state"]["version"] == 1
    assert set(sd["state"][0]) == {"step", "m1_code", "m1_quant_state", "m2_code", "m2_quant_state"}
    assert sd["state"][0]["m1_quant_state"]["packed"] is True
    c = [torch.nn.Parameter(p.detach().clone()) for p in b]
    oc = make(c)
    oc.load_state_dict(sd)
    for k in range(3, 6):
        for p, g in zip(c, grads[k]):
            p.grad = g.to(H.DEVICE)
        oc.step()
    torch.cuda.synchronize()
    for pa, pc in zip(a, c):
        assert torch.equal(H.bits(pa), H.bits(pc))
    for pa, pc in zip(a, c):
        sa, sc = H.state_of(oa, pa), H.state_of(oc, pc)
        for key in sa:
            if key == "step":
                assert sa[key] == sc[key]
            else:
                assert torch.equal(H.bits(sa[key]), H.bits(sc[key])), key


def test_legacy_unpacked_codes_are_repacked():
    """Quantized state holding one code per byte (unpacked, as older checkpoints store it,
    _moment_buffer.py:127-141) is packed on the next step and continues bit-exactly."""
    log("legacy unpacked codes")
    gen = torch.Generator().manual_seed(8)
    shape = (128, 256)
    init = torch.randn(shape, generator=gen) * 0.02
    grads = [H.heavy_tailed(shape, gen) for _ in range(4)]
    a = torch.nn.Parameter(init.clone().to(H.DEVICE))
    b = torch.nn.Parameter(init.clone().to(H.DEVICE))
    oa, ob = aw.ZEEDENAdamW4Bit([a], optimized=True), aw.ZEEDENAdamW4Bit([b], optimized=True)
    for k in range(4):
        if k == 2:
            st = ob.state[b]
            for m in ("m1", "m2"):
                st[f"{m}_code"] = q.unpack_4bit_codes(st[f"{m}_code"], numel=b.numel()).to(torch.uint8)
                st[f"{m}_quant_state"].packed = False
        for p, o in ((a, oa), (b, ob)):
            p.grad = grads[k].to(H.DEVICE)
            o.step()
    torch.cuda.synchronize()
    assert torch.equal(H.bits(a), H.bits(b))
    sa, sb = H.state_of(oa, a), H.state_of(ob, b)
    for key in sa:
        if key != "step":
            assert torch.equal(H.bits(sa[key]), H.bits(sb[key])), key
    assert ob.state[b]["m1_code"].numel() == (b.numel() + 1) // 2 and ob.state[b]["m1_quant_state"].packed


def test_reference_checkpoint_loads_on_gpu():
    """A state_dict written by the reference (CPU) loads onto GPU parameters; its CPU RNG
    streams cannot move to another device type, as in the reference (adamw.py:306-320)."""
    sd = torch.load("tests/golden/zipsr_state_dict.pt", weights_only=True)
    params = torch.load("tests/golden/zipsr_state_dict_params.pt", weights_only=True)
    p = torch.nn.Parameter(params["p"].to(H.DEVICE))
    qv = torch.nn.Parameter(params["q"].to(H.DEVICE))
    opt = aw.ZIPSRAdamW4Bit([p, qv], quant_rng_seed=11, optimized=True)
    opt.load_state_dict(sd)
    st = opt.state[p]
    assert st["m2_code"].device.type == "cuda" and st["m2_quant_state"].absmax.device.type == "cuda"
    assert torch.equal(st["m2_code"].cpu(), sd["state"][0]["m2_code"])
    p.grad = torch.zeros_like(p)
    qv.grad = torch.zeros_like(qv)
    with pytest.raises(ValueError, match="Unable to restore quantization RNG state"):
        opt.step()


# ---------------------------------------------------------------------------
# On-device draws: statistics
# ---------------------------------------------------------------------------

def test_state_sr_on_device_draws_are_value_unbiased():
    log("state-SR statistics")
    gen = torch.Generator().manual_seed(6)
    block = torch.rand(128, generator=gen) * 2 - 1
    block[0] = 1.0
    reps = 8192
    values = block.repeat(reps)
    cb = ref.codebook("nf4_sr")
    n = values.numel()
    codes = torch.empty(n // 2, dtype=torch.uint8, device=H.DEVICE)
    scales = torch.empty(n // 128, dtype=torch.float32, device=H.DEVICE)
    m = moment_desc("nf4_sr", False, True, codes, scales)
    m["rng_seed"], m["rng_offset"] = 12345, 0
    v = values.to(H.DEVICE)
    _lib.quantize(v.data_ptr(), n, m, stream())
    got = q.unpack_4bit_codes(codes.cpu(), numel=n).view(reps, 128).long()
    mean = cb[got].double().mean(0)
    lower, upper, a, b = ref._endpoints(block, cb)
    width = (b - a).double()
    p_hi = ((block.double() - a.double()) / width.clamp_min(1e-12)).clamp(0, 1)
    sd = (width * torch.sqrt(p_hi * (1 - p_hi) / reps)).clamp_min(1e-9)
    assert ((mean - block.double()).abs() <= 5 * sd + 1e-7).all()
    # code histogram: only the two neighbours occur, with frequency P(hi)
    assert bool(((got == lower.long()) | (got == upper.long())).all())
    freq = (got == upper.long()).double().mean(0)
    mid = (lower != upper)
    assert ((freq - p_hi).abs()[mid] <= 5 * torch.sqrt(p_hi * (1 - p_hi) / reps)[mid] + 1e-3).all()


def test_update_sr_on_device_draws_are_preconditioner_unbiased():
    log("update-SR statistics")
    gen = torch.Generator().manual_seed(7)
    block = torch.rand(128, generator=gen) ** 6 * 1e-6
    block[0] = 1e-6
    reps = 8192
    values = block.repeat(reps)
    n = values.numel()
    bias, eps = 0.0975, 1e-8
    codes = torch.empty(n // 2, dtype=torch.uint8, device=H.DEVICE)
    scales = torch.empty(n // 128, dtype=torch.float32, device=H.DEVICE)
    m = moment_desc("dyn4_upd_sr_fp32read", False, True, codes, scales, bias=bias, eps=eps)
    m["rng_seed"], m["rng_offset"] = 777, 4096
    v = values.to(H.DEVICE)
    _lib.quantize(v.data_ptr(), n, m, stream())
    got = q.unpack_4bit_codes(codes.cpu(), numel=n).view(reps, 128).long()
    cb = ref.codebook("dyn4").double()
    s = block.abs().max().double()

    def f(level):
        return 1.0 / (torch.sqrt(torch.clamp(s * level / bias, min=0.0)) + eps)

    est = f(cb[got]).mean(0)
    x = block.double() / s
    target = f(x)
    lower, upper, a, b = ref._endpoints((block / block.abs().max()).contiguous(), cb.float())
    fa, fb = f(a.double()), f(b.double())
    p_lo = ((target - fb) / (fa - fb).clamp_min(1e-300)).clamp(0, 1)
    sd = (fa - fb).abs() * torch.sqrt(p_lo * (1 - p_lo) / reps)
    assert ((est - target).abs() <= 5 * sd + 1e-5 * target).all()
