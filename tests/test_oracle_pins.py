"""Pins for the CPU oracle that do not depend on the golden fixtures.

Known answers from the reference's own tests (cited per test), closed forms,
invariants, brute force over the 16 levels, and planted mistakes that the golden
trajectories must reject.
"""

import math
import struct

import numpy as np
import pytest
import torch

from adamw4bit_amd import quantization as q
from oracle import reference_step as ref
from tests._fixtures import bits, load
from tests.test_oracle_golden import run_oracle

MODES = ["nf4", "sdyn4", "lin4", "lin4_nz", "dyn4"]


def _bits(values):
    return tuple(struct.unpack("<I", struct.pack("<f", float(v)))[0] for v in values)


@pytest.mark.parametrize("mode", MODES)
def test_codebook_closed_forms_match_shipped_bit_patterns(mode):
    cb_id = q.SCHEMES[mode][0]
    assert _bits(ref.codebook(mode).tolist()) == q.CODEBOOK_BITS[cb_id]


def test_codebooks_match_reference_known_values():
    # tests/quantization/test_utils.py:176-210 (same tolerance as torch.testing.assert_close).
    sdyn4 = [-0.8875, -0.6625, -0.4375, -0.2125, -0.0775, -0.0325, -0.0055, 0.0,
             0.0055, 0.0325, 0.0775, 0.2125, 0.4375, 0.6625, 0.8875, 1.0]
    dyn4 = [0.0, 0.00325, 0.00775, 0.02125, 0.04375, 0.06625, 0.08875, 0.15625,
            0.26875, 0.38125, 0.49375, 0.60625, 0.71875, 0.83125, 0.94375, 1.0]
    torch.testing.assert_close(ref.codebook("sdyn4"), torch.tensor(sdyn4))
    torch.testing.assert_close(ref.codebook("dyn4"), torch.tensor(dyn4))
    torch.testing.assert_close(ref.codebook("lin4_nz"), torch.linspace(0.0, 1.0, 17)[1:])
    assert ref.codebook("dyn4")[0].item() == 0.0 and ref.codebook("dyn4")[1].item() > 0.0


def test_nibble_order():
    # test_utils.py:92-100
    packed = ref.pack(torch.tensor([1, 2, 15], dtype=torch.uint8))
    assert packed.tolist() == [0x21, 0x0F]
    assert q.pack_4bit_codes(torch.tensor([1, 2, 15], dtype=torch.uint8)).tolist() == [0x21, 0x0F]
    codes = torch.arange(16, dtype=torch.uint8)
    assert torch.equal(q.unpack_4bit_codes(q.pack_4bit_codes(codes), numel=16), codes)


def _pad(values):
    t = torch.zeros(128)
    t[: len(values)] = torch.tensor(values)
    return t


def test_round_to_nearest_ties_go_up():
    # test_utils.py:233-243 (block scale is 1.0 so x equals the value)
    codes, _ = ref.encode(_pad([0.09375, 0.96875, 1.0, 0.0]), "lin4_nz")
    assert codes[:4].tolist() == [1, 15, 15, 0]
    codes, _ = ref.encode(_pad([0.00275, -0.00275, 1.0, 0.0]), "sdyn4")
    assert codes[:4].tolist() == [8, 7, 15, 7]


@pytest.mark.parametrize("mode", ["nf4", "nf4_sr", "sdyn4", "lin4", "lin4_nz", "dyn4", "dyn4_nz",
                                  "dyn4_sr", "dyn4_upd_sr_fp32read"])
def test_scale_floor(mode):
    # test_utils.py:246-257
    draws = torch.zeros(1, 128) if ref.is_stochastic(mode) else None
    _, scales = ref.encode(torch.zeros(128), mode, draws=draws)
    assert scales.tolist() == [torch.tensor(1e-12, dtype=torch.float32).item()]


def test_dyn4_nz_floor():
    # test_utils.py:165-173
    codes, _ = ref.encode(_pad([0.0, 1e-6, 0.01, 1.0]), "dyn4_nz")
    assert int(codes.min()) >= 1


@pytest.mark.parametrize("mode,eden", [(m, e) for m in ["nf4", "nf4_sr", "sdyn4", "lin4", "lin4_nz",
                                                      "dyn4", "dyn4_nz", "dyn4_upd_sr_fp32read"]
                                      for e in (False, True)])
def test_initial_code_and_scale_is_encoded_zero(mode, eden):
    draws = torch.rand(1, 128) if ref.is_stochastic(mode) else None
    codes, scales = ref.encode(torch.zeros(128), mode, eden=eden, draws=draws)
    code, scale = q.initial_code_and_scale(mode, eden)
    assert set(codes.tolist()) == {code}
    assert scales.tolist() == [scale]


def test_eden_invariant():
    # test_upd_sr_store_eden.py:17-36: <x, x_hat> equals ||x||^2 per block after correction.
    gen = torch.Generator().manual_seed(0)
    v = torch.rand(128 * 64, generator=gen) ** 4
    for mode in ("dyn4_nz", "dyn4", "lin4_nz"):
        codes, scales = ref.encode(v, mode, eden=True)
        xhat = ref.codebook(mode)[codes.long()].view(-1, 128) * scales.unsqueeze(1)
        vb = v.view(-1, 128)
        torch.testing.assert_close((vb * xhat).double().sum(1), (vb * vb).double().sum(1), rtol=1e-5, atol=0)


def test_rtn_brute_force():
    gen = torch.Generator().manual_seed(1)
    for mode in MODES:
        cb = ref.codebook(mode)
        lo = -1.0 if cb[0] < 0 else 0.0
        x = torch.rand(128 * 32, generator=gen) * (1.0 - lo) + lo
        x.view(-1, 128)[:, 0] = 1.0  # pin the block scale to 1 so the codec sees x itself
        codes, _ = ref.encode(x, mode)
        cb64 = cb.double()
        for xi, ci in zip(x.tolist()[:2000], codes.tolist()[:2000]):
            d = [abs(xi - c) for c in cb64.tolist()]
            best = min(d)
            # nearest level; on an exact tie the upper one
            expect = max(j for j, dj in enumerate(d) if dj == best)
            assert ci == expect, (mode, xi, ci, expect)


def test_state_sr_is_value_unbiased():
    gen = torch.Generator().manual_seed(2)
    x = torch.rand(128, generator=gen) * 2 - 1
    x[0] = 1.0
    cb = ref.codebook("nf4_sr")
    acc = torch.zeros(128, dtype=torch.float64)
    trials = 4000
    for _ in range(trials):
        codes, _ = ref.encode(x, "nf4_sr", draws=torch.rand(1, 128, generator=gen))
        acc += cb[codes.long()].double()
    err = (acc / trials - x.double()).abs()
    width = (cb[1:] - cb[:-1]).max().item()
    assert err.max().item() < 5 * width / math.sqrt(trials)


def test_update_sr_is_preconditioner_unbiased():
    # The mean of 1/(sqrt(s*level/bias)+eps) over draws equals the value at x
    # (the property test_dyn4_la_upd_sr.py:44-79 checks for the lookahead variant).
    gen = torch.Generator().manual_seed(3)
    v = torch.rand(128, generator=gen) ** 6 * 1e-6
    v[0] = 1e-6
    bias, eps = 0.0975, 1e-8
    cb = ref.codebook("dyn4").double()
    s = v.abs().max().double()

    def f(level):
        return 1.0 / (torch.sqrt(torch.clamp(s * level / bias, min=0.0)) + eps)

    # Draws on a uniform grid of K points give the expectation up to (f(a) - f(b)) / K,
    # without the heavy tail a Monte-Carlo estimate has next to the zero level (f(0) = 1/eps).
    grid = 4096
    draws = ((torch.arange(grid, dtype=torch.float64) + 0.5) / grid).float().view(-1, 1).expand(grid, 128)
    codes, _ = ref.encode(v.repeat(grid), "dyn4_upd_sr_fp32read", draws=draws.contiguous(), bias=bias, eps=eps)
    levels = f(cb[codes.long()].view(grid, 128))
    expectation = levels.mean(0)
    x = v.double() / s
    target = f(x)
    idx = torch.searchsorted(cb.float(), (v / v.abs().max()).contiguous())
    a, b = cb[(idx - 1).clamp(min=0)], cb[idx.clamp(max=15)]
    slack = (f(a) - f(b)).abs() / grid + 1e-5 * target
    assert ((expectation - target).abs() <= slack).all()


def test_correctly_rounded_sqrt_is_correctly_rounded():
    """sqrt_correctly_rounded(v) = r with (r - ulp/2)^2 <= v <= (r + ulp/2)^2, checked in float64,
    where these squares are exact (25-bit operands), over every fp32 binade, with subnormals."""
    rng = np.random.default_rng(21)
    v = np.concatenate([
        (rng.random(200_000) * 2.0 ** rng.integers(-149, 128, 200_000)).astype(np.float32),
        np.array([0.0, 1.0, 2.0, 4.0, 0.25, 1e-45, 3.4e38], dtype=np.float32)])
    v = v[np.isfinite(v)]
    r = ref.sqrt_correctly_rounded(torch.from_numpy(v)).numpy().astype(np.float64)
    h = np.spacing(r.astype(np.float32)).astype(np.float64) / 2
    lo = np.where(r > 0, (r - h) ** 2, 0.0)
    hi = (r + h) ** 2
    assert np.all(lo <= v) and np.all(v <= hi)
    # ATen's CPU root on this host is within one ulp of it
    aten = torch.from_numpy(v).sqrt().numpy().astype(np.float64)
    assert np.all(np.abs(aten - r) <= 2 * h)


def test_update_sr_codes_depend_on_the_square_root_only_where_the_roots_differ():
    """The oracle's two update-SR square roots ("aten", the reference's host call, and "cr")
    change a code only where ATen's root of one of the value's three preconditioner arguments
    (its level pair and itself) is not the correctly rounded one.  The draws sit exactly on the
    correctly rounded probability, the draw most sensitive to the difference, so the check is
    not vacuous: codes do differ, and each difference is such a value."""
    gen = torch.Generator().manual_seed(29)
    blocks = 4096
    m = (torch.rand(blocks, 128, generator=gen) ** 4) * torch.exp(torch.randn(blocks, 1, generator=gen) * 4 - 14)
    values = m.reshape(-1)
    bias, eps = 0.0975, 1e-8
    scales = m.abs().amax(dim=1).clamp_min(1e-12)
    x = (m / scales[:, None])
    cb = ref.codebook("dyn4")
    _, _, a, b = ref._endpoints(x, cb)
    s = scales[:, None]

    def arg(level):
        return (s * level / bias).clamp_min(0.0)

    def f(level, root):
        return torch.reciprocal(root(arg(level)) + eps)

    cr = ref.sqrt_correctly_rounded
    fa, fb, fx = f(a, cr), f(b, cr), f(x, cr)
    p = ((fx - fb) / (fa - fb).clamp_min(1e-30)).clamp(0.0, 1.0)
    draws = p.contiguous()
    got = {mode: ref.encode(values, "dyn4_upd_sr_fp32read", draws=draws, bias=bias, eps=eps, usr_sqrt=mode)[0]
           for mode in ("aten", "cr")}
    differ = (got["aten"] != got["cr"]).view(blocks, 128)
    roots_agree = torch.ones_like(differ)
    for level in (a, b, x):
        v = arg(level)
        roots_agree &= v.sqrt() == cr(v)
    assert int(differ.sum()) > 0
    assert not bool((differ & roots_agree).any())


@pytest.mark.parametrize("recipe", ["zeeden", "zipsr"])
def test_first_step_equals_torch_adamw(recipe):
    # test_checkpoint_io.py:173-185 (ZE-EDEN) and test_dyn4_la_upd_sr.py:151-191 (ZIP-SR family).
    p = torch.zeros(4096)
    r = torch.nn.Parameter(p.clone())
    m2 = "dyn4_nz" if recipe == "zeeden" else "dyn4_upd_sr_fp32read"
    oracle = ref.Oracle([p], ref.Hyper(1e-3, (0.9, 0.95), 1e-8, 0.0), ["nf4"], [m2],
                        [recipe == "zeeden"], seed=0)
    adamw = torch.optim.AdamW([r], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)
    g = torch.full((4096,), 1e-8)
    oracle.step([g])
    r.grad = g.clone()
    adamw.step()
    torch.testing.assert_close(p, r.detach(), rtol=1e-6, atol=0)
    torch.testing.assert_close(p, torch.full_like(p, -0.0005), rtol=1e-6, atol=0)


# ---------------------------------------------------------------------------
# Planted mistakes: each plausible slip must break a golden comparison.
# ---------------------------------------------------------------------------

def _trajectory_matches(name):
    cfg, arrays = load(name)
    _, snaps = run_oracle(cfg, arrays)
    step = max(snaps)
    p, st = snaps[step][0]
    from tests._fixtures import tensor
    ok = torch.equal(bits(p), bits(tensor(arrays[f"after{step}_p0"], cfg["dtype"]).reshape(p.shape)))
    for key in ("m1_code", "m2_code", "m1_scale", "m2_scale"):
        if f"after{step}_p0_{key}" in arrays:
            ok &= torch.equal(bits(st[key]), bits(torch.from_numpy(arrays[f"after{step}_p0_{key}"])))
    return ok


def test_planted_mistakes_are_caught(monkeypatch):
    assert _trajectory_matches("traj_zeeden_f32.npz")
    assert _trajectory_matches("traj_zipsr_f32_seed0.npz")
    original_encode = ref.encode

    # 1. EDEN sums in plain sequential order instead of ATen's 8-lane x 4-accumulator order.
    def sequential_eden(values, mode, *, eden=False, **kw):
        codes, scales = original_encode(values, mode, eden=False, **kw)
        if eden:
            x = values.view(-1, 128) / values.view(-1, 128).abs().max(1).values.clamp_min(1e-12)[:, None]
            lv = ref.codebook(mode)[codes.long()].view_as(x)
            num = torch.zeros(x.shape[0])
            den = torch.zeros(x.shape[0])
            for j in range(128):
                num += x[:, j] * x[:, j]
                den += x[:, j] * lv[:, j]
            scales = scales * (num / den.clamp_min(1e-12))
        return codes, scales
    monkeypatch.setattr(ref, "encode", sequential_eden)
    assert not _trajectory_matches("traj_zeeden_f32.npz")
    monkeypatch.setattr(ref, "encode", original_encode)

    # 2. Round-to-nearest ties to the lower level.
    def ties_down(values, mode, **kw):
        codes, scales = original_encode(values, mode, **kw)
        if mode in ref.RTN_SCHEMES:
            x = values.view(-1, 128) / values.view(-1, 128).abs().max(1).values.clamp_min(1e-12)[:, None]
            lower, upper, a, b = ref._endpoints(x, ref.codebook(mode))
            c = torch.where((x - a).abs() <= (b - x).abs(), lower, upper).to(torch.uint8).reshape(-1)
            if mode == "dyn4_nz":
                c = c.masked_fill(c == 0, 1)
            codes = c
        return codes, scales
    monkeypatch.setattr(ref, "encode", ties_down)
    cfg, arrays = load("codec_vectors.npz")
    key = "lin4_nz_plain"
    codes, _ = ref.encode(torch.from_numpy(arrays[f"{key}_values"]), "lin4_nz")
    assert not np.array_equal(codes.numpy(), arrays[f"{key}_codes"])
    monkeypatch.setattr(ref, "encode", original_encode)

    # 3. Update-SR without the optimized path's endpoint guards.
    def no_guards(values, mode, **kw):
        kw["guards"] = False
        return original_encode(values, mode, **kw)
    monkeypatch.setattr(ref, "encode", no_guards)
    entries, arrays = load("codec_vectors.npz")
    mismatched = 0
    for e in entries:
        if not e["stochastic"]:
            continue
        codes, _ = ref.encode(torch.from_numpy(arrays[f"{e['key']}_values"]), e["mode"], eden=e["eden"],
                              draws=torch.from_numpy(arrays[f"{e['key']}_draws"]), bias=e["bias"], eps=e["eps"])
        mismatched += int(not np.array_equal(codes.numpy(), arrays[f"{e['key']}_codes"]))
    assert mismatched > 0
    monkeypatch.setattr(ref, "encode", original_encode)

    # 4. lerp written as unfused m + w*(g - m).
    original_lerp = torch.Tensor.lerp_

    def unfused(self, end, weight):
        return self.add_((end - self) * weight)
    monkeypatch.setattr(torch.Tensor, "lerp_", unfused)
    assert not _trajectory_matches("traj_zeeden_f32.npz")
    monkeypatch.setattr(torch.Tensor, "lerp_", original_lerp)

    # 5. Draws consumed for the whole tensor at initialization instead of one tile.
    original_init = ref.Oracle._init_moment

    def whole_tensor_init(self, index, moment, scheme, eden):
        saved = self.optimized
        self.optimized = False
        try:
            return original_init(self, index, moment, scheme, eden)
        finally:
            self.optimized = saved
    monkeypatch.setattr(ref.Oracle, "_init_moment", whole_tensor_init)
    cfg, arrays = load("traj_zipsr_chunked.npz")
    _, snaps = run_oracle(cfg, arrays)
    step = max(snaps)
    _, st = snaps[step][0]
    assert not torch.equal(st["m2_code"], torch.from_numpy(arrays[f"after{step}_p0_m2_code"]))


# ---------------------------------------------------------------------------
# Lookahead update-SR (quantization.py:779-895, adamw.py:566-614)
# ---------------------------------------------------------------------------

def _next_preconditioner(prev, grad, beta2, bias, eps):
    # The target of test_dyn4_la_upd_sr.py:14-23, written out in float64.
    return 1.0 / (((beta2 * prev + (1.0 - beta2) * grad.square()) / bias).sqrt() + eps)


def test_lookahead_block_scale_is_dyn4s():
    # test_dyn4_la_upd_sr.py:26-41
    z = torch.linspace(1e-4, 0.5, steps=128, dtype=torch.float32)
    g = torch.linspace(-0.2, 0.2, steps=128, dtype=torch.float32)
    _, la_scale, _ = ref.encode_lookahead(z, g, beta2=0.95, bias=0.25, eps=1e-8,
                                          draws=torch.rand(128, dtype=torch.float64))
    _, dyn4_scale = ref.encode(z, "dyn4")
    assert torch.equal(la_scale, dyn4_scale)


def _grid_draws(grid, n):
    return ((torch.arange(grid, dtype=torch.float64) + 0.5) / grid).view(-1, 1).expand(grid, n).contiguous()


@pytest.mark.parametrize("scale", [1.0, 1e-16])
def test_lookahead_is_next_preconditioner_unbiased(scale):
    # test_dyn4_la_upd_sr.py:44-79 by Monte Carlo; here on a uniform grid of draws, whose mean
    # is the expectation up to (f(lo) - f(hi)) / grid.  Negative and zero state clamps to 0.
    # scale 1e-16: sqrt(n / bias) is comparable to eps, where the bias does not cancel.
    gen = torch.Generator().manual_seed(5)
    z = torch.rand(128, generator=gen) ** 4 * 0.5 * scale
    z[:4] = torch.tensor([0.0, -1e-3, 0.5, 0.03125]) * scale
    g = (torch.rand(128, generator=gen) - 0.5) * 0.3 * math.sqrt(scale)
    beta2, bias, eps = 0.95, 0.4, 1e-8
    grid = 4096
    _, s, samples = ref.encode_lookahead(z.repeat(grid), g.repeat(grid), beta2=beta2, bias=bias, eps=eps,
                                         draws=_grid_draws(grid, 128))
    f = _next_preconditioner(samples.double().view(grid, 128), g.double(), beta2, bias, eps)
    expectation = f.mean(0)
    target = _next_preconditioner(z.clamp_min(0).double(), g.double(), beta2, bias, eps)
    cb = ref.codebook("dyn4").double()
    lo_hi = [_next_preconditioner(s[0].double() * cb[k], g.double(), beta2, bias, eps) for k in (0, 15)]
    slack = (lo_hi[0] - lo_hi[1]).abs() / grid + 1e-9 * target
    assert ((expectation - target).abs() <= slack).all()
    # values at a level (and the clamped zeros) are stored exactly; at scale 1e-16 the block
    # maximum sits below the 1e-12 scale floor and is no level
    for i in (0, 1, 2) if scale == 1.0 else (0, 1):
        assert torch.all(samples.view(grid, 128)[:, i] == z[i].clamp_min(0))


def test_lookahead_flat_interval_is_value_unbiased():
    # A fresh term that swamps beta2 * q makes f flat over the interval: the rule falls back to
    # value-unbiased rounding, E[sample] = z.
    # (levels 1e-9 apart against n ~ 5e4: relative differences of f near 1e-14 < 1e-12)
    gen = torch.Generator().manual_seed(6)
    z = torch.rand(128, generator=gen) * 1e-9
    g = torch.full((128,), 1e3)
    grid = 4096
    _, s, samples = ref.encode_lookahead(z.repeat(grid), g.repeat(grid), beta2=0.95, bias=1.0, eps=1e-8,
                                         draws=_grid_draws(grid, 128))
    mean = samples.double().view(grid, 128).mean(0)
    cb = ref.codebook("dyn4").double()
    width = s[0].double() * (cb[1:] - cb[:-1]).max()
    assert ((mean - z.double()).abs() <= width / grid + 1e-6 * z.double()).all()
    # both neighbours drawn (the fallback, not a guard) except at the block maximum, a level
    assert samples.view(grid, 128).std(0)[z != z.max()].min() > 0


@pytest.mark.parametrize("scheme", ["dyn4_la_upd_sr", "dyn4_proxy_la_upd_sr", "dyn4_vproxy_la_upd_sr"])
def test_lookahead_first_step_equals_torch_adamw(scheme):
    # test_dyn4_la_upd_sr.py:82-114 (pending state = (1 - beta2) g^2) and :276-316 (proxies).
    values = torch.linspace(-1.0, 1.0, steps=4096)
    grad = torch.linspace(-0.5, 0.5, steps=4096)
    p = values.clone()
    r = torch.nn.Parameter(values.clone())
    oracle = ref.Oracle([p], ref.Hyper(1e-3, (0.9, 0.95), 1e-8, 0.0), ["fp32"], [scheme], [False], seed=0,
                        optimized=False)
    adamw = torch.optim.AdamW([r], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)
    oracle.step([grad.clone()])
    r.grad = grad.clone()
    adamw.step()
    torch.testing.assert_close(p, r.detach(), rtol=1e-6, atol=1e-6)
    m2 = oracle.states[0].m2
    if scheme == "dyn4_la_upd_sr":
        torch.testing.assert_close(m2.values, (1.0 - 0.95) * grad.square())
        assert m2.codes is None
    else:
        assert m2.codes.numel() == 2048 and torch.isfinite(ref.decode(m2.codes, m2.scales, "dyn4", 4096)).all()


def _all_params_match(name):
    cfg, arrays = load(name)
    _, snaps = run_oracle(cfg, arrays)
    step = max(snaps)
    from tests._fixtures import tensor
    ok = True
    for i, (p, st) in enumerate(snaps[step]):
        ok &= torch.equal(bits(p), bits(tensor(arrays[f"after{step}_p{i}"], cfg["dtype"]).reshape(p.shape)))
        for key in ("m2_code", "m2_scale", "m2_pending"):
            if f"after{step}_p{i}_{key}" in arrays:
                ok &= torch.equal(bits(st[key]), bits(torch.from_numpy(arrays[f"after{step}_p{i}_{key}"])))
    return ok


def test_lookahead_planted_mistakes_are_caught(monkeypatch):
    name = "traj_lookahead_groups.npz"
    assert _all_params_match(name)
    original = ref.encode_lookahead

    # 1. v-proxy with the gradient's fresh term instead of (1 - beta2) m2.
    monkeypatch.setattr(ref, "encode_lookahead", lambda *a, fresh_proxy=None, **kw: original(*a, **kw))
    assert not _all_params_match(name)
    # 2. Probabilities without the next step's beta2 decay of the candidate levels.
    monkeypatch.setattr(ref, "encode_lookahead", lambda *a, beta2, **kw: original(*a, beta2=1.0 - 1e-12, **kw))
    assert not _all_params_match(name)
    # 3. Bias corrections one step behind (1 - beta2^(k-1) for 1 - beta2^k).  The bias cancels
    # from P(lo) wherever sqrt(m2 / bias) >> eps, so this needs the small-gradient trajectory.
    small = "traj_lookahead_small_grad.npz"
    monkeypatch.setattr(ref, "encode_lookahead", original)
    assert _all_params_match(small)

    def step_behind(*a, bias, **kw):
        k = round(math.log(1.0 - bias) / math.log(0.95))
        return original(*a, bias=1.0 - 0.95 ** (k - 1) if k > 1 else bias, **kw)
    monkeypatch.setattr(ref, "encode_lookahead", step_behind)
    assert not _all_params_match(small)


# ---------------------------------------------------------------------------
# Gradient clipping before the step (examples/train_gpt_small.py:214)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtypes", [[torch.float32] * 3, [torch.bfloat16] * 3, [torch.float16] * 3,
                                    [torch.bfloat16, torch.float32, torch.float16]])
def test_clip_restatement_matches_torch(dtypes):
    # The float64 restatement the device follows against torch.nn.utils.clip_grad_norm_ itself:
    # within torch's fp32 accumulation error (one storage ulp for 16-bit norms), and the same
    # coefficient arithmetic bit for bit given the total.
    gen = torch.Generator().manual_seed(8)
    shapes = [(300, 700), (4097,), (5,)]
    for scale in (1e-3, 1.0):
        grads = [(torch.randn(s, generator=gen) * scale).to(dt) for s, dt in zip(shapes, dtypes)]
        for max_norm in (1e-4, 1e4):
            t64, c64 = ref.clip_grad_norm_f64(grads, max_norm)
            tt, ct = ref.clip_grad_norm(grads, max_norm)
            assert t64.dtype == tt.dtype
            ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}.get(tt.dtype, 0.0)
            assert abs(float(t64) - float(tt)) <= max(2e-5, 2 * ulp) * float(tt)
            assert torch.equal(c64, torch.clamp(max_norm / (t64 + 1e-6), max=1.0))
            assert (float(c64) == 1.0) == (max_norm == 1e4)


def test_clip_scaling_is_one_rounding_to_the_gradient_dtype():
    # _foreach_mul_ by the coefficient: an fp32 product rounded once to the gradient's dtype
    # (exact for two 16-bit operands), which the step reproduces in-register.
    g = [torch.randn(1000).to(torch.bfloat16), torch.randn(1000)]
    for coef in (torch.tensor(0.3, dtype=torch.bfloat16), torch.tensor(0.3)):
        out = ref.scale_grads(g, coef)
        for a, b in zip(out, g):
            expect = (b.float() * coef.float()).to(b.dtype)
            assert torch.equal(bits(a), bits(expect))
