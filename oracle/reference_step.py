"""CPU oracle for the 4-bit AdamW step -- test infrastructure, never shipped.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
import this module, and only as the checker (or, in the bench, as the timed CPU
restatement of the reference's own eager update).  The product
(``adamw4bit_amd``) never imports it.

It restates, with PyTorch CPU tensor operations in the reference's exact operation
order, the parts of ``adamw4bit`` that the fused HIP step replaces:

* the bounded-chunk update of the optimized backend: ``_step_chunk``
  (``src/adamw4bit/_optimized.py:206-234``), its moment views
  (``_moment_buffer.py:89-179``), chunk codec (``_optimized_quantization.py:37-107``)
  and rounding rules with endpoint guards (``_compiled_quantization.py:30-109``);
* the per-parameter driver around it: state initialization, step counting, bias
  corrections, chunk loop and random-draw consumption
  (``_optimized.py:145-203``, ``adamw.py:281-324``);
* the default reference step (``adamw.py:472-805``) for the scheme set shared with
  the optimized path; it differs only in having no endpoint guards in stochastic
  rounding (``quantization.py:279-377``) and in drawing ``numel`` uniforms when a
  stochastic moment is initialized (``adamw.py:524-545``);
* the reference step's read-back m2 schemes (``dyn4_upd_sr``, ``lin4_upd_sr``,
  ``*_upd_sr_store_eden``, ``adamw.py:615-656``), whose update uses the m2 just
  encoded (``_update_sampled_read``), and its lookahead update-SR schemes
  (``dyn4_la_upd_sr``, ``dyn4_proxy_la_upd_sr``, ``dyn4_vproxy_la_upd_sr``,
  ``adamw.py:566-614``) with their float64 quantizer (``encode_lookahead``,
  ``quantization.py:779-895``).  A parameter whose schemes the optimized
  backend does not accept takes the reference step, as the backend's preflight
  sends it there (``_optimized.py:94-126``).

Because the operations are ATen CPU kernels called in the reference's order, the
element arithmetic (lerp as a fused multiply-add, true division, the 8-lane by
4-accumulator order of the per-block sums, bf16/fp16 rounding points) is the
reference's own.  Random draws come from ``torch.Generator`` CPU streams seeded
exactly as the reference seeds them, and every draw tensor consumed is recorded so
a device implementation can be fed the same draws.

Pinning (see ``tests/test_oracle_*.py``): golden trajectories written by
``tests/golden/make_golden.py`` from the reference itself, the reference's
known-answer tests (codebooks, nibble order, tie rule, scale floor, zero floor,
first step equal to ``torch.optim.AdamW``), the EDEN invariant and brute force over
all 16 levels on small blocks.  ``encode_lookahead`` and the lookahead flows: the
reference's lookahead trajectories (one with gradients near 1e-8, where the bias
correction matters), the next-step preconditioner's unbiasedness over a grid of draws
against an independently written preconditioner, the flat-interval fallback's value
unbiasedness and planted mistakes.  The gradient clipping that precedes a step:
``clip_grad_norm`` is torch's own ``clip_grad_norm_`` on CPU copies;
``clip_grad_norm_f64`` (float64 sums, torch's rounding points) is checked against it
within torch's fp32 accumulation error, with the coefficient bit for bit, and
``scale_grads`` against the single rounding of an fp32 product to the gradient dtype.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

BLOCK = 128
CHUNK_NUMEL = 1 << 19  # _optimized.py:33
QUANT_RNG_OFFSETS = {"m1": 0x1A2B3C4D, "m2": 0x5E6F7789}  # adamw.py:122-125

# Codebooks from the reference's closed forms (quantization.py:201-237, 401-422, 457-497).
_NF4 = [-1.0000000, -0.6961928, -0.5250731, -0.3949175, -0.2844414, -0.1847734, -0.0910500, 0.0,
        0.0795803, 0.1609302, 0.2461123, 0.3379152, 0.4407098, 0.5626170, 0.7229568, 1.0000000]


def _dynamic_map(signed: bool) -> torch.Tensor:
    """Dettmers dynamic map with 3 exponent bits and 4 total bits (quantization.py:201-237)."""
    values: List[float] = []
    for i in range(3):
        items = (2 ** i + 1) if signed else (2 ** (i + 1) + 1)
        edges = torch.linspace(0.1, 1, items)
        mids = (edges[:-1] + edges[1:]) / 2.0
        values += ((10 ** (-2 + i)) * mids).tolist()
        if signed:
            values += (-(10 ** (-2 + i)) * mids).tolist()
    values += [0.0, 1.0]
    values.sort()
    return torch.tensor(values, dtype=torch.float32)


def codebook(mode: str) -> torch.Tensor:
    if mode.startswith("nf4"):
        return torch.tensor(_NF4, dtype=torch.float32)
    if mode.startswith("sdyn4"):
        return _dynamic_map(True)
    if mode == "lin4_nz":
        return torch.linspace(0.0, 1.0, 17, dtype=torch.float32)[1:]
    if mode.startswith("lin4"):
        return torch.linspace(0.0, 1.0, 16, dtype=torch.float32)
    if mode.startswith("dyn4"):
        return _dynamic_map(False)
    raise ValueError(f"no 16-level codebook for {mode!r}")


RTN_SCHEMES = {"nf4", "sdyn4", "lin4", "lin4_nz", "dyn4", "dyn4_nz"}
STATE_SR_SCHEMES = {"nf4_sr", "sdyn4_sr", "lin4_sr", "dyn4_sr"}
FP32_READ_SCHEMES = {"lin4_upd_sr_fp32read", "dyn4_upd_sr_fp32read", "dyn4_lookahead_sr",
                     "dyn4_upd_sr_fp32read_nextbc"}
# Reference-step m2 schemes whose update reads the sampled value back (adamw.py:636-656), and
# those that read it with the pre-EDEN scale, store the EDEN-calibrated scale and keep
# 1 / denominator as "m2_read_preconditioner" (adamw.py:615-635).  Same update-SR rule
# (quantization.py:318-377, 486-526).
SAMPLED_READ_SCHEMES = {"lin4_upd_sr", "dyn4_upd_sr"}
STORE_EDEN_SCHEMES = {"lin4_upd_sr_store_eden", "dyn4_upd_sr_store_eden"}
UPDATE_SR_SCHEMES = FP32_READ_SCHEMES | SAMPLED_READ_SCHEMES | STORE_EDEN_SCHEMES
# Lookahead update-SR (adamw.py:118-120): the pending form keeps m2 in fp32 and samples it
# before each update; the proxies store m2 sampled for the next step's update.
PENDING_LOOKAHEAD_SCHEMES = {"dyn4_la_upd_sr"}
VPROXY_LOOKAHEAD_SCHEMES = {"dyn4_vproxy_la_upd_sr"}
LOOKAHEAD_SCHEMES = PENDING_LOOKAHEAD_SCHEMES | VPROXY_LOOKAHEAD_SCHEMES | {"dyn4_proxy_la_upd_sr"}
NEXT_BIAS_SCHEMES = {"dyn4_lookahead_sr", "dyn4_upd_sr_fp32read_nextbc"}
M1_SCHEMES = {"fp32", "nf4", "nf4_sr", "sdyn4", "sdyn4_sr"}            # _optimized.py:36
M2_SCHEMES = {"fp32", "lin4", "lin4_sr", "lin4_nz", "dyn4", "dyn4_sr", "dyn4_nz"} | FP32_READ_SCHEMES


def is_stochastic(mode: str) -> bool:
    return mode in STATE_SR_SCHEMES or mode in UPDATE_SR_SCHEMES or mode in LOOKAHEAD_SCHEMES


# ---------------------------------------------------------------------------
# Codec
# ---------------------------------------------------------------------------

def decode(packed: torch.Tensor, scales: torch.Tensor, mode: str, numel: int) -> torch.Tensor:
    """Packed nibbles -> float32 values (``_optimized_quantization.py:91-107``)."""
    codes = torch.empty(numel, dtype=torch.uint8)
    codes[0::2] = packed & 0x0F
    codes[1::2] = packed[: numel // 2] >> 4
    levels = torch.index_select(codebook(mode), 0, codes.to(torch.int32))
    return (levels.view(-1, BLOCK) * scales.unsqueeze(1)).view(-1)


def _endpoints(x: torch.Tensor, cb: torch.Tensor):
    """searchsorted-left neighbours (``_compiled_quantization.py:30-38``)."""
    idx = torch.searchsorted(cb, x, out_int32=True)
    lower = (idx - 1).clamp(min=0)
    upper = idx.clamp(max=cb.numel() - 1)
    return lower, upper, cb[lower.long()], cb[upper.long()]


def sqrt_correctly_rounded(v: torch.Tensor) -> torch.Tensor:
    """The correctly rounded fp32 square root: the float64 root of an fp32 value, rounded once
    to fp32 (float64 carries more than the 2 * 24 + 2 bits that make this single rounding exact)."""
    return v.to(torch.float64).sqrt().to(torch.float32)


def encode(values: torch.Tensor, mode: str, *, eden: bool = False,
           draws: Optional[torch.Tensor] = None, bias: float = 1.0, eps: float = 1e-8,
           guards: bool = True, usr_sqrt: str = "aten") -> Tuple[torch.Tensor, torch.Tensor]:
    """float32 values (length a multiple of 128) -> (unpacked uint8 codes, float32 scales).

    ``guards=True`` is the optimized path (``_optimized_quantization.py:46-88`` with the
    rounding of ``_compiled_quantization.py``); ``guards=False`` is the reference
    step's strategies (``quantization.py:254-377``, ``:898-971``).

    ``usr_sqrt`` is the square root of the update-SR preconditioner
    ``1 / (sqrt((s * l) / bias) + eps)`` (``_compiled_quantization.py:74-109``): ``"aten"``
    is ATen's CPU ``sqrt`` as the reference calls it (vectorised, within one ulp of the
    correctly rounded root, host-dependent), ``"cr"`` the correctly rounded root.  Every other
    operation is the same in both.
    """
    if usr_sqrt not in ("aten", "cr"):
        raise ValueError(f"usr_sqrt must be 'aten' or 'cr', got {usr_sqrt!r}")
    blocked = values.view(-1, BLOCK)
    scales = blocked.abs().max(dim=1).values.clamp_min(1e-12)
    x = blocked / scales.unsqueeze(1)
    cb = codebook(mode)
    lower, upper, a, b = _endpoints(x, cb)
    if mode in RTN_SCHEMES:
        pick_lower = (x - a).abs() < (b - x).abs()
        codes = torch.where(pick_lower, lower, upper)
    elif mode in STATE_SR_SCHEMES:
        assert draws is not None and draws.shape == x.shape
        width = b - a
        p = (x - a) / width.clamp_min(1e-12)
        p = torch.where(width > 0, p, 0.0).clamp(0.0, 1.0)
        if guards:
            p = torch.where(x >= b, 1.0, p)
            p = torch.where(x <= a, 0.0, p)
        codes = torch.where(draws < p, upper, lower)
    elif mode in UPDATE_SR_SCHEMES:
        assert draws is not None and draws.shape == x.shape
        s = scales.unsqueeze(1)
        bias_c = max(float(bias), 1e-12)

        def preconditioner(level: torch.Tensor) -> torch.Tensor:
            v_hat = (s * level / bias_c).clamp_min(0.0)
            root = v_hat.sqrt() if usr_sqrt == "aten" else sqrt_correctly_rounded(v_hat)
            return torch.reciprocal(root + eps)  # ``1.0 / t`` is reciprocal(t) * 1.0

        f_a, f_b, f_x = preconditioner(a), preconditioner(b), preconditioner(x)
        den = f_a - f_b
        p = (f_x - f_b) / den.clamp_min(1e-30)
        p = torch.where((b > a) & (den > 0), p, 1.0).clamp(0.0, 1.0)
        if guards:
            p = torch.where(x >= b, 0.0, p)
            p = torch.where(x <= a, 1.0, p)
        codes = torch.where(draws < p, lower, upper)
    else:
        raise ValueError(f"unsupported scheme {mode!r}")
    codes = codes.to(torch.uint8)
    if mode == "dyn4_nz":
        codes = codes.masked_fill(codes == 0, 1)
    if eden:
        levels = torch.index_select(cb, 0, codes.reshape(-1).to(torch.int32)).view_as(x)
        num = (x * x).sum(dim=1)
        den = (x * levels).sum(dim=1)
        scales = scales * (num / den.clamp_min(1e-12))
    return codes.reshape(-1), scales


def encode_lookahead(z_prev: torch.Tensor, grad: torch.Tensor, *, beta2: float, bias: float, eps: float,
                     draws: torch.Tensor, fresh_proxy: Optional[torch.Tensor] = None):
    """Lookahead update-SR of a second moment (``quantize_dyn4_la_upd_sr``, quantization.py:779-895).

    The dyn4 neighbours lo <= x <= hi of x = clamp(z / s, 0, 1) (s the block absmax floored at
    1e-12, in fp32) are chosen so that the NEXT step's preconditioner is unbiased: with
    q = s * level and n(q) = max(beta2 q + fresh, 0) in float64,
        P(lo) = (f(n(z)) - f(n(q_hi))) / max(f(n(q_lo)) - f(n(q_hi)), 1e-300),
        f(n) = 1 / (sqrt(n / bias) + eps),
    or 1 - clamp((z - q_lo) / (q_hi - q_lo), 0, 1) where f is flat over the interval and 1 where
    the interval is empty; fresh is (1 - beta2) g^2 in float64 or a caller's proxy.  Returns
    (unpacked codes, fp32 scales, fp32 samples s * level).  ``draws``: float64 uniforms.
    """
    z = z_prev.reshape(-1, BLOCK).clamp_min(0)
    s = z.abs().max(dim=1).values.clamp_min(1e-12)
    x = (z / s.unsqueeze(1)).clamp(0.0, 1.0)
    cb = codebook("dyn4")
    lower, upper, _, _ = _endpoints(x, cb)
    cb64 = cb.to(torch.float64)
    s64 = s.to(torch.float64).unsqueeze(1)
    if fresh_proxy is None:
        fresh = (1.0 - float(beta2)) * grad.reshape(-1, BLOCK).to(torch.float64).square()
    else:
        fresh = fresh_proxy.reshape(-1, BLOCK).clamp_min(0).to(torch.float64)
    bias = max(float(bias), 1e-12)

    def f(q: torch.Tensor) -> torch.Tensor:
        n = (float(beta2) * q + fresh).clamp_min(0.0)
        return 1.0 / (n.div(bias).sqrt() + float(eps))

    q_lo, q_hi = s64 * cb64[lower.long()], s64 * cb64[upper.long()]
    f_lo, f_z, f_hi = f(q_lo), f(z.to(torch.float64)), f(q_hi)
    den, width = f_lo - f_hi, q_hi - q_lo
    raw = (f_z - f_hi) / den.clamp_min(1e-300)
    fallback = 1.0 - ((z.to(torch.float64) - q_lo) / width.clamp_min(1e-300)).clamp(0.0, 1.0)
    empty = width <= 0.0
    flat = ~empty & (den.abs() <= 1e-12 * torch.maximum(f_lo.abs(), f_hi.abs()).clamp_min(1.0))
    p_lo = torch.where(empty, 1.0, torch.where(flat, fallback, raw)).clamp(0.0, 1.0)
    take_lo = draws.reshape(p_lo.shape) < p_lo
    codes = torch.where(take_lo, lower, upper).to(torch.uint8)
    samples = torch.where(take_lo, q_lo, q_hi).to(torch.float32)
    return codes.reshape(-1), s, samples.reshape(-1)


def clip_grad_norm(grads: List[torch.Tensor], max_norm: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """The gradient clipping the reference's trainer runs before each step (an HF Trainer with
    ``max_grad_norm``, examples/train_gpt_small.py:214): ``torch.nn.utils.clip_grad_norm_``
    (norm type 2) on CPU copies.  Returns (total norm, clip coefficient), both in the promoted
    gradient dtype, as torch computes them (clip_grad.py: per-tensor ``_foreach_norm``, the norm
    of the stacked norms, ``max_norm / (total + 1e-6)`` clamped at 1)."""
    params = []
    for g in grads:
        p = torch.nn.Parameter(torch.empty(g.shape, dtype=g.dtype))
        p.grad = g.detach().clone()
        params.append(p)
    total = torch.nn.utils.clip_grad_norm_(params, max_norm)
    return total, torch.clamp(max_norm / (total + 1e-6), max=1.0)


def clip_grad_norm_f64(grads: List[torch.Tensor], max_norm: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """``clip_grad_norm`` with float64 sums of squares in place of torch's fp32 accumulation and
    torch's rounding points otherwise: norm_t = grad_dtype(fp32(sqrt(sum g^2))), total =
    R(fp32(sqrt(sum norm_t^2))) with R the promoted dtype, and the coefficient computed by torch's
    own operations on that total."""
    dtype = grads[0].dtype
    for g in grads[1:]:
        if g.dtype != dtype:
            dtype = torch.float32
    sq = 0.0
    for g in grads:
        n = math.sqrt(float(g.detach().to(torch.float64).square().sum()))
        n = float(torch.tensor(n, dtype=torch.float64).to(torch.float32).to(g.dtype))
        sq += n * n
    total = torch.tensor(math.sqrt(sq), dtype=torch.float64).to(torch.float32).to(dtype)
    return total, torch.clamp(max_norm / (total + 1e-6), max=1.0)


def scale_grads(grads: List[torch.Tensor], coef: torch.Tensor) -> List[torch.Tensor]:
    """The in-place ``_foreach_mul_`` of the clipping, on copies: each gradient becomes
    grad_dtype(fp32(g * coef))."""
    out = [g.detach().clone() for g in grads]
    torch._foreach_mul_(out, coef)
    return out


def pack(codes: torch.Tensor) -> torch.Tensor:
    out = codes[0::2].clone()
    out[: codes.numel() // 2] |= codes[1::2] << 4
    return out


# ---------------------------------------------------------------------------
# Per-parameter state and the step driver
# ---------------------------------------------------------------------------

@dataclass
class Hyper:
    lr: float = 1e-3
    betas: Tuple[float, float] = (0.9, 0.95)
    eps: float = 1e-8
    weight_decay: float = 0.1


@dataclass
class MomentState:
    scheme: str                      # effective scheme ("fp32" when ineligible)
    values: Optional[torch.Tensor] = None   # fp32 state
    codes: Optional[torch.Tensor] = None    # packed uint8 [(n+1)//2]
    scales: Optional[torch.Tensor] = None   # fp32 [n/128]


@dataclass
class ParamState:
    step: int = 0
    m1: Optional[MomentState] = None
    m2: Optional[MomentState] = None
    read_preconditioner: Optional[torch.Tensor] = None  # store-EDEN schemes: 1 / denominator


@dataclass
class DrawLog:
    """Uniform draws consumed by one write of one moment of one parameter."""
    param: int
    moment: str
    step: int
    draws: torch.Tensor  # flat float32, one per element


def effective_scheme(numel: int, scheme: str) -> str:
    """TorchAO eligibility (``adamw.py:807-817``)."""
    if scheme == "fp32" or (numel >= 4096 and numel % BLOCK == 0):
        return scheme
    return "fp32"


class Oracle:
    """Multi-parameter optimizer restatement over CPU tensors.

    ``optimized=True`` follows the bounded-chunk backend; ``optimized=False`` the
    reference step.  ``m1_schemes``/``m2_schemes``/``eden`` are per parameter so
    mixed-scheme parameter lists (runtime ``nf4_sr`` switches, ablation slices) can
    be expressed.
    """

    def __init__(self, params: List[torch.Tensor], hyper: Hyper, m1_schemes: List[str],
                 m2_schemes: List[str], eden: List[bool], *, seed: Optional[int] = None,
                 optimized: bool = True, chunk: int = CHUNK_NUMEL, record_draws: bool = False,
                 draw_fn=None, usr_sqrt: str = "aten"):
        self.params = params
        self.hyper = hyper
        self.m1_schemes = list(m1_schemes)
        self.m2_schemes = list(m2_schemes)
        self.eden = list(eden)
        self.optimized = optimized
        self.chunk = chunk
        self.states = [ParamState() for _ in params]
        self.generators: Dict[str, Optional[torch.Generator]] = {}
        for moment, offset in QUANT_RNG_OFFSETS.items():
            if seed is None:
                self.generators[moment] = None
            else:
                gen = torch.Generator()
                gen.manual_seed((seed + offset) % ((1 << 63) - 1))
                self.generators[moment] = gen
        self.record_draws = record_draws
        # Optional source of uniforms: draw_fn(moment, n) -> n float32 values, used in place of
        # the CPU generators (to replay the draws a device implementation consumed).
        self.draw_fn = draw_fn
        # Square root of the update-SR preconditioners (``encode``): "aten" as the reference
        # computes it on this host, "cr" correctly rounded.
        self.usr_sqrt = usr_sqrt
        self.draw_log: List[DrawLog] = []
        self.draw_counts = {"m1": 0, "m2": 0}
        self._param_optimized = True  # the optimized backend accepts the parameter's schemes

    # -- random draws -------------------------------------------------------
    def _draw(self, moment: str, n: int, param: int, step: int, log: bool,
              dtype: torch.dtype = torch.float32) -> torch.Tensor:
        if self.draw_fn is not None:
            u = self.draw_fn(moment, n).reshape(n // BLOCK, BLOCK).to(dtype)
        else:
            u = torch.rand((n // BLOCK, BLOCK), dtype=dtype, generator=self.generators[moment])
        self.draw_counts[moment] += n
        if self.record_draws and log:
            self.draw_log.append(DrawLog(param, moment, step, u.reshape(-1).clone()))
        return u

    # -- initialization -------------------------------------------------------
    def _init_moment(self, index: int, moment: str, scheme: str, eden: bool) -> MomentState:
        p = self.params[index]
        n = p.numel()
        if scheme == "fp32":
            return MomentState("fp32", values=torch.zeros(n, dtype=torch.float32))
        if scheme in PENDING_LOOKAHEAD_SCHEMES:  # adamw.py:534-535
            return MomentState(scheme, values=torch.zeros(n, dtype=torch.float32))
        if scheme in LOOKAHEAD_SCHEMES:  # the proxies store zeros with plain dyn4 (quantization.py:583-584)
            codes, scales = encode(torch.zeros(n, dtype=torch.float32), "dyn4")
            return MomentState(scheme, codes=pack(codes), scales=scales)
        optimized = self.optimized and self._param_optimized
        if optimized:
            # _moment_buffer.py:106-126: encode one zero tile, broadcast its first byte/scale.
            tile = n if n <= self.chunk else math.lcm(BLOCK, 2)
        else:
            tile = n  # adamw.py:524-545 encodes the whole zero tensor
        draws = self._draw(moment, tile, index, 0, log=False) if is_stochastic(scheme) else None
        codes, scales = encode(torch.zeros(tile, dtype=torch.float32), scheme, eden=eden,
                               draws=draws, guards=optimized, usr_sqrt=self.usr_sqrt)
        byte = pack(codes)[:1]
        return MomentState(scheme, codes=byte.expand((n + 1) // 2).clone(),
                           scales=scales[:1].expand(n // BLOCK).clone())

    # -- one step -------------------------------------------------------------
    def step(self, grads: List[torch.Tensor]) -> None:
        for index, (p, g) in enumerate(zip(self.params, grads)):
            self._step_param(index, p, g)

    def _step_param(self, index: int, p: torch.Tensor, grad: torch.Tensor) -> None:
        st = self.states[index]
        n = p.numel()
        s1 = effective_scheme(n, self.m1_schemes[index])
        s2 = effective_scheme(n, self.m2_schemes[index])
        eden = self.eden[index]
        # The optimized backend's preflight sends other scheme pairs to the reference step
        # (_optimized.py:94-126).
        self._param_optimized = s1 in M1_SCHEMES and s2 in M2_SCHEMES
        optimized = self.optimized and self._param_optimized
        if st.step == 0:
            st.m1 = self._init_moment(index, "m1", s1, False)
            st.m2 = self._init_moment(index, "m2", s2, eden)
        else:
            # A runtime m1 switch (nf4 <-> nf4_sr) keeps the codes and changes only the rule.
            st.m1.scheme = s1
        st.step += 1
        b1, b2 = self.hyper.betas
        bc1, bc2 = 1 - b1 ** st.step, 1 - b2 ** st.step
        storage_bc = 1 - b2 ** (st.step + 1) if s2 in NEXT_BIAS_SCHEMES else bc2
        flat_p = p.view(-1)
        flat_g = grad.reshape(-1)
        if s2 in SAMPLED_READ_SCHEMES or s2 in STORE_EDEN_SCHEMES:
            self._update_sampled_read(index, st, flat_p, flat_g, s2, eden, bc1, bc2)
            return
        if s2 in LOOKAHEAD_SCHEMES:
            self._update_lookahead(index, st, flat_p, flat_g, s2, bc1, bc2)
            return
        chunk = self._chunk_size(s1, s2) if optimized else n
        for start in range(0, n, chunk):
            stop = min(start + chunk, n)
            self._update_chunk(index, st, flat_p[start:stop], flat_g[start:stop], start, stop,
                               s1, s2, eden, bc1, bc2, storage_bc)

    def _chunk_size(self, s1: str, s2: str) -> int:
        sizes = [BLOCK for s in (s1, s2) if s != "fp32"]
        align = math.lcm(2, *sizes) if sizes else 1
        return self.chunk // align * align

    def _update_chunk(self, index, st, p, grad, start, stop, s1, s2, eden, bc1, bc2, storage_bc):
        """``_step_chunk`` (_optimized.py:206-234) on elements [start, stop)."""
        hp = self.hyper
        n = stop - start
        g = grad.to(dtype=torch.float32)
        m1 = self._read(st.m1, start, stop)
        m2 = self._read(st.m2, start, stop)
        m1.lerp_(g, 1 - hp.betas[0])
        m2.lerp_(g.square(), 1 - hp.betas[1])
        den = m2.sqrt().div_(math.sqrt(bc2)).add_(hp.eps)
        p.mul_(1 - hp.lr * hp.weight_decay)
        p.addcdiv_(m1, den, value=-hp.lr / bc1)
        draws = self._draw("m1", n, index, st.step, True) if is_stochastic(s1) else None
        self._write(st.m1, m1, start, stop, eden=False, draws=draws, bias=1.0, eps=1e-8)
        draws = self._draw("m2", n, index, st.step, True) if is_stochastic(s2) else None
        self._write(st.m2, m2, start, stop, eden=eden, draws=draws, bias=storage_bc, eps=hp.eps)
        if s2 not in STORE_EDEN_SCHEMES:
            st.read_preconditioner = None

    def _update_sampled_read(self, index, st, p, grad, s2, eden, bc1, bc2):
        """The reference step for m2 schemes read back after their encode (adamw.py:615-656):
        m2 is encoded first (update-SR towards the current bias correction) and the
        denominator uses cb[code] * scale -- the stored scale, or for ``*_store_eden`` the scale
        before EDEN, whose calibration goes only to the stored scale
        (``quantize_with_dequantized``, ``apply_eden_correction_to_quant_state``,
        quantization.py:748-776, 1007-1037)."""
        hp = self.hyper
        n = p.numel()
        g = grad.to(dtype=torch.float32)
        m1 = self._read(st.m1, 0, n)
        m2 = self._read(st.m2, 0, n)
        m1.lerp_(g, 1 - hp.betas[0])
        m2.lerp_(g.square(), 1 - hp.betas[1])
        draws = self._draw("m2", n, index, st.step, True)
        store_eden = s2 in STORE_EDEN_SCHEMES
        codes, read_scales = encode(m2, s2, eden=eden and not store_eden, draws=draws, bias=bc2, eps=hp.eps,
                                    guards=False, usr_sqrt=self.usr_sqrt)
        stored_scales = read_scales
        if store_eden:
            _, stored_scales = encode(m2, s2, eden=True, draws=draws, bias=bc2, eps=hp.eps, guards=False,
                                      usr_sqrt=self.usr_sqrt)
        packed = pack(codes)
        m2_read = decode(packed, read_scales, s2, n)
        den = (m2_read.sqrt() / math.sqrt(bc2)).add_(hp.eps)
        st.read_preconditioner = den.reciprocal() if store_eden else None
        p.mul_(1 - hp.lr * hp.weight_decay)
        p.addcdiv_(m1, den, value=-hp.lr / bc1)
        draws = self._draw("m1", n, index, st.step, True) if is_stochastic(st.m1.scheme) else None
        self._write(st.m1, m1, 0, n, eden=False, draws=draws, bias=1.0, eps=1e-8)
        st.m2.codes[:] = packed
        st.m2.scales[:] = stored_scales

    def _update_lookahead(self, index, st, p, grad, s2, bc1, bc2):
        """The reference step for lookahead update-SR m2 (adamw.py:566-614, 771-790).

        Pending form: a lookahead sample A of the pending fp32 state (bias_c2), then
        m2 = A * beta2 + (1 - beta2) g^2 (``mul`` then ``addcmul``), kept in fp32 as the next
        pending state.  Proxies: m2 = lerp(decoded m2, g^2, 1 - beta2) for the update, stored
        as codes sampled for the next step's bias correction with fresh term (1 - beta2) g^2
        (proxy) or (1 - beta2) m2 (v-proxy).  Every write draws numel float64 uniforms."""
        hp = self.hyper
        b1, b2 = hp.betas
        n = p.numel()
        g = grad.to(dtype=torch.float32)
        m1 = self._read(st.m1, 0, n)
        m1.lerp_(g, 1 - b1)
        draws = self._draw("m2", n, index, st.step, True, dtype=torch.float64)
        if s2 in PENDING_LOOKAHEAD_SCHEMES:
            _, _, sample = encode_lookahead(st.m2.values, g, beta2=b2, bias=bc2, eps=hp.eps, draws=draws)
            m2 = sample.mul(b2).addcmul(g, g, value=1 - b2)
        else:
            m2 = self._read(st.m2, 0, n)
            m2.lerp_(g.square(), 1 - b2)
        den = (m2.sqrt() / math.sqrt(bc2)).add_(hp.eps)
        if s2 not in PENDING_LOOKAHEAD_SCHEMES:
            proxy = (1 - b2) * m2 if s2 in VPROXY_LOOKAHEAD_SCHEMES else None
            codes, scales, _ = encode_lookahead(m2, g, beta2=b2, bias=1 - b2 ** (st.step + 1), eps=hp.eps,
                                                draws=draws, fresh_proxy=proxy)
        p.mul_(1 - hp.lr * hp.weight_decay)
        p.addcdiv_(m1, den, value=-hp.lr / bc1)
        self._write(st.m1, m1, 0, n, eden=False, draws=None, bias=1.0, eps=1e-8)  # fp32 or nf4
        if s2 in PENDING_LOOKAHEAD_SCHEMES:
            st.m2.values = m2
        else:
            st.m2.codes[:] = pack(codes)
            st.m2.scales[:] = scales
        st.read_preconditioner = None

    @staticmethod
    def _read(ms: MomentState, start: int, stop: int) -> torch.Tensor:
        if ms.scheme == "fp32":
            return ms.values[start:stop]  # a view: updated in place like MomentBuffer.read
        return decode(ms.codes[start // 2:(stop + 1) // 2], ms.scales[start // BLOCK:stop // BLOCK],
                      ms.scheme, stop - start)

    def _write(self, ms: MomentState, value, start, stop, *, eden, draws, bias, eps) -> None:
        if ms.scheme == "fp32":
            return  # the read view was updated in place
        codes, scales = encode(value, ms.scheme, eden=eden, draws=draws, bias=bias, eps=eps,
                               guards=self.optimized and self._param_optimized, usr_sqrt=self.usr_sqrt)
        ms.codes[start // 2:(stop + 1) // 2] = pack(codes)
        ms.scales[start // BLOCK:stop // BLOCK] = scales
