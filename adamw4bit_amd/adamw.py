"""``QuantizedAdamW`` and its 4-bit recipes, stepped by one fused HIP launch per step.

Drop-in for the optimizer API of ``adamw4bit`` (reference ``src/adamw4bit/adamw.py``):
same constructor arguments and validation (``adamw.py:127-239``), the
ZIP-SR / ZE-EDEN recipe subclasses (``:869-892``), runtime m1 retargeting
(``:251-279``), the per-(moment, device) quantization RNG streams keyed by
``quant_rng_seed`` (``:281-324``) and the packed-code / block-scale
``state_dict`` layout with its ``_quant_rng_state`` payload (``:326-470``).

``step()`` gathers every parameter with a gradient into a launch table and
calls ``aw4_fused_step`` once per device: decode -> AdamW -> re-encode for all
tensors, fp32-state tensors included, in one kernel.  With ``optimized=True`` a
parameter follows the optimized backend's semantics (``_optimized.py:85-234``:
exact-level guards in stochastic rounding, one-tile initial draws); parameters
the backend's preflight would reject, and every parameter when
``optimized=False``, follow the reference step (``adamw.py:472-805``), which
differs only in those two points.

The reference-step m2 variants that read the stored m2 back for the current update
(``dyn4_upd_sr``, ``lin4_upd_sr``, ``*_upd_sr_store_eden``, ``adamw.py:615-656``) and
the lookahead update-SR variants (``dyn4_la_upd_sr`` and its proxies, ``adamw.py:566-614``)
run in the same launch, in kernels of their own.

Not provided (``NotImplementedError`` on construction): 8-bit state
(``linear``/``dynamic``, ``AdamW8bit``), update clipping, diagnostics recording and
telemetry callbacks.  Parameters must live on a HIP device; there is no CPU
implementation.
"""

from __future__ import annotations

import array
import bisect
import functools
import itertools
import math
import operator
import struct
from collections.abc import Mapping
from typing import Any, Dict, Iterable, Iterator, List, Optional, Tuple

import numpy as np
import torch
from torch.optim import optimizer as _torch_optimizer
from torch.optim.optimizer import Optimizer

from . import _lib, _ops
from ._rng import GlobalStream, PhiloxStream
from .quantization import (
    LOOKAHEAD_SCHEMES,
    NEXT_BIAS_SCHEMES,
    PENDING_KEY,
    PENDING_LOOKAHEAD_SCHEMES,
    VPROXY_LOOKAHEAD_SCHEMES,
    SAMPLED_READ_SCHEMES,
    STORE_EDEN_SCHEMES,
    QuantState,
    ROUND_LOOKAHEAD_SR,
    ROUND_STATE_SR,
    ROUND_UPDATE_SR,
    SCHEMES,
    default_block_size,
    initial_code_and_scale,
    pack_4bit_codes,
)

_TORCHAO_MIN_QUANT_NUMEL = 4096           # adamw.py:19
# Classes whose instances hold a quantized moment's block scales: this package's QuantState, and
# those of optimizers driven through HipOptimizedBackend (the reference's own, same fields).
_QUANT_STATE_TYPES: Tuple[type, ...] = (QuantState,)


def register_quant_state_type(cls: type) -> None:
    """Accept instances of `cls` (fields absmax, shape, dtype, blocksize, packed) as moment state."""
    global _QUANT_STATE_TYPES
    if cls not in _QUANT_STATE_TYPES:
        _QUANT_STATE_TYPES = _QUANT_STATE_TYPES + (cls,)


_CHUNK_NUMEL = 1 << 19                    # _optimized.py:33
_CHUNK_KEY = "max_chunk_numel"            # _optimized.py:34
_FALLBACK_KEY = "_optimized_full_fallback"  # _optimized.py:35
# Schemes the optimized backend accepts (_optimized.py:36-41).
_OPT_M1_SCHEMES = {"fp32", "nf4", "nf4_sr", "sdyn4", "sdyn4_sr"}
_OPT_M2_SCHEMES = {
    "fp32", "lin4", "lin4_sr", "lin4_nz", "dyn4", "dyn4_sr", "dyn4_nz",
    "lin4_upd_sr_fp32read", "dyn4_upd_sr_fp32read", "dyn4_lookahead_sr", "dyn4_upd_sr_fp32read_nextbc",
}
_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float64: _lib.F64}
_CLIP_DTYPES = (torch.float32, torch.bfloat16, torch.float16)  # gradients the fused clip and unscale read
_UNSUPPORTED_SCHEMES = {"linear": "8-bit linear state", "dynamic": "8-bit dynamic state"}
_SR_ROUNDINGS = (ROUND_STATE_SR, ROUND_UPDATE_SR, ROUND_LOOKAHEAD_SR)  # roundings that draw uniforms


def _f32(x: float) -> float:
    return float(np.float32(x))


def _rcp32(x: float) -> float:
    """Correctly rounded fp32 reciprocal of the fp32 value ``x``: the float64 quotient rounded to
    fp32 (a double rounding that cannot differ from one rounding, 53 >= 2 * 24 + 2 bits); 1/0 is
    inf with the sign of the zero."""
    if x == 0.0:
        return math.copysign(math.inf, x)
    return array.array("f", (1.0 / x,)).tolist()[0]


def _rcp32s(*values: float) -> list:
    """``_rcp32`` of each fp32 value, with one rounding call."""
    return array.array("f", [1.0 / x if x != 0.0 else math.copysign(math.inf, x) for x in values]).tolist()


def _step_fields() -> np.dtype:
    """View of a launch-table row holding only what a reused plan rewrites each step: the
    gradient address and scale pointer, the flags word with the seven fp32 step constants
    after it (``words``, 8 x 32 bits), the m2 update-SR constants (``m2_sr``, 3 x 32 bits),
    both random-stream keys and positions (a stream drawn from torch's generator takes
    that generator's current seed) and the float64 constants of float64 parameters (``f64``)."""
    T = _lib.TENSOR
    m1, m2 = T.fields["m1"][1], T.fields["m2"][1]
    M = T.fields["m2"][0]
    words = ("flags", "w1", "w2", "decay", "step_coef", "bc2_sqrt", "bc2_sqrt_rcp", "eps")
    assert [T.fields[k][1] for k in words] == [T.fields["flags"][1] + 4 * i for i in range(8)]
    assert [M.fields[k][1] for k in ("sr_bias", "sr_bias_rcp", "sr_eps")] == [M.fields["sr_bias"][1] + 4 * i
                                                                            for i in range(3)]
    assert T.fields["step_coef_f64"][1] == T.fields["decay_f64"][1] + 8
    return np.dtype({"names": ["grad", "grad_scale", "words", "m2_sr", "m1_rng_seed", "m2_rng_seed",
                               "m1_rng_offset", "m2_rng_offset", "f64"],
                     "formats": ["<u8", "<u8", ("<u4", 8), ("<u4", 3), "<u8", "<u8", "<u8", "<u8", ("<f8", 2)],
                     "offsets": [T.fields["grad"][1], T.fields["grad_scale"][1], T.fields["flags"][1],
                                 m2 + M.fields["sr_bias"][1], m1 + M.fields["rng_seed"][1],
                                 m2 + M.fields["rng_seed"][1], m1 + M.fields["rng_offset"][1],
                                 m2 + M.fields["rng_offset"][1], T.fields["decay_f64"][1]],
                     "itemsize": T.itemsize})


_STEP_FIELDS = _step_fields()
# The same per-step fields as byte offsets within a row, for small plans, which pack them in place.
_OFF_WORDS = _lib.TENSOR.fields["flags"][1]
_OFF_GRAD = _lib.TENSOR.fields["grad"][1]
_OFF_M2_SR = _lib.TENSOR.fields["m2"][1] + _lib.MOMENT.fields["sr_bias"][1]
_OFF_F64 = _lib.TENSOR.fields["decay_f64"][1]
_OFF_RNG = {m: _lib.TENSOR.fields[m][1] + _lib.MOMENT.fields["rng_seed"][1] for m in ("m1", "m2")}
assert _lib.MOMENT.fields["rng_offset"][1] == _lib.MOMENT.fields["rng_seed"][1] + 8
_PACK_WORDS = struct.Struct("<i7f").pack_into    # flags word and the seven fp32 step constants
_PACK_U64 = struct.Struct("<Q").pack_into
_PACK_M2_SR = struct.Struct("<3f").pack_into     # update-SR bias, its reciprocal, eps
_PACK_F64 = struct.Struct("<2d").pack_into       # decay_f64, step_coef_f64
_PACK_RNG = struct.Struct("<QQ").pack_into       # rng_seed, rng_offset
_STEP_WORDS = np.dtype([("flags", "<i4")] + [(k, "<f4") for k in ("w1", "w2", "decay", "step_coef", "bc2_sqrt",
                                                                   "bc2_sqrt_rcp", "eps")])


def _byte_range(t: torch.Tensor) -> Tuple[str, int, int]:
    """Storage interval of a tensor (``_moment_buffer.py:13-20``)."""
    if t.is_contiguous():
        start = t.data_ptr()
        return str(t.device), start, start + t.numel() * t.element_size()
    storage = t.untyped_storage()
    return str(t.device), storage.data_ptr(), storage.data_ptr() + storage.nbytes()


def _overlaps(a, b) -> bool:
    return a[0] == b[0] and a[1] < b[2] and b[1] < a[2]


class _RangeSet:
    """Byte ranges a launch writes in place, for the overlap test of ``_overlaps`` against all of
    them in O(log n): per device, the union of the non-empty ranges as sorted disjoint intervals
    (empty ranges, which overlap only what strictly contains their address, kept aside)."""

    __slots__ = ("_starts", "_ends", "_points")

    def __init__(self):
        self._starts: Dict[str, List[int]] = {}
        self._ends: Dict[str, List[int]] = {}
        self._points: List[Tuple[str, int, int]] = []

    def overlaps(self, r) -> bool:
        key, a, b = r
        ends = self._ends.get(key)
        if ends:
            i = bisect.bisect_right(ends, a)  # the first interval ending after a
            if i < len(ends) and self._starts[key][i] < b:
                return True
        return any(_overlaps(r, q) for q in self._points)

    def add(self, r) -> None:
        key, a, b = r
        if b <= a:
            self._points.append(r)
            return
        starts = self._starts.setdefault(key, [])
        ends = self._ends.setdefault(key, [])
        i = bisect.bisect_left(ends, a)     # the first interval ending at or after a
        j = bisect.bisect_right(starts, b)  # the first interval starting after b
        if i < j:
            a, b = min(a, starts[i]), max(b, ends[j - 1])
        starts[i:j] = [a]
        ends[i:j] = [b]


def _f32s(*values: float) -> list:
    """Each value rounded to fp32 (to nearest, as numpy's float32 conversion; out of range: inf)."""
    return array.array("f", values).tolist()


_HYPER_CACHE: Dict[tuple, tuple] = {}


def _hyper_constants(beta1, beta2, lr, wd, eps) -> tuple:
    """The step-independent constants of a group's hyperparameters: the lerp flags, fp32 lerp
    weights (w - 1 with the LARGE flag), fp32 decay 1 - lr*wd and eps, and the float64 decay.
    Cached for Python-number hyperparameters (a tensor-valued one is computed each time: its
    value may change in place)."""
    key = (beta1, beta2, lr, wd, eps)
    cacheable = all(type(v) in (float, int) for v in key)
    if cacheable:
        hit = _HYPER_CACHE.get(key)
        if hit is not None:
            return hit
    w1, w2, decay, eps32 = _f32s(1 - beta1, 1 - beta2, 1 - lr * wd, eps)
    flags = 0
    if not abs(w1) < 0.5:  # ATen lerp switches formulas at |weight| >= 0.5
        flags |= _lib.TENSOR_LERP1_LARGE
        w1 = w1 - 1.0  # exact for w1 in [0.5, 1] (and NaN stays NaN), as in fp32
    if not abs(w2) < 0.5:
        flags |= _lib.TENSOR_LERP2_LARGE
        w2 = w2 - 1.0
    out = (flags, w1, w2, decay, eps32, float(1 - lr * wd))
    if cacheable:
        if len(_HYPER_CACHE) >= 256:
            _HYPER_CACHE.clear()
        _HYPER_CACHE[key] = out
    return out


class _StepConstants:
    """The fp32 step constants of one (group, step), computed in float64 and rounded once to
    fp32 as the reference does (``_optimized.py:168-173``).  ``words`` and ``m2_sr`` are their
    bit patterns as the launch table holds them (the flags word and the seven fp32 constants;
    the m2 update-SR bias, its reciprocal and eps)."""

    __slots__ = ("lerp_flags", "w1", "w2", "decay", "step_coef", "bc2_sqrt", "bc2_sqrt_rcp", "eps", "storage_bias",
                 "decay_f64", "step_coef_f64", "_words", "_m2_sr", "_m2_vals")

    def __init__(self, group, step: int, m2_scheme: str):
        beta1, beta2 = group["betas"]
        lr, wd, eps = group["lr"], group["weight_decay"], group["eps"]
        bias1, bias2 = 1 - beta1 ** step, 1 - beta2 ** step
        self.storage_bias = 1 - beta2 ** (step + 1) if m2_scheme in NEXT_BIAS_SCHEMES else bias2
        self.lerp_flags, self.w1, self.w2, self.decay, self.eps, self.decay_f64 = _hyper_constants(
            beta1, beta2, lr, wd, eps)
        # a float64 parameter is updated with the float64 coefficient (_optimized.py:221-222)
        self.step_coef_f64 = float(-lr / bias1)
        # one fp32 rounding of the step's values, then of the two reciprocals (the update-SR bias
        # is floored at 1e-12 before its rounding, _optimized_quantization.py:66-67)
        self.step_coef, self.bc2_sqrt, sr_bias = _f32s(-lr / bias1, math.sqrt(bias2),
                                                       max(float(self.storage_bias), 1e-12))
        self.bc2_sqrt_rcp, sr_bias_rcp = _rcp32s(self.bc2_sqrt, sr_bias)
        self._m2_vals = (sr_bias, sr_bias_rcp, self.eps)
        self._words = self._m2_sr = None

    def words(self) -> np.ndarray:
        if self._words is None:
            self._words = np.frombuffer(struct.pack("<i7f", self.lerp_flags, self.w1, self.w2, self.decay,
                                                    self.step_coef, self.bc2_sqrt, self.bc2_sqrt_rcp, self.eps),
                                        dtype=np.uint32)
        return self._words

    def m2_sr_values(self) -> tuple:
        """fp32 update-SR storage bias max(c, 1e-12), its correctly rounded reciprocal, and eps."""
        return self._m2_vals

    def m2_sr(self) -> np.ndarray:
        if self._m2_sr is None:
            self._m2_sr = np.frombuffer(struct.pack("<3f", *self.m2_sr_values()), dtype=np.uint32)
        return self._m2_sr


def _step_constants(group, step: int, m2_scheme: str) -> _StepConstants:
    return _StepConstants(group, step, m2_scheme)


def _vec_aligned(p: torch.Tensor, grad: torch.Tensor) -> bool:
    """Parameter and gradient allow 4-value vector access."""
    psize = 4 * p.element_size()
    gsize = 4 * grad.element_size()
    return p.data_ptr() % psize == 0 and grad.data_ptr() % gsize == 0


def _table_tensor(table: np.ndarray) -> torch.Tensor:
    """The rows of a launch table as the CPU uint8 tensor a launch record carries; the tensor also
    keeps the rows for the eager launch (``_aw4_rows``)."""
    t = torch.from_numpy(table.view(np.uint8))
    t._aw4_rows = _lib.rows_of(table)
    return t


try:
    from torch._C import _cuda_getCurrentRawStream as _raw_stream  # torch's own (inductor's get_raw_stream)
except ImportError:  # pragma: no cover - other torch builds
    def _raw_stream(index: int) -> int:
        return torch.cuda.current_stream(index).cuda_stream


def _launch(params: List[torch.Tensor], written: List[torch.Tensor], read: List[torch.Tensor],
            table: torch.Tensor, refs: torch.Tensor, copy_back: List[Tuple[torch.Tensor, torch.Tensor]]) -> None:
    """Launch one device's step on its current stream (a launch record of ``_DeviceBatch.launch``).

    Under ``torch.compile`` the launch is the custom operator ``adamw4bit_hip::fused_step_``,
    which declares the tensors it writes and reads and takes their addresses from the tensors it
    receives (``refs``).  In eager mode the operator's dispatch (argument flattening and one
    version bump per tensor) costs about 5 us per tensor, so the library is called directly on
    the table, whose addresses are already filled in, and the version counters of everything
    written in place are bumped in one call, as the operator would; ``read`` is referenced by
    the caller until the call returns, and the kernels are ordered on the stream like any torch
    kernel.  Strided parameters were stepped as contiguous copies, copied back here."""
    if torch.compiler.is_compiling():
        _ops.fused_step_(params, written, read, table, refs)
    else:
        device = params[0].device
        if device.type != "cuda":
            raise ValueError("the fused 4-bit step runs on HIP devices only")
        rows = getattr(table, "_aw4_rows", None)
        if rows is None:
            rows = table.numpy().view(_lib.TENSOR)
        if torch.cuda.current_device() != device.index:
            with torch.cuda.device(device):
                _lib.fused_step(rows, _raw_stream(device.index))
        else:
            _lib.fused_step(rows, _raw_stream(device.index))
        torch.autograd.graph.increment_version(params + written)
    for p, staged in copy_back:
        p.copy_(staged)


def _lean_step(func):
    """``Optimizer.step`` wrapper with torch's behaviour and less fixed cost.

    torch wraps every optimizer's ``step`` (``Optimizer.profile_hook_step``) in a profiler range
    ``Optimizer.step#<class>.step`` around the step pre-hooks, the step and the post-hooks; the
    range alone costs about 15 us per call, a third of the host time of a one-tensor step.  This
    wrapper runs torch's own wrapper whenever a profiler is running or a step hook is registered
    (globally or on the optimizer), and otherwise calls the step and ``_optimizer_step_code``
    directly.  ``hooked`` tells ``Optimizer._patch_step_function`` not to wrap it again."""
    torch_wrapped = Optimizer.profile_hook_step(func)

    @functools.wraps(func)
    def step(self, *args, **kwargs):
        if (torch.autograd._profiler_enabled() or self._optimizer_step_pre_hooks
                or self._optimizer_step_post_hooks or _torch_optimizer._global_optimizer_pre_hooks
                or _torch_optimizer._global_optimizer_post_hooks):
            return torch_wrapped(self, *args, **kwargs)
        out = func(self, *args, **kwargs)
        self._optimizer_step_code()
        return out

    step.hooked = True
    return step


def _moment_tensors(state: Dict[str, Any]) -> List[torch.Tensor]:
    """Writable moment buffers of one parameter (``_moment_buffer.py:22-41``)."""
    out = []
    for key in ("m1", "m2"):
        for name in (key, f"{key}_code"):
            value = state.get(name)
            if isinstance(value, torch.Tensor) and value.layout == torch.strided and value.numel():
                out.append(value)
        meta = state.get(f"{key}_quant_state")
        if (isinstance(meta, _QUANT_STATE_TYPES) and isinstance(meta.absmax, torch.Tensor)
                and meta.absmax.layout == torch.strided and meta.absmax.numel()):
            out.append(meta.absmax)
    return out


class QuantizedAdamW(Optimizer):
    r"""AdamW with 4-bit or fp32 moment storage, stepped on the GPU by one fused kernel.

    Arguments, defaults and validation follow ``adamw4bit.QuantizedAdamW``
    (reference ``adamw.py:46-239``).  ``optimized`` selects the optimized
    backend's stochastic-rounding guards and initial-draw accounting; both
    settings run the same fused kernel.
    """

    _VALID_SCHEMES = (
        "linear", "dynamic",
        "sdyn4", "sdyn4_sr", "nf4", "nf4_sr",
        "lin4", "lin4_sr", "lin4_upd_sr", "lin4_upd_sr_store_eden", "lin4_upd_sr_fp32read", "lin4_nz",
        "dyn4", "dyn4_sr", "dyn4_upd_sr", "dyn4_upd_sr_store_eden", "dyn4_upd_sr_fp32read",
        "dyn4_lookahead_sr", "dyn4_upd_sr_fp32read_nextbc", "dyn4_la_upd_sr", "dyn4_proxy_la_upd_sr",
        "dyn4_vproxy_la_upd_sr", "dyn4_nz",
        "fp32",
    )
    _UPDATE_SR_STORE_EDEN_SCHEMES = {"lin4_upd_sr_store_eden", "dyn4_upd_sr_store_eden"}
    _ORACLE_LOOKAHEAD_UPDATE_SR_SCHEMES = {"dyn4_la_upd_sr"}
    _PROXY_LOOKAHEAD_UPDATE_SR_SCHEMES = {"dyn4_proxy_la_upd_sr"}
    _VPROXY_LOOKAHEAD_UPDATE_SR_SCHEMES = {"dyn4_vproxy_la_upd_sr"}
    _QUANT_RNG_STATE_KEY = "_quant_rng_state"
    _QUANT_RNG_OFFSETS = {"m1": 0x1A2B3C4D, "m2": 0x5E6F7789}  # adamw.py:122-125
    _quant_state_type: type = QuantState  # the class new quantized moment state is created as

    def __init__(self,
                 params: Iterator[torch.nn.Parameter],
                 lr: float = 1e-3,
                 betas: Tuple[float, float] = (0.9, 0.95),
                 eps: float = 1e-8,
                 weight_decay: float = 1e-1,
                 block_size: Optional[int] = None,
                 quant_scheme: str = "linear",
                 use_eden_m2: bool = False,
                 m1_quant_scheme: Optional[str] = None,
                 m2_quant_scheme: Optional[str] = None,
                 quant_rng_seed: Optional[int] = None,
                 telemetry=None,
                 update_sign_clip: Optional[float] = None,
                 update_norm_clip: Optional[float] = None,
                 record_update_direction_every: Optional[int] = None,
                 record_preconditioner_every: Optional[int] = None,
                 record_preconditioner_steps=None,
                 optimized: bool = False):
        # Validation, messages and order as adamw.py:148-208.
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if quant_rng_seed is not None and (
            isinstance(quant_rng_seed, bool) or not isinstance(quant_rng_seed, int) or quant_rng_seed < 0
        ):
            raise ValueError(f"quant_rng_seed must be a non-negative integer or None, got {quant_rng_seed!r}")
        if update_sign_clip is not None and not update_sign_clip > 0.0:
            raise ValueError(f"update_sign_clip must be positive or None, got {update_sign_clip}")
        if update_norm_clip is not None and not update_norm_clip > 0.0:
            raise ValueError(f"update_norm_clip must be positive or None, got {update_norm_clip}")
        if update_sign_clip is not None and update_norm_clip is not None:
            raise ValueError("Set at most one of update_sign_clip / update_norm_clip "
                             "(they are alternative update-clip mechanisms).")
        if record_update_direction_every is not None and record_update_direction_every <= 0:
            raise ValueError("record_update_direction_every must be positive or None, "
                             f"got {record_update_direction_every}")
        if record_preconditioner_every is not None and record_preconditioner_every <= 0:
            raise ValueError("record_preconditioner_every must be positive or None, "
                             f"got {record_preconditioner_every}")
        if record_preconditioner_steps is not None:
            record_preconditioner_steps = tuple(sorted(set(int(s) for s in record_preconditioner_steps)))
            if any(s <= 0 for s in record_preconditioner_steps):
                raise ValueError("record_preconditioner_steps must contain positive optimizer steps")

        m1_scheme = m1_quant_scheme or quant_scheme
        m2_scheme = m2_quant_scheme or quant_scheme
        for name, s in (("quant_scheme", quant_scheme), ("m1_quant_scheme", m1_scheme),
                        ("m2_quant_scheme", m2_scheme)):
            if s not in self._VALID_SCHEMES:
                raise ValueError(f"{name} must be one of {self._VALID_SCHEMES}, got {s!r}")
        if use_eden_m2 and m2_scheme in {"lin4_sr", "dyn4_sr"}:
            raise ValueError("Vanilla stochastic-rounding m2 schemes should not be combined with use_eden_m2")
        if use_eden_m2 and m2_scheme in self._UPDATE_SR_STORE_EDEN_SCHEMES:
            raise ValueError("Do not set use_eden_m2 with *_upd_sr_store_eden; EDEN is built into the store path")
        if m2_scheme in (self._ORACLE_LOOKAHEAD_UPDATE_SR_SCHEMES | self._PROXY_LOOKAHEAD_UPDATE_SR_SCHEMES
                         | self._VPROXY_LOOKAHEAD_UPDATE_SR_SCHEMES):
            if m1_scheme not in {"fp32", "nf4"}:
                raise ValueError("lookahead update-SR currently supports m1_quant_scheme='fp32' or 'nf4'")
            if use_eden_m2:
                raise ValueError("lookahead update-SR should not be combined with use_eden_m2")
            if update_sign_clip is not None or update_norm_clip is not None:
                raise ValueError("lookahead update-SR should not be combined with update clipping")

        # The parts of the reference API outside the fused 4-bit path.
        for name, s in (("m1_quant_scheme", m1_scheme), ("m2_quant_scheme", m2_scheme)):
            if s in _UNSUPPORTED_SCHEMES:
                raise NotImplementedError(
                    f"{name}={s!r} ({_UNSUPPORTED_SCHEMES[s]}) is not part of the fused 4-bit HIP step")
        for name, value in (("telemetry", telemetry), ("update_sign_clip", update_sign_clip),
                            ("update_norm_clip", update_norm_clip),
                            ("record_update_direction_every", record_update_direction_every),
                            ("record_preconditioner_every", record_preconditioner_every),
                            ("record_preconditioner_steps", record_preconditioner_steps)):
            if value is not None:
                raise NotImplementedError(f"{name} is not part of the fused 4-bit HIP step")
        if block_size is not None and block_size != _lib.BLOCK:
            raise NotImplementedError(f"block_size={block_size}: the fused step encodes {_lib.BLOCK}-value blocks")

        self.telemetry = telemetry
        self._m1_quant_scheme_overrides: Dict[int, str] = {}
        self._quant_rng_seed = quant_rng_seed
        self._quant_generators: Dict[str, Dict[str, PhiloxStream]] = {"m1": {}, "m2": {}}
        self._pending_quant_rng_states: Dict[str, Dict[str, torch.Tensor]] = {"m1": {}, "m2": {}}
        self._global_streams: Dict[str, Dict[str, GlobalStream]] = {"m1": {}, "m2": {}}
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                        block_size=block_size, quant_scheme=quant_scheme, use_eden_m2=use_eden_m2,
                        m1_quant_scheme=m1_scheme, m2_quant_scheme=m2_scheme,
                        update_sign_clip=update_sign_clip, update_norm_clip=update_norm_clip,
                        record_update_direction_every=record_update_direction_every,
                        record_preconditioner_every=record_preconditioner_every,
                        record_preconditioner_steps=record_preconditioner_steps)
        super().__init__(params, defaults)
        self._optimized = optimized
        # Test hook: callable(param, moment, numel, device) -> fp32 uniforms used instead of the
        # on-device Philox draws of a stochastic write (bit-exact comparisons with fed draws).
        self._draw_provider = None
        self._launch_plan: Optional[_LaunchPlan] = None
        self._pending_finish = None  # commit / undo of the step being launched
        self._inconsistent: Optional[str] = None  # why step() refuses to run (a partly enqueued step)
        # Gradient clipping computed by clip_grad_norm_ and applied by the next step:
        # (device, the float pair {inverse loss scale, clip coefficient} on that device, the row
        # flags that apply them) or None.
        self._grad_clip: Optional[Tuple[torch.device, torch.Tensor, int]] = None
        if optimized:
            for group in self.param_groups:
                group.setdefault(_CHUNK_KEY, _CHUNK_NUMEL)
            self.register_load_state_dict_post_hook(self._after_load)

    # ------------------------------------------------------------------
    # Scheme resolution (adamw.py:241-279, 807-817)
    # ------------------------------------------------------------------
    def _m1_scheme_for(self, parameter: torch.Tensor, group_scheme: str) -> str:
        return self._m1_quant_scheme_overrides.get(id(parameter), group_scheme)

    def set_m1_quant_scheme_for_parameters(self, parameters: Iterable[torch.nn.Parameter], scheme: str) -> None:
        """Retarget future m1 writes for existing optimizer parameters."""
        if scheme not in {"nf4", "nf4_sr"}:
            raise ValueError("runtime m1 retargeting supports only nf4 and nf4_sr")
        optimizer_parameter_ids = {id(p) for group in self.param_groups for p in group["params"]}
        selected = list(parameters)
        if not selected:
            raise ValueError("runtime m1 retargeting requires parameters")
        if any(id(p) not in optimizer_parameter_ids for p in selected):
            raise ValueError("runtime m1 retargeting received parameters outside optimizer")
        for p in selected:
            self._m1_quant_scheme_overrides[id(p)] = scheme
        self._launch_plan = None

    @staticmethod
    def _eligible_for_quantized_state(p: torch.Tensor, block_size: int) -> bool:
        n = p.numel()
        return n >= _TORCHAO_MIN_QUANT_NUMEL and n % block_size == 0

    @classmethod
    def _effective_scheme(cls, p: torch.Tensor, scheme: str, block_size: int) -> str:
        if scheme == "fp32" or cls._eligible_for_quantized_state(p, block_size):
            return scheme
        return "fp32"

    # ------------------------------------------------------------------
    # Quantization RNG streams (adamw.py:281-324)
    # ------------------------------------------------------------------
    def _quant_generator(self, moment: str, device: torch.device) -> Optional[PhiloxStream]:
        if self._quant_rng_seed is None:
            return None
        if moment not in self._QUANT_RNG_OFFSETS:
            raise ValueError(f"Unsupported quantization RNG stream: {moment!r}")
        device_key = str(device)
        generators = self._quant_generators[moment]
        if device_key in generators:
            return generators[device_key]
        stream = PhiloxStream((self._quant_rng_seed + self._QUANT_RNG_OFFSETS[moment]) % ((1 << 63) - 1))
        pending = self._pending_quant_rng_states[moment]
        state = pending.pop(device_key, None)
        if state is None:
            compatible = [k for k in pending if k.split(":", maxsplit=1)[0] == device.type]
            if len(compatible) == 1:
                state = pending.pop(compatible[0])
            elif pending:
                raise ValueError(f"Unable to restore quantization RNG state for {moment} on {device}; "
                                 f"saved devices={sorted(pending)}")
        if state is not None:
            stream.set_state(state)
        generators[device_key] = stream
        return stream

    def _stream(self, moment: str, device: torch.device):
        """The stream a stochastic write of ``moment`` draws from on ``device``."""
        stream = self._quant_generator(moment, device)
        if stream is not None:
            return stream
        # quant_rng_seed=None: the reference draws from torch's default generator of the device;
        # so does this stream, write by write (GlobalStream).
        key = str(device)
        streams = self._global_streams[moment]
        if key not in streams:
            if device.type != "cuda":
                raise NotImplementedError("the fused 4-bit step runs on HIP devices only")
            torch.cuda.init()  # fills torch.cuda.default_generators
            generator = torch.cuda.default_generators[device.index if device.index is not None
                                                      else torch.cuda.current_device()]
            # the moment's constant (adamw.py:122-125) spread over 64 bits
            streams[key] = GlobalStream(generator, (self._QUANT_RNG_OFFSETS[moment] * 0x9E3779B97F4A7C15))
        return streams[key]

    def _all_streams(self) -> list:
        """Every random stream this optimizer has opened."""
        return [s for table in (self._quant_generators, self._global_streams) for streams in table.values()
                for s in streams.values()]

    # ------------------------------------------------------------------
    # Checkpoints (adamw.py:326-470, _optimized.py:53-83)
    # ------------------------------------------------------------------
    def state_dict(self):
        result = super().state_dict()
        result["state"] = {
            index: {key: vars(value).copy() if isinstance(value, _QUANT_STATE_TYPES) else value
                    for key, value in parameter_state.items()}
            for index, parameter_state in result["state"].items()
        }
        if self._quant_rng_seed is None:
            return result
        states = {moment: {device: state.detach().cpu().clone()
                           for device, state in self._pending_quant_rng_states[moment].items()}
                  for moment in self._QUANT_RNG_OFFSETS}
        for moment, generators in self._quant_generators.items():
            states[moment].update({device: g.get_state() for device, g in generators.items()})
        result[self._QUANT_RNG_STATE_KEY] = {"version": 1, "seed": self._quant_rng_seed, "states": states}
        return result

    def load_state_dict(self, state_dict):
        """Restore fp32 moments and integer codes on each parameter's device."""
        rng_payload = state_dict.get(self._QUANT_RNG_STATE_KEY)
        optimizer_state = {k: v for k, v in state_dict.items() if k != self._QUANT_RNG_STATE_KEY}

        def capture_state(_optimizer, loaded_state):
            nonlocal optimizer_state
            optimizer_state = loaded_state

        def restore_moments(_optimizer):
            for group, saved_group in zip(self.param_groups, optimizer_state["param_groups"]):
                for parameter, saved_index in zip(group["params"], saved_group["params"]):
                    original = optimizer_state["state"].get(saved_index, {})
                    if not original:
                        continue
                    state = self.state[parameter]
                    for key in ("m1", "m2", "lookahead_pending_exp_avg_sq", "m2_read_preconditioner"):
                        if key in original:
                            state[key] = original[key].to(device=parameter.device, dtype=torch.float32)
                    for key in ("m1_quant_state", "m2_quant_state"):
                        if key in original:
                            value = original[key]
                            fields = dict(value) if isinstance(value, Mapping) else vars(value).copy()
                            fields["absmax"] = fields["absmax"].to(device=parameter.device, dtype=torch.float32)
                            state[key] = QuantState(**fields)
                    schemes = {"m1": self._m1_scheme_for(parameter, group["m1_quant_scheme"]),
                               "m2": group["m2_quant_scheme"]}
                    for key, scheme in schemes.items():
                        code_key = f"{key}_code"
                        if code_key in original:
                            code_dtype = torch.int8 if scheme == "linear" else torch.uint8
                            state[code_key] = original[code_key].to(device=parameter.device, dtype=code_dtype)

        capture_hook = self.register_load_state_dict_pre_hook(capture_state)
        restore_hook = self.register_load_state_dict_post_hook(restore_moments, prepend=True)
        try:
            result = super().load_state_dict(optimizer_state)
        finally:
            capture_hook.remove()
            restore_hook.remove()
        self._quant_generators = {"m1": {}, "m2": {}}
        self._pending_quant_rng_states = {"m1": {}, "m2": {}}
        self._launch_plan = None
        self._inconsistent = None  # the loaded state replaces whatever a failed step left
        if rng_payload is not None:
            if not isinstance(rng_payload, Mapping):
                raise ValueError("Invalid quantization RNG checkpoint payload")
            if rng_payload.get("version") != 1:
                raise ValueError(f"Unsupported quantization RNG checkpoint version: {rng_payload.get('version')!r}")
            if self._quant_rng_seed is None:
                raise ValueError("Checkpoint contains separated quantization RNG state, but quant_rng_seed is disabled")
            saved_seed = rng_payload.get("seed")
            if saved_seed != self._quant_rng_seed:
                raise ValueError(f"Quantization RNG seed mismatch: checkpoint={saved_seed!r}, "
                                 f"configured={self._quant_rng_seed!r}")
            saved_states = rng_payload.get("states")
            if not isinstance(saved_states, Mapping):
                raise ValueError("Quantization RNG checkpoint states are missing")
            for moment in self._QUANT_RNG_OFFSETS:
                moment_states = saved_states.get(moment, {})
                if not isinstance(moment_states, Mapping):
                    raise ValueError(f"Invalid quantization RNG states for {moment}")
                for device, state in moment_states.items():
                    if not isinstance(device, str) or not torch.is_tensor(state):
                        raise ValueError(f"Invalid quantization RNG state entry for {moment}")
                    self._pending_quant_rng_states[moment][device] = state.detach().cpu().clone()
        return result

    @staticmethod
    def _after_load(optimizer: "QuantizedAdamW") -> None:
        """Mark parameters whose loaded moment storage aliases another's (``_optimized.py:53-83``)."""
        intervals = []
        for group in optimizer.param_groups:
            group.setdefault(_CHUNK_KEY, _CHUNK_NUMEL)
            for parameter in group["params"]:
                for tensor in _moment_tensors(optimizer.state.get(parameter, {})):
                    intervals.append((*_byte_range(tensor), id(parameter)))
        intervals.sort()
        aliased, owners = set(), set()
        device, end, count = "", 0, 0
        for current_device, start, stop, owner in intervals:
            if current_device != device or start >= end:
                if count > 1:
                    aliased.update(owners)
                device, end, count, owners = current_device, stop, 1, {owner}
            else:
                end = max(end, stop)
                count += 1
                owners.add(owner)
        if count > 1:
            aliased.update(owners)
        for group in optimizer.param_groups:
            for parameter in group["params"]:
                if id(parameter) in aliased:
                    optimizer.state[parameter][_FALLBACK_KEY] = True

    # ------------------------------------------------------------------
    # Gradient clipping fused into the step
    # ------------------------------------------------------------------
    @torch.no_grad()
    def clip_grad_norm_(self, max_norm: float, norm_type: float = 2.0, error_if_nonfinite: bool = False,
                        foreach: Optional[bool] = None, *, grad_scaler=None) -> torch.Tensor:
        """``torch.nn.utils.clip_grad_norm_`` over this optimizer's parameters, fused into the next
        ``step()``.

        The reference's training examples clip before every step (an HF Trainer with
        ``max_grad_norm=1.0``, ``examples/train_gpt_small.py:214``).  Here one pass over the
        gradients computes the total norm and the coefficient ``min(max_norm / (norm + 1e-6), 1)``
        on the device with torch's dtype rounding points (``aw4_clip_coefficient``), and the next
        ``step()`` reads every gradient value as ``grad_dtype(g * coef)`` -- what torch's in-place
        ``_foreach_mul_`` would have stored -- instead of scaling the gradients in memory.  The
        gradients themselves are left unscaled.  Returns the total norm (a 0-dim tensor on the
        parameters' device, in the promoted gradient dtype), like torch.  Only the 2-norm of
        parameters on one HIP device; one pending clip per step (``zero_grad()`` drops a pending
        clip whose step was skipped).

        With ``grad_scaler`` (an enabled ``torch.amp.GradScaler`` whose scaled loss produced the
        gradients), this is ``grad_scaler.unscale_(self)`` followed by the clip, in the same single
        read of the gradients (``aw4_unscale_clip_coefficient``): each value is unscaled as torch's
        ``_amp_foreach_non_finite_check_and_unscale_`` would leave it, the norm is that of the
        unscaled gradients, and the scaler records this optimizer's ``found_inf`` (any scaled value
        not finite) and its stage as unscaled, so ``grad_scaler.step(self)`` skips an overflowed
        step as usual.  The gradients in memory stay scaled; the next ``step()`` reads them
        unscaled and clipped.
        """
        if float(norm_type) != 2.0:
            raise NotImplementedError("the fused clip computes the 2-norm only")
        return self._fused_prologue(float(max_norm), grad_scaler, error_if_nonfinite, clip=True)

    @torch.no_grad()
    def unscale_grads_(self, grad_scaler) -> None:
        """``grad_scaler.unscale_(self)`` fused into the next ``step()``: one read of the gradients
        checks them for non-finite values (the scaler's ``found_inf`` for this optimizer, as
        ``_amp_foreach_non_finite_check_and_unscale_`` computes it, and its stage set to unscaled),
        and ``step()`` reads every gradient value as ``grad_dtype(g * inv_scale)`` instead of torch
        writing the unscaled gradients back.  Call it where ``grad_scaler.unscale_(optimizer)``
        would be called (or let ``grad_scaler.step`` call torch's own)."""
        self._fused_prologue(math.inf, grad_scaler, False, clip=False)

    def _scaler_begin(self, grad_scaler):
        """The scaler's per-optimizer state for a fused unscale (GradScaler.unscale_'s checks), or
        None without an enabled scaler."""
        if grad_scaler is None or not grad_scaler.is_enabled():
            return None
        from torch.amp.grad_scaler import OptState

        grad_scaler._check_scale_growth_tracker("unscale_")
        state = grad_scaler._per_optimizer_states[id(self)]
        if state["stage"] is OptState.UNSCALED:
            raise RuntimeError("unscale_() has already been called on this optimizer since the last update().")
        if state["stage"] is OptState.STEPPED:
            raise RuntimeError("unscale_() is being called after step().")
        return state

    def _fused_prologue(self, max_norm: float, grad_scaler, error_if_nonfinite: bool, clip: bool):
        scaler_state = self._scaler_begin(grad_scaler)
        prepared = self._prepare_clip()
        if prepared is None:
            if scaler_state is not None:
                from torch.amp.grad_scaler import OptState

                scaler_state["found_inf_per_device"] = {}
                scaler_state["stage"] = OptState.UNSCALED
            return torch.tensor(0.0)
        grads, table, out, result_dtype = prepared
        flags = _lib.TENSOR_GRAD_SCALE if clip else 0
        if scaler_state is not None and any(g.dtype == torch.float16 for g in grads):
            self._grad_clip = None
            raise ValueError("Attempting to unscale FP16 gradients.")  # GradScaler.unscale_ (allow_fp16=False)
        if scaler_state is not None:
            # torch carries out the reciprocal of the scale in float64 (GradScaler.unscale_)
            out[2:3].copy_(grad_scaler._scale.double().reciprocal().float().reshape(1).to(out.device))
            flags |= _lib.TENSOR_GRAD_UNSCALE
            if torch.compiler.is_compiling():
                _ops.unscale_clip_coefficient_(grads, out, table, max_norm)
            else:
                with torch.cuda.device(out.device):
                    p = out.data_ptr()
                    _lib.unscale_clip_coefficient(table.numpy().view(_lib.TENSOR), p + 8, max_norm, p, p + 12, p + 4,
                                                  torch.cuda.current_stream(out.device).cuda_stream)
        elif torch.compiler.is_compiling():
            _ops.clip_coefficient_(grads, out, table, max_norm)
        else:  # the operator's dispatch over every gradient costs more than the call (see _launch)
            with torch.cuda.device(out.device):
                p = out.data_ptr()
                _lib.clip_coefficient(table.numpy().view(_lib.TENSOR), max_norm, p, p + 12,
                                      torch.cuda.current_stream(out.device).cuda_stream)
        total = out[0].to(result_dtype)
        if error_if_nonfinite and bool(torch.logical_or(total.isnan(), total.isinf())):
            raise RuntimeError(
                f"The total norm of order 2.0 for gradients from `parameters` is non-finite, so it "
                "cannot be clipped. To disable this error and scale the gradients by the non-finite norm anyway, "
                "set `error_if_nonfinite=False`")
        if scaler_state is not None:
            from torch.amp.grad_scaler import OptState

            scaler_state["found_inf_per_device"] = {out.device: out[1]}
            scaler_state["stage"] = OptState.UNSCALED
        self._set_grad_clip(out, flags)
        return total

    @torch.compiler.disable
    def _prepare_clip(self):
        """Gradients, launch table (as a CPU uint8 tensor) and the output pair of a clip, or None
        without gradients."""
        if self._grad_clip is not None:
            raise RuntimeError("a gradient clip is already pending: call step() before clipping again")
        params = [p for group in self.param_groups for p in group["params"] if p.grad is not None]
        if not params:
            return None
        devices = {p.device for p in params}
        device = params[0].device
        if len(devices) != 1 or device.type != "cuda":
            raise NotImplementedError("the fused clip runs over gradients on one HIP device")
        grads = []
        for p in params:
            g = p.grad
            if g.layout != torch.strided or g.dtype not in _CLIP_DTYPES:
                raise NotImplementedError("the fused clip reads dense float32/bfloat16/float16 gradients")
            grads.append(g if g.is_contiguous() else g.contiguous())
        table = np.zeros(len(grads), dtype=_lib.TENSOR)
        table["grad"] = [g.data_ptr() for g in grads]
        table["numel"] = [g.numel() for g in grads]
        table["grad_dtype"] = [_DTYPES[g.dtype] for g in grads]
        table["flags"] = [_lib.TENSOR_VEC_ALIGNED if g.data_ptr() % (4 * g.element_size()) == 0 else 0 for g in grads]
        # [total norm, found_inf, then the pair the step reads: inverse loss scale, clip coefficient]
        out = torch.empty(4, dtype=torch.float32, device=device)
        result_dtype = grads[0].dtype
        for g in grads[1:]:
            if g.dtype != result_dtype:
                result_dtype = torch.float32  # torch.stack promotes the per-tensor norms
        return grads, torch.from_numpy(table.view(np.uint8)), out, result_dtype

    @torch.compiler.disable
    def _set_grad_clip(self, out: torch.Tensor, flags: int) -> None:
        self._grad_clip = (out.device, out[2:4], flags)

    def zero_grad(self, set_to_none: bool = True) -> None:
        """``Optimizer.zero_grad``; also drops a pending gradient clip, whose gradients are gone
        (a step skipped after the clip, as a GradScaler skips one on overflow, leaves it)."""
        self._grad_clip = None
        super().zero_grad(set_to_none=set_to_none)

    def _take_grad_clip(self, device: torch.device) -> Optional[Tuple[torch.Tensor, int]]:
        """The pending (unscale, clip) pair on `device` and its row flags, or None."""
        clip = self._grad_clip
        if clip is None or clip[0] != device:
            return None
        return clip[1], clip[2]

    # ------------------------------------------------------------------
    # The step
    # ------------------------------------------------------------------
    @_lean_step
    def step(self, closure=None):  # type: ignore[override]
        """One fused launch per device over every parameter with a gradient (``adamw.py:472-502``).

        The host work -- validation, state initialisation, the launch tables -- runs eagerly, also
        under ``torch.compile`` (``_prepare_launches`` is compiler-disabled); the launch itself is
        the custom operator ``adamw4bit_hip::fused_step_`` when compiled and a direct library call
        otherwise.  A step changes nothing unless it launches: every parameter is checked before
        any state changes, and a failed launch restores step counts, moment state and random
        stream positions.  Like the reference's, the step runs under ``torch.no_grad()``, except
        an eager step without closure that reuses the last step's launch tables: it runs no torch
        operation (a library call and version-counter bumps), so it skips the grad-mode switch."""
        if self._inconsistent is not None:
            raise RuntimeError(self._inconsistent)
        plan = self._launch_plan
        if closure is None and plan is not None and not torch.compiler.is_compiling():
            prepared = plan.prepare(self, records=False)
            if prepared is not None:
                self._pending_finish = prepared[1]
                done = 0
                incomplete = False
                try:
                    for dev in plan.devices:
                        try:
                            dev.launch_eager()
                        except _lib.HipLaunchIncomplete:
                            incomplete = True
                            raise
                        done += 1
                finally:
                    self._finish_launches(done, len(plan.devices), incomplete)
                return None
            self._launch_plan = None  # stale: the full path rebuilds it
        return self._step_full(closure)

    @torch.no_grad()
    def _step_full(self, closure):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        launches = self._prepare_launches()
        done = 0
        incomplete = False
        try:
            for launch in launches:
                try:
                    _launch(*launch)
                except _lib.HipLaunchIncomplete:
                    incomplete = True
                    raise
                done += 1
        finally:
            self._finish_step(done, len(launches), incomplete)
        return loss

    @torch.compiler.disable
    def _finish_step(self, done: int, total: int, incomplete: bool = False) -> None:
        self._finish_launches(done, total, incomplete)

    def _finish_launches(self, done: int, total: int, incomplete: bool = False) -> None:
        """Commit the prepared step after its launches (``done == total``), or undo it if no step
        kernel was enqueued.  A step that failed after enqueuing some of its kernels (a launch that
        failed part way, or one device's launch after another's) cannot be undone: the tensors may
        be partly updated, so the optimizer refuses further steps until a checkpoint is loaded."""
        finish, self._pending_finish = self._pending_finish, None
        if finish is None:
            return
        if done == total or (done == 0 and not incomplete):
            finish(done, total)
            return
        self._launch_plan = None
        self._inconsistent = (
            f"a step failed after {'some of its kernels' if incomplete else f'{done} of its {total} launches'} "
            "were enqueued: parameters and moment state may be partly updated; load a checkpoint with "
            "load_state_dict() before stepping again")

    @torch.compiler.disable
    def _prepare_launches(self):
        """Launch records of this step (see ``_launch``); leaves the step's commit / undo in
        ``_pending_finish`` for ``_finish_step``."""
        self._pending_finish = None
        plan = self._launch_plan
        if plan is not None:
            prepared = plan.prepare(self)
            if prepared is not None:
                launches, self._pending_finish = prepared
                return launches
        self._launch_plan = None
        checked = [self._preflight(p, group) for group in self.param_groups for p in group["params"]
                   if p.grad is not None]
        undo = _StepUndo(self, [c.state for c in checked])
        batches: Dict[torch.device, _DeviceBatch] = {}
        try:
            for c in checked:
                batch = batches.get(c.param.device)
                if batch is None:
                    batch = batches[c.param.device] = _DeviceBatch()
                self._prepare(c, batch)
            launches = [batch.launch(self._take_grad_clip(device)) for device, batch in batches.items()]
        except BaseException:
            undo.restore()
            raise

        def finish(done: int, total: int) -> None:
            if done == total:
                self._grad_clip = None
                self._launch_plan = _LaunchPlan.build(self, list(batches.values()), checked)
            elif done == 0:
                undo.restore()

        self._pending_finish = finish
        return launches

    def _moment_compatible(self, state, key: str, scheme: str, size: int, p: torch.Tensor) -> bool:
        """The optimized backend's check of existing moment state (``_moment_buffer.py:54-87``)."""
        if "step" not in state:
            return True
        if scheme == "fp32":
            value = state.get(key)
            return (isinstance(value, torch.Tensor) and value.layout == torch.strided and value.is_contiguous()
                    and value.shape == p.shape and value.device == p.device and value.dtype == torch.float32)
        codes = state.get(f"{key}_code")
        meta = state.get(f"{key}_quant_state")
        if not isinstance(codes, torch.Tensor) or not isinstance(meta, _QUANT_STATE_TYPES):
            return False
        n = p.numel()
        absmax = meta.absmax
        if not (codes.layout == torch.strided and codes.is_contiguous() and codes.dtype == torch.uint8
                and codes.device == p.device and meta.shape == p.shape and meta.blocksize == size
                and meta.dtype == torch.float32 and isinstance(absmax, torch.Tensor) and absmax.ndim == 1
                and absmax.numel() == n // size and absmax.is_contiguous() and absmax.dtype == torch.float32
                and absmax.device == p.device):
            return False
        if getattr(meta, "packed", False):
            return codes.numel() == (n + 1) // 2
        return codes.numel() in {n, (n + 1) // 2}

    def _plan_accepts(self, p: torch.Tensor, grad: torch.Tensor, group, requested, sizes, schemes, state) -> bool:
        """Whether the optimized backend's preflight takes this parameter (``_optimized.py:85-136``):
        otherwise it follows the reference step."""
        if not self._optimized or state.get(_FALLBACK_KEY, False):
            return False
        if requested[0] not in _OPT_M1_SCHEMES or requested[1] not in _OPT_M2_SCHEMES:
            return False
        if not p.is_contiguous() or not grad.is_contiguous():
            return False
        if "step" in state and not isinstance(state["step"], int):
            return False
        if not all(self._moment_compatible(state, key, scheme, size, p)
                   for key, scheme, size in zip(("m1", "m2"), schemes, sizes)):
            return False
        occupied = [_byte_range(p), _byte_range(grad)]
        if _overlaps(occupied[0], occupied[1]):
            return False
        for tensor in _moment_tensors(state):
            region = _byte_range(tensor)
            if any(_overlaps(region, prev) for prev in occupied):
                return False
            occupied.append(region)
        limit = group.get(_CHUNK_KEY, _CHUNK_NUMEL)
        if isinstance(limit, bool) or not isinstance(limit, int) or limit <= 0:
            return False
        return limit >= (_lib.BLOCK if any(s != "fp32" for s in schemes) else 1)

    def _chunk_numel(self, group, schemes) -> int:
        limit = group.get(_CHUNK_KEY, _CHUNK_NUMEL)
        align = _lib.BLOCK if any(s != "fp32" for s in schemes) else 1
        return limit // align * align

    def _preflight(self, p: torch.Tensor, group) -> "_Checked":
        """Everything that can reject this parameter, checked without changing its state."""
        if not p.is_cuda:
            raise NotImplementedError("the fused 4-bit step runs on HIP devices only; move the parameters to the GPU")
        if p.dtype not in _DTYPES:
            raise NotImplementedError(f"parameter dtype {p.dtype} (supported: float32, bfloat16, float16, float64)")
        if p.layout != torch.strided:
            raise NotImplementedError("the fused step updates dense (strided) parameters in place")
        grad = p.grad
        if grad.layout != torch.strided or grad.dtype not in _DTYPES or grad.device != p.device:
            raise NotImplementedError("gradients must be dense float32/bfloat16/float16/float64 tensors on the "
                                      "parameter's device")
        if grad.shape != p.shape:
            raise ValueError(f"gradient shape {tuple(grad.shape)} does not match parameter shape {tuple(p.shape)}")
        state = self.state[p]
        requested = (self._m1_scheme_for(p, group["m1_quant_scheme"]), group["m2_quant_scheme"])
        sizes = tuple(group["block_size"] if group["block_size"] is not None else default_block_size(m)
                      for m in requested)
        schemes = tuple(self._effective_scheme(p, m, s) for m, s in zip(requested, sizes))
        optimized = self._plan_accepts(p, grad, group, requested, sizes, schemes, state)
        if "step" in state:
            for moment, scheme in zip(("m1", "m2"), schemes):
                self._check_moment(p, state, moment, scheme)
        # Streams are opened (and checkpointed streams restored) before any state changes, so a
        # restore failure leaves every parameter untouched (_optimized.py:157-158).
        for moment in ("m1", "m2"):
            self._stream(moment, p.device)
        return _Checked(p, group, grad, state, schemes, sizes, optimized)

    def _prepare(self, c: "_Checked", batch: "_DeviceBatch") -> None:
        """State initialisation, step count and the launch-table row of one checked parameter."""
        p, group, grad, state, schemes, sizes, optimized = (c.param, c.group, c.grad, c.state, c.schemes, c.sizes,
                                                             c.optimized)
        if optimized:
            group.setdefault(_CHUNK_KEY, _CHUNK_NUMEL)
        else:
            # The reference step writes fresh tensors: detach state and gradients that alias the
            # parameter, each other, or what an earlier row of this launch writes in place (state
            # shared between parameters after a checkpoint load, _optimized.py:53-83).
            occupied = [_byte_range(p)]
            if _overlaps(occupied[0], _byte_range(grad)):
                grad = grad.clone()
            occupied.append(_byte_range(grad))

            def taken(r) -> bool:
                return batch.occupied.overlaps(r) or any(_overlaps(r, q) for q in occupied)

            for key in ("m1", "m2", "m1_code", "m2_code", PENDING_KEY):
                value = state.get(key)
                if isinstance(value, torch.Tensor):
                    if taken(_byte_range(value)):
                        state[key] = value = value.clone()
                    occupied.append(_byte_range(value))
            for key in ("m1_quant_state", "m2_quant_state"):
                meta = state.get(key)
                if isinstance(meta, _QUANT_STATE_TYPES) and isinstance(meta.absmax, torch.Tensor):
                    if taken(_byte_range(meta.absmax)):
                        meta.absmax = meta.absmax.clone()
                    occupied.append(_byte_range(meta.absmax))
        if not grad.is_contiguous():
            grad = grad.contiguous()
        target = p
        if not p.is_contiguous():
            # The reference step updates a strided parameter element by element in logical order;
            # the kernel updates a contiguous copy in that order, which is copied back after it.
            target = p.detach().contiguous()
            batch.copy_back.append((p, target))
        c.staged = target is not p

        n = p.numel()
        if "step" not in state:
            chunk = self._chunk_numel(group, schemes) if optimized else n
            for moment, scheme, size, eden in (("m1", schemes[0], sizes[0], False),
                                               ("m2", schemes[1], sizes[1], group["use_eden_m2"])):
                self._init_moment(p, state, moment, scheme, size, eden, chunk)
            state["step"] = 0
        else:
            for moment, scheme in zip(("m1", "m2"), schemes):
                self._normalize_moment(p, state, moment, scheme)
        state["step"] = int(state["step"]) + 1
        step = state["step"]

        c_ = _step_constants(group, step, schemes[1])
        flags = c_.lerp_flags
        if _vec_aligned(target, grad):
            flags |= _lib.TENSOR_VEC_ALIGNED
        refs = {_COL["param"]: batch.ref("p", target), _COL["grad"]: batch.ref("r", grad)}
        m1 = self._moment_row(p, state, "m1", schemes[0], False, optimized, 1.0, 1e-8, batch, refs)
        m2 = self._moment_row(p, state, "m2", schemes[1], group["use_eden_m2"], optimized,
                              c_.storage_bias, group["eps"], batch, refs)
        if schemes[1] in LOOKAHEAD_SCHEMES:
            # adamw.py:566-614: the pending form samples the fp32 state with bias_c2 before the
            # update; the proxies encode the new m2 for the next step's bias correction.
            beta2 = float(group["betas"][1])
            bias = 1 - beta2 ** step if schemes[1] in PENDING_LOOKAHEAD_SCHEMES else 1 - beta2 ** (step + 1)
            m2_flags = m2[8] | (_lib.MOMENT_FRESH_PROXY if schemes[1] in VPROXY_LOOKAHEAD_SCHEMES else 0)
            m2 = m2[:8] + (m2_flags,) + m2[9:12] + (beta2, 1.0 - beta2, max(float(bias), 1e-12), float(group["eps"]))
            state.pop("m2_read_preconditioner", None)
        elif schemes[1] in STORE_EDEN_SCHEMES:
            # Reads with the scale before EDEN; stores the calibrated scale and 1/denominator.
            pre = state.get("m2_read_preconditioner")
            if not (isinstance(pre, torch.Tensor) and pre.shape == p.shape and pre.dtype == torch.float32
                    and pre.device == p.device and pre.is_contiguous() and pre.data_ptr() % 16 == 0):
                pre = state["m2_read_preconditioner"] = torch.empty(p.shape, dtype=torch.float32, device=p.device)
            refs[_COL["m2.values"]] = batch.ref("w", pre)
            m2 = m2[:8] + (m2[8] | _lib.MOMENT_SAMPLED_READ | _lib.MOMENT_READ_RAW_SCALE | _lib.MOMENT_EDEN,) + m2[9:]
        else:
            state.pop("m2_read_preconditioner", None)  # adamw.py:568-686, _optimized.py:156
            if schemes[1] in SAMPLED_READ_SCHEMES:
                m2 = m2[:8] + (m2[8] | _lib.MOMENT_SAMPLED_READ,) + m2[9:]
        batch.rows.append((0, 0, 0, n, _DTYPES[p.dtype], _DTYPES[grad.dtype], flags, c_.w1, c_.w2, c_.decay,
                           c_.step_coef, c_.bc2_sqrt, c_.bc2_sqrt_rcp, c_.eps, m1, m2, c_.decay_f64,
                           c_.step_coef_f64))
        batch.refs.append(refs)
        pre = state.get("m2_read_preconditioner")
        for t in [target] + _moment_tensors(state) + ([pre] if isinstance(pre, torch.Tensor) else []):
            batch.occupied.add(_byte_range(t))

    def _init_moment(self, p, state, moment, scheme, size, eden, chunk) -> None:
        """Zero state (``_moment_buffer.py:89-126`` / ``adamw.py:524-545``)."""
        n = p.numel()
        if scheme == "fp32":
            state[moment] = torch.zeros(p.shape, device=p.device, dtype=torch.float32)
            state.pop(f"{moment}_code", None)
            state.pop(f"{moment}_quant_state", None)
            return
        if scheme in PENDING_LOOKAHEAD_SCHEMES:  # adamw.py:534-535
            state[PENDING_KEY] = torch.zeros(p.shape, device=p.device, dtype=torch.float32)
            return
        code, scale = initial_code_and_scale(scheme, eden)
        state[f"{moment}_code"] = torch.full(((n + 1) // 2,), code | (code << 4), dtype=torch.uint8, device=p.device)
        absmax = torch.full((n // size,), scale, dtype=torch.float32, device=p.device)
        state[f"{moment}_quant_state"] = self._quant_state_type(absmax=absmax, shape=p.shape, dtype=torch.float32,
                                                    blocksize=size, packed=True)
        state.pop(moment, None)
        if SCHEMES[scheme][1] in (ROUND_STATE_SR, ROUND_UPDATE_SR):
            # Encoding the zero tile consumes draws without affecting the codes.
            tile = n if n <= chunk else math.lcm(size, 2)
            self._stream(moment, p.device).advance(tile)

    def _check_moment(self, p, state, moment, scheme) -> None:
        """Reject existing state the kernel cannot step (``_moment_buffer.py:54-87,127-141``); changes
        nothing (``_normalize_moment`` then brings accepted state into the kernel's layout)."""
        n = p.numel()
        if scheme == "fp32" or scheme in PENDING_LOOKAHEAD_SCHEMES:
            key = moment if scheme == "fp32" else PENDING_KEY
            value = state.get(key)
            if value is None and f"{moment}_code" in state:
                raise NotImplementedError(f"{moment}: quantized state found where the scheme keeps fp32 state")
            if not (isinstance(value, torch.Tensor) and value.device == p.device and value.dtype == torch.float32
                    and value.numel() == n):
                raise ValueError(f"{key}: fp32 state does not match the parameter")
            return
        codes = state.get(f"{moment}_code")
        meta = state.get(f"{moment}_quant_state")
        if not isinstance(codes, torch.Tensor) or not isinstance(meta, _QUANT_STATE_TYPES):
            raise NotImplementedError(f"{moment}: fp32 state found where the scheme is quantized")
        if not isinstance(meta.absmax, torch.Tensor):
            raise ValueError(f"{moment}: quantization scales must be a tensor")
        if meta.blocksize != _lib.BLOCK or meta.absmax.numel() != n // _lib.BLOCK:
            raise NotImplementedError(f"{moment}: block size {meta.blocksize} state")
        if codes.dtype != torch.uint8 or codes.device != p.device:
            raise ValueError(f"{moment}: codes must be uint8 on {p.device}")
        legacy = codes.numel() == n and not getattr(meta, "packed", False)
        if not legacy and codes.numel() != (n + 1) // 2:
            raise ValueError(f"{moment}: {codes.numel()} code bytes for {n} values")

    def _normalize_moment(self, p, state, moment, scheme) -> None:
        """Bring state that ``_check_moment`` accepted into the kernel's layout: contiguous, on the
        parameter's device, packed codes (legacy unpacked codes are repacked), codes 8-byte and
        fp32 values 16-byte aligned (the kernel's vector accesses)."""
        if scheme == "fp32" or scheme in PENDING_LOOKAHEAD_SCHEMES:
            key = moment if scheme == "fp32" else PENDING_KEY
            value = state[key]
            if not value.is_contiguous() or value.data_ptr() % 16:
                state[key] = value.contiguous() if not value.is_contiguous() else value.clone()
            return
        codes = state[f"{moment}_code"]
        meta = state[f"{moment}_quant_state"]
        n = p.numel()
        if meta.absmax.device != p.device or meta.absmax.dtype != torch.float32 or not meta.absmax.is_contiguous():
            meta.absmax = meta.absmax.to(device=p.device, dtype=torch.float32).contiguous()
        if codes.numel() == n and not getattr(meta, "packed", False):
            codes = pack_4bit_codes(codes.reshape(-1))  # legacy unpacked codes
        if not codes.is_contiguous():
            codes = codes.contiguous()
        if codes.data_ptr() % 8:
            codes = codes.clone()
        state[f"{moment}_code"] = codes
        meta.packed = True

    def _moment_row(self, p, state, moment, scheme, eden, optimized, bias, eps, batch, refs) -> Tuple:
        """The ``aw4_moment`` fields of one moment (addresses 0: ``refs`` names their tensors)."""
        n = p.numel()
        if scheme == "fp32":
            refs[_COL[f"{moment}.values"]] = batch.ref("w", state[moment])
            return (0, 0, 0, 0, 0, 0, 0, _lib.ROUND_FP32, 0, 1.0, 1.0, _f32(1e-8), 0.0, 0.0, 0.0, 0.0)
        codebook, rounding, floor_zero = SCHEMES[scheme]
        flags = (_lib.MOMENT_ZERO_FLOOR if floor_zero else 0) | (_lib.MOMENT_EDEN if eden else 0)
        if optimized:
            flags |= _lib.MOMENT_GUARDS
        seed = offset = 0
        if rounding in _SR_ROUNDINGS:
            stream = self._stream(moment, p.device)
            seed, offset = stream.seed, stream.take(n)
            if self._draw_provider is not None:
                # lookahead update-SR draws float64 uniforms (quantization.py:873-878)
                dtype = torch.float64 if rounding == ROUND_LOOKAHEAD_SR else torch.float32
                u = self._draw_provider(p, moment, n, p.device)
                if u.dtype != dtype or u.numel() != n or u.device != p.device:
                    raise ValueError(f"draw provider must return n {dtype} uniforms on the parameter's device")
                u = u.contiguous()
                if u.data_ptr() % 16:
                    u = u.clone()
                refs[_COL[f"{moment}.draws"]] = batch.ref("r", u)
                flags |= _lib.MOMENT_EXT_DRAWS
        sr_bias = _f32(max(float(bias), 1e-12))
        if scheme in PENDING_LOOKAHEAD_SCHEMES:
            refs[_COL[f"{moment}.values"]] = batch.ref("w", state[PENDING_KEY])
            return (0, 0, 0, 0, seed, offset, codebook, rounding, flags | _lib.MOMENT_PENDING, sr_bias,
                    _rcp32(sr_bias), _f32(eps), 0.0, 0.0, 0.0, 0.0)
        refs[_COL[f"{moment}.codes"]] = batch.ref("w", state[f"{moment}_code"])
        refs[_COL[f"{moment}.scales"]] = batch.ref("w", state[f"{moment}_quant_state"].absmax)
        return (0, 0, 0, 0, seed, offset, codebook, rounding, flags, sr_bias, _rcp32(sr_bias), _f32(eps),
                0.0, 0.0, 0.0, 0.0)


# Column of each address field in a launch record's ``refs`` (adamw4bit_amd._ops.ADDRESS_FIELDS).
_COL = {".".join(path): k for k, path in enumerate(_ops.ADDRESS_FIELDS)}


class _Checked:
    """A parameter that passed ``_preflight``: what its step will do."""

    __slots__ = ("param", "group", "grad", "state", "schemes", "sizes", "optimized", "staged")

    def __init__(self, param, group, grad, state, schemes, sizes, optimized):
        self.param, self.group, self.grad, self.state = param, group, grad, state
        self.schemes, self.sizes, self.optimized = schemes, sizes, optimized
        self.staged = False


class _DeviceBatch:
    """The rows of one device's launch and the tensors their addresses point into."""

    __slots__ = ("rows", "refs", "params", "written", "read", "copy_back", "occupied")

    def __init__(self):
        self.occupied = _RangeSet()  # byte ranges the rows so far write in place
        self.rows: List[Tuple] = []
        self.refs: List[Dict[int, Tuple[str, int]]] = []  # per row: column -> (list, index)
        self.params: List[torch.Tensor] = []   # updated in place
        self.written: List[torch.Tensor] = []  # moment state, updated in place
        self.read: List[torch.Tensor] = []     # gradients, clip coefficient, caller draws
        self.copy_back: List[Tuple[torch.Tensor, torch.Tensor]] = []  # (strided parameter, its staged copy)

    def ref(self, kind: str, tensor: torch.Tensor) -> Tuple[str, int]:
        target = self.params if kind == "p" else self.written if kind == "w" else self.read
        target.append(tensor)
        return kind, len(target) - 1

    def launch(self, clip: Optional[Tuple[torch.Tensor, int]]) -> Tuple:
        """The launch record: (params, written, read, table, refs, copy_back), the table a CPU uint8
        tensor of rows with every address filled in, refs its (rows, fields) int64 references.
        `clip`: the pending (unscale, clip) pair and its row flags."""
        table = np.array(self.rows, dtype=_lib.TENSOR)
        if clip is not None:
            pair, flags = clip
            k = self.ref("r", pair)
            for r in self.refs:
                r[_COL["grad_scale"]] = k
            table["flags"] |= flags
        base = {"p": 0, "w": len(self.params), "r": len(self.params) + len(self.written)}
        refs = np.full((len(self.rows), len(_ops.ADDRESS_FIELDS)), -1, dtype=np.int64)
        for i, row in enumerate(self.refs):
            for col, (kind, index) in row.items():
                refs[i, col] = base[kind] + index
        _ops.resolve_addresses(table, refs, self.params + self.written + self.read)
        return (self.params, self.written, self.read, _table_tensor(table), torch.from_numpy(refs), self.copy_back)


class _StepUndo:
    """What preparing a step changes before it launches: the state entries of its parameters
    (and the scales and packing flag of their QuantStates), and every random stream's position."""

    def __init__(self, opt: "QuantizedAdamW", states: List[Dict[str, Any]]):
        self.states = [(st, dict(st), [(q, q.absmax, q.packed) for q in st.values()
                                       if isinstance(q, _QUANT_STATE_TYPES)])
                       for st in states]
        self.streams = [(s, s.offset) for s in opt._all_streams()]

    def restore(self) -> None:
        for st, saved, quants in self.states:
            st.clear()
            st.update(saved)
            for q, absmax, packed in quants:
                q.absmax, q.packed = absmax, packed
        for s, offset in self.streams:
            s.offset = offset


# Plans of at most this many rows per device check and refresh their rows in Python loops,
# larger ones with numpy (whose fixed cost per operation is about a microsecond).
_SMALL_PLAN = 16
_REPEAT_STEP, _REPEAT_INT = itertools.repeat("step"), itertools.repeat(int)


class _PlanDevice:
    """One device's part of a launch plan: its table (rows with every address filled in) and
    the views and per-row facts its per-step refresh needs."""

    __slots__ = ("table", "params", "written", "entries", "states", "device", "small", "lo", "hi", "ranges",
                 "gbytes", "gbytes_list", "pvec", "pvec_list", "gvec", "gvec_list", "fields", "words",
                 "m2_sr", "seed_cols", "offset_cols", "grad_col", "qrows", "qsel", "qrows_any", "la_rows", "la_next",
                 "f64", "f64_rows", "refs", "table_t", "refs_t", "scale_ptr", "scale_ref", "buf", "row_plans",
                 "rows", "index", "bump", "gchecked")

    def __init__(self, table: np.ndarray, params, written, entries, lo, hi, ranges, refs: np.ndarray):
        n = len(params)
        self.table = table
        self.params = list(params)
        self.written = list(written)
        self.entries = entries
        self.states = [e[0] for e in entries]
        self.device = params[0].device
        self.small = n <= _SMALL_PLAN
        self.lo, self.hi = lo, hi
        self.ranges = ranges  # per row: the (start, end) byte ranges a gradient may not overlap
        self.gbytes_list = [p.numel() * p.element_size() for p in params]
        self.gbytes = np.array(self.gbytes_list, dtype=np.int64)
        self.pvec_list = [p.data_ptr() % (4 * p.element_size()) == 0 for p in params]
        self.pvec = np.array(self.pvec_list, dtype=bool)
        self.gvec_list = [4 * p.element_size() for p in params]
        self.gvec = np.array(self.gvec_list, dtype=np.int64)
        # views into the table
        self.fields = table.view(_STEP_FIELDS)
        self.words = self.fields["words"]
        self.m2_sr = self.fields["m2_sr"]
        self.seed_cols = {"m1": self.fields["m1_rng_seed"], "m2": self.fields["m2_rng_seed"]}
        self.offset_cols = {"m1": self.fields["m1_rng_offset"], "m2": self.fields["m2_rng_offset"]}
        self.grad_col = self.fields["grad"]
        self.qrows = np.flatnonzero(table["m2"]["rounding"] != _lib.ROUND_FP32)
        self.qrows_any = len(self.qrows) > 0
        self.qsel = slice(None) if len(self.qrows) == n else self.qrows
        # lookahead m2 rows: their float64 beta2, 1 - beta2, bias correction and eps are per
        # step too (the pending form's bias is bias_c2 of the step, the proxies' that of the next)
        self.la_rows = np.flatnonzero(table["m2"]["rounding"] == _lib.ROUND_LOOKAHEAD_SR)
        self.la_next = (table["m2"]["flags"][self.la_rows] & _lib.MOMENT_PENDING) == 0
        # float64 parameters: their float64 decay and step coefficient are per step too
        self.f64 = self.fields["f64"]
        self.f64_rows = np.flatnonzero(table["param_dtype"] == _lib.F64)
        self.refs = refs
        self.table_t = _table_tensor(table)
        self.rows = self.table_t._aw4_rows
        self.refs_t = torch.from_numpy(refs)
        self.scale_ptr = self.scale_ref = None  # what the grad_scale fields hold (unknown: rewrite)
        self.index = self.device.index
        self.bump = self.params + self.written  # what an eager launch writes in place
        self.gchecked = None  # the gradient addresses whose overlap check last passed
        # small plans write each row's per-step fields in place (struct.pack_into at the row's
        # offsets): per row whether m2 takes the update-SR constants, is float64, is lookahead
        self.buf = memoryview(table.view(np.uint8)).cast("B")
        rounding, pdtype = table["m2"]["rounding"], table["param_dtype"]
        self.row_plans = [(i * _lib.TENSOR.itemsize, bool(rounding[i] != _lib.ROUND_FP32),
                           bool(pdtype[i] == _lib.F64)) for i in range(n)] if self.small else None

    def launch_eager(self) -> None:
        """The eager launch of a refreshed plan (as ``_launch`` for its record)."""
        index = self.index
        if torch.cuda.current_device() != index:
            with torch.cuda.device(index):
                _lib.fused_step(self.rows, _raw_stream(index))
        else:
            _lib.fused_step(self.rows, _raw_stream(index))
        torch.autograd.graph.increment_version(self.bump)


class _LaunchPlan:
    """Launch tables of the last full step, reused by the next steps while only per-step values
    change: gradient addresses, step counts, the fp32 step constants (one per group and step,
    computed by the same code as the full path), random-stream keys and positions, the update-SR
    storage bias and the lookahead constants.  Any structural change -- other parameters with gradients, a parameter whose
    storage, dtype, size or layout changed (``p.data = ...``, ``module.to(dtype)``), new state
    objects, other schemes or chunking in a group, an m1 retarget, a checkpoint load, a draw
    provider, a gradient that is not contiguous or overlaps its parameter or state -- sends the
    step through the full path, which rebuilds the plan.  (A gradient always has its parameter's
    dtype, shape and device: the ``.grad`` setter enforces it.)
    """

    _STRUCTURE_KEYS = ("m1_quant_scheme", "m2_quant_scheme", "use_eden_m2", "block_size", _CHUNK_KEY)
    _STATE_KEYS = ("m1", "m2", "m1_code", "m2_code", "m1_quant_state", "m2_quant_state", "m2_read_preconditioner",
                   PENDING_KEY)
    _MAX_RANGES = 6  # a parameter and its writable moment tensors

    def __init__(self):
        self.groups: list = []     # (group, structure, parameter count)
        self.streams: list = []    # the random streams the planned rows draw from
        self.params: List[torch.Tensor] = []
        self.pdtypes: list = []    # each parameter's dtype, numel and data address at build time
        self.pnumel: list = []
        self.pptr: list = []
        self.one_small = False
        self.devices: list = []    # per device: see build
        # what the tables were built from, checked by identity each step, as parallel lists:
        # (params, their state dicts), (state dict, key, value) for every state key,
        # (QuantState, its absmax tensor)
        self.owners: Tuple[list, list] = ([], [])
        self.state_refs: Tuple[list, list, list] = ([], [], [])
        self.quant_refs: Tuple[list, list] = ([], [])

    @classmethod
    def build(cls, opt: "QuantizedAdamW", batches: List[_DeviceBatch], checked: List[_Checked]):
        if opt._draw_provider is not None or any(c.staged for c in checked):
            return None  # caller draws and staged copies are per step
        plan = cls()
        meta = {id(c.param): c.schemes for c in checked}
        group_of = {}
        for gi, group in enumerate(opt.param_groups):
            plan.groups.append((group, tuple(group.get(k) for k in cls._STRUCTURE_KEYS), len(group["params"])))
            for p in group["params"]:
                group_of[id(p)] = gi
        for batch in batches:
            params = batch.params
            n = len(params)
            lo = np.zeros((n, cls._MAX_RANGES), dtype=np.int64)
            hi = np.zeros((n, cls._MAX_RANGES), dtype=np.int64)
            row_ranges = []
            entries = []
            for i, p in enumerate(params):
                state = opt.state[p]
                schemes = meta[id(p)]
                pre = state.get("m2_read_preconditioner")
                extra = [pre] if isinstance(pre, torch.Tensor) else []
                ranges = [_byte_range(t)[1:] for t in [p] + _moment_tensors(state) + extra]
                if len(ranges) > cls._MAX_RANGES:
                    return None
                # The full path decided this parameter's semantics with this gradient; the plan
                # repeats that decision only for contiguous gradients that overlap nothing.
                g = p.grad
                g0 = g.data_ptr()
                g1 = g0 + g.numel() * g.element_size()
                if not g.is_contiguous() or any(a < g1 and g0 < b for a, b in ranges):
                    return None
                for k, (a, b) in enumerate(ranges):
                    lo[i, k], hi[i, k] = a, b
                row_ranges.append(ranges)
                sr = tuple((moment, opt._stream(moment, p.device))
                           for moment, scheme in (("m1", schemes[0]), ("m2", schemes[1]))
                           if scheme != "fp32" and SCHEMES[scheme][1] in _SR_ROUNDINGS)
                entries.append((state, group_of[id(p)], schemes[1], sr, p.numel()))
                plan.owners[0].append(p)
                plan.owners[1].append(state)
                for k in cls._STATE_KEYS + (_FALLBACK_KEY,):
                    plan.state_refs[0].append(state)
                    plan.state_refs[1].append(k)
                    plan.state_refs[2].append(state.get(k))
                for q in (state.get("m1_quant_state"), state.get("m2_quant_state")):
                    if isinstance(q, _QUANT_STATE_TYPES):
                        plan.quant_refs[0].append(q)
                        plan.quant_refs[1].append(q.absmax)
            table = np.array(batch.rows, dtype=_lib.TENSOR)
            refs = np.full((n, len(_ops.ADDRESS_FIELDS)), -1, dtype=np.int64)
            # the plan's read list is [p.grad for p in params] (+ the clip coefficient)
            n_p, n_w = n, len(batch.written)
            base = {"p": 0, "w": n_p, "r": n_p + n_w}
            for i, row in enumerate(batch.refs):
                for col, (kind, index) in row.items():
                    if col == _COL["grad_scale"]:
                        continue  # set per step
                    if kind == "r":
                        if col != _COL["grad"]:
                            return None  # caller draws: never planned (draw provider)
                        refs[i, col] = base["r"] + i
                    else:
                        refs[i, col] = base[kind] + index
            _ops.resolve_addresses(table, refs, list(params) + list(batch.written) + [p.grad for p in params])
            plan.devices.append(_PlanDevice(table, params, batch.written, entries, lo, hi, row_ranges, refs))
            for _, _, _, sr, _ in entries:
                for _, stream in sr:
                    if not any(stream is s for s in plan.streams):
                        plan.streams.append(stream)
            plan.params.extend(params)
            plan.pdtypes.extend(p.dtype for p in params)
            plan.pnumel.extend(p.numel() for p in params)
            plan.pptr.extend(p.data_ptr() for p in params)
        plan.one_small = len(plan.devices) == 1 and plan.devices[0].small
        return plan

    def _valid(self, opt: "QuantizedAdamW"):
        """Per-device gradient addresses if the plan still describes this step, else None."""
        if opt._draw_provider is not None or len(self.groups) != len(opt.param_groups):
            return None
        params = self.params
        dtypes = self.pdtypes
        one = self.one_small  # one device with few rows: its storage checks join the first loop
        numels, pptrs, gptrs = self.pnumel, self.pptr, []
        i = 0
        n = len(params)
        strided = torch.strided
        for (group, structure, count), current in zip(self.groups, opt.param_groups):
            if current is not group or len(group["params"]) != count:
                return None
            if tuple(map(group.get, self._STRUCTURE_KEYS)) != structure:
                return None
            for p in group["params"]:
                g = p.grad
                if g is None:
                    continue
                if (i >= n or p is not params[i] or p.dtype is not dtypes[i] or g.layout is not strided
                        or not g.is_contiguous() or not p.is_contiguous()):
                    return None
                if one:
                    # the parameter's size and storage are still what the tables hold (p.data
                    # can be swapped without changing the Parameter object)
                    if p.numel() != numels[i] or p.data_ptr() != pptrs[i]:
                        return None
                    gptrs.append(g.data_ptr())
                i += 1
        if i != n:
            return None
        if not one and (list(map(torch.Tensor.numel, params)) != numels
                        or list(map(torch.Tensor.data_ptr, params)) != pptrs):
            return None
        # identity checks in C-level loops (map/all): about 1,300 of them for 148 parameters
        state_map = opt.state
        owners, states = self.owners
        if not all(map(operator.is_, map(state_map.get, owners), states)):
            return None
        if not all(map(operator.is_, map(type, map(dict.get, states, _REPEAT_STEP)), _REPEAT_INT)):
            return None
        ref_states, ref_keys, ref_values = self.state_refs
        if not all(map(operator.is_, map(dict.get, ref_states, ref_keys), ref_values)):
            return None
        quant, absmax = self.quant_refs
        if not all(map(operator.is_, map(operator.attrgetter("absmax"), quant), absmax)):
            return None
        out = []
        for dev in self.devices:
            g0 = gptrs if one else [p.grad.data_ptr() for p in dev.params]
            if dev.small:
                # a gradient may not overlap its row's tensors (the plan's ranges); a gradient at
                # the address checked last step passes again
                if g0 != dev.gchecked:
                    for g, nbytes, ranges in zip(g0, dev.gbytes_list, dev.ranges):
                        g1 = g + nbytes
                        for a, b in ranges:
                            if a < g1 and g < b:
                                return None
                    dev.gchecked = g0
            else:
                g0 = np.array(g0, dtype=np.int64)
                g1 = g0 + dev.gbytes
                if bool(((dev.lo < g1[:, None]) & (g0[:, None] < dev.hi)).any()):
                    return None
            out.append(g0)
        return out

    def prepare(self, opt: "QuantizedAdamW", records: bool = True):
        """Launch records and ``finish`` of the step from the cached tables (as
        ``QuantizedAdamW._prepare_launches``), or None (nothing changed) if the plan is stale.
        Without ``records`` the launches are the devices' ``launch_eager`` (the list is None)."""
        grads = self._valid(opt)
        if grads is None:
            return None
        saved_steps = [(state, state["step"]) for dev in self.devices for state in dev.states]
        saved_streams = [(s, s.offset) for s in self.streams]
        # one _StepConstants per (group, step, m2 scheme): the update-SR storage bias depends on
        # the tensor's m2 scheme (an fp32-state tensor of a group has the fp32 scheme)
        constants: Dict[Tuple[int, int, str], int] = {}
        consts: List[_StepConstants] = []
        launches = []

        def constants_of(gi: int, step: int, m2_scheme: str) -> int:
            k = constants.get((gi, step, m2_scheme))
            if k is None:
                k = constants[(gi, step, m2_scheme)] = len(consts)
                consts.append(_StepConstants(self.groups[gi][0], step, m2_scheme))
            return k

        for dev, g0 in zip(self.devices, grads):
            entries = dev.entries
            clip = opt._take_grad_clip(dev.device)
            coef, extra = clip if clip is not None else (None, 0)
            if dev.small:
                # each row's per-step fields packed in place at its offsets
                buf = dev.buf
                for (state, gi, m2_scheme, sr, numel), (off, q2, f64), g, pvec, gvec in zip(
                        entries, dev.row_plans, g0, dev.pvec_list, dev.gvec_list):
                    step = state["step"] + 1
                    state["step"] = step
                    c = consts[constants_of(gi, step, m2_scheme)]
                    flags = c.lerp_flags | extra | (_lib.TENSOR_VEC_ALIGNED if pvec and g % gvec == 0 else 0)
                    _PACK_WORDS(buf, off + _OFF_WORDS, flags, c.w1, c.w2, c.decay, c.step_coef, c.bc2_sqrt,
                                c.bc2_sqrt_rcp, c.eps)
                    _PACK_U64(buf, off + _OFF_GRAD, g)
                    if q2:
                        _PACK_M2_SR(buf, off + _OFF_M2_SR, *c.m2_sr_values())
                    if f64:
                        _PACK_F64(buf, off + _OFF_F64, c.decay_f64, c.step_coef_f64)
                    for moment, stream in sr:
                        _PACK_RNG(buf, off + _OFF_RNG[moment], stream.seed, stream.take(numel))
                ks = None
            else:
                ks = []  # constants index of each row
                seeds, offsets = dev.seed_cols, dev.offset_cols
                for i, (state, gi, m2_scheme, sr, numel) in enumerate(entries):
                    step = state["step"] + 1
                    state["step"] = step
                    ks.append(constants_of(gi, step, m2_scheme))
                    for moment, stream in sr:
                        seeds[moment][i] = stream.seed
                        offsets[moment][i] = stream.take(numel)
                # the flags word and the seven fp32 step constants (bit patterns), and the m2
                # update-SR constants of the rows whose m2 is quantized
                one = ks.count(ks[0]) == len(ks)
                if one:
                    dev.words[:] = consts[ks[0]].words()
                else:
                    index = np.array(ks, dtype=np.intp)
                    dev.words[:] = np.stack([c.words() for c in consts])[index]
                dev.words[:, 0] |= (np.where(dev.pvec & (g0 % dev.gvec == 0), _lib.TENSOR_VEC_ALIGNED, 0)
                                    | extra).astype(np.uint32)
                if dev.qrows_any:
                    if one:
                        dev.m2_sr[dev.qsel] = consts[ks[0]].m2_sr()
                    else:
                        dev.m2_sr[dev.qrows] = np.stack([c.m2_sr() for c in consts])[index[dev.qrows]]
                if len(dev.f64_rows):
                    dev.f64[dev.f64_rows] = [(consts[ks[i]].decay_f64, consts[ks[i]].step_coef_f64)
                                             for i in dev.f64_rows.tolist()]
                dev.grad_col[:] = g0
            if len(dev.la_rows):
                # the lookahead fields, by the full path's arithmetic (Python floats)
                la = []
                for i, nxt in zip(dev.la_rows.tolist(), dev.la_next.tolist()):
                    state, gi = entries[i][0], entries[i][1]
                    group = self.groups[gi][0]
                    beta2 = float(group["betas"][1])
                    la.append((beta2, 1.0 - beta2, max(float(1 - beta2 ** (state["step"] + int(nxt))), 1e-12),
                               float(group["eps"])))
                m2 = dev.table["m2"]
                for k, name in enumerate(("la_beta2", "la_fresh_weight", "la_bias", "la_eps")):
                    m2[name][dev.la_rows] = [v[k] for v in la]
            params, written = dev.params, dev.written
            scale_ref = -1
            if coef is not None:
                scale_ref = len(params) + len(written) + len(params)
            scale_ptr = 0 if coef is None else coef.data_ptr()
            if scale_ptr != dev.scale_ptr:
                dev.fields["grad_scale"] = scale_ptr
                dev.scale_ptr = scale_ptr
            if scale_ref != dev.scale_ref:
                dev.refs[:, _COL["grad_scale"]] = scale_ref
                dev.scale_ref = scale_ref
            if records:
                read = [p.grad for p in params]
                if coef is not None:
                    read.append(coef)
                launches.append((params, written, read, dev.table_t, dev.refs_t, []))

        def finish(done: int, total: int) -> None:
            if done == total:
                opt._grad_clip = None
            elif done == 0:
                for state, step in saved_steps:
                    state["step"] = step
                for s, offset in saved_streams:
                    s.offset = offset

        return (launches if records else None), finish


class AdamW8bit(QuantizedAdamW):
    """Compatibility name of the reference's 8-bit defaults (``adamw.py:865-866``); 8-bit state is
    outside the fused 4-bit step, so construction raises ``NotImplementedError``."""


class ZIPSRAdamW4Bit(QuantizedAdamW):
    """NF4 first moments and zero-inclusive Dyn4 preconditioner-space SR (``adamw.py:869-879``)."""

    def __init__(self, params, **kwargs):
        super().__init__(params, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_upd_sr_fp32read",
                         use_eden_m2=False, **kwargs)


class ZEEDENAdamW4Bit(QuantizedAdamW):
    """NF4 first moments and zero-exclusive Dyn4 second moments with EDEN (``adamw.py:882-892``)."""

    def __init__(self, params, **kwargs):
        super().__init__(params, m1_quant_scheme="nf4", m2_quant_scheme="dyn4_nz", use_eden_m2=True, **kwargs)
