"""``HipOptimizedBackend``: the fused HIP step behind the reference optimizer's own plug-in point.

The reference's ``QuantizedAdamW(..., optimized=True)`` builds an ``OptimizedBackend``
(``adamw.py:235-239``, ``_optimized.py:45-51``) and, in ``step()``, offers it every parameter with
a gradient through ``try_step_parameter(optimizer, parameter, group) -> bool``
(``adamw.py:497-502``): ``True`` means the parameter and its state were updated in place (and its
step count incremented); ``False`` means nothing changed and no randomness was consumed, and the
reference then runs its own step for that parameter (``_optimized.py:128-143``).

This class keeps that contract with this package's launch preparation and HIP kernels:

* the reference's preflight decides the same way (``_plan``, ``_optimized.py:85-126``: schemes,
  contiguity, compatible state, overlaps, chunk size, the aliased-state mark of a checkpoint
  load), so a ``False`` here is a ``False`` there;
* state lives in the reference optimizer's ``state`` as the reference lays it out, with the
  reference's own ``QuantState`` objects, so its ``state_dict`` / ``load_state_dict`` are unchanged;
* the stochastic rounding draws come from the reference's per-moment generators
  (``_quant_generator``, ``adamw.py:281-305``; torch's default generator of the device when
  ``quant_rng_seed`` is None): each write keys Philox4x32-10 with the generator's seed and takes
  its positions from, and advances, the generator's offset, so the reference's checkpoint of its
  generators resumes the stream exactly.  The draws equal those of this package's own
  ``QuantizedAdamW`` with the same seed;
* parameters the kernels do not take (on the CPU, of a dtype other than float32, bfloat16, float16
  and float64, with a gradient of another dtype) go to the reference's own ``OptimizedBackend``,
  whose answer is returned.

Each accepted parameter is launched at once (``deferred=False``), or, with ``deferred=True``, the
accepted parameters of a step are prepared one by one and launched together by ``flush(optimizer)``
-- one launch per device, which a maintainer calls after the parameter loop of ``step()``.  A
parameter offered again while its previous step is still pending flushes first.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from . import _lib
from ._rng import GlobalStream
from .adamw import (_CHUNK_KEY, _CHUNK_NUMEL, _DTYPES, QuantizedAdamW, _DeviceBatch, _launch, _StepUndo,
                    register_quant_state_type)
from .quantization import default_block_size

# Group settings under which the reference's backend declines every parameter (_optimized.py:131-135).
_DECLINING_GROUP_KEYS = ("update_sign_clip", "update_norm_clip", "record_update_direction_every",
                         "record_preconditioner_every", "record_preconditioner_steps")


class _Engine(QuantizedAdamW):
    """This package's launch preparation bound to another optimizer's state, parameter groups, m1
    scheme overrides and random generators (it is never stepped itself)."""

    def __init__(self, target, quant_state_type: type):  # noqa: D401 -- no Optimizer.__init__
        self._target = target
        self._optimized = True
        self._draw_provider = None
        self._quant_rng_seed = getattr(target, "_quant_rng_seed", None)
        self._global_streams: Dict[str, Dict[str, GlobalStream]] = {"m1": {}, "m2": {}}
        self._wrapped: Dict[int, GlobalStream] = {}
        self._grad_clip = None
        self._quant_state_type = quant_state_type
        register_quant_state_type(quant_state_type)

    @property
    def state(self):
        return self._target.state

    @property
    def param_groups(self):
        return self._target.param_groups

    def _m1_scheme_for(self, parameter: torch.Tensor, group_scheme: str) -> str:
        return self._target._m1_scheme_for(parameter, group_scheme)

    def _effective_scheme(self, p: torch.Tensor, scheme: str, block_size: int) -> str:
        return self._target._effective_scheme(p, scheme, block_size)

    def _quant_generator(self, moment: str, device: torch.device):
        """The target's generator of `moment` on `device` as a stream (None without a seed)."""
        generator = self._target._quant_generator(moment, device)
        if generator is None:
            return None
        stream = self._wrapped.get(id(generator))
        if stream is None or stream.generator is not generator:
            # the generator is seeded with the moment's seed: key Philox with it as it is
            stream = self._wrapped[id(generator)] = GlobalStream(generator, 0)
        return stream

    def _all_streams(self) -> list:
        return list(self._wrapped.values()) + [s for streams in self._global_streams.values()
                                               for s in streams.values()]


class HipOptimizedBackend:
    """Drop-in for ``adamw4bit._optimized.OptimizedBackend`` (see the module docstring).

    ``reference_backend``: what takes the parameters the kernels do not (by default the
    reference's ``OptimizedBackend(optimizer)``); ``quant_state_type``: the class of new moment
    state (by default the reference's ``adamw4bit.quantization.QuantState``)."""

    def __init__(self, optimizer, *, deferred: bool = False, reference_backend: Any = None,
                 quant_state_type: Optional[type] = None) -> None:
        if reference_backend is None:
            from adamw4bit._optimized import OptimizedBackend  # the reference package

            reference_backend = OptimizedBackend(optimizer)
        if quant_state_type is None:
            from adamw4bit.quantization import QuantState as quant_state_type  # the reference package
        self._reference = reference_backend
        self._engine = _Engine(optimizer, quant_state_type)
        self._deferred = deferred
        self._pending: Dict[torch.device, list] = {}  # device -> [batch, per-parameter undos, params]
        for group in optimizer.param_groups:
            group.setdefault(_CHUNK_KEY, _CHUNK_NUMEL)
        # the aliased-state mark after a checkpoint load (_optimized.py:53-83)
        optimizer.register_load_state_dict_post_hook(QuantizedAdamW._after_load)

    def try_step_parameter(self, optimizer, parameter: torch.Tensor, group: Dict[str, Any]) -> bool:
        """Step `parameter` (``True``), or decline it with nothing changed and no draws consumed
        (``False``), as ``OptimizedBackend.try_step_parameter`` (``_optimized.py:128-143``)."""
        if optimizer is not self._engine._target:
            raise ValueError("this backend belongs to another optimizer")
        if getattr(optimizer, "telemetry", None) is not None or any(group.get(k) is not None
                                                                    for k in _DECLINING_GROUP_KEYS):
            return False
        if not parameter.is_cuda or parameter.dtype not in _DTYPES:
            return bool(self._reference.try_step_parameter(optimizer, parameter, group))
        if self._deferred:
            pending = self._pending.get(parameter.device)
            if pending is not None and any(p is parameter for p in pending[2]):
                self.flush(optimizer)  # the previous step's launch was never flushed
        engine = self._engine
        if not self._plan(parameter, group):
            return False
        try:
            checked = engine._preflight(parameter, group)
        except NotImplementedError:
            # a layout or dtype the kernels do not step (e.g. a gradient of another dtype)
            return bool(self._reference.try_step_parameter(optimizer, parameter, group))
        if not checked.optimized:
            return False
        for name in ("_last_update_directions", "_last_preconditioners", "_last_effective_preconditioners"):
            records = getattr(optimizer, name, None)
            if records is not None:
                records.pop(parameter, None)
        if self._deferred:
            pending = self._pending.get(parameter.device)
            if pending is None:
                pending = self._pending[parameter.device] = [_DeviceBatch(), [], []]
            batch, undos, params = pending
            undos.append(_StepUndo(engine, [checked.state]))
            try:
                engine._prepare(checked, batch)
            except BaseException:
                self._pending.pop(parameter.device, None)
                for undo in reversed(undos):
                    undo.restore()
                raise
            params.append(parameter)
            return True
        batch = _DeviceBatch()
        undo = _StepUndo(engine, [checked.state])
        try:
            engine._prepare(checked, batch)
            _launch(*batch.launch(None))
        except _lib.HipLaunchIncomplete:
            raise
        except BaseException:
            undo.restore()
            raise
        return True

    def _plan(self, parameter: torch.Tensor, group: Dict[str, Any]) -> bool:
        """The reference's preflight (``_optimized.py:85-126``), checked without creating state."""
        engine = self._engine
        grad = parameter.grad
        if parameter.layout != torch.strided or grad.layout != torch.strided:
            return False
        state = engine.state.get(parameter, {})
        requested = (engine._m1_scheme_for(parameter, group["m1_quant_scheme"]), group["m2_quant_scheme"])
        sizes = tuple(group["block_size"] if group["block_size"] is not None else default_block_size(m)
                      for m in requested)
        schemes = tuple(engine._effective_scheme(parameter, m, b) for m, b in zip(requested, sizes))
        return engine._plan_accepts(parameter, grad, group, requested, sizes, schemes, state)

    def flush(self, optimizer) -> None:
        """Launch the parameters prepared since the last flush (``deferred=True``): one launch per
        device.  A launch that fails before any kernel is enqueued is undone for all of them."""
        pending, self._pending = self._pending, {}
        for batch, undos, _ in pending.values():
            try:
                _launch(*batch.launch(None))
            except _lib.HipLaunchIncomplete:
                raise
            except BaseException:
                for undo in reversed(undos):
                    undo.restore()
                raise
