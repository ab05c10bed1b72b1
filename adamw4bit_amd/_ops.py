"""The fused step and its clipping prologue as torch custom operators,
``adamw4bit_hip::fused_step_`` and ``adamw4bit_hip::clip_coefficient_``.

They wrap the C ABI's ``aw4_fused_step`` and ``aw4_clip_coefficient``
(``include/adamw4bit_hip.h``) so that a launch is one opaque operator to PyTorch: it declares
which tensors it writes (parameters and moment states, updated in place) and which it reads
(gradients, the clip coefficient, caller-provided draws), and it runs on the current stream of
the parameters' device.

``table`` is a CPU uint8 tensor of ``aw4_tensor`` rows (296 bytes each) holding everything but
device addresses; ``refs`` (CPU int64, one row per table row, :data:`ADDRESS_FIELDS` columns)
says which tensor each address field points into: an index into ``params + states + inputs``,
or -1 for "no buffer".  The operator reads the addresses from the tensors it receives at call
time, so it stays correct when functionalization hands it copies of the declared tensors (under
``torch.compile``), which a table of raw addresses taken earlier would miss.  There is no
implementation other than the HIP library.
"""

from __future__ import annotations

from typing import List, Sequence

import numpy as np
import torch

from . import _lib

# Address fields of an aw4_tensor row, in the column order of ``refs``.
ADDRESS_FIELDS = (
    ("param",), ("grad",), ("grad_scale",),
    ("m1", "codes"), ("m1", "scales"), ("m1", "values"), ("m1", "draws"),
    ("m2", "codes"), ("m2", "scales"), ("m2", "values"), ("m2", "draws"),
)


def _field(rows: np.ndarray, path: Sequence[str]) -> np.ndarray:
    view = rows
    for name in path:
        view = view[name]
    return view


def resolve_addresses(rows: np.ndarray, refs: np.ndarray, tensors: Sequence[torch.Tensor]) -> None:
    """Write ``tensors[refs[i, k]].data_ptr()`` into address field ``k`` of row ``i`` (0 where the
    reference is -1).  Every referenced tensor must be contiguous."""
    if refs.shape != (len(rows), len(ADDRESS_FIELDS)):
        raise ValueError(f"refs must have shape ({len(rows)}, {len(ADDRESS_FIELDS)}), got {tuple(refs.shape)}")
    if len(refs) and (refs.max(initial=-1) >= len(tensors) or refs.min(initial=-1) < -1):
        raise ValueError("refs index outside the tensor lists")
    for t in tensors:
        if not t.is_contiguous():
            raise ValueError("tensors referenced by a launch table must be contiguous")
    ptrs = np.array([t.data_ptr() for t in tensors] + [0], dtype=np.uint64)
    for k, path in enumerate(ADDRESS_FIELDS):
        _field(rows, path)[...] = ptrs[refs[:, k]]


@torch.library.custom_op("adamw4bit_hip::fused_step_", mutates_args=("params", "states"))
def fused_step_(params: List[torch.Tensor], states: List[torch.Tensor], inputs: List[torch.Tensor],
                table: torch.Tensor, refs: torch.Tensor) -> None:
    """One fused 4-bit AdamW step over the rows of ``table`` (one launch per kernel the rows need)."""
    if table.dtype != torch.uint8 or table.device.type != "cpu" or table.numel() % _lib.TENSOR.itemsize:
        raise ValueError("table must be a CPU uint8 tensor of aw4_tensor rows")
    if refs.dtype != torch.int64 or refs.device.type != "cpu":
        raise ValueError("refs must be a CPU int64 tensor")
    if not params:
        return
    device = params[0].device
    if device.type != "cuda":
        raise ValueError("the fused 4-bit step runs on HIP devices only")
    rows = table.contiguous().numpy().view(_lib.TENSOR).copy()
    resolve_addresses(rows, refs.contiguous().numpy(), list(params) + list(states) + list(inputs))
    with torch.cuda.device(device):
        _lib.fused_step(rows, torch.cuda.current_stream(device).cuda_stream)


@fused_step_.register_fake
def _fused_step_fake(params, states, inputs, table, refs) -> None:
    return None


def _norm_rows(grads: List[torch.Tensor], out: torch.Tensor, table: torch.Tensor) -> np.ndarray:
    if table.dtype != torch.uint8 or table.device.type != "cpu" or table.numel() % _lib.TENSOR.itemsize:
        raise ValueError("table must be a CPU uint8 tensor of aw4_tensor rows")
    if out.dtype != torch.float32 or out.numel() < 4 or out.device.type != "cuda" or not out.is_contiguous():
        raise ValueError("out must be 4 contiguous float32 values on a HIP device")
    rows = table.contiguous().numpy().view(_lib.TENSOR).copy()
    if len(rows) != len(grads) or not all(g.is_contiguous() for g in grads):
        raise ValueError("one contiguous gradient per table row")
    rows["grad"] = [g.data_ptr() for g in grads]
    return rows


@torch.library.custom_op("adamw4bit_hip::clip_coefficient_", mutates_args=("out",))
def clip_coefficient_(grads: List[torch.Tensor], out: torch.Tensor, table: torch.Tensor, max_norm: float) -> None:
    """Total gradient 2-norm and clipping coefficient of ``grads`` (row i of ``table`` describes
    ``grads[i]``; its address is taken from the tensor), written to ``out[0]`` and ``out[3]``
    (fp32, on the gradients' device; ``out[2:4]`` is the pair the step reads)."""
    rows = _norm_rows(grads, out, table)
    with torch.cuda.device(out.device):
        p = out.data_ptr()
        _lib.clip_coefficient(rows, max_norm, p, p + 12, torch.cuda.current_stream(out.device).cuda_stream)


@clip_coefficient_.register_fake
def _clip_coefficient_fake(grads, out, table, max_norm) -> None:
    return None


@torch.library.custom_op("adamw4bit_hip::unscale_clip_coefficient_", mutates_args=("out",))
def unscale_clip_coefficient_(grads: List[torch.Tensor], out: torch.Tensor, table: torch.Tensor,
                              max_norm: float) -> None:
    """``clip_coefficient_`` of the gradients unscaled by the inverse loss scale in ``out[2]``:
    total norm to ``out[0]``, found_inf (1.0 if any scaled value is not finite) to ``out[1]`` and
    the coefficient to ``out[3]``."""
    rows = _norm_rows(grads, out, table)
    with torch.cuda.device(out.device):
        p = out.data_ptr()
        _lib.unscale_clip_coefficient(rows, p + 8, max_norm, p, p + 12, p + 4,
                                      torch.cuda.current_stream(out.device).cuda_stream)


@unscale_clip_coefficient_.register_fake
def _unscale_clip_coefficient_fake(grads, out, table, max_norm) -> None:
    return None
