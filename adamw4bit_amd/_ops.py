"""The fused step and its clipping prologue as torch custom operators,
``adamw4bit_hip::fused_step_`` and ``adamw4bit_hip::clip_coefficient_``.

It wraps the C ABI's ``aw4_fused_step`` (``include/adamw4bit_hip.h``) so that the launch is one
opaque operator to PyTorch: it declares which tensors it writes (parameters and moment
states, updated in place) and which it reads (gradients, caller-provided draws), and it runs
on the current stream of the parameters' device.  ``table`` is the launch table, a CPU uint8
tensor of ``aw4_tensor`` rows (280 bytes each) that hold the device addresses of the listed
tensors.  There is no implementation other than the HIP library.
"""

from __future__ import annotations

from typing import List

import torch

from . import _lib


@torch.library.custom_op("adamw4bit_hip::fused_step_", mutates_args=("params", "states"))
def fused_step_(params: List[torch.Tensor], states: List[torch.Tensor], inputs: List[torch.Tensor],
                table: torch.Tensor) -> None:
    """One fused 4-bit AdamW step over the rows of ``table`` (one launch per kernel the rows need)."""
    if table.dtype != torch.uint8 or table.device.type != "cpu" or table.numel() % _lib.TENSOR.itemsize:
        raise ValueError("table must be a CPU uint8 tensor of aw4_tensor rows")
    if not params:
        return
    device = params[0].device
    if device.type != "cuda":
        raise ValueError("the fused 4-bit step runs on HIP devices only")
    rows = table.contiguous().numpy().view(_lib.TENSOR)
    with torch.cuda.device(device):
        _lib.fused_step(rows, torch.cuda.current_stream(device).cuda_stream)


@fused_step_.register_fake
def _fused_step_fake(params, states, inputs, table) -> None:
    return None


@torch.library.custom_op("adamw4bit_hip::clip_coefficient_", mutates_args=("out",))
def clip_coefficient_(grads: List[torch.Tensor], out: torch.Tensor, table: torch.Tensor, max_norm: float) -> None:
    """Total gradient 2-norm and clipping coefficient of the rows of ``table`` (the gradients in
    ``grads``), written to ``out[0]`` and ``out[1]`` (fp32, on the gradients' device)."""
    if table.dtype != torch.uint8 or table.device.type != "cpu" or table.numel() % _lib.TENSOR.itemsize:
        raise ValueError("table must be a CPU uint8 tensor of aw4_tensor rows")
    if out.dtype != torch.float32 or out.numel() < 2 or out.device.type != "cuda" or not out.is_contiguous():
        raise ValueError("out must be 2 contiguous float32 values on a HIP device")
    rows = table.contiguous().numpy().view(_lib.TENSOR)
    with torch.cuda.device(out.device):
        _lib.clip_coefficient(rows, max_norm, out.data_ptr(), out.data_ptr() + 4,
                              torch.cuda.current_stream(out.device).cuda_stream)


@clip_coefficient_.register_fake
def _clip_coefficient_fake(grads, out, table, max_norm) -> None:
    return None
