"""ctypes binding of ``libadamw4bit_hip.so`` (declared in ``include/adamw4bit_hip.h``).

The launch table handed to ``aw4_fused_step`` is a numpy structured array whose
dtype (:data:`TENSOR`) mirrors ``aw4_tensor`` byte for byte.  The library is
required: a missing or stale build raises instead of falling back to any other
implementation.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libadamw4bit_hip.so")

ABI_VERSION = 7
BLOCK = 128

# Error codes
OK, EINVAL, EHIP, EALIGN, ELAUNCHED = 0, -1, -2, -3, -4

# Codebooks / rounding / flags (AW4_* in the header)
CB_NF4, CB_SDYN4, CB_DYN4, CB_LIN4, CB_LIN4_NZ = 0, 1, 2, 3, 4
ROUND_FP32, ROUND_RTN, ROUND_STATE_SR, ROUND_UPDATE_SR, ROUND_LOOKAHEAD_SR = 0, 1, 2, 3, 4
MOMENT_ZERO_FLOOR, MOMENT_EDEN, MOMENT_GUARDS, MOMENT_EXT_DRAWS = 0x1, 0x2, 0x4, 0x8
MOMENT_SAMPLED_READ, MOMENT_READ_RAW_SCALE, MOMENT_FRESH_PROXY, MOMENT_PENDING = 0x10, 0x20, 0x40, 0x80
F32, BF16, F16, F64 = 0, 1, 2, 3
TENSOR_LERP1_LARGE, TENSOR_LERP2_LARGE, TENSOR_VEC_ALIGNED, TENSOR_GRAD_SCALE = 0x1, 0x2, 0x4, 0x8
TENSOR_GRAD_UNSCALE = 0x10

NUM_LUTS, LUT_HALF, LUT_EXP0 = 11, 89, 936
NOALLOC_TABLE_BYTES = 1 << 20
LUT_ENTRIES = 2 * LUT_HALF

MOMENT = np.dtype([
    ("codes", "<u8"), ("scales", "<u8"), ("values", "<u8"), ("draws", "<u8"),
    ("rng_seed", "<u8"), ("rng_offset", "<u8"),
    ("codebook", "<i4"), ("rounding", "<i4"), ("flags", "<i4"),
    ("sr_bias", "<f4"), ("sr_bias_rcp", "<f4"), ("sr_eps", "<f4"),
    ("la_beta2", "<f8"), ("la_fresh_weight", "<f8"), ("la_bias", "<f8"), ("la_eps", "<f8"),
])
TENSOR = np.dtype([
    ("param", "<u8"), ("grad", "<u8"), ("grad_scale", "<u8"), ("numel", "<i8"),
    ("param_dtype", "<i4"), ("grad_dtype", "<i4"), ("flags", "<i4"),
    ("w1", "<f4"), ("w2", "<f4"), ("decay", "<f4"), ("step_coef", "<f4"),
    ("bc2_sqrt", "<f4"), ("bc2_sqrt_rcp", "<f4"), ("eps", "<f4"),
    ("m1", MOMENT), ("m2", MOMENT),
    ("decay_f64", "<f8"), ("step_coef_f64", "<f8"),
])
assert MOMENT.itemsize == 104 and TENSOR.itemsize == 296

# Every function the header declares, with its ctypes signature.
SIGNATURES = {
    "aw4_abi_version": (ctypes.c_int, []),
    "aw4_last_error": (ctypes.c_char_p, []),
    "aw4_fused_step": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]),
    "aw4_fused_step_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]),
    "aw4_quantize": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]),
    "aw4_dequantize": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]),
    "aw4_uniforms": (ctypes.c_int, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p,
                                    ctypes.c_void_p]),
    "aw4_encode_tables": (ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64]),
    "aw4_clip_coefficient": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_void_p]),
    "aw4_unscale_clip_coefficient": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_float,
                                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "aw4_inject_launch_failure": (None, [ctypes.c_int32]),
}


class HipLibraryError(RuntimeError):
    """A call into the HIP library failed (the message is aw4_last_error()).  Unless it is a
    HipLaunchIncomplete, the call enqueued no step kernel."""


class HipLaunchIncomplete(HipLibraryError):
    """A step failed after some of its kernels were enqueued (AW4_ELAUNCHED): the parameters and
    moment state it covers may be partly updated."""


_lib: Optional[ctypes.CDLL] = None


def library() -> ctypes.CDLL:
    """Load the in-tree library once; raise if it is missing or of another ABI."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise ImportError(
            f"{LIBRARY} is missing: build it with `python -m adamw4bit_amd.build` "
            "(the 4-bit AdamW step has no implementation without it)")
    lib = ctypes.CDLL(LIBRARY)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.aw4_abi_version()
    if version != ABI_VERSION:
        raise ImportError(f"{LIBRARY} has ABI {version}, expected {ABI_VERSION}: rebuild it")
    _lib = lib
    return lib


def check(rc: int, what: str) -> int:
    if rc < 0:
        message = library().aw4_last_error().decode(errors="replace")
        raise (HipLaunchIncomplete if rc == ELAUNCHED else HipLibraryError)(f"{what} failed ({rc}): {message}")
    return rc


class Rows(np.ndarray):
    """Launch-table rows (dtype :data:`TENSOR`, C-contiguous) with their host address resolved
    once (``ptr``; numpy's ``ctypes.data`` costs about half a microsecond per call): a launch
    plan hands the same rows to every step.  Views and copies do not keep the address."""

    def __array_finalize__(self, obj) -> None:
        self.ptr = None


def rows_of(table: np.ndarray) -> Rows:
    """``table`` as :class:`Rows` (the same memory)."""
    assert table.dtype == TENSOR and table.flags.c_contiguous
    rows = table.view(Rows)
    rows.ptr = rows.ctypes.data
    return rows


def fused_step(table: np.ndarray, stream: int) -> None:
    """Launch one fused step over the rows of ``table`` (dtype :data:`TENSOR`)."""
    ptr = table.ptr if type(table) is Rows else None
    if ptr is None:
        assert table.dtype == TENSOR and table.flags.c_contiguous
        ptr = table.ctypes.data
    check(library().aw4_fused_step(ptr, len(table), stream), "aw4_fused_step")


def fused_step_noalloc(table: np.ndarray, stream: int) -> None:
    """``fused_step`` through ``aw4_fused_step_noalloc`` (no device allocation; tables of at most
    NOALLOC_TABLE_BYTES)."""
    assert table.dtype == TENSOR and table.flags.c_contiguous
    check(library().aw4_fused_step_noalloc(table.ctypes.data, len(table), stream), "aw4_fused_step_noalloc")


def quantize(values_ptr: int, numel: int, moment: np.ndarray, stream: int) -> None:
    assert moment.dtype == MOMENT and moment.shape == ()
    check(library().aw4_quantize(values_ptr, numel, moment.ctypes.data, stream), "aw4_quantize")


def dequantize(moment: np.ndarray, numel: int, out_ptr: int, stream: int) -> None:
    assert moment.dtype == MOMENT and moment.shape == ()
    check(library().aw4_dequantize(moment.ctypes.data, numel, out_ptr, stream), "aw4_dequantize")


def clip_coefficient(table: np.ndarray, max_norm: float, norm_ptr: int, coef_ptr: int, stream: int) -> None:
    """Global gradient norm of the rows of ``table`` and the clipping coefficient, written to
    the device floats at ``norm_ptr`` and ``coef_ptr``."""
    assert table.dtype == TENSOR and table.flags.c_contiguous
    check(library().aw4_clip_coefficient(table.ctypes.data, len(table), max_norm, norm_ptr, coef_ptr, stream),
          "aw4_clip_coefficient")


def unscale_clip_coefficient(table: np.ndarray, inv_scale_ptr: int, max_norm: float, norm_ptr: int, coef_ptr: int,
                             found_inf_ptr: int, stream: int) -> None:
    """``clip_coefficient`` over gradients scaled by a loss scale: each value is unscaled by the
    device float at ``inv_scale_ptr`` as it is read, and ``found_inf_ptr`` receives 1.0 if any
    scaled value is not finite."""
    assert table.dtype == TENSOR and table.flags.c_contiguous
    check(library().aw4_unscale_clip_coefficient(table.ctypes.data, len(table), inv_scale_ptr, max_norm, norm_ptr,
                                                 coef_ptr, found_inf_ptr, stream), "aw4_unscale_clip_coefficient")


def inject_launch_failure(after: int) -> None:
    """Make the next fused step on this thread fail after `after` step kernel launches (tests of
    error handling; no launch is attempted at that point).  Negative: clear."""
    library().aw4_inject_launch_failure(after)


def uniforms(seed: int, offset: int, n: int, out_ptr: int, stream: int) -> None:
    check(library().aw4_uniforms(seed, offset, n, out_ptr, stream), "aw4_uniforms")


def encode_tables() -> np.ndarray:
    """The kernels' encode lookup tables, shape (NUM_LUTS, LUT_ENTRIES, 4) uint32 words
    {threshold bits, base, level_lo bits, level_hi bits} (host only)."""
    lib = library()
    size = check(lib.aw4_encode_tables(None, 0), "aw4_encode_tables")
    out = np.zeros(size // 4, dtype=np.uint32)
    check(lib.aw4_encode_tables(out.ctypes.data, size), "aw4_encode_tables")
    return out.reshape(NUM_LUTS, LUT_ENTRIES, 4)
