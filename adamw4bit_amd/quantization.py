"""Moment-state layout and 4-bit codec tables shared by the host code and the HIP kernel.

This module owns everything about the persistent optimizer-state format that the
fused step reads and writes in place:

* ``QuantState`` -- the per-moment scale container kept in ``optimizer.state``
  (same attribute names as ``adamw4bit.quantization.QuantState``,
  reference ``src/adamw4bit/quantization.py:15-30``).
* packed nibble storage: element ``2j`` in the low nibble of byte ``j``, element
  ``2j+1`` in the high nibble (reference ``quantization.py:627-654``).
* the five 16-level codebooks the optimized path can use, as exact float32 bit
  patterns.  They are the values of the reference's closed forms
  (``quantization.py:201-237`` dynamic maps, ``:401-422`` NF4, ``:457-497``
  linear grids); the tests recompute them from those formulas.
* the scheme table: which codebook, which rounding rule (round-to-nearest,
  value-space stochastic rounding, preconditioner-space stochastic rounding) and
  whether code 0 is floored to code 1 (``dyn4_nz``), for every scheme name the
  reference accepts on its optimized path (``_optimized.py:36-41``).
"""

from __future__ import annotations

import struct
from typing import Dict, Tuple

import torch


class QuantState:
    """Block-scale container for one quantized moment.

    ``absmax`` is a 1-D float32 tensor with one scale per ``blocksize`` values,
    ``shape`` the logical shape of the moment, ``dtype`` its logical dtype and
    ``packed`` whether the codes are stored two per byte.
    Mirrors reference ``quantization.py:15-30``.
    """

    def __init__(self, absmax, shape=None, dtype=None, blocksize=None, packed: bool = False):
        self.absmax = absmax
        self.shape = shape
        self.dtype = dtype
        self.blocksize = blocksize
        self.packed = packed

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return (f"QuantState(absmax=<{tuple(self.absmax.shape)} {self.absmax.dtype} "
                f"{self.absmax.device}>, shape={tuple(self.shape) if self.shape is not None else None}, "
                f"dtype={self.dtype}, blocksize={self.blocksize}, packed={self.packed})")


# --------------------------------------------------------------------------
# Codebooks (float32 bit patterns, sorted ascending; code = index)
# --------------------------------------------------------------------------

def _from_bits(words: Tuple[int, ...]) -> Tuple[float, ...]:
    return tuple(struct.unpack("<f", struct.pack("<I", w))[0] for w in words)


# NF4 (QLoRA NormalFloat4 table, reference quantization.py:401-422).
_NF4_BITS = (
    0xBF800000, 0xBF3239B1, 0xBF066B31, 0xBECA32A0, 0xBE91A24E, 0xBE3D353D, 0xBDBA786C, 0x00000000,
    0x3DA2FAFF, 0x3E24CAE3, 0x3E7C04DD, 0x3EAD0339, 0x3EE1A4B7, 0x3F1007AB, 0x3F3913B2, 0x3F800000,
)
# Signed dynamic map, 3 exponent bits, 4 total bits (quantization.py:201-237, :386-398).
_SDYN4_BITS = (
    0xBF633333, 0xBF29999A, 0xBEE00000, 0xBE599999, 0xBD9EB852, 0xBD051EB9, 0xBBB43958, 0x00000000,
    0x3BB43958, 0x3D051EB9, 0x3D9EB852, 0x3E599999, 0x3EE00000, 0x3F29999A, 0x3F633333, 0x3F800000,
)
# Unsigned dynamic map, 3 exponent bits, 4 total bits (quantization.py:201-237, :500-552).
_DYN4_BITS = (
    0x00000000, 0x3B54FDF4, 0x3BFDF3B5, 0x3CAE147B, 0x3D333333, 0x3D87AE15, 0x3DB5C28F, 0x3E200000,
    0x3E89999A, 0x3EC33333, 0x3EFCCCCD, 0x3F1B3334, 0x3F380000, 0x3F54CCCC, 0x3F71999A, 0x3F800000,
)
# torch.linspace(0, 1, 16) in float32 (quantization.py:457-463).
_LIN4_BITS = (
    0x00000000, 0x3D888889, 0x3E088889, 0x3E4CCCCE, 0x3E888889, 0x3EAAAAAB, 0x3ECCCCCE, 0x3EEEEEF0,
    0x3F088888, 0x3F199999, 0x3F2AAAAA, 0x3F3BBBBC, 0x3F4CCCCD, 0x3F5DDDDE, 0x3F6EEEEF, 0x3F800000,
)
# torch.linspace(0, 1, 17)[1:] = k/16 (quantization.py:466-472).
_LIN4_NZ_BITS = tuple(struct.unpack("<I", struct.pack("<f", k / 16.0))[0] for k in range(1, 17))

# Codebook ids are part of the C ABI (include/adamw4bit_hip.h, AW4_CB_*).
CB_NF4, CB_SDYN4, CB_DYN4, CB_LIN4, CB_LIN4_NZ = 0, 1, 2, 3, 4
CODEBOOK_BITS: Dict[int, Tuple[int, ...]] = {
    CB_NF4: _NF4_BITS,
    CB_SDYN4: _SDYN4_BITS,
    CB_DYN4: _DYN4_BITS,
    CB_LIN4: _LIN4_BITS,
    CB_LIN4_NZ: _LIN4_NZ_BITS,
}
CODEBOOK_VALUES: Dict[int, Tuple[float, ...]] = {k: _from_bits(v) for k, v in CODEBOOK_BITS.items()}

# Rounding rules (AW4_ROUND_* in the C ABI).
ROUND_NONE = 0      # fp32 state, no codec
ROUND_RTN = 1       # nearest level, ties to the upper level (_compiled_quantization.py:41-45)
ROUND_STATE_SR = 2  # value-unbiased stochastic rounding (_compiled_quantization.py:60-71)
ROUND_UPDATE_SR = 3  # preconditioner-space stochastic rounding (_compiled_quantization.py:74-109)
ROUND_LOOKAHEAD_SR = 4  # next-step preconditioner stochastic rounding (quantization.py:779-895)

# scheme -> (codebook id, rounding rule, floor code 0 to code 1)
# Covers every scheme the reference's optimized path accepts (_optimized.py:36-41)
# plus the reference-step update-SR names that share a codebook and rule: the
# fp32-read, sampled-read and store-side-EDEN variants differ only in what the
# step reads back and stores (adamw.py:615-683).
SCHEMES: Dict[str, Tuple[int, int, bool]] = {
    "nf4": (CB_NF4, ROUND_RTN, False),
    "nf4_sr": (CB_NF4, ROUND_STATE_SR, False),
    "sdyn4": (CB_SDYN4, ROUND_RTN, False),
    "sdyn4_sr": (CB_SDYN4, ROUND_STATE_SR, False),
    "lin4": (CB_LIN4, ROUND_RTN, False),
    "lin4_sr": (CB_LIN4, ROUND_STATE_SR, False),
    "lin4_nz": (CB_LIN4_NZ, ROUND_RTN, False),
    "lin4_upd_sr_fp32read": (CB_LIN4, ROUND_UPDATE_SR, False),
    "dyn4": (CB_DYN4, ROUND_RTN, False),
    "dyn4_sr": (CB_DYN4, ROUND_STATE_SR, False),
    "dyn4_nz": (CB_DYN4, ROUND_RTN, True),
    "dyn4_upd_sr_fp32read": (CB_DYN4, ROUND_UPDATE_SR, False),
    "dyn4_lookahead_sr": (CB_DYN4, ROUND_UPDATE_SR, False),
    "dyn4_upd_sr_fp32read_nextbc": (CB_DYN4, ROUND_UPDATE_SR, False),
    "lin4_upd_sr": (CB_LIN4, ROUND_UPDATE_SR, False),
    "dyn4_upd_sr": (CB_DYN4, ROUND_UPDATE_SR, False),
    "lin4_upd_sr_store_eden": (CB_LIN4, ROUND_UPDATE_SR, False),
    "dyn4_upd_sr_store_eden": (CB_DYN4, ROUND_UPDATE_SR, False),
    "dyn4_la_upd_sr": (CB_DYN4, ROUND_LOOKAHEAD_SR, False),
    "dyn4_proxy_la_upd_sr": (CB_DYN4, ROUND_LOOKAHEAD_SR, False),
    "dyn4_vproxy_la_upd_sr": (CB_DYN4, ROUND_LOOKAHEAD_SR, False),
}

# m2 schemes whose update reads back the sampled value (adamw.py:636-656) and those that
# also keep 1 / denominator as state "m2_read_preconditioner" and apply EDEN to the stored
# scale only (adamw.py:615-635).
SAMPLED_READ_SCHEMES = frozenset({"lin4_upd_sr", "dyn4_upd_sr"})
STORE_EDEN_SCHEMES = frozenset({"lin4_upd_sr_store_eden", "dyn4_upd_sr_store_eden"})

# Lookahead update-SR m2 schemes (adamw.py:118-120, 566-614): the pending form keeps the new
# m2 in fp32 as state "lookahead_pending_exp_avg_sq" and updates from a lookahead sample of
# it; the proxy forms store codes sampled for the next step's update, with the fresh term
# (1 - beta2) g^2 of the current gradient (proxy) or (1 - beta2) m2 (v-proxy).
PENDING_LOOKAHEAD_SCHEMES = frozenset({"dyn4_la_upd_sr"})
PROXY_LOOKAHEAD_SCHEMES = frozenset({"dyn4_proxy_la_upd_sr"})
VPROXY_LOOKAHEAD_SCHEMES = frozenset({"dyn4_vproxy_la_upd_sr"})
LOOKAHEAD_SCHEMES = PENDING_LOOKAHEAD_SCHEMES | PROXY_LOOKAHEAD_SCHEMES | VPROXY_LOOKAHEAD_SCHEMES
PENDING_KEY = "lookahead_pending_exp_avg_sq"

STOCHASTIC_ROUNDING = (ROUND_STATE_SR, ROUND_UPDATE_SR)

# Every scheme name the reference constructor accepts (adamw.py:103-110).
VALID_SCHEMES = (
    "linear", "dynamic",
    "sdyn4", "sdyn4_sr", "nf4", "nf4_sr",
    "lin4", "lin4_sr", "lin4_upd_sr", "lin4_upd_sr_store_eden", "lin4_upd_sr_fp32read", "lin4_nz",
    "dyn4", "dyn4_sr", "dyn4_upd_sr", "dyn4_upd_sr_store_eden", "dyn4_upd_sr_fp32read",
    "dyn4_lookahead_sr", "dyn4_upd_sr_fp32read_nextbc", "dyn4_la_upd_sr", "dyn4_proxy_la_upd_sr",
    "dyn4_vproxy_la_upd_sr", "dyn4_nz",
    "fp32",
)

# Schemes whose storage bias correction is the next step's (adamw.py:114-117, _optimized.py:42).
NEXT_BIAS_SCHEMES = frozenset({"dyn4_lookahead_sr", "dyn4_upd_sr_fp32read_nextbc"})

# Bit widths (quantization.py:587-592) and the block-size defaults keyed by them (:593).
_EIGHT_BIT = frozenset({"linear", "dynamic"})
DEFAULT_BLOCK_SIZE_BY_BITS = {8: 256, 4: 128}
MIN_QUANT_NUMEL = 4096  # TorchAO eligibility threshold (adamw.py:19)


def is_4bit_scheme(mode: str) -> bool:
    """Whether ``mode`` stores 16-level codes (reference ``quantization.py:596-598``)."""
    return mode in VALID_SCHEMES and mode not in _EIGHT_BIT and mode != "fp32"


def default_block_size(mode: str) -> int:
    """128 for 4-bit schemes, 256 otherwise (reference ``quantization.py:694-703``)."""
    return DEFAULT_BLOCK_SIZE_BY_BITS[4] if is_4bit_scheme(mode) else DEFAULT_BLOCK_SIZE_BY_BITS[8]


def default_min_scale(mode: str) -> float:
    """Block-scale floor: 1e-12 for 4-bit schemes, 1e-8 for 8-bit (``quantization.py:706-712``)."""
    return 1e-12 if is_4bit_scheme(mode) else 1e-8


def codebook_tensor(mode: str, device: torch.device | str = "cpu") -> torch.Tensor:
    """The scheme's 16 levels as a float32 tensor."""
    cb_id = SCHEMES[mode][0]
    return torch.tensor(CODEBOOK_VALUES[cb_id], dtype=torch.float32, device=device)


def pack_4bit_codes(codes: torch.Tensor) -> torch.Tensor:
    """Two codes per byte, even element in the low nibble (``quantization.py:627-638``)."""
    if codes.dtype != torch.uint8:
        raise TypeError(f"4-bit codes must use torch.uint8, found {codes.dtype}")
    flat = codes.reshape(-1)
    n = flat.numel()
    out = flat[0::2].clone()
    if n > 1:
        out[: n // 2] |= flat[1::2] << 4
    return out


def unpack_4bit_codes(codes: torch.Tensor, *, numel: int) -> torch.Tensor:
    """Inverse of :func:`pack_4bit_codes` (``quantization.py:641-654``)."""
    if codes.dtype != torch.uint8:
        raise TypeError(f"Packed 4-bit codes must use torch.uint8, found {codes.dtype}")
    expected = (numel + 1) // 2
    if codes.numel() != expected:
        raise ValueError(f"Packed code length mismatch: expected {expected}, found {codes.numel()}")
    flat = codes.reshape(-1)
    out = torch.empty(flat.numel() * 2, dtype=torch.uint8, device=flat.device)
    out[0::2] = flat & 0x0F
    out[1::2] = flat >> 4
    return out[:numel]


def initial_code_and_scale(mode: str, eden: bool) -> Tuple[int, float]:
    """Code and block scale that encode an all-zero moment under ``mode``.

    The reference initializes a quantized moment by encoding zeros
    (``_moment_buffer.py:106-126``, ``adamw.py:524-545``): every block gets the
    floor scale 1e-12, every value normalizes to 0.0, and the code is the
    rounding rule's choice for 0.0 (deterministic for every rule: 0.0 either is a
    level or rounds up to the level the guards select).  ``dyn4_nz`` floors code
    0 to code 1.  With EDEN the scale becomes ``1e-12 * (0 / 1e-12) = 0``.
    """
    cb_id, rounding, floor_zero = SCHEMES[mode]
    levels = CODEBOOK_VALUES[cb_id]
    x = 0.0
    count = sum(1 for v in levels if v < x)          # searchsorted, side="left"
    lower, upper = max(count - 1, 0), min(count, 15)
    a, b = levels[lower], levels[upper]
    if rounding in (ROUND_RTN, ROUND_LOOKAHEAD_SR):
        # the proxy lookahead schemes store their zero state with plain dyn4 (quantization.py:583-584)
        code = lower if abs(x - a) < abs(b - x) else upper
    elif rounding == ROUND_STATE_SR:
        # P(upper) is 1 at x >= b and 0 at x <= a; otherwise x is strictly inside.
        code = upper if x >= b else lower if x <= a else None
    else:
        # P(lower) is 1 at x <= a and 0 at x >= b.
        code = lower if x <= a else upper if x >= b else None
    if code is None:  # pragma: no cover - no shipped codebook has 0 strictly between levels
        raise AssertionError(f"zero is not deterministic under {mode}")
    if floor_zero and code == 0:
        code = 1
    scale = 0.0 if eden else float(torch.tensor(1e-12, dtype=torch.float32))
    return code, scale
