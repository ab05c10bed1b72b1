"""Counter-based random streams for stochastic rounding.

Each (moment, device) pair owns one Philox4x32-10 stream, keyed by the seed
the reference gives that moment's ``torch.Generator``
(``(quant_rng_seed + offset) mod (2**63 - 1)``, ``adamw.py:281-305``).  A
stochastic write of ``n`` values consumes stream positions
``offset .. offset + n - 1`` (element ``k`` of the write uses position
``offset + k``), and the stream then advances by ``n`` rounded up to a
multiple of 128, as the reference's generators advance by the ``n`` uniforms
``_uniform_draws`` takes (``_optimized_quantization.py:37-43``); every
quantized write covers whole 128-value blocks, so nothing is skipped.  Writes
start at multiples of 128: the kernels draw a block's uniforms from one
position group.  The draws depend only on (seed, position), never on launch
geometry.

The checkpointed state is a 16-byte ``uint8`` tensor: the key and the position
as little-endian uint64 (the layout of a CUDA ``torch.Generator`` state).
"""

from __future__ import annotations

import struct

import torch

STATE_BYTES = 16


class PhiloxStream:
    __slots__ = ("seed", "offset")

    def __init__(self, seed: int, offset: int = 0):
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.offset = int(offset)

    def take(self, n: int) -> int:
        """Reserve ``n`` positions and return the first (a multiple of 128)."""
        first = self.offset
        self.offset += (int(n) + 127) // 128 * 128
        return first

    def advance(self, n: int) -> None:
        self.take(n)

    def get_state(self) -> torch.Tensor:
        raw = struct.pack("<QQ", self.seed, self.offset)
        return torch.frombuffer(bytearray(raw), dtype=torch.uint8).clone()

    def set_state(self, state: torch.Tensor) -> None:
        if not torch.is_tensor(state) or state.dtype != torch.uint8 or state.numel() != STATE_BYTES:
            raise ValueError(
                "quantization RNG state must be a 16-byte uint8 tensor (Philox key and position), "
                f"got {getattr(state, 'dtype', type(state))} with {getattr(state, 'numel', lambda: '?')()} elements")
        seed, offset = struct.unpack("<QQ", bytes(state.detach().cpu().contiguous().numpy().tobytes()))
        if offset % 128:
            raise ValueError(f"quantization RNG position {offset} is not a multiple of 128")
        self.seed, self.offset = seed, offset


class GlobalStream:
    """The stream of a (moment, device) when ``quant_rng_seed`` is None: the reference then draws
    every stochastic write from torch's default generator of the device
    (``torch.rand(..., generator=None)``, ``_optimized_quantization.py:37-43``).  Here each write
    keys Philox4x32-10 with that generator's seed, mixed with the moment's constant, and takes its
    positions from the generator's offset, which it moves past them.  So reseeding torch, or any
    other random number torch draws on the device, changes the next writes' draws, and saving and
    restoring torch's RNG state (``torch.cuda.get_rng_state``) saves and restores them, as with the
    reference.  Positions are 128-value groups; each group moves the generator's offset by 4 (its
    offsets are multiples of 4)."""

    __slots__ = ("generator", "mix")
    UNIT = 4

    def __init__(self, generator: torch.Generator, mix: int):
        self.generator = generator
        self.mix = int(mix) & 0xFFFFFFFFFFFFFFFF

    @property
    def seed(self) -> int:
        return (self.generator.initial_seed() ^ self.mix) & 0xFFFFFFFFFFFFFFFF

    @property
    def offset(self) -> int:
        return -(-self.generator.get_offset() // self.UNIT) * 128

    @offset.setter
    def offset(self, value: int) -> None:
        self.generator.set_offset(int(value) // 128 * self.UNIT)

    def take(self, n: int) -> int:
        """Reserve ``n`` positions and return the first (a multiple of 128)."""
        first = self.offset
        self.offset = first + (int(n) + 127) // 128 * 128
        return first

    def advance(self, n: int) -> None:
        self.take(n)
