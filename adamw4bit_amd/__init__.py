"""MI355X-native fused 4-bit AdamW (ZIP-SR / ZE-EDEN) behind the ``adamw4bit`` optimizer API.

``QuantizedAdamW``, ``ZIPSRAdamW4Bit``, ``ZEEDENAdamW4Bit`` and ``AdamW8bit`` mirror
the reference package's exports (reference ``src/adamw4bit/__init__.py:3-5``).
Every ``step()`` runs one hand-written HIP kernel launch per device
(``libadamw4bit_hip.so``, built by ``python -m adamw4bit_amd.build``).
"""

from .adamw import AdamW8bit, QuantizedAdamW, ZEEDENAdamW4Bit, ZIPSRAdamW4Bit
from .quantization import QuantState

__all__ = ["QuantizedAdamW", "ZIPSRAdamW4Bit", "ZEEDENAdamW4Bit", "AdamW8bit", "QuantState"]
