"""MI355X-native fused 4-bit AdamW (ZIP-SR / ZE-EDEN) behind the ``adamw4bit`` optimizer API."""
