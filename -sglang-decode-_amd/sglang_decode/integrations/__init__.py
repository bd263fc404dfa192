"""Framework adapters (SGLang)."""
