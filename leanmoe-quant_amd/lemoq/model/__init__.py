"""Fixed-shape OLMoE decode-step module and session (no HF monkey-patching)."""
