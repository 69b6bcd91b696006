"""Per-step metadata context."""
