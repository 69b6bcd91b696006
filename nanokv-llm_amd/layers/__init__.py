"""Attention layer, compression step and scoring policy."""
