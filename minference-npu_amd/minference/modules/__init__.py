"""Patched attention forward and per-layer dispatch plan."""
