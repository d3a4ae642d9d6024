"""Platforms of this package (only `rocm`)."""
