"""Backends of Difflet's op surface built in this package (only `rocm`)."""
