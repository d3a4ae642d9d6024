"""The text encoders (T5-XXL, UMT5-XXL) on the gfx950 kernels."""
