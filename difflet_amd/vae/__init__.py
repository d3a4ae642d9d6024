"""The VAE decoder (FLUX.1) on the gfx950 kernels."""
