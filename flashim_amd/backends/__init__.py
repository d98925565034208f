"""Kernel backends of this package: ``hip`` (hand-written gfx950 kernels behind ``libflashim_amd.so``)."""
