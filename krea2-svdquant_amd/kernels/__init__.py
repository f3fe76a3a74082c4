"""Kernel backends: ``hip`` (gfx950 HIP kernels through the C-ABI in include/svdq_gfx950.h)."""
