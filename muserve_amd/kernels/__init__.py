"""Kernel wrappers with the reference's muserve/kernels names."""
