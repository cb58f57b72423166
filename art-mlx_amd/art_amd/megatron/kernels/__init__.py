"""Mirrors of art.megatron.kernels."""
