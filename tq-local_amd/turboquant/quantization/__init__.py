"""Quantizer parameters: Lloyd-Max codebook, Haar rotation, QJL matrix."""

from turboquant.quantization.turboquant_mse import (
    build_scalar_codebook,
    codebook_f32,
    generate_qjl_matrix,
    random_rotation_matrix,
)

__all__ = ["build_scalar_codebook", "codebook_f32", "generate_qjl_matrix", "random_rotation_matrix"]
