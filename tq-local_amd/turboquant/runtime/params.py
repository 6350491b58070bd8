"""Seed and bit-width schedule of a packed layer, uploaded once to the device.

Reference: ``PackedMSELayer._build_codebook_tensors`` / ``lazy_initialization``
(runtime/packed_qmse_cache.py:226-283).

* Q_prod (``use_qjl_keys``): keys use the (bits-1)-bit codebook with rotation
  R(seed+1) and the QJL matrix S(seed+31337); values use the bits-bit codebook
  with R(seed).
* Q_mse: keys and values both use the bits-bit codebook with R(seed).
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

import numpy as np
import torch

from turboquant.quantization.turboquant_mse import (
    DEFAULT_GRID_SIZE,
    KEY_ROTATION_SEED_OFFSET,
    QJL_SEED_OFFSET,
    codebook_f32,
    generate_qjl_matrix,
    random_rotation_matrix,
)
from turboquant.runtime.kernels import CodecParams


@dataclass
class LayerCodecs:
    bits: int
    use_qjl_keys: bool
    key: CodecParams
    value: CodecParams
    qjl: torch.Tensor | None  # fp32 [D, D] or None

    @property
    def key_bits(self) -> int:
        return self.key.bits

    @property
    def value_bits(self) -> int:
        return self.value.bits


@lru_cache(maxsize=64)
def _host_codec(dim: int, bits: int, seed: int, grid_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    centers, boundaries = codebook_f32(dim, bits, grid_size)
    return random_rotation_matrix(dim, seed), centers, boundaries


_device_cache: dict[tuple, LayerCodecs] = {}


def _codec(dim: int, bits: int, seed: int, device: torch.device, grid_size: int) -> CodecParams:
    rot, c, b = _host_codec(dim, bits, seed, grid_size)
    return CodecParams(
        bits=bits,
        rotation=torch.from_numpy(np.ascontiguousarray(rot)).to(device=device, dtype=torch.float32),
        centers=torch.from_numpy(c).to(device=device),
        boundaries=torch.from_numpy(b).to(device=device),
    )


def layer_codecs(dim: int, bits: int, seed: int, use_qjl_keys: bool, device: torch.device | str,
                 grid_size: int = DEFAULT_GRID_SIZE) -> LayerCodecs:
    """Device parameters for one packed layer (shared by all layers with the same schedule)."""
    device = torch.device(device)
    if bits < 1 or bits > 4:
        raise ValueError(f"bits must be in 1..4, got {bits}")
    if use_qjl_keys and bits < 2:
        raise ValueError("Q_prod needs bits >= 2 (bits-1 MSE bits for keys)")
    key = (dim, bits, seed, use_qjl_keys, device.type, device.index, grid_size)
    hit = _device_cache.get(key)
    if hit is not None:
        return hit
    value = _codec(dim, bits, seed, device, grid_size)
    if use_qjl_keys:
        kc = _codec(dim, bits - 1, seed + KEY_ROTATION_SEED_OFFSET, device, grid_size)
        qjl = generate_qjl_matrix(dim, seed + QJL_SEED_OFFSET).to(device)
    else:
        kc, qjl = value, None
    out = LayerCodecs(bits=bits, use_qjl_keys=use_qjl_keys, key=kc, value=value, qjl=qjl)
    _device_cache[key] = out
    return out
