"""Seed and bit-width schedule of a packed layer, uploaded once to the device.

Reference: ``PackedMSELayer._build_codebook_tensors`` / ``lazy_initialization``
(runtime/packed_qmse_cache.py:226-283).

* Q_prod (``use_qjl_keys``): keys use the (bits-1)-bit codebook with rotation
  R(seed+1) and the QJL matrix S(seed+31337); values use the bits-bit codebook
  with R(seed).
* Q_mse: keys and values both use the bits-bit codebook with R(seed).

Outlier-split layers (``split_codecs``; reference :243-273) have two channel
groups, each with parameters of its own dimension: the normal channels at
``bits`` with seed s, the outlier channels at ``bits + outlier_extra_bits`` with
seed s+7919.  Q_prod keys use (group bits - 1) MSE bits with the seed + 1 and
the QJL matrices S(s+31337) (normal) and S(s+31337+1) (outlier).
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

import numpy as np
import torch

from turboquant.quantization.turboquant_mse import (
    DEFAULT_GRID_SIZE,
    KEY_ROTATION_SEED_OFFSET,
    OUTLIER_SEED_OFFSET,
    QJL_SEED_OFFSET,
    codebook_f32,
    generate_qjl_matrix,
    random_rotation_matrix,
)
from turboquant.runtime.kernels import CodecParams, GroupCodec, group_matrix

#: widest code libtq's channel-group kernels pack
MAX_GROUP_BITS = 8


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


@dataclass
class SplitCodecs:
    """Device parameters of an outlier-split layer (two channel groups)."""

    bits: int
    outlier_bits: int
    use_qjl_keys: bool
    normal_indices: torch.Tensor  # int64 [d_n] on the device, ascending
    outlier_indices: torch.Tensor  # int64 [d_o] on the device, ascending
    value_normal: GroupCodec
    value_outlier: GroupCodec
    key_normal: GroupCodec  # the value groups themselves for Q_mse keys
    key_outlier: GroupCodec
    # the groups' channel-space matrices stacked into one D x D matrix per role (rows of the
    # normal group first): the rotated space of tq_decode_attention_groups
    key_stack: torch.Tensor
    value_stack: torch.Tensor
    qjl_stack: torch.Tensor | None


def _group(channels: np.ndarray, bits: int, seed: int, device: torch.device, grid_size: int,
           qjl_seed: int | None = None) -> GroupCodec:
    d = int(channels.shape[0])
    if d < 3:
        # the coordinate density (1 - x^2)^((d-3)/2) / Gamma((d-1)/2) has no Lloyd-Max solution below d = 3
        raise ValueError(f"a channel group needs at least 3 channels (got {d})")
    if not 1 <= bits <= MAX_GROUP_BITS:
        raise ValueError(f"channel-group bit width must be in 1..{MAX_GROUP_BITS}, got {bits}")
    rot, c, b = _host_codec(d, bits, seed, grid_size)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)  # noqa: E731
    qjl = qjl_ch = None
    if qjl_seed is not None:
        s = generate_qjl_matrix(d, qjl_seed)
        qjl, qjl_ch = s.to(device), dev(group_matrix(s.numpy(), channels))
    return GroupCodec(channels=channels, bits=bits, rotation=dev(rot), centers=dev(c), boundaries=dev(b),
                      rotation_ch=dev(group_matrix(rot, channels)), qjl=qjl, qjl_ch=qjl_ch)


_split_cache: dict[tuple, SplitCodecs] = {}


def split_codecs(normal_channels, outlier_channels, bits: int, outlier_extra_bits: int, seed: int,
                 use_qjl_keys: bool, device: torch.device | str, grid_size: int = DEFAULT_GRID_SIZE) -> SplitCodecs:
    """Parameters of a layer whose channels are split into a normal and an outlier group
    (reference ``PackedMSELayer.lazy_initialization``, runtime/packed_qmse_cache.py:243-273)."""
    device = torch.device(device)
    normal = np.ascontiguousarray(np.asarray(normal_channels, dtype=np.int64).astype(np.int32))
    outlier = np.ascontiguousarray(np.asarray(outlier_channels, dtype=np.int64).astype(np.int32))
    outlier_bits = bits + outlier_extra_bits
    if use_qjl_keys and (bits < 2 or outlier_bits < 2):
        raise ValueError("Q_prod needs bits >= 2 in both channel groups (bits-1 MSE bits for keys)")
    key = (tuple(normal.tolist()), tuple(outlier.tolist()), bits, outlier_extra_bits, seed, use_qjl_keys,
           device.type, device.index, grid_size)
    hit = _split_cache.get(key)
    if hit is not None:
        return hit
    oseed = seed + OUTLIER_SEED_OFFSET
    vn = _group(normal, bits, seed, device, grid_size)
    vo = _group(outlier, outlier_bits, oseed, device, grid_size)
    if use_qjl_keys:
        kn = _group(normal, bits - 1, seed + KEY_ROTATION_SEED_OFFSET, device, grid_size,
                    qjl_seed=seed + QJL_SEED_OFFSET)
        ko = _group(outlier, outlier_bits - 1, oseed + KEY_ROTATION_SEED_OFFSET, device, grid_size,
                    qjl_seed=seed + QJL_SEED_OFFSET + 1)
    else:
        kn, ko = vn, vo
    stack = lambda a, b: torch.cat((a[:len(normal)], b[:len(outlier)])).contiguous()  # noqa: E731
    out = SplitCodecs(bits=bits, outlier_bits=outlier_bits, use_qjl_keys=use_qjl_keys,
                      normal_indices=torch.from_numpy(normal.astype(np.int64)).to(device),
                      outlier_indices=torch.from_numpy(outlier.astype(np.int64)).to(device),
                      value_normal=vn, value_outlier=vo, key_normal=kn, key_outlier=ko,
                      key_stack=stack(kn.rotation_ch, ko.rotation_ch), value_stack=stack(vn.rotation_ch, vo.rotation_ch),
                      qjl_stack=stack(kn.qjl_ch, ko.qjl_ch) if use_qjl_keys else None)
    _split_cache[key] = out
    return out
