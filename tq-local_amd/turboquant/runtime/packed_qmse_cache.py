"""Packed TurboQuant KV cache (a transformers ``CacheLayerMixin``) backed by libtq.

Drop-in for reference ``runtime/packed_qmse_cache.py``: the same container
types (``PackedTensorMSE``, ``PackedQJL``), the same per-layer attribute names
(``keys_packed``, ``_keys_qjl``, ``values_packed``, ``_dense_keys``, ...), the
same packed layout, seed schedule, norm guard and reconstruction report.

Differences, all on purpose:
* Storage is capacity-preallocated ``[B, H, cap, row]`` buffers; decode-append
  encodes the new token straight into slot ``N`` (one kernel launch per tensor)
  instead of the reference's ``torch.cat`` of the whole history
  (``runtime/packed_qmse_cache.py:81-92, 135-140``).  ``keys_packed`` etc. are
  ``[:, :, :N]`` views of those buffers.
* Every encode / decode is a libtq HIP kernel; there is no CPU path.
* ``get_mask_sizes(query_length)`` / ``get_max_length()`` follow the installed
  transformers (5.x) cache-layer protocol.
* The outlier-channel split (``num_outlier_channels > 0``, reference :95-114,
  :437-535) encodes and decodes each channel group with libtq's channel-group
  kernels, in prefill and in decode-append alike (the reference's lazy
  decode-append ignores the split and hands the 128-channel token to the
  normal group's smaller rotation).
"""

from __future__ import annotations

import sys
from dataclasses import dataclass
from math import sqrt
from typing import Any

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from turboquant.runtime import kernels as K
from turboquant.runtime.params import LayerCodecs, SplitCodecs, layer_codecs, split_codecs

#: growth step of the capacity buffers when decode-append runs out of slots
DEFAULT_RESERVE_TOKENS = 256


@dataclass
class PackedTensorMSE:
    """Packed Q_mse codes of one tensor [B, H, N, D] (reference :58-92)."""

    packed_indices: torch.Tensor  # u8 [B, H, N, ceil(D*bits/8)]
    norms: torch.Tensor  # f16 [B, H, N]
    original_shape: tuple[int, int, int, int]
    original_dtype: torch.dtype
    bits: int

    @property
    def num_vectors(self) -> int:
        b, h, n, _ = self.original_shape
        return int(b * h * n)

    @property
    def dimension(self) -> int:
        return int(self.original_shape[-1])

    def storage_bytes(self) -> int:
        return int(self.packed_indices.numel() * self.packed_indices.element_size()
                   + self.norms.numel() * self.norms.element_size())

    def append(self, other: "PackedTensorMSE") -> "PackedTensorMSE":
        """A new container holding this one's tokens followed by ``other``'s (reference :81-92).
        The cache layer itself never calls this: it writes new tokens into capacity slots."""
        if self.original_shape[:2] != other.original_shape[:2] or self.dimension != other.dimension:
            raise ValueError("Packed tensor append requires matching batch, head, and dimension shape.")
        b, h, n, d = self.original_shape
        return PackedTensorMSE(torch.cat((self.packed_indices, other.packed_indices), dim=2).contiguous(),
                               torch.cat((self.norms, other.norms), dim=2).contiguous(),
                               (b, h, n + other.original_shape[2], d), self.original_dtype, self.bits)


@dataclass
class PackedQJL:
    """1-bit QJL sign sketch and residual norms (reference :121-140)."""

    packed_signs: torch.Tensor  # u8 [B, H, N, D/8]
    residual_norms: torch.Tensor  # f16 [B, H, N]
    dimension: int

    def storage_bytes(self) -> int:
        return int(self.packed_signs.numel() * self.packed_signs.element_size()
                   + self.residual_norms.numel() * self.residual_norms.element_size())

    def append(self, other: "PackedQJL") -> "PackedQJL":
        """A new sketch holding this one's tokens followed by ``other``'s (reference :135-140)."""
        return PackedQJL(torch.cat((self.packed_signs, other.packed_signs), dim=2).contiguous(),
                         torch.cat((self.residual_norms, other.residual_norms), dim=2).contiguous(),
                         self.dimension)


def _codec_of(rotation: torch.Tensor, centers: torch.Tensor | None, boundaries: torch.Tensor | None,
              bits: int) -> K.CodecParams:
    """libtq codec from the reference's parameter tensors (fp32, contiguous, on the device).
    Copies made here are freed after the launch; the caching allocator hands their blocks
    only to work ordered after the kernel on the same stream."""
    f32 = lambda t: None if t is None else (t if t.dtype == torch.float32 and t.is_contiguous()  # noqa: E731
                                            else t.float().contiguous())
    return K.CodecParams(bits=int(bits), rotation=f32(rotation), centers=f32(centers), boundaries=f32(boundaries))


def _packed_rows(t: torch.Tensor) -> torch.Tensor:
    """A packed [B, H, N, ...] tensor as libtq reads it (groups N slots apart)."""
    return t if t.is_contiguous() else t.contiguous()


def detect_outlier_channels(key_states: torch.Tensor, value_states: torch.Tensor,
                            num_outlier_channels: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(outlier, normal) channel indices, both ascending: the channels of largest
    combined key + value energy (reference runtime/packed_qmse_cache.py:95-114)."""
    combined = key_states.float().pow(2).sum(dim=(0, 1, 2)) + value_states.float().pow(2).sum(dim=(0, 1, 2))
    outlier = torch.topk(combined, num_outlier_channels).indices.sort().values
    keep = torch.ones(combined.shape[0], dtype=torch.bool, device=combined.device)
    keep[outlier] = False
    return outlier, torch.arange(combined.shape[0], device=combined.device)[keep]


class _Store:
    """Capacity buffers of one packed layer; slots [0, length) are valid.

    ``spec`` maps each buffer name to (trailing row shape, dtype), or to None for a
    buffer the layer does not have; buffers are [B, H, cap, *row] and are reachable
    as attributes of the store (None when absent)."""

    def __init__(self, B: int, H: int, cap: int, device: torch.device,
                 spec: dict[str, tuple[tuple, torch.dtype] | None]):
        self.B, self.H, self.device, self.spec = B, H, device, spec
        self.length = 0
        self.cap = 0
        for name in spec:
            setattr(self, name, None)
        self._alloc(cap)

    def _alloc(self, cap: int) -> None:
        n = self.length
        for name, entry in self.spec.items():
            if entry is None:
                continue
            row, dtype = entry
            buf = torch.zeros(self.B, self.H, cap, *row, dtype=dtype, device=self.device)
            old = getattr(self, name)
            if old is not None and n:
                buf[:, :, :n].copy_(old[:, :, :n])
            setattr(self, name, buf)
        self.cap = cap

    def reserve(self, extra: int, reserve_tokens: int) -> None:
        need = self.length + extra
        if need > self.cap:
            self._alloc(max(need + reserve_tokens, 2 * self.cap))


def _flat_spec(D: int, c: LayerCodecs) -> dict[str, tuple[tuple, torch.dtype] | None]:
    spec = {"kc": ((K.row_bytes(D, c.key_bits),), torch.uint8), "kn": ((), torch.float16),
            "vc": ((K.row_bytes(D, c.value_bits),), torch.uint8), "vn": ((), torch.float16)}
    qjl = c.use_qjl_keys
    spec.update(ks=((K.row_bytes(D, 1),), torch.uint8) if qjl else None, kr=((), torch.float16) if qjl else None)
    return spec


def _split_spec(sc: SplitCodecs) -> dict[str, tuple[tuple, torch.dtype] | None]:
    """Normal group: kc kn (ks kr) vc vn; outlier group: the same names with an 'o'."""
    spec = {}
    for sfx, kg, vg in (("", sc.key_normal, sc.value_normal), ("o", sc.key_outlier, sc.value_outlier)):
        spec["kc" + sfx] = ((K.row_bytes(kg.dim, kg.bits),), torch.uint8)
        spec["kn" + sfx] = ((), torch.float16)
        spec["ks" + sfx] = ((K.row_bytes(kg.dim, 1),), torch.uint8) if sc.use_qjl_keys else None
        spec["kr" + sfx] = ((), torch.float16) if sc.use_qjl_keys else None
        spec["vc" + sfx] = ((K.row_bytes(vg.dim, vg.bits),), torch.uint8)
        spec["vn" + sfx] = ((), torch.float16)
    return spec


class PackedMSELayer(CacheLayerMixin):
    """One decoder layer's TurboQuant-compressed KV cache."""

    is_sliding = False
    is_compileable = False

    def __init__(self, bits: int, seed: int = 0, grid_size: int = 32769, num_outlier_channels: int = 0,
                 outlier_extra_bits: int = 1, use_qjl_keys: bool = False, quantize_decode: bool = False,
                 reserve_tokens: int = DEFAULT_RESERVE_TOKENS):
        super().__init__()
        self.bits = bits
        self.seed = seed
        self.grid_size = grid_size
        self.num_outlier_channels = num_outlier_channels
        self.outlier_extra_bits = outlier_extra_bits
        self.use_qjl_keys = use_qjl_keys
        self.quantize_decode = quantize_decode
        self.reserve_tokens = reserve_tokens
        self.device: torch.device | None = None
        self.dtype: torch.dtype | None = None
        self.codecs: LayerCodecs | None = None  # unsplit layers
        self._split: SplitCodecs | None = None  # outlier-split layers
        self._store: _Store | None = None
        self._shape: tuple[int, int, int] | None = None  # (B, H, D)
        self._force_dense = False
        self._lazy_update = False
        self._dense_buf: tuple[torch.Tensor, torch.Tensor] | None = None  # capacity buffers [B, H, cap, D]
        self._dense_len = 0

    # ------------------------------------------------------------- parameters
    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Reference :237-283.  With 0 < num_outlier_channels < D the channels are split by
        the first K/V seen (the prefill) and every later token uses the same split."""
        self.dtype = key_states.dtype
        self.device = key_states.device
        D = int(key_states.shape[-1])
        if 0 < self.num_outlier_channels < D:
            outlier, normal = detect_outlier_channels(key_states, value_states, self.num_outlier_channels)
            self._split = split_codecs(normal.cpu().numpy(), outlier.cpu().numpy(), self.bits,
                                       self.outlier_extra_bits, self.seed, self.use_qjl_keys, self.device,
                                       self.grid_size)
        else:
            self.codecs = layer_codecs(D, self.bits, self.seed, self.use_qjl_keys, self.device, self.grid_size)
        self.is_initialized = True

    # reference-compatible parameter attributes (the normal group's on split layers)
    def _value_codec(self):
        return self._split.value_normal if self._split is not None else (self.codecs and self.codecs.value)

    def _key_codec(self):
        return self._split.key_normal if self._split is not None else (self.codecs and self.codecs.key)

    @property
    def rotation(self):
        c = self._value_codec()
        return None if c is None else c.rotation

    @property
    def centers(self):
        c = self._value_codec()
        return None if c is None else c.centers

    @property
    def boundaries(self):
        c = self._value_codec()
        return None if c is None else c.boundaries

    @property
    def _key_rotation(self):
        c = self._key_codec()
        return None if c is None else c.rotation

    @property
    def _key_centers(self):
        c = self._key_codec()
        return None if c is None else c.centers

    @property
    def _key_boundaries(self):
        c = self._key_codec()
        return None if c is None else c.boundaries

    @property
    def _qjl_matrix(self):
        if self._split is not None:
            return self._split.key_normal.qjl
        return None if self.codecs is None else self.codecs.qjl

    @property
    def _outlier_enabled(self) -> bool:
        return self._split is not None

    @property
    def _outlier_indices(self):
        return None if self._split is None else self._split.outlier_indices

    @property
    def _normal_indices(self):
        return None if self._split is None else self._split.normal_indices

    @property
    def _outlier_rotation(self):
        return None if self._split is None else self._split.value_outlier.rotation

    @property
    def _outlier_centers(self):
        return None if self._split is None else self._split.value_outlier.centers

    @property
    def _outlier_boundaries(self):
        return None if self._split is None else self._split.value_outlier.boundaries

    @property
    def _key_outlier_rotation(self):
        return self._split.key_outlier.rotation if self._split is not None and self.use_qjl_keys else None

    @property
    def _key_outlier_centers(self):
        return self._split.key_outlier.centers if self._split is not None and self.use_qjl_keys else None

    @property
    def _key_outlier_boundaries(self):
        return self._split.key_outlier.boundaries if self._split is not None and self.use_qjl_keys else None

    @property
    def _qjl_outlier_matrix(self):
        return None if self._split is None else self._split.key_outlier.qjl

    # ---------------------------------------------------------- packed views
    def packed_seq_length(self) -> int:
        return 0 if self._store is None else self._store.length

    def _packed(self, codes: str, norms: str, dim: int, bits: int) -> PackedTensorMSE | None:
        s = self._store
        if s is None:
            return None
        n = s.length
        B, H, _ = self._shape
        return PackedTensorMSE(getattr(s, codes)[:, :, :n], getattr(s, norms)[:, :, :n], (B, H, n, dim), self.dtype,
                               bits)

    def _qjl(self, signs: str, rnorms: str, dim: int) -> PackedQJL | None:
        s = self._store
        if s is None or not self.use_qjl_keys:
            return None
        n = s.length
        return PackedQJL(getattr(s, signs)[:, :, :n], getattr(s, rnorms)[:, :, :n], dim)

    @property
    def keys_packed(self) -> PackedTensorMSE | None:
        if self._split is not None:
            g = self._split.key_normal
            return self._packed("kc", "kn", g.dim, g.bits)
        return None if self._store is None else self._packed("kc", "kn", self._shape[2], self.codecs.key_bits)

    @property
    def values_packed(self) -> PackedTensorMSE | None:
        if self._split is not None:
            g = self._split.value_normal
            return self._packed("vc", "vn", g.dim, g.bits)
        return None if self._store is None else self._packed("vc", "vn", self._shape[2], self.codecs.value_bits)

    @property
    def _keys_qjl(self) -> PackedQJL | None:
        if self._store is None:
            return None
        dim = self._split.key_normal.dim if self._split is not None else self._shape[2]
        return self._qjl("ks", "kr", dim)

    @property
    def _keys_outlier(self) -> PackedTensorMSE | None:
        if self._split is None:
            return None
        g = self._split.key_outlier
        return self._packed("kco", "kno", g.dim, g.bits)

    @property
    def _values_outlier(self) -> PackedTensorMSE | None:
        if self._split is None:
            return None
        g = self._split.value_outlier
        return self._packed("vco", "vno", g.dim, g.bits)

    @property
    def _keys_outlier_qjl(self) -> PackedQJL | None:
        if self._split is None:
            return None
        return self._qjl("kso", "kro", self._split.key_outlier.dim)

    # --------------------------------------- reference-named kernel boundary
    # The reference's quantizer boundary (runtime/packed_qmse_cache.py:285-330, 376-435), with
    # its signatures and return types, each one libtq launch on the current stream.  Inputs
    # must be on the GPU with head_dim 128 (there is no CPU path); the decoders return bf16
    # rows (bf16((C[idx] R) n), plus the bf16 QJL correction for keys) cast to the packed
    # tensor's original dtype, which is the reference's result for bf16 models.
    @staticmethod
    def _encode_group(tensor: torch.Tensor, rotation: torch.Tensor, centers: torch.Tensor,
                      boundaries: torch.Tensor, bits: int) -> PackedTensorMSE:
        """Q_mse encoder: norms, rotation, bucketize and bit packing (reference :376-402)."""
        B, H, N, D = (int(v) for v in tensor.shape)
        codes = torch.empty(B, H, N, K.row_bytes(D, bits), dtype=torch.uint8, device=tensor.device)
        norms = torch.empty(B, H, N, dtype=torch.float16, device=tensor.device)
        K.quantize_mse(tensor, _codec_of(rotation, centers, boundaries, bits), codes, norms)
        return PackedTensorMSE(codes, norms, (B, H, N, D), tensor.dtype, int(bits))

    @staticmethod
    def _decode_group(packed: PackedTensorMSE, rotation: torch.Tensor, centers: torch.Tensor) -> torch.Tensor:
        """Q_mse decoder: (C[idx] @ R) * norm (reference :404-435)."""
        B, H, N, D = packed.original_shape
        out = K.dequantize_mse(_packed_rows(packed.packed_indices), _packed_rows(packed.norms), N,
                               _codec_of(rotation, centers, None, packed.bits), dim=D)
        return out.to(packed.original_dtype)

    def _encode_keys_qjl_group(self, key_states: torch.Tensor, rotation: torch.Tensor, centers: torch.Tensor,
                               boundaries: torch.Tensor, bits: int,
                               qjl_matrix: torch.Tensor) -> tuple[PackedTensorMSE, PackedQJL]:
        """Q_prod key encoder: (bits)-bit Q_mse codes plus the QJL sign sketch of the residual
        (reference :285-310)."""
        B, H, N, D = (int(v) for v in key_states.shape)
        dev = key_states.device
        codes = torch.empty(B, H, N, K.row_bytes(D, bits), dtype=torch.uint8, device=dev)
        norms = torch.empty(B, H, N, dtype=torch.float16, device=dev)
        signs = torch.empty(B, H, N, K.row_bytes(D, 1), dtype=torch.uint8, device=dev)
        rnorms = torch.empty(B, H, N, dtype=torch.float16, device=dev)
        S = qjl_matrix if qjl_matrix.dtype == torch.float32 and qjl_matrix.is_contiguous() else \
            qjl_matrix.float().contiguous()
        K.quantize_prod(key_states, _codec_of(rotation, centers, boundaries, bits), S, codes, norms, signs, rnorms)
        return (PackedTensorMSE(codes, norms, (B, H, N, D), key_states.dtype, int(bits)),
                PackedQJL(signs, rnorms, D))

    def _decode_keys_qjl_group(self, mse_packed: PackedTensorMSE, qjl: PackedQJL, rotation: torch.Tensor,
                               centers: torch.Tensor, qjl_matrix: torch.Tensor) -> torch.Tensor:
        """Q_prod key decoder: MSE reconstruction plus QJL correction (reference :312-330)."""
        B, H, N, D = mse_packed.original_shape
        S = qjl_matrix if qjl_matrix.dtype == torch.float32 and qjl_matrix.is_contiguous() else \
            qjl_matrix.float().contiguous()
        out = K.dequantize_prod(_packed_rows(mse_packed.packed_indices), _packed_rows(mse_packed.norms),
                                _packed_rows(qjl.packed_signs), _packed_rows(qjl.residual_norms), N,
                                _codec_of(rotation, centers, None, mse_packed.bits), S, dim=D)
        return out.to(mse_packed.original_dtype)

    # ------------------------------------------------------------- encoding
    def initialize_from_dense(self, key_states: torch.Tensor, value_states: torch.Tensor, *,
                              force_dense: bool = False) -> None:
        """Prefill: compress the whole dense K/V (reference :332-374)."""
        if force_dense:
            self.device, self.dtype = key_states.device, key_states.dtype
            self._append_dense(key_states, value_states)
            self._force_dense = True
            self.is_initialized = True
            return
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self._append_packed(key_states, value_states)

    def _append_packed(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Encode [B, H, T, D] keys / values into slots [N, N + T) of the capacity buffers."""
        B, H, T, D = (int(v) for v in key_states.shape)
        if self._store is None:
            self._shape = (B, H, D)
            spec = _split_spec(self._split) if self._split is not None else _flat_spec(D, self.codecs)
            self._store = _Store(B, H, max(T + self.reserve_tokens, 1), key_states.device, spec)
        elif (B, H, D) != self._shape:
            raise ValueError(f"append of shape {tuple(key_states.shape)} to a cache of {self._shape}")
        s = self._store
        s.reserve(T, self.reserve_tokens)
        off = s.length
        if self._split is not None:
            sc = self._split
            qjl = sc.use_qjl_keys
            for sfx, kg, vg in (("", sc.key_normal, sc.value_normal), ("o", sc.key_outlier, sc.value_outlier)):
                K.quantize_group(key_states, kg, getattr(s, "kc" + sfx), getattr(s, "kn" + sfx),
                                 getattr(s, "ks" + sfx) if qjl else None, getattr(s, "kr" + sfx) if qjl else None,
                                 offset=off)
                K.quantize_group(value_states, vg, getattr(s, "vc" + sfx), getattr(s, "vn" + sfx), offset=off)
        else:
            c = self.codecs
            if c.use_qjl_keys:
                K.quantize_prod(key_states, c.key, c.qjl, s.kc, s.kn, s.ks, s.kr, offset=off)
            else:
                K.quantize_mse(key_states, c.key, s.kc, s.kn, offset=off)
            K.quantize_mse(value_states, c.value, s.vc, s.vn, offset=off)
        s.length += T

    # ------------------------------------------------------------- decoding
    def _decode_split(self, pre: str, normal, outlier, start: int, end: int) -> torch.Tensor:
        """Both channel groups of slots [start, end) decoded into one [B, H, end - start, D]
        bf16 tensor (reference _decode_merge / _decode_keys_merge_qjl, :456-515)."""
        s = self._store
        B, H, D = self._shape
        out = torch.empty(B, H, end - start, D, dtype=torch.bfloat16, device=s.device)
        qjl = pre == "k" and self.use_qjl_keys
        for sfx, g, merge in (("", normal, False), ("o", outlier, True)):
            K.dequantize_group(getattr(s, pre + "c" + sfx), getattr(s, pre + "n" + sfx), end - start, g, out, merge,
                               signs=getattr(s, "ks" + sfx) if qjl else None,
                               rnorms=getattr(s, "kr" + sfx) if qjl else None, start=start)
        return out

    def _decode_keys_range(self, start: int, end: int) -> torch.Tensor:
        """Keys of packed positions [start, end) (reference :564-584)."""
        s = self._store
        if self._split is not None:
            return self._decode_split("k", self._split.key_normal, self._split.key_outlier, start, end).to(self.dtype)
        c = self.codecs
        if c.use_qjl_keys:
            return K.dequantize_prod(s.kc, s.kn, s.ks, s.kr, end - start, c.key, c.qjl, start=start).to(self.dtype)
        return K.dequantize_mse(s.kc, s.kn, end - start, c.key, start=start).to(self.dtype)

    def _decode_values_range(self, start: int, end: int) -> torch.Tensor:
        """Values of packed positions [start, end) (reference :586-592)."""
        s = self._store
        if self._split is not None:
            return self._decode_split("v", self._split.value_normal, self._split.value_outlier, start,
                                      end).to(self.dtype)
        return K.dequantize_mse(s.vc, s.vn, end - start, self.codecs.value, start=start).to(self.dtype)

    def _decode_keys_full(self) -> torch.Tensor | None:
        return None if self._store is None else self._decode_keys_range(0, self._store.length)

    def _decode_values_full(self) -> torch.Tensor | None:
        return None if self._store is None else self._decode_values_range(0, self._store.length)

    # ------------------------------------------------------------ HF protocol
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args: Any,
               **kwargs: Any) -> tuple[torch.Tensor, torch.Tensor]:
        """Reference :600-624.  With the TurboQuant attention backend wired
        (``_lazy_update``) only the new token is stored and returned; otherwise
        the decoded history plus the new tokens is returned for dense attention."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if self._lazy_update and not self._force_dense:
            return self._update_lazy(key_states, value_states)
        if self._force_dense or not self.quantize_decode:
            return self._update_dense_decode(key_states, value_states)
        prev_k = self._decode_keys_full()
        prev_v = self._decode_values_full()
        self._append_packed(key_states, value_states)
        if prev_k is None:
            return key_states, value_states
        return torch.cat((prev_k, key_states), dim=-2), torch.cat((prev_v, value_states), dim=-2)

    def _update_lazy(self, key_states: torch.Tensor, value_states: torch.Tensor):
        """Reference :626-679: store the new token without touching the history."""
        if self.quantize_decode:
            self._append_packed(key_states, value_states)
        else:
            self._append_dense(key_states, value_states)
        return key_states, value_states

    @property
    def _dense_keys(self) -> torch.Tensor | None:
        """Tokens kept dense (reference attribute): a [:, :, :n] view of the capacity buffer."""
        return None if self._dense_buf is None else self._dense_buf[0][:, :, :self._dense_len]

    @property
    def _dense_values(self) -> torch.Tensor | None:
        return None if self._dense_buf is None else self._dense_buf[1][:, :, :self._dense_len]

    def _append_dense(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """Append [B, H, T, D] tokens to the dense buffers in place (the reference concatenates
        the whole history each step, runtime/packed_qmse_cache.py:670-677, 695-702)."""
        T = int(key_states.shape[-2])
        n = self._dense_len
        if self._dense_buf is None or n + T > self._dense_buf[0].shape[2]:
            cap = max(n + T + self.reserve_tokens, 2 * (0 if self._dense_buf is None else self._dense_buf[0].shape[2]))
            new = tuple(torch.empty(*x.shape[:2], cap, x.shape[3], dtype=x.dtype, device=x.device)
                        for x in (key_states, value_states))
            if self._dense_buf is not None and n:
                for dst, src in zip(new, self._dense_buf):
                    dst[:, :, :n].copy_(src[:, :, :n])
            self._dense_buf = new
        self._dense_buf[0][:, :, n:n + T].copy_(key_states)
        self._dense_buf[1][:, :, n:n + T].copy_(value_states)
        self._dense_len = n + T

    def _update_dense_decode(self, key_states: torch.Tensor, value_states: torch.Tensor):
        """Reference :681-705: generated tokens stay dense; history is decoded."""
        pk, pv = self._decode_keys_full(), self._decode_values_full()
        self._append_dense(key_states, value_states)
        if pk is None:  # nothing packed (norm-guarded layer): the dense buffers themselves
            return self._dense_keys, self._dense_values
        return torch.cat((pk, self._dense_keys), dim=-2), torch.cat((pv, self._dense_values), dim=-2)

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        if torch.is_tensor(query_length):  # older callers pass cache_position
            query_length = int(query_length.shape[0])
        return self.get_seq_length() + int(query_length), 0

    def get_seq_length(self) -> int:
        dense = 0 if self._dense_keys is None else int(self._dense_keys.shape[-2])
        return self.packed_seq_length() + dense

    def get_max_length(self) -> int:
        return -1

    def get_max_cache_shape(self) -> int:
        return -1

    def storage_bytes(self) -> int:
        """Logical storage (N valid tokens, as the reference counts it; :874-885)."""
        total = 0
        for p in (self.keys_packed, self.values_packed, self._keys_qjl, self._keys_outlier, self._values_outlier,
                  self._keys_outlier_qjl):
            if p is not None:
                total += p.storage_bytes()
        for d in (self._dense_keys, self._dense_values):
            if d is not None:
                total += d.numel() * d.element_size()
        return int(total)


_APPROX_DMSE_UNIT: dict[int, float] = {2: 0.079, 3: 0.030, 4: 0.009, 5: 0.003, 6: 0.0008, 7: 0.0002, 8: 0.00005}


def _auto_norm_threshold(bits: int, head_dim: int, mse_budget: float = 1.0) -> float:
    """Largest mean key norm a layer may have before the norm guard keeps it dense
    (reference :888-900): norm^2 * D_mse(bits) / D < budget."""
    return sqrt(mse_budget * head_dim / _APPROX_DMSE_UNIT.get(bits, 0.03))


def _layer_kv(past_key_values):
    if hasattr(past_key_values, "layers"):
        return [(layer.keys, layer.values) for layer in past_key_values.layers]
    return [(k, v) for k, v, *_ in past_key_values]


def build_packed_mse_cache(past_key_values, bits: int, seed: int = 0, grid_size: int = 32769,
                           num_outlier_channels: int = 0, outlier_extra_bits: int = 1, use_qjl_keys: bool = False,
                           quantize_decode: bool = False, norm_guard: bool = True,
                           reserve_tokens: int = DEFAULT_RESERVE_TOKENS) -> Cache:
    """Compress a prefilled dense cache layer by layer (reference :903-951)."""
    data = _layer_kv(past_key_values)
    if not data:
        return Cache(layers=[])
    # one host sync for all layers' mean key norms (reference: one .item() per layer)
    norms = torch.stack([k.float().norm(dim=-1).mean().to(data[0][0].device) for k, _ in data]).tolist()
    head_dim = int(data[0][0].shape[-1])
    threshold = _auto_norm_threshold(bits, head_dim) if norm_guard else float("inf")
    layers = []
    for (k, v), n in zip(data, norms):
        layer = PackedMSELayer(bits=bits, seed=seed, grid_size=grid_size, num_outlier_channels=num_outlier_channels,
                               outlier_extra_bits=outlier_extra_bits, use_qjl_keys=use_qjl_keys,
                               quantize_decode=quantize_decode, reserve_tokens=reserve_tokens)
        layer.initialize_from_dense(k, v, force_dense=n > threshold)
        layers.append(layer)
    dense_ids = [i for i, n in enumerate(norms) if n > threshold]
    if dense_ids:
        print(f"[TurboQuant] norm_guard: {len(dense_ids)}/{len(layers)} layers kept dense "
              f"(threshold={threshold:.1f}, layers={dense_ids})", file=sys.stderr)
    return Cache(layers=layers)


def verify_packed_reconstruction(original_cache, packed_cache: Cache) -> list[dict[str, Any]]:
    """Per-layer reconstruction quality of the packed cache (reference :954-1009)."""
    out: list[dict[str, Any]] = []
    for idx, (ko, vo) in enumerate(_layer_kv(original_cache)):
        layer: PackedMSELayer = packed_cache.layers[idx]
        kr, vr = layer._decode_keys_full(), layer._decode_values_full()
        dense = kr is None and layer._dense_keys is not None
        if dense:
            kr, vr = layer._dense_keys, layer._dense_values
        ko32, kr32, vo32, vr32 = ko.float(), kr.float(), vo.float(), vr.float()
        ke, ve = ko32 - kr32, vo32 - vr32
        D = ko32.shape[-1]
        stats = torch.stack([
            (ke ** 2).mean(),
            torch.nn.functional.cosine_similarity(ko32.reshape(-1, D), kr32.reshape(-1, D), dim=-1).mean(),
            ke.abs().max(),
            ko32.norm(dim=-1).mean(),
            (ve ** 2).mean(),
            torch.nn.functional.cosine_similarity(vo32.reshape(-1, D), vr32.reshape(-1, D), dim=-1).mean(),
            ve.abs().max(),
            vo32.norm(dim=-1).mean(),
        ]).tolist()
        out.append({
            "layer": idx, "dense": dense,
            "key_mse": round(stats[0], 6), "key_cosine_sim": round(stats[1], 6),
            "key_max_abs_error": round(stats[2], 6), "key_mean_norm": round(stats[3], 4),
            "val_mse": round(stats[4], 6), "val_cosine_sim": round(stats[5], 6),
            "val_max_abs_error": round(stats[6], 6), "val_mean_norm": round(stats[7], 4),
        })
    return out


def packed_cache_storage_bytes(cache: Cache) -> int:
    return sum(int(layer.storage_bytes()) for layer in cache.layers if hasattr(layer, "storage_bytes"))


def packed_cache_storage_breakdown(cache: Cache) -> dict[str, int]:
    sizes = [int(layer.storage_bytes()) for layer in cache.layers if hasattr(layer, "storage_bytes")]
    return {
        "packed_total_bytes": int(sum(sizes)),
        "packed_layer_mean_bytes": int(sum(sizes) / len(sizes)) if sizes else 0,
        "packed_num_layers": len(sizes),
    }
