"""Torch-facing wrappers of the libtq C ABI (PyTorch-ROCm supplies memory and streams).

Every function validates dtype / shape / device on the host, then makes one
C-ABI call on ``torch.cuda.current_stream()``.  There is no CPU path: a CPU
tensor, or a missing libtq.so, raises.

Reference interfaces replaced:
  quantize_mse   -> PackedMSELayer._encode_group           runtime/packed_qmse_cache.py:376-402
  quantize_prod  -> PackedMSELayer._encode_keys_qjl_group  runtime/packed_qmse_cache.py:285-310
  dequantize_mse -> PackedMSELayer._decode_group           runtime/packed_qmse_cache.py:404-435
  decode_attention -> fused_attention                      runtime/triton_kernels.py:238-368
  quantize_group -> PackedMSELayer._encode_split / _encode_keys_split_qjl (one channel group)
                                                           runtime/packed_qmse_cache.py:481-496, 437-454
  dequantize_group -> PackedMSELayer._decode_merge / _decode_keys_merge_qjl (one channel group)
                                                           runtime/packed_qmse_cache.py:498-515, 456-479
  decode_attention_groups -> the reference's attention over outlier-split layers, which its
                    fused kernel refuses (runtime/triton_kernels.py:252-253) and its chunked
                    path dequantises (runtime/attention.py:215-304)
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from turboquant.runtime import _lib

HEAD_DIM = 128
MAX_GROUP = 8  # query heads per KV head the decode-attention kernels take (TQ_MAX_GROUP)


def _vp(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _at_slot(t: torch.Tensor | None, start: int):
    """Pointer to token slot ``start`` of a [B, H, cap, ...] buffer (the group stride stays cap)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr() + start * t.stride(2) * t.element_size())


#: the current stream's handle as an int: torch's raw accessor is one C call, where
#: torch.cuda.current_stream() builds a Stream object (~2 us per call)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _stream(device: torch.device):
    return ctypes.c_void_p(_stream_handle(device))


def _require_gpu(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"TurboQuant kernels run on the GPU only (libtq, gfx950); got a tensor on {t.device}"
            )


def row_bytes(dim: int, bits: int) -> int:
    return (dim * bits + 7) // 8


@dataclass
class CodecParams:
    """Device-resident parameters of one Q_mse codec (rotation, codebook).

    ``attn_centers`` caches the codebook's fp16 form for the decode attention's value sums
    (``attention_value_centers``).
    """

    bits: int
    rotation: torch.Tensor  # fp32 [D, D]
    centers: torch.Tensor  # fp32 [2^bits]
    boundaries: torch.Tensor  # fp32 [2^bits - 1]
    attn_centers: torch.Tensor | None = None  # fp32 [2^bits], fp16-exact values


@dataclass
class GroupCodec:
    """Device-resident codec of one channel group (the outlier-channel split).

    ``rotation`` / ``qjl`` are the group's own d x d matrices (the reference's
    attributes); ``rotation_ch`` / ``qjl_ch`` are the same matrices in channel
    space (``group_matrix``), which is what libtq takes.  ``qjl`` is set only for
    Q_prod key groups.  ``attn_centers`` caches a value group's fp16 codebook for the
    decode attention (``attention_value_centers``).
    """

    channels: np.ndarray  # int32 [d], host, strictly ascending
    bits: int
    rotation: torch.Tensor  # fp32 [d, d]
    centers: torch.Tensor  # fp32 [2^bits]
    boundaries: torch.Tensor  # fp32 [2^bits - 1]
    rotation_ch: torch.Tensor  # fp32 [D, D]
    qjl: torch.Tensor | None = None  # fp32 [d, d]
    qjl_ch: torch.Tensor | None = None  # fp32 [D, D]
    attn_centers: torch.Tensor | None = None  # fp32 [2^bits], fp16-exact values

    @property
    def dim(self) -> int:
        return int(self.channels.shape[0])


def group_matrix(sub: np.ndarray, channels: np.ndarray, dim: int = HEAD_DIM) -> np.ndarray:
    """Channel-space form of a group's d x d matrix (host): out[j, channels[i]] = sub[j, i]."""
    sub = np.ascontiguousarray(sub, dtype=np.float32)
    ch = np.ascontiguousarray(channels, dtype=np.int32)
    if sub.shape != (ch.size, ch.size):
        raise ValueError(f"group matrix {sub.shape} does not match {ch.size} channels")
    out = np.empty((dim, dim), np.float32)
    _lib.call("tq_group_matrix", sub.ctypes.data, ch.size, ch.ctypes.data, dim, out.ctypes.data)
    return out


def _as_encoder_input(x: torch.Tensor) -> torch.Tensor:
    if x.dim() != 4:
        raise ValueError(f"expected [batch, heads, tokens, dim], got {tuple(x.shape)}")
    if x.shape[-1] != HEAD_DIM:
        raise ValueError(f"head_dim {x.shape[-1]} unsupported (kernels are built for {HEAD_DIM})")
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    aligned = x.stride(-1) == 1 and all(s % 8 == 0 for s in x.stride()[:3]) and x.data_ptr() % 16 == 0
    return x if aligned else x.contiguous()


def quantize_mse(x: torch.Tensor, codec: CodecParams, codes: torch.Tensor, norms: torch.Tensor,
                 offset: int = 0) -> None:
    """Encode x [B,H,T,D] into codes [B,H,cap,row] / norms [B,H,cap] at token slot ``offset``."""
    x = _as_encoder_input(x)
    _require_gpu(x, codes, norms, codec.rotation)
    B, H, T, D = x.shape
    cap = codes.shape[2]
    if codes.shape != (B, H, cap, row_bytes(D, codec.bits)) or codes.dtype != torch.uint8 or not codes.is_contiguous():
        raise ValueError(f"codes buffer {tuple(codes.shape)} {codes.dtype} does not match {B, H, cap}")
    if norms.shape != (B, H, cap) or norms.dtype != torch.float16 or not norms.is_contiguous():
        raise ValueError("norms buffer must be contiguous float16 [B, H, cap]")
    _lib.call("tq_quantize_mse", _vp(x), B, H, T, D, x.stride(0), x.stride(1), x.stride(2), codec.bits,
              _vp(codec.rotation), _vp(codec.boundaries), _vp(codes), _vp(norms), cap, offset, _stream(x.device))


def quantize_prod(x: torch.Tensor, codec: CodecParams, qjl: torch.Tensor, codes: torch.Tensor,
                  norms: torch.Tensor, signs: torch.Tensor, rnorms: torch.Tensor, offset: int = 0) -> None:
    """Q_prod keys: (codec.bits)-bit MSE codes + 1-bit QJL signs of the residual, at slot ``offset``."""
    x = _as_encoder_input(x)
    _require_gpu(x, codes, norms, signs, rnorms, qjl)
    B, H, T, D = x.shape
    cap = codes.shape[2]
    if codes.shape != (B, H, cap, row_bytes(D, codec.bits)) or not codes.is_contiguous():
        raise ValueError("codes buffer shape mismatch")
    if signs.shape != (B, H, cap, D // 8) or not signs.is_contiguous():
        raise ValueError("signs buffer shape mismatch")
    for t in (norms, rnorms):
        if t.shape != (B, H, cap) or t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError("norm buffers must be contiguous float16 [B, H, cap]")
    _lib.call("tq_quantize_prod", _vp(x), B, H, T, D, x.stride(0), x.stride(1), x.stride(2), codec.bits,
              _vp(codec.rotation), _vp(codec.centers), _vp(codec.boundaries), _vp(qjl), _vp(codes), _vp(norms),
              _vp(signs), _vp(rnorms), cap, offset, _stream(x.device))


def quantize_group(x: torch.Tensor, g: GroupCodec, codes: torch.Tensor, norms: torch.Tensor,
                   signs: torch.Tensor | None = None, rnorms: torch.Tensor | None = None, offset: int = 0) -> None:
    """Encode channel group ``g`` of x [B,H,T,D] at token slot ``offset``: Q_mse codes,
    plus the QJL sketch when ``g`` is a Q_prod key group (``signs`` / ``rnorms`` then required).
    codes [B,H,cap,ceil(d*bits/8)], norms / rnorms [B,H,cap], signs [B,H,cap,ceil(d/8)]."""
    x = _as_encoder_input(x)
    prod = g.qjl_ch is not None
    _require_gpu(x, codes, norms, signs, rnorms, g.rotation_ch)
    B, H, T, D = x.shape
    cap = codes.shape[2]
    if codes.shape != (B, H, cap, row_bytes(g.dim, g.bits)) or codes.dtype != torch.uint8 or not codes.is_contiguous():
        raise ValueError(f"codes buffer {tuple(codes.shape)} does not match group ({g.dim} channels, {g.bits} bits)")
    if prod:
        if signs is None or rnorms is None:
            raise ValueError("a Q_prod key group needs signs and rnorms buffers")
        if signs.shape != (B, H, cap, row_bytes(g.dim, 1)) or not signs.is_contiguous():
            raise ValueError("signs buffer shape mismatch")
    for t in (norms, rnorms if prod else None):
        if t is not None and (t.shape != (B, H, cap) or t.dtype != torch.float16 or not t.is_contiguous()):
            raise ValueError("norm buffers must be contiguous float16 [B, H, cap]")
    _lib.call("tq_quantize_group", _vp(x), B, H, T, D, x.stride(0), x.stride(1), x.stride(2), g.channels.ctypes.data,
              g.dim, g.bits, _vp(g.rotation_ch), _vp(g.centers), _vp(g.boundaries), _vp(g.qjl_ch), _vp(codes),
              _vp(norms), _vp(signs if prod else None), _vp(rnorms if prod else None), cap, offset, _stream(x.device))


def dequantize_group(codes: torch.Tensor, norms: torch.Tensor, tokens: int, g: GroupCodec, out: torch.Tensor,
                     merge: bool, signs: torch.Tensor | None = None, rnorms: torch.Tensor | None = None,
                     start: int = 0) -> None:
    """Decode channel group ``g`` of slots [start, start + tokens) of codes [B,H,cap,row] into
    out bf16 [B,H,tokens,D] (its channels; the others are zeroed, or kept when ``merge``).
    QJL-corrected when ``g`` is a Q_prod key group."""
    _require_gpu(codes, norms, out, signs, rnorms)
    B, H, cap, _ = codes.shape
    qjl = g.qjl_ch is not None
    if qjl and (signs is None or rnorms is None):
        raise ValueError("a Q_prod key group needs its signs and rnorms")
    if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.shape[:3] != (B, H, tokens):
        raise ValueError("out must be a contiguous bf16 [B, H, tokens, D] tensor")
    if start < 0 or start + tokens > cap:
        raise ValueError(f"slots [{start}, {start + tokens}) outside the capacity {cap}")
    _lib.call("tq_dequantize_group", _at_slot(codes, start), _at_slot(norms, start),
              _at_slot(signs if qjl else None, start), _at_slot(rnorms if qjl else None, start), B * H, tokens,
              cap, out.shape[-1], g.channels.ctypes.data, g.dim,
              g.bits, _vp(g.rotation_ch), _vp(g.centers), _vp(g.qjl_ch), int(bool(merge)), _vp(out),
              _stream(codes.device))


def dequantize_mse(codes: torch.Tensor, norms: torch.Tensor, tokens: int, codec: CodecParams,
                   dim: int = HEAD_DIM, start: int = 0) -> torch.Tensor:
    """Slots [start, start + tokens) of codes [B,H,cap,row] -> bf16 [B,H,tokens,D] =
    bf16((C[codes] @ R) * norm)."""
    _require_gpu(codes, norms)
    B, H, cap, _ = codes.shape
    if start < 0 or start + tokens > cap:
        raise ValueError(f"slots [{start}, {start + tokens}) outside the capacity {cap}")
    out = torch.empty(B, H, tokens, dim, dtype=torch.bfloat16, device=codes.device)
    _lib.call("tq_dequantize_mse", _at_slot(codes, start), _at_slot(norms, start), B * H, tokens, cap, dim, codec.bits,
              _vp(codec.rotation), _vp(codec.centers), _vp(out), _stream(codes.device))
    return out


def dequantize_prod(codes: torch.Tensor, norms: torch.Tensor, signs: torch.Tensor, rnorms: torch.Tensor,
                    tokens: int, codec: CodecParams, qjl: torch.Tensor, dim: int = HEAD_DIM,
                    start: int = 0) -> torch.Tensor:
    """Slots [start, start + tokens) of Q_prod keys [B,H,cap,...] -> bf16 [B,H,tokens,D]:
    MSE reconstruction + QJL correction."""
    _require_gpu(codes, norms, signs, rnorms)
    B, H, cap, _ = codes.shape
    if start < 0 or start + tokens > cap:
        raise ValueError(f"slots [{start}, {start + tokens}) outside the capacity {cap}")
    out = torch.empty(B, H, tokens, dim, dtype=torch.bfloat16, device=codes.device)
    _lib.call("tq_dequantize_prod", _at_slot(codes, start), _at_slot(norms, start), _at_slot(signs, start),
              _at_slot(rnorms, start), B * H, tokens, cap, dim,
              codec.bits, _vp(codec.rotation), _vp(codec.centers), _vp(qjl), _vp(out), _stream(codes.device))
    return out


#: attention workspace (the split partials) per (device, stream):
#: calls on one stream are ordered, so they can share one; calls on two streams get two
_workspaces: dict[tuple, torch.Tensor] = {}
#: workspaces replaced by a larger one stay allocated: a HIP graph that captured a call keeps
#: the old pointer and may be replayed later
_retired: list[torch.Tensor] = []
_ws_bytes: dict[tuple, int] = {}


def _workspace_for(device: torch.device, stream: int, batch: int, q_heads: int, kv_heads: int) -> torch.Tensor:
    shape = (batch, q_heads, kv_heads)
    need = _ws_bytes.get(shape)
    if need is None:
        # sized for any token count (the split count is bounded by the workgroup cap)
        need = int(_lib.load().tq_decode_attention_workspace_bytes(batch, q_heads, kv_heads, HEAD_DIM, 1))
        if need == 0:
            raise ValueError("invalid attention shape for workspace sizing")
        _ws_bytes[shape] = need
    key = (device.index, stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _retired.append(ws)
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def attention_workspace(device: torch.device, batch: int, q_heads: int, kv_heads: int, max_tokens: int) -> torch.Tensor:
    """The partials workspace of ``tq_decode_attention`` for the current stream of ``device``."""
    return _workspace_for(device, _stream_handle(device), batch, q_heads, kv_heads)


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def value_codebook_f16(centers: np.ndarray, bits: int, dim: int = HEAD_DIM) -> np.ndarray:
    """The fp16 value codebook of tq_decode_attention (host; tq_value_codebook_f16): each
    centroid's fp16 neighbour below or above, chosen so that the rounding errors cancel
    over the codes' probabilities instead of adding up over long contexts."""
    c = np.ascontiguousarray(centers, dtype=np.float32)
    if c.shape != (1 << bits,):
        raise ValueError(f"expected {1 << bits} centers for {bits} bits, got {c.shape}")
    out = np.empty_like(c)
    _lib.call("tq_value_codebook_f16", c.ctypes.data, bits, dim, out.ctypes.data)
    return out


def attention_value_centers(codec: CodecParams | GroupCodec) -> torch.Tensor:
    """The value codebook tq_decode_attention is given: ``value_codebook_f16`` of the
    codec's centers (at the group's dimension for a channel group), on the codec's
    device, computed once per codec."""
    if codec.attn_centers is None:
        dim = codec.dim if isinstance(codec, GroupCodec) else HEAD_DIM
        host = value_codebook_f16(codec.centers.detach().cpu().numpy(), codec.bits, dim)
        codec.attn_centers = torch.from_numpy(host).to(codec.centers.device)
    return codec.attn_centers


def decode_attention(q: torch.Tensor, *, k_codes: torch.Tensor, k_norms: torch.Tensor, v_codes: torch.Tensor,
                     v_norms: torch.Tensor, n_tokens: int, key: CodecParams, value: CodecParams,
                     k_signs: torch.Tensor | None = None, k_rnorms: torch.Tensor | None = None,
                     qjl: torch.Tensor | None = None, seq_lens: torch.Tensor | None = None,
                     seq_starts: torch.Tensor | None = None, scale: float | None = None,
                     want_f32: bool = False, want_lse: bool = False):
    """Fused decode attention for one query token per sequence.

    q: [B, Hq, D] or [B, Hq, 1, D] (any float dtype; bf16 is passed through).
    Packed buffers are [B, Hkv, cap, ...] with ``n_tokens`` valid slots; row b
    attends to slots [seq_starts[b], seq_lens[b]) when those are given.
    Returns bf16 [B, Hq, D], then fp32 [B, Hq, D] if ``want_f32`` and the fp32
    log-sum-exp [B, Hq] of the scaled logits if ``want_lse``.

    This runs once per layer and decode step, so the host path is kept short: one
    stream lookup, plain integer pointers into the ctypes call, no copies of inputs
    that are already bf16 and contiguous.
    """
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise ValueError("decode_attention takes exactly one query token per sequence")
        q = q[:, :, 0, :]
    if q.dtype != torch.bfloat16:
        q = q.to(torch.bfloat16)
    if not q.is_contiguous() or q.data_ptr() % 16:
        q = q.contiguous() if q.data_ptr() % 16 == 0 else q.clone(memory_format=torch.contiguous_format)
    if not (q.is_cuda and k_codes.is_cuda and v_codes.is_cuda):
        _require_gpu(q, k_codes, v_codes)
    B, Hq, D = q.shape
    Hkv, cap = k_codes.shape[1], k_codes.shape[2]
    dev = q.device
    stream = _stream_handle(dev)
    out_bf16 = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=dev)
    out_f32 = torch.empty((B, Hq, D), dtype=torch.float32, device=dev) if want_f32 else None
    lse = torch.empty((B, Hq), dtype=torch.float32, device=dev) if want_lse else None
    ws = _workspace_for(dev, stream, B, Hq, Hkv)
    if seq_lens is not None and (seq_lens.dtype != torch.int32 or seq_lens.device != dev
                                 or not seq_lens.is_contiguous()):
        seq_lens = seq_lens.to(device=dev, dtype=torch.int32).contiguous()
    if seq_starts is not None and (seq_starts.dtype != torch.int32 or seq_starts.device != dev
                                   or not seq_starts.is_contiguous()):
        seq_starts = seq_starts.to(device=dev, dtype=torch.int32).contiguous()
    s = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    fn = _lib.load().tq_decode_attention
    st = fn(q.data_ptr(), B, Hq, Hkv, D, _ptr(seq_starts), _ptr(seq_lens), int(n_tokens), cap,
            k_codes.data_ptr(), k_norms.data_ptr(), _ptr(k_signs), _ptr(k_rnorms), v_codes.data_ptr(),
            v_norms.data_ptr(), key.bits, value.bits, int(k_signs is not None), key.rotation.data_ptr(),
            key.centers.data_ptr(), _ptr(qjl), value.rotation.data_ptr(), attention_value_centers(value).data_ptr(), s,
            _ptr(out_f32), out_bf16.data_ptr(), _ptr(lse), ws.data_ptr(), ws.numel(), stream)
    if st != _lib.TQ_OK:
        _lib.check("tq_decode_attention", st)
    if want_f32:
        return (out_bf16, out_f32, lse) if want_lse else (out_bf16, out_f32)
    return (out_bf16, lse) if want_lse else out_bf16


def decode_attention_groups(q: torch.Tensor, groups: list[dict], *, n_tokens: int, key_stack: torch.Tensor,
                            value_stack: torch.Tensor, qjl_stack: torch.Tensor | None = None,
                            seq_lens: torch.Tensor | None = None, seq_starts: torch.Tensor | None = None,
                            scale: float | None = None, want_f32: bool = False, want_lse: bool = False):
    """Fused decode attention over a layer quantized in channel groups (the outlier split).

    ``groups``: per group a dict with ``key`` / ``value`` (GroupCodec), ``k_codes``,
    ``k_norms``, ``v_codes``, ``v_norms`` and, with QJL, ``k_signs`` / ``k_rnorms``, each
    [B, Hkv, cap, ...].  ``key_stack`` / ``value_stack`` / ``qjl_stack`` are the groups'
    channel-space matrices stacked into D x D.  Returns as ``decode_attention``.
    """
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise ValueError("decode_attention_groups takes exactly one query token per sequence")
        q = q[:, :, 0, :]
    q = q.to(torch.bfloat16).contiguous()
    if q.data_ptr() % 16:  # a view at an odd storage offset: the kernels read q 16 bytes at a time
        q = q.clone()
    first = groups[0]
    _require_gpu(q, first["k_codes"], first["v_codes"], key_stack, value_stack)
    B, Hq, D = q.shape
    Hkv, cap = first["k_codes"].shape[1], first["k_codes"].shape[2]
    has_qjl = qjl_stack is not None
    n = len(groups)

    def arr(ctype, values):
        return (ctype * n)(*values)

    P = ctypes.c_void_p
    keep = []  # ctypes arrays must outlive the call
    for g in groups:
        for name in ("k_codes", "k_norms", "v_codes", "v_norms") + (("k_signs", "k_rnorms") if has_qjl else ()):
            t = g[name]
            if t.shape[:3] != (B, Hkv, cap) or not t.is_contiguous():
                raise ValueError(f"{name}: expected a contiguous [B, Hkv, cap, ...] buffer, got {tuple(t.shape)}")
    dims = arr(ctypes.c_int, [g["key"].dim for g in groups])
    kbits = arr(ctypes.c_int, [g["key"].bits for g in groups])
    vbits = arr(ctypes.c_int, [g["value"].bits for g in groups])
    ptr = lambda name: arr(P, [g[name].data_ptr() if g.get(name) is not None else None for g in groups])  # noqa: E731
    kc, kn, vc, vn = ptr("k_codes"), ptr("k_norms"), ptr("v_codes"), ptr("v_norms")
    ks = ptr("k_signs") if has_qjl else None
    kr = ptr("k_rnorms") if has_qjl else None
    ck = arr(P, [g["key"].centers.data_ptr() for g in groups])
    # with two groups the normal group's value sums may run in fp16 on the matrix cores: its
    # codebook goes in the fp16 form that keeps long-context sums unbiased
    vcen = [g["value"].centers for g in groups]
    if n == 2 and groups[0]["value"].bits <= 4:
        vcen[0] = attention_value_centers(groups[0]["value"])
    cv = arr(P, [c.data_ptr() for c in vcen])
    keep += [dims, kbits, vbits, kc, kn, vc, vn, ks, kr, ck, cv]
    out_bf16 = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=q.device)
    out_f32 = torch.empty(B, Hq, D, dtype=torch.float32, device=q.device) if want_f32 else None
    lse = torch.empty(B, Hq, dtype=torch.float32, device=q.device) if want_lse else None
    ws = attention_workspace(q.device, B, Hq, Hkv, max(int(n_tokens), 1))
    if seq_lens is not None:
        seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
    if seq_starts is not None:
        seq_starts = seq_starts.to(device=q.device, dtype=torch.int32).contiguous()
    s = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    _lib.call("tq_decode_attention_groups", _vp(q), B, Hq, Hkv, D, _vp(seq_starts), _vp(seq_lens), int(n_tokens), cap,
              n, dims, kbits, vbits, int(has_qjl), kc, kn, ks, kr, vc, vn, _vp(key_stack), ck, _vp(qjl_stack),
              _vp(value_stack), cv, ctypes.c_float(s), _vp(out_f32), _vp(out_bf16), _vp(lse), _vp(ws), ws.numel(),
              _stream(q.device))
    outs = (out_bf16,) + ((out_f32,) if want_f32 else ()) + ((lse,) if want_lse else ())
    return outs if len(outs) > 1 else out_bf16
