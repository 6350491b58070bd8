"""TurboQuant attention -- HF Transformers ``AttentionInterface`` backend.

``turboquant_attention_forward`` is registered under the name "turboquant"
(reference ``runtime/attention.py:28-120``).  With a packed cache layer on
the module (``module._tq_cache_layer``) a decode step runs the fused libtq
kernel over the packed history; without one (prefill, norm-guarded dense
layers) it is plain SDPA, as in the reference.

``fused_attention`` replaces the reference's Triton host wrapper
(``runtime/triton_kernels.py:238-368``).  Unlike the reference it accepts any
batch size (one query token per row) and honours left/right padding from the
attention mask; it has no fallback path -- shapes it does not cover raise.

Outlier-split layers run libtq's channel-group attention kernel
(``tq_decode_attention_groups``), which scores each channel group in its own
rotated space; the reference's fused kernel refuses such layers
(``triton_kernels.py:252-253``) and its chunked path
(``runtime/attention.py:215-304``) dequantises K and V for every step instead.
"""

from __future__ import annotations

import math
from typing import TYPE_CHECKING

import torch
import torch.nn.functional as F

from turboquant.runtime import kernels as K

if TYPE_CHECKING:
    from turboquant.runtime.packed_qmse_cache import PackedMSELayer


def _valid_range(attention_mask: torch.Tensor | None, B: int, total: int, device):
    """First / one-past-last attended slot per row from an HF decode mask.

    The mask is [B, 1, Sq, kv] (bool: True = attend, or additive float) or
    [B, kv].  Returns (starts, ends) int32 tensors on the device, or (None, None)
    when no mask is given.  Attended slots are assumed contiguous (padding only at
    the ends), which holds for left- or right-padded batched generation.
    """
    if attention_mask is None:
        return None, None
    m = attention_mask
    if m.dim() == 4:
        m = m[:, 0, -1, :]
    if m.dtype != torch.bool:
        m = m > torch.finfo(m.dtype).min / 2 if m.is_floating_point() else m != 0
    m = m[:, :total]
    if m.shape[0] == 1 and B > 1:
        m = m.expand(B, -1)
    idx = torch.arange(m.shape[1], device=m.device, dtype=torch.int32)
    big = torch.iinfo(torch.int32).max
    starts = torch.where(m, idx, torch.full_like(idx, big)).amin(dim=1)
    ends = torch.where(m, idx + 1, torch.zeros_like(idx)).amax(dim=1)
    starts = torch.minimum(starts, ends)
    return starts.to(device=device, dtype=torch.int32), ends.to(device=device, dtype=torch.int32)


def _group_buffers(layer: "PackedMSELayer") -> list[dict]:
    """The store's capacity buffers of each channel group of a split layer."""
    s, sc = layer._store, layer._split
    qjl = sc.use_qjl_keys
    out = []
    for sfx, kg, vg in (("", sc.key_normal, sc.value_normal), ("o", sc.key_outlier, sc.value_outlier)):
        out.append({"key": kg, "value": vg, "k_codes": getattr(s, "kc" + sfx), "k_norms": getattr(s, "kn" + sfx),
                    "k_signs": getattr(s, "ks" + sfx) if qjl else None,
                    "k_rnorms": getattr(s, "kr" + sfx) if qjl else None,
                    "v_codes": getattr(s, "vc" + sfx), "v_norms": getattr(s, "vn" + sfx)})
    return out


def fused_attention(query_states: torch.Tensor, packed_layer: "PackedMSELayer", n_kv_groups: int,
                    attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention of [B, Hq, 1, D] queries over a packed layer -> [B, Hq, 1, D].

    The logit scale is 1/sqrt(D) (reference ``triton_kernels.py:285``).  Tokens
    kept dense (``quantize_decode=False``) are merged by log-sum-exp.  Outlier-split
    layers go through the channel-group kernel (where the reference returns None and
    its caller takes the chunked path).
    """
    B, Hq, Sq, D = query_states.shape
    if Sq != 1:
        raise NotImplementedError("TurboQuant fused attention takes one decode token per sequence "
                                  f"(got {Sq}); prefill runs dense SDPA before the cache is packed")
    store = packed_layer._store
    n_packed = packed_layer.packed_seq_length()
    n_dense = 0 if packed_layer._dense_keys is None else int(packed_layer._dense_keys.shape[-2])
    scale = 1.0 / math.sqrt(D)
    starts, ends = _valid_range(attention_mask, B, n_packed + n_dense, query_states.device)
    p_ends = None if ends is None else torch.clamp(ends, max=n_packed)
    kw = dict(n_tokens=n_packed, seq_starts=starts, seq_lens=p_ends, scale=scale, want_f32=n_dense > 0,
              want_lse=n_dense > 0)
    if packed_layer._outlier_enabled:
        sc = packed_layer._split
        outs = K.decode_attention_groups(query_states, _group_buffers(packed_layer), key_stack=sc.key_stack,
                                         value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, **kw)
    else:
        c = packed_layer.codecs
        outs = K.decode_attention(query_states, k_codes=store.kc, k_norms=store.kn, v_codes=store.vc,
                                  v_norms=store.vn, key=c.key, value=c.value, k_signs=store.ks, k_rnorms=store.kr,
                                  qjl=c.qjl, **kw)
    if n_dense == 0:
        return outs.to(query_states.dtype).view(B, Hq, 1, D)
    _, o_packed, lse_packed = outs
    # dense decode buffer: exact attention on the few generated tokens, merged by LSE
    dk = packed_layer._dense_keys.float().repeat_interleave(n_kv_groups, dim=1)  # [B, Hq, n, D]
    dv = packed_layer._dense_values.float().repeat_interleave(n_kv_groups, dim=1)
    logits = (query_states.float() @ dk.transpose(-2, -1)).squeeze(2) * scale  # [B, Hq, n]
    if starts is not None:
        pos = torch.arange(n_packed, n_packed + n_dense, device=logits.device)
        ok = (pos[None, :] >= starts[:, None]) & (pos[None, :] < ends[:, None])
        logits = logits.masked_fill(~ok[:, None, :], float("-inf"))
    lse_dense = torch.logsumexp(logits, dim=-1)  # [B, Hq]
    m = torch.maximum(lse_packed, lse_dense)
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    wp = torch.exp(lse_packed - m)
    wd = torch.exp(logits - m[..., None])  # [B, Hq, n]
    num = o_packed * wp[..., None] + (wd[..., None] * dv).sum(dim=2)
    den = (wp + wd.sum(dim=-1)).clamp(min=1e-30)[..., None]
    return (num / den).to(query_states.dtype).view(B, Hq, 1, D)


def _sdpa_fallback(module, query, key, value, attention_mask, scaling):
    """Standard SDPA for prefill and norm-guarded dense layers (reference :75-99)."""
    causal = attention_mask is None and query.shape[-2] > 1
    n_kv_groups = getattr(module, "num_key_value_groups", 1)
    out = F.scaled_dot_product_attention(query, key, value, attn_mask=attention_mask, dropout_p=0.0,
                                         is_causal=causal, scale=scaling, enable_gqa=n_kv_groups > 1)
    return out.transpose(1, 2).contiguous(), None


def turboquant_attention_forward(module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                                 value: torch.Tensor, attention_mask: torch.Tensor | None, dropout: float = 0.0,
                                 scaling: float | None = None, is_causal: bool | None = None, **kwargs):
    """HF attention-interface function: returns ([B, Sq, Hq, D], None)."""
    layer = getattr(module, "_tq_cache_layer", None)
    if layer is None or layer._force_dense or layer.packed_seq_length() == 0:
        return _sdpa_fallback(module, query, key, value, attention_mask, scaling)
    out = fused_attention(query, layer, getattr(module, "num_key_value_groups", 1), attention_mask)
    return out.transpose(1, 2).contiguous(), None


def _register_attention_backend() -> None:
    """Register "turboquant" with HF's attention and mask interfaces (idempotent)."""
    try:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    except ImportError:  # pragma: no cover - transformers is a hard dependency of the adapter
        return
    if "turboquant" not in ALL_ATTENTION_FUNCTIONS:
        ALL_ATTENTION_FUNCTIONS.register("turboquant", turboquant_attention_forward)
    try:
        from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

        if "turboquant" not in ALL_MASK_ATTENTION_FUNCTIONS:
            ALL_MASK_ATTENTION_FUNCTIONS.register("turboquant", ALL_MASK_ATTENTION_FUNCTIONS["sdpa"])
    except (ImportError, KeyError):  # pragma: no cover
        pass


_register_attention_backend()
