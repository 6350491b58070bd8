"""TurboQuant attention -- HF Transformers ``AttentionInterface`` backend.

``turboquant_attention_forward`` is registered under the name "turboquant"
(reference ``runtime/attention.py:28-120``).  With a packed cache layer on
the module (``module._tq_cache_layer``) a decode step runs the fused libtq
kernel over the packed history, and several query tokens at once run
``chunked_turboquant_attention`` (libtq decoding, fp32 online softmax); without a
packed layer (prefill, norm-guarded dense layers) it is plain SDPA, as in the
reference.

``fused_attention`` replaces the reference's Triton host wrapper
(``runtime/triton_kernels.py:238-368``) with its contract (None = not applicable,
which here means more than one query token, a GQA group wider than 8 query heads
per KV head, or a mask whose attended slots are not contiguous).  Unlike the
reference it accepts any batch size and honours left padding (and right padding
before the packed history ends) from the attention mask.

Outlier-split layers run libtq's channel-group attention kernel
(``tq_decode_attention_groups``), which scores each channel group in its own
rotated space; the reference's fused kernel refuses such layers
(``triton_kernels.py:252-253``) and its chunked path
(``runtime/attention.py:215-304``) dequantises K and V for every step instead.
"""

from __future__ import annotations

import math
import threading
from typing import TYPE_CHECKING

import torch
import torch.nn.functional as F

from turboquant.runtime import _lib
from turboquant.runtime import kernels as K

if TYPE_CHECKING:
    from turboquant.runtime.packed_qmse_cache import PackedMSELayer


def _attend_mask(attention_mask: torch.Tensor, B: int, total: int) -> torch.Tensor:
    """The decode row of an HF mask as bool [B, total] (True = attend).

    The mask is [B, 1, Sq, kv] (bool, or additive float) or [B, kv]."""
    m = attention_mask
    if m.dim() == 4:
        m = m[:, 0, -1, :]
    if m.dtype != torch.bool:
        m = m > torch.finfo(m.dtype).min / 2 if m.is_floating_point() else m != 0
    m = m[:, :total]
    if m.shape[0] == 1 and B > 1:
        m = m.expand(B, -1)
    return m


#: the ranges of the last mask seen, per host thread (an HF forward hands every layer the same
#: mask tensor): (mask, its version counter, B, total, check) -> (starts, ends); holding the mask
#: keeps its memory from being reused by another tensor while the entry is live
_tls = threading.local()


def _valid_range(attention_mask: torch.Tensor | None, B: int, total: int, device, check_contiguous: bool = True):
    """Per-row attended slot range [start, end) from an HF decode mask.

    Returns (starts, ends) int32 device tensors, or (None, None) without a mask.  The
    kernel attends to every slot of the range, so a row whose attended slots have a
    hole (right padding followed by generated tokens) cannot take this path: with
    ``check_contiguous`` such masks raise ``_HoleyMask`` (one host sync to find out);
    callers that know the mask's shape pass False.  The result for one mask tensor is
    computed once and reused by the following layers of the same forward.
    """
    if attention_mask is None:
        return None, None
    c = getattr(_tls, "last_range", None)
    if (c is not None and c[0] is attention_mask and c[1] == attention_mask._version
            and c[2:6] == (B, total, check_contiguous, device)):
        if c[6] is None:
            raise _HoleyMask
        return c[6]
    try:
        result = _compute_range(attention_mask, B, total, device, check_contiguous)
    except _HoleyMask:
        _tls.last_range = (attention_mask, attention_mask._version, B, total, check_contiguous, device, None)
        raise
    _tls.last_range = (attention_mask, attention_mask._version, B, total, check_contiguous, device, result)
    return result


def _compute_range(attention_mask: torch.Tensor, B: int, total: int, device, check_contiguous: bool):
    m = _attend_mask(attention_mask, B, total)
    idx = torch.arange(m.shape[1], device=m.device, dtype=torch.int32)
    big = torch.iinfo(torch.int32).max
    starts = torch.where(m, idx, torch.full_like(idx, big)).amin(dim=1)
    ends = torch.where(m, idx + 1, torch.zeros_like(idx)).amax(dim=1)
    starts = torch.minimum(starts, ends)
    if check_contiguous and bool(((ends - starts) != m.sum(dim=1, dtype=torch.int32)).any()):
        raise _HoleyMask
    return starts.to(device=device, dtype=torch.int32), ends.to(device=device, dtype=torch.int32)


class _HoleyMask(Exception):
    """A decode mask whose attended slots are not one contiguous range per row."""


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
                    attention_mask: torch.Tensor | None = None) -> torch.Tensor | None:
    """Decode attention of [B, Hq, 1, D] queries over a packed layer -> [B, Hq, 1, D].

    The logit scale is 1/sqrt(D) (reference ``triton_kernels.py:285``).  Tokens
    kept dense (``quantize_decode=False``) are merged by log-sum-exp.  Outlier-split
    layers go through the channel-group kernel (where the reference returns None and
    its caller takes the chunked path).  The result has the query's dtype; an fp32
    query gets the kernel's fp32 output (no bf16 rounding).

    Returns None (the reference's "not applicable": the caller takes
    ``chunked_turboquant_attention``) for several query tokens, for GQA groups wider
    than the kernels' 8 query heads per KV head, and for a mask whose attended slots are
    not one contiguous range per row.  The cache layer's ``_tq_mask_contiguous`` (set by
    the generation loop from the prompt mask) spares the host sync of that last check.
    """
    B, Hq, Sq, D = query_states.shape
    if Sq != 1:
        return None  # the caller takes chunked_turboquant_attention (reference contract)
    store = packed_layer._store
    Hkv = store.kc.shape[1] if store is not None else Hq // max(n_kv_groups, 1)
    if Hq // Hkv > K.MAX_GROUP:
        return None
    n_packed = packed_layer.packed_seq_length()
    n_dense = 0 if packed_layer._dense_keys is None else int(packed_layer._dense_keys.shape[-2])
    scale = 1.0 / math.sqrt(D)
    known = getattr(packed_layer, "_tq_mask_contiguous", None)
    if attention_mask is not None and known is False:
        return None
    try:
        starts, ends = _valid_range(attention_mask, B, n_packed + n_dense, query_states.device,
                                    check_contiguous=known is None)
    except _HoleyMask:
        return None
    # the kernel sees the packed slots only; ends beyond them (dense tokens) are clamped
    p_ends = ends if ends is None or n_dense == 0 else torch.clamp(ends, max=n_packed)
    f32 = query_states.dtype == torch.float32
    kw = dict(n_tokens=n_packed, seq_starts=starts, seq_lens=p_ends, scale=scale, want_f32=f32 or n_dense > 0,
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
        out = outs[1] if f32 else outs
        return out.to(query_states.dtype).view(B, Hq, 1, D)
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


_DEFAULT_CHUNK_SIZE = 1024


def triton_available() -> bool:
    """Reference API (runtime/triton_kernels.py): whether the fused decode kernels are usable.
    Here that is libtq.so (there is no Triton in this build)."""
    try:
        _lib.load()
    except (ImportError, OSError):
        return False
    return True


def _repeat_kv(t: torch.Tensor, n_rep: int) -> torch.Tensor:
    return t if n_rep == 1 else t.repeat_interleave(n_rep, dim=1)


def _additive_mask(mask: torch.Tensor | None) -> torch.Tensor | None:
    if mask is None:
        return None
    if mask.dtype == torch.bool:
        return torch.zeros(mask.shape, dtype=torch.float32, device=mask.device).masked_fill(~mask, float("-inf"))
    return mask.float()


def chunked_turboquant_attention(query_states: torch.Tensor, packed_layer: "PackedMSELayer",
                                 new_key: torch.Tensor | None = None, new_value: torch.Tensor | None = None,
                                 n_kv_groups: int = 1, attention_mask: torch.Tensor | None = None,
                                 chunk_size: int = _DEFAULT_CHUNK_SIZE) -> torch.Tensor:
    """Any-shape attention over a packed layer -> [B, Q, Sq, D] (reference runtime/attention.py:215-304).

    The packed history is decoded by libtq ``chunk_size`` tokens at a time into bf16 K / V
    rows (reference ``_decode_keys_range`` / ``_decode_values_range``), then the dense decode
    buffer and ``new_key`` / ``new_value`` follow; logits are fp32 ``q . K / sqrt(D)`` plus
    the mask slice of each part, merged by an online softmax and normalised with the 1e-8
    clamp.  A boolean mask (True = attend) is applied as 0 / -inf; the reference adds
    ``mask.float()``, which is only right for additive masks.  Rows with nothing to attend
    to return zeros (the reference's running maximum turns them into NaN).
    """
    B, Q, Sq, D = query_states.shape
    scale = 1.0 / math.sqrt(D)
    qf = query_states.float()
    mask = _additive_mask(attention_mask)
    m = torch.full((B, Q, Sq, 1), float("-inf"), device=qf.device)
    s = torch.zeros(B, Q, Sq, 1, device=qf.device)
    o = torch.zeros(B, Q, Sq, D, device=qf.device)
    off = 0

    def attend(keys: torch.Tensor, values: torch.Tensor) -> None:
        nonlocal m, s, o, off
        n = int(keys.shape[-2])
        logits = (qf @ _repeat_kv(keys, n_kv_groups).float().transpose(-2, -1)) * scale
        if mask is not None:
            logits = logits + mask[..., off:off + n]
        new_m = torch.maximum(m, logits.amax(dim=-1, keepdim=True))
        safe = torch.where(torch.isfinite(new_m), new_m, torch.zeros_like(new_m))
        corr = torch.exp(m - safe)
        e = torch.exp(logits - safe)
        s = s * corr + e.sum(dim=-1, keepdim=True)
        o = o * corr + e @ _repeat_kv(values, n_kv_groups).float()
        m = new_m
        off += n

    n_packed = packed_layer.packed_seq_length()
    for a in range(0, n_packed, chunk_size):
        b = min(a + chunk_size, n_packed)
        attend(packed_layer._decode_keys_range(a, b), packed_layer._decode_values_range(a, b))
    if packed_layer._dense_keys is not None:
        attend(packed_layer._dense_keys, packed_layer._dense_values)
    if new_key is not None:
        attend(new_key, new_value)
    return (o / s.clamp(min=1e-8)).to(query_states.dtype)


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
    n_kv_groups = getattr(module, "num_key_value_groups", 1)
    out = fused_attention(query, layer, n_kv_groups, attention_mask) if query.shape[-2] == 1 else None
    if out is None:  # several query tokens, or a shape / mask the fused kernel does not take
        out = chunked_turboquant_attention(query, layer, n_kv_groups=n_kv_groups, attention_mask=attention_mask)
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
