"""KV byte accounting and GPU memory probes for the telemetry schema.

Same fields and arithmetic as reference ``runtime/memory_accounting.py:34-109``.
"""

from __future__ import annotations

from math import ceil
from typing import Any

import torch


def _layer_tensors(layer_cache) -> list[torch.Tensor]:
    if isinstance(layer_cache, (tuple, list)):
        return [t for t in layer_cache if torch.is_tensor(t)]
    out = []
    for name in ("keys", "values", "_sliding_window_tensor"):
        t = getattr(layer_cache, name, None)
        if torch.is_tensor(t):
            out.append(t)
    return out


def _nbytes(t: torch.Tensor) -> int:
    return int(t.numel() * t.element_size())


def past_key_values_memory_breakdown(past_key_values) -> dict[str, Any]:
    """Dense KV bytes of a prefilled cache (reference :34-64)."""
    layers = past_key_values.layers if hasattr(past_key_values, "layers") else past_key_values
    kb = vb = extra = n_layers = n_vec = 0
    dim = None
    for layer in layers:
        ts = _layer_tensors(layer)
        if len(ts) < 2:
            continue
        k, v, *rest = ts
        kb += _nbytes(k)
        vb += _nbytes(v)
        extra += sum(_nbytes(t) for t in rest)
        n_layers += 1
        if dim is None:
            dim = int(k.shape[-1])
        n_vec += int(k.shape[0] * k.shape[1] * k.shape[2])
    return {
        "num_layers": n_layers,
        "vector_dimension": dim,
        "num_key_value_vectors_per_kind": n_vec,
        "key_bytes": kb,
        "value_bytes": vb,
        "dense_kv_bytes": kb + vb,
        "extra_tensor_bytes": extra,
        "total_cache_tensor_bytes": kb + vb + extra,
    }


def turboquant_mse_packed_bytes(*, num_vectors_per_kind: int, vector_dimension: int, bits: int,
                                norm_bytes: int = 2) -> dict[str, int | str]:
    """Packed-size estimate: codes + one norm per vector, for K and V (reference :67-85)."""
    index_bytes = ceil(num_vectors_per_kind * vector_dimension * bits / 8)
    norm_total = num_vectors_per_kind * norm_bytes
    return {
        "bits": bits,
        "norm_bytes_per_vector": norm_bytes,
        "norm_dtype_assumption": "float16" if norm_bytes == 2 else f"{norm_bytes * 8}-bit",
        "packed_kv_bytes": 2 * (index_bytes + norm_total),
        "packed_index_bytes": 2 * index_bytes,
        "packed_norm_bytes": 2 * norm_total,
    }


def gpu_peak_memory_bytes() -> dict[str, int | None]:
    if not torch.cuda.is_available():
        return {"peak_allocated_bytes": None, "peak_reserved_bytes": None}
    return {"peak_allocated_bytes": int(torch.cuda.max_memory_allocated()),
            "peak_reserved_bytes": int(torch.cuda.max_memory_reserved())}


def gpu_current_memory_bytes() -> dict[str, int | None]:
    if not torch.cuda.is_available():
        return {"allocated_bytes": None, "reserved_bytes": None}
    return {"allocated_bytes": int(torch.cuda.memory_allocated()),
            "reserved_bytes": int(torch.cuda.memory_reserved())}
