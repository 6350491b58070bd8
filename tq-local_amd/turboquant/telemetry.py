"""Telemetry summary of a generate() call (reference ``telemetry.py``).

``TelemetrySummary.to_dict()`` is the ``last_telemetry()`` schema: exactly the
15 keys of the reference (``telemetry.py:22-36``).
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Any

from turboquant.runtime.generation import GenerationMetrics


def _fmt_bytes(num_bytes: int | float | None) -> str:
    if num_bytes is None:
        return "n/a"
    value = float(num_bytes)
    for unit in ("B", "KB", "MB", "GB", "TB"):
        if value < 1024.0 or unit == "TB":
            return f"{value:.2f} {unit}"
        value /= 1024.0
    return f"{num_bytes} B"  # pragma: no cover


@dataclass(frozen=True)
class TelemetrySummary:
    variant: str
    qmse_bits: int | None
    prompt_tokens: int
    completion_tokens: int
    dense_kv_bytes: int
    packed_estimate_bytes: int | None
    packed_actual_bytes: int | None
    payload_savings_fraction: float | None
    payload_savings_percent: float | None
    post_cache_setup_allocated_bytes: int | None
    post_cache_setup_reserved_bytes: int | None
    peak_allocated_bytes: int | None
    peak_reserved_bytes: int | None
    generation_seconds: float
    quantization_seconds: float

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    def format(self, compact: bool = False) -> str:
        return self._format_compact() if compact else self._format_full()

    def _format_compact(self) -> str:
        dense_mb = self.dense_kv_bytes / (1024 * 1024)
        packed = self.packed_actual_bytes or self.packed_estimate_bytes
        packed_mb = packed / (1024 * 1024) if packed else 0
        savings = f"{self.payload_savings_percent:.0f}% saved" if self.payload_savings_percent else ""
        peak = f" | peak {self.peak_allocated_bytes / 1e9:.1f} GB" if self.peak_allocated_bytes else ""
        return (f"[TurboQuant] {self.prompt_tokens}→{self.completion_tokens} tok"
                f" | KV {dense_mb:.0f}→{packed_mb:.0f} MB ({savings}){peak}")

    def _format_full(self) -> str:
        mode = f"{self.qmse_bits}-bit {self.variant}" if self.qmse_bits else self.variant
        savings = f"{self.payload_savings_percent:.1f}%" if self.payload_savings_percent else "n/a"
        tok_s = f"{self.completion_tokens / self.generation_seconds:.1f}" if self.generation_seconds > 0 else "n/a"
        packed = self.packed_actual_bytes or self.packed_estimate_bytes
        lines = ["", "  TurboQuant Telemetry", "  " + "─" * 50, "",
                 f"    Mode:               {mode}",
                 f"    KV savings:         {savings}",
                 f"    Generation:         {self.generation_seconds:.2f}s  ({tok_s} tok/s)",
                 f"    Quantization:       {self.quantization_seconds:.3f}s", "",
                 f"    Prompt tokens:      {self.prompt_tokens}",
                 f"    Completion tokens:  {self.completion_tokens}", "",
                 f"    Dense KV cache:     {_fmt_bytes(self.dense_kv_bytes)}",
                 f"    Packed KV cache:    {_fmt_bytes(packed)}"]
        if self.post_cache_setup_allocated_bytes is not None:
            lines += ["", f"    GPU after setup:    {_fmt_bytes(self.post_cache_setup_allocated_bytes)}"]
        if self.peak_allocated_bytes is not None:
            lines.append(f"    GPU peak:           {_fmt_bytes(self.peak_allocated_bytes)}")
        lines.append("")
        return "\n".join(lines)


def _get_int(d: dict | None, key: str) -> int | None:
    if d is None or d.get(key) is None:
        return None
    return int(d[key])


def summarize_generation_metrics(metrics: GenerationMetrics | dict[str, Any]) -> TelemetrySummary:
    """Reference ``telemetry.py:98-156``: savings = 1 - packed_actual (else estimate) / dense."""
    m = metrics.to_dict() if isinstance(metrics, GenerationMetrics) else metrics
    dense = int(m["prefill_cache"]["dense_kv_bytes"])
    est = _get_int(m.get("turboquant_mse_packed_estimate"), "packed_kv_bytes")
    act = _get_int(m.get("turboquant_mse_packed_actual"), "packed_total_bytes")
    eff = act if act is not None else est
    frac = pct = None
    if eff is not None and dense > 0:
        frac = 1.0 - eff / dense
        pct = frac * 100.0
    post, peak = m.get("post_cache_setup_gpu_memory"), m.get("gpu_peak_memory")
    return TelemetrySummary(
        variant=str(m["variant"]), qmse_bits=m.get("qmse_bits"), prompt_tokens=int(m["prompt_tokens"]),
        completion_tokens=int(m["completion_tokens"]), dense_kv_bytes=dense, packed_estimate_bytes=est,
        packed_actual_bytes=act, payload_savings_fraction=frac, payload_savings_percent=pct,
        post_cache_setup_allocated_bytes=_get_int(post, "allocated_bytes"),
        post_cache_setup_reserved_bytes=_get_int(post, "reserved_bytes"),
        peak_allocated_bytes=_get_int(peak, "peak_allocated_bytes"),
        peak_reserved_bytes=_get_int(peak, "peak_reserved_bytes"),
        generation_seconds=float(m["generation_seconds"]), quantization_seconds=float(m["quantization_seconds"]),
    )
