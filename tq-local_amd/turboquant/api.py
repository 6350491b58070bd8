"""Public API re-exports (reference ``api.py``)."""

from turboquant.adapters.transformers import (
    CompatibilityReport,
    TransformersLoadConfig,
    TurboQuantSession,
    activate,
    deactivate,
    inspect_transformers_model_compatibility,
    is_active,
    last_metrics,
    last_telemetry,
    load_transformers_model,
    print_telemetry,
)
from turboquant.telemetry import TelemetrySummary, summarize_generation_metrics

__all__ = [
    "CompatibilityReport",
    "TelemetrySummary",
    "TransformersLoadConfig",
    "TurboQuantSession",
    "activate",
    "deactivate",
    "inspect_transformers_model_compatibility",
    "is_active",
    "last_metrics",
    "last_telemetry",
    "load_transformers_model",
    "print_telemetry",
    "summarize_generation_metrics",
]
