"""TurboQuant KV-cache compression for HuggingFace Transformers -- MI355X-native (libtq, gfx950).

Same public API as the reference package ``turboquant`` 0.1.0.
"""

from turboquant.api import (
    CompatibilityReport,
    TelemetrySummary,
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
    summarize_generation_metrics,
)

__all__ = [
    "__version__",
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

__version__ = "0.1.0"
