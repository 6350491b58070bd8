"""Drop-in API surface on the CPU: names, activate/deactivate state machine,
error behaviour, telemetry schema and arithmetic, and the absence of a CPU
fallback (generation on a CPU model raises instead of computing)."""

import math

import pytest
import torch

import turboquant
from turboquant.runtime.attention import _valid_range
from turboquant.runtime.memory_accounting import turboquant_mse_packed_bytes
from turboquant.runtime.packed_qmse_cache import PackedMSELayer, _auto_norm_threshold
from turboquant.telemetry import TelemetrySummary, summarize_generation_metrics

from ._tiny_model import CharTokenizer, tiny_llama

REFERENCE_EXPORTS = {
    "__version__", "CompatibilityReport", "TelemetrySummary", "TransformersLoadConfig", "TurboQuantSession",
    "activate", "deactivate", "inspect_transformers_model_compatibility", "is_active", "last_metrics",
    "last_telemetry", "load_transformers_model", "print_telemetry", "summarize_generation_metrics",
}

TELEMETRY_KEYS = [
    "variant", "qmse_bits", "prompt_tokens", "completion_tokens", "dense_kv_bytes", "packed_estimate_bytes",
    "packed_actual_bytes", "payload_savings_fraction", "payload_savings_percent",
    "post_cache_setup_allocated_bytes", "post_cache_setup_reserved_bytes", "peak_allocated_bytes",
    "peak_reserved_bytes", "generation_seconds", "quantization_seconds",
]


def test_public_names_match_reference():
    assert set(turboquant.__all__) == REFERENCE_EXPORTS
    for name in REFERENCE_EXPORTS - {"__version__"}:
        assert hasattr(turboquant, name)
    assert turboquant.__version__ == "0.1.0"


def test_activate_deactivate_state_machine(capsys):
    model = tiny_llama()
    orig = model.generate
    assert not turboquant.is_active(model)
    turboquant.activate(model, CharTokenizer(), quiet=True)
    assert turboquant.is_active(model) and model.generate is not orig
    with pytest.raises(RuntimeError, match="already active"):
        turboquant.activate(model, CharTokenizer(), quiet=True)
    assert turboquant.last_telemetry(model) is None and turboquant.last_metrics(model) is None
    turboquant.print_telemetry(model)
    assert "No generation data yet" in capsys.readouterr().out
    turboquant.deactivate(model)
    assert not turboquant.is_active(model) and model.generate == orig
    turboquant.deactivate(model)  # second call is a no-op with a message
    assert "Not active" in capsys.readouterr().out


def test_activate_banner_and_errors(capsys):
    model = tiny_llama()
    turboquant.activate(model, CharTokenizer(), bits=3, use_qjl_keys=False)
    out = capsys.readouterr().out
    assert "3-bit Q_mse" in out and "TurboQuant activated" in out
    turboquant.deactivate(model, quiet=True)
    model.config._name_or_path = ""
    with pytest.raises(ValueError, match="tokenizer"):
        turboquant.activate(model, None, quiet=True)
    with pytest.raises(ValueError, match="outlier bits"):
        turboquant.activate(model, CharTokenizer(), num_outlier_channels=4, outlier_extra_bits=5, quiet=True)
    model.config.use_cache = False
    with pytest.raises(ValueError, match="not compatible"):
        turboquant.activate(model, CharTokenizer(), quiet=True)


def test_compatibility_report():
    model = tiny_llama()
    r = turboquant.inspect_transformers_model_compatibility(model)
    assert r.compatible and r.backend == "transformers" and r.details["num_key_value_heads"] == 2
    assert set(r.to_dict()) == {"compatible", "backend", "reasons", "warnings", "details"}


def test_no_cpu_fallback_generate_raises():
    """The packed path runs only on libtq/GPU: a CPU model fails loudly."""
    model = tiny_llama()
    turboquant.activate(model, CharTokenizer(), quiet=True)
    ids = torch.tensor([[1, 2, 3, 4]])
    with pytest.raises(RuntimeError, match="GPU"):
        model.generate(ids, max_new_tokens=3)
    # the attention interface was restored despite the failure
    assert model.config._attn_implementation != "turboquant"


def test_norm_guard_threshold_closed_form():
    """sqrt(D / D_mse(bits)) with D_mse(4)=0.009, D_mse(3)=0.030 (reference :888-900)."""
    assert math.isclose(_auto_norm_threshold(4, 128), math.sqrt(128 / 0.009))
    assert round(_auto_norm_threshold(4, 128), 1) == 119.3
    assert round(_auto_norm_threshold(3, 128), 1) == 65.3


def test_telemetry_schema_and_savings_arithmetic():
    """4-bit Q_prod stores 134 B per token-head against 512 B dense: 73.8% saved."""
    n_vec = 2 * 8 * 100  # layers * heads * tokens, per kind
    metrics = {
        "variant": "qmse_packed", "qmse_bits": 4, "quantization_seconds": 0.5, "generation_seconds": 2.0,
        "prompt_tokens": 100, "completion_tokens": 10,
        "prefill_cache": {"dense_kv_bytes": 2 * n_vec * 256},
        "turboquant_mse_packed_estimate": turboquant_mse_packed_bytes(num_vectors_per_kind=n_vec,
                                                                      vector_dimension=128, bits=4),
        "turboquant_mse_packed_actual": {"packed_total_bytes": n_vec * 134},
        "post_cache_setup_gpu_memory": {"allocated_bytes": 1, "reserved_bytes": 2},
        "gpu_peak_memory": {"peak_allocated_bytes": 3, "peak_reserved_bytes": None},
    }
    t = summarize_generation_metrics(metrics)
    d = t.to_dict()
    assert list(d) == TELEMETRY_KEYS
    assert round(d["payload_savings_percent"], 1) == 73.8
    assert d["packed_estimate_bytes"] == 2 * (n_vec * 128 * 4 // 8 + 2 * n_vec)  # 132 B per token-head
    assert d["peak_reserved_bytes"] is None
    assert "73.8%" in t.format() and "74% saved" in t.format(compact=True)
    assert isinstance(t, TelemetrySummary)


def test_cache_layer_protocol_without_data():
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=True)
    assert layer.get_seq_length() == 0 and layer.get_max_length() == -1
    assert layer.get_mask_sizes(1) == (1, 0)
    assert layer.keys_packed is None and layer._keys_qjl is None and layer.storage_bytes() == 0
    split = PackedMSELayer(bits=4, num_outlier_channels=2)
    assert split._keys_outlier is None and split._keys_outlier_qjl is None and not split._outlier_enabled


def test_valid_range_from_masks():
    bool_mask = torch.tensor([[True, True, True, True], [False, False, True, True], [True, True, False, False]])
    s, e = _valid_range(bool_mask[:, None, None, :], 3, 4, "cpu")
    assert s.tolist() == [0, 2, 0] and e.tolist() == [4, 4, 2]
    add = torch.where(bool_mask, 0.0, torch.finfo(torch.float32).min)[:, None, None, :]
    s2, e2 = _valid_range(add, 3, 4, "cpu")
    assert s2.tolist() == s.tolist() and e2.tolist() == e.tolist()
    assert _valid_range(None, 3, 4, "cpu") == (None, None)


def test_valid_range_rejects_masks_with_holes():
    """Right padding followed by generated tokens leaves a hole; the fused kernel takes one
    range per row, so the range helper refuses such a mask (fused_attention then returns
    None) unless the caller vouches for contiguity."""
    from turboquant.runtime.attention import _HoleyMask

    m = torch.tensor([[1, 1, 1, 1, 1], [1, 1, 0, 0, 1]], dtype=torch.bool)
    with pytest.raises(_HoleyMask):
        _valid_range(m[:, None, None, :], 2, 5, "cpu")
    s, e = _valid_range(m[:, None, None, :], 2, 5, "cpu", check_contiguous=False)
    assert s.tolist() == [0, 0] and e.tolist() == [5, 5]
    left = torch.tensor([[0, 0, 1, 1, 1]], dtype=torch.bool)  # left padding stays contiguous
    s, e = _valid_range(left, 1, 5, "cpu")
    assert s.tolist() == [2] and e.tolist() == [5]


def test_loader_takes_local_directories_only(tmp_path):
    """No hub downloads in this build: a model id that is not a local directory raises
    FileNotFoundError before transformers is asked to fetch anything."""
    from turboquant.adapters.transformers import TransformersLoadConfig, TurboQuantSession, load_transformers_model

    with pytest.raises(FileNotFoundError, match="local model directory"):
        load_transformers_model(TransformersLoadConfig("some-org/some-model"))
    with pytest.raises(FileNotFoundError):
        TurboQuantSession.from_pretrained(str(tmp_path / "missing"))


def test_session_settings_and_bit_checks():
    from turboquant.adapters.transformers import TurboQuantSession

    model = tiny_llama()
    s = TurboQuantSession(model=model, tokenizer=CharTokenizer())
    # the reference's session defaults differ from activate's
    assert (s.bits, s.use_qjl_keys, s.quantize_decode, s.variant) == (3, False, False, "qmse_packed")
    assert s.compatibility_report()["compatible"] and s.last_telemetry() is None
    with pytest.raises(ValueError, match="unsupported"):
        TurboQuantSession(model=model, tokenizer=CharTokenizer(), bits=1, use_qjl_keys=True)
    # settings are plain attributes, as the reference's: an assignment reaches the next generate
    s.bits, s.use_qjl_keys = 4, True
    assert (s.codec.bits, s.codec.use_qjl_keys, s.codec.mode()) == (4, True, "Q_prod")
    s.bits = 9
    with pytest.raises(ValueError, match="unsupported"):
        s.generate(prompt="ab", max_new_tokens=1)
    with pytest.raises(ValueError, match="out of range"):
        turboquant.activate(model, CharTokenizer(), bits=4, num_outlier_channels=4, outlier_extra_bits=5, quiet=True)
    assert not turboquant.is_active(model)
