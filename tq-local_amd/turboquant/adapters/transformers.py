"""HuggingFace Transformers front end: ``activate`` / ``deactivate`` / telemetry.

Public surface of reference ``adapters/transformers.py`` (names, signatures,
exception types, the activation banner and the telemetry schema are the drop-in
contract).  The implementation is this build's:

* ``_Codec`` is the frozen set of TurboQuant settings one call runs with; it
  validates them against what the libtq kernels pack and turns them into the
  arguments of ``greedy_decode_with_prefill_cache``.
* ``_ActiveState`` is what ``activate`` leaves on the model (``model._tq_state``):
  the codec, the ``generate`` it replaced and a call counter.  Its bound
  ``generate`` method replaces ``model.generate``.
* Compatibility is a table of (predicate, message) rules over the model's config.
* Models load from a local directory only: this build has no hub access, so the
  reference's download path (``from_pretrained`` of a hub id) is out of scope and
  raises ``FileNotFoundError`` with that explanation.

Kept reference behaviours (documented quirks): ``generate`` returns only batch
row 0 as [1, prompt + completion] with the completion ids re-encoded from the
decoded text; ``max_length`` is read as a new-token budget; the EOS check looks at
row 0; ``TurboQuantSession`` defaults differ from ``activate``'s.
"""

from __future__ import annotations

import os
from dataclasses import asdict, dataclass, field
from typing import Any, Callable

import torch
from transformers.cache_utils import Cache

from turboquant.constants import DEFAULT_MAX_NEW_TOKENS
from turboquant.runtime.generation import GenerationOutput, greedy_decode_with_prefill_cache
from turboquant.telemetry import summarize_generation_metrics

NO_DATA = "[TurboQuant] No generation data yet."


# ------------------------------------------------------------------ loading (local only)
@dataclass(frozen=True)
class TransformersLoadConfig:
    model_id_or_path: str
    revision: str | None = None
    dtype: str | torch.dtype = "auto"
    device_map: str | dict[str, Any] = "auto"
    attn_implementation: str = "sdpa"
    trust_remote_code: bool = False
    token: str | None = None
    cache_dir: str | None = None


def load_transformers_model(config: TransformersLoadConfig):
    """(tokenizer, model) from a local model directory, model in eval mode.

    Hub ids are not fetched (no network in this build): anything that is not an
    existing directory raises ``FileNotFoundError``."""
    where = os.path.expanduser(str(config.model_id_or_path))
    if not os.path.isdir(where):
        raise FileNotFoundError(
            f"{config.model_id_or_path!r} is not a local model directory; this build loads models from disk "
            "only (no hub downloads)")
    from transformers import AutoModelForCausalLM, AutoTokenizer

    dtype = config.dtype
    if isinstance(dtype, str) and dtype != "auto":
        dtype = getattr(torch, dtype)
    shared = {"local_files_only": True, "revision": config.revision, "cache_dir": config.cache_dir,
              "trust_remote_code": config.trust_remote_code}
    tokenizer = AutoTokenizer.from_pretrained(where, **shared)
    model = AutoModelForCausalLM.from_pretrained(where, dtype=dtype, device_map=config.device_map,
                                                 attn_implementation=config.attn_implementation, **shared)
    return tokenizer, model.eval()


# ------------------------------------------------------------------ compatibility
@dataclass(frozen=True)
class CompatibilityReport:
    compatible: bool
    backend: str
    reasons: list[str] = field(default_factory=list)
    warnings: list[str] = field(default_factory=list)
    details: dict[str, Any] = field(default_factory=dict)

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


_Rule = tuple[Callable[[dict[str, Any]], bool], str]

#: conditions that make a model unusable (reference :66-104 lists the same)
_BLOCKING: tuple[_Rule, ...] = (
    (lambda f: not f["has_generate"], "Model does not expose a generate() method."),
    (lambda f: f["is_encoder_decoder"], "Encoder-decoder models are not supported in v1."),
    (lambda f: not f["use_cache"], "Model config disables use_cache."),
    (lambda f: f["num_hidden_layers"] is None or f["num_attention_heads"] is None,
     "Model is missing standard decoder attention metadata."),
)
#: conditions that only earn a warning
_CAVEATS: tuple[_Rule, ...] = (
    (lambda f: f["sliding_window"] is not None, "Sliding-window attention is not explicitly supported in v1."),
    (lambda f: f["attention_chunk_size"] is not None, "Chunked attention is not explicitly supported in v1."),
    (lambda f: f["num_kv_shared_layers"] is not None, "Shared-KV-layer models are not explicitly supported in v1."),
)
#: config fields reported in CompatibilityReport.details, in this order
_REPORTED = ("model_type", "is_encoder_decoder", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
             "sliding_window", "attention_chunk_size", "has_generate", "has_model_layers", "use_cache")


def _model_facts(model) -> dict[str, Any]:
    cfg = model.config
    facts = {name: getattr(cfg, name, None) for name in _REPORTED}
    facts["is_encoder_decoder"] = bool(facts["is_encoder_decoder"])
    facts["use_cache"] = getattr(cfg, "use_cache", True)
    facts["has_generate"] = hasattr(model, "generate")
    facts["has_model_layers"] = _decoder_layers(model) is not None
    facts["num_kv_shared_layers"] = getattr(cfg, "num_kv_shared_layers", None)
    return facts


def inspect_transformers_model_compatibility(model) -> CompatibilityReport:
    facts = _model_facts(model)
    reasons = [msg for test, msg in _BLOCKING if test(facts)]
    warnings = [msg for test, msg in _CAVEATS if test(facts)]
    return CompatibilityReport(compatible=not reasons, backend="transformers", reasons=reasons, warnings=warnings,
                               details={name: facts[name] for name in _REPORTED})


# ------------------------------------------------------------------ attention wiring
def _decoder_layers(model):
    inner = getattr(model, "model", None)
    return getattr(inner, "layers", None) if inner is not None else None


def enable_turboquant_attention(model, packed_cache: Cache) -> str | None:
    """Switch the model to the "turboquant" attention interface and hand every attention
    module its packed cache layer (reference :107-131).  Returns the previous setting."""
    import turboquant.runtime.attention  # noqa: F401  (registers the backend)

    layers = _decoder_layers(model)
    if layers is None:
        raise RuntimeError("Cannot locate model decoder layers for TurboQuant attention wiring.")
    previous = getattr(model.config, "_attn_implementation", None)
    for block, cache_layer in zip(layers, packed_cache.layers):
        block.self_attn._tq_cache_layer = cache_layer
        cache_layer._lazy_update = True  # the cache appends decode tokens itself
    model.config._attn_implementation = "turboquant"
    return previous


def disable_turboquant_attention(model, packed_cache: Cache, old_impl: str | None = "sdpa") -> None:
    """Undo ``enable_turboquant_attention`` (reference :134-147)."""
    layers = _decoder_layers(model)
    if layers is None:
        return
    model.config._attn_implementation = old_impl or "sdpa"
    cache_layers = list(packed_cache.layers) if packed_cache is not None else []
    for i, block in enumerate(layers):
        _drop(block.self_attn, "_tq_cache_layer")
        if i < len(cache_layers):
            cache_layers[i]._lazy_update = False
            _drop(cache_layers[i], "_tq_mask_contiguous")


def _drop(obj, name: str) -> None:
    if hasattr(obj, name):
        delattr(obj, name)


# ------------------------------------------------------------------ one call's settings
@dataclass(frozen=True)
class _Codec:
    bits: int
    rotation_seed: int
    num_outlier_channels: int
    outlier_extra_bits: int
    use_qjl_keys: bool
    quantize_decode: bool
    norm_guard: bool

    def check(self) -> "_Codec":
        """Reject settings the libtq kernels cannot pack (ValueError, as the reference's
        own argument errors)."""
        lowest = 2 if self.use_qjl_keys else 1
        if not lowest <= self.bits <= 4:
            raise ValueError(f"bits={self.bits} unsupported (Q_mse: 1-4, Q_prod: 2-4)")
        if self.num_outlier_channels and not 1 <= self.bits + self.outlier_extra_bits <= 8:
            raise ValueError(f"outlier bits {self.bits}+{self.outlier_extra_bits} out of range "
                             "(the channel-group kernels pack 1-8)")
        return self

    def mode(self) -> str:
        return "Q_prod" if self.use_qjl_keys else "Q_mse"

    def run(self, model, tokenizer, inputs: dict, max_new_tokens: int,
            variant: str = "qmse_packed") -> GenerationOutput:
        return greedy_decode_with_prefill_cache(
            model=model, tokenizer=tokenizer, inputs=inputs, max_new_tokens=max_new_tokens, variant=variant,
            qmse_bits=self.bits, rotation_seed=self.rotation_seed, num_outlier_channels=self.num_outlier_channels,
            outlier_extra_bits=self.outlier_extra_bits, use_qjl_keys=self.use_qjl_keys,
            quantize_decode=self.quantize_decode, norm_guard=self.norm_guard)


def _encode_prompt(tokenizer, prompt: str | None, messages, add_generation_prompt: bool):
    """Tokenise a prompt string or a chat (reference :158-177 accepts the same inputs)."""
    if messages is not None:
        if not hasattr(tokenizer, "apply_chat_template"):
            raise ValueError("Tokenizer does not support apply_chat_template, so messages input is unavailable.")
        prompt = tokenizer.apply_chat_template(messages, tokenize=False, add_generation_prompt=add_generation_prompt)
    elif prompt is None:
        raise ValueError("Either prompt or messages must be provided.")
    return tokenizer(prompt, return_tensors="pt")


def _summary(output: GenerationOutput | None):
    return None if output is None else summarize_generation_metrics(output.metrics)


# ------------------------------------------------------------------ explicit sessions
class TurboQuantSession:
    """A model + tokenizer pair generating through TurboQuant on every call (reference
    :180-311).  Its defaults (3-bit Q_mse, dense decode tokens) differ from ``activate``'s,
    as the reference's do."""

    def __init__(self, *, model, tokenizer, variant: str = "qmse_packed", bits: int = 3, rotation_seed: int = 0,
                 num_outlier_channels: int = 0, outlier_extra_bits: int = 1, use_qjl_keys: bool = False,
                 quantize_decode: bool = False, norm_guard: bool = True) -> None:
        report = inspect_transformers_model_compatibility(model)
        if not report.compatible:
            raise ValueError(f"Incompatible model for TurboQuantSession: {report.reasons}")
        self.model = model
        self.tokenizer = tokenizer
        self.variant = variant
        self.compatibility = report
        # plain attributes, as the reference's (assigning one changes the next generate)
        self.bits = bits
        self.rotation_seed = rotation_seed
        self.num_outlier_channels = num_outlier_channels
        self.outlier_extra_bits = outlier_extra_bits
        self.use_qjl_keys = use_qjl_keys
        self.quantize_decode = quantize_decode
        self.norm_guard = norm_guard
        self.codec.check()
        self._last_output: GenerationOutput | None = None

    @property
    def codec(self) -> _Codec:
        """The settings as they stand now (built on every read, so assignments take effect)."""
        return _Codec(self.bits, self.rotation_seed, self.num_outlier_channels, self.outlier_extra_bits,
                      self.use_qjl_keys, self.quantize_decode, self.norm_guard)

    @classmethod
    def from_pretrained(cls, model_id_or_path: str, *, revision=None, dtype="auto", device_map="auto",
                        attn_implementation="sdpa", trust_remote_code=False, token=None, cache_dir=None,
                        variant="qmse_packed", bits=3, rotation_seed=0, num_outlier_channels=0, outlier_extra_bits=1,
                        use_qjl_keys=False, quantize_decode=False, norm_guard=True) -> "TurboQuantSession":
        """A session over a model loaded from a local directory (``load_transformers_model``)."""
        tokenizer, model = load_transformers_model(TransformersLoadConfig(
            model_id_or_path, revision=revision, dtype=dtype, device_map=device_map,
            attn_implementation=attn_implementation, trust_remote_code=trust_remote_code, token=token,
            cache_dir=cache_dir))
        return cls(model=model, tokenizer=tokenizer, variant=variant, bits=bits, rotation_seed=rotation_seed,
                   num_outlier_channels=num_outlier_channels, outlier_extra_bits=outlier_extra_bits,
                   use_qjl_keys=use_qjl_keys, quantize_decode=quantize_decode, norm_guard=norm_guard)

    def generate(self, *, prompt: str | None = None, messages=None, max_new_tokens: int = DEFAULT_MAX_NEW_TOKENS,
                 add_generation_prompt: bool = True, return_output: bool = False):
        encoded = _encode_prompt(self.tokenizer, prompt, messages, add_generation_prompt)
        device = next(self.model.parameters()).device
        inputs = {name: t.to(device) for name, t in encoded.items()}
        self._last_output = self.codec.check().run(self.model, self.tokenizer, inputs, max_new_tokens, self.variant)
        return self._last_output if return_output else self._last_output.text

    def last_metrics(self) -> dict[str, Any] | None:
        return None if self._last_output is None else self._last_output.metrics.to_dict()

    def last_telemetry(self) -> dict[str, Any] | None:
        s = _summary(self._last_output)
        return None if s is None else s.to_dict()

    def print_telemetry(self) -> None:
        s = _summary(self._last_output)
        print(NO_DATA if s is None else s.format(compact=False))

    def compatibility_report(self) -> dict[str, Any]:
        return self.compatibility.to_dict()


# ------------------------------------------------------------------ activate / deactivate
class _ActiveState:
    """Left on the model as ``model._tq_state`` by ``activate``.  Its ``generate`` replaces
    ``model.generate``: prefill, pack the KV cache, greedy decode over the packed cache."""

    def __init__(self, model, codec: _Codec, original_generate) -> None:
        self.model = model
        self.codec = codec
        self.original_generate = original_generate
        self.call_count = 0

    def generate(self, input_ids=None, **kwargs):
        # the reference reads max_length as a budget of new tokens, defaulting to 20
        budget = kwargs.pop("max_new_tokens", None) or kwargs.pop("max_length", None) or 20
        mask = kwargs.pop("attention_mask", None)
        if input_ids is None:
            raise ValueError("input_ids is required for TurboQuant generate().")
        inputs = {"input_ids": input_ids} if mask is None else {"input_ids": input_ids, "attention_mask": mask}
        self.call_count += 1
        tokenizer = self.model._tq_tokenizer
        output = self.codec.run(self.model, tokenizer, inputs, budget)
        self.model._tq_last_output = output
        # row 0 only, its completion re-encoded from the decoded text (reference behaviour)
        completion = torch.tensor(tokenizer.encode(output.text, add_special_tokens=False), dtype=input_ids.dtype,
                                  device=input_ids.device)
        return torch.cat((input_ids[0], completion)).unsqueeze(0)


def _default_tokenizer(model):
    """The tokenizer next to a locally loaded model (no downloads)."""
    source = getattr(model.config, "_name_or_path", None)
    if source:
        from transformers import AutoTokenizer

        try:
            return AutoTokenizer.from_pretrained(source, local_files_only=True)
        except (OSError, ValueError) as exc:
            raise ValueError(f"Cannot auto-detect tokenizer. Pass tokenizer= explicitly. ({exc})") from exc
    raise ValueError("Cannot auto-detect tokenizer. Pass tokenizer= explicitly.")


def _print_banner(model, codec: _Codec) -> None:
    cfg = model.config
    lines = ("", "  TurboQuant activated",
             f"    Model:      {getattr(cfg, 'model_type', 'unknown')} ({getattr(cfg, 'num_hidden_layers', '?')} layers)",
             f"    Bits:       {codec.bits}-bit {codec.mode()}",
             f"    Norm guard: {'on' if codec.norm_guard else 'off'}",
             f"    Decode:     {'quantized' if codec.quantize_decode else 'dense'}",
             "", "  model.generate() now uses TurboQuant compression.",
             "  Call turboquant.deactivate(model) to restore original behavior.", "")
    print("\n".join(lines))


def activate(model, tokenizer=None, *, bits: int = 4, rotation_seed: int = 0, num_outlier_channels: int = 0,
             outlier_extra_bits: int = 1, use_qjl_keys: bool = True, quantize_decode: bool = True,
             norm_guard: bool = True, quiet: bool = False) -> None:
    """Make ``model.generate`` compress the KV cache with TurboQuant (reference :329-450).

    Raises RuntimeError if TurboQuant is already active on the model, ValueError if the
    model is incompatible, a bit width cannot be packed or no tokenizer is found.
    """
    if hasattr(model, "_tq_state"):
        raise RuntimeError("TurboQuant is already active on this model. Call turboquant.deactivate(model) first.")
    report = inspect_transformers_model_compatibility(model)
    if not report.compatible:
        raise ValueError(f"Model is not compatible with TurboQuant: {report.reasons}")
    codec = _Codec(bits, rotation_seed, num_outlier_channels, outlier_extra_bits, use_qjl_keys, quantize_decode,
                   norm_guard).check()
    if tokenizer is None:
        tokenizer = _default_tokenizer(model)
    state = _ActiveState(model, codec, model.generate)
    model._tq_state = state
    model._tq_tokenizer = tokenizer
    model.generate = state.generate
    if not quiet:
        _print_banner(model, codec)


def deactivate(model, quiet: bool = False) -> None:
    """Give the model its own ``generate`` back (reference :453-468)."""
    state: _ActiveState | None = getattr(model, "_tq_state", None)
    if state is None:
        if not quiet:
            print("[TurboQuant] Not active on this model, nothing to deactivate.")
        return
    model.generate = state.original_generate
    for name in ("_tq_state", "_tq_tokenizer", "_tq_last_output"):
        _drop(model, name)
    if not quiet:
        print(f"[TurboQuant] Deactivated after {state.call_count} calls.")


def is_active(model) -> bool:
    return hasattr(model, "_tq_state")


def last_metrics(model) -> dict[str, Any] | None:
    output = getattr(model, "_tq_last_output", None)
    return None if output is None else output.metrics.to_dict()


def last_telemetry(model) -> dict[str, Any] | None:
    s = _summary(getattr(model, "_tq_last_output", None))
    return None if s is None else s.to_dict()


def print_telemetry(model, *, verbose: bool = False) -> None:
    s = _summary(getattr(model, "_tq_last_output", None))
    print(NO_DATA if s is None else s.format(compact=not verbose))
