"""Prefill -> pack -> greedy decode loop (reference ``runtime/generation.py:65-203``).

Same inputs, outputs and metrics as the reference.  Differences:
* the prefill asks the model for the last position's logits only
  (``logits_to_keep=1`` when the forward accepts it) -- the greedy token is the
  same, without materialising [B, prompt, vocab] logits;
* decode steps with the packed cache run the fused libtq kernel for every batch
  size (the reference's fused path is batch-1 only);
* a prompt mask without padding is dropped for the decode steps, and one look at it
  tells the attention backend whether every row's attended slots stay contiguous;
* the research "qmse" fake-quantisation variant is not provided.
"""

from __future__ import annotations

import inspect
import time
from dataclasses import asdict, dataclass
from typing import Any

from turboquant.runtime.memory_accounting import (
    gpu_current_memory_bytes,
    gpu_peak_memory_bytes,
    past_key_values_memory_breakdown,
    turboquant_mse_packed_bytes,
)
from turboquant.runtime.packed_qmse_cache import (
    build_packed_mse_cache,
    packed_cache_storage_breakdown,
    verify_packed_reconstruction,
)

VARIANTS = ("baseline", "qmse_packed")


@dataclass(frozen=True)
class GenerationMetrics:
    variant: str
    qmse_bits: int | None
    quantization_seconds: float
    generation_seconds: float
    prompt_tokens: int
    completion_tokens: int
    prefill_cache: dict[str, Any]
    turboquant_mse_packed_estimate: dict[str, Any] | None
    turboquant_mse_packed_actual: dict[str, Any] | None
    post_cache_setup_gpu_memory: dict[str, Any] | None
    gpu_peak_memory: dict[str, Any] | None
    reconstruction_quality: list[dict[str, Any]] | None = None

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


@dataclass(frozen=True)
class GenerationOutput:
    text: str
    metrics: GenerationMetrics
    token_ids: Any = None  # [B, completion] generated ids (not in the reference; handy for callers)


def validate_generation_variant(variant: str) -> None:
    if variant == "qmse":
        raise NotImplementedError("the research 'qmse' fake-quantisation variant is not part of the MI355X build; "
                                  "use 'qmse_packed'")
    if variant not in VARIANTS:
        raise ValueError(f"Unsupported generation variant={variant!r}. Choose from {list(VARIANTS)}.")


def eos_token_ids(model, tokenizer) -> set[int]:
    eos = getattr(getattr(model, "generation_config", None), "eos_token_id", None)
    if eos is None and tokenizer is not None:
        eos = getattr(tokenizer, "eos_token_id", None)
    if eos is None:
        return set()
    if isinstance(eos, int):
        return {eos}
    return {int(i) for i in eos}


def _accepts_logits_to_keep(model) -> bool:
    try:
        return "logits_to_keep" in inspect.signature(model.forward).parameters
    except (TypeError, ValueError):  # pragma: no cover
        return False


def greedy_decode_with_prefill_cache(*, model, tokenizer, inputs, max_new_tokens: int, variant: str,
                                     qmse_bits: int, rotation_seed: int = 0, num_outlier_channels: int = 0,
                                     outlier_extra_bits: int = 1, use_qjl_keys: bool = False,
                                     quantize_decode: bool = False, norm_guard: bool = True) -> GenerationOutput:
    import torch

    validate_generation_variant(variant)
    if max_new_tokens <= 0:
        raise ValueError("max_new_tokens must be positive.")
    t_start = time.monotonic()
    quant_s = 0.0
    eos_ids = eos_token_ids(model, tokenizer)
    extra = {"logits_to_keep": 1} if _accepts_logits_to_keep(model) else {}

    with torch.inference_mode():
        out = model(**inputs, use_cache=True, **extra)
        past = out.past_key_values
        next_token = torch.argmax(out.logits[:, -1, :], dim=-1, keepdim=True)
        dense_breakdown = past_key_values_memory_breakdown(past)
        estimate = (turboquant_mse_packed_bytes(num_vectors_per_kind=dense_breakdown["num_key_value_vectors_per_kind"],
                                                vector_dimension=dense_breakdown["vector_dimension"], bits=qmse_bits)
                    if variant == "qmse_packed" else None)
        actual = recon = packed = old_impl = None
        if variant == "qmse_packed":
            if torch.cuda.is_available():
                # the prefill kernels are still running: without this wait their tail would be
                # counted as quantization time at the packing's first host sync
                torch.cuda.synchronize()
            t0 = time.monotonic()
            packed = build_packed_mse_cache(past, bits=qmse_bits, seed=rotation_seed,
                                            num_outlier_channels=num_outlier_channels,
                                            outlier_extra_bits=outlier_extra_bits, use_qjl_keys=use_qjl_keys,
                                            quantize_decode=quantize_decode, norm_guard=norm_guard,
                                            reserve_tokens=max_new_tokens)
            recon = verify_packed_reconstruction(past, packed)
            del past
            past = packed
            actual = packed_cache_storage_breakdown(packed)
            quant_s += time.monotonic() - t0
            from turboquant.adapters.transformers import enable_turboquant_attention

            old_impl = enable_turboquant_attention(model, packed)
        del out
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        generated = [next_token]
        mask = inputs.get("attention_mask")
        if mask is not None:
            # One look at the prompt mask decides the decode masks of the whole call: with no
            # padding the decode steps need none (nothing to range-check per layer and step);
            # the fused kernel takes one attended range per row, so right padding (a hole once
            # generated tokens follow) sends those layers to the chunked path instead.
            attend = mask.bool()
            hole = bool(((attend.cumsum(dim=-1) > 0) & ~attend).any())
            if packed is not None:
                for layer in packed.layers:
                    layer._tq_mask_contiguous = not hole
            if bool(attend.all()):
                mask = None
        post_setup = gpu_current_memory_bytes()
        if torch.cuda.is_available():
            torch.cuda.reset_peak_memory_stats()
        try:
            for _ in range(max_new_tokens - 1):
                if eos_ids and int(next_token[0, 0].item()) in eos_ids:
                    break
                if mask is not None:
                    mask = torch.cat((mask, mask.new_ones((mask.shape[0], 1))), dim=-1)
                out = model(input_ids=next_token, attention_mask=mask, past_key_values=past, use_cache=True,
                            **extra)
                past = out.past_key_values
                next_token = torch.argmax(out.logits[:, -1, :], dim=-1, keepdim=True)
                generated.append(next_token)
        finally:
            if variant == "qmse_packed":
                from turboquant.adapters.transformers import disable_turboquant_attention

                disable_turboquant_attention(model, packed, old_impl)

    ids = torch.cat(generated, dim=-1)
    text = tokenizer.decode(ids[0], skip_special_tokens=True).strip() if tokenizer is not None else ""
    metrics = GenerationMetrics(
        variant=variant,
        qmse_bits=qmse_bits if variant == "qmse_packed" else None,
        quantization_seconds=round(quant_s, 4),
        generation_seconds=round(time.monotonic() - t_start, 4),
        prompt_tokens=int(inputs["input_ids"].shape[-1]),
        completion_tokens=int(ids.shape[-1]),
        prefill_cache=dense_breakdown,
        turboquant_mse_packed_estimate=estimate,
        turboquant_mse_packed_actual=actual,
        post_cache_setup_gpu_memory=post_setup,
        gpu_peak_memory=gpu_peak_memory_bytes(),
        reconstruction_quality=recon,
    )
    return GenerationOutput(text=text, metrics=metrics, token_ids=ids)
