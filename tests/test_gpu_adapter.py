"""End-to-end drop-in on the GPU: activate -> generate on a random-init tiny
Llama (GQA 4, head_dim 128), the decode-step attention of a real model checked
against the fp64 oracle, the dense decode buffer (quantize_decode=False) and
left-padded batched decode."""

import math

import numpy as np
import pytest
import torch

import turboquant
from oracle import oracle as O
from turboquant.runtime.attention import fused_attention
from turboquant.runtime.packed_qmse_cache import PackedMSELayer, build_packed_mse_cache
from turboquant.runtime.synthetic import kv_bf16, query_bf16

from ._tiny_model import CharTokenizer, tiny_llama

pytestmark = pytest.mark.gpu

D = 128
TOL = 2e-3


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_layer(layer: PackedMSELayer) -> dict:
    s, c, n = layer._store, layer.codecs, layer.packed_seq_length()
    return {
        "kcodes": s.kc[:, :, :n].cpu().numpy(), "knorms": u16(s.kn[:, :, :n]),
        "vcodes": s.vc[:, :, :n].cpu().numpy(), "vnorms": u16(s.vn[:, :, :n]),
        "signs": None if s.ks is None else s.ks[:, :, :n].cpu().numpy(),
        "rnorms": None if s.kr is None else u16(s.kr[:, :, :n]),
        "Rk": c.key.rotation.cpu().numpy(), "Ck": c.key.centers.cpu().numpy(),
        "Rv": c.value.rotation.cpu().numpy(), "Cv": c.value.centers.cpu().numpy(),
        "S": None if c.qjl is None else c.qjl.cpu().numpy(), "kbits": c.key_bits, "vbits": c.value_bits,
    }


@pytest.mark.parametrize("bits,qjl", [(4, True), (3, False)])
def test_activate_generate_telemetry(cuda, bits, qjl):
    model = tiny_llama(device=cuda, dtype=torch.bfloat16)
    tok = CharTokenizer()
    turboquant.activate(model, tok, bits=bits, use_qjl_keys=qjl, quiet=True)
    ids = torch.randint(0, 94, (1, 300), generator=torch.Generator().manual_seed(0)).to(cuda)
    out = model.generate(ids, max_new_tokens=12)
    assert out.shape == (1, 312) and torch.equal(out[0, :300], ids[0])
    t = turboquant.last_telemetry(model)
    assert list(t) == ["variant", "qmse_bits", "prompt_tokens", "completion_tokens", "dense_kv_bytes",
                       "packed_estimate_bytes", "packed_actual_bytes", "payload_savings_fraction",
                       "payload_savings_percent", "post_cache_setup_allocated_bytes",
                       "post_cache_setup_reserved_bytes", "peak_allocated_bytes", "peak_reserved_bytes",
                       "generation_seconds", "quantization_seconds"]
    assert t["prompt_tokens"] == 300 and t["completion_tokens"] == 12 and t["qmse_bits"] == bits
    per_tok = (48 + 2 + 16 + 2 + 64 + 2) if qjl else (48 + 2 + 48 + 2)
    assert t["packed_actual_bytes"] == 2 * 2 * 300 * per_tok  # layers * kv_heads * prompt tokens
    assert t["payload_savings_percent"] == pytest.approx(100 * (1 - per_tok / 512))
    recon = turboquant.last_metrics(model)["reconstruction_quality"]
    assert len(recon) == 2 and all(r["key_cosine_sim"] > 0.9 and r["val_cosine_sim"] > 0.97 for r in recon)
    turboquant.deactivate(model, quiet=True)
    assert model.config._attn_implementation == "sdpa"


def test_decode_step_matches_oracle_attention_in_a_model(cuda):
    """One decode forward of a real model: the turboquant attention output of every
    layer equals the fp64 fused formula over that layer's packed cache."""
    model = tiny_llama(device=cuda, dtype=torch.bfloat16, layers=2)
    from turboquant.adapters.transformers import disable_turboquant_attention, enable_turboquant_attention

    ids = torch.randint(0, 94, (1, 200), generator=torch.Generator().manual_seed(1)).to(cuda)
    with torch.inference_mode():
        pre = model(input_ids=ids, use_cache=True)
        packed = build_packed_mse_cache(pre.past_key_values, bits=4, use_qjl_keys=True, quantize_decode=True)
        old = enable_turboquant_attention(model, packed)
        captured = []  # attention output = input of o_proj, [1, 1, Hq * D]
        hooks = [layer.self_attn.o_proj.register_forward_pre_hook(
            lambda mod, args: captured.append(args[0].detach().clone())) for layer in model.model.layers]
        nxt = pre.logits[:, -1:].argmax(-1)
        queries = []
        qhooks = [layer.self_attn.q_proj.register_forward_hook(lambda m, a, o: queries.append(o.detach().clone()))
                  for layer in model.model.layers]
        model(input_ids=nxt, past_key_values=packed, use_cache=True)
        for h in hooks + qhooks:
            h.remove()
        disable_turboquant_attention(model, packed, old)
    assert packed.layers[0].packed_seq_length() == 201  # the decode token was appended
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    # recompute each layer's attention from its packed cache with the oracle, using the
    # post-RoPE query the layer saw (q_proj output through the layer's rotary embedding)
    for li in range(len(model.model.layers)):
        q = queries[li].view(1, 1, -1, D).transpose(1, 2)  # [1, Hq, 1, D] pre-RoPE
        cos, sin = model.model.rotary_emb(q, torch.tensor([[200]], device=cuda))
        q_rot, _ = apply_rotary_pos_emb(q, q, cos, sin)
        q16 = q_rot.to(torch.bfloat16)
        ref = O.fused_attention_f64(u16(q16[:, :, 0, :]), host_layer(packed.layers[li]))
        # the same call with an fp32 query returns the kernel's fp32 output (held to the
        # contract); the model saw its bf16 rounding
        got32 = fused_attention(q16.float(), packed.layers[li], model.config.num_attention_heads //
                                model.config.num_key_value_heads)
        err = np.abs(got32[:, :, 0].cpu().numpy() - ref).max()
        assert err <= TOL * np.abs(ref).max(), (li, err)
        seen = u16(captured[li].view(1, -1, D))
        assert np.array_equal(seen, O.f32_to_bf16_bits(got32[:, :, 0].cpu().numpy())), li


def test_dense_decode_buffer_merge(cuda):
    """quantize_decode=False: generated tokens stay dense and are merged with the
    packed history by log-sum-exp (GQA-correct, unlike the reference's merge)."""
    B, Hq, Hkv, N, n_dense = 2, 8, 2, 700, 5
    k = kv_bf16((B, Hkv, N, D), seed=1, device=cuda)
    v = kv_bf16((B, Hkv, N, D), seed=2, device=cuda)
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=False)
    layer.initialize_from_dense(k, v)
    layer._lazy_update = True
    dk = kv_bf16((B, Hkv, n_dense, D), seed=3, device=cuda)
    dv = kv_bf16((B, Hkv, n_dense, D), seed=4, device=cuda)
    for t in range(n_dense):
        layer.update(dk[:, :, t:t + 1], dv[:, :, t:t + 1])
    assert layer.packed_seq_length() == N and layer.get_seq_length() == N + n_dense
    q = query_bf16(B, Hq, D, seed=5, device=cuda)
    out = fused_attention(q.float().unsqueeze(2), layer, Hq // Hkv)[:, :, 0].cpu().numpy()
    kh, vh = O.dequant_layer_f64(host_layer(layer))
    kk = np.concatenate([kh, O.bf16_bits_to_f32(u16(dk)).astype(np.float64)], axis=2)
    vv = np.concatenate([vh, O.bf16_bits_to_f32(u16(dv)).astype(np.float64)], axis=2)
    qf = O.bf16_bits_to_f32(u16(q)).astype(np.float64)
    g = Hq // Hkv
    ref = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            lg = kk[b, h // g] @ qf[b, h] / math.sqrt(D)
            p = np.exp(lg - lg.max())
            ref[b, h] = p @ vv[b, h // g] / p.sum()
    assert np.abs(out - ref).max() <= TOL * np.abs(ref).max()


def test_left_padded_batch_decode(cuda):
    """Batch of 3 with left padding: each row attends to its own valid slots only."""
    B, Hq, Hkv, N = 3, 8, 2, 600
    k = kv_bf16((B, Hkv, N, D), seed=11, device=cuda)
    v = kv_bf16((B, Hkv, N, D), seed=12, device=cuda)
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(k, v)
    pad = [0, 37, 400]
    mask = torch.ones(B, N, dtype=torch.bool, device=cuda)
    for b, p in enumerate(pad):
        mask[b, :p] = False
    q = query_bf16(B, Hq, D, seed=13, device=cuda)
    out = fused_attention(q.float().unsqueeze(2), layer, Hq // Hkv, mask[:, None, None, :])[:, :, 0].cpu().numpy()
    ref = O.fused_attention_f64(u16(q), host_layer(layer), n_start=np.array(pad))
    assert np.abs(out - ref).max() <= TOL * np.abs(ref).max()


class _AttnModule(torch.nn.Module):
    """The attributes the attention backend reads from an HF attention module."""

    def __init__(self, layer, groups):
        super().__init__()
        self._tq_cache_layer = layer
        self.num_key_value_groups = groups


def _dense_rows_reference(layer: PackedMSELayer, q: torch.Tensor, attend: np.ndarray) -> np.ndarray:
    """fp64 attention over the layer's decoded bf16 K / V rows (what the chunked path attends
    to), with an arbitrary boolean mask attend[B, N]."""
    n = layer.packed_seq_length()
    kk = O.bf16_bits_to_f32(u16(layer._decode_keys_range(0, n))).astype(np.float64)
    vv = O.bf16_bits_to_f32(u16(layer._decode_values_range(0, n))).astype(np.float64)
    qf = O.bf16_bits_to_f32(u16(q)).astype(np.float64)
    B, Hq, _ = qf.shape
    g = Hq // kk.shape[1]
    ref = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            lg = kk[b, h // g] @ qf[b, h] / math.sqrt(D)
            lg[~attend[b]] = -np.inf
            p = np.exp(lg - lg.max())
            ref[b, h] = p @ vv[b, h // g] / p.sum()
    return ref


def test_right_padded_batch_takes_the_exact_path(cuda):
    """Right padding followed by generated tokens leaves a hole in a row's attended slots.
    The fused kernel takes one range per row, so fused_attention declines (None) and the
    backend attends through the chunked path with the full mask: the padded slots are
    excluded exactly."""
    from turboquant.runtime.attention import turboquant_attention_forward

    B, Hq, Hkv, N, T = 2, 8, 2, 600, 3
    k = kv_bf16((B, Hkv, N + T, D), seed=61, device=cuda)
    v = kv_bf16((B, Hkv, N + T, D), seed=62, device=cuda)
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(k[:, :, :N], v[:, :, :N])
    layer._lazy_update = True
    for t in range(N, N + T):
        layer.update(k[:, :, t:t + 1], v[:, :, t:t + 1])
    attend = torch.ones(B, N + T, dtype=torch.bool, device=cuda)
    attend[1, 500:N] = False  # row 1: a 500-token prompt right-padded to 600, then 3 generated
    mask4 = attend[:, None, None, :]
    q = query_bf16(B, Hq, D, seed=63, device=cuda)
    assert fused_attention(q.unsqueeze(2), layer, Hq // Hkv, mask4) is None
    # an fp32 query: the chunked path's fp32 result over the decoded bf16 rows
    out, _ = turboquant_attention_forward(_AttnModule(layer, Hq // Hkv), q.float().unsqueeze(2), None, None, mask4)
    ref = _dense_rows_reference(layer, q, attend.cpu().numpy())
    err = np.abs(out[:, 0].cpu().numpy() - ref).max()
    assert err <= TOL * np.abs(ref).max(), err
    # the same layer without the hole goes through the fused kernel
    attend[1, 500:N] = True
    assert fused_attention(q.unsqueeze(2), layer, Hq // Hkv, attend[:, None, None, :]) is not None


def test_gqa_wider_than_the_kernels_takes_the_chunked_path(cuda):
    """16 query heads per KV head: the fused kernels take at most 8, so fused_attention
    returns None (the reference's "not applicable") and the backend falls through to the
    chunked path instead of failing."""
    from turboquant.runtime.attention import turboquant_attention_forward

    B, Hq, Hkv, N = 1, 32, 2, 300
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(kv_bf16((B, Hkv, N, D), seed=71, device=cuda),
                                kv_bf16((B, Hkv, N, D), seed=72, device=cuda))
    q = query_bf16(B, Hq, D, seed=73, device=cuda)
    assert fused_attention(q.unsqueeze(2), layer, Hq // Hkv) is None
    out, _ = turboquant_attention_forward(_AttnModule(layer, Hq // Hkv), q.float().unsqueeze(2), None, None, None)
    ref = _dense_rows_reference(layer, q, np.ones((B, N), bool))
    assert np.abs(out[:, 0].cpu().numpy() - ref).max() <= TOL * np.abs(ref).max()
