"""BASELINE config 5 on the GPU: decode attention at its final shape, and a
reduced-depth QwQ-32B-architecture model run end to end through
``turboquant.activate``.

* The kernel at the config-5 decode shape (B=1, Hq=40, Hkv=8 -- GQA 5 --, N=131,584,
  4-bit Q_prod keys / 4-bit Q_mse values), KV groups 0 and 7 against the fp64 oracle.
* A random-init Qwen2 model with QwQ-32B dimensions (hidden 5120, 40 / 8 heads,
  head_dim 128, SwiGLU 27648, vocab 152064, rope theta 1e6, bf16) but 2 layers instead
  of 64: a 131,072-token prompt, then 3 greedy tokens with EOS disabled.  Every layer's
  attention output at the last decode step is recomputed with an fp32 query (held to
  2e-3 * ||out||_inf against the oracle on two KV groups) and the model saw its bf16
  rounding; the telemetry's byte counts follow from the shape.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from turboquant.runtime import kernels as K
from turboquant.runtime.attention import fused_attention
from turboquant.runtime.params import layer_codecs
from turboquant.runtime.synthetic import kv_bf16, query_bf16

pytestmark = pytest.mark.gpu

D = 128
TOL = 2e-3
HQ, HKV = 40, 8
G = HQ // HKV
CHECK_GROUPS = (0, HKV - 1)


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_groups(store, codecs, n, groups):
    """Host copy of batch row 0, KV heads `groups`, slots [0, n) of a packed store."""
    idx = list(groups)
    pick = lambda t: t[:1, idx, :n]  # noqa: E731
    return {"kcodes": pick(store["kc"]).cpu().numpy(), "knorms": u16(pick(store["kn"])),
            "vcodes": pick(store["vc"]).cpu().numpy(), "vnorms": u16(pick(store["vn"])),
            "signs": pick(store["ks"]).cpu().numpy(), "rnorms": u16(pick(store["kr"])),
            "Rk": codecs.key.rotation.cpu().numpy(), "Ck": codecs.key.centers.cpu().numpy(),
            "Rv": codecs.value.rotation.cpu().numpy(), "Cv": codecs.value.centers.cpu().numpy(),
            "S": codecs.qjl.cpu().numpy(), "kbits": codecs.key_bits, "vbits": codecs.value_bits}


def query_heads(q, groups):
    """The query heads [B, len(groups) * G, ...] of KV heads `groups`."""
    return torch.cat([q[:, g * G:(g + 1) * G] for g in groups], dim=1)


def test_c5_shape_decode_attention(cuda):
    N = 131072 + 512
    lc = layer_codecs(D, 4, 0, True, cuda)
    k = kv_bf16((1, HKV, N, D), seed=51, device=cuda)
    v = kv_bf16((1, HKV, N, D), seed=52, device=cuda)
    st = {"kc": torch.empty(1, HKV, N, 48, dtype=torch.uint8, device=cuda),
          "kn": torch.empty(1, HKV, N, dtype=torch.float16, device=cuda),
          "ks": torch.empty(1, HKV, N, 16, dtype=torch.uint8, device=cuda),
          "kr": torch.empty(1, HKV, N, dtype=torch.float16, device=cuda),
          "vc": torch.empty(1, HKV, N, 64, dtype=torch.uint8, device=cuda),
          "vn": torch.empty(1, HKV, N, dtype=torch.float16, device=cuda)}
    K.quantize_prod(k, lc.key, lc.qjl, st["kc"], st["kn"], st["ks"], st["kr"])
    K.quantize_mse(v, lc.value, st["vc"], st["vn"])
    del k, v
    q = query_bf16(1, HQ, D, seed=53, device=cuda)
    _, out32 = K.decode_attention(q, k_codes=st["kc"], k_norms=st["kn"], v_codes=st["vc"], v_norms=st["vn"],
                                  n_tokens=N, key=lc.key, value=lc.value, k_signs=st["ks"], k_rnorms=st["kr"],
                                  qjl=lc.qjl, want_f32=True)
    torch.cuda.synchronize()
    ref = O.fused_attention_f64(u16(query_heads(q, CHECK_GROUPS)), host_groups(st, lc, N, CHECK_GROUPS))
    got = query_heads(out32, CHECK_GROUPS).cpu().numpy()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    print(f"[c5] decode attention N={N}: max err {err:.2e} of |out|_inf", flush=True)
    assert err <= TOL, err


class IdTokenizer:
    """Bijective id <-> character map over the whole vocabulary (no tokenizer files offline)."""

    eos_token_id = None
    pad_token_id = None
    BASE = 0x20000

    def encode(self, text, add_special_tokens=True):
        return [ord(c) - self.BASE for c in text]

    def decode(self, ids, skip_special_tokens=True):
        return "".join(chr(self.BASE + int(i)) for i in ids)


def qwq_model(device, layers):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=152064, hidden_size=5120, intermediate_size=27648, num_hidden_layers=layers,
                      num_attention_heads=HQ, num_key_value_heads=HKV, max_position_embeddings=131072 + 64,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6}, rms_norm_eps=1e-5,
                      tie_word_embeddings=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen2ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    model.generation_config.eos_token_id = None
    return model


@pytest.mark.parametrize("LAYERS,checked", [(2, (0, 1)), (64, (0, 63))])
def test_c5_architecture_activate_generate(cuda, LAYERS, checked):
    """QwQ-32B dimensions through turboquant.activate: a 131,072-token prompt and 3 greedy
    tokens, with 2 layers and with the full 64 (32.76 B parameters, the configuration's model
    size).  The checked layers' last decode step is held against the oracle."""
    import turboquant
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    P, NEW = 131072, 3
    model = qwq_model(cuda, LAYERS)
    turboquant.activate(model, IdTokenizer(), bits=4, use_qjl_keys=True, quantize_decode=True, quiet=True)
    seen = {li: {} for li in range(LAYERS)}
    hooks = []
    for li, dec in enumerate(model.model.layers):
        att = dec.self_attn

        def pre(mod, args, kwargs, li=li):
            if getattr(mod, "_tq_cache_layer", None) is not None:
                seen[li]["layer"] = mod._tq_cache_layer

        hooks.append(att.register_forward_pre_hook(pre, with_kwargs=True))
        hooks.append(att.q_proj.register_forward_hook(
            lambda m, a, o, li=li: seen[li].__setitem__("q", o.detach().clone()) if o.shape[1] == 1 else None))
        hooks.append(att.o_proj.register_forward_pre_hook(
            lambda m, a, li=li: seen[li].__setitem__("o", a[0].detach().clone()) if a[0].shape[1] == 1 else None))
    ids = torch.randint(0, 152064, (1, P), generator=torch.Generator().manual_seed(5)).to(cuda)
    print(f"[c5] generate: prompt {P}, {NEW} new tokens, {LAYERS} layers", flush=True)
    out = model.generate(ids, max_new_tokens=NEW)
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    assert out.shape == (1, P + NEW) and torch.equal(out[0, :P], ids[0])
    tel = turboquant.last_telemetry(model)
    turboquant.deactivate(model, quiet=True)
    # telemetry: 2 layers x 8 KV heads x P prompt tokens, 134 packed bytes per token-head
    # (48 + 2 + 16 + 2 + 64 + 2) against 2 x 128 x 2 dense bf16 bytes
    assert tel["prompt_tokens"] == P and tel["completion_tokens"] == NEW
    assert tel["dense_kv_bytes"] == LAYERS * HKV * P * 2 * D * 2
    assert tel["packed_actual_bytes"] == LAYERS * HKV * P * 134
    assert tel["payload_savings_percent"] == pytest.approx(100 * (1 - 134 / 512))
    pos = P + NEW - 2  # the last decode step fed token NEW - 1 at this position
    for li in checked:
        layer = seen[li]["layer"]
        n = layer.packed_seq_length()
        assert n == P + NEW - 1  # the prompt plus every token fed back so far
        qr = seen[li]["q"].view(1, 1, HQ, D).transpose(1, 2)  # [1, Hq, 1, D] before RoPE
        cos, sin = model.model.rotary_emb(qr, torch.tensor([[pos]], device=cuda))
        q16, _ = apply_rotary_pos_emb(qr, qr, cos, sin)
        q16 = q16.to(torch.bfloat16)
        got32 = fused_attention(q16.float(), layer, G)[:, :, 0]  # the kernel's fp32 output
        # the model attended with the bf16 query: its output is the RNE rounding of got32
        assert np.array_equal(u16(seen[li]["o"].view(1, HQ, D)), O.f32_to_bf16_bits(got32.cpu().numpy())), li
        s = layer._store
        store = {"kc": s.kc, "kn": s.kn, "ks": s.ks, "kr": s.kr, "vc": s.vc, "vn": s.vn}
        ref = O.fused_attention_f64(u16(query_heads(q16[:, :, 0], CHECK_GROUPS)),
                                    host_groups(store, layer.codecs, n, CHECK_GROUPS))
        err = np.abs(query_heads(got32, CHECK_GROUPS).cpu().numpy() - ref).max() / np.abs(ref).max()
        print(f"[c5] layer {li}: N={n}, max err {err:.2e} of |out|_inf", flush=True)
        assert err <= TOL, (li, err)
    del model, seen, layer, s, store
    torch.cuda.empty_cache()  # the 64-layer model holds ~66 GB
