"""chunked_turboquant_attention (reference runtime/attention.py:215-304) on the GPU: any
number of query tokens against a packed layer, libtq decoding the history chunk by chunk.
Checked against the reference's own chunked output on the golden layer, against fp64
attention over the same decoded rows (with masks, the dense buffer and split layers), and
against the fused kernel for one query token."""

import math

import numpy as np
import pytest
import torch

from turboquant.runtime.attention import chunked_turboquant_attention, fused_attention, turboquant_attention_forward
from turboquant.runtime.packed_qmse_cache import PackedMSELayer
from turboquant.runtime.synthetic import kv_bf16

pytestmark = pytest.mark.gpu

D = 128


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f64(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("name", ["prod4", "mse3"])
def test_chunked_matches_reference_chunked_output(cuda, golden_dir, name):
    """The reference's chunked output on its golden layer, bit for bit up to one bf16 ulp
    (fp32 summation order on the GPU vs the reference's CPU)."""
    att = np.load(golden_dir / "attention_small.npz")
    bits, qjl, hq, hkv, n = (int(v) for v in att[f"{name}_meta"])
    layer = PackedMSELayer(bits=bits, use_qjl_keys=bool(qjl), quantize_decode=True)
    dummy = torch.zeros(1, hkv, n, D, dtype=torch.bfloat16, device=cuda)
    layer.initialize_from_dense(dummy, dummy)
    s = layer._store
    put = lambda buf, arr, f16=False: buf[:, :, :n].copy_(  # noqa: E731
        torch.from_numpy(arr.view(np.float16) if f16 else arr).to(cuda))
    put(s.kc, att[f"{name}_kcodes"])
    put(s.kn, att[f"{name}_knorms"], True)
    put(s.vc, att[f"{name}_vcodes"])
    put(s.vn, att[f"{name}_vnorms"], True)
    if qjl:
        put(s.ks, att[f"{name}_signs"])
        put(s.kr, att[f"{name}_rnorms"], True)
    q = torch.from_numpy(att[f"{name}_q_bf16"].view(np.int16)).view(torch.bfloat16).to(cuda)
    out = chunked_turboquant_attention(q, layer, n_kv_groups=hq // hkv)
    got = f64(out)
    ref = (att[f"{name}_out_bf16"].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert np.abs(got - ref).max() <= 2 ** -8 * np.abs(ref).max()
    assert (u16(out) == att[f"{name}_out_bf16"]).mean() > 0.95  # nearly all elements bit-identical


def _oracle(q, keys, values, mask, g):
    """fp64 softmax attention; q [B,Q,Sq,D], keys/values [B,Hkv,T,D], mask additive [B,1,Sq,T]."""
    B, Q, Sq, _ = q.shape
    out = np.zeros(q.shape)
    for b in range(B):
        for h in range(Q):
            lg = q[b, h] @ keys[b, h // g].T / math.sqrt(D) + mask[b, 0]
            mx = lg.max(axis=-1, keepdims=True)
            p = np.where(np.isfinite(lg), np.exp(lg - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
            ssum = p.sum(axis=-1, keepdims=True)
            out[b, h] = (p @ values[b, h // g]) / np.maximum(ssum, 1e-8)
    return out


@pytest.mark.parametrize("split", [False, True])
def test_chunked_multi_token_with_masks_and_dense_buffer(cuda, split):
    """3 query tokens, a packed history spanning three 1024-token chunks, 2 dense tokens, a
    boolean mask with a left-padded row and a causal tail: fp64 attention over the same
    decoded bf16 rows."""
    B, Hq, Hkv, N, nd, Sq = 2, 8, 2, 2500, 2, 3
    k = kv_bf16((B, Hkv, N + nd, D), seed=91, device=cuda, outlier_channels=4)
    v = kv_bf16((B, Hkv, N + nd, D), seed=92, device=cuda)
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=False, num_outlier_channels=4 if split else 0)
    layer.initialize_from_dense(k[:, :, :N], v[:, :, :N])
    layer._lazy_update = True
    for t in range(N, N + nd):
        layer.update(k[:, :, t:t + 1], v[:, :, t:t + 1])
    assert layer._outlier_enabled == split
    T = N + nd
    mask = torch.ones(B, 1, Sq, T, dtype=torch.bool, device=cuda)
    mask[1, :, :, :100] = False          # left padding of row 1
    mask[:, :, 0, T - 2:] = False        # causal tail: query 0 sees neither dense token
    mask[:, :, 1, T - 1:] = False
    q = torch.randn(B, Hq, Sq, D, generator=torch.Generator(device=cuda).manual_seed(93), device=cuda)
    q = q.to(torch.bfloat16).float()  # fp32 query -> fp32 output
    out = chunked_turboquant_attention(q, layer, n_kv_groups=Hq // Hkv, attention_mask=mask)
    keys = np.concatenate([f64(layer._decode_keys_full()), f64(k[:, :, N:])], axis=2)
    values = np.concatenate([f64(layer._decode_values_full()), f64(v[:, :, N:])], axis=2)
    add = np.where(mask.cpu().numpy(), 0.0, -np.inf)
    ref = _oracle(f64(q), keys, values, add, Hq // Hkv)
    assert np.abs(f64(out) - ref).max() <= 1e-5 * np.abs(ref).max()


def test_chunked_one_token_agrees_with_fused_and_backend_routes_multi_token(cuda):
    """One query token: the chunked path (bf16 K/V rows, the reference's arithmetic) lies
    within the bf16-rounding band of the fused kernel (unrounded formula).  Several query
    tokens through the attention backend go to the chunked path."""
    B, Hq, Hkv, N = 1, 8, 2, 1500
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(kv_bf16((B, Hkv, N, D), seed=94, device=cuda),
                                kv_bf16((B, Hkv, N, D), seed=95, device=cuda))
    q = torch.randn(B, Hq, 2, D, generator=torch.Generator(device=cuda).manual_seed(96), device=cuda)
    q = q.to(torch.bfloat16).float()
    fused = fused_attention(q[:, :, :1], layer, Hq // Hkv)
    chunk = chunked_turboquant_attention(q[:, :, :1], layer, n_kv_groups=Hq // Hkv)
    assert np.abs(f64(chunk) - f64(fused)).max() <= 3e-2 * np.abs(f64(fused)).max()
    assert fused_attention(q, layer, Hq // Hkv) is None  # reference contract for several tokens

    class Attn(torch.nn.Module):
        num_key_value_groups = Hq // Hkv

    mod = Attn()
    mod._tq_cache_layer = layer
    out, _ = turboquant_attention_forward(mod, q, None, None, None)
    assert out.shape == (B, 2, Hq, D)
    ref = chunked_turboquant_attention(q, layer, n_kv_groups=Hq // Hkv)
    assert torch.equal(out, ref.transpose(1, 2))
