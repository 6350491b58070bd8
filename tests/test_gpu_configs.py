"""BASELINE config 4 end to end on the GPU: a Qwen2.5-7B-style 28-layer cache with
norm-asymmetric keys, the norm guard, 256 decode-append steps and decode attention.

Generator (the choices the configuration leaves open):
* key directions iid N(0, 1) with 2 outlier channels (0 and 1; 1% of 128 rounds to 1-2)
  scaled x10 before normalising, so the norms below are exactly the drawn ones;
* key norms lognormal with sigma 0.5 and mean 200 in layers 0 and 27 (mu = ln 200 - 0.125),
  mean 16.8 elsewhere (the reference's notes for Qwen 2.5 7B: ~16.8 in the regular layers,
  239-274 in layers 0 and 27), so the norm guard's threshold sqrt(D / 0.009) = 119.3 keeps
  exactly layers 0 and 27 dense;
* value norms lognormal with mean 5, sigma 0.3.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from turboquant.runtime.attention import fused_attention
from turboquant.runtime.packed_qmse_cache import build_packed_mse_cache
from turboquant.runtime.synthetic import query_bf16

pytestmark = pytest.mark.gpu

D = 128
TOL = 2e-3
B, HQ, HKV, N, LAYERS, STEPS = 4, 28, 4, 32768, 28, 256


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _kv(shape, mean, sigma, seed, device, outliers=0):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(*shape, generator=g, device=device)
    if outliers:
        x[..., :outliers] *= 10.0
    x = x / x.norm(dim=-1, keepdim=True)
    mu = math.log(mean) - sigma ** 2 / 2
    return (x * torch.exp(mu + sigma * torch.randn(*shape[:-1], generator=g, device=device))[..., None]).to(
        torch.bfloat16)


def _layer_kv(li, T, seed, device):
    kmean = 200.0 if li in (0, LAYERS - 1) else 16.8
    k = _kv((B, HKV, T, D), kmean, 0.5, seed, device, outliers=2)
    v = _kv((B, HKV, T, D), 5.0, 0.3, seed + 1, device)
    return k, v


def _host_layer(layer, b):
    s, c, n = layer._store, layer.codecs, layer.packed_seq_length()
    return {"kcodes": s.kc[b:b + 1, :, :n].cpu().numpy(), "knorms": u16(s.kn[b:b + 1, :, :n]),
            "vcodes": s.vc[b:b + 1, :, :n].cpu().numpy(), "vnorms": u16(s.vn[b:b + 1, :, :n]),
            "signs": s.ks[b:b + 1, :, :n].cpu().numpy(), "rnorms": u16(s.kr[b:b + 1, :, :n]),
            "Rk": c.key.rotation.cpu().numpy(), "Ck": c.key.centers.cpu().numpy(),
            "Rv": c.value.rotation.cpu().numpy(), "Cv": c.value.centers.cpu().numpy(),
            "S": c.qjl.cpu().numpy(), "kbits": c.key_bits, "vbits": c.value_bits}


def test_c4_norm_guard_decode_append_and_attention(cuda):
    kv = [_layer_kv(li, N, 100 + 2 * li, cuda) for li in range(LAYERS)]
    cache = build_packed_mse_cache(kv, bits=4, use_qjl_keys=True, quantize_decode=True)
    dense = [i for i, layer in enumerate(cache.layers) if layer._force_dense]
    assert dense == [0, LAYERS - 1]
    for layer in cache.layers:
        layer._lazy_update = True  # as the attention backend wires it
    # 256 decode steps: each appends one token per layer and attends over every packed layer
    new = [_layer_kv(li, STEPS, 9000 + 2 * li, cuda) for li in range(LAYERS)]
    q = query_bf16(B, HQ, D, seed=5, device=cuda).unsqueeze(2)
    for t in range(STEPS):
        for li, layer in enumerate(cache.layers):
            layer.update(new[li][0][:, :, t:t + 1], new[li][1][:, :, t:t + 1])
            if not layer._force_dense:
                fused_attention(q, layer, HQ // HKV)
    torch.cuda.synchronize()
    assert cache.layers[0].get_seq_length() == N + STEPS and cache.layers[0].packed_seq_length() == 0
    layer = cache.layers[1]
    assert layer.packed_seq_length() == N + STEPS
    # decode-appended tokens are encoded exactly as prefill would encode them
    c = layer.codecs
    ks = u16(new[1][0]).reshape(-1, D)
    rc, rn, rs, rr = O.encode_prod(ks, 3, c.key.rotation.cpu().numpy(), c.key.centers.cpu().numpy(),
                                   c.key.boundaries.cpu().numpy(), c.qjl.cpu().numpy())
    s = layer._store
    assert np.array_equal(s.kc[:, :, N:N + STEPS].cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(s.ks[:, :, N:N + STEPS].cpu().numpy().reshape(rs.shape), rs)
    assert np.array_equal(u16(s.kn[:, :, N:N + STEPS]).reshape(-1), rn)
    assert np.array_equal(u16(s.kr[:, :, N:N + STEPS]).reshape(-1), rr)
    vc, vn = O.encode_mse(u16(new[1][1]).reshape(-1, D), 4, c.value.rotation.cpu().numpy(),
                          c.value.boundaries.cpu().numpy())
    assert np.array_equal(s.vc[:, :, N:N + STEPS].cpu().numpy().reshape(vc.shape), vc)
    assert np.array_equal(u16(s.vn[:, :, N:N + STEPS]).reshape(-1), vn)
    # attention over the final 33,024-token cache of batch row 3 (GQA 7) against the fp64 formula
    got = fused_attention(q.float(), layer, HQ // HKV)  # fp32 query: the kernel's fp32 output
    assert got.dtype == torch.float32
    ref = O.fused_attention_f64(u16(q[3:4, :, 0]), _host_layer(layer, 3))
    err = np.abs(got[3:4, :, 0].cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= TOL, err
    # the bf16 result of a bf16 query is the RNE rounding of that fp32 output
    got16 = fused_attention(q, layer, HQ // HKV)
    assert np.array_equal(u16(got16), O.f32_to_bf16_bits(got.cpu().numpy()))
    # dense layers attend through SDPA in the model; their cache holds the raw tokens
    assert torch.equal(cache.layers[0]._dense_keys[:, :, N:], new[0][0])
