"""Faithful torch restatement of the reference's CPU path -- TEST INFRASTRUCTURE ONLY.

This is the "repo's torch reference quantize+dequant path on CPU" that the
benchmark times as its CPU baseline, and the source of reference-style
outputs at sizes the committed golden vectors do not cover.  It issues the
same torch operations in the same order as the reference, so on the same
torch build it reproduces the reference's bits:

  pack_indices            runtime/packed_qmse_cache.py:13-43
  unpack_indices          runtime/packed_qmse_cache.py:46-55
  encode_group            runtime/packed_qmse_cache.py:376-402
  decode_group (CPU)      runtime/packed_qmse_cache.py:428-435
  encode_keys_qjl_group   runtime/packed_qmse_cache.py:285-310, 148-154
  decode_keys_qjl_group   runtime/packed_qmse_cache.py:312-330
  chunked_attention       runtime/attention.py:189-304 (packed history only)
  detect_outlier_channels runtime/packed_qmse_cache.py:95-114
  encode_split            runtime/packed_qmse_cache.py:481-496 (+ :437-454 for Q_prod keys)
  decode_merge            runtime/packed_qmse_cache.py:498-515 (+ :456-479 for Q_prod keys)

Pinned by tests/test_oracle_golden.py against the reference's own outputs.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import ceil, pi, sqrt

import torch


def pack_indices(indices: torch.Tensor, bits: int) -> torch.Tensor:
    m, d = indices.shape
    flat = indices.reshape(-1).to(torch.int32)
    planes = ((flat.unsqueeze(1) >> torch.arange(bits, dtype=torch.int32)) & 1).to(torch.uint8).reshape(-1)
    nbytes = ceil(d * bits / 8)
    pad = nbytes * 8 - d * bits
    stream = planes.view(m, d * bits)
    if pad:
        stream = torch.cat((stream, torch.zeros((m, pad), dtype=torch.uint8)), dim=1)
    stream = stream.reshape(-1)
    tail = (-int(stream.numel())) % 8
    if tail:
        stream = torch.cat((stream, torch.zeros(tail, dtype=torch.uint8)))
    weights = (2 ** torch.arange(8, dtype=torch.int32)).to(torch.uint8)
    return (stream.view(-1, 8) * weights).sum(dim=1).to(torch.uint8).view(m, nbytes).contiguous()


def unpack_indices(packed: torch.Tensor, bits: int, dim: int) -> torch.Tensor:
    m = packed.shape[0]
    b = ((packed.to(torch.int32).unsqueeze(-1) >> torch.arange(8, dtype=torch.int32)) & 1).reshape(-1)
    b = b.view(m, -1)[:, : dim * bits].reshape(-1).view(m * dim, bits)
    return (b * 2 ** torch.arange(bits, dtype=torch.int32)).sum(dim=1).to(torch.int64).view(m, dim)


@dataclass
class Packed:
    codes: torch.Tensor  # u8 [B,H,N,row]
    norms: torch.Tensor  # f16 [B,H,N]
    shape: tuple
    dtype: torch.dtype
    bits: int


def encode_group(x: torch.Tensor, rotation, centers, boundaries, bits: int) -> Packed:
    x32 = x.detach().to(torch.float32)
    shape = tuple(int(s) for s in x32.shape)
    flat = x32.reshape(-1, shape[-1])
    n = torch.linalg.norm(flat, dim=1)
    n = torch.where(n > 0, n, torch.ones_like(n))
    idx = torch.bucketize((flat / n.unsqueeze(1)) @ rotation.T, boundaries).to(torch.int64)
    return Packed(pack_indices(idx, bits).view(shape[0], shape[1], shape[2], -1),
                  n.to(torch.float16).view(shape[0], shape[1], shape[2]), shape, x.dtype, bits)


def decode_group(p: Packed, rotation, centers) -> torch.Tensor:
    m = p.shape[0] * p.shape[1] * p.shape[2]
    idx = unpack_indices(p.codes.view(m, -1), p.bits, p.shape[-1])
    rec = (centers[idx] @ rotation) * p.norms.view(-1).to(torch.float32).unsqueeze(1)
    return rec.view(p.shape).to(p.dtype)


def encode_keys_qjl_group(x, rotation, centers, boundaries, bits, qjl):
    mse = encode_group(x, rotation, centers, boundaries, bits)
    res = x.float() - decode_group(mse, rotation, centers).float()
    shape = tuple(int(s) for s in x.shape)
    flat = res.reshape(-1, shape[-1])
    rn = torch.linalg.norm(flat, dim=1)
    rn = torch.where(rn > 0, rn, torch.ones_like(rn))
    s = torch.sign((flat / rn.unsqueeze(1)) @ qjl.T)
    s[s == 0] = 1.0
    sign_bits = ((s.reshape(-1, shape[-1]) + 1) // 2).to(torch.int64)
    signs = pack_indices(sign_bits, 1).view(shape[0], shape[1], shape[2], -1)
    return mse, signs, rn.to(torch.float16).view(shape[0], shape[1], shape[2])


def decode_keys_qjl_group(mse: Packed, signs, rnorms, rotation, centers, qjl) -> torch.Tensor:
    base = decode_group(mse, rotation, centers)
    dim = mse.shape[-1]
    m = mse.shape[0] * mse.shape[1] * mse.shape[2]
    pm = 2 * unpack_indices(signs.view(m, -1), 1, dim).to(torch.float32) - 1
    corr = (pm @ qjl) * rnorms.view(-1).to(torch.float32).unsqueeze(1) * (sqrt(pi / 2) / dim)
    return base + corr.view(mse.shape).to(base.dtype)


def _slice(p: Packed, a: int, b: int) -> Packed:
    return Packed(p.codes[:, :, a:b, :].contiguous(), p.norms[:, :, a:b].contiguous(),
                  (p.shape[0], p.shape[1], b - a, p.shape[3]), p.dtype, p.bits)


def chunked_attention(q: torch.Tensor, layer: dict, n_kv_groups: int, chunk_size: int = 1024) -> torch.Tensor:
    """q [B,Q,Sq,D]; ``layer`` holds Packed keys/values (+ signs, rnorms) and fp32 params."""
    B, Q, Sq, D = q.shape
    hs = 1.0 / sqrt(D)
    qf = q.float()
    m_run = torch.tensor(float("-inf")).expand(B, Q, Sq, 1).clone()
    s_run = torch.zeros(B, Q, Sq, 1)
    o_run = torch.zeros(B, Q, Sq, D)
    keys: Packed = layer["keys"]
    vals: Packed = layer["values"]
    total = keys.shape[2]
    for a in range(0, total, chunk_size):
        b = min(a + chunk_size, total)
        ks = _slice(keys, a, b)
        if layer.get("signs") is not None:
            kc = decode_keys_qjl_group(ks, layer["signs"][:, :, a:b].contiguous(),
                                       layer["rnorms"][:, :, a:b].contiguous(), layer["Rk"], layer["Ck"], layer["S"])
        else:
            kc = decode_group(ks, layer["Rk"], layer["Ck"])
        kc = kc.repeat_interleave(n_kv_groups, dim=1) if n_kv_groups > 1 else kc
        logits = (qf @ kc.float().transpose(-2, -1)) * hs
        vc = decode_group(_slice(vals, a, b), layer["Rv"], layer["Cv"])
        vc = vc.repeat_interleave(n_kv_groups, dim=1) if n_kv_groups > 1 else vc
        cmax = logits.max(dim=-1, keepdim=True).values
        m_new = torch.maximum(m_run, cmax)
        corr = torch.exp(m_run - m_new)
        s_run = s_run * corr
        o_run = o_run * corr
        e = torch.exp(logits - m_new)
        s_run = s_run + e.sum(dim=-1, keepdim=True)
        o_run = o_run + e @ vc.float()
        m_run = m_new
    return (o_run / s_run.clamp(min=1e-8)).to(q.dtype)


def encode_layer(k: torch.Tensor, v: torch.Tensor, params: dict, use_qjl: bool, bits: int) -> dict:
    """Reference initialize_from_dense (runtime/packed_qmse_cache.py:359-374) on CPU."""
    out = dict(params)
    if use_qjl:
        out["keys"], out["signs"], out["rnorms"] = encode_keys_qjl_group(
            k, params["Rk"], params["Ck"], params["Bk"], bits - 1, params["S"])
    else:
        out["keys"] = encode_group(k, params["Rk"], params["Ck"], params["Bk"], bits)
        out["signs"] = out["rnorms"] = None
    out["values"] = encode_group(v, params["Rv"], params["Cv"], params["Bv"], bits)
    return out


def detect_outlier_channels(k: torch.Tensor, v: torch.Tensor, n: int) -> tuple[torch.Tensor, torch.Tensor]:
    combined = k.float().pow(2).sum(dim=(0, 1, 2)) + v.float().pow(2).sum(dim=(0, 1, 2))
    _, top = torch.topk(combined, n)
    outlier = top.sort().values
    mask = torch.ones(k.shape[-1], dtype=torch.bool)
    mask[outlier] = False
    return outlier, torch.arange(k.shape[-1])[mask]


def encode_split(x: torch.Tensor, groups: list[dict], use_qjl: bool) -> list[dict]:
    """Each group dict holds ``idx`` (channels), ``R``, ``C``, ``B``, ``bits`` (MSE bits) and,
    for Q_prod keys, ``S``.  Returns per group {"packed", "signs", "rnorms"}."""
    out = []
    for g in groups:
        sub = x[..., g["idx"]]
        if use_qjl:
            mse, signs, rn = encode_keys_qjl_group(sub, g["R"], g["C"], g["B"], g["bits"], g["S"])
            out.append({"packed": mse, "signs": signs, "rnorms": rn})
        else:
            out.append({"packed": encode_group(sub, g["R"], g["C"], g["B"], g["bits"]), "signs": None,
                        "rnorms": None})
    return out


def decode_merge(encoded: list[dict], groups: list[dict], full_dim: int) -> torch.Tensor:
    parts = []
    for e, g in zip(encoded, groups):
        if e["signs"] is not None:
            parts.append(decode_keys_qjl_group(e["packed"], e["signs"], e["rnorms"], g["R"], g["C"], g["S"]))
        else:
            parts.append(decode_group(e["packed"], g["R"], g["C"]))
    b, h, n = parts[0].shape[:3]
    full = torch.zeros(b, h, n, full_dim, dtype=parts[0].dtype)
    for part, g in zip(parts, groups):
        full[..., g["idx"]] = part
    return full
