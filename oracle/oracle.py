"""CPU oracle for the TurboQuant hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker.  The product
(``tq-local_amd/turboquant``) never imports it.

Contents
--------
* ctypes bindings of ``tq_oracle.c`` (fixed-order fp32 encoder, bit-identical
  to the HIP quantizer):  ``encode_mse``, ``encode_prod``, ``decode_mse``,
  ``rotated``.
* numpy restatements of the packed layout (reference
  ``runtime/packed_qmse_cache.py:13-55``): ``pack_codes``, ``unpack_codes``.
* ``fused_attention_f64`` -- the fused decode-attention formula of reference
  ``runtime/triton_kernels.py:84-198`` (per-tile logits, softmax, value
  accumulation) and ``:289-366`` (q-side rotations, cross-tile merge, final
  un-rotation), evaluated in fp64 over the whole sequence at once.
* ``dequant_attention_f64`` -- the same attention computed the long way:
  dequantise K (MSE reconstruction + QJL correction, reference
  ``runtime/packed_qmse_cache.py:312-330``) and V to dense fp64 vectors, then
  plain softmax attention.  Agreement of the two pins the rotation algebra.

* ``split_dequant_f64`` / ``dense_attention_f64`` / ``split_fused_attention_f64`` --
  the outlier-split layer (two channel groups): its fp64 dequantisation, plain
  attention over dense rows, and the fused formula summed over the groups.
  The split encoder itself is ``encode_mse`` / ``encode_prod`` at D = d applied
  to the gathered sub-vectors x[..., channels].

Parity status of each function is pinned by tests/test_oracle_*.py:
  encode_mse / encode_prod  -- reference golden vectors (tie-band), brute force
  pack_codes / unpack_codes -- hand-computed bytes, golden vectors, round trip
  fused_attention_f64       -- dequant_attention_f64 identity, golden chunked
                               output of the reference, LSE-merge identity
  encode_* at D = d < 128   -- tie-band against the torch restatement of the
                               reference (itself bit-exact on the golden vectors),
                               nearest-centroid brute force
  split_dequant_f64         -- the torch restatement's decode_merge (bf16) to
                               within its roundings
  split_fused_attention_f64 -- identity with dense_attention_f64 over
                               split_dequant_f64; one group of all D channels
                               reduces to fused_attention_f64
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "libtq_oracle.so"

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        L.tq_oracle_encode_mse.argtypes = [P, I64, I, I, P, P, P, P]
        L.tq_oracle_encode_prod.argtypes = [P, I64, I, I, P, P, P, P, P, P, P, P]
        L.tq_oracle_decode_mse.argtypes = [P, P, I64, I, I, P, P, P]
        L.tq_oracle_rotated.argtypes = [P, I64, I, P, P]
        L.tq_oracle_decode_prod.argtypes = [P, P, P, P, I64, I, I, P, P, P, P]
        L.tq_oracle_norms.argtypes = [P, I64, I, P]
        L.tq_oracle_f32_to_f16_array.argtypes = [P, I64, P]
        L.tq_oracle_f32_to_bf16_array.argtypes = [P, I64, P]
        for fn in ("tq_oracle_encode_mse", "tq_oracle_encode_prod", "tq_oracle_decode_mse", "tq_oracle_decode_prod",
                   "tq_oracle_rotated", "tq_oracle_norms", "tq_oracle_f32_to_f16_array", "tq_oracle_f32_to_bf16_array"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ----------------------------------------------------------------- numerics
def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().tq_oracle_f32_to_bf16_array(_p(f), f.size, _p(out))
    return out


def f32_to_f16_bits(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().tq_oracle_f32_to_f16_array(_p(f), f.size, _p(out))
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def row_bytes(dim: int, bits: int) -> int:
    return (dim * bits + 7) // 8


# ------------------------------------------------------------------- layout
def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """[M, D] ints -> [M, ceil(D*bits/8)] u8, LSB-first bit stream per row."""
    m, d = codes.shape
    c = codes.astype(np.uint32)
    bitplanes = ((c[:, :, None] >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.uint8)
    stream = bitplanes.reshape(m, d * bits)
    pad = row_bytes(d, bits) * 8 - d * bits
    if pad:
        stream = np.concatenate([stream, np.zeros((m, pad), np.uint8)], axis=1)
    return np.packbits(stream.reshape(m, -1, 8), axis=2, bitorder="little").reshape(m, -1)


def unpack_codes(packed: np.ndarray, bits: int, dim: int) -> np.ndarray:
    """[M, row] u8 -> [M, D] int64 (inverse of pack_codes)."""
    m = packed.shape[0]
    if m == 0:
        return np.zeros((0, dim), np.int64)
    stream = np.unpackbits(packed.reshape(m, -1, 1), axis=2, bitorder="little").reshape(m, -1)
    stream = stream[:, : dim * bits].reshape(m, dim, bits).astype(np.int64)
    return (stream << np.arange(bits, dtype=np.int64)).sum(axis=2)


# ------------------------------------------------------------------ encoder
def encode_mse(x_bf16: np.ndarray, bits: int, R: np.ndarray, boundaries: np.ndarray):
    """x_bf16: [M, D] uint16 -> (codes [M,row] u8, norms [M] u16 f16 bits)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, d = x.shape
    codes = np.zeros((m, row_bytes(d, bits)), np.uint8)
    norms = np.zeros(m, np.uint16)
    lib().tq_oracle_encode_mse(_p(x), m, d, bits, _p(np.ascontiguousarray(R, np.float32)),
                               _p(np.ascontiguousarray(boundaries, np.float32)), _p(codes), _p(norms))
    return codes, norms


def encode_prod(x_bf16: np.ndarray, mse_bits: int, R: np.ndarray, centers: np.ndarray,
                boundaries: np.ndarray, S: np.ndarray):
    """Q_prod keys -> (codes, norms, signs [M, D/8] u8, rnorms)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, d = x.shape
    codes = np.zeros((m, row_bytes(d, mse_bits)), np.uint8)
    norms = np.zeros(m, np.uint16)
    signs = np.zeros((m, row_bytes(d, 1)), np.uint8)
    rnorms = np.zeros(m, np.uint16)
    lib().tq_oracle_encode_prod(_p(x), m, d, mse_bits, _p(np.ascontiguousarray(R, np.float32)),
                                _p(np.ascontiguousarray(centers, np.float32)),
                                _p(np.ascontiguousarray(boundaries, np.float32)),
                                _p(np.ascontiguousarray(S, np.float32)),
                                _p(codes), _p(norms), _p(signs), _p(rnorms))
    return codes, norms, signs, rnorms


def decode_mse(codes: np.ndarray, norms: np.ndarray, bits: int, dim: int, R: np.ndarray, centers: np.ndarray):
    codes = np.ascontiguousarray(codes, np.uint8)
    norms = np.ascontiguousarray(norms, np.uint16)
    m = codes.shape[0]
    out = np.zeros((m, dim), np.uint16)
    lib().tq_oracle_decode_mse(_p(codes), _p(norms), m, dim, bits, _p(np.ascontiguousarray(R, np.float32)),
                               _p(np.ascontiguousarray(centers, np.float32)), _p(out))
    return out


def decode_prod(codes, norms, signs, rnorms, mse_bits: int, dim: int, R, centers, S):
    """Q_prod keys -> bf16 bits [M, D]: MSE reconstruction + bf16 QJL correction."""
    codes = np.ascontiguousarray(codes, np.uint8)
    m = codes.shape[0]
    out = np.zeros((m, dim), np.uint16)
    lib().tq_oracle_decode_prod(_p(codes), _p(np.ascontiguousarray(norms, np.uint16)),
                                _p(np.ascontiguousarray(signs, np.uint8)), _p(np.ascontiguousarray(rnorms, np.uint16)),
                                m, dim, mse_bits, _p(np.ascontiguousarray(R, np.float32)),
                                _p(np.ascontiguousarray(centers, np.float32)), _p(np.ascontiguousarray(S, np.float32)),
                                _p(out))
    return out


def norms(x_bf16: np.ndarray) -> np.ndarray:
    """fp16 bits of the encoder's stored norms, [M] (the norm step of encode_mse alone)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, d = x.shape
    out = np.zeros(m, np.uint16)
    lib().tq_oracle_norms(_p(x), m, d, _p(out))
    return out


def rotated(x_bf16: np.ndarray, R: np.ndarray) -> np.ndarray:
    """fp32 pre-images z = (x/|x|) @ R^T in the encoder's exact order."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, d = x.shape
    z = np.zeros((m, d), np.float32)
    lib().tq_oracle_rotated(_p(x), m, d, _p(np.ascontiguousarray(R, np.float32)), _p(z))
    return z


# ---------------------------------------------------------------- attention
def _sign_pm1(signs_u8: np.ndarray, dim: int) -> np.ndarray:
    return 2.0 * unpack_codes(signs_u8, 1, dim).astype(np.float64) - 1.0


def fused_attention_f64(q_bf16, layer: dict, n_valid: np.ndarray | None = None,
                        n_start: np.ndarray | None = None) -> np.ndarray:
    """Fused decode attention in fp64.

    q_bf16: [B, Hq, D] uint16.  ``layer`` holds (numpy) packed tensors
    ``kcodes [B,Hkv,N,rowk]``, ``knorms [B,Hkv,N]`` (f16 bits), ``vcodes``,
    ``vnorms``, optional ``signs``/``rnorms`` and the fp32 params
    ``Rk, Ck, Rv, Cv, S`` plus ``kbits, vbits``.  Batch row b attends to tokens
    [n_start[b], n_valid[b]) (defaults: 0 and N).  Returns fp64 [B, Hq, D].

    logit_t = (n_k <q Rk^T, Ck[kidx_t]> + sqrt(pi/2)/D * rho_t <q S^T, s_t>) / sqrt(D)
    out     = (sum_t softmax(logit)_t n_v,t Cv[vidx_t]) @ Rv
    """
    q = bf16_bits_to_f32(np.asarray(q_bf16)).astype(np.float64)
    B, Hq, D = q.shape
    kc = layer["kcodes"]
    Hkv, N = kc.shape[1], kc.shape[2]
    g = Hq // Hkv
    Rk = layer["Rk"].astype(np.float64)
    Rv = layer["Rv"].astype(np.float64)
    Ck = layer["Ck"].astype(np.float64)
    Cv = layer["Cv"].astype(np.float64)
    has_qjl = layer.get("signs") is not None
    hs = 1.0 / math.sqrt(D)
    qs = math.sqrt(math.pi / 2) / D
    out = np.zeros((B, Hq, D))
    for b in range(B):
        nb = N if n_valid is None else int(n_valid[b])
        sb = 0 if n_start is None else int(n_start[b])
        if nb <= sb:
            continue  # an empty sequence attends to nothing: output stays zero
        sl = slice(sb, nb)
        for h in range(Hkv):
            kidx = unpack_codes(kc[b, h, sl], layer["kbits"], D)
            vidx = unpack_codes(layer["vcodes"][b, h, sl], layer["vbits"], D)
            kn = f16_bits_to_f32(layer["knorms"][b, h, sl]).astype(np.float64)
            vn = f16_bits_to_f32(layer["vnorms"][b, h, sl]).astype(np.float64)
            qq = q[b, h * g:(h + 1) * g]  # [g, D]
            q_rot = qq @ Rk.T
            logits = (q_rot @ Ck[kidx].T) * kn[None, :]
            if has_qjl:
                q_proj = qq @ layer["S"].astype(np.float64).T
                sg = _sign_pm1(layer["signs"][b, h, sl], D)
                rn = f16_bits_to_f32(layer["rnorms"][b, h, sl]).astype(np.float64)
                logits = logits + qs * rn[None, :] * (q_proj @ sg.T)
            logits = logits * hs
            m = logits.max(axis=1, keepdims=True)
            p = np.exp(logits - m)
            ssum = p.sum(axis=1, keepdims=True)
            o_rot = (p * vn[None, :]) @ Cv[vidx]
            out[b, h * g:(h + 1) * g] = (o_rot / np.maximum(ssum, 1e-8)) @ Rv
    return out


def dequant_layer_f64(layer: dict) -> tuple[np.ndarray, np.ndarray]:
    """fp64 K^ [B,Hkv,N,D] (MSE reconstruction + QJL correction) and V^, unrounded."""
    kc = layer["kcodes"]
    B, Hkv, N = kc.shape[:3]
    D = layer["Rk"].shape[0]
    qs = math.sqrt(math.pi / 2) / D
    kh = np.zeros((B, Hkv, N, D))
    vh = np.zeros((B, Hkv, N, D))
    for b in range(B):
        for h in range(Hkv):
            kidx = unpack_codes(kc[b, h], layer["kbits"], D)
            kn = f16_bits_to_f32(layer["knorms"][b, h]).astype(np.float64)
            kh[b, h] = (layer["Ck"].astype(np.float64)[kidx] @ layer["Rk"].astype(np.float64)) * kn[:, None]
            if layer.get("signs") is not None:
                sg = _sign_pm1(layer["signs"][b, h], D)
                rn = f16_bits_to_f32(layer["rnorms"][b, h]).astype(np.float64)
                kh[b, h] += (sg @ layer["S"].astype(np.float64)) * (rn[:, None] * qs)
            vidx = unpack_codes(layer["vcodes"][b, h], layer["vbits"], D)
            vn = f16_bits_to_f32(layer["vnorms"][b, h]).astype(np.float64)
            vh[b, h] = (layer["Cv"].astype(np.float64)[vidx] @ layer["Rv"].astype(np.float64)) * vn[:, None]
    return kh, vh


def dequant_attention_f64(q_bf16, layer: dict) -> np.ndarray:
    """Same attention via explicit fp64 dequantisation of K and V (no bf16 rounding)."""
    q = bf16_bits_to_f32(np.asarray(q_bf16)).astype(np.float64)
    B, Hq, D = q.shape
    kc = layer["kcodes"]
    Hkv, N = kc.shape[1], kc.shape[2]
    g = Hq // Hkv
    out = np.zeros((B, Hq, D))
    qs = math.sqrt(math.pi / 2) / D
    for b in range(B):
        for h in range(Hkv):
            kidx = unpack_codes(kc[b, h], layer["kbits"], D)
            vidx = unpack_codes(layer["vcodes"][b, h], layer["vbits"], D)
            kn = f16_bits_to_f32(layer["knorms"][b, h]).astype(np.float64)
            vn = f16_bits_to_f32(layer["vnorms"][b, h]).astype(np.float64)
            khat = (layer["Ck"].astype(np.float64)[kidx] @ layer["Rk"].astype(np.float64)) * kn[:, None]
            if layer.get("signs") is not None:
                sg = _sign_pm1(layer["signs"][b, h], D)
                rn = f16_bits_to_f32(layer["rnorms"][b, h]).astype(np.float64)
                khat = khat + (sg @ layer["S"].astype(np.float64)) * (rn[:, None] * qs)
            vhat = (layer["Cv"].astype(np.float64)[vidx] @ layer["Rv"].astype(np.float64)) * vn[:, None]
            for j in range(g):
                lg = khat @ q[b, h * g + j] / math.sqrt(D)
                p = np.exp(lg - lg.max())
                out[b, h * g + j] = (p @ vhat) / p.sum()
    return out


# ------------------------------------------------------------ channel groups
def split_dequant_f64(groups: list[dict], full_dim: int) -> tuple[np.ndarray, np.ndarray]:
    """fp64 K^ and V^ [B,Hkv,N,full_dim] of an outlier-split layer, unrounded: each group
    (a ``dequant_layer_f64`` dict of its own dimension plus ``channels``) decoded and
    scattered to its channels (reference _decode_merge / _decode_keys_merge_qjl,
    runtime/packed_qmse_cache.py:456-515, without the bf16 roundings)."""
    B, Hkv, N = groups[0]["kcodes"].shape[:3]
    kh = np.zeros((B, Hkv, N, full_dim))
    vh = np.zeros((B, Hkv, N, full_dim))
    for g in groups:
        k, v = dequant_layer_f64(g)
        kh[..., g["channels"]] = k
        vh[..., g["channels"]] = v
    return kh, vh


def dense_attention_f64(q_bf16, keys: np.ndarray, values: np.ndarray, n_start=None, n_valid=None) -> np.ndarray:
    """softmax(q . K / sqrt(D)) V in fp64 over dense [B,Hkv,N,D] rows; query head h reads
    KV head h // (Hq/Hkv); row b attends to [n_start[b], n_valid[b]) (empty -> 0)."""
    q = bf16_bits_to_f32(np.asarray(q_bf16)).astype(np.float64)
    B, Hq, D = q.shape
    Hkv, N = keys.shape[1], keys.shape[2]
    g = Hq // Hkv
    out = np.zeros((B, Hq, D))
    for b in range(B):
        lo = 0 if n_start is None else int(n_start[b])
        hi = N if n_valid is None else int(n_valid[b])
        if hi <= lo:
            continue
        for h in range(Hq):
            k = keys[b, h // g, lo:hi].astype(np.float64)
            lg = k @ q[b, h] / math.sqrt(D)
            p = np.exp(lg - lg.max())
            out[b, h] = (p @ values[b, h // g, lo:hi].astype(np.float64)) / p.sum()
    return out


def split_fused_attention_f64(q_bf16, groups: list[dict], full_dim: int) -> np.ndarray:
    """The fused formula over channel groups, in fp64 and in each group's rotated space:
    logit_t = sum_g (n_g <q[ch_g] R_k,g^T, C_k,g[kidx]> + sqrt(pi/2)/d_g rho_g <q[ch_g] S_g^T, s>) / sqrt(D),
    out[ch_g] = (sum_t p_t n_v,g C_v,g[vidx]) R_v,g / sum_t p_t."""
    q = bf16_bits_to_f32(np.asarray(q_bf16)).astype(np.float64)
    B, Hq, D = q.shape
    Hkv, N = groups[0]["kcodes"].shape[1:3]
    G = Hq // Hkv
    out = np.zeros((B, Hq, full_dim))
    for b in range(B):
        for h in range(Hkv):
            qq = q[b, h * G:(h + 1) * G]
            logits = np.zeros((G, N))
            for g in groups:
                d, ch = len(g["channels"]), g["channels"]
                kidx = unpack_codes(g["kcodes"][b, h], g["kbits"], d)
                kn = f16_bits_to_f32(g["knorms"][b, h]).astype(np.float64)
                logits += ((qq[:, ch] @ g["Rk"].astype(np.float64).T) @ g["Ck"].astype(np.float64)[kidx].T) * kn
                if g.get("signs") is not None:
                    sg = _sign_pm1(g["signs"][b, h], d)
                    rn = f16_bits_to_f32(g["rnorms"][b, h]).astype(np.float64)
                    logits += math.sqrt(math.pi / 2) / d * rn * ((qq[:, ch] @ g["S"].astype(np.float64).T) @ sg.T)
            logits /= math.sqrt(D)
            p = np.exp(logits - logits.max(axis=1, keepdims=True))
            ssum = p.sum(axis=1, keepdims=True)
            for g in groups:
                d, ch = len(g["channels"]), g["channels"]
                vidx = unpack_codes(g["vcodes"][b, h], g["vbits"], d)
                vn = f16_bits_to_f32(g["vnorms"][b, h]).astype(np.float64)
                o_rot = (p * vn) @ g["Cv"].astype(np.float64)[vidx]
                out[b, h * G:(h + 1) * G][:, ch] = (o_rot / ssum) @ g["Rv"].astype(np.float64)
    return out


def tie_distance(z: np.ndarray, boundaries: np.ndarray) -> np.ndarray:
    """Distance of each pre-image to its nearest codebook boundary (for tie-band checks)."""
    b = np.asarray(boundaries, np.float64)
    return np.min(np.abs(z.astype(np.float64)[..., None] - b), axis=-1)


def cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
