"""Outlier-channel split, CPU side: pin the oracle at group dimensions d < 128 and the
split attention algebra, check the seed schedule, outlier detection and the host-side
checks of the channel-group C ABI (no GPU)."""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_ref as T
from turboquant.quantization.turboquant_mse import (
    build_scalar_codebook,
    codebook_f32,
    coordinate_density,
    generate_qjl_matrix,
    random_rotation_matrix,
)
from turboquant.runtime import _lib
from turboquant.runtime import kernels as K
from turboquant.runtime.packed_qmse_cache import PackedMSELayer, detect_outlier_channels
from turboquant.runtime.params import split_codecs

D = 128
FAKE = ctypes.c_void_p(1 << 20)  # aligned, never dereferenced: validation fails first


def _x(n: int, seed: int, outliers=(3, 77), scale=10.0) -> torch.Tensor:
    """bf16 [n, D] rows with planted high-energy channels."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, D, generator=g) * torch.exp(0.3 * torch.randn(n, 1, generator=g))
    x[:, list(outliers)] *= scale
    return x.to(torch.bfloat16)


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ C ABI (host)
def test_group_matrix_scatter():
    ch = np.array([1, 4, 5], np.int32)
    sub = np.arange(9, dtype=np.float32).reshape(3, 3) + 1
    m = K.group_matrix(sub, ch, dim=8)
    ref = np.zeros((8, 8), np.float32)
    for j in range(3):
        for i, c in enumerate(ch):
            ref[j, c] = sub[j, i]
    assert np.array_equal(m, ref)
    # x @ M^T on the full row equals x[ch] @ sub^T on the gathered sub-vector
    x = np.random.default_rng(0).standard_normal(8).astype(np.float32)
    assert np.allclose((x @ m.T)[:3], x[ch] @ sub.T, rtol=1e-6)


@pytest.mark.parametrize("channels", [[3, 2, 9], [1, 1, 5], [0, 128, 5], [-1, 2]])
def test_group_matrix_rejects_bad_channel_lists(channels):
    ch = np.array(channels, np.int32)
    with pytest.raises(_lib.TQError):
        K.group_matrix(np.zeros((ch.size, ch.size), np.float32), ch)


def test_group_kernels_reject_bad_arguments_on_host():
    lib = _lib.load()
    ok = np.array([0, 5, 9], np.int32)
    bad = np.array([5, 0, 9], np.int32)

    def q(ch=ok, sub=3, bits=4, dim=128, qjl=None, cap=1, off=0):
        return lib.tq_quantize_group(FAKE, 1, 1, 1, dim, 128, 128, 128, ch.ctypes.data, sub, bits, FAKE, FAKE, FAKE,
                                     qjl, FAKE, FAKE, None, None, cap, off, None)

    assert q(ch=bad) == 1          # not ascending
    assert q(sub=0) == 1           # empty group
    assert q(bits=9) == 1 and q(bits=0) == 1
    assert q(dim=64) == 2          # head_dim 64 is not built
    assert q(qjl=FAKE) == 1        # Q_prod without signs / rnorms
    assert q(off=1) == 1           # writes past the capacity

    def dq(ch=ok, bits=4, out=FAKE, qjl=None):
        return lib.tq_dequantize_group(FAKE, FAKE, None, None, 1, 1, 1, 128, ch.ctypes.data, 3, bits, FAKE, FAKE,
                                       qjl, 0, out, None)

    assert dq(ch=bad) == 1 and dq(bits=9) == 1 and dq(qjl=FAKE) == 1
    assert dq(out=ctypes.c_void_p((1 << 20) + 2)) == 2  # misaligned output rows


def test_group_attention_rejects_bad_arguments_on_host():
    lib = _lib.load()
    P2 = ctypes.c_void_p * 2
    I2 = ctypes.c_int * 2
    ptrs = P2(FAKE, FAKE)

    def call(n_groups=2, dims=(124, 4), kb=(3, 4), vb=(4, 5), qjl=1, q_heads=8, ws=FAKE, cap=16):
        return lib.tq_decode_attention_groups(FAKE, 1, q_heads, 2, 128, None, None, 16, cap, n_groups, I2(*dims),
                                              I2(*kb), I2(*vb), qjl, ptrs, ptrs, ptrs, ptrs, ptrs, ptrs, FAKE, ptrs,
                                              FAKE, FAKE, ptrs, ctypes.c_float(0.0), FAKE, None, None, ws, 1 << 30,
                                              None)

    assert call(n_groups=3) == 1 and call(n_groups=0) == 1
    assert call(dims=(120, 4)) == 1     # the groups must cover all 128 channels
    assert call(kb=(3, 9)) == 1 and call(vb=(0, 5)) == 1
    assert call(q_heads=9) == 1          # Hq not a multiple of Hkv
    assert call(q_heads=18) == 2         # GQA group 9 > 8
    assert call(ws=None) == 3
    assert call(cap=8) == 1              # n_tokens > cap


def test_group_wrappers_refuse_cpu_tensors():
    sc = split_codecs(np.arange(4, D), np.arange(4), 4, 1, 0, False, "cpu")
    x = torch.zeros(1, 1, 4, D, dtype=torch.bfloat16)
    codes = torch.zeros(1, 1, 4, K.row_bytes(4, 5), dtype=torch.uint8)
    norms = torch.zeros(1, 1, 4, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        K.quantize_group(x, sc.value_outlier, codes, norms)


# ------------------------------------------------------------- seed schedule
@pytest.mark.parametrize("qjl", [False, True])
def test_split_seed_schedule(qjl):
    """Reference lazy_initialization (runtime/packed_qmse_cache.py:243-273): normal group
    bits / seed s, outlier group bits+extra / seed s+7919; Q_prod keys one bit less with
    seed+1 and S(s+31337), S(s+31338)."""
    outl = np.array([3, 40, 77, 100])
    normal = np.setdiff1d(np.arange(D), outl)
    sc = split_codecs(normal, outl, 4, 2, 5, qjl, "cpu")
    assert sc.outlier_bits == 6 and sc.value_normal.bits == 4 and sc.value_outlier.bits == 6
    assert np.array_equal(sc.value_normal.rotation.numpy(), random_rotation_matrix(124, 5))
    assert np.array_equal(sc.value_outlier.rotation.numpy(), random_rotation_matrix(4, 5 + 7919))
    assert np.array_equal(sc.value_outlier.centers.numpy(), codebook_f32(4, 6)[0])
    if qjl:
        assert sc.key_normal.bits == 3 and sc.key_outlier.bits == 5
        assert np.array_equal(sc.key_normal.rotation.numpy(), random_rotation_matrix(124, 6))
        assert np.array_equal(sc.key_outlier.rotation.numpy(), random_rotation_matrix(4, 5 + 7920))
        assert torch.equal(sc.key_normal.qjl, generate_qjl_matrix(124, 5 + 31337))
        assert torch.equal(sc.key_outlier.qjl, generate_qjl_matrix(4, 5 + 31338))
        assert np.array_equal(sc.key_outlier.qjl_ch.numpy(), K.group_matrix(sc.key_outlier.qjl.numpy(), outl))
    else:
        assert sc.key_normal is sc.value_normal and sc.key_outlier.qjl is None
    # channel-space rotation: rows j < d carry R's rows on the group's channels
    rc = sc.value_outlier.rotation_ch.numpy()
    assert np.array_equal(rc[:4][:, outl], sc.value_outlier.rotation.numpy())
    assert not rc[4:].any() and not np.delete(rc, outl, axis=1).any()


def test_split_rejects_groups_below_three_channels():
    with pytest.raises(ValueError, match="at least 3"):
        split_codecs(np.arange(2, D), np.arange(2), 4, 1, 0, False, "cpu")
    with pytest.raises(ValueError, match="1..8"):
        split_codecs(np.arange(4, D), np.arange(4), 4, 5, 0, False, "cpu")


# ---------------------------------------------------------- outlier detection
def test_detect_outlier_channels_planted_and_matches_restatement():
    k = torch.randn(2, 2, 50, D)
    v = torch.randn(2, 2, 50, D)
    k[..., [7, 90]] *= 10
    v[..., 31] *= 10
    out, normal = detect_outlier_channels(k.to(torch.bfloat16), v.to(torch.bfloat16), 3)
    assert out.tolist() == [7, 31, 90]
    assert normal.tolist() == [c for c in range(D) if c not in (7, 31, 90)]
    ro, rn = T.detect_outlier_channels(k.to(torch.bfloat16), v.to(torch.bfloat16), 3)
    assert torch.equal(out, ro) and torch.equal(normal, rn)


def test_layer_accepts_split_and_stays_gpu_only():
    layer = PackedMSELayer(bits=4, num_outlier_channels=4, use_qjl_keys=True, quantize_decode=True)
    assert not layer._outlier_enabled and layer._keys_outlier is None
    k = _x(20, 1, outliers=(3, 30, 77, 100)).view(1, 1, 20, D)
    with pytest.raises(RuntimeError, match="GPU"):
        layer.initialize_from_dense(k, k)
    assert layer._outlier_enabled and layer._outlier_indices.tolist() == [3, 30, 77, 100]
    assert layer.rotation.shape == (124, 124) and layer._outlier_rotation.shape == (4, 4)
    assert layer._key_outlier_rotation.shape == (4, 4) and layer._qjl_outlier_matrix.shape == (4, 4)


# ------------------------------------------------------- oracle at d < 128
@pytest.mark.parametrize("d,bits", [(3, 2), (8, 5), (8, 8), (13, 3), (120, 4), (125, 1)])
def test_c_oracle_subdim_vs_torch_restatement_tie_band(d, bits):
    """The C oracle at D = d (the split encoder's definition) against the faithful torch
    restatement of the reference on the same gathered sub-vectors: every code that
    differs is a tie (pre-image within 1e-6 of a boundary), norms within one fp16 ulp."""
    ch = np.sort(np.random.default_rng(d).choice(D, d, replace=False))
    xt = _x(3000, d)[:, ch].contiguous()
    x = _u16(xt)
    c, b = codebook_f32(d, bits)
    R = random_rotation_matrix(d, 11)
    codes, norms = O.encode_mse(x, bits, R, b)
    p = T.encode_group(xt.view(1, 1, -1, d), torch.from_numpy(R), torch.from_numpy(c), torch.from_numpy(b), bits)
    i_c = O.unpack_codes(codes, bits, d)
    i_t = O.unpack_codes(p.codes.numpy().reshape(codes.shape), bits, d)
    diff = i_c != i_t
    assert np.all(O.tie_distance(O.rotated(x, R)[diff], b) < 1e-6)
    tn = _u16(p.norms).reshape(-1)
    assert np.all(np.abs(norms.astype(np.int32) - tn.astype(np.int32)) <= 1)
    assert np.array_equal(p.codes.numpy().reshape(codes.shape)[~diff.any(axis=1)], codes[~diff.any(axis=1)])


@pytest.mark.parametrize("d,bits", [(8, 5), (13, 3)])
def test_c_oracle_subdim_codes_are_nearest_centroid(d, bits):
    """Brute force: each code is the centroid nearest to its fp32 pre-image z = u R^T
    (the fp64 recomputation of z agrees to 1e-5), ties aside."""
    xt = _x(500, 100 + d)[:, :d].contiguous()
    x = _u16(xt)
    c, b = codebook_f32(d, bits)
    R = random_rotation_matrix(d, 2)
    codes, _ = O.encode_mse(x, bits, R, b)
    z = O.rotated(x, R).astype(np.float64)
    nearest = np.argmin(np.abs(z[..., None] - c.astype(np.float64)), axis=-1)
    assert np.all((O.unpack_codes(codes, bits, d) == nearest) | (O.tie_distance(z, b) < 1e-6))
    xd = O.bf16_bits_to_f32(x).astype(np.float64)
    assert np.abs(z - (xd / np.linalg.norm(xd, axis=1, keepdims=True)) @ R.astype(np.float64).T).max() < 1e-5


@pytest.mark.parametrize("d,bits", [(120, 3), (8, 4)])
def test_c_oracle_subdim_prod_vs_torch_restatement(d, bits):
    ch = np.arange(D - d, D) if d > 64 else np.arange(d)
    xt = _x(2000, 5 + d)[:, ch].contiguous()
    x = _u16(xt)
    c, b = codebook_f32(d, bits)
    R = random_rotation_matrix(d, 3)
    S = generate_qjl_matrix(d, 9)
    codes, norms, signs, rn = O.encode_prod(x, bits, R, c, b, S.numpy())
    mse, tsig, trn = T.encode_keys_qjl_group(xt.view(1, 1, -1, d), torch.from_numpy(R), torch.from_numpy(c),
                                             torch.from_numpy(b), bits, S)
    same_codes = (mse.codes.numpy().reshape(codes.shape) == codes).all(axis=1)
    # rows whose codes agree reconstruct the same k^, so signs and residual norms agree up to
    # near-zero projections / one fp16 ulp
    sd = O.unpack_codes(tsig.numpy().reshape(signs.shape), 1, d) != O.unpack_codes(signs, 1, d)
    assert sd[same_codes].mean() < 2e-3
    assert np.all(np.abs(rn[same_codes].astype(np.int32) - _u16(trn).reshape(-1)[same_codes].astype(np.int32)) <= 1)
    assert same_codes.mean() > 0.99


@pytest.mark.parametrize("d,bits,tol", [(120, 4, 1e-8), (3, 2, 1e-8), (8, 5, 5e-4), (8, 8, 5e-4)])
def test_codebook_centroid_condition_other_dims(d, bits, tol):
    """Lloyd-Max fixed point of the d-dimensional sphere marginal (the groups' codebooks).
    The reference iterates at most 200 times (quantization/turboquant_mse.py:70-110); the
    wide books of small groups stop there, about 2e-4 short of the fixed point, and the
    builder reproduces that stop, so their bound is looser."""
    cb = build_scalar_codebook(d, bits)
    cc = cb.centers
    assert np.all(np.diff(cc) > 0) and np.allclose(cc, -cc[::-1], atol=1e-4)
    grid = np.linspace(-1.0, 1.0, 32769)
    dens = coordinate_density(d, grid)
    edges = np.concatenate(([-1.0], cb.boundaries, [1.0]))
    for i in range(len(cc)):
        sel = (grid >= edges[i]) & (grid <= edges[i + 1])
        xs, w = grid[sel], dens[sel]
        assert abs(np.trapezoid(xs * w, xs) / np.trapezoid(w, xs) - cc[i]) < tol


def test_three_dim_marginal_is_uniform():
    """d = 3: one coordinate of a uniform point on S^2 is uniform on [-1, 1] (Archimedes), so
    the b-bit Lloyd-Max book is the uniform quantizer: centers -1 + (2i+1)/2^b."""
    for bits in (1, 2, 3):
        L = 1 << bits
        assert np.allclose(build_scalar_codebook(3, bits).centers, -1 + (2 * np.arange(L) + 1) / L, atol=1e-4)


# ------------------------------------------------------ split attention algebra
def _split_layer(seed: int, B=1, Hkv=2, N=40, outl=(3, 40, 77, 100), bits=4, qjl=True):
    """A packed outlier-split layer built with the oracle encoder (numpy dicts per group)."""
    rng = torch.Generator().manual_seed(seed)
    kx = (torch.randn(B, Hkv, N, D, generator=rng) * 2)
    vx = torch.randn(B, Hkv, N, D, generator=rng)
    kx[..., list(outl)] *= 8
    kx, vx = kx.to(torch.bfloat16), vx.to(torch.bfloat16)
    outl = np.array(outl)
    normal = np.setdiff1d(np.arange(D), outl)
    groups = []
    for gi, (ch, gb, s) in enumerate(((normal, bits, 0), (outl, bits + 1, 7919))):
        kb = gb - 1 if qjl else gb
        d = len(ch)
        ck, bk = codebook_f32(d, kb)
        cv, bv = codebook_f32(d, gb)
        Rk = random_rotation_matrix(d, s + (1 if qjl else 0))
        Rv = random_rotation_matrix(d, s)
        S = generate_qjl_matrix(d, 31337 + gi).numpy() if qjl else None
        kg = _u16(kx[..., ch].contiguous()).reshape(-1, d)
        vg = _u16(vx[..., ch].contiguous()).reshape(-1, d)
        g = {"channels": ch, "kbits": kb, "vbits": gb, "Rk": Rk, "Ck": ck, "Rv": Rv, "Cv": cv, "S": S}
        if qjl:
            kc, kn, sg, rn = O.encode_prod(kg, kb, Rk, ck, bk, S)
            g.update(signs=sg.reshape(B, Hkv, N, -1), rnorms=rn.reshape(B, Hkv, N))
        else:
            kc, kn = O.encode_mse(kg, kb, Rk, bk)
            g.update(signs=None, rnorms=None)
        vc, vn = O.encode_mse(vg, gb, Rv, bv)
        g.update(kcodes=kc.reshape(B, Hkv, N, -1), knorms=kn.reshape(B, Hkv, N), vcodes=vc.reshape(B, Hkv, N, -1),
                 vnorms=vn.reshape(B, Hkv, N))
        groups.append(g)
    return groups


@pytest.mark.parametrize("qjl", [True, False])
def test_split_fused_formula_equals_dequant_attention(qjl):
    groups = _split_layer(1, qjl=qjl)
    q = _u16(torch.randn(1, 8, D).to(torch.bfloat16))
    f = O.split_fused_attention_f64(q, groups, D)
    kh, vh = O.split_dequant_f64(groups, D)
    d = O.dense_attention_f64(q, kh, vh)
    assert np.abs(f - d).max() <= 1e-12 * np.abs(f).max()


def test_split_formula_with_one_group_is_the_unsplit_formula():
    """One group holding all D channels is the unsplit layer: same codes, same formula."""
    rng = torch.Generator().manual_seed(3)
    kx = torch.randn(1, 2, 30, D, generator=rng).to(torch.bfloat16)
    vx = torch.randn(1, 2, 30, D, generator=rng).to(torch.bfloat16)
    ck, bk = codebook_f32(D, 3)
    cv, bv = codebook_f32(D, 4)
    Rk, Rv = random_rotation_matrix(D, 1), random_rotation_matrix(D, 0)
    S = generate_qjl_matrix(D, 31337).numpy()
    kc, kn, sg, rn = O.encode_prod(_u16(kx).reshape(-1, D), 3, Rk, ck, bk, S)
    vc, vn = O.encode_mse(_u16(vx).reshape(-1, D), 4, Rv, bv)
    layer = {"kcodes": kc.reshape(1, 2, 30, -1), "knorms": kn.reshape(1, 2, 30), "vcodes": vc.reshape(1, 2, 30, -1),
             "vnorms": vn.reshape(1, 2, 30), "signs": sg.reshape(1, 2, 30, -1), "rnorms": rn.reshape(1, 2, 30),
             "Rk": Rk, "Ck": ck, "Rv": Rv, "Cv": cv, "S": S, "kbits": 3, "vbits": 4}
    q = _u16(torch.randn(1, 8, D).to(torch.bfloat16))
    whole = dict(layer, channels=np.arange(D))
    assert np.allclose(O.split_fused_attention_f64(q, [whole], D), O.fused_attention_f64(q, layer),
                       rtol=0, atol=1e-12 * np.abs(O.fused_attention_f64(q, layer)).max())


def test_split_dequant_matches_torch_restatement_decode_merge():
    """fp64 group dequantisation scattered to the channels against the reference-order
    torch restatement (bf16 per group, then scattered): equal up to its bf16 roundings."""
    groups = _split_layer(4, qjl=True)
    kh, vh = O.split_dequant_f64(groups, D)
    tg, enc = [], []
    for g in groups:
        d = len(g["channels"])
        shp = g["kcodes"].shape[:3] + (d,)
        tg.append({"idx": torch.from_numpy(g["channels"]), "R": torch.from_numpy(g["Rk"]),
                   "C": torch.from_numpy(g["Ck"]), "S": torch.from_numpy(g["S"])})
        enc.append({"packed": T.Packed(torch.from_numpy(g["kcodes"]), torch.from_numpy(g["knorms"].view(np.float16)),
                                       shp, torch.bfloat16, g["kbits"]),
                    "signs": torch.from_numpy(g["signs"]), "rnorms": torch.from_numpy(g["rnorms"].view(np.float16))})
    full = T.decode_merge(enc, tg, D).float().numpy()
    assert np.abs(full - kh).max() <= 2 ** -7 * np.abs(kh).max()
    # the planted x8 outlier channels carry the largest reconstructed energy
    energy = (kh ** 2).sum(axis=(0, 1, 2))
    assert set(np.argsort(energy)[-4:].tolist()) == set(groups[1]["channels"].tolist())
