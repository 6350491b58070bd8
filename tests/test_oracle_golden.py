"""Pin the CPU oracle before trusting it: against the reference's own outputs
(tests/golden/*.npz, written by tests/golden/make_golden.py), hand-computed
bytes, brute force on tiny inputs and closed-form identities."""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_ref as T
from turboquant.quantization.turboquant_mse import codebook_f32, generate_qjl_matrix, random_rotation_matrix

D = 128


@pytest.fixture(scope="module")
def enc(golden_dir):
    return np.load(golden_dir / "encode_small.npz")


@pytest.fixture(scope="module")
def att(golden_dir):
    return np.load(golden_dir / "attention_small.npz")


# --------------------------------------------------------------------- layout
def test_pack_hand_computed_bytes():
    """3-bit codes 1..7,0: sum c_d << 3d = 0x1F58D1 -> bytes D1 58 1F (LSB first)."""
    codes = np.array([[1, 2, 3, 4, 5, 6, 7, 0]])
    assert O.pack_codes(codes, 3).tolist() == [[0xD1, 0x58, 0x1F]]
    assert T.pack_indices(torch.tensor(codes), 3).tolist() == [[0xD1, 0x58, 0x1F]]
    # 1-bit signs: bit i of byte k is sign 8k+i
    s = np.zeros((1, D), np.int64)
    s[0, [0, 9, 127]] = 1
    assert O.pack_codes(s, 1).tolist() == [[1, 2] + [0] * 13 + [128]]


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_matches_big_integer_closed_form(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(50, D))
    packed = O.pack_codes(codes, bits)
    assert packed.shape == (50, (D * bits + 7) // 8)
    for row, cr in zip(packed, codes):
        val = int.from_bytes(row.tobytes(), "little")
        assert all(((val >> (d * bits)) & ((1 << bits) - 1)) == cr[d] for d in range(D))
        assert val >> (D * bits) == 0  # zero padding
    assert np.array_equal(O.unpack_codes(packed, bits, D), codes)
    assert np.array_equal(T.pack_indices(torch.from_numpy(codes), bits).numpy(), packed)
    assert np.array_equal(T.unpack_indices(torch.from_numpy(packed), bits, D).numpy(), codes)


def test_three_bit_codes_straddle_words():
    """3-bit codes straddle 32-bit words at d = 10, 21, 42, ... (3d mod 32 in {30, 31})."""
    straddle = [d for d in range(D) if (3 * d) % 32 > 29]
    assert straddle == [10, 21, 42, 53, 74, 85, 106, 117]
    codes = np.zeros((1, D), np.int64)
    codes[0, straddle] = 7
    words = O.pack_codes(codes, 3).view("<u4")[0]
    for d in straddle:
        w, sh = divmod(3 * d, 32)
        assert (words[w] >> sh) & ((1 << (32 - sh)) - 1) == (1 << (32 - sh)) - 1
        assert words[w + 1] & ((1 << (3 - (32 - sh))) - 1) == (1 << (3 - (32 - sh))) - 1


# ------------------------------------------------------------------- numerics
def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    specials = np.array([0.0, -0.0, 1.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8,
                         2.9802322e-08, 1e-10, np.inf, -np.inf], np.float32)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    bits = bits[np.isfinite(bits)]
    scaled = (rng.standard_normal(1_000_000) * np.exp(rng.uniform(-25, 12, 1_000_000))).astype(np.float32)
    for arr in (specials, bits, scaled):
        assert np.array_equal(O.f32_to_f16_bits(arr), arr.astype(np.float16).view(np.uint16))


def test_norm_is_correctly_rounded_at_an_fp16_tie(golden_dir):
    """A bf16 row (from the config-4 generator) whose fp32 norm rounds correctly to exactly
    the fp16 midpoint 5.435546875, so a sqrt one ulp low stores 0x456F instead of 0x4570.
    Exact rational arithmetic fixes the expected bits: the fp32 fma chain of squares, the
    correctly rounded fp32 square root, then fp16 round-to-nearest-even."""
    from decimal import Decimal, getcontext
    from fractions import Fraction

    row = np.load(golden_dir / "norm_tie_row.npy")

    def rn32(fr):
        if fr == 0:
            return Fraction(0)
        e = fr.numerator.bit_length() - fr.denominator.bit_length()
        while Fraction(2) ** e > fr:
            e -= 1
        while Fraction(2) ** (e + 1) <= fr:
            e += 1
        ulp = Fraction(2) ** (e - 23)
        q, r = divmod(fr, ulp)
        if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
            q += 1
        return q * ulp

    ss = Fraction(0)
    for v in O.bf16_bits_to_f32(row).astype(np.float64):
        ss = rn32(Fraction(v) * Fraction(v) + ss)
    getcontext().prec = 60
    root = (Decimal(ss.numerator) / Decimal(ss.denominator)).sqrt()
    n = rn32(Fraction(str(root)))
    assert n == Fraction(5.435546875)  # an fp16 midpoint, exactly
    assert np.float16(float(n)).view(np.uint16) == 0x4570  # ties to even
    assert O.norms(row.reshape(1, -1))[0] == 0x4570
    assert O.encode_mse(row.reshape(1, -1), 4, np.eye(D, dtype=np.float32), codebook_f32(D, 4)[1])[1][0] == 0x4570


def test_norms_function_equals_encoder_norms():
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.standard_normal((3000, D)).astype(np.float32) * 7).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.norms(xb), O.encode_mse(xb, 2, np.eye(D, dtype=np.float32), codebook_f32(D, 2)[1])[1])


def test_bf16_conversion_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(1_000_000) * np.exp(rng.uniform(-30, 30, 1_000_000))).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(x), ref)


# -------------------------------------------------------------------- encoder
def _params(bits, seed):
    c, b = codebook_f32(D, bits)
    return random_rotation_matrix(D, seed), c, b


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_oracle_encode_mse_matches_reference(enc, bits):
    x = enc["x_bf16"].reshape(-1, D)
    R, _, b = _params(bits, 0)
    codes, norms = O.encode_mse(x, bits, R, b)
    assert np.array_equal(codes, enc[f"mse{bits}_codes"].reshape(codes.shape))
    assert np.array_equal(norms, enc[f"mse{bits}_norms"].reshape(-1))


def test_oracle_encode_prod_matches_reference(enc):
    x = enc["x_bf16"].reshape(-1, D)
    R, c, b = _params(3, 1)
    S = generate_qjl_matrix(D, 31337).numpy()
    codes, norms, signs, rn = O.encode_prod(x, 3, R, c, b, S)
    assert np.array_equal(codes, enc["prod4_codes"].reshape(codes.shape))
    assert np.array_equal(norms, enc["prod4_norms"].reshape(-1))
    assert np.array_equal(signs, enc["prod4_signs"].reshape(signs.shape))
    assert np.array_equal(rn, enc["prod4_rnorms"].reshape(-1))
    assert np.array_equal(O.decode_mse(codes, norms, 3, D, R, c), enc["prod4_khat_bf16"].reshape(-1, D))


def test_oracle_decode_prod_matches_reference(enc):
    """Q_prod key reconstruction (MSE + bf16 QJL correction) equals the reference's
    _decode_keys_qjl_group output bit for bit."""
    R, c, _ = _params(3, 1)
    S = generate_qjl_matrix(D, 31337).numpy()
    out = O.decode_prod(enc["prod4_codes"].reshape(-1, 48), enc["prod4_norms"].reshape(-1),
                        enc["prod4_signs"].reshape(-1, 16), enc["prod4_rnorms"].reshape(-1), 3, D, R, c, S)
    assert np.array_equal(out, enc["prod4_kfull_bf16"].reshape(-1, D))


def test_torch_restatement_matches_reference(enc):
    x = torch.from_numpy(enc["x_bf16"].view(np.int16)).view(torch.bfloat16)
    for bits in (2, 3, 4):
        R, c, b = (torch.from_numpy(a) for a in _params(bits, 0))
        p = T.encode_group(x, R, c, b, bits)
        assert np.array_equal(p.codes.numpy(), enc[f"mse{bits}_codes"])
    R, c, b = (torch.from_numpy(a) for a in _params(3, 1))
    mse, signs, rn = T.encode_keys_qjl_group(x, R, c, b, 3, generate_qjl_matrix(D, 31337))
    assert np.array_equal(mse.codes.numpy(), enc["prod4_codes"])
    assert np.array_equal(signs.numpy(), enc["prod4_signs"])
    assert np.array_equal(rn.view(torch.int16).numpy().view(np.uint16), enc["prod4_rnorms"])


def test_zero_vector_quirks(enc):
    """Zero input: stored norm 1.0 (0x3C00) and every code = middle bucket (z = 0 <= b_mid)."""
    x = enc["x_bf16"].reshape(1, 2, 64, D)[0, 0, 60:61]
    assert not x.any()
    for bits in (2, 3, 4):
        R, _, b = _params(bits, 0)
        codes, norms = O.encode_mse(x, bits, R, b)
        assert norms[0] == 0x3C00
        mid = int(np.sum(b < 0.0))
        assert np.all(O.unpack_codes(codes, bits, D) == mid)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_codes_are_nearest_centroid_brute_force(bits):
    """Lloyd-Max boundaries are midpoints, so each code must be the nearest centroid
    to its fp32 pre-image, except for pre-images within 1e-6 of a boundary."""
    rng = np.random.default_rng(bits)
    xf = rng.standard_normal((400, D)).astype(np.float32)
    x = torch.from_numpy(xf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    R, c, b = _params(bits, 0)
    codes, _ = O.encode_mse(x, bits, R, b)
    idx = O.unpack_codes(codes, bits, D)
    z = O.rotated(x, R).astype(np.float64)
    nearest = np.argmin(np.abs(z[..., None] - c.astype(np.float64)), axis=-1)
    tie = O.tie_distance(z, b) < 1e-6
    assert np.all((idx == nearest) | tie)
    # and z itself is (x/|x|) @ R^T to fp32 accuracy
    xd = O.bf16_bits_to_f32(x).astype(np.float64)
    zd = (xd / np.linalg.norm(xd, axis=1, keepdims=True)) @ R.astype(np.float64).T
    assert np.abs(z - zd).max() < 1e-5


def test_c_oracle_vs_torch_restatement_tie_band():
    """Over 20k random vectors every disagreement between the fixed-order C oracle and
    the reference-order torch path is a tie: the pre-image is within 1e-6 of a boundary."""
    rng = np.random.default_rng(7)
    xf = (rng.standard_normal((20000, D)) * 3).astype(np.float32)
    xt = torch.from_numpy(xf).to(torch.bfloat16)
    x = xt.view(torch.int16).numpy().view(np.uint16)
    R, c, b = _params(4, 0)
    codes, norms = O.encode_mse(x, 4, R, b)
    p = T.encode_group(xt.view(1, 1, -1, D), torch.from_numpy(R), torch.from_numpy(c), torch.from_numpy(b), 4)
    i_c = O.unpack_codes(codes, 4, D)
    i_t = O.unpack_codes(p.codes.numpy().reshape(-1, 64), 4, D)
    diff = i_c != i_t
    z = O.rotated(x, R)
    assert np.all(O.tie_distance(z[diff], b) < 1e-6)
    assert diff.mean() < 1e-4
    nd = norms != p.norms.view(torch.int16).numpy().view(np.uint16).reshape(-1)
    assert np.all(np.abs(norms[nd].astype(np.int32) - p.norms.view(torch.int16).numpy().view(np.uint16).reshape(-1)[nd]) <= 1)


def test_qjl_estimator_is_unbiased():
    """E[sqrt(pi/2)/D * |r| <S q, sign(S r^)>] = <q, r> over random Gaussian S."""
    rng = np.random.default_rng(3)
    errs = []
    for _ in range(400):
        q = rng.standard_normal(D)
        r = rng.standard_normal(D)
        S = rng.standard_normal((D, D))
        est = math.sqrt(math.pi / 2) / D * np.linalg.norm(r) * ((S @ q) @ np.sign(S @ (r / np.linalg.norm(r))))
        errs.append(est - q @ r)
    errs = np.array(errs)
    assert abs(errs.mean()) < 4 * errs.std() / math.sqrt(len(errs))


# ------------------------------------------------------------------ attention
def _golden_layer(att, name):
    bits, qjl, hq, hkv, n = (int(v) for v in att[f"{name}_meta"])
    kb = bits - 1 if qjl else bits
    ck, _ = codebook_f32(D, kb)
    cv, _ = codebook_f32(D, bits)
    layer = {"kcodes": att[f"{name}_kcodes"], "knorms": att[f"{name}_knorms"], "vcodes": att[f"{name}_vcodes"],
             "vnorms": att[f"{name}_vnorms"], "signs": att[f"{name}_signs"] if qjl else None,
             "rnorms": att[f"{name}_rnorms"] if qjl else None, "Rk": random_rotation_matrix(D, 1 if qjl else 0),
             "Ck": ck, "Rv": random_rotation_matrix(D, 0), "Cv": cv,
             "S": generate_qjl_matrix(D, 31337).numpy() if qjl else None, "kbits": kb, "vbits": bits}
    return layer, att[f"{name}_q_bf16"][:, :, 0, :], hq // hkv


@pytest.mark.parametrize("name", ["prod4", "mse3"])
def test_fused_formula_equals_explicit_dequant(att, name):
    layer, q, _ = _golden_layer(att, name)
    f = O.fused_attention_f64(q, layer)
    d = O.dequant_attention_f64(q, layer)
    assert np.abs(f - d).max() <= 1e-12 * np.abs(f).max()


#: max |fused formula - reference chunked output| / ||out||_inf on the golden layers
CHUNKED_GAP = {"prod4": 1.6e-2, "mse3": 5.5e-3}


@pytest.mark.parametrize("name", ["prod4", "mse3"])
def test_fused_formula_vs_reference_chunked_output(att, name):
    """The reference's CPU chunked path rounds dequantised K and V to bf16 (and the
    output); the fused formula does not.  The gap is that rounding alone: the torch
    restatement reproduces the reference's bits exactly, and the fp64 formula lies
    within a bf16-rounding-sized band of it."""
    layer, q, g = _golden_layer(att, name)
    chunked = O.bf16_bits_to_f32(att[f"{name}_out_bf16"][:, :, 0, :]).astype(np.float64)
    f = O.fused_attention_f64(q, layer)
    # measured gap: 1.485e-2 (prod4: bf16 K^ carries the rounded QJL correction too) and
    # 4.79e-3 (mse3) of ||out||_inf; the bounds sit just above
    assert np.abs(f - chunked).max() <= CHUNKED_GAP[name] * np.abs(f).max()
    P = {"Rk": torch.from_numpy(layer["Rk"]), "Ck": torch.from_numpy(layer["Ck"]),
         "Rv": torch.from_numpy(layer["Rv"]), "Cv": torch.from_numpy(layer["Cv"]),
         "S": None if layer["S"] is None else torch.from_numpy(layer["S"])}
    shp = (1,) + layer["kcodes"].shape[1:3] + (D,)
    P["keys"] = T.Packed(torch.from_numpy(layer["kcodes"]), torch.from_numpy(layer["knorms"].view(np.float16)),
                         shp, torch.bfloat16, layer["kbits"])
    P["values"] = T.Packed(torch.from_numpy(layer["vcodes"]), torch.from_numpy(layer["vnorms"].view(np.float16)),
                           shp, torch.bfloat16, layer["vbits"])
    P["signs"] = None if layer["signs"] is None else torch.from_numpy(layer["signs"])
    P["rnorms"] = None if layer["rnorms"] is None else torch.from_numpy(layer["rnorms"].view(np.float16))
    qt = torch.from_numpy(att[f"{name}_q_bf16"].view(np.int16)).view(torch.bfloat16)
    out = T.chunked_attention(qt, P, g).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(out, att[f"{name}_out_bf16"])


def test_fused_formula_invariants(att):
    """Token order does not matter (K and V rows stay paired) and a row-count
    limit of N equals no limit; a huge logit gap reduces to that token's value."""
    layer, q, _ = _golden_layer(att, "prod4")
    base = O.fused_attention_f64(q, layer)
    perm = np.random.default_rng(0).permutation(layer["kcodes"].shape[2])
    pl = dict(layer)
    for k in ("kcodes", "knorms", "vcodes", "vnorms", "signs", "rnorms"):
        pl[k] = layer[k][:, :, perm]
    assert np.abs(O.fused_attention_f64(q, pl) - base).max() <= 1e-12 * np.abs(base).max()
    n = layer["kcodes"].shape[2]
    assert np.array_equal(O.fused_attention_f64(q, layer, n_valid=np.array([n])), base)
    # one-token cache: output is exactly that token's dequantised value, un-rotated
    one = {k: (v[:, :, :1] if isinstance(v, np.ndarray) and v.ndim >= 3 else v) for k, v in layer.items()}
    out = O.fused_attention_f64(q, one)
    vidx = O.unpack_codes(layer["vcodes"][0, :, 0], 4, D)
    vn = O.f16_bits_to_f32(layer["vnorms"][0, :, 0]).astype(np.float64)
    vhat = (layer["Cv"].astype(np.float64)[vidx] @ layer["Rv"].astype(np.float64)) * vn[:, None]
    g = q.shape[1] // vidx.shape[0]
    assert np.allclose(out[0], np.repeat(vhat, g, axis=0), rtol=1e-12, atol=1e-12)


def test_lse_merge_identity(att):
    """Splitting the sequence and merging (o, m, s) partials by log-sum-exp equals
    the single-pass softmax (the identity the split kernel relies on)."""
    rng = np.random.default_rng(11)
    logits = rng.standard_normal(1000) * 3
    vals = rng.standard_normal((1000, 8))
    full = (np.exp(logits - logits.max()) @ vals) / np.exp(logits - logits.max()).sum()
    parts = []
    for a, b in ((0, 300), (300, 301), (301, 1000)):
        m = logits[a:b].max()
        e = np.exp(logits[a:b] - m)
        parts.append((e @ vals[a:b], m, e.sum()))
    M = max(p[1] for p in parts)
    o = sum(np.exp(p[1] - M) * p[0] for p in parts)
    s = sum(np.exp(p[1] - M) * p[2] for p in parts)
    assert np.allclose(o / s, full, rtol=1e-12)
