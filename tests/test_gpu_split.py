"""Outlier-channel split on the GPU: libtq's channel-group encoder and decoder are
bit-identical to the CPU oracle run at D = d on the gathered sub-vectors (the oracle is
pinned at d < 128 in tests/test_oracle_split.py), and the split layer's decode
attention matches fp64 attention over the same decoded rows."""

import numpy as np
import pytest
import torch

import turboquant
from oracle import oracle as O
from turboquant.quantization.turboquant_mse import codebook_f32
from turboquant.runtime import kernels as K
from turboquant.runtime.attention import _group_buffers, fused_attention
from turboquant.runtime.packed_qmse_cache import PackedMSELayer
from turboquant.runtime.params import split_codecs
from turboquant.runtime.synthetic import kv_bf16, query_bf16

from ._tiny_model import CharTokenizer, tiny_llama

pytestmark = pytest.mark.gpu

D = 128
TOL = 2e-3


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _host(g):
    return g.rotation.cpu().numpy(), g.centers.cpu().numpy(), g.boundaries.cpu().numpy()


def _with_specials(x: torch.Tensor, ch: np.ndarray) -> torch.Tensor:
    """Append rows that are zero on the group, nonzero only outside it, tiny, huge and
    one-hot inside it."""
    B, H = x.shape[:2]
    s = torch.zeros(5, D)
    outside = np.setdiff1d(np.arange(D), ch)
    s[1, outside] = 3.0  # zero on the group: stored norm 1.0, middle codes
    s[2, ch] = 1e-3
    s[3, ch] = 3000.0 / len(ch) ** 0.5
    s[4, ch[-1]] = -5.0
    return torch.cat([x, s.to(torch.bfloat16).to(x.device).expand(B, H, 5, D)], dim=2)


def _channels(d: int, seed: int) -> np.ndarray:
    return np.sort(np.random.default_rng(seed).choice(D, d, replace=False))


@pytest.mark.parametrize("d,extra", [(3, 4), (8, 1), (13, 4), (40, 2)])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_quantize_group_mse_bit_exact(cuda, d, extra, bits):
    """Both groups of a split (the outlier group at bits + extra, up to 8 bits) at a token
    offset inside a larger capacity: codes and norms equal the oracle on x[..., ch]."""
    outl = _channels(d, 10 * d + bits)
    sc = split_codecs(np.setdiff1d(np.arange(D), outl), outl, bits, extra, 0, False, cuda)
    x = _with_specials(kv_bf16((2, 3, 131, D), seed=bits + d, device=cuda, outlier_channels=2), outl)
    n = x.shape[2]
    cap, off = n + 7, 4
    for g in (sc.value_normal, sc.value_outlier):
        codes = torch.zeros(2, 3, cap, K.row_bytes(g.dim, g.bits), dtype=torch.uint8, device=cuda)
        norms = torch.zeros(2, 3, cap, dtype=torch.float16, device=cuda)
        K.quantize_group(x, g, codes, norms, offset=off)
        torch.cuda.synchronize()
        R, _, bnd = _host(g)
        rc, rn = O.encode_mse(u16(x).reshape(-1, D)[:, g.channels], g.bits, R, bnd)
        got = codes[:, :, off:off + n].cpu().numpy().reshape(rc.shape)
        assert np.array_equal(got, rc), f"{g.dim} ch, {g.bits} bits: {(got != rc).sum()} code bytes differ"
        assert np.array_equal(u16(norms[:, :, off:off + n]).reshape(-1), rn)
        assert int(codes[:, :, :off].count_nonzero()) == 0 and int(codes[:, :, off + n:].count_nonzero()) == 0


@pytest.mark.parametrize("d,bits,extra", [(4, 2, 1), (8, 4, 1), (13, 3, 4), (40, 4, 2)])
def test_quantize_group_prod_bit_exact(cuda, d, bits, extra):
    outl = _channels(d, d + bits)
    sc = split_codecs(np.setdiff1d(np.arange(D), outl), outl, bits, extra, 3, True, cuda)
    x = _with_specials(kv_bf16((2, 2, 97, D), seed=50 + d, device=cuda), outl)
    B, H, n, _ = x.shape
    for g in (sc.key_normal, sc.key_outlier):
        codes = torch.zeros(B, H, n, K.row_bytes(g.dim, g.bits), dtype=torch.uint8, device=cuda)
        norms = torch.zeros(B, H, n, dtype=torch.float16, device=cuda)
        signs = torch.zeros(B, H, n, K.row_bytes(g.dim, 1), dtype=torch.uint8, device=cuda)
        rnorms = torch.zeros(B, H, n, dtype=torch.float16, device=cuda)
        K.quantize_group(x, g, codes, norms, signs, rnorms)
        torch.cuda.synchronize()
        R, C, bnd = _host(g)
        rc, rn, rs, rr = O.encode_prod(u16(x).reshape(-1, D)[:, g.channels], g.bits, R, C, bnd, g.qjl.cpu().numpy())
        assert np.array_equal(codes.cpu().numpy().reshape(rc.shape), rc), (g.dim, g.bits)
        assert np.array_equal(u16(norms).reshape(-1), rn)
        got_s = signs.cpu().numpy().reshape(rs.shape)
        assert np.array_equal(got_s, rs), f"{(got_s != rs).sum()} sign bytes differ ({g.dim} ch)"
        assert np.array_equal(u16(rnorms).reshape(-1), rr)


@pytest.mark.parametrize("prod", [False, True])
def test_group_small_batch_and_lane_encoders_agree(cuda, prod):
    """One group of 8192 vectors encoded by one call (the lane-per-vector kernel, 8192 and up) and
    by calls of 8191 and 1 vectors (the small-batch kernel) is bit-identical."""
    outl = _channels(13, 5)
    sc = split_codecs(np.setdiff1d(np.arange(D), outl), outl, 3, 2, 0, True, cuda)
    g = sc.key_outlier if prod else sc.value_normal
    x = _with_specials(kv_bf16((1, 1, 8187, D), seed=77, device=cuda), outl)
    n = x.shape[2]
    assert n == 8192

    def bufs():
        b = [torch.zeros(1, 1, n, K.row_bytes(g.dim, g.bits), dtype=torch.uint8, device=cuda),
             torch.zeros(1, 1, n, dtype=torch.float16, device=cuda)]
        if prod:
            b += [torch.zeros(1, 1, n, K.row_bytes(g.dim, 1), dtype=torch.uint8, device=cuda),
                  torch.zeros(1, 1, n, dtype=torch.float16, device=cuda)]
        return b

    whole, parts = bufs(), bufs()
    K.quantize_group(x, g, *whole)
    K.quantize_group(x[:, :, :n - 1], g, *parts, offset=0)
    K.quantize_group(x[:, :, n - 1:], g, *parts, offset=n - 1)
    torch.cuda.synchronize()
    for a, b in zip(whole, parts):
        assert torch.equal(a, b)


def test_quantize_group_strided_input_and_decode_append(cuda):
    base = kv_bf16((1, 4, 3, D), seed=7, device=cuda)
    x = base.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)  # [B,H,T,D] view of a [B,T,H,D] buffer
    assert not x.is_contiguous()
    outl = np.array([5, 6, 70, 71, 127])
    sc = split_codecs(np.setdiff1d(np.arange(D), outl), outl, 4, 2, 0, True, cuda)
    g = sc.key_outlier
    B, H, T, _ = x.shape
    bufs = [torch.zeros(B, H, T, K.row_bytes(5, g.bits), dtype=torch.uint8, device=cuda),
            torch.zeros(B, H, T, dtype=torch.float16, device=cuda),
            torch.zeros(B, H, T, 1, dtype=torch.uint8, device=cuda),
            torch.zeros(B, H, T, dtype=torch.float16, device=cuda)]
    K.quantize_group(x[:, :, :1], g, *bufs, offset=0)
    for t in range(1, T):
        K.quantize_group(x[:, :, t:t + 1], g, *bufs, offset=t)
    torch.cuda.synchronize()
    R, C, bnd = _host(g)
    rc, rn, rs, rr = O.encode_prod(u16(x).reshape(-1, D)[:, outl], g.bits, R, C, bnd, g.qjl.cpu().numpy())
    assert np.array_equal(bufs[0].cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(bufs[2].cpu().numpy().reshape(rs.shape), rs)
    assert np.array_equal(u16(bufs[1]).reshape(-1), rn) and np.array_equal(u16(bufs[3]).reshape(-1), rr)


@pytest.mark.parametrize("qjl", [False, True])
def test_dequantize_groups_merge_into_full_rows(cuda, qjl):
    """Normal group (merge=0), then outlier group (merge=1): the full bf16 row equals the
    oracle's per-group decode scattered to the channels; merge=0 zeroes the other channels."""
    outl = _channels(9, 3)
    sc = split_codecs(np.setdiff1d(np.arange(D), outl), outl, 4, 1, 0, qjl, cuda)
    x = kv_bf16((1, 2, 150, D), seed=9, device=cuda, outlier_channels=3)
    B, H, N, _ = x.shape
    out = torch.full((B, H, N, D), 7.0, dtype=torch.bfloat16, device=cuda)
    ref = np.zeros((B * H * N, D), np.uint16)
    for gi, g in enumerate((sc.key_normal, sc.key_outlier)):
        codes = torch.zeros(B, H, N + 3, K.row_bytes(g.dim, g.bits), dtype=torch.uint8, device=cuda)
        norms = torch.zeros(B, H, N + 3, dtype=torch.float16, device=cuda)
        extra = {}
        if qjl:
            extra = dict(signs=torch.zeros(B, H, N + 3, K.row_bytes(g.dim, 1), dtype=torch.uint8, device=cuda),
                         rnorms=torch.zeros(B, H, N + 3, dtype=torch.float16, device=cuda))
        K.quantize_group(x, g, codes, norms, extra.get("signs"), extra.get("rnorms"))
        K.dequantize_group(codes, norms, N, g, out, merge=gi == 1, **extra)
        if gi == 0:
            torch.cuda.synchronize()
            assert not u16(out).reshape(-1, D)[:, outl].any()  # merge=0 zeroed the other group's channels
        R, C, _ = _host(g)
        hc = codes[:, :, :N].cpu().numpy().reshape(B * H * N, -1)
        hn = u16(norms[:, :, :N]).reshape(-1)
        if qjl:
            dec = O.decode_prod(hc, hn, extra["signs"][:, :, :N].cpu().numpy().reshape(B * H * N, -1),
                                u16(extra["rnorms"][:, :, :N]).reshape(-1), g.bits, g.dim, R, C, g.qjl.cpu().numpy())
        else:
            dec = O.decode_mse(hc, hn, g.bits, g.dim, R, C)
        ref[:, g.channels] = dec
    torch.cuda.synchronize()
    assert np.array_equal(u16(out).reshape(-1, D), ref)
    # the group encodes stay faithful: outlier channels reconstruct to a cosine > 0.97
    xf = x.float().reshape(-1, D)[:, torch.from_numpy(outl).to(cuda)]
    of = out.float().reshape(-1, D)[:, torch.from_numpy(outl).to(cuda)]
    assert torch.nn.functional.cosine_similarity(xf, of, dim=-1).mean().item() > 0.97


def _host_groups(layer: PackedMSELayer) -> list[dict]:
    """Per-group numpy views of a split layer, in the form the fp64 oracle takes."""
    s, sc, n = layer._store, layer._split, layer.packed_seq_length()
    out = []
    for sfx, kg, vg in (("", sc.key_normal, sc.value_normal), ("o", sc.key_outlier, sc.value_outlier)):
        qjl = kg.qjl is not None
        out.append({"channels": kg.channels.astype(np.int64),
                    "kcodes": getattr(s, "kc" + sfx)[:, :, :n].cpu().numpy(),
                    "knorms": u16(getattr(s, "kn" + sfx)[:, :, :n]),
                    "vcodes": getattr(s, "vc" + sfx)[:, :, :n].cpu().numpy(),
                    "vnorms": u16(getattr(s, "vn" + sfx)[:, :, :n]),
                    "signs": getattr(s, "ks" + sfx)[:, :, :n].cpu().numpy() if qjl else None,
                    "rnorms": u16(getattr(s, "kr" + sfx)[:, :, :n]) if qjl else None,
                    "Rk": kg.rotation.cpu().numpy(), "Ck": kg.centers.cpu().numpy(), "kbits": kg.bits,
                    "Rv": vg.rotation.cpu().numpy(), "Cv": vg.centers.cpu().numpy(), "vbits": vg.bits,
                    "S": kg.qjl.cpu().numpy() if qjl else None})
    return out


def _oracle_rows(layer: PackedMSELayer) -> tuple[np.ndarray, np.ndarray]:
    """bf16 K^ / V^ rows (as fp64) decoded by the oracle group by group and scattered."""
    B, H, _ = layer._shape
    n = layer.packed_seq_length()
    kk = np.zeros((B * H * n, D), np.uint16)
    vv = np.zeros((B * H * n, D), np.uint16)
    for g in _host_groups(layer):
        d = len(g["channels"])
        kc, kn = g["kcodes"].reshape(B * H * n, -1), g["knorms"].reshape(-1)
        if g["signs"] is not None:
            kd = O.decode_prod(kc, kn, g["signs"].reshape(B * H * n, -1), g["rnorms"].reshape(-1), g["kbits"], d,
                               g["Rk"], g["Ck"], g["S"])
        else:
            kd = O.decode_mse(kc, kn, g["kbits"], d, g["Rk"], g["Ck"])
        kk[:, g["channels"]] = kd
        vv[:, g["channels"]] = O.decode_mse(g["vcodes"].reshape(B * H * n, -1), g["vnorms"].reshape(-1), g["vbits"],
                                            d, g["Rv"], g["Cv"])
    f = lambda a: O.bf16_bits_to_f32(a).astype(np.float64).reshape(B, H, n, D)  # noqa: E731
    return f(kk), f(vv)


@pytest.mark.parametrize("T", [1001, 3001, 12001])
@pytest.mark.parametrize("k,bits,extra,qjl,role", [(3, 4, 1, True, "key"), (9, 2, 4, False, "key"),
                                                   (40, 3, 5, True, "key"), (5, 4, 4, False, "value"),
                                                   (40, 4, 2, False, "value")])
def test_dequantize_group_arbitrary_rows_match_oracle(cuda, k, bits, extra, qjl, role, T):
    """Arbitrary code and sign bytes with fp16 norms over nine decades (zeros included) for both
    groups of a split, decoded from a slot offset into one row (normal group merge=0, outlier
    group merge=1): run-time widths 2..8 and groups of 3..125 channels, the decoded range ending
    at the buffers' last byte.  3 x T vectors are 188 / 563 / 2251 tiles of 16 (the last ragged):
    on a 256-CU GPU the matrix-core decoder of groups wider than 24 channels then splits a tile's
    row tiles over 4 waves, over 2, or runs whole tiles per wave, so every variant is checked
    on a QJL key group and a value group of 40 outlier channels."""
    rng = np.random.default_rng(700 + 10 * k + bits + T)
    outl = _channels(k, k)
    sc = split_codecs(np.setdiff1d(np.arange(D), outl), outl, bits, extra, 0, qjl and role == "key", cuda)
    groups = (sc.key_normal, sc.key_outlier) if role == "key" else (sc.value_normal, sc.value_outlier)
    B, H, start = 1, 3, 19
    cap = start + T
    out = torch.full((B, H, T, D), 7.0, dtype=torch.bfloat16, device=cuda)
    ref = np.zeros((B * H * T, D), np.uint16)
    sl = slice(start, start + T)
    for gi, g in enumerate(groups):
        prod = g.qjl_ch is not None
        rb = K.row_bytes(g.dim, g.bits)
        codes_h = rng.integers(0, 256, (B, H, cap, rb), dtype=np.uint8)
        norms_h = (10.0 ** rng.uniform(-6.0, 3.0, (B, H, cap))).astype(np.float16)
        norms_h.reshape(-1)[rng.integers(0, norms_h.size, 20)] = 0.0
        extra_args = {}
        if prod:
            signs_h = rng.integers(0, 256, (B, H, cap, K.row_bytes(g.dim, 1)), dtype=np.uint8)
            rnorms_h = (10.0 ** rng.uniform(-6.0, 3.0, (B, H, cap))).astype(np.float16)
            extra_args = dict(signs=torch.from_numpy(signs_h).to(cuda), rnorms=torch.from_numpy(rnorms_h).to(cuda))
        K.dequantize_group(torch.from_numpy(codes_h).to(cuda), torch.from_numpy(norms_h).to(cuda), T, g, out,
                           merge=gi == 1, start=start, **extra_args)
        R, C, _ = _host(g)
        hc = codes_h[:, :, sl].reshape(B * H * T, -1)
        hn = norms_h[:, :, sl].reshape(-1).view(np.uint16)
        if prod:
            dec = O.decode_prod(hc, hn, signs_h[:, :, sl].reshape(B * H * T, -1),
                                rnorms_h[:, :, sl].reshape(-1).view(np.uint16), g.bits, g.dim, R, C,
                                g.qjl.cpu().numpy())
        else:
            dec = O.decode_mse(hc, hn, g.bits, g.dim, R, C)
        ref[:, g.channels] = dec
    torch.cuda.synchronize()
    got = u16(out).reshape(-1, D)
    assert np.array_equal(got, ref), f"{(got != ref).any(axis=1).sum()} of {ref.shape[0]} rows differ"


@pytest.mark.parametrize("qjl,bits,Hq", [(True, 4, 8), (False, 3, 8), (True, 3, 16)])
def test_split_layer_prefill_append_and_attention(cuda, qjl, bits, Hq):
    """Prefill + lazy decode-append of a split layer: packed groups bit-exact against the
    oracle encoder, decoded rows bit-exact against the oracle decoder; the channel-group
    attention kernel (fp32 out) against the fp64 fused formula over the groups at 2e-3."""
    B, Hkv, N, T = 2, 2, 333, 3
    k = kv_bf16((B, Hkv, N + T, D), seed=21, device=cuda, outlier_channels=4)
    v = kv_bf16((B, Hkv, N + T, D), seed=22, device=cuda)
    layer = PackedMSELayer(bits=bits, num_outlier_channels=4, use_qjl_keys=qjl, quantize_decode=True)
    layer.initialize_from_dense(k[:, :, :N], v[:, :, :N])
    layer._lazy_update = True
    for t in range(N, N + T):
        layer.update(k[:, :, t:t + 1], v[:, :, t:t + 1])
    assert layer._outlier_indices.tolist() == [0, 1, 2, 3]  # kv_bf16 plants the outliers at 0..3
    assert layer.packed_seq_length() == N + T
    xs_k, xs_v = u16(k).reshape(-1, D), u16(v).reshape(-1, D)
    groups = _host_groups(layer)
    for g in groups:
        ch, d = g["channels"], len(g["channels"])
        _, bk = codebook_f32(d, g["kbits"])
        _, bv = codebook_f32(d, g["vbits"])
        if g["signs"] is not None:
            rc, rn, rs, rr = O.encode_prod(xs_k[:, ch], g["kbits"], g["Rk"], g["Ck"], bk, g["S"])
            assert np.array_equal(g["signs"].reshape(rs.shape), rs) and np.array_equal(g["rnorms"].reshape(-1), rr)
        else:
            rc, rn = O.encode_mse(xs_k[:, ch], g["kbits"], g["Rk"], bk)
        assert np.array_equal(g["kcodes"].reshape(rc.shape), rc) and np.array_equal(g["knorms"].reshape(-1), rn)
        vc, vn = O.encode_mse(xs_v[:, ch], g["vbits"], g["Rv"], bv)
        assert np.array_equal(g["vcodes"].reshape(vc.shape), vc) and np.array_equal(g["vnorms"].reshape(-1), vn)
    kh, vh = _oracle_rows(layer)
    assert np.array_equal(O.bf16_bits_to_f32(u16(layer._decode_keys_full())).astype(np.float64), kh)
    assert np.array_equal(O.bf16_bits_to_f32(u16(layer._decode_values_full())).astype(np.float64), vh)
    q = query_bf16(B, Hq, D, seed=23, device=cuda)
    sc = layer._split
    _, out = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N + T, key_stack=sc.key_stack,
                                       value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True)
    out = out.cpu().numpy()
    ref = O.split_fused_attention_f64(u16(q), groups, D)
    err = np.abs(out - ref).max() / np.abs(ref).max()
    assert err <= TOL, err
    # the reference's own strategy for split layers (bf16 K^ / V^ rows, exact softmax) lies
    # within the bf16-rounding band of the formula
    assert np.abs(O.dense_attention_f64(u16(q), kh, vh) - ref).max() <= 3e-2 * np.abs(ref).max()
    # through the attention backend: an fp32 query gets the fp32 output (held to the
    # contract), a bf16 query its RNE rounding
    of = fused_attention(q.float().unsqueeze(2), layer, Hq // Hkv)
    assert of.dtype == torch.float32
    assert np.abs(of[:, :, 0].cpu().numpy() - ref).max() <= TOL * np.abs(ref).max()
    ob = fused_attention(q.unsqueeze(2), layer, Hq // Hkv)
    assert ob.dtype == torch.bfloat16
    assert np.array_equal(u16(ob), O.f32_to_bf16_bits(of.cpu().numpy()))


def test_split_layer_dense_buffer_and_left_padding(cuda):
    """quantize_decode=False keeps generated tokens dense after the split history; a
    left-padded batch attends to its own valid slots only (row 2: dense tokens only)."""
    B, Hq, Hkv, N, nd = 3, 8, 2, 210, 4
    k = kv_bf16((B, Hkv, N + nd, D), seed=31, device=cuda, outlier_channels=4)
    v = kv_bf16((B, Hkv, N + nd, D), seed=32, device=cuda)
    layer = PackedMSELayer(bits=4, num_outlier_channels=6, use_qjl_keys=True, quantize_decode=False)
    layer.initialize_from_dense(k[:, :, :N], v[:, :, :N])
    layer._lazy_update = True
    for t in range(N, N + nd):
        layer.update(k[:, :, t:t + 1], v[:, :, t:t + 1])
    assert layer.packed_seq_length() == N and layer.get_seq_length() == N + nd
    pad = [0, 17, N]
    mask = torch.ones(B, N + nd, dtype=torch.bool, device=cuda)
    for b, p in enumerate(pad):
        mask[b, :p] = False
    q = query_bf16(B, Hq, D, seed=33, device=cuda)
    out = fused_attention(q.float().unsqueeze(2), layer, Hq // Hkv, mask[:, None, None, :])[:, :, 0].cpu().numpy()
    kh, vh = O.split_dequant_f64(_host_groups(layer), D)  # unrounded rows: the fused formula
    kk = np.concatenate([kh, O.bf16_bits_to_f32(u16(k[:, :, N:])).astype(np.float64)], axis=2)
    vv = np.concatenate([vh, O.bf16_bits_to_f32(u16(v[:, :, N:])).astype(np.float64)], axis=2)
    ref = O.dense_attention_f64(u16(q), kk, vv, n_start=np.array(pad))
    assert np.abs(out - ref).max() <= TOL * np.abs(ref).max()


def test_split_full_size_c2_layer_subsample(cuda):
    """A BASELINE config-2-sized key layer (B=8, Hkv=8, N=32768) split 124 + 4 channels,
    4-bit Q_prod: a random 2048-vector subsample of both groups is bit-exact against the
    oracle; every stored norm is |x[..., ch]| to fp16 rounding."""
    B, H, N = 8, 8, 32768
    x = kv_bf16((B, H, N, D), seed=2025, device=cuda, outlier_channels=4)
    outl = np.arange(4)
    sc = split_codecs(np.arange(4, D), outl, 4, 1, 0, True, cuda)
    idx = torch.randperm(B * H * N, generator=torch.Generator().manual_seed(6))[:2048]
    xs = u16(x).reshape(-1, D)[idx.numpy()]
    for g in (sc.key_normal, sc.key_outlier):
        rb, sb = K.row_bytes(g.dim, g.bits), K.row_bytes(g.dim, 1)
        codes = torch.empty(B, H, N, rb, dtype=torch.uint8, device=cuda)
        norms = torch.empty(B, H, N, dtype=torch.float16, device=cuda)
        signs = torch.empty(B, H, N, sb, dtype=torch.uint8, device=cuda)
        rnorms = torch.empty(B, H, N, dtype=torch.float16, device=cuda)
        K.quantize_group(x, g, codes, norms, signs, rnorms)
        torch.cuda.synchronize()
        ch_t = torch.from_numpy(g.channels.astype(np.int64)).to(cuda)
        ref_norm = x.float()[..., ch_t].norm(dim=-1)
        assert ((norms.float() - ref_norm).abs() / ref_norm).max().item() < 1e-3
        R, C, bnd = _host(g)
        rc, rn, rs, rr = O.encode_prod(xs[:, g.channels], g.bits, R, C, bnd, g.qjl.cpu().numpy())
        assert np.array_equal(codes.view(-1, rb)[idx.to(cuda)].cpu().numpy(), rc)
        assert np.array_equal(u16(norms).reshape(-1)[idx.numpy()], rn)
        assert np.array_equal(signs.view(-1, sb)[idx.to(cuda)].cpu().numpy(), rs)
        assert np.array_equal(u16(rnorms).reshape(-1)[idx.numpy()], rr)


def test_activate_generate_with_outlier_split(cuda):
    """activate(num_outlier_channels=4) end to end: every packed layer is split, decode
    tokens are appended to both groups and the storage counts both groups."""
    model = tiny_llama(device=cuda, dtype=torch.bfloat16)
    turboquant.activate(model, CharTokenizer(), bits=4, num_outlier_channels=4, quiet=True)
    ids = torch.randint(0, 94, (1, 150), generator=torch.Generator().manual_seed(2)).to(cuda)
    out = model.generate(ids, max_new_tokens=6)
    assert out.shape == (1, 156) and torch.equal(out[0, :150], ids[0])
    t = turboquant.last_telemetry(model)
    # per token-kvhead: normal 124 ch (3-bit codes 47 B + 2, signs 16 B + 2, 4-bit values 62 B + 2)
    # + outlier 4 ch (4-bit codes 2 B + 2, signs 1 B + 2, 5-bit values 3 B + 2)
    per_tok = (47 + 2 + 16 + 2 + 62 + 2) + (2 + 2 + 1 + 2 + 3 + 2)
    assert t["packed_actual_bytes"] == 2 * 2 * 150 * per_tok
    turboquant.deactivate(model, quiet=True)


def test_activate_generate_gqa7_outlier_split_against_oracle(cuda):
    """activate(num_outlier_channels=4) on a GQA-7 model (14 query heads, 2 KV heads): every
    layer's decode attention runs on the 5-8-head split kernel; at the last decode step each
    layer's attention output (captured before o_proj) is the RNE rounding of the kernel's fp32
    output for the same RoPE'd query, which lies within 2e-3 of the fp64 formula over the groups."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    HQ, HKV, P, NEW = 14, 2, 300, 4
    model = tiny_llama(device=cuda, dtype=torch.bfloat16, heads=HQ, kv_heads=HKV, hidden=224)
    turboquant.activate(model, CharTokenizer(), bits=4, num_outlier_channels=4, use_qjl_keys=True,
                        quantize_decode=True, quiet=True)
    seen = [{} for _ in model.model.layers]
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
    ids = torch.randint(0, 94, (1, P), generator=torch.Generator().manual_seed(3)).to(cuda)
    out = model.generate(ids, max_new_tokens=NEW)
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    assert out.shape == (1, P + NEW) and torch.equal(out[0, :P], ids[0])
    pos = P + NEW - 2  # the last decode step fed token NEW - 1 at this position
    for li, rec in enumerate(seen):
        layer = rec["layer"]
        assert layer._split is not None and layer.packed_seq_length() == P + NEW - 1
        qr = rec["q"].view(1, 1, HQ, D).transpose(1, 2)
        cos, sin = model.model.rotary_emb(qr, torch.tensor([[pos]], device=cuda))
        q16, _ = apply_rotary_pos_emb(qr, qr, cos, sin)
        q16 = q16.to(torch.bfloat16)
        got32 = fused_attention(q16.float(), layer, HQ // HKV)[:, :, 0]
        assert np.array_equal(u16(rec["o"].view(1, HQ, D)), O.f32_to_bf16_bits(got32.cpu().numpy())), li
        ref = O.split_fused_attention_f64(u16(q16[:, :, 0]), _host_groups(layer), D)
        err = np.abs(got32.cpu().numpy() - ref).max() / np.abs(ref).max()
        print(f"[split-gqa7] layer {li}: {err:.2e} of |out|_inf", flush=True)
        assert err <= TOL, (li, err)
    turboquant.deactivate(model, quiet=True)


@pytest.mark.parametrize("Hq,Hkv,bits,extra,k,qjl", [
    (28, 4, 4, 1, 3, True),    # GQA 7 (heads 7 of 8 in the wide kernel)
    (8, 8, 2, 3, 13, True),    # one query head per KV head
    (16, 2, 1, 2, 64, False),  # 1-bit normal group, half the channels outliers
    (12, 4, 3, 5, 5, False),   # 8-bit outlier values
])
def test_group_attention_shapes(cuda, Hq, Hkv, bits, extra, k, qjl):
    """tq_decode_attention_groups against the fp64 formula over the groups across GQA
    widths, group sizes and bit widths (ragged token count, partial last tile)."""
    B, N = 2, 777
    kx = kv_bf16((B, Hkv, N, D), seed=60 + k, device=cuda, outlier_channels=k)
    vx = kv_bf16((B, Hkv, N, D), seed=61 + k, device=cuda)
    layer = PackedMSELayer(bits=bits, num_outlier_channels=k, outlier_extra_bits=extra, use_qjl_keys=qjl,
                           quantize_decode=True)
    layer.initialize_from_dense(kx, vx)
    sc = layer._split
    q = query_bf16(B, Hq, D, seed=62, device=cuda)
    _, out = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N, key_stack=sc.key_stack,
                                       value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True)
    ref = O.split_fused_attention_f64(u16(q), _host_groups(layer), D)
    err = np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= TOL, err


def _rows_range(groups: list[dict], b: int, start: int, end: int) -> list[dict]:
    """Batch row b, tokens [start, end) of the oracle's per-group views."""
    out = []
    for g in groups:
        h = dict(g)
        for name in ("kcodes", "knorms", "vcodes", "vnorms", "signs", "rnorms"):
            if h[name] is not None:
                h[name] = h[name][b:b + 1, :, start:end]
        out.append(h)
    return out


@pytest.mark.parametrize("bits,qjl,k,extra,Hq,Hkv", [
    (4, True, 4, 1, 8, 2),    # the split of the headline configuration (GQA 4, 124 + 4 channels)
    (4, True, 8, 1, 6, 2),    # 8 outlier channels, GQA 3
    (3, True, 5, 2, 4, 4),    # 3-bit Q_prod (2-bit keys, 3-bit values), one head per KV head
    (2, True, 3, 3, 4, 2),    # the smallest group (3 channels)
    (4, False, 3, 4, 8, 2),   # 8-bit outlier codes
    (3, False, 7, 1, 8, 2),
    (2, False, 3, 2, 4, 1),
    (1, False, 6, 3, 12, 3),
    (4, True, 4, 1, 28, 4),   # 5-8 heads per KV head (one bit wider outlier group): GQA 7
    (4, True, 8, 1, 40, 8),   # GQA 5, 8 outlier channels
    (3, True, 3, 1, 16, 2),   # GQA 8, 3-bit Q_prod
    (2, False, 5, 1, 24, 4),  # GQA 6, 2-bit Q_mse
    (4, False, 4, 1, 12, 2),  # GQA 6, 4-bit Q_mse
])
def test_split_layer_matrix_core_attention(cuda, bits, qjl, k, extra, Hq, Hkv):
    """Two-group layers with at most 8 outlier channels (and, at 5-8 query heads per KV head,
    an outlier group one bit wider) run on the matrix-core split kernel (group 0's rows at any
    byte alignment, group 1 per lane): fp32 output against the fp64 formula over the groups
    at 2e-3, over the whole range and over per-row ranges (a 1-token row, an offset start)."""
    B, N = 3, 1237
    kx = kv_bf16((B, Hkv, N, D), seed=70 + k, device=cuda, outlier_channels=k)
    vx = kv_bf16((B, Hkv, N, D), seed=71 + k, device=cuda)
    layer = PackedMSELayer(bits=bits, num_outlier_channels=k, outlier_extra_bits=extra, use_qjl_keys=qjl,
                           quantize_decode=True)
    layer.initialize_from_dense(kx, vx)
    sc = layer._split
    q = query_bf16(B, Hq, D, seed=72 + bits, device=cuda)
    host = _host_groups(layer)
    kw = dict(key_stack=sc.key_stack, value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True)
    _, out = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N, **kw)
    ref = O.split_fused_attention_f64(u16(q), host, D)
    err = np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()
    print(f"[split-mfma] bits {bits} qjl {qjl} k {k} extra {extra} G {Hq // Hkv}: whole range {err:.2e}", flush=True)
    assert err <= TOL, err
    starts, ends = [0, 5, 301], [N, 1000, 302]
    _, out = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N,
                                       seq_starts=torch.tensor(starts, dtype=torch.int32),
                                       seq_lens=torch.tensor(ends, dtype=torch.int32), **kw)
    out = out.cpu().numpy()
    for b in range(B):
        ref = O.split_fused_attention_f64(u16(q)[b:b + 1], _rows_range(host, b, starts[b], ends[b]), D)[0]
        err = np.abs(out[b] - ref).max() / np.abs(ref).max()
        assert err <= TOL, (b, err)


@pytest.mark.parametrize("Hq", [8, 14])
def test_split_layer_empty_ranges_are_zero(cuda, Hq):
    """The matrix-core split path (GQA 4 and 7) with nothing to attend to: an empty cache
    (n_tokens = 0) gives zeros and a -inf log-sum-exp, and so does a batch row whose range is
    empty while the other row is held to the fp64 formula."""
    B, Hkv, N = 2, 2, 257
    kx = kv_bf16((B, Hkv, N, D), seed=81, device=cuda, outlier_channels=4)
    vx = kv_bf16((B, Hkv, N, D), seed=82, device=cuda)
    layer = PackedMSELayer(bits=4, num_outlier_channels=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(kx, vx)
    sc = layer._split
    q = query_bf16(B, Hq, D, seed=83, device=cuda)
    kw = dict(key_stack=sc.key_stack, value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True,
              want_lse=True)
    _, out, lse = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=0, **kw)
    assert float(out.abs().max()) == 0.0 and bool(torch.isneginf(lse).all())
    starts, ends = torch.tensor([0, 100], dtype=torch.int32), torch.tensor([N, 100], dtype=torch.int32)
    _, out, lse = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N, seq_starts=starts, seq_lens=ends,
                                            **kw)
    out = out.cpu().numpy()
    assert np.abs(out[1]).max() == 0.0 and bool(torch.isneginf(lse[1]).all())
    ref = O.split_fused_attention_f64(u16(q)[:1], _rows_range(_host_groups(layer), 0, 0, N), D)[0]
    assert np.abs(out[0] - ref).max() <= TOL * np.abs(ref).max()


def test_split_layer_graph_replay_matches_eager(cuda):
    """tq_decode_attention_groups on the matrix-core split path (GQA 4 and GQA 7 layers)
    captured in a HIP graph: bit-identical output on every replay, with eager calls between
    the replays."""
    cases = []
    for Hq, Hkv, N, seed in ((8, 2, 777, 91), (14, 2, 1500, 92)):
        kx = kv_bf16((2, Hkv, N, D), seed=seed, device=cuda, outlier_channels=4)
        vx = kv_bf16((2, Hkv, N, D), seed=seed + 1, device=cuda)
        layer = PackedMSELayer(bits=4, num_outlier_channels=4, use_qjl_keys=True, quantize_decode=True)
        layer.initialize_from_dense(kx, vx)
        cases.append((layer, query_bf16(2, Hq, D, seed=seed + 2, device=cuda), N))

    def call(layer, q, n):
        sc = layer._split
        return K.decode_attention_groups(q, _group_buffers(layer), n_tokens=n, key_stack=sc.key_stack,
                                         value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True)[1]

    eager = [call(*c).clone() for c in cases]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [call(*c) for c in cases]
    for _ in range(3):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
        call(*cases[0])  # eager work between replays
        torch.cuda.synchronize()


def test_split_full_size_c2_layer_attention(cuda):
    """The headline configuration (B=8, Hq=32, Hkv=8, N=32768, 4-bit Q_prod) split 124 + 4
    channels, at the split kernel's full launch geometry: batch rows 0 and 7 against the fp64
    formula over the groups at 2e-3, and the bf16 output the RNE rounding of the fp32 one."""
    B, Hq, Hkv, N = 8, 32, 8, 32768
    kx = kv_bf16((B, Hkv, N, D), seed=2026, device=cuda, outlier_channels=4)
    vx = kv_bf16((B, Hkv, N, D), seed=2027, device=cuda)
    layer = PackedMSELayer(bits=4, num_outlier_channels=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(kx, vx)
    del kx, vx
    sc = layer._split
    q = query_bf16(B, Hq, D, seed=2028, device=cuda)
    ob, of = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N, key_stack=sc.key_stack,
                                       value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True)
    of = of.cpu().numpy()
    assert np.array_equal(u16(ob), O.f32_to_bf16_bits(of))
    host = _host_groups(layer)
    for b in (0, 7):
        ref = O.split_fused_attention_f64(u16(q)[b:b + 1], _rows_range(host, b, 0, N), D)[0]
        err = np.abs(of[b] - ref).max() / np.abs(ref).max()
        print(f"[split-mfma] C2 split layer, row {b}: {err:.2e}", flush=True)
        assert err <= TOL, (b, err)


def test_split_full_size_c4_layer_attention(cuda):
    """The config 4 shape (B=4, Hq=28, Hkv=4, N=32768, 4-bit Q_prod, GQA 7) split 124 + 4
    channels, on the 5-8-head matrix-core split kernel: batch rows 0 and 3 against the fp64
    formula over the groups at 2e-3."""
    B, Hq, Hkv, N = 4, 28, 4, 32768
    kx = kv_bf16((B, Hkv, N, D), seed=2036, device=cuda, outlier_channels=4)
    vx = kv_bf16((B, Hkv, N, D), seed=2037, device=cuda)
    layer = PackedMSELayer(bits=4, num_outlier_channels=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(kx, vx)
    del kx, vx
    sc = layer._split
    q = query_bf16(B, Hq, D, seed=2038, device=cuda)
    _, of = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N, key_stack=sc.key_stack,
                                      value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True)
    of = of.cpu().numpy()
    host = _host_groups(layer)
    for b in (0, 3):
        ref = O.split_fused_attention_f64(u16(q)[b:b + 1], _rows_range(host, b, 0, N), D)[0]
        err = np.abs(of[b] - ref).max() / np.abs(ref).max()
        print(f"[split-mfma] C4 split layer, row {b}: {err:.2e}", flush=True)
        assert err <= TOL, (b, err)


@pytest.mark.parametrize("bits,qjl", [(4, True), (3, False)])
def test_split_layer_diffuse_softmax_long_context(cuda, bits, qjl):
    """An evenly spread softmax over 131,072 tokens (queries scaled by 1e-3) on the
    matrix-core path of a split layer: the normal group's fp16 value sums take the balanced
    codebook at its own dimension (124 channels), which keeps the near-cancelling average
    within 2e-3 of the fp64 formula."""
    B, Hq, Hkv, N = 1, 8, 2, 131072
    kx = kv_bf16((B, Hkv, N, D), seed=90 + bits, device=cuda, outlier_channels=4)
    vx = kv_bf16((B, Hkv, N, D), seed=91 + bits, device=cuda)
    layer = PackedMSELayer(bits=bits, num_outlier_channels=4, use_qjl_keys=qjl, quantize_decode=True)
    layer.initialize_from_dense(kx, vx)
    del kx, vx
    sc = layer._split
    q = (query_bf16(B, Hq, D, seed=92, device=cuda).float() * 1e-3).to(torch.bfloat16)
    _, out = K.decode_attention_groups(q, _group_buffers(layer), n_tokens=N, key_stack=sc.key_stack,
                                       value_stack=sc.value_stack, qjl_stack=sc.qjl_stack, want_f32=True)
    ref = O.split_fused_attention_f64(u16(q), _host_groups(layer), D)
    err = np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()
    print(f"[split-diffuse] bits {bits} qjl {qjl}: {err:.2e} of |out|_inf", flush=True)
    assert err <= TOL, err


@pytest.mark.parametrize("bits,qjl", [(5, False), (8, False), (6, True)])
def test_single_group_attention_at_wide_bit_widths(cuda, bits, qjl):
    """One group of all 128 channels (n_groups = 1): the unsplit layer at widths the MFMA
    kernel does not take, against the unsplit fp64 formula."""
    from turboquant.runtime.params import _group

    B, Hq, Hkv, N = 1, 8, 2, 300
    ch = np.arange(D, dtype=np.int32)
    kg = _group(ch, bits - 1 if qjl else bits, 1 if qjl else 0, cuda, 32769, qjl_seed=31337 if qjl else None)
    vg = _group(ch, bits, 0, cuda, 32769)
    kx = kv_bf16((B, Hkv, N, D), seed=70 + bits, device=cuda)
    vx = kv_bf16((B, Hkv, N, D), seed=71 + bits, device=cuda)
    buf = {"key": kg, "value": vg,
           "k_codes": torch.zeros(B, Hkv, N, K.row_bytes(D, kg.bits), dtype=torch.uint8, device=cuda),
           "k_norms": torch.zeros(B, Hkv, N, dtype=torch.float16, device=cuda),
           "k_signs": torch.zeros(B, Hkv, N, D // 8, dtype=torch.uint8, device=cuda) if qjl else None,
           "k_rnorms": torch.zeros(B, Hkv, N, dtype=torch.float16, device=cuda) if qjl else None,
           "v_codes": torch.zeros(B, Hkv, N, K.row_bytes(D, bits), dtype=torch.uint8, device=cuda),
           "v_norms": torch.zeros(B, Hkv, N, dtype=torch.float16, device=cuda)}
    K.quantize_group(kx, kg, buf["k_codes"], buf["k_norms"], buf["k_signs"], buf["k_rnorms"])
    K.quantize_group(vx, vg, buf["v_codes"], buf["v_norms"])
    q = query_bf16(B, Hq, D, seed=72, device=cuda)
    _, out = K.decode_attention_groups(q, [buf], n_tokens=N, key_stack=kg.rotation_ch, value_stack=vg.rotation_ch,
                                       qjl_stack=kg.qjl_ch, want_f32=True)
    layer = {"kcodes": buf["k_codes"].cpu().numpy(), "knorms": u16(buf["k_norms"]),
             "vcodes": buf["v_codes"].cpu().numpy(), "vnorms": u16(buf["v_norms"]),
             "signs": buf["k_signs"].cpu().numpy() if qjl else None, "rnorms": u16(buf["k_rnorms"]) if qjl else None,
             "Rk": kg.rotation.cpu().numpy(), "Ck": kg.centers.cpu().numpy(), "Rv": vg.rotation.cpu().numpy(),
             "Cv": vg.centers.cpu().numpy(), "S": kg.qjl.cpu().numpy() if qjl else None, "kbits": kg.bits,
             "vbits": bits}
    ref = O.fused_attention_f64(u16(q), layer)
    err = np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= TOL, err
    # the codes themselves are the oracle's at D = 128
    _, _, bv = _host(vg)
    rc, rn = O.encode_mse(u16(vx).reshape(-1, D), bits, vg.rotation.cpu().numpy(), bv)
    assert np.array_equal(buf["v_codes"].cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(u16(buf["v_norms"]).reshape(-1), rn)
