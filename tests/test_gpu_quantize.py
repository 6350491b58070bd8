"""GPU quantizer parity: libtq codes / norms / QJL signs / residual norms are
bit-identical to the CPU oracle (oracle/tq_oracle.c), which itself matches the
reference's golden vectors (tests/test_oracle_golden.py)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from turboquant.runtime import kernels as K
from turboquant.runtime.params import layer_codecs
from turboquant.runtime.synthetic import kv_bf16

pytestmark = pytest.mark.gpu

D = 128


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _special_rows(device) -> torch.Tensor:
    """Zero, tiny, huge-norm, one-hot and exactly-representable vectors (1 x 1 x 6 x D)."""
    x = torch.zeros(1, 1, 6, D)
    g = torch.Generator().manual_seed(99)
    x[0, 0, 1] = 1e-3 * torch.randn(D, generator=g)
    x[0, 0, 2] = 3000.0 * torch.randn(D, generator=g) / D**0.5
    x[0, 0, 3, 17] = -5.0
    x[0, 0, 4] = 1.0
    x[0, 0, 5, ::2] = 0.25
    return x.to(torch.bfloat16).to(device)


def _host(codec):
    return codec.rotation.cpu().numpy(), codec.centers.cpu().numpy(), codec.boundaries.cpu().numpy()


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_quantize_mse_bit_exact(cuda, bits):
    x = kv_bf16((2, 3, 301, D), seed=10 + bits, device=cuda)
    x = torch.cat([x, _special_rows(cuda).expand(2, 3, 6, D)], dim=2)
    codec = layer_codecs(D, bits, 0, False, cuda).value
    cap, off = x.shape[2] + 9, 5
    codes = torch.zeros(2, 3, cap, K.row_bytes(D, bits), dtype=torch.uint8, device=cuda)
    norms = torch.zeros(2, 3, cap, dtype=torch.float16, device=cuda)
    K.quantize_mse(x, codec, codes, norms, offset=off)
    torch.cuda.synchronize()
    R, _, bnd = _host(codec)
    rc, rn = O.encode_mse(u16(x).reshape(-1, D), bits, R, bnd)
    n = x.shape[2]
    got_c = codes[:, :, off:off + n].cpu().numpy().reshape(-1, rc.shape[1])
    got_n = u16(norms[:, :, off:off + n]).reshape(-1)
    assert np.array_equal(got_c, rc), f"{(got_c != rc).sum()} code bytes differ"
    assert np.array_equal(got_n, rn)
    # slots outside [off, off+n) untouched
    assert int(codes[:, :, :off].count_nonzero()) == 0 and int(codes[:, :, off + n:].count_nonzero()) == 0


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quantize_prod_bit_exact(cuda, bits):
    x = kv_bf16((2, 2, 257, D), seed=20 + bits, device=cuda)
    x = torch.cat([x, _special_rows(cuda).expand(2, 2, 6, D)], dim=2)
    lc = layer_codecs(D, bits, 0, True, cuda)
    B, H, n, _ = x.shape
    codes = torch.zeros(B, H, n, K.row_bytes(D, bits - 1), dtype=torch.uint8, device=cuda)
    norms = torch.zeros(B, H, n, dtype=torch.float16, device=cuda)
    signs = torch.zeros(B, H, n, D // 8, dtype=torch.uint8, device=cuda)
    rnorms = torch.zeros(B, H, n, dtype=torch.float16, device=cuda)
    K.quantize_prod(x, lc.key, lc.qjl, codes, norms, signs, rnorms)
    torch.cuda.synchronize()
    R, C, bnd = _host(lc.key)
    rc, rn, rs, rr = O.encode_prod(u16(x).reshape(-1, D), bits - 1, R, C, bnd, lc.qjl.cpu().numpy())
    assert np.array_equal(codes.cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(u16(norms).reshape(-1), rn)
    assert np.array_equal(signs.cpu().numpy().reshape(rs.shape), rs), f"{(signs.cpu().numpy().reshape(rs.shape) != rs).sum()} sign bytes differ"
    assert np.array_equal(u16(rnorms).reshape(-1), rr)


def _matrix_core_input(cuda, seed, T=2101):
    """[2, 3, T, D] bf16 keys as a strided [B, H, T, D] view of a [B, T, H, D] buffer, with the
    special rows at tokens 100..105: 6 T vectors (>= 4096, so the matrix-core encoder runs),
    a tile count that is not a multiple of 16 vectors."""
    x = kv_bf16((2, 3, T, D), seed=seed, device=cuda)
    x[:, :, 100:106] = _special_rows(cuda)[0, 0]
    x = x.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    assert not x.is_contiguous() and x.shape[0] * x.shape[1] * x.shape[2] % 16 != 0
    return x


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_quantize_mse_matrix_core_bit_exact(cuda, bits):
    x = _matrix_core_input(cuda, 30 + bits)
    codec = layer_codecs(D, bits, 0, False, cuda).value
    B, H, n, _ = x.shape
    cap, off = n + 7, 3
    codes = torch.zeros(B, H, cap, K.row_bytes(D, bits), dtype=torch.uint8, device=cuda)
    norms = torch.zeros(B, H, cap, dtype=torch.float16, device=cuda)
    K.quantize_mse(x, codec, codes, norms, offset=off)
    torch.cuda.synchronize()
    R, _, bnd = _host(codec)
    rc, rn = O.encode_mse(u16(x).reshape(-1, D), bits, R, bnd)
    got_c = codes[:, :, off:off + n].cpu().numpy().reshape(-1, rc.shape[1])
    assert np.array_equal(got_c, rc), f"{(got_c != rc).sum()} code bytes differ"
    assert np.array_equal(u16(norms[:, :, off:off + n]).reshape(-1), rn)
    assert int(codes[:, :, :off].count_nonzero()) == 0 and int(codes[:, :, off + n:].count_nonzero()) == 0
    assert int(norms[:, :, :off].count_nonzero()) == 0 and int(norms[:, :, off + n:].count_nonzero()) == 0


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quantize_prod_matrix_core_bit_exact(cuda, bits):
    x = _matrix_core_input(cuda, 50 + bits)
    lc = layer_codecs(D, bits, 0, True, cuda)
    B, H, n, _ = x.shape
    cap, off = n + 5, 2
    codes = torch.zeros(B, H, cap, K.row_bytes(D, bits - 1), dtype=torch.uint8, device=cuda)
    norms = torch.zeros(B, H, cap, dtype=torch.float16, device=cuda)
    signs = torch.zeros(B, H, cap, D // 8, dtype=torch.uint8, device=cuda)
    rnorms = torch.zeros(B, H, cap, dtype=torch.float16, device=cuda)
    K.quantize_prod(x, lc.key, lc.qjl, codes, norms, signs, rnorms, offset=off)
    torch.cuda.synchronize()
    R, C, bnd = _host(lc.key)
    rc, rn, rs, rr = O.encode_prod(u16(x).reshape(-1, D), bits - 1, R, C, bnd, lc.qjl.cpu().numpy())
    sl = slice(off, off + n)
    got_c = codes[:, :, sl].cpu().numpy().reshape(rc.shape)
    got_s = signs[:, :, sl].cpu().numpy().reshape(rs.shape)
    assert np.array_equal(got_c, rc), f"{(got_c != rc).sum()} code bytes differ"
    assert np.array_equal(u16(norms[:, :, sl]).reshape(-1), rn)
    assert np.array_equal(got_s, rs), f"{(got_s != rs).sum()} sign bytes differ"
    assert np.array_equal(u16(rnorms[:, :, sl]).reshape(-1), rr)
    for t in (codes, norms, signs, rnorms):
        assert int(t[:, :, :off].count_nonzero()) == 0 and int(t[:, :, off + n:].count_nonzero()) == 0


@pytest.mark.parametrize("irregular", ["repeated", "outlying", "unsorted"])
def test_quantize_mse_matrix_core_irregular_boundaries(cuda, irregular):
    """Boundary sets the uniform bucketize grid does not cover (a repeated boundary, one far
    outside the others, an unsorted pair) go through the binary search; codes still equal the
    oracle's #{b < z}.  For the unsorted set the search no longer counts (it assumes order),
    so only its own determinism is checked there."""
    x = _matrix_core_input(cuda, 77)
    base = layer_codecs(D, 4, 0, False, cuda).value
    b = base.boundaries.clone()
    if irregular == "repeated":
        b[8] = b[7]
    elif irregular == "outlying":
        b[14] = 1.0e3
    else:
        b[3], b[4] = base.boundaries[4], base.boundaries[3]
    codec = K.CodecParams(bits=4, rotation=base.rotation, centers=base.centers, boundaries=b)
    B, H, n, _ = x.shape
    codes = torch.zeros(B, H, n, 64, dtype=torch.uint8, device=cuda)
    norms = torch.zeros(B, H, n, dtype=torch.float16, device=cuda)
    K.quantize_mse(x, codec, codes, norms)
    torch.cuda.synchronize()
    if irregular == "unsorted":
        again = torch.zeros_like(codes)
        K.quantize_mse(x, codec, again, norms)
        assert torch.equal(codes, again)
        return
    rc, rn = O.encode_mse(u16(x).reshape(-1, D), 4, base.rotation.cpu().numpy(), b.cpu().numpy())
    got = codes.cpu().numpy().reshape(rc.shape)
    assert np.array_equal(got, rc), f"{(got != rc).sum()} code bytes differ"
    assert np.array_equal(u16(norms).reshape(-1), rn)


def test_quantize_strided_input_and_decode_append(cuda):
    """A [B,T,H,D] buffer viewed as [B,H,T,D] (HF layout), appended one token at a time."""
    base = kv_bf16((1, 4, 40, D), seed=7, device=cuda)  # [B, T=4?]
    x = base.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)  # non-contiguous [B,H,T,D] view
    assert not x.is_contiguous()
    lc = layer_codecs(D, 4, 0, True, cuda)
    B, H, T, _ = x.shape
    bufs = [torch.zeros(B, H, T, K.row_bytes(D, 3), dtype=torch.uint8, device=cuda),
            torch.zeros(B, H, T, dtype=torch.float16, device=cuda),
            torch.zeros(B, H, T, D // 8, dtype=torch.uint8, device=cuda),
            torch.zeros(B, H, T, dtype=torch.float16, device=cuda)]
    K.quantize_prod(x[:, :, :30], lc.key, lc.qjl, *bufs, offset=0)
    for t in range(30, T):  # decode-append path: one token per call
        K.quantize_prod(x[:, :, t:t + 1], lc.key, lc.qjl, *bufs, offset=t)
    torch.cuda.synchronize()
    R, C, bnd = _host(lc.key)
    rc, rn, rs, rr = O.encode_prod(u16(x).reshape(-1, D), 3, R, C, bnd, lc.qjl.cpu().numpy())
    assert np.array_equal(bufs[0].cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(u16(bufs[1]).reshape(-1), rn)
    assert np.array_equal(bufs[2].cpu().numpy().reshape(rs.shape), rs)
    assert np.array_equal(u16(bufs[3]).reshape(-1), rr)


@pytest.mark.parametrize("bits,prod", [(1, False), (3, False), (4, False), (2, True), (4, True)])
def test_small_batch_and_matrix_core_encoders_agree(cuda, bits, prod):
    """The same 4096 vectors encoded by one call (the matrix-core kernel, 4096 and up) and by
    two calls of 4095 and 1 vectors (the small-batch kernel) are bit-identical: codes, norms,
    and for Q_prod signs and residual norms."""
    B, H, T = 4, 8, 128  # 4096 vectors
    x = kv_bf16((B, H, T, D), seed=60 + bits, device=cuda).reshape(1, 1, B * H * T, D)
    lc = layer_codecs(D, bits, 0, prod, cuda)
    codec = lc.key if prod else lc.value
    n = x.shape[2]

    def bufs():
        b = [torch.zeros(1, 1, n, K.row_bytes(D, codec.bits), dtype=torch.uint8, device=cuda),
             torch.zeros(1, 1, n, dtype=torch.float16, device=cuda)]
        if prod:
            b += [torch.zeros(1, 1, n, D // 8, dtype=torch.uint8, device=cuda),
                  torch.zeros(1, 1, n, dtype=torch.float16, device=cuda)]
        return b

    def enc(xs, b, off):
        if prod:
            K.quantize_prod(xs, codec, lc.qjl, *b, offset=off)
        else:
            K.quantize_mse(xs, codec, *b, offset=off)

    whole, parts = bufs(), bufs()
    enc(x, whole, 0)
    enc(x[:, :, :n - 1], parts, 0)
    enc(x[:, :, n - 1:], parts, n - 1)
    torch.cuda.synchronize()
    for a, b in zip(whole, parts):
        assert torch.equal(a, b)


def test_quantize_full_size_c2_key_layer(cuda):
    """BASELINE config 2 key layer (B=8, Hkv=8, N=32768, 4-bit Q_prod: 3-bit codes + QJL):
    all 2,097,152 vectors' codes, norms, sign bits and residual norms bit-exact against the
    oracle (run on the host's cores in chunks: the oracle's C calls release the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    B, H, N = 8, 8, 32768
    x = kv_bf16((B, H, N, D), seed=2024, device=cuda)
    lc = layer_codecs(D, 4, 0, True, cuda)
    codes = torch.empty(B, H, N, 48, dtype=torch.uint8, device=cuda)
    norms = torch.empty(B, H, N, dtype=torch.float16, device=cuda)
    signs = torch.empty(B, H, N, 16, dtype=torch.uint8, device=cuda)
    rnorms = torch.empty(B, H, N, dtype=torch.float16, device=cuda)
    K.quantize_prod(x, lc.key, lc.qjl, codes, norms, signs, rnorms)
    torch.cuda.synchronize()
    xs = u16(x).reshape(-1, D)
    del x
    R, C, bnd = _host(lc.key)
    S = lc.qjl.cpu().numpy()
    got = (codes.view(-1, 48).cpu().numpy(), u16(norms).reshape(-1), signs.view(-1, 16).cpu().numpy(),
           u16(rnorms).reshape(-1))
    chunk = 1 << 15
    starts = range(0, xs.shape[0], chunk)

    def one(s):
        ref = O.encode_prod(xs[s:s + chunk], 3, R, C, bnd, S)
        return [int((g[s:s + chunk] != r).sum()) for g, r in zip(got, ref)]

    with ThreadPoolExecutor(max_workers=min(16, O.cpu_count())) as pool:
        bad = np.array(list(pool.map(one, starts))).sum(axis=0)
    assert bad.tolist() == [0, 0, 0, 0], f"differing code bytes / norms / sign bytes / rnorms: {bad.tolist()}"


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_dequantize_matches_oracle(cuda, bits):
    x = kv_bf16((1, 2, 200, D), seed=40 + bits, device=cuda)
    codec = layer_codecs(D, bits, 0, False, cuda).value
    codes = torch.zeros(1, 2, 210, K.row_bytes(D, bits), dtype=torch.uint8, device=cuda)
    norms = torch.zeros(1, 2, 210, dtype=torch.float16, device=cuda)
    K.quantize_mse(x, codec, codes, norms)
    out = K.dequantize_mse(codes, norms, 200, codec)
    torch.cuda.synchronize()
    R, C, _ = _host(codec)
    ref = O.decode_mse(codes[:, :, :200].cpu().numpy().reshape(400, -1), u16(norms[:, :, :200]).reshape(-1),
                       bits, D, R, C)
    assert np.array_equal(u16(out).reshape(400, D), ref)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_dequantize_prod_matches_oracle(cuda, bits):
    x = kv_bf16((1, 2, 150, D), seed=60 + bits, device=cuda)
    lc = layer_codecs(D, bits, 0, True, cuda)
    kb = bits - 1
    codes = torch.zeros(1, 2, 160, K.row_bytes(D, kb), dtype=torch.uint8, device=cuda)
    norms = torch.zeros(1, 2, 160, dtype=torch.float16, device=cuda)
    signs = torch.zeros(1, 2, 160, D // 8, dtype=torch.uint8, device=cuda)
    rnorms = torch.zeros(1, 2, 160, dtype=torch.float16, device=cuda)
    K.quantize_prod(x, lc.key, lc.qjl, codes, norms, signs, rnorms)
    out = K.dequantize_prod(codes, norms, signs, rnorms, 150, lc.key, lc.qjl)
    torch.cuda.synchronize()
    R, C, _ = _host(lc.key)
    ref = O.decode_prod(codes[:, :, :150].cpu().numpy().reshape(300, -1), u16(norms[:, :, :150]).reshape(-1),
                        signs[:, :, :150].cpu().numpy().reshape(300, -1), u16(rnorms[:, :, :150]).reshape(-1),
                        kb, D, R, C, lc.qjl.cpu().numpy())
    assert np.array_equal(u16(out).reshape(300, D), ref)


@pytest.mark.parametrize("T", [3001, 12001])
@pytest.mark.parametrize("bits,prod", [(1, False), (2, False), (3, False), (4, False), (1, True), (2, True),
                                       (3, True)])
def test_dequantize_arbitrary_rows_match_oracle(cuda, bits, prod, T):
    """Arbitrary code and sign bytes with fp16 norms over nine decades (zeros and subnormals
    included), decoded from a slot offset of a capacity buffer.  3 x 3001 vectors are 563 tiles
    of 16 (each tile's row tiles split over 2 or 4 waves), 3 x 12001 are 2251 (whole tiles per
    wave, several per wave); the last tile is ragged.  The larger case checks 1500 random rows
    and the last 40 against the oracle."""
    rng = np.random.default_rng(900 + 10 * bits + prod + T)
    B, H, start = 1, 3, 57
    cap = start + T + 40
    lc = layer_codecs(D, bits + 1 if prod else bits, 0, prod, cuda)
    codec = lc.key if prod else lc.value
    assert codec.bits == bits

    def norms16():
        n = (10.0 ** rng.uniform(-6.0, 3.0, (B, H, cap))).astype(np.float16)
        n.reshape(-1)[rng.integers(0, n.size, 40)] = 0.0
        return n

    row = K.row_bytes(D, bits)
    codes_h = rng.integers(0, 256, (B, H, cap, row), dtype=np.uint8)
    norms_h = norms16()
    codes, norms = torch.from_numpy(codes_h).to(cuda), torch.from_numpy(norms_h).to(cuda)
    R, C, _ = _host(codec)
    n = B * H * T
    rows = np.arange(n) if T < 5000 else np.union1d(rng.choice(n, 1500, replace=False), np.arange(n - 40, n))
    sl = slice(start, start + T)
    pick = lambda a: a[:, :, sl].reshape(n, -1)[rows]  # noqa: E731
    if prod:
        signs_h = rng.integers(0, 256, (B, H, cap, D // 8), dtype=np.uint8)
        rnorms_h = norms16()
        out = K.dequantize_prod(codes, norms, torch.from_numpy(signs_h).to(cuda),
                                torch.from_numpy(rnorms_h).to(cuda), T, codec, lc.qjl, start=start)
        ref = O.decode_prod(pick(codes_h), pick(norms_h[..., None].view(np.uint16)).reshape(-1), pick(signs_h),
                            pick(rnorms_h[..., None].view(np.uint16)).reshape(-1), bits, D, R, C,
                            lc.qjl.cpu().numpy())
    else:
        out = K.dequantize_mse(codes, norms, T, codec, start=start)
        ref = O.decode_mse(pick(codes_h), pick(norms_h[..., None].view(np.uint16)).reshape(-1), bits, D, R, C)
    torch.cuda.synchronize()
    got = u16(out).reshape(-1, D)[rows]
    assert np.array_equal(got, ref), f"{(got != ref).any(axis=1).sum()} of {ref.shape[0]} rows differ"


def test_norms_correctly_rounded_over_a_million_vectors(cuda, golden_dir):
    """Stored norms are fp16(correctly rounded sqrt(fma chain)) for 1M vectors; about one in
    4000 lands on an fp16 rounding midpoint, where a square root one ulp low (the bare
    hardware instruction) stores the other neighbour.  Includes a known midpoint row."""
    tie = torch.from_numpy(np.load(golden_dir / "norm_tie_row.npy").view(np.int16)).view(torch.bfloat16)
    x = kv_bf16((8, 8, 16384, D), seed=77, device=cuda)
    x[0, 0, 0] = tie.to(cuda)
    codec = layer_codecs(D, 4, 0, False, cuda).value
    codes = torch.empty(8, 8, 16384, 64, dtype=torch.uint8, device=cuda)
    norms = torch.empty(8, 8, 16384, dtype=torch.float16, device=cuda)
    K.quantize_mse(x, codec, codes, norms)
    torch.cuda.synchronize()
    got = u16(norms).reshape(-1)
    ref = O.norms(u16(x).reshape(-1, D))
    assert got[0] == 0x4570
    assert np.array_equal(got, ref), f"{(got != ref).sum()} of {ref.size} norms differ"


def test_residual_norms_correctly_rounded(cuda):
    """The same for the Q_prod residual norms (32K keys against the full oracle encoder)."""
    x = kv_bf16((2, 4, 4096, D), seed=78, device=cuda)
    lc = layer_codecs(D, 4, 0, True, cuda)
    bufs = [torch.empty(2, 4, 4096, 48, dtype=torch.uint8, device=cuda),
            torch.empty(2, 4, 4096, dtype=torch.float16, device=cuda),
            torch.empty(2, 4, 4096, 16, dtype=torch.uint8, device=cuda),
            torch.empty(2, 4, 4096, dtype=torch.float16, device=cuda)]
    K.quantize_prod(x, lc.key, lc.qjl, *bufs)
    torch.cuda.synchronize()
    R, C, bnd = _host(lc.key)
    rc, rn, rs, rr = O.encode_prod(u16(x).reshape(-1, D), 3, R, C, bnd, lc.qjl.cpu().numpy())
    assert np.array_equal(u16(bufs[1]).reshape(-1), rn)
    assert np.array_equal(u16(bufs[3]).reshape(-1), rr)
    assert np.array_equal(bufs[0].cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(bufs[2].cpu().numpy().reshape(rs.shape), rs)
