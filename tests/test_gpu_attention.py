"""GPU fused decode attention parity against the fp64 fused-formula oracle.

Tolerance (north star): max |out_gpu - out_oracle| <= 2e-3 * ||out_oracle||_inf on
the fp32 output, before the bf16 cast.  The kernel accumulates in fp32.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from turboquant.runtime import kernels as K
from turboquant.runtime.params import layer_codecs
from turboquant.runtime.synthetic import kv_bf16, query_bf16

pytestmark = pytest.mark.gpu

D = 128
TOL = 2e-3


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def build_layer(cuda, B, Hkv, N, bits, qjl, seed, cap=None, kv_mu=None, v_mu=None, v_sigma=None):
    cap = cap or N
    lc = layer_codecs(D, bits, 0, qjl, cuda)
    kw = {} if kv_mu is None else {"mu": kv_mu}
    vw = {} if v_mu is None else {"mu": v_mu}
    if v_sigma is not None:
        vw["sigma"] = v_sigma
    k = kv_bf16((B, Hkv, N, D), seed=seed, device=cuda, **kw)
    v = kv_bf16((B, Hkv, N, D), seed=seed + 1, device=cuda, **vw)
    L = {
        "kcodes": torch.zeros(B, Hkv, cap, K.row_bytes(D, lc.key_bits), dtype=torch.uint8, device=cuda),
        "knorms": torch.zeros(B, Hkv, cap, dtype=torch.float16, device=cuda),
        "vcodes": torch.zeros(B, Hkv, cap, K.row_bytes(D, lc.value_bits), dtype=torch.uint8, device=cuda),
        "vnorms": torch.zeros(B, Hkv, cap, dtype=torch.float16, device=cuda),
        "signs": None, "rnorms": None,
    }
    if qjl:
        L["signs"] = torch.zeros(B, Hkv, cap, D // 8, dtype=torch.uint8, device=cuda)
        L["rnorms"] = torch.zeros(B, Hkv, cap, dtype=torch.float16, device=cuda)
        K.quantize_prod(k, lc.key, lc.qjl, L["kcodes"], L["knorms"], L["signs"], L["rnorms"])
    else:
        K.quantize_mse(k, lc.key, L["kcodes"], L["knorms"])
    K.quantize_mse(v, lc.value, L["vcodes"], L["vnorms"])
    return lc, L


def host_layer(lc, L, N):
    h = {
        "kcodes": L["kcodes"][:, :, :N].cpu().numpy(), "knorms": u16(L["knorms"][:, :, :N]),
        "vcodes": L["vcodes"][:, :, :N].cpu().numpy(), "vnorms": u16(L["vnorms"][:, :, :N]),
        "signs": None if L["signs"] is None else L["signs"][:, :, :N].cpu().numpy(),
        "rnorms": None if L["rnorms"] is None else u16(L["rnorms"][:, :, :N]),
        "Rk": lc.key.rotation.cpu().numpy(), "Ck": lc.key.centers.cpu().numpy(),
        "Rv": lc.value.rotation.cpu().numpy(), "Cv": lc.value.centers.cpu().numpy(),
        "S": None if lc.qjl is None else lc.qjl.cpu().numpy(),
        "kbits": lc.key_bits, "vbits": lc.value_bits,
    }
    return h


def run(lc, L, q, N, seq_lens=None):
    return K.decode_attention(q, k_codes=L["kcodes"], k_norms=L["knorms"], v_codes=L["vcodes"], v_norms=L["vnorms"],
                              n_tokens=N, key=lc.key, value=lc.value, k_signs=L["signs"], k_rnorms=L["rnorms"],
                              qjl=lc.qjl, seq_lens=seq_lens, want_f32=True)


def check(out32, ref, tol=TOL):
    ref_inf = np.abs(ref).max()
    err = np.abs(out32.cpu().numpy().astype(np.float64) - ref).max()
    assert err <= tol * ref_inf, f"max err {err:.3e} > {tol} * {ref_inf:.3e}"
    return err / max(ref_inf, 1e-30)


CASES = [
    # (B, Hq, Hkv, N, bits, qjl)
    (1, 32, 8, 4096, 4, True),    # BASELINE config 1 shape
    (2, 8, 2, 1000, 4, True),     # ragged N (not a tile multiple)
    (1, 8, 2, 700, 3, False),     # 3-bit Q_mse (codes straddle bytes and words)
    (2, 10, 2, 513, 4, True),     # GQA 5
    (1, 28, 4, 600, 4, True),     # GQA 7
    (1, 4, 4, 300, 2, False),     # MHA, 2-bit
    (1, 16, 2, 257, 3, True),     # GQA 8, 3-bit Q_prod
    (1, 6, 2, 100, 1, False),     # GQA 3, 1-bit
    (3, 12, 2, 333, 4, False),    # GQA 6, 4-bit Q_mse
    (1, 2, 2, 1, 4, True),        # a single token
    (1, 8, 2, 777, 2, True),      # 2-bit Q_prod (1-bit MSE keys + QJL, 2-bit values)
    (2, 12, 2, 450, 3, False),    # GQA 6, 3-bit Q_mse (3-bit value pairs across lanes)
    (40, 32, 8, 200, 4, True),    # 320 groups: more workgroups than the GPU holds at once
    (80, 28, 4, 100, 4, True),    # GQA 7, 320 groups
]


@pytest.mark.parametrize("B,Hq,Hkv,N,bits,qjl", CASES)
def test_attention_matches_fp64_oracle(cuda, B, Hq, Hkv, N, bits, qjl):
    lc, L = build_layer(cuda, B, Hkv, N, bits, qjl, seed=100 + N + bits)
    q = query_bf16(B, Hq, D, seed=7 + N, device=cuda)
    out16, out32 = run(lc, L, q, N)
    torch.cuda.synchronize()
    ref = O.fused_attention_f64(u16(q), host_layer(lc, L, N))
    check(out32, ref)
    # the bf16 output is the RNE rounding of the fp32 output
    assert np.array_equal(u16(out16), O.f32_to_bf16_bits(out32.cpu().numpy()))


def test_attention_capacity_and_seq_lens(cuda):
    """cap > n_tokens, per-row valid lengths (including an empty row and a row longer
    than the split size) and garbage in the unused slots."""
    B, Hq, Hkv, N, cap = 4, 8, 2, 3000, 3500
    lc, L = build_layer(cuda, B, Hkv, cap, 4, True, seed=555, cap=cap)
    q = query_bf16(B, Hq, D, seed=3, device=cuda)
    lens = torch.tensor([3000, 0, 1, 2049], dtype=torch.int32)
    out16, out32 = run(lc, L, q, N, seq_lens=lens)
    torch.cuda.synchronize()
    hl = host_layer(lc, L, N)
    ref = O.fused_attention_f64(u16(q), hl, n_valid=lens.numpy())
    assert np.all(out32[1].cpu().numpy() == 0.0)  # empty sequence -> zeros
    check(out32, ref)


@pytest.mark.parametrize("Hq,Hkv,bits,qjl", [(8, 2, 4, True), (10, 2, 3, False)])
def test_attention_seq_starts_and_lens(cuda, Hq, Hkv, bits, qjl):
    """Per-row attended ranges [seq_starts[b], seq_lens[b]) (what a left- or right-padded mask
    becomes): starts and ends off the 16-token blocks, a range inside the last few of the
    group's splits (every earlier split empty), a single token, start = end and start > end
    (both empty: zero output), with real data in the slots outside every range and past
    n_tokens.  Four and five query heads per KV head (the two split-kernel families)."""
    B, N, cap = 6, 5000, 5200
    lc, L = build_layer(cuda, B, Hkv, cap, bits, qjl, seed=909 + bits, cap=cap)
    q = query_bf16(B, Hq, D, seed=91, device=cuda)
    starts = np.array([0, 37, 4900, 1, 2500, 3000], dtype=np.int32)
    lens = np.array([5000, 4999, 5000, 2, 2500, 2000], dtype=np.int32)
    out16, out32 = K.decode_attention(q, k_codes=L["kcodes"], k_norms=L["knorms"], v_codes=L["vcodes"],
                                      v_norms=L["vnorms"], n_tokens=N, key=lc.key, value=lc.value,
                                      k_signs=L["signs"], k_rnorms=L["rnorms"], qjl=lc.qjl,
                                      seq_lens=torch.from_numpy(lens), seq_starts=torch.from_numpy(starts),
                                      want_f32=True)
    torch.cuda.synchronize()
    ref = O.fused_attention_f64(u16(q), host_layer(lc, L, N), n_valid=lens, n_start=starts)
    assert np.all(out32[4:].cpu().numpy() == 0.0)  # empty ranges attend to nothing
    check(out32, ref)
    assert np.array_equal(u16(out16), O.f32_to_bf16_bits(out32.cpu().numpy()))


@pytest.mark.parametrize("bits,qjl", [(4, True), (3, False)])
def test_attention_diffuse_softmax_long_context(cuda, bits, qjl):
    """An evenly spread softmax over 131,072 tokens (queries scaled by 1e-3): the output is a
    near-cancelling average of the values, where a value centroid's fp16 rounding error,
    the same for every token that carries the code, would add up (as sqrt(tokens) against
    the output).  The kernel is given the balanced fp16 codebook (tq_value_codebook_f16);
    the nearest-even codebook's error on the same inputs is printed beside it."""
    from dataclasses import replace

    B, Hq, Hkv, N = 1, 8, 2, 131072
    lc, L = build_layer(cuda, B, Hkv, N, bits, qjl, seed=4242 + bits)
    q = (query_bf16(B, Hq, D, seed=77, device=cuda).float() * 1e-3).to(torch.bfloat16)
    _, out32 = run(lc, L, q, N)
    nearest = replace(lc.value, attn_centers=lc.value.centers)  # rounded to fp16 in the kernel
    _, out_rne = K.decode_attention(q, k_codes=L["kcodes"], k_norms=L["knorms"], v_codes=L["vcodes"],
                                    v_norms=L["vnorms"], n_tokens=N, key=lc.key, value=nearest,
                                    k_signs=L["signs"], k_rnorms=L["rnorms"], qjl=lc.qjl, want_f32=True)
    torch.cuda.synchronize()
    ref = O.fused_attention_f64(u16(q), host_layer(lc, L, N))
    inf = np.abs(ref).max()
    err_rne = np.abs(out_rne.cpu().numpy().astype(np.float64) - ref).max() / inf
    err = check(out32, ref)
    print(f"[diffuse] bits {bits}: balanced codebook {err:.2e}, nearest-even {err_rne:.2e} of |out|_inf")


def test_attention_empty_cache_is_zero(cuda):
    lc, L = build_layer(cuda, 1, 2, 4, 4, True, seed=1)
    q = query_bf16(1, 8, D, seed=1, device=cuda)
    out16, out32 = run(lc, L, q, 0)
    torch.cuda.synchronize()
    assert float(out32.abs().max()) == 0.0


def test_attention_full_length_c2_rows(cuda):
    """BASELINE config 2 sequence length (N=32768, GQA 4, 4-bit Q_prod) on 2 batch rows."""
    B, Hq, Hkv, N = 2, 32, 8, 32768
    lc, L = build_layer(cuda, B, Hkv, N, 4, True, seed=77)
    q = query_bf16(B, Hq, D, seed=77, device=cuda)
    _, out32 = run(lc, L, q, N)
    torch.cuda.synchronize()
    check(out32, O.fused_attention_f64(u16(q), host_layer(lc, L, N)))


def test_attention_c2_geometry(cuda):
    """BASELINE config 2 exactly as the bench launches it: B=8, Hq=32, Hkv=8, N=32768, 4-bit
    Q_prod keys / 4-bit Q_mse values, so the kernel runs its 64-group x 4-split grid of
    8192-token workgroups.  Batch rows 0 and 7 against the fp64 oracle (2e-3 of |out| on the
    fp32 output); the bf16 output of every row is the RNE rounding of the fp32 output."""
    B, Hq, Hkv, N = 8, 32, 8, 32768
    lc, L = build_layer(cuda, B, Hkv, N, 4, True, seed=808)
    q = query_bf16(B, Hq, D, seed=808, device=cuda)
    out16, out32 = run(lc, L, q, N)
    torch.cuda.synchronize()
    assert np.array_equal(u16(out16), O.f32_to_bf16_bits(out32.cpu().numpy()))
    for b in (0, B - 1):
        row = host_layer(lc, {k: (None if v is None else v[b:b + 1]) for k, v in L.items()}, N)
        check(out32[b:b + 1], O.fused_attention_f64(u16(q[b:b + 1]), row))


def test_attention_full_size_c3(cuda):
    """BASELINE config 3 at its full shape (B=16, Hq=32, Hkv=8, N=65536, 3-bit Q_mse keys and
    values, codes straddling bytes and words): rows 0 and 15 against the fp64 oracle."""
    B, Hq, Hkv, N = 16, 32, 8, 65536
    lc, L = build_layer(cuda, B, Hkv, N, 3, False, seed=303)
    q = query_bf16(B, Hq, D, seed=303, device=cuda)
    _, out32 = run(lc, L, q, N)
    torch.cuda.synchronize()
    for b in (0, B - 1):
        row = host_layer(lc, {k: (None if v is None else v[b:b + 1]) for k, v in L.items()}, N)
        check(out32[b:b + 1], O.fused_attention_f64(u16(q[b:b + 1]), row))


def test_attention_sharp_softmax(cuda):
    """Large key norms make the softmax nearly one-hot (stresses max tracking across splits)."""
    lc, L = build_layer(cuda, 1, 2, 5000, 4, True, seed=9, kv_mu=float(np.log(400.0)))
    q = query_bf16(1, 8, D, seed=9, device=cuda)
    _, out32 = run(lc, L, q, 5000)
    torch.cuda.synchronize()
    check(out32, O.fused_attention_f64(u16(q), host_layer(lc, L, 5000)))


@pytest.mark.parametrize("Hq,v_mu,v_sigma", [
    (8, float(np.log(2e-3)), 0.3),   # tiny value norms (f16 exponents near the bottom of the range)
    (8, float(np.log(4e3)), 0.3),    # large value norms
    (8, float(np.log(20.0)), 2.0),   # norms spread over five decades within one sequence
    (14, float(np.log(20.0)), 2.0),  # the same through the 5-8-head kernel
])
def test_attention_extreme_value_norms(cuda, Hq, v_mu, v_sigma):
    """The fp16 value sum takes p |v| as an fp16 weight; the lazy maximum tracks the value norm's
    exponent so that those weights neither overflow nor lose their leading bits."""
    lc, L = build_layer(cuda, 1, 2, 3000, 4, True, seed=23, v_mu=v_mu, v_sigma=v_sigma)
    q = query_bf16(1, Hq, D, seed=23, device=cuda)
    _, out32 = run(lc, L, q, 3000)
    torch.cuda.synchronize()
    check(out32, O.fused_attention_f64(u16(q), host_layer(lc, L, 3000)))


def test_attention_on_reference_golden_layer(cuda, golden_dir):
    """Run the fused kernel on the packed layer the reference itself produced, and
    compare to (a) the fp64 oracle (tolerance) and (b) the reference's CPU chunked
    output, which rounds K^ and V^ to bf16 (looser, informational bound)."""
    g = np.load(golden_dir / "attention_small.npz")
    for name in ("prod4", "mse3"):
        bits, qjl, hq, hkv, n = (int(v) for v in g[f"{name}_meta"])
        lc = layer_codecs(D, bits, 0, bool(qjl), cuda)
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
        L = {"kcodes": dev(g[f"{name}_kcodes"]), "knorms": dev(g[f"{name}_knorms"].view(np.float16)),
             "vcodes": dev(g[f"{name}_vcodes"]), "vnorms": dev(g[f"{name}_vnorms"].view(np.float16)),
             "signs": dev(g[f"{name}_signs"]) if qjl else None,
             "rnorms": dev(g[f"{name}_rnorms"].view(np.float16)) if qjl else None}
        q = dev(g[f"{name}_q_bf16"].view(np.int16)).view(torch.bfloat16)
        out16, out32 = run(lc, L, q, n)
        torch.cuda.synchronize()
        ref = O.fused_attention_f64(g[f"{name}_q_bf16"][:, :, 0, :], host_layer(lc, L, n))
        check(out32, ref)
        chunked = O.bf16_bits_to_f32(g[f"{name}_out_bf16"][:, :, 0, :]).astype(np.float64)
        # the fp64 formula's own gap to this output is 1.485e-2 (prod4) / 4.79e-3 (mse3)
        bound = {"prod4": 1.6e-2, "mse3": 5.5e-3}[name]
        assert np.abs(out32.cpu().numpy() - chunked).max() <= bound * np.abs(chunked).max()


def test_graph_replay_matches_eager(cuda):
    """tq_decode_attention captured in a HIP graph (two layers, two batch shapes) gives
    bit-identical output on every replay, with eager calls between the replays."""
    lcs = [build_layer(cuda, 2, 2, 777, 4, True, seed=31), build_layer(cuda, 1, 4, 1500, 3, False, seed=32)]
    qs = [query_bf16(2, 8, D, seed=31, device=cuda), query_bf16(1, 4, D, seed=32, device=cuda)]
    ns = [777, 1500]
    eager = [run(lc, L, q, n)[1].clone() for (lc, L), q, n in zip(lcs, qs, ns)]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [run(lc, L, q, n)[1] for (lc, L), q, n in zip(lcs, qs, ns)]
    for _ in range(3):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
        run(*lcs[0], qs[0], ns[0])  # eager work between replays
        torch.cuda.synchronize()


def test_query_at_unaligned_offset(cuda):
    """A contiguous bf16 query view at a storage offset that is not 16-byte aligned (the
    kernels read q 16 bytes at a time) gives the aligned query's output."""
    lc, L = build_layer(cuda, 2, 2, 300, 4, True, seed=12)
    q = query_bf16(2, 8, D, seed=12, device=cuda)
    base = torch.empty(q.numel() + 1, dtype=torch.bfloat16, device=cuda)
    qv = base[1:].view(2, 8, D)
    qv.copy_(q)
    assert qv.data_ptr() % 16 != 0 and qv.is_contiguous()
    _, want = run(lc, L, q, 300)
    _, got = run(lc, L, qv, 300)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
