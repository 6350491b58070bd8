#!/usr/bin/env python3
"""TurboQuant hot-path benchmark on one MI355X.

Workload: Llama-3.1-8B KV shape -- batch 8, 32 query heads,
8 KV heads, head_dim 128, context 32768 -- with 4-bit Q_prod keys (3-bit MSE +
1-bit QJL) and 4-bit Q_mse values, 32 independently seeded layers of
synthetic K/V (iid N(0,1) directions, lognormal(ln 20, 0.3) norms) quantized
on the GPU by the prefill quantizer.

A "step" is one decode step: the fused decode attention over all 32 layers
(one query token per sequence, every layer a different packed cache, so the
9 GB working set defeats the 256 MB Infinity Cache).  ``value`` is the
whole-job packed-KV read rate in GB/s over the timed steps (inputs resident
in HBM).  The prefill quantizer is timed separately and reported beside it.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 5]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "tq-local_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
VALU_FP32_PEAK_TFLOPS = 157.3

# BASELINE decode-attention shapes (B, Hq, Hkv, N, bits, qjl) -> the configuration they are
_SHAPES = {(8, 32, 8, 32768, 4, True): "BASELINE config 2",
           (16, 32, 8, 65536, 3, False): "BASELINE config 3 shape",
           (4, 28, 4, 32768, 4, True): "BASELINE config 4 shape",
           (1, 40, 8, 131584, 4, True): "BASELINE config 5 shape"}


def _shape_name(B, Hq, Hkv, N, bits, qjl):
    return _SHAPES.get((B, Hq, Hkv, N, bits, qjl), "custom shape")


def packed_bytes_per_token_head(dim: int, bits: int, qjl: bool) -> int:
    kb = bits - 1 if qjl else bits
    b = math.ceil(dim * kb / 8) + 2 + math.ceil(dim * bits / 8) + 2
    if qjl:
        b += dim // 8 + 2
    return b


def measured_traffic() -> int | None:
    """HBM bytes per call from the committed PMC summary, if it was measured on this kernel source."""
    import hashlib

    summary = ROOT / "profiles" / "tq_decode_attention_c2_traffic.txt"
    source = ROOT / "tq-local_amd" / "csrc" / "tq_attention.hip"
    try:
        fields = dict(line.split(":", 1) for line in summary.read_text().splitlines() if ":" in line and not line.startswith("#"))
        if fields["attention_source_sha256"].strip() != hashlib.sha256(source.read_bytes()).hexdigest():
            return None  # stale: the kernel changed since the counters were taken
        return int(fields["traffic_bytes_per_call"].strip())
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(bits: int = 4) -> dict:
    """BASELINE config 1 (B=1, Hq=32, Hkv=8, N=4096) through the torch restatement of
    the reference's CPU path: encode (K Q_prod + V Q_mse) and one decode-attention step."""
    import numpy as np
    import torch

    from oracle import torch_ref
    from turboquant.quantization.turboquant_mse import codebook_f32, generate_qjl_matrix, random_rotation_matrix
    from turboquant.runtime.synthetic import kv_bf16, query_bf16

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    B, Hq, Hkv, N, D = 1, 32, 8, 4096, 128
    ck, bk = codebook_f32(D, bits - 1)
    cv, bv = codebook_f32(D, bits)
    params = {
        "Rk": torch.from_numpy(random_rotation_matrix(D, 1)), "Ck": torch.from_numpy(ck), "Bk": torch.from_numpy(bk),
        "Rv": torch.from_numpy(random_rotation_matrix(D, 0)), "Cv": torch.from_numpy(cv), "Bv": torch.from_numpy(bv),
        "S": generate_qjl_matrix(D, 31337),
    }
    k = kv_bf16((B, Hkv, N, D), seed=11, device="cpu")
    v = kv_bf16((B, Hkv, N, D), seed=12, device="cpu")
    q = query_bf16(B, Hq, D, seed=13, device="cpu").unsqueeze(2)

    def timed(fn, reps=5, warm=2):
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    layer = torch_ref.encode_layer(k, v, params, True, bits)
    t_enc = timed(lambda: torch_ref.encode_layer(k, v, params, True, bits))
    t_att = timed(lambda: torch_ref.chunked_attention(q, layer, Hq // Hkv))
    nbytes = B * Hkv * N * packed_bytes_per_token_head(D, bits, True)
    cpu_model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(nbytes / t_att / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config 1 (B=1, Hq=32, Hkv=8, D=128, N=4096, 4-bit Q_prod) through oracle/torch_ref.py "
                   f"(reference CPU path): decode attention {t_att * 1e6:.0f} us/layer "
                   f"({nbytes} packed bytes), encode K+V {t_enc * 1e3:.1f} ms; median of 5 after 2 warmups"),
        "attention_us_per_layer": round(t_att * 1e6, 1),
        "encode_ms_per_layer": round(t_enc * 1e3, 2),
        "cpu_model": cpu_model,
        "affinity_cpus": threads,
    }


def bench_split(args, dev) -> dict:
    """Outlier-split layers (num_outlier_channels = --outliers): prefill through the
    channel-group encoders (tq_quantize_group), then decode steps through the channel-group
    attention kernel (tq_decode_attention_groups).  Launches are eager."""
    import torch

    from turboquant.runtime.attention import fused_attention
    from turboquant.runtime.packed_qmse_cache import PackedMSELayer
    from turboquant.runtime.synthetic import kv_bf16, query_bf16

    B, Hq, Hkv, N, D, bits = args.batch, args.q_heads, args.kv_heads, args.context, 128, args.bits
    qjl = not args.no_qjl
    layers, queries, q_ms = [], [], []
    for li in range(args.layers):
        k = kv_bf16((B, Hkv, N, D), seed=1000 + 2 * li, device=dev, outlier_channels=args.outliers)
        v = kv_bf16((B, Hkv, N, D), seed=1001 + 2 * li, device=dev)
        layer = PackedMSELayer(bits=bits, num_outlier_channels=args.outliers, use_qjl_keys=qjl, quantize_decode=True,
                               reserve_tokens=0)
        layer.lazy_initialization(k, v)  # channel detection and codecs, outside the timed encode
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        layer.initialize_from_dense(k, v)
        e1.record()
        torch.cuda.synchronize()
        q_ms.append(e0.elapsed_time(e1))
        del k, v
        layers.append(layer)
        queries.append(query_bf16(B, Hq, D, seed=5000 + li, device=dev).unsqueeze(2))
    print(f"[bench] split-quantized {args.layers} layers: {statistics.median(q_ms):.3f} ms/layer (median)",
          file=sys.stderr, flush=True)

    def attn(li):
        return fused_attention(queries[li], layers[li], Hq // Hkv)

    for _ in range(args.warmup):
        for li in range(args.layers):
            attn(li)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        for li in range(args.layers):
            attn(li)
    e1.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    avg_us = e0.elapsed_time(e1) * 1e3 / (args.steps * args.layers)
    layer_bytes = int(layers[0].storage_bytes())
    achieved = layer_bytes / (avg_us * 1e-6) / 1e9
    # at most 8 outlier channels, and with 5-8 heads per KV head not 3-bit Q_mse (the outlier
    # group here is one bit wider): the split kernel's matrix-core path
    mfma = args.outliers <= 8 and (Hq // Hkv <= 4 or qjl or bits != 3)
    return {
        "metric": "outlier-split decode-attn us/layer, 8B KV shape @32K",
        "value": round(avg_us, 1),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8 codes; int8/fp16 MFMA (normal group), fp32 (outlier group)" if mfma else "u8 codes; fp32 VALU",
        "data": "synthetic",
        "config": {
            "workload": (f"outlier split, {args.outliers} channels: {args.layers} layers, B={B}, Hq={Hq}, Hkv={Hkv}, "
                         f"D={D}, N={N}, {bits}-bit normal / {bits + 1}-bit outlier group, "
                         + ("Q_prod keys" if qjl else "Q_mse keys")),
            "packed_bytes_per_layer": layer_bytes,
            "layers": args.layers,
        },
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "tq_decode_attention_groups = " + ("split_kernel (two groups)" if mfma else "group_attn_kernel")
                     + " + merge_kernel, eager calls"},
        "prefill_quantizer": {"ms_per_layer": round(statistics.median(q_ms), 3)},
    }


class _IdTokenizer:
    """Bijective id <-> character map over the whole vocabulary (no tokenizer files offline):
    id i is the code point 0x20000 + i, so decode -> encode returns the same ids."""

    eos_token_id = None
    pad_token_id = None
    BASE = 0x20000

    def encode(self, text, add_special_tokens=True):
        return [ord(c) - self.BASE for c in text]

    def decode(self, ids, skip_special_tokens=True):
        return "".join(chr(self.BASE + int(i)) for i in ids)


def bench_c5(args, dev) -> dict:
    """a random-init QwQ-32B-architecture model (Qwen2, 64 layers, hidden
    5120, 40/8 heads, SwiGLU 27648, vocab 152064, rope theta 1e6, bf16) on one GPU; 131072
    uniform random prompt ids, then 512 greedy tokens with EOS disabled, through
    turboquant.activate(bits=4, Q_prod keys, quantize_decode=True) and model.generate;
    with --outliers K every packed layer is split (num_outlier_channels=K)."""
    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM

    import turboquant
    from turboquant.runtime import kernels as K
    from turboquant.runtime.params import layer_codecs
    from turboquant.runtime.synthetic import kv_bf16, query_bf16

    prompt, new = args.c5_prompt, args.c5_new
    cfg = Qwen2Config(vocab_size=152064, hidden_size=5120, intermediate_size=27648, num_hidden_layers=args.c5_layers,
                      num_attention_heads=40, num_key_value_heads=8, max_position_embeddings=prompt + new,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6}, rms_norm_eps=1e-5,
                      tie_word_embeddings=False)
    cfg._attn_implementation = "sdpa"
    t0 = time.perf_counter()
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Qwen2ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    model.generation_config.eos_token_id = None
    init_s = time.perf_counter() - t0
    print(f"[bench] c5 model ready in {init_s:.1f} s ({sum(p.numel() for p in model.parameters()) / 1e9:.2f} B "
          "parameters)", file=sys.stderr, flush=True)
    turboquant.activate(model, _IdTokenizer(), bits=4, use_qjl_keys=True, quantize_decode=True, quiet=True,
                        num_outlier_channels=args.outliers)
    ids = torch.randint(0, cfg.vocab_size, (1, prompt), generator=torch.Generator().manual_seed(5)).to(dev)
    model.generate(ids[:, :2048], max_new_tokens=4)  # untimed: kernel loading, GEMM heuristics, allocator
    runs = {}
    for n_new in (2, new):  # the difference isolates the decode steps from prefill + packing
        torch.cuda.synchronize()
        t = time.perf_counter()
        out = model.generate(ids, max_new_tokens=n_new)
        torch.cuda.synchronize()
        runs[n_new] = time.perf_counter() - t
        assert out.shape == (1, prompt + n_new) and torch.equal(out[0, :prompt], ids[0])
        print(f"[bench] c5 generate {n_new} tokens: {runs[n_new]:.2f} s", file=sys.stderr, flush=True)
    tel = turboquant.last_telemetry(model)
    turboquant.deactivate(model, quiet=True)
    decode_s = runs[new] - runs[2]
    step_ms = decode_s / (new - 2) * 1e3
    del model
    torch.cuda.empty_cache()
    # the decode attention kernel alone on one packed layer of the final shape (N = prompt + new)
    N = prompt + new
    k, v = kv_bf16((1, 8, N, 128), seed=1, device=dev), kv_bf16((1, 8, N, 128), seed=2, device=dev)
    q = query_bf16(1, 40, 128, seed=3, device=dev)
    if args.outliers:
        from turboquant.runtime.attention import _group_buffers
        from turboquant.runtime.packed_qmse_cache import PackedMSELayer

        layer = PackedMSELayer(bits=4, num_outlier_channels=args.outliers, use_qjl_keys=True, quantize_decode=True,
                               reserve_tokens=0)
        layer.initialize_from_dense(k, v)
        sc, gb = layer._split, _group_buffers(layer)

        def call():
            K.decode_attention_groups(q, gb, n_tokens=N, key_stack=sc.key_stack, value_stack=sc.value_stack,
                                      qjl_stack=sc.qjl_stack)
    else:
        lc = layer_codecs(128, 4, 0, True, dev)
        L = {"k_codes": torch.empty(1, 8, N, 48, dtype=torch.uint8, device=dev),
             "k_norms": torch.empty(1, 8, N, dtype=torch.float16, device=dev),
             "k_signs": torch.empty(1, 8, N, 16, dtype=torch.uint8, device=dev),
             "k_rnorms": torch.empty(1, 8, N, dtype=torch.float16, device=dev),
             "v_codes": torch.empty(1, 8, N, 64, dtype=torch.uint8, device=dev),
             "v_norms": torch.empty(1, 8, N, dtype=torch.float16, device=dev)}
        K.quantize_prod(k, lc.key, lc.qjl, L["k_codes"], L["k_norms"], L["k_signs"], L["k_rnorms"])
        K.quantize_mse(v, lc.value, L["v_codes"], L["v_norms"])

        def call():
            K.decode_attention(q, n_tokens=N, key=lc.key, value=lc.value, qjl=lc.qjl, **L)
    for _ in range(3):
        call()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        call()
    e1.record()
    torch.cuda.synchronize()
    attn_us = e0.elapsed_time(e1) * 1e3 / 20
    return {
        "metric": "config 5 end-to-end decode tokens/s (random-init QwQ-32B architecture, 128K prompt)",
        "value": round((new - 2) / decode_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "higher_is_better": True,
        "vs_baseline": None,
        "dtype": "bf16 model; u8 packed KV",
        "data": "synthetic (uniform random ids, random-init weights)",
        "config": {"workload": f"QwQ-32B architecture, {cfg.num_hidden_layers} layers, prompt {prompt}, "
                               f"{new} greedy tokens, batch 1, 4-bit Q_prod K / 4-bit Q_mse V, quantize_decode"
                               + (f", outlier split ({args.outliers} channels)" if args.outliers else ""),
                   "model_init_s": round(init_s, 1)},
        "decode_ms_per_token": round(step_ms, 3),
        "prefill_and_pack_s": round(runs[2], 2),
        "generate_s": round(runs[new], 2),
        "attention_us_per_layer": round(attn_us, 2),
        "attention_share_of_decode_step": round(cfg.num_hidden_layers * attn_us * 1e-3 / step_ms, 4),
        "telemetry": tel,
    }


def bench_host(args, dev) -> dict:
    """Host cost of one decode-attention call: the Python path an HF decode step takes
    (fused_attention on a packed cache layer) and the bare libtq wrapper, timed over many
    back-to-back calls on a small layer (the device time per call is reported beside it,
    so a host-bound loop shows as wall time above device time)."""
    import torch

    from turboquant.runtime import kernels as K
    from turboquant.runtime.attention import fused_attention
    from turboquant.runtime.packed_qmse_cache import PackedMSELayer
    from turboquant.runtime.synthetic import kv_bf16, query_bf16

    B, Hq, Hkv, N, D = 1, 40, 8, 4096, 128  # config-5 heads, a short history
    layer = PackedMSELayer(bits=4, use_qjl_keys=True, quantize_decode=True)
    layer.initialize_from_dense(kv_bf16((B, Hkv, N, D), seed=1, device=dev), kv_bf16((B, Hkv, N, D), seed=2, device=dev))
    q = query_bf16(B, Hq, D, seed=3, device=dev).unsqueeze(2)
    mask = torch.ones(B, 1, 1, N, dtype=torch.bool, device=dev)
    s, c = layer._store, layer.codecs
    calls = {
        "fused_attention": lambda: fused_attention(q, layer, Hq // Hkv),
        "fused_attention_masked": lambda: fused_attention(q, layer, Hq // Hkv, mask),
        "kernels.decode_attention": lambda: K.decode_attention(
            q, k_codes=s.kc, k_norms=s.kn, v_codes=s.vc, v_norms=s.vn, n_tokens=N, key=c.key, value=c.value,
            k_signs=s.ks, k_rnorms=s.kr, qjl=c.qjl),
    }
    out = {}
    for name, fn in calls.items():
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        reps = 2000
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        t_host = time.perf_counter() - t0
        torch.cuda.synchronize()
        t_wall = time.perf_counter() - t0
        out[name] = {"host_us_per_call": round(t_host / reps * 1e6, 2),
                     "wall_us_per_call": round(t_wall / reps * 1e6, 2),
                     "device_us_per_call": round(e0.elapsed_time(e1) * 1e3 / reps, 2)}
        print(f"[bench] host {name}: {out[name]}", file=sys.stderr, flush=True)
    return {"metric": "decode-attention host cost per call", "unit": "us",
            "config": {"workload": f"B={B}, Hq={Hq}, Hkv={Hkv}, N={N}, 4-bit Q_prod, 2000 back-to-back calls"},
            "calls": out}


def bench_dequant(args, dev) -> dict:
    """The decoders (`tq_dequantize_prod` for keys, `tq_dequantize_mse` for values) on
    `--context` tokens of every (batch row, KV head): a whole C2 layer by default; 1024 tokens is
    one range of the chunked attention path.  Device time per call (HIP events on the launch
    stream), and the fp32 matrix work against the MI355X dense fp32 matrix peak."""
    import torch

    from turboquant.runtime import kernels as K
    from turboquant.runtime.params import layer_codecs

    B, Hkv, N, D, bits = args.batch, args.kv_heads, args.context, 128, args.bits
    qjl = not args.no_qjl
    lc = layer_codecs(D, bits, 0, qjl, dev)
    gen = torch.Generator(device=dev).manual_seed(5)

    def rand_bytes(*shape):
        return torch.randint(0, 256, shape, dtype=torch.uint8, device=dev, generator=gen)

    def rand_norms():
        return torch.rand(B, Hkv, N, device=dev, generator=gen).half()

    kc, kn = rand_bytes(B, Hkv, N, K.row_bytes(D, lc.key_bits)), rand_norms()
    ks, kr = rand_bytes(B, Hkv, N, D // 8), rand_norms()
    vc, vn = rand_bytes(B, Hkv, N, K.row_bytes(D, bits)), rand_norms()

    def dec_k():
        if qjl:
            K.dequantize_prod(kc, kn, ks, kr, N, lc.key, lc.qjl)
        else:
            K.dequantize_mse(kc, kn, N, lc.key)

    def dec_v():
        K.dequantize_mse(vc, vn, N, lc.value)

    if args.outliers:
        # outlier-split layers: both channel groups of K and of V into full rows, the first
        # --outliers channels as the outlier group, one bit wider
        import numpy as np

        from turboquant.runtime.params import split_codecs

        sc = split_codecs(np.arange(args.outliers, D), np.arange(args.outliers), bits, 1, 0, qjl, dev)
        out = torch.empty(B, Hkv, N, D, dtype=torch.bfloat16, device=dev)

        def group_data(g):
            d = [rand_bytes(B, Hkv, N, K.row_bytes(g.dim, g.bits)), rand_norms()]
            if g.qjl_ch is not None:
                d += [rand_bytes(B, Hkv, N, K.row_bytes(g.dim, 1)), rand_norms()]
            return g, d

        kg = [group_data(g) for g in (sc.key_normal, sc.key_outlier)]
        vg = [group_data(g) for g in (sc.value_normal, sc.value_outlier)]

        def dec_groups(gs):
            for i, (g, d) in enumerate(gs):
                extra = {"signs": d[2], "rnorms": d[3]} if len(d) == 4 else {}
                K.dequantize_group(d[0], d[1], N, g, out, merge=i == 1, **extra)

        def dec_k():  # noqa: F811
            dec_groups(kg)

        def dec_v():  # noqa: F811
            dec_groups(vg)

    def device_us(fn):
        for _ in range(max(args.warmup, 1)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / args.steps

    n_vec = B * Hkv * N
    k_us, v_us = device_us(dec_k), device_us(dec_v)
    # one D x D fp32 matrix-vector product per vector (C[code] @ R), a second one for the QJL correction
    k_tflops = n_vec * (2 if qjl else 1) * 2 * D * D / (k_us * 1e-6) / 1e12
    v_tflops = n_vec * 2 * D * D / (v_us * 1e-6) / 1e12
    peak = 157.3
    return {"metric": "decode (dequantize) per call", "value": round(k_us + v_us, 2), "unit": "us",
            "higher_is_better": False, "dtype": "f32",
            "config": {"workload": f"{N} tokens of B={B} x Hkv={Hkv}: {lc.key_bits}-bit "
                                   f"{'Q_prod' if qjl else 'Q_mse'} keys, {bits}-bit Q_mse values"
                                   + (f", outlier split ({args.outliers} channels at {bits + 1} bits; both "
                                      "groups of K and of V; the flop figures count 128-channel chains)"
                                      if args.outliers else ""),
                       "vectors_per_call": n_vec},
            "steps": args.steps,
            "keys": {"us": round(k_us, 2), "tflops": round(k_tflops, 1), "frac": round(k_tflops / peak, 3)},
            "values": {"us": round(v_us, 2), "tflops": round(v_tflops, 1), "frac": round(v_tflops / peak, 3)},
            "peak_tflops": peak}


def bench_append(args, dev) -> dict:
    """Decode-append: the encoders on one new token per (batch row, KV head), writing in place
    at a slot of a capacity buffer, as a decode step does for every packed layer.  K (Q_prod or
    Q_mse) and V (Q_mse) per layer, timed eagerly (launch included) and as a HIP graph of
    `--layers` layers (device time)."""
    import torch

    from turboquant.runtime import kernels as K
    from turboquant.runtime.params import layer_codecs
    from turboquant.runtime.synthetic import kv_bf16

    B, Hkv, D, bits, cap = args.batch, args.kv_heads, 128, args.bits, 64
    qjl = not args.no_qjl
    lc = layer_codecs(D, bits, 0, qjl, dev)
    kb = lc.key_bits
    buf = {"kc": torch.zeros(B, Hkv, cap, K.row_bytes(D, kb), dtype=torch.uint8, device=dev),
           "kn": torch.zeros(B, Hkv, cap, dtype=torch.float16, device=dev),
           "ks": torch.zeros(B, Hkv, cap, D // 8, dtype=torch.uint8, device=dev),
           "kr": torch.zeros(B, Hkv, cap, dtype=torch.float16, device=dev),
           "vc": torch.zeros(B, Hkv, cap, K.row_bytes(D, bits), dtype=torch.uint8, device=dev),
           "vn": torch.zeros(B, Hkv, cap, dtype=torch.float16, device=dev)}
    k = kv_bf16((B, Hkv, 1, D), seed=1, device=dev)
    v = kv_bf16((B, Hkv, 1, D), seed=2, device=dev)

    def enc_k(slot):
        if qjl:
            K.quantize_prod(k, lc.key, lc.qjl, buf["kc"], buf["kn"], buf["ks"], buf["kr"], offset=slot)
        else:
            K.quantize_mse(k, lc.key, buf["kc"], buf["kn"], offset=slot)

    def enc_v(slot):
        K.quantize_mse(v, lc.value, buf["vc"], buf["vn"], offset=slot)

    if args.outliers:
        # outlier-split layers: both channel groups, the first --outliers channels as the outlier
        # group (the split's encoders take any sorted channel subset; which ones does not change
        # the work), the outlier group one bit wider
        import numpy as np

        from turboquant.runtime.params import split_codecs

        outl = np.arange(args.outliers)
        sc = split_codecs(np.arange(args.outliers, D), outl, bits, 1, 0, qjl, dev)

        def group_bufs(g, prod):
            b = [torch.zeros(B, Hkv, cap, K.row_bytes(g.dim, g.bits), dtype=torch.uint8, device=dev),
                 torch.zeros(B, Hkv, cap, dtype=torch.float16, device=dev)]
            if prod:
                b += [torch.zeros(B, Hkv, cap, K.row_bytes(g.dim, 1), dtype=torch.uint8, device=dev),
                      torch.zeros(B, Hkv, cap, dtype=torch.float16, device=dev)]
            return b

        kgroups = [(g, group_bufs(g, qjl)) for g in (sc.key_normal, sc.key_outlier)]
        vgroups = [(g, group_bufs(g, False)) for g in (sc.value_normal, sc.value_outlier)]

        def enc_k(slot):  # noqa: F811
            for g, b in kgroups:
                K.quantize_group(k, g, *b, offset=slot)

        def enc_v(slot):  # noqa: F811
            for g, b in vgroups:
                K.quantize_group(v, g, *b, offset=slot)

    def eager_us(fn, reps=400):
        for i in range(20):
            fn(i % cap)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            fn(i % cap)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    k_us, v_us = eager_us(enc_k), eager_us(enc_v)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li in range(args.layers):
            enc_k(li % cap)
            enc_v(li % cap)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    layer_us = e0.elapsed_time(e1) * 1e3 / (args.steps * args.layers)
    return {"metric": "decode-append encode, K + V per layer and decode step", "value": round(layer_us, 2),
            "unit": "us", "higher_is_better": False,
            "config": {"workload": f"one token per (batch row, KV head): B={B}, Hkv={Hkv}, {bits}-bit "
                                   f"{'Q_prod' if qjl else 'Q_mse'} keys, {bits}-bit Q_mse values"
                                   + (f", outlier split ({args.outliers} channels at {bits + 1} bits; "
                                      "both groups of K and of V)" if args.outliers else ""),
                       "vectors_per_call": B * Hkv},
            "graph_layers": args.layers, "steps": args.steps,
            "eager_us_per_call": {"keys": round(k_us, 2), "values": round(v_us, 2)}}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--q-heads", type=int, default=32)
    ap.add_argument("--kv-heads", type=int, default=8)
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--no-qjl", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="replay one captured HIP graph per step instead of launching every layer from Python "
                         "(on ROCm 7 the graph's kernel nodes cost ~3 us more per call than stream launches)")
    ap.add_argument("--eager", action="store_true", help="stream launches (the default; kept for old command lines)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed region, run a plain elementwise copy of one layer's packed size "
                         "(reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--outliers", type=int, default=0,
                    help="measure outlier-split layers with this many outlier channels instead of the C2 line "
                         "(with --c5: split every layer of the end-to-end run)")
    ap.add_argument("--c5", action="store_true",
                    help="BASELINE config 5 end to end (random-init QwQ-32B architecture) instead of the C2 line")
    ap.add_argument("--c5-layers", type=int, default=64)
    ap.add_argument("--c5-prompt", type=int, default=131072)
    ap.add_argument("--c5-new", type=int, default=512)
    ap.add_argument("--host", action="store_true",
                    help="host cost per decode-attention call (Python wrappers) instead of the C2 line")
    ap.add_argument("--append", action="store_true",
                    help="decode-append encoders (one new token per batch row and KV head) instead of the C2 line")
    ap.add_argument("--dequant", action="store_true",
                    help="the decoders on --context tokens per (batch row, KV head) instead of the C2 line")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the TurboQuant decode path is single-GPU "
              "(every configuration fits one MI355X); multi-GPU sharding is design-only.", file=sys.stderr)
        return 2

    import torch

    from turboquant.runtime import kernels as K
    from turboquant.runtime.params import layer_codecs
    from turboquant.runtime.synthetic import kv_bf16, query_bf16

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.append:
        print(json.dumps(bench_append(args, dev)))
        return 0
    if args.dequant:
        print(json.dumps(bench_dequant(args, dev)))
        return 0
    if args.c5:
        print(json.dumps(bench_c5(args, dev)))
        return 0
    if args.outliers:
        print(json.dumps(bench_split(args, dev)))
        return 0
    if args.host:
        print(json.dumps(bench_host(args, dev)))
        return 0
    B, Hq, Hkv, N, D, bits = args.batch, args.q_heads, args.kv_heads, args.context, 128, args.bits
    qjl = not args.no_qjl
    lc = layer_codecs(D, bits, 0, qjl, dev)
    per_tok = packed_bytes_per_token_head(D, bits, qjl)
    layer_bytes = B * Hkv * N * per_tok

    # ------------------------------------------------ prefill quantize all layers
    layers, queries, q_ms = [], [], []
    for li in range(args.layers):
        k = kv_bf16((B, Hkv, N, D), seed=1000 + 2 * li, device=dev)
        v = kv_bf16((B, Hkv, N, D), seed=1001 + 2 * li, device=dev)
        L = {
            "k_codes": torch.empty(B, Hkv, N, K.row_bytes(D, lc.key_bits), dtype=torch.uint8, device=dev),
            "k_norms": torch.empty(B, Hkv, N, dtype=torch.float16, device=dev),
            "v_codes": torch.empty(B, Hkv, N, K.row_bytes(D, bits), dtype=torch.uint8, device=dev),
            "v_norms": torch.empty(B, Hkv, N, dtype=torch.float16, device=dev),
            "k_signs": torch.empty(B, Hkv, N, D // 8, dtype=torch.uint8, device=dev) if qjl else None,
            "k_rnorms": torch.empty(B, Hkv, N, dtype=torch.float16, device=dev) if qjl else None,
        }
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        if qjl:
            K.quantize_prod(k, lc.key, lc.qjl, L["k_codes"], L["k_norms"], L["k_signs"], L["k_rnorms"])
        else:
            K.quantize_mse(k, lc.key, L["k_codes"], L["k_norms"])
        K.quantize_mse(v, lc.value, L["v_codes"], L["v_norms"])
        e1.record()
        torch.cuda.synchronize()
        q_ms.append(e0.elapsed_time(e1))
        del k, v
        layers.append(L)
        queries.append(query_bf16(B, Hq, D, seed=5000 + li, device=dev))
    print(f"[bench] quantized {args.layers} layers: {statistics.median(q_ms):.3f} ms/layer (median)",
          file=sys.stderr, flush=True)

    def attn(li):
        L = layers[li]
        return K.decode_attention(queries[li], n_tokens=N, key=lc.key, value=lc.value, qjl=lc.qjl, **L)

    for _ in range(args.warmup):
        for li in range(args.layers):
            attn(li)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)

    # per-call HIP events on the launch stream (eager calls; each brackets the split
    # and merge kernels of one tq_decode_attention call)
    n_ev = min(args.steps, 10) * args.layers
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    torch.cuda.synchronize()
    for i in range(n_ev):
        starts[i].record(stream)
        attn(i % args.layers)
        ends[i].record(stream)
    torch.cuda.synchronize()
    eager_call_us = statistics.fmean(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))

    # one decode step = all layers launched back to back on one stream, as an HF decode step
    # launches them (the host enqueues a call in ~15 us, well ahead of the GPU, so the timed region
    # holds GPU work only); with --graph the step is captured once in a HIP graph and replayed.
    # Either way the outputs are checked to repeat bit for bit.
    ref = [attn(li) for li in range(args.layers)]
    torch.cuda.synchronize()
    again = [attn(li) for li in range(args.layers)]
    torch.cuda.synchronize()
    bad = [li for li in range(args.layers) if not torch.equal(again[li], ref[li])]
    if bad:
        print(f"[bench] a repeated call differs on layers {bad}", file=sys.stderr)
        return 1
    del again
    graph = None
    if args.graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = [attn(li) for li in range(args.layers)]
        for rep in range(2):
            graph.replay()
            torch.cuda.synchronize()
            bad = [li for li in range(args.layers) if not torch.equal(outs[li], ref[li])]
            if bad:
                print(f"[bench] graph replay {rep} differs from eager on layers {bad}", file=sys.stderr)
                return 1
            attn(0)  # eager work between replays
        torch.cuda.synchronize()

    def step():
        if graph is not None:
            graph.replay()
        else:
            for li in range(args.layers):
                attn(li)

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_us = e0.elapsed_time(e1) * 1e3 / args.steps
    avg_us = step_us / args.layers
    ms_per_step = elapsed * 1e3 / args.steps
    value = layer_bytes * args.layers * args.steps / elapsed / 1e9
    achieved = layer_bytes / (avg_us * 1e-6) / 1e9

    copy_cal = None
    if args.copy_calibration:
        # torch.neg over fp32: one read and one write of exactly `layer_bytes` each
        src = torch.randn(layer_bytes // 4, device=dev)
        dst = torch.empty_like(src)
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.neg(src, out=dst)
        c0.record(stream)
        for _ in range(3):
            torch.neg(src, out=dst)
        c1.record(stream)
        torch.cuda.synchronize()
        copy_cal = {"kernel": "torch.neg fp32 (elementwise)", "read_bytes": src.numel() * 4,
                    "write_bytes": dst.numel() * 4, "us": round(c0.elapsed_time(c1) * 1e3 / 3, 2)}
        del src, dst

    # prefill quantizer: bytes = bf16 K+V in + packed out; flops = 2 D^2 per matvec (4 for Q_prod K + V)
    q_s = statistics.median(q_ms) * 1e-3
    n_vec = B * Hkv * N
    q_bytes = n_vec * (4 * D + per_tok)
    q_flops = n_vec * 2 * D * D * (4 if qjl else 2)

    is_c2 = (B, Hq, Hkv, N, bits, qjl) == (8, 32, 8, 32768, 4, True)
    traffic = measured_traffic() if is_c2 else None
    line = {
        "metric": "fused decode-attn us/layer + packed-KV GB/s (% HBM peak), 8B KV shape @32K",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "us_per_layer": round(avg_us, 3),
        "launch": "eager" if graph is None else "hip_graph",
        "hbm_peak_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("u8 codes; int8-limb key MFMAs (<= 4 heads per KV head, else bf16 hi/lo), fp16 value "
                  "MFMAs, fp32 accumulate"),
        "data": "synthetic",
        "config": {
            "workload": (f"{_shape_name(B, Hq, Hkv, N, bits, qjl)}: decode attention over {args.layers} "
                         f"independently seeded packed "
                         f"layers, B={B}, Hq={Hq}, Hkv={Hkv}, D={D}, N={N}, "
                         + (f"{bits}-bit Q_prod K ({bits - 1}-bit MSE + 1-bit QJL) / {bits}-bit Q_mse V" if qjl
                            else f"{bits}-bit Q_mse K and V")),
            "packed_bytes_per_layer": layer_bytes,
            "packed_bytes_per_token_head": per_tok,
            "layers": args.layers,
            "batch": B,
            "context": N,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": ("tq_decode_attention = split_kernel + merge_kernel; duration = HIP events around the "
                       "timed steps on the launch stream / (steps x layers)"),
            "us_per_call": round(avg_us, 3),
            "eager_us_per_call": round(eager_call_us, 3),
        },
        "prefill_quantizer": {
            "ms_per_layer": round(q_s * 1e3, 3),
            "GB_per_s": round(q_bytes / q_s / 1e9, 1),
            "TFLOP_per_s": round(q_flops / q_s / 1e12, 2),
            "fp32_valu_peak_tflops": VALU_FP32_PEAK_TFLOPS,
        },
    }
    if copy_cal is not None:
        line["copy_calibration"] = copy_cal
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(bits)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
