"""tq_decode_attention_noalloc (no workspace argument, no allocation) against
tq_decode_attention, called through the C ABI.  Named to be collected last: it must
pass after every other GPU test as well as alone.

Both entry points run the same kernels on the same split, so their outputs must be
bit-identical; the fp32 output is also held to the fp64 oracle at 2e-3 * ||out||_inf.
Two calls in a row, the second smaller, check that the shared device array carries
nothing from one call into the next.  A shape whose partials exceed the array is
rejected on the host (TQ_ERR_WORKSPACE) before any launch.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from turboquant.runtime import _lib
from turboquant.runtime import kernels as K
from turboquant.runtime.params import layer_codecs
from turboquant.runtime.synthetic import kv_bf16, query_bf16

pytestmark = pytest.mark.gpu

D = 128
TOL = 2e-3
SCRATCH_BYTES = 8 << 20  # TQ_NOALLOC_SCRATCH_BYTES in include/tq.h


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def vp(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def make_layer(dev, B, Hkv, N, seed):
    lc = layer_codecs(D, 4, 0, True, dev)
    k = kv_bf16((B, Hkv, N, D), seed=seed, device=dev)
    v = kv_bf16((B, Hkv, N, D), seed=seed + 1, device=dev)
    L = {"kc": torch.empty(B, Hkv, N, 48, dtype=torch.uint8, device=dev),
         "kn": torch.empty(B, Hkv, N, dtype=torch.float16, device=dev),
         "ks": torch.empty(B, Hkv, N, 16, dtype=torch.uint8, device=dev),
         "kr": torch.empty(B, Hkv, N, dtype=torch.float16, device=dev),
         "vc": torch.empty(B, Hkv, N, 64, dtype=torch.uint8, device=dev),
         "vn": torch.empty(B, Hkv, N, dtype=torch.float16, device=dev)}
    K.quantize_prod(k, lc.key, lc.qjl, L["kc"], L["kn"], L["ks"], L["kr"])
    K.quantize_mse(v, lc.value, L["vc"], L["vn"])
    return lc, L


def common_args(q, lc, L, B, Hq, Hkv, N):
    return [vp(q), B, Hq, Hkv, D, None, None, N, N, vp(L["kc"]), vp(L["kn"]), vp(L["ks"]), vp(L["kr"]),
            vp(L["vc"]), vp(L["vn"]), 3, 4, 1, vp(lc.key.rotation), vp(lc.key.centers), vp(lc.qjl),
            vp(lc.value.rotation), vp(lc.value.centers), ctypes.c_float(0.0)]


def outputs(dev, B, Hq):
    return (torch.full((B, Hq, D), float("nan"), device=dev), torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev),
            torch.full((B, Hq), float("nan"), device=dev))


def run_pair(dev, B, Hq, Hkv, N, seed):
    lib = _lib.load()
    lc, L = make_layer(dev, B, Hkv, N, seed)
    q = query_bf16(B, Hq, D, seed=seed + 2, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    a32, a16, alse = outputs(dev, B, Hq)
    ws = torch.empty(int(lib.tq_decode_attention_workspace_bytes(B, Hq, Hkv, D, N)), dtype=torch.uint8, device=dev)
    st = lib.tq_decode_attention(*common_args(q, lc, L, B, Hq, Hkv, N), vp(a32), vp(a16), vp(alse), vp(ws),
                                 ws.numel(), stream)
    assert st == 0, st
    b32, b16, blse = outputs(dev, B, Hq)
    st = lib.tq_decode_attention_noalloc(*common_args(q, lc, L, B, Hq, Hkv, N), vp(b32), vp(b16), vp(blse), stream)
    assert st == 0, st
    torch.cuda.synchronize()
    assert torch.equal(a32, b32) and torch.equal(a16, b16) and torch.equal(alse, blse)
    host = {"kcodes": L["kc"].cpu().numpy(), "knorms": u16(L["kn"]), "vcodes": L["vc"].cpu().numpy(),
            "vnorms": u16(L["vn"]), "signs": L["ks"].cpu().numpy(), "rnorms": u16(L["kr"]),
            "Rk": lc.key.rotation.cpu().numpy(), "Ck": lc.key.centers.cpu().numpy(),
            "Rv": lc.value.rotation.cpu().numpy(), "Cv": lc.value.centers.cpu().numpy(),
            "S": lc.qjl.cpu().numpy(), "kbits": 3, "vbits": 4}
    ref = O.fused_attention_f64(u16(q), host)
    err = np.abs(b32.cpu().numpy() - ref).max()
    assert err <= TOL * np.abs(ref).max(), err


def test_noalloc_matches_workspace_entry_point_twice(cuda):
    print("[no_alloc] call 1: B=4 Hq=32 Hkv=8 N=5000", flush=True)
    run_pair(cuda, 4, 32, 8, 5000, seed=41)
    print("[no_alloc] call 2 (smaller): B=1 Hq=8 Hkv=2 N=700", flush=True)
    run_pair(cuda, 1, 8, 2, 700, seed=43)


def test_noalloc_rejects_partials_beyond_the_array(cuda):
    """B=128, Hq=128, Hkv=16: 2048 groups -> one split, 16384 partial rows of 130 fp32 =
    8.5 MB > 8 MiB.  The buffers are real and sized for the call, so nothing would fault
    even if the host check were missing; the status must be TQ_ERR_WORKSPACE."""
    lib = _lib.load()
    B, Hq, Hkv, N = 128, 128, 16, 16
    assert lib.tq_decode_attention_workspace_bytes(B, Hq, Hkv, D, N) > SCRATCH_BYTES
    lc, L = make_layer(cuda, B, Hkv, N, seed=45)
    q = query_bf16(B, Hq, D, seed=46, device=cuda)
    o32, o16, olse = outputs(cuda, B, Hq)
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    st = lib.tq_decode_attention_noalloc(*common_args(q, lc, L, B, Hq, Hkv, N), vp(o32), vp(o16), vp(olse), stream)
    torch.cuda.synchronize()
    assert st == 3, st  # TQ_ERR_WORKSPACE
    assert torch.isnan(o32).all()  # nothing was launched
