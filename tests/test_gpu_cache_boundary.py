"""GPU parity of the reference-named quantizer boundary of the cache layer
(PackedMSELayer._encode_group, _encode_keys_qjl_group, _decode_group,
_decode_keys_qjl_group; reference runtime/packed_qmse_cache.py:285-330, 376-435):
codes, norms, QJL signs and residual norms bit-exact against the CPU oracle, decoded
rows bit-exact against the oracle decoders."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from turboquant.runtime.packed_qmse_cache import PackedMSELayer, PackedQJL, PackedTensorMSE
from turboquant.runtime.params import layer_codecs
from turboquant.runtime.synthetic import kv_bf16

pytestmark = pytest.mark.gpu

D = 128


def u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_encode_group_and_decode_group_match_oracle(cuda, bits):
    c = layer_codecs(D, bits, 0, False, cuda).value
    x = kv_bf16((2, 3, 157, D), seed=40 + bits, device=cuda)
    p = PackedMSELayer._encode_group(x, c.rotation, c.centers, c.boundaries, bits)
    torch.cuda.synchronize()
    assert isinstance(p, PackedTensorMSE) and p.original_shape == (2, 3, 157, D) and p.bits == bits
    assert p.packed_indices.shape == (2, 3, 157, D * bits // 8) and p.norms.dtype == torch.float16
    R, C, Bd = (t.cpu().numpy() for t in (c.rotation, c.centers, c.boundaries))
    rc, rn = O.encode_mse(u16(x).reshape(-1, D), bits, R, Bd)
    assert np.array_equal(p.packed_indices.cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(u16(p.norms).reshape(-1), rn)
    dec = PackedMSELayer._decode_group(p, c.rotation, c.centers)
    torch.cuda.synchronize()
    assert dec.dtype == torch.bfloat16 and dec.shape == x.shape
    ref = O.decode_mse(rc, rn, bits, D, R, C)
    assert np.array_equal(u16(dec).reshape(-1, D), ref)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_encode_keys_qjl_group_and_decode_match_oracle(cuda, bits):
    lc = layer_codecs(D, bits, 0, True, cuda)
    k = kv_bf16((1, 4, 211, D), seed=60 + bits, device=cuda)
    layer = PackedMSELayer(bits=bits, use_qjl_keys=True)
    mse, qjl = layer._encode_keys_qjl_group(k, lc.key.rotation, lc.key.centers, lc.key.boundaries, bits - 1, lc.qjl)
    torch.cuda.synchronize()
    assert isinstance(mse, PackedTensorMSE) and isinstance(qjl, PackedQJL) and qjl.dimension == D
    R, C, Bd, S = (t.cpu().numpy() for t in (lc.key.rotation, lc.key.centers, lc.key.boundaries, lc.qjl))
    rc, rn, rs, rr = O.encode_prod(u16(k).reshape(-1, D), bits - 1, R, C, Bd, S)
    assert np.array_equal(mse.packed_indices.cpu().numpy().reshape(rc.shape), rc)
    assert np.array_equal(u16(mse.norms).reshape(-1), rn)
    assert np.array_equal(qjl.packed_signs.cpu().numpy().reshape(rs.shape), rs)
    assert np.array_equal(u16(qjl.residual_norms).reshape(-1), rr)
    dec = layer._decode_keys_qjl_group(mse, qjl, lc.key.rotation, lc.key.centers, lc.qjl)
    torch.cuda.synchronize()
    ref = O.decode_prod(rc, rn, rs, rr, bits - 1, D, R, C, S)
    assert np.array_equal(u16(dec).reshape(-1, D), ref)


def test_decode_group_of_a_capacity_view(cuda):
    """The packed views a cache layer hands out ([:, :, :N] of capacity buffers) decode the
    same as the compact tensors."""
    layer = PackedMSELayer(bits=4, use_qjl_keys=False, reserve_tokens=64)
    k = kv_bf16((1, 2, 90, D), seed=5, device=cuda)
    layer.initialize_from_dense(k, k)
    kp = layer.keys_packed
    assert not kp.packed_indices.is_contiguous()
    c = layer.codecs.key
    got = PackedMSELayer._decode_group(kp, c.rotation, c.centers)
    compact = PackedTensorMSE(kp.packed_indices.contiguous(), kp.norms.contiguous(), kp.original_shape,
                              kp.original_dtype, kp.bits)
    assert torch.equal(got, PackedMSELayer._decode_group(compact, c.rotation, c.centers))
    assert torch.equal(got, layer._decode_keys_full())
