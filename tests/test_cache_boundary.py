"""The reference-named quantizer boundary of the cache layer (CPU part): the static and
instance methods the reference's callers use exist with the reference's parameter names
(runtime/packed_qmse_cache.py:285-330, 376-435), and the containers' ``append`` concatenates
along the token axis (:81-92, 135-140)."""

import inspect

import pytest
import torch

from turboquant.runtime.packed_qmse_cache import PackedMSELayer, PackedQJL, PackedTensorMSE

# parameter lists of the reference's definitions (runtime/packed_qmse_cache.py)
REFERENCE_SIGNATURES = {
    "_encode_group": ["tensor", "rotation", "centers", "boundaries", "bits"],                # :376-383 (static)
    "_decode_group": ["packed", "rotation", "centers"],                                     # :404-409 (static)
    "_encode_keys_qjl_group": ["self", "key_states", "rotation", "centers", "boundaries", "bits",
                               "qjl_matrix"],                                               # :285-293
    "_decode_keys_qjl_group": ["self", "mse_packed", "qjl", "rotation", "centers", "qjl_matrix"],  # :312-319
}
STATIC = {"_encode_group", "_decode_group"}


@pytest.mark.parametrize("name", sorted(REFERENCE_SIGNATURES))
def test_reference_method_signatures(name):
    raw = inspect.getattr_static(PackedMSELayer, name)
    assert isinstance(raw, staticmethod) == (name in STATIC), f"{name}: static-ness differs from the reference"
    params = list(inspect.signature(raw.__func__ if isinstance(raw, staticmethod) else raw).parameters)
    assert params == REFERENCE_SIGNATURES[name]


def _packed(n, seed, bits=4, B=2, H=3, D=128):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (B, H, n, D * bits // 8), generator=g, dtype=torch.uint8)
    norms = torch.rand(B, H, n, generator=g).to(torch.float16)
    return PackedTensorMSE(codes, norms, (B, H, n, D), torch.bfloat16, bits)


def test_packed_tensor_append_concatenates_tokens():
    a, b = _packed(5, 1), _packed(3, 2)
    c = a.append(b)
    assert c.original_shape == (2, 3, 8, 128) and c.bits == 4 and c.original_dtype == torch.bfloat16
    assert torch.equal(c.packed_indices[:, :, :5], a.packed_indices)
    assert torch.equal(c.packed_indices[:, :, 5:], b.packed_indices)
    assert torch.equal(c.norms, torch.cat((a.norms, b.norms), dim=2))
    assert c.packed_indices.is_contiguous() and c.num_vectors == 2 * 3 * 8
    assert c.storage_bytes() == a.storage_bytes() + b.storage_bytes()
    with pytest.raises(ValueError):
        a.append(_packed(2, 3, H=4))


def test_packed_qjl_append_concatenates_tokens():
    g = torch.Generator().manual_seed(7)
    s1 = PackedQJL(torch.randint(0, 256, (1, 2, 4, 16), generator=g, dtype=torch.uint8),
                   torch.rand(1, 2, 4, generator=g).half(), 128)
    s2 = PackedQJL(torch.randint(0, 256, (1, 2, 1, 16), generator=g, dtype=torch.uint8),
                   torch.rand(1, 2, 1, generator=g).half(), 128)
    s = s1.append(s2)
    assert s.dimension == 128 and s.packed_signs.shape == (1, 2, 5, 16)
    assert torch.equal(s.packed_signs[:, :, 4], s2.packed_signs[:, :, 0])
    assert torch.equal(s.residual_norms[:, :, :4], s1.residual_norms)


def test_reference_methods_refuse_cpu_tensors():
    """No CPU path: the product raises instead of falling back."""
    from turboquant.runtime.params import layer_codecs

    lc = layer_codecs(128, 4, 0, False, "cpu")
    x = torch.zeros(1, 1, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        PackedMSELayer._encode_group(x, lc.value.rotation, lc.value.centers, lc.value.boundaries, 4)
