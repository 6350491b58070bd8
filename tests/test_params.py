"""Quantizer parameters (a1-a4): pinned to the reference's own outputs (golden
params.json) and to closed-form properties of the Lloyd-Max quantizer."""

import hashlib
import json
import math

import numpy as np
import pytest
import torch

from turboquant.quantization.turboquant_mse import (
    build_scalar_codebook,
    codebook_f32,
    coordinate_density,
    generate_qjl_matrix,
    random_rotation_matrix,
)
from turboquant.runtime.params import layer_codecs

D = 128


@pytest.fixture(scope="module")
def golden(golden_dir):
    return json.loads((golden_dir / "params.json").read_text())


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_bit_identical_to_reference(golden, bits):
    c, b = codebook_f32(D, bits)
    g = golden["codebooks"][str(bits)]
    assert [x.tobytes().hex() for x in c] == g["centers_f32_hex"]
    assert [x.tobytes().hex() for x in b] == g["boundaries_f32_hex"]


@pytest.mark.parametrize("seed", [0, 1])
def test_rotation_bit_identical_to_reference(golden, seed):
    r = random_rotation_matrix(D, seed)
    assert hashlib.sha256(r.tobytes()).hexdigest() == golden["rotations"][str(seed)]["sha256"]


def test_qjl_matrix_bit_identical_to_reference(golden):
    s = generate_qjl_matrix(D, 31337)
    assert hashlib.sha256(s.numpy().tobytes()).hexdigest() == golden["qjl"]["31337"]["sha256"]


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_lloyd_max_fixed_point(bits):
    """Centroid condition on the reference's own grid: every center is the
    conditional mean of its cell and boundaries are midpoints.  The book is odd
    only up to the grid discretisation (the cell test includes both end points,
    so the point shared by two cells counts twice): |c_i + c_{L-1-i}| < 1e-4."""
    cb = build_scalar_codebook(D, bits)
    c = cb.centers
    assert np.all(np.diff(c) > 0)
    assert np.allclose(c, -c[::-1], atol=1e-4)
    assert np.allclose(cb.boundaries, (c[:-1] + c[1:]) / 2)
    grid = np.linspace(-1.0, 1.0, 32769)
    dens = coordinate_density(D, grid)
    edges = np.concatenate(([-1.0], cb.boundaries, [1.0]))
    for i in range(len(c)):
        sel = (grid >= edges[i]) & (grid <= edges[i + 1])
        x, w = grid[sel], dens[sel]
        assert abs(np.trapezoid(x * w, x) / np.trapezoid(w, x) - c[i]) < 1e-9


def test_one_bit_codebook_is_mean_absolute_coordinate():
    """1-bit Lloyd-Max = +-E|x_1| for x uniform on S^{D-1}: Gamma(D/2)/(sqrt(pi) Gamma((D+1)/2))."""
    c = build_scalar_codebook(D, 1).centers
    exact = math.exp(math.lgamma(D / 2) - math.lgamma((D + 1) / 2)) / math.sqrt(math.pi)
    assert abs(c[1] - exact) < 1e-4 and abs(c[0] + exact) < 1e-4


@pytest.mark.parametrize("bits,gauss", [
    (2, [0.4528, 1.5104]),
    (3, [0.2451, 0.7560, 1.3440, 2.1520]),
    (4, [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326]),
])
def test_codebook_near_gaussian_lloyd_max(bits, gauss):
    """Textbook Lloyd-Max levels of N(0,1), scaled by 1/sqrt(D); the sphere marginal
    differs from the Gaussian at O(1/D), so a 2% band pins the construction."""
    c = build_scalar_codebook(D, bits).centers
    pos = c[len(c) // 2:] * math.sqrt(D)
    assert np.allclose(pos, gauss, rtol=0.02)


@pytest.mark.parametrize("seed", [0, 1, 7])
def test_rotation_is_orthogonal(seed):
    r = random_rotation_matrix(D, seed).astype(np.float64)
    assert np.abs(r @ r.T - np.eye(D)).max() < 1e-5


def test_qjl_matrix_is_standard_normal():
    s = generate_qjl_matrix(D, 31337).numpy().astype(np.float64)
    assert abs(s.mean()) < 5.0 / D and abs(s.std() - 1.0) < 0.02  # 5 sigma of the sample mean


def test_seed_schedule_qprod_and_qmse():
    """Q_prod: keys (bits-1) with R(seed+1) + S(seed+31337); values bits with R(seed).
    Q_mse: keys and values share bits and R(seed).  (runtime/packed_qmse_cache.py:226-283)"""
    lc = layer_codecs(D, 4, 5, True, "cpu")
    assert lc.key.bits == 3 and lc.value.bits == 4
    assert np.array_equal(lc.key.rotation.numpy(), random_rotation_matrix(D, 6))
    assert np.array_equal(lc.value.rotation.numpy(), random_rotation_matrix(D, 5))
    assert torch.equal(lc.qjl, generate_qjl_matrix(D, 5 + 31337))
    lm = layer_codecs(D, 3, 5, False, "cpu")
    assert lm.key is lm.value and lm.key.bits == 3 and lm.qjl is None
