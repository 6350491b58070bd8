"""tq_value_codebook_f16: the fp16 value codebook of the decode attention (host helper).

Checked against an independent restatement: the cell probabilities from the exact Beta CDF
of one coordinate of a uniform point on S^(d-1) ((x + 1) / 2 ~ Beta((d-1)/2, (d-1)/2)), and a
brute force over every choice of fp16 neighbours.
"""

import ctypes

import numpy as np
import pytest
from scipy.special import betainc

from turboquant.quantization.turboquant_mse import build_scalar_codebook
from turboquant.runtime import _lib
from turboquant.runtime import kernels as K


def neighbours(c32: np.ndarray):
    h = c32.astype(np.float16)
    hv = h.astype(np.float64)
    c = c32.astype(np.float64)
    down = np.where(hv > c, np.nextafter(h, np.float16(-np.inf)), h).astype(np.float64)
    up = np.where(hv < c, np.nextafter(h, np.float16(np.inf)), h).astype(np.float64)
    return down, up


def cell_probabilities(c32: np.ndarray, dim: int) -> np.ndarray:
    c = c32.astype(np.float64)
    edges = np.concatenate([[-1.0], (c[1:] + c[:-1]) / 2, [1.0]])
    a = (dim - 1) / 2.0
    cdf = betainc(a, a, (edges + 1.0) / 2.0)
    return np.diff(cdf)


def best_bias(c32: np.ndarray, P: np.ndarray) -> float:
    down, up = neighbours(c32)
    n = c32.size
    sel = ((np.arange(1 << n)[:, None] >> np.arange(n)[None, :]) & 1).astype(bool)
    vals = np.where(sel, up[None, :], down[None, :])
    return float(np.abs(((vals - c32.astype(np.float64)[None, :]) * P[None, :]).sum(1)).min())


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("dim", [128, 124, 64, 16])  # 124: a split layer's normal group
def test_codebook_f16_is_the_least_biased_choice_of_neighbours(bits, dim):
    c32 = build_scalar_codebook(dim, bits).centers.astype(np.float32)
    out = K.value_codebook_f16(c32, bits, dim)
    down, up = neighbours(c32)
    o = out.astype(np.float64)
    # every value is fp16-exact and one of the centroid's two fp16 neighbours
    assert np.array_equal(out.astype(np.float16).astype(np.float32), out)
    assert np.all((o == down) | (o == up))
    P = cell_probabilities(c32, dim)
    bias = abs(float(((o - c32.astype(np.float64)) * P).sum()))
    rne = abs(float(((c32.astype(np.float16).astype(np.float64) - c32) * P).sum()))
    # within integration accuracy of the brute-force optimum, and never worse than nearest-even
    assert bias <= best_bias(c32, P) + 1e-12
    assert bias <= rne + 1e-12


def test_codebook_f16_rejects_bad_arguments():
    lib = _lib.load()
    c = build_scalar_codebook(128, 3).centers.astype(np.float32)
    out = np.empty_like(c)
    vp = ctypes.c_void_p
    assert lib.tq_value_codebook_f16(None, 3, 128, vp(out.ctypes.data)) == 1
    assert lib.tq_value_codebook_f16(vp(c.ctypes.data), 3, 128, None) == 1
    for bits, dim in ((0, 128), (5, 128), (3, 2)):
        assert lib.tq_value_codebook_f16(vp(c.ctypes.data), bits, dim, vp(out.ctypes.data)) == 1
    bad = c.copy()
    bad[3] = bad[2]  # not strictly increasing
    assert lib.tq_value_codebook_f16(vp(bad.ctypes.data), 3, 128, vp(out.ctypes.data)) == 1
    bad = c.copy()
    bad[-1] = 1.0  # outside (-1, 1)
    assert lib.tq_value_codebook_f16(vp(bad.ctypes.data), 3, 128, vp(out.ctypes.data)) == 1
    bad = c.copy()
    bad[0] = np.nan
    assert lib.tq_value_codebook_f16(vp(bad.ctypes.data), 3, 128, vp(out.ctypes.data)) == 1
