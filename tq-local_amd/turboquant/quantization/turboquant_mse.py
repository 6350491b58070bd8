"""TurboQuant quantizer parameters: Lloyd-Max codebook, Haar rotation, QJL matrix.

These are one-time host computations (fp64 numpy / CPU torch RNG) whose
results are uploaded to HBM once per layer.  They follow the reference's
parameter generators step for step, because the parameters must be
bit-identical for the packed codes to be:

* ``build_scalar_codebook``  -- reference ``quantization/turboquant_mse.py:37-110``
* ``random_rotation_matrix`` -- reference ``quantization/turboquant_mse.py:113-121``
* ``generate_qjl_matrix``    -- reference ``runtime/packed_qmse_cache.py:143-145``

The codebook is the Lloyd-Max quantizer of one coordinate of a uniformly
random unit vector in R^D, whose density is
``Gamma(D/2) / (sqrt(pi) Gamma((D-1)/2)) * (1 - x^2)^((D-3)/2)`` on [-1, 1].
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache
from math import gamma, pi, sqrt

import numpy as np
import torch

#: seed offsets of the reference's seed schedule
#: (``runtime/packed_qmse_cache.py:117-118, 255, 262, 265, 278``)
KEY_ROTATION_SEED_OFFSET = 1
QJL_SEED_OFFSET = 31337
OUTLIER_SEED_OFFSET = 7919

DEFAULT_GRID_SIZE = 32769


@dataclass(frozen=True)
class ScalarCodebook:
    dimension: int
    bits: int
    centers: np.ndarray  # fp64 [2^bits]
    boundaries: np.ndarray  # fp64 [2^bits - 1], midpoints of the fp64 centers
    grid_size: int


def coordinate_density(dimension: int, x: np.ndarray) -> np.ndarray:
    """Marginal density of one coordinate of a uniform point on S^{D-1}."""
    out = np.zeros_like(x, dtype=np.float64)
    inside = np.abs(x) <= 1.0
    coef = gamma(dimension / 2.0) / (sqrt(np.pi) * gamma((dimension - 1.0) / 2.0))
    out[inside] = coef * np.power(1.0 - np.square(x[inside]), (dimension - 3.0) / 2.0)
    return out


def _normalised_cdf(grid: np.ndarray, density: np.ndarray) -> np.ndarray:
    step = grid[1] - grid[0]
    cdf = np.cumsum(density) * step
    cdf /= cdf[-1]
    cdf[0] = 0.0
    cdf[-1] = 1.0
    return cdf


def _cell_centroid(grid: np.ndarray, density: np.ndarray, lo: float, hi: float) -> float:
    """Trapezoid-rule centroid of the density over the grid points in [lo, hi]."""
    if hi <= lo:
        return (lo + hi) / 2.0
    sel = (grid >= lo) & (grid <= hi)
    xs = grid[sel]
    if xs.size == 0:
        return (lo + hi) / 2.0
    ws = density[sel]
    mass = np.trapezoid(ws, xs)
    if mass <= 0:
        return (lo + hi) / 2.0
    return float(np.trapezoid(xs * ws, xs) / mass)


@lru_cache(maxsize=32)
def build_scalar_codebook(
    dimension: int,
    bits: int,
    grid_size: int = DEFAULT_GRID_SIZE,
    max_iters: int = 200,
    tol: float = 1e-10,
) -> ScalarCodebook:
    """Lloyd-Max iteration from quantile initialisation (fp64)."""
    if bits <= 0:
        raise ValueError("bits must be positive for TurboQuant_mse.")
    n_levels = 1 << bits
    grid = np.linspace(-1.0, 1.0, grid_size, dtype=np.float64)
    density = coordinate_density(dimension, grid)
    cdf = _normalised_cdf(grid, density)
    probs = np.linspace(0.0, 1.0, n_levels + 2, dtype=np.float64)[1:-1]
    centers = np.interp(probs, cdf, grid)
    for _ in range(max_iters):
        mids = (centers[:-1] + centers[1:]) / 2.0
        edges = np.concatenate(([-1.0], mids, [1.0]))
        nxt = np.array(
            [_cell_centroid(grid, density, edges[i], edges[i + 1]) for i in range(n_levels)],
            dtype=np.float64,
        )
        done = np.max(np.abs(nxt - centers)) < tol
        centers = nxt
        if done:
            break
    return ScalarCodebook(
        dimension=dimension,
        bits=bits,
        centers=centers,
        boundaries=(centers[:-1] + centers[1:]) / 2.0,
        grid_size=grid_size,
    )


@lru_cache(maxsize=16)
def random_rotation_matrix(dimension: int, seed: int) -> np.ndarray:
    """Haar-random orthogonal matrix: QR of a PCG64 Gaussian, columns sign-fixed by diag(R)."""
    g = np.random.default_rng(seed).standard_normal((dimension, dimension))
    q, r = np.linalg.qr(g)
    s = np.sign(np.diag(r))
    s[s == 0.0] = 1.0
    return (q * s).astype(np.float32)


def generate_qjl_matrix(dimension: int, seed: int) -> torch.Tensor:
    """i.i.d. N(0,1) fp32 [D, D] from torch's CPU mt19937 generator."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(dimension, dimension, generator=gen, dtype=torch.float32)


def codebook_f32(dimension: int, bits: int, grid_size: int = DEFAULT_GRID_SIZE) -> tuple[np.ndarray, np.ndarray]:
    """(centers, boundaries) as fp32, each cast from fp64 independently
    (reference ``runtime/packed_qmse_cache.py:233-234``)."""
    cb = build_scalar_codebook(dimension, bits, grid_size)
    return cb.centers.astype(np.float32), cb.boundaries.astype(np.float32)


def approx_pi_over_2_scale(dimension: int) -> float:
    """QJL estimator scale sqrt(pi/2)/D (reference ``runtime/packed_qmse_cache.py:326``)."""
    return sqrt(pi / 2) / dimension
