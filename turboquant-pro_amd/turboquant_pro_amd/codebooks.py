"""Host-side constants of the codecs: PolarQuant value codebooks and the
seeded random rotation.  Computed once per cache on the host (NumPy) and
uploaded; every per-token operation runs in the gfx950 kernels.

The tables and their fp32 rounding have to be identical to the reference's for
the codes to be bit-exact: Lloyd-Max N(0,1) levels (turboquant_pro/core.py:70-93),
scaled by 1/sqrt(d) in float64 then rounded to fp32, with fp32 midpoints as
boundaries (turboquant_pro/core.py:229-240); the rotation is the Q factor of
``default_rng(seed).standard_normal((d, d))`` in fp32 (turboquant_pro/core.py:252-263).
"""

from __future__ import annotations

import math

import numpy as np

LLOYD_MAX_LEVELS = {
    2: (-1.510, -0.453, 0.453, 1.510),
    3: (-1.748, -1.050, -0.500, -0.069, 0.069, 0.500, 1.050, 1.748),
    4: (-2.401, -1.844, -1.437, -1.099, -0.800, -0.524, -0.262, -0.066,
        0.066, 0.262, 0.524, 0.800, 1.099, 1.437, 1.844, 2.401),
}

SUPPORTED_BITS = tuple(sorted(LLOYD_MAX_LEVELS))


def value_codebook(bits: int, head_dim: int) -> tuple[np.ndarray, np.ndarray]:
    """``(centroids, boundaries)`` fp32 for ``bits``-bit PolarQuant values."""
    if bits not in LLOYD_MAX_LEVELS:
        raise ValueError(f"Unsupported bits={bits}; choose from {list(SUPPORTED_BITS)}")
    levels = np.asarray(LLOYD_MAX_LEVELS[bits], dtype=np.float64) * (1.0 / math.sqrt(head_dim))
    cent = levels.astype(np.float32)
    bnd = ((cent[:-1] + cent[1:]) / np.float32(2.0)).astype(np.float32)
    return cent, bnd


def random_rotation(seed, head_dim: int) -> tuple[np.ndarray, np.ndarray]:
    """``(Pi, Pi_T)``: rotate with ``x @ Pi_T``, unrotate with ``y @ Pi``."""
    gauss = np.random.default_rng(seed).standard_normal((head_dim, head_dim)).astype(np.float32)
    q, _ = np.linalg.qr(gauss)
    return np.ascontiguousarray(q), np.ascontiguousarray(q.T)


def outliers_per_channel(group_tokens: int, outlier_frac: float) -> int:
    """Outliers kept per (head, channel) in a group: ``max(1, round(G * f))``
    with Python's round (turboquant_pro/per_channel_kv.py:274); 0 when f == 0."""
    if outlier_frac <= 0.0:
        return 0
    return max(1, int(round(group_tokens * outlier_frac)))


def group_tokens_for(hot_window: int) -> int:
    """Tokens per flush for a hot window of W tokens: ``(W + 1) // 2``."""
    return (hot_window + 1) // 2


def n_groups_for(length: int, hot_window: int) -> int:
    """Flushed groups after ``length`` appends (first flush at W + 1 tokens)."""
    G = group_tokens_for(hot_window)
    if G == 0 or length <= hot_window:
        return 0
    return (length - (hot_window + 1)) // G + 1
