"""Host-side constants of the codecs: PolarQuant value codebooks, the seeded
random rotation, and the config-derived key zero points (RoPE-averaged k_proj
bias, DC-channel mask).  Computed once per cache on the host (NumPy) and
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
# head dims the gfx950 kernels are built for (the MFMA decode serves 128, the
# VALU decode 64 and 256)
HEAD_DIMS = (64, 128, 256)


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


# --------------------------------------------------------------------------- #
# Zero points of asym-NF4 keys that come from the model config, not the data   #
# (turboquant_pro/per_channel_kv.py:234-267).  Computed on the host in float64 #
# NumPy with the reference's operation order, rounded to fp32 where it does.   #
# --------------------------------------------------------------------------- #


def dc_channel_mask(rope_theta: float, head_dim: int, window: int) -> np.ndarray:
    """``(head_dim,)`` bool: channels whose rotary wavelength exceeds ``window``
    tokens (``zero_point="sparse"`` keeps the channel mean only there)."""
    half = head_dim // 2
    inv = rope_theta ** (-2.0 * np.arange(half) / head_dim)
    wl = 2.0 * np.pi / inv
    return np.tile(wl, 2)[:head_dim] > float(window)


def dc_mask_words(mask: np.ndarray) -> list[int]:
    """A ``(head_dim,)`` bool channel mask (head_dim <= 256) as the
    descriptor's eight uint32 words: channel j is bit j % 32 of word j // 32,
    words past the mask are 0."""
    m = np.asarray(mask, bool).reshape(-1)
    if m.size > 256 or m.size % 32:
        raise ValueError(f"channel mask of {m.size} channels")
    words = [int(sum(1 << b for b in range(32) if m[32 * w + b])) for w in range(m.size // 32)]
    return words + [0] * (8 - len(words))


def rope_averaged_bias(k_bias: np.ndarray, rope_theta: float, head_dim: int, start: int,
                       n: int) -> np.ndarray:
    """``(H, head_dim)`` fp32 zero point of ``zero_point="bias"``: the k_proj
    bias rotated by RoPE and averaged over positions ``[start, start + n)``,
    ``b * mean(cos) + rotate_half(b) * mean(sin)``."""
    half = head_dim // 2
    inv = rope_theta ** (-2.0 * np.arange(half, dtype=np.float64) / head_dim)
    pos = np.arange(start, start + n, dtype=np.float64)
    ang = pos[:, None] * inv[None, :]
    mc = np.cos(ang).mean(axis=0)
    ms = np.sin(ang).mean(axis=0)
    c_full = np.concatenate([mc, mc]).astype(np.float32)
    s_full = np.concatenate([ms, ms]).astype(np.float32)
    b = np.asarray(k_bias, dtype=np.float32).reshape(-1, head_dim)
    rh = np.concatenate([-b[:, half:], b[:, :half]], axis=1)
    return (b * c_full[None, :] + rh * s_full[None, :]).astype(np.float32)
