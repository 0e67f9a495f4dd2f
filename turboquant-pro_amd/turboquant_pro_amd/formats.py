"""Conversions between the HBM layout of the gfx950 cache and the reference's
container byte layouts (host side, NumPy; used for export and inspection).

* Key codes are stored exactly as the reference packs them
  (turboquant_pro/per_channel_kv.py:87-93): 64 bytes per (token, head).
* Value codes are the reference's little-endian pack
  (turboquant_pro/core.py:350-398) when stored per token; with the MFMA-tiled
  order (page_tokens % 16 == 0 and group_tokens % 32 == 0) each 16-token tile
  holds 64 units of vrow/4 bytes -- unit (lg, c) carries tokens
  [4lg, 4lg+4) x channels [8c, 8c+8), the codes of token pairs (0,1) and (2,3)
  of one channel side by side -- a lossless permutation of the same bits.
"""

from __future__ import annotations

import numpy as np


def pack_values(codes: np.ndarray, bits: int) -> np.ndarray:
    """Flat codes -> reference value bytes (3-bit: 8 codes per 24-bit LE word)."""
    v = np.ascontiguousarray(codes, dtype=np.uint32).reshape(-1)
    per = {2: 4, 3: 8, 4: 2}[bits]
    pad = (-v.size) % per
    if pad:
        v = np.concatenate([v, np.zeros(pad, np.uint32)])
    v = v.reshape(-1, per)
    word = np.zeros(v.shape[0], np.uint32)
    for k in range(per):
        word |= v[:, k] << np.uint32(bits * k)
    if bits == 3:
        return np.stack([(word >> s) & 0xFF for s in (0, 8, 16)], 1).astype(np.uint8).reshape(-1)
    return word.astype(np.uint8)


def unit_bit(u: int, nt: int, vb: int) -> int:
    """Bit of (token u of the unit, channel nt of the unit) inside a tiled unit."""
    return (2 * nt + (u >> 1)) * (2 * vb) + (u & 1) * vb


def untile_values(tile_bytes: np.ndarray, vb: int, D: int = 128) -> np.ndarray:
    """Codes ``(16, D)`` of one 16-token tile stored in the tiled order."""
    vrow = D * vb // 8
    unit = vrow // 4
    raw = np.asarray(tile_bytes, np.uint8).reshape(64, unit)
    bits = np.unpackbits(raw, axis=1, bitorder="little")          # (64, unit*8)
    out = np.zeros((16, D), np.uint8)
    for lg in range(4):
        for c in range(16):
            ub = bits[16 * lg + c]
            for u in range(4):
                for nt in range(8):
                    b0 = unit_bit(u, nt, vb)
                    val = 0
                    for k in range(vb):
                        val |= int(ub[b0 + k]) << k
                    out[4 * lg + u, 8 * c + nt] = val
    return out


def untile_value_rows(rows: np.ndarray, vb: int, D: int = 128) -> np.ndarray:
    """Tiled value bytes of ``n`` tokens (n % 16 == 0, tile-aligned) -> codes (n, D)."""
    vrow = D * vb // 8
    rows = np.asarray(rows, np.uint8).reshape(-1, 16 * vrow)
    return np.concatenate([untile_values(t, vb, D) for t in rows], axis=0)
