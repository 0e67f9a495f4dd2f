"""Conversions between the HBM layout of the gfx950 cache and the reference's
container byte layouts (host side, NumPy; used for export and inspection).

* Key codes are stored as the reference packs them
  (turboquant_pro/per_channel_kv.py:87-93), 64 bytes per (token, head), with
  one difference: at every position held in the fp16 outlier side-list the
  stored code is the NF4 zero level (7), so a decode's dense pass contributes
  exactly the channel mean there and the side-list adds ``val - mean``.  The
  reference's code at such a position is the nearest level to the stored fp16
  value; :func:`restore_outlier_codes` puts it back on export.
* 3- and 2-bit key codes (uniform grid) are stored as 32-channel chunks of
  pair fields (:func:`key_rows_from_codes`), a permutation of the reference's
  bit stream (:func:`pack_key_codes`) that gives every decode lane its 32
  channels in one load and a channel pair in one field.
* Value codes are the reference's little-endian pack
  (turboquant_pro/core.py:350-398) when stored per token; with the MFMA-tiled
  order (page_tokens % 16 == 0 and group_tokens % 32 == 0) each 16-token tile
  holds 64 units of vrow/4 bytes -- unit (lg, c) carries tokens
  [4lg, 4lg+4) x channels [8c, 8c+8), the codes of token pairs (0,1) and (2,3)
  of one channel side by side -- a lossless permutation of the same bits.
"""

from __future__ import annotations

import numpy as np

# NormalFloat-4 levels (turboquant_pro/per_channel_kv.py:64-84), as the fp32
# constants the kernels use.
NF4 = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
    0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0], dtype=np.float32)
NF4_ZERO_CODE = 7


def _rev4(c: np.ndarray) -> np.ndarray:
    c = c.astype(np.uint8)
    return (((c & 1) << 3) | ((c & 2) << 1) | ((c & 4) >> 1) | ((c & 8) >> 3)).astype(np.uint8)


def nf4_codes(x: np.ndarray, scale: np.ndarray, mean: np.ndarray) -> np.ndarray:
    """Nearest-level NF4 code of fp32 ``x`` given per-element ``scale``/``mean``,
    in the reference's arithmetic (turboquant_pro/per_channel_kv.py:347-383):
    centroid ``mean + scale * NF4[l]`` rounded to fp32 per operation, first
    index of the smallest ``|x - centroid|`` (a NaN distance wins, as
    ``np.argmin`` has it)."""
    x = np.asarray(x, np.float32)[..., None]
    cent = (np.asarray(mean, np.float32)[..., None] + np.asarray(scale, np.float32)[..., None] * NF4)
    return np.argmin(np.abs(x - cent), axis=-1).astype(np.uint8)


def uniform_codes(x: np.ndarray, scale: np.ndarray, zero: np.ndarray, bits: int = 4) -> np.ndarray:
    """Uniform key code of fp32 ``x`` (turboquant_pro/per_channel_kv.py:306):
    ``clip(round_half_even((x - zero) / scale), 0, 2**bits - 1)`` in fp32."""
    x = np.asarray(x, np.float32)
    q = (x - np.asarray(zero, np.float32)) / np.asarray(scale, np.float32)
    return np.clip(np.round(q), 0, (1 << bits) - 1).astype(np.uint8)


def pack_key_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Flat key codes -> the reference's key bytes (turboquant_pro/per_channel_kv.py:87-93):
    each code's ``bits`` low bits least significant first, the bit stream
    filling every byte from its most significant bit."""
    c = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    stream = ((c[:, None] >> np.arange(bits, dtype=np.uint8)) & 1).astype(np.uint8).reshape(-1)
    stream = np.concatenate([stream, np.zeros((-stream.size) % 8, np.uint8)]).reshape(-1, 8)
    return (stream << np.arange(7, -1, -1, dtype=np.uint8)).sum(axis=1, dtype=np.uint32).astype(np.uint8)


def unpack_key_codes(packed: np.ndarray, n_values: int, bits: int) -> np.ndarray:
    """The inverse of :func:`pack_key_codes` (turboquant_pro/per_channel_kv.py:94-100)."""
    b = np.asarray(packed, np.uint8).reshape(-1)
    stream = ((b[:, None] >> np.arange(7, -1, -1, dtype=np.uint8)) & 1).reshape(-1)[: n_values * bits]
    return (stream.reshape(n_values, bits).astype(np.uint16) << np.arange(bits, dtype=np.uint16)).sum(
        axis=1).astype(np.uint8)


def key_rows_from_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Codes ``(n, D)`` -> stored key rows ``(n, D * bits / 8)``: 4-bit keys in
    the reference's pack; 3- and 2-bit keys as four 32-channel chunks of
    little-endian pair fields (field i of chunk c = code(32c + 2i) |
    code(32c + 2i + 1) << bits at bit 2 * bits * i)."""
    codes = np.asarray(codes, np.uint8)
    n, D = codes.shape
    if bits == 4:
        return pack_key_codes(codes, 4).reshape(n, D // 2)
    # inside a chunk, channel k's code starts at bit bits * k (fields are
    # consecutive pairs), its bits least significant first
    bitv = ((codes[:, :, None] >> np.arange(bits, dtype=np.uint8)) & 1).astype(np.uint8)
    return np.packbits(bitv.reshape(n, D // 32, 32 * bits), axis=-1, bitorder="little").reshape(n, D * bits // 8)


def codes_from_key_rows(rows: np.ndarray, bits: int, D: int = 128) -> np.ndarray:
    """The inverse of :func:`key_rows_from_codes`: stored rows -> codes ``(n, D)``."""
    rows = np.asarray(rows, np.uint8)
    n = rows.shape[0]
    if bits == 4:
        return unpack_keys(rows.reshape(-1), n * D).reshape(n, D)
    bitv = np.unpackbits(rows.reshape(n, D // 32, 4 * bits), axis=-1, bitorder="little")
    bitv = bitv.reshape(n, D, bits).astype(np.uint8)
    return (bitv << np.arange(bits, dtype=np.uint8)).sum(axis=-1, dtype=np.uint32).astype(np.uint8)


def restore_outlier_codes(kp: np.ndarray, idx: np.ndarray, val: np.ndarray,
                          scale: np.ndarray, mean: np.ndarray, grid: str = "nf4_asym") -> np.ndarray:
    """Put the reference's key codes back at outlier positions.

    ``kp`` (H, G, D/2) packed codes as stored; ``idx`` flat positions into
    (H, G, D) and ``val`` their fp16 values; ``scale``/``mean`` (H, D) (for
    uniform keys ``grid="uniform"``: scale and zero)."""
    kp = np.array(kp, dtype=np.uint8, copy=True)
    H, G, half = kp.shape
    D = 2 * half
    if idx.size == 0:
        return kp
    idx = idx.astype(np.int64)
    h, t, j = idx // (G * D), (idx // D) % G, idx % D
    code = (uniform_codes if grid == "uniform" else nf4_codes)(val.astype(np.float32), scale[h, j], mean[h, j])
    nib = _rev4(code)
    # even channels in the high nibble, odd in the low one; one parity at a
    # time so two outliers sharing a byte both land
    for par in (0, 1):
        m = (j % 2) == par
        hh, tt, bb, nn = h[m], t[m], j[m] // 2, nib[m]
        byte = kp[hh, tt, bb]
        kp[hh, tt, bb] = ((byte & 0x0F) | (nn << 4)) if par == 0 else ((byte & 0xF0) | nn)
    return kp


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


def tile_value_rows(codes: np.ndarray, vb: int) -> np.ndarray:
    """Codes ``(n, D)`` (n % 16 == 0) -> the tiled value bytes ``(n, D*vb/8)``,
    the inverse of :func:`untile_value_rows`: unit (lg, c) of a 16-token tile
    holds tokens 4lg..4lg+3 x channels 8c..8c+7, code bit k of (token u,
    channel nt) at unit bit ``unit_bit(u, nt, vb) + k``."""
    codes = np.asarray(codes, np.uint8)
    n, D = codes.shape
    if n % 16 or D % 8:
        raise ValueError("tiling needs whole 16-token tiles and D % 8 == 0")
    vrow = D * vb // 8
    unit_bits = vrow // 4 * 8
    # (tile, lg, u, c, nt) view of the codes
    t = codes.reshape(n // 16, 4, 4, D // 8, 8)
    bits = np.zeros((n // 16, 4, D // 8, unit_bits), np.uint8)       # (tile, lg, c, bit)
    for u in range(4):
        for nt in range(8):
            b0 = unit_bit(u, nt, vb)
            for k in range(vb):
                bits[:, :, :, b0 + k] = (t[:, :, u, :, nt] >> k) & 1
    packed = np.packbits(bits, axis=-1, bitorder="little")           # (tile, lg, c, unit bytes)
    return packed.reshape(n // 16, 16 * vrow).reshape(n, vrow)


def untile_value_rows(rows: np.ndarray, vb: int, D: int = 128) -> np.ndarray:
    """Tiled value bytes of ``n`` tokens (n % 16 == 0, tile-aligned) -> codes (n, D)."""
    vrow = D * vb // 8
    rows = np.asarray(rows, np.uint8).reshape(-1, 16 * vrow)
    return np.concatenate([untile_values(t, vb, D) for t in rows], axis=0)


def unpack_keys(packed: np.ndarray, n_values: int) -> np.ndarray:
    """Reference 4-bit key bytes -> flat codes (turboquant_pro/per_channel_kv.py:94-100):
    byte n holds code 2n bit-reversed in its high nibble and code 2n + 1
    bit-reversed in its low nibble."""
    kp = np.asarray(packed, np.uint8).reshape(-1)
    codes = np.empty(2 * kp.size, np.uint8)
    codes[0::2] = _rev4(kp >> 4)
    codes[1::2] = _rev4(kp & 0x0F)
    return codes[:n_values]


def mark_outlier_codes(kp: np.ndarray, idx: np.ndarray, grid: str = "nf4_asym") -> np.ndarray:
    """The stored form of reference key bytes: at every outlier position the
    code whose level is the group's mean term -- NF4's zero level (code 7), or
    code 0 of uniform keys.  ``kp`` (H, G, D/2) packed codes, ``idx`` flat
    positions into (H, G, D); the inverse of :func:`restore_outlier_codes`
    up to the codes it recomputes."""
    kp = np.array(kp, dtype=np.uint8, copy=True)
    H, G, half = kp.shape
    D = 2 * half
    if idx.size == 0:
        return kp
    idx = idx.astype(np.int64)
    h, t, j = idx // (G * D), (idx // D) % G, idx % D
    nib = int(_rev4(np.array([0 if grid == "uniform" else NF4_ZERO_CODE]))[0])
    for par in (0, 1):
        m = (j % 2) == par
        hh, tt, bb = h[m], t[m], j[m] // 2
        byte = kp[hh, tt, bb]
        kp[hh, tt, bb] = ((byte & 0x0F) | (nib << 4)) if par == 0 else ((byte & 0xF0) | nib)
    return kp


def unpack_values(packed: np.ndarray, n_values: int, bits: int) -> np.ndarray:
    """Reference value bytes -> flat codes (turboquant_pro/core.py:400-441), the
    inverse of :func:`pack_values`."""
    b = np.asarray(packed, np.uint8).reshape(-1)
    per = {2: 4, 3: 8, 4: 2}[bits]
    if bits == 3:
        b = np.concatenate([b, np.zeros((-b.size) % 3, np.uint8)]).reshape(-1, 3).astype(np.uint32)
        word = b[:, 0] | (b[:, 1] << np.uint32(8)) | (b[:, 2] << np.uint32(16))
    else:
        word = b.astype(np.uint32)
    mask = np.uint32((1 << bits) - 1)
    codes = np.stack([(word >> np.uint32(bits * k)) & mask for k in range(per)], 1)
    return codes.reshape(-1)[:n_values].astype(np.uint8)
