"""CPU oracle for TurboQuant Pro's decode-on-codes KV attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or shipped.
The product path (``turboquant-pro_amd/``) never imports it.

This is a from-scratch NumPy restatement of the reference algorithm.  Every
function cites the reference ``file:line`` it restates (paths relative to the
reference repository root).  Where bit-exactness depends on NumPy's reduction
order the restatement uses the very same NumPy primitive on the same array
shape, so the oracle reproduces the reference bit for bit on the same NumPy
build; ``oracle/tqk_oracle.c`` spells the same operation order out in scalar C
(sequential channel mean, 8-lane pairwise norm, sequential non-fused rotation)
and the tests check the two agree bit for bit.

Pinning (what fixes each function independently of this file):
  * codebooks / NF4 table / pack layouts: reference literals and the 3-bit
    known-answer test (tests/test_core.py:228-256), the 4-bit LUT
    (turboquant_pro/volta_kernels.py:270-280);
  * encode / decompress / cache cadence: golden vectors written by
    ``tests/golden/make_golden.py`` from the reference itself;
  * attention: closed-form checks (uniform keys -> mean of values, one-hot
    softmax) and the merge-partials associativity invariant.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

# --------------------------------------------------------------------------- #
# Tables                                                                        #
# --------------------------------------------------------------------------- #

# NormalFloat-4 levels, turboquant_pro/per_channel_kv.py:64-84 (QLoRA NF4).
NF4 = np.array(
    [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
     -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
     0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
     0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
     0.7229568362236023, 1.0],
    dtype=np.float32,
)

# Lloyd-Max N(0,1) levels, turboquant_pro/core.py:70-93 (float64 literals).
_LLOYD_MAX = {
    2: [-1.510, -0.453, 0.453, 1.510],
    3: [-1.748, -1.050, -0.500, -0.069, 0.069, 0.500, 1.050, 1.748],
    4: [-2.401, -1.844, -1.437, -1.099, -0.800, -0.524, -0.262, -0.066,
        0.066, 0.262, 0.524, 0.800, 1.099, 1.437, 1.844, 2.401],
}


def polar_codebook(bits: int, head_dim: int) -> tuple[np.ndarray, np.ndarray]:
    """(centroids, boundaries) fp32 for the PolarQuant value codec.

    turboquant_pro/core.py:229-240: ``c = fp32(raw_f64 * (1/sqrt(d)))`` and
    ``bnd = (c[:-1] + c[1:]) / 2`` evaluated in fp32.
    """
    raw = np.asarray(_LLOYD_MAX[bits], dtype=np.float64)
    c = (raw * (1.0 / math.sqrt(head_dim))).astype(np.float32)
    bnd = (c[:-1] + c[1:]) / np.float32(2.0)
    return c, bnd.astype(np.float32)


def rotation(seed, head_dim: int) -> tuple[np.ndarray, np.ndarray]:
    """(Pi, Pi_T) for the full-QR random rotation, turboquant_pro/core.py:252-263.

    ``Q = qr(default_rng(seed).standard_normal((d, d)).astype(fp32))``; rotate is
    ``x @ Pi_T`` and unrotate ``y @ Pi``.  LAPACK-dependent, so the tests pin
    seed 0 against a committed fixture.
    """
    g = np.random.default_rng(seed).standard_normal((head_dim, head_dim))
    q, _ = np.linalg.qr(g.astype(np.float32))
    return q, q.T.copy()


# --------------------------------------------------------------------------- #
# Bit-pack layouts                                                              #
# --------------------------------------------------------------------------- #


def pack_key_codes(codes: np.ndarray, bits: int = 4) -> np.ndarray:
    """Key-code bitstream, turboquant_pro/per_channel_kv.py:87-93.

    Bit ``t`` of flat value ``i`` lands at stream bit ``p = bits*i + t``, stored
    in byte ``p >> 3`` at bit ``7 - (p & 7)`` (MSB-first bytes, LSB-first values).
    """
    v = np.ascontiguousarray(codes).reshape(-1).astype(np.uint8)
    n_bits = v.size * bits
    stream = np.zeros(((n_bits + 7) // 8) * 8, dtype=np.uint8)
    pos = np.arange(v.size, dtype=np.int64) * bits
    for t in range(bits):
        stream[pos + t] = (v >> t) & 1
    weights = (1 << np.arange(7, -1, -1)).astype(np.uint8)
    return (stream.reshape(-1, 8) * weights).sum(axis=1).astype(np.uint8)


def unpack_key_codes(packed: np.ndarray, n_values: int, bits: int = 4) -> np.ndarray:
    """Inverse of :func:`pack_key_codes` (turboquant_pro/per_channel_kv.py:96-100)."""
    b = np.asarray(packed, dtype=np.uint8).reshape(-1)
    stream = ((b[:, None] >> np.arange(7, -1, -1)) & 1).reshape(-1)
    stream = stream[: n_values * bits].reshape(n_values, bits).astype(np.uint16)
    return (stream << np.arange(bits, dtype=np.uint16)).sum(axis=1).astype(np.uint8)


def pack_value_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """PolarQuant value pack, turboquant_pro/core.py:350-398.

    3-bit: 8 flat codes -> 24-bit little-endian word -> 3 bytes.  4-bit:
    ``v0 | v1 << 4``.  2-bit: ``v0 | v1<<2 | v2<<4 | v3<<6``.  Zero-padded tail.
    """
    v = np.ascontiguousarray(codes).reshape(-1).astype(np.uint32)
    per = {2: 4, 3: 8, 4: 2}[bits]
    pad = (-v.size) % per
    if pad:
        v = np.concatenate([v, np.zeros(pad, dtype=np.uint32)])
    v = v.reshape(-1, per)
    word = np.zeros(v.shape[0], dtype=np.uint32)
    for k in range(per):
        word |= v[:, k] << np.uint32(bits * k)
    if bits == 3:
        return np.stack([(word >> s) & 0xFF for s in (0, 8, 16)], axis=1).astype(np.uint8).reshape(-1)
    return word.astype(np.uint8)


def unpack_value_codes(packed: np.ndarray, n_values: int, bits: int) -> np.ndarray:
    """Inverse of :func:`pack_value_codes` (turboquant_pro/core.py:400-441)."""
    b = np.asarray(packed, dtype=np.uint8).reshape(-1).astype(np.uint32)
    if bits == 3:
        b = b.reshape(-1, 3)
        word = b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16)
        per = 8
    else:
        word = b
        per = 8 // bits
    mask = (1 << bits) - 1
    out = np.stack([(word >> (bits * k)) & mask for k in range(per)], axis=1)
    return out.reshape(-1)[:n_values].astype(np.uint8)


# --------------------------------------------------------------------------- #
# Encode (quantize-on-flush)                                                    #
# --------------------------------------------------------------------------- #


@dataclass
class KeyGroup:
    """One flushed key group of one sequence: the reference's
    ``CompressedPerChannelKV`` fields (turboquant_pro/per_channel_kv.py:103-143)
    for the asym-NF4 calibrated mode, shape ``(1, H, S, D)``."""

    codes: np.ndarray            # (H, S, D) uint8 (unpacked view)
    packed: np.ndarray           # flat uint8, the storage of record
    nf4_scale: np.ndarray        # (H, D) fp32 abs-max of the centred channel
    nf4_mean: np.ndarray         # (H, D) fp32 channel mean
    outlier_idx: np.ndarray | None   # int32 flat indices into (1, H, S, D)
    outlier_val: np.ndarray | None   # fp16 values at those indices
    shape: tuple = ()
    # "nf4_asym", or "uniform": then nf4_scale / nf4_mean hold the reference's
    # per-channel scale / zero (its (1, H, 1, D) arrays without the unit axes)
    grid: str = "nf4_asym"
    bits: int = 4                # code width (2 or 3 only with the uniform grid)


@dataclass
class ValueGroup:
    """One flushed value group: ``CompressedKV`` fields (turboquant_pro/core.py:96-136)."""

    codes: np.ndarray            # (H, S, D) uint8
    packed: np.ndarray           # flat uint8
    norms: np.ndarray            # (H, S) fp32
    bits: int = 3


def outlier_count_per_channel(n_tokens: int, outlier_frac: float) -> int:
    """``k = max(1, int(round(S * f)))``, turboquant_pro/per_channel_kv.py:274
    (Python's round-half-even on the float product)."""
    return max(1, int(round(n_tokens * outlier_frac)))


def key_outliers(x4: np.ndarray, outlier_frac: float):
    """Dense-sparse outliers of a (1, H, S, D) block, turboquant_pro/per_channel_kv.py:269-283:
    the k largest |x| per (head, channel) and every tie, as flat int32
    indices in C order and their fp16 values; (None, None) when f == 0."""
    if outlier_frac <= 0.0:
        return None, None
    S = x4.shape[2]
    k = outlier_count_per_channel(S, outlier_frac)
    mag = np.abs(x4)
    if k >= S:
        sel = np.ones(x4.shape, dtype=bool)
    else:
        # k-th largest magnitude per (head, channel); >= keeps every tie.
        thr = np.partition(mag, S - k, axis=2)[:, :, S - k:S - k + 1, :]
        sel = mag >= thr
    oidx = np.flatnonzero(sel).astype(np.int32)
    return oidx, x4.reshape(-1)[oidx].astype(np.float16)


def encode_keys_uniform(x: np.ndarray, outlier_frac: float, bits: int = 4) -> KeyGroup:
    """Uniform asymmetric per-channel key encode of one group ``x`` (H, S, D)
    fp32, turboquant_pro/per_channel_kv.py:303-317 with ``qmax = 2**bits - 1``
    (:179): per channel ``mn``/``mx`` over the tokens,
    ``scale = max(mx - mn, 1e-8) / qmax``,
    ``code = clip(round_half_even((x - mn) / scale), 0, qmax)``; outliers as for
    NF4 (the codes at their positions are kept)."""
    x4 = np.asarray(x, dtype=np.float32)[None]
    _, H, S, D = x4.shape
    qmax = (1 << bits) - 1
    oidx, oval = key_outliers(x4, outlier_frac)
    mn = x4.min(axis=2, keepdims=True)
    mx = x4.max(axis=2, keepdims=True)
    scale = np.maximum(mx - mn, 1e-8) / qmax
    codes = np.clip(np.round((x4 - mn) / scale), 0, qmax).astype(np.uint8)
    return KeyGroup(codes=codes[0], packed=pack_key_codes(codes, bits),
                    nf4_scale=scale[0, :, 0, :].astype(np.float32), nf4_mean=mn[0, :, 0, :].astype(np.float32),
                    outlier_idx=oidx, outlier_val=oval, shape=(1, H, S, D), grid="uniform", bits=bits)


def dc_channel_mask(rope_theta: float, head_dim: int, window: int) -> np.ndarray:
    """Channels whose rotary wavelength exceeds ``window`` tokens,
    turboquant_pro/per_channel_kv.py:234-243 (float64)."""
    half = head_dim // 2
    inv = rope_theta ** (-2.0 * np.arange(half) / head_dim)
    return np.tile(2.0 * np.pi / inv, 2)[:head_dim] > float(window)


def rope_averaged_bias(k_bias: np.ndarray, rope_theta: float, head_dim: int, start: int,
                       n: int) -> np.ndarray:
    """Position-averaged rotation of the k_proj bias over ``[start, start + n)``,
    turboquant_pro/per_channel_kv.py:245-267: float64 mean cos/sin per
    frequency, rounded to fp32, then ``b * c + rotate_half(b) * s`` in fp32."""
    half = head_dim // 2
    inv = rope_theta ** (-2.0 * np.arange(half, dtype=np.float64) / head_dim)
    ang = np.arange(start, start + n, dtype=np.float64)[:, None] * inv[None, :]
    c = np.tile(np.cos(ang).mean(axis=0), 2).astype(np.float32)
    sn = np.tile(np.sin(ang).mean(axis=0), 2).astype(np.float32)
    b = np.asarray(k_bias, dtype=np.float32).reshape(-1, head_dim)
    return b * c[None, :] + np.concatenate([-b[:, half:], b[:, :half]], axis=1) * sn[None, :]


def encode_keys(x: np.ndarray, outlier_frac: float, zero_point: str = "calibrated",
                rope_theta: float | None = None, k_bias=None, position_start: int = 0) -> KeyGroup:
    """Asym-NF4 per-channel key encode of one group ``x`` (H, S, D) fp32.

    Restates turboquant_pro/per_channel_kv.py:269-283 (outliers) and
    :285-401 (nf4_asym) with the zero point of :327-345: the channel mean
    ("calibrated"), the mean on the DC channels only ("sparse"), the
    RoPE-averaged k_proj bias of positions ``[position_start, +S)`` ("bias"),
    or none ("symmetric": symmetric NF4, :354-357).
    ``nf4_mean`` holds the zero point of every channel (the reference stores
    only the DC channels for "sparse" and nothing for "bias").  The reference
    works on a ``(1, H, S, D)`` array; the same shape is used here so NumPy's
    reduction order (and therefore every rounding) is the same.
    """
    x4 = np.asarray(x, dtype=np.float32)[None]
    _, H, S, D = x4.shape
    oidx, oval = key_outliers(x4, outlier_frac)
    if zero_point == "bias":
        mean = np.broadcast_to(rope_averaged_bias(k_bias, rope_theta, D, position_start, S)[None],
                               (1, H, D))
    elif zero_point == "symmetric":
        # PerChannelKV(nf4=True) without nf4_asym (per_channel_kv.py:354-357):
        # the raw channel's abs-max scales the grid, no mean (zero here, and
        # 0 + fl(amax * NF4[l]) is fl(amax * NF4[l]) exactly)
        mean = np.zeros((1, H, D), np.float32)
    elif zero_point == "sparse":
        mean = x4.mean(axis=2) * dc_channel_mask(rope_theta, D, S)[None, None, :]
    else:
        mean = x4.mean(axis=2)                               # (1, H, D)
    centred = x4 - mean[:, :, None, :]
    amax = np.maximum(np.abs(centred).max(axis=2), 1e-8)     # (1, H, D)
    grid = (mean[..., None] + amax[..., None] * NF4[None, None, None, :]).astype(np.float32)
    dist = np.abs(np.moveaxis(x4, 2, -1)[..., None, :] - grid[..., :, None])  # (1,H,D,16,S)
    codes = np.moveaxis(dist.argmin(axis=-2).astype(np.uint8), -1, 2)        # (1,H,S,D)
    return KeyGroup(
        codes=codes[0], packed=pack_key_codes(codes, 4),
        nf4_scale=amax[0].astype(np.float32), nf4_mean=mean[0].astype(np.float32),
        outlier_idx=oidx, outlier_val=oval, shape=(1, H, S, D))


def encode_values(v: np.ndarray, pi_t: np.ndarray, bnd: np.ndarray, bits: int) -> ValueGroup:
    """PolarQuant value encode of one group ``v`` (H, S, D), CPU full-QR branch.

    Restates turboquant_pro/core.py:542-617 (``kind="value"``, ``packed=True``):
    L2 norm, divide by ``max(norm, 1e-30)``, rotate by ``Pi_T`` (einsum),
    ``searchsorted(boundaries, y)`` (left: code = #{b < y}), pack.
    """
    x = np.asarray(v, dtype=np.float32)[None]
    norms = np.linalg.norm(x, axis=-1)
    unit = x / np.maximum(norms, 1e-30)[..., None]
    rot = np.einsum("...d,de->...e", unit, pi_t)
    codes = np.searchsorted(bnd, rot).astype(np.uint8)
    return ValueGroup(codes=codes[0], packed=pack_value_codes(codes, bits),
                      norms=norms[0].astype(np.float32), bits=bits)


# --------------------------------------------------------------------------- #
# Decode (dequantize-then-attend: the parity target)                            #
# --------------------------------------------------------------------------- #


def decode_keys(g: KeyGroup) -> np.ndarray:
    """Reconstruct (H, S, D) fp32 keys, turboquant_pro/per_channel_kv.py:497-539
    (nf4 branch with calibrated mean, then the fp16 outlier overwrite)."""
    _, H, S, D = g.shape
    codes = unpack_key_codes(g.packed, H * S * D, g.bits).reshape(1, H, S, D)
    if g.grid == "uniform":
        # per_channel_kv.py:529-530: idx * scale + zero, two fp32 roundings
        out = codes.astype(np.float32) * g.nf4_scale[None, :, None, :] + g.nf4_mean[None, :, None, :]
        out = out.astype(np.float32)
    else:
        grid = g.nf4_scale[None, ..., None] * NF4[None, None, None, :]
        grid = grid + g.nf4_mean[None, ..., None]
        out = np.take_along_axis(grid.astype(np.float32), np.moveaxis(codes, 2, -1), axis=-1)
        out = np.moveaxis(out, -1, 2).astype(np.float32)
    if g.outlier_idx is not None:
        flat = out.reshape(-1)
        flat[g.outlier_idx] = g.outlier_val.astype(np.float32)
        out = flat.reshape(1, H, S, D)
    return out[0]


def decode_values(g: ValueGroup, cent: np.ndarray, pi: np.ndarray) -> np.ndarray:
    """Reconstruct (H, S, D) fp32 values, turboquant_pro/core.py:619-654:
    ``(cent[code] @ Pi) * norm``."""
    H, S = g.norms.shape
    D = pi.shape[0]
    codes = unpack_value_codes(g.packed, H * S * D, g.bits).reshape(1, H, S, D)
    y = cent[codes]
    x = np.einsum("...d,de->...e", y, pi)
    return (x * g.norms[None, ..., None])[0]


def softmax_rows(s: np.ndarray) -> np.ndarray:
    """turboquant_pro/kv_fused.py:46-49: subtract the row max, exp, normalise."""
    s = s - np.amax(s, axis=-1, keepdims=True)
    e = np.exp(s)
    return e / np.sum(e, axis=-1, keepdims=True)


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """fp32 softmax attention with the GQA head map (q-head i -> kv-head i // g).

    The MHA case is the reference's oracle formula,
    tests/test_kv_fused_pck.py:202-208: ``softmax(q k^T / sqrt(d)) v``.
    ``q`` (Hq, D); ``k``, ``v`` (Hkv, L, D).  Returns (Hq, D) fp32.
    """
    q = np.asarray(q, dtype=np.float32)
    Hq, D = q.shape
    Hkv = k.shape[0]
    grp = Hq // Hkv
    kk = np.repeat(np.asarray(k, np.float32), grp, axis=0)
    vv = np.repeat(np.asarray(v, np.float32), grp, axis=0)
    sc = np.einsum("hd,hsd->hs", q, kk) / np.sqrt(D)
    p = softmax_rows(sc)
    return np.einsum("hs,hsd->hd", p, vv)


def merge_partials(parts):
    """Online-softmax merge of ``(m, l, acc)`` states, turboquant_pro/kv_fused.py:139-153."""
    big = parts[0][0]
    for m, _, _ in parts[1:]:
        big = np.maximum(big, m)
    num = np.zeros_like(parts[0][2])
    den = np.zeros_like(parts[0][1])
    for m, l, acc in parts:
        w = np.exp(m - big)
        num = num + acc * w[:, None]
        den = den + l * w
    return num / den[:, None]


# --------------------------------------------------------------------------- #
# Two-tier cache cadence                                                        #
# --------------------------------------------------------------------------- #


def group_tokens(hot_window: int) -> int:
    """Tokens per flush: ``len(hot) // 2`` at ``len(hot) == hot_window + 1``
    (turboquant_pro/core.py:1006-1016)."""
    return (hot_window + 1) // 2


def n_groups(length: int, hot_window: int) -> int:
    """Number of flushed groups after ``length`` one-token appends
    (turboquant_pro/core.py:986-1038): the first flush fires when the hot list
    reaches ``hot_window + 1``, then every ``group_tokens`` appends."""
    G = group_tokens(hot_window)
    if G == 0 or length <= hot_window:
        return 0
    return (length - (hot_window + 1)) // G + 1


@dataclass
class SequenceCache:
    """State of one ``TurboQuantKVCache`` after appending ``L`` tokens.

    Bulk restatement of the append/flush loop: group ``i`` holds tokens
    ``[G*i, G*(i+1))`` (each flush takes the oldest hot tokens, and the
    flushed block's ``position_start`` is the running cold length); the hot
    window is the rest, kept as appended (fp16 in, upcast on read,
    turboquant_pro/core.py:1107-1113).
    """

    hot_window: int
    value_bits: int
    outlier_frac: float
    seed: int | None = 0
    # or "uniform" (per_channel_kv.py:303-317), or "polar": PolarQuant keys
    # (per_channel_keys=False, turboquant_pro/core.py:1028-1029 -- the value
    # encode with kind="key", whose codebook is key_bits' = value_bits' here)
    key_grid: str = "nf4_asym"
    key_bits: int = 4                # uniform keys: 2, 3 or 4
    zero_point: str = "calibrated"   # asym-NF4: or "sparse" / "bias" (per_channel_kv.py:327-345)
    rope_theta: float | None = None
    k_bias: np.ndarray | None = None
    keys: list = field(default_factory=list)
    values: list = field(default_factory=list)
    hot_k: np.ndarray | None = None
    hot_v: np.ndarray | None = None

    def build(self, k: np.ndarray, v: np.ndarray, pi: np.ndarray, pi_t: np.ndarray):
        """``k``, ``v``: (H, L, D) as appended (fp16).  Encodes every group."""
        H, L, D = k.shape
        G = group_tokens(self.hot_window)
        ng = n_groups(L, self.hot_window)
        cent, bnd = polar_codebook(self.value_bits, D)
        self.keys, self.values = [], []
        for i in range(ng):
            sl = slice(G * i, G * (i + 1))
            if self.key_grid == "polar":
                if self.key_bits != self.value_bits:
                    raise ValueError("polar keys here take key_bits == value_bits")
                self.keys.append(encode_values(k[:, sl].astype(np.float32), pi_t, bnd, self.value_bits))
            elif self.key_grid == "uniform":
                self.keys.append(encode_keys_uniform(k[:, sl].astype(np.float32), self.outlier_frac,
                                                     self.key_bits))
            else:
                # the flushed block's position_start is the cold length before it
                self.keys.append(encode_keys(k[:, sl].astype(np.float32), self.outlier_frac,
                                             self.zero_point, self.rope_theta, self.k_bias, G * i))
            self.values.append(encode_values(v[:, sl].astype(np.float32), pi_t, bnd, self.value_bits))
        self.hot_k = k[:, G * ng:]
        self.hot_v = v[:, G * ng:]
        self._cent, self._pi = cent, pi
        return self

    def get_keys(self) -> np.ndarray:
        """(H, L, D) fp32, ``get_keys(0, L)[0]`` (turboquant_pro/core.py:1040-1117)."""
        parts = [decode_values(g, self._cent, self._pi) if isinstance(g, ValueGroup) else decode_keys(g)
                 for g in self.keys] + [self.hot_k.astype(np.float32)]
        return np.concatenate(parts, axis=1)

    def get_values(self) -> np.ndarray:
        parts = [decode_values(g, self._cent, self._pi) for g in self.values]
        parts.append(self.hot_v.astype(np.float32))
        return np.concatenate(parts, axis=1)

    def attend(self, q: np.ndarray) -> np.ndarray:
        return attend(q, self.get_keys(), self.get_values())


# --------------------------------------------------------------------------- #
# Synthetic inputs (the measurement spec)                                       #
# --------------------------------------------------------------------------- #


def rope_rotate_half(x: np.ndarray, theta: float = 10000.0, start: int = 0) -> np.ndarray:
    """RoPE with the ``rotate_half`` convention (turboquant_pro/per_channel_kv.py:258-267,
    turboquant_pro/rope.py): ``x*cos + rotate_half(x)*sin`` over the token axis -2."""
    D = x.shape[-1]
    half = D // 2
    inv = theta ** (-2.0 * np.arange(half, dtype=np.float64) / D)
    pos = np.arange(start, start + x.shape[-2], dtype=np.float64)
    ang = pos[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], axis=1).astype(np.float32)
    sin = np.concatenate([np.sin(ang), np.sin(ang)], axis=1).astype(np.float32)
    rh = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return (x * cos + rh * sin).astype(np.float32)


def synthetic_kv(seed: int, B: int, Hkv: int, Hq: int, L: int, D: int = 128,
                 outlier_channel_frac: float = 0.02, theta: float = 10000.0):
    """Seeded synthetic keys/values/queries, all fp16.

    Keys: N(0,1) x per-(seq, head, channel) lognormal(0,1); ``round(0.02*D)``
    channels per head x10; RoPE at positions 0..L-1.  Values, queries: N(0,1).
    Returns ``k (B,Hkv,L,D)``, ``v (B,Hkv,L,D)``, ``q (B,Hq,D)`` as float16.
    """
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, Hkv, L, D), dtype=np.float32)
    scale = rng.lognormal(0.0, 1.0, size=(B, Hkv, 1, D)).astype(np.float32)
    n_hot = int(round(outlier_channel_frac * D))
    for b in range(B):
        for h in range(Hkv):
            ch = rng.choice(D, size=n_hot, replace=False)
            scale[b, h, 0, ch] *= 10.0
    k = rope_rotate_half(k * scale, theta)
    v = rng.standard_normal((B, Hkv, L, D), dtype=np.float32)
    q = rng.standard_normal((B, Hq, D), dtype=np.float32)
    return k.astype(np.float16), v.astype(np.float16), q.astype(np.float16)


# --------------------------------------------------------------------------- #
# Byte accounting (the roofline numerator)                                      #
# --------------------------------------------------------------------------- #


def decode_step_bytes(seq_lens, Hkv: int, Hq: int, D: int = 128, kbits: int = 4,
                      vbits: int = 3, hot_window: int = 512, n_out: int | None = None,
                      out_bytes: int = 2) -> int:
    """Canonical compressed bytes one decode step must read, per the storage of
    record: per (sequence, kv head) ``n_cold*(D*kb/8 + D*vb/8 + 4)`` +
    ``n_grp*(2*D*4 + n_out*6)`` + ``n_hot*2*D*2`` + q and output per q-head."""
    G = group_tokens(hot_window)
    if n_out is None:
        n_out = outlier_count_per_channel(G, 0.02) * D
    total = 0
    g = Hq // Hkv
    for L in seq_lens:
        ng = n_groups(int(L), hot_window)
        n_cold = G * ng
        n_hot = int(L) - n_cold
        per_head = (n_cold * (D * kbits // 8 + D * vbits // 8 + 4) + ng * (2 * D * 4 + n_out * 6)
                    + n_hot * 2 * D * 2 + g * D * (2 + out_bytes))
        total += per_head * Hkv
    return total
