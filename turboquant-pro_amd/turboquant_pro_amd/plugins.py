"""Quantizer plugin registry and the two in-tree KV formats, on the gfx950
library (turboquant_pro/plugins.py:60-360).

The registry keeps the reference's surface: targets as plain strings,
:class:`PluginSpec`, :func:`register` / :func:`get_plugin` / :func:`create` /
:func:`available_plugins`, out-of-tree discovery through the
``turboquant_pro.plugins`` entry-point group, and the optional-capability
probes :func:`affine_params` / :func:`affine_codes` / :func:`outlier_csr` /
:func:`native_dtype`.

In-tree formats:

* ``"per_channel"`` -- :class:`PerChannelKVQuantizer`, asym-NF4 4-bit keys with
  the fp16 outlier side-list (turboquant_pro/per_channel_kv.py:182-401).
  ``compress`` runs the GPU encode of one group per sequence (up to 256 tokens,
  the cache's group size bound) and returns the reference container, bit for
  bit for fp16-valued input (keys enter the cache as fp16); ``decompress``
  runs the GPU dequant.  The affine capability (``grid_params`` / ``codes`` /
  ``outlier_csr``) reads the container on the host, as the reference's
  (turboquant_pro/kv_fused_pck.py:47-127).
* ``"polar"`` -- :class:`PolarQuantizer`, PolarQuant values
  (turboquant_pro/core.py:139-654) at 3 or 4 bits: ``compress`` /
  ``decompress`` on the GPU, any number of tokens.

Configurations the library has no gfx950 form for raise
``NotImplementedError`` at construction.
"""

from __future__ import annotations

import logging
from collections.abc import Callable
from dataclasses import dataclass, field
from importlib import metadata
from typing import Any, Protocol, runtime_checkable

import numpy as np

from .codebooks import group_tokens_for, random_rotation
from .formats import NF4, pack_values, unpack_keys, unpack_values

logger = logging.getLogger(__name__)

__all__ = [
    "TARGET_KV_KEY", "TARGET_KV_VALUE", "TARGET_WEIGHT", "TARGET_EMBEDDING",
    "Quantizer", "PluginSpec", "register", "get_plugin", "create", "available_plugins",
    "load_entry_point_plugins", "affine_params", "affine_codes", "outlier_csr", "native_dtype",
    "CompressedPerChannelKV", "CompressedKV", "PerChannelKVQuantizer", "PolarQuantizer",
]

TARGET_KV_KEY = "kv_key"
TARGET_KV_VALUE = "kv_value"
TARGET_WEIGHT = "weight"
TARGET_EMBEDDING = "embedding"
_TARGETS = frozenset({TARGET_KV_KEY, TARGET_KV_VALUE, TARGET_WEIGHT, TARGET_EMBEDDING})
_TIERS = frozenset({"stable", "beta", "experimental"})
ENTRY_POINT_GROUP = "turboquant_pro.plugins"

# one encode group holds at most this many tokens (the library's group bound)
_MAX_GROUP_TOKENS = 256


@runtime_checkable
class Quantizer(Protocol):
    """What every plugin instance provides: ``compress`` to an opaque
    container and ``decompress`` back to a float array of the input shape."""

    def compress(self, x: np.ndarray, **kwargs: Any) -> Any: ...

    def decompress(self, c: Any) -> np.ndarray: ...


@dataclass(frozen=True)
class PluginSpec:
    """A named quantizer factory (``factory(**config)`` -> :class:`Quantizer`)."""

    name: str
    factory: Callable[..., Any]
    targets: frozenset[str]
    tier: str = "experimental"
    description: str = ""

    def __post_init__(self) -> None:
        if not self.name or "/" in self.name:
            raise ValueError(f"invalid plugin name: {self.name!r}")
        unknown = sorted(set(self.targets) - _TARGETS)
        if unknown:
            raise ValueError(f"unknown targets {unknown}; valid: {sorted(_TARGETS)}")
        if self.tier not in _TIERS:
            raise ValueError(f"tier must be one of {sorted(_TIERS)}")


_registry: dict[str, PluginSpec] = {}
_entry_points_done = False


def register(spec: PluginSpec, *, overwrite: bool = False) -> PluginSpec:
    """Add ``spec``; a taken name raises unless ``overwrite``."""
    if spec.name in _registry and not overwrite:
        raise ValueError(f"plugin {spec.name!r} already registered (pass overwrite=True to replace)")
    _registry[spec.name] = spec
    return spec


def get_plugin(name: str) -> PluginSpec:
    """The spec registered as ``name`` (entry points are loaded on a miss)."""
    if name not in _registry:
        load_entry_point_plugins()
    if name not in _registry:
        names = ", ".join(sorted(_registry)) or "<none>"
        raise KeyError(f"no quantizer plugin {name!r}; available: {names}")
    return _registry[name]


def create(name: str, **config: Any) -> Any:
    """An instance of plugin ``name``, e.g. ``create("per_channel", nf4_asym=True)``."""
    q = get_plugin(name).factory(**config)
    if not isinstance(q, Quantizer):
        raise TypeError(f"plugin {name!r} factory returned {type(q).__name__}, "
                        "which does not provide compress/decompress")
    return q


def available_plugins(*, target: str | None = None) -> dict[str, PluginSpec]:
    """Registered plugins by name (entry points included), optionally of one target."""
    load_entry_point_plugins()
    out = {n: _registry[n] for n in sorted(_registry)}
    if target is not None:
        out = {n: s for n, s in out.items() if target in s.targets}
    return out


def load_entry_point_plugins(*, force: bool = False) -> list[str]:
    """Register the specs published under the ``turboquant_pro.plugins``
    entry-point group (a spec, an iterable of specs, or a zero-argument
    callable returning either).  A broken entry point is logged and skipped.
    Returns the names added."""
    global _entry_points_done
    if _entry_points_done and not force:
        return []
    _entry_points_done = True
    added: list[str] = []
    try:
        eps = metadata.entry_points(group=ENTRY_POINT_GROUP)
    except Exception:  # importlib.metadata variations
        logger.exception("entry-point discovery failed")
        return added
    for ep in eps:
        try:
            obj = ep.load()
            if callable(obj) and not isinstance(obj, PluginSpec):
                obj = obj()
            for spec in ([obj] if isinstance(obj, PluginSpec) else list(obj)):
                if spec.name in _registry:
                    continue
                register(spec)
                added.append(spec.name)
        except Exception:
            logger.exception("skipping broken plugin entry point %r", ep.name)
    return added


# ---------------------------------------------------------------- probes
def affine_params(q: Any, c: Any):
    """``(mu (H, D), weight (H, D), grid (L,))`` when ``q`` exposes the affine
    contract for container ``c``, else ``None`` (decompress-then-attend)."""
    fn = getattr(q, "grid_params", None)
    if fn is None:
        return None
    try:
        return fn(c)
    except NotImplementedError:
        return None


def affine_codes(q: Any, c: Any):
    """Unpacked codes ``(B, H, S, D)`` uint8 of the affine contract, or ``None``."""
    fn = getattr(q, "codes", None)
    if fn is None:
        return None
    try:
        return fn(c)
    except NotImplementedError:
        return None


def outlier_csr(q: Any, c: Any):
    """Token-major CSR ``(row_ptr, cols, deltas)`` of the sparse overlay, or ``None``."""
    fn = getattr(q, "outlier_csr", None)
    return None if fn is None else fn(c)


def native_dtype(q: Any) -> str | None:
    """Hardware dtype for passthrough execution, or ``None``."""
    fn = getattr(q, "native_dtype", None)
    return None if fn is None else fn()


# ------------------------------------------------------------ containers
@dataclass
class CompressedPerChannelKV:
    """Key container, field for field the reference's
    (turboquant_pro/per_channel_kv.py:103-138)."""

    indices: np.ndarray
    scale: np.ndarray | None
    zero: np.ndarray | None
    bits: int
    shape: tuple[int, ...]
    packed: bool = False
    levels: np.ndarray | None = None
    nf4_scale: np.ndarray | None = None
    nf4_mean: np.ndarray | None = None
    original_dtype: np.dtype = field(default_factory=lambda: np.dtype("float32"))
    outlier_idx: np.ndarray | None = None
    outlier_val: np.ndarray | None = None
    zp_mode: str = "calibrated"
    rope_theta: float | None = None
    position_start: int = 0

    def nbytes(self) -> int:
        return int(sum(a.nbytes for a in (self.indices, self.scale, self.zero, self.levels,
                                          self.nf4_scale, self.nf4_mean, self.outlier_idx,
                                          self.outlier_val) if a is not None))


@dataclass
class CompressedKV:
    """Value container, field for field the reference's (turboquant_pro/core.py:96-137)."""

    indices: np.ndarray
    norms: np.ndarray
    bits: int
    original_dtype: np.dtype = field(default_factory=lambda: np.dtype("float32"))
    packed: bool = False
    n_values: int = 0
    shape: tuple[int, ...] = ()

    def nbytes(self) -> int:
        return int(self.indices.nbytes + self.norms.nbytes)


# --------------------------------------------------------------- formats
def _pool(H: int, S: int, value_bits: int, outlier_frac: float, B: int, seed=None, device=None,
          outlier_cap: int | None = None, key_grid: str = "nf4_asym", rotation=None):
    """A B-sequence pool whose groups are exactly S tokens, one token per page
    (value codes stored per token, in the reference's pack)."""
    from .pool import TQKVPool

    W = 2 * S - 1
    assert group_tokens_for(W) == S
    return TQKVPool(n_kv_heads=H, n_q_heads=H, max_batch=B, max_seq_len=2 * S, hot_window=W,
                    value_bits=value_bits, outlier_frac=outlier_frac, page_tokens=1, seed=seed,
                    rotation=rotation, device=device, outlier_cap=outlier_cap, key_grid=key_grid)


def _fp16_tokens(x: np.ndarray):
    from .pool import _torch

    torch = _torch()
    x = np.asarray(x)
    if x.ndim != 4:
        raise ValueError(f"expected (B,H,S,D), got shape {x.shape}")
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float16))


class PerChannelKVQuantizer:
    """``"per_channel"`` keys on the gfx950 library: asym-NF4 4-bit or uniform
    4-bit (the reference's default mode), with the fp16 outlier side-list,
    one encode group per sequence.

    The constructor validates like ``PerChannelKV.__init__``
    (turboquant_pro/per_channel_kv.py:182-213) and raises
    ``NotImplementedError`` for the modes the library does not encode
    (2/3-bit uniform, symmetric NF4, data-fit quantiles, zero-point
    "sparse"/"bias", head_dim != 128)."""

    _ZP_MODES = ("calibrated", "sparse", "bias")

    def __init__(self, head_dim: int = 128, n_heads: int = 32, bits: int = 4, nuq: bool = False,
                 nf4: bool = False, nf4_asym: bool = False, outlier_frac: float = 0.0,
                 zero_point: str = "calibrated", rope_theta: float | None = None, k_bias=None,
                 device=None) -> None:
        if bits not in (2, 3, 4):
            raise ValueError(f"bits must be one of (2, 3, 4), got {bits}")
        if nf4_asym:
            nf4 = True
        if nf4 and bits != 4:
            raise ValueError("nf4=True requires bits=4")
        if not 0.0 <= outlier_frac < 1.0:
            raise ValueError("outlier_frac must be in [0, 1)")
        if zero_point not in self._ZP_MODES:
            raise ValueError(f"zero_point must be one of {self._ZP_MODES}")
        if zero_point != "calibrated":
            if not nf4_asym:
                raise ValueError(f"zero_point={zero_point!r} requires nf4_asym=True")
            if rope_theta is None:
                raise ValueError(f"zero_point={zero_point!r} requires rope_theta")
        if zero_point == "bias" and k_bias is None:
            raise ValueError('zero_point="bias" requires k_bias')
        uniform = bits == 4 and not nf4 and not nuq
        if not ((nf4_asym and zero_point == "calibrated") or uniform) or head_dim != 128:
            raise NotImplementedError("the gfx950 key encode is per-channel asym-NF4 (calibrated zero "
                                      "points) or uniform, 4-bit, at head_dim 128")
        self.head_dim, self.n_heads, self.bits = head_dim, n_heads, bits
        self.uniform = uniform
        self.key_grid = "uniform" if uniform else "nf4_asym"
        self.nuq, self.nf4, self.nf4_asym = nuq, nf4, nf4_asym
        self.outlier_frac, self.zero_point = outlier_frac, zero_point
        self.rope_theta, self.k_bias = rope_theta, None
        self.device = device

    def compress(self, x: np.ndarray, packed: bool = False, position_start: int = 0) -> CompressedPerChannelKV:
        """``(B, H, S, D)`` keys, S <= 256, as one group per sequence; the
        values are taken as fp16 (the form the cache stores)."""
        from .pool import _torch

        torch = _torch()
        xt = _fp16_tokens(x)
        B, H, S, D = xt.shape
        if D != self.head_dim:
            raise ValueError(f"head_dim {D} != {self.head_dim}")
        if not 1 <= S <= _MAX_GROUP_TOKENS:
            raise NotImplementedError(f"one gfx950 key group holds 1..{_MAX_GROUP_TOKENS} tokens, got {S}")
        pool = _pool(H, S, 3, self.outlier_frac, B, device=self.device, key_grid=self.key_grid)
        k = torch.cat([xt, torch.zeros_like(xt)], dim=2).to(pool.device)
        pool.append(k, torch.zeros_like(k))
        parts = [pool.export_group(b, 0) for b in range(B)]
        kp = np.concatenate([p["kpacked"] for p in parts])
        oidx = oval = None
        if self.outlier_frac > 0:
            oidx = np.concatenate([p["outlier_idx"].astype(np.int64) + b * H * S * D
                                   for b, p in enumerate(parts)]).astype(np.int32)
            oval = np.concatenate([p["outlier_val"] for p in parts]).astype(np.float16)
        indices = kp if packed else unpack_keys(kp, B * H * S * D).reshape(B, H, S, D)
        if self.uniform:
            # per_channel_kv.py:303-317: (B, H, 1, D) scale and zero, no NF4 fields
            return CompressedPerChannelKV(
                indices, np.stack([p["nf4_scale"] for p in parts]).astype(np.float32)[:, :, None, :],
                np.stack([p["nf4_mean"] for p in parts]).astype(np.float32)[:, :, None, :],
                self.bits, (B, H, S, D), packed, outlier_idx=oidx, outlier_val=oval)
        return CompressedPerChannelKV(
            indices, None, None, self.bits, (B, H, S, D), packed,
            nf4_scale=np.stack([p["nf4_scale"] for p in parts]).astype(np.float32),
            nf4_mean=np.stack([p["nf4_mean"] for p in parts]).astype(np.float32),
            outlier_idx=oidx, outlier_val=oval, zp_mode="calibrated", rope_theta=None,
            position_start=position_start)

    def decompress(self, c: CompressedPerChannelKV) -> np.ndarray:
        """fp32 ``(B, H, S, D)``: ``mean + scale * NF4[code]``, outliers overwritten
        by their fp16 values (turboquant_pro/per_channel_kv.py:497-539), on the GPU."""
        B, H, S, D = c.shape
        uniform = c.nf4_scale is None and c.levels is None and c.scale is not None and c.zero is not None
        if not uniform and (c.nf4_scale is None or c.nf4_mean is None or c.zp_mode != "calibrated"):
            raise NotImplementedError("the gfx950 dequant reads calibrated asym-NF4 or uniform containers")
        if uniform and c.bits != 4:
            raise NotImplementedError("the gfx950 dequant reads 4-bit uniform containers")
        gscale = np.asarray(c.scale)[:, :, 0, :] if uniform else np.asarray(c.nf4_scale)
        gmean = np.asarray(c.zero)[:, :, 0, :] if uniform else np.asarray(c.nf4_mean)
        if not 1 <= S <= _MAX_GROUP_TOKENS or D != 128:
            raise NotImplementedError(f"one gfx950 key group holds 1..{_MAX_GROUP_TOKENS} tokens at head_dim 128")
        kp = c.indices if c.packed else _pack_keys(np.asarray(c.indices))
        kp = np.asarray(kp, np.uint8).reshape(B, H * S * D // 2)
        has_out = c.outlier_idx is not None and c.outlier_val is not None
        flat = np.asarray(c.outlier_idx, np.int64).reshape(-1) if has_out else np.zeros(0, np.int64)
        vals = np.asarray(c.outlier_val, np.float16).reshape(-1) if has_out else np.zeros(0, np.float16)
        # side-list sized for the container's own counts (ties can exceed k per channel)
        per_head = np.bincount(flat // (S * D), minlength=B * H) if flat.size else np.zeros(1, np.int64)
        cap = max(1, int(per_head.max()))
        frac = self.outlier_frac if self.outlier_frac > 0 else 0.02
        pool = _pool(H, S, 3, frac if has_out else 0.0, B, device=self.device,
                     outlier_cap=cap if has_out else 0, key_grid="uniform" if uniform else "nf4_asym")
        for b in range(B):
            m = (flat // (H * S * D)) == b
            pool.import_group(b, 0, keys={
                "kpacked": kp[b], "nf4_scale": gscale[b], "nf4_mean": gmean[b],
                "outlier_idx": flat[m] - b * H * S * D, "outlier_val": vals[m]})
        keys, _ = pool.dequant_groups([(b, 0) for b in range(B)])
        return keys.cpu().numpy().reshape(B, H, S, D)

    # affine capability (turboquant_pro/kv_fused_pck.py:47-127), on the container
    def grid_params(self, c: CompressedPerChannelKV):
        """``mu (H, D)``, ``weight (H, D)``, ``grid (16,)`` with
        dequant = mu + weight * grid[code]; B must be 1."""
        B = c.shape[0]
        if B != 1:
            raise ValueError("fused decode operates on single-batch blocks (B=1)")
        if c.nf4_scale is None and c.levels is None and c.scale is not None:
            # uniform: dequant = zero + scale * code
            return (np.asarray(c.zero)[0, :, 0, :].astype(np.float32),
                    np.asarray(c.scale)[0, :, 0, :].astype(np.float32), np.arange(16, dtype=np.float32))
        if c.nf4_scale is None:
            raise NotImplementedError("only NF4-family and uniform containers carry the affine grid here")
        mu = (np.asarray(c.nf4_mean)[0] if c.nf4_mean is not None
              else np.zeros(np.asarray(c.nf4_scale)[0].shape, np.float32))
        return mu.astype(np.float32), np.asarray(c.nf4_scale)[0].astype(np.float32), NF4.copy()

    def codes(self, c: CompressedPerChannelKV) -> np.ndarray:
        """Unpacked codes ``(B, H, S, D)`` uint8."""
        B, H, S, D = c.shape
        if c.packed:
            return unpack_keys(c.indices, B * H * S * D).reshape(B, H, S, D)
        return np.asarray(c.indices)

    def outlier_csr(self, c: CompressedPerChannelKV):
        """Token-major CSR of the outliers as deltas against the dense dequant:
        ``row_ptr (H*S + 1,) int32``, ``cols (nnz,) uint16`` channels,
        ``deltas (nnz,) float32`` = fp32(val) - (mu + weight * grid[code]);
        ``None`` without outliers."""
        if c.outlier_idx is None:
            return None
        B, H, S, D = c.shape
        if B != 1:
            raise ValueError("fused decode operates on single-batch blocks (B=1)")
        mu, weight, grid = self.grid_params(c)
        codes = self.codes(c)
        flat = np.asarray(c.outlier_idx, np.int64)
        h, s, j = (flat // (S * D)) % H, (flat // D) % S, flat % D
        dense = mu[h, j] + weight[h, j] * grid[codes[0, h, s, j]]
        deltas = np.asarray(c.outlier_val, np.float16).astype(np.float32) - dense
        order = np.lexsort((j, s, h))
        h, s, j, deltas = h[order], s[order], j[order], deltas[order]
        counts = np.bincount(h * S + s, minlength=H * S)
        row_ptr = np.zeros(H * S + 1, np.int32)
        np.cumsum(counts, out=row_ptr[1:])
        return row_ptr, j.astype(np.uint16), deltas.astype(np.float32)

    def native_dtype(self) -> str | None:
        return None


def _pack_keys(codes: np.ndarray) -> np.ndarray:
    """Flat 4-bit codes -> reference key bytes (code 2n bit-reversed in the
    high nibble, 2n + 1 in the low one)."""
    from .formats import _rev4

    v = np.asarray(codes, np.uint8).reshape(-1, 2)
    return ((_rev4(v[:, 0]) << 4) | _rev4(v[:, 1])).astype(np.uint8)


class PolarQuantizer:
    """``"polar"`` values on the gfx950 library: PolarQuant (norm + rotated
    direction on the Lloyd-Max grid) at 3 or 4 bits.

    Constructor as ``TurboQuantKV.__init__`` (turboquant_pro/core.py:178-228):
    ``bits`` is the default width, ``key_bits`` / ``value_bits`` override it
    per kind; the rotation is the reference's ``seed`` recipe.  Widths other
    than 3 and 4, ``head_dim`` other than 128, and PolarQuant *keys* have no
    gfx950 form."""

    def __init__(self, head_dim: int = 128, n_heads: int = 32, bits: int = 3,
                 key_bits: int | None = None, value_bits: int | None = None, use_gpu: bool = True,
                 device_id: int = 0, seed: int | None = None, device=None) -> None:
        self.key_bits = key_bits if key_bits is not None else bits
        self.value_bits = value_bits if value_bits is not None else bits
        for name, v in (("bits", bits), ("key_bits", self.key_bits), ("value_bits", self.value_bits)):
            if v not in (2, 3, 4):
                raise ValueError(f"Unsupported {name}={v}; choose from [2, 3, 4]")
        if head_dim != 128:
            raise NotImplementedError("the gfx950 value encode serves head_dim 128")
        self.head_dim, self.n_heads, self.bits, self.seed = head_dim, n_heads, bits, seed
        self.device = device
        # drawn once, as TurboQuantKV does (core.py:178-228): with seed=None the
        # instance's compress and decompress still share one rotation
        self.rotation = random_rotation(seed, head_dim)

    def _width(self, kind: str | None) -> int:
        if kind == "key":
            raise NotImplementedError("PolarQuant keys have no gfx950 form (the cache's keys are asym-NF4)")
        if kind not in (None, "value"):
            raise ValueError(f"kind must be 'key', 'value' or None, got {kind!r}")
        w = self.value_bits if kind == "value" else self.bits
        if w not in (3, 4):
            raise NotImplementedError(f"the gfx950 value encode is 3 or 4 bits, not {w}")
        return w

    def compress(self, tensor: np.ndarray, packed: bool = False, kind: str | None = None) -> CompressedKV:
        """``(B, H, S, D)`` values (taken as fp16) -> codes + fp32 norms, in
        groups of up to 256 tokens (PolarQuant is per token)."""
        from .pool import _torch

        torch = _torch()
        bits = self._width(kind)
        orig = np.asarray(tensor).dtype
        vt = _fp16_tokens(tensor)
        B, H, S, D = vt.shape
        codes = np.zeros((B, H, S, D), np.uint8)
        norms = np.zeros((B, H, S), np.float32)
        for t0 in range(0, S, _MAX_GROUP_TOKENS):
            n = min(_MAX_GROUP_TOKENS, S - t0)
            pool = _pool(H, n, bits, 0.0, B, rotation=self.rotation, device=self.device)
            chunk = vt[:, :, t0:t0 + n]
            v = torch.cat([chunk, torch.zeros_like(chunk)], dim=2).to(pool.device)
            pool.append(torch.zeros_like(v), v)
            for b in range(B):
                e = pool.export_group(b, 0)
                codes[b, :, t0:t0 + n] = unpack_values(e["vpacked"], H * n * D, bits).reshape(H, n, D)
                norms[b, :, t0:t0 + n] = e["vnorms"]
        shape = (B, H, S, D)
        if packed:
            return CompressedKV(pack_values(codes, bits), norms, bits, np.dtype(orig), True,
                                int(codes.size), shape)
        return CompressedKV(codes, norms, bits, np.dtype(orig), False, int(codes.size), shape)

    def decompress(self, compressed: CompressedKV) -> np.ndarray:
        """fp32 ``(B, H, S, D)`` = norm * (centroids[code] @ Pi), on the GPU
        (turboquant_pro/core.py:619-654)."""
        bits = compressed.bits
        if bits not in (3, 4):
            raise NotImplementedError(f"the gfx950 value dequant is 3 or 4 bits, not {bits}")
        B, H, S, D = compressed.shape
        codes = (unpack_values(compressed.indices, compressed.n_values, bits) if compressed.packed
                 else np.asarray(compressed.indices, np.uint8)).reshape(B, H, S, D)
        norms = np.asarray(compressed.norms, np.float32).reshape(B, H, S)
        out = np.zeros((B, H, S, D), np.float32)
        for t0 in range(0, S, _MAX_GROUP_TOKENS):
            n = min(_MAX_GROUP_TOKENS, S - t0)
            pool = _pool(H, n, bits, 0.0, B, rotation=self.rotation, device=self.device)
            for b in range(B):
                pool.import_group(b, 0, values={
                    "vpacked": pack_values(codes[b, :, t0:t0 + n], bits),
                    "vnorms": norms[b, :, t0:t0 + n]})
            _, vals = pool.dequant_groups([(b, 0) for b in range(B)])
            out[:, :, t0:t0 + n] = vals.cpu().numpy().reshape(B, H, n, D)
        return out


def _per_channel_factory(**config: Any) -> PerChannelKVQuantizer:
    return PerChannelKVQuantizer(**config)


def _polar_factory(**config: Any) -> PolarQuantizer:
    return PolarQuantizer(**config)


register(PluginSpec(
    name="per_channel", factory=_per_channel_factory, targets=frozenset({TARGET_KV_KEY}), tier="beta",
    description="per-channel asym-NF4 4-bit keys with the fp16 outlier side-list on the gfx950 "
                "library; full affine contract"))
register(PluginSpec(
    name="polar", factory=_polar_factory, targets=frozenset({TARGET_KV_VALUE}), tier="stable",
    description="PolarQuant values (rotation + norm/direction codes) at 3 or 4 bits on the gfx950 "
                "library"))
