"""Quantizer plugin registry and the two in-tree KV formats, on the gfx950
library (turboquant_pro/plugins.py:60-360).

The registry keeps the reference's surface: targets as plain strings,
:class:`PluginSpec`, :func:`register` / :func:`get_plugin` / :func:`create` /
:func:`available_plugins`, out-of-tree discovery through the
``turboquant_pro.plugins`` entry-point group, and the optional-capability
probes :func:`affine_params` / :func:`affine_codes` / :func:`outlier_csr` /
:func:`native_dtype`.

In-tree formats:

* ``"per_channel"`` -- :class:`PerChannelKVQuantizer`, per-channel 4-bit keys
  (asym-NF4 with a calibrated, sparse or bias zero point, or uniform) with the
  fp16 outlier side-list (turboquant_pro/per_channel_kv.py:182-401).
  ``compress`` runs the GPU block encode, every (b, h) pair one group of any
  length S, and returns the reference container bit for bit for fp32 or fp16
  input; ``decompress`` runs the GPU block dequant.  The affine capability
  (``grid_params`` / ``codes`` / ``outlier_csr``) reads the container on the
  host, as the reference's (turboquant_pro/kv_fused_pck.py:47-127).
* ``"polar"`` -- :class:`PolarQuantizer`, PolarQuant
  (turboquant_pro/core.py:139-654) at 2, 3 or 4 bits, of values or keys:
  ``compress`` / ``decompress`` on the GPU, any number of tokens.

Configurations the library has no gfx950 form for raise
``NotImplementedError`` at construction.
"""

from __future__ import annotations

import ctypes
import logging
from collections.abc import Callable
from dataclasses import dataclass, field
from importlib import metadata
from typing import Any, Protocol, runtime_checkable

import numpy as np

from .codebooks import HEAD_DIMS, outliers_per_channel, random_rotation
from .formats import NF4, pack_values, unpack_key_codes, unpack_values

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
def _torch():
    import torch
    return torch


def _device_tokens(x, device):
    """A ``(B, H, S, D)`` block on the GPU as the block kernels read it, and
    whether it is fp32: fp16 input stays fp16 (exact either way, half the
    bytes); anything else becomes fp32, as ``np.asarray(x, dtype=np.float32)``
    makes it in the reference (turboquant_pro/per_channel_kv.py:293)."""
    torch = _torch()
    dev = torch.device(device if device is not None else "cuda")
    if isinstance(x, torch.Tensor):
        t = x.detach()
        if t.dtype != torch.float16:
            t = t.to(torch.float32)
    else:
        a = np.asarray(x)
        a = a if a.dtype == np.float16 else np.asarray(a, dtype=np.float32)
        t = torch.from_numpy(np.ascontiguousarray(a))
    if t.dim() != 4:
        raise ValueError(f"expected (B,H,S,D), got shape {tuple(t.shape)}")
    return t.to(dev).contiguous(), int(t.dtype == torch.float32)


def _block_desc(shape, bits: int, key_grid: int = 0, zero_point: int = 0, k: int = 0, cap: int = 0,
                f32: int = 1, dc=None):
    from . import _native as N
    from .codebooks import dc_mask_words
    B, H, S, D = (int(v) for v in shape)
    d = N.BlockDesc(batch=B, n_heads=H, tokens=S, head_dim=D, bits=bits, key_grid=key_grid,
                    zero_point=zero_point, outliers_per_channel=k, outlier_cap=cap, input_f32=f32)
    if dc is not None:
        d.dc_mask[:] = dc_mask_words(dc)
    return d


def _stream():
    return ctypes.c_void_p(_torch().cuda.current_stream().cuda_stream)


# the block descriptor's zero points; symmetric NF4 is its "sparse" mode with
# no DC channel (every mean 0)
_ZERO_POINTS = {"calibrated": 0, "sparse": 1, "bias": 2, "symmetric": 1}


class PerChannelKVQuantizer:
    """``"per_channel"`` keys on the gfx950 library: asym-NF4 4-bit (zero
    point "calibrated", "sparse" or "bias"), symmetric NF4 (``nf4=True``
    without ``nf4_asym``) or uniform 2-, 3- or 4-bit (the reference's default
    mode), with the fp16 outlier side-list; every (b, h) pair of a block is
    one group.

    The constructor validates like ``PerChannelKV.__init__``
    (turboquant_pro/per_channel_kv.py:182-213) and raises
    ``NotImplementedError`` for the modes the library does not encode
    (data-fit quantiles, head_dim other than 64, 128 or 256)."""

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
        uniform = not nf4 and not nuq
        if nuq or head_dim not in HEAD_DIMS:
            raise NotImplementedError("the gfx950 key encode is per-channel asym-NF4 (any zero point), "
                                      "symmetric NF4 "
                                      f"or uniform 2/3/4-bit, at head_dim {HEAD_DIMS}")
        self.head_dim, self.n_heads, self.bits = head_dim, n_heads, bits
        self.uniform = uniform
        # symmetric NF4 (nf4 without nf4_asym): the asym-NF4 encode with no mean
        self.symmetric = nf4 and not nf4_asym
        self.key_grid = "uniform" if uniform else "nf4_asym"
        self.nuq, self.nf4, self.nf4_asym = nuq, nf4, nf4_asym
        self.outlier_frac, self.zero_point = outlier_frac, zero_point
        self.rope_theta = rope_theta
        self.k_bias = (np.asarray(k_bias, dtype=np.float32).reshape(n_heads, head_dim)
                       if zero_point == "bias" else None)
        self.device = device

    def compress(self, x, packed: bool = False, position_start: int = 0) -> CompressedPerChannelKV:
        """``(B, H, S, D)`` keys, any S, each (b, h) one group, on the GPU
        (turboquant_pro/per_channel_kv.py:285-401); fp32 (or fp16) input is
        encoded as given, bit for bit."""
        from . import _native as N
        from .codebooks import dc_channel_mask, rope_averaged_bias

        torch = _torch()
        xt, f32 = _device_tokens(x, self.device)
        B, H, S, D = xt.shape
        if D != self.head_dim:
            raise ValueError(f"head_dim {D} != {self.head_dim}")
        k = outliers_per_channel(S, self.outlier_frac)
        zp_mode = "calibrated" if self.uniform else "symmetric" if self.symmetric else self.zero_point
        dc = (dc_channel_mask(self.rope_theta, D, S) if zp_mode == "sparse"
              else np.zeros(D, bool) if zp_mode == "symmetric" else None)
        zp = None
        if zp_mode == "bias":
            if H != self.n_heads:
                raise ValueError(f"input has {H} heads but k_bias was given for {self.n_heads}; "
                                 "zero_point='bias' needs them equal")
            zp = torch.from_numpy(rope_averaged_bias(self.k_bias, self.rope_theta, D, position_start, S)
                                  ).to(xt.device)
        u8, f32t, i32 = torch.uint8, torch.float32, torch.int32
        kp = torch.empty(B * H * S * D * self.bits // 8, dtype=u8, device=xt.device)
        scale = torch.empty((B, H, D), dtype=f32t, device=xt.device)
        zero = torch.empty_like(scale)
        count = torch.zeros(B * H, dtype=i32, device=xt.device)
        cap = min(S * D, 4 * k * D) if k else 0
        while True:
            pos = torch.empty((B * H, max(cap, 1)), dtype=torch.int32, device=xt.device)
            val = torch.empty((B * H, max(cap, 1)), dtype=torch.float16, device=xt.device)
            d = _block_desc(xt.shape, self.bits, int(self.uniform), _ZERO_POINTS[zp_mode], k, cap, f32, dc)
            N.check(N.lib().tqk_encode_key_block(
                ctypes.byref(d), xt.data_ptr(), zp.data_ptr() if zp is not None else None,
                kp.data_ptr(), scale.data_ptr(), zero.data_ptr(), pos.data_ptr(), val.data_ptr(),
                count.data_ptr(), _stream()), "tqk_encode_key_block")
            cnt = count.cpu().numpy()
            if k == 0 or int(cnt.max()) <= cap:
                break
            cap = int(cnt.max())  # magnitude ties: more than k per channel
        kp_np = kp.cpu().numpy()
        oidx = oval = None
        if k:
            pos_np = pos.cpu().numpy().view(np.uint32)
            val_np = val.cpu().numpy()
            oidx = np.concatenate([pos_np[i, :cnt[i]].astype(np.int64) + i * S * D
                                   for i in range(B * H)]).astype(np.int32)
            oval = np.concatenate([val_np[i, :cnt[i]] for i in range(B * H)]).astype(np.float16)
        indices = kp_np if packed else unpack_key_codes(kp_np, B * H * S * D, self.bits).reshape(B, H, S, D)
        sc, zr = scale.cpu().numpy(), zero.cpu().numpy()
        if self.uniform:
            # per_channel_kv.py:303-317: (B, H, 1, D) scale and zero, no NF4 fields
            return CompressedPerChannelKV(indices, sc[:, :, None, :], zr[:, :, None, :], self.bits,
                                          (B, H, S, D), packed, outlier_idx=oidx, outlier_val=oval)
        # the stored zero point: every channel's, the DC channels', or none
        # (bias: recomputed; symmetric NF4: there is none, and its container
        # says "calibrated", per_channel_kv.py:354-357)
        mean = {"calibrated": zr, "sparse": zr[:, :, dc] if dc is not None else None, "bias": None,
                "symmetric": None}[zp_mode]
        stored_mode = "calibrated" if zp_mode == "symmetric" else zp_mode
        return CompressedPerChannelKV(
            indices, None, None, self.bits, (B, H, S, D), packed, nf4_scale=sc, nf4_mean=mean,
            outlier_idx=oidx, outlier_val=oval, zp_mode=stored_mode,
            rope_theta=self.rope_theta if stored_mode != "calibrated" else None,
            position_start=position_start)

    def decompress(self, c: CompressedPerChannelKV) -> np.ndarray:
        """fp32 ``(B, H, S, D)``: ``zero point + scale * NF4[code]`` (or
        ``zero + scale * code``), outliers overwritten by their fp16 values
        (turboquant_pro/per_channel_kv.py:497-539), on the GPU."""
        from . import _native as N
        from .codebooks import dc_channel_mask, rope_averaged_bias

        torch = _torch()
        B, H, S, D = c.shape
        uniform = c.nf4_scale is None and c.levels is None and c.scale is not None and c.zero is not None
        if c.levels is not None or (not uniform and c.nf4_scale is None):
            raise NotImplementedError("data-fit (quantile) key grids have no gfx950 dequant")
        if c.bits not in (2, 3, 4) or (c.bits != 4 and not uniform) or D not in HEAD_DIMS:
            raise NotImplementedError("the gfx950 dequant reads asym-NF4 4-bit or uniform 2/3/4-bit "
                                      f"keys at head_dim {HEAD_DIMS}")
        if uniform:
            scale = np.asarray(c.scale, np.float32)[:, :, 0, :]
            zero = np.asarray(c.zero, np.float32)[:, :, 0, :]
        else:
            scale = np.asarray(c.nf4_scale, np.float32)
            if c.zp_mode == "bias":
                if self.k_bias is None:
                    raise ValueError('container was compressed with zero_point="bias"; decompress '
                                     "needs a quantizer built with the same k_bias")
                zero = np.broadcast_to(rope_averaged_bias(self.k_bias, c.rope_theta, D, c.position_start, S)[None],
                                       (B, H, D))
            elif c.zp_mode == "sparse":
                zero = np.zeros((B, H, D), np.float32)
                zero[:, :, dc_channel_mask(c.rope_theta, D, S)] = c.nf4_mean
            elif c.nf4_mean is not None:
                zero = np.asarray(c.nf4_mean, np.float32)
            else:  # symmetric NF4 container: no zero point
                zero = np.zeros((B, H, D), np.float32)
        kp = np.asarray(c.indices if c.packed else _pack_keys(np.asarray(c.indices), c.bits),
                        np.uint8).reshape(-1)
        has_out = c.outlier_idx is not None and c.outlier_val is not None
        _check_key_container(kp, scale, zero, c, B * H * S * D, (B, H, D), has_out)
        dev = torch.device(self.device if self.device is not None else "cuda")
        # a writable host copy: containers may hold read-only arrays (np.load)
        t = lambda a, dt: torch.from_numpy(np.array(a, dt, order="C")).to(dev)  # noqa: E731
        kp_d, sc_d, zr_d = t(kp, np.uint8), t(scale, np.float32), t(zero, np.float32)
        n_out = int(np.asarray(c.outlier_idx).size) if has_out else 0
        idx_d = t(np.asarray(c.outlier_idx, np.int32).reshape(-1), np.int32) if n_out else None
        val_d = t(np.asarray(c.outlier_val, np.float16).reshape(-1).view(np.int16), np.int16) if n_out else None
        out = torch.empty((B, H, S, D), dtype=torch.float32, device=dev)
        d = _block_desc(c.shape, c.bits, int(uniform))
        N.check(N.lib().tqk_dequant_key_block(
            ctypes.byref(d), kp_d.data_ptr(), sc_d.data_ptr(), zr_d.data_ptr(), n_out,
            idx_d.data_ptr() if n_out else None, val_d.data_ptr() if n_out else None, out.data_ptr(),
            _stream()), "tqk_dequant_key_block")
        return out.cpu().numpy()

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
                    np.asarray(c.scale)[0, :, 0, :].astype(np.float32), np.arange(1 << c.bits, dtype=np.float32))
        if c.nf4_scale is None:
            raise NotImplementedError("only NF4-family and uniform containers carry the affine grid here")
        mu = (np.asarray(c.nf4_mean)[0] if c.nf4_mean is not None
              else np.zeros(np.asarray(c.nf4_scale)[0].shape, np.float32))
        return mu.astype(np.float32), np.asarray(c.nf4_scale)[0].astype(np.float32), NF4.copy()

    def codes(self, c: CompressedPerChannelKV) -> np.ndarray:
        """Unpacked codes ``(B, H, S, D)`` uint8."""
        B, H, S, D = c.shape
        if c.packed:
            return unpack_key_codes(c.indices, B * H * S * D, c.bits).reshape(B, H, S, D)
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


def _pack_keys(codes: np.ndarray, bits: int = 4) -> np.ndarray:
    """Flat key codes -> reference key bytes (turboquant_pro/per_channel_kv.py:87-93)."""
    from .formats import pack_key_codes

    return pack_key_codes(codes, bits)


class PolarQuantizer:
    """``"polar"`` on the gfx950 library: PolarQuant (norm + rotated direction
    on the Lloyd-Max grid) at 2, 3 or 4 bits.

    Constructor as ``TurboQuantKV.__init__`` (turboquant_pro/core.py:178-228):
    ``bits`` is the default width, ``key_bits`` / ``value_bits`` override it
    per kind (``compress(kind=...)``); the rotation is the reference's
    ``seed`` recipe.  ``head_dim`` is 64, 128 or 256 (the gfx950 kernels')."""

    def __init__(self, head_dim: int = 128, n_heads: int = 32, bits: int = 3,
                 key_bits: int | None = None, value_bits: int | None = None, use_gpu: bool = True,
                 device_id: int = 0, seed: int | None = None, device=None) -> None:
        self.key_bits = key_bits if key_bits is not None else bits
        self.value_bits = value_bits if value_bits is not None else bits
        for name, v in (("bits", bits), ("key_bits", self.key_bits), ("value_bits", self.value_bits)):
            if v not in (2, 3, 4):
                raise ValueError(f"Unsupported {name}={v}; choose from [2, 3, 4]")
        if head_dim not in HEAD_DIMS:
            raise NotImplementedError(f"the gfx950 PolarQuant encode serves head_dim {HEAD_DIMS}")
        self.head_dim, self.n_heads, self.bits, self.seed = head_dim, n_heads, bits, seed
        self.device = device
        # drawn once, as TurboQuantKV does (core.py:178-228): with seed=None the
        # instance's compress and decompress still share one rotation
        self.rotation = random_rotation(seed, head_dim)
        self._dev_consts: dict = {}

    def _width(self, kind: str | None) -> int:
        if kind not in (None, "key", "value"):
            raise ValueError(f"kind must be 'key', 'value' or None, got {kind!r}")
        return self.key_bits if kind == "key" else self.value_bits if kind == "value" else self.bits

    def _consts(self, bits: int):
        """Device copies of Pi and the bits-wide codebook."""
        torch = _torch()
        got = self._dev_consts.get(bits)
        if got is None:
            from .codebooks import value_codebook
            dev = torch.device(self.device if self.device is not None else "cuda")
            cent, bnd = value_codebook(bits, self.head_dim)
            got = tuple(torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
                        for a in (self.rotation[0], cent, bnd))
            self._dev_consts[bits] = got
        return got

    def compress(self, tensor, packed: bool = False, kind: str | None = None) -> CompressedKV:
        """``(B, H, S, D)`` -> codes + fp32 norms (turboquant_pro/core.py:542-617),
        any S, on the GPU; fp32 (or fp16) input is encoded as given, bit for bit."""
        from . import _native as N

        torch = _torch()
        bits = self._width(kind)
        orig = np.dtype(str(tensor.dtype).replace("torch.", "")) if isinstance(tensor, torch.Tensor) \
            else np.asarray(tensor).dtype
        xt, f32 = _device_tokens(tensor, self.device)
        B, H, S, D = xt.shape
        pi, _, bnd = self._consts(bits)
        out = torch.empty(B * H * S * D * bits // 8, dtype=torch.uint8, device=xt.device)
        norms = torch.empty((B, H, S), dtype=torch.float32, device=xt.device)
        d = _block_desc(xt.shape, bits, f32=f32)
        N.check(N.lib().tqk_encode_value_block(ctypes.byref(d), xt.data_ptr(), pi.data_ptr(),
                                               bnd.data_ptr(), out.data_ptr(), norms.data_ptr(),
                                               _stream()), "tqk_encode_value_block")
        pk, nv = out.cpu().numpy(), norms.cpu().numpy()
        shape, n = (B, H, S, D), B * H * S * D
        if packed:
            return CompressedKV(pk, nv, bits, orig, True, n, shape)
        return CompressedKV(unpack_values(pk, n, bits).reshape(shape), nv, bits, orig, False, n, shape)

    def decompress(self, compressed: CompressedKV) -> np.ndarray:
        """fp32 ``(B, H, S, D)`` = norm * (centroids[code] @ Pi), on the GPU
        (turboquant_pro/core.py:619-654)."""
        from . import _native as N

        torch = _torch()
        bits = compressed.bits
        if bits not in (2, 3, 4):
            raise NotImplementedError(f"the gfx950 PolarQuant dequant is 2, 3 or 4 bits, not {bits}")
        B, H, S, D = compressed.shape
        n = B * H * S * D
        pk = (np.asarray(compressed.indices, np.uint8).reshape(-1)[: n * bits // 8] if compressed.packed
              else pack_values(np.asarray(compressed.indices, np.uint8), bits))
        norms = np.ascontiguousarray(compressed.norms, np.float32).reshape(-1)
        if pk.size != n * bits // 8 or norms.size != B * H * S:
            raise ValueError(f"value container holds {pk.size} code bytes and {norms.size} norms, "
                             f"shape {compressed.shape} needs {n * bits // 8} and {B * H * S}")
        pi, cent, _ = self._consts(bits)
        dev = pi.device
        pk_d = torch.from_numpy(np.ascontiguousarray(pk)).to(dev)
        nv_d = torch.from_numpy(norms).to(dev)
        out = torch.empty((B, H, S, D), dtype=torch.float32, device=dev)
        d = _block_desc(compressed.shape, bits)
        N.check(N.lib().tqk_dequant_value_block(ctypes.byref(d), pk_d.data_ptr(), nv_d.data_ptr(),
                                                pi.data_ptr(), cent.data_ptr(), out.data_ptr(),
                                                _stream()), "tqk_dequant_value_block")
        return out.cpu().numpy()


def _check_key_container(kp, scale, zero, c, n, bhd, has_out) -> None:
    """Sizes and side-list indices of a key container before its arrays go to
    the GPU (a container read from a store may be damaged or foreign)."""
    if kp.size != n * c.bits // 8:
        raise ValueError(f"key container holds {kp.size} code bytes, shape {c.shape} needs {n * c.bits // 8}")
    if scale.shape != bhd or zero.shape != bhd:
        raise ValueError(f"key container scale {scale.shape} / zero point {zero.shape}, expected {bhd}")
    if has_out:
        idx = np.asarray(c.outlier_idx).reshape(-1)
        if idx.size != np.asarray(c.outlier_val).size:
            raise ValueError("outlier index and value lists differ in length")
        if idx.size and (int(idx.min()) < 0 or int(idx.max()) >= n):
            raise ValueError(f"outlier index outside [0, {n})")


def _per_channel_factory(**config: Any) -> PerChannelKVQuantizer:
    return PerChannelKVQuantizer(**config)


def _polar_factory(**config: Any) -> PolarQuantizer:
    return PolarQuantizer(**config)


register(PluginSpec(
    name="per_channel", factory=_per_channel_factory, targets=frozenset({TARGET_KV_KEY}), tier="beta",
    description="per-channel 4-bit keys (asym-NF4, any zero point, or uniform) with the fp16 outlier side-list on the gfx950 "
                "library; full affine contract"))
register(PluginSpec(
    name="polar", factory=_polar_factory, targets=frozenset({TARGET_KV_VALUE}), tier="stable",
    description="PolarQuant values (rotation + norm/direction codes) at 2, 3 or 4 bits on the gfx950 "
                "library"))
