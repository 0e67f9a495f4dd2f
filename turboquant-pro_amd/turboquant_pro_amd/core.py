"""Drop-in ``TurboQuantKVCache`` backed by the gfx950 kernels.

Same constructor, methods and return conventions as the reference's
``TurboQuantKVCache`` (turboquant_pro/core.py:818-1307): one sequence, an fp16
hot window of ``hot_window`` tokens, and flushed groups of
``(hot_window + 1) // 2`` tokens coded as per-channel keys (4-bit asym-NF4
with a calibrated, sparse or bias zero point, or uniform 2/3/4-bit -- the
reference's default) with an fp16 outlier side-list, or as PolarQuant
(``per_channel_keys=False``), plus 2/3/4-bit PolarQuant values.  Storage and compute live on the GPU:
``append`` runs the quantize-on-flush kernel when a group completes,
``fused_decode`` runs the fused split-K kernel, ``get_keys``/``get_values``
reconstruct on the GPU.

Differences from the reference, all deliberate:
  * the fused path supports ``key_bits != value_bits`` (the reference raises
    NotImplementedError, turboquant_pro/core.py:1193-1194; K4/V3 is the
    AutoConfig default and the point of this build);
  * keys/values/queries are converted to fp16 on entry (the serving dtype the
    kernels consume); codes are bit-exact with the reference for fp16 inputs;
  * ``per_channel_keys=False`` (PolarQuant keys, turboquant_pro/core.py:1028-1029)
    requires ``key_bits == value_bits``, as the reference's fused decode does;
  * configurations without a gfx950 form (quantile keys; head_dim other than
    64, 128 or 256) raise
    NotImplementedError at construction instead of silently running on the CPU;
  * an optional ``n_q_heads`` (a multiple of ``n_heads``) serves GQA queries.
"""

from __future__ import annotations

import logging

import numpy as np

from .codebooks import HEAD_DIMS, SUPPORTED_BITS, group_tokens_for, n_groups_for
from .pool import TQKVPool

logger = logging.getLogger(__name__)


def _torch():
    import torch
    return torch


def merge_partials(parts):
    """Final attention output ``(H, D)`` of unnormalised online-softmax states
    ``[(m (H,), l (H,), acc (H, D)), ...]`` over disjoint key sets -- e.g.
    :meth:`TurboQuantKVCache.fused_decode_partials` and a state over extra
    keys (the contract of turboquant_pro/kv_fused.py:139-153).  NumPy arrays or
    torch tensors; each state is rescaled to the largest running max."""
    if not parts:
        raise ValueError("no partial states to merge")
    torch = _torch() if any(isinstance(p[0], _torch().Tensor) for p in parts) else None
    if torch is not None:
        m = torch.stack([torch.as_tensor(p[0]) for p in parts])
        l_ = torch.stack([torch.as_tensor(p[1]) for p in parts])
        acc = torch.stack([torch.as_tensor(p[2]) for p in parts])
        w = torch.exp(m - m.max(dim=0).values)
    else:
        m, l_, acc = (np.stack([np.asarray(p[i]) for p in parts]) for i in range(3))
        w = np.exp(m - m.max(axis=0))
    return (acc * w[..., None]).sum(0) / (l_ * w).sum(0)[..., None]


class TurboQuantKVCache:
    """GPU-resident two-tier KV cache of one sequence (see module docstring)."""

    @classmethod
    def robust(cls, head_dim: int = 128, n_heads: int = 32, *, key_bits: int = 4,
               value_bits: int = 4, hot_window: int = 512, outlier_frac: float = 0.02,
               **kwargs) -> "TurboQuantKVCache":
        """Asym-NF4 keys + ``outlier_frac`` fp16 outliers (turboquant_pro/core.py:856-884)."""
        return cls(head_dim=head_dim, n_heads=n_heads, key_bits=key_bits, value_bits=value_bits,
                   hot_window=hot_window, key_nf4_asym=True, key_outlier_frac=outlier_frac,
                   **kwargs)

    def __init__(self, head_dim: int = 128, n_heads: int = 32, bits: int = 3,
                 key_bits: int | None = None, value_bits: int | None = None,
                 hot_window: int = 512, use_gpu: bool = True, device_id: int = 0,
                 seed: int | None = None, per_channel_keys: bool = True, key_nuq: bool = False,
                 key_nf4: bool = False, key_nf4_asym: bool = False,
                 key_outlier_frac: float = 0.0, key_zero_point: str = "calibrated",
                 key_rope_theta: float | None = None, key_k_bias=None, *,
                 n_q_heads: int | None = None, capacity: int = 4096,
                 input_dtype: str | None = None) -> None:
        self.head_dim = head_dim
        self.n_heads = n_heads
        self.n_q_heads = n_heads if n_q_heads is None else n_q_heads
        self.bits = bits
        self.key_bits = key_bits if key_bits is not None else bits
        self.value_bits = value_bits if value_bits is not None else bits
        self.hot_window = hot_window
        self.per_channel_keys = per_channel_keys
        self.key_outlier_frac = key_outlier_frac
        self.key_zero_point = key_zero_point
        self.seed = seed
        for name, b in (("bits", bits), ("key_bits", self.key_bits), ("value_bits", self.value_bits)):
            if b not in SUPPORTED_BITS:
                raise ValueError(f"Unsupported {name}={b}; choose from {list(SUPPORTED_BITS)}")
        if not (0.0 <= key_outlier_frac < 1.0):
            raise ValueError("outlier_frac must be in [0, 1)")
        if key_zero_point not in ("calibrated", "sparse", "bias"):
            raise ValueError("zero_point must be one of ('calibrated', 'sparse', 'bias')")
        if key_nf4_asym:
            key_nf4 = True
        if not per_channel_keys:
            # PolarQuant keys (turboquant_pro/core.py:1028-1029): the per-channel
            # flags configure a quantizer the reference then never builds
            key_nf4 = key_nf4_asym = key_nuq = False
            key_zero_point, key_rope_theta, key_k_bias = "calibrated", None, None
            self.key_zero_point = key_zero_point
            if self.key_bits != self.value_bits:
                raise NotImplementedError(
                    "PolarQuant keys on the gfx950 cache share the value codebook: key_bits must "
                    "equal value_bits (the reference's fused decode has the same requirement)")
        if key_nf4 and self.key_bits != 4:
            raise ValueError("nf4=True requires bits=4")
        # zero-point checks of PerChannelKV.__init__ (turboquant_pro/per_channel_kv.py:199-213)
        if key_zero_point != "calibrated":
            if not key_nf4_asym:
                raise ValueError(f"zero_point={key_zero_point!r} requires nf4_asym=True")
            if key_rope_theta is None:
                raise ValueError(f"zero_point={key_zero_point!r} requires rope_theta")
        if key_zero_point == "bias":
            if key_k_bias is None:
                raise ValueError('zero_point="bias" requires k_bias')
            key_k_bias = np.asarray(key_k_bias, dtype=np.float32).reshape(n_heads, head_dim)
        self.key_rope_theta, self.key_k_bias = key_rope_theta, key_k_bias
        # per-channel keys: asym-NF4 (robust / build_cache) or, without any NF4
        # or quantile flag, the reference's uniform mode (its default, at 2, 3 or
        # 4 bits); per_channel_keys=False: PolarQuant keys
        uniform = per_channel_keys and not key_nuq and not key_nf4
        if per_channel_keys and key_nuq:
            raise NotImplementedError(
                "the gfx950 cache codes keys per channel as asym-NF4 (TurboQuantKVCache.robust / "
                "AutoConfig.build_cache), symmetric NF4 or uniform 2/3/4-bit, or as PolarQuant "
                "(per_channel_keys=False); data-fit quantile keys have no GPU form here")
        self.key_grid = "polar" if not per_channel_keys else "uniform" if uniform else "nf4_asym"
        # symmetric NF4 (key_nf4 without key_nf4_asym, per_channel_kv.py:354-357):
        # the asym-NF4 encode with no mean
        self._pool_zero_point = ("symmetric" if per_channel_keys and key_nf4 and not key_nf4_asym
                                 else key_zero_point)
        if head_dim not in HEAD_DIMS:
            raise NotImplementedError(f"head_dim {head_dim}: the gfx950 kernels serve {HEAD_DIMS}")
        if group_tokens_for(hot_window) > 256 or hot_window < 1:
            raise NotImplementedError("hot_window must be in [1, 512] for the gfx950 kernels")
        self._device = _torch().device(f"cuda:{device_id}")
        self._capacity = max(capacity, hot_window + 1)
        # the precision the cache takes its tokens in: fixed ("float16",
        # "float32") or, with None, that of the first tokens appended to the
        # empty cache -- fp16 tokens make an fp16 cache, any other float dtype
        # (fp32, bf16: both exact in fp32) an fp32 one, whose codes are the
        # reference's on the same fp32 values
        if input_dtype not in (None, "float16", "float32"):
            raise ValueError(f"input_dtype must be None, 'float16' or 'float32', not {input_dtype!r}")
        self.input_dtype = input_dtype
        self._pool_dtype = input_dtype or "float16"
        self._pool = self._new_pool(self._capacity, rotation=None)
        self._rotation = (self._pool.pi.cpu().numpy(), self._pool.pi_t.cpu().numpy())

    def _new_pool(self, capacity: int, rotation):
        return TQKVPool(n_kv_heads=self.n_heads, n_q_heads=self.n_q_heads, head_dim=self.head_dim,
                        max_batch=1, max_seq_len=capacity, hot_window=self.hot_window,
                        key_bits=self.key_bits, value_bits=self.value_bits,
                        outlier_frac=self.key_outlier_frac if self.key_grid != "polar" else 0.0,
                        seed=self.seed, rotation=rotation,
                        device=self._device, key_grid=self.key_grid,
                        zero_point=self._pool_zero_point, rope_theta=self.key_rope_theta,
                        k_bias=self.key_k_bias, input_dtype=self._pool_dtype)

    def _grow(self, need: int) -> None:
        """Reallocate to hold ``need`` tokens (at least doubling), moving the
        coded groups and the hot ring as they are."""
        cap = max(need, 2 * self._capacity)
        self._pool, self._capacity = self._pool.grown(cap), cap

    # ---------------------------------------------------------------- sizes --
    @property
    def length(self) -> int:
        return self._pool.lengths[0]

    @property
    def cold_length(self) -> int:
        return self._pool.n_groups(0) * self._pool.group_tokens

    @property
    def hot_length(self) -> int:
        return self.length - self.cold_length

    # --------------------------------------------------------------- append --
    def _as_tokens(self, x):
        """(H, D) / (1, H, 1, D) / (H, n, D) -> device tensor (1, H, n, D) in the
        pool's input dtype."""
        torch = _torch()
        t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x))
        if t.dim() == 2:
            t = t[None, :, None, :]
        elif t.dim() == 3:
            t = t[None]
        if t.dim() != 4 or t.shape[0] != 1 or t.shape[1] != self.n_heads or t.shape[3] != self.head_dim:
            raise ValueError(f"expected (H, D), (1, H, 1, D) or (H, n, D) with H={self.n_heads}, "
                             f"D={self.head_dim}; got {tuple(x.shape)}")
        return t.to(device=self._device, dtype=self._pool.dtype).contiguous()

    def _adopt_dtype(self, x) -> None:
        """With no fixed input_dtype, an empty cache takes the precision of the
        tokens appended to it (a fresh pool of the same rotation)."""
        if self.input_dtype is not None or self.length:
            return
        torch = _torch()
        dt = x.dtype if isinstance(x, torch.Tensor) else np.asarray(x).dtype
        want = "float16" if dt in (torch.float16, np.float16) else "float32"
        if want != self._pool_dtype:
            self._pool_dtype = want
            self._pool = self._new_pool(self._capacity, rotation=self._rotation)

    def append(self, key, value) -> None:
        """Add one token's key/value ``(H, D)`` or ``(1, H, 1, D)``
        (turboquant_pro/core.py:986-1009); flushes to coded storage on the GPU."""
        self.extend(key, value)

    def extend(self, keys, values) -> None:
        """Append several tokens at once, ``(H, n, D)`` or ``(1, H, n, D)``;
        identical to n ``append`` calls."""
        self._adopt_dtype(keys)
        k, v = self._as_tokens(keys), self._as_tokens(values)
        if k.shape != v.shape:
            raise ValueError("keys and values must have the same shape")
        n = int(k.shape[2])
        if self.length + n > self._capacity:
            self._grow(self.length + n)
        self._pool.append(k, v)

    # ------------------------------------------------------------- readback --
    def _range(self, start: int, end: int, which: int) -> np.ndarray:
        torch = _torch()
        H, D, G = self.n_heads, self.head_dim, self._pool.group_tokens
        start, end = max(0, int(start)), min(int(end), self.length)
        if end <= start:
            return np.zeros((1, H, 0, D), dtype=np.float32)
        parts = []
        g0, g1 = start // G, min(self._pool.n_groups(0), (end + G - 1) // G)
        if g1 > g0 and start < self.cold_length:
            kk, vv = self._pool.dequant_groups([(0, g) for g in range(g0, g1)])
            rec = (kk if which == 0 else vv).permute(1, 0, 2, 3).reshape(H, (g1 - g0) * G, D)
            lo = start - g0 * G
            hi = min(end, g1 * G) - g0 * G
            parts.append(rec[:, lo:hi])
        if end > self.cold_length:
            hk, hv = self._pool.hot_window_tokens(0)
            hot = (hk if which == 0 else hv).float()
            lo = max(start, self.cold_length) - self.cold_length
            parts.append(hot[:, lo:end - self.cold_length])
        return torch.cat(parts, dim=1)[None].cpu().numpy()

    def get_keys(self, start: int, end: int) -> np.ndarray:
        """fp32 keys ``(1, H, end-start, D)`` (turboquant_pro/core.py:1040-1056)."""
        return self._range(start, end, 0)

    def get_values(self, start: int, end: int) -> np.ndarray:
        """fp32 values ``(1, H, end-start, D)`` (turboquant_pro/core.py:1058-1073)."""
        return self._range(start, end, 1)

    # --------------------------------------------------------------- decode --
    def fused_decode(self, query, method: str = "warp"):
        """One decode step over the whole cache: ``(Hq, D)`` or ``(1, Hq, 1, D)``
        query -> ``(Hq, D)`` fp32 output (turboquant_pro/core.py:1168-1265).
        Returns NumPy for NumPy input, a device tensor for tensor input."""
        torch = _torch()
        if self.length == 0:
            raise RuntimeError("cache is empty")
        is_np = not isinstance(query, torch.Tensor)
        q = query if not is_np else torch.from_numpy(np.asarray(query))
        # an fp32 cache takes the query in fp32; an fp16 cache rounds it to fp16
        q = q.reshape(self.n_q_heads, self.head_dim).to(device=self._device, dtype=self._pool.dtype)
        out = self._pool.decode(q[None].contiguous())[0]
        return out.cpu().numpy() if is_np else out

    def fused_decode_partials(self, query):
        """Unnormalised ``(m (Hq,), l (Hq,), acc (Hq, D))`` of one step, mergeable
        with :func:`merge_partials`."""
        torch = _torch()
        q = torch.as_tensor(np.asarray(query) if not isinstance(query, torch.Tensor) else query)
        q = q.reshape(self.n_q_heads, self.head_dim).to(device=self._device, dtype=self._pool.dtype)
        m, l_, acc = self._pool.decode_partials(q[None].contiguous())
        return m[0], l_[0], acc[0]

    # ---------------------------------------------------------------- stats --
    def memory_stats(self) -> dict[str, float]:
        """Byte accounting in the reference's container terms
        (turboquant_pro/core.py:1267-1295); hot tokens are held in the
        cache's input dtype (fp16 or fp32)."""
        H, D, G = self.n_heads, self.head_dim, self._pool.group_tokens
        ng = self._pool.n_groups(0)
        n_out = int(self._pool.ocount[:ng, :, -1].sum().item()) if ng else 0
        # stored zero point: every channel, the DC channels ("sparse") or none ("bias")
        zp_ch = {"calibrated": D, "bias": 0}.get(self.key_zero_point, None)
        if zp_ch is None:
            zp_ch = int(self._pool.dc_mask.sum())
        if self.key_grid == "polar":
            # CompressedKV: packed codes + one f32 norm per token and head
            key_bytes = ng * (-(-H * G * D * self.key_bits // 8) + H * G * 4)
        else:
            key_bytes = ng * (H * G * D * self.key_bits // 8 + H * D * 4 + H * zp_ch * 4) + n_out * 6
        val_bytes = ng * (H * G * D * self.value_bits // 8 + H * G * 4)
        cold = float(key_bytes + val_bytes)
        hot = float(self.hot_length * H * D * 2 * self._pool.hot_k.element_size())
        unc = float(self.length * H * D * 4 * 2)
        return {"cold_bytes": cold, "hot_bytes": hot, "total_bytes": cold + hot,
                "uncompressed_equivalent_bytes": unc,
                "effective_ratio": unc / max(cold + hot, 1.0)}

    def clear(self) -> None:
        """Reset to empty (turboquant_pro/core.py:1297-1307)."""
        self._pool.reset()

    @property
    def pool(self) -> TQKVPool:
        return self._pool

    def n_groups(self) -> int:
        return n_groups_for(self.length, self.hot_window)
