"""HuggingFace ``transformers`` cache backed by the gfx950 KV pool, with the
decode step attending on codes.

Mirrors turboquant_pro/hf_cache.py (``TurboQuantCache``, ``TurboQuantLayer``,
``enable_turboquant_cache``; the v5 ``Cache`` / ``CacheLayerMixin``
contract).  The reference's layer returns the whole cache as dense K/V on
every ``update`` -- every cold token dequantized again at every step
(hf_cache.py:205-214).  Here each layer keeps a :class:`TQKVPool` on the
GPU (quantize-on-append in the encode kernel) and:

* a decode step (one new token) of a model whose attention implementation
  is ``"tqk_gfx950"`` (``enable_turboquant_cache`` sets it) runs the fused
  decode-on-codes kernel: ``update`` hands the attention function the layer
  instead of dense K/V, and nothing is dequantized;
* prefill, masked (padded) batches, and models on another attention
  implementation get dense K/V -- the cold groups dequantized by the GPU
  dequant kernel, bit-exact to the reference's decompress -- as in the
  reference.

Differences from the reference layer, by design of the pool: tokens leave
the hot window in groups of ``(hot_window + 1) // 2`` (the cadence of
``TurboQuantKVCache``, turboquant_pro/core.py:1015-1038) instead of
overflow-sized spills; the hot window is kept in fp16 (or fp32 with
``input_dtype="float32"``); head_dim is 64, 128 or 256; a
layer starts with room for 4096 tokens per sequence (or twice its first
chunk) and doubles on demand, moving its codes, up to ``max_cache_len`` (else
the model config's ``max_position_embeddings``) as a bound only.
``crop``/``reorder_cache``/batch edits re-ingest dense K/V, as the reference
does (hf_cache.py:247-299).
"""

from __future__ import annotations

from functools import partial

try:
    import torch
    from transformers.cache_utils import Cache, CacheLayerMixin
    _HAS_TRANSFORMERS = True
except Exception:  # pragma: no cover - exercised only without transformers
    torch = None
    _HAS_TRANSFORMERS = False

    class Cache:  # type: ignore[no-redef]
        pass

    class CacheLayerMixin:  # type: ignore[no-redef]
        pass

__all__ = ["TurboQuantCache", "TurboQuantLayer", "enable_turboquant_cache", "tqk_attention",
           "ATTN_IMPLEMENTATION"]

ATTN_IMPLEMENTATION = "tqk_gfx950"
# first allocation per layer, in tokens per sequence; layers grow by doubling
_INITIAL_CAPACITY = 4096


class TurboQuantLayer(CacheLayerMixin):
    """One layer's two-tier cache on the GPU (hf_cache.py:73-120)."""

    is_compileable = False
    is_sliding = False

    def __init__(self, hot_window: int = 512, key_bits: int = 4, value_bits: int = 4,
                 outlier_frac: float = 0.02, seed: int = 0, n_q_heads: int | None = None,
                 max_cache_len: int | None = None, fused_decode: bool = False,
                 input_dtype: str = "float16") -> None:
        super().__init__()
        if hot_window < 1:
            raise ValueError("hot_window must be >= 1")
        self.hot_window, self.key_bits, self.value_bits = int(hot_window), int(key_bits), int(value_bits)
        self.outlier_frac, self.seed = float(outlier_frac), int(seed)
        self.n_q_heads = n_q_heads
        self.max_cache_len = max_cache_len
        self.fused_decode = bool(fused_decode)
        # "float16": states rounded to fp16 (the MFMA decode); "float32": kept
        # exactly (bf16 and fp32 models; codes the reference's, VALU decode)
        self.input_dtype = input_dtype
        self.pool = None
        self.head_dim = self.n_kv_heads = self.batch = None

    # ------------------------------------------------------------ lifecycle
    def lazy_initialization(self, key_states, value_states) -> None:
        from .pool import TQKVPool
        self.dtype, self.device = key_states.dtype, key_states.device
        b, h, _, d = key_states.shape
        self.batch, self.n_kv_heads, self.head_dim = int(b), int(h), int(d)
        # start small and grow on demand (max_cache_len is an upper bound only)
        first = int(key_states.shape[-2])
        cap = max(_INITIAL_CAPACITY, 2 * first)
        if self.max_cache_len:
            cap = min(cap, int(self.max_cache_len))
        self.pool = TQKVPool(
            n_kv_heads=self.n_kv_heads, n_q_heads=self.n_q_heads or self.n_kv_heads,
            head_dim=self.head_dim, max_batch=self.batch, max_seq_len=max(cap, first),
            hot_window=self.hot_window, key_bits=self.key_bits, value_bits=self.value_bits,
            outlier_frac=self.outlier_frac, seed=self.seed, device=self.device,
            input_dtype=self.input_dtype)
        self.is_initialized = True

    def _ingest(self, key_states, value_states) -> None:
        n = int(key_states.shape[-2])
        if n == 0:
            return
        if tuple(key_states.shape[:2]) != (self.batch, self.n_kv_heads):
            raise ValueError(f"cache layer holds (batch, kv heads) = ({self.batch}, {self.n_kv_heads}); "
                             f"got {tuple(key_states.shape[:2])}")
        need = self.get_seq_length() + n
        if need > self.pool.max_seq_len:
            if self.max_cache_len and need > int(self.max_cache_len):
                raise ValueError(f"sequence length {need} exceeds max_cache_len={self.max_cache_len}")
            cap = max(need, 2 * self.pool.max_seq_len)
            if self.max_cache_len:
                cap = min(cap, int(self.max_cache_len))
            self.pool = self.pool.grown(cap)
        self.pool.append(key_states.to(self.pool.dtype).contiguous(),
                         value_states.to(self.pool.dtype).contiguous())

    def update(self, key_states, value_states, *args, **kwargs):
        """Append the new tokens; return dense K/V, or for a fused decode step
        empty K/V tagged with this layer (read by :func:`tqk_attention`)."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self._ingest(key_states, value_states)
        if self.fused_decode and int(key_states.shape[-2]) == 1:
            k = key_states.new_empty((self.batch, self.n_kv_heads, 0, self.head_dim))
            v = value_states.new_empty((self.batch, self.n_kv_heads, 0, self.head_dim))
            k._tq_layer = self
            v._tq_layer = self
            return k, v
        return self.dense()

    def dense(self, dtype=None):
        """The whole cache as dense ``(B, H, L, D)`` K/V in ``dtype`` (the model
        dtype by default): coded groups through the GPU dequant (fp32), then
        the hot window."""
        pool = self.pool
        B, H, D, G = self.batch, self.n_kv_heads, self.head_dim, pool.group_tokens
        ng = pool.n_groups(0)
        keys, values = [], []
        if ng:
            kk, vv = pool.dequant_groups([(b, g) for b in range(B) for g in range(ng)])
            keys.append(kk.view(B, ng, H, G, D).permute(0, 2, 1, 3, 4).reshape(B, H, ng * G, D))
            values.append(vv.view(B, ng, H, G, D).permute(0, 2, 1, 3, 4).reshape(B, H, ng * G, D))
        hot = [pool.hot_window_tokens(b) for b in range(B)]
        keys.append(torch.stack([h[0] for h in hot]).float())
        values.append(torch.stack([h[1] for h in hot]).float())
        dt = self.dtype if dtype is None else dtype
        return torch.cat(keys, dim=2).to(dt), torch.cat(values, dim=2).to(dt)

    def decode(self, query, scaling: float):
        """Fused decode of one query token per sequence: ``(B, Hq, 1, D)`` ->
        ``(B, Hq, D)`` fp32, attending on codes."""
        pool = self.pool
        if query.shape[1] != pool.n_q_heads:
            raise ValueError(f"the layer's pool serves {pool.n_q_heads} query heads, "
                             f"got {query.shape[1]} (pass the model config)")
        pool.desc.sm_scale = float(scaling)
        return pool.decode(query[:, :, 0].to(pool.dtype).contiguous())

    # ------------------------------------------------------------ contract
    def get_seq_length(self) -> int:
        return self.pool.lengths[0] if self.is_initialized else 0

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_max_cache_shape(self) -> int:
        return -1

    def get_max_length(self) -> int:
        # grows like a dynamic layer (its capacity is an allocation bound only)
        return -1

    def reset(self) -> None:
        if self.is_initialized:
            self.pool.reset()

    def _reload(self, keys, values) -> None:
        """Drop all state and re-ingest dense K/V (hf_cache.py:258-269)."""
        if int(keys.shape[0]) != self.batch:
            self.batch = int(keys.shape[0])
            self.is_initialized = False
            self.lazy_initialization(keys, values)
        else:
            self.pool.reset()
        self._ingest(keys, values)

    def crop(self, max_length: int) -> None:
        if not self.is_initialized:
            return
        n = self.get_seq_length()
        if max_length < 0:
            max_length = n - abs(max_length)
        if n <= max_length:
            return
        keys, values = self.dense()
        self._reload(keys[:, :, :max_length], values[:, :, :max_length])

    def reorder_cache(self, beam_idx) -> None:
        if not self.is_initialized or self.get_seq_length() == 0:
            return
        keys, values = self.dense()
        idx = beam_idx.to(keys.device)
        self._reload(keys.index_select(0, idx), values.index_select(0, idx))

    def batch_repeat_interleave(self, repeats: int) -> None:
        if not self.is_initialized or self.get_seq_length() == 0:
            return
        keys, values = self.dense()
        self._reload(keys.repeat_interleave(repeats, dim=0), values.repeat_interleave(repeats, dim=0))

    def batch_select_indices(self, indices) -> None:
        if not self.is_initialized or self.get_seq_length() == 0:
            return
        keys, values = self.dense()
        self._reload(keys[indices, ...], values[indices, ...])

    def offload(self) -> None:  # the pool stays in HBM
        pass

    def prefetch(self) -> None:
        pass


def _mask_is_trivial(mask, kv_len: int) -> bool:
    """True when ``mask`` lets every query attend every cached token."""
    if mask is None:
        return True
    m = mask[..., -kv_len:]
    if m.dtype == torch.bool:
        return bool(m.all())
    return bool((m == 0).all())


def tqk_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                  scaling: float | None = None, **kwargs):
    """Attention function registered as ``"tqk_gfx950"``: a decode step on a
    :class:`TurboQuantLayer` runs the fused kernel; anything else (prefill,
    padded batches, dropout, dense K/V) runs PyTorch SDPA on dense K/V."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    layer = getattr(key, "_tq_layer", None)
    if layer is not None:
        sc = float(scaling) if scaling is not None else layer.head_dim ** -0.5
        if (query.shape[2] == 1 and dropout == 0.0
                and _mask_is_trivial(attention_mask, layer.get_seq_length())):
            out = layer.decode(query, sc)                       # (B, Hq, D) fp32
            return out.to(query.dtype)[:, None], None            # (B, 1, Hq, D)
        key, value = layer.dense()
    return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                  scaling=scaling, **kwargs)


def _register() -> None:
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    AttentionInterface.register(ATTN_IMPLEMENTATION, tqk_attention)
    AttentionMaskInterface.register(ATTN_IMPLEMENTATION, sdpa_mask)


class TurboQuantCache(Cache):
    """Drop-in ``transformers`` cache (hf_cache.py:302-348): one
    :class:`TurboQuantLayer` per model layer.  ``config`` (the model config)
    gives the query-head count the fused decode needs and the default
    capacity; ``fused_decode`` routes decode steps to the kernel and needs the
    model's attention implementation to be ``"tqk_gfx950"``; ``input_dtype``
    "float32" keeps bf16/fp32 states exact (the reference's codes) instead
    of rounding them to fp16."""

    def __init__(self, hot_window: int = 512, key_bits: int = 4, value_bits: int = 4,
                 outlier_frac: float = 0.02, seed: int = 0, *, config=None,
                 max_cache_len: int | None = None, fused_decode: bool = False,
                 input_dtype: str = "float16") -> None:
        if not _HAS_TRANSFORMERS:  # pragma: no cover - dependency guard
            raise ImportError("TurboQuantCache requires transformers (v5+) and torch")
        self.hot_window, self.key_bits, self.value_bits = int(hot_window), int(key_bits), int(value_bits)
        self.outlier_frac, self.seed = float(outlier_frac), int(seed)
        n_q = getattr(config, "num_attention_heads", None) if config is not None else None
        if max_cache_len is None and config is not None:
            max_cache_len = getattr(config, "max_position_embeddings", None)
        if fused_decode:
            _register()
        super().__init__(layer_class_to_replicate=partial(
            TurboQuantLayer, hot_window=self.hot_window, key_bits=self.key_bits,
            value_bits=self.value_bits, outlier_frac=self.outlier_frac, seed=self.seed,
            n_q_heads=n_q, max_cache_len=max_cache_len, fused_decode=fused_decode,
            input_dtype=input_dtype))


def enable_turboquant_cache(model, **kwargs):
    """Make ``model.generate`` use a fused-decode :class:`TurboQuantCache`
    whenever no cache is passed, and switch the model's attention to
    ``"tqk_gfx950"`` (SDPA for everything but fused decode steps).  Returns the
    model (hf_cache.py:351-371)."""
    if not _HAS_TRANSFORMERS:  # pragma: no cover - dependency guard
        raise ImportError("enable_turboquant_cache requires transformers and torch")
    _register()
    model.set_attn_implementation(ATTN_IMPLEMENTATION)
    model._turboquant_cache_kwargs = dict(kwargs)
    if getattr(model, "_turboquant_generate_patched", False):
        return model
    original_generate = model.generate

    def generate(*args, **gen_kwargs):
        if gen_kwargs.get("use_cache", True) and gen_kwargs.get("past_key_values") is None:
            gen_kwargs["past_key_values"] = TurboQuantCache(
                config=model.config, fused_decode=True, **model._turboquant_cache_kwargs)
        return original_generate(*args, **gen_kwargs)

    model.generate = generate
    model._turboquant_generate_patched = True
    return model
