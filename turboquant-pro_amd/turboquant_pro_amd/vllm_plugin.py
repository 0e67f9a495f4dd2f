"""Multi-layer KV cache manager and its vLLM-style backend wrapper, over the
gfx950 ``TurboQuantKVCache``.

Same classes, methods and return conventions as the reference's
``turboquant_pro/vllm_plugin.py``: :class:`TurboQuantKVManager` keeps one
two-tier cache per transformer layer (``store`` appends one token's K/V to a
layer, ``load`` reconstructs a token range, ``memory_stats`` /
``layer_stats`` / ``estimate_capacity`` account for them) and
:class:`TurboQuantKVBackend` wraps a manager for a model once its shape is
known.  Each layer's cache is the GPU cache built with the constructor's
arguments, so a layer's coded groups are bit-exact to the reference's for the
same configuration and fp16-valued input (the reference's default, 3-bit
uniform keys and values, and PolarQuant keys with ``per_channel_keys=False``
included); configurations the GPU cache has no form for (quantile keys,
PolarQuant keys of another width than the values) raise
``NotImplementedError`` at construction.  ``fused_decode`` runs one layer's
decode step on codes.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass

import numpy as np

from .core import TurboQuantKVCache

logger = logging.getLogger(__name__)

__all__ = ["LayerStats", "TurboQuantKVManager", "TurboQuantKVBackend"]


@dataclass
class LayerStats:
    """One layer's cache statistics (turboquant_pro/vllm_plugin.py:49-61)."""

    layer_id: int
    length: int
    cold_length: int
    hot_length: int
    cold_bytes: int
    hot_bytes: int
    total_bytes: int
    uncompressed_bytes: int
    compression_ratio: float


class TurboQuantKVManager:
    """Per-layer GPU caches of a whole model (turboquant_pro/vllm_plugin.py:64-269).

    The reference's arguments, plus the GPU cache's own keywords passed
    through to every layer (``key_nf4_asym``, ``key_outlier_frac``, ``seed``,
    ``n_q_heads``, ``capacity``, ...)."""

    def __init__(self, n_layers: int = 32, n_kv_heads: int = 8, head_dim: int = 128, bits: int = 3,
                 key_bits: int | None = None, value_bits: int | None = None, hot_window: int = 512,
                 use_gpu: bool = False, device_id: int = 0, **cache_kwargs) -> None:
        self._n_layers = n_layers
        self._n_kv_heads = n_kv_heads
        self._head_dim = head_dim
        self._bits = bits
        self._key_bits = key_bits if key_bits is not None else bits
        self._value_bits = value_bits if value_bits is not None else bits
        self._hot_window = hot_window
        self._caches = [TurboQuantKVCache(head_dim=head_dim, n_heads=n_kv_heads, bits=bits,
                                          key_bits=key_bits, value_bits=value_bits,
                                          hot_window=hot_window, use_gpu=use_gpu,
                                          device_id=device_id, **cache_kwargs)
                        for _ in range(n_layers)]
        logger.info("TurboQuantKVManager: %d layers, %d heads, %d head_dim, bits=%d (key=%d, value=%d), "
                    "hot_window=%d", n_layers, n_kv_heads, head_dim, bits, self._key_bits,
                    self._value_bits, hot_window)

    @property
    def n_layers(self) -> int:
        return self._n_layers

    def cache(self, layer_id: int) -> TurboQuantKVCache:
        """The GPU cache of one layer."""
        return self._caches[layer_id]

    def store(self, layer_id: int, keys, values) -> None:
        """Append one token's K/V ``(n_kv_heads, head_dim)`` or
        ``(1, n_kv_heads, 1, head_dim)`` to a layer (several tokens
        ``(n_kv_heads, n, head_dim)`` at once are appended in order)."""
        self._caches[layer_id].extend(keys, values)

    def load(self, layer_id: int, start: int = 0, end: int | None = None):
        """``(keys, values)`` fp32 ``(1, n_kv_heads, end - start, head_dim)`` of a
        layer, coded groups reconstructed on the GPU."""
        cache = self._caches[layer_id]
        if end is None:
            end = cache.length
        return cache.get_keys(start, end), cache.get_values(start, end)

    def fused_decode(self, layer_id: int, query):
        """One decode step of a layer over its whole cache, on codes."""
        return self._caches[layer_id].fused_decode(query)

    def length(self, layer_id: int = 0) -> int:
        return self._caches[layer_id].length

    def clear(self) -> None:
        for cache in self._caches:
            cache.clear()

    def layer_stats(self, layer_id: int) -> LayerStats:
        cache = self._caches[layer_id]
        st = cache.memory_stats()
        uncompressed = cache.length * self._n_kv_heads * self._head_dim * 4 * 2
        return LayerStats(layer_id=layer_id, length=cache.length, cold_length=cache.cold_length,
                          hot_length=cache.hot_length, cold_bytes=st["cold_bytes"],
                          hot_bytes=st["hot_bytes"], total_bytes=st["total_bytes"],
                          uncompressed_bytes=uncompressed,
                          compression_ratio=st.get("effective_ratio", 1.0))

    def memory_stats(self) -> dict:
        cold = hot = unc = tokens = 0
        for i in range(self._n_layers):
            ls = self.layer_stats(i)
            cold += ls.cold_bytes
            hot += ls.hot_bytes
            unc += ls.uncompressed_bytes
            tokens = max(tokens, ls.length)
        total = cold + hot
        ratio = unc / max(total, 1) if total > 0 else 1.0
        return {"n_layers": self._n_layers, "total_tokens": tokens, "cold_bytes": cold,
                "hot_bytes": hot, "total_bytes": total, "total_mb": round(total / 1048576, 1),
                "uncompressed_bytes": unc, "uncompressed_mb": round(unc / 1048576, 1),
                "compression_ratio": round(ratio, 1),
                "saved_mb": round((unc - total) / 1048576, 1), "bits": self._bits,
                "hot_window": self._hot_window}

    def estimate_capacity(self, max_memory_gb: float) -> int:
        """Context length a memory budget holds, with the reference's estimate
        (turboquant_pro/vllm_plugin.py:237-269): the hot window at fp32, the
        rest at the bit width's approximate compression ratio."""
        per_token_hot = self._n_layers * self._n_kv_heads * self._head_dim * 4 * 2
        approx_ratio = {2: 7.5, 3: 5.1, 4: 3.9}.get(self._bits, 5.0)
        per_token_cold = per_token_hot / approx_ratio
        remaining = max_memory_gb * 1073741824 - self._hot_window * per_token_hot
        if remaining <= 0:
            return self._hot_window
        return self._hot_window + int(remaining / per_token_cold)


class TurboQuantKVBackend:
    """vLLM-style backend over a :class:`TurboQuantKVManager`
    (turboquant_pro/vllm_plugin.py:277-343)."""

    def __init__(self, bits: int = 3, hot_window: int = 512, **manager_kwargs) -> None:
        self._bits = bits
        self._hot_window = hot_window
        self._manager_kwargs = manager_kwargs
        self._manager: TurboQuantKVManager | None = None

    def initialize(self, n_layers: int, n_kv_heads: int, head_dim: int, **kwargs) -> None:
        self._manager = TurboQuantKVManager(n_layers=n_layers, n_kv_heads=n_kv_heads,
                                            head_dim=head_dim, bits=self._bits,
                                            hot_window=self._hot_window,
                                            **{**self._manager_kwargs, **kwargs})

    def store_block(self, layer_id: int, keys, values) -> None:
        if self._manager is None:
            raise RuntimeError("Backend not initialized")
        self._manager.store(layer_id, keys, values)

    def load_block(self, layer_id: int, start: int = 0, end: int | None = None):
        if self._manager is None:
            raise RuntimeError("Backend not initialized")
        return self._manager.load(layer_id, start, end)

    def memory_stats(self) -> dict:
        return {} if self._manager is None else self._manager.memory_stats()

    def supports_async(self) -> bool:
        return False
