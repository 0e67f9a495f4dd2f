"""``AutoConfig`` for the gfx950 cache: the reference's parameter resolution
(turboquant_pro/autoconfig.py:175-486) with ``build_cache`` returning the
GPU-backed :class:`~turboquant_pro_amd.core.TurboQuantKVCache`.

Resolution is the reference's: HF-style config keys map to (head_dim,
n_kv_heads, n_layers, rope_theta, max_seq_len); a target preset sets
(key_bits, value_bits, rope_aware); overrides win.  ``from_pretrained`` only
resolves the built-in registry and its aliases -- this build never reaches for
the network, so an unknown name raises ``ValueError`` (the reference's own
error when neither the registry nor ``transformers`` resolves it).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass

logger = logging.getLogger(__name__)

# Model shapes of the reference registry (turboquant_pro/autoconfig.py:51-116):
# name -> (head_dim, q heads, kv heads, layers, rope_theta, max positions).
_SHAPES = {
    "llama-3-8b": (128, 32, 8, 32, 500000.0, 8192),
    "llama-3-70b": (128, 64, 8, 80, 500000.0, 8192),
    "gemma-2-27b": (128, 32, 16, 46, 10000.0, 8192),
    "gemma-2-9b": (256, 16, 8, 42, 10000.0, 8192),
    "gemma-4-27b-a4b": (256, 8, 1, 48, 10000.0, 262144),
    "qwen2.5-7b": (128, 28, 4, 28, 1000000.0, 131072),
    "qwen2.5-72b": (128, 64, 8, 80, 1000000.0, 131072),
    "mistral-7b": (128, 32, 8, 32, 10000.0, 32768),
}
MODEL_REGISTRY = {
    name: dict(head_dim=s[0], num_attention_heads=s[1], num_key_value_heads=s[2],
               num_hidden_layers=s[3], rope_theta=s[4], max_position_embeddings=s[5])
    for name, s in _SHAPES.items()
}
# HF-style names (lower case) -> registry key (turboquant_pro/autoconfig.py:119-131)
MODEL_ALIASES = {
    "meta-llama/llama-3-8b": "llama-3-8b",
    "meta-llama/meta-llama-3-8b": "llama-3-8b",
    "meta-llama/llama-3-70b": "llama-3-70b",
    "meta-llama/meta-llama-3-70b": "llama-3-70b",
    "google/gemma-2-27b": "gemma-2-27b",
    "google/gemma-2-9b": "gemma-2-9b",
    "google/gemma-4-27b-a4b": "gemma-4-27b-a4b",
    "qwen/qwen2.5-7b": "qwen2.5-7b",
    "qwen/qwen2.5-72b": "qwen2.5-72b",
    "mistralai/mistral-7b-v0.1": "mistral-7b",
    "mistralai/mistral-7b": "mistral-7b",
}
# target -> (key_bits, value_bits, rope_aware) (turboquant_pro/autoconfig.py:146-171)
TARGETS = {
    "quality": (4, 4, True),
    "balanced": (4, 3, True),
    "compression": (4, 2, True),
    "extreme": (2, 2, False),
}


@dataclass
class AutoConfig:
    """Model shape + compression target; ``build_cache`` makes the GPU cache."""

    head_dim: int = 128
    n_kv_heads: int = 8
    n_layers: int = 32
    rope_theta: float = 10000.0
    max_seq_len: int = 8192
    key_bits: int = 4
    value_bits: int = 3
    rope_aware: bool = True
    target: str = "balanced"
    model_name: str = ""
    key_zero_point: str = "auto"
    n_q_heads: int | None = None   # query heads (GQA), from num_attention_heads

    @classmethod
    def from_dict(cls, config: dict, target: str = "balanced", **overrides) -> "AutoConfig":
        """HF-style dict -> AutoConfig (turboquant_pro/autoconfig.py:216-285)."""
        if target not in TARGETS:
            raise ValueError(f"Unknown target '{target}'. Choose from: {sorted(TARGETS)}")
        kb, vb, rope = TARGETS[target]
        n_q = config.get("num_attention_heads", 32)
        head_dim = config.get("head_dim")
        if head_dim is None:
            head_dim = config.get("hidden_size", 4096) // n_q
        kwargs = dict(
            head_dim=head_dim,
            n_kv_heads=config.get("num_key_value_heads", n_q),
            n_layers=config.get("num_hidden_layers", 32),
            rope_theta=config.get("rope_theta", 10000.0),
            max_seq_len=config.get("max_position_embeddings", 8192),
            key_bits=kb, value_bits=vb, rope_aware=rope, target=target,
            model_name=config.get("model_type", ""), n_q_heads=n_q)
        kwargs.update(overrides)
        cfg = cls(**kwargs)
        logger.info("AutoConfig: %s target=%s key=%d-bit value=%d-bit head_dim=%d n_kv_heads=%d",
                    cfg.model_name or "custom", target, cfg.key_bits, cfg.value_bits,
                    cfg.head_dim, cfg.n_kv_heads)
        return cfg

    @classmethod
    def from_pretrained(cls, model_name_or_path: str, target: str = "balanced",
                        **overrides) -> "AutoConfig":
        """Registry name or alias -> AutoConfig (turboquant_pro/autoconfig.py:287-346,
        without the Hub lookup)."""
        key = model_name_or_path.lower().strip("/")
        key = MODEL_ALIASES.get(key, key)
        if key not in MODEL_REGISTRY:
            raise ValueError(
                f"Could not resolve model '{model_name_or_path}'. Known models: "
                f"{sorted(MODEL_REGISTRY)}. Pass a config dict via AutoConfig.from_dict().")
        cfg = cls.from_dict(MODEL_REGISTRY[key], target=target, **overrides)
        cfg.model_name = key
        return cfg

    @property
    def is_qwen_family(self) -> bool:
        return "qwen" in (self.model_name or "").lower()

    def resolve_key_zero_point(self, has_k_bias: bool) -> str:
        """``auto`` -> ``bias`` for Qwen with a k_proj bias, else ``calibrated``
        (turboquant_pro/autoconfig.py:374-402)."""
        mode = self.key_zero_point
        if mode == "auto":
            return "bias" if (self.is_qwen_family and has_k_bias) else "calibrated"
        if mode == "bias" and not has_k_bias:
            raise ValueError('key_zero_point="bias" requires k_bias (per-layer k_proj bias)')
        return mode

    def build_cache(self, hot_window: int = 512, use_gpu: bool = True, seed: int | None = None,
                    robust: bool = True, outlier_frac: float = 0.02, k_bias=None, *,
                    n_q_heads: int | None = None, capacity: int = 4096):
        """The GPU cache with this config's K/V bits (turboquant_pro/autoconfig.py:439-486):
        asym-NF4 keys with the resolved zero point (``bias`` needs this layer's
        ``k_bias``) + ``outlier_frac`` fp16 outliers.  ``n_q_heads`` (default:
        one query per kv-head, as the reference's cache) serves GQA queries.
        ``robust=False`` builds uniform keys at the config's key width, as the
        reference's plain per-channel cache."""
        from .core import TurboQuantKVCache
        zp = self.resolve_key_zero_point(k_bias is not None) if robust else "calibrated"
        return TurboQuantKVCache(
            head_dim=self.head_dim, n_heads=self.n_kv_heads, bits=self.value_bits,
            key_bits=self.key_bits, value_bits=self.value_bits, hot_window=hot_window,
            use_gpu=use_gpu, seed=seed, key_nf4_asym=robust,
            key_outlier_frac=outlier_frac if robust else 0.0, key_zero_point=zp,
            key_rope_theta=self.rope_theta if zp != "calibrated" else None,
            key_k_bias=k_bias if zp == "bias" else None, n_q_heads=n_q_heads, capacity=capacity)


def list_models() -> list[str]:
    """Registry names (turboquant_pro/autoconfig.py:661-663)."""
    return sorted(MODEL_REGISTRY)


def list_targets() -> dict[str, str]:
    """Target presets and their bit allocation (turboquant_pro/autoconfig.py:666-668)."""
    return {t: f"K{kb}/V{vb}" + (" + RoPE boost" if rope else "")
            for t, (kb, vb, rope) in TARGETS.items()}
