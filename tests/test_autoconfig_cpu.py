"""AutoConfig resolution, mirroring the reference's own cases
(tests/test_autoconfig.py:21-129 of the reference): dict keys, presets,
overrides, registry, aliases, and the errors."""

import pytest

from turboquant_pro_amd import AutoConfig, list_models, list_targets


def test_basic_dict():
    cfg = AutoConfig.from_dict({"head_dim": 128, "num_key_value_heads": 8, "num_hidden_layers": 32})
    assert (cfg.head_dim, cfg.n_kv_heads, cfg.n_layers) == (128, 8, 32)


def test_infer_head_dim_from_hidden_size():
    assert AutoConfig.from_dict({"hidden_size": 4096, "num_attention_heads": 32}).head_dim == 128


@pytest.mark.parametrize("target,kb,vb,rope", [
    ("quality", 4, 4, True), ("balanced", 4, 3, True),
    ("compression", 4, 2, True), ("extreme", 2, 2, False)])
def test_targets(target, kb, vb, rope):
    cfg = AutoConfig.from_dict({"head_dim": 128}, target=target)
    assert (cfg.key_bits, cfg.value_bits, cfg.rope_aware) == (kb, vb, rope)


def test_invalid_target_raises():
    with pytest.raises(ValueError, match="Unknown target"):
        AutoConfig.from_dict({"head_dim": 128}, target="turbo")


def test_overrides():
    cfg = AutoConfig.from_dict({"head_dim": 128}, target="balanced", key_bits=3, rope_aware=False)
    assert (cfg.key_bits, cfg.value_bits, cfg.rope_aware) == (3, 3, False)


def test_rope_theta_and_max_seq_len():
    cfg = AutoConfig.from_dict({"head_dim": 128, "rope_theta": 500000.0,
                                "max_position_embeddings": 131072})
    assert cfg.rope_theta == 500000.0 and cfg.max_seq_len == 131072


def test_registry_models_and_aliases():
    cfg = AutoConfig.from_pretrained("llama-3-8b")
    assert (cfg.head_dim, cfg.n_kv_heads, cfg.n_layers, cfg.model_name) == (128, 8, 32, "llama-3-8b")
    assert cfg.n_q_heads == 32
    assert AutoConfig.from_pretrained("Llama-3-8B").head_dim == 128
    assert AutoConfig.from_pretrained("meta-llama/Llama-3-8B").model_name == "llama-3-8b"
    g = AutoConfig.from_pretrained("gemma-2-27b")
    assert (g.head_dim, g.n_kv_heads, g.n_layers) == (128, 16, 46)
    q = AutoConfig.from_pretrained("qwen2.5-7b")
    assert (q.rope_theta, q.max_seq_len) == (1000000.0, 131072)
    for m in list_models():
        c = AutoConfig.from_pretrained(m)
        assert c.head_dim > 0 and c.n_kv_heads > 0 and c.n_layers > 0
    assert set(list_targets()) == {"quality", "balanced", "compression", "extreme"}


def test_unknown_model_raises():
    with pytest.raises(ValueError, match="Could not resolve"):
        AutoConfig.from_pretrained("totally-unknown-model-xyz")


def test_zero_point_resolution():
    assert AutoConfig.from_pretrained("llama-3-8b").resolve_key_zero_point(True) == "calibrated"
    assert AutoConfig.from_pretrained("qwen2.5-7b").resolve_key_zero_point(True) == "bias"
    assert AutoConfig.from_pretrained("qwen2.5-7b").resolve_key_zero_point(False) == "calibrated"
    with pytest.raises(ValueError):
        AutoConfig(key_zero_point="bias").resolve_key_zero_point(False)
