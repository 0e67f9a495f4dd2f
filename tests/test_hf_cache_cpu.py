"""The HuggingFace cache module on a machine without a GPU: it imports,
builds lazily (turboquant_pro/hf_cache.py:302-348 builds layers on first
``update``), validates its arguments, and refuses to run on the CPU instead
of falling back to a CPU path."""

import pytest

torch = pytest.importorskip("torch")
pytest.importorskip("transformers")


def test_lazy_construction_and_gpu_requirement():
    from turboquant_pro_amd import hf_cache as HC
    c = HC.TurboQuantCache(hot_window=512, value_bits=4)
    assert c.hot_window == 512 and c.value_bits == 4 and c.key_bits == 4
    with pytest.raises(ValueError):
        HC.TurboQuantLayer(hot_window=0)
    layer = HC.TurboQuantLayer(hot_window=64, n_q_heads=4)
    assert layer.get_seq_length() == 0 and layer.get_mask_sizes(3) == (3, 0)
    assert layer.get_max_cache_shape() == -1
    if not torch.cuda.is_available():
        k = torch.zeros((1, 2, 4, 128), dtype=torch.float16)
        with pytest.raises(RuntimeError, match="GPU"):
            layer.update(k, k)


def test_mask_triviality():
    from turboquant_pro_amd.hf_cache import _mask_is_trivial
    assert _mask_is_trivial(None, 5)
    m = torch.ones((2, 1, 1, 7), dtype=torch.bool)
    assert _mask_is_trivial(m, 5)
    m[0, 0, 0, 3] = False
    assert not _mask_is_trivial(m, 5)
    f = torch.zeros((2, 1, 1, 7))
    assert _mask_is_trivial(f, 5)
    f[1, 0, 0, -1] = float("-inf")
    assert not _mask_is_trivial(f, 5)
