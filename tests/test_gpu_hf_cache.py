"""The HuggingFace cache on the GPU (turboquant_pro/hf_cache.py, routed to the
fused decode kernel).

* Layer level: a ``TurboQuantLayer`` fed a 1200-token prefill and then one
  token at a time (crossing a flush) answers each decode step through the
  fused kernel within the north-star bar (max-abs 2e-3, relative 1e-2) of
  dequantize-then-attend -- the oracle's ``SequenceCache.attend`` over the
  same tokens -- and of SDPA over the layer's own dense K/V.
* Model level (a tiny fp16 GQA Llama with head_dim 128, random weights, no
  downloads): teacher-forced decode steps through ``enable_turboquant_cache``
  (fused) give the logits of the same cache read densely (the reference's
  path: SDPA over dequantized K/V), and with nothing compressed those of
  ``DynamicCache``; the fused kernel ran for every decode step; ``generate``
  runs end to end.
"""

import numpy as np
import pytest

from gpu_util import assert_attn_close
from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _sdpa_ref(q, k, v):
    """fp32 attention of q (B, Hq, D) over dense k, v (B, Hkv, L, D)."""
    B, Hq, D = q.shape
    g = Hq // k.shape[1]
    kk = k.float().repeat_interleave(g, dim=1)
    vv = v.float().repeat_interleave(g, dim=1)
    s = torch.einsum("bhd,bhld->bhl", q.float(), kk) / D ** 0.5
    return torch.einsum("bhl,bhld->bhd", torch.softmax(s, dim=-1), vv)


def test_layer_fused_decode_matches_dequant_attend():
    from turboquant_pro_amd.hf_cache import TurboQuantLayer, tqk_attention
    B, Hkv, Hq, L0, L1 = 2, 2, 8, 1200, 1290
    print(f"[hf layer] B={B} Hkv={Hkv} Hq={Hq} prefill {L0}, decode to {L1}", flush=True)
    k, v, _ = O.synthetic_kv(41, B, Hkv, Hq, L1)
    rng = np.random.default_rng(5)
    layer = TurboQuantLayer(hot_window=512, value_bits=3, n_q_heads=Hq, max_cache_len=2048,
                            fused_decode=True)
    kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    dk, dv = layer.update(kd[:, :, :L0], vd[:, :, :L0])
    assert dk.shape == (B, Hkv, L0, 128) and dk.dtype == torch.float16
    pi, pi_t = O.rotation(0, 128)
    for t in range(L0, L1):
        kt, vt = layer.update(kd[:, :, t:t + 1], vd[:, :, t:t + 1])
        assert kt.shape[2] == 0 and getattr(kt, "_tq_layer", None) is layer
        q = rng.standard_normal((B, Hq, 128)).astype(np.float16)
        qd = torch.from_numpy(q).cuda()
        out, _ = tqk_attention(None, qd[:, :, None], kt, vt, None, scaling=128 ** -0.5)
        assert out.shape == (B, 1, Hq, 128) and out.dtype == torch.float16
        got = layer.decode(qd[:, :, None], 128 ** -0.5)      # the kernel's fp32 output
        assert torch.equal(out[:, 0], got.half())
        if t in (L0, 1280, 1281, L1 - 1):     # around the flush at 1281 tokens
            dense_k, dense_v = layer.dense(torch.float32)
            want = _sdpa_ref(qd, dense_k, dense_v)
            for b in range(B):
                assert_attn_close(got[b].cpu().numpy(), want[b].cpu().numpy(), what=f"sdpa t={t} b={b}")
                sc = O.SequenceCache(hot_window=512, value_bits=3, outlier_frac=0.02).build(
                    k[b, :, :t + 1], v[b, :, :t + 1], pi, pi_t)
                assert_attn_close(got[b].cpu().numpy(), sc.attend(q[b]), what=f"oracle t={t} b={b}")
    assert layer.get_seq_length() == L1 and layer.pool.n_groups(0) == 4


def _tiny_llama():
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=128, intermediate_size=1024, vocab_size=256,
                      max_position_embeddings=2048)
    return LlamaForCausalLM(cfg).to("cuda", torch.float16).eval(), cfg


@torch.no_grad()
def _teacher_forced(model, cache, prompt, steps):
    out = model(input_ids=prompt, past_key_values=cache, use_cache=True)
    logits = [out.logits[:, -1].float()]
    for t in range(steps.shape[1]):
        out = model(input_ids=steps[:, t:t + 1], past_key_values=cache, use_cache=True)
        logits.append(out.logits[:, -1].float())
    return torch.stack(logits, 1)


def test_model_fused_decode_logits(monkeypatch):
    from transformers.cache_utils import DynamicCache
    from turboquant_pro_amd import hf_cache as HC
    model, cfg = _tiny_llama()
    HC.enable_turboquant_cache(model, hot_window=512, value_bits=4)
    calls = {"n": 0}
    real = HC.TurboQuantLayer.decode

    def counted(self, q, s):
        calls["n"] += 1
        return real(self, q, s)

    monkeypatch.setattr(HC.TurboQuantLayer, "decode", counted)
    g = torch.Generator().manual_seed(3)
    for plen in (700, 100):            # with coded groups / hot window only
        print(f"[hf model] prompt {plen}", flush=True)
        prompt = torch.randint(0, 256, (2, plen), generator=g).cuda()
        steps = torch.randint(0, 256, (2, 12), generator=g).cuda()
        calls["n"] = 0
        fused = _teacher_forced(model, HC.TurboQuantCache(hot_window=512, value_bits=4, config=cfg,
                                                          fused_decode=True), prompt, steps)
        assert calls["n"] == 12 * cfg.num_hidden_layers
        dense = _teacher_forced(model, HC.TurboQuantCache(hot_window=512, value_bits=4, config=cfg),
                                prompt, steps)
        scale = dense.abs().max().item()
        err = (fused - dense).abs().max().item()
        assert err <= 2e-2 * scale, f"prompt {plen}: fused vs dense logits {err:.3e} (scale {scale:.3e})"
        if plen < 512:
            ref = _teacher_forced(model, DynamicCache(config=cfg), prompt, steps)
            err = (fused - ref).abs().max().item()
            assert err <= 2e-2 * scale, f"hot only: fused vs DynamicCache {err:.3e}"
    out = model.generate(input_ids=prompt, max_new_tokens=8, do_sample=False)
    assert out.shape == (2, prompt.shape[1] + 8)
