"""Connector records produced on the GPU are the reference's bytes.

The gfx950 ``per_channel`` (asym-NF4, 2 % outliers) and ``polar`` (3-bit,
seed 0) plugins compress the fixture's keys and values; the record blob
(``tqp-kv-npz/1``, turboquant_pro/connectors/vllm_v1.py:118-143) equals the
blob the reference's ``_rec_to_blob`` wrote for the same inputs
(tests/golden/connector_blob.npz), unpacked and packed.  The block store's
``save`` (default configuration, a 3-D layer block as vLLM hands it over)
exports that same blob; ``load`` returns the oracle's dequantization; and a
record adopted from the reference's blob loads to the same arrays.
"""

import hashlib
import os

import numpy as np
import pytest

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def _gold():
    z = np.load(os.path.join(GOLD, "connector_blob.npz"), allow_pickle=False)
    return z["k"], z["v"], {t: z[f"blob_{t}"].tobytes() for t in ("default", "packed")}


def _oracle_kv(k, v):
    g = O.encode_keys(k, 0.02)
    pi, pi_t = O.rotation(0, 128)
    cent, bnd = O.polar_codebook(3, 128)
    return O.decode_keys(g), O.decode_values(O.encode_values(v, pi_t, bnd, 3), cent, pi)


@pytest.mark.parametrize("packed", [False, True])
def test_gpu_record_blob_is_reference_blob(packed):
    print(f"[connector] plugin record blob packed={packed}", flush=True)
    from turboquant_pro_amd import plugins as PL
    from turboquant_pro_amd.connectors import BlockRecord, rec_to_blob
    k, v, blobs = _gold()
    H, S, D = k.shape
    kq = PL.create("per_channel", head_dim=D, n_heads=H, nf4_asym=True, outlier_frac=0.02)
    vq = PL.create("polar", head_dim=D, n_heads=H, bits=3, seed=0)
    kw = {"packed": True} if packed else {}
    rec = BlockRecord(key_payload=kq.compress(k[None], **kw), value_payload=vq.compress(v[None], **kw),
                      shape=(H, S, D), dtype="float32", num_tokens=S, head_dim=D, n_heads=H)
    assert rec_to_blob(rec) == blobs["packed" if packed else "default"]


def test_store_save_export_load():
    print("[connector] store save / export / load", flush=True)
    from turboquant_pro_amd.connectors import (ENCODER_VERSION, KVIdentityProfile,
                                               TurboQuantBlockStore)
    k, v, blobs = _gold()
    st = TurboQuantBlockStore()
    st.save("req", "model.layers.0.attn", torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    assert st.matched_tokens("req") == 200
    prof = KVIdentityProfile(
        model_repo="org/model", model_revision="abc123", weight_fingerprint="wf0",
        tokenizer_fingerprint="tf0", architecture="LlamaForCausalLM", adapter_identity="",
        rope={"theta": 500000.0}, attention_backend="tqk-gfx950", kv_layout_version="tqk-paged/1",
        sliding_window=0, n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, tp_size=1,
        pp_size=1, kv_dtype="auto", block_size=16, quant=st.quant_descriptor(),
        encoder_version=ENCODER_VERSION)
    st.profile = prof
    state = st.export_state()
    item = state["records"]["req\x00model.layers.0.attn"]
    assert item["blob"] == blobs["default"]
    assert item["sha256"] == hashlib.sha256(blobs["default"]).hexdigest()
    kk, vv = st.load("req", "model.layers.0.attn")
    ok, ov = _oracle_kv(k, v)
    assert kk.shape == k.shape and np.array_equal(kk, ok) and np.array_equal(vv, ov)
    # the reference's packed blob, adopted, loads to the same arrays
    other = TurboQuantBlockStore(profile=prof)
    assert other.import_state({**state, "records": {"r\x00l": {
        "blob": blobs["packed"], "sha256": hashlib.sha256(blobs["packed"]).hexdigest()}}}) == 1
    k2, v2 = other.load("r", "l")
    assert np.array_equal(k2, ok) and np.array_equal(v2, ov)
    # an undecodable record (its code bytes cut short) is a miss, and is dropped
    rec = other.record("r", "l")
    rec.key_payload.indices = np.asarray(rec.key_payload.indices).reshape(-1)[:10]
    assert other.load("r", "l") is None and other.record("r", "l") is None
