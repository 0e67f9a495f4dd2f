"""Write the golden vectors for the KV connector's record format.

Run once, in the build container only (the reference tree does not exist on
the GPU box):

    python tests/golden/make_connector_golden.py /path/to/reference

The reference pins its record codec (``tqp-kv-npz/1``,
turboquant_pro/connectors/vllm_v1.py:66-198) and its identity digest
(``tqp-kv-identity/1``, turboquant_pro/connectors/identity.py:45-238) only by
self-consistency tests (tests/test_connector_beta.py,
tests/test_kv_identity.py), so this script drives the reference's own codec
and profile on small seeded inputs and stores the inputs and the outputs:

* ``connector_blob.npz``: fp32 keys/values ``(2, 200, 128)`` (exact fp16
  values), and the record blobs the reference writes for them with the
  ``per_channel`` (asym-NF4, 2 % outliers) and ``polar`` (3-bit, seed 0)
  plugins, unpacked (the block store's default call) and packed;
* ``connector_identity.npz``: one complete profile's fields (JSON), its
  digest, the prefix-block hashes of a token list, and the digest of an
  incomplete profile.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def main(ref: str) -> None:
    sys.path.insert(0, ref)
    from turboquant_pro.connectors import identity as I
    from turboquant_pro.connectors import vllm_v1 as V
    from turboquant_pro.plugins import create

    rng = np.random.default_rng(2024)
    H, S, D = 2, 200, 128
    scale = rng.lognormal(0.0, 1.0, size=(H, 1, D)).astype(np.float32)
    k = (rng.standard_normal((H, S, D)).astype(np.float32) * scale).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((H, S, D)).astype(np.float16).astype(np.float32)
    kq = create("per_channel", head_dim=D, n_heads=H, nf4_asym=True, outlier_frac=0.02)
    vq = create("polar", head_dim=D, n_heads=H, bits=3, seed=0)
    out = {"k": k, "v": v}
    for tag, packed in (("default", False), ("packed", True)):
        kw = {"packed": True} if packed else {}
        rec = V._BlockRecord(key_payload=kq.compress(k[None], **kw),
                             value_payload=vq.compress(v[None], **kw),
                             shape=(H, S, D), dtype="float32", num_tokens=S, head_dim=D, n_heads=H)
        out[f"blob_{tag}"] = np.frombuffer(V._rec_to_blob(rec), dtype=np.uint8)
    np.savez_compressed(HERE / "connector_blob.npz", **out)

    fields = dict(model_repo="org/model", model_revision="abc123", weight_fingerprint="wf0",
                  tokenizer_fingerprint="tf0", architecture="LlamaForCausalLM", adapter_identity="",
                  rope={"theta": 500000.0, "scaling": None, "max_position_embeddings": 131072},
                  attention_backend="tqk-gfx950", kv_layout_version="tqk-paged/1", sliding_window=0,
                  n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, tp_size=1, pp_size=1,
                  kv_dtype="auto", block_size=16,
                  quant={"key": "per_channel", "value": "polar",
                         "key_config": {"nf4_asym": True, "outlier_frac": 0.02},
                         "value_config": {"bits": 3, "seed": 0}},
                  encoder_version="2.0.0a2")
    p = I.KVIdentityProfile(**fields)
    tokens = list(range(1000, 1040))
    hashes = I.prefix_block_hashes(p, tokens, block_size=16)
    incomplete = I.KVIdentityProfile(model_repo="org/model", n_heads=32)
    np.savez_compressed(
        HERE / "connector_identity.npz",
        fields=np.frombuffer(json.dumps(fields).encode(), dtype=np.uint8),
        digest=np.array(p.digest()), tokens=np.array(tokens, dtype=np.int64),
        hashes=np.array(hashes), incomplete_digest=np.array(incomplete.digest()),
        incomplete_unknown=np.array(sorted(incomplete.unknown_fields)))
    print("done")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
