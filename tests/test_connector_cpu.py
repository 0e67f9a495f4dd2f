"""Connector formats on the CPU, against the reference's own outputs.

* Identity (turboquant_pro/connectors/identity.py): a profile with the fields
  of tests/golden/connector_identity.npz has the reference's digest, prefix
  block hashes and, when incomplete, the same digest and unknown fields;
  compatibility needs two complete profiles with equal digests; non-finite
  floats are refused.
* Record codec ``tqp-kv-npz/1`` (turboquant_pro/connectors/vllm_v1.py:66-198):
  the reference's blobs (tests/golden/connector_blob.npz, written by
  ``_rec_to_blob``) decode, re-encode to the same bytes (also through this
  build's container dataclasses), and hold the codes, stats, outliers and
  norms the oracle computes for the same inputs; unknown codecs, non-numeric
  dtypes and oversized blobs are refused (tests/test_connector_beta.py:113-135).
* Store persistence (vllm_v1.py:466-664): export/import and the directory
  layout round-trip the reference's blobs unchanged; the profile gate, the
  COMMIT marker, per-record integrity and manifest file names behave as the
  reference's tests expect (tests/test_connector_beta.py:136-220).
"""

import io
import json
import os

import numpy as np
import pytest

from oracle import tq_oracle as O
from turboquant_pro_amd import plugins as PL
from turboquant_pro_amd.connectors import (BLOB_CODEC, IncompatibleProfile, KVIdentityProfile,
                                           TurboQuantBlockStore, prefix_block_hashes, rec_from_blob,
                                           rec_to_blob)
from turboquant_pro_amd.connectors.store import STATE_SCHEMA

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _identity():
    z = np.load(os.path.join(GOLD, "connector_identity.npz"), allow_pickle=False)
    return json.loads(bytes(z["fields"]).decode()), z


def _blobs():
    z = np.load(os.path.join(GOLD, "connector_blob.npz"), allow_pickle=False)
    return z, {t: z[f"blob_{t}"].tobytes() for t in ("default", "packed")}


def _profile(**over):
    fields, _ = _identity()
    fields.update(over)
    return KVIdentityProfile(**fields)


# ------------------------------------------------------------------ identity
def test_profile_digest_and_prefix_hashes_match_reference():
    fields, z = _identity()
    p = KVIdentityProfile(**fields)
    assert p.is_complete and p.digest() == str(z["digest"])
    assert prefix_block_hashes(p, z["tokens"].tolist(), block_size=16) == z["hashes"].tolist()
    inc = KVIdentityProfile(model_repo="org/model", n_heads=32)
    assert inc.digest() == str(z["incomplete_digest"])
    assert sorted(inc.unknown_fields) == z["incomplete_unknown"].tolist()


def test_profile_compatibility_rules():
    a, b = _profile(), _profile()
    assert a.compatible(b) and a.digest() == b.digest()
    c = _profile(quant={**a.quant, "value_config": {"bits": 4, "seed": 0}})
    assert not a.compatible(c)
    with pytest.raises(IncompatibleProfile, match="mismatch"):
        a.require_compatible(c)
    inc = _profile(weight_fingerprint=None)
    assert not inc.compatible(inc)          # incomplete: compatible with nothing
    with pytest.raises(IncompatibleProfile, match="incomplete"):
        a.require_compatible(inc)
    with pytest.raises(IncompatibleProfile):
        prefix_block_hashes(inc, [1, 2, 3])
    # whole blocks only; any profile change changes every hash
    h = prefix_block_hashes(a, list(range(40)), block_size=16)
    assert len(h) == 2 and prefix_block_hashes(a, list(range(47)))[:2] == h
    assert set(prefix_block_hashes(c, list(range(40)))).isdisjoint(h)
    with pytest.raises(ValueError):
        _profile(rope={"theta": float("nan")}).digest()


# ------------------------------------------------------------------- records
@pytest.mark.parametrize("tag", ["default", "packed"])
def test_reference_blob_round_trips_byte_exact(tag):
    _, blobs = _blobs()
    blob = blobs[tag]
    rec = rec_from_blob(blob)
    assert rec.shape == (2, 200, 128) and rec.num_tokens == 200 and rec.n_heads == 2
    assert rec_to_blob(rec) == blob
    typed = rec_from_blob(blob, key_cls=PL.CompressedPerChannelKV, value_cls=PL.CompressedKV)
    assert isinstance(typed.key_payload, PL.CompressedPerChannelKV)
    assert typed.key_payload.packed == (tag == "packed") and typed.value_payload.bits == 3
    assert rec_to_blob(typed) == blob


@pytest.mark.parametrize("tag", ["default", "packed"])
def test_reference_blob_holds_oracle_codes(tag):
    z, blobs = _blobs()
    rec = rec_from_blob(blobs[tag], key_cls=PL.CompressedPerChannelKV, value_cls=PL.CompressedKV)
    k, v = z["k"], z["v"]
    g = O.encode_keys(k, 0.02)
    kp = rec.key_payload
    codes = kp.indices.reshape(-1) if not kp.packed else O.unpack_key_codes(kp.indices, k.size, 4)
    assert np.array_equal(codes.reshape(k.shape), g.codes)
    if kp.packed:
        assert np.array_equal(kp.indices, g.packed)
    assert np.array_equal(kp.nf4_scale[0], g.nf4_scale) and np.array_equal(kp.nf4_mean[0], g.nf4_mean)
    assert np.array_equal(kp.outlier_idx, g.outlier_idx)
    assert np.array_equal(kp.outlier_val.view(np.uint16), g.outlier_val.view(np.uint16))
    _, pi_t = O.rotation(0, 128)
    _, bnd = O.polar_codebook(3, 128)
    gv = O.encode_values(v, pi_t, bnd, 3)
    vp = rec.value_payload
    vc = vp.indices if not vp.packed else O.unpack_value_codes(vp.indices, v.size, 3)
    assert np.array_equal(np.asarray(vc).reshape(v.shape), gv.codes)
    assert np.array_equal(vp.norms[0], gv.norms)


def _rewrite(blob, header_edit=None, extra=None):
    with np.load(io.BytesIO(blob), allow_pickle=False) as z:
        header = json.loads(bytes(z["__header__"]).decode())
        arrays = {n: z[n] for n in z.files if n != "__header__"}
    if header_edit:
        header_edit(header)
    arrays.update(extra or {})
    out = io.BytesIO()
    np.savez(out, __header__=np.frombuffer(json.dumps(header).encode(), dtype=np.uint8), **arrays)
    return out.getvalue()


def test_blob_refusals():
    _, blobs = _blobs()
    blob = blobs["packed"]
    future = _rewrite(blob, lambda h: h.__setitem__("codec", "tqp-kv-npz/99"))
    with pytest.raises(ValueError, match="unknown record codec"):
        rec_from_blob(future)
    odd = _rewrite(blob, extra={"k.extra": np.zeros(4, np.complex64)})
    with pytest.raises(ValueError, match="whitelisted"):
        rec_from_blob(odd)
    with pytest.raises(ValueError, match="max_bytes"):
        rec_from_blob(blob, max_bytes=1000)
    # a compressed archive whose arrays expand beyond the limit (a zip bomb)
    bomb = io.BytesIO()
    header = {"codec": BLOB_CODEC, "shape": [1], "dtype": "float32", "num_tokens": 1,
              "head_dim": 1, "n_heads": 1, "key_scalars": {}, "value_scalars": {}}
    np.savez_compressed(bomb, __header__=np.frombuffer(json.dumps(header).encode(), dtype=np.uint8),
                        **{"k.indices": np.zeros(4_000_000, np.uint8)})
    assert len(bomb.getvalue()) < 100_000
    with pytest.raises(ValueError, match="max_bytes"):
        rec_from_blob(bomb.getvalue(), max_bytes=1_000_000)
    assert BLOB_CODEC == "tqp-kv-npz/1"


# ------------------------------------------------------------- persistence
def _loaded_store(profile=None):
    """A store holding the reference's two blobs (no GPU needed to adopt them)."""
    import hashlib
    _, blobs = _blobs()
    p = profile or _profile()
    st = TurboQuantBlockStore(profile=p)
    records = {f"req1\x00layer.{i}": {"blob": b, "sha256": hashlib.sha256(b).hexdigest()}
               for i, b in enumerate(blobs.values())}
    n = st.import_state({"schema": STATE_SCHEMA, "profile_digest": p.digest(), "records": records,
                         "tokens": {"req1": 200}})
    assert n == 2
    return st, blobs


def test_export_import_and_directory_round_trip(tmp_path):
    st, blobs = _loaded_store()
    assert st.matched_tokens("req1") == 200 and st.stats()["records"] == 2
    state = st.export_state()
    assert state["schema"] == STATE_SCHEMA
    assert {k: v["blob"] for k, v in state["records"].items()} == \
        {f"req1\x00layer.{i}": b for i, b in enumerate(blobs.values())}
    d = tmp_path / "store"
    assert st.save_to_dir(str(d)) == 2
    assert (d / "COMMIT").read_text() == st.profile.digest()
    recs = sorted(p.name for p in d.glob("*.rec"))
    assert len(recs) == 2 and all(len(n) == 28 for n in recs)
    assert (d / recs[0]).read_bytes()[:2] == b"PK"
    dst = TurboQuantBlockStore(profile=_profile())
    assert dst.load_from_dir(str(d)) == 2
    assert dst.export_state()["records"] == state["records"]
    assert dst.evict("req1") == 2 and dst.matched_tokens("req1") == 0


def test_persistence_gates(tmp_path):
    st, _ = _loaded_store()
    d = tmp_path / "store"
    st.save_to_dir(str(d))
    with pytest.raises(IncompatibleProfile):
        TurboQuantBlockStore(profile=_profile(model_revision="other")).load_from_dir(str(d))
    with pytest.raises(IncompatibleProfile):
        TurboQuantBlockStore(profile=_profile(weight_fingerprint=None)).load_from_dir(str(d))
    with pytest.raises(IncompatibleProfile):
        TurboQuantBlockStore().export_state()
    state = st.export_state()
    with pytest.raises(IncompatibleProfile, match="schema"):
        TurboQuantBlockStore(profile=_profile()).import_state({**state, "schema": "x"})
    # a corrupt record is skipped, the intact one loads
    key = next(iter(state["records"]))
    bad = dict(state["records"])
    bad[key] = {"blob": bad[key]["blob"][:-7] + b"garbage", "sha256": bad[key]["sha256"]}
    assert TurboQuantBlockStore(profile=_profile()).import_state({**state, "records": bad}) == 1
    # a manifest naming a path outside the store is refused
    m = json.loads((d / "manifest.json").read_text())
    m["records"][key]["file"] = "..\\..\\evil.rec"
    (d / "manifest.json").write_text(json.dumps(m))
    assert TurboQuantBlockStore(profile=_profile()).load_from_dir(str(d)) == 1
    # no COMMIT marker: the directory is invisible
    os.remove(d / "COMMIT")
    with pytest.raises(IncompatibleProfile, match="COMMIT"):
        TurboQuantBlockStore(profile=_profile()).load_from_dir(str(d))


def test_quant_descriptor_names_the_bytes():
    st = TurboQuantBlockStore()
    q = st.quant_descriptor()
    assert q == {"key": "per_channel", "value": "polar",
                 "key_config": {"nf4_asym": True, "outlier_frac": 0.02},
                 "value_config": {"bits": 3, "seed": 0}}
    fields, _ = _identity()
    assert fields["quant"] == q      # the golden profile describes this store's default


def test_connector_protocol_host_side():
    """Scheduler-side answers and eviction of the connector (vllm_v1.py:750-814),
    over a store holding the reference's records; without vLLM, ``register``
    reports False instead of failing."""
    from turboquant_pro_amd.connectors import TurboQuantKVConnector
    from turboquant_pro_amd.connectors.vllm import TurboQuantConnectorMetadata, register
    st, _ = _loaded_store()
    conn = TurboQuantKVConnector(store=st)
    req = type("Req", (), {"request_id": "req1"})()
    assert conn.get_num_new_matched_tokens(req, 0) == (200, False)
    assert conn.get_num_new_matched_tokens(req, 150) == (50, False)
    assert conn.get_num_new_matched_tokens(req, 500) == (0, False)
    meta = conn.build_connector_meta()
    assert isinstance(meta, TurboQuantConnectorMetadata) and meta.loads == []
    assert conn.request_finished(req) == (False, None)
    conn.bind_connector_metadata(TurboQuantConnectorMetadata(loads=[("req1", 0, 200)]))
    assert conn.start_load_kv(None) == 0      # no pool bound: nothing to restore into
    conn.get_finished({"req1"})
    assert st.matched_tokens("req1") == 0 and st.stats()["records"] == 0
    m = conn.get_metrics()
    assert m["evictions"] == st.metrics.to_dict()["evictions"] > 0
    assert register() is False


class _RecordingStore:
    """A store stand-in for the connector's metadata flow: what the worker
    was asked to restore, where."""

    def __init__(self, tokens):
        from turboquant_pro_amd.connectors.metrics import ConnectorMetrics
        self.tokens, self.calls, self.metrics = dict(tokens), [], ConnectorMetrics()

    def matched_tokens(self, rid):
        return self.tokens.get(rid, 0)

    def load_into_pool(self, rid, layer, pool, slot):
        self.calls.append((rid, layer, pool, slot))
        return self.tokens.get(rid, 0)

    def evict(self, rid):
        return int(self.tokens.pop(rid, None) is not None)


def _metadata_round(mod):
    """Scheduler -> metadata -> worker, as vLLM V1 drives a connector: the
    scheduler instance answers the match, takes the allocation of requests
    that load, and builds the step's metadata; the worker instance is bound
    to it and restores each request into its slot of every bound pool."""
    store = _RecordingStore({"a": 600, "b": 1300, "c": 40})
    sched = mod.TurboQuantKVConnector(role=mod.KVConnectorRole.SCHEDULER, store=store)
    work = mod.TurboQuantKVConnector(role=mod.KVConnectorRole.WORKER, store=store)
    pools = {"layers.0.attn": object(), "layers.1.attn": object()}
    for name, p in pools.items():
        work.bind_pool(name, p)
    reqs = {r: type("Req", (), {"request_id": r})() for r in "abcd"}
    for r, computed in (("a", 0), ("b", 256), ("c", 40), ("d", 0)):
        n, pending = sched.get_num_new_matched_tokens(reqs[r], computed)
        assert not pending
        sched.update_state_after_alloc(reqs[r], [], n)
    meta = sched.build_connector_meta()
    assert isinstance(meta, mod.TurboQuantConnectorMetadata)
    # only the requests with tokens to take from the store load, in order,
    # each in its own slot
    assert meta.loads == [("a", 0, 600), ("b", 1, 1044)]
    assert sched.build_connector_meta().loads == []      # handed over once
    work.bind_connector_metadata(meta)
    assert work.start_load_kv(None) == 2 * (600 + 1300)
    assert sorted((c[0], c[1], c[3]) for c in store.calls) == sorted(
        (r, layer, s) for r, s in (("a", 0), ("b", 1)) for layer in pools)
    assert all(c[2] is pools[c[1]] for c in store.calls)
    work.clear_connector_metadata()
    assert work.start_load_kv(None) == 0
    # a finished request frees its slot for the next one
    assert sched.request_finished(reqs["a"], []) == (False, None)
    sched.update_state_after_alloc(reqs["c"], [], 40)
    assert sched.build_connector_meta().loads == [("c", 0, 40)]
    assert sched.slot_of(reqs["b"]) == 1 and sched.slot_of(reqs["a"]) is None
    return sched, work


def test_connector_metadata_flow_without_vllm():
    from turboquant_pro_amd.connectors import vllm as mod
    _metadata_round(mod)


def test_connector_metadata_flow_with_stubbed_vllm(monkeypatch):
    """With vLLM importable (stub modules, as the reference's own connector
    test does, tests/test_vllm_connector.py:89-119), the connector is a
    subclass of vLLM's KVConnectorBase_V1, its metadata of
    KVConnectorMetadata, and the base's bind/clear hooks carry the flow."""
    import importlib
    import sys
    import types

    class KVConnectorRole:
        SCHEDULER = "scheduler"
        WORKER = "worker"

    class KVConnectorMetadata:
        pass

    class KVConnectorBase_V1:  # noqa: N801
        def __init__(self, vllm_config, role):
            self._vllm_config, self._role = vllm_config, role
            self._connector_metadata = None

        def bind_connector_metadata(self, m):
            self._connector_metadata = m

        def clear_connector_metadata(self):
            self._connector_metadata = None

        def _get_connector_metadata(self):
            return self._connector_metadata

    names = ["vllm", "vllm.distributed", "vllm.distributed.kv_transfer",
             "vllm.distributed.kv_transfer.kv_connector", "vllm.distributed.kv_transfer.kv_connector.v1"]
    for n in names:
        monkeypatch.setitem(sys.modules, n, types.ModuleType(n))
    base = types.ModuleType("vllm.distributed.kv_transfer.kv_connector.v1.base")
    base.KVConnectorBase_V1, base.KVConnectorMetadata, base.KVConnectorRole = (
        KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole)
    monkeypatch.setitem(sys.modules, base.__name__, base)
    from turboquant_pro_amd.connectors import vllm as mod
    try:
        mod = importlib.reload(mod)
        assert issubclass(mod.TurboQuantKVConnector, KVConnectorBase_V1)
        assert mod.KVConnectorRole is KVConnectorRole
        sched, work = _metadata_round(mod)
        assert isinstance(sched.build_connector_meta(), KVConnectorMetadata)
        assert work._role == KVConnectorRole.WORKER
    finally:
        monkeypatch.undo()
        importlib.reload(mod)
