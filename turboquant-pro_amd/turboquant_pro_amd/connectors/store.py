"""Block store of quantized KV layers, keyed by (request, layer), with the
reference's persistence and handoff formats.

Mirrors ``TurboQuantBlockStore`` (turboquant_pro/connectors/vllm_v1.py:213-
664): ``save`` quantizes one layer's K/V through the plugin registry
(``per_channel`` keys, ``polar`` values -- here the gfx950 encode), ``load``
dequantizes it (the gfx950 dequant), and the persistence hooks are gated by
a complete, matching :class:`KVIdentityProfile`:

* ``export_state`` / ``import_state``: schema ``tqp-kv-store-state/2``, one
  ``tqp-kv-npz/1`` blob and its SHA-256 per record, keys
  ``request + "\\0" + layer``; the profile is checked first (a mismatch
  refuses everything), then each record's integrity (a bad record is
  skipped, the rest load);
* ``save_to_dir`` / ``load_from_dir``: ``<sha256(key)[:24]>.rec`` blobs, a
  ``manifest.json`` (schema, digest, tokens, per-record file + SHA-256) and a
  ``COMMIT`` marker holding the digest, written last by atomic rename after
  fsync; no marker, or a marker for another digest, is a miss; manifest
  file names other than 24 hex digits + ``.rec`` are refused.

A ``load`` that cannot decode a record is a miss: the record is dropped and
``None`` returned.  Every save, load, miss (by cause), eviction and restore is
counted in ``metrics`` (:class:`ConnectorMetrics`, the reference's counter
names).  Saves are synchronous (the reference's async queue and backpressure
are serving-side glue that this build leaves to the caller).
"""

from __future__ import annotations

import hashlib
import json
import logging
import os
import re
import tempfile
import threading
from typing import Any

import numpy as np

from .identity import IncompatibleProfile, KVIdentityProfile
from .metrics import ConnectorMetrics
from .records import BlockRecord, RawTokens, payload_nbytes, rec_from_blob, rec_to_blob

logger = logging.getLogger(__name__)

__all__ = ["TurboQuantBlockStore", "STATE_SCHEMA", "ENCODER_VERSION"]

STATE_SCHEMA = "tqp-kv-store-state/2"
# The reference encoder release whose container bytes the gfx950 encode
# reproduces bit for bit (per_channel asym-NF4 keys, polar values); a
# profile's ``encoder_version`` names it so that stores hand over both ways.
ENCODER_VERSION = "2.0.0a2"
_REC_NAME = re.compile(r"[0-9a-f]{24}\.rec")


def _sha256(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


class TurboQuantBlockStore:
    """Quantized KV blocks on the host, encoded and decoded on the GPU.

    ``quantizer_config`` goes to both plugins, as in the reference (a plugin
    that refuses a keyword gets its defaults); ``key_config`` and
    ``value_config`` are applied on top, per plugin.  Without any of them the
    store uses the cache's own format: asym-NF4 keys with 2 % outliers, 3-bit
    values with rotation seed 0.  ``quantizer_config={}`` gives the reference's
    plugin defaults instead (uniform 4-bit keys without outliers, a rotation
    drawn per store), which the gfx950 plugins also serve; records of an
    unseeded rotation decode only in the process that wrote them.
    """

    DEFAULT_KEY_CONFIG = {"nf4_asym": True, "outlier_frac": 0.02}
    DEFAULT_VALUE_CONFIG = {"bits": 3, "seed": 0}

    def __init__(self, key_plugin: str = "per_channel", value_plugin: str = "polar",
                 quantizer_config: dict | None = None, profile: KVIdentityProfile | None = None,
                 key_config: dict | None = None, value_config: dict | None = None, device=None):
        self.key_plugin, self.value_plugin = key_plugin, value_plugin
        self.quantizer_config = dict(quantizer_config or {})
        explicit = quantizer_config is not None or key_config is not None or value_config is not None
        self.key_config = dict(key_config or ({} if explicit else self.DEFAULT_KEY_CONFIG))
        self.value_config = dict(value_config or ({} if explicit else self.DEFAULT_VALUE_CONFIG))
        self.profile = profile
        self.device = device
        self._records: dict[tuple[str, str], BlockRecord] = {}
        self._tokens: dict[str, int] = {}
        self._quantizers: dict[tuple, Any] = {}
        self._lock = threading.Lock()
        self.metrics = ConnectorMetrics()

    # ------------------------------------------------------------ plugins
    def quant_descriptor(self) -> dict:
        """The ``quant`` field of a :class:`KVIdentityProfile` for this store:
        plugin names and every parameter that changes the stored bytes."""
        return {"key": self.key_plugin, "value": self.value_plugin,
                "key_config": {**self.quantizer_config, **self.key_config},
                "value_config": {**self.quantizer_config, **self.value_config}}

    def _quantizer(self, kind: str, head_dim: int, n_heads: int):
        name = self.key_plugin if kind == "key" else self.value_plugin
        extra = self.key_config if kind == "key" else self.value_config
        cache_key = (kind, name, head_dim, n_heads)
        q = self._quantizers.get(cache_key)
        if q is None:
            from .. import plugins
            geometry = {"head_dim": head_dim, "n_heads": n_heads}
            if self.device is not None:
                geometry["device"] = self.device
            try:
                q = plugins.create(name, **{**geometry, **self.quantizer_config, **extra})
            except TypeError:
                # a plugin that does not take the shared keywords (vllm_v1.py:258-275)
                q = plugins.create(name, **{**geometry, **extra})
            self._quantizers[cache_key] = q
        return q

    @staticmethod
    def _host_f32(x: Any) -> np.ndarray:
        if hasattr(x, "detach"):
            x = x.detach().float().cpu().numpy()
        return np.ascontiguousarray(x, dtype=np.float32)

    @staticmethod
    def _as_bhsd(x: np.ndarray) -> np.ndarray:
        """Any engine layout as (B, H, S, D): tokens on axis -2, channels on
        axis -1, leading axes folded into the batch (vllm_v1.py:284-296)."""
        if x.ndim == 4:
            return x
        if x.ndim < 4:
            return x.reshape((1,) * (4 - x.ndim) + x.shape)
        return x.reshape((-1,) + x.shape[-3:])

    # ---------------------------------------------------------------- API
    def make_record(self, keys: Any, values: Any, packed: bool = False,
                    position_start: int = 0) -> BlockRecord:
        """Quantize one layer block into a record (the body of ``save``);
        ``position_start`` is the block's first token position (the RoPE
        zero point of ``bias`` keys depends on it)."""
        k, v = self._host_f32(keys), self._host_f32(values)
        if k.shape != v.shape:
            raise ValueError(f"keys {k.shape} and values {v.shape} differ in shape")
        k4, v4 = self._as_bhsd(k), self._as_bhsd(v)
        d, h = int(k4.shape[-1]), int(k4.shape[1])
        kw = {"packed": True} if packed else {}
        kkw = dict(kw, position_start=int(position_start)) if position_start else kw
        return BlockRecord(key_payload=self._quantizer("key", d, h).compress(k4, **kkw),
                           value_payload=self._quantizer("value", d, h).compress(v4, **kw),
                           shape=tuple(int(s) for s in k.shape), dtype="float32",
                           num_tokens=int(k4.shape[-2]), head_dim=d, n_heads=h)

    # ------------------------------------------------- paged (pool) records
    @staticmethod
    def _group_name(layer_name: str, g: int) -> str:
        return f"{layer_name}#g{g}"

    def save_sequence(self, request_id: str, layer_name: str, keys: Any, values: Any,
                      group_tokens: int, hot_window: int) -> int:
        """Store one sequence's layer K/V ``(H, L, D)`` the way a paged pool
        holds it: one record per coded group of the flush cadence
        (``<layer>#g<i>``, ``group_tokens`` tokens each, so each is exactly the
        pool's group) and the hot window as it is (``<layer>#hot0``, a
        :class:`RawTokens` payload: fp16 for fp16 K/V, fp32 otherwise, the
        precision of the pool they came from), so that a restore is the pool
        it came from.  The group records are ``tqp-kv-npz/1`` records the
        reference reads; the hot record is this library's own.  Returns the
        groups."""
        from ..codebooks import n_groups_for
        hot_dtype = np.float16 if str(getattr(keys, "dtype", "")).endswith("float16") else np.float32
        k, v = self._host_f32(keys), self._host_f32(values)
        k4, v4 = self._as_bhsd(k), self._as_bhsd(v)
        if k4.shape[0] != 1 or k4.shape != v4.shape:
            raise ValueError("save_sequence takes one sequence: (H, L, D) keys and values")
        L, G = int(k4.shape[2]), int(group_tokens)
        ng = n_groups_for(L, int(hot_window))
        recs = {self._group_name(layer_name, g): self.make_record(
                    k4[:, :, g * G:(g + 1) * G], v4[:, :, g * G:(g + 1) * G], packed=True,
                    position_start=g * G)
                for g in range(ng)}
        if L > ng * G:
            hk = np.ascontiguousarray(k4[:, :, ng * G:], dtype=hot_dtype)
            hv = np.ascontiguousarray(v4[:, :, ng * G:], dtype=hot_dtype)
            recs[f"{layer_name}#hot0"] = BlockRecord(
                key_payload=RawTokens(hk), value_payload=RawTokens(hv), shape=tuple(hk.shape[1:]),
                dtype=np.dtype(hot_dtype).name, num_tokens=int(hk.shape[2]), head_dim=int(hk.shape[3]),
                n_heads=int(hk.shape[1]))
        with self._lock:
            for name, rec in recs.items():
                self._records[(request_id, name)] = rec
            self._tokens[request_id] = L
        for rec in recs.values():
            self._count_save(rec)
        return ng

    def load_into_pool(self, request_id: str, layer_name: str, pool, b: int) -> int:
        """Restore a sequence saved by :meth:`save_sequence` into sequence ``b``
        of ``pool`` (empty): the coded groups go in as codes, unchanged (no
        dequantize / re-encode), the hot window as the tokens it held.
        Returns the tokens restored, 0 when nothing is stored (a miss).
        Raises ``ValueError`` when the records are not in the pool's format
        (key grid, zero point and, for sparse/bias zero points, rope_theta and
        group positions, value width, rotation, group size)."""
        groups = []
        with self._lock:
            while (request_id, self._group_name(layer_name, len(groups))) in self._records:
                groups.append(self._records[(request_id, self._group_name(layer_name, len(groups)))])
            hot = self._records.get((request_id, f"{layer_name}#hot0"))
        if not groups and hot is None:
            self.metrics.miss("empty")
            return 0
        with self.metrics.timed("load"):
            try:
                n = self._restore(groups, hot, pool, b)
            except ValueError:
                self.metrics.miss("incompatible")
                raise
        self.metrics.inc("loads")
        self.metrics.inc("hits")
        self.metrics.inc("records_restored", len(groups) + (hot is not None))
        return n

    def _restore(self, groups: list, hot, pool, b: int) -> int:
        """The body of :meth:`load_into_pool`: format checks, then the import."""
        import torch

        H, D, G = pool.n_kv_heads, pool.head_dim, pool.group_tokens
        vq = self._quantizer("value", D, H)
        if getattr(vq, "value_bits", None) != pool.value_bits:
            raise ValueError(f"stored values are {getattr(vq, 'value_bits', None)}-bit, the pool's "
                             f"{pool.value_bits}-bit")
        # the instance's own rotation (drawn once, also for an unseeded store)
        if not np.array_equal(np.asarray(vq.rotation[0], np.float32), pool.pi.cpu().numpy()):
            raise ValueError("the pool's value rotation is not the store's")
        items = []
        for rec in groups:
            kp, vp = rec.key_payload, rec.value_payload
            if rec.num_tokens != G or rec.n_heads != H or rec.head_dim != D or not kp.packed \
                    or not vp.packed:
                raise ValueError("a stored group does not match the pool's group format")
            uniform = getattr(kp, "nf4_scale", None) is None and getattr(kp, "scale", None) is not None
            if ("uniform" if uniform else "nf4_asym") != pool.key_grid:
                raise ValueError(f"stored keys are {'uniform' if uniform else 'asym-NF4'}, the pool's "
                                 f"{pool.key_grid}")
            zp = "calibrated" if uniform else getattr(kp, "zp_mode", "calibrated")
            if zp == "calibrated" and not uniform and getattr(kp, "nf4_mean", None) is None:
                zp = "symmetric"  # symmetric NF4: no mean stored (per_channel_kv.py:354-357)
            if zp != pool.zero_point:
                raise ValueError(f"stored key zero point {zp!r}, the pool's {pool.zero_point!r}")
            if zp != "calibrated":
                # the zero point of a sparse/bias group is a function of its
                # rope_theta and first position (per_channel_kv.py:234-267):
                # the pool rebuilds it from its own, so both must match
                theta = getattr(kp, "rope_theta", None)
                if theta is None or float(theta) != float(pool.rope_theta):
                    raise ValueError(f"stored keys use rope_theta={theta}, the pool's "
                                     f"{pool.rope_theta}")
                start = int(getattr(kp, "position_start", 0))
                if start != len(items) * G:
                    raise ValueError(f"stored group {len(items)} starts at position {start}, "
                                     f"not {len(items) * G}")
            if uniform:
                scale, mean = np.asarray(kp.scale)[0, :, 0, :], np.asarray(kp.zero)[0, :, 0, :]
            else:
                scale = np.asarray(kp.nf4_scale)[0]
                mean = None if kp.nf4_mean is None else np.asarray(kp.nf4_mean)[0]
            items.append(({"kpacked": kp.indices, "nf4_scale": scale, "nf4_mean": mean,
                           "outlier_idx": kp.outlier_idx, "outlier_val": kp.outlier_val},
                          {"vpacked": vp.indices, "vnorms": vp.norms[0]}))
        if hot is not None:
            hk = torch.from_numpy(np.ascontiguousarray(hot.key_payload.data)[0])
            hv = torch.from_numpy(np.ascontiguousarray(hot.value_payload.data)[0])
            if pool.dtype == torch.float16 and hk.dtype != torch.float16:
                raise ValueError("the stored hot window is fp32; this pool holds fp16 tokens")
        else:
            hk = hv = torch.zeros((H, 0, D), dtype=pool.dtype)
        pool.load_sequence(b, items, hk, hv)
        return len(items) * G + int(hk.shape[1])

    def _count_save(self, rec: BlockRecord) -> None:
        self.metrics.inc("saves")
        n = 1
        for dim in rec.shape:
            n *= int(dim)
        self.metrics.bytes_saved(logical=2 * 4 * n,  # fp32 keys and values
                                 physical=payload_nbytes(rec.key_payload) + payload_nbytes(rec.value_payload))

    def save(self, request_id: str, layer_name: str, keys: Any, values: Any) -> None:
        """Quantize and store one layer's KV for ``request_id``."""
        with self.metrics.timed("save"):
            rec = self.make_record(keys, values)
            with self._lock:
                self._records[(request_id, layer_name)] = rec
                self._tokens[request_id] = rec.num_tokens
        self._count_save(rec)

    def record(self, request_id: str, layer_name: str) -> BlockRecord | None:
        with self._lock:
            return self._records.get((request_id, layer_name))

    def load(self, request_id: str, layer_name: str):
        """``(keys, values)`` fp32 in the saved shape, or ``None`` (nothing
        stored, or a record that does not decode -- then it is dropped)."""
        rec = self.record(request_id, layer_name)
        if rec is None:
            self.metrics.miss("empty")
            return None
        if hasattr(rec.key_payload, "data") and not hasattr(rec.key_payload, "indices"):
            # a live-path hot window, stored as it is
            self.metrics.inc("loads")
            self.metrics.inc("hits")
            return (np.asarray(rec.key_payload.data, np.float32).reshape(rec.shape),
                    np.asarray(rec.value_payload.data, np.float32).reshape(rec.shape))
        try:
            with self.metrics.timed("load"):
                k = self._quantizer("key", rec.head_dim, rec.n_heads).decompress(rec.key_payload)
                v = self._quantizer("value", rec.head_dim, rec.n_heads).decompress(rec.value_payload)
                out = (np.asarray(k, dtype=np.float32).reshape(rec.shape),
                       np.asarray(v, dtype=np.float32).reshape(rec.shape))
            self.metrics.inc("loads")
            self.metrics.inc("hits")
            return out
        except Exception:
            logger.warning("undecodable KV record (%s, %s): treated as a miss", request_id,
                           layer_name, exc_info=True)
            self.metrics.miss("corrupt")
            self.metrics.inc("integrity_failures")
            with self._lock:
                self._records.pop((request_id, layer_name), None)
            return None

    def matched_tokens(self, request_id: str) -> int:
        with self._lock:
            return self._tokens.get(request_id, 0)

    def evict(self, request_id: str) -> int:
        with self._lock:
            gone = [key for key in self._records if key[0] == request_id]
            for key in gone:
                del self._records[key]
            self._tokens.pop(request_id, None)
        if gone:
            self.metrics.inc("evictions", len(gone))
        return len(gone)

    def stats(self) -> dict:
        with self._lock:
            return {"requests": len(self._tokens), "records": len(self._records),
                    "key_plugin": self.key_plugin, "value_plugin": self.value_plugin,
                    "bytes_physical": sum(payload_nbytes(r.key_payload) + payload_nbytes(r.value_payload)
                                          for r in self._records.values())}

    # -------------------------------------------------------- persistence
    def _require_profile(self, what: str) -> None:
        if self.profile is None or not self.profile.is_complete:
            raise IncompatibleProfile(f"{what} requires a complete KVIdentityProfile "
                                      "(uncertain identity is never persisted or adopted)")

    def export_state(self) -> dict:
        """Every record as a blob + SHA-256 under the profile's digest."""
        self._require_profile("export")
        with self._lock:
            items = list(self._records.items())
            tokens = dict(self._tokens)
        records = {}
        for (rid, layer), rec in items:
            blob = rec_to_blob(rec)
            records[rid + "\x00" + layer] = {"blob": blob, "sha256": _sha256(blob)}
        return {"schema": STATE_SCHEMA, "profile_digest": self.profile.digest(),
                "records": records, "tokens": tokens}

    def import_state(self, state: dict) -> int:
        """Adopt exported records; returns how many were accepted."""
        self._require_profile("import")
        if state.get("schema") != STATE_SCHEMA:
            raise IncompatibleProfile(f"unknown state schema {state.get('schema')!r} (safe refusal)")
        if state.get("profile_digest") != self.profile.digest():
            raise IncompatibleProfile("profile digest mismatch: every record refused (safe miss)")
        accepted = 0
        for key, item in state.get("records", {}).items():
            blob = item["blob"]
            if _sha256(blob) != item.get("sha256"):
                logger.warning("integrity failure on %r: skipped", key)
                self.metrics.inc("integrity_failures")
                continue
            try:
                rec = rec_from_blob(blob)
            except Exception:
                logger.warning("undecodable record %r: skipped", key, exc_info=True)
                self.metrics.inc("integrity_failures")
                continue
            rid, layer = key.split("\x00", 1)
            with self._lock:
                self._records[(rid, layer)] = rec
                self._tokens[rid] = rec.num_tokens
            accepted += 1
        self.metrics.inc("records_restored", accepted)
        return accepted

    def save_to_dir(self, path: str) -> int:
        """Persist atomically: records and manifest first, ``COMMIT`` last."""
        state = self.export_state()
        os.makedirs(path, exist_ok=True)

        def write_synced(data, name: str) -> None:
            binary = isinstance(data, bytes)
            with tempfile.NamedTemporaryFile("wb" if binary else "w", dir=path, delete=False,
                                             **({} if binary else {"encoding": "utf-8"})) as f:
                f.write(data)
                f.flush()
                os.fsync(f.fileno())
                tmp = f.name
            os.replace(tmp, os.path.join(path, name))

        def sync_dir() -> None:
            try:
                fd = os.open(path, os.O_RDONLY)
                try:
                    os.fsync(fd)
                finally:
                    os.close(fd)
            except OSError:
                pass

        manifest = {"schema": state["schema"], "profile_digest": state["profile_digest"],
                    "tokens": state["tokens"], "records": {}}
        for key, item in state["records"].items():
            fname = _sha256(key.encode())[:24] + ".rec"
            write_synced(item["blob"], fname)
            manifest["records"][key] = {"file": fname, "sha256": item["sha256"]}
        write_synced(json.dumps(manifest), "manifest.json")
        sync_dir()
        write_synced(state["profile_digest"], "COMMIT")
        sync_dir()
        self.metrics.inc("records_persisted", len(manifest["records"]))
        return len(manifest["records"])

    def load_from_dir(self, path: str) -> int:
        """Restore what ``save_to_dir`` committed; returns records accepted."""
        self._require_profile("restore")
        marker = os.path.join(path, "COMMIT")
        if not os.path.exists(marker):
            raise IncompatibleProfile("no COMMIT marker: uncommitted persistence (safe miss)")
        with open(marker, encoding="utf-8") as f:
            if f.read().strip() != self.profile.digest():
                raise IncompatibleProfile("COMMIT profile digest mismatch (safe miss)")
        with open(os.path.join(path, "manifest.json"), encoding="utf-8") as f:
            manifest = json.load(f)
        records = {}
        for key, meta in manifest.get("records", {}).items():
            fname = meta.get("file", "")
            if not _REC_NAME.fullmatch(fname):
                logger.warning("manifest names a suspicious file %r: refused", fname)
                continue
            try:
                with open(os.path.join(path, fname), "rb") as f:
                    records[key] = {"blob": f.read(), "sha256": meta.get("sha256")}
            except OSError:
                continue
        return self.import_state({"schema": manifest.get("schema"),
                                  "profile_digest": manifest.get("profile_digest"),
                                  "records": records, "tokens": manifest.get("tokens", {})})
