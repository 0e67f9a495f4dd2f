"""KV connector with the reference's vLLM V1 protocol surface and a live
load path into the gfx950 paged pool.

Mirrors ``TurboQuantKVConnector`` (turboquant_pro/connectors/vllm_v1.py:
688-836): one class for both roles, derived from vLLM's
``KVConnectorBase_V1`` when vLLM is importable and from a stand-in base with
the same metadata hooks otherwise (the reference's shim, vllm_v1.py:688-711).

vLLM tells a worker what to load through connector metadata, and this class
follows that flow:

* scheduler side: ``get_num_new_matched_tokens`` reports the stored tokens
  beyond vLLM's own prefix; ``update_state_after_alloc(request, blocks,
  num_external_tokens)`` gives every request that will load a sequence slot
  of the worker's paged pools (a slot allocator of ``max_num_seqs`` slots,
  freed by ``request_finished``) and queues the load; ``build_connector_meta``
  hands the queued loads over as a :class:`TurboQuantConnectorMetadata`;
* worker side: vLLM binds that metadata (``bind_connector_metadata``) before
  the forward pass, and ``start_load_kv(forward_context)`` restores each
  queued request into its slot of every layer bound to a :class:`TQKVPool`
  (``bind_pool``): the coded groups go in as codes, unchanged
  (``TurboQuantBlockStore.load_into_pool``), the hot window as the fp16
  tokens it held, so decode resumes on codes without re-encoding.  A layer
  bound to a pool is saved in the pool's own group cadence
  (``TurboQuantBlockStore.save_sequence``); unbound layers save and load as
  in the reference (one dense-restorable record per layer).

The reference's ``start_load_kv`` is a no-op (its store only returns dense
K/V).  ``get_metrics`` returns the store's counters (vllm_v1.py:804-806).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, field
from typing import Any

from .store import TurboQuantBlockStore

logger = logging.getLogger(__name__)

__all__ = ["TurboQuantKVConnector", "TurboQuantConnectorMetadata", "KVConnectorRole", "register"]

CONNECTOR_NAME = "TurboQuantConnector"


def _resolve_base() -> tuple[type, type, Any]:
    """vLLM's connector base, metadata base and role enum, or stand-ins with
    the same hooks when vLLM is not importable."""
    try:
        from vllm.distributed.kv_transfer.kv_connector.v1.base import (  # type: ignore
            KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole)
        return KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole
    except Exception:
        pass

    class KVConnectorRole:  # noqa: N801 - vLLM's name
        SCHEDULER = 0
        WORKER = 1

    class KVConnectorMetadata:  # noqa: N801
        """Base of the scheduler-to-worker metadata."""

    class KVConnectorBase_V1:  # noqa: N801
        """The metadata hooks of vLLM's base: the worker's copy of the
        scheduler's metadata for the current step."""

        def __init__(self, vllm_config: Any = None, role: Any = None, *args: Any, **kwargs: Any):
            self._vllm_config = vllm_config
            self._role = role
            self._connector_metadata = None

        def bind_connector_metadata(self, connector_metadata: Any) -> None:
            self._connector_metadata = connector_metadata

        def clear_connector_metadata(self) -> None:
            self._connector_metadata = None

        def _get_connector_metadata(self) -> Any:
            return self._connector_metadata

    return KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole


_Base, _MetaBase, KVConnectorRole = _resolve_base()


@dataclass
class TurboQuantConnectorMetadata(_MetaBase):  # type: ignore[misc, valid-type]
    """What the scheduler tells the workers for one step: the requests to
    restore, each as (request id, pool sequence slot, tokens to load)."""

    loads: list = field(default_factory=list)
    version: int = 1


class TurboQuantKVConnector(_Base):  # type: ignore[misc, valid-type]
    """Both connector roles over one :class:`TurboQuantBlockStore`."""

    def __init__(self, vllm_config: Any = None, role: Any = None, *args: Any,
                 store: TurboQuantBlockStore | None = None, **kwargs: Any):
        try:
            super().__init__(vllm_config, role, *args, **kwargs)
        except TypeError:  # base signature drift between vLLM releases
            super().__init__()
        self.vllm_config, self.role = vllm_config, role
        if not hasattr(self, "_connector_metadata"):
            self._connector_metadata = None
        cfg = getattr(getattr(vllm_config, "kv_transfer_config", None), "kv_connector_extra_config", None)
        cfg = dict(cfg) if isinstance(cfg, dict) else {}
        self.store = store or TurboQuantBlockStore(
            key_plugin=cfg.get("key_plugin", "per_channel"),
            value_plugin=cfg.get("value_plugin", "polar"),
            quantizer_config=cfg.get("quantizer_config"))
        # scheduler side: sequence slots of the workers' paged pools
        n = cfg.get("max_num_seqs") or getattr(getattr(vllm_config, "scheduler_config", None),
                                                  "max_num_seqs", None)
        self.max_slots = int(n) if n else None
        self._slot_of: dict[str, int] = {}
        self._free_slots: list[int] = []
        self._next_slot = 0
        self._pending_loads: list[tuple[str, int, int]] = []
        # worker side
        self._pools: dict[str, Any] = {}
        self._loaded: dict[tuple[str, str], int] = {}

    # ---------------------------------------------------------- worker setup
    def bind_pool(self, layer_name: str, pool) -> None:
        """Serve ``layer_name`` from ``pool``: saves follow its group cadence and
        ``start_load_kv`` restores into it."""
        self._pools[layer_name] = pool

    # ------------------------------------------------------ scheduler side
    @staticmethod
    def _rid(request: Any) -> str:
        return str(getattr(request, "request_id", None) or request)

    def slot_of(self, request: Any) -> int | None:
        """The pool sequence slot the scheduler gave ``request`` (or None)."""
        return self._slot_of.get(self._rid(request))

    def _take_slot(self, rid: str) -> int:
        if rid in self._slot_of:
            return self._slot_of[rid]
        if self._free_slots:
            slot = self._free_slots.pop()
        else:
            if self.max_slots is not None and self._next_slot >= self.max_slots:
                raise RuntimeError(f"no free sequence slot: {self.max_slots} requests hold them all")
            slot = self._next_slot
            self._next_slot += 1
        self._slot_of[rid] = slot
        return slot

    def get_num_new_matched_tokens(self, request: Any, num_computed_tokens: int, *args: Any,
                                   **kwargs: Any) -> tuple[int, bool]:
        """Tokens the store can supply beyond those already computed (loads
        are synchronous: nothing is pending)."""
        return max(0, self.store.matched_tokens(self._rid(request)) - int(num_computed_tokens)), False

    def update_state_after_alloc(self, request: Any = None, blocks: Any = None,
                                 num_external_tokens: int = 0, *args: Any, **kwargs: Any) -> None:
        """vLLM allocated blocks for ``request``; when it will take
        ``num_external_tokens`` > 0 from the store, the request gets a
        sequence slot and its load is queued for the next metadata."""
        if request is None or int(num_external_tokens) <= 0:
            return None
        rid = self._rid(request)
        self._pending_loads.append((rid, self._take_slot(rid), int(num_external_tokens)))
        return None

    def build_connector_meta(self, scheduler_output: Any = None, **kwargs: Any) -> TurboQuantConnectorMetadata:
        """The loads queued since the last step, for the workers."""
        meta = TurboQuantConnectorMetadata(loads=list(self._pending_loads))
        self._pending_loads.clear()
        return meta

    def request_finished(self, request: Any = None, block_ids: Any = None,
                         **kwargs: Any) -> tuple[bool, dict | None]:
        """The request's slot is free again; its blocks are not held (the
        store keeps its own copy)."""
        slot = self._slot_of.pop(self._rid(request), None) if request is not None else None
        if slot is not None:
            self._free_slots.append(slot)
        return False, None

    # --------------------------------------------------------- worker side
    @staticmethod
    def _request_id(attn_metadata: Any, kwargs: dict) -> str:
        return str(getattr(attn_metadata, "request_id", kwargs.get("request_id", "_")))

    def save_kv_layer(self, layer_name: str, kv_layer: Any, attn_metadata: Any = None,
                      **kwargs: Any) -> None:
        """Quantize one layer's ``kv_layer[0]`` keys and ``kv_layer[1]``
        values ``(H, L, D)`` of the request into the store (GPU encode)."""
        rid = self._request_id(attn_metadata, kwargs)
        keys, values = kv_layer[0], kv_layer[1]
        pool = self._pools.get(layer_name)
        if pool is None:
            self.store.save(rid, layer_name, keys, values)
        else:
            self.store.save_sequence(rid, layer_name, keys, values, pool.group_tokens, pool.hot_window)

    def start_load_kv(self, forward_context: Any = None, **kwargs: Any) -> int:
        """Restore the requests of the bound metadata into their slots of the
        bound pools.  Returns the tokens restored over all layers; a request
        with nothing stored is a miss (its slot stays empty and vLLM
        recomputes it)."""
        meta = self._get_connector_metadata()
        total = 0
        for rid, slot, _n in getattr(meta, "loads", None) or ():
            for layer_name, pool in self._pools.items():
                n = self.store.load_into_pool(str(rid), layer_name, pool, int(slot))
                self._loaded[(str(rid), layer_name)] = n
                total += n
        return total

    def wait_for_layer_load(self, layer_name: str, **kwargs: Any) -> None:
        return None

    def wait_for_save(self, **kwargs: Any) -> None:
        return None

    def get_finished(self, finished_req_ids: Any = None, **kwargs: Any) -> tuple[set | None, set | None]:
        for rid in finished_req_ids or ():
            self.store.evict(str(rid))
        return None, None

    def get_metrics(self) -> dict:
        """The store's counters (the reference's ``get_metrics`` keys)."""
        return self.store.metrics.to_dict()


def register(name: str = CONNECTOR_NAME) -> bool:
    """Register with vLLM's connector factory when vLLM is installed
    (vllm_v1.py:817-836); ``False`` otherwise."""
    try:
        from vllm.distributed.kv_transfer.kv_connector.factory import KVConnectorFactory
    except Exception:
        logger.info("vLLM not installed; %s not registered", name)
        return False
    try:
        KVConnectorFactory.register_connector(name, __name__, "TurboQuantKVConnector")
    except ValueError:
        pass
    return True
