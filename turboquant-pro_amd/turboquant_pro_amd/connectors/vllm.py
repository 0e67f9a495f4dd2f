"""KV connector with the reference's vLLM V1 protocol surface and a live
load path into the gfx950 paged pool.

Mirrors ``TurboQuantKVConnector`` (turboquant_pro/connectors/vllm_v1.py:
714-814): one class for both roles; scheduler-side
``get_num_new_matched_tokens`` / ``update_state_after_alloc`` /
``build_connector_meta`` / ``request_finished``; worker-side
``save_kv_layer``, ``start_load_kv``, ``wait_for_layer_load``,
``wait_for_save``, ``get_finished``.  The reference's ``start_load_kv`` is a
no-op (its store only returns dense K/V).  Here a layer bound to a
:class:`TQKVPool` (``bind_pool``) is saved in the pool's own group cadence
(``TurboQuantBlockStore.save_sequence``) and ``start_load_kv`` restores a
request's saved prefix into its pool slot as codes -- the coded groups are
imported unchanged, only the hot tokens come back dequantized -- so decode
resumes on codes without re-encoding.  Unbound layers save and load as in the
reference (one dense-restorable record per layer).

vLLM itself is not a dependency: without it the class stands alone, with the
same method names and arguments (the reference's shim, vllm_v1.py:667-711).
"""

from __future__ import annotations

import logging
from typing import Any

from .store import TurboQuantBlockStore

logger = logging.getLogger(__name__)

__all__ = ["TurboQuantKVConnector", "register"]

CONNECTOR_NAME = "TurboQuantConnector"


class TurboQuantKVConnector:
    """Both connector roles over one :class:`TurboQuantBlockStore`."""

    def __init__(self, vllm_config: Any = None, role: Any = None, *, store: TurboQuantBlockStore | None = None,
                 **kwargs: Any):
        self.vllm_config, self.role = vllm_config, role
        cfg = getattr(getattr(vllm_config, "kv_transfer_config", None), "kv_connector_extra_config", None)
        cfg = dict(cfg) if isinstance(cfg, dict) else {}
        self.store = store or TurboQuantBlockStore(
            key_plugin=cfg.get("key_plugin", "per_channel"),
            value_plugin=cfg.get("value_plugin", "polar"),
            quantizer_config=cfg.get("quantizer_config"))
        self._pools: dict[str, Any] = {}
        self._loaded: dict[tuple[str, str], int] = {}

    # ---------------------------------------------------------- worker setup
    def bind_pool(self, layer_name: str, pool) -> None:
        """Serve ``layer_name`` from ``pool``: saves follow its group cadence and
        ``start_load_kv`` restores into it."""
        self._pools[layer_name] = pool

    # ------------------------------------------------------ scheduler side
    def get_num_new_matched_tokens(self, request: Any, num_computed_tokens: int, *args: Any,
                                   **kwargs: Any) -> tuple[int, bool]:
        """Tokens the store can supply beyond those already computed (loads
        are synchronous: nothing is pending)."""
        rid = getattr(request, "request_id", None) or str(request)
        return max(0, self.store.matched_tokens(rid) - int(num_computed_tokens)), False

    def update_state_after_alloc(self, *args: Any, **kwargs: Any) -> None:
        return None

    def build_connector_meta(self, scheduler_output: Any = None, **kwargs: Any) -> dict:
        return {"version": 1}

    def request_finished(self, request: Any = None, block_ids: Any = None,
                         **kwargs: Any) -> tuple[bool, dict | None]:
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

    def start_load_kv(self, forward_context: Any = None, *, requests: dict | None = None,
                      **kwargs: Any) -> int:
        """Restore saved prefixes into the bound pools: ``requests`` maps a
        request id to its sequence slot in every bound pool.  Returns the
        tokens restored over all layers; a request with nothing stored is a
        miss (it stays empty and is recomputed)."""
        total = 0
        for rid, slot in (requests or {}).items():
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
