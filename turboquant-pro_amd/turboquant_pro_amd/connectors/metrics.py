"""Counters of the KV tier, with the reference's counter names.

``ConnectorMetrics.to_dict`` returns the keys the reference's connector
reports from ``get_metrics`` (turboquant_pro/connectors/metrics.py:38-126;
vllm_v1.py:804-806): event counters, misses by cause, logical and physical
bytes, and save/load latency quantiles from a bounded window.  The names and
the derived fields (``misses_total``, ``hit_rate``, ``effective_expansion``,
``<op>_latency_p50/p95/p99_s``) are the interface an operator's dashboards
read; the bookkeeping below is this build's own.
"""

from __future__ import annotations

import math
import threading
import time
from collections import deque
from contextlib import contextmanager

__all__ = ["ConnectorMetrics", "MISS_CAUSES"]

MISS_CAUSES = ("empty", "corrupt", "incompatible", "timeout", "declined")
COUNTERS = ("saves", "loads", "hits", "evictions", "integrity_failures", "backpressure_blocked",
            "backpressure_dropped", "worker_fallbacks", "bytes_logical", "bytes_physical",
            "records_persisted", "records_restored")
WINDOW = 1024  # latency samples kept per operation


class ConnectorMetrics:
    """Thread-safe counters and latency windows."""

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._n = dict.fromkeys(COUNTERS + tuple(f"misses_{c}" for c in MISS_CAUSES), 0)
        self._lat = {"save": deque(maxlen=WINDOW), "load": deque(maxlen=WINDOW)}

    def inc(self, name: str, by: float = 1) -> None:
        with self._lock:
            if name not in self._n:
                raise KeyError(f"unknown counter {name!r}")
            self._n[name] += by

    def miss(self, cause: str) -> None:
        if cause not in MISS_CAUSES:
            raise KeyError(f"unknown miss cause {cause!r}; one of {MISS_CAUSES}")
        self.inc(f"misses_{cause}")

    def bytes_saved(self, logical: int, physical: int) -> None:
        with self._lock:
            self._n["bytes_logical"] += logical
            self._n["bytes_physical"] += physical

    @contextmanager
    def timed(self, op: str):
        """Record the seconds the ``with`` body takes under ``op``."""
        t0 = time.perf_counter()
        try:
            yield
        finally:
            with self._lock:
                self._lat[op].append(time.perf_counter() - t0)

    @staticmethod
    def _quantile(xs: list, q: float) -> float:
        # linear interpolation between order statistics (NumPy's default)
        if not xs:
            return float("nan")
        s = sorted(xs)
        pos = (len(s) - 1) * q
        lo = math.floor(pos)
        hi = min(lo + 1, len(s) - 1)
        return s[lo] + (s[hi] - s[lo]) * (pos - lo)

    def to_dict(self) -> dict:
        with self._lock:
            out = dict(self._n)
            lat = {op: list(v) for op, v in self._lat.items()}
        miss = sum(out[f"misses_{c}"] for c in MISS_CAUSES)
        looks = out["hits"] + miss
        out["misses_total"] = miss
        out["hit_rate"] = out["hits"] / looks if looks else float("nan")
        out["effective_expansion"] = (out["bytes_logical"] / out["bytes_physical"]
                                      if out["bytes_physical"] else float("nan"))
        for op in ("save", "load"):
            for name, q in (("p50", 0.50), ("p95", 0.95), ("p99", 0.99)):
                out[f"{op}_latency_{name}_s"] = self._quantile(lat[op], q)
        return out
