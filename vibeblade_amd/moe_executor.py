"""Hot / cold MoE executor -- drop-in for vibeblade/moe_executor.py.

Same constructor, ``dispatch`` signature, stats dict keys and accounting as
the reference (vibeblade/moe_executor.py:31-406).  One MI355X holds every
expert of every layer in HBM, so there is no CPU expert path: the experts a
``HotColdMap`` marks hot are uploaded when the executor is built, the others
on the first dispatch that needs their layer, and every routed expert runs in
one grouped GPU launch sequence.  The counters keep their reference names and
meaning for the map: ``gpu_hits`` = routed experts that are hot,
``cpu_falls`` = routed experts that are cold (here: served from the on-demand
tier, still on the GPU); ``cpu_latency_ms`` is the time spent uploading cold
experts.  Unlike the reference, which routes only the first token of a batch
(vibeblade/moe_executor.py:210-212), every token is routed.
"""
from __future__ import annotations

import threading
import time
from dataclasses import dataclass

import numpy as np
import torch

from .moe import grouped_ffn, _dense_ffn, _sanitize

__all__ = ["ExecutorStats", "HotColdExecutor"]


_COUNTS = ("gpu_hits", "cpu_falls")
_TIMES_MS = ("gpu_latency_ms", "cpu_latency_ms", "sync_latency_ms")


@dataclass
class ExecutorStats:
    """Routed-expert counters and time spent, for one dispatch or summed over
    dispatches.  A dataclass with the reference's fields, order and defaults;
    ``hit_rate`` and the ``to_dict`` keys and rounding are the reference's
    interface (vibeblade/moe_executor.py:31-54)."""

    gpu_hits: int = 0
    cpu_falls: int = 0
    gpu_latency_ms: float = 0.0
    cpu_latency_ms: float = 0.0
    sync_latency_ms: float = 0.0

    @property
    def hit_rate(self) -> float:
        """Hot share of the routed experts (0 before anything was routed)."""
        routed = self.gpu_hits + self.cpu_falls
        return self.gpu_hits / routed if routed else 0.0

    def add(self, other: "ExecutorStats") -> "ExecutorStats":
        """Accumulate another record into this one (counts and times)."""
        for name in _COUNTS + _TIMES_MS:
            setattr(self, name, getattr(self, name) + getattr(other, name))
        return self

    def copy(self) -> "ExecutorStats":
        return ExecutorStats().add(self)

    def to_dict(self) -> dict:
        d = {name: getattr(self, name) for name in _COUNTS}
        d.update((name, round(getattr(self, name), 3)) for name in _TIMES_MS)
        d["hit_rate"] = round(self.hit_rate, 4)
        return d


class HotColdExecutor:
    """MoE FFN executor over a hot / cold expert map, all experts on the GPU."""

    def __init__(self, hot_cold_map, routers: dict, experts: dict, shared_experts: dict = None,
                 gpu_backend=None, cpu_threads: int = 8, tiered_mgr=None):
        self._hot_map = hot_cold_map
        self._routers = routers
        self._experts = experts
        self._shared = shared_experts or {}
        self._gpu = gpu_backend
        self._cpu_threads = cpu_threads
        self._tiered_mgr = tiered_mgr
        self._open = True
        self._uploaded: set = set()
        self._total_stats = ExecutorStats()
        self._stats_lock = threading.Lock()
        for layer_idx, hot_ids in self._hot_map.hot_experts.items():
            if hot_ids and self._experts.get(layer_idx) is not None:
                self._upload(layer_idx)

    def _upload(self, layer_idx: int) -> float:
        """Make the layer's experts device-resident; returns the ms spent."""
        if layer_idx in self._uploaded:
            return 0.0
        t0 = time.perf_counter()
        self._experts[layer_idx].device_experts()
        torch.cuda.synchronize()
        self._uploaded.add(layer_idx)
        return (time.perf_counter() - t0) * 1000.0

    @property
    def stats(self) -> ExecutorStats:
        with self._stats_lock:
            return self._total_stats.copy()

    def reset_stats(self) -> None:
        with self._stats_lock:
            self._total_stats = ExecutorStats()

    def dispatch(self, layer_idx: int, x: np.ndarray):
        """Route and run the MoE FFN of one layer for x: (shared_dim,),
        (1, shared_dim) or (tokens, shared_dim).  Returns (output same shape
        as x, stats dict)."""
        orig_shape = np.asarray(x).shape
        squeeze = np.asarray(x).ndim == 1
        x2 = np.atleast_2d(np.asarray(x, dtype=np.float32))
        router = self._routers.get(layer_idx)
        expert_set = self._experts.get(layer_idx)
        if router is None or expert_set is None:
            stats = {"gpu_hits": 0, "cpu_falls": 0, "hit_rate": 0.0, "gpu_latency_ms": 0.0,
                     "cpu_latency_ms": 0.0, "sync_latency_ms": 0.0,
                     "expert_indices": np.array([]), "expert_weights": np.array([])}
            return np.zeros(orig_shape, dtype=np.float32), stats

        cpu_ms = self._upload(layer_idx)
        t0 = time.perf_counter()
        logits = router._logits_dev(x2)
        out, indices, weights = grouped_ffn(expert_set, x2, logits, router.topk)
        t1 = time.perf_counter()
        shared = self._shared.get(layer_idx)
        if shared is not None and shared[0] is not None:
            out = out + np.atleast_2d(_dense_ffn(x2, *shared))
        output = _sanitize(out).astype(np.float32)
        t2 = time.perf_counter()

        routed = np.asarray(indices).reshape(-1)
        hits = int(np.count_nonzero(np.isin(routed, list(self._hot_map.hot_experts.get(layer_idx, ())))))
        per = ExecutorStats(gpu_hits=hits, cpu_falls=int(routed.size) - hits, gpu_latency_ms=(t1 - t0) * 1000.0,
                            cpu_latency_ms=cpu_ms, sync_latency_ms=(t2 - t1) * 1000.0)
        with self._stats_lock:
            self._total_stats.add(per)
        # per-dispatch dict: to_dict's keys and rounding, except an unrounded
        # hit rate, plus the routing of the (first, for 1-D x) token(s)
        stats = per.to_dict()
        stats["hit_rate"] = per.hit_rate
        stats["expert_indices"] = indices[0] if squeeze else indices
        stats["expert_weights"] = weights[0] if squeeze else weights
        return (output[0] if squeeze else output.reshape(orig_shape)), stats

    def _expert_counts(self, layer_idx=None):
        """(hot, cold) expert counts of one layer, or of every layer (None)."""
        maps = (self._hot_map.hot_experts, self._hot_map.cold_experts)
        if layer_idx is not None:
            return tuple(len(m.get(layer_idx, ())) for m in maps)
        return tuple(sum(map(len, m.values())) for m in maps)

    def layer_stats(self, layer_idx: int) -> dict:
        """Hot and cold expert counts of a layer and the hot share in percent
        (keys of vibeblade/moe_executor.py:363-372)."""
        hot, cold = self._expert_counts(layer_idx)
        return {"layer": layer_idx, "hot_experts": hot, "cold_experts": cold,
                "hot_pct": 100.0 * hot / max(hot + cold, 1)}

    def memory_estimate(self, expert_dim: int, shared_dim: int, bytes_per_param: float = 0.5) -> dict:
        """Bytes held by the hot and the cold experts of the whole map; an
        expert is three shared_dim x expert_dim matrices (gate, up, down) of
        ``bytes_per_param`` per element (keys of
        vibeblade/moe_executor.py:374-400; GB and MB are binary)."""
        expert_bytes = 3.0 * shared_dim * expert_dim * bytes_per_param
        hot, cold = self._expert_counts()
        gib, mib = float(1 << 30), float(1 << 20)
        return {"hot_vram_gb": hot * expert_bytes / gib, "cold_ram_gb": cold * expert_bytes / gib,
                "per_expert_mb": expert_bytes / mib, "total_hot_experts": hot, "total_cold_experts": cold}

    def shutdown(self) -> None:
        """Release host resources (there is no thread pool); dispatch keeps
        working afterwards, as in the reference."""
        self._open = False
