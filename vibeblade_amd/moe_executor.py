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


@dataclass
class ExecutorStats:
    """Per-token execution statistics (vibeblade/moe_executor.py:31-54)."""

    gpu_hits: int = 0
    cpu_falls: int = 0
    gpu_latency_ms: float = 0.0
    cpu_latency_ms: float = 0.0
    sync_latency_ms: float = 0.0

    @property
    def hit_rate(self) -> float:
        total = self.gpu_hits + self.cpu_falls
        return self.gpu_hits / total if total > 0 else 0.0

    def to_dict(self) -> dict:
        return {
            "gpu_hits": self.gpu_hits,
            "cpu_falls": self.cpu_falls,
            "gpu_latency_ms": round(self.gpu_latency_ms, 3),
            "cpu_latency_ms": round(self.cpu_latency_ms, 3),
            "sync_latency_ms": round(self.sync_latency_ms, 3),
            "hit_rate": round(self.hit_rate, 4),
        }


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
            s = self._total_stats
            return ExecutorStats(s.gpu_hits, s.cpu_falls, s.gpu_latency_ms, s.cpu_latency_ms, s.sync_latency_ms)

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

        hot_ids = set(self._hot_map.hot_experts.get(layer_idx, []))
        hits = int(sum(1 for e in indices.ravel() if int(e) in hot_ids))
        falls = int(indices.size - hits)
        per = ExecutorStats(gpu_hits=hits, cpu_falls=falls, gpu_latency_ms=(t1 - t0) * 1000.0,
                            cpu_latency_ms=cpu_ms, sync_latency_ms=(t2 - t1) * 1000.0)
        with self._stats_lock:
            s = self._total_stats
            s.gpu_hits += per.gpu_hits
            s.cpu_falls += per.cpu_falls
            s.gpu_latency_ms += per.gpu_latency_ms
            s.cpu_latency_ms += per.cpu_latency_ms
            s.sync_latency_ms += per.sync_latency_ms
        stats = {
            "gpu_hits": per.gpu_hits,
            "cpu_falls": per.cpu_falls,
            "hit_rate": per.hit_rate,
            "gpu_latency_ms": round(per.gpu_latency_ms, 3),
            "cpu_latency_ms": round(per.cpu_latency_ms, 3),
            "sync_latency_ms": round(per.sync_latency_ms, 3),
            "expert_indices": indices[0] if squeeze else indices,
            "expert_weights": weights[0] if squeeze else weights,
        }
        return (output[0] if squeeze else output.reshape(orig_shape)), stats

    def layer_stats(self, layer_idx: int) -> dict:
        hot = self._hot_map.hot_experts.get(layer_idx, [])
        cold = self._hot_map.cold_experts.get(layer_idx, [])
        return {"layer": layer_idx, "hot_experts": len(hot), "cold_experts": len(cold),
                "hot_pct": len(hot) / max(len(hot) + len(cold), 1) * 100}

    def memory_estimate(self, expert_dim: int, shared_dim: int, bytes_per_param: float = 0.5) -> dict:
        per_expert = 3 * shared_dim * expert_dim * bytes_per_param
        total_hot = sum(len(v) for v in self._hot_map.hot_experts.values())
        total_cold = sum(len(v) for v in self._hot_map.cold_experts.values())
        return {"hot_vram_gb": total_hot * per_expert / (1024 ** 3),
                "cold_ram_gb": total_cold * per_expert / (1024 ** 3),
                "per_expert_mb": per_expert / (1024 ** 2),
                "total_hot_experts": total_hot,
                "total_cold_experts": total_cold}

    def shutdown(self) -> None:
        """Release host resources (there is no thread pool); dispatch keeps
        working afterwards, as in the reference."""
        self._open = False
