"""Hot / cold expert map -- drop-in for ``HotColdMap``
(vibeblade/moe_profiler.py:8-62): per-layer expert ids pinned in HBM (hot)
or uploaded on first use (cold), with the same JSON format."""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass

import numpy as np


@dataclass
class HotColdMap:
    hot_experts: dict    # {layer_idx: [expert_ids]}
    cold_experts: dict   # {layer_idx: [expert_ids]}
    num_layers: int
    num_experts: int
    profile_tokens: int = 0
    profile_dataset: str = ""

    def hit_rate(self, layer_idx: int, expert_indices: np.ndarray) -> float:
        hot = set(self.hot_experts.get(layer_idx, []))
        flat = np.asarray(expert_indices).flatten()
        return sum(1 for e in flat if int(e) in hot) / max(len(flat), 1)

    def overall_hit_rate(self) -> float:
        if not self.hot_experts or self.num_layers == 0:
            return 0.0
        return sum(len(v) for v in self.hot_experts.values()) / (self.num_layers * self.num_experts)

    def summary(self) -> str:
        lines = [f"HotColdMap: {self.num_layers} layers, {self.num_experts} experts",
                 f"Profile tokens: {self.profile_tokens}",
                 f"Dataset: {self.profile_dataset or '(none)'}"]
        for layer_idx in sorted(self.hot_experts):
            lines.append(f"  Layer {layer_idx:3d}: hot={len(self.hot_experts[layer_idx])}, "
                         f"cold={len(self.cold_experts.get(layer_idx, []))}")
        return "\n".join(lines)

    def save(self, path: str) -> None:
        data = asdict(self)
        data["hot_experts"] = {str(k): v for k, v in data["hot_experts"].items()}
        data["cold_experts"] = {str(k): v for k, v in data["cold_experts"].items()}
        with open(path, "w") as f:
            json.dump(data, f, indent=2)

    @classmethod
    def load(cls, path: str) -> "HotColdMap":
        with open(path) as f:
            data = json.load(f)
        data["hot_experts"] = {int(k): v for k, v in data["hot_experts"].items()}
        data["cold_experts"] = {int(k): v for k, v in data["cold_experts"].items()}
        return cls(**data)
