"""Hot / cold expert map -- drop-in for ``HotColdMap``
(vibeblade/moe_profiler.py:8-62).

The map names, per MoE layer, the experts kept resident in HBM from the
start ("hot") and the ones uploaded on first use ("cold").  What must match
the reference is the interface: the constructor's keyword names, the
attributes ``hot_experts`` / ``cold_experts`` ({layer: [expert ids]}),
``num_layers``, ``num_experts``, ``profile_tokens``, ``profile_dataset``, the
methods ``hit_rate``, ``overall_hit_rate``, ``summary``, ``save`` / ``load``
and the JSON file format (one object with those six keys; the layer keys of
the two maps written as strings, since JSON keys are strings).
"""
from __future__ import annotations

import json
from dataclasses import dataclass

import numpy as np

# The JSON object's keys, in the order the files carry them.
_FIELDS = ("hot_experts", "cold_experts", "num_layers", "num_experts", "profile_tokens", "profile_dataset")
_LAYER_MAPS = ("hot_experts", "cold_experts")


def _keys_to(layer_map: dict, conv) -> dict:
    return {conv(layer): list(ids) for layer, ids in layer_map.items()}


@dataclass
class HotColdMap:
    """Per-layer hot and cold expert ids of a MoE model.  A dataclass with the
    reference's fields, order and defaults, so ``dataclasses.asdict``,
    ``replace``, ``fields`` and ``is_dataclass`` work on it as on the
    reference's."""

    hot_experts: dict    # {layer: [expert ids]} kept resident in HBM
    cold_experts: dict   # {layer: [expert ids]} uploaded on first use
    num_layers: int
    num_experts: int
    profile_tokens: int = 0
    profile_dataset: str = ""

    # ---- queries ----------------------------------------------------------

    def hit_rate(self, layer_idx: int, expert_indices) -> float:
        """Share of the routed expert ids (any shape) that are hot in this layer;
        0 when nothing was routed."""
        routed = np.asarray(expert_indices).reshape(-1).astype(np.int64)
        if routed.size == 0:
            return 0.0
        hot = np.fromiter((int(e) for e in self.hot_experts.get(layer_idx, ())), dtype=np.int64)
        return float(np.count_nonzero(np.isin(routed, hot))) / routed.size

    def overall_hit_rate(self) -> float:
        """Hot experts over all (layer, expert) slots of the model: the hit rate
        of uniform routing.  0 for an empty map or a model without layers."""
        slots = self.num_layers * self.num_experts
        if not self.hot_experts or self.num_layers == 0:
            return 0.0
        return sum(map(len, self.hot_experts.values())) / slots

    def summary(self) -> str:
        """A header (layers and experts, profile tokens, dataset) and one line per
        layer of the hot map with its hot and cold counts."""
        out = [f"HotColdMap: {self.num_layers} layers, {self.num_experts} experts",
               f"Profile tokens: {self.profile_tokens}",
               f"Dataset: {self.profile_dataset if self.profile_dataset else '(none)'}"]
        out += [f"  Layer {layer:3d}: hot={len(self.hot_experts[layer])}, "
                f"cold={len(self.cold_experts.get(layer, ()))}" for layer in sorted(self.hot_experts)]
        return "\n".join(out)

    # ---- persistence ------------------------------------------------------

    def to_json_dict(self) -> dict:
        d = {name: getattr(self, name) for name in _FIELDS}
        for name in _LAYER_MAPS:
            d[name] = _keys_to(d[name], str)
        return d

    @classmethod
    def from_json_dict(cls, d: dict) -> "HotColdMap":
        d = dict(d)
        for name in _LAYER_MAPS:
            d[name] = _keys_to(d[name], int)
        return cls(**d)

    def save(self, path: str) -> None:
        with open(path, "w") as f:
            json.dump(self.to_json_dict(), f, indent=2)

    @classmethod
    def load(cls, path: str) -> "HotColdMap":
        with open(path) as f:
            return cls.from_json_dict(json.load(f))
