"""Mixture-of-Experts FFN -- drop-in for vibeblade/moe.py.

Same names, shapes and stats as the reference (vibeblade/moe.py:21-612).
Routing (logits, softmax, top-k, renormalisation) and every expert FFN run on
the GPU: ``moe_ffn_silu`` is one grouped launch sequence over all tokens
(libvbhip's vb_moe_grouped_ffn: tokens grouped per expert, each expert's
weights streamed once, SwiGLU on MFMA, deterministic weighted combine).

Expert weights are fp32 arrays in the reference's GGUF layout (gate / up
(E, expert_dim, shared_dim), down (E, shared_dim, expert_dim)), uploaded
once as exact F32 tensors zero-padded to multiples of 256 (padding adds zero
terms only), or lists of ``QTensor`` handles (GGUF Q4_K experts).
``ExpertRouter.route`` orders the selected experts by descending weight (the
reference's argpartition order is unspecified).
"""
from __future__ import annotations

import re
from dataclasses import dataclass

import numpy as np
import torch

from .tensor import QTensor, as_qtensor, gemv, moe_route, moe_grouped_ffn, sparse_ffn, ACT_SILU, DOWN_GGUF

__all__ = [
    "MoEConfig", "ExpertRouter", "MoEExpertSet", "detect_moe_config", "moe_ffn_silu",
    "load_moe_weights_from_layer", "_silu", "_dense_ffn",
]

_CLIP = 65504.0


def _silu(x: np.ndarray) -> np.ndarray:
    """SiLU (vibeblade/moe.py:36-50), on the GPU."""
    from .sparse import silu
    out = silu(np.asarray(x, dtype=np.float32))
    return np.nan_to_num(out, nan=0.0)


def _sanitize(a: np.ndarray) -> np.ndarray:
    return np.clip(np.nan_to_num(a, nan=0.0, posinf=_CLIP, neginf=-_CLIP), -_CLIP, _CLIP)


def _ffn_rows(gate_rows: QTensor, up_rows: QTensor, down_rows: QTensor, x2d: np.ndarray) -> np.ndarray:
    """down(silu(gate x) * up x) per row of x, all on the GPU (the full neuron
    set through the sparse FFN kernels is the dense SwiGLU FFN)."""
    inter = gate_rows.rows
    dev = gate_rows.device
    allidx = torch.arange(inter, dtype=torch.int32, device=dev)
    xt = torch.from_numpy(np.ascontiguousarray(x2d, dtype=np.float32)).to(dev)
    out = torch.empty((xt.shape[0], down_rows.rows), dtype=torch.float32, device=dev)
    for t in range(xt.shape[0]):
        sparse_ffn(gate_rows, up_rows, down_rows, xt[t], allidx, ACT_SILU, DOWN_GGUF, out=out[t])
    return out.cpu().numpy()


def _dense_ffn(x: np.ndarray, gate_w, up_w, down_w) -> np.ndarray:
    """SwiGLU FFN in the MoE weight convention (vibeblade/moe.py:53-81):
    gate_w / up_w (shared_dim, expert_dim), down_w (expert_dim, shared_dim)."""
    squeeze = np.asarray(x).ndim == 1
    x2 = np.atleast_2d(np.asarray(x, dtype=np.float32))
    g = as_qtensor(np.ascontiguousarray(np.asarray(gate_w, dtype=np.float32).T))
    u = as_qtensor(np.ascontiguousarray(np.asarray(up_w, dtype=np.float32).T))
    d = as_qtensor(np.ascontiguousarray(np.asarray(down_w, dtype=np.float32).T))
    out = _sanitize(_ffn_rows(g, u, d, x2))
    return out[0] if squeeze else out


def _softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    x_max = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - x_max)
    return e / np.sum(e, axis=axis, keepdims=True)


@dataclass
class MoEConfig:
    """Architecture parameters of one MoE FFN layer (vibeblade/moe.py:96-143)."""

    num_experts: int
    num_active: int
    expert_dim: int
    shared_dim: int
    router_topk: int | None = None
    has_shared_expert: bool = False

    def __post_init__(self):
        if self.router_topk is None:
            self.router_topk = self.num_active

    @classmethod
    def from_tensors(cls, router_w, gate_exps, up_exps, down_exps, num_active: int = 2) -> "MoEConfig":
        return cls(num_experts=int(router_w.shape[1]), num_active=num_active,
                   expert_dim=int(gate_exps.shape[1]), shared_dim=int(gate_exps.shape[2]))

    def __repr__(self) -> str:
        parts = [f"num_experts={self.num_experts}", f"num_active={self.num_active}",
                 f"expert_dim={self.expert_dim}", f"shared_dim={self.shared_dim}"]
        if self.has_shared_expert:
            parts.append("shared_expert=True")
        return f"MoEConfig({', '.join(parts)})"


class ExpertRouter:
    """Top-k expert router (vibeblade/moe.py:151-216): logits = x @ W_router on
    the GPU, then softmax (logits clamped to +-50), top-k and renormalisation
    in one device kernel."""

    def __init__(self, router_weight: np.ndarray, topk: int = 2):
        self.weight = np.asarray(router_weight, dtype=np.float32)
        self.topk = int(topk)
        self.num_experts = int(self.weight.shape[1])
        self.shared_dim = int(self.weight.shape[0])
        self._dev_w: QTensor | None = None

    def _wdev(self) -> QTensor:
        if self._dev_w is None:
            self._dev_w = as_qtensor(np.ascontiguousarray(self.weight.T))  # experts x shared_dim
        return self._dev_w

    def _logits_dev(self, x2d: np.ndarray) -> torch.Tensor:
        w = self._wdev()
        xt = torch.from_numpy(np.ascontiguousarray(x2d, dtype=np.float32)).to(w.device)
        out = torch.empty((xt.shape[0], self.num_experts), dtype=torch.float32, device=w.device)
        for t in range(xt.shape[0]):
            gemv(w, xt[t], out=out[t])
        return out

    def route(self, x: np.ndarray):
        squeeze = np.asarray(x).ndim == 1
        x2 = np.atleast_2d(np.asarray(x, dtype=np.float32))
        idx, w = moe_route(self._logits_dev(x2), self.topk)
        idx = idx.cpu().numpy().astype(np.int64)
        w = w.cpu().numpy().astype(np.float32)
        if squeeze:
            return idx[0], w[0]
        return idx, w

    def predict(self, x: np.ndarray) -> np.ndarray:
        squeeze = np.asarray(x).ndim == 1
        logits = self._logits_dev(np.atleast_2d(np.asarray(x, dtype=np.float32))).cpu().numpy()
        return logits[0] if squeeze else logits


def _pad_to(a: np.ndarray, rows: int, cols: int) -> np.ndarray:
    if a.shape == (rows, cols):
        return np.ascontiguousarray(a, dtype=np.float32)
    out = np.zeros((rows, cols), dtype=np.float32)
    out[:a.shape[0], :a.shape[1]] = a
    return out


def _round256(v: int) -> int:
    return (v + 255) // 256 * 256


class MoEExpertSet:
    """Expert weights of one MoE layer (vibeblade/moe.py:224-300).

    gate / up: (E, expert_dim, shared_dim), down: (E, shared_dim, expert_dim)
    fp32 -- or three lists of E ``QTensor`` handles (gate / up expert_dim rows
    x shared_dim, down shared_dim rows x expert_dim), the quantized path."""

    def __init__(self, gate_weights, up_weights, down_weights):
        self._q = isinstance(gate_weights, (list, tuple)) and len(gate_weights) > 0 and \
            isinstance(gate_weights[0], QTensor)
        if self._q:
            self._qg, self._qu, self._qd = list(gate_weights), list(up_weights), list(down_weights)
            g0 = self._qg[0]
            assert len(self._qg) == len(self._qu) == len(self._qd), "expert counts differ"
            for g, u, d in zip(self._qg, self._qu, self._qd):
                assert g.shape == u.shape == (g0.rows, g0.k) and d.shape == (g0.k, g0.rows), \
                    f"gate {g.shape} incompatible with down {d.shape}"
            self._shape = (len(self._qg), g0.rows, g0.k)
            self.gate = self.up = self.down = None
        else:
            self.gate = np.asarray(gate_weights, dtype=np.float32)
            self.up = np.asarray(up_weights, dtype=np.float32)
            self.down = np.asarray(down_weights, dtype=np.float32)
            assert self.gate.shape == self.up.shape, f"gate {self.gate.shape} != up {self.up.shape}"
            assert self.gate.shape[0] == self.down.shape[0] and self.gate.shape[1] == self.down.shape[2] and \
                self.gate.shape[2] == self.down.shape[1], \
                f"gate {self.gate.shape} incompatible with down {self.down.shape}"
            self._shape = self.gate.shape
        self._dev = None

    @property
    def num_experts(self) -> int:
        return int(self._shape[0])

    @property
    def expert_dim(self) -> int:
        return int(self._shape[1])

    @property
    def shared_dim(self) -> int:
        return int(self._shape[2])

    @property
    def expert_dim_real(self) -> int:
        return int(self._shape[1])

    @property
    def quantized(self) -> bool:
        return self._q

    def get_expert(self, idx: int):
        """(gate_w, up_w, down_w) in the MoE convention: (shared_dim,
        expert_dim), (shared_dim, expert_dim), (expert_dim, shared_dim).
        For a quantized set: the expert's three ``QTensor`` handles."""
        if self._q:
            return self._qg[idx], self._qu[idx], self._qd[idx]
        return self.gate[idx].T, self.up[idx].T, self.down[idx].T

    def get_experts_batch(self, indices: np.ndarray):
        if self._q:
            raise TypeError("get_experts_batch returns dense arrays; not available for quantized experts")
        idx = np.asarray(indices)
        return (np.transpose(self.gate[idx], (0, 2, 1)), np.transpose(self.up[idx], (0, 2, 1)),
                np.transpose(self.down[idx], (0, 2, 1)))

    def device_experts(self):
        """(gates, ups, downs, shared_dim padded) -- lists of device tensors in
        the GGUF orientation, uploaded once."""
        if self._dev is None:
            if self._q:
                self._dev = (self._qg, self._qu, self._qd, self.shared_dim)
            else:
                hp, ip = _round256(self.shared_dim), _round256(self.expert_dim)
                gs = [as_qtensor(_pad_to(self.gate[e], ip, hp)) for e in range(self.num_experts)]
                us = [as_qtensor(_pad_to(self.up[e], ip, hp)) for e in range(self.num_experts)]
                ds = [as_qtensor(_pad_to(self.down[e], hp, ip)) for e in range(self.num_experts)]
                self._dev = (gs, us, ds, hp)
        return self._dev

    def device_expert(self, idx: int):
        """One expert's device tensors (gate, up, down), uploading only it."""
        if self._dev is not None or self._q:
            g, u, d, _ = self.device_experts()
            return g[idx], u[idx], d[idx]
        return (as_qtensor(np.ascontiguousarray(self.gate[idx])), as_qtensor(np.ascontiguousarray(self.up[idx])),
                as_qtensor(np.ascontiguousarray(self.down[idx])))


def grouped_ffn(experts: MoEExpertSet, x2d: np.ndarray, logits: torch.Tensor, topk: int):
    """Route every token and run the grouped expert FFN on the GPU.
    Returns (out (T, shared_dim) fp32 numpy, indices, weights)."""
    gs, us, ds, hp = experts.device_experts()
    h = experts.shared_dim
    xp = np.zeros((x2d.shape[0], hp), dtype=np.float32)
    xp[:, :h] = x2d
    y, idx, w = moe_grouped_ffn(gs, us, ds, torch.from_numpy(xp), logits, topk)
    return y[:, :h].cpu().numpy(), idx.cpu().numpy().astype(np.int64), w.cpu().numpy()


# Tensor-name patterns of the two MoE naming conventions (vibeblade/moe.py:308-315)
_RE_GGUF_ROUTER = re.compile(r"^blk\.\d+\.ffn_gate_inp\.weight$")
_RE_GGUF_GATE = re.compile(r"^blk\.\d+\.ffn_gate_exps\.weight$")
_RE_GGUF_SHARED = re.compile(r"^blk\.\d+\.ffn_gate_shunt\.weight$")
_RE_ALT_ROUTER = re.compile(r"^blk\.\d+\.ffn_router\.weight$")
_RE_ALT_EXPERT = re.compile(r"^blk\.(\d+)\.expert\.(\d+)\.(ffn_gate|ffn_up|ffn_down)\.weight$")


def _orient_router(router_w: np.ndarray, gate_w: np.ndarray) -> np.ndarray:
    """(num_experts, hidden) GGUF router -> (hidden, num_experts)."""
    if router_w.ndim == 2 and gate_w.ndim >= 2:
        ne = gate_w.shape[0]
        if router_w.shape[0] == ne and router_w.shape[1] != ne:
            return router_w.T.copy()
    return router_w


def detect_moe_config(weights: dict) -> MoEConfig | None:
    """Detect an MoE layer from tensor names (vibeblade/moe.py:318-399)."""
    keys = set(weights.keys())
    routers = sorted(k for k in keys if _RE_GGUF_ROUTER.match(k))
    gates = sorted(k for k in keys if _RE_GGUF_GATE.match(k))
    if routers and gates:
        gate_w = weights[gates[0]]
        router_w = _orient_router(weights[routers[0]], gate_w)
        return MoEConfig(num_experts=int(router_w.shape[1]), num_active=2, expert_dim=int(gate_w.shape[1]),
                         shared_dim=int(router_w.shape[0]),
                         has_shared_expert=any(_RE_GGUF_SHARED.match(k) for k in keys))
    alt_routers = sorted(k for k in keys if _RE_ALT_ROUTER.match(k))
    alt_experts = sorted(k for k in keys if _RE_ALT_EXPERT.match(k))
    if alt_routers and alt_experts:
        router_w = weights[alt_routers[0]]
        shared_dim = int(router_w.shape[0])
        gate_keys = [k for k in alt_experts if ".ffn_gate.weight" in k]
        sample = weights[gate_keys[0] if gate_keys else alt_experts[0]]
        expert_dim = int(sample.shape[0])
        if sample.ndim == 2 and sample.shape[0] == shared_dim:
            expert_dim = int(sample.shape[1])
        return MoEConfig(num_experts=int(router_w.shape[1]), num_active=2, expert_dim=expert_dim,
                         shared_dim=shared_dim)
    return None


def load_moe_weights_from_layer(weights: dict, layer_idx: int):
    """(router_weight, MoEExpertSet, extra) of layer `layer_idx`, or
    (None, None, extra) (vibeblade/moe.py:508-608)."""
    pfx = f"blk.{layer_idx}"
    keys = set(weights.keys())
    extra: dict = {}
    router_w = gate_w = up_w = down_w = None
    if f"{pfx}.ffn_gate_inp.weight" in keys and f"{pfx}.ffn_gate_exps.weight" in keys:
        gate_w = weights[f"{pfx}.ffn_gate_exps.weight"]
        up_w = weights.get(f"{pfx}.ffn_up_exps.weight")
        down_w = weights.get(f"{pfx}.ffn_down_exps.weight")
        router_w = _orient_router(weights[f"{pfx}.ffn_gate_inp.weight"], gate_w)
        for suffix in ("shexp", "shunt"):
            gk = f"{pfx}.ffn_gate_{suffix}.weight"
            if gk in keys:
                extra["shared_gate"] = weights[gk]
                if f"{pfx}.ffn_up_{suffix}.weight" in keys:
                    extra["shared_up"] = weights[f"{pfx}.ffn_up_{suffix}.weight"]
                if f"{pfx}.ffn_down_{suffix}.weight" in keys:
                    extra["shared_down"] = weights[f"{pfx}.ffn_down_{suffix}.weight"]
                break
    elif f"{pfx}.ffn_router.weight" in keys:
        router_w = weights[f"{pfx}.ffn_router.weight"]
        g, u, d = [], [], []
        for e in range(int(router_w.shape[1])):
            for lst, name in ((g, "ffn_gate"), (u, "ffn_up"), (d, "ffn_down")):
                k = f"{pfx}.expert.{e}.{name}.weight"
                if k in keys:
                    lst.append(weights[k])
        if g and u and d:
            gate_w, up_w, down_w = np.stack(g), np.stack(u), np.stack(d)
    if router_w is None or gate_w is None or up_w is None or down_w is None:
        return None, None, extra
    return router_w, MoEExpertSet(gate_w, up_w, down_w), extra


_load_moe_weights_from_layer = load_moe_weights_from_layer


def moe_ffn_silu(x: np.ndarray, router: ExpertRouter, experts: MoEExpertSet, shared_expert_gate=None,
                 shared_expert_up=None, shared_expert_down=None):
    """MoE SwiGLU FFN (vibeblade/moe.py:407-500): route every token to its
    top-k experts, weighted sum of the expert FFNs, plus the optional shared
    expert (MoE weight convention).  Returns (output, stats)."""
    squeeze = np.asarray(x).ndim == 1
    x2 = np.atleast_2d(np.asarray(x, dtype=np.float32))
    logits = router._logits_dev(x2)
    moe_out, indices, weights = grouped_ffn(experts, x2, logits, router.topk)
    has_shared = shared_expert_gate is not None
    if has_shared:
        moe_out = moe_out + np.atleast_2d(_dense_ffn(x2, shared_expert_gate, shared_expert_up, shared_expert_down))
    output = _sanitize(moe_out)
    stats = {
        "expert_indices": indices,
        "expert_weights": weights,
        "num_experts": experts.num_experts,
        "topk": router.topk,
        "has_shared_expert": has_shared,
        "batch_size": x2.shape[0],
    }
    return (output[0] if squeeze else output), stats
