"""TurboSparse activation-sparse FFN -- drop-in for vibeblade/sparse.py.

Same names, signatures, return shapes and stats dicts as the reference
module (vibeblade/sparse.py:30-650).  The matrix work runs on the GPU through
libvbhip; weights may be fp32 arrays in the reference's orientation (uploaded
as exact GGUF F32 tensors) or ``QTensor`` handles of GGUF-quantized weights
(Q8_0 / Q4_K / Q6_K) resident in HBM, which is the path this package exists
for.  Results are fp32 (the reference returns the numpy result dtype).

Host-side helpers that only build masks or apply thresholds to arrays the
caller holds (``drelu_activation``, ``drelu_gate``, ``predict_activations``,
``compute_sparsity``, ``topk_activation_mask``, ``batch_drelu`` and the
predictor bookkeeping) keep the reference's numpy semantics: they have no
matrix work to offload.
"""
from __future__ import annotations

import numpy as np
import torch

from .tensor import QTensor, as_qtensor, gemv, sparse_ffn, topk_indices, activation, ACT_SILU, DOWN_GGUF

__all__ = [
    "drelu_activation", "drelu_gate", "predict_activations", "compute_sparsity", "sparse_matmul",
    "topk_activation_mask", "batch_drelu", "sparse_ffn_silu", "silu", "SparsePredictor",
    "EMANeuronPredictor", "DeviceEMAPredictor",
]


def drelu_activation(x: np.ndarray, threshold: float = 0.0) -> np.ndarray:
    """``x * (x > threshold)`` (vibeblade/sparse.py:30-45)."""
    return x * (x > threshold).astype(np.float64)


def drelu_gate(x: np.ndarray) -> np.ndarray:
    """``max(0, x) * max(0, -x)`` -- identically zero, as in the reference
    (vibeblade/sparse.py:48-73)."""
    return np.maximum(0, x) * np.maximum(0, -x)


def predict_activations(x: np.ndarray, threshold: float = 0.0) -> np.ndarray:
    """Boolean mask ``x > threshold`` (vibeblade/sparse.py:76-91)."""
    return x > threshold


def compute_sparsity(x: np.ndarray, threshold: float = 0.0) -> float:
    """Fraction of entries ``<= threshold``; 0.0 for an empty array
    (vibeblade/sparse.py:94-113)."""
    total = x.size
    if total == 0:
        return 0.0
    return float(np.count_nonzero(x <= threshold)) / float(total)


def _device_weight_rows(w) -> QTensor:
    """Weights given as (hidden, output) fp32 -> device tensor of `output` rows."""
    if isinstance(w, QTensor):
        return w
    return as_qtensor(np.ascontiguousarray(np.asarray(w, dtype=np.float32).T))


def _rows_matmul(a: np.ndarray, w: QTensor) -> np.ndarray:
    """(seq, k) fp32 activations times a device weight (rows = outputs)."""
    dev_a = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(w.device)
    out = torch.empty((dev_a.shape[0], w.rows), dtype=torch.float32, device=w.device)
    for t in range(dev_a.shape[0]):
        gemv(w, dev_a[t], out=out[t])
    return out.cpu().numpy()


def sparse_matmul(activations: np.ndarray, weights, mask: np.ndarray) -> np.ndarray:
    """``(activations * mask) @ weights`` (vibeblade/sparse.py:116-139).

    ``weights``: (hidden, output) fp32, or a ``QTensor`` of ``output`` rows by
    ``hidden`` (GGUF orientation).  Computed on the GPU in fp32."""
    acts = np.atleast_2d(np.asarray(activations))
    masked = (acts * np.asarray(mask)[np.newaxis, :]).astype(np.float32)
    return _rows_matmul(masked, _device_weight_rows(weights))


def topk_activation_mask(x: np.ndarray, k: int) -> np.ndarray:
    """Boolean mask with the top-k entries of each row set
    (vibeblade/sparse.py:142-168).  Ties resolve to the lowest indices."""
    x = np.asarray(x)
    if k <= 0:
        return np.zeros_like(x, dtype=bool)
    if k >= x.shape[1]:
        return np.ones_like(x, dtype=bool)
    order = np.argsort(-x, axis=1, kind="stable")[:, :k]
    mask = np.zeros_like(x, dtype=bool)
    mask[np.arange(x.shape[0])[:, None], order] = True
    return mask


def batch_drelu(x: np.ndarray, threshold: float = 0.0):
    """``(x * (x > threshold), x > threshold)`` (vibeblade/sparse.py:171-191)."""
    mask = x > threshold
    return x * mask.astype(np.float64), mask


def silu(x: np.ndarray) -> np.ndarray:
    """SiLU on the GPU, fp32 (vibeblade/sparse.py:286-289)."""
    a = np.asarray(x, dtype=np.float32)
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return activation(t, ACT_SILU).cpu().numpy().reshape(a.shape)


def sparse_ffn_silu(x: np.ndarray, gate_w, up_w, down_w, sparse_ratio: float = 0.1):
    """PowerInfer-style sparse SwiGLU FFN (vibeblade/sparse.py:199-283).

    x: (seq, hidden).  gate_w / up_w: (intermediate, hidden); down_w:
    (hidden, intermediate) -- fp32 arrays or ``QTensor`` handles of the same
    orientation (GGUF).  Steps, all on the GPU: dense gate GEMV, top-k of the
    gate per token (k = max(1, int(intermediate * sparse_ratio))), the union
    of the per-token sets for seq > 1, then the fused sparse FFN over the
    sorted active set (gate and up on the active rows only, silu(g) * u, down
    over the active columns).  Returns (out (seq, hidden) fp32, stats)."""
    x = np.atleast_2d(np.asarray(x, dtype=np.float32))
    g = gate_w if isinstance(gate_w, QTensor) else as_qtensor(gate_w)
    u = up_w if isinstance(up_w, QTensor) else as_qtensor(up_w)
    d = down_w if isinstance(down_w, QTensor) else as_qtensor(down_w)
    inter, hidden = g.rows, g.k
    if x.shape[1] != hidden:
        raise ValueError(f"x has hidden size {x.shape[1]}, weights expect {hidden}")
    k = max(1, int(inter * sparse_ratio))
    dev = g.device
    xt = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    sets = []
    for t in range(x.shape[0]):
        gate = gemv(g, xt[t])
        sets.append(topk_indices(gate, min(k, inter)))
    if len(sets) == 1:
        active = sets[0]
    else:  # neuron active for any position (vibeblade/sparse.py:256-259)
        active = torch.from_numpy(np.unique(torch.cat(sets).cpu().numpy()).astype(np.int32)).to(dev)
    out = torch.empty((x.shape[0], hidden), dtype=torch.float32, device=dev)
    for t in range(x.shape[0]):
        sparse_ffn(g, u, d, xt[t], active, ACT_SILU, DOWN_GGUF, out=out[t])
    n_active = int(active.numel())
    stats = {
        "active_neurons": n_active,
        "total_neurons": inter,
        "sparsity_ratio": 1.0 - (n_active / inter),
    }
    return out.cpu().numpy(), stats


def _gate_values(hidden_state: np.ndarray, gate_w) -> np.ndarray:
    g = gate_w if isinstance(gate_w, QTensor) else as_qtensor(gate_w)
    xt = torch.from_numpy(np.ascontiguousarray(np.atleast_2d(hidden_state)[0], dtype=np.float32)).to(g.device)
    return gemv(g, xt).cpu().numpy()


class SparsePredictor:
    """Per-layer neuron predictor (vibeblade/sparse.py:292-423); the gate
    projection runs on the GPU, the activation statistics stay on the host."""

    def __init__(self, n_layers: int, intermediate_dim: int, sparse_ratio: float = 0.1, mode: str = "online"):
        self.n_layers = n_layers
        self.intermediate_dim = intermediate_dim
        self.sparse_ratio = sparse_ratio
        self.mode = mode
        self.heavy_hitters = [np.array([], dtype=np.int64) for _ in range(n_layers)]
        self._activation_counts = [np.zeros(intermediate_dim, dtype=np.float64) for _ in range(n_layers)]
        self._calibration_samples = 0

    def calibrate_update(self, layer_idx: int, hidden_state: np.ndarray, gate_w) -> None:
        if layer_idx >= self.n_layers:
            return
        gate = _gate_values(hidden_state, gate_w)
        self._activation_counts[layer_idx] += (gate > 0).astype(np.float64)
        self._calibration_samples += 1

    def calibrate_finish(self, threshold_ratio: float = 0.3) -> None:
        for layer_idx in range(self.n_layers):
            counts = self._activation_counts[layer_idx]
            if self._calibration_samples > 0:
                freq = counts / self._calibration_samples
                self.heavy_hitters[layer_idx] = np.where(freq >= threshold_ratio)[0].astype(np.int64)
            min_k = max(1, int(len(counts) * self.sparse_ratio))
            if len(self.heavy_hitters[layer_idx]) < min_k:
                top = np.argsort(-counts, kind="stable")[:min_k]
                self.heavy_hitters[layer_idx] = np.sort(np.unique(np.concatenate([self.heavy_hitters[layer_idx], top])))
        self.mode = "offline"

    def predict(self, layer_idx: int, hidden_state: np.ndarray, gate_w) -> np.ndarray:
        g = gate_w if isinstance(gate_w, QTensor) else None
        inter = g.rows if g is not None else np.asarray(gate_w).shape[0]
        k = max(1, int(inter * self.sparse_ratio))
        if self.mode == "offline" and len(self.heavy_hitters[layer_idx]) > 0:
            mask = np.zeros(inter, dtype=bool)
            mask[self.heavy_hitters[layer_idx]] = True
            return mask
        gq = g if g is not None else as_qtensor(gate_w)
        xt = torch.from_numpy(np.ascontiguousarray(np.atleast_2d(hidden_state)[0], dtype=np.float32)).to(gq.device)
        idx = topk_indices(gemv(gq, xt), min(k, inter)).cpu().numpy()
        mask = np.zeros(inter, dtype=bool)
        mask[idx] = True
        return mask

    @property
    def is_calibrated(self) -> bool:
        return self.mode == "offline"


class EMANeuronPredictor:
    """EMA neuron-activation predictor (vibeblade/sparse.py:431-650): host
    bookkeeping of per-neuron activation probabilities."""

    def __init__(self, hidden_dim: int, n_layers: int, ema_decay: float = 0.1, sparse_ratio: float = 0.1,
                 activation_threshold: float = 0.3) -> None:
        self.hidden_dim = hidden_dim
        self.n_layers = n_layers
        self.ema_decay = ema_decay
        self.sparse_ratio = sparse_ratio
        self.activation_threshold = activation_threshold
        self._ema_probs = np.zeros((n_layers, hidden_dim), dtype=np.float32)
        self._update_counts = np.zeros(n_layers, dtype=np.int32)
        self._total_updates = 0

    def update(self, layer_idx: int, activation_mask: np.ndarray) -> None:
        if layer_idx < 0 or layer_idx >= self.n_layers:
            return
        obs = activation_mask.astype(np.float32)
        a = self.ema_decay
        self._ema_probs[layer_idx] = a * obs + (1.0 - a) * self._ema_probs[layer_idx]
        self._update_counts[layer_idx] += 1
        self._total_updates += 1

    def _topk_mask(self, values: np.ndarray, k: int) -> np.ndarray:
        mask = np.zeros(self.hidden_dim, dtype=bool)
        mask[np.argsort(-values, kind="stable")[:k]] = True
        return mask

    def predict(self, layer_idx: int, gate_values: np.ndarray | None = None) -> np.ndarray:
        if layer_idx < 0 or layer_idx >= self.n_layers:
            return np.ones(self.hidden_dim, dtype=bool)
        k = max(1, int(self.hidden_dim * self.sparse_ratio))
        probs = self._ema_probs[layer_idx]
        if self._update_counts[layer_idx] > 5:
            ema_mask = probs >= self.activation_threshold
            if np.sum(ema_mask) < k:
                remaining = k - int(np.sum(ema_mask))
                inactive = np.where(~ema_mask)[0]
                if len(inactive) > 0:
                    order = inactive[np.argsort(-probs[inactive], kind="stable")[:remaining]]
                    ema_mask[order] = True
            return ema_mask
        if gate_values is not None:
            return self._topk_mask(np.asarray(gate_values), k)
        mask = np.zeros(self.hidden_dim, dtype=bool)
        mask[:k] = True
        return mask

    def predict_combined(self, layer_idx: int, gate_values: np.ndarray) -> np.ndarray:
        ema_mask = self.predict(layer_idx, gate_values=None)
        k = max(1, int(self.hidden_dim * self.sparse_ratio))
        return ema_mask | self._topk_mask(np.asarray(gate_values), k)

    def get_activation_probabilities(self, layer_idx: int) -> np.ndarray:
        if 0 <= layer_idx < self.n_layers:
            return self._ema_probs[layer_idx].copy()
        return np.zeros(self.hidden_dim, dtype=np.float32)

    def get_top_neurons(self, layer_idx: int, k: int = 10) -> np.ndarray:
        probs = self.get_activation_probabilities(layer_idx)
        top_k = min(k, self.hidden_dim)
        return np.argsort(-probs, kind="stable")[:top_k]

    @property
    def total_updates(self) -> int:
        return self._total_updates

    @property
    def is_warmed_up(self) -> bool:
        return bool(np.all(self._update_counts > 5))

    def reset(self) -> None:
        self._ema_probs.fill(0)
        self._update_counts.fill(0)
        self._total_updates = 0


class DeviceEMAPredictor:
    """EMANeuronPredictor (vibeblade/sparse.py:431-650) with its state on the
    GPU: the per-layer probabilities live in device memory and update,
    predict and the active-index compaction are device launches
    (vb_ema_update, vb_ema_predict), so a decode step hands its predicted
    active set to the sparse FFN block (``sparse_ffn(..., count=)``) without a
    host round trip.

    Same constructor arguments, methods and results as ``EMANeuronPredictor``
    (ties at a top-k threshold go to the lowest indices; the EMA step is
    bit-identical).  ``predict`` / ``predict_combined`` return numpy bool
    masks like the reference (one device-to-host copy); ``predict_active``
    keeps everything on the device.  The warm-up counters stay on the host:
    they decide which rule a prediction uses."""

    def __init__(self, hidden_dim: int, n_layers: int, ema_decay: float = 0.1, sparse_ratio: float = 0.1,
                 activation_threshold: float = 0.3, device=None) -> None:
        from .tensor import _dev
        self.hidden_dim = hidden_dim
        self.n_layers = n_layers
        self.ema_decay = ema_decay
        self.sparse_ratio = sparse_ratio
        self.activation_threshold = activation_threshold
        self.device = _dev(device)
        self._probs = torch.zeros((n_layers, hidden_dim), dtype=torch.float32, device=self.device)
        self._update_counts = np.zeros(n_layers, dtype=np.int32)
        self._total_updates = 0

    def _k(self) -> int:
        return min(self.hidden_dim, max(1, int(self.hidden_dim * self.sparse_ratio)))

    def update(self, layer_idx: int, activation_mask) -> None:
        """EMA step with an observed mask: numpy bool array, or a device
        bool / uint8 tensor (e.g. the mask of ``predict_active``)."""
        from . import _lib
        from .tensor import _stream
        if layer_idx < 0 or layer_idx >= self.n_layers:
            return
        m = torch.as_tensor(activation_mask).to(device=self.device, dtype=torch.uint8).contiguous().reshape(-1)
        if m.numel() != self.hidden_dim:
            raise ValueError(f"update: mask has {m.numel()} entries, expected {self.hidden_dim}")
        _lib.call("vb_ema_update", self._probs[layer_idx].data_ptr(), self.hidden_dim, m.data_ptr(),
                  float(self.ema_decay), _stream())
        self._update_counts[layer_idx] += 1
        self._total_updates += 1

    def predict_active(self, layer_idx: int, gate_values=None, combined: bool = False):
        """(active int32 indices ascending, count int32 (1,), mask uint8) on
        the device; ``active`` has room for every neuron and is valid up to
        ``count``.  combined: the ``predict_combined`` rule."""
        from . import _lib
        from .tensor import _stream
        n = self.hidden_dim
        active = torch.empty(n, dtype=torch.int32, device=self.device)
        count = torch.empty(1, dtype=torch.int32, device=self.device)
        mask = torch.empty(n, dtype=torch.uint8, device=self.device)
        if layer_idx < 0 or layer_idx >= self.n_layers:  # the reference: every neuron
            torch.arange(n, dtype=torch.int32, device=self.device, out=active)
            count.fill_(n)
            mask.fill_(1)
            return active, count, mask
        g = None
        if gate_values is not None:
            g = torch.as_tensor(gate_values).to(device=self.device, dtype=torch.float32).contiguous().reshape(-1)
            if g.numel() != n:
                raise ValueError(f"predict: gate_values has {g.numel()} entries, expected {n}")
        if combined and g is None:
            raise ValueError("predict_combined needs gate_values")
        warm = int(self._update_counts[layer_idx] > 5)
        _lib.call("vb_ema_predict", self._probs[layer_idx].data_ptr(), None if g is None else g.data_ptr(), n,
                  self._k(), float(self.activation_threshold), warm, int(bool(combined)), mask.data_ptr(),
                  active.data_ptr(), count.data_ptr(), _stream())
        return active, count, mask

    def predict(self, layer_idx: int, gate_values=None) -> np.ndarray:
        return self.predict_active(layer_idx, gate_values)[2].cpu().numpy().astype(bool)

    def predict_combined(self, layer_idx: int, gate_values) -> np.ndarray:
        return self.predict_active(layer_idx, gate_values, combined=True)[2].cpu().numpy().astype(bool)

    def get_activation_probabilities(self, layer_idx: int) -> np.ndarray:
        if 0 <= layer_idx < self.n_layers:
            return self._probs[layer_idx].cpu().numpy().copy()
        return np.zeros(self.hidden_dim, dtype=np.float32)

    def get_top_neurons(self, layer_idx: int, k: int = 10) -> np.ndarray:
        probs = self.get_activation_probabilities(layer_idx)
        return np.argsort(-probs, kind="stable")[:min(k, self.hidden_dim)]

    @property
    def total_updates(self) -> int:
        return self._total_updates

    @property
    def is_warmed_up(self) -> bool:
        return bool(np.all(self._update_counts > 5))

    def reset(self) -> None:
        self._probs.zero_()
        self._update_counts.fill(0)
        self._total_updates = 0
