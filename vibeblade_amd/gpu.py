"""HIP backend with the ``GPUBackend`` duck type (vibeblade/gpu.py:40-198).

``HipBackend`` (also exported as ``GPUBackend``) is the device hook the MoE
executor and callers use: ``is_gpu``, ``drelu``, ``silu``, ``rms_norm``,
``softmax`` and ``matmul`` run as libvbhip kernels on the GPU.  ``matmul``
also takes a ``QTensor`` for ``b`` (GGUF orientation: rows = outputs), which
is the dequant-fused quantized path (GEMV per row, or the MFMA GEMM for Q4_K
with two or more rows).  There is no numpy fallback.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ggml
from .tensor import QTensor, as_qtensor, gemv, gemm, activation, _dev, _stream
from . import _lib

__all__ = ["GPUBackend", "HipBackend", "available_backends"]


def available_backends() -> list:
    """Backends this package provides ("hip" when a GPU is visible)."""
    return ["hip"] if torch.cuda.is_available() else []


def _to_dev(a, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=np.float32))).to(device)


class HipBackend:
    """gfx950 backend; ``backend`` accepts "auto" or "hip"."""

    def __init__(self, backend: str = "auto", device_index: int = 0):
        if backend not in ("auto", "hip"):
            raise ValueError(f"Unknown backend '{backend}'. Choose from: {available_backends()}")
        self.backend_name = "hip"
        self._device = _dev(f"cuda:{device_index}")
        self._device_name = torch.cuda.get_device_name(self._device)

    def __repr__(self) -> str:
        return f"GPUBackend(backend={self.backend_name!r}, device={self._device_name!r})"

    @property
    def is_gpu(self) -> bool:
        return True

    def drelu(self, x: np.ndarray) -> np.ndarray:
        """max(x, 0) (vibeblade/gpu.py:100-111)."""
        a = np.asarray(x, dtype=np.float32)
        return activation(_to_dev(a, self._device), 1).cpu().numpy().reshape(a.shape)

    def silu(self, x: np.ndarray) -> np.ndarray:
        """x * sigmoid(x) (vibeblade/gpu.py:113-124)."""
        a = np.asarray(x, dtype=np.float32)
        return activation(_to_dev(a, self._device), 0).cpu().numpy().reshape(a.shape)

    def rms_norm(self, x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
        """x / sqrt(mean(x^2) + eps) * weight over the last axis (vibeblade/gpu.py:126-146)."""
        a = np.asarray(x, dtype=np.float32)
        w = np.asarray(weight, dtype=np.float32)
        xt = _to_dev(a.reshape(-1, w.shape[0]), self._device)
        out = torch.empty_like(xt)
        _lib.call("vb_rms_norm", xt.data_ptr(), _to_dev(w, self._device).data_ptr(), out.data_ptr(),
                  xt.shape[0], w.shape[0], float(eps), _stream())
        return out.cpu().numpy().reshape(a.shape)

    def softmax(self, x: np.ndarray, axis: int = -1) -> np.ndarray:
        """Softmax along `axis` (vibeblade/gpu.py:192-198)."""
        a = np.moveaxis(np.asarray(x, dtype=np.float32), axis, -1)
        xt = _to_dev(a.reshape(-1, a.shape[-1]), self._device)
        out = torch.empty_like(xt)
        _lib.call("vb_softmax", xt.data_ptr(), out.data_ptr(), xt.shape[0], xt.shape[1], _stream())
        return np.moveaxis(out.cpu().numpy().reshape(a.shape), -1, axis)

    def matmul(self, a: np.ndarray, b) -> np.ndarray:
        """C = A x B (vibeblade/gpu.py:148-168).  a: (M, K) fp32.  b: (K, N)
        fp32, or a ``QTensor`` with N rows of K (GGUF orientation)."""
        a2 = np.atleast_2d(np.asarray(a, dtype=np.float32))
        w = b if isinstance(b, QTensor) else as_qtensor(np.ascontiguousarray(np.asarray(b, dtype=np.float32).T),
                                                        device=self._device)
        if a2.shape[1] != w.k:
            raise ValueError(f"matmul: a has {a2.shape[1]} columns, b has {w.k} rows")
        xt = _to_dev(a2, w.device)
        if w.qtype == ggml.GGML_TYPE_Q4_K and a2.shape[0] >= 2:
            return gemm(w, xt).cpu().numpy()
        out = torch.empty((a2.shape[0], w.rows), dtype=torch.float32, device=w.device)
        for t in range(a2.shape[0]):
            gemv(w, xt[t], out=out[t])
        return out.cpu().numpy()

    def rotor_unpack(self, packed: np.ndarray, rotor: np.ndarray, n: int) -> np.ndarray:
        """4-bit unpack with per-group rotor scaling (vibeblade/gpu.py:170-190,
        the reference's numpy path; RotorQuant is not a GGUF format)."""
        from .quant import unpack_nibbles
        unpacked = unpack_nibbles(packed, n).astype(np.float32)
        for i in range(0, n, 4):
            g = min(4, n - i)
            r = rotor[i:i + g] if rotor.ndim == 1 else np.diag(rotor[:g, :g])
            unpacked[i:i + g] *= r[:g]
        return unpacked


GPUBackend = HipBackend
