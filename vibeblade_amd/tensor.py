"""Device-resident GGUF tensors and the functional ops over them.

``QTensor`` holds one GGUF weight matrix in HBM in its on-disk block layout:
``rows`` outputs x ``k`` inputs, each row a run of blocks along k.  PyTorch
provides the device memory and the stream; every op below is one or more
libvbhip launches on ``torch.cuda.current_stream()``.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from . import ggml


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(device=None) -> torch.device:
    d = torch.device(device if device is not None else "cuda")
    if d.type != "cuda":
        raise ValueError("vibeblade_amd ops run on the GPU only (device must be cuda)")
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU visible: vibeblade_amd has no CPU path")
    idx = d.index if d.index is not None else torch.cuda.current_device()
    _lib.init(idx)
    return torch.device("cuda", idx)


def _as_f32_dev(x, device) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        t = x.to(device=device, dtype=torch.float32)
    else:
        t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(device)
    return t.contiguous()


class QTensor:
    """A GGUF tensor (rows x k, type ``qtype``) resident on one GPU."""

    def __init__(self, data: torch.Tensor, qtype: int, rows: int, k: int):
        rb = ggml.row_bytes(qtype, k)
        if data.dtype != torch.uint8 or data.device.type != "cuda":
            raise ValueError("QTensor data must be a cuda uint8 tensor")
        if data.numel() != rows * rb:
            raise ValueError(f"QTensor: {data.numel()} bytes != {rows} rows x {rb}")
        if qtype not in ggml.DEVICE_TYPES:
            raise ValueError(f"no device kernels for ggml type {qtype}")
        self.data = data.contiguous().view(rows, rb)
        self.qtype = int(qtype)
        self.rows = int(rows)
        self.k = int(k)

    @property
    def shape(self) -> tuple:
        return (self.rows, self.k)

    @property
    def nbytes(self) -> int:
        return self.data.numel()

    @property
    def device(self) -> torch.device:
        return self.data.device

    def ptr(self) -> int:
        return self.data.data_ptr()

    def __repr__(self) -> str:
        return f"QTensor({ggml.NAMES[self.qtype]}, rows={self.rows}, k={self.k}, {self.device})"

    @classmethod
    def from_bytes(cls, raw, qtype: int, rows: int, k: int, device=None) -> "QTensor":
        """Upload GGUF bytes (numpy/bytes/torch uint8, rows*row_bytes long)."""
        dev = _dev(device)
        if isinstance(raw, torch.Tensor):
            t = raw.to(device=dev, dtype=torch.uint8).reshape(-1)
        else:
            arr = np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray)) \
                else np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
            t = torch.from_numpy(arr.copy()).to(dev)
        return cls(t, qtype, rows, k)

    @classmethod
    def quantize(cls, w, qtype: int, device=None) -> "QTensor":
        """Quantize an fp32 (rows, k) matrix on the device (vb_quantize_rows)."""
        dev = _dev(device if device is not None else
                   (w.device if isinstance(w, torch.Tensor) and w.is_cuda else None))
        src = _as_f32_dev(w, dev)
        if src.dim() != 2:
            raise ValueError("quantize expects a 2-D (rows, k) matrix")
        rows, k = src.shape
        out = torch.empty(rows * ggml.row_bytes(qtype, k), dtype=torch.uint8, device=dev)
        _lib.call("vb_quantize_rows", src.data_ptr(), out.data_ptr(), rows, k, qtype, _stream())
        return cls(out, qtype, rows, k)

    def dequantize(self) -> torch.Tensor:
        """Decode to fp32 (rows, k) on the device (vb_dequant_rows)."""
        out = torch.empty((self.rows, self.k), dtype=torch.float32, device=self.device)
        _lib.call("vb_dequant_rows", self.ptr(), out.data_ptr(), self.rows, self.k,
                  self.qtype, _stream())
        return out

    def to_numpy_bytes(self) -> np.ndarray:
        return self.data.cpu().numpy()


def gemv(w: QTensor, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = W x for one activation vector (len k) -> (rows,) fp32."""
    x = _as_f32_dev(x, w.device).reshape(-1)
    if x.numel() != w.k:
        raise ValueError(f"gemv: x has {x.numel()} elements, W has k={w.k}")
    if out is None:
        out = torch.empty(w.rows, dtype=torch.float32, device=w.device)
    _lib.call("vb_gemv", w.ptr(), x.data_ptr(), out.data_ptr(), w.rows, w.k, w.qtype, _stream())
    return out


X_F32 = 0
X_F16 = 1
GEMM_AUTO, GEMM_SKINNY, GEMM_TILED = 0, 1, 2


def gemm(w: QTensor, x: torch.Tensor, out: torch.Tensor | None = None,
         variant: int = GEMM_AUTO) -> torch.Tensor:
    """Y = X W^T for a batch of activations X (m, k) fp16 or fp32 -> (m, rows) fp32
    (MFMA path; fp16 operands, fp32 accumulation)."""
    if not isinstance(x, torch.Tensor):
        x = torch.from_numpy(np.ascontiguousarray(x))
    x = x.to(w.device)
    if x.dtype not in (torch.float16, torch.float32):
        x = x.to(torch.float32)
    x = x.contiguous()
    if x.dim() != 2 or x.shape[1] != w.k:
        raise ValueError(f"gemm: x must be (m, {w.k}), got {tuple(x.shape)}")
    m = x.shape[0]
    if out is None:
        out = torch.empty((m, w.rows), dtype=torch.float32, device=w.device)
    xdt = X_F16 if x.dtype == torch.float16 else X_F32
    _lib.call("vb_gemm", w.ptr(), x.data_ptr(), xdt, out.data_ptr(), m, w.rows, w.k, w.qtype,
              variant, _stream())
    return out
