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


def _check_out(out: torch.Tensor, numel: int, device, what: str) -> torch.Tensor:
    """A caller-supplied output must be a contiguous fp32 tensor of exactly
    ``numel`` elements on ``device``: the kernels write through its pointer."""
    if not isinstance(out, torch.Tensor):
        raise ValueError(f"{what}: out must be a torch tensor")
    if out.dtype != torch.float32 or out.device != torch.device(device) or not out.is_contiguous():
        raise ValueError(f"{what}: out must be a contiguous float32 tensor on {device} "
                         f"(got {out.dtype} on {out.device}, contiguous={out.is_contiguous()})")
    if out.numel() != numel:
        raise ValueError(f"{what}: out has {out.numel()} elements, {numel} expected")
    return out


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


def embed_rows(table: QTensor, tokens, out: torch.Tensor | None = None) -> torch.Tensor:
    """Decoded rows ``tokens`` of an embedding table, (n_tokens, k) fp32 on
    the device (vb_embed_rows; ids outside the table give zero rows)."""
    dev = table.device
    ids = torch.as_tensor(tokens, dtype=torch.int32).to(dev).contiguous().reshape(-1)
    n = ids.numel()
    if out is None:
        out = torch.empty((n, table.k), dtype=torch.float32, device=dev)
    _check_out(out, n * table.k, dev, "embed_rows")
    _lib.call("vb_embed_rows", table.ptr(), table.qtype, table.rows, table.k, ids.data_ptr() if n else None, n,
              out.data_ptr(), _stream())
    return out


def gemv(w: QTensor, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = W x for one activation vector (len k) -> (rows,) fp32."""
    x = _as_f32_dev(x, w.device).reshape(-1)
    if x.numel() != w.k:
        raise ValueError(f"gemv: x has {x.numel()} elements, W has k={w.k}")
    if out is None:
        out = torch.empty(w.rows, dtype=torch.float32, device=w.device)
    _check_out(out, w.rows, w.device, "gemv")
    _lib.call("vb_gemv", w.ptr(), x.data_ptr(), out.data_ptr(), w.rows, w.k, w.qtype, _stream())
    return out


X_F32 = 0
X_F16 = 1
GEMM_AUTO, GEMM_SKINNY, GEMM_TILED, GEMM_SPLIT, GEMM_KSPLIT, GEMM_XREG = 0, 1, 2, 3, 4, 5


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
    _check_out(out, m * w.rows, w.device, "gemm")
    xdt = X_F16 if x.dtype == torch.float16 else X_F32
    lib = _lib.load()
    nb = int(lib.vb_gemm_workspace(m, w.rows, w.k, w.qtype, xdt, variant))
    if nb > 0:
        # the packed-X kernel's workspace, from torch's caching allocator
        ws = torch.empty(nb, dtype=torch.uint8, device=w.device)
        _lib.call("vb_gemm_ws", w.ptr(), x.data_ptr(), xdt, out.data_ptr(), m, w.rows, w.k, w.qtype,
                  variant, ws.data_ptr(), nb, _stream())
        return out
    _lib.call("vb_gemm", w.ptr(), x.data_ptr(), xdt, out.data_ptr(), m, w.rows, w.k, w.qtype,
              variant, _stream())
    return out


def as_qtensor(w, device=None) -> QTensor:
    """A QTensor as is; an fp32 (rows, k) array / tensor uploaded as a GGUF
    F32 tensor (no quantization: the values stay exact)."""
    if isinstance(w, QTensor):
        return w
    dev = _dev(device if device is not None else
               (w.device if isinstance(w, torch.Tensor) and w.is_cuda else None))
    t = _as_f32_dev(w, dev)
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D weight matrix, got shape {tuple(t.shape)}")
    rows, k = t.shape
    return QTensor(t.contiguous().view(torch.uint8).reshape(-1), ggml.GGML_TYPE_F32, rows, k)


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


ACT_SILU = 0   # silu(g) * u
ACT_RELU2 = 1  # relu(g) * relu(u)
ACT_GELU_TANH = 2  # gelu_tanh(g) * u (GeGLU)
DOWN_GGUF = 0          # down weight (h rows x i)
DOWN_NEURON_MAJOR = 1  # down^T (i rows x h)


def topk_indices(v: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest entries of a 1-D fp32 device vector, ascending
    (ties at the threshold go to the lowest indices)."""
    v = v.to(torch.float32).contiguous().reshape(-1)
    n = v.numel()
    k = int(k)
    if k < 0 or k > n:
        raise ValueError(f"topk_indices: k={k} out of range for n={n}")
    out = torch.empty(k, dtype=torch.int32, device=v.device)
    _lib.call("vb_topk_indices", v.data_ptr(), n, k, out.data_ptr(), _stream())
    return out


def sparse_ffn(gate: QTensor, up: QTensor, down: QTensor, x: torch.Tensor, active: torch.Tensor,
               act: int = ACT_SILU, down_layout: int = DOWN_GGUF,
               out: torch.Tensor | None = None, norm_w=None, eps: float = 1e-5,
               residual: bool = False, count: torch.Tensor | None = None) -> torch.Tensor:
    """One token through the activation-sparse FFN over the sorted active set.
    With ``norm_w`` the FFN input is rms_norm(x, norm_w, eps) (normalised
    inside the gate/up launch); with ``residual`` y = x + FFN (``out`` may
    be ``x``).  ``count``: a device int32 holding the set's size (an on-device
    prediction); ``active`` is then read up to it, with no host sync."""
    h, i = gate.k, gate.rows
    if up.shape != gate.shape or up.qtype != gate.qtype or down.qtype != gate.qtype:
        raise ValueError("sparse_ffn: gate/up/down must share shape conventions and type")
    want_down = (h, i) if down_layout == DOWN_GGUF else (i, h)
    if down.shape != want_down:
        raise ValueError(f"sparse_ffn: down has shape {down.shape}, expected {want_down}")
    dev = gate.device
    x = _as_f32_dev(x, dev).reshape(-1)
    if x.numel() != h:
        raise ValueError(f"sparse_ffn: x has {x.numel()} elements, expected {h}")
    active = active.to(device=dev, dtype=torch.int32).contiguous().reshape(-1)
    n_active = active.numel()
    if out is None:
        out = torch.empty(h, dtype=torch.float32, device=dev)
    _check_out(out, h, dev, "sparse_ffn")
    nbytes = _lib.load().vb_sparse_ffn_workspace(h, i, n_active, down_layout)
    if nbytes < 0:
        raise ValueError("sparse_ffn: bad shape")
    ws = _workspace(nbytes, dev)
    if count is not None:
        count = count.to(device=dev, dtype=torch.int32)
    if norm_w is None and not residual and count is None:
        _lib.call("vb_sparse_ffn", gate.ptr(), up.ptr(), down.ptr(), down_layout, x.data_ptr(),
                  active.data_ptr() if n_active else None, n_active, act, out.data_ptr(), h, i, gate.qtype,
                  ws.data_ptr(), ws.numel(), _stream())
        return out
    nw = None
    if norm_w is not None:
        nw = _as_f32_dev(norm_w, dev).reshape(-1)
        if nw.numel() != h:
            raise ValueError(f"sparse_ffn: norm_w has {nw.numel()} elements, expected {h}")
    _lib.call("vb_sparse_ffn_block", gate.ptr(), up.ptr(), down.ptr(), down_layout, x.data_ptr(),
              None if nw is None else nw.data_ptr(), float(eps), active.data_ptr() if n_active else None,
              n_active, None if count is None else count.data_ptr(), act, int(bool(residual)), out.data_ptr(), h, i,
              gate.qtype, ws.data_ptr(), ws.numel(), _stream())
    return out


def ffn_block(gate: QTensor, up: QTensor, down: QTensor, x: torch.Tensor, norm_w=None, eps: float = 1e-5,
              act: int = ACT_SILU, residual: bool = True, out: torch.Tensor | None = None) -> torch.Tensor:
    """One token through the FFN block: y = [x +] down(act(gate(n), up(n))),
    n = rms_norm(x, norm_w, eps) (n = x without norm_w).  Two launches for
    Q4_K / Q6_K / Q8_0 weights (vb_ffn_block).  ``out`` may be ``x``."""
    hd, inter = gate.k, gate.rows
    if up.shape != gate.shape or up.qtype != gate.qtype:
        raise ValueError("ffn_block: gate and up must have one shape and type")
    if down.shape != (hd, inter):
        raise ValueError(f"ffn_block: down has shape {down.shape}, expected {(hd, inter)}")
    dev = gate.device
    x = _as_f32_dev(x, dev).reshape(-1)
    if x.numel() != hd:
        raise ValueError(f"ffn_block: x has {x.numel()} elements, expected {hd}")
    nw = None
    if norm_w is not None:
        nw = _as_f32_dev(norm_w, dev).reshape(-1)
        if nw.numel() != hd:
            raise ValueError(f"ffn_block: norm_w has {nw.numel()} elements, expected {hd}")
    if out is None:
        out = torch.empty(hd, dtype=torch.float32, device=dev)
    _check_out(out, hd, dev, "ffn_block")
    ws = _workspace(_lib.load().vb_ffn_block_workspace(hd, inter), dev)
    _lib.call("vb_ffn_block", x.data_ptr(), None if nw is None else nw.data_ptr(), float(eps), gate.ptr(),
              up.ptr(), gate.qtype, down.ptr(), down.qtype, hd, inter, int(act), int(bool(residual)),
              out.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    return out


def moe_route(logits: torch.Tensor, topk: int):
    """(indices int32 (T, topk), weights fp32 (T, topk)) from router logits (T, E)."""
    logits = logits.to(torch.float32).contiguous()
    t, e = logits.shape
    idx = torch.empty((t, topk), dtype=torch.int32, device=logits.device)
    w = torch.empty((t, topk), dtype=torch.float32, device=logits.device)
    _lib.call("vb_moe_route", logits.data_ptr(), t, e, topk, idx.data_ptr(), w.data_ptr(), _stream())
    return idx, w


def moe_grouped_ffn(gates, ups, downs, x: torch.Tensor, logits: torch.Tensor, topk: int):
    """Top-k MoE over experts (lists of QTensors: gate/up i x h, down h x i;
    gate/up of one ggml type, down of the same or another).  Returns (y (T, h) fp32, indices (T, topk) int32, weights (T, topk) fp32)."""
    import ctypes
    n_exp = len(gates)
    if not (len(ups) == len(downs) == n_exp) or n_exp == 0:
        raise ValueError("moe_grouped_ffn: need the same number of gate/up/down experts")
    g0 = gates[0]
    h, i = g0.k, g0.rows
    gu_type, dn_type = g0.qtype, downs[0].qtype
    for e in range(n_exp):
        if gates[e].shape != (i, h) or ups[e].shape != (i, h) or downs[e].shape != (h, i):
            raise ValueError(f"moe_grouped_ffn: expert {e} has inconsistent shapes")
        if not (gates[e].qtype == ups[e].qtype == gu_type and downs[e].qtype == dn_type):
            raise ValueError("moe_grouped_ffn: every expert's gate/up must share one ggml type, "
                             "and every expert's down another (or the same)")
    dev = g0.device
    x = _as_f32_dev(x, dev)
    if x.dim() == 1:
        x = x.reshape(1, -1)
    t = x.shape[0]
    logits = _as_f32_dev(logits, dev).reshape(t, n_exp)
    y = torch.empty((t, h), dtype=torch.float32, device=dev)
    idx = torch.empty((t, topk), dtype=torch.int32, device=dev)
    w = torch.empty((t, topk), dtype=torch.float32, device=dev)
    arr = ctypes.c_void_p * n_exp
    pg = arr(*[g.ptr() for g in gates])
    pu = arr(*[u.ptr() for u in ups])
    pd = arr(*[d.ptr() for d in downs])
    nbytes = _lib.load().vb_moe_workspace(t, topk, h, i)
    if nbytes < 0:
        raise ValueError("moe_grouped_ffn: bad shape")
    ws = _workspace(nbytes, dev)
    vp = ctypes.c_void_p
    _lib.call("vb_moe_grouped_ffn_types", ctypes.cast(pg, vp), ctypes.cast(pu, vp), ctypes.cast(pd, vp), n_exp,
              x.data_ptr(), t, logits.data_ptr(), topk, y.data_ptr(), idx.data_ptr(), w.data_ptr(), h, i,
              gu_type, dn_type, ws.data_ptr(), ws.numel(), _stream())
    return y, idx, w


def activation(x: torch.Tensor, kind: int) -> torch.Tensor:
    """silu (kind 0) or relu (kind 1), elementwise on the device."""
    x = x.to(torch.float32).contiguous()
    out = torch.empty_like(x)
    _lib.call("vb_activation", x.data_ptr(), out.data_ptr(), x.numel(), kind, _stream())
    return out
