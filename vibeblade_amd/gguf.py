"""GGUF ingestion: a .gguf file's metadata and tensor table, and its tensors
on the GPU in their GGUF block layout.

The file is parsed natively (libvbhip, ``vb_gguf_*``: the file is mapped
read-only, never copied whole into RAM) and tensors are uploaded through
pinned staging buffers without decoding: the kernels read GGUF blocks as
stored.

``GGUFFile`` keeps the names of the reference's C++ reader
(cpp/include/gguf.h:29-60): ``tensor_data``, ``tensor_info``,
``meta_string`` / ``meta_int`` / ``meta_float`` / ``meta_bool`` and the
``*_array`` accessors with the same defaults for absent keys, ``tensors()``,
``version()``, ``file_size()``.  ``GGUFLoader`` keeps the Python reader's
surface (vibeblade/loader.py:490-783): ``metadata``, ``tensor_infos``,
``tensor_names()``, ``tensor_info(name)`` (a dict with the GGUF dims
reversed into a row-major ``shape``; KeyError when absent, as
loader.py:616), ``load_tensor(name)`` (fp32 numpy) and the context manager.
Both add ``load_qtensor(name)``: the tensor as a device ``QTensor``.

Differences from the reference, on purpose: the data section follows
``general.alignment`` when the file sets it (the reference always uses 32);
every metadata type is kept (the reference drops 16-bit values and most
array element types); ``load_tensor`` decodes the quantized types that have
device kernels (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K;
bit-exact GGUF decoding on the GPU) and raises ValueError for the others
(Q8_1, Q8_K), where the reference's Python decoders use non-GGUF bit layouts
for several of them.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

from . import _lib, ggml

# GGUF metadata value types
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL = range(8)
GGUF_STRING, GGUF_ARRAY, GGUF_U64, GGUF_I64, GGUF_F64 = 8, 9, 10, 11, 12
_INT_TYPES = (GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_U64, GGUF_I64)
_FLOAT_TYPES = (GGUF_F32, GGUF_F64)


@dataclass(frozen=True)
class TensorInfo:
    """One tensor table entry (cpp/include/gguf.h:20-27): GGUF dims
    (``dims[0]`` along the row, unused dims 1), ``offset`` from the start of
    the data section (as stored), ``size`` in bytes."""
    name: str
    n_dims: int
    dims: tuple
    type: int
    offset: int
    size: int

    @property
    def shape(self) -> tuple:
        """Row-major shape (GGUF dims reversed, as loader.py:564 does)."""
        return tuple(reversed(self.dims[: self.n_dims]))

    @property
    def rows(self) -> int:
        n = 1
        for d in self.dims[1: self.n_dims]:
            n *= d
        return n


class _Mapping:
    """Owner of the native handle (the file mapping).  ``GGUFFile`` and every
    ``tensor_data`` view hold a reference, so the mapping outlives
    ``close()`` for as long as a view of it is alive."""

    def __init__(self, lib, h):
        self._lib, self.h = lib, h

    def __del__(self) -> None:
        h, self.h = self.h, None
        if h is not None and h.value:
            try:
                self._lib.vb_gguf_close(h)
            except Exception:
                pass


class GGUFFile:
    """A parsed .gguf file (see the module docstring)."""

    def __init__(self, path: str):
        path = os.fspath(path)
        if not os.path.exists(path):
            raise FileNotFoundError(f"Cannot open GGUF: {path}")
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        _lib.check("vb_gguf_open", self._lib.vb_gguf_open(path.encode(), ctypes.byref(h)))
        self._map = _Mapping(self._lib, h)
        self._h = h
        self.path = path
        ver, align = ctypes.c_uint32(), ctypes.c_uint64()
        doff, fsize = ctypes.c_uint64(), ctypes.c_uint64()
        _lib.check("vb_gguf_info", self._lib.vb_gguf_info(h, ctypes.byref(ver), ctypes.byref(align),
                                                          ctypes.byref(doff), ctypes.byref(fsize)))
        self._version, self.alignment = ver.value, align.value
        self.data_offset, self._file_size = doff.value, fsize.value
        self._tensors = [self._read_tensor(i) for i in range(self._lib.vb_gguf_n_tensors(h))]
        self._by_name = {t.name: i for i, t in enumerate(self._tensors)}
        self.metadata = {}
        self._meta_types = {}
        for i in range(self._lib.vb_gguf_n_kv(h)):
            key, vtype, etype, count = self._kv_info(i)
            self._meta_types[key] = (vtype, etype)
            self.metadata[key] = self._kv_value(i, vtype, etype, count)

    # ---- table ----------------------------------------------------------------

    def _read_tensor(self, i: int) -> TensorInfo:
        name, t, nd = ctypes.c_char_p(), ctypes.c_int32(), ctypes.c_int32()
        dims = (ctypes.c_int64 * 4)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        _lib.check("vb_gguf_tensor_info", self._lib.vb_gguf_tensor_info(
            self._h, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd), dims, ctypes.byref(off),
            ctypes.byref(nb)))
        return TensorInfo(name.value.decode("utf-8"), nd.value, tuple(dims), t.value,
                          off.value - self.data_offset, nb.value)

    def _kv_info(self, i: int):
        key, vt, et, cnt = ctypes.c_char_p(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_uint64()
        _lib.check("vb_gguf_kv_info", self._lib.vb_gguf_kv_info(self._h, i, ctypes.byref(key), ctypes.byref(vt),
                                                                ctypes.byref(et), ctypes.byref(cnt)))
        return key.value.decode("utf-8"), vt.value, et.value, cnt.value

    def _elem(self, i: int, t: int, j: int):
        if t in _INT_TYPES or t == GGUF_BOOL:
            v = ctypes.c_int64()
            _lib.check("vb_gguf_kv_int", self._lib.vb_gguf_kv_int(self._h, i, j, ctypes.byref(v)))
            if t == GGUF_BOOL:
                return v.value != 0
            if t == GGUF_U64:
                return v.value & 0xFFFFFFFFFFFFFFFF
            return v.value
        if t in _FLOAT_TYPES:
            v = ctypes.c_double()
            _lib.check("vb_gguf_kv_float", self._lib.vb_gguf_kv_float(self._h, i, j, ctypes.byref(v)))
            return v.value
        if t == GGUF_STRING:
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            _lib.check("vb_gguf_kv_str", self._lib.vb_gguf_kv_str(self._h, i, j, ctypes.byref(p), ctypes.byref(n)))
            return ctypes.string_at(p.value, n.value).decode("utf-8", errors="replace") if n.value else ""
        raise ValueError(f"unsupported GGUF value type {t}")

    def _kv_value(self, i: int, vtype: int, etype: int, count: int):
        if vtype == GGUF_ARRAY:
            return [self._elem(i, etype, j) for j in range(count)]
        return self._elem(i, vtype, 0)

    # ---- GGUFFile accessors (cpp/include/gguf.h) ------------------------------

    def tensors(self) -> list:
        return list(self._tensors)

    def version(self) -> int:
        return self._version

    def file_size(self) -> int:
        return self._file_size

    def tensor_info(self, name: str):
        """TensorInfo, or None when absent (gguf.h:41 returns nullptr)."""
        i = self._by_name.get(name)
        return None if i is None else self._tensors[i]

    def tensor_data(self, name: str):
        """Read-only numpy uint8 view of the tensor's bytes in the mapping, or
        None when absent (gguf.h:38).  The view keeps the mapping alive: it
        stays valid after ``close()`` or after this object is dropped."""
        i = self._by_name.get(name)
        if i is None:
            return None
        p = ctypes.c_void_p()
        _lib.check("vb_gguf_tensor_data", self._lib.vb_gguf_tensor_data(self._handle(), i, ctypes.byref(p)))
        n = self._tensors[i].size
        buf = (ctypes.c_uint8 * n).from_address(p.value) if n else (ctypes.c_uint8 * 0)()
        buf._owner = self._map  # the view's base holds the mapping
        arr = np.frombuffer(buf, dtype=np.uint8)
        arr.flags.writeable = False
        return arr

    def _scalar(self, key: str, types, default):
        if key not in self.metadata or self._meta_types[key][0] not in types:
            return default
        return self.metadata[key]

    def meta_string(self, key: str) -> str:
        return self._scalar(key, (GGUF_STRING,), "")

    def meta_int(self, key: str, default_val: int = 0) -> int:
        return self._scalar(key, _INT_TYPES, default_val)

    def meta_float(self, key: str, default_val: float = 0.0) -> float:
        return self._scalar(key, _FLOAT_TYPES, default_val)

    def meta_bool(self, key: str, default_val: bool = False) -> bool:
        return self._scalar(key, (GGUF_BOOL,), default_val)

    def _array(self, key: str, etypes) -> list:
        vt = self._meta_types.get(key)
        if vt is None or vt[0] != GGUF_ARRAY or vt[1] not in etypes:
            return []
        return list(self.metadata[key])

    def meta_string_array(self, key: str) -> list:
        return self._array(key, (GGUF_STRING,))

    def meta_int_array(self, key: str) -> list:
        return self._array(key, _INT_TYPES)

    def meta_float_array(self, key: str) -> list:
        return self._array(key, _FLOAT_TYPES)

    # ---- device ---------------------------------------------------------------

    def load_qtensor(self, name: str, device=None):
        """The tensor as a QTensor (rows x k, k = dims[0]) on the GPU, GGUF
        blocks unchanged.  ValueError for types without device kernels."""
        import torch

        from .tensor import QTensor, _dev, _stream
        h = self._handle()
        i = self._by_name.get(name)
        if i is None:
            raise KeyError(f"Tensor not found: {name}")
        t = self._tensors[i]
        if t.type not in ggml.DEVICE_TYPES:
            raise ValueError(f"tensor '{name}': no device kernels for type {ggml.NAMES.get(t.type, t.type)}")
        dev = _dev(device)
        buf = torch.empty(t.size, dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            _lib.check("vb_gguf_upload", self._lib.vb_gguf_upload(h, i, buf.data_ptr(), _stream()))
        return QTensor(buf, t.type, t.rows, t.dims[0])

    # ---- lifetime -------------------------------------------------------------

    def _handle(self):
        if getattr(self, "_h", None) is None:
            raise ValueError("GGUF file is closed")
        return self._h

    def close(self) -> None:
        """Release this object's hold on the mapping; it is unmapped once no
        ``tensor_data`` view of it is left."""
        self._h = None
        self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class GGUFLoader(GGUFFile):
    """GGUFLoader's surface (vibeblade/loader.py:490-783) over GGUFFile."""

    def __init__(self, path: str, progress_cb=None) -> None:
        super().__init__(path)
        self._progress_cb = progress_cb
        self.n_tensors = len(self._tensors)
        self.n_kv = len(self.metadata)
        self.tensor_infos = [{"name": t.name, "shape": t.shape, "dtype": t.type, "offset": t.offset}
                             for t in self._tensors]
        if progress_cb:
            progress_cb("tensor info", self.n_tensors, self.n_tensors, loading=True)

    def tensor_names(self) -> list:
        return [t.name for t in self._tensors]

    def tensor_info(self, name: str) -> dict:
        i = self._by_name.get(name)
        if i is None:
            raise KeyError(f"Tensor not found: {name}")
        return self.tensor_infos[i]

    def load_tensor(self, name: str, dtype=np.dtype("float32"), progress_cb=None) -> np.ndarray:
        """The tensor decoded to ``dtype`` (fp32 or fp16) numpy, row-major
        shape.  F32 / F16 / BF16 come straight from the file; Q8_0 / Q4_K /
        Q6_K are decoded on the GPU (bit-exact GGUF decoding); other types
        raise ValueError."""
        i = self._by_name.get(name)
        if i is None:
            raise KeyError(f"Tensor not found: {name}")
        t = self._tensors[i]
        raw = GGUFFile.tensor_data(self, name)
        if t.type == ggml.GGML_TYPE_F32:
            arr = raw.view(np.float32)
        elif t.type == ggml.GGML_TYPE_F16:
            arr = raw.view(np.float16)
        elif t.type == ggml.GGML_TYPE_BF16:
            arr = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif t.type in ggml.DEVICE_TYPES:
            arr = self.load_qtensor(name).dequantize().cpu().numpy()
        else:
            raise ValueError(f"Unsupported tensor type {t.type} ({ggml.NAMES.get(t.type, '?')}) "
                             f"for tensor '{name}'")
        out = arr.reshape(t.shape)
        if dtype == np.float16:
            return np.clip(out, -65504.0, 65504.0).astype(np.float16)
        return out.astype(dtype, copy=True)

    def load_all_tensors(self, dtype=np.dtype("float32"), progress_cb=None) -> dict:
        return {n: self.load_tensor(n, dtype) for n in self.tensor_names()}
