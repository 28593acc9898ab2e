"""CPU oracle for the GGUF quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package; it is the checker, never the thing
measured or shipped.  ``vibeblade_amd`` never imports it.

Contents
--------
* ctypes bindings to ``vb_oracle.c`` (plain C restatement of the reference's
  decoders, quantizers and GEMV loops; see the header of that file for the
  reference file:line each function follows);
* optional bindings to ``_ref/libvbref_*.so``, the reference's own
  ``cpp/src/dequant.cpp`` + ``fp16_compat.cpp`` compiled by ``Makefile`` target
  ``ref`` (built only where the reference tree exists);
* numpy compositions for the FFN-level configs (sparse FFN, MoE), written in
  float64 over the bit-exact decoded weights.

Parity status of each function is listed in ``PARITY`` below; every entry is
pinned by a test in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_0 = 2
TYPE_Q4_1 = 3
TYPE_Q5_0 = 6
TYPE_Q5_1 = 7
TYPE_Q8_0 = 8
TYPE_Q2_K = 10
TYPE_Q3_K = 11
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_BF16 = 30
TYPE_Q6_K_VBREF = 1014   # cpp/src/dequant.cpp:359-402 gather (test only)
TYPE_Q8_0_VBREF = 1008   # cpp/src/dequant.cpp:99-112 float-scale read (timing only)

BLOCK_ELEMS = {TYPE_F32: 1, TYPE_F16: 1, TYPE_BF16: 1, TYPE_Q4_0: 32, TYPE_Q4_1: 32, TYPE_Q5_0: 32,
               TYPE_Q5_1: 32, TYPE_Q8_0: 32, TYPE_Q2_K: 256, TYPE_Q3_K: 256, TYPE_Q4_K: 256, TYPE_Q5_K: 256,
               TYPE_Q6_K: 256,
               TYPE_Q6_K_VBREF: 256, TYPE_Q8_0_VBREF: 32}
BLOCK_BYTES = {TYPE_F32: 4, TYPE_F16: 2, TYPE_BF16: 2, TYPE_Q4_0: 18, TYPE_Q4_1: 20, TYPE_Q5_0: 22,
               TYPE_Q5_1: 24, TYPE_Q8_0: 34, TYPE_Q2_K: 84, TYPE_Q3_K: 110, TYPE_Q4_K: 144, TYPE_Q5_K: 176,
               TYPE_Q6_K: 210,
               TYPE_Q6_K_VBREF: 210, TYPE_Q8_0_VBREF: 34}

PARITY = {
    "dequant Q4_K": "pinned: golden vectors from compiled reference dequant.cpp + KATs",
    "dequant Q6_K": "pinned: layout-invariant KATs (reference tests/test_kquants.py:134-175) "
                    "+ single-position index-map blocks + VBREF golden vectors",
    "dequant Q8_0": "pinned: closed forms (d=1 -> q, d=0 -> 0) on loader.py:129-133 layout",
    "dequant Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q5_K / Q2_K / Q3_K": "pinned: ggml's published dequantize_row_* "
        "loop forms restated in the tests (sequential outputs, ggml's own scale / fifth-bit / hmask "
        "unpacking) on random blocks, plus a moved-code-bit negative control",
    "gemv / gemm": "pinned: brute force over integer-valued blocks + fp64 numpy",
    "sparse_ffn": "pinned: closed form S=all equals dense, S=empty gives 0, order invariance",
    "ffn_block": "pinned: rms_norm closed forms (constant rows, scale invariance, eps), "
                 "activation special values, the tanh-form GeGLU against the identity "
                 "0.5(1 + tanh z) = 1/(1 + e^-2z), composition = sparse_ffn with S = all plus the residual",
    "moe": "pinned: weights sum to 1, grouped == per-token loop, single-expert == one GEMM",
    "ema_update / ema_predict": "pinned: the reference's own known answers (tests/test_ema_neuron.py: "
                                "decay, cold start with and without gate values, warm threshold set, "
                                "combined union), the closed form 1 - (1 - a)^t, brute force on tiny inputs",
}


def _cpu_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return " avx512f" in flags and " avx512vl" in flags
    except OSError:
        return False


def simd_variant() -> str:
    return "avx512" if _cpu_has_avx512() else "avx2"


def build(with_ref: bool = True) -> None:
    """Compile the oracle (and the reference, when its tree is present)."""
    targets = ["oracle"]
    if with_ref and os.path.isdir("/root/reference/cpp/src"):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", _HERE] + targets, check=True)


_lib = None
_ref = None


def _load():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, f"liboracle_{simd_variant()}.so")
        if not os.path.exists(path):
            build(with_ref=False)
        lib = ctypes.CDLL(path)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.orc_dequant_rows.argtypes = [vp, vp, i64, i64, i32]
        lib.orc_quantize_rows.argtypes = [vp, vp, i64, i64, i32]
        lib.orc_gemv.argtypes = [vp, vp, vp, i64, i64, i32]
        lib.orc_gemm.argtypes = [vp, vp, vp, i64, i64, i64, i32]
        lib.orc_gemv_kn.argtypes = [vp, vp, vp, i64, i64, i32, vp]
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f16_to_f32.restype = ctypes.c_float
        lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        lib.orc_f32_to_f16.restype = ctypes.c_uint16
        lib.orc_row_bytes.argtypes = [i32, i64]
        lib.orc_row_bytes.restype = i64
        _lib = lib
    return _lib


def ref_available() -> bool:
    return os.path.exists(os.path.join(_HERE, "_ref", f"libvbref_{simd_variant()}.so"))


def _load_ref():
    """The compiled reference (``_ref/``); raises if it was not built."""
    global _ref
    if _ref is None:
        path = os.path.join(_HERE, "_ref", f"libvbref_{simd_variant()}.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        lib = ctypes.CDLL(path)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        lib.ref_dequantize_row.argtypes = [vp, vp, i64, i32]
        lib.ref_gemv_dequant.argtypes = [vp, vp, vp, i64, i64, i32, vp]
        lib.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.ref_f16_to_f32.restype = ctypes.c_float
        _ref = lib
    return _ref


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def row_bytes(qtype: int, k: int) -> int:
    rb = _load().orc_row_bytes(qtype, k)
    if rb < 0:
        raise ValueError(f"bad type/row length: type={qtype} k={k}")
    return int(rb)


def f16_to_f32(h: int) -> float:
    return float(_load().orc_f16_to_f32(int(h)))


def f32_to_f16(f: float) -> int:
    return int(_load().orc_f32_to_f16(float(f)))


def quantize(w: np.ndarray, qtype: int) -> np.ndarray:
    """Quantize an fp32 (rows, k) matrix to GGUF bytes, shape (rows, row_bytes)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    out = np.zeros((rows, row_bytes(qtype, k)), dtype=np.uint8)
    if _load().orc_quantize_rows(_ptr(w), _ptr(out), rows, k, qtype):
        raise ValueError("quantize failed")
    return out


def dequantize(wq: np.ndarray, k: int, qtype: int) -> np.ndarray:
    """Decode GGUF bytes (rows, row_bytes) to fp32 (rows, k)."""
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    rows = wq.shape[0] if wq.ndim == 2 else wq.size // row_bytes(qtype, k)
    out = np.empty((rows, k), dtype=np.float32)
    if _load().orc_dequant_rows(_ptr(wq), _ptr(out), rows, k, qtype):
        raise ValueError("dequant failed")
    return out


def gemv(wq: np.ndarray, x: np.ndarray, n: int, k: int, qtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n, dtype=np.float32)
    if _load().orc_gemv(_ptr(np.ascontiguousarray(wq)), _ptr(x), _ptr(y), n, k, qtype):
        raise ValueError("gemv failed")
    return y


def gemm(wq: np.ndarray, x: np.ndarray, n: int, k: int, qtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    if _load().orc_gemm(_ptr(np.ascontiguousarray(wq)), _ptr(x), _ptr(y), m, n, k, qtype):
        raise ValueError("gemm failed")
    return y


def gemv_kn(x: np.ndarray, wq: np.ndarray, K: int, N: int, qtype: int,
            scratch: np.ndarray | None = None) -> np.ndarray:
    """The reference gemv_dequant loop restated: out = x . W, W = K rows of N."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(N, dtype=np.float32)
    if scratch is None:
        scratch = np.empty(N, dtype=np.float32)
    if _load().orc_gemv_kn(_ptr(x), _ptr(wq), _ptr(out), K, N, qtype, _ptr(scratch)):
        raise ValueError("gemv_kn failed")
    return out


def ref_dequantize(wq: np.ndarray, n: int, qtype: int) -> np.ndarray:
    """Decode with the compiled reference's vibeblade::dequantize_row."""
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if _load_ref().ref_dequantize_row(_ptr(wq), _ptr(out), n, qtype):
        raise ValueError("reference dequantize_row threw")
    return out


def ref_gemv_dequant(x: np.ndarray, wq: np.ndarray, K: int, N: int, qtype: int,
                     scratch: np.ndarray | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(N, dtype=np.float32)
    if scratch is None:
        scratch = np.empty(N, dtype=np.float32)
    if _load_ref().ref_gemv_dequant(_ptr(x), _ptr(wq), _ptr(out), K, N, qtype, _ptr(scratch)):
        raise ValueError("reference gemv_dequant threw")
    return out


def ref_f16_to_f32(h: int) -> float:
    return float(_load_ref().ref_f16_to_f32(int(h)))


# ---------------------------------------------------------------------------
# FFN-level compositions (float64 over bit-exact decoded weights)
# ---------------------------------------------------------------------------

def silu64(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def relu64(v: np.ndarray) -> np.ndarray:
    return np.maximum(np.asarray(v, dtype=np.float64), 0.0)


ACT_SILU = 0   # silu(g) * u         (vibeblade/sparse.py:269-272)
ACT_DRELU = 1  # relu(g) * relu(u)   (ReLU after both projections, config 4)
ACT_GELU_TANH = 2  # gelu_tanh(g) * u (cpp/src/fast_model.cpp:943-948)


def gelu_tanh64(v: np.ndarray) -> np.ndarray:
    """0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))), as
    cpp/src/fast_model.cpp:945-946 writes it."""
    v = np.asarray(v, dtype=np.float64)
    return 0.5 * v * (1.0 + np.tanh(0.7978845608 * (v + 0.044715 * v * v * v)))


def act_pair(g: np.ndarray, u: np.ndarray, act: int) -> np.ndarray:
    if act == ACT_SILU:
        return silu64(g) * u
    if act == ACT_GELU_TANH:
        return gelu_tanh64(g) * u
    return relu64(g) * relu64(u)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * w per row, fp64 (cpp/src/fast_model.cpp:61-71)."""
    x = np.asarray(x, dtype=np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * np.asarray(w, dtype=np.float64)


def ffn_block(gate: np.ndarray, up: np.ndarray, down: np.ndarray, x: np.ndarray, norm_w, eps: float,
              act: int, add_residual: bool) -> np.ndarray:
    """One token's FFN block, fp64 over decoded weights (cpp/src/fast_model.cpp:837-975):
    n = rms_norm(x) (or x when norm_w is None); y = [x +] down @ act(gate @ n, up @ n).
    gate/up: decoded (I, H); down: decoded (H, I)."""
    x = np.asarray(x, dtype=np.float64)
    n = x if norm_w is None else rms_norm(x, norm_w, eps)
    g = gate.astype(np.float64) @ n
    u = up.astype(np.float64) @ n
    y = down.astype(np.float64) @ act_pair(g, u, act)
    return x + y if add_residual else y


def sparse_ffn(gate: np.ndarray, up: np.ndarray, down: np.ndarray, x: np.ndarray,
               active: np.ndarray, act: int) -> np.ndarray:
    """y = sum_{i in S} act(g_i, u_i) * down[:, i]  (fp64).

    gate/up: decoded (I, H) fp32; down: decoded (H, I) fp32 (GGUF layout);
    x: (M, H); active: sorted neuron ids.  This equals the dense FFN with the
    hidden vector masked to S (vibeblade/sparse.py:138-139,
    vibeblade/transformer.py:204-206).
    """
    x = np.atleast_2d(np.asarray(x, dtype=np.float64))
    idx = np.asarray(active, dtype=np.int64)
    g = x @ gate[idx].astype(np.float64).T
    u = x @ up[idx].astype(np.float64).T
    return act_pair(g, u, act) @ down[:, idx].astype(np.float64).T


def ema_update(probs: np.ndarray, mask: np.ndarray, alpha: float) -> np.ndarray:
    """EMANeuronPredictor.update (vibeblade/sparse.py:494-515): the float32
    numpy expression alpha * obs + (1 - alpha) * probs, evaluated as numpy
    evaluates it."""
    obs = np.asarray(mask).astype(np.float32)
    return (alpha * obs + (1.0 - alpha) * np.asarray(probs, dtype=np.float32)).astype(np.float32)


def _top_k_lowest(values: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest values; ties to the lowest indices."""
    return np.argsort(-np.asarray(values, dtype=np.float64), kind="stable")[:k]


def ema_predict(probs: np.ndarray, k: int, threshold: float, warm: bool, gate=None,
                combined: bool = False) -> np.ndarray:
    """EMANeuronPredictor.predict / predict_combined (vibeblade/sparse.py:517-598)
    as written there: warm -> the threshold mask, topped up to k with the most
    probable neurons below it; cold -> top-k of the gate values, else the
    first k; combined -> the gate-less prediction | top-k(gate).  Where the
    reference's argpartition leaves ties open, the lowest indices win."""
    p = np.asarray(probs, dtype=np.float32)
    n = p.size

    def base(g):
        if warm:
            m = p >= np.float32(threshold)
            c = int(m.sum())
            if c < k:
                below = np.flatnonzero(~m)
                m[below[_top_k_lowest(p[below], k - c)]] = True
            return m
        m = np.zeros(n, dtype=bool)
        if g is not None:
            m[_top_k_lowest(g, k)] = True
        else:
            m[:k] = True
        return m
    if combined:
        m = base(None)
        m[_top_k_lowest(gate, k)] = True
        return m
    return base(gate)


def route_top_k(logits: np.ndarray, topk: int):
    """softmax over experts, top-k, renormalise (vibeblade/moe.py:186-200,
    cpp/src/fast_model.cpp:534-548).  Ties resolve to the lower expert id."""
    z = np.asarray(logits, dtype=np.float64)
    z = np.clip(z, -50.0, 50.0)
    p = np.exp(z - z.max(axis=-1, keepdims=True))
    p = p / p.sum(axis=-1, keepdims=True)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :topk]
    w = np.take_along_axis(p, order, axis=-1)
    w = w / w.sum(axis=-1, keepdims=True)
    return order.astype(np.int32), w


def moe_ffn(gates, ups, downs, x: np.ndarray, logits: np.ndarray, topk: int):
    """Per-token top-k SwiGLU MoE (vibeblade/moe_executor.py:342-344 expert FFN,
    vibeblade/moe.py:457-482 weighted sum).  gates/ups: lists of decoded (I, H);
    downs: decoded (H, I).  Returns (Y fp64 (T, H), idx, w)."""
    x = np.asarray(x, dtype=np.float64)
    idx, w = route_top_k(logits, topk)
    y = np.zeros((x.shape[0], downs[0].shape[0]), dtype=np.float64)
    for t in range(x.shape[0]):
        for s in range(topk):
            e = int(idx[t, s])
            g = gates[e].astype(np.float64) @ x[t]
            u = ups[e].astype(np.float64) @ x[t]
            y[t] += w[t, s] * (downs[e].astype(np.float64) @ (silu64(g) * u))
    return y, idx, w


def moe_ffn_grouped(experts, x: np.ndarray, logits: np.ndarray, topk: int):
    """moe_ffn with tokens grouped per expert: ``experts(e)`` returns expert e's
    decoded (gate (I, H), up (I, H), down (H, I)) and is called once per hit
    expert, so large experts are decoded one at a time.  Same fp64 sums as
    moe_ffn (each token's slots added in slot order).  Returns (Y, idx, w)."""
    x = np.asarray(x, dtype=np.float64)
    idx, w = route_top_k(logits, topk)
    parts = {}
    for e in sorted(set(idx.ravel().tolist())):
        g, u, d = experts(e)
        rows = [(t, s) for t in range(x.shape[0]) for s in range(topk) if idx[t, s] == e]
        xe = x[[t for t, _ in rows]]
        he = silu64(xe @ g.astype(np.float64).T) * (xe @ u.astype(np.float64).T)
        ye = he @ d.astype(np.float64).T
        for r, (t, s) in enumerate(rows):
            parts[(t, s)] = ye[r]
    y = np.zeros((x.shape[0], parts[(0, 0)].shape[0]), dtype=np.float64)
    for t in range(x.shape[0]):
        for s in range(topk):
            y[t] += w[t, s] * parts[(t, s)]
    return y, idx, w


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
