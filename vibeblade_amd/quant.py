"""RotorQuant 4-bit packing -- drop-in for vibeblade/quant.py.

Same functions, signatures, validation errors and results as the reference
(vibeblade/quant.py:13-304).  RotorQuant is an SO(4)-rotation 4-bit scheme
of the reference's own, not a GGUF format; it runs at weight-conversion time
on the host, so these are host functions over numpy arrays.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = ["pack_nibbles", "unpack_nibbles", "build_so4_rotor", "quantize_4bit", "dequantize_4bit",
           "quantization_error"]


def pack_nibbles(values: np.ndarray) -> np.ndarray:
    """Two 4-bit values per byte: values[2i] low nibble, values[2i+1] high."""
    v = np.asarray(values, dtype=np.uint8)
    if v.ndim != 1:
        raise ValueError("pack_nibbles expects a 1-D array")
    if v.size and np.any(v > 15):
        raise ValueError("pack_nibbles: all values must be in 0..15")
    if v.size % 2:
        v = np.concatenate([v, np.zeros(1, np.uint8)])
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray, n: int) -> np.ndarray:
    """Inverse of pack_nibbles: the first n 4-bit values."""
    p = np.asarray(packed, dtype=np.uint8)
    if p.ndim != 1:
        raise ValueError("unpack_nibbles expects a 1-D array")
    need = math.ceil(n / 2)
    if p.size < need:
        raise ValueError(f"unpack_nibbles: need at least {need} bytes for n={n}, got {p.size}")
    out = np.empty(2 * p.size, dtype=np.uint8)
    out[0::2] = p & 0x0F
    out[1::2] = p >> 4
    return out[:n]


def build_so4_rotor(weights: np.ndarray) -> np.ndarray:
    """Block-diagonal SO(4) matrix of two Givens rotations, one per pair
    (w0, w1) and (w2, w3), each turning its pair onto the first axis."""
    w = np.asarray(weights, dtype=np.float32)
    if w.shape != (4,):
        raise ValueError(f"build_so4_rotor expects shape (4,), got {w.shape}")
    r = np.eye(4, dtype=np.float32)
    for i, j in ((0, 1), (2, 3)):
        a, b = float(w[i]), float(w[j])
        if abs(a) < 1e-12 and abs(b) < 1e-12:
            continue
        th = math.atan2(b, a)
        c, s = math.cos(th), math.sin(th)
        r[i, i], r[i, j], r[j, i], r[j, j] = c, s, -s, c
    return r


def quantize_4bit(weights: np.ndarray, group_size: int = 32):
    """RotorQuant encode: per 4-element sub-group, rotate by its SO(4) rotor
    and affine-quantize to 0..15.  Returns (packed, scales (G, 2, S),
    rotors (G, S, 4, 4)), S = group_size / 4."""
    w = np.asarray(weights, dtype=np.float32)
    if w.ndim != 1:
        raise ValueError("quantize_4bit expects a 1-D weight array")
    if group_size % 4 != 0:
        raise ValueError("group_size must be divisible by 4")
    if w.size % group_size != 0:
        raise ValueError(f"Weight length ({w.size}) must be divisible by group_size ({group_size})")
    ng, sg = w.size // group_size, group_size // 4
    scales = np.empty((ng, 2, sg), dtype=np.float32)
    rotors = np.empty((ng, sg, 4, 4), dtype=np.float32)
    codes = np.empty((ng, sg, 4), dtype=np.uint8)
    sub = w.reshape(ng, sg, 4)
    for g in range(ng):
        for s in range(sg):
            r = build_so4_rotor(sub[g, s])
            rot = r @ sub[g, s]
            rotors[g, s] = r
            lo, hi = float(rot.min()), float(rot.max())
            if hi - lo < 1e-12:  # constant sub-group -> midpoint code
                codes[g, s] = 8
                scales[g, 0, s], scales[g, 1, s] = float(rot[0]), 0.0
            else:
                step = (hi - lo) / 15.0
                scales[g, 0, s], scales[g, 1, s] = lo, step
                codes[g, s] = np.clip(np.round((rot - lo) / step), 0, 15).astype(np.uint8)
    return pack_nibbles(codes.reshape(-1)), scales, rotors


def dequantize_4bit(packed: np.ndarray, scales: np.ndarray, rotors: np.ndarray, n: int) -> np.ndarray:
    """Inverse of quantize_4bit: R^T (lo + q * step) per sub-group."""
    scales = np.asarray(scales, dtype=np.float32)
    rotors = np.asarray(rotors, dtype=np.float32)
    ng, sg = rotors.shape[0], rotors.shape[1]
    if ng * sg * 4 != n:
        raise ValueError(f"Mismatch: num_groups({ng}) * group_size({sg * 4}) = {ng * sg * 4} != n({n})")
    q = unpack_nibbles(packed, n).reshape(ng, sg, 4).astype(np.float32)
    out = np.empty((ng, sg, 4), dtype=np.float32)
    for g in range(ng):
        for s in range(sg):
            lo, step = scales[g, 0, s], scales[g, 1, s]
            vals = np.full(4, lo, dtype=np.float32) if step < 1e-12 else lo + q[g, s] * step
            out[g, s] = rotors[g, s].T @ vals
    return out.reshape(-1)


def quantization_error(original: np.ndarray, reconstructed: np.ndarray) -> float:
    """RMS error between two weight vectors of the same size."""
    a = np.asarray(original, dtype=np.float32).ravel()
    b = np.asarray(reconstructed, dtype=np.float32).ravel()
    if a.shape != b.shape:
        raise ValueError(f"Shape mismatch: original {a.shape} vs reconstructed {b.shape}")
    return float(np.sqrt(np.mean((a - b) ** 2)))
