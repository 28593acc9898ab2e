"""GGUF type ids and block geometry.

Same table as ``ggml_type`` / ``ggml_blck_size`` / ``ggml_type_size`` /
``tensor_nbytes`` (cpp/include/ggml_types.h:11-71, :195-199) and the Python
twins ``_QBLOCK_SIZE`` / ``_QBLOCK_BYTES`` (vibeblade/loader.py:86-115).  The
loader's Q3_K entry (178 bytes) disagrees with ggml (110), and the C++
table's Q8_1 entry (40 bytes, ggml_types.h:62: fp32 d and s) is the older
ggml layout (fp16 d and s, 36 bytes, since); ggml's current values are used
here.  Only the types with device kernels are marked in ``DEVICE_TYPES``.
"""
from __future__ import annotations

GGML_TYPE_F32 = 0
GGML_TYPE_F16 = 1
GGML_TYPE_Q4_0 = 2
GGML_TYPE_Q4_1 = 3
GGML_TYPE_Q5_0 = 6
GGML_TYPE_Q5_1 = 7
GGML_TYPE_Q8_0 = 8
GGML_TYPE_Q8_1 = 9
GGML_TYPE_Q2_K = 10
GGML_TYPE_Q3_K = 11
GGML_TYPE_Q4_K = 12
GGML_TYPE_Q5_K = 13
GGML_TYPE_Q6_K = 14
GGML_TYPE_Q8_K = 15
GGML_TYPE_BF16 = 30

# type -> (elements per block, bytes per block)
BLOCK = {
    GGML_TYPE_F32: (1, 4),
    GGML_TYPE_F16: (1, 2),
    GGML_TYPE_BF16: (1, 2),
    GGML_TYPE_Q4_0: (32, 18),
    GGML_TYPE_Q4_1: (32, 20),
    GGML_TYPE_Q5_0: (32, 22),
    GGML_TYPE_Q5_1: (32, 24),
    GGML_TYPE_Q8_0: (32, 34),
    GGML_TYPE_Q8_1: (32, 36),
    GGML_TYPE_Q2_K: (256, 84),
    GGML_TYPE_Q3_K: (256, 110),
    GGML_TYPE_Q4_K: (256, 144),
    GGML_TYPE_Q5_K: (256, 176),
    GGML_TYPE_Q6_K: (256, 210),
    GGML_TYPE_Q8_K: (256, 292),
}

NAMES = {
    GGML_TYPE_F32: "F32", GGML_TYPE_F16: "F16", GGML_TYPE_BF16: "BF16",
    GGML_TYPE_Q4_0: "Q4_0", GGML_TYPE_Q4_1: "Q4_1", GGML_TYPE_Q5_0: "Q5_0",
    GGML_TYPE_Q5_1: "Q5_1", GGML_TYPE_Q8_0: "Q8_0", GGML_TYPE_Q8_1: "Q8_1",
    GGML_TYPE_Q2_K: "Q2_K", GGML_TYPE_Q3_K: "Q3_K", GGML_TYPE_Q4_K: "Q4_K",
    GGML_TYPE_Q5_K: "Q5_K", GGML_TYPE_Q6_K: "Q6_K", GGML_TYPE_Q8_K: "Q8_K",
}

# Types with gfx950 kernels in libvbhip (decode, embedding rows, GEMV).
DEVICE_TYPES = (GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_BF16, GGML_TYPE_Q4_0, GGML_TYPE_Q4_1, GGML_TYPE_Q5_0,
                GGML_TYPE_Q5_1, GGML_TYPE_Q8_0, GGML_TYPE_Q2_K, GGML_TYPE_Q3_K, GGML_TYPE_Q4_K, GGML_TYPE_Q5_K,
                GGML_TYPE_Q6_K)
# Of those, the types the quantizer (vb_quantize_rows) writes.
QUANTIZE_TYPES = (GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q8_0, GGML_TYPE_Q4_K, GGML_TYPE_Q6_K)


def ggml_blck_size(t: int) -> int:
    return BLOCK.get(t, (1, 4))[0]


def ggml_type_size(t: int) -> int:
    return BLOCK.get(t, (1, 4))[1]


def tensor_nbytes(t: int, n_values: int) -> int:
    """Bytes of n_values elements, rounded up to whole blocks
    (cpp/include/ggml_types.h:195-199)."""
    be, bb = BLOCK.get(t, (1, 4))
    return ((n_values + be - 1) // be) * bb


def row_bytes(t: int, k: int) -> int:
    """Bytes of one row of k elements; ValueError unless k is whole blocks."""
    if t not in BLOCK:
        raise ValueError(f"unknown ggml type {t}")
    be, bb = BLOCK[t]
    if k <= 0 or k % be:
        raise ValueError(f"row length {k} is not a multiple of the {NAMES[t]} block ({be})")
    return (k // be) * bb
