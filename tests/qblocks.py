"""Random GGUF blocks for types without a quantizer here (Q4_0, Q4_1, Q5_0,
Q5_1, Q2_K, Q3_K, Q5_K): random bytes with every fp16 scale / min set to a modest normal
value of random sign, so decoded weights are finite and of moderate size."""
import numpy as np

from vibeblade_amd import ggml

# byte offsets of the fp16 scale / min fields in each block
SCALE_OFFSETS = {
    ggml.GGML_TYPE_Q4_0: [0], ggml.GGML_TYPE_Q4_1: [0, 2], ggml.GGML_TYPE_Q5_0: [0], ggml.GGML_TYPE_Q5_1: [0, 2],
    ggml.GGML_TYPE_Q8_0: [0], ggml.GGML_TYPE_Q4_K: [0, 2], ggml.GGML_TYPE_Q5_K: [0, 2], ggml.GGML_TYPE_Q6_K: [208],
    ggml.GGML_TYPE_Q2_K: [80, 82], ggml.GGML_TYPE_Q3_K: [108],
}


def rand_qblocks(qtype: int, rows: int, k: int, seed: int) -> np.ndarray:
    """(rows, row_bytes) uint8."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, (rows, ggml.row_bytes(qtype, k)), dtype=np.uint8)
    blk = raw.reshape(-1, ggml.BLOCK[qtype][1])
    for o in SCALE_OFFSETS[qtype]:
        # fp16 sign random, exponent 8..11 (2^-7 .. 2^-4), mantissa random
        blk[:, o + 1] = (blk[:, o + 1] & 0x83) | (0x20 + (blk[:, o] & 0x0C))
    return raw
