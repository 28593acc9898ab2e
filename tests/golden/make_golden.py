"""Write tests/golden/ref_vectors.npz from the compiled reference.

Runs the reference's own cpp/src/dequant.cpp and fp16_compat.cpp, built from
the reference tree by ``make -C oracle ref`` into ``oracle/_ref/`` (never
copied into this repository), on seeded inputs, and stores inputs and
outputs as plain arrays:

* ``q4k_blocks`` / ``q4k_out``: random Q4_K blocks (fp16 d and dmin forced
  to normal values) and vibeblade::dequantize_row's output (type 12);
* ``q6k_blocks`` / ``q6k_vbref_out``: random Q6_K blocks and the reference's
  Q6_K decode (its own gather, cpp/src/dequant.cpp:359-402);
* ``f16_bits`` / ``f16_ref``: vibeblade::f16_to_f32 on all fp16 subnormals,
  a sample of normals and the infinities (documents the subnormal behaviour of fp16_compat.cpp:13-35);
* ``kn_*``: vibeblade::gemv_dequant on a small Q4_K matrix in its own
  orientation (K rows of N), the loop the CPU baseline restates.

Usage: ``python tests/golden/make_golden.py`` (needs /root/reference).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402

SEED = 20261201


def _f16bits(v):
    return np.asarray(v, dtype=np.float16).view(np.uint16)


def main() -> None:
    O.build(with_ref=True)
    rng = np.random.default_rng(SEED)

    nb = 48
    q4 = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    d = _f16bits(rng.uniform(1e-3, 2.0, nb))
    dm = _f16bits(rng.uniform(1e-3, 2.0, nb))
    q4[:, 0], q4[:, 1] = d & 0xFF, d >> 8
    q4[:, 2], q4[:, 3] = dm & 0xFF, dm >> 8
    q4_out = O.ref_dequantize(q4.ravel(), 256 * nb, O.TYPE_Q4_K)

    q6 = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    d6 = _f16bits(rng.uniform(1e-3, 2.0, nb))
    q6[:, 208], q6[:, 209] = d6 & 0xFF, d6 >> 8
    q6_out = O.ref_dequantize(q6.ravel(), 256 * nb, O.TYPE_Q6_K)

    sub = np.arange(0, 0x400, dtype=np.uint16)
    bits = np.concatenate([sub, sub | 0x8000,
                           rng.integers(0x400, 0x7C00, 512).astype(np.uint16),
                           np.array([0x7C00, 0xFC00, 0x3C00, 0xBC00], dtype=np.uint16)])
    f16_ref = np.array([O.ref_f16_to_f32(int(b)) for b in bits], dtype=np.float32)

    # gemv_dequant in the reference orientation: K rows of N elements.
    K, N = 24, 512
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    wq = O.quantize(w, O.TYPE_Q4_K)
    x = rng.standard_normal(K).astype(np.float32)
    kn_out = O.ref_gemv_dequant(x, wq.ravel(), K, N, O.TYPE_Q4_K)

    np.savez_compressed(
        os.path.join(HERE, "ref_vectors.npz"),
        seed=np.int64(SEED),
        q4k_blocks=q4, q4k_out=q4_out.reshape(nb, 256),
        q6k_blocks=q6, q6k_vbref_out=q6_out.reshape(nb, 256),
        f16_bits=bits, f16_ref=f16_ref,
        kn_w=wq, kn_x=x, kn_out=kn_out, kn_shape=np.array([K, N], dtype=np.int64),
    )
    print("wrote", os.path.join(HERE, "ref_vectors.npz"))


if __name__ == "__main__":
    main()
