"""vibeblade_amd: gfx950 (MI355X) GGUF quantized matmul behind VibeBlade's op surface.

The device work is hand-written HIP in ``csrc/`` built into ``libvbhip.so``
(C ABI: ``include/vbhip.h``) and called through ``ctypes``.  Modules:

* ``ggml``          -- GGUF type ids and block geometry
* ``tensor``        -- ``QTensor`` (GGUF weights resident in HBM) and the ops
                       on it: gemv, gemm, sparse_ffn, topk_indices,
                       moe_grouped_ffn, moe_route
* ``sparse``        -- drop-in for vibeblade/sparse.py (TurboSparse FFN)
* ``moe``           -- drop-in for vibeblade/moe.py (router, experts, MoE FFN)
* ``moe_executor``  -- drop-in for vibeblade/moe_executor.py (HotColdExecutor)
* ``moe_profiler``  -- ``HotColdMap``
* ``gpu``           -- ``GPUBackend`` duck type on HIP (``HipBackend``)
* ``quant``         -- drop-in for vibeblade/quant.py (RotorQuant packing)
* ``build``         -- compiles ``libvbhip.so`` in-tree with hipcc for gfx950

Importing the package does not touch the GPU; the first op loads the library
and selects the device (there is no CPU fallback).
"""
from . import ggml  # noqa: F401

__all__ = ["ggml", "tensor", "sparse", "moe", "moe_executor", "moe_profiler", "gpu", "quant"]
__version__ = "0.1.0"
