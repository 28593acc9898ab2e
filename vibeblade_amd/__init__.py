"""vibeblade_amd: gfx950 (MI355X) GGUF quantized matmul behind VibeBlade's op surface.

The device work is hand-written HIP in ``csrc/`` built into ``libvbhip.so``
(C ABI: ``include/vbhip.h``) and called through ``ctypes``.  Modules:

* ``ggml``    -- GGUF type ids and block geometry
* ``tensor``  -- ``QTensor`` (GGUF weights resident in HBM) and the ops on it
* ``build``   -- compiles ``libvbhip.so`` in-tree with hipcc for gfx950
"""
from . import ggml  # noqa: F401

__all__ = ["ggml"]
__version__ = "0.1.0"
