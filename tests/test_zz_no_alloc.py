"""The allocation-free sparse FFN entry point (vb_sparse_ffn_noalloc): its
workspace is the library's static device scratch.  Checked through the C
ABI against vb_sparse_ffn with a caller workspace (same kernels, so the same
bits) and against the fp64 oracle (rel-L2 <= 1e-3), on two calls in a row,
the second with a smaller input; sizes beyond the scratch are refused with
an error before any launch."""
import numpy as np
import pytest
import torch

import oracle as O
from vibeblade_amd import _lib, ggml
from vibeblade_amd.tensor import QTensor, ACT_RELU2, ACT_SILU

pytestmark = pytest.mark.gpu
Q4K = ggml.GGML_TYPE_Q4_K


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    _lib.init(0)
    yield


def dec(qt):
    return O.dequantize(qt.to_numpy_bytes(), qt.k, qt.qtype)


def case(h, i, layout, p_active, seed):
    rng = np.random.default_rng(seed)
    g = QTensor.quantize((rng.standard_normal((i, h)) * 0.02).astype(np.float32), Q4K)
    u = QTensor.quantize((rng.standard_normal((i, h)) * 0.02).astype(np.float32), Q4K)
    dshape = (h, i) if layout == 0 else (i, h)
    d = QTensor.quantize((rng.standard_normal(dshape) * 0.02).astype(np.float32), Q4K)
    s = np.flatnonzero(rng.random(i) < p_active).astype(np.int32)
    x = rng.standard_normal(h).astype(np.float32)
    return g, u, d, s, x


def run_pair(lib, g, u, d, s, x, layout, act):
    """(no-alloc result, workspace result, fp64 oracle) for one case."""
    h, i = x.size, g.rows
    xd = torch.from_numpy(x).cuda()
    sd = torch.from_numpy(s).cuda()
    y0 = torch.full((h,), float("nan"), device="cuda")
    y1 = torch.full((h,), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.vb_sparse_ffn_noalloc(g.ptr(), u.ptr(), d.ptr(), layout, xd.data_ptr(), sd.data_ptr(), s.size, act,
                                   y0.data_ptr(), h, i, Q4K, st)
    _lib.check("vb_sparse_ffn_noalloc", rc)
    nbytes = lib.vb_sparse_ffn_workspace(h, i, s.size, layout)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    _lib.check("vb_sparse_ffn", lib.vb_sparse_ffn(g.ptr(), u.ptr(), d.ptr(), layout, xd.data_ptr(), sd.data_ptr(),
                                                  s.size, act, y1.data_ptr(), h, i, Q4K, ws.data_ptr(), ws.numel(),
                                                  st))
    torch.cuda.synchronize()
    dd = dec(d) if layout == 0 else np.ascontiguousarray(dec(d).T)
    want = O.sparse_ffn(dec(g), dec(u), dd, x, s, O.ACT_SILU if act == ACT_SILU else O.ACT_DRELU)[0]
    return y0.cpu().numpy(), y1.cpu().numpy(), want


@pytest.mark.parametrize("layout", [1, 0])
def test_noalloc_matches_workspace_entry_twice(layout):
    """Config-4 shape, then a smaller one (fewer neurons, smaller h): the
    second call reuses the scratch the first one left behind."""
    lib = _lib.load()
    for (h, i, p, seed, act) in ((4096, 14336, 0.10, 3, ACT_RELU2), (2048, 4096, 0.05, 4, ACT_SILU)):
        g, u, d, s, x = case(h, i, layout, p, seed)
        y0, y1, want = run_pair(lib, g, u, d, s, x, layout, act)
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32)), (layout, h, i)
        assert O.rel_l2(y0, want) <= 1e-3, (layout, h, i)


def test_noalloc_rejects_beyond_scratch():
    """Every neuron active at h = 4096 on the fused path needs 29 MB of
    partials, beyond the 8 MiB scratch: an error, y untouched."""
    lib = _lib.load()
    h, i = 4096, 14336
    need = lib.vb_sparse_ffn_workspace(h, i, i, 1)
    assert need > (8 << 20)
    g, u, d, _, x = case(h, i, 1, 0.0, 5)
    s = torch.arange(i, dtype=torch.int32, device="cuda")
    xd = torch.from_numpy(x).cuda()
    y = torch.full((h,), 7.0, device="cuda")
    rc = lib.vb_sparse_ffn_noalloc(g.ptr(), u.ptr(), d.ptr(), 1, xd.data_ptr(), s.data_ptr(), i, ACT_RELU2,
                                   y.data_ptr(), h, i, Q4K, torch.cuda.current_stream().cuda_stream)
    assert rc == -1
    assert b"scratch" in lib.vb_last_error()
    torch.cuda.synchronize()
    assert bool(torch.all(y == 7.0))
