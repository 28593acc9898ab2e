"""GPU parity of the MFMA GEMM (Q4_K weights, fp16 / fp32 activations).

Bar: rel-L2 <= 5e-3 against the fp64 product of the oracle-decoded weights
(the fp16 MFMA path rounds each weight once to fp16).
"""
import numpy as np
import pytest
import torch

import oracle as O
from vibeblade_amd import ggml
from vibeblade_amd._lib import VBError
from vibeblade_amd import _lib
from vibeblade_amd.tensor import (QTensor, gemm, GEMM_AUTO, GEMM_SKINNY, GEMM_TILED, GEMM_SPLIT, GEMM_KSPLIT,
                                  GEMM_XREG)

pytestmark = pytest.mark.gpu

TOL = 5e-3
Q4K = ggml.GGML_TYPE_Q4_K
Q6K = ggml.GGML_TYPE_Q6_K
Q80 = ggml.GGML_TYPE_Q8_0


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield


def ref_gemm(qt, x):
    w = O.dequantize(qt.to_numpy_bytes(), qt.k, qt.qtype).astype(np.float64)
    return x.astype(np.float64) @ w.T


def make(m, n, k, seed, outliers=True, qtype=Q4K):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if outliers:
        mask = rng.random((m, k)) < 0.001
        x[mask] *= 20.0
    return QTensor.quantize(w, qtype), x


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (3, 50, 512), (8, 300, 1024), (16, 64, 4096),
                                   (5, 33, 14336)])
def test_skinny(dtype, m, n, k):
    qt, x = make(m, n, k, m * 7 + n)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_SKINNY).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL


@pytest.mark.parametrize("qtype", [Q4K, Q6K, Q80])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("n,k", [(64, 256), (14336, 4096), (4096, 14336), (1000, 2048)])
def test_one_row_runs_the_gemv(qtype, dtype, n, k):
    """M = 1 (variant 0) takes the GEMV path: fp32 X for every type, fp16 X on
    the short-row kernels (Q4_K k <= 4096, Q6_K k = 2048 / 4096, Q8_0
    k % 256 == 0 up to 4096) and the split-row kernels (k = 14336); other fp16
    shapes stay on the MFMA kernels.
    Same results as vb_gemv on the same (rounded) activations."""
    qt, x = make(1, n, k, n + k + qtype, qtype=qtype)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (1, n)
    assert O.rel_l2(y, want) <= TOL
    short = {Q4K: True, Q6K: k in (2048, 4096, 14336), Q80: k % 256 == 0}[qtype]
    if dtype == torch.float32 or short:
        from vibeblade_amd.tensor import gemv
        yv = gemv(qt, xt.float().reshape(-1)).cpu().numpy()
        assert np.array_equal(y.reshape(-1).view(np.uint32), yv.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(17, 16, 256), (40, 130, 512), (300, 257, 1024), (256, 128, 4096),
                                   (513, 200, 768)])
def test_tiled(dtype, m, n, k):
    qt, x = make(m, n, k, m + n * 3)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL
    # every row of the output is populated
    assert np.all(np.abs(y).sum(axis=1) > 0)


@pytest.mark.parametrize("nf", ["6", "8"])
def test_tiled_column_tiles(knob, nf):
    """Both workgroup widths (96 and 128 columns), ragged M and N edges."""
    knob("VB_GEMM_NF", nf)
    qt, x = make(300, 333, 1280, 21)
    for dtype in (torch.float16, torch.float32):
        xt = torch.from_numpy(x).to("cuda", dtype)
        y = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
        want = O.gemm(qt.to_numpy_bytes(), xt.float().cpu().numpy(), 333, 1280, qt.qtype)
        assert O.rel_l2(y, want) <= TOL, (nf, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(17, 16, 256), (24, 300, 1024), (32, 64, 4096), (20, 33, 14336),
                                   (32, 4100, 4096)])
def test_skinny_two_tiles(dtype, m, n, k):
    """17 <= M <= 32: two activation tiles share every dequantized weight
    fragment (4-wave workgroups); ragged row counts and tokens past M."""
    qt, x = make(m, n, k, m * 11 + n)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_SKINNY).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL
    assert np.all(np.abs(y).sum(axis=1) > 0)  # every token row written


@pytest.mark.parametrize("m,n,k", [(33, 16, 256), (48, 300, 1024), (64, 4100, 4096), (40, 14336, 4096),
                                   (57, 33, 14336)])
def test_skinny_four_tiles(m, n, k):
    """33 <= M <= 64, fp16 X: four activation tiles share every dequantized
    weight fragment (4-wave workgroups, the final sums in LDS past the
    staging areas); ragged row counts and tokens past M; the default route
    at N >= 8192 gives the same bits."""
    qt, x = make(m, n, k, m * 13 + n)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt, variant=GEMM_SKINNY).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL
    assert np.all(np.abs(y).sum(axis=1) > 0)
    if n >= 8192:
        assert np.array_equal(gemm(qt, xt).cpu().numpy().view(np.uint32), y.view(np.uint32))


def test_tiled_matches_skinny_on_overlap():
    qt, x = make(16, 96, 1024, 5)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    a = gemm(qt, xt, variant=GEMM_SKINNY).cpu().numpy()
    b = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(a, b) <= 1e-5


def test_gemm_rejects_bad_shapes():
    qt, x = make(4, 16, 256, 1)
    with pytest.raises(ValueError):
        gemm(qt, torch.zeros((4, 255), device="cuda"))
    with pytest.raises(ValueError):
        gemm(qt, torch.zeros((33, 256), device="cuda"), variant=GEMM_SKINNY)  # fp32 X: M <= 32
    with pytest.raises(ValueError):
        gemm(qt, torch.zeros((65, 256), device="cuda", dtype=torch.float16), variant=GEMM_SKINNY)


@pytest.mark.parametrize("m", [8, 512])
def test_config_shapes(m):
    """Q4_K GEMM at M in {8, 512}, N=14336, K=4096, fp16 X ~ N(0,1) with 0.1%
    outliers x20, fp32 output."""
    n, k = 14336, 4096
    gen = torch.Generator(device="cuda").manual_seed(m)
    w = torch.randn((n, k), generator=gen, device="cuda") * 0.02
    qt = QTensor.quantize(w, Q4K)
    del w
    x = torch.randn((m, k), generator=gen, device="cuda")
    mask = torch.rand((m, k), generator=gen, device="cuda") < 0.001
    x[mask] *= 20.0
    xh = x.half()
    y = gemm(qt, xh).cpu().numpy()
    want = ref_gemm(qt, xh.float().cpu().numpy())
    assert O.rel_l2(y, want) <= TOL


@pytest.mark.parametrize("cfg", ["4,2,8", "4,2,6", "2,4,8", "2,2,4", "2,2,6", "1,4,4", "1,4,8", "1,2,4"])
def test_tiled_tile_configs(knob, cfg):
    """Every tile configuration (VB_GEMM_TILE=wm,wn,nf), ragged M and N edges,
    fp16 and fp32 X."""
    knob("VB_GEMM_TILE", cfg)
    qt, x = make(200, 333, 1280, 23)
    for dtype in (torch.float16, torch.float32):
        xt = torch.from_numpy(x).to("cuda", dtype)
        y = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
        want = O.gemm(qt.to_numpy_bytes(), xt.float().cpu().numpy(), 333, 1280, qt.qtype)
        assert O.rel_l2(y, want) <= TOL, (cfg, dtype)
        assert np.all(np.abs(y).sum(axis=1) > 0)


@pytest.mark.parametrize("m", [17, 64, 100, 128, 129, 256])
def test_mid_m_at_config_shape(m):
    """The mid-M sizes of speculative verify and chunked prefill at
    N = 14336, K = 4096 (fp16 X with 0.1 % outliers x20), on the default tile
    for each M."""
    n, k = 14336, 4096
    gen = torch.Generator(device="cuda").manual_seed(m)
    qt = QTensor.quantize(torch.randn((n, k), generator=gen, device="cuda") * 0.02, Q4K)
    x = torch.randn((m, k), generator=gen, device="cuda")
    x[torch.rand((m, k), generator=gen, device="cuda") < 0.001] *= 20.0
    xh = x.half()
    y = gemm(qt, xh).cpu().numpy()
    want = ref_gemm(qt, xh.float().cpu().numpy())
    assert O.rel_l2(y, want) <= TOL


@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (257, 113, 512), (300, 257, 1024), (512, 224, 4096),
                                   (600, 50, 768), (1000, 333, 256)])
def test_split(m, n, k):
    """The role-split kernel (variant 3, fp16 X): ragged M (rows past M) and
    N (column tiles of 112), one to several M-tiles of 256 rows."""
    qt, x = make(m, n, k, m * 5 + n)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt, variant=GEMM_SPLIT).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL
    assert np.all(np.abs(y).sum(axis=1) > 0)


def test_split_matches_tiled(knob):
    """Same dequantized fragments, same MFMAs in the same order per output:
    the role-split and tiled kernels agree bit for bit (the tiled kernel
    without K halves, which sum in another order)."""
    knob("VB_GEMM_TILE", "2,2,4,1")
    qt, x = make(520, 250, 2048, 31)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    a = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    b = gemm(qt, xt, variant=GEMM_SPLIT).cpu().numpy()
    assert np.array_equal(a, b)


def test_split_rejects_fp32_x():
    qt, x = make(300, 16, 256, 2)
    with pytest.raises(ValueError):
        gemm(qt, torch.from_numpy(x).to("cuda", torch.float32), variant=GEMM_SPLIT)


# ---- packed-X kernel (gemm_xr.hip, variant 5 / variant 0 with a workspace) ---

@pytest.mark.parametrize("m,n,k", [(256, 224, 256), (300, 4096, 1024), (512, 14336, 4096), (600, 1136, 512),
                                   (777, 128, 2048), (256, 16, 768)])
def test_xreg(m, n, k):
    """The packed-X kernel: one or several 256-row M-tiles (a last partial
    tile moved back to end at row M, its shared rows computed twice), ragged
    N (column tiles of 112, rows past N clamped), K of 1 to 16 super-blocks."""
    qt, x = make(m, n, k, m * 3 + n + k)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt, variant=GEMM_XREG).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL
    assert np.all(np.abs(y).sum(axis=1) > 0)


def test_xreg_matches_tiled():
    """Same fp16 weights and MFMA order per output as the tiled kernel's one
    k-group configuration: agreement to fp32 rounding of the same sums."""
    qt, x = make(512, 14336, 4096, 11)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    a = gemm(qt, xt, variant=GEMM_XREG).cpu().numpy()
    b = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(a, b.astype(np.float64)) <= 1e-5


def test_xreg_auto_route():
    """Variant 0 with a workspace takes the packed-X kernel at M > 256, N >=
    8192 (fp16 X): vb_gemm_workspace says how much, and the result equals an
    explicit variant 5 call bit for bit."""
    lib = _lib.load()
    assert lib.vb_gemm_workspace(512, 14336, 4096, Q4K, 1, 0) == 512 * 4096 * 2
    assert lib.vb_gemm_workspace(300, 14336, 4096, Q4K, 1, 0) == 512 * 4096 * 2  # whole 256-row tiles
    assert lib.vb_gemm_workspace(256, 14336, 4096, Q4K, 1, 0) == 0   # M = 256: another kernel
    # N < 8192 with fewer output tiles than CUs: K splits (3 at 37 x 2 tiles),
    # the packed X plus one fp32 partial product per split
    assert lib.vb_gemm_workspace(512, 4096, 14336, Q4K, 1, 0) == 512 * 14336 * 2 + 3 * 512 * 4096 * 4
    assert lib.vb_gemm_workspace(1024, 4096, 4096, Q4K, 1, 0) == 0   # 148 tiles: no split, another kernel
    assert lib.vb_gemm_workspace(512, 14336, 4096, Q4K, 0, 0) == 0   # fp32 X
    assert lib.vb_gemm_workspace(512, 14336, 4096, Q6K, 1, 0) == 512 * 4096 * 2  # Q6_K / Q8_0 too
    assert lib.vb_gemm_workspace(512, 14336, 4096, Q80, 1, 0) == 512 * 4096 * 2
    assert lib.vb_gemm_workspace(256, 64, 256, Q4K, 1, 5) == 256 * 256 * 2
    qt, x = make(384, 8192, 1024, 5)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    a = gemm(qt, xt).cpu().numpy()
    b = gemm(qt, xt, variant=GEMM_XREG).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert O.rel_l2(a, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL


@pytest.mark.parametrize("m,n,k,splits", [(512, 4096, 14336, 3), (300, 2000, 8192, 4), (256, 64, 4096, 2)])
def test_xreg_ksplit(m, n, k, splits):
    """The packed-X kernel with K splits (output tiles fewer than the CUs):
    each split sums its super-blocks into a partial product, a second launch
    adds them in split order.  The FFN down shape (4096 x 14336, M = 512),
    ragged M and N with four splits, one tile with two.  Against the oracle,
    the tiled kernel (to fp32 rounding of the same fp16 products), and the
    default route (the same bits)."""
    lib = _lib.load()
    xf = -(-m // 256) * 256 * k * 2
    assert lib.vb_gemm_workspace(m, n, k, Q4K, 1, GEMM_XREG) == xf + splits * m * n * 4
    qt, x = make(m, n, k, m + n + k + 1)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt, variant=GEMM_XREG).cpu().numpy()
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    assert np.all(np.abs(y).sum(axis=1) > 0)
    t = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5
    if m > 256:
        assert np.array_equal(gemm(qt, xt).cpu().numpy().view(np.uint32), y.view(np.uint32))


def test_xreg_rejects():
    lib = _lib.load()
    qt, x = make(300, 64, 256, 2)
    with pytest.raises(ValueError):
        gemm(qt, torch.from_numpy(x).to("cuda", torch.float32), variant=GEMM_XREG)
    qt, x = make(255, 64, 256, 3)
    with pytest.raises(ValueError):
        gemm(qt, torch.from_numpy(x).to("cuda", torch.float16), variant=GEMM_XREG)
    # variant 5 without a workspace (vb_gemm) or with one that is too small
    qt, x = make(256, 64, 256, 4)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = torch.empty((256, 64), dtype=torch.float32, device="cuda")
    rc = lib.vb_gemm(qt.ptr(), xt.data_ptr(), 1, y.data_ptr(), 256, 64, 256, Q4K, GEMM_XREG, None)
    assert rc == -1
    ws = torch.empty(1024, dtype=torch.uint8, device="cuda")
    rc = lib.vb_gemm_ws(qt.ptr(), xt.data_ptr(), 1, y.data_ptr(), 256, 64, 256, Q4K, GEMM_XREG, ws.data_ptr(),
                        1024, None)
    assert rc == -1
    assert b"workspace" in lib.vb_last_error()


@pytest.mark.parametrize("qtype", [Q6K, Q80])
@pytest.mark.parametrize("m,n,k", [(256, 224, 256), (300, 4096, 1024), (600, 1136, 512), (777, 128, 2048),
                                   (256, 16, 768), (257, 5, 2304), (512, 14336, 4096)])
def test_xreg_types(qtype, m, n, k):
    """Q6_K and Q8_0 on the packed-X kernel (one raw buffer, two barriers per
    super-block): one or several 256-row M-tiles with a moved-back last tile,
    ragged N, K of 1 to 16 super-blocks; Q6_K rows of k = 2304 (1890 bytes)
    and 5 rows put super-blocks at every even byte offset within their
    16-byte window.  Against the oracle, and against the tiled kernel, which
    decodes the same fp16 weights."""
    qt, x = make(m, n, k, m * 5 + n + k + qtype, qtype=qtype)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt, variant=GEMM_XREG).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL, (qtype, m, n, k)
    assert np.all(np.abs(y).sum(axis=1) > 0)
    t = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("qtype", [Q6K, Q80])
@pytest.mark.parametrize("m,n,k,splits", [(512, 4096, 14336, 3), (300, 2000, 8192, 4), (384, 1000, 4096, 2)])
def test_xreg_types_ksplit(knob, qtype, m, n, k, splits):
    """Q6_K / Q8_0 on the packed-X kernel with K splits: the default route at
    M > 256 with a workspace (the same bits as variant 5), against the
    oracle and the tiled kernel with its own K splits (VB_GEMM_XR_KQ=0)."""
    lib = _lib.load()
    xf = -(-m // 256) * 256 * k * 2
    assert lib.vb_gemm_workspace(m, n, k, qtype, 1, 0) == xf + splits * m * n * 4
    qt, x = make(m, n, k, m + n + k + qtype, qtype=qtype)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt).cpu().numpy()
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    assert np.all(np.abs(y).sum(axis=1) > 0)
    assert np.array_equal(gemm(qt, xt, variant=GEMM_XREG).cpu().numpy().view(np.uint32), y.view(np.uint32))
    knob("VB_GEMM_XR_KQ", "0")
    t = gemm(qt, xt).cpu().numpy()
    assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5


def test_xreg_types_rejects():
    """Variant 5 with Q8_0 needs K % 256 == 0 (the other Q8_0 kernels take
    K % 128 == 0)."""
    qt, x = make(256, 64, 384, 6, qtype=Q80)
    with pytest.raises(VBError):
        gemm(qt, torch.from_numpy(x).to("cuda", torch.float16), variant=GEMM_XREG)


# ---- Q6_K and Q8_0 weights (gemm_kq.hip) ----------------------------------

@pytest.mark.parametrize("qtype", [Q6K, Q80])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (8, 300, 1024), (16, 33, 768), (17, 100, 512),
                                   (40, 50, 256), (64, 257, 1280), (65, 70, 512), (300, 130, 1024)])
def test_kq_types(qtype, dtype, m, n, k):
    """Q6_K and Q8_0 weights at every M tile (16 rows up to M = 16, one tile
    of 32 / 48 / 64 rows up to 64, 64- or 32-row tiles above), ragged M and N,
    K split over the 8 waves unevenly (k / 128 steps not a multiple of 8),
    fp16 and fp32 X."""
    qt, x = make(m, n, k, m * 11 + n + qtype, qtype=qtype)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL, (qtype, dtype, m, n, k)
    assert np.all(np.abs(y).sum(axis=1) > 0)


@pytest.mark.parametrize("qtype", [Q6K, Q80])
@pytest.mark.parametrize("n", [8192, 16400])
def test_kq_wide(qtype, n):
    """Wide weights at small M: two and four 16-row column groups per
    workgroup."""
    qt, x = make(5, n, 256, n + qtype, qtype=qtype)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert O.rel_l2(y, want) <= TOL


def test_kq_rows_misaligned():
    """Odd row counts of 2-byte-aligned rows: a Q8_0 row of K = 384 is 408
    bytes and a Q6_K row of K = 256 210 bytes, so every other row starts 2
    bytes into a dword; the last row's last block ends the tensor."""
    for qtype, k in ((Q80, 384), (Q6K, 256), (Q6K, 768)):
        qt, x = make(9, 7, k, k + qtype, qtype=qtype)
        xt = torch.from_numpy(x).to("cuda", torch.float16)
        y = gemm(qt, xt).cpu().numpy()
        want = ref_gemm(qt, xt.float().cpu().numpy())
        assert O.rel_l2(y, want) <= TOL, (qtype, k)


@pytest.mark.parametrize("m", [8, 512])
def test_kq_q6k_down_shape(m):
    """Q6_K 4096 x 14336 (the down projection of a Q4_K_M file) at M = 8 and
    M = 512, fp16 X ~ N(0, 1) with 0.1 % outliers x20."""
    n, k = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(100 + m)
    qt = QTensor.quantize(torch.randn((n, k), generator=gen, device="cuda") * 0.02, Q6K)
    x = torch.randn((m, k), generator=gen, device="cuda")
    x[torch.rand((m, k), generator=gen, device="cuda") < 0.001] *= 20.0
    xh = x.half()
    y = gemm(qt, xh).cpu().numpy()
    w = O.dequantize(qt.to_numpy_bytes(), k, Q6K).astype(np.float32)
    want = xh.float().cpu().numpy().astype(np.float64) @ w.T.astype(np.float64)
    assert O.rel_l2(y, want) <= TOL


def test_kq_matches_gemv_rows():
    """Row r of the Q6_K / Q8_0 GEMM against the GEMV of the same weights
    with x = X[r] (two independent kernels, fp32 X)."""
    from vibeblade_amd.tensor import gemv
    for qtype in (Q6K, Q80):
        qt, x = make(6, 96, 2048, 77 + qtype, qtype=qtype)
        xt = torch.from_numpy(x).to("cuda", torch.float32)
        y = gemm(qt, xt).cpu().numpy()
        for r in range(6):
            yr = gemv(qt, xt[r]).cpu().numpy()
            assert O.rel_l2(y[r], yr) <= TOL, (qtype, r)


@pytest.mark.parametrize("m", [1, 2])
def test_q8_0_k_rule_at_every_m(m):
    """Q8_0 needs K % 128 == 0 in vb_gemm at every M: the one-row case, which
    runs on the GEMV (which itself takes K % 32 == 0 through vb_gemv), is
    refused the same way as M = 2, so a shape valid at M = 1 stays valid at
    M = 2."""
    qt, x = make(m, 16, 192, 5, qtype=Q80)
    with pytest.raises(VBError, match="K % 128"):
        gemm(qt, torch.from_numpy(x).to("cuda", torch.float16))
    from vibeblade_amd.tensor import gemv
    y = gemv(qt, torch.from_numpy(x[0]).cuda())  # the GEMV entry takes it
    assert O.rel_l2(y.cpu().numpy(), ref_gemm(qt, x[:1].astype(np.float32))[0]) <= TOL


def test_kq_rejects():
    qt, x = make(4, 16, 256, 3, qtype=Q80)  # Q8_0 K = 256 is fine
    gemm(qt, torch.from_numpy(x).to("cuda", torch.float16))
    q8, x8 = make(4, 16, 96, 3, qtype=Q80)  # K % 128 != 0
    with pytest.raises(VBError):
        gemm(q8, torch.from_numpy(x8).to("cuda", torch.float16))
    for variant in (GEMM_SKINNY, GEMM_SPLIT):  # Q4_K-only kernels
        with pytest.raises(VBError):
            gemm(qt, torch.from_numpy(x).to("cuda", torch.float16), variant=variant)
    q8, x8 = make(4, 16, 384, 3, qtype=Q80)  # the tiled kernel takes K % 256 == 0
    with pytest.raises(VBError):
        gemm(q8, torch.from_numpy(x8).to("cuda", torch.float16), variant=GEMM_TILED)
    gemm(q8, torch.from_numpy(x8).to("cuda", torch.float16), variant=GEMM_KSPLIT)


# ---- Q6_K and Q8_0 on the LDS-tiled kernel (gemm.hip) ---------------------

@pytest.mark.parametrize("qtype", [Q6K, Q80])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (17, 33, 512), (65, 70, 512), (130, 257, 1024),
                                   (300, 130, 768), (256, 128, 4096), (520, 100, 2304)])
def test_tiled_types(qtype, dtype, m, n, k):
    """Q6_K and Q8_0 weights on the tiled kernel (variant 2) at every tile
    shape the default picks, ragged M and N, Q6_K rows of K = 768 (630 bytes:
    every other row starts 2 bytes into a dword): against the oracle, and
    against the K-split kernel, which rounds the same weights to the same fp16
    values and sums in another order."""
    qt, x = make(m, n, k, m * 7 + n + qtype, qtype=qtype)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n)
    assert O.rel_l2(y, want) <= TOL, (qtype, dtype, m, n, k)
    assert np.all(np.abs(y).sum(axis=1) > 0)
    other = gemm(qt, xt, variant=GEMM_KSPLIT).cpu().numpy()
    assert O.rel_l2(y, other) <= 1e-5
    # the default runs the tiled kernel from M = 65 on (at N < 8192: Q6_K
    # above M = 256 with fp16 X, both types above 128 with fp32 X)
    kq_max = (256 if qtype == Q6K else 0) if dtype == torch.float16 else 128
    if m >= 65 and not (n < 8192 and m <= kq_max):
        assert np.array_equal(gemm(qt, xt).cpu().numpy(), y)


@pytest.mark.parametrize("qtype", [Q6K, Q80])
@pytest.mark.parametrize("cfg", ["4,2,8", "4,2,6", "4,2,4", "2,4,8", "2,4,4", "2,2,8", "2,2,6", "2,2,4",
                                 "1,4,8", "1,4,4", "1,2,4", "1,2,6"])
def test_tiled_types_tile_configs(knob, qtype, cfg):
    """Every tile configuration with Q6_K / Q8_0 weights, ragged edges, fp16
    and fp32 X."""
    knob("VB_GEMM_TILE", cfg)
    qt, x = make(200, 333, 1280, 29 + qtype, qtype=qtype)
    for dtype in (torch.float16, torch.float32):
        xt = torch.from_numpy(x).to("cuda", dtype)
        y = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
        want = ref_gemm(qt, xt.float().cpu().numpy())
        assert O.rel_l2(y, want) <= TOL, (cfg, dtype)
        assert np.all(np.abs(y).sum(axis=1) > 0)


@pytest.mark.parametrize("qtype", [Q4K, Q6K, Q80])
@pytest.mark.parametrize("cfg", ["2,2,4", "1,4,4", "1,4,8", "1,2,4"])
def test_tiled_k_halves(knob, qtype, cfg):
    """K halves per workgroup (VB_GEMM_TILE=wm,wn,nf,2): against the oracle
    and the same tile without halves, which sums the same fp16 products in
    another order.  K = 1536 (24 steps: 12 a half) and K = 1280 (20 steps: not
    a whole number of 4-step rounds a half, so the tile runs without
    halves)."""
    for k in (1536, 1280):
        qt, x = make(200, 333, k, 31 + qtype + k, qtype=qtype)
        for dtype in (torch.float16, torch.float32):
            xt = torch.from_numpy(x).to("cuda", dtype)
            knob("VB_GEMM_TILE", cfg + ",2")
            y = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
            want = ref_gemm(qt, xt.float().cpu().numpy())
            assert O.rel_l2(y, want) <= TOL, (cfg, dtype, k)
            assert np.all(np.abs(y).sum(axis=1) > 0)
            knob("VB_GEMM_TILE", cfg)
            one = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
            assert O.rel_l2(y, one) <= 1e-5, (cfg, dtype, k)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m", [40, 200, 512, 1000])
def test_narrow_n_defaults(dtype, m):
    """Q4_K at N < 8192 on the default path: the K-split kernel at
    33 <= M <= 64, 64- and 128-row tiles with K halves up to M = 768, 128 x 128
    tiles above (K = 1536: 12 steps a half)."""
    qt, x = make(m, 1000, 1536, 41 + m, qtype=Q4K)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert O.rel_l2(y, want) <= TOL, (dtype, m)
    assert np.all(np.abs(y).sum(axis=1) > 0)


@pytest.mark.parametrize("m", [2, 5, 8, 16])
def test_small_m_long_k_runs_ksplit(m):
    """Q4_K at 2 <= M <= 16, N < 8192, K >= 8192 takes the K-split kernel by
    default: equal to variant 4 bit for bit, and to the oracle."""
    qt, x = make(m, 300, 8192, 53 + m, qtype=Q4K)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt).cpu().numpy()
    assert np.array_equal(y, gemm(qt, xt, variant=GEMM_KSPLIT).cpu().numpy())
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL


@pytest.mark.parametrize("qtype", [Q6K, Q80])
@pytest.mark.parametrize("m,n,k,zs", [(400, 1000, 4096, 4), (384, 4096, 14336, 4)])
def test_tiled_types_zsplit(knob, qtype, m, n, k, zs):
    """Q6_K / Q8_0, fp16 X, M >= 384, N < 8192, with the packed-X kernel
    switched off (VB_GEMM_XR_KQ=0): the tiled kernel splits K between
    workgroups of 256 x 128 tiles (partial products in the workspace, added in
    split order): ragged M and N with four splits, and the down shape at
    M = 384.  Against the oracle and the unsplit tiled kernel (same fp16
    products, sums grouped differently)."""
    knob("VB_GEMM_XR_KQ", "0")
    lib = _lib.load()
    assert lib.vb_gemm_workspace(m, n, k, qtype, 1, 0) == zs * m * n * 4
    assert lib.vb_gemm_workspace(m, n, k, qtype, 0, 0) == 0  # fp32 X: no split
    qt, x = make(m, n, k, m + n + qtype, qtype=qtype)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt).cpu().numpy()
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    assert np.all(np.abs(y).sum(axis=1) > 0)
    t = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("qtype", [Q6K, Q80])
def test_tiled_types_down_shape(qtype):
    """4096 x 14336 Q6_K / Q8_0 weights (the down projection) at M = 512 on
    the default path (the packed-X kernel with K split three ways between
    workgroups), against the K-split kernel and the oracle; fp16 X with 0.1 %
    outliers x20."""
    n, k, m = 4096, 14336, 512
    gen = torch.Generator(device="cuda").manual_seed(300 + qtype)
    qt = QTensor.quantize(torch.randn((n, k), generator=gen, device="cuda") * 0.02, qtype)
    x = torch.randn((m, k), generator=gen, device="cuda")
    x[torch.rand((m, k), generator=gen, device="cuda") < 0.001] *= 20.0
    xh = x.half()
    y = gemm(qt, xh).cpu().numpy()
    w = O.dequantize(qt.to_numpy_bytes(), k, qtype).astype(np.float32)
    want = xh.float().cpu().numpy().astype(np.float64) @ w.T.astype(np.float64)
    assert O.rel_l2(y, want) <= TOL
    assert O.rel_l2(y, gemm(qt, xh, variant=GEMM_KSPLIT).cpu().numpy()) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (8, 300, 1024), (17, 100, 512), (40, 50, 256),
                                   (64, 257, 1280), (100, 70, 512)])
def test_ksplit_q4k(dtype, m, n, k):
    """Q4_K on the K-split kernel (variant 4) at every M tile: against the
    oracle, and against the skinny / tiled kernel, which rounds the same
    weights to the same fp16 values and sums in another order (one row goes
    to the GEMV by default, so the skinny kernel is named for it)."""
    qt, x = make(m, n, k, m * 13 + n, qtype=Q4K)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_KSPLIT).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert O.rel_l2(y, want) <= TOL
    other = gemm(qt, xt, variant=GEMM_SKINNY if m == 1 else GEMM_AUTO).cpu().numpy()
    assert O.rel_l2(y, other) <= 1e-5


# ---- the other GGUF types: decoded once to fp16, then the tiled kernel ------

OTHER_TYPES = [ggml.GGML_TYPE_Q4_0, ggml.GGML_TYPE_Q4_1, ggml.GGML_TYPE_Q5_0, ggml.GGML_TYPE_Q5_1,
               ggml.GGML_TYPE_Q5_K, ggml.GGML_TYPE_Q2_K, ggml.GGML_TYPE_Q3_K, ggml.GGML_TYPE_BF16,
               ggml.GGML_TYPE_F16, ggml.GGML_TYPE_F32]


B32_TYPES = [ggml.GGML_TYPE_Q4_0, ggml.GGML_TYPE_Q4_1, ggml.GGML_TYPE_Q5_0, ggml.GGML_TYPE_Q5_1]


def make_other(qtype, n, k, seed):
    """Weights of `qtype` as raw GGUF bytes: random blocks with moderate
    scales for the block types, N(0, 0.02) values for the plain ones."""
    if qtype in (ggml.GGML_TYPE_F32, ggml.GGML_TYPE_F16, ggml.GGML_TYPE_BF16):
        w = (np.random.default_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
        if qtype == ggml.GGML_TYPE_F32:
            raw = w.view(np.uint8)
        elif qtype == ggml.GGML_TYPE_F16:
            raw = w.astype(np.float16).view(np.uint8)
        else:
            raw = (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        return QTensor.from_bytes(np.ascontiguousarray(raw).reshape(n, -1), qtype, n, k)
    from qblocks import rand_qblocks
    return QTensor.from_bytes(rand_qblocks(qtype, n, k, seed), qtype, n, k)


@pytest.mark.parametrize("qtype", OTHER_TYPES)
@pytest.mark.parametrize("m,n,k,dtype", [(8, 300, 512, torch.float16), (65, 200, 768, torch.float32),
                                         (1, 129, 256, torch.float16), (300, 1000, 1024, torch.float16),
                                         (2, 64, 4096, torch.float32)])
def test_gemm_other_types(qtype, m, n, k, dtype):
    """Q2_K / Q3_K / BF16 / F32 weights are decoded once to fp16 (one
    rounding, as the fused decoders round) and run on the tiled kernel; F16
    weights in place; Q5_K and the 32-element types with their own decoders
    (no workspace at these shapes).  Against the fp64 product of the
    oracle's decode; the workspace the call asks for; without a workspace
    (decoded into a stream-ordered allocation) the same bits."""
    lib = _lib.load()
    qt = make_other(qtype, n, k, m + n + k + qtype)
    x = np.random.default_rng(m + k).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).to("cuda", dtype)
    xdt = 1 if dtype == torch.float16 else 0
    # the 32-element types decode themselves, except Q5_0 / Q5_1 between the
    # K-split kernel's range (M <= 256 at N < 8192, 128 above) and the packed-X one
    five_bit_pass = qtype in (ggml.GGML_TYPE_Q5_0, ggml.GGML_TYPE_Q5_1) and m > (256 if n < 8192 else 128)
    in_place = qtype in (ggml.GGML_TYPE_F16, ggml.GGML_TYPE_Q5_K) or (qtype in B32_TYPES and not five_bit_pass)
    want_ws = 0 if in_place or (m == 1 and xdt == 0) else n * k * 2
    assert lib.vb_gemm_workspace(m, n, k, qtype, xdt, 0) == want_ws
    y = gemm(qt, xt).cpu().numpy()
    want = ref_gemm(qt, xt.float().cpu().numpy())
    assert y.shape == (m, n) and np.all(np.isfinite(y))
    assert O.rel_l2(y, want) <= TOL
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    rc = lib.vb_gemm(qt.ptr(), xt.data_ptr(), xdt, out.data_ptr(), m, n, k, qtype, 0, s)
    assert rc == 0
    assert np.array_equal(out.cpu().numpy().view(np.uint32), y.view(np.uint32))


def test_gemm_other_types_rejects():
    """Shapes and variants the kernels do not take fail with a clear error:
    a 32-element type with K not a multiple of 128 on the K-split kernel or
    of 256 above its range (the tiled kernel), a variant other than 0 / 2 on
    the decode pass."""
    qt = make_other(ggml.GGML_TYPE_Q4_0, 64, 288, 5)
    xt = torch.randn((4, 288), device="cuda", dtype=torch.float16)
    with pytest.raises(VBError, match="128"):
        gemm(qt, xt)
    xt = torch.randn((300, 288), device="cuda", dtype=torch.float16)
    with pytest.raises(VBError, match="256"):
        gemm(qt, xt)
    qt = make_other(ggml.GGML_TYPE_Q4_1, 64, 384, 7)
    with pytest.raises(ValueError):  # variant 5: k % 256
        gemm(qt, torch.randn((256, 384), device="cuda", dtype=torch.float16), variant=GEMM_XREG)
    qt = make_other(ggml.GGML_TYPE_Q5_K, 64, 512, 6)
    with pytest.raises(VBError, match="Q5_K runs the tiled"):
        gemm(qt, torch.randn((4, 512), device="cuda", dtype=torch.float16), variant=GEMM_SKINNY)


@pytest.mark.parametrize("m,n,k,dtype", [(8, 300, 512, torch.float16), (300, 1000, 1024, torch.float16),
                                         (65, 200, 768, torch.float32)])
def test_gemm_q5k_fused_matches_fp16_decode(m, n, k, dtype):
    """The fused Q5_K decoder (d sc and dmin m rounded to fp16, then one fma
    per weight) against the same tiled kernel fed the oracle's decode rounded
    to fp16 as F16 weights: the two differ only by those roundings."""
    qt = make_other(ggml.GGML_TYPE_Q5_K, n, k, m + n + 1)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt).cpu().numpy()
    wf16 = torch.from_numpy(O.dequantize(qt.to_numpy_bytes(), k, qt.qtype).astype(np.float16)).cuda()
    qh = QTensor.from_bytes(wf16.view(torch.uint8).reshape(-1), ggml.GGML_TYPE_F16, n, k)
    y16 = gemm(qh, xt).cpu().numpy()
    assert O.rel_l2(y, y16.astype(np.float64)) <= 2e-3
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
@pytest.mark.parametrize("qtype", B32_TYPES)
@pytest.mark.parametrize("m,n,k,dtype", [(1, 300, 512, torch.float16), (2, 130, 384, torch.float32),
                                         (8, 1000, 4096, torch.float16), (17, 64, 1280, torch.float16),
                                         (64, 257, 2048, torch.float32), (40, 9000, 256, torch.float16)])
def test_b32_ksplit_kernel(qtype, m, n, k, dtype):
    """Q4_0 / Q4_1 / Q5_0 / Q5_1 on the K-split kernel (one 18-24-byte block
    per lane group, odd 18- and 22-byte blocks 2 bytes into a dword; K = 384
    and 1280 leave steps over the 8 waves unevenly): variant 4 against the
    oracle, the default route up to M = 128 (no workspace; the same bits), and
    the fp16 decode pass on the tiled kernel (the same fp16 weights)."""
    lib = _lib.load()
    qt = make_other(qtype, n, k, m * 7 + n + k + qtype)
    x = np.random.default_rng(m + 9).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_KSPLIT).cpu().numpy()
    assert y.shape == (m, n) and np.all(np.abs(y).sum(axis=1) > 0)
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    if m <= 128 and not (m == 1 and dtype == torch.float32):
        assert lib.vb_gemm_workspace(m, n, k, qtype, 1 if dtype == torch.float16 else 0, 0) == 0
        assert np.array_equal(gemm(qt, xt).cpu().numpy().view(np.uint32), y.view(np.uint32))
    if k % 256 == 0:
        t = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
        assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("qtype", B32_TYPES)
@pytest.mark.parametrize("m,n,k,dtype", [(200, 300, 512, torch.float16), (129, 1000, 2048, torch.float32),
                                         (256, 8192, 256, torch.float16), (40, 90, 768, torch.float16)])
def test_b32_tiled_kernel(qtype, m, n, k, dtype):
    """The 32-element types on the tiled kernel with their own decoder
    (variant 2 at any M; the default for Q4_0 / Q4_1 at N >= 8192 and 128 < M
    <= 256): against the oracle, and against the same kernel fed the oracle's
    decode rounded to fp16 as F16 weights (the same fp16 weights, so the same
    sums to fp32 rounding)."""
    lib = _lib.load()
    qt = make_other(qtype, n, k, m * 5 + n + k + qtype)
    x = np.random.default_rng(m + 11).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert y.shape == (m, n) and np.all(np.abs(y).sum(axis=1) > 0)
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    wf16 = torch.from_numpy(O.dequantize(qt.to_numpy_bytes(), k, qtype).astype(np.float16)).cuda()
    qh = QTensor.from_bytes(wf16.view(torch.uint8).reshape(-1), ggml.GGML_TYPE_F16, n, k)
    y16 = gemm(qh, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(y, y16.astype(np.float64)) <= 1e-5
    if 128 < m <= 256 and n >= 8192 and qtype in (ggml.GGML_TYPE_Q4_0, ggml.GGML_TYPE_Q4_1):
        assert lib.vb_gemm_workspace(m, n, k, qtype, 1 if dtype == torch.float16 else 0, 0) == 0
        assert np.array_equal(gemm(qt, xt).cpu().numpy().view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("qtype", B32_TYPES)
@pytest.mark.parametrize("m,n,k", [(256, 224, 256), (300, 8192, 1024), (777, 128, 2048), (512, 4096, 14336)])
def test_b32_xreg(qtype, m, n, k):
    """The 32-element types on the packed-X kernel (9-12-piece windows of
    eight blocks): variant 5 against the oracle and the tiled kernel on the
    fp16 decode; the default route takes it at M > 256 where Q4_K does (the
    same bits), with K splits at the down shape."""
    lib = _lib.load()
    qt = make_other(qtype, n, k, m + n + k + 3 * qtype)
    x = np.random.default_rng(m + 10).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt, variant=GEMM_XREG).cpu().numpy()
    assert y.shape == (m, n) and np.all(np.abs(y).sum(axis=1) > 0)
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    t = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5
    if m > 256 and (n >= 8192 or k >= 8192):
        assert lib.vb_gemm_workspace(m, n, k, qtype, 1, 0) == lib.vb_gemm_workspace(m, n, k, qtype, 1, GEMM_XREG) > 0
        assert np.array_equal(gemm(qt, xt).cpu().numpy().view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("m,n,k,dtype", [(2, 300, 512, torch.float16), (8, 1000, 4096, torch.float32),
                                         (17, 64, 768, torch.float16), (64, 257, 2048, torch.float16),
                                         (300, 130, 1024, torch.float32)])
def test_q5k_ksplit_kernel(m, n, k, dtype):
    """Q5_K on the K-split kernel (variant 4, and variant 0 up to M = 64 at
    N < 8192, 32 above; half a super-block per step, the fifth bits from qh):
    against the oracle, and against the tiled kernel, which multiplies the
    same fp16 weights."""
    qt = make_other(ggml.GGML_TYPE_Q5_K, n, k, m * 3 + n + k)
    x = np.random.default_rng(m + 5).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).to("cuda", dtype)
    y = gemm(qt, xt, variant=GEMM_KSPLIT).cpu().numpy()
    if m <= (64 if n < 8192 else 32):  # the default route at small M
        assert np.array_equal(gemm(qt, xt).cpu().numpy().view(np.uint32), y.view(np.uint32))
    assert y.shape == (m, n) and np.all(np.abs(y).sum(axis=1) > 0)
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    t = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("m,n,k", [(256, 224, 256), (300, 4096, 1024), (777, 128, 2048), (512, 14336, 4096),
                                   (512, 4096, 14336)])
def test_q5k_xreg(m, n, k):
    """Q5_K on the packed-X kernel (11-piece raw windows, two raw buffers):
    variant 5 against the oracle and the tiled kernel (same fp16 weights);
    the default route with a workspace takes it at M > 256 where Q4_K does
    (bit-identical to variant 5), K split at the down shape."""
    lib = _lib.load()
    qt = make_other(ggml.GGML_TYPE_Q5_K, n, k, m + n + k + 13)
    x = np.random.default_rng(m + 6).standard_normal((m, k)).astype(np.float32)
    xt = torch.from_numpy(x).to("cuda", torch.float16)
    y = gemm(qt, xt, variant=GEMM_XREG).cpu().numpy()
    assert y.shape == (m, n) and np.all(np.abs(y).sum(axis=1) > 0)
    assert O.rel_l2(y, ref_gemm(qt, xt.float().cpu().numpy())) <= TOL
    t = gemm(qt, xt, variant=GEMM_TILED).cpu().numpy()
    assert O.rel_l2(y, t.astype(np.float64)) <= 1e-5
    auto = lib.vb_gemm_workspace(m, n, k, ggml.GGML_TYPE_Q5_K, 1, 0)
    if m > 256 and (n >= 8192 or k >= 8192):
        assert auto == lib.vb_gemm_workspace(m, n, k, ggml.GGML_TYPE_Q5_K, 1, GEMM_XREG) > 0
        assert np.array_equal(gemm(qt, xt).cpu().numpy().view(np.uint32), y.view(np.uint32))


