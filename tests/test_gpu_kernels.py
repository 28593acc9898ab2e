"""GPU parity: block decode, quantize and GEMV through the C ABI vs the oracle.

Bars: bit-exact for decoded weights and quantized bytes; rel-L2 <= 1e-3 for
GEMV outputs (fp32 accumulation).  Small shapes are compared against the
oracle directly; the config shapes run at full size.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vibeblade_amd import ggml
from vibeblade_amd.tensor import QTensor, gemv

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
QTYPES = [ggml.GGML_TYPE_Q4_K, ggml.GGML_TYPE_Q6_K, ggml.GGML_TYPE_Q8_0]


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rand_weights(rows, k, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)


def test_dequant_matches_compiled_reference_vectors():
    g = np.load("tests/golden/ref_vectors.npz", allow_pickle=False)
    blocks = g["q4k_blocks"]
    qt = QTensor.from_bytes(blocks.ravel(), ggml.GGML_TYPE_Q4_K, 1, 256 * blocks.shape[0])
    out = qt.dequantize().cpu().numpy().ravel()
    assert np.array_equal(bits(out), bits(g["q4k_out"].ravel()))


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("rows,k", [(1, 256), (7, 512), (33, 4096), (5, 14336)])
def test_dequant_random_bytes_bit_exact(qtype, rows, k):
    rng = np.random.default_rng(rows * 131 + k)
    rb = ggml.row_bytes(qtype, k)
    raw = rng.integers(0, 256, (rows, rb), dtype=np.uint8)
    # keep fp16 scales finite (random bytes may form inf/nan halves)
    be, bb = ggml.BLOCK[qtype]
    blk = raw.reshape(-1, bb)
    offs = {ggml.GGML_TYPE_Q4_K: [0, 2], ggml.GGML_TYPE_Q6_K: [208], ggml.GGML_TYPE_Q8_0: [0]}[qtype]
    for o in offs:
        blk[:, o + 1] &= 0x7B  # exponent < 31
    want = O.dequantize(raw, k, qtype)
    got = QTensor.from_bytes(raw, qtype, rows, k).dequantize().cpu().numpy()
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("qtype", [ggml.GGML_TYPE_F32, ggml.GGML_TYPE_F16])
def test_dequant_plain_types(qtype):
    w = rand_weights(9, 37, 1)
    raw = w.tobytes() if qtype == ggml.GGML_TYPE_F32 else w.astype(np.float16).tobytes()
    got = QTensor.from_bytes(raw, qtype, 9, 37).dequantize().cpu().numpy()
    want = w if qtype == ggml.GGML_TYPE_F32 else w.astype(np.float16).astype(np.float32)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("qtype", QTYPES)
def test_quantize_matches_oracle_bytes(qtype):
    w = rand_weights(24, 1024, 2)
    w[3, :256] = 0.0            # all-zero block
    w[4, 5] = 0.5               # outlier
    qt = QTensor.quantize(w, qtype)
    assert np.array_equal(qt.to_numpy_bytes(), O.quantize(w, qtype))


@pytest.mark.parametrize("qtype", QTYPES + [ggml.GGML_TYPE_F32, ggml.GGML_TYPE_F16])
@pytest.mark.parametrize("rows,k", [(1, 256), (13, 512), (70, 4096), (37, 14336), (9, 28672)])
def test_gemv_small_vs_oracle(qtype, rows, k):
    w = rand_weights(rows, k, rows + k)
    qt = QTensor.quantize(w, qtype)
    x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    # and each output individually close (no dropped row)
    scale = np.abs(want).max()
    assert np.max(np.abs(y - want)) <= 1e-3 * scale + 1e-6


@pytest.fixture
def q4k_mfma_path(knob):
    """Route Q4_K GEMVs through the int8-MFMA kernel (VB_GEMV_Q4K_PATH=mfma)."""
    knob("VB_GEMV_Q4K_PATH", "mfma")


@pytest.mark.parametrize("rows,k", [(1, 256), (13, 512), (70, 4096), (37, 14336), (9, 28672), (300, 1280)])
def test_gemv_q4k_mfma_path_vs_oracle(q4k_mfma_path, rows, k):
    w = rand_weights(rows, k, rows * 7 + k)
    qt = QTensor.quantize(w, ggml.GGML_TYPE_Q4_K)
    x = np.random.default_rng(k + 1).standard_normal(k).astype(np.float32)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("cfg", ["2,1", "4,4", "8,8", "16,16", "8,2", "6,3"])
def test_gemv_q4k_mfma_launch_shapes(q4k_mfma_path, knob, cfg):
    """Every k-slice / workgroup split gives the same rows (k = 4096: 16
    super-blocks; "6,3" leaves a ragged last slice)."""
    knob("VB_GEMV_MFMA_CFG", cfg)
    rows, k = 200, 4096
    qt = QTensor.quantize(rand_weights(rows, k, 11), ggml.GGML_TYPE_Q4_K)
    x = np.random.default_rng(12).standard_normal(k).astype(np.float32)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL


@pytest.mark.parametrize("cfg", ["8,1", "8,3", "16,2", "4,9", "8,7"])
@pytest.mark.parametrize("ring", ["", "1", "2", "3", "4"])
def test_gemv_dot_launch_shapes(knob, cfg, ring):
    """v_dot4 kernel launch overrides: rows per wave x ring depth (1-4; rows
    not a multiple of the depth take padding steps), one k-slice (k = 4096)
    and four (k = 14336)."""
    knob("VB_GEMV_Q4K_PATH", "dot")  # Q4_K, Q6_K and Q8_0 through the general kernel too
    knob("VB_GEMV_Q6K_PATH", "dot")
    knob("VB_GEMV_Q8_PATH", "dot")
    knob("VB_GEMV_CFG", cfg)
    if ring:
        knob("VB_GEMV_RING", ring)
    for qtype in QTYPES:
        for rows, k in ((333, 4096), (70, 14336)):
            qt = QTensor.quantize(rand_weights(rows, k, 13), qtype)
            x = np.random.default_rng(14).standard_normal(k).astype(np.float32)
            y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
            want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qtype)
            assert O.rel_l2(y, want) <= GEMV_TOL, (cfg, ring, qtype, rows, k)


def test_gemv_zero_rows_and_errors():
    qt = QTensor.quantize(rand_weights(4, 256, 3), ggml.GGML_TYPE_Q4_K)
    x = torch.zeros(256, device="cuda")
    with pytest.raises(ValueError):
        gemv(qt, torch.zeros(255, device="cuda"))
    from vibeblade_amd import _lib
    y = torch.full((4,), 7.0, device="cuda")
    _lib.call("vb_gemv", qt.ptr(), x.data_ptr(), y.data_ptr(), 0, 256, qt.qtype, 0)
    torch.cuda.synchronize()
    assert torch.all(y == 7.0)  # n = 0 writes nothing
    with pytest.raises(ValueError):
        _lib.call("vb_gemv", qt.ptr(), x.data_ptr(), y.data_ptr(), 4, 100, qt.qtype, 0)


def test_gemv_extreme_activations():
    """Outliers, zeros and tiny values in x still meet the bound."""
    k = 4096
    qt = QTensor.quantize(rand_weights(64, k, 4), ggml.GGML_TYPE_Q4_K)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(k).astype(np.float32)
    x[:64] = 0.0
    x[100] = 300.0
    x[2000:2032] = 1e-30
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, 64, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL


@pytest.mark.parametrize("qtype,k", [(ggml.GGML_TYPE_Q4_K, 4096), (ggml.GGML_TYPE_Q6_K, 4096),
                                     (ggml.GGML_TYPE_Q8_0, 4096), (ggml.GGML_TYPE_Q4_K, 14336),
                                     (ggml.GGML_TYPE_Q6_K, 14336), (ggml.GGML_TYPE_Q8_0, 14336)])
def test_gemv_outlier_unit_precision(qtype, k):
    """A 300x outlier sets the scale of its 64-element unit in the 15-bit
    activation encoding of the short-row (k = 4096) and split-row (k = 14336)
    kernels.  The whole-vector rel-L2 is dominated by the outlier's own
    product, so its exact fp64 contribution W[:, 100] x[100] is taken out of
    both outputs: the remainder (every other element, the 63 in the outlier's
    unit included) must still meet the bound."""
    n = 512
    qt = QTensor.quantize(rand_weights(n, k, 7), qtype)
    rng = np.random.default_rng(k + qtype)
    x = rng.standard_normal(k).astype(np.float32)
    x[100] = 300.0
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy().astype(np.float64)
    w = O.dequantize(qt.to_numpy_bytes(), k, qtype).astype(np.float64)
    want = w @ x.astype(np.float64)
    out = w[:, 100] * 300.0
    assert O.rel_l2(y - out, want - out) <= GEMV_TOL


CONFIG_SHAPES = [
    (ggml.GGML_TYPE_Q8_0, 4096, 4096),     # Q8_0 GEMV 4096x4096
    (ggml.GGML_TYPE_Q4_K, 14336, 4096),    # Q4_K gate/up
    (ggml.GGML_TYPE_Q4_K, 4096, 14336),    # Q4_K down
    (ggml.GGML_TYPE_Q6_K, 128256, 4096),   # Q6_K lm_head
]


@pytest.mark.parametrize("qtype,rows,k", CONFIG_SHAPES)
def test_gemv_config_shapes(qtype, rows, k):
    gen = torch.Generator(device="cuda").manual_seed(rows + k)
    w = torch.randn((rows, k), generator=gen, device="cuda") * 0.02
    qt = QTensor.quantize(w, qtype)
    del w
    x = torch.randn(k, generator=gen, device="cuda")
    y = gemv(qt, x).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x.cpu().numpy(), rows, k, qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    # the decode of the same bytes is bit-exact at full size too
    if rows * k <= 14336 * 4096:
        got = qt.dequantize().cpu().numpy()
        assert np.array_equal(bits(got), bits(O.dequantize(qt.to_numpy_bytes(), k, qtype)))


@pytest.mark.parametrize("qtype", QTYPES + [ggml.GGML_TYPE_F32, ggml.GGML_TYPE_F16])
def test_embed_rows_bit_exact(qtype):
    """Token-embedding rows decoded from device ids: equal to the oracle's
    decode of the same rows; ids outside the table give zero rows."""
    from vibeblade_amd.tensor import embed_rows
    vocab, k = 1000, 512
    rng = np.random.default_rng(77)
    if qtype in QTYPES:
        rb = ggml.row_bytes(qtype, k)
        raw = rng.integers(0, 256, (vocab, rb), dtype=np.uint8)
        be, bb = ggml.BLOCK[qtype]
        blk = raw.reshape(-1, bb)
        offs = {ggml.GGML_TYPE_Q4_K: [0, 2], ggml.GGML_TYPE_Q6_K: [208], ggml.GGML_TYPE_Q8_0: [0]}[qtype]
        for o in offs:
            blk[:, o + 1] &= 0x7B  # finite fp16 scales
        want_all = O.dequantize(raw, k, qtype)
    else:
        w = rand_weights(vocab, k, 5)
        raw = w if qtype == ggml.GGML_TYPE_F32 else w.astype(np.float16)
        want_all = raw.astype(np.float32)
        raw = np.frombuffer(raw.tobytes(), np.uint8).reshape(vocab, -1)
    table = QTensor.from_bytes(raw, qtype, vocab, k)
    ids = np.array([0, 999, 17, 17, -1, 1000, 500, 2 ** 31 - 1], np.int32)
    got = embed_rows(table, torch.from_numpy(ids)).cpu().numpy()
    for t, i in enumerate(ids):
        want = want_all[i] if 0 <= i < vocab else np.zeros(k, np.float32)
        assert np.array_equal(bits(got[t]), bits(want)), (t, i)
    assert embed_rows(table, torch.zeros(0, dtype=torch.int32)).shape == (0, k)


# ---- Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q2_K / Q3_K / Q5_K / BF16 --------------------

NEW_TYPES = [ggml.GGML_TYPE_Q4_0, ggml.GGML_TYPE_Q4_1, ggml.GGML_TYPE_Q5_0, ggml.GGML_TYPE_Q5_1, ggml.GGML_TYPE_Q5_K,
             ggml.GGML_TYPE_Q2_K, ggml.GGML_TYPE_Q3_K]


@pytest.mark.parametrize("qtype", NEW_TYPES)
@pytest.mark.parametrize("rows,k", [(3, 256), (17, 4096), (5, 14336)])
def test_new_types_decode_bit_exact(qtype, rows, k):
    from qblocks import rand_qblocks
    raw = rand_qblocks(qtype, rows, k, rows * 7 + k + qtype)
    got = QTensor.from_bytes(raw, qtype, rows, k).dequantize().cpu().numpy()
    assert np.array_equal(bits(got), bits(O.dequantize(raw, k, qtype)))


@pytest.mark.parametrize("qtype", NEW_TYPES + [ggml.GGML_TYPE_Q8_0])
@pytest.mark.parametrize("rows,k", [(1, 256), (33, 4096), (5, 14336), (300, 1024), (7, 64), (9, 128), (3, 192)])
def test_new_types_gemv(qtype, rows, k):
    """Against the fp64 oracle on the same blocks.  Rows of 64 / 128 / 192
    elements (fewer than 4 lane units) for the 32-element types; Q8_0 is
    here for those short rows too."""
    from qblocks import rand_qblocks
    if k % ggml.BLOCK[qtype][0]:
        pytest.skip("row not a whole number of blocks")
    raw = rand_qblocks(qtype, rows, k, rows + k + 3 * qtype)
    x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
    y = gemv(QTensor.from_bytes(raw, qtype, rows, k), torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(raw, x, rows, k, qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL


def test_bf16_decode_and_gemv():
    w = rand_weights(9, 100, 8)
    raw = (w.view(np.uint32) >> 16).astype(np.uint16)
    wd = (raw.astype(np.uint32) << 16).view(np.float32)
    qt = QTensor.from_bytes(raw.view(np.uint8), ggml.GGML_TYPE_BF16, 9, 100)
    assert np.array_equal(bits(qt.dequantize().cpu().numpy()), bits(wd))
    x = np.random.default_rng(1).standard_normal(100).astype(np.float32)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    assert O.rel_l2(y, wd.astype(np.float64) @ x.astype(np.float64)) <= GEMV_TOL


@pytest.mark.parametrize("qtype", NEW_TYPES)
def test_new_types_embed_rows(qtype):
    from qblocks import rand_qblocks
    from vibeblade_amd.tensor import embed_rows
    raw = rand_qblocks(qtype, 300, 512, qtype)
    ids = np.array([0, 299, 5, -1, 300, 5], np.int32)
    got = embed_rows(QTensor.from_bytes(raw, qtype, 300, 512), torch.from_numpy(ids)).cpu().numpy()
    want = O.dequantize(raw, 512, qtype)
    for t, i in enumerate(ids):
        assert np.array_equal(bits(got[t]), bits(want[i] if 0 <= i < 300 else np.zeros(512, np.float32)))


# ---- the short-row Q4_K kernel (k <= 4096, up to 8 rows per wave) ----------

def _q4k_case(rows, k, seed):
    qt = QTensor.quantize(rand_weights(rows, k, seed), ggml.GGML_TYPE_Q4_K)
    x = np.random.default_rng(seed + 1).standard_normal(k).astype(np.float32)
    return qt, x


@pytest.mark.parametrize("wpg", [8, 16])
@pytest.mark.parametrize("rpw", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("ring", ["", "1", "2", "3", "4"])
@pytest.mark.parametrize("dma", ["", "0"])
def test_gemv_q4k_short_rows_per_wave(knob, wpg, rpw, ring, dma):
    """Every rows-per-wave count with 8- and 16-wave workgroups (forced with
    VB_GEMV_CFG), at each ring depth, 8-wave workgroups with the rows landing
    in LDS by DMA (the default) and in the register ring (VB_GEMV_DMA=0);
    three full workgroups and a ragged one."""
    if wpg == 16 and dma == "0":
        pytest.skip("16-wave workgroups always use the register ring")
    knob("VB_GEMV_CFG", f"{wpg},{rpw}")
    if ring:
        knob("VB_GEMV_RING", ring)
    if dma:
        knob("VB_GEMV_DMA", dma)
    rows = 3 * wpg * rpw + 5
    qt, x = _q4k_case(rows, 4096, 10 * wpg + rpw)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, 4096, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6  # no row dropped or swapped


@pytest.mark.parametrize("rows", [1, 2047, 4096, 14336, 28672, 32768])
def test_gemv_q4k_short_default_shapes(rows):
    """The default launch shape at row counts from 1 to the largest it takes
    (32768 = 256 CUs x 16 waves x 8 rows)."""
    qt, x = _q4k_case(rows, 4096, rows)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, 4096, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("rows,k", [(1, 256), (3, 256), (17, 768), (64, 1280), (129, 2048), (1, 4096)])
def test_gemv_q4k_short_k_idle_lanes(rows, k):
    """k < 4096 leaves lanes idle: they load one of the row's own units (in
    bounds) and must contribute nothing (counted twice, it would show here)."""
    qt, x = _q4k_case(rows, k, rows + k)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6


# ---- the short-row Q6_K / Q8_0 kernel (rows of whole 16-byte slots, k <= 4096) --

SHORT_TYPES = [ggml.GGML_TYPE_Q6_K, ggml.GGML_TYPE_Q8_0]


def _short_case(qtype, rows, k, seed):
    qt = QTensor.quantize(rand_weights(rows, k, seed), qtype)
    x = np.random.default_rng(seed + 1).standard_normal(k).astype(np.float32)
    return qt, x


@pytest.mark.parametrize("qtype", SHORT_TYPES)
@pytest.mark.parametrize("rpw", [1, 2, 3, 5, 7, 8, 9, 16, 63])
@pytest.mark.parametrize("ring", ["", "1", "2"])
def test_gemv_short_rows_per_wave(knob, qtype, rpw, ring):
    """Rows per wave forced with VB_GEMV_CFG: one group of up to 8 rows, or
    8-row groups with a ragged last group (9, 63); each ring depth (ring 2
    past 8 rows per wave falls back to 3 rows in flight); three full
    workgroups and a ragged one."""
    knob("VB_GEMV_CFG", f"8,{rpw}")
    if ring:
        knob("VB_GEMV_RING", ring)
    rows = 3 * 8 * rpw + 5
    qt, x = _short_case(qtype, rows, 4096, 100 + rpw)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, 4096, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6  # no row dropped or swapped


@pytest.mark.parametrize("qtype,rows,k", [(ggml.GGML_TYPE_Q6_K, 1, 2048), (ggml.GGML_TYPE_Q6_K, 129, 2048),
                                          (ggml.GGML_TYPE_Q6_K, 4096, 2048), (ggml.GGML_TYPE_Q6_K, 1, 4096),
                                          (ggml.GGML_TYPE_Q6_K, 1024, 4096), (ggml.GGML_TYPE_Q6_K, 14336, 4096),
                                          (ggml.GGML_TYPE_Q6_K, 40000, 4096), (ggml.GGML_TYPE_Q8_0, 1, 256),
                                          (ggml.GGML_TYPE_Q8_0, 33, 512), (ggml.GGML_TYPE_Q8_0, 300, 1024),
                                          (ggml.GGML_TYPE_Q8_0, 129, 2816), (ggml.GGML_TYPE_Q8_0, 4096, 4096),
                                          (ggml.GGML_TYPE_Q8_0, 14336, 4096), (ggml.GGML_TYPE_Q8_0, 40000, 4096)])
def test_gemv_short_default_shapes(qtype, rows, k):
    """Default shapes: k < 4096 leaves lanes idle (they read a unit of their
    own row and contribute nothing); row counts from 1 to 20 rows per wave."""
    qt, x = _short_case(qtype, rows, k, rows + k)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6


def test_gemv_q8_short_integer_range():
    """Q8_0 codes at -128 / 127 with x at a constant magnitude (every x16 =
    +-16383): each block's integer sum reaches 32 * 128 * 16383; random bytes
    in the other rows (finite fp16 d)."""
    k, rows = 4096, 64
    rng = np.random.default_rng(10)
    raw = rng.integers(0, 256, (rows, ggml.row_bytes(ggml.GGML_TYPE_Q8_0, k)), dtype=np.uint8)
    blk = raw.reshape(rows, -1, 34)
    blk[:, :, 1] &= 0x7B  # fp16 d finite
    blk[0, :, 2:] = 0x80  # -128
    blk[1, :, 2:] = 0x7F  # 127
    blk[:2, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    for x in (np.ones(k, np.float32), -np.ones(k, np.float32)):
        qt = QTensor.from_bytes(raw, ggml.GGML_TYPE_Q8_0, rows, k)
        y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
        want = O.gemv(raw, x, rows, k, ggml.GGML_TYPE_Q8_0)
        assert np.allclose(y[:2], want[:2], rtol=1e-5, atol=0), (y[:2], want[:2])
        assert O.rel_l2(y, want) <= GEMV_TOL


def test_gemv_q6k_short_integer_range():
    """Codes and scales at the ends of their ranges: q6 = 0 (q = -32) or 63,
    scales -128 / 127, and x at a constant magnitude, so every x16 is
    +-16383 and each run's integer sum reaches 16 * 32 * 16383; the pair
    sums S_01 / S_23 then sit just below 2^31.  Random bytes in other rows
    (finite fp16 d)."""
    k, rows = 4096, 64
    rng = np.random.default_rng(9)
    raw = rng.integers(0, 256, (rows, ggml.row_bytes(ggml.GGML_TYPE_Q6_K, k)), dtype=np.uint8)
    blk = raw.reshape(rows, -1, 210)
    blk[:, :, 209] &= 0x7B            # fp16 d finite
    blk[0, :, :192] = 0               # q6 = 0 everywhere: q = -32
    blk[0, :, 192:208] = 0x80         # scales -128
    blk[1, :, :192] = 0xFF            # q6 = 63: q = 31
    blk[1, :, 192:208] = 0x7F         # scales 127
    blk[2, :, :192] = 0
    blk[2, :, 192:208] = 0x7F
    blk[:3, :, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    for x in (np.ones(k, np.float32), -np.ones(k, np.float32), np.where(np.arange(k) % 2, 1.0, -1.0).astype(np.float32)):
        qt = QTensor.from_bytes(raw, ggml.GGML_TYPE_Q6_K, rows, k)
        y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
        want = O.gemv(raw, x, rows, k, ggml.GGML_TYPE_Q6_K)
        assert np.allclose(y[:3], want[:3], rtol=1e-5, atol=0), (y[:3], want[:3])
        assert O.rel_l2(y, want) <= GEMV_TOL


@pytest.mark.parametrize("qtype,rows,env", [(ggml.GGML_TYPE_Q6_K, 128256, "VB_GEMV_Q6K_PATH"),
                                            (ggml.GGML_TYPE_Q8_0, 4096, "VB_GEMV_Q8_PATH")])
def test_gemv_short_matches_general_kernel(knob, qtype, rows, env):
    """The short-row kernel and the general kernel agree at the lm_head and
    Q8_0 4096 x 4096 shapes, both close to the oracle; repeated launches are
    bit-identical."""
    k = 4096
    gen = torch.Generator(device="cuda").manual_seed(79)
    qt = QTensor.quantize(torch.randn((rows, k), generator=gen, device="cuda") * 0.02, qtype)
    x = torch.randn(k, generator=gen, device="cuda")
    y_short = gemv(qt, x).cpu().numpy()
    assert np.array_equal(bits(gemv(qt, x).cpu().numpy()), bits(y_short))
    knob(env, "dot")
    y_gen = gemv(qt, x).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x.cpu().numpy(), rows, k, qt.qtype)
    assert O.rel_l2(y_short, want) <= 2e-4 and O.rel_l2(y_gen, want) <= 2e-4


# ---- the split-row Q6_K / Q8_0 kernel (4096 < k <= 16384) --------------------

# (rows, k): 2 slices per row (Q6_K k = 4608: slices of 40 and 32 units; Q8_0
# k = 4352: 36 and 32; k = 7168), 4 (k = 14336), 8 with a short last slice
# (k = 14848: 7 x 32 + 8 units), rows per wave 1 to 8
TSPLIT_SHAPES = [(1, 4608), (2049, 4608), (3000, 7168), (4096, 14336), (8192, 14336), (1000, 14848),
                 (513, 16384)]


@pytest.mark.parametrize("qtype", SHORT_TYPES)
@pytest.mark.parametrize("rows,k", TSPLIT_SHAPES + [(77, 4352), (4096, 11264)])
def test_gemv_split_rows(qtype, rows, k):
    """Q6_K rows need k % 512 == 0 for the split kernel (Q6_K k = 4352 takes the
    general kernel); every case against the oracle."""
    qt, x = _short_case(qtype, rows, k, rows + k + qtype)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6  # no row or slice dropped


@pytest.mark.parametrize("cfg", ["2,1", "4,1", "4,3", "8,2", "8,4"])
def test_gemv_split_knob(knob, cfg):
    """VB_GEMV_SPLIT="slices,rows in flight" on the Q6_K / Q8_0 split kernel
    (4 rows in flight run as 3; 2 slices of 112-unit rows exceed a 56-unit
    slice: the general kernel takes k = 14336 then)."""
    knob("VB_GEMV_SPLIT", cfg)
    for qtype in SHORT_TYPES:
        for rows, k in ((5000, 7168), (4096, 14336)):
            qt, x = _short_case(qtype, rows, k, rows + k + 2)
            y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
            want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
            assert O.rel_l2(y, want) <= GEMV_TOL, (cfg, qtype, rows, k)
            assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("qtype,env", [(ggml.GGML_TYPE_Q6_K, "VB_GEMV_Q6K_PATH"),
                                       (ggml.GGML_TYPE_Q8_0, "VB_GEMV_Q8_PATH")])
def test_gemv_split_matches_general_kernel(knob, qtype, env):
    """At the FFN down shape (4096 x 14336) the split-row kernel and the
    general kernel agree, both close to the oracle; repeated launches are
    bit-identical (fixed-order slice sums)."""
    rows, k = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(80)
    qt = QTensor.quantize(torch.randn((rows, k), generator=gen, device="cuda") * 0.02, qtype)
    x = torch.randn(k, generator=gen, device="cuda")
    y_split = gemv(qt, x).cpu().numpy()
    assert np.array_equal(bits(gemv(qt, x).cpu().numpy()), bits(y_split))
    knob(env, "dot")
    y_gen = gemv(qt, x).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x.cpu().numpy(), rows, k, qt.qtype)
    assert O.rel_l2(y_split, want) <= 2e-4 and O.rel_l2(y_gen, want) <= 2e-4


# ---- the split-row Q4_K kernel (4096 < k <= 16384, rows over 2/4/8 waves) --

# (rows, k): 2 slices per row up to 112 units (k = 7168), 4 up to 224
# (k = 14336), 8 above; rows per wave from 1 to 8 on 256 CUs (2048, 1024 and
# 512 row groups), ragged row counts, a last slice of 4 units (k = 14592)
SPLIT_SHAPES = [(1, 4352), (2049, 4352), (16384, 7168), (10000, 7168), (7, 7424), (3000, 7424),
                (4096, 14336), (8192, 14336), (1000, 14592), (513, 16384), (4096, 16384)]


@pytest.mark.parametrize("rows,k", SPLIT_SHAPES)
def test_gemv_q4k_split_rows(rows, k):
    qt, x = _q4k_case(rows, k, rows + k)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL
    assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6  # no row or slice dropped


@pytest.mark.parametrize("cfg", ["2,1", "2,3", "4,1", "4,4", "8,2", "8,3"])
def test_gemv_q4k_split_knob(knob, cfg):
    """VB_GEMV_SPLIT="slices,rows in flight": every ring depth at 2, 4 and 8
    slices per row (2 slices of 112-unit rows exceed a 56-unit slice, so
    k = 14336 then takes the general kernel)."""
    knob("VB_GEMV_SPLIT", cfg)
    for rows, k in ((5000, 7168), (4096, 14336)):
        qt, x = _q4k_case(rows, k, rows + k + 1)
        y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
        want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
        assert O.rel_l2(y, want) <= GEMV_TOL, (cfg, rows, k)
        assert np.max(np.abs(y - want)) <= 1e-3 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("rows,k", [(8193, 14336), (300, 16640)])
def test_gemv_q4k_split_declines(rows, k):
    """Past 8 rows per wave or 256 units the general kernel takes the launch."""
    qt, x = _q4k_case(rows, k, rows + k)
    y = gemv(qt, torch.from_numpy(x).cuda()).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y, want) <= GEMV_TOL


def test_gemv_q4k_split_matches_general_kernel(knob):
    """The split-row kernel and the general v_dot4 kernel agree at the FFN
    down shape (4096 x 14336), both close to the oracle; repeated launches
    are bit-identical (fixed-order slice sums)."""
    rows, k = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(78)
    qt = QTensor.quantize(torch.randn((rows, k), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
    x = torch.randn(k, generator=gen, device="cuda")
    y_split = gemv(qt, x).cpu().numpy()
    assert np.array_equal(bits(gemv(qt, x).cpu().numpy()), bits(y_split))
    knob("VB_GEMV_Q4K_PATH", "dot")
    y_gen = gemv(qt, x).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x.cpu().numpy(), rows, k, qt.qtype)
    assert O.rel_l2(y_split, want) <= 2e-4 and O.rel_l2(y_gen, want) <= 2e-4


@pytest.mark.parametrize("rows,k", [(14336, 4096), (2047, 4096), (129, 2048), (17, 768), (1, 256),
                                    (4096, 14336), (129, 8192), (5, 16384)])
def test_gemv_q4k_dma_rows_match_register_ring(knob, rows, k):
    """Rows (k <= 4096) or row slices (the split-row kernel, k > 4096) landing
    in LDS by DMA and the same through the register ring feed the same
    arithmetic: the outputs are bit-identical."""
    qt, x = _q4k_case(rows, k, 3 * rows + k)
    xt = torch.from_numpy(x).cuda()
    y_dma = gemv(qt, xt).cpu().numpy()
    knob("VB_GEMV_DMA", "0")
    y_reg = gemv(qt, xt).cpu().numpy()
    assert np.array_equal(bits(y_dma), bits(y_reg))
    want = O.gemv(qt.to_numpy_bytes(), x, rows, k, qt.qtype)
    assert O.rel_l2(y_dma, want) <= GEMV_TOL


def test_stream_read_probe_modes():
    """The floor probe runs in its register and DMA modes and refuses rings
    it does not have (it computes nothing: only the return codes are checked)."""
    from vibeblade_amd import _lib
    lib = _lib.load()
    rows, k = 14336, 4096
    rb = ggml.row_bytes(ggml.GGML_TYPE_Q4_K, k)
    w = torch.zeros(rows * rb, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    for ring in (-3, -2, -1, 0, 1, 3, 8):
        assert lib.vb_stream_read(w.data_ptr(), rows, rb, ring, sink.data_ptr(), s) == 0, ring
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0  # zeros fold to 0, never the sink's trigger value
    for ring in (-4, 9):
        assert lib.vb_stream_read(w.data_ptr(), rows, rb, ring, sink.data_ptr(), s) != 0, ring


def test_gemv_q4k_short_matches_general_kernel(knob):
    """The short-row kernel and the general v_dot4 kernel agree at the
    headline shape (both against the oracle; 16-bit vs 15-bit x encodings)."""
    rows, k = 14336, 4096
    gen = torch.Generator(device="cuda").manual_seed(77)
    qt = QTensor.quantize(torch.randn((rows, k), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
    x = torch.randn(k, generator=gen, device="cuda")
    y_short = gemv(qt, x).cpu().numpy()
    knob("VB_GEMV_Q4K_PATH", "dot")
    y_gen = gemv(qt, x).cpu().numpy()
    want = O.gemv(qt.to_numpy_bytes(), x.cpu().numpy(), rows, k, qt.qtype)
    assert O.rel_l2(y_short, want) <= 2e-4 and O.rel_l2(y_gen, want) <= 2e-4
