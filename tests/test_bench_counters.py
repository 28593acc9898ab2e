"""bench.py's counter table: per-kernel means over rocprofv3 counter_collection.csv
rows and the figures derived from them (CPU only, synthetic CSV)."""
import csv
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(FIELDS, r)))


def test_counter_table_derived_figures(tmp_path, capsys):
    gemm = "void vb::(anonymous namespace)::gemm_q4k_tiled<1, 8, 2>(unsigned char const*, int)"
    neg = "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda>(int)"
    rows = []
    # two dispatches; counters split over two instances per dispatch (summed per dispatch)
    for d, mops in ((1, 1.0e8), (2, 1.2e8)):
        rows += [(d, gemm, "SQ_INSTS_VALU_MFMA_MOPS_F16", mops / 2), (d, gemm, "SQ_INSTS_VALU_MFMA_MOPS_F16", mops / 2),
                 (d, gemm, "SQ_VALU_MFMA_BUSY_CYCLES", 1024 * 1000 * 0.25),
                 (d, gemm, "GRBM_GUI_ACTIVE", 8 * 1000), (d, gemm, "FETCH_SIZE", 1000.0)]
    rows += [(3, neg, "FETCH_SIZE", bench.CALIB_BYTES / 1024 / 2)]  # the copy reads half its bytes
    p = tmp_path / "run_counter_collection.csv"
    _write(p, rows)
    bench.counter_table([str(p)])
    out = capsys.readouterr().out.splitlines()
    # one column per library kernel (the copy is not one), one row per counter
    assert "gemm_q4k_tiled<1, 8, 2>" in out[0] and "neg_kernel" not in out[0]
    row = {l.split("|")[1].strip(): l.split("|")[2].strip() for l in out[2:]}
    assert row["dispatches"] == "2"
    assert row["MFMA f16 GFLOP"] == f"{1.1e8 * 512 / 1e9:.3f}"  # mean of 1.0e8 and 1.2e8, x 512 FLOP
    assert row["MFMA busy"] == "25.0%"                        # GRBM summed over 8 XCDs
    assert row["read MB (copy-scaled)"] == f"{1000.0 * 1024 * 2 / 1e6:.2f}"  # copy factor 2 applied to KiB


def test_counter_table_mangled_names(tmp_path, capsys):
    """Kernel names left mangled by the profiler (_Float16 parameters) still
    count as the library's, under a readable name."""
    name = "_ZN2vb12_GLOBAL__N_115moe_gate_up_q4kILi4EEEvNS0_10ExpertPtrsES2_PKDF16_PKiS6_iiiijjPDF16_"
    p = tmp_path / "run_counter_collection.csv"
    _write(p, [(1, name, "SQ_WAVES", 7168.0)])
    bench.counter_table([str(p)])
    out = capsys.readouterr().out.splitlines()
    assert "`vb::moe_gate_up_q4k<4>`" in out[0]
    assert out[3].split("|")[1].strip() == "SQ_WAVES" and out[3].split("|")[2].strip() == "7168"


def test_random_blocks_decode_to_finite_moderate_weights():
    """The random weight blocks of the GEMM lines for Q5_K and the 32-element
    types decode (oracle) to finite weights of moderate size: the fp16 scale
    fields get exponents 2^-7 .. 2^-4 whatever the random bytes were."""
    import numpy as np
    import oracle as O
    from vibeblade_amd import ggml
    rng = np.random.default_rng(3)
    for qtype in (ggml.GGML_TYPE_Q4_0, ggml.GGML_TYPE_Q4_1, ggml.GGML_TYPE_Q5_0, ggml.GGML_TYPE_Q5_1,
                  ggml.GGML_TYPE_Q5_K):
        raw = bench.random_blocks(qtype, 7, 512, rng)
        assert raw.shape == (7, ggml.row_bytes(qtype, 512)) and raw.dtype == np.uint8
        w = O.dequantize(raw, 512, qtype)
        assert np.all(np.isfinite(w))
        # |d| < 2^-3 times at most 31 (Q5_0 / Q5_1 codes; Q5_K times a 6-bit sub-block scale, 63)
        assert 0 < np.abs(w).max() < (300 if qtype == ggml.GGML_TYPE_Q5_K else 8) and np.abs(w).mean() > 1e-4
