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
    out = capsys.readouterr().out
    line = next(l for l in out.splitlines() if "gemm_q4k_tiled<1, 8, 2>" in l)
    assert "| 2 |" in line                                  # dispatches
    assert f"MFMA f16 {1.1e8 * 512 / 1e9:.3f} GFLOP" in line  # mean of 1.0e8 and 1.2e8, x 512 FLOP
    assert "MFMA busy 25.0%" in line                        # GRBM summed over 8 XCDs
    assert f"read {1000.0 * 1024 * 2 / 1e6:.2f} MB" in line  # copy factor 2 applied to KiB
