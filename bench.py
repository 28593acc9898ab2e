"""Benchmark: Q4_K GEMV effective HBM GB/s at 14336x4096, M=1, on one MI355X.

One step = one dequant-fused GEMV y = W x with W a GGUF Q4_K 14336x4096 matrix
(Llama-3-8B FFN gate/up shape), x fp32 (4096), y fp32 (14336).  Weights are
drawn N(0, 0.02) from a fixed seed and quantized on the device; 16 distinct
weight copies (528 MB, more than the 256 MB MALL) are used round robin so
that every step streams its weights from HBM.  Steps are launched as a HIP
graph of 16 GEMVs (one per copy) so host launch overhead is off the clock.
GPU time is taken with HIP events on the launch stream around the K timed
steps (bracketed by synchronize).

value = algorithmic bytes per step / (time per step), algorithmic bytes =
weights read once + x read once + y written once = 33,103,872 B.

cpu_baseline: the reference's CPU path (cpp/src/dequant.cpp gemv_dequant,
compiled from the reference sources into oracle/_ref with its release flags)
on the same shape, single thread, on a bounded sample (~10 s), reported as
the same GB/s metric; the oracle's restatement of that loop is used when the
compiled reference is absent.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--extra]
  --extra also measures the other single-GPU GEMV shapes and prints one JSON
  line per shape to stderr (the main line stays the headline metric).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join("profiles", "q4k_gemv_14336x4096_traffic.json")
GEMV_KERNEL = "gemv_q_kernel<12"  # the Q4_K v_dot4 GEMV instantiations
CALIB_BYTES = 256 << 20            # bytes read and written by the calibration copy
MFMA_FP16_PEAK_TFS = 2500.0  # dense fp16 MFMA, MI355X
NCOPIES = 16
SEED = 1234


def alg_bytes_gemv(qtype: int, n: int, k: int) -> int:
    from vibeblade_amd import ggml
    return n * ggml.row_bytes(qtype, k) + 4 * k + 4 * n


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--extra", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--pmc-pass", nargs="?", const="gemv", choices=["gemv", "gemm8", "gemm512"],
                   help="eager launches for rocprofv3 --pmc: 32 headline GEMVs (gemv) or 16 Q4_K GEMMs "
                        "14336x4096 at M=8 / 512 (gemm8, gemm512), then a 256 MiB copy (torch.neg) "
                        "that calibrates FETCH_SIZE / WRITE_SIZE")
    p.add_argument("--counter-table", nargs="+", metavar="CSV",
                   help="per-kernel means of every counter in rocprofv3 counter_collection.csv files, "
                        "as a markdown table, with the MFMA and traffic figures derived from them")
    p.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                   help="turn the counter_collection.csv files of two --pmc-pass runs (FETCH_SIZE, "
                        "WRITE_SIZE) into " + TRAFFIC_FILE)
    return p.parse_args()


def make_copies(qtype, n, k, ncopies, gen):
    import torch
    from vibeblade_amd.tensor import QTensor
    copies = []
    for _ in range(ncopies):
        w = torch.randn((n, k), generator=gen, device="cuda") * 0.02
        copies.append(QTensor.quantize(w, qtype))
        del w
    torch.cuda.synchronize()
    return copies


GRAPH_LAUNCHES = 128  # launches captured per graph: amortizes the gap between replays


def time_launches(launch_fns, steps, warmup):
    """Capture calls of the closures in `launch_fns` (each takes a stream
    handle; rounds over the list until about GRAPH_LAUNCHES launches) in a
    HIP graph and replay it; returns (ms per launch, graph used, launches
    timed).  HIP events on the replay stream bracket the timed region."""
    import torch
    stream = torch.cuda.Stream()
    rounds = max(1, GRAPH_LAUNCHES // len(launch_fns))
    nl = rounds * len(launch_fns)

    def launch_all(s):
        for _ in range(rounds):
            for f in launch_fns:
                f(s)

    graph = None
    with torch.cuda.stream(stream):
        launch_all(stream.cuda_stream)  # warm the code objects
        stream.synchronize()
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                launch_all(torch.cuda.current_stream().cuda_stream)
        except Exception as e:  # graph capture unavailable: direct launches
            print(f"[bench] graph capture failed ({e}); timing direct launches", file=sys.stderr)
            graph = None
    reps_w = max(1, warmup // nl)
    reps = max(1, (steps + nl - 1) // nl)

    def run(nrep):
        with torch.cuda.stream(stream):
            for _ in range(nrep):
                if graph is not None:
                    graph.replay()
                else:
                    launch_all(stream.cuda_stream)

    run(reps_w)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    run(reps)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    return ms / (reps * nl), graph is not None, reps * nl


def time_gemv(qtype, n, k, steps, warmup, ncopies=NCOPIES):
    """Returns (ms_per_step, graph_used, steps_timed, copies, x, ys)."""
    import torch
    from vibeblade_amd import _lib
    gen = torch.Generator(device="cuda").manual_seed(SEED)
    copies = make_copies(qtype, n, k, ncopies, gen)
    x = torch.randn(k, generator=gen, device="cuda")
    ys = torch.empty((ncopies, n), dtype=torch.float32, device="cuda")
    lib = _lib.load()

    def mk(i, c):
        args = (c.ptr(), x.data_ptr(), ys[i].data_ptr(), n, k, qtype)

        def f(s):
            rc = lib.vb_gemv(*args, s)
            if rc != 0:
                _lib.check("vb_gemv", rc)
        return f
    ms, graph_used, nsteps = time_launches([mk(i, c) for i, c in enumerate(copies)], steps, warmup)
    return ms, graph_used, nsteps, copies, x, ys


def time_gemm(m, n, k, steps, warmup, ncopies):
    """Q4_K GEMM with fp16 X (0.1% outliers x20); returns (ms, rel-L2 of copy 0)."""
    import torch
    import oracle as O
    from vibeblade_amd import _lib, ggml
    gen = torch.Generator(device="cuda").manual_seed(SEED + m)
    copies = make_copies(ggml.GGML_TYPE_Q4_K, n, k, ncopies, gen)
    x = torch.randn((m, k), generator=gen, device="cuda")
    x[torch.rand((m, k), generator=gen, device="cuda") < 0.001] *= 20.0
    xh = x.half().contiguous()
    ys = torch.empty((ncopies, m, n), dtype=torch.float32, device="cuda")
    lib = _lib.load()

    def mk(i, c):
        args = (c.ptr(), xh.data_ptr(), 1, ys[i].data_ptr(), m, n, k, c.qtype, 0)

        def f(s):
            rc = lib.vb_gemm(*args, s)
            if rc != 0:
                _lib.check("vb_gemm", rc)
        return f
    ms, _, _ = time_launches([mk(i, c) for i, c in enumerate(copies)], steps, warmup)
    w = O.dequantize(copies[0].to_numpy_bytes(), k, copies[0].qtype).astype(np.float64)
    want = xh.float().cpu().numpy().astype(np.float64) @ w.T
    err = O.rel_l2(ys[0].cpu().numpy(), want)
    return ms, err


def time_sparse(layout, steps, warmup, ncopies=8, block=False):
    """TurboSparse FFN, H=4096, I=14336, Q4_K, S ~ Bernoulli(0.1), relu(g)*relu(u);
    block: with the pre-FFN RMSNorm and the residual (vb_sparse_ffn_block).
    Returns (ms per call, |S|, algorithmic bytes)."""
    import torch
    from vibeblade_amd import _lib, ggml
    from vibeblade_amd.tensor import QTensor, ACT_RELU2
    h, i = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(SEED + 4)
    sets = []
    for _ in range(ncopies):
        g = QTensor.quantize(torch.randn((i, h), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        u = QTensor.quantize(torch.randn((i, h), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        dshape = (h, i) if layout == 0 else (i, h)
        d = QTensor.quantize(torch.randn(dshape, generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        sets.append((g, u, d))
    rng = np.random.default_rng(42)
    s = torch.from_numpy(np.flatnonzero(rng.random(i) < 0.10).astype(np.int32)).cuda()
    x = torch.randn(h, generator=gen, device="cuda")
    y = torch.empty(h, device="cuda")
    lib = _lib.load()
    nbytes = lib.vb_sparse_ffn_workspace(h, i, s.numel(), layout)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")

    nw = 1.0 + 0.1 * torch.randn(h, generator=gen, device="cuda")

    def mk(g, u, d):
        def f(st):
            if block:
                _lib.check("vb_sparse_ffn_block", lib.vb_sparse_ffn_block(
                    g.ptr(), u.ptr(), d.ptr(), layout, x.data_ptr(), nw.data_ptr(), 1e-5, s.data_ptr(),
                    s.numel(), None, ACT_RELU2, 1, y.data_ptr(), h, i, g.qtype, ws.data_ptr(), ws.numel(), st))
                return
            rc = lib.vb_sparse_ffn(g.ptr(), u.ptr(), d.ptr(), layout, x.data_ptr(), s.data_ptr(), s.numel(),
                                   ACT_RELU2, y.data_ptr(), h, i, g.qtype, ws.data_ptr(), ws.numel(), st)
            if rc != 0:
                _lib.check("vb_sparse_ffn", rc)
        return f
    ms, _, _ = time_launches([mk(*t) for t in sets], steps, warmup)
    n_s = int(s.numel())
    rb = 2304
    down_b = h * 8064 if layout == 0 else n_s * rb
    ab = 2 * n_s * rb + down_b + 4 * h + 4 * h + 4 * n_s + (8 * h if block else 0)
    return ms, n_s, ab


def time_ffn_block(down_type, fused, steps, warmup, ncopies=8):
    """One token through the FFN block, hd=4096, inter=14336, Q4_K gate/up,
    down Q4_K or Q6_K (the two Q4_K_M mixes), RMSNorm + SiLU + residual.
    fused: vb_ffn_block (2 launches); else the reference's step order as
    separate launches (rms_norm, gate GEMV, up GEMV, silu, multiply, down
    GEMV, residual add).  Returns (ms per call, algorithmic bytes)."""
    import torch
    from vibeblade_amd import _lib, ggml
    from vibeblade_amd.tensor import QTensor, ACT_SILU
    hd, inter = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(SEED + 6)
    sets = []
    for _ in range(ncopies):
        g = QTensor.quantize(torch.randn((inter, hd), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        u = QTensor.quantize(torch.randn((inter, hd), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        d = QTensor.quantize(torch.randn((hd, inter), generator=gen, device="cuda") * 0.02, down_type)
        sets.append((g, u, d))
    x = torch.randn(hd, generator=gen, device="cuda")
    nw = 1.0 + 0.1 * torch.randn(hd, generator=gen, device="cuda")
    y = torch.empty(hd, device="cuda")
    lib = _lib.load()
    ws = torch.empty(lib.vb_ffn_block_workspace(hd, inter), dtype=torch.uint8, device="cuda")
    xn, gb, ub, hb = (torch.empty(n, device="cuda") for n in (hd, inter, inter, inter))
    db = torch.empty(hd, device="cuda")

    def mk(g, u, d):
        def f(st):
            if fused:
                _lib.check("vb_ffn_block", lib.vb_ffn_block(
                    x.data_ptr(), nw.data_ptr(), 1e-5, g.ptr(), u.ptr(), g.qtype, d.ptr(), d.qtype, hd, inter,
                    ACT_SILU, 1, y.data_ptr(), ws.data_ptr(), ws.numel(), st))
                return
            _lib.check("vb_rms_norm", lib.vb_rms_norm(x.data_ptr(), nw.data_ptr(), xn.data_ptr(), 1, hd, 1e-5, st))
            _lib.check("vb_gemv", lib.vb_gemv(g.ptr(), xn.data_ptr(), gb.data_ptr(), inter, hd, g.qtype, st))
            _lib.check("vb_gemv", lib.vb_gemv(u.ptr(), xn.data_ptr(), ub.data_ptr(), inter, hd, u.qtype, st))
            _lib.check("vb_activation", lib.vb_activation(gb.data_ptr(), hb.data_ptr(), inter, 0, st))
            torch.mul(hb, ub, out=hb)
            _lib.check("vb_gemv", lib.vb_gemv(d.ptr(), hb.data_ptr(), db.data_ptr(), hd, inter, d.qtype, st))
            torch.add(x, db, out=y)
        return f
    ms, _, _ = time_launches([mk(*t) for t in sets], steps, warmup)
    ab = 2 * inter * 2304 + hd * ggml.row_bytes(down_type, inter) + 4 * hd * 4 + 8 * inter
    return ms, ab


def time_sparse_predicted(steps, warmup, ncopies=8, predict_only=False):
    """One TurboSparse token step with the active set predicted on the device:
    vb_ema_predict (warm EMA state, k = 10 %), vb_sparse_ffn_block over the
    predicted set through its device count (RMSNorm + relu(g)*relu(u) +
    residual, neuron-major Q4_K down, H=4096, I=14336) and vb_ema_update with
    the used mask.  Returns (ms per step, mean |S|)."""
    import torch
    from vibeblade_amd import _lib, ggml
    from vibeblade_amd.tensor import QTensor, ACT_RELU2
    h, i = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(SEED + 7)
    sets = []
    for _ in range(ncopies):
        g = QTensor.quantize(torch.randn((i, h), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        u = QTensor.quantize(torch.randn((i, h), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        d = QTensor.quantize(torch.randn((i, h), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        sets.append((g, u, d))
    lib = _lib.load()
    # a warm EMA state: about 10 % of the neurons at or above the threshold
    probs = (torch.rand(i, generator=gen, device="cuda") * 0.34).contiguous()
    x = torch.randn(h, generator=gen, device="cuda")
    nw = 1.0 + 0.1 * torch.randn(h, generator=gen, device="cuda")
    y = torch.empty(h, device="cuda")
    mask = torch.empty(i, dtype=torch.uint8, device="cuda")
    active = torch.empty(i, dtype=torch.int32, device="cuda")
    count = torch.empty(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(lib.vb_sparse_ffn_workspace(h, i, i, 1), dtype=torch.uint8, device="cuda")
    k = i // 10

    def mk(g, u, d):
        def f(st):
            _lib.check("vb_ema_predict", lib.vb_ema_predict(probs.data_ptr(), None, i, k, 0.3, 1, 0, mask.data_ptr(),
                                                            active.data_ptr(), count.data_ptr(), st))
            if predict_only:
                return
            _lib.check("vb_sparse_ffn_block", lib.vb_sparse_ffn_block(
                g.ptr(), u.ptr(), d.ptr(), 1, x.data_ptr(), nw.data_ptr(), 1e-5, active.data_ptr(), i,
                count.data_ptr(), ACT_RELU2, 1, y.data_ptr(), h, i, g.qtype, ws.data_ptr(), ws.numel(), st))
            _lib.check("vb_ema_update", lib.vb_ema_update(probs.data_ptr(), i, mask.data_ptr(), 0.1, st))
        return f
    ms, _, _ = time_launches([mk(*t) for t in sets], steps, warmup)
    return ms, int(count.item())


def time_moe(steps, warmup):
    """8 Q4_K experts (gate/up 14336x4096, down 4096x14336), 16 tokens, top-2.
    Returns (ms per call, experts hit, algorithmic bytes)."""
    import torch
    from vibeblade_amd import ggml
    from vibeblade_amd.tensor import QTensor, moe_grouped_ffn
    import ctypes
    from vibeblade_amd import _lib
    e_n, h, i, t, topk = 8, 4096, 14336, 16, 2
    gen = torch.Generator(device="cuda").manual_seed(SEED + 5)
    q = lambda shape: QTensor.quantize(torch.randn(shape, generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
    gates = [q((i, h)) for _ in range(e_n)]
    ups = [q((i, h)) for _ in range(e_n)]
    downs = [q((h, i)) for _ in range(e_n)]
    x = torch.randn((t, h), generator=gen, device="cuda")
    logits = torch.randn((t, e_n), generator=gen, device="cuda")
    y, idx, w = moe_grouped_ffn(gates, ups, downs, x, logits, topk)
    hit = len(set(idx.cpu().numpy().ravel().tolist()))
    lib = _lib.load()
    arr = ctypes.c_void_p * e_n
    pg, pu, pd = arr(*[g.ptr() for g in gates]), arr(*[u.ptr() for u in ups]), arr(*[d.ptr() for d in downs])
    nbytes = lib.vb_moe_workspace(t, topk, h, i)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    yo = torch.empty((t, h), device="cuda")
    vp = ctypes.c_void_p

    def f(st):
        rc = lib.vb_moe_grouped_ffn(ctypes.cast(pg, vp), ctypes.cast(pu, vp), ctypes.cast(pd, vp), e_n,
                                    x.data_ptr(), t, logits.data_ptr(), topk, yo.data_ptr(), None, None, h, i,
                                    ggml.GGML_TYPE_Q4_K, ws.data_ptr(), ws.numel(), st)
        if rc != 0:
            _lib.check("vb_moe_grouped_ffn", rc)
    ms, _, _ = time_launches([f], steps, warmup)
    ab = hit * 3 * i * 2304 + t * h * 4 * 2 + t * e_n * 4
    return ms, hit, ab


def time_gguf_ingest(n_tensors=32, reps=3):
    """GGUF ingestion: a file of n_tensors Q4_K 14336x4096 tensors (random
    block bytes, 33 MB each) in the page cache, opened and every tensor
    uploaded to HBM (vb_gguf_open + vb_gguf_upload).  Returns the best
    rate over reps in GB/s, the bytes moved, the file and the open time."""
    import tempfile
    import torch
    from vibeblade_amd import ggml
    from vibeblade_amd.gguf import GGUFFile
    from vibeblade_amd.gguf_write import write_gguf
    rows, k = 14336, 4096
    blob = np.random.default_rng(0).integers(0, 256, rows * ggml.row_bytes(ggml.GGML_TYPE_Q4_K, k),
                                            dtype=np.uint8)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    write_gguf(path, [], [(f"blk.{i}.ffn_up.weight", (k, rows), ggml.GGML_TYPE_Q4_K, blob)
                          for i in range(n_tensors)])
    total = n_tensors * blob.size
    best, t_open = None, None
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with GGUFFile(path) as f:
            t1 = time.perf_counter()
            ws = [f.load_qtensor(f"blk.{i}.ffn_up.weight", "cuda:0") for i in range(n_tensors)]
            torch.cuda.synchronize()
            dt = time.perf_counter() - t1
        if best is None or dt < best:
            best, t_open = dt, t1 - t0
        ok = bool(torch.equal(ws[-1].data.reshape(-1), torch.from_numpy(blob).cuda()))
        del ws
        torch.cuda.empty_cache()
        if not ok:
            os.remove(path)
            raise RuntimeError("GGUF upload: device bytes differ from the file")
    return total / best / 1e9, total, path, t_open


def gguf_reader_cpu_baseline(path):
    """The reference's GGUFFile (cpp/src/gguf.cpp) opening the same file:
    it reads the whole file into RAM (gguf.cpp:199-251), the host half of
    its ingestion.  None where that reader is not built."""
    import ctypes
    lib_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle", "_ref", "libvbref_gguf.so")
    if not os.path.exists(lib_path):
        return None
    lib = ctypes.CDLL(lib_path)
    lib.ref_gguf_open.restype = ctypes.c_void_p
    lib.ref_gguf_open.argtypes = [ctypes.c_char_p]
    lib.ref_gguf_close.argtypes = [ctypes.c_void_p]
    best = None
    for _ in range(2):
        t0 = time.perf_counter()
        h = lib.ref_gguf_open(path.encode())
        dt = time.perf_counter() - t0
        if not h:
            return None
        lib.ref_gguf_close(h)
        best = dt if best is None else min(best, dt)
    return os.path.getsize(path) / best / 1e9


def check_parity(qtype, n, k, copies, x, ys):
    """Oracle check of the first copy's output (the timed results)."""
    import oracle as O
    y = ys[0].cpu().numpy()
    want = O.gemv(copies[0].to_numpy_bytes(), x.cpu().numpy(), n, k, qtype)
    return O.rel_l2(y, want)


def cpu_baseline(qtype, n, k, seconds):
    """Reference gemv_dequant (its own orientation: K rows of N) on the same
    bytes count, single thread, 10 % trimmed mean (vibeblade/benchmark.py:61-79)."""
    import oracle as O
    rng = np.random.default_rng(SEED)
    # the reference walks W as k rows of n elements: same bytes, transposed roles
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    wq = O.quantize(w, qtype)
    del w
    x = rng.standard_normal(k).astype(np.float32)
    scratch = np.empty(n, np.float32)
    kind = "reference" if O.ref_available() else "port"
    fn = O.ref_gemv_dequant if kind == "reference" else O.gemv_kn
    fn(x, wq, k, n, qtype, scratch)  # warmup
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        fn(x, wq, k, n, qtype, scratch)
        times.append(time.perf_counter() - t0)
    ts = np.sort(np.array(times))
    trim = int(len(ts) * 0.1)
    ts = ts[trim:len(ts) - trim] if len(ts) > 2 * trim + 1 else ts
    sec = float(ts.mean())
    return {
        "value": round(alg_bytes_gemv(qtype, n, k) / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": (f"{len(times)} calls of gemv_dequant Q4_K (K={k} rows x N={n}), "
                   f"{O.simd_variant()} build, 10% trimmed mean {sec * 1e3:.2f} ms/call; "
                   f"host nproc={os.cpu_count()}"),
    }


def pmc_pass(workload="gemv"):
    """Launches for counter collection: no graph (per-dispatch counters), no
    timing.  The GEMVs rotate over 16 weight copies as in the timed run; the
    GEMMs (fp16 X with 0.1% outliers x20, as timed) over 4."""
    import torch
    from vibeblade_amd import _lib, ggml
    _lib.init(0)
    qtype, n, k = ggml.GGML_TYPE_Q4_K, 14336, 4096
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    if workload == "gemv":
        gen = torch.Generator(device="cuda").manual_seed(SEED)
        copies = make_copies(qtype, n, k, NCOPIES, gen)
        x = torch.randn(k, generator=gen, device="cuda")
        y = torch.empty(n, device="cuda")
        for i in range(32):
            c = copies[i % NCOPIES]
            _lib.check("vb_gemv", lib.vb_gemv(c.ptr(), x.data_ptr(), y.data_ptr(), n, k, qtype, st))
        what = "32 GEMV dispatches"
    else:
        m = 8 if workload == "gemm8" else 512
        gen = torch.Generator(device="cuda").manual_seed(SEED + m)
        copies = make_copies(qtype, n, k, 4, gen)
        x = torch.randn((m, k), generator=gen, device="cuda")
        x[torch.rand((m, k), generator=gen, device="cuda") < 0.001] *= 20.0
        xh = x.half().contiguous()
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        for i in range(16):
            c = copies[i % 4]
            _lib.check("vb_gemm", lib.vb_gemm(c.ptr(), xh.data_ptr(), 1, y.data_ptr(), m, n, k, qtype, 0, st))
        what = f"16 GEMM dispatches at M={m}"
    torch.cuda.synchronize()
    del copies
    torch.cuda.empty_cache()
    src = torch.randn(CALIB_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(f"[bench] pmc pass done: {what}, 4 calibration copies", file=sys.stderr)


def _counter_means(path, counter):
    """Mean counter value per kernel name (all dispatches) from a rocprofv3
    counter_collection.csv."""
    import csv
    sums, cnt = {}, {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            key = (r["Kernel_Name"], r.get("Dispatch_Id", ""))
            sums[key] = sums.get(key, 0.0) + float(r["Counter_Value"])
    per_kernel = {}
    for (name, _), v in sums.items():
        per_kernel.setdefault(name, []).append(v)
    return {name: (sum(v) / len(v), len(v)) for name, v in per_kernel.items()}


def counter_table(paths):
    """Markdown table of per-kernel mean counter values (per dispatch) over
    rocprofv3 counter_collection.csv files, plus derived figures:
    MFMA FLOPs = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 (the counter counts units
    of 512 FLOPs), MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8
    XCDs x 256 CUs x 4 SIMDs), and FETCH_SIZE / WRITE_SIZE scaled by the calibration
    copy (CALIB_BYTES read and written) when it is in the same file."""
    import csv
    rows = {}
    for path in paths:
        with open(path) as f:
            recs = list(csv.DictReader(f))
        counters = sorted({r["Counter_Name"] for r in recs})
        for c in counters:
            for name, (v, cnt) in _counter_means(path, c).items():
                rows.setdefault(name, {})[c] = (v, cnt)
    calib = {c: v for name, d in rows.items() if "neg_kernel" in name for c, (v, _) in d.items()}
    names = sorted({c for d in rows.values() for c in d})
    print("| Kernel | dispatches | " + " | ".join(names) + " | derived |")
    print("|---" * (len(names) + 3) + "|")
    for kname, d in sorted(rows.items(), key=lambda t: t[0]):
        short = kname.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:80]
        nd = max(cnt for _, cnt in d.values())
        cells = [f"{d[c][0]:.4g}" if c in d else "" for c in names]
        der = []
        if "SQ_INSTS_VALU_MFMA_MOPS_F16" in d:
            der.append(f"MFMA f16 {d['SQ_INSTS_VALU_MFMA_MOPS_F16'][0] * 512 / 1e9:.3f} GFLOP")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in d and "GRBM_GUI_ACTIVE" in d:
            # GRBM_GUI_ACTIVE comes summed over the 8 XCDs' GRBM instances
            der.append("MFMA busy {:.1%}".format(
                d["SQ_VALU_MFMA_BUSY_CYCLES"][0] / (d["GRBM_GUI_ACTIVE"][0] / 8 * 256 * 4)))
        for c, fac_name in (("FETCH_SIZE", "read"), ("WRITE_SIZE", "write")):
            if c in d and calib.get(c):
                der.append(f"{fac_name} {d[c][0] * CALIB_BYTES / calib[c] / 1e6:.2f} MB (copy-scaled)")
        print(f"| `{short}` | {nd} | " + " | ".join(cells) + " | " + "; ".join(der) + " |")


def summarize_pmc(fetch_csv, write_csv):
    """Traffic per GEMV launch = FETCH_SIZE x read factor + WRITE_SIZE x write
    factor, the factors being what the calibration copy (CALIB_BYTES read and
    written) shows for the same counters (KiB per dispatch)."""
    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        means = _counter_means(path, counter)
        gemv = [(v, c, name) for name, (v, c) in means.items() if GEMV_KERNEL in name]
        calib = [(v, c, name) for name, (v, c) in means.items() if "neg_kernel" in name]
        if not gemv or not calib:
            raise SystemExit(f"{path}: no {counter} rows for the GEMV or the calibration copy")
        g_kib, g_n, g_name = max(gemv, key=lambda t: t[1])
        c_kib, c_n, _ = max(calib, key=lambda t: t[1])
        factor = CALIB_BYTES / (c_kib * 1024.0)
        out[counter] = {"gemv_kib_per_dispatch": round(g_kib, 1), "gemv_dispatches": g_n,
                        "calib_kib_per_dispatch": round(c_kib, 1), "calib_dispatches": c_n,
                        "scale_factor": round(factor, 4), "gemv_bytes": round(g_kib * 1024.0 * factor)}
        out["kernel"] = g_name
    out["traffic_bytes_per_launch"] = out["FETCH_SIZE"]["gemv_bytes"] + out["WRITE_SIZE"]["gemv_bytes"]
    out["workload"] = "Q4_K GEMV 14336x4096, M=1"
    with open(os.path.join(ROOT, TRAFFIC_FILE), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def load_traffic():
    """HBM bytes per launch from the committed counter summary, if any."""
    try:
        with open(os.path.join(ROOT, TRAFFIC_FILE)) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main():
    args = parse()
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.counter_table:
        counter_table(args.counter_table)
        return
    if args.pmc_pass:
        pmc_pass(args.pmc_pass)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)
    import torch
    from vibeblade_amd import _lib, ggml
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    _lib.init(0)

    qtype, n, k = ggml.GGML_TYPE_Q4_K, 14336, 4096
    print(f"[bench] Q4_K GEMV {n}x{k}: building {NCOPIES} weight copies", file=sys.stderr, flush=True)
    ms, graph_used, nsteps, copies, x, ys = time_gemv(qtype, n, k, args.steps, args.warmup)
    err = check_parity(qtype, n, k, copies, x, ys)
    ab = alg_bytes_gemv(qtype, n, k)
    gbs = ab / (ms * 1e-3) / 1e9
    print(f"[bench] {ms * 1e3:.2f} us/step, {gbs:.0f} GB/s, rel-L2 vs oracle {err:.2e}",
          file=sys.stderr, flush=True)
    if err > 1e-3:
        print("[bench] PARITY FAILURE", file=sys.stderr)
        sys.exit(3)
    del copies, ys
    torch.cuda.empty_cache()

    if args.extra:
        extra_shapes = [
            ("Q8_0 GEMV 4096x4096", ggml.GGML_TYPE_Q8_0, 4096, 4096),
            ("Q4_K GEMV 4096x14336 (down)", ggml.GGML_TYPE_Q4_K, 4096, 14336),
            ("Q6_K GEMV 128256x4096 (lm_head)", ggml.GGML_TYPE_Q6_K, 128256, 4096),
        ]
        for name, t, nn, kk in extra_shapes:
            ncop = 2 if nn * kk > 100e6 else NCOPIES
            ms2, _, _, cps, xx, yy = time_gemv(t, nn, kk, max(200, args.steps // 4), 50, ncop)
            e2 = check_parity(t, nn, kk, cps, xx, yy)
            b2 = alg_bytes_gemv(t, nn, kk)
            print(json.dumps({"workload": name, "us_per_call": round(ms2 * 1e3, 3),
                              "GB/s": round(b2 / (ms2 * 1e-3) / 1e9, 1),
                              "frac_hbm": round(b2 / (ms2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              "rel_l2": e2}), file=sys.stderr, flush=True)
            del cps, yy
            torch.cuda.empty_cache()
        for layout, block in ((1, False), (0, False), (1, True), (0, True)):
            ms4, n_s, b4 = time_sparse(layout, 400, 40, block=block)
            what = "block (RMSNorm + FFN + residual)" if block else "FFN"
            print(json.dumps({"workload": f"TurboSparse {what} H=4096 I=14336 |S|={n_s} down_layout={layout}",
                              "us_per_call": round(ms4 * 1e3, 3), "alg_bytes": b4,
                              "GB/s": round(b4 / (ms4 * 1e-3) / 1e9, 1),
                              "frac_hbm": round(b4 / (ms4 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}),
                  file=sys.stderr, flush=True)
            torch.cuda.empty_cache()
        ms5, hit, b5 = time_moe(50, 5)
        print(json.dumps({"workload": f"MoE 8x Q4_K experts, 16 tokens top-2 ({hit} experts hit)",
                          "us_per_call": round(ms5 * 1e3, 3), "alg_bytes": b5,
                          "GB/s": round(b5 / (ms5 * 1e-3) / 1e9, 1),
                          "frac_hbm": round(b5 / (ms5 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}),
              file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        for only in (True, False):
            ms8, n_s8 = time_sparse_predicted(400, 40, predict_only=only)
            what = ("EMA predict + compaction alone (I=14336, k=1433)" if only else
                    "TurboSparse token step on the device: EMA predict + sparse block over the device count "
                    "+ EMA update, H=4096 I=14336")
            print(json.dumps({"workload": what, "us_per_call": round(ms8 * 1e3, 3), "active": n_s8}),
                  file=sys.stderr, flush=True)
            torch.cuda.empty_cache()
        for dt_name, dt in (("Q4_K", ggml.GGML_TYPE_Q4_K), ("Q6_K", ggml.GGML_TYPE_Q6_K)):
            for fused in (True, False):
                ms7, b7 = time_ffn_block(dt, fused, 400, 40)
                print(json.dumps({"workload": f"FFN block hd=4096 inter=14336 Q4_K gate/up, {dt_name} down, "
                                              f"RMSNorm+SiLU+residual, {'fused (2 launches)' if fused else 'unfused (7 launches)'}",
                                  "us_per_call": round(ms7 * 1e3, 3), "alg_bytes": b7,
                                  "GB/s": round(b7 / (ms7 * 1e-3) / 1e9, 1),
                                  "frac_hbm": round(b7 / (ms7 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}),
                      file=sys.stderr, flush=True)
                torch.cuda.empty_cache()
        gbs6, b6, gpath, t_open = time_gguf_ingest()
        ref_gbs = gguf_reader_cpu_baseline(gpath) if not args.no_cpu_baseline else None
        os.remove(gpath)
        print(json.dumps({"workload": "GGUF ingestion: open + upload 32 Q4_K 14336x4096 tensors (page cache)",
                          "bytes": b6, "GB/s": round(gbs6, 2), "open_ms": round(t_open * 1e3, 3),
                          "cpu_baseline": None if ref_gbs is None else
                          {"value": round(ref_gbs, 2), "unit": "GB/s", "cores": 1, "kind": "reference",
                           "sample": "reference GGUFFile opening the same file (reads it into RAM)"}}),
              file=sys.stderr, flush=True)
        for m, ncop in ((8, NCOPIES), (512, 4)):
            ms3, e3 = time_gemm(m, 14336, 4096, 400 if m == 8 else 100, 40, ncop)
            flops = 2.0 * m * 14336 * 4096
            b3 = 14336 * 2304 + 2 * m * 4096 + 4 * m * 14336
            print(json.dumps({"workload": f"Q4_K GEMM M={m} N=14336 K=4096 fp16 X",
                              "us_per_call": round(ms3 * 1e3, 3),
                              "TFLOP/s": round(flops / (ms3 * 1e-3) / 1e12, 2),
                              "frac_mfma_fp16": round(flops / (ms3 * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFS, 4),
                              "GB/s": round(b3 / (ms3 * 1e-3) / 1e9, 1),
                              "frac_hbm": round(b3 / (ms3 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              "rel_l2": e3}), file=sys.stderr, flush=True)
            torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline (reference gemv_dequant, 1 thread)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(qtype, n, k, args.cpu_seconds)

    line = {
        "metric": "Q4_K GEMV eff. HBM GB/s (14336x4096, M=1) + % of MI355X peak",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": nsteps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 dot (v_dot4_i32_i8) -> i32, f32 scales",
        "data": "synthetic: W ~ N(0,0.02) quantized to GGUF Q4_K on device (16 rotating copies), x ~ N(0,1)",
        "config": {"workload": "Q4_K GEMV M=1, N=14336 rows x K=4096 (Llama-3-8B FFN gate/up)",
                   "n": n, "k": k, "m": 1, "weight_copies": NCOPIES, "hip_graph": graph_used,
                   "rel_l2_vs_oracle": float(f"{err:.3e}")},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic(),
                     "alg_bytes_per_launch": ab, "us_per_launch": round(ms * 1e3, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
