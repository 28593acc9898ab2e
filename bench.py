"""Benchmark: Q4_K GEMV effective HBM GB/s at 14336x4096, M=1, on one MI355X.

Workload: one dequant-fused GEMV y = W x with W a GGUF Q4_K 14336x4096 matrix
(Llama-3-8B FFN gate/up shape), x fp32 (4096), y fp32 (14336).  Weights are
drawn N(0, 0.02) from a fixed seed and quantized on the device; 16 distinct
weight copies (528 MB, more than the 256 MB MALL) are used round robin so
that every launch streams its weights from HBM.

A step is eight passes over the 16 copies: 128 GEMV launches, captured once
as a HIP graph and replayed, so host launch overhead is off the clock and the
replay boundary is spread over 128 launches.  W untimed warmup steps, then
exactly K timed steps; a HIP event on the replay stream is recorded before
the first step and after every step, so each step is timed on its own.  The
reported time per launch is the median over the K steps of (step time /
128); K = 20 is 2560 launches.

value = algorithmic bytes per launch / median time per launch, algorithmic
bytes = weights read once + x read once + y written once = 33,103,872 B.

cpu_baseline: the oracle's C restatement of the reference CPU path
(cpp/src/dequant.cpp:739-780 gemv_dequant: decode each of the K rows into an
fp32 scratch row, then a saxpy; single thread, like the reference's
gemv_dequant_mt at :783-792) on the same shape, on a bounded sample (about
10 s), reported as the same GB/s metric with the host CPU model.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--extra [LIST]]
  --extra also measures the other configurations (comma list of gemv,
  sparse, moe, predict, ffn, gguf, gemm, msweep, cpu; default all) and
  prints one JSON line per workload to stderr (the main line stays the
  headline metric).  Every workload rotates more than 512 MB of distinct
  weights.
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
GEMV_KERNELS = ("gemv_q4k_dma_kernel<", "gemv_q4k_kernel<")  # the Q4_K short-row GEMV instantiations
CALIB_BYTES = 256 << 20            # bytes read and written by the calibration copy
MFMA_FP16_PEAK_TFS = 2500.0  # dense fp16 MFMA, MI355X
NCOPIES = 16
MIN_ROTATION_BYTES = 512 << 20     # every timed rotation touches more than this
SEED = 1234
EXTRA_ALL = ("gemv", "sparse", "moe", "predict", "ffn", "gguf", "gemm", "msweep", "cpu")
# Arithmetic of the GEMV kernels that the GEMV lines time (the short-row Q4_K
# kernel of the headline, the short-row Q6_K / Q8_0 kernels and the split-row
# kernels): x encoded per workgroup as 15-bit fixed point (|x16| <= 16383) with
# one fp32 scale per 64-element unit, each value split into two signed bytes;
# weights as stored (4-, 6- or 8-bit codes); v_dot4_i32_i8 integer dot
# products, integer scale/min combination per run, fp32 per unit and row.
DTYPE_GEMV = ("i8 x i8 dot (v_dot4_i32_i8) -> i32; x as 15-bit fixed point with one f32 scale per "
              "64-element unit (two int8 halves per value); f32 scale combination per unit, f32 accumulate")


DTYPE_GEMM = "fp16 X x W dequantized to fp16 (one rounding) on v_mfma_f32_16x16x32_f16, f32 accumulate"


def alg_bytes_gemv(qtype: int, n: int, k: int) -> int:
    from vibeblade_amd import ggml
    return n * ggml.row_bytes(qtype, k) + 4 * k + 4 * n


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--extra", nargs="?", const=",".join(EXTRA_ALL), default=None,
                   help="comma list of extra workloads: " + ",".join(EXTRA_ALL))
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--pmc-pass", nargs="?", const="gemv",
                   choices=["gemv", "lmhead", "down", "gemm8", "gemm512", "down512", "down512q6", "sparse", "moe"],
                   help="eager launches for rocprofv3 --pmc: 32 headline GEMVs (gemv), 16 Q4_K GEMMs "
                        "14336x4096 at M=8 / 512 (gemm8, gemm512) or 4096x14336 at M=512 (down512; Q6_K: "
                        "down512q6), 16 "
                        "neuron-major TurboSparse FFN calls (sparse) or 8 MoE calls (moe), each as the timed "
                        "run launches it, then a 256 MiB copy (torch.neg) that calibrates FETCH_SIZE / "
                        "WRITE_SIZE")
    p.add_argument("--counter-table", nargs="+", metavar="CSV",
                   help="per-kernel means of every counter in rocprofv3 counter_collection.csv files, "
                        "as a markdown table, with the MFMA and traffic figures derived from them")
    p.add_argument("--floor", action="store_true",
                   help="one-launch floor table for the headline shape (same protocol: rotating weight copies, "
                        "128-launch graph replays): the GEMV beside a read-only probe with its launch shape and "
                        "loads (vb_stream_read, several rings), torch's reduction and copy over the same bytes, "
                        "and a one-workgroup launch; one JSON line each on stderr")
    p.add_argument("--mfma-ceiling", action="store_true",
                   help="what the chip's fp16 MFMA reaches on the GEMM shapes with the vendor library: "
                        "torch.matmul (hipBLASLt) on fp16 weights (no decode) at 14336x4096, M = 512 / 1024 / "
                        "2048 / 4096, and 4096x14336 at M = 512, with random and with all-zero X, beside the "
                        "Q4_K GEMM at the same shapes; one JSON line each on stderr")
    p.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                   help="turn the counter_collection.csv files of two --pmc-pass runs (FETCH_SIZE, "
                        "WRITE_SIZE) into " + TRAFFIC_FILE)
    return p.parse_args()


def copies_for(bytes_per_copy: int, minimum: int = NCOPIES) -> int:
    """Distinct weight copies so that one rotation touches > MIN_ROTATION_BYTES."""
    return max(minimum, MIN_ROTATION_BYTES // max(1, bytes_per_copy) + 1)


def random_blocks(qtype, n, k, rng):
    """(n, row_bytes) uint8 of random blocks whose fp16 scale fields (d, and
    dmin / m where the type has one) have exponent 2^-7 .. 2^-4 and a random
    sign and mantissa: for the types vb_quantize_rows does not write."""
    from vibeblade_amd import ggml
    offsets = {ggml.GGML_TYPE_Q4_0: (0,), ggml.GGML_TYPE_Q4_1: (0, 2), ggml.GGML_TYPE_Q5_0: (0,),
               ggml.GGML_TYPE_Q5_1: (0, 2), ggml.GGML_TYPE_Q5_K: (0, 2)}[qtype]
    raw = rng.integers(0, 256, (n, ggml.row_bytes(qtype, k)), dtype=np.uint8)
    blk = raw.reshape(-1, ggml.BLOCK[qtype][1])
    for o in offsets:
        blk[:, o + 1] = (blk[:, o + 1] & 0x83) | (0x20 + (blk[:, o] & 0x0C))
    return raw


def make_copies(qtype, n, k, ncopies, gen):
    """Weight copies: N(0, 0.02) quantized on the device for Q4_K / Q6_K /
    Q8_0, random blocks (random_blocks) for the other block types."""
    import torch
    from vibeblade_amd import ggml
    from vibeblade_amd.tensor import QTensor
    copies = []
    if qtype not in (ggml.GGML_TYPE_Q4_K, ggml.GGML_TYPE_Q6_K, ggml.GGML_TYPE_Q8_0):
        rng = np.random.default_rng(SEED + qtype)
        for _ in range(ncopies):
            copies.append(QTensor.from_bytes(random_blocks(qtype, n, k, rng), qtype, n, k))
        torch.cuda.synchronize()
        return copies
    for _ in range(ncopies):
        w = torch.randn((n, k), generator=gen, device="cuda") * 0.02
        copies.append(QTensor.quantize(w, qtype))
        del w
    torch.cuda.synchronize()
    return copies


class Timing:
    """Per-launch times of a timed run: median over steps of (step time /
    launches per step), the plain mean, and the counts."""

    def __init__(self, step_ms, per_step, total_ms, graph):
        self.steps = len(step_ms)
        self.per_step = per_step
        self.launches = self.steps * per_step
        self.step_ms = float(np.median(step_ms))
        self.ms = self.step_ms / per_step               # median per launch
        self.mean_ms = total_ms / self.launches          # mean per launch
        self.graph = graph

    def us(self):
        return round(self.ms * 1e3, 3)


GRAPH_MIN_LAUNCHES = 128  # launches per graph replay: spreads the replay boundary over them


def time_launches(launch_fns, steps, warmup, min_launches=200):
    """One step = `passes` rounds of calls of every closure in `launch_fns`
    (each takes a stream handle; passes = ceil(GRAPH_MIN_LAUNCHES / len)),
    captured once as a HIP graph and replayed.  `warmup` untimed steps, then
    max(steps, ceil(min_launches / launches per step)) timed steps, each
    bracketed by HIP events on the replay stream.  Returns a Timing."""
    import torch
    # the inputs were made on torch's current stream, and the closures run on
    # a new one: wait for every pending kernel first, so no buffer (nor a
    # block the caching allocator handed out again) is still being written
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    passes = -(-GRAPH_MIN_LAUNCHES // len(launch_fns))
    nl = passes * len(launch_fns)
    steps = max(steps, -(-min_launches // nl))

    def launch_all(s):
        for _ in range(passes):
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

    def one():
        if graph is not None:
            graph.replay()
        else:
            launch_all(stream.cuda_stream)

    with torch.cuda.stream(stream):
        for _ in range(warmup):
            one()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    with torch.cuda.stream(stream):
        evs[0].record(stream)
        for i in range(steps):
            one()
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    step_ms = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    return Timing(step_ms, nl, evs[0].elapsed_time(evs[-1]), graph is not None)


def time_gemv(qtype, n, k, steps, warmup, ncopies=None):
    """Returns (Timing, copies, x, ys)."""
    import torch
    from vibeblade_amd import _lib, ggml
    if ncopies is None:
        ncopies = copies_for(n * ggml.row_bytes(qtype, k))
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
    tm = time_launches([mk(i, c) for i, c in enumerate(copies)], steps, warmup)
    return tm, copies, x, ys


def gemm_inputs(m, k, gen):
    """fp16 X (m, k) ~ N(0, 1) with 0.1 % of the entries scaled x20."""
    import torch
    x = torch.randn((m, k), generator=gen, device="cuda")
    x[torch.rand((m, k), generator=gen, device="cuda") < 0.001] *= 20.0
    return x.half().contiguous()


def time_gemm(m, n, k, steps, warmup, qtype=None):
    """Q4_K (or `qtype`) GEMM with fp16 X; weight copies rotate over > 512 MB.
    Returns (Timing, rel-L2 of copy 0 against the fp64 oracle product)."""
    import torch
    import oracle as O
    from vibeblade_amd import _lib, ggml
    qtype = ggml.GGML_TYPE_Q4_K if qtype is None else qtype
    gen = torch.Generator(device="cuda").manual_seed(SEED + m)
    copies = make_copies(qtype, n, k, copies_for(n * ggml.row_bytes(qtype, k)), gen)
    xh = gemm_inputs(m, k, gen)
    ys = torch.empty((len(copies), m, n), dtype=torch.float32, device="cuda")
    lib = _lib.load()
    # the workspace vb_gemm_ws needs for this shape (the packed-X kernel's X
    # in fragment order; 0 for the other kernels), allocated once, as a
    # serving loop would
    nb = int(lib.vb_gemm_workspace(m, n, k, qtype, 1, 0))
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")

    def mk(i, c):
        args = (c.ptr(), xh.data_ptr(), 1, ys[i].data_ptr(), m, n, k, c.qtype, 0, ws.data_ptr(), nb)

        def f(s):
            rc = lib.vb_gemm_ws(*args, s)
            if rc != 0:
                _lib.check("vb_gemm_ws", rc)
        return f
    tm = time_launches([mk(i, c) for i, c in enumerate(copies)], steps, warmup)
    w = O.dequantize(copies[0].to_numpy_bytes(), k, copies[0].qtype).astype(np.float64)
    want = xh.float().cpu().numpy().astype(np.float64) @ w.T
    err = O.rel_l2(ys[0].cpu().numpy(), want)
    return tm, err


SPARSE_COPIES = 64  # 64 x 9.9 MB (neuron-major) = 634 MB touched per rotation


def time_sparse(layout, steps, warmup, block=False):
    """TurboSparse FFN, H=4096, I=14336, Q4_K, relu(g)*relu(u); block: with the
    pre-FFN RMSNorm and the residual (vb_sparse_ffn_block).  SPARSE_COPIES
    weight sets, each with its own active set S ~ Bernoulli(0.1), so one
    rotation reads more than 512 MB.  Returns (Timing, mean |S|, mean
    algorithmic bytes per call, rel-L2 of set 0 against the fp64 oracle)."""
    import torch
    import oracle as O
    from vibeblade_amd import _lib, ggml
    from vibeblade_amd.tensor import QTensor, ACT_RELU2
    h, i = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(SEED + 4)
    rng = np.random.default_rng(42)
    sets = []
    for _ in range(SPARSE_COPIES):
        g = QTensor.quantize(torch.randn((i, h), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        u = QTensor.quantize(torch.randn((i, h), generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        dshape = (h, i) if layout == 0 else (i, h)
        d = QTensor.quantize(torch.randn(dshape, generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        s = torch.from_numpy(np.flatnonzero(rng.random(i) < 0.10).astype(np.int32)).cuda()
        sets.append((g, u, d, s))
    x = torch.randn(h, generator=gen, device="cuda")
    ys = torch.empty((SPARSE_COPIES, h), device="cuda")
    lib = _lib.load()
    nbytes = max(lib.vb_sparse_ffn_workspace(h, i, t[3].numel(), layout) for t in sets)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    nw = 1.0 + 0.1 * torch.randn(h, generator=gen, device="cuda")

    def mk(j, g, u, d, s):
        y = ys[j]

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
    tm = time_launches([mk(j, *t) for j, t in enumerate(sets)], steps, warmup)
    n_s = np.array([t[3].numel() for t in sets], dtype=np.float64)
    rb = 2304
    down_b = h * 8064 if layout == 0 else n_s * rb
    ab = float(np.mean(2 * n_s * rb + down_b + 4 * h + 4 * h + 4 * n_s + (8 * h if block else 0)))
    err = None
    if not block:
        g, u, d, s = sets[0]
        dec = lambda q: O.dequantize(q.to_numpy_bytes(), q.k, q.qtype)
        dd = dec(d) if layout == 0 else dec(d).T
        want = O.sparse_ffn(dec(g), dec(u), dd, x.cpu().numpy(), s.cpu().numpy(), O.ACT_DRELU)[0]
        err = O.rel_l2(ys[0].cpu().numpy(), want)
    return tm, float(n_s.mean()), ab, err


def time_ffn_block(down_type, fused, steps, warmup, ncopies=8):
    """One token through the FFN block, hd=4096, inter=14336, Q4_K gate/up,
    down Q4_K or Q6_K (the two Q4_K_M mixes), RMSNorm + SiLU + residual.
    8 weight sets (8 x 99-114 MB per rotation).
    fused: vb_ffn_block (2 launches); else the reference's step order as
    separate launches (rms_norm, gate GEMV, up GEMV, silu, multiply, down
    GEMV, residual add).  Returns (Timing, algorithmic bytes)."""
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
    tm = time_launches([mk(*t) for t in sets], steps, warmup)
    ab = 2 * inter * 2304 + hd * ggml.row_bytes(down_type, inter) + 4 * hd * 4 + 8 * inter
    return tm, ab


def time_sparse_predicted(steps, warmup, predict_only=False):
    """One TurboSparse token step with the active set predicted on the device:
    vb_ema_predict (warm EMA state, k = 10 %), vb_sparse_ffn_block over the
    predicted set through its device count (RMSNorm + relu(g)*relu(u) +
    residual, neuron-major Q4_K down, H=4096, I=14336) and vb_ema_update with
    the used mask.  SPARSE_COPIES weight sets (> 512 MB of active rows per
    rotation).  Returns (Timing, |S| of the last step)."""
    import torch
    from vibeblade_amd import _lib, ggml
    from vibeblade_amd.tensor import QTensor, ACT_RELU2
    h, i = 4096, 14336
    gen = torch.Generator(device="cuda").manual_seed(SEED + 7)
    sets = []
    for _ in range(1 if predict_only else SPARSE_COPIES):
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
    tm = time_launches([mk(*t) for t in sets], steps, warmup)
    return tm, int(count.item())


def time_moe(steps, warmup):
    """8 Q4_K experts (gate/up 14336x4096, down 4096x14336), 16 tokens, top-2
    (793 MB of weights per call when all 8 are hit).  Returns (Timing,
    experts hit, algorithmic bytes, rel-L2 against the fp64 oracle)."""
    import ctypes
    import torch
    import oracle as O
    from vibeblade_amd import _lib, ggml
    from vibeblade_amd.tensor import QTensor, moe_grouped_ffn
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
    tm = time_launches([f], steps, warmup)
    ab = hit * 3 * i * 2304 + t * h * 4 * 2 + t * e_n * 4

    def expert(e):
        dec = lambda qt: O.dequantize(qt.to_numpy_bytes(), qt.k, qt.qtype)
        return dec(gates[e]), dec(ups[e]), dec(downs[e])
    want, _, _ = O.moe_ffn_grouped(expert, x.cpu().numpy(), logits.cpu().numpy(), topk)
    err = O.rel_l2(yo.cpu().numpy(), want)
    return tm, hit, ab, err


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


def check_parity(qtype, n, k, copies, x, ys):
    """Oracle check of the first copy's output (the timed results)."""
    import oracle as O
    y = ys[0].cpu().numpy()
    want = O.gemv(copies[0].to_numpy_bytes(), x.cpu().numpy(), n, k, qtype)
    return O.rel_l2(y, want)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def _trimmed_mean(fn, seconds, min_calls=3):
    """Warmup call, then calls for about `seconds`; 10 % trimmed mean
    (vibeblade/benchmark.py:61-79).  Returns (seconds per call, calls)."""
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_calls:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    ts = np.sort(np.array(times))
    trim = int(len(ts) * 0.1)
    ts = ts[trim:len(ts) - trim] if len(ts) > 2 * trim + 1 else ts
    return float(ts.mean()), len(times)


def _quantized_kn(qtype, K, N, rng, chunk_rows=256):
    """GGUF bytes of a K x N matrix (the reference's orientation: K rows of N)
    of N(0, 0.02) weights, quantized by the oracle in row chunks."""
    import oracle as O
    parts = []
    for r0 in range(0, K, chunk_rows):
        w = rng.standard_normal((min(chunk_rows, K - r0), N), dtype=np.float32) * np.float32(0.02)
        parts.append(O.quantize(w, qtype))
    return np.ascontiguousarray(np.concatenate(parts, axis=0))


def cpu_gemv_sample(qtype, K, N, seconds, rng=None):
    """The oracle's restatement of the reference loop (gemv_dequant,
    cpp/src/dequant.cpp:739-780) on one K x N matrix: seconds per call."""
    import oracle as O
    rng = np.random.default_rng(SEED) if rng is None else rng
    wq = _quantized_kn(qtype, K, N, rng)
    x = rng.standard_normal(K).astype(np.float32)
    scratch = np.empty(N, np.float32)
    sec, calls = _trimmed_mean(lambda: O.gemv_kn(x, wq, K, N, qtype, scratch), seconds)
    return sec, calls


def cpu_baseline(qtype, n, k, seconds):
    """The oracle's C restatement of the reference gemv_dequant (its own
    orientation: k rows of n) on the same bytes, one thread, 10 % trimmed mean."""
    import oracle as O
    sec, calls = cpu_gemv_sample(qtype, k, n, seconds)
    return {
        "value": round(alg_bytes_gemv(qtype, n, k) / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{calls} calls of the oracle's restatement of gemv_dequant (cpp/src/dequant.cpp:739-780) "
                   f"on Q4_K K={k} rows x N={n}, {O.simd_variant()} build (-O3), 10% trimmed mean "
                   f"{sec * 1e3:.2f} ms/call; host {cpu_model()}, nproc={os.cpu_count()}"),
    }


def cpu_table(seconds):
    """One-core CPU time per call for every configuration: the oracle's
    restatements of the reference's CPU paths.  GEMV shapes: the gemv_dequant
    loop; batched M: the reference's per-token loop of it
    (cpp/src/fast_model.cpp:644-669), timed on a sample of tokens and scaled;
    TurboSparse and MoE: the reference's numpy steps over fp32 weights
    (vibeblade/sparse.py:199-283, vibeblade/moe_executor.py:331-344) with
    BLAS held to one thread.  Yields one dict per configuration."""
    from vibeblade_amd import ggml
    from threadpoolctl import threadpool_limits
    rng = np.random.default_rng(SEED + 11)
    per = max(1.0, seconds)
    for name, qt, n, k in (("1: Q8_0 GEMV 4096x4096", ggml.GGML_TYPE_Q8_0, 4096, 4096),
                           ("2: Q4_K GEMV 14336x4096 (gate/up)", ggml.GGML_TYPE_Q4_K, 14336, 4096),
                           ("2: Q4_K GEMV 4096x14336 (down)", ggml.GGML_TYPE_Q4_K, 4096, 14336),
                           ("2: Q6_K GEMV 128256x4096 (lm_head)", ggml.GGML_TYPE_Q6_K, 128256, 4096)):
        sec, calls = cpu_gemv_sample(qt, k, n, per, rng)
        yield {"config": name, "cpu_us_per_call": round(sec * 1e6, 1), "calls": calls,
               "GB/s": round(alg_bytes_gemv(qt, n, k) / sec / 1e9, 3)}
    sec1, calls = cpu_gemv_sample(ggml.GGML_TYPE_Q4_K, 4096, 14336, per, rng)
    for m in (8, 512):
        yield {"config": f"3: Q4_K GEMM M={m} 14336x4096", "cpu_us_per_call": round(m * sec1 * 1e6, 1),
               "sample": f"per-token loop: {m} x the gate/up GEMV time ({calls} calls timed)"}
    h, i = 4096, 14336
    with threadpool_limits(limits=1):
        w002 = np.float32(0.02)
        gate = rng.standard_normal((i, h), dtype=np.float32) * w002
        up = rng.standard_normal((i, h), dtype=np.float32) * w002
        down = rng.standard_normal((h, i), dtype=np.float32) * w002
        x = rng.standard_normal((1, h), dtype=np.float32)
        kk = max(1, int(i * 0.1))

        def sparse_step():
            g = x @ gate.T
            top = np.argpartition(g[0], -kk)[-kk:]
            act = np.sort(top)
            ua = x @ up[act].T
            ga = g[:, act]
            hid = ga * (1.0 / (1.0 + np.exp(-ga))) * ua
            return hid @ down.T[act]
        sec, calls = _trimmed_mean(sparse_step, per)
        yield {"config": "4: TurboSparse FFN H=4096 I=14336 (10% active)", "cpu_us_per_call": round(sec * 1e6, 1),
               "calls": calls, "sample": "reference sparse_ffn_silu steps in numpy fp32 (dense gate, top-k, "
                                         "gathered up and down), 1 BLAS thread"}
        xe = rng.standard_normal((4, h), dtype=np.float32)
        gt, ut, dt = gate.T, up.T, down.T  # moe convention: no transpose copies

        def expert_step():
            go = xe @ gt
            return (go * (1.0 / (1.0 + np.exp(-go))) * (xe @ ut)) @ dt
        sec, calls = _trimmed_mean(expert_step, per)
        yield {"config": "5: MoE 8 experts, 16 tokens top-2", "cpu_us_per_call": round(8 * sec * 1e6, 1),
               "calls": calls, "sample": "8 x one expert's _compute_single_expert_cpu on its 4 tokens "
                                         "(16 x 2 / 8), numpy fp32, 1 BLAS thread"}
        del gate, up, down


def pmc_pass(workload="gemv"):
    """Launches for counter collection: no graph (per-dispatch counters), no
    timing.  The GEMVs rotate over 16 weight copies as in the timed run; the
    GEMMs (fp16 X with 0.1% outliers x20, as timed) likewise."""
    import torch
    from vibeblade_amd import _lib, ggml
    _lib.init(0)
    qtype, n, k = ggml.GGML_TYPE_Q4_K, 14336, 4096
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    if workload in ("gemv", "lmhead", "down"):
        if workload == "lmhead":  # Q6_K output projection 128256 x 4096, 2 copies (862 MB)
            qtype, n, ncop = ggml.GGML_TYPE_Q6_K, 128256, 2
        elif workload == "down":  # Q4_K 4096 x 14336
            n, k, ncop = 4096, 14336, NCOPIES
        else:
            ncop = NCOPIES
        gen = torch.Generator(device="cuda").manual_seed(SEED)
        copies = make_copies(qtype, n, k, ncop, gen)
        x = torch.randn(k, generator=gen, device="cuda")
        y = torch.empty(n, device="cuda")
        ndisp = 8 if workload == "lmhead" else 32
        for i in range(ndisp):
            c = copies[i % ncop]
            _lib.check("vb_gemv", lib.vb_gemv(c.ptr(), x.data_ptr(), y.data_ptr(), n, k, qtype, st))
        what = f"{ndisp} GEMV dispatches ({workload})"
    elif workload == "sparse":
        from vibeblade_amd.tensor import QTensor, ACT_RELU2
        h, i = 4096, 14336
        gen = torch.Generator(device="cuda").manual_seed(SEED + 4)
        rng = np.random.default_rng(42)
        q = lambda shape: QTensor.quantize(torch.randn(shape, generator=gen, device="cuda") * 0.02, qtype)
        copies = [(q((i, h)), q((i, h)), q((i, h)),
                   torch.from_numpy(np.flatnonzero(rng.random(i) < 0.10).astype(np.int32)).cuda())
                  for _ in range(NCOPIES)]
        x = torch.randn(h, generator=gen, device="cuda")
        y = torch.empty(h, device="cuda")
        nb = max(lib.vb_sparse_ffn_workspace(h, i, c[3].numel(), 1) for c in copies)
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        for j in range(16):
            g, u, d, s = copies[j % NCOPIES]
            _lib.check("vb_sparse_ffn", lib.vb_sparse_ffn(g.ptr(), u.ptr(), d.ptr(), 1, x.data_ptr(), s.data_ptr(),
                                                          s.numel(), ACT_RELU2, y.data_ptr(), h, i, qtype,
                                                          ws.data_ptr(), ws.numel(), st))
        what = "16 neuron-major sparse FFN calls"
    elif workload == "moe":
        import ctypes
        from vibeblade_amd.tensor import QTensor
        e_n, h, i, t, topk = 8, 4096, 14336, 16, 2
        gen = torch.Generator(device="cuda").manual_seed(SEED + 5)
        q = lambda shape: QTensor.quantize(torch.randn(shape, generator=gen, device="cuda") * 0.02, qtype)
        copies = [q((i, h)) for _ in range(2 * e_n)] + [q((h, i)) for _ in range(e_n)]
        arr = ctypes.c_void_p * e_n
        pg, pu, pd = (arr(*[c.ptr() for c in copies[a * e_n:(a + 1) * e_n]]) for a in range(3))
        x = torch.randn((t, h), generator=gen, device="cuda")
        logits = torch.randn((t, e_n), generator=gen, device="cuda")
        ws = torch.empty(lib.vb_moe_workspace(t, topk, h, i), dtype=torch.uint8, device="cuda")
        y = torch.empty((t, h), device="cuda")
        vp = ctypes.c_void_p
        for _ in range(8):
            _lib.check("vb_moe_grouped_ffn", lib.vb_moe_grouped_ffn(
                ctypes.cast(pg, vp), ctypes.cast(pu, vp), ctypes.cast(pd, vp), e_n, x.data_ptr(), t,
                logits.data_ptr(), topk, y.data_ptr(), None, None, h, i, qtype, ws.data_ptr(), ws.numel(), st))
        what = "8 MoE calls"
    else:
        m = 8 if workload == "gemm8" else 512
        if workload in ("down512", "down512q6"):
            n, k = 4096, 14336
        if workload == "down512q6":
            qtype = ggml.GGML_TYPE_Q6_K
        gen = torch.Generator(device="cuda").manual_seed(SEED + m)
        copies = make_copies(qtype, n, k, NCOPIES, gen)
        xh = gemm_inputs(m, k, gen)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        nb = int(lib.vb_gemm_workspace(m, n, k, qtype, 1, 0))
        ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")
        for i in range(16):
            c = copies[i % NCOPIES]
            _lib.check("vb_gemm_ws", lib.vb_gemm_ws(c.ptr(), xh.data_ptr(), 1, y.data_ptr(), m, n, k, qtype, 0,
                                                    ws.data_ptr(), nb, st))
        what = f"16 GEMM dispatches at M={m}, {n}x{k}"
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
    """Markdown table of per-dispatch mean counter values of the library's
    kernels (namespace vb) over rocprofv3 counter_collection.csv files, one
    row per counter and one column per kernel, plus derived rows:
    MFMA FLOPs = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 (the counter counts units
    of 512 FLOPs); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8
    XCDs x 256 CUs x 4 SIMDs); wait / issue shares of the wave lifetime
    (SQ_WAIT_ANY, SQ_ACTIVE_INST_ANY over SQ_WAVE_CYCLES); lanes per VALU
    instruction (SQ_THREAD_CYCLES_VALU / SQ_ACTIVE_INST_VALU); and FETCH_SIZE /
    WRITE_SIZE scaled by the calibration copy (CALIB_BYTES read and written)
    when it is in the same file."""
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

    def demangle(name):
        # the library's kernels in an anonymous namespace: _ZN2vb12_GLOBAL__N_1<len><name>...
        # (some rocprofv3 builds leave names with _Float16 parameters mangled)
        import re
        m = re.match(r"_ZN2vb12_GLOBAL__N_1(\d+)", name)
        if not m:
            return name
        n = int(m.group(1))
        base = name[m.end():m.end() + n]
        rest = name[m.end() + n:]
        tmpl = re.match(r"IL[ij](\d+)E", rest)
        return f"vb::{base}" + (f"<{tmpl.group(1)}>" if tmpl else "")
    rows = {demangle(k): d for k, d in rows.items()}
    kern = sorted(k for k in rows if "vb::" in k)
    short = [k.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:70] for k in kern]
    names = sorted({c for k in kern for c in rows[k]})
    print("| Counter | " + " | ".join(f"`{s}`" for s in short) + " |")
    print("|---" * (len(kern) + 1) + "|")
    print("| dispatches | " + " | ".join(str(max(n for _, n in rows[k].values())) for k in kern) + " |")
    for c in names:
        print(f"| {c} | " + " | ".join(f"{rows[k][c][0]:.4g}" if c in rows[k] else "" for k in kern) + " |")

    def derived(label, fn):
        vals = []
        for k in kern:
            try:
                vals.append(fn(rows[k]))
            except (KeyError, ZeroDivisionError):
                vals.append("")
        if any(vals):
            print(f"| {label} | " + " | ".join(vals) + " |")
    v = lambda d, c: d[c][0]
    derived("MFMA f16 GFLOP", lambda d: f"{v(d, 'SQ_INSTS_VALU_MFMA_MOPS_F16') * 512 / 1e9:.3f}")
    derived("MFMA busy", lambda d: "{:.1%}".format(
        v(d, "SQ_VALU_MFMA_BUSY_CYCLES") / (v(d, "GRBM_GUI_ACTIVE") / 8 * 256 * 4)))
    derived("waiting / wave lifetime", lambda d: "{:.1%}".format(v(d, "SQ_WAIT_ANY") / v(d, "SQ_WAVE_CYCLES")))
    derived("issuing / wave lifetime", lambda d: "{:.1%}".format(
        v(d, "SQ_ACTIVE_INST_ANY") / v(d, "SQ_WAVE_CYCLES")))
    derived("lanes per VALU instruction", lambda d: "{:.1f}".format(
        v(d, "SQ_THREAD_CYCLES_VALU") / v(d, "SQ_ACTIVE_INST_VALU")))
    derived("LDS bank conflict / LDS active", lambda d: "{:.1%}".format(
        v(d, "SQ_LDS_BANK_CONFLICT") / v(d, "SQ_ACTIVE_INST_LDS")))
    for c, lab in (("FETCH_SIZE", "read MB (copy-scaled)"), ("WRITE_SIZE", "written MB (copy-scaled)")):
        if calib.get(c):
            derived(lab, lambda d, c=c: f"{v(d, c) * CALIB_BYTES / calib[c] / 1e6:.2f}")


def summarize_pmc(fetch_csv, write_csv):
    """Traffic per GEMV launch = FETCH_SIZE x read factor + WRITE_SIZE x write
    factor, the factors being what the calibration copy (CALIB_BYTES read and
    written) shows for the same counters (KiB per dispatch)."""
    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        means = _counter_means(path, counter)
        gemv = [(v, c, name) for name, (v, c) in means.items() if any(k in name for k in GEMV_KERNELS)]
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


def run_mfma_ceiling(steps, warmup):
    """fp16 GEMM on the vendor library (torch.matmul -> hipBLASLt) with fp16
    weights already in HBM (nothing to decode; 3.5x the Q4_K bytes), rotating
    over > 512 MB of weight copies like the other lines, at the Q4_K GEMM
    shapes: the MFMA rate this chip sustains on them with random fp16 data
    (and with all-zero X, which draws less power), beside time_gemm's Q4_K
    numbers for the same shapes."""
    import torch
    shapes = ((512, 14336, 4096), (1024, 14336, 4096), (2048, 14336, 4096), (4096, 14336, 4096),
              (512, 4096, 14336))
    gen = torch.Generator(device="cuda").manual_seed(SEED + 7)
    for m, n, k in shapes:
        ncop = copies_for(n * k * 2, 2)
        ws = [torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float16) * 0.02 for _ in range(ncop)]
        x = torch.randn((m, k), generator=gen, device="cuda", dtype=torch.float16)
        outs = [torch.empty((m, n), device="cuda", dtype=torch.float16) for _ in range(ncop)]
        line = {"kernel": "torch.matmul fp16 (hipBLASLt)", "m": m, "n": n, "k": k, "weight_copies": ncop}
        for label, xx in (("random", x), ("zero", torch.zeros_like(x))):
            for i in range(warmup * ncop):
                torch.matmul(xx, ws[i % ncop].t(), out=outs[i % ncop])
            torch.cuda.synchronize()
            it = steps * ncop
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(it):
                torch.matmul(xx, ws[i % ncop].t(), out=outs[i % ncop])
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / it
            line[f"us_{label}_x"] = round(us, 2)
            line[f"frac_{label}_x"] = round(2 * m * n * k / (us * 1e-6) / 2.5e15, 4)
        del ws, outs
        torch.cuda.empty_cache()
        tm, err = time_gemm(m, n, k, steps, warmup)
        line["q4k_us"] = tm.us()
        line["q4k_frac"] = round(2 * m * n * k / (tm.ms * 1e-3) / 2.5e15, 4)
        line["q4k_rel_l2"] = float(f"{err:.3g}")
        torch.cuda.empty_cache()
        print(json.dumps(line), file=sys.stderr, flush=True)


def run_floor(steps, warmup):
    """The headline GEMV (14336 x 4096 Q4_K) and what one launch over the same
    33 MB costs without the GEMV's arithmetic, all under the bench protocol
    (16 rotating weight copies, graphs of 128 launches, HIP events on the
    replay stream):
      * vb_stream_read: the GEMV's grid (256 workgroups of 8 waves, 7 rows
        per wave) and row-contiguous non-temporal loads, nothing computed;
        into registers (ring 3 is the register-ring GEMV's schedule, ring 0
        issues a wave's 7 rows at once) or into LDS by DMA (DMA ring 2 is
        the default GEMV's schedule);
      * torch.sum over the copy viewed as int32 (a vendor reduction kernel);
      * torch copy_ of the copy into a second buffer (reads and writes 33 MB);
      * vb_stream_read of one row (one workgroup): the launch cost alone."""
    import torch
    from vibeblade_amd import _lib, ggml
    qtype, n, k = ggml.GGML_TYPE_Q4_K, 14336, 4096
    rb = ggml.row_bytes(qtype, k)
    ab = alg_bytes_gemv(qtype, n, k)
    tm, copies, x, ys = time_gemv(qtype, n, k, steps, warmup, NCOPIES)
    lib = _lib.load()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    rows = [("GEMV (vb_gemv, the headline kernel)", tm)]

    def probe(ring, nrows):
        def mk(c):
            def f(s):
                rc = lib.vb_stream_read(c.ptr(), nrows, rb, ring, sink.data_ptr(), s)
                if rc != 0:
                    _lib.check("vb_stream_read", rc)
            return f
        return time_launches([mk(c) for c in copies], steps, warmup)

    for ring in (-2, -1, -3, 3, 1, 2, 4, 6, 0):
        what = ("all 7 rows of a wave at once" if ring == 0 else
                f"rows into LDS by DMA, ring {-ring}" if ring < 0 else f"rows into registers, ring {ring}")
        rows.append((f"read-only probe, GEMV shape and loads, {what}", probe(ring, n)))
    views = [c.data.reshape(-1).view(torch.int32) for c in copies]
    out = torch.empty((), dtype=torch.int64, device="cuda")

    def red(v):
        def f(s):
            torch.sum(v, dim=0, dtype=torch.int64, out=out)
        return f
    rows.append(("torch.sum over the copy (int32 view)", time_launches([red(v) for v in views], steps, warmup)))
    dst = torch.empty_like(views[0])

    def cp(v):
        def f(s):
            dst.copy_(v)
        return f
    rows.append(("torch copy_ of the copy (reads + writes 33 MB)", time_launches([cp(v) for v in views], steps,
                                                                                   warmup)))
    rows.append(("one-workgroup launch (vb_stream_read of 1 row)", probe(3, 1)))
    for name, t in rows:
        gbs = ab / (t.ms * 1e-3) / 1e9
        emit({"floor": name, "us_per_launch": t.us(), "GB/s_of_33.1MB": round(gbs, 1),
              "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "launches": t.launches})
    return rows


def emit(d):
    print(json.dumps(d), file=sys.stderr, flush=True)


def run_extra(which, args):
    """The other configurations, one JSON line each on stderr."""
    import torch
    from vibeblade_amd import ggml

    def frac(b, tm):
        gbs = b / (tm.ms * 1e-3) / 1e9
        return round(gbs, 1), round(gbs / HBM_PEAK_GBS, 4)

    if "gemv" in which:
        for name, t, nn, kk in (("1: Q8_0 GEMV 4096x4096", ggml.GGML_TYPE_Q8_0, 4096, 4096),
                                ("2: Q4_K GEMV 4096x14336 (down)", ggml.GGML_TYPE_Q4_K, 4096, 14336),
                                ("2: Q6_K GEMV 128256x4096 (lm_head)", ggml.GGML_TYPE_Q6_K, 128256, 4096)):
            tm, cps, xx, yy = time_gemv(t, nn, kk, 20, 3)
            e2 = check_parity(t, nn, kk, cps, xx, yy)
            b2 = alg_bytes_gemv(t, nn, kk)
            gbs, fr = frac(b2, tm)
            emit({"workload": name, "us_per_call": tm.us(), "mean_us": round(tm.mean_ms * 1e3, 3),
                  "launches": tm.launches, "weight_copies": len(cps), "GB/s": gbs, "frac_hbm": fr, "rel_l2": e2,
                  "dtype": DTYPE_GEMV})
            del cps, yy
            torch.cuda.empty_cache()
    if "sparse" in which:
        for layout, block in ((1, False), (0, False), (1, True), (0, True)):
            tm, n_s, b4, err = time_sparse(layout, 20, 3, block=block)
            what = "block (RMSNorm + FFN + residual)" if block else "FFN"
            gbs, fr = frac(b4, tm)
            emit({"workload": f"4: TurboSparse {what} H=4096 I=14336 mean |S|={n_s:.0f} down_layout={layout}",
                  "us_per_call": tm.us(), "launches": tm.launches, "weight_sets": SPARSE_COPIES,
                  "alg_bytes": round(b4), "GB/s": gbs, "frac_hbm": fr, "rel_l2": err})
            torch.cuda.empty_cache()
    if "moe" in which:
        tm, hit, b5, err = time_moe(5, 1)
        gbs, fr = frac(b5, tm)
        emit({"workload": f"5: MoE 8x Q4_K experts, 16 tokens top-2 ({hit} experts hit)",
              "us_per_call": tm.us(), "launches": tm.launches, "alg_bytes": b5, "GB/s": gbs, "frac_hbm": fr,
              "rel_l2": err, "dtype": "x and the hidden rows rounded to fp16, fp16 MFMA, fp32 accumulate"})
        torch.cuda.empty_cache()
    if "predict" in which:
        for only in (True, False):
            tm, n_s8 = time_sparse_predicted(10, 2, predict_only=only)
            what = ("EMA predict + compaction alone (I=14336, k=1433)" if only else
                    "TurboSparse token step on the device: EMA predict + sparse block over the device count "
                    "+ EMA update, H=4096 I=14336")
            emit({"workload": what, "us_per_call": tm.us(), "launches": tm.launches, "active": n_s8})
            torch.cuda.empty_cache()
    if "ffn" in which:
        for dt_name, dt in (("Q4_K", ggml.GGML_TYPE_Q4_K), ("Q6_K", ggml.GGML_TYPE_Q6_K)):
            for fused in (True, False):
                tm, b7 = time_ffn_block(dt, fused, 40, 3)
                gbs, fr = frac(b7, tm)
                emit({"workload": f"FFN block hd=4096 inter=14336 Q4_K gate/up, {dt_name} down, RMSNorm+SiLU+"
                                  f"residual, {'fused (2 launches)' if fused else 'unfused (7 launches)'}",
                      "us_per_call": tm.us(), "launches": tm.launches, "alg_bytes": b7, "GB/s": gbs, "frac_hbm": fr})
                torch.cuda.empty_cache()
    if "gguf" in which:
        gbs6, b6, gpath, t_open = time_gguf_ingest()
        os.remove(gpath)
        emit({"workload": "GGUF ingestion: open + upload 32 Q4_K 14336x4096 tensors (page cache)",
              "bytes": b6, "GB/s": round(gbs6, 2), "open_ms": round(t_open * 1e3, 3)})
    ms_list = []
    if "gemm" in which:
        ms_list += [8, 512]
    if "msweep" in which:
        ms_list += [m for m in (1, 4, 16, 17, 32, 64, 100, 128, 256, 1024) if m not in ms_list]
    for m in ms_list:
        tm, e3 = time_gemm(m, 14336, 4096, 20, 2)
        flops = 2.0 * m * 14336 * 4096
        b3 = 14336 * 2304 + 2 * m * 4096 + 4 * m * 14336
        tfs = flops / (tm.ms * 1e-3) / 1e12
        gbs, fr = frac(b3, tm)
        emit({"workload": f"3: Q4_K GEMM M={m} N=14336 K=4096 fp16 X", "us_per_call": tm.us(),
              "launches": tm.launches, "TFLOP/s": round(tfs, 2), "frac_mfma_fp16": round(tfs / MFMA_FP16_PEAK_TFS, 4),
              "GB/s": gbs, "frac_hbm": fr, "rel_l2": e3, "dtype": DTYPE_GEMM if m > 1 else DTYPE_GEMV})
        torch.cuda.empty_cache()
    if "gemm" in which:
        # the other weight types at the gate/up shape: Q6_K / Q8_0 (quantized
        # on the device), Q5_K / Q4_0 (random blocks)
        for qtype, name in ((ggml.GGML_TYPE_Q6_K, "Q6_K"), (ggml.GGML_TYPE_Q8_0, "Q8_0"),
                            (ggml.GGML_TYPE_Q5_K, "Q5_K"), (ggml.GGML_TYPE_Q4_0, "Q4_0")):
            n, k = 14336, 4096
            wb = n * ggml.row_bytes(qtype, k)
            for m in (8, 512):
                tm, e3 = time_gemm(m, n, k, 20, 2, qtype=qtype)
                tfs = 2.0 * m * n * k / (tm.ms * 1e-3) / 1e12
                gbs, fr = frac(wb + 2 * m * k + 4 * m * n, tm)
                emit({"workload": f"3: {name} GEMM M={m} N={n} K={k} fp16 X", "us_per_call": tm.us(),
                      "launches": tm.launches, "TFLOP/s": round(tfs, 2),
                      "frac_mfma_fp16": round(tfs / MFMA_FP16_PEAK_TFS, 4), "GB/s": gbs, "frac_hbm": fr,
                      "rel_l2": e3, "dtype": DTYPE_GEMM})
                torch.cuda.empty_cache()
        # the down projection: Q6_K in a Q4_K_M file, Q4_K in a Q4_K_S file,
        # Q8_0 in a Q8_0 file
        for qtype, name in ((ggml.GGML_TYPE_Q6_K, "Q6_K"), (ggml.GGML_TYPE_Q4_K, "Q4_K"),
                            (ggml.GGML_TYPE_Q8_0, "Q8_0")):
            n, k = 4096, 14336
            wb = n * ggml.row_bytes(qtype, k)
            for m in (8, 512):
                tm, e3 = time_gemm(m, n, k, 20, 2, qtype=qtype)
                tfs = 2.0 * m * n * k / (tm.ms * 1e-3) / 1e12
                gbs, fr = frac(wb + 2 * m * k + 4 * m * n, tm)
                emit({"workload": f"3: {name} GEMM M={m} N={n} K={k} fp16 X", "us_per_call": tm.us(),
                      "launches": tm.launches, "TFLOP/s": round(tfs, 2),
                      "frac_mfma_fp16": round(tfs / MFMA_FP16_PEAK_TFS, 4), "GB/s": gbs, "frac_hbm": fr,
                      "rel_l2": e3, "dtype": DTYPE_GEMM})
                torch.cuda.empty_cache()
    if "cpu" in which and not args.no_cpu_baseline:
        for row in cpu_table(min(args.cpu_seconds, 3.0)):
            row["cores"] = 1
            row["host"] = cpu_model()
            emit(row)


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
    if args.floor:
        import torch
        from vibeblade_amd import _lib
        _lib.init(0)
        run_floor(args.steps, args.warmup)
        return
    if args.mfma_ceiling:
        import torch
        from vibeblade_amd import _lib
        torch.zeros(1, device="cuda")
        _lib.init(0)
        run_mfma_ceiling(args.steps, args.warmup)
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
    tm, copies, x, ys = time_gemv(qtype, n, k, args.steps, args.warmup, NCOPIES)
    err = check_parity(qtype, n, k, copies, x, ys)
    ab = alg_bytes_gemv(qtype, n, k)
    gbs = ab / (tm.ms * 1e-3) / 1e9
    print(f"[bench] {tm.us():.2f} us per launch (median over {tm.steps} steps of {tm.per_step}; mean "
          f"{tm.mean_ms * 1e3:.2f}), {gbs:.0f} GB/s, rel-L2 vs oracle {err:.2e}", file=sys.stderr, flush=True)
    if err > 1e-3:
        print("[bench] PARITY FAILURE", file=sys.stderr)
        sys.exit(3)
    del copies, ys
    torch.cuda.empty_cache()

    if args.extra:
        which = {w.strip() for w in args.extra.split(",") if w.strip()}
        bad = which - set(EXTRA_ALL)
        if bad:
            print(f"unknown --extra workloads: {sorted(bad)}", file=sys.stderr)
            sys.exit(2)
        run_extra(which, args)

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline (oracle restatement of gemv_dequant, 1 thread)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(qtype, n, k, args.cpu_seconds)

    line = {
        "metric": "Q4_K GEMV eff. HBM GB/s (14336x4096, M=1) + % of MI355X peak",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": tm.steps,
        "warmup": args.warmup,
        "ms_per_step": round(tm.step_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_GEMV,
        "data": f"synthetic: W ~ N(0,0.02) quantized to GGUF Q4_K on device ({NCOPIES} rotating copies, "
                f"{NCOPIES * n * 2304 / 1e6:.0f} MB), x ~ N(0,1)",
        "config": {"workload": "Q4_K GEMV M=1, N=14336 rows x K=4096 (Llama-3-8B FFN gate/up)",
                   "n": n, "k": k, "m": 1, "weight_copies": NCOPIES, "hip_graph": tm.graph,
                   "step": f"{tm.per_step // NCOPIES} passes over the {NCOPIES} weight copies ({tm.per_step} GEMV launches, "
                           "one HIP graph replay)",
                   "launches_timed": tm.launches, "us_per_launch_median": tm.us(),
                   "us_per_launch_mean": round(tm.mean_ms * 1e3, 3),
                   "rel_l2_vs_oracle": float(f"{err:.3e}")},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic(),
                     "alg_bytes_per_launch": ab, "us_per_launch": tm.us()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
