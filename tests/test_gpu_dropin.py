"""GPU tests of the drop-in surface (vibeblade_amd.sparse / moe /
moe_executor / gpu), mirroring the reference's own tests
(tests/test_sparse.py, test_moe.py, test_moe_executor.py) plus parity
against fp64 restatements and the quantized-weight (QTensor) paths.  fp32
weights run as exact F32 tensors; bounds are fp32-accumulation tolerances
(the MoE experts run on fp16 MFMA: 5e-3)."""
import numpy as np
import pytest
import torch

import oracle as O
from vibeblade_amd import ggml
from vibeblade_amd.gpu import GPUBackend, HipBackend, available_backends
from vibeblade_amd.moe import ExpertRouter, MoEExpertSet, moe_ffn_silu, _dense_ffn
from vibeblade_amd.moe_executor import HotColdExecutor
from vibeblade_amd.moe_profiler import HotColdMap
from vibeblade_amd.sparse import SparsePredictor, sparse_ffn_silu, sparse_matmul, silu
from vibeblade_amd.tensor import QTensor

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield


def silu64(v):
    return v / (1.0 + np.exp(-v))


def dense_ffn64(x, g, u, d):
    """transformer.ffn_silu semantics (vibeblade/transformer.py:177-208), fp64."""
    x = x.astype(np.float64)
    return (silu64(x @ g.T.astype(np.float64)) * (x @ u.T.astype(np.float64))) @ d.T.astype(np.float64)


def ffn_weights(seed, hidden, inter, scale=1.0):
    rng = np.random.RandomState(seed)
    return (rng.randn(1, hidden).astype(np.float32), (rng.randn(inter, hidden) * scale).astype(np.float32),
            (rng.randn(inter, hidden) * scale).astype(np.float32), (rng.randn(hidden, inter) * scale).astype(np.float32))


class TestSparseFFN:
    def test_shapes_and_stats(self):
        rng = np.random.RandomState(42)
        x = rng.randn(2, 64).astype(np.float32)
        g, u = rng.randn(128, 64).astype(np.float32), rng.randn(128, 64).astype(np.float32)
        d = rng.randn(64, 128).astype(np.float32)
        out, st = sparse_ffn_silu(x, g, u, d, sparse_ratio=0.1)
        assert out.shape == (2, 64)
        assert set(st) == {"active_neurons", "total_neurons", "sparsity_ratio"}

    def test_ratio_controls_active_count(self):
        x, g, u, d = ffn_weights(42, 64, 256)
        _, s10 = sparse_ffn_silu(x, g, u, d, 0.1)
        _, s50 = sparse_ffn_silu(x, g, u, d, 0.5)
        _, s100 = sparse_ffn_silu(x, g, u, d, 1.0)
        assert s10["sparsity_ratio"] > s50["sparsity_ratio"]
        assert s100["sparsity_ratio"] == 0.0 and s100["active_neurons"] == 256
        x1, g1, u1, d1 = ffn_weights(7, 32, 64)
        out, st = sparse_ffn_silu(x1, g1, u1, d1, 0.25)
        assert out.shape == (1, 32) and st["active_neurons"] == 16

    def test_full_ratio_equals_dense(self):
        x, g, u, d = ffn_weights(99, 16, 32)
        out, _ = sparse_ffn_silu(x, g, u, d, 1.0)
        assert np.allclose(out, dense_ffn64(x, g, u, d), rtol=1e-4, atol=1e-4)

    def test_matches_masked_dense(self):
        """Output = dense FFN with the hidden vector masked to the top-k of the gate."""
        x, g, u, d = ffn_weights(3, 256, 1024, 0.05)
        out, st = sparse_ffn_silu(x, g, u, d, 0.1)
        gate = x.astype(np.float64) @ g.T.astype(np.float64)
        k = st["active_neurons"]
        assert k == 102
        active = np.sort(np.argsort(-gate[0], kind="stable")[:k])
        want = O.sparse_ffn(g, u, d, x, active, O.ACT_SILU)
        assert O.rel_l2(out, want) <= 1e-4

    def test_quantized_weights(self):
        h, i = 4096, 14336
        gen = torch.Generator(device="cuda").manual_seed(3)
        q = lambda shape: QTensor.quantize(torch.randn(shape, generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        g, u, d = q((i, h)), q((i, h)), q((h, i))
        x = np.random.default_rng(1).standard_normal((1, h)).astype(np.float32)
        out, st = sparse_ffn_silu(x, g, u, d, 0.1)
        gd, ud, dd = (O.dequantize(t.to_numpy_bytes(), t.k, t.qtype) for t in (g, u, d))
        gate = gd.astype(np.float64) @ x[0].astype(np.float64)
        active = np.sort(np.argsort(-gate, kind="stable")[:st["active_neurons"]])
        want = O.sparse_ffn(gd, ud, dd, x, active, O.ACT_SILU)
        assert O.rel_l2(out, want) <= 1e-3

    def test_sparse_matmul(self):
        rng = np.random.RandomState(123)
        a, w = rng.randn(4, 8), rng.randn(8, 6)
        mask = np.array([True, False] * 4)
        got = sparse_matmul(a, w, mask)
        assert np.allclose(got, (a * mask[None, :]) @ w, rtol=1e-5, atol=1e-5)
        assert np.allclose(sparse_matmul(a, w, np.ones(8, bool)), a @ w, rtol=1e-5, atol=1e-5)

    def test_predictor_and_silu(self):
        pred = SparsePredictor(n_layers=2, intermediate_dim=64, sparse_ratio=0.1)
        rng = np.random.RandomState(42)
        x, gw = rng.randn(1, 32).astype(np.float32), rng.randn(64, 32).astype(np.float32)
        m = pred.predict(0, x, gw)
        assert m.shape == (64,) and m.sum() == 6
        assert set(np.flatnonzero(m)) == set(np.argsort(-(x @ gw.T)[0])[:6])
        for _ in range(3):
            pred.calibrate_update(0, x, gw)
        pred.calibrate_finish(0.3)
        assert pred.is_calibrated and pred.predict(0, x, gw).sum() >= 6
        v = rng.randn(100).astype(np.float32)
        assert np.allclose(silu(v), v / (1 + np.exp(-v)), rtol=1e-5, atol=1e-6)


def make_router(shared_dim=16, num_experts=4, topk=2):
    w = np.random.RandomState(42).randn(shared_dim, num_experts).astype(np.float32)
    w[:, 0] += 3.0
    w[:, 1] += 1.0
    return ExpertRouter(w, topk=topk)


def make_expert_set(num_experts=4, shared_dim=16, expert_dim=32):
    rng = np.random.RandomState(123)
    g = rng.randn(num_experts, expert_dim, shared_dim).astype(np.float32) * 0.1
    u = rng.randn(num_experts, expert_dim, shared_dim).astype(np.float32) * 0.1
    d = rng.randn(num_experts, shared_dim, expert_dim).astype(np.float32) * 0.1
    return MoEExpertSet(g, u, d)


def make_executor(hot_ids=(0,), num_experts=4, topk=2, shared=False):
    cold = [i for i in range(num_experts) if i not in hot_ids]
    hmap = HotColdMap(hot_experts={0: list(hot_ids)}, cold_experts={0: cold}, num_layers=1, num_experts=num_experts)
    sh = {}
    if shared:
        rng = np.random.RandomState(99)
        sh[0] = (rng.randn(16, 32).astype(np.float32) * 0.1, rng.randn(16, 32).astype(np.float32) * 0.1,
                 rng.randn(32, 16).astype(np.float32) * 0.1)
    return HotColdExecutor(hmap, {0: make_router(16, num_experts, topk)}, {0: make_expert_set(num_experts)},
                           shared_experts=sh, gpu_backend=HipBackend())


def moe_ref(x2, router, es, shared=None):
    """Per-token restatement (vibeblade/moe.py:457-482) in fp64."""
    logits = x2.astype(np.float64) @ router.weight.astype(np.float64)
    idx, w = O.route_top_k(logits, router.topk)
    y = np.zeros((x2.shape[0], es.shared_dim))
    for t in range(x2.shape[0]):
        for k in range(router.topk):
            e = idx[t, k]
            gw, uw, dw = es.get_expert(e)
            y[t] += w[t, k] * dense_ffn64(x2[t:t + 1], gw.T, uw.T, dw.T)[0]
    if shared is not None:
        y += dense_ffn64(x2, shared[0].T, shared[1].T, shared[2].T)
    return y, idx, w


class TestExecutor:
    def test_shapes_stats_accounting(self):
        ex = make_executor(hot_ids=[0, 1, 2, 3])
        x = np.random.randn(16).astype(np.float32)
        out, st = ex.dispatch(0, x)
        assert out.shape == (16,) and np.all(np.isfinite(out))
        for key in ["gpu_hits", "cpu_falls", "hit_rate", "gpu_latency_ms", "cpu_latency_ms", "sync_latency_ms",
                    "expert_indices", "expert_weights"]:
            assert key in st
        assert st["gpu_hits"] == 2 and st["cpu_falls"] == 0
        out2, _ = ex.dispatch(0, x[None, :])
        assert out2.shape == (1, 16)
        for _ in range(3):
            ex.dispatch(0, x)
        assert ex.stats.gpu_hits == 10
        ex.reset_stats()
        assert ex.stats.gpu_hits == 0 and ex.stats.gpu_latency_ms == 0.0
        cold = make_executor(hot_ids=[])
        _, st = cold.dispatch(0, x)
        assert st["gpu_hits"] == 0 and st["cpu_falls"] == 2
        assert 0.0 <= make_executor(hot_ids=[0]).dispatch(0, x)[1]["hit_rate"] <= 1.0

    def test_matches_reference_math(self):
        ex = make_executor()
        x = np.random.RandomState(5).randn(16).astype(np.float32)
        out, st = ex.dispatch(0, x)
        want, idx, w = moe_ref(x[None, :], ex._routers[0], ex._experts[0])
        assert np.array_equal(np.sort(st["expert_indices"]), np.sort(idx[0]))
        assert O.rel_l2(out, want[0]) <= 5e-3

    def test_batch_routes_every_token(self):
        ex = make_executor()
        x = np.random.RandomState(6).randn(5, 16).astype(np.float32)
        out, st = ex.dispatch(0, x)
        assert out.shape == (5, 16) and st["expert_indices"].shape == (5, 2)
        want, _, _ = moe_ref(x, ex._routers[0], ex._experts[0])
        assert O.rel_l2(out, want) <= 5e-3

    def test_shared_missing_shutdown(self):
        x = np.random.RandomState(77).randn(16).astype(np.float32)
        a, _ = make_executor(shared=False).dispatch(0, x)
        ex = make_executor(shared=True)
        b, _ = ex.dispatch(0, x)
        assert not np.allclose(a, b) and np.all(np.isfinite(b))
        want, _, _ = moe_ref(x[None, :], ex._routers[0], ex._experts[0], ex._shared[0])
        assert O.rel_l2(b, want[0]) <= 5e-3
        z, st = ex.dispatch(99, x)
        assert z.shape == (16,) and np.all(z == 0) and st["gpu_hits"] == 0
        ex.shutdown()
        assert ex.dispatch(0, x)[0].shape == (16,)
        est = ex.memory_estimate(expert_dim=32, shared_dim=16, bytes_per_param=4.0)
        assert abs(est["per_expert_mb"] - 3 * 16 * 32 * 4.0 / 1024 ** 2) < 1e-10
        ls = make_executor(hot_ids=[0, 1]).layer_stats(0)
        assert ls["hot_experts"] == 2 and abs(ls["hot_pct"] - 50.0) < 1e-10


class TestMoE:
    def test_router(self):
        r = make_router(16, 8, 3)
        x = np.random.randn(5, 16).astype(np.float32)
        idx, w = r.route(x)
        assert idx.shape == (5, 3) and np.allclose(w.sum(-1), 1.0, atol=1e-6) and np.all(w >= 0)
        x1 = np.random.randn(16).astype(np.float32)
        i1, _ = r.route(x1)
        logits = r.predict(x1)
        assert logits.shape == (8,) and np.allclose(logits, r.predict(x1[None])[0])
        assert set(i1.tolist()) == set(np.argsort(logits)[-3:].tolist())
        assert np.allclose(logits, x1 @ r.weight, rtol=1e-5, atol=1e-5)

    def test_moe_ffn_silu(self):
        r, es = make_router(16, 4, 2), make_expert_set(4, 16, 32)
        x = np.random.RandomState(1).randn(5, 16).astype(np.float32)
        out, st = moe_ffn_silu(x, r, es)
        assert out.shape == (5, 16) and st["batch_size"] == 5 and st["expert_indices"].shape == (5, 2)
        want, _, _ = moe_ref(x, r, es)
        assert O.rel_l2(out, want) <= 5e-3
        o1, s1 = moe_ffn_silu(x[0], r, es)
        assert o1.shape == (16,) and s1["expert_indices"].shape == (1, 2) and s1["has_shared_expert"] is False
        o2, _ = moe_ffn_silu(x[0], r, es)
        assert np.array_equal(o1, o2)
        rng = np.random.default_rng(7)
        sh = (rng.standard_normal((16, 32)).astype(np.float32), rng.standard_normal((16, 32)).astype(np.float32),
              rng.standard_normal((32, 16)).astype(np.float32))
        o3, s3 = moe_ffn_silu(x[0], r, es, *sh)
        assert s3["has_shared_expert"] is True and not np.allclose(o1, o3)
        assert np.allclose(_dense_ffn(x[0], *sh), dense_ffn64(x[:1], sh[0].T, sh[1].T, sh[2].T)[0],
                           rtol=1e-4, atol=1e-4)

    def test_quantized_experts(self):
        e_n, h, i = 4, 512, 1024
        gen = torch.Generator(device="cuda").manual_seed(11)
        q = lambda shape: QTensor.quantize(torch.randn(shape, generator=gen, device="cuda") * 0.02, ggml.GGML_TYPE_Q4_K)
        es = MoEExpertSet([q((i, h)) for _ in range(e_n)], [q((i, h)) for _ in range(e_n)],
                          [q((h, i)) for _ in range(e_n)])
        r = ExpertRouter(np.random.RandomState(2).randn(h, e_n).astype(np.float32) * 0.05, topk=2)
        x = np.random.RandomState(3).randn(6, h).astype(np.float32)
        out, st = moe_ffn_silu(x, r, es)
        dq = lambda t: O.dequantize(t.to_numpy_bytes(), t.k, t.qtype)
        ref = MoEExpertSet(np.stack([dq(t) for t in es._qg]), np.stack([dq(t) for t in es._qu]),
                           np.stack([dq(t) for t in es._qd]))
        want, _, _ = moe_ref(x, r, ref)
        assert O.rel_l2(out, want) <= 5e-3


class TestBackend:
    def test_ops(self):
        be = GPUBackend()
        assert be.is_gpu and be.backend_name == "hip" and available_backends() == ["hip"]
        x = np.random.randn(7, 33).astype(np.float32)
        assert np.allclose(be.drelu(x), np.maximum(x, 0))
        assert np.allclose(be.silu(x), x / (1 + np.exp(-x)), rtol=1e-5, atol=1e-6)
        w = np.random.rand(33).astype(np.float32)
        want = x / np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + 1e-6) * w
        assert np.allclose(be.rms_norm(x, w), want, rtol=1e-5, atol=1e-6)
        e = np.exp(x - x.max(axis=-1, keepdims=True))
        assert np.allclose(be.softmax(x), e / e.sum(-1, keepdims=True), rtol=1e-5, atol=1e-7)
        assert np.allclose(be.softmax(x, axis=0), np.exp(x - x.max(0)) / np.exp(x - x.max(0)).sum(0),
                           rtol=1e-5, atol=1e-7)
        a, b = np.random.randn(3, 33).astype(np.float32), np.random.randn(33, 5).astype(np.float32)
        assert np.allclose(be.matmul(a, b), a @ b, rtol=1e-4, atol=1e-4)
        with pytest.raises(ValueError):
            HipBackend("metal")

    def test_quantized_matmul(self):
        be = HipBackend()
        w = (np.random.default_rng(0).standard_normal((300, 1024)) * 0.02).astype(np.float32)
        qt = QTensor.quantize(w, ggml.GGML_TYPE_Q4_K)
        wd = O.dequantize(qt.to_numpy_bytes(), 1024, qt.qtype).astype(np.float64)
        for m in (1, 12):
            a = np.random.default_rng(m).standard_normal((m, 1024)).astype(np.float32)
            assert O.rel_l2(be.matmul(a, qt), a @ wd.T) <= 5e-3
