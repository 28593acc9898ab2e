"""Host-side parts of the drop-in surface (CPU only): RotorQuant packing,
sparse mask helpers, HotColdMap persistence, ExecutorStats, MoE weight
containers and tensor-name detection.  Mirrors the reference's own tests
(tests/test_quant.py, test_sparse.py, test_moe_executor.py, test_moe.py,
test_ema_neuron.py)."""
import numpy as np
import pytest

from vibeblade_amd import quant, sparse
from vibeblade_amd.moe import MoEConfig, MoEExpertSet, detect_moe_config, load_moe_weights_from_layer
from vibeblade_amd.moe_executor import ExecutorStats
from vibeblade_amd.moe_profiler import HotColdMap


class TestRotorQuant:
    def test_pack_unpack(self):
        v = np.random.default_rng(42).integers(0, 16, 101).astype(np.uint8)
        assert np.array_equal(quant.unpack_nibbles(quant.pack_nibbles(v), v.size), v)
        assert quant.pack_nibbles(np.zeros(11, np.uint8)).shape == (6,)
        assert quant.pack_nibbles(np.array([3, 11], np.uint8))[0] == 0xB3
        assert quant.pack_nibbles(np.array([7], np.uint8))[0] == 0x07
        with pytest.raises(ValueError):
            quant.pack_nibbles(np.array([16], np.uint8))
        with pytest.raises(ValueError):
            quant.unpack_nibbles(np.array([0xAB], np.uint8), n=3)

    def test_rotor(self):
        rng = np.random.default_rng(123)
        for _ in range(20):
            r = quant.build_so4_rotor(rng.standard_normal(4).astype(np.float32))
            assert abs(np.linalg.det(r) - 1.0) < 1e-5
            assert np.allclose(r @ r.T, np.eye(4), atol=1e-5)
        assert np.array_equal(quant.build_so4_rotor(np.zeros(4, np.float32)), np.eye(4, dtype=np.float32))
        with pytest.raises(ValueError):
            quant.build_so4_rotor(np.zeros(3))

    def test_roundtrip_and_errors(self):
        w = np.random.default_rng(0).standard_normal(256).astype(np.float32)
        packed, scales, rotors = quant.quantize_4bit(w, 32)
        assert packed.shape == (128,) and scales.shape == (8, 2, 8) and rotors.shape == (8, 8, 4, 4)
        back = quant.dequantize_4bit(packed, scales, rotors, w.size)
        assert quant.quantization_error(w, back) < 0.15
        c = np.full(64, 0.75, np.float32)
        assert np.allclose(quant.dequantize_4bit(*quant.quantize_4bit(c), 64), c, atol=1e-6)
        with pytest.raises(ValueError):
            quant.quantize_4bit(np.zeros(30, np.float32), 32)
        with pytest.raises(ValueError):
            quant.quantize_4bit(np.zeros(32, np.float32), 6)
        with pytest.raises(ValueError):
            quant.dequantize_4bit(packed, scales, rotors, 100)
        assert quant.quantization_error(w, w) == 0.0
        assert abs(quant.quantization_error(np.zeros(4), np.ones(4)) - 1.0) < 1e-7
        with pytest.raises(ValueError):
            quant.quantization_error(np.zeros(3), np.zeros(4))


class TestSparseHost:
    def test_drelu_and_masks(self):
        x = np.array([-2.0, -1.0, 0.0, 0.5, 3.0])
        assert np.allclose(sparse.drelu_activation(x), [0, 0, 0, 0.5, 3.0])
        assert np.allclose(sparse.drelu_activation(np.array([-1.0, 0, 0.5, 1, 1.5, 2]), 1.0), [0, 0, 0, 0, 1.5, 2])
        assert np.all(sparse.drelu_gate(np.linspace(-5, 5, 101)) == 0)
        assert sparse.predict_activations(np.array([-1.0, 0.0, 0.5, 1.5])).tolist() == [False, False, True, True]
        assert sparse.compute_sparsity(np.zeros(100)) == pytest.approx(1.0)
        assert sparse.compute_sparsity(np.ones(100)) == pytest.approx(0.0)
        assert sparse.compute_sparsity(np.zeros(0)) == 0.0

    def test_topk_mask(self):
        x = np.random.RandomState(7).randn(5, 10)
        m = sparse.topk_activation_mask(x, 3)
        assert m.shape == (5, 10) and all(np.count_nonzero(r) == 3 for r in m)
        assert sparse.topk_activation_mask(np.array([[1.0, 5, 3, 2, 4]]), 2).tolist() == \
            [[False, True, False, False, True]]
        assert not sparse.topk_activation_mask(x, 0).any()
        assert sparse.topk_activation_mask(x, 10).all()

    def test_batch_drelu(self):
        act, mask = sparse.batch_drelu(np.array([[[-1.0, 0.0, 2.0]]]))
        assert act.tolist() == [[[0.0, 0.0, 2.0]]] and mask.tolist() == [[[False, False, True]]]
        a2, m2 = sparse.batch_drelu(np.random.randn(3, 5, 7))
        assert a2.shape == m2.shape == (3, 5, 7) and a2.dtype == np.float64 and m2.dtype == bool

    def test_ema_predictor(self):
        p = sparse.EMANeuronPredictor(hidden_dim=100, n_layers=2, ema_decay=0.5, sparse_ratio=0.1)
        assert p.predict(0).sum() == 10  # cold start, no gate values: first k
        gv = np.arange(100, dtype=np.float32)
        assert set(np.flatnonzero(p.predict(0, gv))) == set(range(90, 100))
        mask = np.zeros(100, bool)
        mask[:20] = True
        for _ in range(6):
            p.update(0, mask)
        assert p.is_warmed_up is False and p.total_updates == 6
        got = p.predict(0)
        assert got[:20].all() and got.sum() == 20
        assert p.get_top_neurons(0, 5).tolist() == [0, 1, 2, 3, 4]
        assert p.predict(5).all()  # out of range layer -> all active
        p.reset()
        assert p.total_updates == 0 and p.get_activation_probabilities(0).sum() == 0


def test_hot_cold_map_roundtrip(tmp_path):
    m = HotColdMap(hot_experts={0: [0, 1], 3: [2]}, cold_experts={0: [2, 3], 3: [0, 1, 3]}, num_layers=4,
                   num_experts=4, profile_tokens=10)
    p = tmp_path / "map.json"
    m.save(str(p))
    m2 = HotColdMap.load(str(p))
    assert m2 == m
    assert m.hit_rate(0, np.array([0, 2])) == 0.5
    assert m.overall_hit_rate() == 3 / 16
    assert "Layer   0: hot=2, cold=2" in m.summary()


def test_executor_stats():
    s = ExecutorStats(gpu_hits=3, cpu_falls=1, gpu_latency_ms=0.1234567, cpu_latency_ms=1.2, sync_latency_ms=0.1)
    d = s.to_dict()
    assert set(d) == {"gpu_hits", "cpu_falls", "gpu_latency_ms", "cpu_latency_ms", "sync_latency_ms", "hit_rate"}
    assert d["gpu_latency_ms"] == 0.123 and abs(d["hit_rate"] - 0.75) < 1e-4
    assert ExecutorStats().hit_rate == 0.0 and ExecutorStats(gpu_hits=1).hit_rate == 1.0


class TestMoEContainers:
    def test_expert_set(self):
        rng = np.random.default_rng(0)
        g = rng.standard_normal((4, 32, 16)).astype(np.float32)
        d = rng.standard_normal((4, 16, 32)).astype(np.float32)
        es = MoEExpertSet(g, g, d)
        assert (es.num_experts, es.expert_dim, es.shared_dim) == (4, 32, 16)
        gw, uw, dw = es.get_expert(2)
        assert gw.shape == (16, 32) and dw.shape == (32, 16)
        assert np.array_equal(gw, g[2].T)
        gb, ub, db = es.get_experts_batch(np.array([0, 3, 1, 2]))
        assert gb.shape == (4, 16, 32) and np.array_equal(gb[1], g[3].T)
        with pytest.raises(AssertionError):
            MoEExpertSet(g, g, np.zeros((4, 16, 8), np.float32))

    def test_detect_and_load(self):
        rng = np.random.default_rng(0)
        w = {
            "blk.0.ffn_gate_inp.weight": rng.standard_normal((4, 16)).astype(np.float32),  # (E, hidden)
            "blk.0.ffn_gate_exps.weight": rng.standard_normal((4, 32, 16)).astype(np.float32),
            "blk.0.ffn_up_exps.weight": rng.standard_normal((4, 32, 16)).astype(np.float32),
            "blk.0.ffn_down_exps.weight": rng.standard_normal((4, 16, 32)).astype(np.float32),
            "blk.0.ffn_gate_shexp.weight": rng.standard_normal((16, 32)).astype(np.float32),
        }
        cfg = detect_moe_config(w)
        assert (cfg.num_experts, cfg.expert_dim, cfg.shared_dim, cfg.num_active) == (4, 32, 16, 2)
        assert detect_moe_config({"x": np.zeros(3)}) is None
        r, es, extra = load_moe_weights_from_layer(w, 0)
        assert r.shape == (16, 4) and es.num_experts == 4 and "shared_gate" in extra
        assert load_moe_weights_from_layer(w, 1) == (None, None, {})
        alt = {"blk.2.ffn_router.weight": rng.standard_normal((16, 2)).astype(np.float32)}
        for e in range(2):
            alt[f"blk.2.expert.{e}.ffn_gate.weight"] = rng.standard_normal((32, 16)).astype(np.float32)
            alt[f"blk.2.expert.{e}.ffn_up.weight"] = rng.standard_normal((32, 16)).astype(np.float32)
            alt[f"blk.2.expert.{e}.ffn_down.weight"] = rng.standard_normal((16, 32)).astype(np.float32)
        assert detect_moe_config(alt).expert_dim == 32
        r2, es2, _ = load_moe_weights_from_layer(alt, 2)
        assert es2.num_experts == 2 and r2.shape == (16, 2)
        assert repr(MoEConfig(4, 2, 32, 16, has_shared_expert=True)).endswith("shared_expert=True)")


def test_stats_and_map_are_dataclasses():
    """ExecutorStats and HotColdMap are dataclasses with the reference's
    fields, order and defaults (vibeblade/moe_executor.py:31-38,
    vibeblade/moe_profiler.py:8-16): asdict / replace / fields work on them,
    and attributes can be added as on the reference's."""
    import dataclasses
    assert [f.name for f in dataclasses.fields(ExecutorStats)] == [
        "gpu_hits", "cpu_falls", "gpu_latency_ms", "cpu_latency_ms", "sync_latency_ms"]
    st = ExecutorStats(gpu_hits=3, cpu_falls=1, gpu_latency_ms=1.23456)
    assert dataclasses.asdict(st)["gpu_latency_ms"] == 1.23456
    assert dataclasses.replace(st, cpu_falls=3).hit_rate == 0.5
    st.extra = 1  # no __slots__
    assert st.copy() == ExecutorStats(3, 1, 1.23456)
    assert [(f.name, f.default) for f in dataclasses.fields(HotColdMap)][2:] == [
        ("num_layers", dataclasses.MISSING), ("num_experts", dataclasses.MISSING),
        ("profile_tokens", 0), ("profile_dataset", "")]
    m = HotColdMap({0: [1, 2]}, {0: [3]}, 1, 4)
    assert dataclasses.is_dataclass(m) and dataclasses.asdict(m)["hot_experts"] == {0: [1, 2]}
    assert dataclasses.replace(m, profile_tokens=7).profile_tokens == 7
