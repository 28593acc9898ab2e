"""GPU parity of the on-device EMA neuron predictor (vb_ema_update,
vb_ema_predict) and of the sparse FFN block fed by its device-side count.

Bars: the EMA state bit-identical to the oracle's float32 numpy evaluation;
predicted masks, active lists and counts exact; the sparse block with a
device count bit-identical to the same block with the host-side set.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vibeblade_amd import ggml
from vibeblade_amd.sparse import DeviceEMAPredictor, EMANeuronPredictor
from vibeblade_amd.tensor import QTensor, sparse_ffn, ACT_RELU2, ACT_SILU, DOWN_GGUF, DOWN_NEURON_MAJOR

pytestmark = pytest.mark.gpu
Q4K = ggml.GGML_TYPE_Q4_K


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("alpha", [0.1, 0.3, 0.05, 1.0 / 3.0])
def test_ema_update_bit_exact(alpha):
    n = 14336
    rng = np.random.default_rng(int(alpha * 1000))
    pred = DeviceEMAPredictor(n, 2, ema_decay=alpha)
    want = np.zeros(n, np.float32)
    for step in range(20):
        m = rng.random(n) < 0.1 + 0.02 * step
        pred.update(1, m)
        want = O.ema_update(want, m, alpha)
        assert np.array_equal(bits(pred.get_activation_probabilities(1)), bits(want)), step
    assert np.all(pred.get_activation_probabilities(0) == 0.0)
    assert pred.total_updates == 20 and not pred.is_warmed_up


def _device_predict(probs, k, thr, warm, gate=None, combined=False):
    n = probs.size
    pred = DeviceEMAPredictor(n, 1, sparse_ratio=k / n + 1e-9, activation_threshold=thr)
    assert pred._k() == k
    pred._probs[0].copy_(torch.from_numpy(np.ascontiguousarray(probs, np.float32)))
    pred._update_counts[0] = 6 if warm else 0
    active, count, mask = pred.predict_active(0, gate, combined=combined)
    c = int(count.item())
    return mask.cpu().numpy().astype(bool), active.cpu().numpy()[:c], c


@pytest.mark.parametrize("n", [14336, 1000, 64, 3, 20000, 40000])
def test_ema_predict_matches_oracle(n):
    rng = np.random.default_rng(n)
    levels = np.array([0.0, 0.05, 0.1, 0.2, 0.3, 0.31, 0.5, 0.9], np.float32)
    for case in range(12):
        k = int(rng.integers(1, n + 1)) if case % 3 else max(1, n // 10)
        if case % 2:
            probs = rng.choice(levels, n)  # many ties
        else:
            probs = rng.random(n).astype(np.float32) * 0.6
        gate = rng.standard_normal(n).astype(np.float32)
        if case % 4 == 1:
            gate = np.round(gate)  # ties in the gate values too
        thr = 0.3
        for warm, g, comb in [(True, None, False), (False, gate, False), (False, None, False),
                              (True, gate, True), (False, gate, True), (True, gate, False)]:
            want = O.ema_predict(probs, k, thr, warm, gate=g, combined=comb)
            mask, active, c = _device_predict(probs, k, thr, warm, g, comb)
            assert np.array_equal(mask, want), (case, warm, comb)
            assert c == int(want.sum()) and np.array_equal(active, np.flatnonzero(want))


def test_device_predictor_follows_host_predictor():
    """A decode loop: predict, then update with the prediction, on the host
    class and the device class side by side."""
    n, layers = 4096, 3
    host = EMANeuronPredictor(n, layers, ema_decay=0.2, sparse_ratio=0.05, activation_threshold=0.3)
    dev = DeviceEMAPredictor(n, layers, ema_decay=0.2, sparse_ratio=0.05, activation_threshold=0.3)
    rng = np.random.default_rng(3)
    for t in range(12):
        for layer in range(layers):
            gate = rng.standard_normal(n).astype(np.float32)
            gate[: 50 + 10 * layer] += 3.0  # a persistent hot set
            mh = host.predict(layer, gate)
            md = dev.predict(layer, gate)
            assert np.array_equal(mh, md), (t, layer)
            host.update(layer, mh)
            dev.update(layer, md)
            assert np.array_equal(bits(host.get_activation_probabilities(layer)),
                                  bits(dev.get_activation_probabilities(layer)))
        comb_h = host.predict_combined(1, gate)
        comb_d = dev.predict_combined(1, gate)
        assert np.array_equal(comb_h, comb_d)
    assert dev.is_warmed_up and np.array_equal(host.get_top_neurons(2, 20), dev.get_top_neurons(2, 20))
    assert np.all(dev.predict(-1)) and np.all(dev.predict(layers))
    dev.reset()
    assert dev.total_updates == 0 and np.all(dev.get_activation_probabilities(0) == 0)


def _weights(h, i, layout, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    gq = QTensor.quantize(torch.randn((i, h), generator=g, device="cuda") * 0.02, Q4K)
    uq = QTensor.quantize(torch.randn((i, h), generator=g, device="cuda") * 0.02, Q4K)
    shape = (h, i) if layout == DOWN_GGUF else (i, h)
    dq = QTensor.quantize(torch.randn(shape, generator=g, device="cuda") * 0.02, Q4K)
    return gq, uq, dq


@pytest.mark.parametrize("h,i,layout,fused_env", [(4096, 14336, DOWN_NEURON_MAJOR, None),
                                                  (4096, 14336, DOWN_GGUF, None),
                                                  (2048, 4096, DOWN_NEURON_MAJOR, "0"),
                                                  (8192, 2048, DOWN_NEURON_MAJOR, None)])
def test_sparse_block_with_device_count(knob, h, i, layout, fused_env):
    """The predicted set through its device count gives the same bits as the
    same set passed from the host (every path: fused neuron-major, GGUF down,
    gathered neuron-major)."""
    if fused_env is not None:
        knob("VB_SPARSE_FUSED", fused_env)
    gq, uq, dq = _weights(h, i, layout, 11)
    rng = np.random.default_rng(12)
    x = torch.from_numpy(rng.standard_normal(h).astype(np.float32)).cuda()
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(h)).astype(np.float32)).cuda()
    pred = DeviceEMAPredictor(i, 1, sparse_ratio=0.1, activation_threshold=0.3)
    gate = rng.standard_normal(i).astype(np.float32)
    for warm in (False, True):
        if warm:
            for _ in range(6):
                pred.update(0, rng.random(i) < 0.12)
        active, count, mask = pred.predict_active(0, gate)
        y_dev = sparse_ffn(gq, uq, dq, x, active, ACT_RELU2, layout, norm_w=nw, residual=True, count=count)
        s = np.flatnonzero(mask.cpu().numpy())
        assert int(count.item()) == s.size
        y_host = sparse_ffn(gq, uq, dq, x, torch.from_numpy(s.astype(np.int32)), ACT_RELU2, layout, norm_w=nw,
                            residual=True)
        assert np.array_equal(bits(y_dev.cpu().numpy()), bits(y_host.cpu().numpy())), warm


def test_sparse_block_device_count_zero():
    """A device count of 0 (nothing predicted) leaves y = x / y = 0."""
    h, i = 2048, 4096
    for layout in (DOWN_NEURON_MAJOR, DOWN_GGUF):
        gq, uq, dq = _weights(h, i, layout, 13)
        x = torch.randn(h, device="cuda")
        active = torch.zeros(i, dtype=torch.int32, device="cuda")
        zero = torch.zeros(1, dtype=torch.int32, device="cuda")
        y = sparse_ffn(gq, uq, dq, x, active, ACT_SILU, layout, residual=True, count=zero)
        assert torch.equal(y, x)
        y0 = sparse_ffn(gq, uq, dq, x, active, ACT_SILU, layout, residual=False, count=zero)
        assert torch.count_nonzero(y0) == 0


def test_predict_and_block_in_a_graph():
    """predict_active + the sparse block captured in a HIP graph: each replay
    equals the eager result for the predictor state of that moment (the EMA
    state changes eagerly between replays)."""
    h, i = 4096, 14336
    gq, uq, dq = _weights(h, i, DOWN_NEURON_MAJOR, 14)
    rng = np.random.default_rng(15)
    x = torch.from_numpy(rng.standard_normal(h).astype(np.float32)).cuda()
    pred = DeviceEMAPredictor(i, 1, sparse_ratio=0.1, activation_threshold=0.3)
    for _ in range(6):
        pred.update(0, rng.random(i) < 0.15)
    gate = torch.from_numpy(rng.standard_normal(i).astype(np.float32)).cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up outside the capture
        active, count, _ = pred.predict_active(0, gate)
        sparse_ffn(gq, uq, dq, x, active, ACT_RELU2, DOWN_NEURON_MAJOR, residual=True, count=count)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_active, g_count, _ = pred.predict_active(0, gate)
        g_y = sparse_ffn(gq, uq, dq, x, g_active, ACT_RELU2, DOWN_NEURON_MAJOR, residual=True, count=g_count)
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        active, count, _ = pred.predict_active(0, gate)
        y = sparse_ffn(gq, uq, dq, x, active, ACT_RELU2, DOWN_NEURON_MAJOR, residual=True, count=count)
        torch.cuda.synchronize()
        assert int(g_count.item()) == int(count.item())
        assert torch.equal(g_y, y), rep
        pred.update(0, rng.random(i) < 0.2)  # eager work between replays
        torch.cuda.synchronize()
