"""GPU parity for GGUF ingestion: tensors uploaded from a file by
vb_gguf_upload reach HBM byte for byte, and the GEMV and decode kernels
give the oracle's results on them.

Bars: byte-exact upload; bit-exact decode; rel-L2 <= 1e-3 for GEMV.
"""
import numpy as np
import pytest
import torch

import oracle as O
from vibeblade_amd.gguf_write import STRING, U32, write_gguf
from vibeblade_amd import ggml
from vibeblade_amd.gguf import GGUFFile, GGUFLoader
from vibeblade_amd.tensor import gemv

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


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    """A small llama-style file: three quantized FFN weights and a norm."""
    rng = np.random.default_rng(3)
    tensors, weights = [], {}
    for name, (rows, k), qt in [("blk.0.ffn_gate.weight", (96, 1024), ggml.GGML_TYPE_Q4_K),
                                ("blk.0.ffn_down.weight", (64, 768), ggml.GGML_TYPE_Q6_K),
                                ("blk.0.attn_q.weight", (40, 512), ggml.GGML_TYPE_Q8_0)]:
        w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
        q = O.quantize(w, qt)
        weights[name] = (q, rows, k, qt)
        tensors.append((name, (k, rows), qt, q.tobytes()))
    norm = rng.standard_normal(1024).astype(np.float32)
    tensors.append(("blk.0.ffn_norm.weight", (1024,), ggml.GGML_TYPE_F32, norm.tobytes()))
    q8k = rng.integers(0, 256, 2 * ggml.row_bytes(ggml.GGML_TYPE_Q8_K, 256), dtype=np.uint8)
    tensors.append(("blk.0.attn_k.weight", (256, 2), ggml.GGML_TYPE_Q8_K, q8k.tobytes()))
    path = tmp_path_factory.mktemp("gguf") / "tiny.gguf"
    write_gguf(path, [("general.architecture", STRING, "llama"), ("llama.block_count", U32, 1)], tensors,
               alignment=64)
    return path, weights, norm


def test_upload_bytes_and_gemv(model):
    path, weights, norm = model
    rng = np.random.default_rng(9)
    with GGUFFile(path) as f:
        for name, (q, rows, k, qt) in weights.items():
            w = f.load_qtensor(name, "cuda:0")
            assert w.shape == (rows, k) and w.qtype == qt
            assert np.array_equal(w.to_numpy_bytes(), q.reshape(rows, -1)), name
            x = rng.standard_normal(k).astype(np.float32)
            y = gemv(w, torch.from_numpy(x).cuda()).cpu().numpy()
            want = O.gemv(q, x, rows, k, qt)
            assert O.rel_l2(y, want) <= GEMV_TOL, name
        nw = f.load_qtensor("blk.0.ffn_norm.weight", "cuda:0")
        assert nw.shape == (1, 1024)
        assert np.array_equal(bits(nw.dequantize().cpu().numpy().ravel()), bits(norm))
        with pytest.raises(ValueError):
            f.load_qtensor("blk.0.attn_k.weight")  # Q8_K: no device kernels
        with pytest.raises(KeyError):
            f.load_qtensor("missing")


def test_loader_decode_bit_exact(model):
    path, weights, norm = model
    with GGUFLoader(path) as ld:
        for name, (q, rows, k, qt) in weights.items():
            got = ld.load_tensor(name)
            assert got.shape == (rows, k)
            assert np.array_equal(bits(got), bits(O.dequantize(q.reshape(rows, -1), k, qt))), name
        assert np.array_equal(bits(ld.load_tensor("blk.0.ffn_norm.weight")), bits(norm))
        with pytest.raises(ValueError):
            ld.load_tensor("blk.0.attn_k.weight")


def test_upload_larger_than_staging(tmp_path):
    """A 75 MB tensor after a small one: ten staging chunks through two buffers,
    a ragged last chunk, a data offset that is not chunk-aligned."""
    rng = np.random.default_rng(4)
    rows, k = 17, 128
    small = rng.integers(0, 256, rows * ggml.row_bytes(ggml.GGML_TYPE_Q8_0, k), dtype=np.uint8)
    big_rows, big_k = 2311, 32 * 1000
    big = rng.integers(0, 256, big_rows * ggml.row_bytes(ggml.GGML_TYPE_Q8_0, big_k), dtype=np.uint8)
    assert big.size > 64 << 20
    path = tmp_path / "big.gguf"
    write_gguf(path, [], [("small", (k, rows), ggml.GGML_TYPE_Q8_0, small.tobytes()),
                          ("big", (big_k, big_rows), ggml.GGML_TYPE_Q8_0, big.tobytes())])
    with GGUFFile(path) as f:
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            wb = f.load_qtensor("big", "cuda:0")
            ws = f.load_qtensor("small", "cuda:0")
        s.synchronize()
        assert np.array_equal(ws.to_numpy_bytes().ravel(), small)
        got = wb.data.cpu().numpy()
        assert got.size == big.size and np.array_equal(got.ravel(), big)


def test_upload_split_copy_tail(tmp_path):
    """Chunks of at least 4 MiB are copied by several host threads; a chunk
    whose size is 1-3 bytes past a multiple of 16 KiB once lost its last
    bytes to a rounded-down share.  1-D F16 tensors of 4 MiB + 2 and
    12 MiB + 2 bytes (an 8 MiB chunk, then the ragged one) and of
    4 MiB + 16 KiB + 2 bytes come back byte for byte."""
    rng = np.random.default_rng(40)
    tensors, blobs = [], {}
    for name, nbytes in (("a", (4 << 20) + 2), ("b", (12 << 20) + 2), ("c", (4 << 20) + (16 << 10) + 2)):
        blob = rng.integers(0, 256, nbytes, dtype=np.uint8)
        blobs[name] = blob
        tensors.append((name, (nbytes // 2,), ggml.GGML_TYPE_F16, blob.tobytes()))
    path = tmp_path / "tail.gguf"
    write_gguf(path, [], tensors)
    with GGUFFile(path) as f:
        for name, blob in blobs.items():
            qt = f.load_qtensor(name, "cuda:0")
            torch.cuda.synchronize()
            got = qt.data.cpu().numpy().ravel()
            assert got.size == blob.size and np.array_equal(got, blob), name
