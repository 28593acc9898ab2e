"""GGUF ingestion (vb_gguf_* in libvbhip, vibeblade_amd.gguf): parsing on
the CPU, no GPU needed.

Files are written by vibeblade_amd/gguf_write.py from the GGUF format definition.
Parity: every header field, metadata value and tensor byte read back as
written; errors for every malformed case; the same tensor table, bytes and
(kept) metadata as the reference's own parser (cpp/src/gguf.cpp, compiled
into oracle/_ref where the reference tree is present).
"""
import ctypes
import os
import struct

import numpy as np
import pytest

from vibeblade_amd.gguf_write import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64,
                       gguf_bytes, gstr, write_gguf)
from vibeblade_amd import ggml
from vibeblade_amd.gguf import GGUFFile, GGUFLoader

KVS = [
    ("general.architecture", STRING, "llama"),
    ("general.name", STRING, "tiny éè test"),
    ("t.u8", U8, 250), ("t.i8", I8, -7), ("t.u16", U16, 65000), ("t.i16", I16, -30000),
    ("t.u32", U32, 4000000000), ("t.i32", I32, -123456), ("t.f32", F32, 1.5e-3),
    ("t.bool", BOOL, True), ("t.u64", U64, 2 ** 63 + 5), ("t.i64", I64, -(2 ** 40)), ("t.f64", F64, 1.2345678912345e30),
    ("llama.context_length", U32, 8192), ("llama.embedding_length", U32, 4096),
    ("llama.rope.freq_base", F32, 500000.0),
    ("tokenizer.ggml.tokens", ARRAY, (STRING, ["<s>", "</s>", "hello", "", "wörld"])),
    ("tokenizer.ggml.scores", ARRAY, (F32, [0.0, -1.5, 2.25])),
    ("tokenizer.ggml.token_type", ARRAY, (I32, [1, 3, 1, 1, 2])),
    ("t.u8s", ARRAY, (U8, [0, 255, 7])), ("t.i16s", ARRAY, (I16, [-2, 3])), ("t.u64s", ARRAY, (U64, [1, 2 ** 50])),
    ("t.f64s", ARRAY, (F64, [0.5, -0.25])), ("t.bools", ARRAY, (BOOL, [True, False])),
    ("t.empty", ARRAY, (I32, [])),
]


def rand_tensors(rng):
    def raw(gt, dims):
        be, bb = ggml.BLOCK[gt]
        n = 1
        for d in dims:
            n *= d
        return rng.integers(0, 256, n // be * bb, dtype=np.uint8).tobytes()

    spec = [("tok_embd.weight", (512, 8), ggml.GGML_TYPE_Q4_K), ("norm.weight", (64,), ggml.GGML_TYPE_F32),
            ("blk.0.ffn_gate.weight", (256, 6), ggml.GGML_TYPE_Q6_K), ("half", (32, 3), ggml.GGML_TYPE_F16),
            ("bf", (16,), ggml.GGML_TYPE_BF16), ("q8", (64, 2, 3), ggml.GGML_TYPE_Q8_0),
            ("q40", (64, 2), ggml.GGML_TYPE_Q4_0), ("q5k", (256, 2, 1, 2), ggml.GGML_TYPE_Q5_K),
            ("q8k", (256, 3), ggml.GGML_TYPE_Q8_K)]
    return [(n, d, t, raw(t, d)) for n, d, t in spec]


@pytest.fixture()
def sample(tmp_path):
    rng = np.random.default_rng(5)
    tensors = rand_tensors(rng)
    path = tmp_path / "m.gguf"
    data_start, offs = write_gguf(path, KVS, tensors)
    return path, tensors, data_start, offs


def test_roundtrip(sample):
    path, tensors, data_start, offs = sample
    with GGUFFile(path) as f:
        assert f.version() == 3 and f.alignment == 32 and f.data_offset == data_start
        assert f.file_size() == os.path.getsize(path)
        infos = f.tensors()
        assert [t.name for t in infos] == [t[0] for t in tensors]
        for ti, (name, dims, gt, data), off in zip(infos, tensors, offs):
            assert ti.n_dims == len(dims) and ti.dims[: len(dims)] == tuple(dims)
            assert all(d == 1 for d in ti.dims[len(dims):])
            assert ti.type == gt and ti.offset == off and ti.size == len(data)
            assert f.tensor_data(name).tobytes() == data
            assert f.tensor_info(name) == ti
        assert f.tensor_info("nope") is None and f.tensor_data("nope") is None
        for k, t, v in KVS:
            got = f.metadata[k]
            if t == F32:
                assert got == float(np.float32(v))
            elif t == ARRAY and v[0] == F32:
                assert got == [float(np.float32(x)) for x in v[1]]
            else:
                assert got == (list(v[1]) if t == ARRAY else v), k
        assert f.meta_string("general.architecture") == "llama"
        assert f.meta_string("missing") == "" and f.meta_int("missing", 7) == 7
        assert f.meta_int("t.u32") == 4000000000 and f.meta_int("t.u16") == 65000
        assert f.meta_int("general.name", -1) == -1  # wrong type -> default
        assert f.meta_float("t.f64") == 1.2345678912345e30 and f.meta_bool("t.bool") is True
        assert f.meta_string_array("tokenizer.ggml.tokens")[4] == "wörld"
        assert f.meta_int_array("tokenizer.ggml.token_type") == [1, 3, 1, 1, 2]
        assert f.meta_float_array("tokenizer.ggml.scores") == [0.0, -1.5, 2.25]
        assert f.meta_int_array("t.empty") == []


def test_streamed_writer_matches_bytes(sample, tmp_path):
    path, tensors, _, _ = sample
    assert path.read_bytes() == gguf_bytes(KVS, tensors)[0]
    q = tmp_path / "o.gguf"
    write_gguf(q, KVS[:2], tensors[:3], alignment=256, offsets=[512, 0, 4096])
    assert q.read_bytes() == gguf_bytes(KVS[:2], tensors[:3], alignment=256, offsets=[512, 0, 4096])[0]


@pytest.mark.parametrize("alignment", [64, 256])
def test_general_alignment(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    tensors = rand_tensors(rng)
    path = tmp_path / "a.gguf"
    data_start, offs = write_gguf(path, KVS[:3], tensors, alignment=alignment)
    assert data_start % alignment == 0
    with GGUFFile(path) as f:
        assert f.alignment == alignment and f.data_offset == data_start
        for ti, (name, _, _, data), off in zip(f.tensors(), tensors, offs):
            assert ti.offset == off and off % alignment == 0
            assert f.tensor_data(name).tobytes() == data


def test_loader_surface(sample):
    path, tensors, _, offs = sample
    calls = []
    with GGUFLoader(str(path), progress_cb=lambda *a, **k: calls.append(a)) as ld:
        assert ld.tensor_names() == [t[0] for t in tensors]
        assert ld.n_tensors == len(tensors) and ld.n_kv == len(KVS)
        info = ld.tensor_info("q8")
        assert info == {"name": "q8", "shape": (3, 2, 64), "dtype": ggml.GGML_TYPE_Q8_0, "offset": offs[5]}
        with pytest.raises(KeyError):
            ld.tensor_info("missing")
        norm = ld.load_tensor("norm.weight")
        assert norm.dtype == np.float32 and norm.shape == (64,)
        assert np.array_equal(norm.view(np.uint32), np.frombuffer(tensors[1][3], np.uint32))
        half = ld.load_tensor("half", dtype=np.float16)
        assert half.shape == (3, 32)
        assert np.array_equal(half.view(np.uint16).ravel(), np.frombuffer(tensors[3][3], np.uint16))
        bf = ld.load_tensor("bf")
        want = (np.frombuffer(tensors[4][3], np.uint16).astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(bf.view(np.uint32), want.view(np.uint32))
        with pytest.raises(ValueError):
            ld.load_tensor("q8k")  # Q8_K: no device kernels
        assert ld.metadata["llama.context_length"] == 8192
    assert calls


def _corrupt(kind):
    """(file bytes, expected error fragment) for one malformed case."""
    good = [("a", (32,), ggml.GGML_TYPE_F32, bytes(128))]
    kv = [("k", U32, 1)]
    if kind == "magic":
        raw = bytearray(gguf_bytes(kv, good)[0]); raw[0:4] = b"GGML"; return bytes(raw), "bad magic"
    if kind == "version":
        return gguf_bytes(kv, good, version=4)[0], "version"
    if kind == "version0":
        return gguf_bytes(kv, good, version=0)[0], "version"
    if kind == "short_header":
        return gguf_bytes(kv, good)[0][:20], "header"
    if kind == "kv_string":
        raw = gguf_bytes([("k", STRING, "x" * 100)], [])[0]
        return raw[: 24 + 9 + 4 + 8 + 50], "past the end"
    if kind == "huge_string":
        raw = bytearray(gguf_bytes([("k", STRING, "x")], [])[0]); raw[24 + 9 + 4: 24 + 9 + 12] = struct.pack("<Q", 2 ** 62)
        return bytes(raw), "past the end"
    if kind == "kv_type":
        head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1)
        return head + gstr("k") + struct.pack("<I", 13) + bytes(8), "unknown metadata value type"
    if kind == "nested_array":
        head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1)
        return head + gstr("k") + struct.pack("<IIQ", ARRAY, ARRAY, 1) + bytes(16), "unknown array element type"
    if kind == "n_dims":
        return gguf_bytes(kv, [("a", (32, 1, 1, 1, 1), ggml.GGML_TYPE_F32, bytes(128))])[0], "dimensions"
    if kind == "tensor_type":
        return gguf_bytes(kv, [("a", (32,), 99, bytes(128))])[0], "unknown type"
    if kind == "partial_block":
        return gguf_bytes(kv, [("a", (33,), ggml.GGML_TYPE_Q8_0, bytes(34))])[0], "whole number of blocks"
    if kind == "data_past_end":
        raw = gguf_bytes(kv, good)[0]
        return raw[:-8], "past the end"
    if kind == "unaligned_offset":
        return gguf_bytes(kv, good + [("b", (8,), ggml.GGML_TYPE_F32, bytes(32))], offsets=[0, 136])[0], "not aligned"
    if kind == "alignment_value":
        return gguf_bytes(kv, good, alignment=48)[0], "power of two"
    if kind == "alignment_type":
        return gguf_bytes(kv + [("general.alignment", U64, 32)], good)[0], "not a uint32"
    if kind == "duplicate":
        return gguf_bytes(kv, good + [("a", (32,), ggml.GGML_TYPE_F32, bytes(128))])[0], "duplicate"
    if kind == "count":
        raw = bytearray(gguf_bytes(kv, good)[0]); raw[8:16] = struct.pack("<Q", 2 ** 40)
        return bytes(raw), "implausible"
    raise AssertionError(kind)


@pytest.mark.parametrize("kind", ["magic", "version", "version0", "short_header", "kv_string", "huge_string",
                                  "kv_type", "nested_array", "n_dims", "tensor_type", "partial_block",
                                  "data_past_end", "unaligned_offset", "alignment_value", "alignment_type",
                                  "duplicate", "count"])
def test_malformed(tmp_path, kind):
    raw, frag = _corrupt(kind)
    p = tmp_path / "bad.gguf"
    p.write_bytes(raw)
    with pytest.raises(ValueError, match=frag):
        GGUFFile(p)


def test_missing_and_empty(tmp_path):
    with pytest.raises(FileNotFoundError):
        GGUFFile(tmp_path / "nope.gguf")
    p = tmp_path / "empty.gguf"
    p.write_bytes(b"")
    with pytest.raises(ValueError):
        GGUFFile(p)
    # a file with no tensors and no metadata is valid
    q = tmp_path / "min.gguf"
    q.write_bytes(gguf_bytes([], [])[0])
    with GGUFFile(q) as f:
        assert f.tensors() == [] and f.metadata == {}


def test_truncations_and_flips_never_crash(sample):
    """Every prefix of a valid file, and files with bytes flipped in the
    header / metadata / tensor table, parse or raise ValueError: the reader
    never reads outside the mapping."""
    path, tensors, data_start, _ = sample
    raw = path.read_bytes()
    d = path.parent
    rng = np.random.default_rng(11)
    cuts = sorted(set(list(range(0, min(data_start, 600))) + list(rng.integers(0, len(raw), 60))))
    for n in cuts:
        p = d / "cut.gguf"
        p.write_bytes(raw[:n])
        try:
            GGUFFile(p).close()
        except ValueError:
            pass
    for _ in range(300):
        b = bytearray(raw)
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(0, data_start))] = int(rng.integers(0, 256))
        p = d / "flip.gguf"
        p.write_bytes(bytes(b))
        try:
            GGUFFile(p).close()
        except ValueError:
            pass


# ---- the reference's own parser ---------------------------------------------

_REF = os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libvbref_gguf.so")


def _ref_lib():
    if not os.path.exists(_REF):
        pytest.skip("reference GGUF reader not built (oracle/_ref)")
    lib = ctypes.CDLL(_REF)
    vp, i64, i32, u64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64
    lib.ref_gguf_open.restype = vp
    lib.ref_gguf_open.argtypes = [ctypes.c_char_p]
    lib.ref_gguf_close.argtypes = [vp]
    lib.ref_gguf_error.restype = ctypes.c_char_p
    lib.ref_gguf_n_tensors.restype = i64
    lib.ref_gguf_n_tensors.argtypes = [vp]
    lib.ref_gguf_tensor.argtypes = [vp, i64, ctypes.c_char_p, i64, ctypes.POINTER(i32), ctypes.POINTER(i64),
                                    ctypes.POINTER(i32), ctypes.POINTER(u64), ctypes.POINTER(u64)]
    lib.ref_gguf_tensor_bytes.restype = i64
    lib.ref_gguf_tensor_bytes.argtypes = [vp, ctypes.c_char_p, vp, i64]
    lib.ref_gguf_meta_int.restype = i64
    lib.ref_gguf_meta_int.argtypes = [vp, ctypes.c_char_p, i64]
    lib.ref_gguf_meta_float.restype = ctypes.c_float
    lib.ref_gguf_meta_float.argtypes = [vp, ctypes.c_char_p, ctypes.c_float]
    lib.ref_gguf_meta_bool.argtypes = [vp, ctypes.c_char_p, ctypes.c_int]
    lib.ref_gguf_meta_string.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, i64]
    lib.ref_gguf_meta_int_array.restype = i64
    lib.ref_gguf_meta_int_array.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(i64), i64]
    lib.ref_gguf_meta_float_array.restype = i64
    lib.ref_gguf_meta_float_array.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), i64]
    lib.ref_gguf_meta_string_array.argtypes = [vp, ctypes.c_char_p, i64, ctypes.c_char_p, i64]
    lib.ref_gguf_meta_string_array_len.restype = i64
    lib.ref_gguf_meta_string_array_len.argtypes = [vp, ctypes.c_char_p]
    return lib


def test_against_reference_parser(sample):
    """Same tensor table and bytes as cpp/src/gguf.cpp, and the same values
    for the metadata it keeps.  Documented differences: it drops 16-bit
    values (gguf.cpp:89-90), reads uint32 as int32 (:91) and keeps f64 as
    float (:157); the build keeps each value as written."""
    lib = _ref_lib()
    path, tensors, _, offs = sample
    h = lib.ref_gguf_open(str(path).encode())
    assert h, lib.ref_gguf_error()
    try:
        with GGUFFile(path) as f:
            assert lib.ref_gguf_n_tensors(h) == len(f.tensors())
            for i, ti in enumerate(f.tensors()):
                name = ctypes.create_string_buffer(256)
                nd, typ = ctypes.c_int32(), ctypes.c_int32()
                dims = (ctypes.c_int64 * 4)()
                off, size = ctypes.c_uint64(), ctypes.c_uint64()
                lib.ref_gguf_tensor(h, i, name, 256, ctypes.byref(nd), dims, ctypes.byref(typ), ctypes.byref(off),
                                    ctypes.byref(size))
                assert name.value.decode() == ti.name and nd.value == ti.n_dims and tuple(dims) == ti.dims
                assert typ.value == ti.type and off.value == ti.offset and size.value == ti.size
                buf = np.zeros(ti.size, np.uint8)
                assert lib.ref_gguf_tensor_bytes(h, ti.name.encode(), buf.ctypes.data, ti.size) == ti.size
                assert buf.tobytes() == f.tensor_data(ti.name).tobytes()
            for k, t, v in KVS:
                kb = k.encode()
                if t in (U8, I8, I32, I64):
                    assert lib.ref_gguf_meta_int(h, kb, 12345) == v == f.meta_int(k)
                elif t == U32:
                    want = v - 2 ** 32 if v >= 2 ** 31 else v  # the reference reads uint32 as int32
                    assert lib.ref_gguf_meta_int(h, kb, 12345) == want
                    assert f.meta_int(k) == v
                elif t == U64:
                    assert lib.ref_gguf_meta_int(h, kb, 12345) % 2 ** 64 == v == f.meta_int(k)
                elif t in (U16, I16):
                    assert lib.ref_gguf_meta_int(h, kb, 12345) == 12345  # dropped by the reference
                    assert f.meta_int(k) == v
                elif t == F32:
                    assert lib.ref_gguf_meta_float(h, kb, -1.0) == np.float32(v) == np.float32(f.meta_float(k))
                elif t == F64:
                    assert lib.ref_gguf_meta_float(h, kb, -1.0) == np.float32(v)
                    assert f.meta_float(k) == v
                elif t == BOOL:
                    assert bool(lib.ref_gguf_meta_bool(h, kb, 0)) == v == f.meta_bool(k)
                elif t == STRING:
                    sb = ctypes.create_string_buffer(256)
                    lib.ref_gguf_meta_string(h, kb, sb, 256)
                    assert sb.value.decode() == v == f.meta_string(k)
                elif t == ARRAY and v[0] == STRING:
                    n = lib.ref_gguf_meta_string_array_len(h, kb)
                    got = []
                    for j in range(n):
                        sb = ctypes.create_string_buffer(256)
                        lib.ref_gguf_meta_string_array(h, kb, j, sb, 256)
                        got.append(sb.value.decode())
                    assert got == v[1] == f.meta_string_array(k)
                elif t == ARRAY and v[0] in (I32, U32, I64, U64):
                    out = (ctypes.c_int64 * 16)()
                    n = lib.ref_gguf_meta_int_array(h, kb, out, 16)
                    assert [x % 2 ** 64 if v[0] == U64 else x for x in out[:n]] == v[1] == f.meta_int_array(k)
                elif t == ARRAY and v[0] == F32:
                    out = (ctypes.c_float * 16)()
                    n = lib.ref_gguf_meta_float_array(h, kb, out, 16)
                    assert list(out[:n]) == v[1] == f.meta_float_array(k)
    finally:
        lib.ref_gguf_close(h)


def test_tensor_data_outlives_close(sample):
    """A tensor_data view keeps the mapping alive after close() and after the
    GGUFFile is dropped (it used to dangle and crash on access)."""
    import gc
    path, tensors, _, _ = sample
    name, _, _, data = tensors[0]
    f = GGUFFile(path)
    view = f.tensor_data(name)
    f.close()
    assert view.tobytes() == data
    with pytest.raises(ValueError):
        f.load_qtensor(name)
    view2 = GGUFFile(path).tensor_data(tensors[2][0])
    gc.collect()
    assert view2[-1] == tensors[2][3][-1] and view2.tobytes() == tensors[2][3]
    del view, view2, f
    gc.collect()
