"""Pins the CPU oracle before anything is compared against it (CPU only).

Each decoder is checked against something independent of its own code:
golden vectors from the compiled reference, the reference's known-answer
tests, closed forms on blocks whose decoded values are known integers, or
the published ggml loop form of the layout.
"""
import os
import struct

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- fp16 ------------------------------------------------------------------

def test_f16_to_f32_exact_for_all_patterns():
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exact = allbits.view(np.float16).astype(np.float32)
    mine = np.array([O.f16_to_f32(int(b)) for b in allbits], dtype=np.float32)
    nan = np.isnan(exact)
    assert np.array_equal(np.isnan(mine), nan)
    assert np.array_equal(bits(mine[~nan]), bits(exact[~nan]))


def test_reference_f16_doubles_subnormals(gold):
    """cpp/src/fp16_compat.cpp:13-35 returns 2x the value of every fp16
    subnormal; normals and infinities are exact.  The oracle and the GPU follow
    IEEE (v_cvt_f32_f16), i.e. what GGUF files mean."""
    b = gold["f16_bits"]
    ref = gold["f16_ref"]
    exact = b.view(np.float16).astype(np.float32)
    sub = ((b & 0x7C00) == 0) & ((b & 0x3FF) != 0)
    assert np.array_equal(bits(ref[~sub]), bits(exact[~sub]))
    assert np.array_equal(ref[sub], 2.0 * exact[sub])


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(5000) * 10.0 ** rng.integers(-9, 5, 5000)).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8, 3e-8, np.inf])])
    mine = np.array([O.f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(mine, x.astype(np.float16).view(np.uint16))


# ---- Q4_K --------------------------------------------------------------------

def test_q4k_matches_compiled_reference(gold):
    blocks, want = gold["q4k_blocks"], gold["q4k_out"]
    got = O.dequantize(blocks.reshape(1, -1), blocks.shape[0] * 256, O.TYPE_Q4_K)
    assert np.array_equal(bits(got.ravel()), bits(want.ravel()))


def _q4k_unit_block(qs):
    b = bytearray(144)
    b[0:2] = struct.pack("<e", 1.0)
    b[2:4] = struct.pack("<e", 0.0)
    b[4:16] = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])  # sc_j = 1, m_j = 0
    b[16:144] = bytes(qs)
    return np.frombuffer(bytes(b), dtype=np.uint8)


def test_q4k_index_map_single_nibble():
    """d=1, dmin=0, every sc=1: y is the nibble itself.  One non-zero nibble
    per position checks the element -> (byte, nibble) map of
    cpp/src/dequant.cpp:289-296."""
    for byte in range(128):
        for hi in range(2):
            qs = [0] * 128
            qs[byte] = 5 << (4 * hi)
            y = O.dequantize(_q4k_unit_block(qs).reshape(1, -1), 256, O.TYPE_Q4_K).ravel()
            c, l = byte // 32, byte % 32
            e = 64 * c + 32 * hi + l
            want = np.zeros(256, np.float32)
            want[e] = 5.0
            assert np.array_equal(y, want), (byte, hi)


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference (oracle/_ref) not built here")
def test_q4k_every_scale_byte_matches_compiled_reference():
    """256 blocks in which every one of the 12 scale bytes takes all 256
    values (so every 6-bit scale / min field of get_scale_min_k4,
    cpp/src/dequant.cpp:258-266, takes all 64 values in every position),
    decoded by the oracle and by the compiled reference."""
    nb = 256
    rng = np.random.default_rng(7)
    blk = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    for i in range(12):
        blk[:, 4 + i] = (np.arange(nb) * 1 + i * 37) & 255
    blk[:, 0:2] = np.frombuffer(np.float16(0.75).tobytes(), np.uint8)
    blk[:, 2:4] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    got = O.dequantize(blk.reshape(1, -1), nb * 256, O.TYPE_Q4_K)
    want = O.ref_dequantize(blk.ravel(), nb * 256, O.TYPE_Q4_K)
    assert np.array_equal(bits(got.ravel()), bits(np.asarray(want).ravel()))


def test_q4k_min_term():
    b = bytearray(_q4k_unit_block([0x33] * 128).tobytes())
    b[2:4] = struct.pack("<e", 0.5)
    b[4:16] = bytes([2, 2, 2, 2, 3, 3, 3, 3, 0x32, 0x32, 0x32, 0x32])  # sc=2, m=3 everywhere
    y = O.dequantize(np.frombuffer(bytes(b), np.uint8).reshape(1, -1), 256, O.TYPE_Q4_K)
    assert np.all(y == 2.0 * 3 - 0.5 * 3)


# ---- Q6_K --------------------------------------------------------------------

def _q6k_block(fill_ql, fill_qh, scale=1, d=1.0):
    b = bytearray(210)
    b[0:128] = bytes([fill_ql]) * 128
    b[128:192] = bytes([fill_qh]) * 64
    b[192:208] = bytes([scale & 0xFF]) * 16
    b[208:210] = struct.pack("<e", d)
    return np.frombuffer(bytes(b), dtype=np.uint8)


@pytest.mark.parametrize("qtype", [O.TYPE_Q6_K, O.TYPE_Q6_K_VBREF])
def test_q6k_reference_known_answers(qtype):
    """The layout-invariant known answers of tests/test_kquants.py:134-175."""
    y = O.dequantize(_q6k_block(0xFF, 0xFF).reshape(1, -1), 256, qtype)
    assert np.all(y == 31.0)
    y = O.dequantize(_q6k_block(0x00, 0x00).reshape(1, -1), 256, qtype)
    assert np.all(y == -32.0)
    y = O.dequantize(_q6k_block(0x00, 0x55).reshape(1, -1), 256, qtype)
    assert np.all(y == -16.0)


def test_q6k_vbref_matches_compiled_reference(gold):
    blocks, want = gold["q6k_blocks"], gold["q6k_vbref_out"]
    got = O.dequantize(blocks.reshape(1, -1), blocks.shape[0] * 256, O.TYPE_Q6_K_VBREF)
    assert np.array_equal(bits(got.ravel()), bits(want.ravel()))


def _ggml_q6k_loop(block):
    """ggml's published dequantize_row_q6_K loop form (two halves of 128, four
    strided outputs per l), an independent statement of the GGUF layout."""
    ql = block[0:128].astype(np.int32)
    qh = block[128:192].astype(np.int32)
    sc = block[192:208].view(np.int8).astype(np.float32)
    d = np.float32(np.frombuffer(block[208:210].tobytes(), np.float16)[0])
    y = np.zeros(256, np.float32)
    for n in range(2):
        qlp, qhp, scp, yp = ql[64 * n:], qh[32 * n:], sc[8 * n:], 128 * n
        for l in range(32):
            i = l // 16
            q1 = ((qlp[l] & 0xF) | (((qhp[l] >> 0) & 3) << 4)) - 32
            q2 = ((qlp[l + 32] & 0xF) | (((qhp[l] >> 2) & 3) << 4)) - 32
            q3 = ((qlp[l] >> 4) | (((qhp[l] >> 4) & 3) << 4)) - 32
            q4 = ((qlp[l + 32] >> 4) | (((qhp[l] >> 6) & 3) << 4)) - 32
            y[yp + l] = d * scp[i + 0] * q1
            y[yp + l + 32] = d * scp[i + 2] * q2
            y[yp + l + 64] = d * scp[i + 4] * q3
            y[yp + l + 96] = d * scp[i + 6] * q4
    return y


def test_q6k_gguf_layout_against_ggml_loop_form():
    rng = np.random.default_rng(11)
    for _ in range(16):
        blk = rng.integers(0, 256, 210, dtype=np.uint8)
        blk[208:210] = np.frombuffer(np.float16(rng.uniform(1e-3, 2)).tobytes(), np.uint8)
        got = O.dequantize(blk.reshape(1, -1), 256, O.TYPE_Q6_K).ravel()
        assert np.array_equal(bits(got), bits(_ggml_q6k_loop(blk)))


def test_q6k_gguf_and_vbref_differ():
    """Single-position blocks separate the two gathers (the reference's C++
    decoder is not the GGUF one)."""
    blk = _q6k_block(0x00, 0x00).copy()
    blk[0] = 0x0F  # ql[0] low nibble
    g = O.dequantize(blk.reshape(1, -1), 256, O.TYPE_Q6_K).ravel()
    v = O.dequantize(blk.reshape(1, -1), 256, O.TYPE_Q6_K_VBREF).ravel()
    assert g[0] == -17.0 and v[0] == -17.0
    blk = _q6k_block(0x00, 0x00).copy()
    blk[1] = 0xF0  # ql[1] high nibble
    g = O.dequantize(blk.reshape(1, -1), 256, O.TYPE_Q6_K).ravel()
    v = O.dequantize(blk.reshape(1, -1), 256, O.TYPE_Q6_K_VBREF).ravel()
    assert np.flatnonzero(g != -32.0).tolist() == [65]   # GGUF: h=0,t=2,l=1
    assert np.flatnonzero(v != -32.0).tolist() == [3]    # VBREF: e/2=1, odd


# ---- ggml's published loop forms for the other GGUF types -----------------------
#
# Each helper restates ggml's dequantize_row_* loop (ggml-quants.c) in its own
# shape -- sequential outputs, strided reads, ggml's own scale unpacking -- in
# float64, which is exact for these products.  The oracle decodes by element
# index with its own helpers, in float32 (gcc may contract d*q - m into one
# fma), so the comparison allows a few float32 ulps of the terms: far below one
# quantization step, which any layout or bit-map mistake moves by.

def _h16(b):
    return float(np.frombuffer(bytes(b[:2]), np.float16)[0])


def _ulp_ok(got, want, scale):
    """|got - want| within 2^-20 of the per-block magnitude `scale`."""
    return np.all(np.abs(got.astype(np.float64) - want) <= scale * 2.0 ** -20)


def _ggml_scale_min_k4(j, q):
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def _ggml_q4_0(b):
    d, qs = _h16(b[0:2]), [int(v) for v in b[2:18]]
    y = np.zeros(32)
    for j in range(16):
        y[j] = ((qs[j] & 0x0F) - 8) * d
        y[j + 16] = ((qs[j] >> 4) - 8) * d
    return y


def _ggml_q4_1(b):
    d, m, qs = _h16(b[0:2]), _h16(b[2:4]), [int(v) for v in b[4:20]]
    y = np.zeros(32)
    for j in range(16):
        y[j] = (qs[j] & 0x0F) * d + m
        y[j + 16] = (qs[j] >> 4) * d + m
    return y


def _ggml_q5_0(b):
    d = _h16(b[0:2])
    qh = int.from_bytes(bytes(b[2:6]), "little")
    qs = [int(v) for v in b[6:22]]
    y = np.zeros(32)
    for j in range(16):
        xh_0 = ((qh >> (j + 0)) << 4) & 0x10
        xh_1 = (qh >> (j + 12)) & 0x10
        y[j] = (((qs[j] & 0x0F) | xh_0) - 16) * d
        y[j + 16] = (((qs[j] >> 4) | xh_1) - 16) * d
    return y


def _ggml_q5_1(b):
    d, m = _h16(b[0:2]), _h16(b[2:4])
    qh = int.from_bytes(bytes(b[4:8]), "little")
    qs = [int(v) for v in b[8:24]]
    y = np.zeros(32)
    for j in range(16):
        xh_0 = ((qh >> (j + 0)) << 4) & 0x10
        xh_1 = (qh >> (j + 12)) & 0x10
        y[j] = ((qs[j] & 0x0F) | xh_0) * d + m
        y[j + 16] = ((qs[j] >> 4) | xh_1) * d + m
    return y


def _ggml_q5_k(b):
    d, dmin = _h16(b[0:2]), _h16(b[2:4])
    scales = [int(v) for v in b[4:16]]
    qh = [int(v) for v in b[16:48]]
    ql = [int(v) for v in b[48:176]]
    y = np.zeros(256)
    o, is_, u1, u2 = 0, 0, 1, 2
    for j in range(0, 256, 64):
        sc, m = _ggml_scale_min_k4(is_ + 0, scales)
        d1, m1 = d * sc, dmin * m
        sc, m = _ggml_scale_min_k4(is_ + 1, scales)
        d2, m2 = d * sc, dmin * m
        for l in range(32):
            y[j + l] = d1 * ((ql[o + l] & 0xF) + (16 if qh[l] & u1 else 0)) - m1
        for l in range(32):
            y[j + 32 + l] = d2 * ((ql[o + l] >> 4) + (16 if qh[l] & u2 else 0)) - m2
        o += 32
        is_ += 2
        u1 <<= 2
        u2 <<= 2
    return y


def _ggml_q2_k(b):
    scales = [int(v) for v in b[0:16]]
    q = [int(v) for v in b[16:80]]
    d, dmin = _h16(b[80:82]), _h16(b[82:84])
    y, yi, is_ = np.zeros(256), 0, 0
    for n in range(2):
        qq = q[32 * n:]
        shift = 0
        for _ in range(4):
            sc = scales[is_]
            is_ += 1
            dl, ml = d * (sc & 0xF), dmin * (sc >> 4)
            for l in range(16):
                y[yi] = dl * ((qq[l] >> shift) & 3) - ml
                yi += 1
            sc = scales[is_]
            is_ += 1
            dl, ml = d * (sc & 0xF), dmin * (sc >> 4)
            for l in range(16):
                y[yi] = dl * ((qq[l + 16] >> shift) & 3) - ml
                yi += 1
            shift += 2
    return y


def _ggml_q3_k(b):
    hm = [int(v) for v in b[0:32]]
    q = [int(v) for v in b[32:96]]
    aux = [int.from_bytes(bytes(b[96 + 4 * i:100 + 4 * i]), "little") for i in range(3)] + [0]
    d_all = _h16(b[108:110])
    kmask1, kmask2 = 0x03030303, 0x0F0F0F0F
    tmp = aux[2]
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4)
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4)
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4)
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4)
    scales = np.array(aux, dtype="<u4").view(np.int8).astype(int)
    y, yi, is_, m = np.zeros(256), 0, 0, 1
    for n in range(2):
        qq = q[32 * n:]
        shift = 0
        for _ in range(4):
            dl = d_all * (scales[is_] - 32)
            is_ += 1
            for l in range(16):
                y[yi] = dl * (((qq[l] >> shift) & 3) - (0 if hm[l] & m else 4))
                yi += 1
            dl = d_all * (scales[is_] - 32)
            is_ += 1
            for l in range(16):
                y[yi] = dl * (((qq[l + 16] >> shift) & 3) - (0 if hm[l + 16] & m else 4))
                yi += 1
            shift += 2
            m <<= 1
    return y


# type -> (loop form, byte offsets of the fp16 fields, magnitude bound of a
# block's terms in units of its fp16 fields: (field offset, bound))
_LOOP_FORMS = {
    O.TYPE_Q4_0: (_ggml_q4_0, [(0, 8)]),
    O.TYPE_Q4_1: (_ggml_q4_1, [(0, 15), (2, 1)]),
    O.TYPE_Q5_0: (_ggml_q5_0, [(0, 16)]),
    O.TYPE_Q5_1: (_ggml_q5_1, [(0, 31), (2, 1)]),
    O.TYPE_Q5_K: (_ggml_q5_k, [(0, 63 * 31), (2, 63)]),
    O.TYPE_Q2_K: (_ggml_q2_k, [(80, 15 * 3), (82, 15)]),
    O.TYPE_Q3_K: (_ggml_q3_k, [(108, 32 * 4)]),
}


@pytest.mark.parametrize("qtype", sorted(_LOOP_FORMS))
def test_gguf_types_against_ggml_loop_forms(qtype):
    """Oracle decode of Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q5_K / Q2_K / Q3_K equals
    ggml's published loop form on random blocks (every bit pattern of the
    codes, scales and fifth / third bits), with finite random fp16 fields."""
    form, fields = _LOOP_FORMS[qtype]
    qk, bs = O.BLOCK_ELEMS[qtype], O.BLOCK_BYTES[qtype]
    rng = np.random.default_rng(1000 + qtype)
    for _ in range(24):
        blk = rng.integers(0, 256, bs, dtype=np.uint8)
        for off, _bound in fields:
            blk[off:off + 2] = np.frombuffer(np.float16(rng.uniform(-2, 2)).tobytes(), np.uint8)
        got = O.dequantize(blk.reshape(1, -1), qk, qtype).ravel()
        want = form(blk)
        scale = sum(abs(_h16(blk[off:off + 2])) * bound for off, bound in fields)
        assert _ulp_ok(got, want, scale), (qtype, np.flatnonzero(np.abs(got - want) > scale * 2.0 ** -20)[:8])


@pytest.mark.parametrize("qtype", sorted(_LOOP_FORMS))
def test_ggml_loop_forms_detect_a_moved_bit(qtype):
    """The comparison has teeth: decoding a block whose codes were changed
    in one byte differs from the loop form of the original block."""
    form, fields = _LOOP_FORMS[qtype]
    qk, bs = O.BLOCK_ELEMS[qtype], O.BLOCK_BYTES[qtype]
    rng = np.random.default_rng(2000 + qtype)
    blk = rng.integers(0, 256, bs, dtype=np.uint8)
    for off, _bound in fields:
        blk[off:off + 2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    fp16_bytes = {off + i for off, _ in fields for i in (0, 1)}
    byte = next(i for i in range(bs - 1, -1, -1) if i not in fp16_bytes)
    moved = blk.copy()
    moved[byte] ^= 0x11
    got = O.dequantize(moved.reshape(1, -1), qk, qtype).ravel()
    scale = sum(bound for _off, bound in fields)
    assert not _ulp_ok(got, form(blk), scale)


# ---- Q8_0 ----------------------------------------------------------------------

def _q8_block(d, q):
    return np.frombuffer(struct.pack("<e", d) + np.asarray(q, np.int8).tobytes(), np.uint8)


def test_q8_0_closed_forms():
    q = np.arange(-16, 16, dtype=np.int8)
    y = O.dequantize(_q8_block(1.0, q).reshape(1, -1), 32, O.TYPE_Q8_0).ravel()
    assert np.array_equal(y, q.astype(np.float32))
    y = O.dequantize(_q8_block(0.0, q).reshape(1, -1), 32, O.TYPE_Q8_0).ravel()
    assert np.all(y == 0.0)


def test_q8_0_loader_semantics():
    """vibeblade/loader.py:129-133: fp16 scale at [0:2], int8 at [2:34]."""
    rng = np.random.default_rng(5)
    blocks = rng.integers(0, 256, (40, 34), dtype=np.uint8)
    blocks[:, 0:2] = np.frombuffer(np.float16(rng.uniform(-2, 2, 40)).tobytes(), np.uint8).reshape(40, 2)
    want = np.concatenate([
        np.frombuffer(b[2:34].tobytes(), np.int8).astype(np.float32)
        * np.frombuffer(b[:2].tobytes(), np.float16).astype(np.float32)[0] for b in blocks])
    got = O.dequantize(blocks.reshape(1, -1), 40 * 32, O.TYPE_Q8_0).ravel()
    assert np.array_equal(bits(got), bits(want))


# ---- quantizers ------------------------------------------------------------------

@pytest.mark.parametrize("qtype,tol", [(O.TYPE_Q8_0, 0.01), (O.TYPE_Q4_K, 0.12), (O.TYPE_Q6_K, 0.03)])
def test_quantizer_roundtrip(qtype, tol):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    wq = O.quantize(w, qtype)
    assert wq.shape == (8, O.row_bytes(qtype, 1024))
    back = O.dequantize(wq, 1024, qtype)
    assert O.rel_l2(back, w) < tol


def test_quantized_q4k_decodes_identically_in_reference():
    if not O.ref_available():
        pytest.skip("compiled reference not built (no reference tree)")
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((4, 2048)) * 0.02).astype(np.float32)
    wq = O.quantize(w, O.TYPE_Q4_K)
    mine = O.dequantize(wq, 2048, O.TYPE_Q4_K).ravel()
    ref = O.ref_dequantize(wq.ravel(), 4 * 2048, O.TYPE_Q4_K)
    assert np.array_equal(bits(mine), bits(ref))


# ---- products ----------------------------------------------------------------------

def _integer_matrix(qtype, rows, k, rng):
    """GGUF bytes whose decoded values are known integers, plus those values."""
    if qtype == O.TYPE_Q8_0:
        q = rng.integers(-127, 128, (rows, k)).astype(np.int8)
        raw = b"".join(_q8_block(1.0, q[r, 32 * i:32 * i + 32]).tobytes()
                       for r in range(rows) for i in range(k // 32))
        return np.frombuffer(raw, np.uint8).reshape(rows, -1), q.astype(np.float64)
    if qtype == O.TYPE_Q4_K:
        nib = rng.integers(0, 16, (rows, k))
        out = []
        for r in range(rows):
            for s in range(k // 256):
                blk = nib[r, 256 * s:256 * s + 256]
                qs = [(blk[64 * c + l] | (blk[64 * c + 32 + l] << 4)) for c in range(4) for l in range(32)]
                out.append(_q4k_unit_block(qs).tobytes())
        return np.frombuffer(b"".join(out), np.uint8).reshape(rows, -1), nib.astype(np.float64)
    raise ValueError(qtype)


@pytest.mark.parametrize("qtype", [O.TYPE_Q8_0, O.TYPE_Q4_K])
def test_gemv_gemm_brute_force(qtype):
    rng = np.random.default_rng(9)
    rows, k = 6, 512
    wq, wint = _integer_matrix(qtype, rows, k, rng)
    assert np.array_equal(O.dequantize(wq, k, qtype), wint.astype(np.float32))
    x = rng.standard_normal((3, k)).astype(np.float32)
    want = x.astype(np.float64) @ wint.T
    assert np.allclose(O.gemv(wq, x[0], rows, k, qtype), want[0], rtol=1e-6, atol=1e-6)
    assert np.allclose(O.gemm(wq, x, rows, k, qtype), want, rtol=1e-6, atol=1e-6)


def test_gemv_kn_restates_reference_loop(gold):
    K, N = (int(v) for v in gold["kn_shape"])
    got = O.gemv_kn(gold["kn_x"], gold["kn_w"], K, N, O.TYPE_Q4_K)
    assert np.allclose(got, gold["kn_out"], rtol=1e-6, atol=1e-7)


# ---- FFN compositions -----------------------------------------------------------------

def _ffn_weights(rng, H=64, I=256):
    g = (rng.standard_normal((I, H)) * 0.1).astype(np.float32)
    u = (rng.standard_normal((I, H)) * 0.1).astype(np.float32)
    d = (rng.standard_normal((H, I)) * 0.1).astype(np.float32)
    return g, u, d


@pytest.mark.parametrize("act", [O.ACT_SILU, O.ACT_DRELU])
def test_sparse_ffn_invariants(act):
    rng = np.random.default_rng(12)
    g, u, d = _ffn_weights(rng)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    x64 = x.astype(np.float64)
    gd, ud = x64 @ g.T.astype(np.float64), x64 @ u.T.astype(np.float64)
    h = O.silu64(gd) * ud if act == O.ACT_SILU else np.maximum(gd, 0) * np.maximum(ud, 0)
    dense = h @ d.T.astype(np.float64)
    allidx = np.arange(256)
    assert np.allclose(O.sparse_ffn(g, u, d, x, allidx, act), dense, rtol=1e-12, atol=1e-12)
    assert np.all(O.sparse_ffn(g, u, d, x, np.array([], np.int64), act) == 0)
    s = np.sort(rng.choice(256, 40, replace=False))
    masked = (h * np.isin(allidx, s)) @ d.T.astype(np.float64)
    assert np.allclose(O.sparse_ffn(g, u, d, x, s, act), masked, rtol=1e-12, atol=1e-12)
    assert np.allclose(O.sparse_ffn(g, u, d, x, s[::-1], act), masked, rtol=1e-12, atol=1e-12)


def test_moe_invariants():
    rng = np.random.default_rng(13)
    E, H, I, T = 4, 32, 64, 6
    gates = [(rng.standard_normal((I, H)) * 0.1).astype(np.float32) for _ in range(E)]
    ups = [(rng.standard_normal((I, H)) * 0.1).astype(np.float32) for _ in range(E)]
    downs = [(rng.standard_normal((H, I)) * 0.1).astype(np.float32) for _ in range(E)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    y, idx, w = O.moe_ffn(gates, ups, downs, x, logits, 2)
    assert np.allclose(w.sum(axis=1), 1.0)
    assert np.all(idx[:, 0] != idx[:, 1])
    # every token routed to expert 2 first and expert 0 second
    logits2 = np.full((T, E), -5.0, np.float32)
    logits2[:, 2], logits2[:, 0] = 3.0, 1.0
    y2, idx2, w2 = O.moe_ffn(gates, ups, downs, x, logits2, 2)
    x64 = x.astype(np.float64)

    def ffn(e):
        return (O.silu64(x64 @ gates[e].T) * (x64 @ ups[e].T)) @ downs[e].T.astype(np.float64)
    assert np.allclose(y2, w2[:, :1] * ffn(2) + w2[:, 1:] * ffn(0), rtol=1e-12)
    # relabelling experts relabels the routing consistently
    perm = np.array([3, 1, 0, 2])
    y3, idx3, _ = O.moe_ffn([gates[p] for p in perm], [ups[p] for p in perm],
                            [downs[p] for p in perm], x, logits[:, perm], 2)
    assert np.allclose(y3, y, rtol=1e-12)
    assert np.array_equal(perm[idx3], idx)
    # grouped per expert (the bench's form for full-size experts) = per-token loop
    calls = []

    def expert(e):
        calls.append(e)
        return gates[e], ups[e], downs[e]
    yg, idxg, wg = O.moe_ffn_grouped(expert, x, logits, 2)
    assert np.array_equal(idxg, idx) and np.array_equal(wg, w)
    assert np.allclose(yg, y, rtol=1e-12, atol=1e-14)
    assert sorted(calls) == sorted(set(idx.ravel().tolist())) and len(calls) == len(set(calls))


def test_rms_norm_closed_forms():
    w = np.linspace(-2.0, 3.0, 8)
    # constant row, eps = 0: x / |x| * w
    assert np.allclose(O.rms_norm(np.full(8, -3.5), w, 0.0), -w, rtol=0, atol=1e-15)
    # x = (3, 4): mean square 12.5 (a sum instead of a mean, or a product
    # instead of a quotient, fails here)
    got = O.rms_norm(np.array([3.0, 4.0]), np.array([1.0, 2.0]), 0.0)
    assert np.allclose(got, [3.0 / np.sqrt(12.5), 8.0 / np.sqrt(12.5)], rtol=1e-15)
    # eps enters under the root: x = 0 stays finite, eps = mean square halves the scale^2
    assert np.all(O.rms_norm(np.zeros(8), w, 1e-5) == 0.0)
    x = np.array([1.0, -1.0, 1.0, -1.0])
    assert np.allclose(O.rms_norm(x, np.ones(4), 1.0), x / np.sqrt(2.0), rtol=1e-15)
    # scale invariance at eps = 0
    rng = np.random.default_rng(3)
    v = rng.standard_normal(64)
    assert np.allclose(O.rms_norm(1e3 * v, np.ones(64), 0.0), O.rms_norm(v, np.ones(64), 0.0), rtol=1e-12)


def test_activation_forms():
    g = np.array([-30.0, -2.0, -0.5, 0.0, 0.5, 1.0, 2.0, 30.0])
    # GeGLU (tanh form): published value gelu_tanh(1) = 0.8411919906..., zero at 0, identity far right
    assert abs(O.gelu_tanh64(np.array([1.0]))[0] - 0.8411919906082768) < 1e-12
    z = 0.7978845608 * (g + 0.044715 * g ** 3)
    with np.errstate(over="ignore"):  # exp(1972) at g = -30: the quotient is -0
        assert np.allclose(O.gelu_tanh64(g), g / (1.0 + np.exp(-2.0 * z)), rtol=1e-13, atol=1e-300)
    assert O.gelu_tanh64(np.array([0.0]))[0] == 0.0 and abs(O.gelu_tanh64(np.array([30.0]))[0] - 30.0) < 1e-12
    u = np.full_like(g, 3.0)
    assert np.allclose(O.act_pair(g, u, O.ACT_SILU), 3.0 * g / (1.0 + np.exp(-g)), rtol=1e-15)
    assert np.array_equal(O.act_pair(g, -u, O.ACT_DRELU), np.zeros_like(g))
    assert np.array_equal(O.act_pair(g, u, O.ACT_DRELU), 3.0 * np.maximum(g, 0.0))


@pytest.mark.parametrize("act", [O.ACT_SILU, O.ACT_DRELU, O.ACT_GELU_TANH])
def test_ffn_block_composition(act):
    """No norm, no residual: the dense FFN = sparse_ffn over every neuron;
    the residual adds x; the norm feeds rms_norm(x) to the same FFN."""
    rng = np.random.default_rng(14)
    g, u, d = _ffn_weights(rng)
    x = rng.standard_normal(64)
    nw = rng.standard_normal(64)
    allidx = np.arange(256)
    plain = O.ffn_block(g, u, d, x, None, 0.0, act, False)
    assert np.allclose(plain, O.sparse_ffn(g, u, d, x, allidx, act)[0], rtol=1e-12, atol=1e-14)
    assert np.allclose(O.ffn_block(g, u, d, x, None, 0.0, act, True) - x, plain, rtol=1e-12, atol=1e-14)
    normed = O.ffn_block(g, u, d, x, nw, 1e-5, act, True)
    want = x + O.sparse_ffn(g, u, d, O.rms_norm(x, nw, 1e-5), allidx, act)[0]
    assert np.allclose(normed, want, rtol=1e-12, atol=1e-14)


def test_ema_update_known_answers():
    """tests/test_ema_neuron.py:84-97 of the reference (decay), and the closed
    form p_t = 1 - (1 - a)^t for an always-on neuron, 0 for a never-on one."""
    p = np.zeros(128, np.float32)
    mask = np.zeros(128, bool)
    mask[:10] = True
    for _ in range(10):
        p = O.ema_update(p, mask, 0.1)
    assert p[0] > 0.5 and p[50] < 0.01
    assert abs(float(p[0]) - (1 - 0.9 ** 10)) < 1e-6 and p[50] == 0.0
    # one step from p = 1 with the neuron off: 1 - a
    q = O.ema_update(np.ones(4, np.float32), np.zeros(4, bool), 0.25)
    assert np.all(q == np.float32(0.75))


def test_ema_predict_known_answers():
    """The reference's tests/test_ema_neuron.py:99-152 cases."""
    n = 128
    k = max(1, int(n * 0.1))
    m = O.ema_predict(np.zeros(n), k, 0.3, warm=False)  # cold, no gate: first k
    assert m.sum() == 12 and m[:12].all()
    gate = np.random.default_rng(0).standard_normal(32).astype(np.float32)
    gate[5] = 100.0
    assert O.ema_predict(np.zeros(32), 3, 0.3, warm=False, gate=gate)[5]
    p = np.zeros(64, np.float32)
    mk = np.zeros(64, bool)
    mk[:16] = True
    for _ in range(10):
        p = O.ema_update(p, mk, 0.1)
    warm = O.ema_predict(p, 16, 0.2, warm=True)
    assert warm[:16].all()
    g2 = np.zeros(64, np.float32)
    g2[50] = 100.0
    comb = O.ema_predict(p, 6, 0.3, warm=True, gate=g2, combined=True)
    assert comb[50] and comb[:6].all()


def test_ema_predict_brute_force():
    """Tiny inputs against an exhaustive reading of the rule: the threshold
    set, topped up with the largest remaining probabilities (ties: lowest
    index), has max(k, |{p >= thr}|) members and contains every p >= thr."""
    rng = np.random.default_rng(9)
    for _ in range(200):
        n = int(rng.integers(1, 12))
        k = int(rng.integers(1, n + 1))
        p = rng.choice(np.array([0.0, 0.1, 0.25, 0.5, 0.75], np.float32), n)
        thr = float(rng.choice([0.1, 0.3, 0.6]))
        m = O.ema_predict(p, k, thr, warm=True)
        above = p >= np.float32(thr)
        assert m[above].all() and m.sum() == max(k, int(above.sum()))
        # every unselected neuron is below every selected one below the threshold,
        # and among equals the selected ones come first
        sel_below = np.flatnonzero(m & ~above)
        unsel = np.flatnonzero(~m)
        for a in sel_below:
            for b in unsel:
                assert p[a] > p[b] or (p[a] == p[b] and a < b)


# ---- Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q5_K / BF16 (GGUF layouts) -------------------

_BLK = {O.TYPE_Q4_0: 18, O.TYPE_Q4_1: 20, O.TYPE_Q5_0: 22, O.TYPE_Q5_1: 24, O.TYPE_Q5_K: 176}


def _rand_blocks(qtype, nblk, rng, zero_qh=False):
    """Random blocks with normal (non-subnormal, finite) fp16 scales."""
    b = rng.integers(0, 256, (nblk, _BLK[qtype]), dtype=np.uint8)
    scale_offs = {O.TYPE_Q4_0: [0], O.TYPE_Q4_1: [0, 2], O.TYPE_Q5_0: [0], O.TYPE_Q5_1: [0, 2],
                  O.TYPE_Q5_K: [0, 2]}[qtype]
    for o in scale_offs:
        b[:, o + 1] = (b[:, o + 1] & 0x83) | 0x28  # exponent 10..13: normal, modest
    if zero_qh:
        qh = {O.TYPE_Q5_0: (2, 6), O.TYPE_Q5_1: (4, 8), O.TYPE_Q5_K: (16, 48)}[qtype]
        b[:, qh[0]:qh[1]] = 0
    return b


@pytest.mark.parametrize("qtype,zero_qh", [(O.TYPE_Q4_0, False), (O.TYPE_Q4_1, False), (O.TYPE_Q5_0, True),
                                           (O.TYPE_Q5_1, True)])
def test_32_element_types_against_reference_order(qtype, zero_qh):
    """The compiled reference decodes the same values with interleaved
    nibbles (cpp/src/dequant.cpp:23-94): GGUF element j = its element 2j,
    GGUF element j + 16 = its element 2j + 1 (with qh = 0 for the 5-bit
    types, whose fifth bits the two assign differently)."""
    if not O.ref_available():
        pytest.skip("compiled reference not built")
    rng = np.random.default_rng(qtype)
    blocks = _rand_blocks(qtype, 64, rng, zero_qh)
    mine = O.dequantize(blocks.reshape(1, -1), 64 * 32, qtype).reshape(64, 32)
    ref = O.ref_dequantize(blocks.reshape(-1), 64 * 32, qtype).reshape(64, 32)
    assert np.array_equal(mine[:, :16], ref[:, 0::2]) and np.array_equal(mine[:, 16:], ref[:, 1::2])


@pytest.mark.parametrize("qtype", [O.TYPE_Q5_0, O.TYPE_Q5_1])
def test_5bit_types_fifth_bit_map(qtype):
    """d = 1 (m = 0), all nibbles 0, one qh bit e set: only element e moves,
    by exactly 16 (q - 16 for Q5_0: -16 -> 0; d q + m for Q5_1: 0 -> 16)."""
    qh_off = 2 if qtype == O.TYPE_Q5_0 else 4
    base = -16.0 if qtype == O.TYPE_Q5_0 else 0.0
    for e in range(32):
        b = np.zeros(_BLK[qtype], np.uint8)
        b[0:2] = [0x00, 0x3C]  # fp16 1.0
        b[qh_off:qh_off + 4] = np.frombuffer(np.uint32(1 << e).tobytes(), np.uint8)
        y = O.dequantize(b.reshape(1, -1), 32, qtype)[0]
        want = np.full(32, base, np.float32)
        want[e] = base + 16.0
        assert np.array_equal(y, want), e
    # closed forms of the nibbles: Q4_0 with d = 2, qs[j] = j | (15 - j) << 4
    b = np.zeros(18, np.uint8)
    b[0:2] = [0x00, 0x40]  # fp16 2.0
    b[2:] = [j | ((15 - j) << 4) for j in range(16)]
    y = O.dequantize(b.reshape(1, -1), 32, O.TYPE_Q4_0)[0]
    assert np.array_equal(y, 2.0 * np.array([j - 8 for j in range(16)] + [7 - j for j in range(16)], np.float32))


def test_q5k_with_zero_qh_is_q4k_and_bit_map():
    """A Q5_K block with qh = 0 decodes as the Q4_K block with the same d,
    dmin, scales and qs (Q4_K is pinned by the reference's golden vectors);
    each qh bit adds 16 d sc to exactly one element: bit 2c of qh[l] to
    element 64 c + l, bit 2c + 1 to element 64 c + 32 + l."""
    rng = np.random.default_rng(5)
    q5 = _rand_blocks(O.TYPE_Q5_K, 32, rng, zero_qh=True)
    q4 = np.concatenate([q5[:, :16], q5[:, 48:]], axis=1)
    assert np.array_equal(O.dequantize(q5.reshape(1, -1), 32 * 256, O.TYPE_Q5_K),
                          O.dequantize(q4.reshape(1, -1), 32 * 256, O.TYPE_Q4_K))
    blk = q5[0].copy()
    blk[0:2] = [0x00, 0x3C]  # d = 1
    blk[2:4] = 0  # dmin = 0
    blk[4:16] = 0
    blk[4:8] = 1  # scales[0..3]: sub-blocks 0..3 scale 1 (their mins, scales[4..7], stay 0)
    blk[12:16] = 1  # scales[8..11]: sub-blocks 4..7 scale 1 (low nibble), min 0 (high nibble)
    base = O.dequantize(blk.reshape(1, -1), 256, O.TYPE_Q5_K)[0]
    for l in (0, 7, 31):
        for bit in range(8):
            b2 = blk.copy()
            b2[16 + l] = 1 << bit
            y = O.dequantize(b2.reshape(1, -1), 256, O.TYPE_Q5_K)[0]
            e = 64 * (bit // 2) + 32 * (bit % 2) + l
            diff = np.flatnonzero(y != base)
            assert list(diff) == [e] and y[e] - base[e] == 16.0, (l, bit)
    if O.ref_available():  # the reference's first group (qh = 0) agrees
        ref = O.ref_dequantize(q5[:4].reshape(-1), 4 * 256, O.TYPE_Q5_K).reshape(4, 256)
        mine = O.dequantize(q5[:4].reshape(1, -1), 4 * 256, O.TYPE_Q5_K).reshape(4, 256)
        assert np.array_equal(mine[:, :64], ref[:, :64])


def test_bf16_closed_form():
    v = np.array([1.0, -2.5, 3.0e38, 1e-40, 0.0, -0.0], np.float32)
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    y = O.dequantize(bf.view(np.uint8).reshape(1, -1), 6, O.TYPE_BF16)[0]
    assert np.array_equal(y.view(np.uint32), bf.astype(np.uint32) << 16)


def _f16(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def test_q2k_code_and_scale_maps():
    """GGUF Q2_K: element 128 h + 32 j + l = code bits 2j of qs[32 h + l],
    sub-block e / 16 scale (low nibble) and min (high nibble)."""
    base = np.zeros(84, np.uint8)
    base[80:82] = _f16(1.0)
    base[0:16] = 0x01  # scale 1, min 0
    for byte in range(64):
        for j in range(4):
            b = base.copy()
            b[16 + byte] = 1 << (2 * j)
            y = O.dequantize(b.reshape(1, -1), 256, O.TYPE_Q2_K)[0]
            e = 128 * (byte // 32) + 32 * j + byte % 32
            assert list(np.flatnonzero(y)) == [e] and y[e] == 1.0, (byte, j)
    b = base.copy()
    b[16:80] = 0xFF  # every code 3
    b[82:84] = _f16(0.5)  # dmin
    b[0:16] = [((i % 15) + 1) | ((i % 16) << 4) for i in range(16)]
    y = O.dequantize(b.reshape(1, -1), 256, O.TYPE_Q2_K)[0]
    want = np.repeat([3.0 * ((i % 15) + 1) - 0.5 * (i % 16) for i in range(16)], 16).astype(np.float32)
    assert np.array_equal(y, want)


def test_q3k_code_hmask_and_scale_maps():
    """GGUF Q3_K: code bits 2j of qs[32 h + l], third bit = bit 4h + j of
    hmask[l] (clear: minus 4), 6-bit scales minus 32, each field moving exactly
    its own element or sub-block."""
    base = np.zeros(110, np.uint8)
    base[108:110] = _f16(1.0)
    base[96:104] = 0x11  # low 4 bits of every scale = 1
    base[104:108] = 0xAA  # high 2 bits = 2: every scale 33 - 32 = 1
    base[0:32] = 0xFF  # every third bit set: q = code
    y0 = O.dequantize(base.reshape(1, -1), 256, O.TYPE_Q3_K)[0]
    assert np.all(y0 == 0.0)
    for byte in range(64):
        for j in range(4):
            b = base.copy()
            b[32 + byte] = 1 << (2 * j)
            y = O.dequantize(b.reshape(1, -1), 256, O.TYPE_Q3_K)[0]
            e = 128 * (byte // 32) + 32 * j + byte % 32
            assert list(np.flatnonzero(y)) == [e] and y[e] == 1.0, (byte, j)
    for l in range(32):
        for bit in range(8):
            b = base.copy()
            b[l] &= ~np.uint8(1 << bit)
            y = O.dequantize(b.reshape(1, -1), 256, O.TYPE_Q3_K)[0]
            e = 128 * (bit // 4) + 32 * (bit % 4) + l
            assert list(np.flatnonzero(y)) == [e] and y[e] == -4.0, (l, bit)
    ones = base.copy()
    ones[32:96] = 0x55  # every code 1: y = scale - 32 per sub-block
    def sub_scales(b):
        return O.dequantize(b.reshape(1, -1), 256, O.TYPE_Q3_K)[0].reshape(16, 16)[:, 0]
    assert np.all(sub_scales(ones) == 1.0)
    for i in range(16):  # the low 4 bits of scale i: byte i (i < 8) or the high nibble of byte i - 8
        b = ones.copy()
        b[96 + (i % 8)] = (0x12 if i < 8 else 0x21)
        want = np.ones(16, np.float32)
        want[i] = 2.0
        assert np.array_equal(sub_scales(b), want), i
    for t in range(4):  # the high 2 bits of scale 4 t + m: bits 2t of byte 8 + m
        for m in range(4):
            b = ones.copy()
            b[104 + m] = 0xAA ^ (0b11 << (2 * t))  # 2 -> 1: scale 17 - 32 = -15
            want = np.ones(16, np.float32)
            want[4 * t + m] = -15.0
            assert np.array_equal(sub_scales(b), want), (t, m)
