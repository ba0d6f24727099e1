"""Pins the oracle's block decoding and activation encodings.

The reference's ggml is absent, so the checks are: exhaustive comparison of the f16 conversion
with numpy's IEEE binary16; hand-built blocks whose decoded values follow from the GGUF layout
(wrong nibble order, sub-block index or scale packing fails them); quantize->dequantize round trips
through two independent implementations (the generator's quantizer and the oracle's decoder)
within each format's error bound; and quantized dot products against a float64 product.
"""
import numpy as np
import pytest

import oracle_py as O
from zonos2_amd import configs, synth
from zonos2_amd.lib import host_lib
import ctypes as C

L = O.lib()


def test_f16_decode_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(x)) for x in h], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000) * s for s in (1e-6, 1e-3, 1.0, 100.0, 3e4)]).astype(np.float32)
    # exact halfway cases between consecutive halves (round-to-even ties)
    hv = np.arange(0, 0x7bff, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    hn = (np.arange(0, 0x7bff, 97, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    x = np.concatenate([x, ((hv + hn) / 2).astype(np.float32), np.float32([65519.0, 65520.0, 1e-8, -0.0])])
    x = x[np.abs(x) < 65520.0]                      # numpy warns on the overflow to inf
    got = np.array([L.orc_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def _q4k_block(d, dmin, sc, mn, q):
    """GGUF Q4_K block from 8 scales/mins (6-bit) and 256 nibbles (element order)."""
    b = bytearray(144)
    b[0:2] = np.float16(d).tobytes()
    b[2:4] = np.float16(dmin).tobytes()
    for i in range(4):
        b[4 + i] = (sc[i] & 63) | ((sc[i + 4] >> 4) << 6)
        b[8 + i] = (mn[i] & 63) | ((mn[i + 4] >> 4) << 6)
        b[12 + i] = (sc[i + 4] & 15) | ((mn[i + 4] & 15) << 4)
    for p in range(4):
        for l in range(32):
            b[16 + 32 * p + l] = q[64 * p + l] | (q[64 * p + 32 + l] << 4)
    return np.frombuffer(bytes(b), np.uint8)


def test_q4k_known_answer():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, 256)
    sc = [1, 2, 3, 4, 17, 33, 49, 63]          # j >= 4 need the high bits stored in other bytes
    mn = [0, 5, 10, 15, 20, 40, 60, 63]
    blk = _q4k_block(0.5, 0.25, sc, mn, q)
    y = O.dequant(12, blk, 256)
    want = np.array([0.5 * sc[j // 32] * q[j] - 0.25 * mn[j // 32] for j in range(256)], np.float32)
    assert np.array_equal(y, want)


def test_q6k_known_answer():
    rng = np.random.default_rng(2)
    u = rng.integers(0, 64, 256)                  # stored 6-bit values, weight = sc * d * (u - 32)
    sc = rng.integers(-128, 128, 16)
    b = bytearray(210)
    for h in range(2):
        uh = u[128 * h:128 * h + 128]
        for l in range(32):
            b[64 * h + l] = (uh[l] & 15) | ((uh[l + 64] & 15) << 4)
            b[64 * h + l + 32] = (uh[l + 32] & 15) | ((uh[l + 96] & 15) << 4)
            b[128 + 32 * h + l] = (uh[l] >> 4) | ((uh[l + 32] >> 4) << 2) | ((uh[l + 64] >> 4) << 4) | ((uh[l + 96] >> 4) << 6)
    b[192:208] = np.int8(sc).tobytes()
    b[208:210] = np.float16(0.125).tobytes()
    y = O.dequant(14, np.frombuffer(bytes(b), np.uint8), 256)
    want = np.array([np.float32(0.125) * np.float32(sc[j // 16]) * np.float32(u[j] - 32) for j in range(256)], np.float32)
    assert np.array_equal(y, want)


def test_q8_0_known_answer():
    b = bytearray(34)
    b[0:2] = np.float16(0.0625).tobytes()
    q = np.arange(-16, 16, dtype=np.int8)
    b[2:34] = q.tobytes()
    y = O.dequant(8, np.frombuffer(bytes(b), np.uint8), 32)
    assert np.array_equal(y, q.astype(np.float32) * np.float32(0.0625))


@pytest.mark.parametrize("ttype,bound", [(8, 0.5 / 127), (12, 0.5 / 15 + 1.0 / 63), (14, 0.5 / 31 + 1.0 / 127)])
def test_quantize_dequantize_bound(ttype, bound):
    """Generator quantizer -> oracle decoder, error relative to the block's range."""
    rng = np.random.default_rng(ttype)
    n = 4096
    x = (rng.standard_normal(n) * 0.02).astype(np.float32)
    lib = host_lib()
    dst = np.empty(configs.row_bytes(ttype, n), np.uint8)
    assert lib.z2s_quantize(ttype, x.ctypes.data_as(C.c_void_p), dst.ctypes.data_as(C.c_void_p), 1, n, 1) == 0
    y = O.dequant(ttype, dst, n)
    blk = 32 if ttype == 8 else 256
    for b in range(n // blk):
        xs, ys = x[b * blk:(b + 1) * blk], y[b * blk:(b + 1) * blk]
        rng_ = float(np.abs(xs).max()) * 2
        assert np.abs(xs - ys).max() <= bound * rng_ + 1e-7, (ttype, b)


def test_q8k_activation_encoding():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(1024) * 3).astype(np.float32)
    x[300] = -50.0                                    # the block's extreme value is negative
    q = np.empty(1024, np.int8); d = np.empty(4, np.float32); bs = np.empty(64, np.int16)
    O.check(L.orc_quant_act(15, O.ptr(x), 1024, O.ptr(q), O.ptr(d), O.ptr(bs), None))
    for b in range(4):
        xb, qb = x[256 * b:256 * b + 256], q[256 * b:256 * b + 256].astype(np.int32)
        assert np.abs(qb).max() == 127
        assert np.abs(d[b] * qb - xb).max() <= abs(d[b]) * 0.5 + 1e-6
        assert np.array_equal(bs[16 * b:16 * b + 16], qb.reshape(16, 16).sum(1))
    # the extreme element always maps to -127 (iscale = -127 / x_max); the sign lives in d
    assert q[300] == -127 and d[1] > 0


@pytest.mark.parametrize("ttype", [1, 8, 12, 14])
def test_quantized_matmul_vs_float64(ttype):
    """orc_matmul on quantized weights vs float64 product of the dequantized weights."""
    rng = np.random.default_rng(ttype + 10)
    n_in, n_out, T = 512, 96, 3
    t = synth.generate_tensor(f"kat.{ttype}", ttype, (n_in, n_out), (0, 0.0, 0.02), seed=5)
    w = np.stack([O.dequant(ttype, t.data[r * configs.row_bytes(ttype, n_in):(r + 1) * configs.row_bytes(ttype, n_in)], n_in)
                  for r in range(n_out)]).astype(np.float64)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    y = O.matmul(ttype, t.data, n_in, n_out, x)
    ref = x.astype(np.float64) @ w.T
    # activation encoding error: Q8_K/Q8_0 relative step 1/254 per element, f16 2^-11
    rel = {1: 2e-3, 8: 2e-2, 12: 1e-2, 14: 1e-2}[ttype]
    assert np.abs(y - ref).max() <= rel * np.abs(x).max() * np.abs(w).sum(1).max()
    cos = (y * ref).sum() / np.sqrt((y * y).sum() * (ref * ref).sum())
    assert cos > 0.9999
