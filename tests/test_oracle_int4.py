"""Pins the oracle's INT4 restatement (crates/haagenti/src/testing/quantization.rs).

Known answers are computed by hand in the comments; the f16 decoder is
checked against numpy's float16 conversion (a library routine) for all
65,536 codes.
"""
import numpy as np
import pytest

import oracle_lib as O


def test_compressed_size_reference_assertions():
    # quantization.rs:290-300
    assert O.int4_compressed_size(32) == 18
    assert O.int4_compressed_size(64) == 36
    assert O.int4_compressed_size(33) == 21
    assert O.int4_compressed_size(0) == 0
    assert O.int4_compressed_size(10000) == 626 + 5000


def test_single_block_all_ones():
    # scale = 1/7 f32 = 0x3E124925 -> f16 exp 12, frac 0x124925>>13 = 0x92
    q = O.quantize_int4(np.ones(32, np.float32))
    assert len(q) == 18
    assert q[:2] == bytes([0x92, 0x30])
    assert q[2:] == b"\xff" * 16  # q = 7 -> nibble 15 everywhere
    d = O.dequantize_int4(q, 32)
    # 0x3092 = 2^-3 * (1 + 146/1024) = 0.142822265625; 7 * that:
    assert (d == np.float32(0.999755859375)).all()


def test_scale_is_truncated_not_rounded():
    # max_abs = 7*(1+3/4096) -> scale = 1+3/4096 exactly; its f16 mantissa
    # bits 3<<11 are cut by >>13 -> 0x3C00 (RNE would give 0x3C01).
    w = np.zeros(32, np.float32)
    w[0] = 7.005126953125
    q = O.quantize_int4(w)
    assert q[:2] == bytes([0x00, 0x3C])
    assert q[2] == 0x8F and q[3:] == b"\x88" * 15
    d = O.dequantize_int4(q, 32)
    assert d[0] == np.float32(7.0) and (d[1:] == 0).all()
    assert np.float16(np.float32(1.000732421875)).view(np.uint16) == 0x3C01  # RNE differs


def test_round_half_away_from_zero():
    # scale = 7/7 = 1.0 exactly (f16 0x3C00); q = round(v) half away from 0.
    w = np.zeros(32, np.float32)
    w[:8] = [7.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5]
    q = O.quantize_int4(w)
    assert q[:2] == bytes([0x00, 0x3C])
    # nibbles 15,11 | 5,9 | 7,10 | 6,12 | 8...
    assert q[2:6] == bytes([0xBF, 0x95, 0xA7, 0xC6])
    assert q[6:] == b"\x88" * 12
    d = O.dequantize_int4(q, 32)
    assert list(d[:8]) == [7.0, 3.0, -3.0, 1.0, -1.0, 2.0, -2.0, 4.0]


def test_tiny_block_scale_one():
    w = np.full(32, 1e-11, np.float32)
    q = O.quantize_int4(w)
    assert q[:2] == bytes([0x00, 0x3C]) and q[2:] == b"\x88" * 16


def test_odd_tail_low_nibble_only():
    w = np.zeros(33, np.float32)
    w[32] = -1.0  # block 2: scale 1/7 -> q = -7 -> nibble 1
    q = O.quantize_int4(w)
    assert len(q) == 21
    assert q[-1] == 0x01
    d = O.dequantize_int4(q, 33)
    assert d.size == 33 and d[32] == np.float32(-7 * 0.142822265625)


def test_empty_and_short_inputs():
    assert O.quantize_int4(np.zeros(0, np.float32)) == b""
    assert O.dequantize_int4(b"", 0).size == 0
    assert O.dequantize_int4(b"\x00\x3c", 64).size == 0  # shorter than the scales
    # 64 elements, 4 scale bytes, only 10 nibble bytes -> stops after 20
    d = O.dequantize_int4(b"\x00\x3c\x00\x3c" + b"\x9a" * 10, 64)
    assert d.size == 20 and (d[0::2] == 2.0).all() and (d[1::2] == 1.0).all()


def test_reference_roundtrip_tolerance_and_sign():
    # quantization.rs:229-249, :334-355
    w = np.array([(i - 50.0) / 10.0 for i in range(100)], np.float32)
    d = O.dequantize_int4(O.quantize_int4(w), 100)
    assert (np.abs(w - d) < np.abs(w) * 0.15 + 0.1).all()
    d = O.dequantize_int4(O.quantize_int4(np.array([-5.0, 5.0, -2.5, 2.5], np.float32)), 4)
    assert d[0] < 0 < d[1] and d[2] < 0 < d[3]
    assert (np.abs(O.dequantize_int4(O.quantize_int4(np.zeros(64, np.float32)), 64)) < 1e-6).all()


def test_f16_decoder_all_codes_vs_numpy():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mine = O.f16_bits_to_f32_bits(codes).view(np.float32)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert (mine.view(np.uint32)[~nan] == ref.view(np.uint32)[~nan]).all()
    # NaN codes keep their payload unquieted (quantization.rs:189-191):
    c = codes[nan].astype(np.uint32)
    exp = ((c & 0x8000) << 16) | 0x7F800000 | ((c & 0x3FF) << 13)
    assert (mine.view(np.uint32)[nan] == exp).all()


@pytest.mark.parametrize("v,h", [
    (1.0, 0x3C00), (-2.0, 0xC000), (0.5, 0x3800), (65504.0, 0x7BFF),
    (65520.0, 0x7BFF),        # truncation keeps 0x7BFF (RNE would overflow to inf)
    (70000.0, 0x7C00),        # overflow -> inf
    (1e-5, 0x0000),           # f16-subnormal range flushes to zero
    (-1e-5, 0x8000),
    (6.103515625e-05, 0x0400),  # smallest normal f16
    (float("inf"), 0x7C00), (float("-inf"), 0xFC00),
    (0.1, 0x2E66),
])
def test_f16_encoder_known_values(v, h):
    assert O.f32_to_f16_bits(v) == h


def test_f16_encoder_agrees_with_numpy_on_exact_values():
    # For values exactly representable in f16, truncation and RNE agree.
    codes = np.arange(0x0400, 0x7C00, 7, dtype=np.uint16)
    vals = codes.view(np.float16).astype(np.float32)
    assert all(O.f32_to_f16_bits(float(v)) == int(c) for v, c in zip(vals, codes))


def test_dequant_brute_force_all_bytes():
    # Every byte value x a spread of scale codes (normal, subnormal, zero).
    scale_codes = [0x3C00, 0x2E66, 0x0001, 0x03FF, 0x8400, 0x0000, 0x7BFF]
    for sc in scale_codes:
        data = bytes([sc & 0xFF, sc >> 8]) + bytes(range(256))[:16]
        for start in range(0, 256, 16):
            data = bytes([sc & 0xFF, sc >> 8]) + bytes(range(start, start + 16))
            d = O.dequantize_int4(data, 32)
            s = np.float32(np.array([sc], np.uint16).view(np.float16)[0])
            nib = np.array([[b & 15, b >> 4] for b in range(start, start + 16)]).ravel()
            exp = (nib.astype(np.float32) - np.float32(8)) * s
            assert (d.view(np.uint32) == exp.astype(np.float32).view(np.uint32)).all()


def test_dequant_mt_equals_serial():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, 100_003).astype(np.float32)
    q = O.quantize_int4(w)
    a = O.dequantize_int4(q, w.size)
    b = O.dequantize_int4(q, w.size, threads=4)
    assert (a.view(np.uint32) == b.view(np.uint32)).all()
