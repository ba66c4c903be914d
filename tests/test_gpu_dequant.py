"""INT4 dequant on the GPU vs the oracle (testing::dequantize_int4,
crates/haagenti/src/testing/quantization.rs:82-131): bit-exact f32, bf16/f16
equal to the round-to-nearest-even of that f32."""
import numpy as np
import pytest

import gpu_util as G
import oracle_lib as O

pytestmark = pytest.mark.gpu


def _run(q, n, dtype, offset=0):
    import haagenti_amd as H
    T = G.torch()
    q = np.frombuffer(bytes(q), np.uint8)
    buf = np.zeros(q.size + offset + 16, np.uint8)
    buf[offset:offset + q.size] = q
    dq = G.dev(buf)
    esz = 4 if dtype == H.F32 else 2
    out = T.zeros(max(n, 1) * esz + 64, dtype=T.uint8, device="cuda")
    produced = G.ctx().dequant_int4(dq.data_ptr() + offset, q.size, n, out, dtype=dtype,
                                    stream=G.stream())
    G.sync()
    raw = G.host_u8(out)
    if dtype == H.F32:
        return raw[:produced * 4].view(np.float32), produced
    return raw[:produced * 2].view(np.uint16), produced


def test_config1_4096x4096_bit_exact():
    import haagenti_amd as H
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, 4096 * 4096).astype(np.float32)
    q = O.quantize_int4(w)
    assert len(q) == 9_437_184
    ref = O.dequantize_int4(q, w.size, threads=8)
    got, m = _run(q, w.size, H.F32)
    assert m == w.size
    assert G.same_f32(got, ref)
    got16, _ = _run(q, w.size, H.BF16)
    assert (got16 == G.bf16_bits(ref)).all()
    goth, _ = _run(q, w.size, H.F16)
    assert (goth == G.f16_bits(ref)).all()


@pytest.mark.parametrize("n", [1, 2, 3, 7, 8, 31, 32, 33, 97, 255, 1000, 4099])
@pytest.mark.parametrize("offset", [0, 1, 2])
def test_ragged_sizes_and_misaligned_input(n, offset):
    import haagenti_amd as H
    rng = np.random.default_rng(n * 7 + offset)
    w = rng.normal(0, 1, n).astype(np.float32)
    q = O.quantize_int4(w)
    ref = O.dequantize_int4(q, n)
    for dt in (H.F32, H.BF16, H.F16):
        got, m = _run(q, n, dt, offset)
        assert m == n
        if dt == H.F32:
            assert G.same_f32(got, ref)
        elif dt == H.BF16:
            assert (got == G.bf16_bits(ref)).all()
        else:
            assert (got == G.f16_bits(ref)).all()


def test_short_data_stops_early_like_reference():
    import haagenti_amd as H
    q = b"\x00\x3c\x00\x3c" + b"\x9a" * 10        # 64 elements requested, 20 present
    got, m = _run(q, 64, H.F32)
    ref = O.dequantize_int4(q, 64)
    assert m == ref.size == 20 and G.same_f32(got, ref)
    got, m = _run(b"\x00\x3c", 64, H.F32)             # shorter than the scales
    assert m == 0


def test_all_bytes_all_scale_classes():
    # every byte value under normal, subnormal, zero, negative, inf and NaN
    # scales; NaN results compare as NaN.
    import haagenti_amd as H
    scales = [0x3C00, 0x2E66, 0x0001, 0x03FF, 0x8400, 0x0000, 0x7BFF, 0x7C00, 0xFC00, 0x7E01,
              0x7C01, 0xFE00]
    q = bytearray()
    for sc in scales:
        q += bytes([sc & 0xFF, sc >> 8])
    n = 32 * len(scales)
    payload = bytes((i * 37 + 11) & 0xFF for i in range(n // 2))
    data = bytes(q) + payload
    ref = O.dequantize_int4(data, n)
    got, m = _run(data, n, H.F32)
    assert m == n and G.same_f32(got, ref)


def test_random_bytes_fuzz():
    import haagenti_amd as H
    rng = np.random.default_rng(99)
    for trial in range(5):
        n = int(rng.integers(1, 20000))
        data = rng.integers(0, 256, H.int4_compressed_size(n), dtype=np.uint8).tobytes()
        ref = O.dequantize_int4(data, n)
        got, m = _run(data, n, H.F32)
        assert m == n and G.same_f32(got, ref)
