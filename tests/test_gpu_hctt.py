"""HCT-T tile decode (dequant -> bitmap scatter -> 64x64 IDCT on MFMA) on the
GPU vs the oracle (dequantize_int4 + compressive.rs scatter + dct.rs
idct_2d).  Tolerance from the spec of this path: max-abs error <= 1e-3 x
tensor RMS against the f32 CPU IDCT; bf16 output is the RNE of the f32
output."""
import numpy as np
import pytest

import gpu_util as G
import oracle_lib as O

pytestmark = pytest.mark.gpu

TOL = 1e-3   # x RMS, the parity bar for the IDCT


def decode_gpu(tiles, rows, cols, k, dtype=0, status=False):
    import haagenti_amd as H
    T = G.torch()
    d_t = G.dev(np.frombuffer(bytes(tiles), np.uint8) if not isinstance(tiles, np.ndarray) else tiles)
    esz = 4 if dtype == H.F32 else 2
    out = T.full((rows * cols * esz,), 0x7F, dtype=T.uint8, device="cuda")
    ntiles = (rows // 64) * (cols // 64)
    st = T.full((ntiles,), -1, dtype=T.int32, device="cuda") if status else None
    G.ctx().hctt_decode(d_t, d_t.numel(), rows, cols, k, out, dtype=dtype,
                        d_tile_status=st, stream=G.stream())
    G.sync()
    raw = G.host_u8(out)
    arr = raw.view(np.float32) if dtype == H.F32 else raw.view(np.uint16)
    arr = arr.reshape(rows, cols)
    return (arr, st.cpu().numpy()) if status else arr


def _encode(rows, cols, k, seed, std=0.02):
    import haagenti_amd as H
    rng = np.random.default_rng(seed)
    w = rng.normal(0, std, (rows, cols)).astype(np.float32)
    return H.hctt_encode(w, k)


@pytest.mark.parametrize("k", [1024, 1228])
def test_small_tensor_vs_oracle(k):
    rows, cols = 256, 384
    tiles = _encode(rows, cols, k, seed=k)
    rc, ref = O.hctt_decode_tensor(tiles, rows, cols, k)
    assert rc == O.OK
    got = decode_gpu(tiles, rows, cols, k)
    rms = np.sqrt((ref.astype(np.float64) ** 2).mean())
    err = np.abs(got - ref).max()
    assert err <= TOL * rms, err / rms
    # also against the f64 closed form, tile by tile
    tb = O.hctt_tile_bytes(k)
    for t in range(6):
        _, x64 = O.hctt_decode_tile(tiles[t * tb:(t + 1) * tb], k, f64=True)
        tr, tc = divmod(t, cols // 64)
        blk = got[tr * 64:(tr + 1) * 64, tc * 64:(tc + 1) * 64]
        assert np.abs(blk - x64).max() <= 1e-5 * rms


def test_bf16_and_f16_are_rne_of_f32():
    import haagenti_amd as H
    rows, cols, k = 128, 256, 1228
    tiles = _encode(rows, cols, k, seed=5)
    f32 = decode_gpu(tiles, rows, cols, k, H.F32)
    b16 = decode_gpu(tiles, rows, cols, k, H.BF16)
    h16 = decode_gpu(tiles, rows, cols, k, H.F16)
    assert (b16 == G.bf16_bits(f32)).all()
    assert (h16 == G.f16_bits(f32)).all()
    # against the oracle: the f32 result lies within 1e-5 x RMS of the CPU
    # result (the per-tile bar against the f64 inverse), so its RNE to bf16
    # lies within half a bf16 ulp of it plus that
    _, ref = O.hctt_decode_tensor(tiles, rows, cols, k)
    rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
    bv = (b16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    half_ulp = np.ldexp(1.0, np.frexp(np.abs(bv))[1] - 9)
    assert (np.abs(bv - ref) <= half_ulp + 1e-5 * rms).all()
    d = np.abs(b16.astype(np.int32) - G.bf16_bits(ref).astype(np.int32))
    assert (d[np.abs(ref) >= 1e-2 * rms] <= 1).all()   # one bf16 ulp of the rounded CPU result


@pytest.mark.parametrize("k", [1, 7, 777, 2048, 4096])
def test_other_retention_counts(k):
    # 777: odd tile size (951 B) exercises the byte-staging path
    rows, cols = 128, 128
    tiles = _encode(rows, cols, k, seed=100 + k)
    rc, ref = O.hctt_decode_tensor(tiles, rows, cols, k)
    got = decode_gpu(tiles, rows, cols, k)
    rms = np.sqrt((ref.astype(np.float64) ** 2).mean())
    assert np.abs(got - ref).max() <= TOL * rms


def test_wide_dynamic_range_between_tiles():
    # tiles at very different magnitudes exercise the per-tile prescale
    import haagenti_amd as H
    rows, cols, k = 64, 64 * 6, 1228
    rng = np.random.default_rng(8)
    w = rng.normal(0, 1, (rows, cols)).astype(np.float32)
    for i, s in enumerate([1e-6, 1e-3, 1.0, 30.0, 1e3, 5e-5]):
        w[:, 64 * i:64 * (i + 1)] *= s
    tiles = H.hctt_encode(w, k)
    _, ref = O.hctt_decode_tensor(tiles, rows, cols, k)
    got = decode_gpu(tiles, rows, cols, k)
    for i in range(6):
        a, b = got[:, 64 * i:64 * (i + 1)], ref[:, 64 * i:64 * (i + 1)]
        rms = np.sqrt((b.astype(np.float64) ** 2).mean())
        assert np.abs(a - b).max() <= TOL * rms


def test_corrupted_bitmap_tile_reports_and_zeroes():
    rows, cols, k = 128, 128, 1024
    tiles = _encode(rows, cols, k, seed=9).copy()
    tb = O.hctt_tile_bytes(k)
    tiles[2 * tb + 5] ^= 0x10           # tile 2 popcount off by one
    got, st = decode_gpu(tiles, rows, cols, k, status=True)
    assert list(st) == [0, 0, 1, 0]
    assert (got[64:128, 0:64] == 0).all()
    rc, ref = O.hctt_decode_tensor(tiles, rows, cols, k)
    assert rc == O.CORRUPTED
    ok = np.ones((rows, cols), bool)
    ok[64:128, 0:64] = False
    _, good = O.hctt_decode_tensor(_encode(rows, cols, k, seed=9), rows, cols, k)
    rms = np.sqrt((good.astype(np.float64) ** 2).mean())
    assert np.abs(got[ok] - good[ok]).max() <= TOL * rms


def test_shape_limits_are_argument_errors():
    """rows / cols not multiples of 64, or cols above 2^24 (the stores'
    32-bit row offsets), are rejected before any launch."""
    import haagenti_amd as Hm
    T = G.torch()
    k = 1024
    tiles = G.dev(_encode(64, 64, k, seed=3))
    o = T.empty(64 * 64, dtype=T.float32, device="cuda")
    for rows, cols in ((64, 100), (100, 64), (64, (1 << 24) + 64)):
        with pytest.raises(Hm.HaagentiError) as e:
            G.ctx().hctt_decode(tiles, tiles.numel(), rows, cols, k, o)
        assert e.value.code == Hm.INVALID_ARGUMENT, (rows, cols)
    G.ctx().hctt_decode(tiles, tiles.numel(), 64, 64, k, o)
    G.sync()


def test_config3_8192x8192_vs_oracle():
    # 16,384 tiles, top 25% (k = 1024), f32 output against the oracle, plus
    # Parseval per tile (orthonormal IDCT preserves energy).
    rows = cols = 8192
    k = 1024
    tiles = _encode(rows, cols, k, seed=3)
    assert tiles.size == 16384 * 1088 == 17_825_792
    rc, ref = O.hctt_decode_tensor(tiles, rows, cols, k, nthreads=8)
    assert rc == O.OK
    got = decode_gpu(tiles, rows, cols, k)
    rms = np.sqrt((ref.astype(np.float64) ** 2).mean())
    err = np.abs(got - ref).max()
    assert err <= TOL * rms, err / rms
    e_out = (got.astype(np.float64) ** 2).reshape(128, 64, 128, 64).sum(axis=(1, 3))
    e_ref = (ref.astype(np.float64) ** 2).reshape(128, 64, 128, 64).sum(axis=(1, 3))
    assert np.abs(e_out - e_ref).max() <= 1e-4 * e_ref.max()


def test_tile_with_infinite_scale_matches_the_oracle():
    # A constant tile of 1e5 has a DC coefficient of 6.4e6, so its first
    # 32-block's scale max/7 truncates to an infinite f16
    # (quantization.rs:136-163); the reference then dequantizes that block
    # to inf (7 x inf) and nan (0 x inf, its other coefficients) and its
    # inverse DCT spreads nan over the tile.  The GPU decode must agree:
    # the same tile status and the same non-finite pattern, with the finite
    # tiles around it within tolerance.
    import haagenti_amd as H
    rows, cols, k = 128, 128, 1228
    rng = np.random.default_rng(71)
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    w[0:64, 64:128] = 1e5
    tiles = H.hctt_encode(w, k)
    tb = O.hctt_tile_bytes(k)
    scales = np.frombuffer(bytes(tiles[tb + 512:tb + 514]), np.uint16)
    assert scales[0] == 0x7C00  # +inf
    rc, ref = O.hctt_decode_tensor(tiles, rows, cols, k)
    assert rc == O.OK
    got, st = decode_gpu(tiles, rows, cols, k, status=True)
    assert (st == 0).all()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    rms = np.sqrt((ref[fin].astype(np.float64) ** 2).mean())
    assert np.abs(got[fin] - ref[fin]).max() <= TOL * rms
    assert not fin[0:64, 64:128].any()   # the oracle's tile is all nan
