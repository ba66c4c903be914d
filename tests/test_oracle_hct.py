"""Pins the oracle's HCT-T tile codec (compressive.rs rules + quantization.rs
+ dct.rs) and the HCT v1 container (crates/haagenti-hct/src/tensor.rs).
"""
import struct

import numpy as np
import pytest

import oracle_lib as O


def test_tile_bytes():
    assert O.hctt_tile_bytes(1024) == 512 + 64 + 512 == 1088
    assert O.hctt_tile_bytes(1228) == 512 + 78 + 614 == 1204


def _f16_stream(bitmap, coeffs_f16):
    """HCT V3 fragment stream as read by ref/c/hct_decoder.h:322-394."""
    data = struct.pack("<I", len(coeffs_f16)) + bytes(bitmap) + coeffs_f16.astype("<u2").tobytes()
    frag = struct.pack("<HHQI", 0, 0, 0, len(data)) + data
    return struct.pack("<H", 1) + frag


def _random_tile_bytes(rng, k, scale_codes):
    bits = rng.choice(4096, k, replace=False)
    bm = np.zeros(512, np.uint8)
    for b in bits:
        bm[b // 8] |= 1 << (b % 8)
    nsc = (k + 31) // 32
    sc = np.array(rng.choice(scale_codes, nsc), np.uint16)
    nib = rng.integers(0, 16, k).astype(np.uint8)
    packed = np.zeros((k + 1) // 2, np.uint8)
    packed[:] = nib[0::2]
    packed[: k // 2] |= nib[1::2] << 4
    return bm, sc, nib, np.concatenate([bm, sc.view(np.uint8), packed])


@pytest.mark.skipif(not O.ref_available(), reason="reference C decoder not built")
@pytest.mark.parametrize("k", [1024, 1228, 1, 4096])
def test_tile_decode_vs_reference_c_decoder(k):
    # Power-of-two scales make every dequantized value exactly an f16, so the
    # reference's f16 V3 decoder sees the same coefficients.
    rng = np.random.default_rng(k)
    bm, sc, nib, tb = _random_tile_bytes(rng, k, [0x2000, 0x2400, 0x1C00, 0x3C00])
    rc, mine = O.hctt_decode_tile(tb, k)
    assert rc == O.OK
    idx = np.flatnonzero(np.unpackbits(bm, bitorder="little"))
    vals = (nib.astype(np.float32) - 8) * sc.view(np.float16).astype(np.float32)[np.arange(k) // 32]
    f16 = vals.astype(np.float16).view(np.uint16)
    assert (f16.view(np.float16).astype(np.float32) == vals).all()
    ref = O.ref_hct_decode(_f16_stream(bm, f16), 64, 64)
    assert ref is not None
    assert np.abs(mine - ref).max() < 1e-5 * np.abs(ref).max()
    # the scatter itself: ascending bit positions get the values in order
    dense = np.zeros(4096, np.float32)
    dense[idx] = vals
    assert np.abs(O.ref_idct_2d(dense.reshape(64, 64)) - ref).max() == 0.0


def test_tile_encode_decode_gaussian():
    rng = np.random.default_rng(11)
    t = rng.normal(0, 0.02, (64, 64)).astype(np.float32)
    for k in [1024, 1228]:
        tb = O.hctt_encode_tile(t, k)
        assert tb.size == O.hctt_tile_bytes(k)
        assert int(np.unpackbits(tb[:512]).sum()) == k
        rc, x32 = O.hctt_decode_tile(tb, k)
        rc2, x64 = O.hctt_decode_tile(tb, k, f64=True)
        assert rc == rc2 == O.OK
        rms = np.sqrt((x64 ** 2).mean())
        assert np.abs(x32 - x64).max() < 1e-5 * rms
        # White noise has a flat spectrum: keeping the top fraction p of the
        # coefficients keeps E = 2[t phi(t) + 1 - Phi(t)] of the energy, where
        # t is the (1 - p/2) normal quantile, so cos(x, t) ~= sqrt(E).
        from scipy.stats import norm
        p = k / 4096
        thr = norm.ppf(1 - p / 2)
        energy = 2 * (thr * norm.pdf(thr) + norm.sf(thr))
        cos = (x64 * t).sum() / np.sqrt((x64 ** 2).sum() * (t ** 2).sum())
        assert abs(cos - np.sqrt(energy)) < 0.03


def test_tile_keeps_top_k_of_the_dct():
    rng = np.random.default_rng(12)
    t = rng.normal(0, 1, (64, 64)).astype(np.float32)
    k = 300
    tb = O.hctt_encode_tile(t, k)
    c = O.dct_2d(t).ravel()
    expect = sorted(sorted(range(4096), key=lambda i: (-abs(float(c[i])), i))[:k])
    got = list(np.flatnonzero(np.unpackbits(tb[:512], bitorder="little")))
    assert got == expect
    # coefficients quantized in ascending index order
    q = O.quantize_int4(c[expect])
    assert bytes(tb[512:]) == q


def test_tile_bitmap_count_mismatch_is_corrupted():
    rng = np.random.default_rng(13)
    tb = O.hctt_encode_tile(rng.normal(0, 1, (64, 64)).astype(np.float32), 1024)
    bad = tb.copy()
    bad[0] ^= 0xFF
    rc, _ = O.hctt_decode_tile(bad, 1024)
    assert rc == O.CORRUPTED


def test_tensor_tile_order_row_major():
    # Each tile constant -> DC only -> decodes to ~that constant.  Pins the
    # (tile row, tile col) -> tensor placement.
    rows, cols = 128, 192
    w = np.zeros((rows, cols), np.float32)
    vals = {}
    for tr in range(rows // 64):
        for tc in range(cols // 64):
            v = 0.01 * (1 + tr * 3 + tc)
            w[tr * 64:(tr + 1) * 64, tc * 64:(tc + 1) * 64] = v
            vals[(tr, tc)] = v
    tiles = O.hctt_encode_tensor(w, 1, nthreads=2)
    rc, x = O.hctt_decode_tensor(tiles, rows, cols, 1, nthreads=2)
    assert rc == O.OK
    for (tr, tc), v in vals.items():
        blk = x[tr * 64:(tr + 1) * 64, tc * 64:(tc + 1) * 64]
        assert np.abs(blk - v).max() < 2e-3 * v
    # and the tensor decode equals the per-tile decode
    tb = O.hctt_tile_bytes(1)
    for t in range(6):
        rc, xt = O.hctt_decode_tile(tiles[t * tb:(t + 1) * tb], 1)
        tr, tc = divmod(t, cols // 64)
        assert (xt == x[tr * 64:(tr + 1) * 64, tc * 64:(tc + 1) * 64]).all()


# ---------------------------------------------------------------- container
def test_container_bytes_hand_derived():
    data = b"\x12" * 512
    f = O.hct_write_lz4(data, 256, 0, [512])
    blk = bytes([0x2F, 0x12, 0x12, 0x01, 0x00, 0xE6, 0x50]) + b"\x12" * 5  # 12 bytes
    hdr = (b"HCTN" + struct.pack("<I", 1) + bytes([0, 0]) + struct.pack("<H", 0)
           + struct.pack("<QQII", 512, 24, 256, 2) + bytes([1]) + struct.pack("<Q", 512))
    hdr += b"\x00" * (64 - len(hdr))
    idx = struct.pack("<IIII", 0, 12, 12, 12)
    assert f == hdr + idx + blk + blk
    out, e = O.hct_read_all_lz4(f, 1024)
    assert e.kind == O.OK and out == data


@pytest.mark.parametrize("n,bs,nblocks", [(0, 1024, 0), (1000, 1000, 1), (1024, 512, 2),
                                          (1025, 512, 3), (1023, 512, 2), (16384 * 3 + 7, 16384, 4)])
def test_container_block_boundaries(n, bs, nblocks):
    rng = np.random.default_rng(n)
    data = rng.integers(0, 5, n, dtype=np.uint8).tobytes()
    f = O.hct_write_lz4(data, bs, 4, [n])
    assert struct.unpack("<I", f[32:36])[0] == nblocks
    assert struct.unpack("<Q", f[12:20])[0] == n
    out, e = O.hct_read_all_lz4(f, max(n, 1))
    assert e.kind == O.OK and out == data


@pytest.mark.parametrize("patch,kind", [
    ((0, b"XXXX"), O.CORRUPTED),     # magic   (tensor.rs:1447)
    ((4, b"\x03"), O.CORRUPTED),     # version (tensor.rs:1469)
    ((8, b"\x02"), O.CORRUPTED),     # algorithm (tensor.rs:1490)
    ((9, b"\x05"), O.CORRUPTED),     # dtype   (tensor.rs:1511)
])
def test_container_corrupted_header(patch, kind):
    f = bytearray(O.hct_write_lz4(b"\x12" * 512, 256, 0, [512]))
    off, b = patch
    f[off:off + len(b)] = b
    out, e = O.hct_read_all_lz4(bytes(f), 1024)
    assert out is None and e.kind == kind


def test_container_truncations():
    f = O.hct_write_lz4(b"\x12" * 512, 256, 0, [512])
    assert O.hct_read_all_lz4(f[:40], 1024)[1].kind == O.ALGORITHM    # header
    assert O.hct_read_all_lz4(f[:68], 1024)[1].kind == O.ALGORITHM    # index
    assert O.hct_read_all_lz4(f[:-3], 1024)[1].kind == O.ALGORITHM    # block data
    assert O.hct_read_all_lz4(b"\xde\xad\xbe\xef\x12\x34\x56\x78", 1024)[1].kind != O.OK
