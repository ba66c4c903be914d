"""Oracle XXH3-64 and HCT v2 container (crates/haagenti-hct/src/tensor.rs).

XXH3-64 (xxhash-rust 0.8.15 `xxh3_64`, seed 0, called at tensor.rs:729,794,
858,967) is pinned against the xxhash library (python `xxhash`, the C
reference implementation of the published algorithm) on every length that
selects a different code path.  The v2 container restates HctWriterV2 /
HctReaderV2 (:676-1021) and is checked against the reference's own v2 tests
(:1250-1440, 1943-2060) and the byte layout they imply."""
import struct

import numpy as np
import pytest

import oracle_lib as O

xxhash = pytest.importorskip("xxhash")


def test_xxh3_every_short_length_and_long_inputs():
    rng = np.random.default_rng(11)
    lengths = list(range(0, 1100)) + [2047, 2048, 2049, 4095, 4096, 4097, 16384, 65536, 65809]
    for n in lengths:
        d = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert O.xxh3_64(d) == xxhash.xxh3_64_intdigest(d), n


def test_xxh3_structured_inputs():
    # zeros, 0xFF runs and the reference's own test pattern (i % 256)
    for n in [0, 1, 3, 4, 8, 9, 16, 17, 128, 129, 240, 241, 1024, 1025, 16384]:
        for d in (bytes(n), b"\xff" * n, bytes(i % 256 for i in range(n))):
            assert O.xxh3_64(d) == xxhash.xxh3_64_intdigest(d)


def test_xxh3_is_sensitive_to_every_byte_position():
    # tensor.rs:1943-1960 (checksum uniqueness) and :2043-2060 (bit flips)
    base = bytes(i % 251 for i in range(3000))
    h0 = O.xxh3_64(base)
    seen = {h0}
    for pos in range(0, 3000, 7):
        b = bytearray(base)
        b[pos] ^= 1
        h = O.xxh3_64(bytes(b))
        assert h != h0
        seen.add(h)
    assert len(seen) == 1 + len(range(0, 3000, 7))


def _pattern(n):
    return bytes(i % 256 for i in range(n))


def test_v2_roundtrip_and_layout():
    # tensor.rs:1287-1321 test_hct_v2_checksum_valid: 16384 bytes (i % 256), dtype I8
    data = _pattern(16384)
    f = O.hct_write_v2_lz4(data, 16 * 1024, 3, [16384])
    assert f[:4] == b"HCTN" and struct.unpack_from("<I", f, 4)[0] == 2
    flags = struct.unpack_from("<H", f, 10)[0]
    assert flags == O.FLAG_HEADER_CHECKSUM | O.FLAG_BLOCK_CHECKSUMS
    assert struct.unpack_from("<Q", f, 56)[0] == xxhash.xxh3_64_intdigest(f[:56])
    off, csz, sum_ = struct.unpack_from("<IIQ", f, 64)  # BlockIndexV2 (:241-261)
    assert off == 0 and sum_ == xxhash.xxh3_64_intdigest(f[80:80 + csz])
    e, fb = O.hct_validate_v2(f)
    assert e.kind == O.OK and fb == -1
    out, e, fb = O.hct_read_all_v2_lz4(f, len(data))
    assert e.kind == O.OK and out == data


def test_v2_detects_corruption():
    # tensor.rs:1324-1364: flip a byte at offset 100 (index or data)
    data = _pattern(16384)
    f = bytearray(O.hct_write_v2_lz4(data, 16 * 1024, 3, [16384]))
    f[100] ^= 0xFF
    e, fb = O.hct_validate_v2(bytes(f))
    assert e.kind == O.CORRUPTED and e.sub == O.CORRUPT_BLOCK_CHECKSUM and fb == 0
    out, e, fb = O.hct_read_all_v2_lz4(bytes(f), len(data))
    assert out is None and e.sub == O.CORRUPT_BLOCK_CHECKSUM and fb == 0
    # a header byte: header checksum mismatch (:857-865)
    g = bytearray(O.hct_write_v2_lz4(data, 16 * 1024, 3, [16384]))
    g[20] ^= 0x01
    out, e, fb = O.hct_read_all_v2_lz4(bytes(g), len(data))
    assert e.kind == O.CORRUPTED and e.sub == O.CORRUPT_HEADER_CHECKSUM and fb == -1


def test_v2_with_quantization_metadata():
    # tensor.rs:1367-1410: GptqInt4, group 128, scale 0x3C00, I4 data
    data = _pattern(4096)
    quant = bytes([1, 0]) + struct.pack("<H", 0x3C00) + bytes([0]) + (128).to_bytes(3, "little")
    f = O.hct_write_v2_lz4(data, 16 * 1024, 4, [4096],
                           flags=O.FLAG_HEADER_CHECKSUM | O.FLAG_BLOCK_CHECKSUMS | O.FLAG_QUANTIZATION,
                           quant8=quant)
    assert f[64:72] == quant
    out, e, fb = O.hct_read_all_v2_lz4(f, len(data))
    assert e.kind == O.OK and out == data
    # unknown scheme (:158-173)
    g = bytearray(f)
    g[64] = 5
    out, e, fb = O.hct_read_all_v2_lz4(bytes(g), len(data))
    assert e.kind == O.CORRUPTED and e.sub == O.CORRUPT_QUANT_SCHEME


def test_v2_without_block_checksums_has_zero_sums():
    # without_block_checksums (:720-724): index entries stay 16 bytes but the
    # reader, seeing no BLOCK_CHECKSUMS flag, reads 8-byte entries (:877-884)
    data = bytes(np.random.default_rng(2).integers(0, 4, 50000, dtype=np.uint8))
    f = O.hct_write_v2_lz4(data, 16384, 3, [50000], flags=O.FLAG_HEADER_CHECKSUM)
    nblocks = 4
    for b in range(nblocks):
        assert struct.unpack_from("<Q", f, 64 + 16 * b + 8)[0] == 0
    out, e, fb = O.hct_read_all_v2_lz4(f, len(data))
    # the 8-byte reading of 16-byte entries puts the data offset inside the
    # index, so the file does not read back (the reference's writer and
    # reader disagree on this flag combination the same way)
    assert e.kind != O.OK or out != data


def test_v1_files_still_read():
    # tensor.rs:1412-1438: a v1 file through the v2 reader (no checksums)
    data = _pattern(8192)
    f = O.hct_write_lz4(data, 16 * 1024, 3, [8192])
    out, e, fb = O.hct_read_all_v2_lz4(f, len(data))
    assert e.kind == O.OK and out == data


def test_v2_multi_block_short_last_block_and_errors():
    rng = np.random.default_rng(3)
    data = rng.integers(0, 8, 70001, dtype=np.uint8).tobytes()
    f = O.hct_write_v2_lz4(data, 16384, 3, [70001])
    out, e, fb = O.hct_read_all_v2_lz4(f, len(data))
    assert e.kind == O.OK and out == data
    # truncated file: block read fails (Error::Algorithm), first failing block
    out, e, fb = O.hct_read_all_v2_lz4(f[:-10], len(data))
    assert e.kind == O.ALGORITHM and fb == 4
    # output capacity short
    out, e, fb = O.hct_read_all_v2_lz4(f, len(data) - 1)
    assert e.kind == O.BUFFER_TOO_SMALL and fb == 4
