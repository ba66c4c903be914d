"""HCT v2 on the GPU: XXH3-64 of many buffers in one launch
(hh_xxh3_64_batch) against the xxhash library, and HctReaderV2's validated
decode / checksum validation (hh_hct_decompress_all_validated,
hh_hct_validate_checksums) against the oracle's restatement of
crates/haagenti-hct/src/tensor.rs:840-1020: identical bytes, error kinds and
failing block."""
import struct

import numpy as np
import pytest

import gpu_util as G
import oracle_lib as O

pytestmark = pytest.mark.gpu
xxhash = pytest.importorskip("xxhash")


def gpu_hashes(buf, offs, lens):
    T = G.torch()
    d = G.dev(np.frombuffer(bytes(buf), np.uint8) if len(buf) else np.zeros(1, np.uint8))
    d_off = G.dev(np.array(offs, np.uint64))
    d_len = G.dev(np.array(lens, np.uint32))
    out = T.full((len(offs),), -1, dtype=T.int64, device="cuda")
    G.ctx().xxh3_64_batch(d, len(buf), d_off, d_len, len(offs), out, stream=G.stream())
    G.sync()
    return [int(x) & (2 ** 64 - 1) for x in out.cpu().numpy()]


def test_xxh3_batch_every_length_class_and_alignment():
    rng = np.random.default_rng(31)
    lens = list(range(0, 300)) + [1023, 1024, 1025, 1088, 2047, 2048, 2049, 4096, 16383, 16384,
                                  16385, 65536, 65809]
    offs, pos = [], 0
    for i, n in enumerate(lens):
        pos += i % 7            # every start alignment
        offs.append(pos)
        pos += n
    buf = rng.integers(0, 256, pos + 5, dtype=np.uint8).tobytes()
    got = gpu_hashes(buf, offs, lens)
    for o, n, h in zip(offs, lens, got):
        assert h == xxhash.xxh3_64_intdigest(buf[o:o + n]), (o, n)


def test_xxh3_batch_buffer_end_and_out_of_range():
    rng = np.random.default_rng(32)
    buf = rng.integers(0, 256, 5000, dtype=np.uint8).tobytes()
    # buffers ending exactly at the end of the allocation, and one past it
    offs = [5000 - 241, 5000 - 1025, 5000 - 3, 0, 4990]
    lens = [241, 1025, 3, 5000, 20]
    got = gpu_hashes(buf, offs, lens)
    for o, n, h in zip(offs[:4], lens[:4], got[:4]):
        assert h == xxhash.xxh3_64_intdigest(buf[o:o + n])
    assert got[4] == 0


def _v2(data, block_size=16384, dtype=3, shape=None, flags=O.FLAG_HEADER_CHECKSUM | O.FLAG_BLOCK_CHECKSUMS,
        quant8=None):
    return O.hct_write_v2_lz4(data, block_size, dtype, shape or [len(data)], flags=flags, quant8=quant8)


def gpu_read_v2(f, out_cap):
    import haagenti_amd as H
    try:
        r = H.HctReaderV2(f)
    except H.HaagentiError as e:
        return None, e.code, -1, e.status.detail
    try:
        n, d = r.decompress_all_validated_gpu(G.ctx(), out_cap=out_cap, stream=G.stream())
    except H.HaagentiError as e:
        return None, e.code, e.failed_block, e.status.detail
    return G.host_u8(d)[:n].tobytes(), H.OK, -1, 0


def check(f, out_cap):
    got, code, fb, detail = gpu_read_v2(f, out_cap)
    ref, e, rfb = O.hct_read_all_v2_lz4(f, out_cap)
    assert code == e.kind, (code, e.kind)
    if code == O.OK:
        assert got == ref
    else:
        assert fb == rfb
        if code == O.CORRUPTED:
            assert detail == e.sub
    return got, code, fb


def test_reference_v2_checksum_valid():
    # tensor.rs:1287-1321
    data = bytes(i % 256 for i in range(16384))
    got, code, _ = check(_v2(data), len(data))
    assert code == O.OK and got == data


def test_reference_v2_detects_corruption():
    # tensor.rs:1324-1364 (byte 100), and the header and every block region
    import haagenti_amd as H
    data = bytes(np.random.default_rng(33).integers(0, 5, 60000, dtype=np.uint8))
    f = _v2(data)
    for pos in [20, 60, 70, 100, 200, len(f) // 2, len(f) - 1]:
        g = bytearray(f)
        g[pos] ^= 0xFF
        check(bytes(g), len(data))
    # validate_checksums on the GPU
    g = bytearray(f)
    g[len(f) - 1] ^= 1
    r = H.HctReaderV2(bytes(g))
    with pytest.raises(H.HaagentiError) as e:
        r.validate_checksums_gpu(G.ctx(), stream=G.stream())
    _, rfb = O.hct_validate_v2(bytes(g))
    assert e.value.status.detail == H.CORRUPT_BLOCK_CHECKSUM and e.value.failed_block == rfb == 3
    H.HctReaderV2(f).validate_checksums_gpu(G.ctx(), stream=G.stream())


def test_reference_v2_with_quantization_metadata():
    # tensor.rs:1367-1410
    data = bytes(i % 256 for i in range(4096))
    q = bytes([1, 0]) + struct.pack("<H", 0x3C00) + bytes([0]) + (128).to_bytes(3, "little")
    f = _v2(data, dtype=4, flags=O.FLAG_HEADER_CHECKSUM | O.FLAG_BLOCK_CHECKSUMS | O.FLAG_QUANTIZATION,
            quant8=q)
    got, code, _ = check(f, len(data))
    assert code == O.OK and got == data


def test_reference_v1_file_through_v2_reader():
    # tensor.rs:1412-1438
    data = bytes(i % 256 for i in range(8192))
    f = O.hct_write_lz4(data, 16384, 3, [8192])
    got, code, _ = check(f, len(data))
    assert code == O.OK and got == data


def test_v2_blocks_truncation_capacity_and_zero_sums():
    rng = np.random.default_rng(34)
    data = rng.integers(0, 9, 200001, dtype=np.uint8).tobytes()
    f = _v2(data, block_size=20000)
    check(f, len(data))
    check(f[:-7], len(data))            # last block's range past the end
    check(f, len(data) - 1)             # output capacity
    # a block whose index checksum is 0 is not validated (:966)
    g = bytearray(f)
    struct.pack_into("<Q", g, 64 + 16 * 2 + 8, 0)
    g[56:64] = struct.pack("<Q", O.xxh3_64(bytes(g[:56])))
    check(bytes(g), len(data))


def test_v2_large_file_many_blocks():
    # 4 MiB of config-2-like bytes in 64 KiB blocks: every block hashed and
    # decoded in one launch each
    rng = np.random.default_rng(35)
    data = rng.integers(0, 16, 4 << 20, dtype=np.uint8)
    data[np.repeat(rng.random((4 << 20) // 256) < 0.5, 256)] = 0
    data = data.tobytes()
    f = _v2(data, block_size=65536)
    got, code, _ = check(f, len(data))
    assert code == O.OK and got == data
