"""HCT container read on the GPU (hh_hct_decompress_all, one batched LZ4
launch for all blocks) vs the oracle's HctReader::new + decompress_all
restatement (crates/haagenti-hct/src/tensor.rs:417-515): identical bytes and
error kinds, including a short block shifting the rest and the first failing
block winning."""
import struct

import numpy as np
import pytest

import gpu_util as G
import oracle_lib as O

pytestmark = pytest.mark.gpu


def make_file(blocks, block_size, original, dtype=4, shape=None):
    """HCT v1 bytes from already-compressed blocks (tensor.rs:275-375,556-616)."""
    shape = shape or [original]
    comp = sum(len(b) for b in blocks)
    hdr = (b"HCTN" + struct.pack("<I", 1) + bytes([0, dtype]) + struct.pack("<H", 0)
           + struct.pack("<QQII", original, comp, block_size, len(blocks)) + bytes([len(shape)])
           + b"".join(struct.pack("<Q", d) for d in shape))
    hdr += b"\x00" * (64 - len(hdr))
    idx, off = b"", 0
    for b in blocks:
        idx += struct.pack("<II", off, len(b))
        off += len(b)
    return hdr + idx + b"".join(blocks)


def gpu_read(f, out_cap=None):
    import haagenti_amd as H
    r = H.HctReader(f)
    cap = r.header()["original_size"] if out_cap is None else out_cap
    try:
        n, d = r.decompress_all_gpu(G.ctx(), out_cap=cap, stream=G.stream())
    except H.HaagentiError as e:
        return None, e.code, e.failed_block
    return G.host_u8(d)[:n].tobytes(), H.OK, -1


def check(f, out_cap=None):
    cap = out_cap
    if cap is None:
        cap = struct.unpack("<Q", f[12:20])[0] if len(f) >= 20 else 1
    ref, e = O.hct_read_all_lz4(f, max(cap, 1) if cap else 1)
    got, code, fb = gpu_read(f, cap)
    assert code == e.kind, (code, e.kind, fb)
    if e.kind == O.OK:
        assert got == ref
    return got, code, fb


def test_hand_derived_file():
    f = O.hct_write_lz4(b"\x12" * 512, 256, 0, [512])
    got, code, _ = check(f)
    assert code == 0 and got == b"\x12" * 512


@pytest.mark.parametrize("n,bs", [(1, 1024), (1000, 1000), (1024, 512), (1025, 512), (1023, 512),
                                  (16384 * 3 + 7, 16384), (200000, 4096)])
def test_block_boundaries(n, bs):
    rng = np.random.default_rng(n)
    data = rng.integers(0, 5, n, dtype=np.uint8).tobytes()
    got, code, _ = check(O.hct_write_lz4(data, bs, 4, [n]))
    assert code == 0 and got == data


def test_product_writer_file():
    # a file from the product's HctWriter (tensor.rs:519-617), read back on
    # the GPU and by the oracle
    import haagenti_amd as H
    rng = np.random.default_rng(12)
    data = rng.integers(0, 7, 100003, dtype=np.uint8).tobytes()
    w = H.HctWriter(4, [100003], 16384)
    w.compress_data(data, H.Lz4Compressor())
    got, code, _ = check(w.finish())
    assert code == 0 and got == data


def test_int4_payload_in_default_blocks():
    # the example's on-disk layout: [f16 scales][nibbles], DType::I4, 16 KiB blocks
    rng = np.random.default_rng(11)
    w = rng.normal(0, 0.02, 1024 * 1024).astype(np.float32)
    q = O.quantize_int4(w)
    q = bytes(q)
    f = O.hct_write_lz4(q, 16384, 4, [1024, 1024])
    got, code, _ = check(f)
    assert code == 0 and got == q


def test_short_block_shifts_the_rest():
    import haagenti_amd as H
    comp = H.Lz4Compressor()
    # a stream may end right after a match: 5 literals + an offset-1 match of
    # 20 bytes decodes to 25 of the block's 256 bytes, which is success
    # (block.rs:261-366); the blocks after it move up (decompress_all, :506-515)
    short = bytes([0x5F]) + b"abcde" + bytes([1, 0, 1])
    a = b"abcde" + b"e" * 20
    b = bytes((7 * i) & 0xFF for i in range(256))
    c = bytes((3 * i) & 0xFF for i in range(60))
    f = make_file([short, comp.compress(b), comp.compress(c)], 256, 2 * 256 + 60)
    got, code, _ = check(f)
    assert code == 0 and got == a + b + c


def test_first_failing_block_wins():
    import haagenti_amd as H
    comp = H.Lz4Compressor()
    good = comp.compress(bytes(256))
    zero_off = bytes([0x10, 0x61, 0x00, 0x00])  # literal then offset 0: corrupted
    f = make_file([good, zero_off, good, zero_off], 256, 1024)
    _, code, fb = check(f)
    assert code == H.CORRUPTED_DATA and fb == 1


@pytest.mark.parametrize("patch", [(0, b"XXXX"), (4, b"\x03"), (8, b"\x02"), (9, b"\x05"), (36, b"\x04")])
def test_corrupted_header(patch):
    f = bytearray(O.hct_write_lz4(b"\x12" * 512, 256, 0, [512]))
    off, b = patch
    f[off:off + len(b)] = b
    import haagenti_amd as H
    with pytest.raises(H.HaagentiError) as ei:
        H.HctReader(bytes(f))
    ref, e = O.hct_read_all_lz4(bytes(f), 1024)
    assert ei.value.code == e.kind


def test_truncations_and_index_past_end():
    import haagenti_amd as H
    f = O.hct_write_lz4(bytes(range(256)) * 4, 256, 0, [1024])
    for cut in [len(f) - 3, len(f) - 100]:
        _, code, fb = check(f[:cut])
        assert code == H.ALGORITHM
    # an index entry past the end after a corrupt block: the corrupt block wins
    comp = H.Lz4Compressor()
    zero_off = bytes([0x10, 0x61, 0x00, 0x00])
    g = bytearray(make_file([comp.compress(bytes(256)), zero_off, comp.compress(bytes(256))], 256, 768))
    struct.pack_into("<I", g, 64 + 16, 10 ** 6)  # block 2 offset far past the end
    _, code, fb = check(bytes(g))
    assert code == H.CORRUPTED_DATA and fb == 1


def test_output_capacity():
    import haagenti_amd as H
    data = bytes(range(256)) * 8
    f = O.hct_write_lz4(data, 512, 0, [len(data)])
    _, code, fb = check(f, out_cap=len(data) - 1)
    assert code == H.BUFFER_TOO_SMALL and fb == 3


def test_per_block_decompressor_path():
    # decompress_all with the GPU Decompressor object, block by block, as the
    # reference calls it (&impl Decompressor)
    import haagenti_amd as H
    rng = np.random.default_rng(2)
    data = rng.integers(0, 3, 5000, dtype=np.uint8).tobytes()
    f = O.hct_write_lz4(data, 1024, 4, [5000])
    r = H.HctReader(f)
    assert r.decompress_all(H.Lz4Decompressor(G.ctx())) == data
