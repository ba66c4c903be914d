"""Pins the oracle's LZ4 restatement (crates/haagenti-lz4/src/block.rs).

Known answers were derived by hand from block.rs:73-147 (compressor) and the
public LZ4 block format (decoder streams); none of them is produced by the
code under test.
"""
import numpy as np
import pytest

import oracle_lib as O


# ---------------------------------------------------------------- compressor
def test_compress_small_input_literals_only():
    # block.rs:77-79: inputs < 13 bytes are one literal run.
    out, e = O.lz4_compress_block(b"Hello")
    assert out == bytes([0x50]) + b"Hello"


def test_compress_empty_is_single_zero_token():
    # block.rs:380-385 (test_empty_input): a single 0x00 token.
    out, e = O.lz4_compress_block(b"")
    assert out == b"\x00"


def test_compress_40_A_hand_derived():
    # Position 0 never matches (match_pos > 0 guard, block.rs:99), so the
    # first match is found at ip=2 against position 1: ll=2, offset 1,
    # match runs to match_limit = 40-5 = 35 -> ml = 33 (ext byte 33-4-15=14),
    # then 5 last literals.
    out, e = O.lz4_compress_block(b"A" * 40)
    assert out == bytes([0x2F, 0x41, 0x41, 0x01, 0x00, 0x0E, 0x50]) + b"A" * 5


def test_compress_literal_extension_and_match_limit_hand_derived():
    # "0123" at 16 hashes to position 0 -> rejected by the >0 guard; "1234"
    # at 17 matches position 1 (offset 16) and extends to match_limit=23:
    # ml = 6, ll = 17 (token 0xF2, ext byte 2), then 5 last literals.
    src = b"0123456789abcdef0123456vwxyz"
    out, e = O.lz4_compress_block(src)
    exp = bytes([0xF2, 0x02]) + b"0123456789abcdef0" + bytes([0x10, 0x00, 0x50]) + b"vwxyz"
    assert out == exp


def test_compress_256_same_bytes_hand_derived():
    # Used by the container test below: ml = 4 + (251-6) = 249 -> ext 230.
    out, e = O.lz4_compress_block(b"\x12" * 256)
    assert out == bytes([0x2F, 0x12, 0x12, 0x01, 0x00, 0xE6, 0x50]) + b"\x12" * 5


def test_compress_buffer_too_small():
    out, e = O.lz4_compress_block(b"Hello", cap=4)
    assert out is None and e.kind == O.BUFFER_TOO_SMALL
    assert e.required == 1 + 0 + 1 + 5 and e.provided == 4


@pytest.mark.parametrize("src", [
    b"Hello",
    b"A" * 40,
    b"Hello, World! Hello, World! Hello, World! This is a test.",
    (b"The quick brown fox jumps over the lazy dog. " * 300)[:10000],
    b"Hello, LZ4! This is a test for interoperability with lz4_flex.",
    b"Testing compression output compatibility with lz4_flex reference.",
    (b"ABCDEFGH" * 200)[:1000],
])
def test_roundtrip_reference_inputs(src):
    # The reference's own test inputs (block.rs:379-502).
    comp, _ = O.lz4_compress_block(src)
    assert len(comp) <= O.lz4_max_compressed_size(len(src))
    out, e = O.lz4_decompress_block(comp, len(src))
    assert e.kind == O.OK and out == src


def test_roundtrip_compresses_repetitive():
    src = (b"The quick brown fox jumps over the lazy dog. " * 300)[:10000]
    comp, _ = O.lz4_compress_block(src)
    assert len(comp) < len(src)


def test_roundtrip_random_and_structured():
    rng = np.random.default_rng(5)
    for n in [0, 1, 12, 13, 14, 17, 64, 1000, 65536]:
        for kind in range(3):
            if kind == 0:
                src = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
            elif kind == 1:
                src = rng.integers(0, 4, n, dtype=np.uint8).tobytes()
            else:
                a = rng.integers(0, 256, n, dtype=np.uint8)
                a[(np.arange(n) // 256) % 2 == 0] = 0
                src = a.tobytes()
            comp, _ = O.lz4_compress_block(src)
            out, e = O.lz4_decompress_block(comp, n)
            assert e.kind == O.OK and out == src, (n, kind)


# ---------------------------------------------------------------- decoder
def test_decode_empty_token():
    out, e = O.lz4_decompress_block(b"\x00", 0)
    assert e.kind == O.OK and out == b""


def test_decode_offset1_overlap():
    # 'x' then match off=1 len 8, then last literal 'y'
    s = bytes([0x14, ord("x"), 0x01, 0x00, 0x10, ord("y")])
    out, e = O.lz4_decompress_block(s, 10)
    assert out == b"x" * 9 + b"y"


def test_decode_offset3_overlap_then_zero_token():
    s = bytes([0x35]) + b"abc" + bytes([0x03, 0x00, 0x00])
    out, e = O.lz4_decompress_block(s, 12)
    assert out == b"abc" * 4


def test_decode_literal_length_chain():
    lits = bytes(range(256)) + bytes(range(14))
    s = bytes([0xF0, 0xFF, 0x00]) + lits  # 15 + 255 + 0 = 270
    out, e = O.lz4_decompress_block(s, 270)
    assert out == lits


def test_decode_match_length_chain():
    s = bytes([0x1F, ord("z"), 0x01, 0x00, 0xFF, 0x01])  # ml = 4+15+255+1
    out, e = O.lz4_decompress_block(s, 276)
    assert out == b"z" * 276


def test_decode_short_block_is_success():
    # Stream ends right after a match: fewer bytes than output_size, no error.
    s = bytes([0x14, ord("x"), 0x01, 0x00])
    out, e = O.lz4_decompress_block(s, 20)
    assert e.kind == O.OK and out == b"x" * 9


@pytest.mark.parametrize("stream,size,kind,sub,pos,req,prov", [
    (bytes([0x10, 0x61, 0x00, 0x00]), 10, O.CORRUPTED, O.CORRUPT_ZERO_OFFSET, 0, 0, 0),
    (bytes([0x10, 0x61, 0x02, 0x00]), 10, O.CORRUPTED, O.CORRUPT_OFFSET_BEYOND, 1, 0, 0),
    (bytes([0xF0]), 10, O.UNEXPECTED_EOF, 0, 1, 0, 0),
    (bytes([0x30, 0x61]), 10, O.UNEXPECTED_EOF, 0, 1, 0, 0),
    (bytes([0x10, 0x61, 0x01]), 10, O.UNEXPECTED_EOF, 0, 2, 0, 0),
    (bytes([0x1F, 0x61, 0x01, 0x00]), 100, O.UNEXPECTED_EOF, 0, 4, 0, 0),
    (bytes([0x30, 0x61, 0x62, 0x63]), 2, O.BUFFER_TOO_SMALL, 0, 0, 3, 2),
    (bytes([0x14, 0x78, 0x01, 0x00]), 5, O.BUFFER_TOO_SMALL, 0, 0, 9, 5),
    (bytes([0x30, 0x61, 0x62, 0x63]), 10, O.UNEXPECTED_EOF, 0, 4, 0, 0),
])
def test_decode_errors(stream, size, kind, sub, pos, req, prov):
    out, e = O.lz4_decompress_block(stream, size)
    assert out is None
    assert (e.kind, e.sub, e.position, e.required, e.provided) == (kind, sub, pos, req, prov)


def test_batch_matches_single_calls():
    rng = np.random.default_rng(9)
    blocks = [rng.integers(0, 3, rng.integers(1, 5000), dtype=np.uint8).tobytes() for _ in range(37)]
    comp = [O.lz4_compress_block(b)[0] for b in blocks]
    in_off = np.cumsum([0] + [len(c) for c in comp[:-1]])
    out_off = np.cumsum([0] + [len(b) for b in blocks[:-1]])
    out, kinds, written = O.lz4_decompress_batch(b"".join(comp), in_off, [len(c) for c in comp],
                                                 out_off, [len(b) for b in blocks],
                                                 sum(len(b) for b in blocks), nthreads=4)
    assert (kinds == 0).all()
    assert out.tobytes() == b"".join(blocks)
    assert list(written) == [len(b) for b in blocks]
