"""Host zstd decoder (hh_zstd_decompress) against libzstd.

The reference decodes the turbo pipeline's zstd wrapper with the zstd crate
0.13.3 (crates/haagenti/src/pipeline/turbo.rs:389-391,
crates/haagenti-cuda/src/decompress.rs:296-319), i.e. libzstd.  Frames here
are produced by libzstd itself (pyarrow's bundled build) at several levels
and content kinds, so every block type, literal mode and FSE table mode
occurs; decoded bytes must be identical, malformed streams must be reported
(never crash).  XXH64 is pinned against the xxhash library."""
import struct

import numpy as np
import pytest

pa = pytest.importorskip("pyarrow")
xxhash = pytest.importorskip("xxhash")


def H():
    import haagenti_amd as h
    return h


def z(data, level):
    return pa.Codec("zstd", compression_level=level).compress(data, asbytes=True)


def contents():
    rng = np.random.default_rng(0)
    text = b"".join(b"the %d-th weight tile of layer %d holds %d coefficients; " % (i, i % 32, i * 7)
                    for i in range(20000))
    nib = rng.integers(0, 16, 300000, dtype=np.uint8)
    nib[np.repeat(rng.random(300000 // 256 + 1) < 0.5, 256)[:300000]] = 0
    yield "empty", b""
    yield "one", b"x"
    yield "zeros", bytes(1 << 20)
    yield "random", rng.integers(0, 256, 200000, dtype=np.uint8).tobytes()
    yield "text", text
    yield "nibbles", nib.tobytes()
    yield "f16", rng.normal(0, 0.05, 150000).astype(np.float16).tobytes()
    yield "block_edge", text[:131072]
    yield "block_edge1", text[:131073]
    yield "period3", b"abc" * 100000


@pytest.mark.parametrize("level", [-5, 1, 3, 9, 19])
def test_decode_matches_libzstd(level):
    for name, data in contents():
        c = z(data, level)
        got = H().zstd_decompress(c)
        assert got == data, (name, level)


def test_concatenated_and_skippable_frames():
    a, b = b"first frame " * 1000, bytes(range(256)) * 300
    skip = struct.pack("<II", 0x184D2A53, 5) + b"hello"
    stream = z(a, 3) + skip + z(b, 1) + z(b"", 1)
    assert H().zstd_decompress(stream) == a + b


def raw_frame(data, checksum=True, single=True):
    """A frame of raw blocks with the content size and, optionally, the
    XXH64 content checksum (RFC 8878 sections 3.1.1.1-3.1.1.2)."""
    fhd = (3 << 6) | (int(single) << 5) | (int(checksum) << 2)
    out = struct.pack("<IB", 0xFD2FB528, fhd)
    if not single:
        out += bytes([(17 - 10) << 3])                        # window 128 KiB
    out += struct.pack("<Q", len(data))
    blocks = [data[i:i + 65536] for i in range(0, len(data), 65536)] or [b""]
    for i, blk in enumerate(blocks):
        hdr = (len(blk) << 3) | (0 << 1) | int(i == len(blocks) - 1)
        out += struct.pack("<I", hdr)[:3] + blk
    if checksum:
        out += struct.pack("<I", xxhash.xxh64_intdigest(data) & 0xFFFFFFFF)
    return out


def test_checksum_and_raw_frames():
    rng = np.random.default_rng(1)
    data = rng.integers(0, 256, 200000, dtype=np.uint8).tobytes()
    for single in (True, False):
        f = raw_frame(data, True, single)
        assert H().zstd_decompress(f) == data
        assert pa.Codec("zstd").decompress(f, decompressed_size=len(data), asbytes=True) == data
        bad = bytearray(f)
        bad[-1] ^= 1                                          # checksum mismatch
        with pytest.raises(H().HaagentiError):
            H().zstd_decompress(bytes(bad))


def test_xxh64_matches_xxhash():
    rng = np.random.default_rng(2)
    for n in list(range(0, 70)) + [100, 1000, 4096, 100003]:
        d = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        for seed in (0, 1, 2 ** 63 + 5):
            assert H().xxh64(d, seed) == xxhash.xxh64_intdigest(d, seed)


def test_malformed_streams_are_reported():
    rng = np.random.default_rng(3)
    data = b"".join(b"row %d: %s\n" % (i, bytes(rng.integers(97, 123, 20, dtype=np.uint8))) for i in range(5000))
    c = z(data, 3)
    Hm = H()
    outcomes = set()
    for trial in range(300):
        b = bytearray(c)
        k = trial % 3
        if k == 0:
            b = b[:int(rng.integers(1, len(b)))]
        elif k == 1:
            p = int(rng.integers(4, len(b)))
            b[p] ^= 1 << int(rng.integers(0, 8))
        else:
            p = int(rng.integers(4, len(b)))
            b[p] = int(rng.integers(0, 256))
        try:
            got = Hm.zstd_decompress(bytes(b))
            outcomes.add("ok")
            # a stream libzstd also accepts must decode to the same bytes
            try:
                ref = pa.Codec("zstd").decompress(bytes(b), decompressed_size=len(got), asbytes=True)
            except Exception:
                ref = None
            if ref is not None:
                assert got == ref
        except Hm.HaagentiError as e:
            assert e.code == Hm.CORRUPTED_DATA
            outcomes.add("err")
    assert "err" in outcomes
    with pytest.raises(Hm.HaagentiError):
        Hm.zstd_decompress(b"\x28\xb5\x2f\xfd")
    # a dictionary frame cannot be decoded without the dictionary
    d = bytearray(raw_frame(b"abc", False))
    d[4] |= 1
    d[5:5] = b"\x07"
    with pytest.raises(Hm.HaagentiError):
        Hm.zstd_decompress(bytes(d))


def block_modes(frame):
    """(block types, literal types, sequence table modes) of a one-frame
    stream, from the headers alone (RFC 8878 sections 3.1.1.2-3.1.1.3)."""
    p = 4
    fhd = frame[p]
    p += 1
    single, fcs_flag, did = (fhd >> 5) & 1, fhd >> 6, fhd & 3
    p += 0 if single else 1
    p += [0, 1, 2, 4][did]
    p += [1 if single else 0, 2, 4, 8][fcs_flag]
    btypes, ltypes, smodes = set(), set(), set()
    while True:
        bh = frame[p] | (frame[p + 1] << 8) | (frame[p + 2] << 16)
        p += 3
        last, bt, bs = bh & 1, (bh >> 1) & 3, bh >> 3
        btypes.add(bt)
        if bt == 2:
            b = frame[p:p + bs]
            lt, sf = b[0] & 3, (b[0] >> 2) & 3
            ltypes.add(lt)
            if lt in (0, 1):
                hdr = 1 if sf in (0, 2) else (2 if sf == 1 else 3)
                regen = (b[0] >> 3) if hdr == 1 else ((b[0] >> 4) + (b[1] << 4) if hdr == 2
                                                      else (b[0] >> 4) + (b[1] << 4) + (b[2] << 12))
                q = hdr + (regen if lt == 0 else 1)
            else:
                hdr = 3 if sf <= 1 else (4 if sf == 2 else 5)
                h = int.from_bytes(b[:hdr], "little")
                comp = {3: (h >> 14) & 0x3FF, 4: (h >> 18) & 0x3FFF, 5: (h >> 22) & 0x3FFFF}[hdr]
                q = hdr + comp
            n = b[q]
            q += 1 if n < 128 else (2 if n < 255 else 3)
            if n:
                m = b[q]
                smodes.update({m >> 6, (m >> 4) & 3, (m >> 2) & 3})
            p += bs
        else:
            p += 1 if bt == 1 else bs
        if last:
            return btypes, ltypes, smodes


def test_corpus_covers_every_mode():
    bt, lt, sm = set(), set(), set()
    for level in (-5, 1, 3, 9, 19):
        for _, data in contents():
            if data:
                a, b, c = block_modes(z(data, level))
                bt |= a
                lt |= b
                sm |= c
    assert bt >= {0, 1, 2}          # raw, RLE, compressed blocks
    assert lt >= {0, 2, 3}          # raw, Huffman, treeless literals (RLE: below)
    assert sm >= {0, 1, 2, 3}       # predefined, RLE, described, repeated tables


def test_rle_literal_sections():
    # compressed blocks whose literals section is RLE, in each of its three
    # header sizes, and no sequences; libzstd must accept them too
    for regen in (5, 31, 32, 1000, 4095, 4096, 70000):
        if regen < 32:
            lit = bytes([(regen << 3) | 1])
        elif regen < 4096:
            lit = bytes([((regen & 15) << 4) | (1 << 2) | 1, regen >> 4])
        else:
            lit = bytes([((regen & 15) << 4) | (3 << 2) | 1, (regen >> 4) & 0xFF, regen >> 12])
        body = lit + b"\x5a" + b"\x00"                    # the byte, then 0 sequences
        frame = struct.pack("<IB", 0xFD2FB528, (2 << 6) | (1 << 5)) + struct.pack("<I", regen)
        frame += struct.pack("<I", (len(body) << 3) | (2 << 1) | 1)[:3] + body
        want = b"\x5a" * regen
        assert pa.Codec("zstd").decompress(frame, decompressed_size=regen, asbytes=True) == want
        assert H().zstd_decompress(frame) == want
