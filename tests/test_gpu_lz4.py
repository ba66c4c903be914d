"""Batched LZ4 block decode on the GPU vs the oracle
(crates/haagenti-lz4/src/block.rs:261-366): bit-exact bytes and identical
error records."""
import numpy as np
import pytest

import gpu_util as G
import oracle_lib as O

pytestmark = pytest.mark.gpu

# Every test runs on each decoder the batched entry point can dispatch to
# (the context's HH_OPT_LZ4_DECODER): the sequence-batched decoder with its
# 4 and 8 KiB rings, the one-sequence LDS-ring decoder with its 4 (the
# entry point's default), 8, 16 and 32 KiB rings, and the register-window
# decoder.
KERNELS = ["seq", "seq8", "ring4", "ring8", "ring16", "ring32", "window"]


@pytest.fixture(autouse=True, params=KERNELS)
def lz4_kernel(request):
    G.ctx().set_lz4_decoder(request.param)
    yield request.param
    G.ctx().set_lz4_decoder("auto")


def gpu_batch(streams, caps, in_pad=0, out_pad=0, in_align=0, out_align=0):
    """Decode independent blocks in one launch.  Returns (outputs, statuses)."""
    import haagenti_amd as H
    T = G.torch()
    in_off, pos = [], in_align
    for s in streams:
        in_off.append(pos)
        pos += len(s) + in_pad
    comp = np.zeros(max(pos, 1), np.uint8)
    for o, s in zip(in_off, streams):
        comp[o:o + len(s)] = np.frombuffer(bytes(s), np.uint8)
    out_off, opos = [], out_align
    for c in caps:
        out_off.append(opos)
        opos += c + out_pad
    d_in = G.dev(comp)
    d_out = T.full((max(opos, 1),), 0xA5, dtype=T.uint8, device="cuda")
    d_in_off = G.dev(np.array(in_off, np.uint64))
    d_in_len = G.dev(np.array([len(s) for s in streams], np.uint32))
    d_out_off = G.dev(np.array(out_off, np.uint64))
    d_out_cap = G.dev(np.array(caps, np.uint32))
    d_status = T.zeros(len(streams) * 32, dtype=T.uint8, device="cuda")
    rc = G.ctx().lz4_decompress_batch(d_in, comp.size, d_in_off, d_in_len, d_out, d_out_off,
                                      d_out_cap, len(streams), d_status, stream=G.stream())
    assert rc == H.OK
    G.sync()
    st = np.frombuffer(G.host_u8(d_status).tobytes(), dtype=np.dtype(
        [("code", "<i4"), ("detail", "<i4"), ("position", "<u8"), ("required", "<u8"),
         ("written", "<u8")]))
    out = G.host_u8(d_out)
    outs = [out[o:o + int(s["written"])].tobytes() for o, s in zip(out_off, st)]
    # bytes beyond `written` inside each block's capacity, and the padding
    # between blocks, must be untouched (0xA5) -- nothing written out of range
    for o, c, s in zip(out_off, caps, st):
        if s["code"] == 0:
            assert (out[o + int(s["written"]):o + c] == 0xA5).all()
    if out_pad:
        for o, c in zip(out_off, caps):
            assert (out[o + c:o + c + out_pad] == 0xA5).all()
    return outs, st


def check_against_oracle(streams, caps, **kw):
    outs, st = gpu_batch(streams, caps, **kw)
    for s, c, o, r in zip(streams, caps, outs, st):
        ref, e = O.lz4_decompress_block(s, c)
        assert r["code"] == e.kind, (r, e.kind)
        if e.kind == O.OK:
            assert o == ref
        else:
            assert r["detail"] == e.sub
            assert r["position"] == e.position
            assert r["required"] == e.required
    return outs, st


def test_reference_inputs_roundtrip():
    srcs = [b"Hello", b"A" * 40, b"Hello, World! Hello, World! Hello, World! This is a test.",
            (b"The quick brown fox jumps over the lazy dog. " * 300)[:10000],
            (b"ABCDEFGH" * 200)[:1000], b"", b"x"]
    streams = [O.lz4_compress_block(s)[0] for s in srcs]
    outs, st = check_against_oracle(streams, [len(s) for s in srcs])
    assert outs == srcs


def test_hand_written_streams_and_errors():
    cases = [
        (bytes([0x14, 0x78, 0x01, 0x00, 0x10, 0x79]), 10),
        (bytes([0x35]) + b"abc" + bytes([0x03, 0x00, 0x00]), 12),
        (bytes([0xF0, 0xFF, 0x00]) + bytes(range(256)) + bytes(range(14)), 270),
        (bytes([0x1F, 0x7A, 0x01, 0x00, 0xFF, 0x01]), 276),
        (bytes([0x14, 0x78, 0x01, 0x00]), 20),                  # short block: success
        (bytes([0x10, 0x61, 0x00, 0x00]), 10),                  # zero offset
        (bytes([0x10, 0x61, 0x02, 0x00]), 10),                  # offset beyond output
        (bytes([0xF0]), 10),                                    # eof in literal length
        (bytes([0x30, 0x61]), 10),                              # eof in literals
        (bytes([0x10, 0x61, 0x01]), 10),                        # eof in offset
        (bytes([0x1F, 0x61, 0x01, 0x00]), 100),                 # eof in match length
        (bytes([0x30, 0x61, 0x62, 0x63]), 2),                   # literal overflow
        (bytes([0x14, 0x78, 0x01, 0x00]), 5),                   # match overflow
        (bytes([0x30, 0x61, 0x62, 0x63]), 10),                  # eof after literals
        (b"\x00", 0),
    ]
    check_against_oracle([c[0] for c in cases], [c[1] for c in cases], out_pad=7)


def _config2_sources(rng, nsrc):
    """Block contents as in the 64 KiB LZ4 benchmark: packed INT4 nibbles of
    N(0, 0.02) weights, or the same with half of the 256-byte spans zeroed."""
    import haagenti_amd as H
    out = []
    for i in range(nsrc):
        w = rng.normal(0, 0.02, 131072).astype(np.float32)
        q = H.quantize_int4(w)
        nib = q[2 * 4096:].copy()
        assert nib.size == 65536
        if i % 2:
            nib[np.repeat(rng.random(256) < 0.5, 256)] = 0
        out.append(nib.tobytes())
    return out


def test_config2_blocks_vs_oracle():
    import haagenti_amd as H
    rng = np.random.default_rng(2)
    srcs = _config2_sources(rng, 16)
    comp = [H.Lz4Compressor().compress(s) for s in srcs]
    ratios = [len(s) / len(c) for s, c in zip(srcs, comp)]
    assert min(ratios[1::2]) > 1.5  # zeroed spans compress
    outs, st = check_against_oracle(comp, [65536] * len(comp))
    assert outs == srcs


def test_config2_full_256MiB_roundtrip():
    # 4096 x 64 KiB blocks; every block must come back bit-identical.
    import haagenti_amd as H
    rng = np.random.default_rng(3)
    srcs = _config2_sources(rng, 64)
    comp = [H.Lz4Compressor().compress(s) for s in srcs]
    pick = rng.integers(0, 2, 4096) + 2 * rng.integers(0, 32, 4096)   # seeded coin per block
    streams = [comp[i] for i in pick]
    outs, st = gpu_batch(streams, [65536] * 4096)
    assert (st["code"] == 0).all() and (st["written"] == 65536).all()
    for i, o in zip(pick, outs):
        assert o == srcs[i]


def test_unaligned_offsets_and_padding():
    rng = np.random.default_rng(4)
    srcs = []
    for n in [1, 15, 16, 17, 63, 64, 65, 255, 1000, 4097, 20000]:
        a = rng.integers(0, 4, n, dtype=np.uint8)
        a[rng.random(n) < 0.3] = 0
        srcs.append(a.tobytes())
    streams = [O.lz4_compress_block(s)[0] for s in srcs]
    for in_align, out_align, in_pad, out_pad in [(1, 3, 5, 9), (2, 1, 0, 1), (3, 7, 13, 0)]:
        outs, st = check_against_oracle(streams, [len(s) for s in srcs], in_align=in_align,
                                        out_align=out_align, in_pad=in_pad, out_pad=out_pad)
        assert outs == srcs


def test_overlapping_match_periods():
    # offset 1..70 with long matches: periodic copies of every period
    streams, srcs = [], []
    for off in list(range(1, 20)) + [31, 32, 33, 63, 64, 65, 70]:
        lit = bytes((i * 29 + off) & 0xFF for i in range(off))
        ml = 300 + off
        s = bytes([0xFF if off >= 15 else (off << 4) | 15])
        if off >= 15:
            s = bytes([0xFF, off - 15])
        s += lit + bytes([off & 0xFF, off >> 8, 255, ml - 4 - 15 - 255])
        out = bytearray(lit)
        for j in range(ml):
            out.append(out[len(out) - off])
        streams.append(s)
        srcs.append(bytes(out))
    outs, st = check_against_oracle(streams, [len(x) for x in srcs])
    assert outs == srcs


def test_corrupted_stream_fuzz():
    rng = np.random.default_rng(5)
    base = []
    for n in [100, 1000, 5000]:
        a = rng.integers(0, 3, n, dtype=np.uint8).tobytes()
        base.append((O.lz4_compress_block(a)[0], n))
    streams, caps = [], []
    for trial in range(300):
        s, n = base[trial % len(base)]
        b = bytearray(s)
        kind = trial % 3
        if kind == 0:
            for _ in range(int(rng.integers(1, 4))):
                b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        elif kind == 1:
            b = b[:int(rng.integers(0, len(b)))]
        else:
            b[int(rng.integers(0, len(b)))] ^= 0xFF
        streams.append(bytes(b))
        caps.append(n if trial % 5 else int(rng.integers(0, n + 1)))
    check_against_oracle(streams, caps, out_pad=3)


def test_ring_boundaries_far_long_and_periodic_copies():
    # Streams from the oracle compressor whose matches sit on the ring
    # decoder's limits: offsets just below / above what each ring serves
    # (R - 32 for R = 4, 8, 16, 32 KiB), literals longer than the input stage,
    # matches longer than the ring (periodic and not), and far matches that
    # overlap their own output.
    rng = np.random.default_rng(6)
    srcs = []
    for L in [100, 992, 993, 2047, 2049, 4063, 4065, 4097, 8159, 8161, 8200, 16351, 16353, 32735, 32737,
              40000]:
        a = rng.integers(0, 256, L, dtype=np.uint8).tobytes()
        srcs.append(a + a)                                     # one match at offset L
    srcs.append(rng.integers(0, 256, 70000, dtype=np.uint8).tobytes())   # one 70 KB literal
    srcs.append(bytes(200000))                                # offset-1 match of ~200 KB
    srcs.append(bytes((i * 7) & 0xFF for i in range(40)) * 500)          # offset 40, 20 KB
    a = rng.integers(0, 256, 10000, dtype=np.uint8).tobytes()
    srcs.append(a * 6)                                        # offset 10000, 60 KB (overlapping)
    streams = [O.lz4_compress_block(x)[0] for x in srcs]
    for out_align in (0, 5, 11):
        outs, st = check_against_oracle(streams, [len(x) for x in srcs], out_align=out_align,
                                        in_align=out_align % 4, out_pad=17)
        assert outs == srcs


def _lz4_len(n):
    """Extension bytes of a length field whose nibble is 15 (block.rs:277-289)."""
    out = bytearray()
    n -= 15
    while n >= 255:
        out.append(255)
        n -= 255
    out.append(n)
    return bytes(out)


def _seq(lit, off=None, ml=None):
    """One LZ4 sequence; a literal-only last sequence when off is None."""
    mn = 0 if off is None else min(ml - 4, 15)
    s = bytearray([(min(len(lit), 15) << 4) | mn])
    if len(lit) >= 15:
        s += _lz4_len(len(lit))
    s += lit
    if off is not None:
        s += bytes([off & 0xFF, off >> 8])
        if ml - 4 >= 15:
            s += _lz4_len(ml - 4)
    return bytes(s)


def test_long_literals_then_matches_into_them():
    # Literals of 2 KiB and more (the ring decoder copies those straight
    # from the input to the output and keeps only their tail in the ring),
    # each followed by matches whose sources lie in the literal, just inside
    # and just outside the ring's reach (offset R - 32 = 4064 for 4 KiB),
    # before the literal, and periodic; blocks that end with a long literal;
    # and capacities that end inside a long literal or right after it.
    rng = np.random.default_rng(7)
    streams, caps = [], []
    for L in [2048, 2049, 3000, 4064, 4065, 4100, 9000, 20000]:
        for off_kind in range(6):
            head = rng.integers(0, 256, 37, dtype=np.uint8).tobytes()
            lit = rng.integers(0, 256, L, dtype=np.uint8).tobytes()
            off = {0: 1, 1: 17, 2: min(L, 4064), 3: min(L + 30, 4065), 4: L + 30, 5: L // 2}[off_kind]
            ml = [4, 19, 300, 5000][off_kind % 4]
            tail = rng.integers(0, 256, 2500 + 13 * off_kind, dtype=np.uint8).tobytes()
            streams.append(_seq(head, 3, 40) + _seq(lit, off, ml) + _seq(b"xy", 2100, 64) + _seq(tail))
            caps.append(37 + 40 + L + ml + 2 + 64 + len(tail))
    # exact sizes (the block ends with its literal), a cap inside the long
    # literal, and one right after it (early stop: block.rs:309-311)
    lit = rng.integers(0, 256, 6000, dtype=np.uint8).tobytes()
    s = _seq(b"ab", 1, 100) + _seq(lit, 50, 20) + _seq(lit[:3000])
    streams += [s, s, s]
    caps += [102 + 6000 + 20 + 3000, 102 + 3000, 102 + 6000]
    for out_align in (0, 1, 7, 15):
        check_against_oracle(streams, caps, out_align=out_align, in_align=out_align % 3, out_pad=5)


def test_lengths_beyond_32_bits():
    # runs of ~2^24 0xFF extension bytes: lengths just below and above 2^32;
    # a literal that long fails the input-length check, a match that long
    # the capacity check, with the exact 64-bit required size
    streams, want = [], []
    for nrun in ((1 << 24) + 10, (1 << 24) + (1 << 18)):
        run = b"\xff" * nrun
        streams += [bytes([0xF0]) + run + b"\x00" + b"tail", bytes([0x1F]) + b"a" + b"\x01\x00" + run + b"\x00"]
        want.append(1 + 19 + 255 * nrun)
    assert want[0] < 1 << 32 < want[1]
    outs, st = check_against_oracle(streams, [1 << 20] * 4)
    assert [r["code"] for r in st] == [O.UNEXPECTED_EOF, O.BUFFER_TOO_SMALL] * 2
    assert [st[1]["required"], st[3]["required"]] == want


def _reference_decompress(data):
    """Lz4Decompressor::decompress (crates/haagenti-lz4/src/decompress.rs:33-57)
    on the oracle: 4x the input first, max(required, 2x) on BufferTooSmall,
    a 256 MiB limit.  Returns (bytes or None, error kind, attempts).  Note
    that decompress_block only stops early when the output reaches the size
    it is given, so a stream that ends with literals and decodes to less
    than that size runs on into a missing match offset (UnexpectedEof): the
    size-unknown call succeeds only for streams ending with a match."""
    size, tries = len(data) * 4, 0
    while True:
        tries += 1
        out, e = O.lz4_decompress_block(data, size)
        if e.kind == O.OK:
            return out, O.OK, tries
        if e.kind != O.BUFFER_TOO_SMALL:
            return None, e.kind, tries
        size = max(int(e.required), size * 2)
        if size > 256 * 1024 * 1024:
            return None, O.CORRUPTED, tries


def _gpu_decompress(d, c):
    import haagenti_amd as H
    try:
        return d.decompress(c), O.OK
    except H.HaagentiError as e:
        return None, e.code


def test_decompressor_size_unknown_grows_like_the_reference():
    import haagenti_amd as H
    d = H.Lz4Decompressor(G.ctx())
    rng = np.random.default_rng(8)
    # streams ending with a match: one literal then an offset-1 match
    ends_with_match = [bytes([0x1F]) + b"a" + b"\x01\x00" + b"\xff" * n + b"\x07" for n in (0, 3, 400)]
    # two sequences, the second ending with a periodic match of period 3
    ends_with_match.append(bytes([0x3F]) + b"xyz" + b"\x03\x00" + b"\xff" * 50 + b"\x00")
    cases = [(s, True) for s in ends_with_match]
    for src in [b"", rng.integers(0, 4, 5000, dtype=np.uint8).tobytes(), bytes(200000)]:
        cases.append((O.lz4_compress_block(src)[0], False))
    cases.append((b"", True))                    # no input: an empty output
    for c, ok in cases:
        ref, kind, tries = _reference_decompress(c)
        assert (kind == O.OK) == ok, (c[:8], kind)
        got, gkind = _gpu_decompress(d, c)
        assert gkind == kind and got == ref
        if ok and len(c) > 10:
            assert tries >= 2        # the 4x estimate was short
        # decompress_with_size at the true size succeeds for every stream
        if ref is not None:
            assert d.decompress_with_size(c, len(ref)) == ref
    src = bytes(200000)
    c = O.lz4_compress_block(src)[0]
    assert d.decompress_with_size(c, len(src)) == src
    assert _reference_decompress(c)[2] == 3      # grew twice, then ran past the last literals


def test_decompressor_size_unknown_limit():
    # one literal, then an offset-1 match longer than 256 MiB: the first
    # attempt (4x the input) reports the required size, which exceeds the
    # limit -> CorruptedData("decompressed size exceeds limit")
    import haagenti_amd as H
    nrun = (1 << 28) // 255 + 1
    c = bytes([0x1F]) + b"a" + b"\x01\x00" + b"\xff" * nrun + b"\x00"
    ref, kind, tries = _reference_decompress(c)
    assert ref is None and kind == O.CORRUPTED and tries == 1
    with pytest.raises(H.HaagentiError) as ei:
        H.Lz4Decompressor(G.ctx()).decompress(c)
    assert ei.value.code == H.CORRUPTED_DATA
