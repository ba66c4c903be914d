"""C-ABI library: loads, exports every declared symbol, and its host-side
producer (Compressor side) is byte-identical to the oracle.  No GPU."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import haagenti_amd as H
import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "haagenti_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hh_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported():
    declared = _declared()
    assert len(declared) >= 15
    lib = C.CDLL(H.LIB_PATH)
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(H.EXPORTS) == declared


def test_status_categories_mirror_core_error():
    # crates/haagenti-core/src/error.rs:120-134
    assert H.category(H.CORRUPTED_DATA) == "corrupted_data"
    assert H.category(H.BUFFER_TOO_SMALL) == "buffer_too_small"
    assert H.category(H.UNEXPECTED_EOF) == "unexpected_eof"
    assert H.category(H.CHECKSUM_MISMATCH) == "checksum_mismatch"
    assert H.category(H.UNSUPPORTED) == "unsupported"
    assert H.category(H.ALGORITHM) == "algorithm_error"
    assert H.HaagentiError(H.UNEXPECTED_EOF).is_recoverable()
    assert H.HaagentiError(H.BUFFER_TOO_SMALL).is_recoverable()
    assert not H.HaagentiError(H.CORRUPTED_DATA).is_recoverable()
    # numeric values shared with the oracle's error kinds
    assert (H.CORRUPTED_DATA, H.BUFFER_TOO_SMALL, H.UNEXPECTED_EOF, H.ALGORITHM) == \
           (O.CORRUPTED, O.BUFFER_TOO_SMALL, O.UNEXPECTED_EOF, O.ALGORITHM)


def _lz4_inputs():
    rng = np.random.default_rng(21)
    yield b""
    yield b"Hello"
    yield b"A" * 40
    yield b"0123456789abcdef0123456vwxyz"
    yield (b"The quick brown fox jumps over the lazy dog. " * 300)[:10000]
    for n in [13, 100, 4096, 65536]:
        yield rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        yield rng.integers(0, 3, n, dtype=np.uint8).tobytes()
        a = rng.integers(0, 256, n, dtype=np.uint8)
        a[(np.arange(n) // 256) % 2 == 0] = 0
        yield a.tobytes()
    # config-2 style payload: packed INT4 nibbles of Gaussian weights
    w = rng.normal(0, 0.02, 2 * 65536).astype(np.float32)
    q = O.quantize_int4(w)
    yield q[:65536]
    z = np.frombuffer(q[:65536], np.uint8).copy()
    z[np.repeat(rng.random(256) < 0.5, 256)] = 0
    yield z.tobytes()


def test_lz4_compressor_byte_identical_to_oracle():
    comp = H.Lz4Compressor()
    for src in _lz4_inputs():
        mine = comp.compress(src)
        ref, e = O.lz4_compress_block(src)
        assert mine == ref, len(src)
        assert comp.max_compressed_size(len(src)) == O.lz4_max_compressed_size(len(src))


def test_lz4_compressor_buffer_too_small():
    out = C.create_string_buffer(4)
    w = C.c_size_t(0)
    rc = H.lib().hh_lz4_compress_block(b"Hello", 5, out, 4, C.byref(w))
    assert rc == H.BUFFER_TOO_SMALL and w.value == 7


def test_quantize_byte_identical_to_oracle():
    rng = np.random.default_rng(22)
    cases = [rng.normal(0, 0.02, n).astype(np.float32) for n in [1, 31, 32, 33, 97, 1000, 65537]]
    w = np.zeros(64, np.float32)
    w[0] = 7.005126953125
    w[33] = np.nan
    w[40] = np.inf
    cases.append(w)
    cases.append(np.array([(i - 50.0) / 10.0 for i in range(100)], np.float32))
    for w in cases:
        assert H.quantize_int4(w).tobytes() == O.quantize_int4(w)
    assert H.int4_compressed_size(33) == 21


def test_retain_count_and_tile_bytes():
    assert H.hctt_retain_count(0.3) == O.retain_count(4096, 0.3) == 1228
    assert H.hctt_retain_count(0.25) == 1024
    assert H.hctt_retain_count(0.01) == O.retain_count(4096, 0.01)
    assert H.hctt_tile_bytes(1228) == O.hctt_tile_bytes(1228) == 1204


def test_hctt_encoder_matches_oracle_encoder():
    # The producer computes dct_2d as the reference does (f32 Makhoul, rows
    # then columns) in the same order of operations as the oracle, so the
    # tiles are byte-identical, near-ties of the top-k selection included.
    rng = np.random.default_rng(23)
    w = rng.normal(0, 0.02, (128, 192)).astype(np.float32)
    # plus tiles with exact ties and special values: constant, a ramp,
    # zeros, a NaN, infinities and huge/tiny magnitudes
    w[:64, :64] = 0.5
    w[64:, :64] = np.arange(64, dtype=np.float32)[None, :] * 1e-3
    w[:64, 64:128] = 0.0
    w[70, 70] = np.nan
    w[:64, 128:] = rng.normal(0, 1e30, (64, 64)).astype(np.float32)
    w[64:, 128:] = rng.normal(0, 1e-30, (64, 64)).astype(np.float32)
    w[100, 150] = np.inf
    for k in [1, 1024, 1228, 2048, 4096]:
        mine = H.hctt_encode(w, k, threads=2)
        ref = O.hctt_encode_tensor(w, k, nthreads=2)
        assert mine.tobytes() == ref.tobytes(), k


def test_tile_encoder_matches_oracle_across_magnitudes():
    # single tiles whose values span 1e-6 .. 1e6: the f32 DCT, the top-k
    # selection and the f16 scales agree byte for byte at every scale
    rng = np.random.default_rng(29)
    for trial in range(8):
        t = rng.normal(0, 10.0 ** rng.integers(-6, 6), (64, 64)).astype(np.float32)
        assert H.hctt_encode(t, 4096).tobytes() == O.hctt_encode_tensor(t, 4096).tobytes()
        assert H.hctt_encode(t, 777).tobytes() == O.hctt_encode_tensor(t, 777).tobytes()


# ---------------------------------------------------------------- HCT header (host)
def test_hct_header_parse_matches_writer():
    import haagenti_amd as H
    f = O.hct_write_lz4(b"\x12" * 1000, 256, 4, [10, 100])
    h = H.HctReader(f).header()
    assert h == dict(version=1, algorithm=0, dtype=4, flags=0, original_size=1000,
                     compressed_size=h["compressed_size"], block_size=256, num_blocks=4,
                     shape=[10, 100])
    assert h["compressed_size"] == len(f) - 64 - 4 * 8


def test_hct_header_errors_match_oracle():
    import haagenti_amd as H
    f = O.hct_write_lz4(b"\x12" * 512, 256, 0, [512])
    cases = [f[:40], f[:68], b"XXXX" + f[4:], f[:4] + b"\x03" + f[5:], f[:8] + b"\x02" + f[9:],
             f[:9] + b"\x05" + f[10:], f[:36] + b"\x04" + f[37:]]
    for c in cases:
        _, e = O.hct_read_all_lz4(c, 1024)
        with pytest.raises(H.HaagentiError) as ei:
            H.HctReader(c)
        assert ei.value.code == e.kind, (c[:12], ei.value.code, e.kind)


def test_v1_writer_byte_identical_to_oracle():
    # HctWriter (tensor.rs:519-617) against the oracle's restatement, for
    # whole and ragged last blocks and ranks 0..3
    import haagenti_amd as H
    rng = np.random.default_rng(23)
    for n, bs, dtype, shape in [(70001, 16384, 3, [70001]), (4096, 1024, 4, [64, 32]),
                                (1000, 256, 0, [10, 10, 10]), (1, 16384, 2, []), (0, 16384, 1, [0])]:
        data = rng.integers(0, 6, n, dtype=np.uint8).tobytes()
        w = H.HctWriter(dtype, shape, bs)
        w.compress_data(data, H.Lz4Compressor())
        assert w.finish() == O.hct_write_lz4(data, bs, dtype, shape), (n, bs, shape)
        r = H.HctReader(w.finish())
        assert r.header()["shape"] == shape and r.header()["num_blocks"] == (n + bs - 1) // bs
    with pytest.raises(ValueError):
        H.HctWriter(0, [2, 2, 2, 2])


# ---------------------------------------------------------------- HCT v2 (host side)
def test_xxh3_host_matches_xxhash_library():
    xxhash = pytest.importorskip("xxhash")
    rng = np.random.default_rng(21)
    for n in list(range(0, 600)) + [1023, 1024, 1025, 4096, 16384, 65809]:
        d = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert H.xxh3_64(d) == xxhash.xxh3_64_intdigest(d) == O.xxh3_64(d)


def _v2_pair(data, block_size, dtype, shape, quant=None, checksums=True):
    w = H.HctWriterV2(dtype, shape, block_size)
    flags = O.FLAG_HEADER_CHECKSUM | (O.FLAG_BLOCK_CHECKSUMS if checksums else 0)
    if quant:
        w.with_quantization(**quant)
        flags |= O.FLAG_QUANTIZATION
    if not checksums:
        w.without_block_checksums()
    w.compress_data(data, H.Lz4Compressor())
    mine = w.finish()
    q8 = None
    if quant:
        q8 = mine[64:72]
    ref = O.hct_write_v2_lz4(data, block_size, dtype, shape, flags=flags, quant8=q8)
    return mine, ref


def test_v2_writer_byte_identical_to_oracle():
    rng = np.random.default_rng(22)
    data = rng.integers(0, 6, 70001, dtype=np.uint8).tobytes()
    mine, ref = _v2_pair(data, 16384, 3, [70001])
    assert mine == ref
    q = dict(scheme=1, group_size=128, scale_bits=0x3C00, zero_point=-8, has_per_group_scales=True)
    mine, ref = _v2_pair(data, 16384, 4, [271, 259], quant=q)
    assert mine == ref
    mine, ref = _v2_pair(data, 20000, 3, [70001], checksums=False)
    assert mine == ref


def test_v2_header_parse_checksum_and_quantization():
    data = bytes(i % 256 for i in range(4096))
    q = dict(scheme=1, group_size=128, scale_bits=0x3C00, zero_point=0, has_per_group_scales=False)
    f, _ = _v2_pair(data, 16384, 4, [4096], quant=q)
    r = H.HctReaderV2(f)   # tensor.rs:1367-1410
    assert r.quantization() == dict(scheme=1, group_size=128, scale_bits=0x3C00, zero_point=0,
                                    has_per_group_scales=False)
    assert r.header()["version"] == 2 and r.num_blocks() == 1
    r.validate_checksums()
    g = bytearray(f)
    g[20] ^= 1   # header byte: checksum mismatch (:857-865)
    with pytest.raises(H.HaagentiError) as e:
        H.HctReaderV2(bytes(g))
    assert e.value.code == H.CORRUPTED_DATA and e.value.status.detail == H.CORRUPT_HEADER_CHECKSUM
    g = bytearray(f)
    g[64] = 7    # unknown quantization scheme (:158-173); header checksum still valid
    with pytest.raises(H.HaagentiError) as e:
        H.HctReaderV2(bytes(g))
    assert e.value.status.detail == H.CORRUPT_QUANT_SCHEME


def test_v2_block_checksum_detects_corruption_on_host():
    # tensor.rs:1324-1364: byte 100 is inside the data of the one block
    data = bytes(i % 256 for i in range(16384))
    f, _ = _v2_pair(data, 16384, 3, [16384])
    g = bytearray(f)
    g[100] ^= 0xFF
    r = H.HctReaderV2(bytes(g))
    with pytest.raises(H.HaagentiError) as e:
        r.validate_checksums()
    assert e.value.code == H.CORRUPTED_DATA
    e2, fb = O.hct_validate_v2(bytes(g))
    assert e2.sub == O.CORRUPT_BLOCK_CHECKSUM and fb == 0


def test_import_without_the_hip_library_fails_loudly(tmp_path):
    # the package has no CPU fallback: without libhaagenti_hip.so it refuses
    # to import rather than decode on the host
    import shutil
    import subprocess
    import sys
    pkg = tmp_path / "haagenti_amd"
    pkg.mkdir()
    shutil.copy(H.__file__, pkg / "__init__.py")
    r = subprocess.run([sys.executable, "-c", "import haagenti_amd"], cwd=tmp_path, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "ImportError" in r.stderr and "no CPU fallback" in r.stderr
