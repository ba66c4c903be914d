"""ctypes bindings for the CPU oracle (oracle/libhh_oracle.so) and the
reference's own C decoder built into oracle/_ref/.

Test infrastructure: this module is the checker, never the thing measured.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "libhh_oracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libhct_ref.so")

OK, CORRUPTED, BUFFER_TOO_SMALL, UNEXPECTED_EOF, ALGORITHM = 0, 1, 2, 3, 6
CORRUPT_ZERO_OFFSET, CORRUPT_OFFSET_BEYOND, CORRUPT_BITMAP_COUNT, CORRUPT_HEADER = 1, 2, 3, 4


class Err(C.Structure):
    _fields_ = [("kind", C.c_int32), ("sub", C.c_int32), ("position", C.c_uint64),
                ("required", C.c_uint64), ("provided", C.c_uint64)]


def _ensure_built():
    if not os.path.exists(ORACLE_SO):
        subprocess.check_call(["make", "-s", "-C", ORACLE_DIR, "all"])


_lib = None


def lib():
    global _lib
    if _lib is None:
        _ensure_built()
        L = C.CDLL(ORACLE_SO)
        u8p, f32p, f64p = C.c_void_p, C.c_void_p, C.c_void_p
        sz = C.c_size_t
        L.hho_lz4_max_compressed_size.restype = sz
        L.hho_lz4_max_compressed_size.argtypes = [sz]
        L.hho_lz4_compress_block.restype = C.c_int
        L.hho_lz4_compress_block.argtypes = [u8p, sz, u8p, sz, C.POINTER(sz), C.POINTER(Err)]
        L.hho_lz4_decompress_block.restype = C.c_int
        L.hho_lz4_decompress_block.argtypes = [u8p, sz, u8p, sz, sz, C.POINTER(sz), C.POINTER(Err)]
        L.hho_lz4_decompress_batch.restype = None
        L.hho_lz4_decompress_batch.argtypes = [u8p, u8p, u8p, u8p, u8p, u8p, sz, u8p, u8p, C.c_int]
        L.hho_f32_to_f16_bits.restype = C.c_uint16
        L.hho_f32_to_f16_bits.argtypes = [C.c_float]
        L.hho_f16_bits_to_f32.restype = C.c_float
        L.hho_f16_bits_to_f32.argtypes = [C.c_uint16]
        L.hho_f16_bits_to_f32_bits.restype = None
        L.hho_f16_bits_to_f32_bits.argtypes = [u8p, sz, u8p]
        L.hho_int4_compressed_size.restype = sz
        L.hho_int4_compressed_size.argtypes = [sz]
        L.hho_quantize_int4.restype = sz
        L.hho_quantize_int4.argtypes = [f32p, sz, u8p]
        L.hho_dequantize_int4.restype = sz
        L.hho_dequantize_int4.argtypes = [u8p, sz, sz, f32p]
        L.hho_dequantize_int4_mt.restype = sz
        L.hho_dequantize_int4_mt.argtypes = [u8p, sz, sz, f32p, C.c_int]
        for name in ["hho_dct_1d", "hho_dct_1d_direct", "hho_idct_1d", "hho_idct_1d_direct",
                     "hho_dct_1d_f64", "hho_idct_1d_f64"]:
            getattr(L, name).restype = None
            getattr(L, name).argtypes = [f32p, f32p, sz]
        for name in ["hho_dct_2d", "hho_idct_2d", "hho_dct_2d_f64", "hho_idct_2d_f64",
                     "hho_reference_dct_2d", "hho_reference_idct_2d"]:
            getattr(L, name).restype = None
            getattr(L, name).argtypes = [f32p, f32p, sz, sz]
        L.hho_retain_count.restype = sz
        L.hho_retain_count.argtypes = [sz, C.c_float]
        L.hho_topk_bitmap.restype = None
        L.hho_topk_bitmap.argtypes = [f32p, sz, sz, u8p, u8p]
        L.hho_bitmap_index_map.restype = sz
        L.hho_bitmap_index_map.argtypes = [u8p, sz, u8p]
        L.hho_hctt_tile_bytes.restype = sz
        L.hho_hctt_tile_bytes.argtypes = [sz]
        L.hho_hctt_encode_tile.restype = None
        L.hho_hctt_encode_tile.argtypes = [f32p, sz, u8p]
        L.hho_hctt_decode_tile.restype = C.c_int
        L.hho_hctt_decode_tile.argtypes = [u8p, sz, f32p]
        L.hho_hctt_decode_tile_f64.restype = C.c_int
        L.hho_hctt_decode_tile_f64.argtypes = [u8p, sz, f64p]
        L.hho_hctt_encode_tensor.restype = None
        L.hho_hctt_encode_tensor.argtypes = [f32p, sz, sz, sz, u8p, C.c_int]
        L.hho_hctt_decode_tensor.restype = C.c_int
        L.hho_hctt_decode_tensor.argtypes = [u8p, sz, sz, sz, f32p, C.c_int]
        L.hho_hct_file_size.restype = sz
        L.hho_hct_file_size.argtypes = [sz, sz]
        L.hho_hct_write_lz4.restype = sz
        L.hho_hct_write_lz4.argtypes = [u8p, sz, C.c_uint32, C.c_uint8, u8p, C.c_int, u8p, sz]
        L.hho_hct_read_all_lz4.restype = C.c_int
        L.hho_hct_read_all_lz4.argtypes = [u8p, sz, u8p, sz, C.POINTER(sz), C.POINTER(Err)]
        L.hho_xxh3_64.restype = C.c_uint64
        L.hho_xxh3_64.argtypes = [u8p, sz]
        L.hho_xxh3_64_batch.restype = None
        L.hho_xxh3_64_batch.argtypes = [u8p, u8p, u8p, sz, u8p, C.c_int]
        L.hho_hct_write_v2_lz4.restype = sz
        L.hho_hct_write_v2_lz4.argtypes = [u8p, sz, C.c_uint32, C.c_uint8, u8p, C.c_int, C.c_uint16,
                                           u8p, u8p, sz]
        L.hho_hct_read_all_v2_lz4.restype = C.c_int
        L.hho_hct_read_all_v2_lz4.argtypes = [u8p, sz, u8p, sz, C.POINTER(sz), C.POINTER(Err),
                                              C.POINTER(C.c_int64)]
        L.hho_hct_validate_v2.restype = C.c_int
        L.hho_hct_validate_v2.argtypes = [u8p, sz, C.POINTER(Err), C.POINTER(C.c_int64)]
        L.hho_f32_to_f16_rne.restype = C.c_uint16
        L.hho_f32_to_f16_rne.argtypes = [C.c_float]
        L.hho_hct3_coefficients.restype = C.c_int
        L.hho_hct3_coefficients.argtypes = [u8p, sz, sz, f32p]
        L.hho_idct_2d_mt.restype = None
        L.hho_idct_2d_mt.argtypes = [f32p, f32p, sz, sz, C.c_int]
        L.hho_hct3_decode.restype = C.c_int
        L.hho_hct3_decode.argtypes = [u8p, sz, u8p, sz, f32p]
        L.hho_spectral_encode_from_dct.restype = sz
        L.hho_spectral_encode_from_dct.argtypes = [f32p, C.c_uint32, C.c_uint32, C.c_uint16, C.c_float,
                                                   C.c_float, u8p, sz, u8p]
        L.hho_spectral_reconstruct.restype = C.c_int
        L.hho_spectral_reconstruct.argtypes = [u8p, u8p, u8p, C.c_uint32, f32p, sz, C.POINTER(C.c_uint32),
                                               C.POINTER(C.c_uint32), C.POINTER(Err)]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a.size else C.c_void_p(0)


def _u8(b):
    return np.frombuffer(bytes(b), dtype=np.uint8).copy() if not isinstance(b, np.ndarray) \
        else np.ascontiguousarray(b, dtype=np.uint8)


# ---------------------------------------------------------------- LZ4
def lz4_max_compressed_size(n):
    return lib().hho_lz4_max_compressed_size(n)


def lz4_compress_block(data, cap=None):
    """Returns (bytes, err)."""
    src = _u8(data)
    cap = lz4_max_compressed_size(src.size) if cap is None else cap
    dst = np.zeros(max(cap, 1), dtype=np.uint8)
    w = C.c_size_t(0)
    e = Err()
    rc = lib().hho_lz4_compress_block(_p(src), src.size, _p(dst), cap, C.byref(w), C.byref(e))
    return (dst[:w.value].tobytes() if rc == OK else None), e


def lz4_decompress_block(data, out_len, output_size=None):
    """Returns (bytes_or_None, err).  out_len = output.len()."""
    src = _u8(data)
    output_size = out_len if output_size is None else output_size
    dst = np.zeros(max(out_len, 1), dtype=np.uint8)
    w = C.c_size_t(0)
    e = Err()
    rc = lib().hho_lz4_decompress_block(_p(src), src.size, _p(dst), out_len, output_size,
                                        C.byref(w), C.byref(e))
    return (dst[:w.value].tobytes() if rc == OK else None), e


def lz4_decompress_batch(comp, in_off, in_len, out_off, out_cap, total_out, nthreads=0):
    comp = _u8(comp)
    in_off = np.ascontiguousarray(in_off, dtype=np.uint64)
    in_len = np.ascontiguousarray(in_len, dtype=np.uint32)
    out_off = np.ascontiguousarray(out_off, dtype=np.uint64)
    out_cap = np.ascontiguousarray(out_cap, dtype=np.uint32)
    n = in_off.size
    out = np.zeros(total_out, dtype=np.uint8)
    kinds = np.zeros(n, dtype=np.int32)
    written = np.zeros(n, dtype=np.uint64)
    lib().hho_lz4_decompress_batch(_p(comp), _p(in_off), _p(in_len), _p(out), _p(out_off),
                                   _p(out_cap), n, _p(kinds), _p(written), nthreads)
    return out, kinds, written


# ---------------------------------------------------------------- INT4
def f32_to_f16_bits(v):
    return lib().hho_f32_to_f16_bits(float(v))


def f16_bits_to_f32(h):
    return np.float32(lib().hho_f16_bits_to_f32(int(h)))


def f16_bits_to_f32_bits(codes):
    c = np.ascontiguousarray(codes, dtype=np.uint16)
    out = np.zeros(c.size, dtype=np.uint32)
    lib().hho_f16_bits_to_f32_bits(_p(c), c.size, _p(out))
    return out


def int4_compressed_size(n):
    return lib().hho_int4_compressed_size(n)


def quantize_int4(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros(max(int4_compressed_size(w.size), 1), dtype=np.uint8)
    n = lib().hho_quantize_int4(_p(w), w.size, _p(out))
    return out[:n].tobytes()


def dequantize_int4(data, n, threads=None):
    d = _u8(data)
    out = np.zeros(max(n, 1), dtype=np.float32)
    if threads is None:
        m = lib().hho_dequantize_int4(_p(d), d.size, n, _p(out))
    else:
        m = lib().hho_dequantize_int4_mt(_p(d), d.size, n, _p(out), threads)
    return out[:m]


# ---------------------------------------------------------------- DCT
def _call1d(name, x, dtype):
    x = np.ascontiguousarray(x, dtype=dtype)
    out = np.zeros_like(x)
    getattr(lib(), name)(_p(x), _p(out), x.size)
    return out


def dct_1d(x):
    return _call1d("hho_dct_1d", x, np.float32)


def dct_1d_direct(x):
    return _call1d("hho_dct_1d_direct", x, np.float32)


def idct_1d(x):
    return _call1d("hho_idct_1d", x, np.float32)


def idct_1d_direct(x):
    return _call1d("hho_idct_1d_direct", x, np.float32)


def dct_1d_f64(x):
    return _call1d("hho_dct_1d_f64", x, np.float64)


def idct_1d_f64(x):
    return _call1d("hho_idct_1d_f64", x, np.float64)


def _call2d(name, x, dtype, width_height=True):
    x = np.ascontiguousarray(x, dtype=dtype)
    h, w = x.shape
    out = np.zeros_like(x)
    if width_height:
        getattr(lib(), name)(_p(x), _p(out), w, h)
    else:
        getattr(lib(), name)(_p(x), _p(out), h, w)
    return out


def dct_2d(x):
    return _call2d("hho_dct_2d", x, np.float32)


def idct_2d(x):
    return _call2d("hho_idct_2d", x, np.float32)


def dct_2d_f64(x):
    return _call2d("hho_dct_2d_f64", x, np.float64)


def idct_2d_mt(x, nthreads=0):
    """idct_2d on all host threads (bit-identical to idct_2d)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().hho_idct_2d_mt(_p(x), _p(out), x.shape[1], x.shape[0], int(nthreads))
    return out


def idct_2d_f64(x):
    return _call2d("hho_idct_2d_f64", x, np.float64)


def reference_dct_2d(x):
    return _call2d("hho_reference_dct_2d", x, np.float32, width_height=False)


def reference_idct_2d(x):
    return _call2d("hho_reference_idct_2d", x, np.float32, width_height=False)


# ---------------------------------------------------------------- retention / tiles
def retain_count(n, rho):
    return lib().hho_retain_count(n, float(rho))


def topk_bitmap(c, k):
    c = np.ascontiguousarray(c, dtype=np.float32).ravel()
    bm = np.zeros((c.size + 7) // 8, dtype=np.uint8)
    idx = np.zeros(max(k, 1), dtype=np.uint32)
    lib().hho_topk_bitmap(_p(c), c.size, k, _p(bm), _p(idx))
    return bm, idx[:k]


def bitmap_index_map(bm, n):
    bm = _u8(bm)
    idx = np.zeros(max(n, 1), dtype=np.uint32)
    m = lib().hho_bitmap_index_map(_p(bm), n, _p(idx))
    return idx[:m]


def hctt_tile_bytes(k):
    return lib().hho_hctt_tile_bytes(k)


def hctt_encode_tile(tile, k):
    t = np.ascontiguousarray(tile, dtype=np.float32)
    out = np.zeros(hctt_tile_bytes(k), dtype=np.uint8)
    lib().hho_hctt_encode_tile(_p(t), k, _p(out))
    return out


def hctt_decode_tile(tb, k, f64=False):
    tb = _u8(tb)
    out = np.zeros((64, 64), dtype=np.float64 if f64 else np.float32)
    fn = lib().hho_hctt_decode_tile_f64 if f64 else lib().hho_hctt_decode_tile
    rc = fn(_p(tb), k, _p(out))
    return rc, out


def hctt_encode_tensor(w, k, nthreads=0):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.zeros((rows // 64) * (cols // 64) * hctt_tile_bytes(k), dtype=np.uint8)
    lib().hho_hctt_encode_tensor(_p(w), rows, cols, k, _p(out), nthreads)
    return out


def hctt_decode_tensor(tiles, rows, cols, k, nthreads=0):
    t = _u8(tiles)
    out = np.zeros((rows, cols), dtype=np.float32)
    rc = lib().hho_hctt_decode_tensor(_p(t), rows, cols, k, _p(out), nthreads)
    return rc, out


# ---------------------------------------------------------------- HCT container
def hct_write_lz4(data, block_size, dtype, shape):
    d = _u8(data)
    nblocks = (d.size + block_size - 1) // block_size
    cap = 64 + 8 * nblocks + sum(lz4_max_compressed_size(min(block_size, d.size - i * block_size))
                                 for i in range(nblocks))
    out = np.zeros(cap, dtype=np.uint8)
    shp = np.ascontiguousarray(shape, dtype=np.uint64)
    n = lib().hho_hct_write_lz4(_p(d), d.size, block_size, dtype, _p(shp), len(shape), _p(out), cap)
    return out[:n].tobytes() if n else None


def hct_read_all_lz4(file_bytes, out_cap):
    f = _u8(file_bytes)
    out = np.zeros(max(out_cap, 1), dtype=np.uint8)
    w = C.c_size_t(0)
    e = Err()
    rc = lib().hho_hct_read_all_lz4(_p(f), f.size, _p(out), out_cap, C.byref(w), C.byref(e))
    return (out[:w.value].tobytes() if rc == OK else None), e


FLAG_HEADER_CHECKSUM, FLAG_BLOCK_CHECKSUMS, FLAG_QUANTIZATION = 1, 2, 4
CORRUPT_HEADER_CHECKSUM, CORRUPT_BLOCK_CHECKSUM, CORRUPT_QUANT_SCHEME = 6, 7, 8


def xxh3_64(data):
    d = _u8(data)
    return int(lib().hho_xxh3_64(_p(d), d.size))


def xxh3_64_batch(data, offs, lens, nthreads=0):
    d = _u8(data)
    o = np.ascontiguousarray(offs, dtype=np.uint64)
    ln = np.ascontiguousarray(lens, dtype=np.uint32)
    out = np.zeros(o.size, dtype=np.uint64)
    lib().hho_xxh3_64_batch(_p(d), _p(o), _p(ln), o.size, _p(out), nthreads)
    return out


def hct_write_v2_lz4(data, block_size, dtype, shape,
                     flags=FLAG_HEADER_CHECKSUM | FLAG_BLOCK_CHECKSUMS, quant8=None):
    d = _u8(data)
    nblocks = (d.size + block_size - 1) // block_size
    cap = 64 + 8 + 16 * nblocks + sum(lz4_max_compressed_size(min(block_size, d.size - i * block_size))
                                      for i in range(nblocks))
    out = np.zeros(cap, dtype=np.uint8)
    shp = np.ascontiguousarray(shape, dtype=np.uint64)
    q = _u8(quant8 if quant8 is not None else bytes(8))
    n = lib().hho_hct_write_v2_lz4(_p(d), d.size, block_size, dtype, _p(shp), len(shape), flags,
                                   _p(q), _p(out), cap)
    return out[:n].tobytes() if n else None


def hct_read_all_v2_lz4(file_bytes, out_cap):
    """Returns (data or None, err, failed_block)."""
    f = _u8(file_bytes)
    out = np.zeros(max(out_cap, 1), dtype=np.uint8)
    w = C.c_size_t(0)
    e = Err()
    fb = C.c_int64(-1)
    rc = lib().hho_hct_read_all_v2_lz4(_p(f), f.size, _p(out), out_cap, C.byref(w), C.byref(e),
                                       C.byref(fb))
    return (out[:w.value].tobytes() if rc == OK else None), e, fb.value


def hct_validate_v2(file_bytes):
    f = _u8(file_bytes)
    e = Err()
    fb = C.c_int64(-1)
    lib().hho_hct_validate_v2(_p(f), f.size, C.byref(e), C.byref(fb))
    return e, fb.value


# ---------------------------------------------------------------- reference C decoder
_ref = None


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        R = C.CDLL(REF_SO)
        R.hct_decode.restype = C.POINTER(C.c_float)
        R.hct_decode.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t]
        R.hct_idct_2d.restype = None
        R.hct_idct_2d.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t]
        R.hct_dct_2d.restype = None
        R.hct_dct_2d.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t]
        libc = C.CDLL(None)
        libc.free.argtypes = [C.c_void_p]
        R._free = libc.free
        _ref = R
    return _ref


def ref_idct_2d(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    ref().hct_idct_2d(_p(x), _p(out), x.shape[0], x.shape[1])
    return out


def ref_dct_2d(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    ref().hct_dct_2d(_p(x), _p(out), x.shape[0], x.shape[1])
    return out


def ref_hct_decode(data, rows, cols):
    d = _u8(data)
    ptr = ref().hct_decode(_p(d), d.size, rows, cols)
    if not ptr:
        return None
    out = np.ctypeslib.as_array(ptr, shape=(rows * cols,)).copy().reshape(rows, cols)
    ref()._free(C.cast(ptr, C.c_void_p))
    return out


# ------------------------------------------------------------- HCT3 spectral
INVALID_DATA, UNSUPPORTED = 7, 5


def f32_to_f16_rne(v):
    return int(lib().hho_f32_to_f16_rne(float(v)))


def hct3_coefficients(data, total):
    d = _u8(data)
    out = np.zeros(max(int(total), 1), np.float32)
    rc = lib().hho_hct3_coefficients(_p(d), d.size, int(total), _p(out))
    return rc, out[:int(total)]


def hct3_decode(data, shape):
    d = _u8(data)
    shp = np.ascontiguousarray(shape, dtype=np.uint64)
    total = int(np.prod(shape)) if len(shape) else 1
    out = np.zeros(max(total, 1), np.float32)
    rc = lib().hho_hct3_decode(_p(d), d.size, _p(shp), len(shape), _p(out))
    return rc, out[:total]


def spectral_encode_from_dct(dct, width, height, nfrag, retention, essential_ratio=0.2):
    c = np.ascontiguousarray(dct, dtype=np.float32).ravel()
    n = width * height
    cap = 24 + (n + 7) // 8 + 2 * n + 8 * nfrag + 16
    out = np.zeros(cap, np.uint8)
    offs = np.zeros(nfrag + 1, np.uint64)
    w = lib().hho_spectral_encode_from_dct(_p(c), width, height, nfrag, retention, essential_ratio,
                                           _p(out), cap, _p(offs))
    assert w > 0
    raw = out[:w].tobytes()
    return [(f, raw[int(offs[f]):int(offs[f + 1])]) for f in range(nfrag)]


def spectral_reconstruct(fragments, out_cap=None):
    """fragments: list of (index, bytes).  Returns (out, Err, width, height)."""
    bufs = [np.frombuffer(bytes(d), np.uint8).copy() if len(d) else np.zeros(1, np.uint8) for _, d in fragments]
    ptrs = np.array([b.ctypes.data for b in bufs], np.uint64)
    lens = np.array([len(d) for _, d in fragments], np.uint64)
    idx = np.array([i for i, _ in fragments], np.uint16)
    w, h, e = C.c_uint32(0), C.c_uint32(0), Err()
    if out_cap is None:
        d0 = bytes(fragments[0][1])
        out_cap = int.from_bytes(d0[4:8], "little") * int.from_bytes(d0[8:12], "little") if len(d0) >= 12 else 0
    out = np.zeros(max(out_cap, 1), np.float32)
    lib().hho_spectral_reconstruct(_p(ptrs), _p(lens), _p(idx), len(fragments), _p(out), out_cap,
                                   C.byref(w), C.byref(h), C.byref(e))
    return out[:w.value * h.value], e, w.value, h.value
