"""haagenti_amd -- MI355X (gfx950) HCT decode path behind a C ABI.

Python mirror of the reference's decode interfaces, calling
libhaagenti_hip.so through ctypes:

  Lz4Decompressor   haagenti_core::Decompressor for raw LZ4 blocks
                    (crates/haagenti-core/src/traits.rs:56-91,
                    crates/haagenti-lz4/src/decompress.rs:28-68), decoded on GPU
  Lz4Compressor     Compressor side (crates/haagenti-lz4/src/compress.rs:59-99)
  HipContext        GpuContext / GpuDctContext (crates/haagenti-cuda/src/lib.rs:89-230,
                    dct_gpu.rs): idct_2d / dct_2d of whole matrices
  GpuDecompressor   HCT V3 fragment containers decoded on the GPU
                    (crates/haagenti-cuda/src/decompress.rs:108-443)
  CompressiveSpectralDecoder / CompressiveSpectralEncoder
                    crates/haagenti/src/compressive.rs:67-752
  HaagentiError     haagenti_core::Error (crates/haagenti-core/src/error.rs:10-135)

Device entry points take torch tensors (or raw device addresses) for
device memory; torch is only the allocator and stream provider.  There is
no CPU fallback: importing without the built library raises.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhaagenti_hip.so")

OK = 0
CORRUPTED_DATA = 1
BUFFER_TOO_SMALL = 2
UNEXPECTED_EOF = 3
CHECKSUM_MISMATCH = 4
UNSUPPORTED = 5
ALGORITHM = 6
INVALID_ARGUMENT = 7
OUT_OF_MEMORY = 8
DEVICE = 9
KERNEL_LAUNCH = 10
DEVICE_NOT_FOUND = 11

CORRUPT_ZERO_OFFSET = 1
CORRUPT_OFFSET_BEYOND = 2
CORRUPT_BITMAP_COUNT = 3

F32, F16, BF16 = 0, 1, 2

# hh_context_set_option options, LZ4 decoders and whole-matrix transform
# routes (diagnostics and tests)
OPT_LZ4_DECODER, OPT_FUSED_POLL_LIMIT, OPT_DCT_ROUTE, OPT_PIPELINE_ROUTE = 1, 2, 3, 4
LZ4_DECODERS = {"auto": 0, "seq": 1, "seq8": 2, "ring4": 3, "ring8": 4, "ring16": 5, "ring32": 6, "window": 7}
DCT_ROUTES = {"auto": 0, "dense": 1, "fft": 2}
PIPELINE_ROUTES = {"auto": 0, "two-launch": 1, "fused": 2}


class BlockStatus(C.Structure):
    _fields_ = [("code", C.c_int32), ("detail", C.c_int32), ("position", C.c_uint64),
                ("required", C.c_uint64), ("written", C.c_uint64)]


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run `python haagenti_amd/build.py` "
        "(the HIP extension is required, there is no CPU fallback)")

try:
    # torch ships its own HIP runtime under the same soname
    # (libamdhip64.so.7).  Loading torch first makes this library bind to
    # that copy, so the process has one HIP runtime and torch's streams and
    # allocations are valid here.
    import torch  # noqa: F401
except ImportError:
    pass

_lib = C.CDLL(LIB_PATH)
_vp, _sz, _i32, _u32 = C.c_void_p, C.c_size_t, C.c_int32, C.c_uint32


def _sig(name, res, args):
    f = getattr(_lib, name)
    f.restype = res
    f.argtypes = args
    return f


_sig("hh_status_category", C.c_char_p, [_i32])
_sig("hh_status_is_recoverable", _i32, [_i32])
_sig("hh_version", C.c_char_p, [])
_sig("hh_device_count", _i32, [])
_sig("hh_context_create", _i32, [_i32, C.POINTER(_vp)])
_sig("hh_context_destroy", None, [_vp])
_sig("hh_context_stream", _vp, [_vp])
_sig("hh_context_synchronize", _i32, [_vp])
_sig("hh_context_set_option", _i32, [_vp, _i32, C.c_int64])
_sig("hh_lz4_decompress_batch", _i32, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _vp])
_sig("hh_lz4_decompress_to", _i32, [_vp, _vp, _sz, _vp, _sz, C.POINTER(_sz), C.POINTER(BlockStatus)])
_sig("hh_lz4_compress_block", _i32, [_vp, _sz, _vp, _sz, C.POINTER(_sz)])
_sig("hh_lz4_max_compressed_size", _sz, [_sz])
_sig("hh_dequant_int4", _i32, [_vp, _vp, _sz, _sz, _i32, _vp, C.POINTER(_sz), _vp])
_sig("hh_quantize_int4", _sz, [_vp, _sz, _vp])
_sig("hh_int4_compressed_size", _sz, [_sz])
_sig("hh_hctt_tile_bytes", _sz, [_u32])
_sig("hh_hctt_retain_count", _u32, [C.c_float])
_sig("hh_hctt_decode", _i32, [_vp, _vp, _sz, _u32, _u32, _u32, _i32, _vp, _vp, _vp])
_sig("hh_hctt_encode", _i32, [_vp, _u32, _u32, _u32, _vp, _i32])


class HcttTensor(C.Structure):
    """hh_hctt_tensor: one tensor of a batched tile decode."""
    _fields_ = [("d_tiles", _vp), ("tiles_len", _sz), ("rows", _u32), ("cols", _u32),
                ("k", _u32), ("d_out", _vp), ("d_tile_status", _vp)]


_sig("hh_hctt_decode_batch", _i32, [_vp, C.POINTER(HcttTensor), _u32, _i32, _vp])
_sig("hh_hctt_decode_lz4_batch", _i32, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _u32, _vp, C.POINTER(HcttTensor), _u32,
                                        _i32, _vp])
_sig("hh_hctt_decode_lz4_batch_noalloc", _i32, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, _u32, _vp, C.POINTER(HcttTensor),
                                                _u32, _i32, _vp])
NOALLOC_SCRATCH_BYTES = 64 << 20
_sig("hh_hctt_decode_lz4_fused", _i32, [_vp, _vp, _sz, _vp, _vp, _u32, _vp, C.POINTER(HcttTensor), _u32, _u32,
                                        _i32, _vp])
_sig("hh_hctt_decode_lz4_fused_tpb", _i32, [_vp, _vp, _sz, _vp, _vp, _u32, _vp, C.POINTER(HcttTensor), _u32,
                                            C.POINTER(_u32), _i32, _vp])
FUSED_BLOCK_BYTES = 16352


class PoolStats(C.Structure):
    """hh_pool_stats: PoolStats (crates/haagenti-cuda/src/memory.rs:341-347)."""
    _fields_ = [("total_size", C.c_uint64), ("allocated", C.c_uint64), ("available", C.c_uint64),
                ("free_buffers", C.c_uint64), ("free_buffer_bytes", C.c_uint64), ("largest_free", C.c_uint64)]


class PipelineConfig(C.Structure):
    """hh_pipeline_config: PipelineConfig (crates/haagenti-cuda/src/pipeline.rs:35-60)."""
    _fields_ = [("num_staging_buffers", _u32), ("max_blocks", _u32), ("staging_buffer_size", C.c_uint64),
                ("tile_scratch_size", C.c_uint64), ("use_pinned_memory", _u32), ("copy_threads", _u32)]


class PipelineStats(C.Structure):
    """hh_pipeline_stats: PipelineStats (pipeline.rs:121-128)."""
    _fields_ = [("blocks_processed", C.c_uint64), ("bytes_read", C.c_uint64), ("bytes_decompressed", C.c_uint64),
                ("transfer_time_ns", C.c_uint64), ("decompress_time_ns", C.c_uint64), ("units", C.c_uint64),
                ("bytes_output", C.c_uint64)]


class PipelineTimes(C.Structure):
    """hh_pipeline_times: a unit's copy and decode intervals (ms since creation)."""
    _fields_ = [("h2d_start_ms", C.c_double), ("h2d_end_ms", C.c_double), ("decode_start_ms", C.c_double),
                ("decode_end_ms", C.c_double)]


_sig("hh_pinned_alloc", _i32, [_sz, C.POINTER(_vp)])
_sig("hh_pinned_free", _i32, [_vp])
_sig("hh_pool_create", _i32, [_vp, _sz, C.POINTER(_vp)])
_sig("hh_pool_destroy", None, [_vp])
_sig("hh_pool_allocate", _i32, [_vp, _sz, _i32, C.POINTER(_vp)])
_sig("hh_pool_recycle", _i32, [_vp, _vp])
_sig("hh_pool_get_stats", _i32, [_vp, C.POINTER(PoolStats)])
_sig("hh_pipeline_default_config", None, [C.POINTER(PipelineConfig)])
_sig("hh_pipeline_create", _i32, [_vp, _vp, C.POINTER(PipelineConfig), C.POINTER(_vp)])
_sig("hh_pipeline_destroy", None, [_vp])
_sig("hh_pipeline_streams", _i32, [_vp, C.POINTER(_vp), C.POINTER(_vp)])
_sig("hh_pipeline_next_staging", _i32, [_vp, C.POINTER(_vp), C.POINTER(_sz)])
_sig("hh_pipeline_submit", _i32, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, _u32, _vp, C.c_uint64,
                                  C.POINTER(HcttTensor), _u32, _i32, _vp, C.POINTER(C.c_uint64)])
_sig("hh_pipeline_wait", _i32, [_vp, C.c_uint64, _vp, C.POINTER(C.c_int64)])
_sig("hh_pipeline_stream_wait", _i32, [_vp, C.c_uint64, _vp])
_sig("hh_pipeline_get_times", _i32, [_vp, C.c_uint64, C.POINTER(PipelineTimes)])
_sig("hh_pipeline_finish", _i32, [_vp, _vp, C.POINTER(C.c_int64), C.POINTER(C.c_uint64)])
_sig("hh_pipeline_get_stats", _i32, [_vp, C.POINTER(PipelineStats)])
_sig("hh_pipeline_reset_stats", None, [_vp])


class HctInfo(C.Structure):
    """hh_hct_info: HCT v1 header fields (crates/haagenti-hct/src/tensor.rs:275-375)."""
    _fields_ = [("version", C.c_uint32), ("algorithm", C.c_uint8), ("dtype", C.c_uint8),
                ("flags", C.c_uint16), ("original_size", C.c_uint64),
                ("compressed_size", C.c_uint64), ("block_size", C.c_uint32),
                ("num_blocks", C.c_uint32), ("rank", C.c_uint32), ("index_entry_size", C.c_uint32),
                ("shape", C.c_uint64 * 4), ("data_offset", C.c_uint64)]


class HctQuant(C.Structure):
    """hh_hct_quant: QuantizationMetadata of HCT v2 (tensor.rs:180-226)."""
    _fields_ = [("present", C.c_uint8), ("scheme", C.c_uint8), ("has_per_group_scales", C.c_uint8),
                ("zero_point", C.c_int8), ("scale_bits", C.c_uint16), ("pad", C.c_uint16),
                ("group_size", C.c_uint32)]


_sig("hh_hct_read_header", _i32, [_vp, _sz, C.POINTER(HctInfo), C.POINTER(BlockStatus)])
_sig("hh_hct_read_header_v2", _i32, [_vp, _sz, C.POINTER(HctInfo), C.POINTER(HctQuant),
                                      C.POINTER(BlockStatus)])
_sig("hh_hct_decompress_all_validated", _i32, [_vp, _vp, _vp, _sz, _vp, _sz, C.POINTER(_sz),
                                                C.POINTER(BlockStatus), C.POINTER(C.c_int64), _vp])
_sig("hh_hct_validate_checksums", _i32, [_vp, _vp, _vp, _sz, C.POINTER(BlockStatus),
                                          C.POINTER(C.c_int64), _vp])
_sig("hh_xxh3_64", C.c_uint64, [_vp, _sz])
_sig("hh_xxh3_64_batch", _i32, [_vp, _vp, _sz, _vp, _vp, _u32, _vp, _vp])
_sig("hh_hct_decompress_all", _i32, [_vp, _vp, _vp, _sz, _vp, _sz, C.POINTER(_sz),
                                      C.POINTER(BlockStatus), C.POINTER(C.c_int64), _vp])

_sig("hh_hct3_coefficients", _i32, [_vp, _vp, _sz, C.c_uint64, _vp, _vp])
_sig("hh_hct3_decompress", _i32, [_vp, _vp, _sz, _vp, _u32, _i32, _vp, _vp])
_sig("hh_hct3_decompress_device", _i32, [_vp, _vp, _vp, _sz, _vp, _u32, _i32, _vp, _vp])
_sig("hh_spectral_reconstruct", _i32, [_vp, _vp, _vp, _vp, _u32, _i32, _vp, C.c_uint64,
                                       C.POINTER(_u32), C.POINTER(_u32), C.POINTER(BlockStatus), _vp])
_sig("hh_idct_2d", _i32, [_vp, _vp, _u32, _u32, _i32, _vp, _vp])
_sig("hh_dct_2d", _i32, [_vp, _vp, _u32, _u32, _vp, _vp])
_sig("hh_turbo_tensor_decode", _i32, [_vp, _vp, _sz, _i32, _i32, _vp, C.c_uint64, C.POINTER(_u32),
                                      C.POINTER(_u32), C.POINTER(BlockStatus), _vp])
_sig("hh_zstd_decompress", _i32, [_vp, _sz, _vp, _sz, C.POINTER(_sz)])
_sig("hh_xxh64", C.c_uint64, [_vp, _sz, C.c_uint64])
_sig("hh_spectral_encoded_size", _sz, [_u32, _u32, C.c_uint16, C.c_float, C.c_float,
                                        C.POINTER(_u32), C.POINTER(_u32)])
_sig("hh_spectral_encode_from_dct", _i32, [_vp, _u32, _u32, C.c_uint16, C.c_float, C.c_float, _vp,
                                           _sz, _vp, C.POINTER(_sz)])

_sig("hh_hbm_copy", _i32, [_vp, _vp, _vp, C.c_uint64, _vp])

# Every symbol include/haagenti_hip.h declares (checked by the tests).
EXPORTS = [
    "hh_status_category", "hh_status_is_recoverable", "hh_version", "hh_device_count",
    "hh_context_create", "hh_context_destroy", "hh_context_stream", "hh_context_synchronize",
    "hh_context_set_option", "hh_lz4_decompress_batch", "hh_lz4_decompress_to", "hh_lz4_compress_block",
    "hh_lz4_max_compressed_size", "hh_dequant_int4", "hh_quantize_int4",
    "hh_int4_compressed_size", "hh_hctt_tile_bytes", "hh_hctt_retain_count",
    "hh_hctt_decode", "hh_hctt_decode_batch", "hh_hctt_decode_lz4_batch", "hh_hctt_decode_lz4_batch_noalloc",
    "hh_hctt_decode_lz4_fused", "hh_hctt_decode_lz4_fused_tpb",
    "hh_hctt_encode",
    "hh_hct_read_header", "hh_hct_decompress_all",
    "hh_xxh3_64", "hh_xxh3_64_batch", "hh_hct_read_header_v2", "hh_hct_decompress_all_validated",
    "hh_hct_validate_checksums", "hh_hct3_coefficients", "hh_hct3_decompress", "hh_hct3_decompress_device",
    "hh_spectral_reconstruct", "hh_idct_2d", "hh_dct_2d", "hh_spectral_encoded_size",
    "hh_zstd_decompress", "hh_xxh64", "hh_turbo_tensor_decode",
    "hh_spectral_encode_from_dct",
    "hh_pinned_alloc", "hh_pinned_free", "hh_pool_create", "hh_pool_destroy", "hh_pool_allocate",
    "hh_pool_recycle", "hh_pool_get_stats", "hh_pipeline_default_config", "hh_pipeline_create",
    "hh_pipeline_destroy", "hh_pipeline_streams", "hh_pipeline_next_staging", "hh_pipeline_submit",
    "hh_pipeline_wait", "hh_pipeline_stream_wait", "hh_pipeline_get_times", "hh_pipeline_finish",
    "hh_pipeline_get_stats", "hh_pipeline_reset_stats", "hh_hbm_copy",
]

CORRUPT_HEADER_CHECKSUM, CORRUPT_BLOCK_CHECKSUM, CORRUPT_QUANT_SCHEME = 6, 7, 8
FLAG_HEADER_CHECKSUM, FLAG_BLOCK_CHECKSUMS, FLAG_QUANTIZATION = 0x0001, 0x0002, 0x0004


def xxh3_64(data):
    """xxhash_rust::xxh3::xxh3_64 (seed 0) on host bytes (hh_xxh3_64)."""
    b = bytes(data)
    return int(_lib.hh_xxh3_64(b, len(b)))


def lib():
    return _lib


def _zstd_size_hint(b):
    """Content size declared by the first frame header, or None."""
    if len(b) < 6 or b[:4] != b"\x28\xb5\x2f\xfd":
        return None
    fhd = b[4]
    fcs_flag, single, did = fhd >> 6, (fhd >> 5) & 1, fhd & 3
    size = [1 if single else 0, 2, 4, 8][fcs_flag]
    at = 5 + (0 if single else 1) + [0, 1, 2, 4][did]
    if size == 0 or len(b) < at + size:
        return None
    v = int.from_bytes(b[at:at + size], "little")
    return v + 256 if size == 2 else v


def zstd_decompress(data):
    """zstd::decode_all (RFC 8878 frames) on the host (hh_zstd_decompress).
    Raises HaagentiError(CORRUPTED_DATA) on a malformed stream."""
    b = bytes(data)
    n = _sz(0)
    hint = _zstd_size_hint(b)
    cap = hint if hint is not None and hint <= 64 * len(b) + (1 << 20) else 8 * len(b) + (1 << 20)
    out = C.create_string_buffer(max(cap, 1))
    rc = _lib.hh_zstd_decompress(b, len(b), out, cap, C.byref(n))
    if rc == BUFFER_TOO_SMALL:  # more than the hint (concatenated frames) or the estimate
        out = C.create_string_buffer(n.value)
        rc = _lib.hh_zstd_decompress(b, len(b), out, n.value, C.byref(n))
    _check(rc, "zstd decode")
    return out.raw[:n.value]


def xxh64(data, seed=0):
    b = bytes(data)
    return int(_lib.hh_xxh64(b, len(b), int(seed)))


class HaagentiError(Exception):
    """haagenti_core::Error mirror: .code, .category, plus the record fields."""

    def __init__(self, code, message="", status=None):
        self.code = int(code)
        self.category = category(code)
        self.status = status
        super().__init__(f"{self.category}: {message}" if message else self.category)

    def is_recoverable(self):
        return bool(_lib.hh_status_is_recoverable(self.code))


def category(code):
    return _lib.hh_status_category(int(code)).decode()


def version():
    return _lib.hh_version().decode()


def device_count():
    return int(_lib.hh_device_count())


def _check(code, what=""):
    if code != OK:
        raise HaagentiError(code, what)


def _addr(x):
    """Device address of a torch tensor, or an int address."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _host_buf(data):
    b = bytes(data)
    return b, C.cast(C.c_char_p(b), _vp) if b else None


class HipContext:
    """One device context (device id, stream, IDCT basis table).  Not
    thread-safe; use one per host thread, like GpuDctContext."""

    def __init__(self, device=0):
        p = _vp()
        _check(_lib.hh_context_create(int(device), C.byref(p)), "hh_context_create")
        self._p = p
        self.device = device

    @property
    def handle(self):
        return self._p

    @property
    def stream(self):
        return _lib.hh_context_stream(self._p)

    def synchronize(self):
        _check(_lib.hh_context_synchronize(self._p))

    def set_option(self, option, value):
        """hh_context_set_option: OPT_LZ4_DECODER (a value of LZ4_DECODERS),
        OPT_FUSED_POLL_LIMIT (polls per wait of the fused decode, 0 = default),
        OPT_DCT_ROUTE (a value of DCT_ROUTES) or OPT_PIPELINE_ROUTE (a value
        of PIPELINE_ROUTES)."""
        _check(_lib.hh_context_set_option(self._p, int(option), int(value)), "hh_context_set_option")

    def set_lz4_decoder(self, name):
        self.set_option(OPT_LZ4_DECODER, LZ4_DECODERS[name])

    def set_dct_route(self, name):
        """Whole-matrix transform route: "auto" (the FFT route when both sides
        allow it and the larger is at least 1024), "dense" or "fft"."""
        self.set_option(OPT_DCT_ROUTE, DCT_ROUTES[name])

    def set_pipeline_route(self, name):
        """How DecompressionPipeline.submit decodes a unit's tensors: "auto"
        (tensors with k >= 1024 whose blocks hold whole tiles in the fused
        launch, the others through the LZ4 and tile launches), "two-launch"
        or "fused" (every tensor whose blocks allow it)."""
        self.set_option(OPT_PIPELINE_ROUTE, PIPELINE_ROUTES[name])

    def close(self):
        if getattr(self, "_p", None):
            _lib.hh_context_destroy(self._p)
            self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---------------------------------------------------------- device API
    def lz4_decompress_batch(self, d_in, in_total, d_in_off, d_in_len, d_out, d_out_off,
                             d_out_cap, nblocks, d_status, stream=None):
        """Raw device-pointer batch decode (hh_lz4_decompress_batch)."""
        return _lib.hh_lz4_decompress_batch(
            self._p, _addr(d_in), int(in_total), _addr(d_in_off), _addr(d_in_len), _addr(d_out),
            _addr(d_out_off), _addr(d_out_cap), int(nblocks), _addr(d_status), stream)

    def xxh3_64_batch(self, d_data, data_len, d_off, d_len, n, d_out, stream=None):
        """XXH3-64 of n device buffers in one launch (hh_xxh3_64_batch)."""
        _check(_lib.hh_xxh3_64_batch(self._p, _addr(d_data), int(data_len), _addr(d_off), _addr(d_len),
                                     int(n), _addr(d_out), stream), "hh_xxh3_64_batch")

    def dequant_int4(self, d_q, q_len, n, d_out, dtype=F32, stream=None):
        produced = _sz(0)
        _check(_lib.hh_dequant_int4(self._p, _addr(d_q), int(q_len), int(n), int(dtype),
                                    _addr(d_out), C.byref(produced), stream), "hh_dequant_int4")
        return produced.value

    def hctt_decode(self, d_tiles, tiles_len, rows, cols, k, d_out, dtype=F32,
                    d_tile_status=None, stream=None):
        _check(_lib.hh_hctt_decode(self._p, _addr(d_tiles), int(tiles_len), int(rows), int(cols),
                                   int(k), int(dtype), _addr(d_out), _addr(d_tile_status),
                                   stream), "hh_hctt_decode")

    def hctt_decode_batch(self, tensors, dtype=F32, stream=None):
        """tensors: list of (d_tiles, tiles_len, rows, cols, k, d_out[, d_status])."""
        arr = (HcttTensor * len(tensors))()
        for i, t in enumerate(tensors):
            st = t[6] if len(t) > 6 else None
            arr[i] = HcttTensor(_addr(t[0]), int(t[1]), int(t[2]), int(t[3]), int(t[4]),
                                _addr(t[5]), _addr(st))
        _check(_lib.hh_hctt_decode_batch(self._p, arr, len(tensors), int(dtype), stream),
               "hh_hctt_decode_batch")

    def hctt_decode_lz4_batch(self, d_in, in_total, d_in_off, d_in_len, d_scratch, d_out_off, d_out_cap,
                              nblocks, d_status, tensors, dtype=F32, stream=None):
        """LZ4 blocks -> scratch -> tiles of several tensors, two launches on
        one stream (hh_hctt_decode_lz4_batch); tensors as for
        hctt_decode_batch, their d_tiles inside d_scratch."""
        arr = (HcttTensor * len(tensors))()
        for i, t in enumerate(tensors):
            st = t[6] if len(t) > 6 else None
            arr[i] = HcttTensor(_addr(t[0]), int(t[1]), int(t[2]), int(t[3]), int(t[4]), _addr(t[5]), _addr(st))
        _check(_lib.hh_hctt_decode_lz4_batch(
            self._p, _addr(d_in), int(in_total), _addr(d_in_off), _addr(d_in_len), _addr(d_scratch),
            _addr(d_out_off), _addr(d_out_cap), int(nblocks), _addr(d_status), arr, len(tensors), int(dtype),
            stream), "hh_hctt_decode_lz4_batch")

    def hctt_decode_lz4_fused(self, d_in, in_total, d_in_off, d_in_len, nblocks, d_status, tensors,
                              tiles_per_block, dtype=F32, stream=None):
        """LZ4 blocks of whole tiles and their tiles in one launch, the tile
        bytes kept in LDS (hh_hctt_decode_lz4_fused); tensors are (rows,
        cols, k, d_out[, d_status]), tensor i's blocks the next
        ceil(tiles_i / tiles_per_block) of the block tables; tiles_per_block
        is one count for every tensor or a sequence of one per tensor
        (hh_hctt_decode_lz4_fused_tpb).  Returns the status code."""
        arr = (HcttTensor * max(len(tensors), 1))()
        for i, t in enumerate(tensors):
            st = t[4] if len(t) > 4 else None
            arr[i] = HcttTensor(None, 0, int(t[0]), int(t[1]), int(t[2]), _addr(t[3]), _addr(st))
        if isinstance(tiles_per_block, (list, tuple)):
            tpb = (_u32 * max(len(tiles_per_block), 1))(*[int(x) for x in tiles_per_block])
            return _lib.hh_hctt_decode_lz4_fused_tpb(
                self._p, _addr(d_in), int(in_total), _addr(d_in_off), _addr(d_in_len), int(nblocks),
                _addr(d_status), arr, len(tensors), tpb, int(dtype), stream)
        return _lib.hh_hctt_decode_lz4_fused(
            self._p, _addr(d_in), int(in_total), _addr(d_in_off), _addr(d_in_len), int(nblocks), _addr(d_status),
            arr, len(tensors), int(tiles_per_block), int(dtype), stream)

    def hctt_decode_lz4_batch_noalloc(self, d_in, in_total, d_in_off, d_in_len, d_out_off, d_out_cap,
                                      nblocks, d_status, tensors, dtype=F32, stream=None):
        """hh_hctt_decode_lz4_batch_noalloc: as hctt_decode_lz4_batch with the
        tile bytes in the library's own device array; tensors are (tiles_len,
        rows, cols, k, d_out[, d_status]), packed in order in that array, and
        d_out_off are offsets into it.  Returns the status code."""
        arr = (HcttTensor * max(len(tensors), 1))()
        for i, t in enumerate(tensors):
            st = t[5] if len(t) > 5 else None
            arr[i] = HcttTensor(None, int(t[0]), int(t[1]), int(t[2]), int(t[3]), _addr(t[4]), _addr(st))
        return _lib.hh_hctt_decode_lz4_batch_noalloc(
            self._p, _addr(d_in), int(in_total), _addr(d_in_off), _addr(d_in_len), _addr(d_out_off),
            _addr(d_out_cap), int(nblocks), _addr(d_status), arr, len(tensors), int(dtype), stream)

    # ---------------------------------------------------------- host API
    def lz4_decompress_to(self, data, out_cap):
        """Decompressor::decompress_to on host buffers.  Returns
        (bytes, BlockStatus); raises HaagentiError on failure."""
        b, pin = _host_buf(data)
        out = C.create_string_buffer(max(int(out_cap), 1))
        written = _sz(0)
        st = BlockStatus()
        rc = _lib.hh_lz4_decompress_to(self._p, pin, len(b), out, int(out_cap), C.byref(written),
                                       C.byref(st))
        if rc != OK:
            raise HaagentiError(rc, "lz4 decompress", st)
        return out.raw[:written.value], st


class HctReader:
    """HctReader (crates/haagenti-hct/src/tensor.rs:408-516) over an in-memory
    HCT v1 file: header(), num_blocks(), read_block(), decompress_block(),
    decompress_all() with any decompressor object (per block, as the
    reference does), plus decompress_all_gpu(): every block in one batched
    GPU launch (hh_hct_decompress_all)."""

    def __init__(self, data):
        self._data = bytes(data)
        self._info = HctInfo()
        st = BlockStatus()
        rc = _lib.hh_hct_read_header(self._data, len(self._data), C.byref(self._info), C.byref(st))
        if rc != OK:
            raise HaagentiError(rc, "hct header", st)

    def header(self):
        i = self._info
        return dict(version=i.version, algorithm=i.algorithm, dtype=i.dtype, flags=i.flags,
                    original_size=i.original_size, compressed_size=i.compressed_size,
                    block_size=i.block_size, num_blocks=i.num_blocks,
                    shape=list(i.shape[:i.rank]))

    def num_blocks(self):
        return int(self._info.num_blocks)

    def data_offset(self):
        """File offset of the first compressed block (blocks follow each other)."""
        return int(self._info.data_offset)

    def _entry(self, idx):
        import struct
        off, csz = struct.unpack_from("<II", self._data, 64 + 8 * idx)
        return self._info.data_offset + off, csz

    def read_block(self, idx):
        if idx >= self.num_blocks():
            raise HaagentiError(CORRUPTED_DATA, f"block index out of range: {idx} >= {self.num_blocks()}")
        start, csz = self._entry(idx)
        if start + csz > len(self._data):
            raise HaagentiError(ALGORITHM, f"failed to read block {idx}")
        return self._data[start:start + csz]

    def expected_size(self, idx):
        n, bs = self.num_blocks(), self._info.block_size
        if idx == n - 1:
            full = (n - 1) * bs
            if full > self._info.original_size:
                raise HaagentiError(CORRUPTED_DATA, "last block size")
            return self._info.original_size - full
        return bs

    def decompress_block(self, idx, decompressor):
        compressed = self.read_block(idx)
        return decompressor.decompress_with_size(compressed, self.expected_size(idx))

    def decompress_all(self, decompressor):
        return b"".join(self.decompress_block(i, decompressor) for i in range(self.num_blocks()))

    def decompress_all_gpu(self, ctx, d_file=None, d_out=None, out_cap=None, stream=None):
        """Batched GPU decode.  Returns (written, d_out); d_file / d_out are
        allocated with torch when not given.  Raises HaagentiError (with
        .status and .failed_block) on failure."""
        import numpy as np
        import torch
        if d_file is None:
            d_file = torch.from_numpy(np.frombuffer(self._data, np.uint8).copy()).cuda()
        if out_cap is None:
            out_cap = int(self._info.original_size)
        if d_out is None:
            d_out = torch.empty(max(out_cap, 1), dtype=torch.uint8, device="cuda")
        written, st, fb = _sz(0), BlockStatus(), C.c_int64(-1)
        rc = _lib.hh_hct_decompress_all(ctx.handle, self._data, _addr(d_file), len(self._data),
                                        _addr(d_out), int(out_cap), C.byref(written), C.byref(st),
                                        C.byref(fb), stream)
        if rc != OK:
            e = HaagentiError(rc, f"hct block {fb.value}", st)
            e.failed_block = fb.value
            raise e
        return written.value, d_out


class HctReaderV2(HctReader):
    """HctReaderV2 (crates/haagenti-hct/src/tensor.rs:832-1021) over an
    in-memory HCT file: the constructor verifies the header checksum and
    reads the quantization metadata; read_block_validated() checks a block's
    XXH3 when its index entry holds one; decompress_all_validated() works
    block by block through any decompressor, as the reference does;
    decompress_all_validated_gpu() / validate_checksums_gpu() hash every block
    in one GPU launch and decode them in one more."""

    def __init__(self, data):
        self._data = bytes(data)
        self._info = HctInfo()
        self._quant = HctQuant()
        st = BlockStatus()
        rc = _lib.hh_hct_read_header_v2(self._data, len(self._data), C.byref(self._info),
                                        C.byref(self._quant), C.byref(st))
        if rc != OK:
            raise HaagentiError(rc, "hct v2 header", st)

    def quantization(self):
        q = self._quant
        if not q.present:
            return None
        return dict(scheme=q.scheme, group_size=q.group_size, scale_bits=q.scale_bits,
                    zero_point=q.zero_point, has_per_group_scales=bool(q.has_per_group_scales))

    def _entry(self, idx):
        import struct
        e = self._info.index_entry_size
        at = self._info.data_offset - e * self.num_blocks() + e * idx
        off, csz = struct.unpack_from("<II", self._data, at)
        sum_ = struct.unpack_from("<Q", self._data, at + 8)[0] if e == 16 else 0
        return self._info.data_offset + off, csz, sum_

    def read_block(self, idx):
        return self.read_block_validated(idx)

    def read_block_validated(self, idx):
        if idx >= self.num_blocks():
            raise HaagentiError(CORRUPTED_DATA, f"block index out of range: {idx} >= {self.num_blocks()}")
        start, csz, sum_ = self._entry(idx)
        if start + csz > len(self._data):
            raise HaagentiError(ALGORITHM, f"failed to read block {idx}")
        buf = self._data[start:start + csz]
        if sum_ != 0:
            got = xxh3_64(buf)
            if got != sum_:
                raise HaagentiError(CORRUPTED_DATA, f"block {idx} checksum mismatch: expected "
                                                    f"{sum_:016x}, got {got:016x}")
        return buf

    def decompress_block_validated(self, idx, decompressor):
        return self.decompress_block(idx, decompressor)

    def decompress_all_validated(self, decompressor):
        return self.decompress_all(decompressor)

    def validate_checksums(self):
        for i in range(self.num_blocks()):
            self.read_block_validated(i)

    def _gpu(self, ctx, decode, d_file, d_out, out_cap, stream):
        import numpy as np
        import torch
        if d_file is None:
            d_file = torch.from_numpy(np.frombuffer(self._data, np.uint8).copy()).cuda()
        written, st, fb = _sz(0), BlockStatus(), C.c_int64(-1)
        if decode:
            if out_cap is None:
                out_cap = int(self._info.original_size)
            if d_out is None:
                d_out = torch.empty(max(out_cap, 1), dtype=torch.uint8, device="cuda")
            rc = _lib.hh_hct_decompress_all_validated(ctx.handle, self._data, _addr(d_file),
                                                      len(self._data), _addr(d_out), int(out_cap),
                                                      C.byref(written), C.byref(st), C.byref(fb), stream)
        else:
            rc = _lib.hh_hct_validate_checksums(ctx.handle, self._data, _addr(d_file), len(self._data),
                                                C.byref(st), C.byref(fb), stream)
        if rc != OK:
            e = HaagentiError(rc, f"hct block {fb.value}", st)
            e.failed_block = fb.value
            raise e
        return written.value, d_out

    def decompress_all_validated_gpu(self, ctx, d_file=None, d_out=None, out_cap=None, stream=None):
        """Every block hashed and decoded on the GPU.  Returns (written, d_out)."""
        return self._gpu(ctx, True, d_file, d_out, out_cap, stream)

    def validate_checksums_gpu(self, ctx, d_file=None, stream=None):
        self._gpu(ctx, False, d_file, None, 0, stream)


class HctWriter:
    """HctWriter (crates/haagenti-hct/src/tensor.rs:519-617), host producer of
    version-1 files: the 64-byte header (HctHeader::to_bytes, :299-328;
    version 1, flags 0, shape dims at 37 + 8 i), one 8-byte index entry per
    block (offset from the data start, compressed size; :391-396), then the
    blocks in order.  Shapes of rank 4 and more do not fit the header (the
    reference's header serialization indexes past its 64 bytes); they raise
    ValueError."""

    def __init__(self, dtype, shape, block_size=16 * 1024, algorithm=0):
        if len(shape) > 3:
            raise ValueError("an HCT v1 header holds at most 3 dimensions")
        self.dtype, self.shape, self.block_size, self.algorithm = dtype, list(shape), block_size, algorithm
        self.blocks = []
        self.original_size = 0

    def with_block_size(self, block_size):
        self.block_size = block_size
        return self

    def add_block(self, compressed, original_len):
        self.blocks.append(bytes(compressed))
        self.original_size += original_len

    def compress_data(self, data, compressor):
        data = bytes(data)
        for s in range(0, len(data), self.block_size):
            chunk = data[s:s + self.block_size]
            self.add_block(compressor.compress(chunk), len(chunk))

    def finish(self):
        import struct
        index, off = b"", 0
        for c in self.blocks:
            index += struct.pack("<II", off, len(c))
            off += len(c)
        h = bytearray(64)
        h[0:4] = b"HCTN"
        struct.pack_into("<IBBHQQII", h, 4, 1, self.algorithm, self.dtype, 0,
                         self.original_size, off, self.block_size, len(self.blocks))
        h[36] = len(self.shape)
        for i, d in enumerate(self.shape):
            struct.pack_into("<Q", h, 37 + 8 * i, d)
        return bytes(h) + index + b"".join(self.blocks)


class HctWriterV2:
    """HctWriterV2 (tensor.rs:679-829), host producer: header (version 2,
    flags), optional quantization metadata, 16-byte index entries with the
    XXH3 of each compressed block (0 without block checksums), data."""

    def __init__(self, dtype, shape, block_size=16 * 1024, algorithm=0):
        self.dtype, self.shape, self.block_size, self.algorithm = dtype, list(shape), block_size, algorithm
        self.flags = FLAG_HEADER_CHECKSUM | FLAG_BLOCK_CHECKSUMS
        self.quant = None
        self.blocks = []
        self.original_size = 0

    def with_block_size(self, block_size):
        self.block_size = block_size
        return self

    def with_quantization(self, scheme, group_size, scale_bits, zero_point=0, has_per_group_scales=False):
        import struct
        self.quant = (bytes([scheme, 1 if has_per_group_scales else 0]) + struct.pack("<H", scale_bits)
                      + struct.pack("<b", zero_point) + int(group_size).to_bytes(4, "little")[:3])
        self.flags |= FLAG_QUANTIZATION
        return self

    def without_block_checksums(self):
        self.flags &= ~FLAG_BLOCK_CHECKSUMS
        return self

    def add_block(self, compressed, original_len):
        c = bytes(compressed)
        self.blocks.append((c, xxh3_64(c) if self.flags & FLAG_BLOCK_CHECKSUMS else 0))
        self.original_size += original_len

    def compress_data(self, data, compressor):
        data = bytes(data)
        for s in range(0, len(data), self.block_size):
            chunk = data[s:s + self.block_size]
            self.add_block(compressor.compress(chunk), len(chunk))

    def finish(self):
        import struct
        index, off = b"", 0
        for c, sum_ in self.blocks:
            index += struct.pack("<IIQ", off, len(c), sum_)
            off += len(c)
        h = bytearray(64)
        h[0:4] = b"HCTN"
        struct.pack_into("<IBBHQQII", h, 4, 2, self.algorithm, self.dtype, self.flags,
                         self.original_size, off, self.block_size, len(self.blocks))
        h[36] = len(self.shape)
        for i, d in enumerate(self.shape[:4]):
            h[37 + 8 * i:45 + 8 * i] = struct.pack("<Q", d)[:max(0, min(8, 64 - (37 + 8 * i)))]
        struct.pack_into("<Q", h, 56, xxh3_64(bytes(h[:56])))
        return bytes(h) + (self.quant or b"") + index + b"".join(c for c, _ in self.blocks)


class Lz4Decompressor:
    """haagenti_core::Decompressor for raw LZ4 blocks, decoded on the GPU.

    Methods mirror crates/haagenti-lz4/src/decompress.rs:28-68."""

    def __init__(self, ctx=None):
        self.ctx = ctx if ctx is not None else HipContext(0)

    def algorithm(self):
        return "lz4"

    def decompress_to(self, data, out_cap):
        out, st = self.ctx.lz4_decompress_to(data, out_cap)
        return out

    def decompress_with_size(self, data, output_size):
        return self.decompress_to(data, output_size)

    def decompress(self, data):
        """Size unknown: start at 4x the input and grow on BufferTooSmall up
        to 256 MiB (decompress.rs:33-57)."""
        size = len(data) * 4
        while True:
            try:
                return self.decompress_to(data, size)
            except HaagentiError as e:
                if e.code != BUFFER_TOO_SMALL:
                    raise
                size = max(int(e.status.required), size * 2)
                if size > 256 * 1024 * 1024:
                    raise HaagentiError(CORRUPTED_DATA, "decompressed size exceeds limit")


class Lz4Compressor:
    """Compressor side (host): byte-identical to block::compress_block."""

    def algorithm(self):
        return "lz4"

    def max_compressed_size(self, n):
        return int(_lib.hh_lz4_max_compressed_size(int(n)))

    def compress(self, data):
        b, pin = _host_buf(data)
        cap = self.max_compressed_size(len(b))
        out = C.create_string_buffer(cap)
        w = _sz(0)
        _check(_lib.hh_lz4_compress_block(pin, len(b), out, cap, C.byref(w)), "lz4 compress")
        return out.raw[:w.value]


def lz4_max_compressed_size(n):
    return int(_lib.hh_lz4_max_compressed_size(int(n)))


def int4_compressed_size(n):
    return int(_lib.hh_int4_compressed_size(int(n)))


def hctt_tile_bytes(k):
    return int(_lib.hh_hctt_tile_bytes(int(k)))


def hctt_retain_count(rho):
    return int(_lib.hh_hctt_retain_count(float(rho)))


def quantize_int4(w):
    """testing::quantize_int4 on the host; w is a float32 numpy array."""
    import numpy as np
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros(max(int4_compressed_size(w.size), 1), dtype=np.uint8)
    n = _lib.hh_quantize_int4(w.ctypes.data, w.size, out.ctypes.data)
    return out[:n]


def hctt_encode(w, k, threads=0):
    """HCT-T tiles for a float32 (rows, cols) numpy array (host producer)."""
    import numpy as np
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.zeros((rows // 64) * (cols // 64) * hctt_tile_bytes(k), dtype=np.uint8)
    _check(_lib.hh_hctt_encode(w.ctypes.data, rows, cols, int(k), out.ctypes.data, int(threads)),
           "hh_hctt_encode")
    return out


# ------------------------------------------------------------- HCT3 spectral

def _shape_arr(shape):
    shape = [int(d) for d in shape]
    return (C.c_uint64 * max(len(shape), 1))(*shape), len(shape)


def _dims(shape):
    """GpuDecompressor::calculate_dimensions (decompress.rs:430-442)."""
    shape = [int(d) for d in shape]
    if not shape:
        return 1, 1
    w = shape[-1]
    n = 1
    for d in shape:
        n *= d
    return w, (n // w if w else 0)


def _torch_dtype(dtype):
    import torch
    return {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}[dtype]


class GpuDecompressor:
    """GpuDecompressor (crates/haagenti-cuda/src/decompress.rs:108-443) for HCT
    V3 fragment containers: decompress(), decompress_to_gpu(),
    decompress_batch(), plus reconstruct_coefficients_gpu() (the dense DCT
    coefficient matrix before the transform).  zstd-framed input raises
    UNSUPPORTED."""

    def __init__(self, ctx=None):
        self.ctx = ctx if ctx is not None else HipContext(0)

    def reconstruct_coefficients_gpu(self, compressed, total, stream=None):
        import torch
        b = bytes(compressed)
        out = torch.empty(max(int(total), 1), dtype=torch.float32, device="cuda")
        _check(_lib.hh_hct3_coefficients(self.ctx.handle, b, len(b), int(total), _addr(out), stream),
               "hh_hct3_coefficients")
        return out[:int(total)]

    def decompress_to_gpu(self, compressed, shape, dtype=F32, d_out=None, stream=None):
        import torch
        b = bytes(compressed)
        w, h = _dims(shape)
        n = w * h
        if d_out is None:
            d_out = torch.empty(max(n, 1), dtype=_torch_dtype(dtype), device="cuda")
        arr, rank = _shape_arr(shape)
        _check(_lib.hh_hct3_decompress(self.ctx.handle, b, len(b), arr, rank, int(dtype), _addr(d_out),
                                       stream), "hh_hct3_decompress")
        return d_out[:n]

    def decompress_device(self, h_data, d_data, shape, d_out, dtype=F32, stream=None):
        """Decode with the container already on the device (d_data, a copy of
        h_data): asynchronous on the stream (hh_hct3_decompress_device)."""
        b = h_data if isinstance(h_data, bytes) else bytes(h_data)
        arr, rank = _shape_arr(shape)
        _check(_lib.hh_hct3_decompress_device(self.ctx.handle, b, _addr(d_data), len(b), arr, rank, int(dtype),
                                              _addr(d_out), stream), "hh_hct3_decompress_device")
        return d_out

    def decompress(self, compressed, shape):
        """Reconstructed tensor as a flat float32 numpy array."""
        return self.decompress_to_gpu(compressed, shape).cpu().numpy()

    def decompress_batch(self, tensors):
        return [self.decompress(c, s) for c, s in tensors]

    def decompress_batch_pipelined(self, tensors):
        """decompress_batch_pipelined (decompress.rs:228-279): every tensor's
        coefficient matrix first (zstd unwrap, container parse and the
        bitmap scatter: hh_hct3_coefficients), then every inverse DCT
        (hh_idct_2d), with the reference's DecompressStats of the two
        phases.  Returns ([flat float32 numpy arrays], stats dict)."""
        import time
        import torch
        t0 = time.perf_counter()
        stats = dict(num_tensors=len(tensors), total_input_bytes=0, total_output_bytes=0)
        coefs = []
        for compressed, shape in tensors:
            w, h = _dims(shape)
            stats["total_input_bytes"] += len(compressed)
            stats["total_output_bytes"] += w * h * 4
            coefs.append((self.reconstruct_coefficients_gpu(compressed, w * h), w, h))
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        outs = []
        for c, w, h in coefs:
            x = torch.empty(max(w * h, 1), dtype=torch.float32, device="cuda")
            if w * h:
                self.ctx.idct_2d(c, h, w, x)
            outs.append(x[:w * h])
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        stats.update(parse_time_ms=(t1 - t0) * 1e3, idct_time_ms=(t2 - t1) * 1e3, total_time_ms=(t2 - t0) * 1e3)
        return [o.cpu().numpy() for o in outs], stats


class CompressiveSpectralDecoder:
    """CompressiveSpectralDecoder (compressive.rs:420-752): add_essentials()
    (fragment 0) then add_detail() for any subset of the detail fragments;
    quality() as the reference computes it (:716-729); reconstruct() runs the
    scatter and the whole-matrix IDCT on the GPU.  Fragments are
    (index, bytes) pairs or objects with .index and .data."""

    def __init__(self, ctx=None):
        self._ctx = ctx
        self._frags = []
        self.has_essentials = False
        self.total_coeffs = self.essential_count = 0
        self.total_fragments = 0
        self.detail_fragments_loaded = 0
        self.width = self.height = 0

    @property
    def ctx(self):
        if self._ctx is None:
            self._ctx = HipContext(0)
        return self._ctx

    @staticmethod
    def _split(fragment):
        if isinstance(fragment, tuple):
            return int(fragment[0]), bytes(fragment[1])
        return int(fragment.index), bytes(fragment.data)

    def add_essentials(self, fragment):
        import struct
        idx, data = self._split(fragment)
        if idx != 0:
            raise HaagentiError(CORRUPTED_DATA, "fragment 0 must be added first for CompressiveSpectralDecoder")
        self._frags = [(0, data)]
        self._probe()
        self.total_coeffs, self.essential_count = struct.unpack_from("<II", data, 12)
        self.has_essentials = True

    def add_detail(self, fragment):
        import struct
        if not self.has_essentials:
            raise HaagentiError(CORRUPTED_DATA, "must add fragment 0 (essentials) first")
        idx, data = self._split(fragment)
        if idx == 0:
            return
        self._frags.append((idx, data))
        self._probe()
        self.total_fragments = struct.unpack_from("<H", data, 2)[0]
        self.detail_fragments_loaded += 1

    def can_reconstruct(self):
        return self.has_essentials

    def quality(self):
        """compressive.rs:716-729 (f32 arithmetic)."""
        import numpy as np
        if not self.has_essentials:
            return 0.0
        if self.total_fragments <= 1:
            return 1.0
        f = np.float32
        detail = self.total_fragments - 1
        loaded = min(self.detail_fragments_loaded, detail)
        eq = f(self.essential_count) / f(self.total_coeffs)
        dq = f(self.total_coeffs - self.essential_count) / f(self.total_coeffs)
        return float(eq + dq * (f(loaded) / f(detail)))

    def _call(self, dtype=F32, d_out=None, out_cap=0, stream=None):
        n = len(self._frags)
        bufs = [d for _, d in self._frags]
        ptrs = (_vp * n)(*[C.cast(C.c_char_p(d), _vp) for d in bufs])
        lens = (_sz * n)(*[len(d) for d in bufs])
        idx = (C.c_uint16 * n)(*[i for i, _ in self._frags])
        w, h, st = _u32(0), _u32(0), BlockStatus()
        rc = _lib.hh_spectral_reconstruct(self.ctx.handle, ptrs, lens, idx, n, int(dtype), _addr(d_out),
                                          int(out_cap), C.byref(w), C.byref(h), C.byref(st), stream)
        return rc, w.value, h.value, st

    def _probe(self):
        # parse and validate without reconstructing (no output buffer)
        rc, w, h, st = self._call()
        if rc not in (OK, INVALID_ARGUMENT):
            raise HaagentiError(rc, "compressive spectral fragment", st)
        self.width, self.height = w, h

    def reconstruct_gpu(self, dtype=F32, d_out=None, stream=None):
        import torch
        if not self.has_essentials:
            raise HaagentiError(CORRUPTED_DATA, "need essentials fragment to reconstruct")
        n = self.width * self.height
        if d_out is None:
            d_out = torch.empty(max(n, 1), dtype=_torch_dtype(dtype), device="cuda")
        rc, w, h, st = self._call(dtype, d_out, d_out.numel(), stream)
        if rc != OK:
            raise HaagentiError(rc, "compressive spectral reconstruct", st)
        return d_out[:n]

    def reconstruct(self):
        return self.reconstruct_gpu().cpu().numpy()


class CompressiveSpectralEncoder:
    """CompressiveSpectralEncoder (compressive.rs:67-340), producer: the DCT of
    the tensor on the GPU (GpuDctContext::dct_2d, as the turbo encoder uses),
    then retention, bitmap and f16 fragments on the host
    (hh_spectral_encode_from_dct).  Fragments are returned as (index, bytes);
    the forward DCT's rounding differs from the reference's FFT DCT, so
    near-tied magnitudes may be retained differently."""

    def __init__(self, num_fragments, retention_ratio, ctx=None):
        self.num_fragments = int(num_fragments)
        self.retention_ratio = float(retention_ratio)
        self.essential_ratio = 0.2
        self.ctx = ctx

    def with_essential_ratio(self, ratio):
        self.essential_ratio = float(ratio)
        return self

    def encode_2d_from_dct(self, dct_coeffs, width, height):
        import numpy as np
        c = np.ascontiguousarray(dct_coeffs, dtype=np.float32).ravel()
        if c.size != width * height:
            raise HaagentiError(CORRUPTED_DATA, "DCT coefficients size mismatch")
        size = int(_lib.hh_spectral_encoded_size(width, height, self.num_fragments, self.retention_ratio,
                                                 self.essential_ratio, None, None))
        out = C.create_string_buffer(max(size, 1))
        offs = (C.c_uint64 * (self.num_fragments + 1))()
        w = _sz(0)
        _check(_lib.hh_spectral_encode_from_dct(c.ctypes.data, width, height, self.num_fragments,
                                                self.retention_ratio, self.essential_ratio, out, size,
                                                offs, C.byref(w)), "hh_spectral_encode_from_dct")
        raw = out.raw
        return [(f, raw[offs[f]:offs[f + 1]]) for f in range(self.num_fragments)]

    def encode_2d(self, data, width, height):
        import numpy as np
        import torch
        ctx = self.ctx if self.ctx is not None else HipContext(0)
        x = torch.as_tensor(np.ascontiguousarray(data, dtype=np.float32).ravel()).cuda()
        if x.numel() != width * height:
            raise HaagentiError(CORRUPTED_DATA, "data size mismatch")
        c = torch.empty_like(x)
        ctx.dct_2d(x, height, width, c)
        torch.cuda.synchronize()
        return self.encode_2d_from_dct(c.cpu().numpy(), width, height)


def hct3_container(fragments):
    """The fragment container the turbo pipeline serializes before its zstd
    wrapper (crates/haagenti/src/pipeline/turbo.rs:378-387): [u16 n] then per
    fragment index, flags (0), XXH3-64 of the data, u32 length, data."""
    import struct
    out = struct.pack("<H", len(fragments))
    for idx, data in fragments:
        data = bytes(data)
        out += struct.pack("<HHQI", idx, 0, xxh3_64(data), len(data)) + data
    return out


def _hip_dct(self, d_in, rows, cols, d_out, stream=None):
    """Orthonormal 2-D DCT-II of a row-major rows x cols f32 device matrix
    (hh_dct_2d; GpuDctContext::dct_2d)."""
    _check(_lib.hh_dct_2d(self.handle, _addr(d_in), int(rows), int(cols), _addr(d_out), stream), "hh_dct_2d")


def _hip_hbm_copy(self, d_dst, d_src, nbytes, stream=None):
    """Streaming device copy of nbytes (hh_hbm_copy): the bandwidth
    calibration kernel of the measurements."""
    _check(_lib.hh_hbm_copy(self.handle, _addr(d_dst), _addr(d_src), int(nbytes), stream), "hh_hbm_copy")


HipContext.hbm_copy = _hip_hbm_copy


def _hip_idct(self, d_in, rows, cols, d_out, dtype=F32, stream=None):
    """Orthonormal 2-D DCT-III of a row-major rows x cols f32 device matrix
    (hh_idct_2d; GpuDctContext::idct_2d_gpu)."""
    _check(_lib.hh_idct_2d(self.handle, _addr(d_in), int(rows), int(cols), int(dtype), _addr(d_out), stream),
           "hh_idct_2d")


HipContext.dct_2d = _hip_dct
HipContext.idct_2d = _hip_idct
