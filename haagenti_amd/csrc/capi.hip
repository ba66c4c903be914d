// C-ABI entry points: contexts, argument validation, kernel launches.
// Declarations and the reference interface each one replaces are in
// include/haagenti_hip.h.
#include <cmath>
#include <cstring>
#include <vector>

#include "hh_internal.hpp"

namespace hh {

int32_t from_hip(hipError_t e) {
    switch (e) {
        case hipSuccess: return HH_OK;
        case hipErrorOutOfMemory: return HH_ERR_OUT_OF_MEMORY;
        case hipErrorInvalidDevice:
        case hipErrorNoDevice: return HH_ERR_DEVICE_NOT_FOUND;
        case hipErrorInvalidValue: return HH_ERR_INVALID_ARGUMENT;
        case hipErrorLaunchFailure:
        case hipErrorInvalidDeviceFunction:
        case hipErrorInvalidConfiguration: return HH_ERR_KERNEL_LAUNCH;
        default: return HH_ERR_DEVICE;
    }
}

int32_t ensure_scratch(hh_context *ctx, size_t bytes) {
    if (ctx->scratch_bytes >= bytes) return HH_OK;
    if (ctx->d_scratch) {
        hipError_t e = hipFree(ctx->d_scratch);
        ctx->d_scratch = nullptr;
        ctx->scratch_bytes = 0;
        if (e != hipSuccess) return from_hip(e);
    }
    size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
    hipError_t e = hipMalloc(&ctx->d_scratch, sz);
    if (e != hipSuccess) {
        ctx->d_scratch = nullptr;
        return from_hip(e);
    }
    ctx->scratch_bytes = sz;
    return HH_OK;
}

}  // namespace hh

namespace {

using hh::ensure_scratch;
using hh::from_hip;

// The caller's stream is used as given; NULL is HIP's null stream (torch's
// default stream is that null stream).  hh_context_stream() returns the
// context's own stream for callers that want it.
hipStream_t pick_stream(hh_context *, void *stream) {
    return reinterpret_cast<hipStream_t>(stream);
}

}  // namespace

namespace hh {

// MFMA fragments of M' = 256 * M, M[v][j] = a_v cos(pi v (2j+1) / 128),
// split into f16 hi + lo, for the even/odd halves of the frequencies.
// Entry ((hl*2 + par)*2 + s)*64 + lane holds the 8 values
// M'[2 pi(16s + 8h + e) + par][lane%32] for e = 0..7, h = lane/32,
// pi(16s + 8h + e) = 16s + 8(e/4) + 4h + e%4 (the accumulator row order of
// v_mfma_f32_32x32x16_f16).  Only j < 32 is tabulated: the other half
// follows from M[v][63 - j] = (-1)^v M[v][j].
size_t basis_table_bytes() { return 2 * 2 * 2 * 64 * 8 * sizeof(_Float16); }

void build_basis_table(void *buf) {
    _Float16 *t = reinterpret_cast<_Float16 *>(buf);
    const double pi = 3.14159265358979323846;
    for (int hl = 0; hl < 2; hl++)
        for (int par = 0; par < 2; par++)
            for (int s = 0; s < 2; s++)
                for (int lane = 0; lane < 64; lane++)
                    for (int e = 0; e < 8; e++) {
                        const int h = lane >> 5;
                        const int v = 2 * (16 * s + 8 * (e >> 2) + 4 * h + (e & 3)) + par;
                        const int j = lane & 31;
                        const double a = v == 0 ? std::sqrt(1.0 / 64) : std::sqrt(2.0 / 64);
                        const double m = 256.0 * a * std::cos(pi * v * (2 * j + 1) / 128.0);
                        const _Float16 hi = (_Float16)m;
                        const _Float16 lo = (_Float16)(m - (double)hi);
                        t[((((hl * 2 + par) * 2 + s) * 64 + lane) * 8) + e] = hl == 0 ? hi : lo;
                    }
}

}  // namespace hh

namespace hh {
int32_t check_hctt_tensor(const hh_hctt_tensor &T, size_t *ntiles) {
    if (T.rows % 64 || T.cols % 64 || T.cols > (1u << 24) || T.k < 1 || T.k > 4096) return HH_ERR_INVALID_ARGUMENT;
    const size_t nt = (size_t)(T.rows / 64) * (T.cols / 64);
    *ntiles = nt;
    if (nt == 0) return HH_OK;
    if (T.tiles_len < nt * hh_hctt_tile_bytes(T.k)) return HH_ERR_UNEXPECTED_EOF;
    if (!T.d_tiles || !T.d_out || ((uintptr_t)T.d_out & 15u)) return HH_ERR_INVALID_ARGUMENT;
    return HH_OK;
}
}  // namespace hh

extern "C" {

const char *hh_status_category(int32_t code) {
    switch (code) {
        case HH_OK: return "ok";
        case HH_ERR_CORRUPTED_DATA: return "corrupted_data";
        case HH_ERR_BUFFER_TOO_SMALL: return "buffer_too_small";
        case HH_ERR_UNEXPECTED_EOF: return "unexpected_eof";
        case HH_ERR_CHECKSUM_MISMATCH: return "checksum_mismatch";
        case HH_ERR_UNSUPPORTED: return "unsupported";
        case HH_ERR_ALGORITHM: return "algorithm_error";
        case HH_ERR_INVALID_ARGUMENT: return "invalid_argument";
        case HH_ERR_OUT_OF_MEMORY: return "allocation_failed";
        case HH_ERR_DEVICE: return "device_error";
        case HH_ERR_KERNEL_LAUNCH: return "kernel_launch";
        case HH_ERR_DEVICE_NOT_FOUND: return "device_not_found";
        default: return "unknown";
    }
}

int32_t hh_status_is_recoverable(int32_t code) {
    return code == HH_ERR_UNEXPECTED_EOF || code == HH_ERR_BUFFER_TOO_SMALL;
}

const char *hh_version(void) { return "haagenti-hip 0.1.0 (gfx950)"; }

int32_t hh_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int32_t hh_context_create(int32_t device, hh_context **out) {
    if (!out) return HH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
        return HH_ERR_DEVICE_NOT_FOUND;
    hh::DeviceGuard guard(device);
    hipError_t e = guard.status();
    if (e != hipSuccess) return from_hip(e);
    hh_context *ctx = new hh_context();
    ctx->device = device;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        delete ctx;
        return from_hip(e);
    }
    ctx->num_cus = prop.multiProcessorCount;
    // set-up of hh_hctt_decode_lz4_batch_noalloc (its failure is reported
    // by that entry point, not here)
    ctx->noalloc_status = hh::noalloc_scratch(device, &ctx->noalloc_scratch);
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return from_hip(e);
    }
    std::vector<unsigned char> table(hh::basis_table_bytes());
    hh::build_basis_table(table.data());
    e = hipMalloc(&ctx->d_basis, table.size());
    if (e == hipSuccess) e = hipMemcpy(ctx->d_basis, table.data(), table.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hh_context_destroy(ctx);
        return from_hip(e);
    }
    *out = ctx;
    return HH_OK;
}

void hh_context_destroy(hh_context *ctx) {
    if (!ctx) return;
    hh::DeviceGuard guard(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->d_basis) (void)hipFree(ctx->d_basis);
    if (ctx->d_scratch) (void)hipFree(ctx->d_scratch);
    hh::release_dct_resources(ctx);
    hh::release_fft_resources(ctx);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

void *hh_context_stream(hh_context *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int32_t hh_context_synchronize(hh_context *ctx) {
    if (!ctx) return HH_ERR_INVALID_ARGUMENT;
    return from_hip(hipStreamSynchronize(ctx->stream));
}

int32_t hh_context_set_option(hh_context *ctx, int32_t option, int64_t value) {
    if (!ctx) return HH_ERR_INVALID_ARGUMENT;
    switch (option) {
        case HH_OPT_LZ4_DECODER:
            if (value < HH_LZ4_AUTO || value > HH_LZ4_WINDOW) return HH_ERR_INVALID_ARGUMENT;
            ctx->lz4_decoder = (int32_t)value;
            return HH_OK;
        case HH_OPT_FUSED_POLL_LIMIT:
            if (value < 0 || value > (1 << 24)) return HH_ERR_INVALID_ARGUMENT;
            ctx->fused_poll_limit = (uint32_t)value;
            return HH_OK;
        case HH_OPT_DCT_ROUTE:
            if (value < HH_DCT_AUTO || value > HH_DCT_FFT) return HH_ERR_INVALID_ARGUMENT;
            ctx->dct_route = (int32_t)value;
            return HH_OK;
        case HH_OPT_PIPELINE_ROUTE:
            if (value < HH_PIPE_AUTO || value > HH_PIPE_FUSED) return HH_ERR_INVALID_ARGUMENT;
            ctx->pipeline_route = (int32_t)value;
            return HH_OK;
        default: return HH_ERR_INVALID_ARGUMENT;
    }
}

// ---------------------------------------------------------------- LZ4

static int32_t lz4_batch_with(hh_context *ctx, int32_t decoder, const uint8_t *d_in, size_t in_total,
                              const uint64_t *d_in_off, const uint32_t *d_in_len, uint8_t *d_out,
                              const uint64_t *d_out_off, const uint32_t *d_out_cap, uint32_t nblocks,
                              hh_block_status *d_status, void *stream, bool zero_tail = false) {
    if (!ctx) return HH_ERR_INVALID_ARGUMENT;
    if (nblocks == 0) return HH_OK;
    if (!d_in || !d_in_off || !d_in_len || !d_out || !d_out_off || !d_out_cap || !d_status)
        return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(ctx->device);
    hipError_t e = guard.status();
    if (e != hipSuccess) return from_hip(e);
    // the caller's output buffer has no stated size: its block table is trusted
    const hh::Lz4Batch B = {d_in,      in_total,  d_in_off, d_in_len, d_out,    ~0ull,
                            d_out_off, d_out_cap, nblocks,  d_status, zero_tail};
    return from_hip(hh::launch_lz4_batch(B, decoder, pick_stream(ctx, stream)));
}

int32_t hh_lz4_decompress_batch(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                const uint64_t *d_in_off, const uint32_t *d_in_len, uint8_t *d_out,
                                const uint64_t *d_out_off, const uint32_t *d_out_cap,
                                uint32_t nblocks, hh_block_status *d_status, void *stream) {
    if (!ctx) return HH_ERR_INVALID_ARGUMENT;
    return lz4_batch_with(ctx, hh::lz4_decoder_for(ctx, HH_LZ4_RING4), d_in, in_total, d_in_off, d_in_len, d_out,
                          d_out_off, d_out_cap, nblocks, d_status, stream);
}

int32_t hh_lz4_decompress_to(hh_context *ctx, const uint8_t *in, size_t in_len, uint8_t *out,
                             size_t out_cap, size_t *written, hh_block_status *status) {
    if (!ctx || (!in && in_len) || (!out && out_cap)) return HH_ERR_INVALID_ARGUMENT;
    if (in_len > 0xffffffffu || out_cap > 0xffffffffu) return HH_ERR_UNSUPPORTED;
    hh::DeviceGuard guard(ctx->device);
    hipError_t e = guard.status();
    if (e != hipSuccess) return from_hip(e);
    // scratch layout: [status 32][in_off 8][in_len 4 pad 4][out_off 8][out_cap 4 pad 4][in][out]
    const size_t hdr = 64;
    const size_t in_at = hdr, out_at = (hdr + in_len + 255) & ~(size_t)255;
    int32_t rc = ensure_scratch(ctx, out_at + out_cap + 16);
    if (rc != HH_OK) return rc;
    uint8_t *base = reinterpret_cast<uint8_t *>(ctx->d_scratch);
    struct {
        uint64_t in_off;
        uint32_t in_len, pad0;
        uint64_t out_off;
        uint32_t out_cap, pad1;
    } meta = {0, (uint32_t)in_len, 0, 0, (uint32_t)out_cap, 0};
    hipStream_t s = ctx->stream;
    e = hipMemcpyAsync(base + 32, &meta, sizeof(meta), hipMemcpyHostToDevice, s);
    if (e == hipSuccess && in_len)
        e = hipMemcpyAsync(base + in_at, in, in_len, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return from_hip(e);
    const hh::Lz4Batch B = {base + in_at,
                            in_len,
                            reinterpret_cast<uint64_t *>(base + 32),
                            reinterpret_cast<uint32_t *>(base + 40),
                            base + out_at,
                            out_cap,
                            reinterpret_cast<uint64_t *>(base + 48),
                            reinterpret_cast<uint32_t *>(base + 56),
                            1,
                            reinterpret_cast<hh_block_status *>(base)};
    e = hh::launch_lz4_batch(B, hh::lz4_decoder_for(ctx, HH_LZ4_RING4), s);
    if (e != hipSuccess) return from_hip(e);
    hh_block_status st;
    e = hipMemcpyAsync(&st, base, sizeof(st), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return from_hip(e);
    if (st.code == HH_OK && st.written) {
        e = hipMemcpy(out, base + out_at, st.written, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return from_hip(e);
    }
    if (written) *written = st.code == HH_OK ? st.written : 0;
    if (status) *status = st;
    return st.code;
}

// ---------------------------------------------------------------- INT4

int32_t hh_dequant_int4(hh_context *ctx, const uint8_t *d_q, size_t q_len, size_t n,
                        int32_t out_dtype, void *d_out, size_t *produced, void *stream) {
    if (!ctx) return HH_ERR_INVALID_ARGUMENT;
    if (out_dtype != HH_F32 && out_dtype != HH_F16 && out_dtype != HH_BF16)
        return HH_ERR_UNSUPPORTED;
    const size_t groups = (n + 31) / 32;
    size_t m = 0;
    if (n > 0 && q_len >= 2 * groups) {
        const size_t packed = q_len - 2 * groups;
        m = n < 2 * packed ? n : 2 * packed;
    }
    if (produced) *produced = m;
    if (m == 0) return HH_OK;
    if (!d_q || !d_out || ((uintptr_t)d_out & 15u)) return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(ctx->device);
    hipError_t e = guard.status();
    if (e != hipSuccess) return from_hip(e);
    return from_hip(hh::launch_dequant_int4(d_q, m, groups, out_dtype, d_out, ctx->num_cus,
                                            pick_stream(ctx, stream)));
}

// ---------------------------------------------------------------- HCT-T

int32_t hh_hctt_decode_batch(hh_context *ctx, const hh_hctt_tensor *tensors, uint32_t n,
                             int32_t out_dtype, void *stream) {
    if (!ctx || (!tensors && n)) return HH_ERR_INVALID_ARGUMENT;
    if (out_dtype != HH_F32 && out_dtype != HH_F16 && out_dtype != HH_BF16)
        return HH_ERR_UNSUPPORTED;
    size_t total = 0;
    for (uint32_t i = 0; i < n; i++) {
        size_t nt = 0;
        int32_t rc = hh::check_hctt_tensor(tensors[i], &nt);
        if (rc != HH_OK) return rc;
        total += nt;
    }
    if (total == 0) return HH_OK;
    if (total > 0xffffffffu) return HH_ERR_UNSUPPORTED;
    hh::DeviceGuard guard(ctx->device);
    hipError_t e = guard.status();
    if (e != hipSuccess) return from_hip(e);
    return from_hip(hh::launch_hctt_decode(tensors, n, out_dtype, ctx->d_basis, ctx->num_cus,
                                           pick_stream(ctx, stream)));
}

int32_t hh_hctt_decode_lz4_batch(hh_context *ctx, const uint8_t *d_in, size_t in_total, const uint64_t *d_in_off,
                                 const uint32_t *d_in_len, uint8_t *d_scratch, const uint64_t *d_out_off,
                                 const uint32_t *d_out_cap, uint32_t nblocks, hh_block_status *d_status,
                                 const hh_hctt_tensor *tensors, uint32_t ntensors, int32_t out_dtype,
                                 void *stream) {
    // both launches on the caller's stream: the tile decode reads the
    // scratch after every block has been written
    if (!ctx || (!tensors && ntensors)) return HH_ERR_INVALID_ARGUMENT;
    int32_t rc = lz4_batch_with(ctx, hh::lz4_decoder_for_tiles(ctx, tensors, ntensors), d_in, in_total, d_in_off,
                                d_in_len, d_scratch, d_out_off, d_out_cap, nblocks, d_status, stream, true);
    if (rc != HH_OK) return rc;
    return hh_hctt_decode_batch(ctx, tensors, ntensors, out_dtype, stream);
}

int32_t hh_hctt_decode_lz4_fused_tpb(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                     const uint64_t *d_in_off, const uint32_t *d_in_len, uint32_t nblocks,
                                     hh_block_status *d_status, const hh_hctt_tensor *tensors, uint32_t ntensors,
                                     const uint32_t *tiles_per_block, int32_t out_dtype, void *stream) {
    if (!ctx || (!tensors && ntensors) || (!tiles_per_block && ntensors)) return HH_ERR_INVALID_ARGUMENT;
    if (out_dtype != HH_F32 && out_dtype != HH_F16 && out_dtype != HH_BF16) return HH_ERR_UNSUPPORTED;
    uint64_t need = 0, total = 0;
    for (uint32_t i = 0; i < ntensors; i++) {
        const hh_hctt_tensor &T = tensors[i];
        const uint32_t tpb = tiles_per_block[i];
        if (tpb == 0) return HH_ERR_INVALID_ARGUMENT;
        if (T.rows % 64 || T.cols % 64 || T.cols > (1u << 24) || T.k < 1 || T.k > 4096) return HH_ERR_INVALID_ARGUMENT;
        const uint64_t nt = (uint64_t)(T.rows / 64) * (T.cols / 64);
        if (nt == 0) continue;
        if (!T.d_out || ((uintptr_t)T.d_out & 15u)) return HH_ERR_INVALID_ARGUMENT;
        if ((uint64_t)tpb * hh_hctt_tile_bytes(T.k) > hh::fused_block_max()) return HH_ERR_UNSUPPORTED;
        need += (nt + tpb - 1) / tpb;
        total += nt;
    }
    if (need != nblocks) return HH_ERR_INVALID_ARGUMENT;
    if (nblocks == 0) return HH_OK;
    if (total > 0xffffffffu) return HH_ERR_UNSUPPORTED;
    if (!d_in || !d_in_off || !d_in_len || !d_status) return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    return from_hip(hh::launch_hctt_lz4_fused(tensors, ntensors, tiles_per_block, d_in, in_total, d_in_off,
                                              d_in_len, d_status, out_dtype, ctx->d_basis, ctx->num_cus,
                                              ctx->fused_poll_limit,
                                              hh::lz4_decoder_for_tiles(ctx, tensors, ntensors) == HH_LZ4_SEQ,
                                              pick_stream(ctx, stream)));
}

int32_t hh_hctt_decode_lz4_fused(hh_context *ctx, const uint8_t *d_in, size_t in_total, const uint64_t *d_in_off,
                                 const uint32_t *d_in_len, uint32_t nblocks, hh_block_status *d_status,
                                 const hh_hctt_tensor *tensors, uint32_t ntensors, uint32_t tiles_per_block,
                                 int32_t out_dtype, void *stream) {
    if (!ctx || (!tensors && ntensors) || tiles_per_block == 0) return HH_ERR_INVALID_ARGUMENT;
    std::vector<uint32_t> tpb(ntensors, tiles_per_block);
    return hh_hctt_decode_lz4_fused_tpb(ctx, d_in, in_total, d_in_off, d_in_len, nblocks, d_status, tensors,
                                        ntensors, tpb.data(), out_dtype, stream);
}

int32_t hh_hctt_decode(hh_context *ctx, const uint8_t *d_tiles, size_t tiles_len, uint32_t rows,
                       uint32_t cols, uint32_t k, int32_t out_dtype, void *d_out,
                       int32_t *d_tile_status, void *stream) {
    hh_hctt_tensor T = {d_tiles, tiles_len, rows, cols, k, d_out, d_tile_status};
    return hh_hctt_decode_batch(ctx, &T, 1, out_dtype, stream);
}

// ---------------------------------------------------------------- HCT container

namespace {

uint32_t rd_u32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint64_t rd_u64(const uint8_t *p) { return (uint64_t)rd_u32(p) | ((uint64_t)rd_u32(p + 4) << 32); }

int32_t fail(hh_block_status *st, int32_t code, int32_t detail, uint64_t pos = 0,
             uint64_t req = 0) {
    if (st) {
        st->code = code;
        st->detail = detail;
        st->position = pos;
        st->required = req;
        st->written = 0;
    }
    return code;
}

}  // namespace

int32_t hh_hct_read_header(const uint8_t *file, size_t file_len, hh_hct_info *info,
                           hh_block_status *status) {
    if (!info || (!file && file_len)) return HH_ERR_INVALID_ARGUMENT;
    std::memset(info, 0, sizeof(*info));
    if (status) std::memset(status, 0, sizeof(*status));
    const size_t kHeader = 64;
    if (file_len < kHeader) return fail(status, HH_ERR_ALGORITHM, HH_CORRUPT_NONE, file_len);
    if (std::memcmp(file, "HCTN", 4) != 0) return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_HEADER);
    info->version = rd_u32(file + 4);
    if (info->version > 2) return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_HEADER);
    info->algorithm = file[8];
    info->dtype = file[9];
    if (info->algorithm > 1 || info->dtype > 4)
        return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_HEADER);
    info->flags = (uint16_t)(file[10] | (file[11] << 8));
    info->original_size = rd_u64(file + 12);
    info->compressed_size = rd_u64(file + 20);
    info->block_size = rd_u32(file + 28);
    info->num_blocks = rd_u32(file + 32);
    info->rank = file[36];
    // four dimensions would overrun the 64-byte header (37 + 4 * 8 > 64)
    if (info->rank > 3) return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_HEADER);
    for (uint32_t i = 0; i < info->rank; i++) info->shape[i] = rd_u64(file + 37 + 8 * i);
    info->index_entry_size = 8;
    info->data_offset = kHeader + (uint64_t)info->num_blocks * 8;
    if (info->data_offset > file_len) return fail(status, HH_ERR_ALGORITHM, HH_CORRUPT_NONE, file_len);
    return HH_OK;
}

}  // extern "C"

namespace {

// The block loop shared by HctReader::decompress_all (v1, tensor.rs:486-515)
// and HctReaderV2::decompress_all_validated / validate_checksums (:937-1020):
// host checks of every index entry, one batched XXH3 launch (validate) and
// one batched LZ4 launch (decode) over the blocks that can be read, then
// the reference's per-block order of errors: index range, checksum, last
// block size, output capacity, LZ4 result.
int32_t hct_blocks(hh_context *ctx, const uint8_t *h_file, const uint8_t *d_file, size_t file_len,
                   const hh_hct_info &info, bool validate, bool decode, uint8_t *d_out,
                   size_t out_cap, size_t *written, hh_block_status *status, int64_t *failed_block,
                   void *stream) {
    const uint32_t n = info.num_blocks;
    const uint32_t entry = info.index_entry_size;
    const uint8_t *index = h_file + (info.data_offset - (uint64_t)n * entry);
    // blocks [0, m) can be read (:470-480); size_fail: the last one's
    // expected size is inconsistent (:494-500 / :988-994)
    uint32_t m = n;
    bool size_fail = false;
    std::vector<uint64_t> in_off(n), out_off(n), sum(n, 0);
    std::vector<uint32_t> in_len(n), expect(n);
    uint64_t nominal = 0;
    for (uint32_t b = 0; b < n; b++) {
        const uint8_t *ie = index + (size_t)entry * b;
        const uint32_t off = rd_u32(ie), csz = rd_u32(ie + 4);
        if (entry == 16) sum[b] = rd_u64(ie + 8);
        if (info.data_offset + off + csz > file_len) {
            m = b;
            break;
        }
        uint64_t e = info.block_size;
        if (b == n - 1) {
            const uint64_t full = (uint64_t)(n - 1) * info.block_size;
            if (full > info.original_size) {
                size_fail = true;
                e = 0;
            } else {
                e = info.original_size - full;
            }
        }
        if (e > 0xffffffffull) return fail(status, HH_ERR_UNSUPPORTED, HH_CORRUPT_NONE);
        in_off[b] = info.data_offset + off;
        in_len[b] = csz;
        expect[b] = (uint32_t)e;
        out_off[b] = nominal;
        nominal += e;
    }
    // blocks that are decoded: the readable ones, less a last block of
    // inconsistent size
    const uint32_t md = decode ? (size_fail && m == n ? n - 1 : m) : 0;
    hh::DeviceGuard guard(ctx->device);
    hipError_t he = guard.status();
    if (he != hipSuccess) return from_hip(he);
    hipStream_t s = pick_stream(ctx, stream);
    const bool direct = nominal <= out_cap;
    const size_t tab = (size_t)m * (32 + 8 + 8 + 4 + 4 + 8);
    const size_t stage_at = (tab + 255) & ~(size_t)255;
    std::vector<hh_block_status> st(md);
    std::vector<uint64_t> hash(validate ? m : 0);
    int32_t rc = HH_OK;
    uint8_t *base = nullptr;
    if (m > 0) {
        rc = ensure_scratch(ctx, stage_at + (decode && !direct ? nominal : 0) + 16);
        if (rc != HH_OK) return rc;
        base = reinterpret_cast<uint8_t *>(ctx->d_scratch);
        hh_block_status *d_st = reinterpret_cast<hh_block_status *>(base);
        uint64_t *d_in_off = reinterpret_cast<uint64_t *>(base + (size_t)m * 32);
        uint64_t *d_out_off = d_in_off + m;
        uint64_t *d_hash = d_out_off + m;
        uint32_t *d_in_len = reinterpret_cast<uint32_t *>(d_hash + m);
        uint32_t *d_cap = d_in_len + m;
        uint8_t *dst = direct ? d_out : base + stage_at;
        he = hipMemcpyAsync(d_in_off, in_off.data(), 8 * (size_t)m, hipMemcpyHostToDevice, s);
        if (he == hipSuccess)
            he = hipMemcpyAsync(d_in_len, in_len.data(), 4 * (size_t)m, hipMemcpyHostToDevice, s);
        if (he == hipSuccess && validate)
            he = hh::launch_xxh3_batch(d_file, file_len, d_in_off, d_in_len, m, d_hash, s);
        if (he == hipSuccess && validate)
            he = hipMemcpyAsync(hash.data(), d_hash, 8 * (size_t)m, hipMemcpyDeviceToHost, s);
        if (md > 0) {
            if (he == hipSuccess)
                he = hipMemcpyAsync(d_out_off, out_off.data(), 8 * (size_t)md, hipMemcpyHostToDevice, s);
            if (he == hipSuccess)
                he = hipMemcpyAsync(d_cap, expect.data(), 4 * (size_t)md, hipMemcpyHostToDevice, s);
            const hh::Lz4Batch B = {d_file,    file_len, d_in_off, d_in_len, dst, direct ? out_cap : nominal,
                                    d_out_off, d_cap,    md,       d_st};
            if (he == hipSuccess) he = hh::launch_lz4_batch(B, hh::lz4_decoder_for(ctx, HH_LZ4_RING4), s);
            if (he == hipSuccess)
                he = hipMemcpyAsync(st.data(), d_st, 32 * (size_t)md, hipMemcpyDeviceToHost, s);
        }
        if (he == hipSuccess) he = hipStreamSynchronize(s);
        if (he != hipSuccess) return from_hip(he);
    }
    // the reference's loop, block by block
    uint64_t op = 0;
    bool shifted = false;
    for (uint32_t b = 0; b < n; b++) {
        if (b == m) {  // read_block / read_block_validated: read_exact fails
            if (failed_block) *failed_block = b;
            return fail(status, HH_ERR_ALGORITHM, HH_CORRUPT_NONE, file_len);
        }
        if (validate && sum[b] != 0 && hash[b] != sum[b]) {
            if (failed_block) *failed_block = b;
            return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_BLOCK_CHECKSUM);
        }
        if (!decode) continue;
        if (b == n - 1 && size_fail) {
            if (failed_block) *failed_block = b;
            return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_SIZE);
        }
        if (op + expect[b] > out_cap) {
            if (failed_block) *failed_block = b;
            return fail(status, HH_ERR_BUFFER_TOO_SMALL, HH_CORRUPT_NONE, 0, op + expect[b]);
        }
        if (st[b].code != HH_OK) {
            if (failed_block) *failed_block = b;
            if (status) *status = st[b];
            return st[b].code;
        }
        if (op != out_off[b]) shifted = true;
        op += st[b].written;
    }
    if (decode && md > 0 && (shifted || !direct)) {
        // a short block shifts the blocks after it (truncate, then extend)
        if (direct) {  // bounce buffer for the overlapping moves to the left
            uint64_t maxw = 0;
            for (uint32_t b = 0; b < md; b++) maxw = st[b].written > maxw ? st[b].written : maxw;
            rc = ensure_scratch(ctx, stage_at + maxw + 16);
            if (rc != HH_OK) return rc;
        }
        uint8_t *scr = reinterpret_cast<uint8_t *>(ctx->d_scratch);
        uint64_t o = 0;
        for (uint32_t b = 0; b < md && he == hipSuccess; b++) {
            const uint64_t w = st[b].written;
            if (w && (!direct || o != out_off[b])) {
                if (direct) {
                    he = hipMemcpyAsync(scr + stage_at, d_out + out_off[b], w, hipMemcpyDeviceToDevice, s);
                    if (he == hipSuccess)
                        he = hipMemcpyAsync(d_out + o, scr + stage_at, w, hipMemcpyDeviceToDevice, s);
                } else {
                    he = hipMemcpyAsync(d_out + o, scr + stage_at + out_off[b], w, hipMemcpyDeviceToDevice, s);
                }
            }
            o += w;
        }
        if (he == hipSuccess) he = hipStreamSynchronize(s);
        if (he != hipSuccess) return from_hip(he);
    }
    if (written) *written = op;
    if (status) {
        std::memset(status, 0, sizeof(*status));
        status->written = op;
    }
    return HH_OK;
}

}  // namespace

extern "C" {

int32_t hh_hct_decompress_all(hh_context *ctx, const uint8_t *h_file, const uint8_t *d_file,
                              size_t file_len, uint8_t *d_out, size_t out_cap, size_t *written,
                              hh_block_status *status, int64_t *failed_block, void *stream) {
    if (written) *written = 0;
    if (failed_block) *failed_block = -1;
    if (!ctx || !h_file || !d_file || (!d_out && out_cap)) return HH_ERR_INVALID_ARGUMENT;
    hh_hct_info info;
    int32_t rc = hh_hct_read_header(h_file, file_len, &info, status);
    if (rc != HH_OK) return rc;
    return hct_blocks(ctx, h_file, d_file, file_len, info, false, true, d_out, out_cap, written, status,
                      failed_block, stream);
}

uint64_t hh_xxh3_64(const uint8_t *data, size_t len) {
    if (!data && len) return 0;
    return hh::xxh3_64_host(data, len);
}

int32_t hh_xxh3_64_batch(hh_context *ctx, const uint8_t *d_data, size_t data_len, const uint64_t *d_off,
                         const uint32_t *d_len, uint32_t n, uint64_t *d_out, void *stream) {
    if (!ctx) return HH_ERR_INVALID_ARGUMENT;
    if (n == 0) return HH_OK;
    if (!d_data || !d_off || !d_len || !d_out) return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(ctx->device);
    hipError_t e = guard.status();
    if (e == hipSuccess) e = hh::launch_xxh3_batch(d_data, data_len, d_off, d_len, n, d_out, pick_stream(ctx, stream));
    return from_hip(e);
}

int32_t hh_hct_read_header_v2(const uint8_t *file, size_t file_len, hh_hct_info *info,
                              hh_hct_quant *quant, hh_block_status *status) {
    if (!info || (!file && file_len)) return HH_ERR_INVALID_ARGUMENT;
    if (quant) std::memset(quant, 0, sizeof(*quant));
    // header fields (from_bytes); the v1 index geometry is replaced below
    int32_t rc = hh_hct_read_header(file, file_len < 64 ? file_len : 64, info, status);
    if (rc != HH_OK) {
        // a v1-sized index that does not fit is not an error yet: only the
        // header itself was given to the v1 parse
        if (!(rc == HH_ERR_ALGORITHM && file_len >= 64)) return rc;
    }
    if (info->version >= 2 && (info->flags & 0x0001u) &&
        hh::xxh3_64_host(file, 56) != rd_u64(file + 56))
        return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_HEADER_CHECKSUM);
    uint64_t at = 64;
    if (info->flags & 0x0004u) {  // QuantizationMetadata (:868-876, :207-226)
        if (file_len < at + 8) return fail(status, HH_ERR_ALGORITHM, HH_CORRUPT_NONE, file_len);
        const uint8_t *q = file + at;
        if (q[0] > 4) return fail(status, HH_ERR_CORRUPTED_DATA, HH_CORRUPT_QUANT_SCHEME);
        if (quant) {
            quant->present = 1;
            quant->scheme = q[0];
            quant->has_per_group_scales = q[1] != 0;
            quant->scale_bits = (uint16_t)(q[2] | (q[3] << 8));
            quant->zero_point = (int8_t)q[4];
            quant->group_size = (uint32_t)q[5] | ((uint32_t)q[6] << 8) | ((uint32_t)q[7] << 16);
        }
        at += 8;
    }
    info->index_entry_size = (info->version >= 2 && (info->flags & 0x0002u)) ? 16u : 8u;
    info->data_offset = at + (uint64_t)info->num_blocks * info->index_entry_size;
    if (info->data_offset > file_len) return fail(status, HH_ERR_ALGORITHM, HH_CORRUPT_NONE, file_len);
    if (status) std::memset(status, 0, sizeof(*status));
    return HH_OK;
}

int32_t hh_hct_decompress_all_validated(hh_context *ctx, const uint8_t *h_file, const uint8_t *d_file,
                                        size_t file_len, uint8_t *d_out, size_t out_cap,
                                        size_t *written, hh_block_status *status,
                                        int64_t *failed_block, void *stream) {
    if (written) *written = 0;
    if (failed_block) *failed_block = -1;
    if (!ctx || !h_file || !d_file || (!d_out && out_cap)) return HH_ERR_INVALID_ARGUMENT;
    hh_hct_info info;
    int32_t rc = hh_hct_read_header_v2(h_file, file_len, &info, nullptr, status);
    if (rc != HH_OK) return rc;
    return hct_blocks(ctx, h_file, d_file, file_len, info, true, true, d_out, out_cap, written, status,
                      failed_block, stream);
}

int32_t hh_hct_validate_checksums(hh_context *ctx, const uint8_t *h_file, const uint8_t *d_file,
                                  size_t file_len, hh_block_status *status, int64_t *failed_block,
                                  void *stream) {
    if (failed_block) *failed_block = -1;
    if (!ctx || !h_file || !d_file) return HH_ERR_INVALID_ARGUMENT;
    hh_hct_info info;
    int32_t rc = hh_hct_read_header_v2(h_file, file_len, &info, nullptr, status);
    if (rc != HH_OK) return rc;
    return hct_blocks(ctx, h_file, d_file, file_len, info, true, false, nullptr, 0, nullptr, status,
                      failed_block, stream);
}

}  // extern "C"
