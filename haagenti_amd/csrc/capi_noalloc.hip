// hh_hctt_decode_lz4_batch_noalloc: the one-call layer decode
// (hh_hctt_decode_lz4_batch) for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops that forbid hipMalloc): the
// LZ4 output (the layer's tile bytes) goes to a device array the library
// owns instead of a caller-provided scratch.
//
// The array is a file-scope device variable: each GPU the library runs on
// holds one copy of kNoAllocScratchBytes from the moment the code object is
// loaded on it until the process ends.  Host code never uses the array's
// name as an address (on the host it is only a handle for the runtime); the
// device address is looked up once per device with hipGetSymbolAddress, with
// that device current, and kept per device.
//
// Every call on one GPU uses that GPU's single array: calls that overlap on
// one GPU (on different streams, or from different threads) race and must be
// serialised by the caller.  The array keeps the last call's bytes; nothing
// in it needs to start at zero (every tile byte the tile decode reads is
// written first by the LZ4 block that covers it, or zeroed when that block
// fails).
#include <mutex>

#include "hh_internal.hpp"

namespace {

static __device__ __align__(256) uint8_t scratch[HH_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t *g_ptr[kMaxDevices] = {};

}  // namespace

namespace hh {

// Device address of this device's array (the device must be current).
hipError_t noalloc_scratch(int device, uint8_t **out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_ptr[device] = reinterpret_cast<uint8_t *>(p);
    }
    *out = g_ptr[device];
    return hipSuccess;
}

}  // namespace hh

extern "C" {

int32_t hh_hctt_decode_lz4_batch_noalloc(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                         const uint64_t *d_in_off, const uint32_t *d_in_len,
                                         const uint64_t *d_out_off, const uint32_t *d_out_cap, uint32_t nblocks,
                                         hh_block_status *d_status, const hh_hctt_tensor *tensors, uint32_t ntensors,
                                         int32_t out_dtype, void *stream) {
    if (!ctx || (!tensors && ntensors)) return HH_ERR_INVALID_ARGUMENT;
    if (out_dtype != HH_F32 && out_dtype != HH_F16 && out_dtype != HH_BF16) return HH_ERR_UNSUPPORTED;
    if (nblocks && (!d_in || !d_in_off || !d_in_len || !d_out_off || !d_out_cap || !d_status))
        return HH_ERR_INVALID_ARGUMENT;
    // the tensors' tiles are packed in order from the array's start
    uint64_t total = 0;
    for (uint32_t i = 0; i < ntensors; i++) {
        if (tensors[i].d_tiles != nullptr) return HH_ERR_INVALID_ARGUMENT;
        if (tensors[i].tiles_len > HH_NOALLOC_SCRATCH_BYTES - total) return HH_ERR_BUFFER_TOO_SMALL;
        total += tensors[i].tiles_len;
    }
    hh::DeviceGuard guard(ctx->device);
    if (guard.status() != hipSuccess) return hh::from_hip(guard.status());
    if (ctx->noalloc_status != hipSuccess) return hh::from_hip(ctx->noalloc_status);
    uint8_t *base = ctx->noalloc_scratch;
    // every tensor is checked before anything is enqueued
    {
        uint64_t off = 0, ntiles = 0;
        for (uint32_t i = 0; i < ntensors; i++) {
            hh_hctt_tensor t = tensors[i];
            t.d_tiles = base + off;
            size_t nt = 0;
            const int32_t rc = hh::check_hctt_tensor(t, &nt);
            if (rc != HH_OK) return rc;
            off += t.tiles_len;
            ntiles += nt;
        }
        if (ntiles > 0xffffffffull) return HH_ERR_UNSUPPORTED;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (nblocks) {
        // blocks writing outside the packed tile bytes are reported, not run
        const hh::Lz4Batch B = {d_in, in_total, d_in_off, d_in_len, base, total, d_out_off, d_out_cap,
                                nblocks, d_status, 1u};
        const hipError_t e = hh::launch_lz4_batch(B, hh::lz4_decoder_for_tiles(ctx, tensors, ntensors), s);
        if (e != hipSuccess) return hh::from_hip(e);
    }
    // the tile decode, eight tensors at a time from a fixed-size copy
    hh_hctt_tensor local[8];
    uint64_t off = 0;
    for (uint32_t i = 0; i < ntensors; i += 8) {
        const uint32_t n = ntensors - i < 8 ? ntensors - i : 8;
        for (uint32_t j = 0; j < n; j++) {
            local[j] = tensors[i + j];
            local[j].d_tiles = base + off;
            off += local[j].tiles_len;
        }
        const int32_t rc = hh_hctt_decode_batch(ctx, local, n, out_dtype, stream);
        if (rc != HH_OK) return rc;
    }
    return HH_OK;
}

}  // extern "C"
