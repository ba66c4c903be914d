// Streaming device copy: the HBM bandwidth calibration of the measurements
// (the rate a kernel that reads and writes each byte once can reach, and the
// scale of the FETCH_SIZE / WRITE_SIZE counters).  Each workgroup copies one
// contiguous 16 KiB piece: each of its 256 threads moves four 16-byte chunks
// (a wave's 1 KiB apart), all four non-temporal loads issued before the
// stores.  Contiguous pieces per workgroup keep each wave's accesses in few
// DRAM pages; a grid-stride loop over the whole buffer (each thread's chunks
// a grid apart) measured 20-30 % slower.  The bytes before the first
// 16-aligned source address and after the last whole chunk are copied one by
// one.
#include "hh_internal.hpp"

namespace hh {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kThreads) void copy16_kernel(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst,
                                                          uint64_t n16) {
    const uint64_t base = (uint64_t)blockIdx.x * (kThreads * kUnroll) + threadIdx.x;
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const uint64_t j = base + (uint64_t)u * kThreads;
        if (j < n16) v[u] = __builtin_nontemporal_load(src + j);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const uint64_t j = base + (uint64_t)u * kThreads;
        if (j < n16) __builtin_nontemporal_store(v[u], dst + j);
    }
}

__global__ void copy_bytes_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

}  // namespace
}  // namespace hh

int32_t hh_hbm_copy(hh_context *ctx, void *d_dst, const void *d_src, uint64_t bytes, void *stream) {
    if (!ctx) return HH_ERR_INVALID_ARGUMENT;
    if (bytes == 0) return HH_OK;
    if (!d_dst || !d_src) return HH_ERR_INVALID_ARGUMENT;
    const uint8_t *s8 = reinterpret_cast<const uint8_t *>(d_src);
    uint8_t *d8 = reinterpret_cast<uint8_t *>(d_dst);
    if ((s8 < d8 + bytes) && (d8 < s8 + bytes)) return HH_ERR_INVALID_ARGUMENT;  // overlapping ranges
    hh::DeviceGuard guard(ctx->device);
    if (guard.status() != hipSuccess) return hh::from_hip(guard.status());
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // the 16-byte body needs both pointers at the same offset mod 16
    uint64_t head = (16u - ((uintptr_t)s8 & 15u)) & 15u;
    if (((uintptr_t)s8 & 15u) != ((uintptr_t)d8 & 15u)) head = bytes;
    if (head > bytes) head = bytes;
    const uint64_t n16 = (bytes - head) / 16, tail_at = head + 16 * n16, tail = bytes - tail_at;
    if (head)
        hipLaunchKernelGGL(hh::copy_bytes_kernel, dim3((uint32_t)((head + 255) / 256)), dim3(256), 0, s, s8, d8,
                           head);
    // one workgroup per 16 KiB piece, launches of at most 2^31 - 1 pieces
    const uint64_t piece = (uint64_t)hh::kThreads * hh::kUnroll;
    for (uint64_t done = 0; done < n16;) {
        uint64_t n = n16 - done;
        const uint64_t max_n = 0x7fffffffull * piece;
        if (n > max_n) n = max_n;
        const uint64_t grid = (n + piece - 1) / piece;
        hipLaunchKernelGGL(hh::copy16_kernel, dim3((uint32_t)grid), dim3(hh::kThreads), 0, s,
                           reinterpret_cast<const hh::u32x4 *>(s8 + head) + done,
                           reinterpret_cast<hh::u32x4 *>(d8 + head) + done, n);
        done += n;
    }
    if (tail)
        hipLaunchKernelGGL(hh::copy_bytes_kernel, dim3((uint32_t)((tail + 255) / 256)), dim3(256), 0, s,
                           s8 + tail_at, d8 + tail_at, tail);
    return hh::from_hip(hipGetLastError());
}
