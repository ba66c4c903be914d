// Streaming device copy: the HBM bandwidth calibration of the measurements
// (the rate a kernel that reads and writes each byte once can reach, and the
// scale of the FETCH_SIZE / WRITE_SIZE counters).  Each thread of a
// grid-stride loop moves four 16-byte chunks per iteration, all four loads
// issued before the stores; the bytes before the first 16-aligned source
// address and after the last whole chunk are copied one by one.
#include "hh_internal.hpp"

namespace hh {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kThreads) void copy16_kernel(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst,
                                                          uint64_t n16) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < kUnroll; u++) __builtin_nontemporal_store(v[u], dst + i + u * stride);
    }
    for (; i < n16; i += stride) dst[i] = src[i];
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
    if (n16) {
        const uint32_t cus = (uint32_t)(ctx->num_cus > 0 ? ctx->num_cus : 256);
        uint64_t grid = (n16 + hh::kThreads * hh::kUnroll - 1) / (hh::kThreads * hh::kUnroll);
        if (grid > 4ull * cus) grid = 4ull * cus;
        hipLaunchKernelGGL(hh::copy16_kernel, dim3((uint32_t)grid), dim3(hh::kThreads), 0, s,
                           reinterpret_cast<const hh::u32x4 *>(s8 + head), reinterpret_cast<hh::u32x4 *>(d8 + head),
                           n16);
    }
    if (tail)
        hipLaunchKernelGGL(hh::copy_bytes_kernel, dim3((uint32_t)((tail + 255) / 256)), dim3(256), 0, s,
                           s8 + tail_at, d8 + tail_at, tail);
    return hh::from_hip(hipGetLastError());
}
