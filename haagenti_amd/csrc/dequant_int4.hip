// INT4 dequantization with per-32-element f16 scales, streaming kernel.
//
// Semantics: crates/haagenti/src/testing/quantization.rs:82-131
//   out[i] = f32(nibble_i - 8) * f32(scale[i / 32])
// with offset-binary nibbles, low nibble first, and the f16 scale decoded
// exactly (quantization.rs:166-197).  One IEEE f32 multiply per element, so
// the f32 output is bit-identical to the reference; bf16/f16 outputs are the
// round-to-nearest-even of that f32.
//
// Layout in HBM: [G f16 scales][ceil(n/2) packed bytes] (G = ceil(n/32)).
// Each lane produces one 16-byte output vector per step (4 f32 or 8 half
// values), so every wave store covers one contiguous 1 KiB span; its input
// is 2 or 4 packed bytes plus one scale shared by 8 (f32) or 4 (16-bit)
// lanes.  The kernel is HBM-bound: 0.5 B + 1/16 B in, 2 or 4 B out per
// element.
#include "hh_internal.hpp"

namespace hh {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

template <int DT, bool ALIGNED>
__device__ __forceinline__ void dequant_chunk(const uint8_t *__restrict__ q,
                                              const uint8_t *__restrict__ nib, uint64_t c,
                                              void *__restrict__ out) {
    constexpr int E = (DT == HH_F32) ? 4 : 8;  // elements per 16-byte store
    const uint64_t e0 = c * E;
    const uint64_t g = e0 >> 5;
    uint32_t sbits;
    uint32_t w;
    if constexpr (ALIGNED) {
        sbits = reinterpret_cast<const uint16_t *>(q)[g];
        if constexpr (E == 4)
            w = reinterpret_cast<const uint16_t *>(nib)[e0 >> 2];
        else
            w = reinterpret_cast<const uint32_t *>(nib)[e0 >> 3];
    } else {
        sbits = (uint32_t)q[2 * g] | ((uint32_t)q[2 * g + 1] << 8);
        const uint8_t *p = nib + (e0 >> 1);
        w = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
        if constexpr (E == 8) w |= ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    }
    const float s = f16_bits_to_f32(sbits);
    float v[E];
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = (float)((int)((w >> (4 * i)) & 15u) - 8) * s;
    if constexpr (DT == HH_F32) {
        float4 o = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4 *>(out)[c] = o;
    } else {
        uint32_t p[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t lo = DT == HH_BF16 ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
            uint32_t hi = DT == HH_BF16 ? f32_to_bf16_bits(v[2 * i + 1]) : f32_to_f16_bits(v[2 * i + 1]);
            p[i] = lo | (hi << 16);
        }
        reinterpret_cast<uint4 *>(out)[c] = make_uint4(p[0], p[1], p[2], p[3]);
    }
}

template <int DT, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void dequant_int4_kernel(const uint8_t *__restrict__ q,
                                                                uint64_t n, uint64_t ngroups,
                                                                void *__restrict__ out) {
    constexpr int E = (DT == HH_F32) ? 4 : 8;
    const uint8_t *__restrict__ nib = q + 2 * ngroups;
    const uint64_t nchunks = n / E;
    const uint64_t G = (uint64_t)gridDim.x * kThreads;
    for (uint64_t base = (uint64_t)blockIdx.x * kThreads + threadIdx.x; base < nchunks;
         base += G * kUnroll) {
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const uint64_t c = base + (uint64_t)u * G;
            if (c < nchunks) dequant_chunk<DT, ALIGNED>(q, nib, c, out);
        }
    }
    // ragged tail (< E elements), element by element
    if (blockIdx.x == 0 && threadIdx.x < (uint32_t)(n - nchunks * E)) {
        const uint64_t i = nchunks * E + threadIdx.x;
        const uint64_t g = i >> 5;
        const float s = f16_bits_to_f32((uint32_t)q[2 * g] | ((uint32_t)q[2 * g + 1] << 8));
        const uint32_t b = nib[i >> 1];
        const float v = (float)((int)((i & 1) ? (b >> 4) : (b & 15u)) - 8) * s;
        if (DT == HH_F32)
            reinterpret_cast<float *>(out)[i] = v;
        else
            reinterpret_cast<uint16_t *>(out)[i] =
                (uint16_t)(DT == HH_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
    }
}

template <int DT>
hipError_t launch_typed(const uint8_t *d_q, size_t n, size_t ngroups, void *d_out, int num_cus,
                        hipStream_t s) {
    constexpr int E = (DT == HH_F32) ? 4 : 8;
    const uint64_t nchunks = n / E;
    uint64_t want = (nchunks + (uint64_t)kThreads * kUnroll - 1) / ((uint64_t)kThreads * kUnroll);
    uint64_t cap = (uint64_t)(num_cus > 0 ? num_cus : 256) * 16;
    uint32_t grid = (uint32_t)(want < 1 ? 1 : (want > cap ? cap : want));
    const uintptr_t qa = (uintptr_t)d_q, na = qa + 2 * ngroups;
    // Output is 16-byte aligned (checked by the caller); the input may not be.
    const bool aligned = (qa % 2 == 0) && (E == 4 ? na % 2 == 0 : na % 4 == 0);
    if (aligned)
        hipLaunchKernelGGL((dequant_int4_kernel<DT, true>), dim3(grid), dim3(kThreads), 0, s, d_q,
                           (uint64_t)n, (uint64_t)ngroups, d_out);
    else
        hipLaunchKernelGGL((dequant_int4_kernel<DT, false>), dim3(grid), dim3(kThreads), 0, s,
                           d_q, (uint64_t)n, (uint64_t)ngroups, d_out);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dequant_int4(const uint8_t *d_q, size_t n, size_t ngroups, int dtype,
                               void *d_out, int num_cus, hipStream_t s) {
    if (n == 0) return hipSuccess;
    switch (dtype) {
        case HH_F32: return launch_typed<HH_F32>(d_q, n, ngroups, d_out, num_cus, s);
        case HH_F16: return launch_typed<HH_F16>(d_q, n, ngroups, d_out, num_cus, s);
        case HH_BF16: return launch_typed<HH_BF16>(d_q, n, ngroups, d_out, num_cus, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hh
