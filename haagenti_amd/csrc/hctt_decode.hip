// HCT-T tile decode: INT4 dequant + bitmap scatter + 64x64 inverse DCT on
// MFMA, one wavefront per tile.
//
// Reference semantics (per tile):
//   dequantize_int4   crates/haagenti/src/testing/quantization.rs:82-131
//   bitmap scatter    crates/haagenti/src/compressive.rs:620-627, 741-745
//   idct_2d           crates/haagenti-core/src/dct.rs:311-337 (orthonormal
//                     DCT-III along both axes)
//
// Math.  With the basis M[v][j] = a_v cos(pi v (2j+1) / 128) (a_0 = 1/8,
// a_v = 1/sqrt(32)), the tile is X = M^T C M.  It is computed as two 64^3
// contractions on v_mfma_f32_32x32x16_f16:
//   GEMM1  S = C M     (A = C rows from LDS, B = M from registers)
//   GEMM2  X = M^T S   (A = M^T from registers, B = S straight from GEMM1's
//                       accumulators)
// The contraction index of both GEMMs runs in the order pi(k) below, which
// is exactly the row order of the 32x32 accumulator layout, so GEMM1's
// output registers are GEMM2's B fragments without any shuffle or LDS trip,
// and the same M fragments serve as GEMM1's B and GEMM2's A.
//
// Precision.  Every operand is split into f16 hi + lo (x = hi + lo exactly
// for the coefficients, to ~2^-22 for M and S) and each GEMM runs three
// passes hi*hi + hi*lo + lo*hi with f32 accumulation, giving ~f32 accuracy
// (the bar is max-abs error <= 1e-3 x RMS).  Coefficients are prescaled by
// 2^E per tile (E from the largest f16 scale exponent) and M by 2^8 so that
// the lo parts stay in f16's normal range; the output is rescaled exactly.
//
// LDS per wave: staged tile bytes, scaled f32 scales, C hi and C lo
// (64 x 64 f16 each, 16-byte chunks XOR-swizzled by row to spread banks);
// the C area is reused to stage the output tile for coalesced row stores.
#include <cstring>

#include "hh_internal.hpp"

namespace hh {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kCBytes = 2u * 64u * 64u * 2u;  // C hi + C lo
constexpr uint32_t kScaleBytes = 512;               // up to 128 f32 scales

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ floatx16 mfma(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float pow2f(int e) {  // e in [-126, 127]
    return __uint_as_float((uint32_t)(e + 127) << 23);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t o = __shfl_xor(v, d);
        v = v > o ? v : o;
    }
    return v;
}

// Up to kMaxTensors tensors per launch, passed by value as kernel arguments.
// Tiles are numbered across the batch; tensor i owns [start[i], start[i+1]).
constexpr int kMaxTensors = 8;
struct TileBatch {
    const uint8_t *tiles[kMaxTensors];
    void *out[kMaxTensors];
    int32_t *status[kMaxTensors];
    uint32_t start[kMaxTensors + 1];
    uint32_t tiles_per_row[kMaxTensors];
    uint32_t cols[kMaxTensors];
    uint32_t k[kMaxTensors];
    uint32_t tb[kMaxTensors];
    uint32_t dword_ok[kMaxTensors];
    uint32_t n;
    uint32_t wave_lds;
};

template <int DT>
__global__ __launch_bounds__(kThreads, 1) void hctt_decode_kernel(TileBatch B,
                                                                   const half8 *__restrict__ basis) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const uint32_t wave_lds = B.wave_lds;
    uint8_t *wsm = smem + wave * wave_lds;
    const uint32_t payb = wave_lds - kScaleBytes - kCBytes;
    uint8_t *pay = wsm;
    float *sc32 = reinterpret_cast<float *>(wsm + payb);
    _Float16 *chi = reinterpret_cast<_Float16 *>(wsm + payb + kScaleBytes);
    _Float16 *clo = chi + 64 * 64;
    float *xs = reinterpret_cast<float *>(chi);

    half8 mf[2][2][4];  // [hi/lo][column block][k step]
#pragma unroll
    for (int hl = 0; hl < 2; hl++)
#pragma unroll
        for (int jb = 0; jb < 2; jb++)
#pragma unroll
            for (int s = 0; s < 4; s++) mf[hl][jb][s] = basis[((hl * 2 + jb) * 4 + s) * 64 + lane];

    const uint32_t ntiles = B.start[B.n];
    for (uint32_t gt = blockIdx.x * kWaves + wave; gt < ntiles; gt += gridDim.x * kWaves) {
        uint32_t ti = 0;
        while (ti + 1 < B.n && gt >= B.start[ti + 1]) ti++;
        const uint32_t t = gt - B.start[ti];
        const uint32_t k = B.k[ti], tb = B.tb[ti], cols = B.cols[ti];
        const uint32_t tiles_per_row = B.tiles_per_row[ti], dword_ok = B.dword_ok[ti];
        void *__restrict__ out = B.out[ti];
        int32_t *__restrict__ tstatus = B.status[ti];
        const uint32_t nsc = (k + 31) >> 5;
        const uint32_t nib_off = 512 + 2 * nsc;
        const uint8_t *src = B.tiles[ti] + (size_t)t * tb;
        // 1. stage the tile's bytes in LDS
        if (dword_ok) {
            const uint32_t *s32 = reinterpret_cast<const uint32_t *>(src);
            uint32_t *d32 = reinterpret_cast<uint32_t *>(pay);
            for (uint32_t i = lane; i < (tb >> 2); i += 64) d32[i] = s32[i];
        } else {
            for (uint32_t i = lane; i < tb; i += 64) pay[i] = src[i];
        }
        wave_sync();

        // 2. bitmap row `lane`: set-bit count and exclusive prefix over rows
        const uint64_t bits = reinterpret_cast<const uint64_t *>(pay)[lane];
        const uint32_t cnt = (uint32_t)__popcll(bits);
        uint32_t incl = cnt;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t y = __shfl_up(incl, d);
            if (lane >= d) incl += y;
        }
        const uint32_t total = __shfl(incl, 63);
        const bool ok = total == k;
        uint32_t rank = incl - cnt;

        // 3. per-tile power-of-two prescale from the largest scale exponent
        uint32_t emax = 0;
        for (uint32_t g = lane; g < nsc; g += 64) {
            const uint32_t sb = (uint32_t)pay[512 + 2 * g] | ((uint32_t)pay[513 + 2 * g] << 8);
            const uint32_t ex = (sb >> 10) & 31u;
            emax = ex > emax ? ex : emax;
        }
        emax = wave_max_u32(emax);
        const int E = 21 - (int)emax;
        const float pe = pow2f(E);
        for (uint32_t g = lane; g < nsc; g += 64) {
            const uint32_t sb = (uint32_t)pay[512 + 2 * g] | ((uint32_t)pay[513 + 2 * g] << 8);
            sc32[g] = f16_bits_to_f32(sb) * pe;
        }
        wave_sync();

        // 4. dequantize + scatter row `lane` into C hi/lo (swizzled chunks)
#pragma unroll
        for (int g = 0; g < 8; g++) {
            half8 hv, lv;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int v = 8 * g + e;
                float c = 0.0f;
                if (ok && ((bits >> v) & 1ull)) {
                    const uint32_t r = rank++;
                    const uint32_t byte = pay[nib_off + (r >> 1)];
                    const uint32_t q = (r & 1u) ? (byte >> 4) : (byte & 15u);
                    c = (float)((int)q - 8) * sc32[r >> 5];
                }
                const _Float16 hi = (_Float16)c;
                hv[e] = hi;
                lv[e] = (_Float16)(c - (float)hi);
            }
            const int sw = ((g ^ (lane & 7)) << 3);
            *reinterpret_cast<half8 *>(chi + lane * 64 + sw) = hv;
            *reinterpret_cast<half8 *>(clo + lane * 64 + sw) = lv;
        }
        wave_sync();

        // 5-7. Per 32-column block jb of the output:
        //   GEMM1: S[:, jb] = C M[:, jb]    (rows u, contraction over v in pi order)
        //   GEMM2: X[:, jb] = M^T S[:, jb]  (B fragments are GEMM1's accumulator rows)
        // and the block is parked in LDS.  Keeping one column block live at a
        // time halves the accumulator registers.
        const float s_down = 1.0f / 256.0f;
        const float os = pow2f(-(E + 8));
        float xv[2][16];
#pragma unroll
        for (int jb = 0; jb < 2; jb++) {
            floatx16 acc[2];
            acc[0] = floatx16{};
            acc[1] = floatx16{};
#pragma unroll
            for (int s = 0; s < 4; s++) {
#pragma unroll
                for (int ub = 0; ub < 2; ub++) {
                    const int u = 32 * ub + l32;
                    const int o1 = u * 64 + (((2 * s) ^ (u & 7)) << 3) + 4 * h;
                    const int o2 = u * 64 + (((2 * s + 1) ^ (u & 7)) << 3) + 4 * h;
                    const half4 h1 = *reinterpret_cast<const half4 *>(chi + o1);
                    const half4 h2 = *reinterpret_cast<const half4 *>(chi + o2);
                    const half4 q1 = *reinterpret_cast<const half4 *>(clo + o1);
                    const half4 q2 = *reinterpret_cast<const half4 *>(clo + o2);
                    const half8 ahi = __builtin_shufflevector(h1, h2, 0, 1, 2, 3, 4, 5, 6, 7);
                    const half8 alo = __builtin_shufflevector(q1, q2, 0, 1, 2, 3, 4, 5, 6, 7);
                    acc[ub] = mfma(ahi, mf[0][jb][s], acc[ub]);
                    acc[ub] = mfma(ahi, mf[1][jb][s], acc[ub]);
                    acc[ub] = mfma(alo, mf[0][jb][s], acc[ub]);
                }
            }
            floatx16 xacc[2];
            xacc[0] = floatx16{};
            xacc[1] = floatx16{};
#pragma unroll
            for (int ub = 0; ub < 2; ub++) {
#pragma unroll
                for (int t2 = 0; t2 < 2; t2++) {
                    const int sk = 2 * ub + t2;
                    half8 bhi, blo;
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float x = acc[ub][8 * t2 + e] * s_down;
                        const _Float16 hi = (_Float16)x;
                        bhi[e] = hi;
                        blo[e] = (_Float16)(x - (float)hi);
                    }
#pragma unroll
                    for (int ib = 0; ib < 2; ib++) {
                        xacc[ib] = mfma(mf[0][ib][sk], bhi, xacc[ib]);
                        xacc[ib] = mfma(mf[1][ib][sk], bhi, xacc[ib]);
                        xacc[ib] = mfma(mf[0][ib][sk], blo, xacc[ib]);
                    }
                }
            }
            if (jb == 0) {
#pragma unroll
                for (int ib = 0; ib < 2; ib++)
#pragma unroll
                    for (int r = 0; r < 16; r++) xv[ib][r] = xacc[ib][r] * os;
            } else {
                // C has been fully read (both column blocks): park the output
                wave_sync();
#pragma unroll
                for (int ib = 0; ib < 2; ib++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int i = 32 * ib + (r & 3) + 8 * (r >> 2) + 4 * h;
                        xs[i * 64 + l32] = xv[ib][r];
                        xs[i * 64 + 32 + l32] = xacc[ib][r] * os;
                    }
            }
        }
        wave_sync();

        // 8. coalesced row stores
        const uint32_t tr = t / tiles_per_row, tc = t % tiles_per_row;
        const size_t base = (size_t)(64 * tr) * cols + 64 * tc;
        if constexpr (DT == HH_F32) {
            float *o = reinterpret_cast<float *>(out) + base;
#pragma unroll
            for (int it = 0; it < 16; it++) {
                const int row = 4 * it + (lane >> 4), c4 = (lane & 15) * 4;
                const float4 v = *reinterpret_cast<const float4 *>(xs + row * 64 + c4);
                *reinterpret_cast<float4 *>(o + (size_t)row * cols + c4) = v;
            }
        } else {
            uint16_t *o = reinterpret_cast<uint16_t *>(out) + base;
#pragma unroll
            for (int it = 0; it < 8; it++) {
                const int row = 8 * it + (lane >> 3), c8 = (lane & 7) * 8;
                const float4 a = *reinterpret_cast<const float4 *>(xs + row * 64 + c8);
                const float4 b = *reinterpret_cast<const float4 *>(xs + row * 64 + c8 + 4);
                const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                uint32_t p[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t lo = DT == HH_BF16 ? f32_to_bf16_bits(f[2 * q]) : f32_to_f16_bits(f[2 * q]);
                    const uint32_t hi = DT == HH_BF16 ? f32_to_bf16_bits(f[2 * q + 1]) : f32_to_f16_bits(f[2 * q + 1]);
                    p[q] = lo | (hi << 16);
                }
                *reinterpret_cast<uint4 *>(o + (size_t)row * cols + c8) = make_uint4(p[0], p[1], p[2], p[3]);
            }
        }
        if (tstatus != nullptr && lane == 0) tstatus[t] = ok ? HH_OK : HH_ERR_CORRUPTED_DATA;
        wave_sync();
    }
}

}  // namespace

hipError_t launch_hctt_decode(const hh_hctt_tensor *tensors, uint32_t n, int dtype,
                              const void *d_basis, int num_cus, hipStream_t s) {
    for (uint32_t first = 0; first < n; first += kMaxTensors) {
        TileBatch B;
        std::memset(&B, 0, sizeof(B));
        uint32_t max_tb = 0, total = 0;
        B.n = 0;
        for (uint32_t i = first; i < n && B.n < (uint32_t)kMaxTensors; i++) {
            const hh_hctt_tensor &T = tensors[i];
            const uint32_t nt = (T.rows / 64) * (T.cols / 64);
            if (nt == 0) continue;
            const uint32_t j = B.n++;
            const uint32_t tb = (uint32_t)hh_hctt_tile_bytes(T.k);
            B.tiles[j] = T.d_tiles;
            B.out[j] = T.d_out;
            B.status[j] = T.d_tile_status;
            B.start[j] = total;
            B.tiles_per_row[j] = T.cols / 64;
            B.cols[j] = T.cols;
            B.k[j] = T.k;
            B.tb[j] = tb;
            B.dword_ok[j] = ((tb & 3u) == 0 && ((uintptr_t)T.d_tiles & 3u) == 0) ? 1u : 0u;
            total += nt;
            max_tb = tb > max_tb ? tb : max_tb;
        }
        if (B.n == 0) continue;
        B.start[B.n] = total;
        const uint32_t payb = (max_tb + 15u) & ~15u;
        B.wave_lds = payb + kScaleBytes + kCBytes;
        const uint32_t lds = B.wave_lds * kWaves;
        // one 4-wave workgroup per CU (1 wave per SIMD), persistent over tiles
        uint32_t grid = (uint32_t)(num_cus > 0 ? num_cus : 256);
        const uint32_t need = (total + kWaves - 1) / kWaves;
        if (grid > need) grid = need;
        const half8 *basis = reinterpret_cast<const half8 *>(d_basis);
        hipError_t e = hipSuccess;
#define HH_LAUNCH(DTV)                                                                  \
    do {                                                                                \
        e = hipFuncSetAttribute((const void *)hctt_decode_kernel<DTV>,                  \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);  \
        if (e != hipSuccess) return e;                                                  \
        hipLaunchKernelGGL(hctt_decode_kernel<DTV>, dim3(grid), dim3(kThreads), lds, s, \
                           B, basis);                                                   \
    } while (0)
        switch (dtype) {
            case HH_F32: HH_LAUNCH(HH_F32); break;
            case HH_F16: HH_LAUNCH(HH_F16); break;
            case HH_BF16: HH_LAUNCH(HH_BF16); break;
            default: return hipErrorInvalidValue;
        }
#undef HH_LAUNCH
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace hh
