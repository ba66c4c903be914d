// HCT3 whole-tensor spectral decode on the GPU: f16 (or f32) coefficients
// scattered by bitmap rank into the dense DCT coefficient matrix of the
// whole tensor, then the orthonormal 2-D inverse DCT of that matrix.
//
// Reference semantics:
//   coefficient reconstruction  crates/haagenti-cuda/src/decompress.rs:400-427
//       (each set bit, in ascending raster order, takes the fragment's next
//       value while values remain; later fragments overwrite earlier ones)
//   CompressiveSpectralDecoder  crates/haagenti/src/compressive.rs:728-752
//   idct_2d                     crates/haagenti-core/src/dct.rs:311-337
//       (orthonormal DCT-III along both axes; row-major, width contiguous)
//
// Scatter.  A block of 256 threads owns 256 64-bit bitmap words (16384
// coefficients).  Pass 1 counts set bits per block; one block scans the
// block counts; pass 2 recomputes the counts, scans them inside the block
// (giving each word the rank of its first set bit), then writes the block's
// 16384 outputs in coalesced order: output e is set when its bit is, and
// takes value number rank(e) = word rank + popcount(bits below e).
//
// Transform.  With B_n[k][i] = s_k cos(pi k (2i + 1) / 2n) (s_0 = sqrt(1/n),
// s_k = sqrt(2/n)), the inverse DCT of the h x w coefficient matrix C is
// X = B_h^T C B_w, computed as two fp32 GEMMs (rocBLAS): T = C B_w, then
// X = B_h^T T.  The forward DCT-II (dct_2d, dct.rs:282-308) is the
// transpose: C = B_h X B_w^T.  The basis matrices are generated on the GPU
// from an exact integer reduction of the cosine argument and cached per
// context.  fp32 GEMMs with K = n accumulate to ~1e-6 x RMS, against the
// 1e-3 x RMS bar of the tolerance-based IDCT parity.
//
// The inverse runs on the f16 MFMA instead (16x the fp32 MFMA rate): every
// operand is split into f16 hi + lo (x = hi + lo to ~2^-22 relative) and each
// product of two split operands is three f16 GEMMs with f32 accumulation
// (hi*hi + hi*lo + lo*hi; the dropped lo*lo is ~2^-22 relative).  C is first
// scaled by a power of two 2^e chosen from max|C| so that |C 2^e| and the
// intermediate T = B_w^T C 2^e stay below 2^14 (|T| <= max|C| sqrt(w)), far
// from f16 overflow; a last elementwise pass multiplies by 2^-e (exact).
// HH_DCT_F32=1 selects the fp32 GEMMs.
#include <cstdlib>

#include <rocblas/rocblas.h>

#include "hh_internal.hpp"

namespace hh {
namespace {

constexpr int kWordsPerBlock = 256;
constexpr uint64_t kElemsPerBlock = 64ull * kWordsPerBlock;

__device__ __forceinline__ uint64_t word_mask(uint64_t w, uint64_t nbits) {
    const uint64_t lo = 64ull * w;
    if (lo + 64 <= nbits) return ~0ull;
    if (lo >= nbits) return 0ull;
    return (1ull << (nbits - lo)) - 1ull;
}

// Exclusive sum over the 256 threads of the block (4 waves); *total gets the
// block total.  Uses s[0..3].
__device__ __forceinline__ uint32_t block_excl_sum(uint32_t v, uint32_t *s, uint32_t *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(incl, d);
        if (lane >= d) incl += t;
    }
    if (lane == 63) s[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t x = s[i];
        before += i < wave ? x : 0u;
        all += x;
    }
    *total = all;
    return before + incl - v;
}

__global__ __launch_bounds__(256) void hct3_count_kernel(const uint64_t *__restrict__ bits,
                                                         uint64_t nbits,
                                                         uint32_t *__restrict__ block_sums) {
    __shared__ uint32_t s[4];
    const uint64_t w = (uint64_t)blockIdx.x * kWordsPerBlock + threadIdx.x;
    const uint64_t m = word_mask(w, nbits);
    const uint32_t c = m ? (uint32_t)__popcll(bits[w] & m) : 0u;
    uint32_t total;
    block_excl_sum(c, s, &total);
    if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// In-place exclusive scan of n counts, one block of 1024 threads.
__global__ __launch_bounds__(1024) void scan_counts_kernel(uint32_t *__restrict__ d, uint32_t n) {
    __shared__ uint32_t s[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t carry = 0;
    for (uint32_t base = 0; base < n; base += 1024) {
        const uint32_t i = base + threadIdx.x;
        const uint32_t v = i < n ? d[i] : 0u;
        uint32_t incl = v;
#pragma unroll
        for (int k = 1; k < 64; k <<= 1) {
            const uint32_t t = __shfl_up(incl, k);
            if (lane >= k) incl += t;
        }
        if (lane == 63) s[wave] = incl;
        __syncthreads();
        uint32_t before = 0, all = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const uint32_t x = s[k];
            before += k < wave ? x : 0u;
            all += x;
        }
        if (i < n) d[i] = carry + before + incl - v;
        carry += all;
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void hct3_scatter_kernel(const uint64_t *__restrict__ bits,
                                                           uint64_t nbits,
                                                           const uint32_t *__restrict__ block_pref,
                                                           const void *__restrict__ coef,
                                                           uint32_t ncoef, int coef_f32,
                                                           float *__restrict__ dense, int first) {
    __shared__ uint64_t W[kWordsPerBlock];
    __shared__ uint32_t P[kWordsPerBlock];
    __shared__ uint32_t s[4];
    const uint64_t w0 = (uint64_t)blockIdx.x * kWordsPerBlock;
    const uint64_t w = w0 + threadIdx.x;
    const uint64_t m = word_mask(w, nbits);
    const uint64_t b = m ? bits[w] & m : 0ull;
    uint32_t total;
    const uint32_t excl = block_excl_sum((uint32_t)__popcll(b), s, &total);
    W[threadIdx.x] = b;
    P[threadIdx.x] = block_pref[blockIdx.x] + excl;
    __syncthreads();
    const uint64_t e0 = w0 * 64;
    // values are read bytewise: inside a fragment container they may sit
    // at any byte offset
    const uint8_t *cb = reinterpret_cast<const uint8_t *>(coef);
    for (uint32_t j = 0; j < 64; j++) {
        const uint32_t el = threadIdx.x + kWordsPerBlock * j;
        const uint64_t e = e0 + el;
        if (e >= nbits) break;
        const uint64_t bw = W[el >> 6];
        const uint32_t bit = el & 63u;
        float v = 0.0f;
        bool have = false;
        if ((bw >> bit) & 1ull) {
            const uint32_t r = P[el >> 6] + (uint32_t)__popcll(bw & ((1ull << bit) - 1ull));
            if (r < ncoef) {
                if (coef_f32) {
                    const uint8_t *q = cb + 4ull * r;
                    v = __uint_as_float((uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) |
                                        ((uint32_t)q[3] << 24));
                } else {
                    const uint8_t *q = cb + 2ull * r;
                    v = f16_bits_to_f32((uint32_t)q[0] | ((uint32_t)q[1] << 8));
                }
                have = true;
            }
        }
        if (first)
            dense[e] = v;
        else if (have)
            dense[e] = v;
    }
}

// B[k][i] = s_k cos(pi k (2i + 1) / 2n): the argument is reduced exactly in
// integers (k (2i + 1) mod 4n) before the double-precision cosine.
__global__ __launch_bounds__(256) void dct3_basis_kernel(float *__restrict__ B, uint32_t n) {
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)n * n) return;
    const uint32_t k = (uint32_t)(idx / n), i = (uint32_t)(idx % n);
    const uint64_t m = ((uint64_t)k * (2ull * i + 1ull)) % (4ull * n);
    const double sk = k == 0 ? sqrt(1.0 / (double)n) : sqrt(2.0 / (double)n);
    B[idx] = (float)(sk * cospi((double)m / (2.0 * (double)n)));
}

// 64-bit words of a bitmap held at any byte address (nbytes bytes; the last
// word is zero-padded).
__global__ __launch_bounds__(256) void pack_bits_kernel(const uint8_t *__restrict__ src, uint64_t nbytes,
                                                        uint64_t *__restrict__ words, uint64_t nwords) {
    const uint64_t w = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (w >= nwords) return;
    uint64_t v = 0;
    const uint64_t b0 = 8 * w;
#pragma unroll
    for (int i = 0; i < 8; i++)
        if (b0 + i < nbytes) v |= (uint64_t)src[b0 + i] << (8 * i);
    words[w] = v;
}

__global__ __launch_bounds__(256) void f32_convert_kernel(const float *__restrict__ x, uint64_t n,
                                                          int dtype, void *__restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    uint16_t *o = reinterpret_cast<uint16_t *>(out);
    o[i] = (uint16_t)(dtype == HH_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
}

uint32_t blocks_for(uint64_t n, uint32_t per) { return (uint32_t)((n + per - 1) / per); }

// Per-block max |x| over a grid-stride range.
__global__ __launch_bounds__(256) void amax_kernel(const float *__restrict__ x, uint64_t n,
                                                   float *__restrict__ partial) {
    __shared__ float sm[256];
    float m = 0.0f;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
        m = fmaxf(m, fabsf(x[i]));
    sm[threadIdx.x] = m;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) sm[threadIdx.x] = fmaxf(sm[threadIdx.x], sm[threadIdx.x + st]);
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = sm[0];
}

// consts = {0, 1, 2^e, 2^-e} with e the largest integer for which
// max|C| 2^e sqrt(w) <= 2^14 (e = 0 for an all-zero or non-finite C).
__global__ __launch_bounds__(256) void split_scale_kernel(const float *__restrict__ partial, uint32_t np,
                                                          uint32_t w, float *__restrict__ consts) {
    __shared__ float sm[256];
    float m = 0.0f;
    for (uint32_t i = threadIdx.x; i < np; i += 256) m = fmaxf(m, partial[i]);
    sm[threadIdx.x] = m;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) sm[threadIdx.x] = fmaxf(sm[threadIdx.x], sm[threadIdx.x + st]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float mx = sm[0];
        int e = 0;
        if (mx > 0.0f && isfinite(mx)) {
            int q;
            frexpf(16384.0f / (mx * sqrtf((float)w)), &q);  // 2^(q-1) <= ratio < 2^q
            e = q - 1;
            e = e < -120 ? -120 : e > 120 ? 120 : e;
        }
        consts[0] = 0.0f;
        consts[1] = 1.0f;
        consts[2] = ldexpf(1.0f, e);
        consts[3] = ldexpf(1.0f, -e);
    }
}

// hi = f16(x s), lo = f16(x s - hi) (round to nearest even; x s - hi is
// exact in f32); s = *scale, or 1 without one.
__global__ __launch_bounds__(256) void split_f16_kernel(const float *__restrict__ x, uint64_t n,
                                                        const float *__restrict__ scale,
                                                        _Float16 *__restrict__ hi, _Float16 *__restrict__ lo) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = scale ? x[i] * scale[0] : x[i];
    const _Float16 h = (_Float16)v;
    hi[i] = h;
    lo[i] = (_Float16)(v - (float)h);
}

// x *= *scale, in place
__global__ __launch_bounds__(256) void scale_kernel(float *__restrict__ x, uint64_t n, const float *__restrict__ scale) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] *= scale[0];
}

// out = 16-bit RNE of x * *scale (the scale is a power of two: exact)
__global__ __launch_bounds__(256) void scale_convert_kernel(const float *__restrict__ x, uint64_t n,
                                                            const float *__restrict__ scale, int dtype,
                                                            void *__restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = x[i] * scale[0];
    uint16_t *o = reinterpret_cast<uint16_t *>(out);
    o[i] = (uint16_t)(dtype == HH_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
}

}  // namespace

hipError_t launch_hct3_scatter(const uint64_t *d_bits, uint64_t nbits, uint32_t *d_block_sums,
                               const void *d_coef, uint32_t ncoef, int coef_f32, float *d_dense,
                               int first, hipStream_t s) {
    if (nbits == 0) return hipSuccess;
    const uint32_t nwords = blocks_for(nbits, 64);
    const uint32_t nblk = blocks_for(nwords, kWordsPerBlock);
    hipLaunchKernelGGL(hct3_count_kernel, dim3(nblk), dim3(256), 0, s, d_bits, nbits, d_block_sums);
    hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(1024), 0, s, d_block_sums, nblk);
    hipLaunchKernelGGL(hct3_scatter_kernel, dim3(nblk), dim3(256), 0, s, d_bits, nbits, d_block_sums,
                       d_coef, ncoef, coef_f32, d_dense, first);
    return hipGetLastError();
}

hipError_t launch_pack_bits(const uint8_t *d_src, uint64_t nbytes, uint64_t *d_words, hipStream_t s) {
    const uint64_t nwords = (nbytes + 7) / 8;
    if (nwords == 0) return hipSuccess;
    hipLaunchKernelGGL(pack_bits_kernel, dim3(blocks_for(nwords, 256)), dim3(256), 0, s, d_src, nbytes, d_words,
                       nwords);
    return hipGetLastError();
}

size_t hct3_block_sums_bytes(uint64_t nbits) {
    return 4ull * blocks_for(blocks_for(nbits, 64), kWordsPerBlock);
}

hipError_t launch_f32_convert(const float *d_x, uint64_t n, int dtype, void *d_out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(f32_convert_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, d_x, n, dtype, d_out);
    return hipGetLastError();
}

// The context's cached basis B_n (two sizes are kept; the older is replaced).
static int32_t basis_for(hh_context *ctx, uint32_t n, hipStream_t s, const float **out) {
    for (int i = 0; i < 2; i++)
        if (ctx->dct_basis[i].d && ctx->dct_basis[i].n == n) {
            ctx->dct_basis[i].stamp = ++ctx->dct_stamp;
            *out = ctx->dct_basis[i].d;
            return HH_OK;
        }
    const int v = !ctx->dct_basis[0].d ? 0 : !ctx->dct_basis[1].d ? 1
                  : ctx->dct_basis[0].stamp <= ctx->dct_basis[1].stamp ? 0 : 1;
    hh_context::Basis &b = ctx->dct_basis[v];
    if (b.d) {
        hipError_t e = hipFree(b.d);
        if (b.hl && e == hipSuccess) e = hipFree(b.hl);
        b.d = nullptr;
        b.hl = nullptr;
        b.n = 0;
        if (e != hipSuccess) return from_hip(e);
    }
    hipError_t e = hipMalloc(&b.d, (size_t)n * n * sizeof(float));
    if (e != hipSuccess) {
        b.d = nullptr;
        return from_hip(e);
    }
    b.n = n;
    b.stamp = ++ctx->dct_stamp;
    hipLaunchKernelGGL(dct3_basis_kernel, dim3(blocks_for((uint64_t)n * n, 256)), dim3(256), 0, s, b.d, n);
    e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e);
    *out = b.d;
    return HH_OK;
}

// The f16 hi / lo halves of the cached basis B_n (made on first use).
static int32_t basis_split_for(hh_context *ctx, uint32_t n, const float *bd, hipStream_t s, const _Float16 **hi,
                               const _Float16 **lo) {
    for (int i = 0; i < 2; i++) {
        hh_context::Basis &b = ctx->dct_basis[i];
        if (b.d != bd) continue;
        const uint64_t nn = (uint64_t)n * n;
        if (!b.hl) {
            hipError_t e = hipMalloc(&b.hl, 2 * nn * sizeof(uint16_t));
            if (e != hipSuccess) {
                b.hl = nullptr;
                return from_hip(e);
            }
            _Float16 *h = reinterpret_cast<_Float16 *>(b.hl);
            hipLaunchKernelGGL(split_f16_kernel, dim3(blocks_for(nn, 256)), dim3(256), 0, s, b.d, nn,
                               (const float *)nullptr, h, h + nn);
            e = hipGetLastError();
            if (e != hipSuccess) return from_hip(e);
        }
        *hi = reinterpret_cast<const _Float16 *>(b.hl);
        *lo = *hi + nn;
        return HH_OK;
    }
    return HH_ERR_INVALID_ARGUMENT;
}

static int32_t blas_for(hh_context *ctx, hipStream_t s, rocblas_handle *h) {
    if (!ctx->blas) {
        rocblas_handle nh = nullptr;
        if (rocblas_create_handle(&nh) != rocblas_status_success) return HH_ERR_DEVICE;
        ctx->blas = nh;
    }
    *h = reinterpret_cast<rocblas_handle>(ctx->blas);
    return rocblas_set_stream(*h, s) == rocblas_status_success ? HH_OK : HH_ERR_DEVICE;
}

static int32_t blas_status(rocblas_status st) {
    switch (st) {
        case rocblas_status_success: return HH_OK;
        case rocblas_status_memory_error: return HH_ERR_OUT_OF_MEMORY;
        case rocblas_status_invalid_size:
        case rocblas_status_invalid_pointer:
        case rocblas_status_invalid_value: return HH_ERR_INVALID_ARGUMENT;
        default: return HH_ERR_KERNEL_LAUNCH;
    }
}

// X = B_h^T C B_w on the f16 MFMA (see the header): d_tmp holds T in f32.
static int32_t idct_split(hh_context *ctx, rocblas_handle h, const float *d_in, float *d_tmp, float *d_out,
                          uint32_t rows, uint32_t cols, const float *bw, const float *bh, hipStream_t s,
                          bool f16_exact, int32_t cvt_dtype, void *cvt_out) {
    const uint64_t total = (uint64_t)rows * cols;
    const _Float16 *bw_hi, *bw_lo, *bh_hi, *bh_lo;
    int32_t rc = basis_split_for(ctx, cols, bw, s, &bw_hi, &bw_lo);
    if (rc != HH_OK) return rc;
    rc = basis_split_for(ctx, rows, bh, s, &bh_hi, &bh_lo);
    if (rc != HH_OK) return rc;
    // split scratch: hi and lo operand halves, block maxima, constants
    const uint32_t np = 1024;
    const size_t need = 2 * total * sizeof(uint16_t) + (np + 4) * sizeof(float) + 256;
    if (ctx->split_bytes < need) {
        if (ctx->d_split) {
            hipError_t e = hipFree(ctx->d_split);
            ctx->d_split = nullptr;
            ctx->split_bytes = 0;
            if (e != hipSuccess) return from_hip(e);
        }
        hipError_t e = hipMalloc(&ctx->d_split, need);
        if (e != hipSuccess) {
            ctx->d_split = nullptr;
            return from_hip(e);
        }
        ctx->split_bytes = need;
    }
    _Float16 *ohi = reinterpret_cast<_Float16 *>(ctx->d_split);
    _Float16 *olo = ohi + total;
    float *partial = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(ctx->d_split) +
                                               ((2 * total * sizeof(uint16_t) + 255) & ~(size_t)255));
    float *consts = partial + np;
    hipLaunchKernelGGL(amax_kernel, dim3(np), dim3(256), 0, s, d_in, total, partial);
    hipLaunchKernelGGL(split_scale_kernel, dim3(1), dim3(256), 0, s, partial, np, cols, consts);
    hipLaunchKernelGGL(split_f16_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, d_in, total,
                       (const float *)(consts + 2), ohi, olo);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e);
    const int m = (int)cols, n = (int)rows;
    // host scalars (rocBLAS reads device scalars back to the host per call);
    // 2^-e is applied by a last elementwise pass
    const float c0 = 0.0f, c1 = 1.0f;
    const float *k0 = &c0, *k1 = &c1;
    const rocblas_datatype f16 = rocblas_datatype_f16_r, f32 = rocblas_datatype_f32_r;
    auto gemm = [&](rocblas_operation ta, rocblas_operation tb, int k, const float *alpha, const void *a, int lda,
                    const void *b, int ldb, const float *beta, float *c) {
        return rocblas_gemm_ex(h, ta, tb, m, n, k, alpha, a, f16, lda, b, f16, ldb, beta, c, f32, m, c, f32, m, f32,
                               rocblas_gemm_algo_standard, 0, 0);
    };
    const rocblas_operation N = rocblas_operation_none, T = rocblas_operation_transpose;
    // T^T = B_w^T (C 2^e)^T, three passes (column-major views as below)
    rocblas_status st = gemm(N, N, m, k1, bw_hi, m, ohi, m, k0, d_tmp);
    if (st == rocblas_status_success) st = gemm(N, N, m, k1, bw_lo, m, ohi, m, k1, d_tmp);
    // (an input of f16 values scaled by 2^e has no low half)
    if (st == rocblas_status_success && !f16_exact) st = gemm(N, N, m, k1, bw_hi, m, olo, m, k1, d_tmp);
    if (st == rocblas_status_success) {
        hipLaunchKernelGGL(split_f16_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, d_tmp, total,
                           (const float *)nullptr, ohi, olo);
        if (hipGetLastError() != hipSuccess) st = rocblas_status_internal_error;
    }
    // X^T 2^e = T^T B_h, three passes; then X = 2^-e (X 2^e)
    if (st == rocblas_status_success) st = gemm(N, T, n, k1, ohi, m, bh_hi, n, k0, d_out);
    if (st == rocblas_status_success) st = gemm(N, T, n, k1, ohi, m, bh_lo, n, k1, d_out);
    if (st == rocblas_status_success) st = gemm(N, T, n, k1, olo, m, bh_hi, n, k1, d_out);
    if (st != rocblas_status_success) return blas_status(st);
    if (cvt_out)
        hipLaunchKernelGGL(scale_convert_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, d_out, total,
                           (const float *)(consts + 3), (int)cvt_dtype, cvt_out);
    else
        hipLaunchKernelGGL(scale_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, d_out, total,
                           (const float *)(consts + 3));
    return from_hip(hipGetLastError());
}

int32_t dct2d_full(hh_context *ctx, bool inverse, const float *d_in, float *d_tmp, float *d_out,
                   uint32_t rows, uint32_t cols, hipStream_t s, bool f16_exact, int32_t cvt_dtype,
                   void *cvt_out, bool *converted) {
    if (converted) *converted = false;
    if (rows == 0 || cols == 0) return HH_OK;
    const float *bw = nullptr, *bh = nullptr;
    int32_t rc = basis_for(ctx, cols, s, &bw);
    if (rc != HH_OK) return rc;
    rc = basis_for(ctx, rows, s, &bh);
    if (rc != HH_OK) return rc;
    if (rows == cols) bw = bh;  // one cache slot serves both
    rocblas_handle h;
    rc = blas_for(ctx, s, &h);
    if (rc != HH_OK) return rc;
    const float one = 1.0f, zero = 0.0f;
    // Column-major views: a row-major h x w matrix M is the w x h matrix
    // M^T with leading dimension w; a row-major basis B_n is B_n^T.
    //   inverse:  T^T = B_w^T C^T     (m = w, n = h, k = w)
    //             X^T = T^T B_h       (m = w, n = h, k = h)
    //   forward:  T^T = B_w X^T       (m = w, n = h, k = w)
    //             C^T = T^T B_h^T     (m = w, n = h, k = h)
    const int m = (int)cols, n = (int)rows;
    const char *f32env = std::getenv("HH_DCT_F32");
    if (inverse && !(f32env && f32env[0] == '1')) {
        if (converted) *converted = cvt_out != nullptr;
        return idct_split(ctx, h, d_in, d_tmp, d_out, rows, cols, bw, bh, s, f16_exact, cvt_dtype, cvt_out);
    }
    rocblas_status st = rocblas_sgemm(h, inverse ? rocblas_operation_none : rocblas_operation_transpose,
                                      rocblas_operation_none, m, n, m, &one, bw, m, d_in, m, &zero,
                                      d_tmp, m);
    if (st != rocblas_status_success) return blas_status(st);
    st = rocblas_sgemm(h, rocblas_operation_none, inverse ? rocblas_operation_transpose : rocblas_operation_none,
                       m, n, n, &one, d_tmp, m, bh, n, &zero, d_out, m);
    return blas_status(st);
}

void release_dct_resources(hh_context *ctx) {
    for (int i = 0; i < 2; i++) {
        if (ctx->dct_basis[i].d) hipFree(ctx->dct_basis[i].d);
        if (ctx->dct_basis[i].hl) hipFree(ctx->dct_basis[i].hl);
        ctx->dct_basis[i].d = nullptr;
        ctx->dct_basis[i].hl = nullptr;
        ctx->dct_basis[i].n = 0;
    }
    if (ctx->d_split) hipFree(ctx->d_split);
    ctx->d_split = nullptr;
    ctx->split_bytes = 0;
    if (ctx->blas) rocblas_destroy_handle(reinterpret_cast<rocblas_handle>(ctx->blas));
    ctx->blas = nullptr;
}

}  // namespace hh
