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
        b.d = nullptr;
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

int32_t dct2d_full(hh_context *ctx, bool inverse, const float *d_in, float *d_tmp, float *d_out,
                   uint32_t rows, uint32_t cols, hipStream_t s) {
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
        ctx->dct_basis[i].d = nullptr;
        ctx->dct_basis[i].n = 0;
    }
    if (ctx->blas) rocblas_destroy_handle(reinterpret_cast<rocblas_handle>(ctx->blas));
    ctx->blas = nullptr;
}

}  // namespace hh
