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
// X = B_h^T C B_w and the forward DCT-II (dct_2d, dct.rs:282-308) is
// C = B_h X B_w^T; each is two split-f16 MFMA products (dct_gemm.hip)
// against basis planes generated on the GPU from an exact integer reduction
// of the cosine argument and cached per context.  The input is first scaled
// by a power of two 2^e chosen from max |input| (the amax and scale kernels
// below) so that every f16 operand stays far from overflow; the last
// product multiplies by 2^-e (exact).  Error ~1e-6 x RMS, against the
// 1e-3 x RMS bar of the tolerance-based IDCT parity.
#include "hh_internal.hpp"

namespace hh {
namespace {

constexpr int kWordsPerBlock = 256;

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
    const uint8_t *cb = reinterpret_cast<const uint8_t *>(coef);
    if (!coef_f32 && ((uintptr_t)coef & 1u) == 0 && ncoef > 0) {
        // 2-byte aligned f16 values: eight elements' values loaded together
        // (an element without a value loads value 0 and discards it)
        const uint16_t *hv16 = reinterpret_cast<const uint16_t *>(coef);
        for (uint32_t j0 = 0; j0 < 64; j0 += 8) {
            uint32_t x[8];
            bool hv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t el = threadIdx.x + kWordsPerBlock * (j0 + k);
                const uint64_t bw = W[el >> 6];
                const uint32_t bit = el & 63u;
                const uint32_t rk = P[el >> 6] + (uint32_t)__popcll(bw & ((1ull << bit) - 1ull));
                hv[k] = ((bw >> bit) & 1ull) && rk < ncoef;  // bits past nbits are clear
                x[k] = hv16[hv[k] ? rk : 0u];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint64_t e = e0 + threadIdx.x + kWordsPerBlock * (j0 + k);
                if (e < nbits && (first || hv[k])) dense[e] = hv[k] ? f16_bits_to_f32(x[k]) : 0.0f;
            }
        }
        return;
    }
    // values read bytewise: inside a fragment container they may sit at any
    // byte offset
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

// hct3_scatter_kernel's output written as the first product's operand
// plane of the even / odd split inverse DCT (dct2d_eo): element (r, c) of
// the h x w matrix, times scale[0] (a power of two), as f16 at r w + c / 2
// for even c and r w + w / 2 + c / 2 for odd c.  The values are f16, so the
// plane holds them exactly (barring f16 range limits at the scale chosen).
__global__ __launch_bounds__(256) void hct3_scatter_plane_kernel(const uint64_t *__restrict__ bits,
                                                                 uint64_t nbits,
                                                                 const uint32_t *__restrict__ block_pref,
                                                                 const uint8_t *__restrict__ coef, uint32_t ncoef,
                                                                 uint32_t w, const float *__restrict__ scale,
                                                                 _Float16 *__restrict__ plane, int first) {
    __shared__ uint64_t W[kWordsPerBlock];
    __shared__ uint32_t P[kWordsPerBlock];
    __shared__ uint32_t s[4];
    const uint64_t w0 = (uint64_t)blockIdx.x * kWordsPerBlock;
    const uint64_t wd = w0 + threadIdx.x;
    const uint64_t m = word_mask(wd, nbits);
    const uint64_t b = m ? bits[wd] & m : 0ull;
    uint32_t total;
    const uint32_t excl = block_excl_sum((uint32_t)__popcll(b), s, &total);
    W[threadIdx.x] = b;
    P[threadIdx.x] = block_pref[blockIdx.x] + excl;
    __syncthreads();
    const float sc = *scale;
    const uint32_t half = w / 2;
    const uint64_t e0 = w0 * 64 + threadIdx.x;
    // this thread's first element as (row, column); each step advances 256
    // columns (w >= 512: at most one row wrap per step)
    uint64_t r = e0 / w;
    uint32_t c = (uint32_t)(e0 - r * w);
    if (((uintptr_t)coef & 1u) == 0 && ncoef > 0) {
        // 2-byte aligned values: eight elements' values loaded together
        // (an element without a value loads value 0 and discards it)
        const uint16_t *h = reinterpret_cast<const uint16_t *>(coef);
        for (uint32_t j0 = 0; j0 < 64; j0 += 8) {
            uint32_t x[8];
            bool hv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t el = threadIdx.x + kWordsPerBlock * (j0 + k);
                const uint64_t bw = W[el >> 6];
                const uint32_t bit = el & 63u;
                const uint32_t rk = P[el >> 6] + (uint32_t)__popcll(bw & ((1ull << bit) - 1ull));
                hv[k] = ((bw >> bit) & 1ull) && rk < ncoef;  // bits past nbits are clear
                x[k] = h[hv[k] ? rk : 0u];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint64_t e = w0 * 64 + threadIdx.x + kWordsPerBlock * (j0 + k);
                if (e < nbits && (first || hv[k])) {
                    const _Float16 v = hv[k] ? (_Float16)(f16_bits_to_f32(x[k]) * sc) : (_Float16)0.0f;
                    plane[r * w + ((c & 1u) ? half + (c >> 1) : (c >> 1))] = v;
                }
                c += kWordsPerBlock;
                if (c >= w) {
                    c -= w;
                    r++;
                }
            }
        }
        return;
    }
    for (uint32_t j = 0; j < 64; j++) {
        const uint32_t el = threadIdx.x + kWordsPerBlock * j;
        const uint64_t e = w0 * 64 + el;
        if (e >= nbits) break;
        const uint64_t bw = W[el >> 6];
        const uint32_t bit = el & 63u;
        bool have = false;
        _Float16 v = (_Float16)0.0f;
        if ((bw >> bit) & 1ull) {
            const uint32_t rk = P[el >> 6] + (uint32_t)__popcll(bw & ((1ull << bit) - 1ull));
            if (rk < ncoef) {
                const uint8_t *q = coef + 2ull * rk;
                v = (_Float16)(f16_bits_to_f32((uint32_t)q[0] | ((uint32_t)q[1] << 8)) * sc);
                have = true;
            }
        }
        const uint64_t o = r * w + ((c & 1u) ? half + (c >> 1) : (c >> 1));
        if (first || have) plane[o] = v;
        c += kWordsPerBlock;
        if (c >= w) {
            c -= w;
            r++;
        }
    }
}

// Per-block max |v| of n f16 values at any byte address (a grid-stride
// range per block) into partial[blockIdx.x]; 16-bit loads when the values
// are 2-byte aligned, bytes otherwise.
__global__ __launch_bounds__(256) void amax_f16_kernel(const uint8_t *__restrict__ v, uint32_t n,
                                                       float *__restrict__ partial) {
    __shared__ float sm[256];
    float mx = 0.0f;
    if (((uintptr_t)v & 1u) == 0) {
        // eight independent loads in flight per thread
        const uint16_t *h = reinterpret_cast<const uint16_t *>(v);
        const uint32_t st = gridDim.x * 256;
        uint32_t i = blockIdx.x * 256 + threadIdx.x;
        for (; (uint64_t)i + 7ull * st < n; i += 8 * st) {
            uint32_t x[8];
#pragma unroll
            for (int k = 0; k < 8; k++) x[k] = h[i + k * st];
#pragma unroll
            for (int k = 0; k < 8; k++) mx = fmaxf(mx, fabsf(f16_bits_to_f32(x[k])));
        }
        for (; i < n; i += st) mx = fmaxf(mx, fabsf(f16_bits_to_f32(h[i])));
    } else {
        for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
            mx = fmaxf(mx, fabsf(f16_bits_to_f32((uint32_t)v[2ull * i] | ((uint32_t)v[2ull * i + 1] << 8))));
    }
    sm[threadIdx.x] = mx;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) sm[threadIdx.x] = fmaxf(sm[threadIdx.x], sm[threadIdx.x + st]);
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = sm[0];
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

hipError_t launch_scan_counts(uint32_t *d, uint32_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(1024), 0, s, d, n);
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

// The context's cached basis planes: kind 0 B_n, 1 B_n^T, 2 the even / odd
// split of B_n^T; two are kept, the older is replaced.
static int32_t planes_for(hh_context *ctx, uint32_t n, int kind, hipStream_t s, const uint16_t **hi,
                          const uint16_t **lo) {
    const uint64_t plane = kind == 2 ? (uint64_t)n * (n / 2) : (uint64_t)dct_planes_rows(n) * dct_planes_cols(n);
    for (int i = 0; i < 2; i++) {
        hh_context::Basis &b = ctx->dct_basis[i];
        if (b.hl && b.n == n && b.kind == kind) {
            b.stamp = ++ctx->dct_stamp;
            *hi = b.hl;
            *lo = b.hl + plane;
            return HH_OK;
        }
    }
    const int v = !ctx->dct_basis[0].hl ? 0 : !ctx->dct_basis[1].hl ? 1
                  : ctx->dct_basis[0].stamp <= ctx->dct_basis[1].stamp ? 0 : 1;
    hh_context::Basis &b = ctx->dct_basis[v];
    if (b.hl) {
        // the stream may still read the old planes: wait before freeing
        hipError_t e = hipStreamSynchronize(s);
        if (e == hipSuccess) e = hipFree(b.hl);
        b.hl = nullptr;
        b.n = 0;
        if (e != hipSuccess) return from_hip(e);
    }
    hipError_t e = hipMalloc(&b.hl, 2 * plane * sizeof(uint16_t));
    if (e != hipSuccess) {
        b.hl = nullptr;
        return from_hip(e);
    }
    b.n = n;
    b.kind = kind;
    b.stamp = ++ctx->dct_stamp;
    e = kind == 2 ? launch_dct_basis_split_planes(b.hl, b.hl + plane, n, s)
                  : launch_dct_basis_planes(b.hl, b.hl + plane, n, kind == 1, s);
    if (e != hipSuccess) return from_hip(e);
    *hi = b.hl;
    *lo = b.hl + plane;
    return HH_OK;
}

// The context's transform scratch, at least `need` bytes.
static int32_t split_scratch(hh_context *ctx, size_t need, hipStream_t s) {
    if (ctx->split_bytes >= need) return HH_OK;
    if (ctx->d_split) {
        hipError_t e = hipStreamSynchronize(s);
        if (e == hipSuccess) e = hipFree(ctx->d_split);
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
    return HH_OK;
}

// Inverse 2-D DCT of an h x w matrix (both multiples of 512) on the even /
// odd split of the cosine bases: B_n[k][n - 1 - i] = (-1)^k B_n[k][i], so
// row i < n/2 of B_n^T X is E_i + O_i and row n - 1 - i is E_i - O_i, with
// E over the even frequencies and O over the odd ones -- two products of
// half the depth in one launch (the stacked split basis against the input's
// planes with their columns in even / odd order), then a butterfly pass.
//   P  = butterfly(split(B_w)^T (C 2^e)^T)     (w x h, as even / odd planes)
//   X  = 2^-e butterfly(split(B_h)^T P^T)      (h x w)
// dct2d_eo's scratch: block maxima, the constants {0, 1, 2^e, 2^-e}, the
// input's planes, the stacked E / O products (f32), the intermediate's
// planes; and the basis planes.
struct EoScratch {
    float *partial, *consts;
    uint16_t *in_hi, *in_lo, *mid_hi, *mid_lo;
    float *y;
    const uint16_t *wh, *wl, *hh, *hl;
};
constexpr uint32_t kEoPartials = 4096;  // block maxima: 256 per fragment in hct3_decode_eo

static int32_t eo_scratch(hh_context *ctx, uint32_t h, uint32_t w, bool f16_exact, hipStream_t s, EoScratch &S) {
    int32_t rc = planes_for(ctx, w, 2, s, &S.wh, &S.wl);
    if (rc != HH_OK) return rc;
    rc = planes_for(ctx, h, 2, s, &S.hh, &S.hl);
    if (rc != HH_OK) return rc;
    if (h == w) {  // the second lookup may have replaced the first's slot
        S.wh = S.hh;
        S.wl = S.hl;
    }
    const uint64_t total = (uint64_t)h * w;
    const size_t off_in = ((kEoPartials + 4) * sizeof(float) + 255) & ~(size_t)255;
    const size_t off_y = off_in + ((total * (f16_exact ? 2 : 4) + 255) & ~(uint64_t)255);
    const size_t off_mid = off_y + total * 4;
    rc = split_scratch(ctx, off_mid + total * 4, s);
    if (rc != HH_OK) return rc;
    uint8_t *sp = reinterpret_cast<uint8_t *>(ctx->d_split);
    S.partial = reinterpret_cast<float *>(sp);
    S.consts = S.partial + kEoPartials;
    S.in_hi = reinterpret_cast<uint16_t *>(sp + off_in);
    S.in_lo = f16_exact ? nullptr : S.in_hi + total;
    S.y = reinterpret_cast<float *>(sp + off_y);
    S.mid_hi = reinterpret_cast<uint16_t *>(sp + off_mid);
    S.mid_lo = S.mid_hi + total;
    return HH_OK;
}

// The two half-depth products and butterflies of dct2d_eo, from the input's
// planes (C 2^e in even / odd column order) and the constants in S.
static int32_t eo_products(const EoScratch &S, float *d_out, uint32_t h, uint32_t w, hipStream_t s,
                           int32_t cvt_dtype, void *cvt_out, bool *converted) {
    DctGemm g1;
    g1.a_hi = S.wh;
    g1.a_lo = S.wl;
    g1.b_hi = S.in_hi;
    g1.b_lo = S.in_lo;
    g1.out_scale = nullptr;
    g1.d = S.y;
    g1.ldd = h;
    g1.d_dtype = HH_F32;
    g1.d_planes = false;
    g1.M = w;
    g1.N = h;
    g1.K = w / 2;
    g1.lda = w / 2;
    g1.ldb = w;
    g1.m_split = w / 2;
    g1.b_koff = w / 2;
    hipError_t e = launch_dct_gemm(g1, s);
    if (e == hipSuccess) e = launch_dct_butterfly(S.y, w / 2, h, true, nullptr, HH_F32, S.mid_hi, 0, s);
    if (e != hipSuccess) return from_hip(e);
    DctGemm g2;
    g2.a_hi = S.hh;
    g2.a_lo = S.hl;
    g2.b_hi = S.mid_hi;
    g2.b_lo = S.mid_lo;
    g2.out_scale = nullptr;
    g2.d = S.y;
    g2.ldd = w;
    g2.d_dtype = HH_F32;
    g2.d_planes = false;
    g2.M = h;
    g2.N = w;
    g2.K = h / 2;
    g2.lda = h / 2;
    g2.ldb = h;
    g2.m_split = h / 2;
    g2.b_koff = h / 2;
    e = launch_dct_gemm(g2, s);
    const bool cvt = cvt_out != nullptr;
    if (e == hipSuccess)
        e = launch_dct_butterfly(S.y, h / 2, w, false, S.consts + 3, cvt ? cvt_dtype : HH_F32,
                                 cvt ? cvt_out : d_out, w, s);
    if (e != hipSuccess) return from_hip(e);
    if (converted) *converted = cvt;
    return HH_OK;
}

static int32_t dct2d_eo(hh_context *ctx, const float *d_in, float *d_out, uint32_t h, uint32_t w, hipStream_t s,
                        bool f16_exact, int32_t cvt_dtype, void *cvt_out, bool *converted) {
    EoScratch S;
    int32_t rc = eo_scratch(ctx, h, w, f16_exact, s, S);
    if (rc != HH_OK) return rc;
    const uint64_t total = (uint64_t)h * w;
    hipLaunchKernelGGL(amax_kernel, dim3(kEoPartials), dim3(256), 0, s, d_in, total, S.partial);
    hipLaunchKernelGGL(split_scale_kernel, dim3(1), dim3(256), 0, s, S.partial, kEoPartials, w, S.consts);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e);
    e = launch_operand_planes_eo(d_in, h, w, w, S.consts + 2, S.in_hi, S.in_lo, s);
    if (e != hipSuccess) return from_hip(e);
    return eo_products(S, d_out, h, w, s, cvt_dtype, cvt_out, converted);
}

int32_t hct3_decode_eo(hh_context *ctx, const Hct3Frag *frags, uint32_t nfrags, uint32_t h, uint32_t w,
                       int32_t dtype, void *d_out, uint8_t *d_stage, hipStream_t s) {
    const uintptr_t out_addr = (uintptr_t)d_out;
    if (h % 512u || w % 512u || nfrags == 0 || nfrags > kEoPartials / 256u ||
        (out_addr & (dtype == HH_F32 ? 15u : 7u)))
        return HH_ERR_UNSUPPORTED;
    const uint64_t total = (uint64_t)h * w;
    const uint32_t nwords = blocks_for(total, 64);
    const uint32_t nblk = blocks_for(nwords, kWordsPerBlock);
    uint32_t *d_sums = reinterpret_cast<uint32_t *>(d_stage);
    uint64_t *d_bits = reinterpret_cast<uint64_t *>(d_stage + ((hct3_block_sums_bytes(total) + 15u) & ~(size_t)15));
    if (use_fft(ctx, h, w)) {
        // the fragments scattered into the first row pass in LDS, or where
        // its limits do not allow that into an f32 matrix, then the FFT route
        int32_t rc = hct3_decode_fft(ctx, frags, nfrags, h, w, dtype, d_out, s);
        if (rc != HH_ERR_UNSUPPORTED) return rc;
        float *a, *b;
        rc = fft_scratch(ctx, total, s, &a, &b);
        if (rc != HH_OK) return rc;
        for (uint32_t i = 0; i < nfrags; i++) {
            hipError_t e = launch_pack_bits(frags[i].bitmap, (total + 7) / 8, d_bits, s);
            if (e == hipSuccess)
                e = launch_hct3_scatter(d_bits, total, d_sums, frags[i].coef, frags[i].ncoef, 0, a, i == 0 ? 1 : 0,
                                        s);
            if (e != hipSuccess) return from_hip(e);
        }
        return dct2d_fft(ctx, true, a, a, b, h, w, dtype, d_out, s);
    }
    EoScratch S;
    int32_t rc = eo_scratch(ctx, h, w, true, s, S);
    if (rc != HH_OK) return rc;
    // the scale from the largest coefficient of any fragment (at least the
    // largest of the matrix the fragments make)
    for (uint32_t i = 0; i < nfrags; i++)
        hipLaunchKernelGGL(amax_f16_kernel, dim3(256), dim3(256), 0, s, frags[i].coef, frags[i].ncoef,
                           S.partial + 256u * i);
    hipLaunchKernelGGL(split_scale_kernel, dim3(1), dim3(256), 0, s, S.partial, 256u * nfrags, w, S.consts);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e);
    for (uint32_t i = 0; i < nfrags; i++) {
        e = launch_pack_bits(frags[i].bitmap, (total + 7) / 8, d_bits, s);
        if (e != hipSuccess) return from_hip(e);
        hipLaunchKernelGGL(hct3_count_kernel, dim3(nblk), dim3(256), 0, s, d_bits, total, d_sums);
        hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(1024), 0, s, d_sums, nblk);
        hipLaunchKernelGGL(hct3_scatter_plane_kernel, dim3(nblk), dim3(256), 0, s, d_bits, total, d_sums,
                           frags[i].coef, frags[i].ncoef, w, S.consts + 2,
                           reinterpret_cast<_Float16 *>(S.in_hi), i == 0 ? 1 : 0);
        e = hipGetLastError();
        if (e != hipSuccess) return from_hip(e);
    }
    return eo_products(S, reinterpret_cast<float *>(d_out), h, w, s, dtype == HH_F32 ? HH_F32 : dtype,
                       dtype == HH_F32 ? nullptr : d_out, nullptr);
}

int32_t dct2d_full(hh_context *ctx, bool inverse, const float *d_in, float *d_tmp, float *d_out,
                   uint32_t rows, uint32_t cols, hipStream_t s, bool f16_exact, int32_t cvt_dtype,
                   void *cvt_out, bool *converted) {
    if (converted) *converted = false;
    if (rows == 0 || cols == 0) return HH_OK;
    const uint32_t h = rows, w = cols;
    const uint64_t total = (uint64_t)h * w;
    if (use_fft(ctx, h, w)) {
        const bool cvt = inverse && cvt_out != nullptr;
        void *out = cvt ? cvt_out : static_cast<void *>(d_out);
        const int32_t dt = cvt ? cvt_dtype : HH_F32;
        if ((reinterpret_cast<uintptr_t>(out) & (dt == HH_F32 ? 15u : 7u)) == 0 &&
            (inverse || (reinterpret_cast<uintptr_t>(d_in) & 15u) == 0)) {
            float *a, *b;
            int32_t rc = fft_scratch(ctx, total, s, &a, &b);
            if (rc == HH_OK) rc = dct2d_fft(ctx, inverse, d_in, a, b, h, w, dt, out, s);
            if (rc == HH_OK && converted) *converted = cvt;
            return rc;
        }
    }
    // the inverse needs B^T planes, the forward B planes; a square matrix
    // uses one set for both products
    // the inverse of a matrix whose sides are multiples of 512 runs on the
    // even / odd split of the bases (half the MFMA work, see dct2d_eo)
    // (its last pass stores four outputs at a time: 16-byte aligned f32 or
    // 8-byte aligned 16-bit outputs)
    const uintptr_t out_addr = (uintptr_t)(inverse && cvt_out != nullptr ? cvt_out : (void *)d_out);
    const bool out_aligned = (out_addr & (inverse && cvt_out != nullptr ? 7u : 15u)) == 0;
    if (inverse && h % 512u == 0 && w % 512u == 0 && out_aligned)
        return dct2d_eo(ctx, d_in, d_out, h, w, s, f16_exact, cvt_dtype, cvt_out, converted);
    const uint16_t *wh, *wl, *hh_, *hl;
    int32_t rc = planes_for(ctx, w, inverse ? 1 : 0, s, &wh, &wl);
    if (rc != HH_OK) return rc;
    rc = planes_for(ctx, h, inverse ? 1 : 0, s, &hh_, &hl);
    if (rc != HH_OK) return rc;
    if (h == w) {  // the second lookup may have replaced the first's slot
        wh = hh_;
        wl = hl;
    }
    // scratch: block maxima, the constants {0, 1, 2^e, 2^-e}, the input's
    // planes and the intermediate's planes
    const uint32_t np = 1024;
    const uint64_t in_plane = (uint64_t)dct_planes_rows(h) * dct_planes_cols(w);
    const uint64_t mid_plane = (uint64_t)dct_planes_rows(w) * dct_planes_cols(h);
    const bool need_lo = !(inverse && f16_exact);
    const size_t off_in = ((np + 4) * sizeof(float) + 255) & ~(size_t)255;  // after the maxima and constants
    const size_t off_mid = off_in + ((in_plane * (need_lo ? 4 : 2) + 255) & ~(uint64_t)255);
    const size_t need = off_mid + mid_plane * 4;
    rc = split_scratch(ctx, need, s);
    if (rc != HH_OK) return rc;
    uint8_t *sp = reinterpret_cast<uint8_t *>(ctx->d_split);
    float *partial = reinterpret_cast<float *>(sp);
    float *consts = partial + np;
    uint16_t *in_hi = reinterpret_cast<uint16_t *>(sp + off_in);
    uint16_t *in_lo = need_lo ? in_hi + in_plane : nullptr;
    uint16_t *mid_hi = reinterpret_cast<uint16_t *>(sp + off_mid);
    uint16_t *mid_lo = mid_hi + mid_plane;
    (void)d_tmp;
    hipLaunchKernelGGL(amax_kernel, dim3(np), dim3(256), 0, s, d_in, total, partial);
    hipLaunchKernelGGL(split_scale_kernel, dim3(1), dim3(256), 0, s, partial, np, w, consts);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e);
    e = launch_operand_planes(d_in, h, w, w, consts + 2, in_hi, in_lo, s);
    if (e != hipSuccess) return from_hip(e);
    // first product: the w x h matrix P = B_w^T (C 2^e)^T (inverse) or
    // B_w (X 2^e)^T (forward), as the second product's planes
    DctGemm g1;
    g1.a_hi = wh;
    g1.a_lo = wl;
    g1.b_hi = in_hi;
    g1.b_lo = in_lo;
    g1.out_scale = nullptr;
    g1.d = mid_hi;
    g1.ldd = 0;
    g1.d_dtype = HH_F32;
    g1.d_planes = true;
    g1.M = w;
    g1.N = h;
    g1.K = w;
    e = launch_dct_gemm(g1, s);
    if (e != hipSuccess) return from_hip(e);
    // second product: the h x w result 2^-e B_h^T P^T (inverse) or
    // 2^-e B_h P^T (forward), converted on the way out when asked
    const bool cvt = inverse && cvt_out != nullptr;
    DctGemm g2;
    g2.a_hi = hh_;
    g2.a_lo = hl;
    g2.b_hi = mid_hi;
    g2.b_lo = mid_lo;
    g2.out_scale = consts + 3;
    g2.d = cvt ? cvt_out : d_out;
    g2.ldd = w;
    g2.d_dtype = cvt ? cvt_dtype : HH_F32;
    g2.d_planes = false;
    g2.M = h;
    g2.N = w;
    g2.K = h;
    e = launch_dct_gemm(g2, s);
    if (e != hipSuccess) return from_hip(e);
    if (converted) *converted = cvt;
    return HH_OK;
}

void release_dct_resources(hh_context *ctx) {
    for (int i = 0; i < 2; i++) {
        if (ctx->dct_basis[i].hl) (void)hipFree(ctx->dct_basis[i].hl);
        ctx->dct_basis[i].hl = nullptr;
        ctx->dct_basis[i].n = 0;
    }
    if (ctx->d_split) (void)hipFree(ctx->d_split);
    ctx->d_split = nullptr;
    ctx->split_bytes = 0;
}

}  // namespace hh
