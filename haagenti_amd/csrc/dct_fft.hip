// Whole-matrix DCT-II / DCT-III (orthonormal) in O(n^2 log n): a 1-D
// transform along every row, a transpose, the 1-D transform along every
// row of the transposed matrix, and a transpose back (converted to the
// output type on the way).
//
// 1-D transform of a row of length N (N even), by Makhoul's reordering
// (J. Makhoul, "A fast cosine transform in one and two dimensions", IEEE
// Trans. ASSP 28(1), 1980) and the usual packing of a real sequence of
// length N into a complex one of length L = N / 2:
//   forward  v[m] = x[2m], v[N-1-m] = x[2m+1];  z[j] = v[2j] + i v[2j+1];
//            Z = DFT_L(z);  V[k] = E_k - i w_N^-k O_k with
//            E_k = (Z[k] + conj Z[L-k]) / 2, O_k = (Z[k] - conj Z[L-k]) / 2;
//            X[k] = s_k Re(w_4N^-k V[k]), X[N-k] = -s_{N-k} Im(w_4N^-k V[k])
//   inverse  c = s X;  H[0] = c[0], H[k] = w_4N^k (c[k] - i c[N-k]) / 2;
//            Z[k] = (H[k] + H[k+L]) + i w_N^k (H[k] - H[k+L]);
//            z = unnormalised inverse DFT_L(Z);  v[2j] = Re z[j],
//            v[2j+1] = Im z[j];  x[2m] = v[m], x[2m+1] = v[N-1-m]
// with w_n = e^(2 pi i / n), s_0 = sqrt(1/N), s_k = sqrt(2/N).  The complex
// DFT of length L runs in LDS as a Stockham autosort FFT (radix 8, 4, 2, 3,
// 5, 7 passes; each pass reads all its butterflies' inputs into registers,
// then writes the outputs in place), one workgroup per row, with f32
// arithmetic and twiddles rounded from double.
//
// The reference's whole-matrix transforms switch to an FFT above 4096
// (haagenti-cuda/src/dct_gpu.rs:1081,1381-1412, via cufft_ffi.rs:423-506);
// its CPU path is the same Makhoul construction (haagenti-core/src/
// dct.rs:154-259).
#include "hh_internal.hpp"

namespace hh {
namespace {

constexpr uint32_t kMaxLds = 160u * 1024u;
constexpr uint32_t kFftMaxFrags = 16;
constexpr uint32_t kStaticLds = 64;  // the row kernel's scan words, beside the dynamic LDS
// elements (k pairs) per thread of a fused-scatter pre-step, read before any
// write (the row and the FFT points share the LDS)
constexpr uint32_t kScatK = 8;

struct FftRows {
    const float *in;
    float *out;
    // twiddle tables (fft_tables_kernel): per pass q (radix R_q, p_q the
    // product of the earlier radices) w_L^(j k L / (p_q R_q)) at
    // [off_q + (j - 1) p_q + k] for k < p_q, 1 <= j < R_q -- the lanes of a
    // wave read consecutive k, so each load is coalesced; then w_4N^k for
    // k <= N and w_N^k for k < L
    const float2 *ptab;
    const float2 *w4;
    const float2 *wn;
    // the inverse pre-step's combined factors for k < L: alpha_k =
    // s1 w_4N^k (1 + i w_N^k) / 2, beta_k = s1 w_4N^(k+L) (1 - i w_N^k) / 2
    // (x, y = alpha; z, w = beta), so that Z[k] = alpha_k (c[k] - i c[N-k])
    // + beta_k (c[k+L] - i c[L-k]) with the inputs unscaled
    const float4 *ab;
    uint32_t N, L;
    uint32_t nr;
    uint8_t r[16];
    // LDS layout of the L points: point x at x + (x >> psh), one pad slot
    // per 32 points (psh = 5, when L is a multiple of 256) so that the
    // strided writes of the first passes spread over the banks, or none
    // (psh = 31)
    uint32_t psh;
    // HCT3 fragments scattered into the rows in LDS (the fused first pass of
    // an inverse; `in` unused): fragment f's bitmap as 64-bit words, the
    // rank of each row's first bit, its f16 values and their count
    uint32_t nfrag;
    const uint64_t *fbits[kFftMaxFrags];
    const uint32_t *fpref[kFftMaxFrags];
    const uint8_t *fcoef[kFftMaxFrags];
    uint32_t fncoef[kFftMaxFrags];
};

// table[idx]: the table's base (a kernel argument, scalar) plus a 32-bit
// byte offset, so the load needs no 64-bit address arithmetic per lane
__device__ __forceinline__ float2 tab_at(const float2 *__restrict__ table, uint32_t idx) {
    return *reinterpret_cast<const float2 *>(reinterpret_cast<const uint8_t *>(table) + (size_t)(idx * 8u));
}
__device__ __forceinline__ float2 tab_at_byte(const float2 *__restrict__ table, uint32_t off) {
    return *reinterpret_cast<const float2 *>(reinterpret_cast<const uint8_t *>(table) + (size_t)off);
}
// the byte offsets of a pass table's entries (j, k), j = 1 .. R-1: k + (j -
// 1) p, stepped by additions (the empty asm keeps the compiler from turning
// the steps into quarter-rate multiplies)
template <int R>
__device__ __forceinline__ void twiddle_offsets(uint32_t k, uint32_t p, uint32_t (&off)[R]) {
    const uint32_t p8 = p * 8u;
    uint32_t o = k * 8u;
    off[1] = o;
#pragma unroll
    for (int j = 2; j < R; j++) {
        o += p8;
        __asm__("" : "+v"(o));
        off[j] = o;
    }
}

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cconj(float2 a) { return make_float2(a.x, -a.y); }
// i^S a for S = +1 (INV) or -1
template <bool INV>
__device__ __forceinline__ float2 rot90(float2 a) {
    return INV ? make_float2(-a.y, a.x) : make_float2(a.y, -a.x);
}

// In-register DFT of length R with e^(+-2 pi i / R) (+ for INV).
template <int R, bool INV>
struct Dft;

template <bool INV>
struct Dft<2, INV> {
    __device__ __forceinline__ static void run(float2 *x) {
        const float2 a = x[0], b = x[1];
        x[0] = cadd(a, b);
        x[1] = csub(a, b);
    }
};

template <bool INV>
struct Dft<4, INV> {
    __device__ __forceinline__ static void run(float2 *x) {
        const float2 t0 = cadd(x[0], x[2]), t1 = csub(x[0], x[2]);
        const float2 t2 = cadd(x[1], x[3]), t3 = rot90<INV>(csub(x[1], x[3]));
        x[0] = cadd(t0, t2);
        x[2] = csub(t0, t2);
        x[1] = cadd(t1, t3);
        x[3] = csub(t1, t3);
    }
};

template <bool INV>
struct Dft<8, INV> {
    __device__ __forceinline__ static void run(float2 *x) {
        float2 e[4] = {x[0], x[2], x[4], x[6]};
        float2 o[4] = {x[1], x[3], x[5], x[7]};
        Dft<4, INV>::run(e);
        Dft<4, INV>::run(o);
        constexpr float h = 7.071067812e-01f;  // 1 / sqrt(2)
        // o[q] *= w_8^(+-q)
        o[1] = INV ? make_float2(h * (o[1].x - o[1].y), h * (o[1].x + o[1].y))
                   : make_float2(h * (o[1].x + o[1].y), h * (o[1].y - o[1].x));
        o[2] = rot90<INV>(o[2]);
        o[3] = INV ? make_float2(-h * (o[3].x + o[3].y), h * (o[3].x - o[3].y))
                   : make_float2(h * (o[3].y - o[3].x), -h * (o[3].x + o[3].y));
#pragma unroll
        for (int q = 0; q < 4; q++) {
            x[q] = cadd(e[q], o[q]);
            x[q + 4] = csub(e[q], o[q]);
        }
    }
};

template <bool INV>
struct Dft<3, INV> {
    __device__ __forceinline__ static void run(float2 *x) {
        constexpr float s3 = 8.660254038e-01f;  // sin(2 pi / 3)
        const float2 t = cadd(x[1], x[2]);
        const float2 u = rot90<INV>(csub(x[1], x[2]));
        const float2 m = make_float2(x[0].x - 0.5f * t.x, x[0].y - 0.5f * t.y);
        x[0] = cadd(x[0], t);
        x[1] = make_float2(m.x + s3 * u.x, m.y + s3 * u.y);
        x[2] = make_float2(m.x - s3 * u.x, m.y - s3 * u.y);
    }
};

// odd R: y_q = x_0 + sum_m a_m cos(2 pi m q / R) +- i sum_m b_m sin(2 pi m q / R)
// over m = 1 .. (R-1)/2 with a_m = x_m + x_{R-m}, b_m = x_m - x_{R-m}
template <int R, bool INV>
__device__ __forceinline__ void dft_odd(float2 *x, const float *c, const float *sn) {
    constexpr int H = (R - 1) / 2;
    float2 a[H], b[H];
#pragma unroll
    for (int m = 1; m <= H; m++) {
        a[m - 1] = cadd(x[m], x[R - m]);
        b[m - 1] = rot90<INV>(csub(x[m], x[R - m]));
    }
    float2 y[R];
    y[0] = x[0];
#pragma unroll
    for (int m = 0; m < H; m++) y[0] = cadd(y[0], a[m]);
#pragma unroll
    for (int q = 1; q <= H; q++) {
        float2 re = x[0], im = make_float2(0.0f, 0.0f);
#pragma unroll
        for (int m = 1; m <= H; m++) {
            const int j = (m * q) % R;  // cos / sin of 2 pi j / R, j in [1, R)
            const float cj = j <= H ? c[j - 1] : c[R - j - 1];
            const float sj = j <= H ? sn[j - 1] : -sn[R - j - 1];
            re = make_float2(re.x + cj * a[m - 1].x, re.y + cj * a[m - 1].y);
            im = make_float2(im.x + sj * b[m - 1].x, im.y + sj * b[m - 1].y);
        }
        y[q] = cadd(re, im);
        y[R - q] = csub(re, im);
    }
#pragma unroll
    for (int q = 0; q < R; q++) x[q] = y[q];
}

template <bool INV>
struct Dft<5, INV> {
    __device__ __forceinline__ static void run(float2 *x) {
        constexpr float c[2] = {3.090169944e-01f, -8.090169944e-01f};
        constexpr float sn[2] = {9.510565163e-01f, 5.877852523e-01f};
        dft_odd<5, INV>(x, c, sn);
    }
};

template <bool INV>
struct Dft<7, INV> {
    __device__ __forceinline__ static void run(float2 *x) {
        constexpr float c[3] = {6.234898019e-01f, -2.225209340e-01f, -9.009688679e-01f};
        constexpr float sn[3] = {7.818314825e-01f, 9.749279122e-01f, 4.338837391e-01f};
        dft_odd<7, INV>(x, c, sn);
    }
};

// Exclusive sum of v over the workgroup's threads (up to 1024; sm: 16
// words of LDS).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *sm) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(incl, d);
        if (lane >= (uint32_t)d) incl += t;
    }
    if (lane == 63u) sm[wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t i = 0; i < nw; i++) before += i < wave ? sm[i] : 0u;
    __syncthreads();  // sm reusable after
    return before + incl - v;
}

// Set bits per row of a bitmap of `rows` rows of wpr 64-bit words: one wave
// per row.
__global__ __launch_bounds__(256) void row_counts_kernel(const uint64_t *__restrict__ bits, uint32_t wpr,
                                                         uint32_t rows, uint32_t *__restrict__ cnt) {
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (row >= rows) return;
    const uint64_t *rb = bits + (uint64_t)row * wpr;
    uint32_t c = 0;
    for (uint32_t i = lane; i < wpr; i += 64u) c += (uint32_t)__popcll(rb[i]);
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) c += __shfl_xor(c, d);
    if (lane == 0) cnt[row] = c;
}

// Builds row `row` of the coefficient matrix in LDS as N f32 values (rowf)
// from the fragments, in order: zeros, then every set bit whose rank is
// below the fragment's value count takes that value (later fragments
// overwrite earlier ones), as the HCT3 scatter does.  wds / wpre: N / 64
// words of LDS each (the row's bitmap words and their ranks).
__device__ __forceinline__ void scatter_row(const FftRows &P, uint32_t row, float *rowf, uint64_t *wds,
                                            uint32_t *wpre, uint32_t *sm) {
    const uint32_t N = P.N, T = blockDim.x, tid = threadIdx.x, nw = N / 64u;
    for (uint32_t i = tid; i < N / 4u; i += T) reinterpret_cast<float4 *>(rowf)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t f = 0; f < P.nfrag; f++) {
        // this row's words and the rank of each word's first bit (nw <= T)
        uint64_t wv = 0;
        if (tid < nw) wv = P.fbits[f][(uint64_t)row * nw + tid];
        const uint32_t ex = block_excl_scan(tid < nw ? (uint32_t)__popcll(wv) : 0u, sm);
        if (tid < nw) {
            wds[tid] = wv;
            wpre[tid] = P.fpref[f][row] + ex;
        }
        __syncthreads();
        const uint32_t nc = P.fncoef[f];
        const uint8_t *cb = P.fcoef[f];
        if (nc > 0 && ((uintptr_t)cb & 1u) == 0) {
            // eight elements' values loaded together (an element without a
            // value loads value 0 and discards it)
            const uint16_t *c16 = reinterpret_cast<const uint16_t *>(cb);
            for (uint32_t e0 = 0; e0 < N; e0 += 8u * T) {
                uint32_t x[8];
                bool hv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t e = e0 + tid + (uint32_t)u * T;
                    hv[u] = false;
                    uint32_t rk = 0;
                    if (e < N) {
                        const uint64_t bw = wds[e >> 6];
                        const uint32_t bit = e & 63u;
                        rk = wpre[e >> 6] + (uint32_t)__popcll(bw & ((1ull << bit) - 1ull));
                        hv[u] = ((bw >> bit) & 1ull) && rk < nc;
                    }
                    x[u] = c16[hv[u] ? rk : 0u];
                }
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (hv[u]) rowf[e0 + tid + (uint32_t)u * T] = f16_bits_to_f32(x[u]);
            }
        } else {
            // values at an odd byte offset: read bytewise
            for (uint32_t e = tid; e < N; e += T) {
                const uint64_t bw = wds[e >> 6];
                const uint32_t bit = e & 63u;
                const uint32_t rk = wpre[e >> 6] + (uint32_t)__popcll(bw & ((1ull << bit) - 1ull));
                if (((bw >> bit) & 1ull) && rk < nc)
                    rowf[e] = f16_bits_to_f32((uint32_t)cb[2ull * rk] | ((uint32_t)cb[2ull * rk + 1] << 8));
            }
        }
        __syncthreads();  // the next fragment rewrites wds / wpre
    }
}

// One Stockham pass of radix R over the L points in LDS, p = the product
// of the earlier passes' radices: butterfly i (of L / R) takes points
// i + j L/R, multiplies point j by w_L^(+-j k L/(p R)) with k = i mod p
// (an exponent below L), transforms, and writes output j to
// (i - k) R + k + j p.  All inputs are read before the barrier, so the
// pass runs in place.
template <int R, int MAXB, bool INV>
__device__ __forceinline__ void fft_pass(float2 *buf, uint32_t L, uint32_t p, const float2 *__restrict__ ptab,
                                         uint32_t psh) {
    // the twiddles are loaded with the pass's LDS reads, before the barrier,
    // where the registers allow; the first pass (p = 1) has none
    constexpr bool kPre = MAXB * (R - 1) <= 16;
    const bool tw = p > 1;
    const uint32_t T = blockDim.x, tid = threadIdx.x;
    const uint32_t nb = L / R;
    // i mod p without a division: (i + 1/2) / p lies at least 1/(2p) from an
    // integer, and the float product's relative error (2^-23 with 1/p
    // rounded) stays below that for i < 2^22 (i < L <= 20480 here)
    const float invp = 1.0f / (float)p;
    auto mod_p = [&](uint32_t i) { return i - (uint32_t)(((float)i + 0.5f) * invp) * p; };
    float2 x[MAXB][R];
    float2 w[kPre ? MAXB : 1][R - 1];
    // padded layout: point i + j nb at pad(i) + j (nb + nb / 32), point
    // base + j p at pad(base) + j p + j p / 32 (nb and, past the first
    // passes, p are multiples of 32 when padded; the first passes' p R
    // divides 32)
    const uint32_t rstep = nb + (nb >> psh);
#pragma unroll
    for (int b = 0; b < MAXB; b++) {
        const uint32_t i = tid + b * T;
        if (i < nb) {
            const uint32_t ri = i + (i >> psh);
#pragma unroll
            for (int j = 0; j < R; j++) x[b][j] = buf[ri + j * rstep];
            if (kPre && tw) {
                uint32_t off[R];
                twiddle_offsets<R>(mod_p(i), p, off);
#pragma unroll
                for (int j = 1; j < R; j++) w[kPre ? b : 0][j - 1] = tab_at_byte(ptab, off[j]);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < MAXB; b++) {
        const uint32_t i = tid + b * T;
        if (i < nb) {
            const uint32_t k = mod_p(i);
            if (tw) {
                uint32_t off[R];
                if (!kPre) twiddle_offsets<R>(k, p, off);
#pragma unroll
                for (int j = 1; j < R; j++) {
                    float2 t = kPre ? w[kPre ? b : 0][j - 1] : tab_at_byte(ptab, off[j]);
                    if (!INV) t.y = -t.y;
                    x[b][j] = cmul(x[b][j], t);
                }
            }
            Dft<R, INV>::run(x[b]);
            const uint32_t base = (i - k) * R + k;
            const uint32_t wb = base + (base >> psh);
#pragma unroll
            for (int j = 0; j < R; j++) buf[wb + j * p + ((j * p) >> psh)] = x[b][j];
        }
    }
    __syncthreads();
}

template <bool INV, int MAXB, bool SCAT = false>
__global__ __launch_bounds__(1024) void dct_fft_rows_kernel(FftRows P) {
    extern __shared__ float2 buf[];
    __shared__ uint32_t scan_sm[16];
    const uint32_t N = P.N, L = P.L, T = blockDim.x, tid = threadIdx.x;
    const float *__restrict__ in = P.in + (uint64_t)blockIdx.x * N;
    float *__restrict__ out = P.out + (uint64_t)blockIdx.x * N;
    const float2 *__restrict__ w4 = P.w4;
    const float2 *__restrict__ wn = P.wn;
    const float s0 = sqrtf(1.0f / (float)N), s1 = sqrtf(2.0f / (float)N);
    const uint32_t psh = P.psh;
    auto pd = [psh](uint32_t x) { return x + (x >> psh); };  // LDS slot of point x
    // Z[k] and Z[L-k] from c[k], c[N-k], c[k+L], c[L-k] for 0 < k < L/2;
    // k = 0's thread also makes Z[0] (from c[0], c[L]) and the self-paired
    // Z[L/2] (from c[L/2], c[3L/2]); the inputs come as c[k], c[3L/2 or
    // N-k], c[k+L], c[L/2 or L-k]
    // (a - i b) scaled by the factor f: (f.x a + f.y b, f.y a - f.x b)
    auto fm = [](float fx, float fy, float a, float b) {
        return make_float2(__builtin_fmaf(fx, a, fy * b), __builtin_fmaf(fy, a, -(fx * b)));
    };
    const float4 *__restrict__ ab = P.ab;
    auto emit = [&](uint32_t k, float a, float b, float d, float e) {
        if (k == 0) {
            // Z[0] = s0 c[0] (1 + i) + beta_0 (c[L] - i c[L]);
            // Z[L/2] = alpha_{L/2} (c[L/2] - i c[3L/2]) + beta_{L/2} (c[3L/2] - i c[L/2])
            const float4 f0 = ab[0], fm2 = ab[L / 2];
            const float as = a * s0;
            buf[0] = cadd(make_float2(as, as), fm(f0.z, f0.w, d, d));
            buf[pd(L / 2)] = cadd(fm(fm2.x, fm2.y, e, b), fm(fm2.z, fm2.w, b, e));
            return;
        }
        const float4 fk = ab[k], fk2 = ab[L - k];
        buf[pd(k)] = cadd(fm(fk.x, fk.y, a, b), fm(fk.z, fk.w, d, e));
        buf[pd(L - k)] = cadd(fm(fk2.x, fk2.y, e, d), fm(fk2.z, fk2.w, b, a));
    };
    if constexpr (SCAT) {
        // the row built in LDS from the fragments; every thread reads all of
        // its inputs (L/2 <= kScatK T) before any Z overwrites them
        float *rowf = reinterpret_cast<float *>(buf);
        uint64_t *wds = reinterpret_cast<uint64_t *>(buf + pd(L - 1) + 1);
        uint32_t *wpre = reinterpret_cast<uint32_t *>(wds + N / 64u);
        scatter_row(P, blockIdx.x, rowf, wds, wpre, scan_sm);
        float a[kScatK], b[kScatK], d[kScatK], e[kScatK];
#pragma unroll
        for (uint32_t u = 0; u < kScatK; u++) {
            const uint32_t k = tid + u * T;
            if (k < L / 2) {
                a[u] = rowf[k];
                b[u] = rowf[k == 0 ? 3 * L / 2 : N - k];
                d[u] = rowf[k + L];
                e[u] = rowf[k == 0 ? L / 2 : L - k];
            }
        }
        __syncthreads();
#pragma unroll
        for (uint32_t u = 0; u < kScatK; u++) {
            const uint32_t k = tid + u * T;
            if (k < L / 2) emit(k, a[u], b[u], d[u], e[u]);
        }
    } else if (INV) {
        // the row's loads are issued kB per thread at a time, before any use
        constexpr int kB = 4;
        for (uint32_t k0 = 0; k0 < L / 2; k0 += kB * T) {
            float a[kB], b[kB], d[kB], e[kB];
#pragma unroll
            for (int u = 0; u < kB; u++) {
                const uint32_t k = k0 + tid + u * T;
                if (k < L / 2) {
                    a[u] = in[k];
                    b[u] = in[k == 0 ? 3 * L / 2 : N - k];
                    d[u] = in[k + L];
                    e[u] = in[k == 0 ? L / 2 : L - k];
                }
            }
#pragma unroll
            for (int u = 0; u < kB; u++) {
                const uint32_t k = k0 + tid + u * T;
                if (k < L / 2) emit(k, a[u], b[u], d[u], e[u]);
            }
        }
    } else {
        // z[q] = x[4q] + i x[4q+2], z[L-1-q] = x[4q+3] + i x[4q+1]
        constexpr int kB = 4;
        const float4 *in4 = reinterpret_cast<const float4 *>(in);
        for (uint32_t q0 = 0; q0 < L / 2; q0 += kB * T) {
            float4 v[kB];
#pragma unroll
            for (int u = 0; u < kB; u++) {
                const uint32_t q = q0 + tid + u * T;
                if (q < L / 2) v[u] = in4[q];
            }
#pragma unroll
            for (int u = 0; u < kB; u++) {
                const uint32_t q = q0 + tid + u * T;
                if (q < L / 2) {
                    buf[pd(q)] = make_float2(v[u].x, v[u].z);
                    buf[pd(L - 1 - q)] = make_float2(v[u].w, v[u].y);
                }
            }
        }
    }
    __syncthreads();
    uint32_t p = 1, poff = 0;
    for (uint32_t q = 0; q < P.nr; q++) {
        switch (P.r[q]) {
            case 8: fft_pass<8, MAXB, INV>(buf, L, p, P.ptab + poff, psh); break;
            case 4: fft_pass<4, MAXB, INV>(buf, L, p, P.ptab + poff, psh); break;
            case 2: fft_pass<2, MAXB, INV>(buf, L, p, P.ptab + poff, psh); break;
            case 3: fft_pass<3, MAXB, INV>(buf, L, p, P.ptab + poff, psh); break;
            case 5: fft_pass<5, MAXB, INV>(buf, L, p, P.ptab + poff, psh); break;
            default: fft_pass<7, MAXB, INV>(buf, L, p, P.ptab + poff, psh); break;
        }
        poff += p * (P.r[q] - 1u);
        p *= P.r[q];
    }
    if (INV) {
        // x[4q .. 4q+3] = Re z[q], Im z[L-1-q], Im z[q], Re z[L-1-q]
        float4 *out4 = reinterpret_cast<float4 *>(out);
        for (uint32_t q = tid; q < L / 2; q += T) {
            const float2 za = buf[pd(q)], zb = buf[pd(L - 1 - q)];
            out4[q] = make_float4(za.x, zb.y, za.y, zb.x);
        }
    } else {
        // X[k], X[N-k] from V[k], for k and L - k
        for (uint32_t k = tid; k <= L / 2; k += T) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t kk = h == 0 ? k : L - k;
                if (h == 1 && 2 * k == L) break;
                const float2 zk = buf[pd(kk == L ? 0 : kk)];
                const float2 zc = cconj(buf[pd(kk == 0 ? 0 : L - kk)]);
                const float2 E = make_float2(0.5f * (zk.x + zc.x), 0.5f * (zk.y + zc.y));
                const float2 D = make_float2(0.5f * (zk.x - zc.x), 0.5f * (zk.y - zc.y));
                const float2 wq = kk == L ? make_float2(-1.0f, 0.0f) : cconj(tab_at(wn, kk));
                const float2 V = csub(E, rot90<true>(cmul(wq, D)));
                const float2 W = cmul(cconj(tab_at(w4, kk)), V);
                out[kk] = (kk == 0 ? s0 : s1) * W.x;
                if (kk != 0 && kk != L) out[N - kk] = -s1 * W.y;
            }
        }
    }
}

// out (cols x rows) = transpose of in (rows x cols), both multiples of 64,
// converted to OUT (HH_F32, HH_BF16 or HH_F16): 64 x 64 tiles through LDS.
template <int OUT>
__global__ __launch_bounds__(256) void transpose_kernel(const float *__restrict__ in, uint32_t rows, uint32_t cols,
                                                         void *__restrict__ out) {
    __shared__ float tile[64][65];
    const uint32_t c0 = blockIdx.x * 64u, r0 = blockIdx.y * 64u;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = ty + 16 * i;
        const float4 v = *reinterpret_cast<const float4 *>(in + (uint64_t)(r0 + r) * cols + c0 + 4 * tx);
        tile[r][4 * tx + 0] = v.x;
        tile[r][4 * tx + 1] = v.y;
        tile[r][4 * tx + 2] = v.z;
        tile[r][4 * tx + 3] = v.w;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = ty + 16 * i;
        const float a = tile[4 * tx + 0][c], b = tile[4 * tx + 1][c];
        const float d = tile[4 * tx + 2][c], e = tile[4 * tx + 3][c];
        const uint64_t o = (uint64_t)(c0 + c) * rows + r0 + 4 * tx;
        if (OUT == HH_F32) {
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + o) = make_float4(a, b, d, e);
        } else {
            auto cv = [](float v) { return OUT == HH_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v); };
            *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(out) + o) =
                make_uint2(cv(a) | (cv(b) << 16), cv(d) | (cv(e) << 16));
        }
    }
}

// The twiddle tables of a length-N plan (FftRows): the pass tables (L - 1
// entries: sum_q p_q (R_q - 1) = L - 1), then w_4N^k for k <= N, then w_N^k
// for k < L; each entry computed in double and rounded once.
struct TabPlan {
    uint32_t L, N, nr;
    uint8_t r[16];
};
constexpr uint32_t tab_w4(uint32_t L) { return L; }              // after the pass tables (L - 1, one pad)
constexpr uint32_t tab_wn(uint32_t L, uint32_t N) { return L + N + 1; }
constexpr uint32_t tab_ab(uint32_t L, uint32_t N) { return 2 * L + N + 2; }  // 16-byte aligned (one pad)
constexpr uint32_t tab_len(uint32_t L, uint32_t N) { return tab_ab(L, N) + 2 * L; }

__global__ __launch_bounds__(256) void fft_tables_kernel(float2 *__restrict__ tab, TabPlan P) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const uint32_t L = P.L, N = P.N;
    if (i >= tab_len(L, N)) return;
    double s = 0.0, c = 1.0;
    if (i < L) {
        // pass q: entry (j, k) at off_q + (j - 1) p_q + k
        uint32_t p = 1, off = 0;
        for (uint32_t q = 0; q < P.nr; q++) {
            const uint32_t R = P.r[q], n = p * (R - 1u);
            if (i < off + n) {
                const uint32_t j = (i - off) / p + 1u, k = (i - off) % p;
                // w_L^(j k L / (p R)) = e^(2 pi i j k / (p R))
                sincospi(2.0 * (double)(j * k) / (double)(p * R), &s, &c);
                break;
            }
            off += n;
            p *= R;
        }
    } else if (i < tab_wn(L, N)) {
        sincospi((double)(i - L) / (2.0 * (double)N), &s, &c);
    } else if (i < tab_wn(L, N) + L) {
        sincospi(2.0 * (double)(i - tab_wn(L, N)) / (double)N, &s, &c);
    } else if (i >= tab_ab(L, N)) {
        // alpha_k (even entry) or beta_k (odd entry)
        const uint32_t k = (i - tab_ab(L, N)) >> 1, beta = (i - tab_ab(L, N)) & 1u;
        double s4, c4, sn, cn;
        sincospi((double)(k + (beta ? L : 0u)) / (2.0 * (double)N), &s4, &c4);  // w_4N^(k or k+L)
        sincospi(2.0 * (double)k / (double)N, &sn, &cn);                          // w_N^k
        // (1 + i w_N^k) = (1 - sn, cn); (1 - i w_N^k) = (1 + sn, -cn)
        const double fr = beta ? 1.0 + sn : 1.0 - sn, fi = beta ? -cn : cn;
        const double h = 0.5 * sqrt(2.0 / (double)N);
        c = h * (c4 * fr - s4 * fi);
        s = h * (c4 * fi + s4 * fr);
    }
    tab[i] = make_float2((float)c, (float)s);
}

struct Plan {
    uint32_t N = 0, L = 0, threads = 0, maxb = 0, nr = 0, psh = 31;
    uint8_t r[16] = {};
};
// LDS slots of L points in the layout of shift psh (one pad slot per 32
// points when psh = 5)
constexpr uint32_t slots_of(uint32_t L, uint32_t psh) { return L + (psh == 5u ? L / 32u : 0u); }

// Radices of L (8s, then 4 or 2, then 3, 5, 7), the workgroup size and
// the butterflies per thread of the widest pass; false when N is not a
// multiple of 64, L has another prime factor, L points do not fit in LDS
// or a pass would need more than 4 butterflies per thread (more registers
// than a 1024-thread workgroup has: the MAXB = 8 variant spilled).
bool make_plan(uint32_t N, Plan &P) {
    if (N == 0 || N % 64u != 0) return false;
    const uint32_t L = N / 2;
    // the padded layout when every pass keeps its strides multiples of 32
    // (L a multiple of 256)
    const uint32_t psh = L % 256u == 0 ? 5u : 31u;
    if ((uint64_t)slots_of(L, psh) * 8u + kStaticLds > kMaxLds) return false;
    uint32_t n = L, nr = 0;
    uint8_t r[16];
    while (n % 8 == 0) r[nr++] = 8, n /= 8;
    if (n % 4 == 0) r[nr++] = 4, n /= 4;
    if (n % 2 == 0) r[nr++] = 2, n /= 2;
    for (uint32_t f : {3u, 5u, 7u})
        while (n % f == 0 && nr < 16) r[nr++] = (uint8_t)f, n /= f;
    if (n != 1) return false;
    uint32_t T = (L / 8 + 63) / 64 * 64;
    T = T < 64 ? 64 : T > 1024 ? 1024 : T;
    uint32_t mb = 0;
    for (uint32_t q = 0; q < nr; q++) {
        const uint32_t b = (L / r[q] + T - 1) / T;
        mb = b > mb ? b : mb;
    }
    if (mb > 4) return false;
    P.N = N;
    P.L = L;
    P.psh = psh;
    P.threads = T;
    P.maxb = mb <= 1 ? 1 : mb <= 2 ? 2 : 4;
    P.nr = nr;
    for (uint32_t q = 0; q < nr; q++) P.r[q] = r[q];
    return true;
}

template <bool INV, int MAXB, bool SCAT>
hipError_t launch_rows_t(const FftRows &A, uint32_t rows, uint32_t threads, hipStream_t s) {
    const uint32_t lds = slots_of(A.L, A.psh) * 8u + (SCAT ? (A.N / 64u) * 12u : 0u);
    hipError_t e = hipFuncSetAttribute((const void *)dct_fft_rows_kernel<INV, MAXB, SCAT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((dct_fft_rows_kernel<INV, MAXB, SCAT>), dim3(rows), dim3(threads), lds, s, A);
    return hipGetLastError();
}

// The row pass of plan P over `rows` rows; `scat` (an inverse's first pass)
// supplies the HCT3 fragments in place of `in`.
hipError_t launch_rows(bool inverse, const Plan &P, const float *in, float *out, uint32_t rows,
                       const float2 *tab, hipStream_t s, const FftRows *scat = nullptr) {
    FftRows A;
    if (scat) A = *scat;
    else A.nfrag = 0;
    A.in = in;
    A.out = out;
    A.ptab = tab;
    A.w4 = tab + tab_w4(P.L);
    A.wn = tab + tab_wn(P.L, P.N);
    A.ab = reinterpret_cast<const float4 *>(tab + tab_ab(P.L, P.N));
    A.N = P.N;
    A.L = P.L;
    A.psh = P.psh;
    A.nr = P.nr;
    for (int q = 0; q < 16; q++) A.r[q] = P.r[q];
    if (scat) {
        switch (P.maxb) {
            case 1: return launch_rows_t<true, 1, true>(A, rows, P.threads, s);
            case 2: return launch_rows_t<true, 2, true>(A, rows, P.threads, s);
            default: return launch_rows_t<true, 4, true>(A, rows, P.threads, s);
        }
    }
    switch (P.maxb | (inverse ? 16 : 0)) {
        case 1: return launch_rows_t<false, 1, false>(A, rows, P.threads, s);
        case 2: return launch_rows_t<false, 2, false>(A, rows, P.threads, s);
        case 4: return launch_rows_t<false, 4, false>(A, rows, P.threads, s);
        case 17: return launch_rows_t<true, 1, false>(A, rows, P.threads, s);
        case 18: return launch_rows_t<true, 2, false>(A, rows, P.threads, s);
        default: return launch_rows_t<true, 4, false>(A, rows, P.threads, s);
    }
}

// Whether plan P's rows can take the fragments in LDS: every thread's
// pre-step inputs read at once (L/2 <= kScatK threads), one bitmap word per
// thread, and the row's words and ranks beside the points in LDS.
bool scat_ok(const Plan &P) {
    return P.L / 2u <= kScatK * P.threads && P.N / 64u <= P.threads &&
           (uint64_t)slots_of(P.L, P.psh) * 8u + (P.N / 64u) * 12u + kStaticLds <= kMaxLds;
}

hipError_t launch_transpose(const float *in, uint32_t rows, uint32_t cols, int32_t dtype, void *out, hipStream_t s) {
    const dim3 grid(cols / 64u, rows / 64u);
    switch (dtype) {
        case HH_BF16: hipLaunchKernelGGL(transpose_kernel<HH_BF16>, grid, dim3(256), 0, s, in, rows, cols, out); break;
        case HH_F16: hipLaunchKernelGGL(transpose_kernel<HH_F16>, grid, dim3(256), 0, s, in, rows, cols, out); break;
        default: hipLaunchKernelGGL(transpose_kernel<HH_F32>, grid, dim3(256), 0, s, in, rows, cols, out); break;
    }
    return hipGetLastError();
}

// The context's twiddle tables for length n (two cached, the older replaced).
int32_t tables_for(hh_context *ctx, const Plan &P, hipStream_t s, const float2 **out) {
    for (int i = 0; i < 2; i++) {
        hh_context::FftTables &t = ctx->fft_tab[i];
        if (t.tab && t.n == P.N) {
            t.stamp = ++ctx->dct_stamp;
            *out = reinterpret_cast<const float2 *>(t.tab);
            return HH_OK;
        }
    }
    const int v = !ctx->fft_tab[0].tab ? 0 : !ctx->fft_tab[1].tab ? 1
                  : ctx->fft_tab[0].stamp <= ctx->fft_tab[1].stamp ? 0 : 1;
    hh_context::FftTables &t = ctx->fft_tab[v];
    if (t.tab) {
        // the stream may still read the old table: wait before freeing
        hipError_t e = hipStreamSynchronize(s);
        if (e == hipSuccess) e = hipFree(t.tab);
        t.tab = nullptr;
        t.n = 0;
        if (e != hipSuccess) return from_hip(e);
    }
    const uint32_t n = tab_len(P.L, P.N);
    hipError_t e = hipMalloc(&t.tab, (size_t)n * sizeof(float2));
    if (e != hipSuccess) {
        t.tab = nullptr;
        return from_hip(e);
    }
    t.n = P.N;
    t.stamp = ++ctx->dct_stamp;
    TabPlan TP;
    TP.L = P.L;
    TP.N = P.N;
    TP.nr = P.nr;
    for (int q = 0; q < 16; q++) TP.r[q] = P.r[q];
    hipLaunchKernelGGL(fft_tables_kernel, dim3((n + 255) / 256), dim3(256), 0, s,
                       reinterpret_cast<float2 *>(t.tab), TP);
    e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e);
    *out = reinterpret_cast<const float2 *>(t.tab);
    return HH_OK;
}

}  // namespace

bool fft_supported(uint32_t n) {
    Plan P;
    return make_plan(n, P);
}

bool use_fft(const hh_context *ctx, uint32_t rows, uint32_t cols) {
    if (ctx->dct_route == HH_DCT_DENSE) return false;
    if (!fft_supported(rows) || !fft_supported(cols)) return false;
    if (ctx->dct_route == HH_DCT_FFT) return true;
    return (rows > cols ? rows : cols) >= kFftAutoMin;
}

int32_t fft_scratch(hh_context *ctx, uint64_t total, hipStream_t s, float **a, float **b) {
    const size_t mat = ((size_t)total * sizeof(float) + 255) & ~(size_t)255;
    if (ctx->fft_bytes < 2 * mat) {
        if (ctx->d_fft) {
            hipError_t e = hipStreamSynchronize(s);
            if (e == hipSuccess) e = hipFree(ctx->d_fft);
            ctx->d_fft = nullptr;
            ctx->fft_bytes = 0;
            if (e != hipSuccess) return from_hip(e);
        }
        hipError_t e = hipMalloc(&ctx->d_fft, 2 * mat);
        if (e != hipSuccess) {
            ctx->d_fft = nullptr;
            return from_hip(e);
        }
        ctx->fft_bytes = 2 * mat;
    }
    *a = reinterpret_cast<float *>(ctx->d_fft);
    *b = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(ctx->d_fft) + mat);
    return HH_OK;
}

namespace {
int32_t dct2d_fft_impl(hh_context *ctx, bool inverse, const float *d_in, float *d_a, float *d_b, uint32_t h,
                       uint32_t w, int32_t out_dtype, void *d_out, hipStream_t s, const FftRows *scat) {
    Plan Pw, Ph;
    if (!make_plan(w, Pw) || !make_plan(h, Ph)) return HH_ERR_UNSUPPORTED;
    if (reinterpret_cast<uintptr_t>(d_out) & (out_dtype == HH_F32 ? 15u : 7u)) return HH_ERR_UNSUPPORTED;
    // the forward route reads its rows as 16-byte vectors
    if (!inverse && (reinterpret_cast<uintptr_t>(d_in) & 15u)) return HH_ERR_UNSUPPORTED;
    const float2 *tw, *th;
    int32_t rc = tables_for(ctx, Pw, s, &tw);
    if (rc != HH_OK) return rc;
    rc = tables_for(ctx, Ph, s, &th);
    if (rc != HH_OK) return rc;
    if (h == w) tw = th;  // the second lookup may have replaced the first's slot
    // rows of length w: in -> b (h x w); b^T -> a (w x h); rows of length h:
    // a -> b (w x h); b^T -> out (h x w), converted
    hipError_t e = launch_rows(inverse, Pw, d_in, d_b, h, tw, s, scat);
    if (e == hipSuccess) e = launch_transpose(d_b, h, w, HH_F32, d_a, s);
    if (e == hipSuccess) e = launch_rows(inverse, Ph, d_a, d_b, w, th, s);
    if (e == hipSuccess) e = launch_transpose(d_b, w, h, out_dtype, d_out, s);
    return from_hip(e);
}
}  // namespace

int32_t dct2d_fft(hh_context *ctx, bool inverse, const float *d_in, float *d_a, float *d_b, uint32_t h,
                  uint32_t w, int32_t out_dtype, void *d_out, hipStream_t s) {
    return dct2d_fft_impl(ctx, inverse, d_in, d_a, d_b, h, w, out_dtype, d_out, s, nullptr);
}

int32_t hct3_decode_fft(hh_context *ctx, const Hct3Frag *frags, uint32_t nfrags, uint32_t h, uint32_t w,
                        int32_t dtype, void *d_out, hipStream_t s) {
    Plan Pw, Ph;
    if (nfrags == 0 || nfrags > kFftMaxFrags || !make_plan(w, Pw) || !make_plan(h, Ph) || !scat_ok(Pw))
        return HH_ERR_UNSUPPORTED;
    if (reinterpret_cast<uintptr_t>(d_out) & (dtype == HH_F32 ? 15u : 7u)) return HH_ERR_UNSUPPORTED;
    const uint64_t total = (uint64_t)h * w;
    float *a, *b;
    int32_t rc = fft_scratch(ctx, total, s, &a, &b);
    if (rc != HH_OK) return rc;
    // in a (free until the first pass has run): per fragment its bitmap as
    // words (total / 8 bytes: w is a multiple of 64) and its row ranks
    const size_t bits_bytes = (size_t)(total / 8u);
    const size_t pref_bytes = ((size_t)h * 4u + 255u) & ~(size_t)255u;
    uint8_t *pa = reinterpret_cast<uint8_t *>(a);
    FftRows F;
    F.nfrag = nfrags;
    for (uint32_t f = 0; f < nfrags; f++) {
        uint64_t *bits = reinterpret_cast<uint64_t *>(pa + f * (bits_bytes + pref_bytes));
        uint32_t *pref = reinterpret_cast<uint32_t *>(reinterpret_cast<uint8_t *>(bits) + bits_bytes);
        hipError_t e = launch_pack_bits(frags[f].bitmap, bits_bytes, bits, s);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(row_counts_kernel, dim3((h + 3u) / 4u), dim3(256), 0, s, bits, w / 64u, h, pref);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = launch_scan_counts(pref, h, s);
        if (e != hipSuccess) return from_hip(e);
        F.fbits[f] = bits;
        F.fpref[f] = pref;
        F.fcoef[f] = frags[f].coef;
        F.fncoef[f] = frags[f].ncoef;
    }
    return dct2d_fft_impl(ctx, true, nullptr, a, b, h, w, dtype, d_out, s, &F);
}

void release_fft_resources(hh_context *ctx) {
    for (int i = 0; i < 2; i++) {
        if (ctx->fft_tab[i].tab) (void)hipFree(ctx->fft_tab[i].tab);
        ctx->fft_tab[i].tab = nullptr;
        ctx->fft_tab[i].n = 0;
    }
    if (ctx->d_fft) (void)hipFree(ctx->d_fft);
    ctx->d_fft = nullptr;
    ctx->fft_bytes = 0;
}

}  // namespace hh
