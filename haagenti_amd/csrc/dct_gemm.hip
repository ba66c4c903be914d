// Whole-matrix DCT products on the f16 MFMA with split operands:
//
//     D[m][n] = s_out * sum_k A[m][k] Bt[n][k]          (m < M, n < N, k < K)
//
// Both operands are held as two f16 planes hi + lo (hi = f16(x), lo =
// f16(x - hi): x to ~2^-22 relative), row-major with k contiguous and padded
// with zeros to whole tiles (rows) and whole k steps (columns).  A is a DCT
// basis (B_n or its transpose); Bt is the f32 input, split by
// operand_planes_kernel after multiplying by a power of two 2^e, or the
// output of the first product, which writes its result as planes directly.
// Each product runs as three f16 MFMA passes with f32 accumulation,
// hi*hi + lo*hi + hi*lo (the dropped lo*lo is ~2^-22 relative), or two when
// Bt has no low half (its values are f16 values).
//
// The 2-D transforms are two such products (B_n[k][i] = s_k cos(pi k (2i+1)
// / 2n), an h x w matrix row-major):
//   inverse  X = B_h^T C B_w  (idct_2d, crates/haagenti-core/src/dct.rs:311-337):
//            T' = B_w^T (C 2^e)^T   (A = B_w^T, Bt = C:  M = w, N = h, K = w)
//            X  = 2^-e B_h^T T'^T   (A = B_h^T, Bt = T': M = h, N = w, K = h)
//   forward  C = B_h X B_w^T  (dct_2d, dct.rs:282-308):
//            U' = B_w (X 2^e)^T     (A = B_w,   Bt = X:  M = w, N = h, K = w)
//            C  = 2^-e B_h U'^T     (A = B_h,   Bt = U': M = h, N = w, K = h)
// where 2^e is chosen from max |input| so that every f16 operand stays far
// from overflow (|T'|, |U'| <= max|input 2^e| sqrt(w) <= 2^14).
//
// Kernel.  A workgroup of 8 waves computes a 256 x 256 tile of D, each wave
// a 128 x 64 part as 4 x 2 blocks of v_mfma_f32_32x32x16_f16.  K runs in
// steps of 16 through a ring of four 32 KiB LDS stages.  The operands go
// from global memory straight into LDS (global_load_lds_dwordx4: lane l of
// a load writes LDS bytes [16 l, 16 l + 16) of the wave's destination), in
// MFMA fragment order (block of 32 rows, lane), so a fragment is one linear
// 16-byte ds_read per lane and no register holds staged data.  The loads of
// step s + 3 are issued at step s, into the stage step s - 1 used; before
// step s each wave waits only until its loads of step s have landed (the
// later two steps stay in flight) and one barrier makes everyone's
// visible.  Tiles are numbered in groups of 4 tile rows and each of the 8
// XCDs (which take workgroups round robin) is given a contiguous run of tile
// numbers, so the workgroups on one XCD share A and Bt panels in its L2.
#include "hh_internal.hpp"

namespace hh {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define HH_GLOBAL __attribute__((address_space(1)))
#define HH_LDS __attribute__((address_space(3)))

constexpr uint32_t kTile = 256;          // rows of A and of Bt per tile
constexpr uint32_t kBK = 16;             // k per step
constexpr uint32_t kThreads = 512;
constexpr uint32_t kBlock = 64 * 16;     // one fragment block: 64 lanes x 16 bytes
constexpr uint32_t kPlane = 8 * kBlock;  // 8 row blocks of 32 rows: 8 KiB
constexpr uint32_t kStage = 4 * kPlane;  // A hi, A lo, B hi, B lo
constexpr uint32_t kStages = 4;
constexpr uint32_t kAhead = kStages - 1; // steps whose loads are in flight
constexpr uint32_t kLds = kStages * kStage;  // 128 KiB
constexpr uint32_t kGroupRows = 4;       // tile rows per group of the tile order

__device__ __forceinline__ floatx16 mfma(u32x4 a, u32x4 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c,
                                                  0, 0, 0);
}

// s_waitcnt for the vector memory counter only: at most n (< 64) of this
// wave's vector memory operations outstanding (gfx9 encoding: vmcnt bits
// 3:0 and 15:14; expcnt 7 and lgkmcnt 15 do not wait).
template <uint32_t N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((int)((N & 15u) | (7u << 4) | (15u << 8) | ((N >> 4) << 14)));
}

// s_waitcnt lgkmcnt(0) alone (vmcnt 63 and expcnt 7 do not wait).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt((int)(15u | (7u << 4) | (3u << 14))); }

struct GemmArgs {
    const uint16_t *a_hi, *a_lo;  // planes, row stride lda halves
    const uint16_t *b_hi, *b_lo;  // planes, row stride ldb halves; b_lo null: no low half
    uint32_t lda, ldb;
    const float *out_scale;       // device scalar, or null for 1
    void *d;                      // output; planes: hi then lo, d_plane elements apart
    uint64_t d_plane;
    uint32_t ldd;
    uint32_t d_rows, d_cols;      // extent written (planes: the padded extent)
    uint32_t ksteps;
    uint32_t tiles_m, tiles_n;
    uint32_t m_split, b_koff;     // tiles at m0 >= m_split (when not 0) read Bt from column b_koff
};

// OUT: HH_F32 / HH_F16 / HH_BF16, or kOutPlanes (f16 hi / lo planes).
constexpr int kOutPlanes = 100;

template <bool BLO, int OUT>
__global__ __launch_bounds__(kThreads, 1) void dct_gemm_kernel(GemmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave >> 2, wn = wave & 3u;  // wave rows [128 wm, +128), cols [64 wn, +64)

    // tile of this workgroup
    const uint32_t total = g.tiles_m * g.tiles_n;
    uint32_t t = blockIdx.x;
    if ((total & 7u) == 0) t = (blockIdx.x & 7u) * (total >> 3) + (blockIdx.x >> 3);
    const uint32_t per_group = kGroupRows * g.tiles_n;
    const uint32_t grp = t / per_group, in_grp = t % per_group;
    const uint32_t rows_here = min(kGroupRows, g.tiles_m - kGroupRows * grp);
    const uint32_t m0 = (kGroupRows * grp + in_grp % rows_here) * kTile, n0 = (in_grp / rows_here) * kTile;

    // this wave's loads per step: blocks q = kPerWave wave + i of (plane, row
    // block); lane l of a block reads row 32 rb + l % 32 at k 8 (l / 32)
    constexpr uint32_t kPlanes = BLO ? 4u : 3u;
    constexpr uint32_t kPerWave = kPlanes * 8u / 8u;  // 4 or 3
    const uint16_t *src[kPerWave];
    uint32_t dst[kPerWave];
#pragma unroll
    for (uint32_t i = 0; i < kPerWave; i++) {
        const uint32_t q = kPerWave * wave + i;
        const uint32_t p = q >> 3, rb = q & 7u;
        const uint32_t row = 32u * rb + (lane & 31u), k = 8u * (lane >> 5);
        const uint16_t *base = p == 0 ? g.a_hi : p == 1 ? g.a_lo : p == 2 ? g.b_hi : g.b_lo;
        const uint32_t ld = p < 2 ? g.lda : g.ldb;
        const uint32_t r0 = p < 2 ? m0 : n0;
        const uint32_t koff = p >= 2 && g.m_split != 0u && m0 >= g.m_split ? g.b_koff : 0u;
        src[i] = base + (size_t)(r0 + row) * ld + k + koff;
        dst[i] = p * kPlane + rb * kBlock;
    }
    auto issue = [&](uint32_t step) {
        const uint32_t st = step % kStages;
#pragma unroll
        for (uint32_t i = 0; i < kPerWave; i++)
            __builtin_amdgcn_global_load_lds((const void HH_GLOBAL *)(src[i] + (size_t)step * kBK),
                                             (void HH_LDS *)(smem + st * kStage + dst[i]), 16, 0, 0);
    };

    float so = g.out_scale ? *g.out_scale : 1.0f;

    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = floatx16{};

    for (uint32_t i = 0; i < kAhead && i < g.ksteps; i++) issue(i);
    for (uint32_t s = 0; s < g.ksteps; s++) {
        // this wave's loads of step s have landed when at most those of the
        // steps after it (up to kAhead - 1 of them) are outstanding
        const uint32_t later = min(g.ksteps - 1u - s, kAhead - 1u);
        if (later >= 2)
            wait_vm<2 * kPerWave>();
        else if (later == 1)
            wait_vm<kPerWave>();
        else
            wait_vm<0>();
        // everyone's loads of step s are visible, and everyone has finished
        // reading the stage of step s - 1, which the loads of step s + 3 fill
        // (a bare barrier: a workgroup fence would also wait for the loads
        // still in flight; the empty asm keeps the compiler from moving LDS
        // accesses across it)
        wait_lgkm0();
        __asm__ __volatile__("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ __volatile__("" ::: "memory");
        if (s + kAhead < g.ksteps) issue(s + kAhead);
        const uint8_t *base = smem + (s % kStages) * kStage;
        u32x4 ah[4], al[4], bh[2], bl[2];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t o = (4u * wm + i) * kBlock + 16u * lane;
            ah[i] = *reinterpret_cast<const u32x4 *>(base + 0 * kPlane + o);
            al[i] = *reinterpret_cast<const u32x4 *>(base + 1 * kPlane + o);
        }
#pragma unroll
        for (uint32_t j = 0; j < 2; j++) {
            const uint32_t o = (2u * wn + j) * kBlock + 16u * lane;
            bh[j] = *reinterpret_cast<const u32x4 *>(base + 2 * kPlane + o);
            if constexpr (BLO) bl[j] = *reinterpret_cast<const u32x4 *>(base + 3 * kPlane + o);
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; i++)
#pragma unroll
            for (uint32_t j = 0; j < 2; j++) {
                acc[i][j] = mfma(ah[i], bh[j], acc[i][j]);
                acc[i][j] = mfma(al[i], bh[j], acc[i][j]);
                if constexpr (BLO) acc[i][j] = mfma(ah[i], bl[j], acc[i][j]);
            }
    }

    // epilogue: lane l holds column n = l % 32 of each block, register r row
    // (r & 3) + 8 (r >> 2) + 4 (l / 32).  The scale was loaded before the
    // loop; taking it here once keeps the stores below free of waits (a wait
    // for it inside a guarded store would also wait for every earlier store).
    __asm__ __volatile__("" : "+v"(so));
    const uint32_t hf = lane >> 5, c = lane & 31u;
    const bool full = m0 + kTile <= g.d_rows && n0 + kTile <= g.d_cols;
    auto put = [&](uint32_t m, uint32_t n, float a) {
        const float v = a * so;
        const size_t o = (size_t)m * g.ldd + n;
        if constexpr (OUT == HH_F32) {
            reinterpret_cast<float *>(g.d)[o] = v;
        } else if constexpr (OUT == kOutPlanes) {
            const _Float16 h = (_Float16)v;
            const _Float16 l = (_Float16)(v - (float)h);
            reinterpret_cast<_Float16 *>(g.d)[o] = h;
            reinterpret_cast<_Float16 *>(g.d)[o + g.d_plane] = l;
        } else {
            reinterpret_cast<uint16_t *>(g.d)[o] =
                (uint16_t)(OUT == HH_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
        }
    };
#pragma unroll
    for (uint32_t i = 0; i < 4; i++)
#pragma unroll
        for (uint32_t j = 0; j < 2; j++) {
            const uint32_t n = n0 + 64u * wn + 32u * j + c;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t m = m0 + 128u * wm + 32u * i + (r & 3) + 8 * (r >> 2) + 4 * hf;
                if (full || (m < g.d_rows && n < g.d_cols)) put(m, n, acc[i][j][r]);
            }
        }
}

// Basis planes: P[m][k] = split(B_n[k][m]) (transposed) or split(B_n[m][k]),
// for m < Mp (rows past n zero) and k < Kp (columns past n zero).
__global__ __launch_bounds__(256) void basis_planes_kernel(uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                           uint32_t n, uint32_t Mp, uint32_t Kp, int transposed) {
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)Mp * Kp) return;
    const uint32_t m = (uint32_t)(idx / Kp), k = (uint32_t)(idx % Kp);
    double b = 0.0;
    if (m < n && k < n) {
        // B_n[f][i] with the argument reduced exactly in integers
        const uint32_t f = transposed ? k : m, i = transposed ? m : k;
        const uint64_t q = ((uint64_t)f * (2ull * i + 1ull)) % (4ull * n);
        const double sf = f == 0 ? sqrt(1.0 / (double)n) : sqrt(2.0 / (double)n);
        b = sf * cospi((double)q / (2.0 * (double)n));
    }
    const _Float16 h = (_Float16)b;
    const _Float16 l = (_Float16)(b - (double)h);
    hi[idx] = __builtin_bit_cast(uint16_t, h);
    lo[idx] = __builtin_bit_cast(uint16_t, l);
}

// An f32 rows x cols matrix (row stride ld) times *scale as f16 planes of
// Rp x Kp (zeros past rows / cols); lo may be null (the high half only).
__global__ __launch_bounds__(256) void operand_planes_kernel(const float *__restrict__ x, uint32_t rows,
                                                             uint32_t cols, uint32_t ld,
                                                             const float *__restrict__ scale,
                                                             _Float16 *__restrict__ hi, _Float16 *__restrict__ lo,
                                                             uint32_t Rp, uint32_t Kp) {
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)Rp * Kp) return;
    const uint32_t r = (uint32_t)(idx / Kp), k = (uint32_t)(idx % Kp);
    const float v = (r < rows && k < cols) ? x[(size_t)r * ld + k] * *scale : 0.0f;
    const _Float16 h = (_Float16)v;
    hi[idx] = h;
    if (lo) lo[idx] = (_Float16)(v - (float)h);
}

// The even / odd split of B_n^T: P[m][k] = B_n[2k + (m >= n/2)][m mod n/2],
// an n x n/2 plane pair (n a multiple of 512: no padding).
__global__ __launch_bounds__(256) void basis_split_planes_kernel(uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                                 uint32_t n) {
    const uint32_t nh = n / 2;
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)n * nh) return;
    const uint32_t m = (uint32_t)(idx / nh), k = (uint32_t)(idx % nh);
    const uint32_t f = 2u * k + (m >= nh ? 1u : 0u), i = m % nh;
    const uint64_t q = ((uint64_t)f * (2ull * i + 1ull)) % (4ull * n);
    const double sf = f == 0 ? sqrt(1.0 / (double)n) : sqrt(2.0 / (double)n);
    const double b = sf * cospi((double)q / (2.0 * (double)n));
    const _Float16 h = (_Float16)b;
    const _Float16 l = (_Float16)(b - (double)h);
    hi[idx] = __builtin_bit_cast(uint16_t, h);
    lo[idx] = __builtin_bit_cast(uint16_t, l);
}

// operand_planes_kernel with the columns in even / odd order: column k of
// the matrix goes to k / 2, or cols / 2 + k / 2 when odd (cols even, rows
// padded to Rp with zeros).  Each thread takes two adjacent columns.
__global__ __launch_bounds__(256) void operand_planes_eo_kernel(const float *__restrict__ x, uint32_t rows,
                                                                uint32_t cols, uint32_t ld,
                                                                const float *__restrict__ scale,
                                                                _Float16 *__restrict__ hi, _Float16 *__restrict__ lo,
                                                                uint32_t Rp) {
    const uint32_t ch = cols / 2;
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)Rp * ch) return;
    const uint32_t r = (uint32_t)(idx / ch), k2 = (uint32_t)(idx % ch);
    float ve = 0.0f, vo = 0.0f;
    if (r < rows) {
        const float sc = *scale;
        ve = x[(size_t)r * ld + 2u * k2] * sc;
        vo = x[(size_t)r * ld + 2u * k2 + 1u] * sc;
    }
    const size_t oe = (size_t)r * cols + k2, oo = oe + ch;
    const _Float16 he = (_Float16)ve, ho = (_Float16)vo;
    hi[oe] = he;
    hi[oo] = ho;
    if (lo) {
        lo[oe] = (_Float16)(ve - (float)he);
        lo[oo] = (_Float16)(vo - (float)ho);
    }
}

// The butterfly of an even / odd split product (see launch_dct_butterfly);
// each thread takes four adjacent columns of one row pair.
template <int OUT>
__global__ __launch_bounds__(256) void butterfly_kernel(const float *__restrict__ y, uint32_t mh, uint32_t n,
                                                        const float *__restrict__ scale, void *__restrict__ out,
                                                        uint32_t ldd) {
    const uint32_t nq = n / 4;
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)mh * nq) return;
    const uint32_t m = (uint32_t)(idx / nq), c = 4u * (uint32_t)(idx % nq);
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 e = *reinterpret_cast<const f4 *>(y + (size_t)m * n + c);
    const f4 o = *reinterpret_cast<const f4 *>(y + (size_t)(mh + m) * n + c);
    const uint32_t m2 = 2u * mh - 1u - m;
    if constexpr (OUT == kOutPlanes) {
        // columns c, c + 2 -> c / 2, c / 2 + 1; c + 1, c + 3 -> n/2 + the same
        const f4 a = e + o, b = e - o;
        _Float16 *hi = reinterpret_cast<_Float16 *>(out), *lo = hi + (size_t)2 * mh * n;
        const uint32_t ce = c / 2, co = n / 2 + c / 2;
        auto put2 = [&](uint32_t row, float v0, float v1, uint32_t col) {
            const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
            const size_t o2 = (size_t)row * n + col;
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            *reinterpret_cast<h2 *>(hi + o2) = h2{h0, h1};
            *reinterpret_cast<h2 *>(lo + o2) = h2{(_Float16)(v0 - (float)h0), (_Float16)(v1 - (float)h1)};
        };
        put2(m, a[0], a[2], ce);
        put2(m, a[1], a[3], co);
        put2(m2, b[0], b[2], ce);
        put2(m2, b[1], b[3], co);
    } else {
        const float sc = scale ? *scale : 1.0f;
        const f4 a = (e + o) * sc, b = (e - o) * sc;
        if constexpr (OUT == HH_F32) {
            *reinterpret_cast<f4 *>(reinterpret_cast<float *>(out) + (size_t)m * ldd + c) = a;
            *reinterpret_cast<f4 *>(reinterpret_cast<float *>(out) + (size_t)m2 * ldd + c) = b;
        } else {
            typedef uint16_t u4 __attribute__((ext_vector_type(4)));
            auto cv = [](float v) { return (uint16_t)(OUT == HH_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v)); };
            *reinterpret_cast<u4 *>(reinterpret_cast<uint16_t *>(out) + (size_t)m * ldd + c) =
                u4{cv(a[0]), cv(a[1]), cv(a[2]), cv(a[3])};
            *reinterpret_cast<u4 *>(reinterpret_cast<uint16_t *>(out) + (size_t)m2 * ldd + c) =
                u4{cv(b[0]), cv(b[1]), cv(b[2]), cv(b[3])};
        }
    }
}

template <bool BLO, int OUT>
hipError_t launch_one(const GemmArgs &g, hipStream_t s) {
    hipError_t e = hipFuncSetAttribute((const void *)dct_gemm_kernel<BLO, OUT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((dct_gemm_kernel<BLO, OUT>), dim3(g.tiles_m * g.tiles_n), dim3(kThreads), kLds, s, g);
    return hipGetLastError();
}

}  // namespace

uint32_t dct_planes_rows(uint32_t n) { return (n + kTile - 1) / kTile * kTile; }
uint32_t dct_planes_cols(uint32_t n) { return (n + kBK - 1) / kBK * kBK; }

hipError_t launch_dct_basis_planes(uint16_t *hi, uint16_t *lo, uint32_t n, bool transposed, hipStream_t s) {
    const uint32_t Mp = dct_planes_rows(n), Kp = dct_planes_cols(n);
    const uint64_t total = (uint64_t)Mp * Kp;
    hipLaunchKernelGGL(basis_planes_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, hi, lo, n, Mp,
                       Kp, transposed ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_operand_planes(const float *x, uint32_t rows, uint32_t cols, uint32_t ld, const float *scale,
                                 uint16_t *hi, uint16_t *lo, hipStream_t s) {
    const uint32_t Rp = dct_planes_rows(rows), Kp = dct_planes_cols(cols);
    const uint64_t total = (uint64_t)Rp * Kp;
    hipLaunchKernelGGL(operand_planes_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, x, rows, cols,
                       ld, scale, reinterpret_cast<_Float16 *>(hi), reinterpret_cast<_Float16 *>(lo), Rp, Kp);
    return hipGetLastError();
}

hipError_t launch_dct_basis_split_planes(uint16_t *hi, uint16_t *lo, uint32_t n, hipStream_t s) {
    const uint64_t total = (uint64_t)n * (n / 2);
    hipLaunchKernelGGL(basis_split_planes_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, hi, lo, n);
    return hipGetLastError();
}

hipError_t launch_operand_planes_eo(const float *x, uint32_t rows, uint32_t cols, uint32_t ld, const float *scale,
                                    uint16_t *hi, uint16_t *lo, hipStream_t s) {
    const uint32_t Rp = dct_planes_rows(rows);
    const uint64_t total = (uint64_t)Rp * (cols / 2);
    hipLaunchKernelGGL(operand_planes_eo_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, x, rows,
                       cols, ld, scale, reinterpret_cast<_Float16 *>(hi), reinterpret_cast<_Float16 *>(lo), Rp);
    return hipGetLastError();
}

hipError_t launch_dct_butterfly(const float *y, uint32_t mh, uint32_t n, bool eo_planes, const float *scale,
                                int32_t dtype, void *out, uint32_t ldd, hipStream_t s) {
    const uint64_t total = (uint64_t)mh * (n / 4);
    const dim3 grid((uint32_t)((total + 255) / 256));
    if (eo_planes)
        hipLaunchKernelGGL(butterfly_kernel<kOutPlanes>, grid, dim3(256), 0, s, y, mh, n, scale, out, ldd);
    else if (dtype == HH_F32)
        hipLaunchKernelGGL(butterfly_kernel<HH_F32>, grid, dim3(256), 0, s, y, mh, n, scale, out, ldd);
    else if (dtype == HH_F16)
        hipLaunchKernelGGL(butterfly_kernel<HH_F16>, grid, dim3(256), 0, s, y, mh, n, scale, out, ldd);
    else if (dtype == HH_BF16)
        hipLaunchKernelGGL(butterfly_kernel<HH_BF16>, grid, dim3(256), 0, s, y, mh, n, scale, out, ldd);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_dct_gemm(const DctGemm &p, hipStream_t s) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    GemmArgs g;
    g.a_hi = p.a_hi;
    g.a_lo = p.a_lo;
    g.b_hi = p.b_hi;
    g.b_lo = p.b_lo;
    g.lda = p.lda ? p.lda : dct_planes_cols(p.K);
    g.ldb = p.ldb ? p.ldb : dct_planes_cols(p.K);
    g.m_split = p.m_split;
    g.b_koff = p.b_koff;
    g.out_scale = p.out_scale;
    g.d = p.d;
    g.tiles_m = (p.M + kTile - 1) / kTile;
    g.tiles_n = (p.N + kTile - 1) / kTile;
    g.ksteps = dct_planes_cols(p.K) / kBK;
    if (p.d_planes) {
        // the planes of the next product's Bt: its padded extent, zeros included
        g.ldd = dct_planes_cols(p.N);
        g.d_rows = dct_planes_rows(p.M);
        g.d_cols = g.ldd;
        g.d_plane = (uint64_t)g.d_rows * g.ldd;
        return p.b_lo ? launch_one<true, kOutPlanes>(g, s) : launch_one<false, kOutPlanes>(g, s);
    }
    g.ldd = p.ldd;
    g.d_rows = p.M;
    g.d_cols = p.N;
    g.d_plane = 0;
    switch (p.d_dtype) {
        case HH_F32: return p.b_lo ? launch_one<true, HH_F32>(g, s) : launch_one<false, HH_F32>(g, s);
        case HH_F16: return p.b_lo ? launch_one<true, HH_F16>(g, s) : launch_one<false, HH_F16>(g, s);
        case HH_BF16: return p.b_lo ? launch_one<true, HH_BF16>(g, s) : launch_one<false, HH_BF16>(g, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hh
