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
//   GEMM1  S = C M     (A = C, gathered into registers; B = M)
//   GEMM2  X = M^T S   (A = M^T; B = S straight from GEMM1's accumulators)
// The contraction index of both GEMMs runs in the order
//   pi(16 s + 8 h + e) = 16 s + 8 (e / 4) + 4 h + e % 4
// (k step s, lane half h, element e), which is exactly the row order of the
// 32x32 accumulator layout, so GEMM1's output registers are GEMM2's B
// fragments without any shuffle or LDS trip, and one table of M fragments
// serves as GEMM1's B and GEMM2's A.
//
// Precision.  Each retained coefficient (q - 8) * scale is held exactly as
// an f16 pair hi + lo (the scale split into its top 8 and low 3 significant
// bits, each product with q - 8 exact), and GEMM1 runs three passes
// hi*hi + hi*lo + lo*hi against M = M_hi + M_lo (the dropped lo*lo is below
// 2^-8 * 2^-11 = 2^-19 relative).  GEMM1's output S is split the same way by
// rounding (S_hi = f16(S), S_lo = f16(S - S_hi)) and GEMM2 runs three
// passes (the dropped S_lo * M_lo is ~2^-24 relative).  Accumulation is
// f32; the max-abs error is ~4e-6 x RMS against a bar of 1e-3 x RMS (each
// MFMA pass costs about as much as a tenth of the tile's vector work, so
// the fourth GEMM1 pass, worth ~2e-6 x RMS, is left out).  Coefficients are prescaled
// by 2^E per tile (E from the largest f16 scale exponent, so that
// |C 2^E| < 4) and M by 2^8, which puts GEMM1's output directly in the
// range of GEMM2's f16 operands; only scales below ~2^-12 of the tile's
// largest lose low bits to f16 subnormals.  The output is rescaled exactly.
//
// Data flow per tile (per wave):
//   1. each lane reads one 64-bit bitmap row; a wave prefix sum gives every
//      row's first retained index;
//   2. the k retained coefficients are dequantized once, in index order, into
//      a per-wave LDS table V[r] = f16 hi | f16 lo << 16;
//   3. every lane gathers its GEMM1 A fragments (2 rows x 32 columns) from V
//      by bitmap rank, branch-free (unset positions read a zero word);
//   4. GEMM1 / GEMM2 per 32-column block; the M fragments live in LDS, shared
//      by the workgroup;
//   5. the output block is parked in LDS (reusing V's space) and written as
//      coalesced 16-byte row segments.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "hh_internal.hpp"
#include "lz4_ring.hpp"
#include "lz4_seq.hpp"

namespace hh {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Global-address-space views.  Pointers read from LDS are generic; memory
// operations through them would be flat instructions, whose completion also
// counts against the LDS wait counter.
#define HH_GLOBAL __attribute__((address_space(1)))
typedef const uint8_t HH_GLOBAL g_u8;
typedef const u32x4 HH_GLOBAL g_u32x4;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kMTabBytes = 2 * 2 * 2 * 64 * 16;  // [hl][parity][kstep][lane] x 16 B
constexpr uint32_t kZeroBytes = 16;

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A wave-uniform value (read from LDS, say) moved to scalar registers, so
// that addresses built from it are scalar bases.
__device__ __forceinline__ uint64_t uniform(uint64_t v) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
}
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

__device__ __forceinline__ floatx16 mfma(u32x4 a, u32x4 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

__device__ __forceinline__ float pow2f(int e) {  // e in [-126, 127]
    return __uint_as_float((uint32_t)(e + 127) << 23);
}

// Inclusive prefix sum over the 64 lanes with DPP row shifts (1, 2, 4, 8
// within each row of 16 lanes) and the row broadcasts of lanes 15 and 31;
// lanes whose source lies outside the row keep the 0 passed as `old`.
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
    return v;
}

// Largest value of a 5-bit field over the wave (wave-uniform): a binary
// search on ballots, one bit at a time from the top.
__device__ __forceinline__ uint32_t wave_max_u5(uint32_t v) {
    uint32_t m = 0;
#pragma unroll
    for (int b = 4; b >= 0; b--) {
        const uint32_t c = m | (1u << b);
        if (__builtin_amdgcn_ballot_w64(v >= c) != 0) m = c;
    }
    return m;
}

// (a, b) -> f16 hi pair and f16 lo pair with a = hi.x + lo.x, b = hi.y + lo.y
// to ~2^-20 relative (exactly when a, b have at most 21 significant bits):
// lo = round_f16(a * one - hi), where a - hi is exact in f32.  `one` is 1.0
// passed in at run time, so the compiler keeps the FMA and selects the
// mixed-precision FMAs (v_fma_mixlo/hi_f16, one instruction per lo half)
// itself; it then also inserts the wait states an MFMA needs before reading
// their results (inline assembly would hide those writes from it).
__device__ __forceinline__ void split2(float a, float b, float one, uint32_t &hi, uint32_t &lo) {
    const half2v h = __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a, b));
    const half2v l = {(_Float16)__builtin_fmaf(a, one, -(float)h.x), (_Float16)__builtin_fmaf(b, one, -(float)h.y)};
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, l);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef u32x4 __attribute__((address_space(3))) lds_u32x4;
typedef u32x2 __attribute__((address_space(3))) lds_u32x2;

// Row pitch of the parked output tile in LDS: 64 values plus 8 (16-bit) or
// 4 (f32) values of padding, so that the 32 rows written by one instruction
// fall into distinct banks.
template <int DT>
constexpr uint32_t kParkPitch = DT == HH_F32 ? 64u * 4u + 16u : 64u * 2u + 8u;
// The same for one 32-column block of the tile.
template <int DT>
constexpr uint32_t kHalfPitch = DT == HH_F32 ? 32u * 4u + 16u : 32u * 2u + 8u;

// Two outputs rounded to the 16-bit output type, packed low | high.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (DT == HH_BF16) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{a, b}, bf16x2));
    } else {
        // keep the f32 values as such: a fused fma -> f16 (v_fma_mix) would
        // round once from the exact result, not from the f32 output
        __asm__("" : "+v"(a), "+v"(b));
        return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
    }
}

// LDS read at an absolute LDS byte address, used as an LDS pointer as is
// (no base is added to it).
typedef const uint32_t __attribute__((address_space(3))) lds_u32;
__device__ __forceinline__ uint32_t lds_load(uint32_t a) { return *(lds_u32 *)(size_t)a; }

// Up to kMaxTensors tensors per launch, passed by value as kernel arguments.
// Tiles are numbered across the batch; tensor i owns [start[i], start[i+1]).
constexpr int kMaxTensors = 32;
static_assert((kMaxTensors & (kMaxTensors - 1)) == 0 && kMaxTensors <= 64, "tensor_of reads one start per lane");
// Waves per SIMD the tile kernel is compiled for: 3 for 16-bit outputs with
// at most 2 KiB of tile bytes prefetched (168 registers, no spills; the LDS
// also fits 3 workgroups per CU), else 2.
constexpr int kWavesPerSimd(int dt, int np) { return dt != HH_F32 && np == 2 ? 3 : 2; }
struct TileBatch {
    const uint8_t *tiles[kMaxTensors];
    void *out[kMaxTensors];
    int32_t *status[kMaxTensors];
    uint32_t start[kMaxTensors + 1];
    float tpr_inv[kMaxTensors];  // 64 / cols (1 / tiles per row), rounded to f32 on the host
    uint32_t cols[kMaxTensors];
    uint32_t k[kMaxTensors];
    uint32_t tb[kMaxTensors];
    uint32_t n;
    uint32_t wave_lds;  // per-wave LDS bytes: V/output union + staged tile bytes
    uint32_t vo_bytes;  // size of the V/output union
    float one;          // 1.0 and -4, as run-time values (see split2 and the gather)
    int32_t neg4;
};

// The tensor holding batch tile gt (wave-uniform; every lane active): the
// count of tensor starts after the first at or below gt.  The starts ascend,
// start[n] is the tile total and the unused ones past it are all-ones, so no
// start past tensor n - 1 counts.  Lane j compares start[j]: one LDS read
// and a ballot.
__device__ __forceinline__ uint32_t tensor_of(const TileBatch &B, uint32_t gt, int lane) {
    const uint32_t s = B.start[lane & (kMaxTensors - 1)];
    return (uint32_t)__popcll(__builtin_amdgcn_ballot_w64(gt >= s) & (((1ull << kMaxTensors) - 1ull) & ~1ull));
}

// Workgroup LDS layout: [zero word][batch descriptor][M fragment table][per-wave areas].
// The zero word sits at LDS address 0, so a gathered address masked to 0
// reads zeros.  The descriptor is copied from the kernel arguments once:
// indexing the by-value argument with a per-tile tensor index would compile
// to vector loads whose waits also stall on the prefetch and the output
// stores.
constexpr uint32_t kZeroOff = 0;
constexpr uint32_t kBatchOff = kZeroBytes;
constexpr uint32_t kBatchBytes = (sizeof(TileBatch) + 15u) & ~15u;
constexpr uint32_t kMTabOff = kBatchOff + kBatchBytes;
constexpr uint32_t kSharedBytes = kMTabOff + kMTabBytes;

// Loads the bytes of global tile gt (of tensor ti) into registers, 16 bytes per lane per
// KiB, always issuing NP loads (NP KiB cover the tile) so that the wait
// counts stay static.  DW: every tile of the batch starts 4-byte aligned and
// has a size divisible by 4; register chunk i holds tile bytes
// [16*(lane + 64 i), +16) wherever those lie inside the tile (chunks past the
// tile end re-read its last 16 bytes).  Otherwise chunk i holds the bytes
// from 16*(lane + 64 i) on counted from the tile start rounded down to 4
// bytes (staged as is, the tile then starts at byte tile_shift of the
// staging area): 16-byte loads at 4-byte alignment wherever the chunk lies
// inside the tensor's tile bytes, bytes one by one where it would leave them
// (the tensor's first and last chunks), anything for chunks past the tile.
template <bool DW, int NP>
__device__ __forceinline__ void prefetch_tile(const TileBatch &B, uint32_t gt, uint32_t ti, int lane,
                                              u32x4 (&pf)[NP]) {
    const uint32_t tb = uniform(B.tb[ti]), st = uniform(B.start[ti]), sn = uniform(B.start[ti + 1]);
    const uint64_t s0 = uniform((uint64_t)(uintptr_t)B.tiles[ti]);
    g_u8 *src = (g_u8 *)(uintptr_t)s0 + (size_t)(gt - st) * tb;
    {
        // every chunk inside the tensor's tile bytes (all but its first and
        // last tiles, usually): scalar base + 32-bit lane offset, no
        // per-lane checks.  The chunks hold what both forms below hold
        // inside the tile; past its end, don't-care bytes.
        const uint64_t e0 = s0 + (uint64_t)(sn - st) * tb;
        const uint64_t a0 = (uint64_t)(uintptr_t)src & ~(uint64_t)3;
        if (a0 >= s0 && a0 + 1024u * NP <= e0) {
#pragma unroll
            for (int i = 0; i < NP; i++) pf[i] = *(g_u32x4 *)((g_u8 *)(uintptr_t)a0 + 16u * (lane + 64u * i));
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const uint32_t off = 16u * (lane + 64u * i);
        if constexpr (!DW) {
            const uintptr_t e0 = (uintptr_t)s0 + (size_t)(sn - st) * tb;  // >= s0 + 515
            const uintptr_t ts = (uintptr_t)src;
            const uintptr_t a = (ts & ~(uintptr_t)3) + off;
            if (a >= s0 && a + 16 <= e0) {
                pf[i] = *(g_u32x4 *)a;
            } else if (a < ts + tb) {
                uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll 1
                for (int b = 0; b < 16; b++)
                    if (a + b >= s0 && a + b < ts + tb) d[b >> 2] |= (uint32_t)((g_u8 *)(a + b))[0] << (8 * (b & 3));
                pf[i] = u32x4{d[0], d[1], d[2], d[3]};
            } else {
                pf[i] = *(g_u32x4 *)((e0 - 16) & ~(uintptr_t)3);  // not used
            }
        } else {
            // A chunk reaching past the tile end is read at tb - 16 (tiles
            // are >= 515 bytes) and shifted down by s dwords so that byte
            // off lands first; dwords beyond the tile end are don't-care.
            const uint32_t o = off + 16 <= tb ? off : tb - 16;
            const u32x4 v = *(g_u32x4 *)(src + o);
            const uint32_t s = (off - o) >> 2;
            const uint32_t d0 = s == 0 ? v[0] : s == 1 ? v[1] : s == 2 ? v[2] : v[3];
            const uint32_t d1 = s == 0 ? v[1] : s == 1 ? v[2] : v[3];
            const uint32_t d2 = s == 0 ? v[2] : v[3];
            pf[i] = u32x4{d0, d1, d2, v[3]};
        }
    }
}

// Byte offset of global tile gt's first byte in the staging area that
// prefetch_tile<false> fills (its address mod 4); 0 for DW.
template <bool DW>
__device__ __forceinline__ uint32_t tile_shift(const TileBatch &B, uint32_t ti, uint32_t t) {
    if constexpr (DW) return 0u;
    return (uint32_t)(((uintptr_t)B.tiles[ti] + (size_t)t * B.tb[ti]) & 3u);
}

// One tile from its bytes in LDS (`pay`): steps 1-8 of the data flow above,
// with this wave's V table / output park at LDS byte offset wbase (V is the
// same area as a pointer).  `consumed` runs once the tile's bytes are no
// longer read: right after the V table is built (HALF), or just before the
// output stores (whole-tile park; EARLY: right after the V table there too).
// PRIO raises the wave's issue priority over the two products (the tile
// kernel, where every wave decodes tiles; not the fused kernel, whose LZ4
// waves would then starve).
template <int DT, bool HALF, bool EARLY = false, bool PRIO = false, typename Hook>
__device__ __forceinline__ void tile_body(const TileBatch &B, uint32_t ti, uint32_t t, const uint8_t *pay,
                                          uint32_t *V, uint32_t wbase, const u32x4 *mtab, int lane, float one,
                                          int32_t n4, Hook &&consumed) {
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const uint32_t k = uniform(B.k[ti]), cols = uniform(B.cols[ti]);
    const uint32_t nsc = (k + 31) >> 5;
    const uint32_t nib_off = 512 + 2 * nsc;

    // 1. bitmap row `lane`: set-bit count and exclusive prefix over rows
    const uint64_t bits = reinterpret_cast<const uint64_t *>(pay)[lane];
    const uint32_t cnt = (uint32_t)__popcll(bits);
    const uint32_t incl = wave_incl_sum(cnt);
    const bool ok = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63) == k;
    const uint32_t pre = incl - cnt;

    // 2. per-tile power-of-two prescale from the largest scale exponent
    const uint16_t *sc16 = reinterpret_cast<const uint16_t *>(pay + 512);
    uint32_t emax = 0;
    for (uint32_t g = lane; g < nsc; g += 64) {
        const uint32_t ex = ((uint32_t)sc16[g] >> 10) & 31u;
        emax = ex > emax ? ex : emax;
    }
    emax = wave_max_u5(emax);
    // coefficients are scaled by 2^E (|C 2^E| < 4); the basis carries 2^8
    const int E = 13 - (int)emax;
    const float pe = pow2f(E);

    // 3. dense table of the retained coefficients, 8 per lane per pass:
    //    V[r] = hi | lo << 16 with hi + lo = (q_r - 8) * scale * 2^E
    //    exactly.  The scaled scale s = scale * 2^E (11 significant bits)
    //    is split into s_hi (its top 8 bits) + s_lo (the other 3); with
    //    |q - 8| <= 8 (at most 3 significant bits) both (q - 8) s_hi and
    //    (q - 8) s_lo are exact f16 products, formed two at a time by
    //    packed f16 multiplies.
    if (ok) {
        const uint16_t *nib16 = reinterpret_cast<const uint16_t *>(pay + nib_off);
        for (uint32_t c8 = lane; 8 * c8 < k; c8 += 64) {
            const uint32_t r0 = 8 * c8;
            // nibbles r0 .. r0+7, low first (bytes past the tile's end
            // are staged slack; their entries lie past V[k - 1])
            const uint32_t n32 = (uint32_t)nib16[2 * c8] | ((uint32_t)nib16[2 * c8 + 1] << 16);
            const float sf = (float)__builtin_bit_cast(_Float16, sc16[r0 >> 5]) * pe;
            const float shi = __uint_as_float(__float_as_uint(sf) & 0xffff0000u);
            const half2v sc = __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(shi, sf - shi));
            uint32_t v[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                // f16 (1024 + q) for nibbles e and e + 4, minus 1032
                const uint32_t y = ((n32 >> (4 * e)) & 0x000f000fu) | 0x64006400u;
                const half2v q = __builtin_bit_cast(half2v, y) - half2v{(_Float16)1032.0f, (_Float16)1032.0f};
                v[e] = __builtin_bit_cast(uint32_t, half2v{q.x, q.x} * sc);
                v[e + 4] = __builtin_bit_cast(uint32_t, half2v{q.y, q.y} * sc);
            }
            u32x4 *dst = reinterpret_cast<u32x4 *>(V + r0);
            dst[0] = u32x4{v[0], v[1], v[2], v[3]};
            dst[1] = u32x4{v[4], v[5], v[6], v[7]};
        }
    }
    wave_sync();
    // the tile's bytes have all been read (their values feed the V stores)
    if constexpr (HALF || EARLY) consumed();

    // 4. GEMM1 A fragments.  A[upar][vpar][s] holds, for row
    //    u = 2 l32 + upar, the columns v = 2 pi(16 s + 8 h + e) + vpar,
    //    e = 0..7.  For fixed (upar, s) these are two runs of 8
    //    consecutive columns, v0 = 32 s + 16 run + 8 h: even offsets feed
    //    vpar 0, odd offsets vpar 1.
    const uint64_t bits_r[2] = {__shfl(bits, 2 * l32), __shfl(bits, 2 * l32 + 1)};
    const uint32_t pre_r[2] = {__shfl(pre, 2 * l32), __shfl(pre, 2 * l32 + 1)};
    // 5. GEMM1 (even/odd halves of the column frequencies), one row
    //    parity at a time so that only its A fragments are live:
    //    acc[upar][vpar][n] = sum_v C[2m + upar][v] M[v][n], v of parity vpar,
    //    n < 32.  Then S[u][n] = E + O and S[u][63 - n] = E - O.
    floatx16 acc[2][2];
    // PRIO: the wave issues at raised priority from here to its last MFMA
    // (the second column block's output stage), so that the matrix cores are
    // fed while the other waves' gathers, splits and stores fill the VALU
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int up = 0; up < 2; up++) {
        const uint64_t b64 = ok ? bits_r[up] : 0ull;
        // the row shifted so that column 8 h is bit 0: every column this
        // lane needs sits at a compile-time bit position
        const uint64_t bh = b64 >> (8 * h);
        const uint32_t wd[2] = {(uint32_t)bh, (uint32_t)(bh >> 32)};
        const uint32_t rank_h = pre_r[up] + (uint32_t)__popcll(b64 & ((1ull << (8 * h)) - 1ull));
        // LDS byte address of V[rank]; a column that is not retained
        // masks it to 0, the zero word
        uint32_t diff = wbase + 4 * rank_h;
        acc[up][0] = floatx16{};
        acc[up][1] = floatx16{};
        // one k step at a time: its A fragments are gathered, then used
#pragma unroll
        for (int s = 0; s < 2; s++) {
            u32x4 ahi[2], alo[2];  // [vpar]
#pragma unroll
            for (int run = 0; run < 2; run++) {
                const uint32_t word = wd[s];
                uint32_t a[8];  // LDS address of each column's table entry, or 0
#pragma unroll
                for (int o = 0; o < 8; o++) {
                    // all-ones when column 16 run + o of the word is retained
                    const int32_t m = (int32_t)(word << (31 - (16 * run + o))) >> 31;
                    a[o] = (uint32_t)m & diff;
                    diff = (uint32_t)((int32_t)diff + m * n4);  // v_mad_i32_i24
                }
                // columns 16 run + 8 .. 16 run + 15 of this word belong to the
                // other lane half
                diff += (uint32_t)__popc((word >> (16 * run + 8)) & 0xffu) << 2;
                // dword p of a fragment packs elements e = 2p, 2p + 1 (this run
                // supplies e = 4 run .. 4 run + 3, at offsets 2 (e - 4 run) + vpar);
                // a table entry is f16 hi | f16 lo << 16
                uint32_t w[8];
#pragma unroll
                for (int o = 0; o < 8; o++) w[o] = lds_load(a[o]);
#pragma unroll
                for (int vp = 0; vp < 2; vp++) {
                    ahi[vp][2 * run] = __builtin_amdgcn_perm(w[2 + vp], w[vp], 0x05040100u);
                    alo[vp][2 * run] = __builtin_amdgcn_perm(w[2 + vp], w[vp], 0x07060302u);
                    ahi[vp][2 * run + 1] = __builtin_amdgcn_perm(w[6 + vp], w[4 + vp], 0x05040100u);
                    alo[vp][2 * run + 1] = __builtin_amdgcn_perm(w[6 + vp], w[4 + vp], 0x07060302u);
                }
            }
#pragma unroll
            for (int vp = 0; vp < 2; vp++) {
                const u32x4 mh = mtab[((0 * 2 + vp) * 2 + s) * 64 + lane];
                const u32x4 ml = mtab[((1 * 2 + vp) * 2 + s) * 64 + lane];
                acc[up][vp] = mfma(ahi[vp], mh, acc[up][vp]);
                acc[up][vp] = mfma(ahi[vp], ml, acc[up][vp]);
                acc[up][vp] = mfma(alo[vp], mh, acc[up][vp]);
            }
        }
    }
    wave_sync();

    // 6. butterfly in place: acc[upar][0] = E + O = S[u][n],
    //    acc[upar][1] = E - O = S[u][63 - n]
#pragma unroll
    for (int up = 0; up < 2; up++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float e = acc[up][0][r], o = acc[up][1][r];
            acc[up][0][r] = e + o;
            acc[up][1][r] = e - o;
        }
    }

    // 7. GEMM2 transposed, per S column block jb (jb = 0: j = n;
    //    jb = 1: j = 63 - n): X^T[j][i] = sum_u S[u][j] M[u][i], with S
    //    (GEMM1's accumulators) as the A operand and the M fragments as B,
    //    split by u parity into E2 (upar 0) and O2 (upar 1).  Lane l32 then
    //    holds output rows i = l32 and 63 - i (X[63 - i][j] = E2 - O2) and
    //    register r the column j = (r & 3) + 8 (r >> 2) + 4 h (or 63 minus
    //    it): four consecutive columns per register quad, parked in LDS as
    //    one 8-byte (16-bit outputs) or 16-byte (f32) write per row.  The
    //    park holds the whole tile (HALF false: stored once, 16 bytes per
    //    lane over whole rows) or one column block (HALF: stored after each
    //    block, half the LDS).
    const float os = pow2f(-(E + 16));
    constexpr uint32_t pitch = HALF ? kHalfPitch<DT> : kParkPitch<DT>;
    const uint32_t i_lo = wbase + (uint32_t)l32 * pitch;
    const uint32_t i_hi = wbase + (uint32_t)(63 - l32) * pitch;
    constexpr uint32_t esz = DT == HH_F32 ? 4u : 2u;
    const uint32_t tpr = cols >> 6;
    // t / tpr without a division below 2^22 tiles: (t + 1/2) / tpr lies at
    // least 1/(2 tpr) from an integer, beyond the float product's error
    const uint32_t tr = t < (1u << 22) ? uniform((uint32_t)(((float)t + 0.5f) * B.tpr_inv[ti])) : t / tpr;
    const uint32_t tc = t - tr * tpr;
    const size_t base = (size_t)(64 * tr) * cols + 64 * tc;
    // the tile's first output byte and the row pitch, in scalar registers:
    // a store addresses scalar base + 32-bit lane offset (no 64-bit vector
    // arithmetic per store)
    uint8_t HH_GLOBAL *const otile =
        (uint8_t HH_GLOBAL *)uniform((uint64_t)(uintptr_t)((uint8_t HH_GLOBAL *)B.out[ti] + esz * base));
    const uint32_t opitch = uniform(cols * esz);
    // row stores of columns [c0, c0 + ncols) from the park (16 bytes per lane)
    auto store = [&](uint32_t c0, auto ncolc) {
        constexpr uint32_t ncols = decltype(ncolc)::value;
        constexpr uint32_t per_row = ncols * esz / 16;  // lanes per row
        constexpr uint32_t rows_per = 64 / per_row;     // rows per instruction
        const uint32_t rsub = (uint32_t)lane / per_row, csub = (uint32_t)lane % per_row;
        const uint32_t loff = rsub * opitch + esz * c0 + 16 * csub;  // < 16 rows: fits 32 bits
#pragma unroll
        for (uint32_t it = 0; it < 64 / rows_per; it++) {
            const uint32_t row = rows_per * it + rsub;
            const uint32_t a0 = wbase + row * pitch + 16 * csub;
            u32x4 v;
            if constexpr (DT == HH_F32) {
                v = *(lds_u32x4 *)(size_t)a0;
            } else {
                // rows are 8-byte aligned in the park: two 8-byte reads
                const u32x2 lo = *(lds_u32x2 *)(size_t)a0, hi = *(lds_u32x2 *)(size_t)(a0 + 8);
                v = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
            *(u32x4 HH_GLOBAL *)(otile + (size_t)(rows_per * it) * opitch + loff) = v;
        }
    };
    // GEMM2 for both column blocks first (four accumulator chains in
    // flight), then their output stages
    floatx16 x2all[2][2];
#pragma unroll
    for (int jb = 0; jb < 2; jb++) {
        x2all[jb][0] = floatx16{};
        x2all[jb][1] = floatx16{};
#pragma unroll
        for (int up = 0; up < 2; up++) {
#pragma unroll
            for (int s = 0; s < 2; s++) {
                u32x4 shi, slo;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int r0 = 8 * s + 2 * p;
                    uint32_t hp, lp;
                    split2(acc[up][jb][r0], acc[up][jb][r0 + 1], one, hp, lp);
                    shi[p] = hp;
                    slo[p] = lp;
                }
                const u32x4 mh = mtab[((0 * 2 + up) * 2 + s) * 64 + lane];
                const u32x4 ml = mtab[((1 * 2 + up) * 2 + s) * 64 + lane];
                x2all[jb][up] = mfma(shi, mh, x2all[jb][up]);
                x2all[jb][up] = mfma(shi, ml, x2all[jb][up]);
                x2all[jb][up] = mfma(slo, mh, x2all[jb][up]);
            }
        }
    }
#pragma unroll
    for (int jb = 0; jb < 2; jb++) {
        const floatx16 *x2 = x2all[jb];
        if constexpr (PRIO)
            if (jb == 1) __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float va[4], vc[4];  // rows i and 63 - i, columns ascending
#pragma unroll
            for (int t4 = 0; t4 < 4; t4++) {
                const int r = 4 * q + (jb == 0 ? t4 : 3 - t4);
                const float o2 = x2[1][r] * os;
                va[t4] = __builtin_fmaf(x2[0][r], os, o2);
                vc[t4] = __builtin_fmaf(x2[0][r], os, -o2);
            }
            // first of the four columns (relative to 32 jb in a half park)
            const uint32_t jabs = jb == 0 ? 8 * q + 4 * h : 60 - 8 * q - 4 * h;
            const uint32_t j0 = HALF ? jabs - 32u * jb : jabs;
            if constexpr (DT == HH_F32) {
                *(lds_u32x4 *)(size_t)(i_lo + esz * j0) =
                    u32x4{__float_as_uint(va[0]), __float_as_uint(va[1]), __float_as_uint(va[2]),
                          __float_as_uint(va[3])};
                *(lds_u32x4 *)(size_t)(i_hi + esz * j0) =
                    u32x4{__float_as_uint(vc[0]), __float_as_uint(vc[1]), __float_as_uint(vc[2]),
                          __float_as_uint(vc[3])};
            } else {
                *(lds_u32x2 *)(size_t)(i_lo + esz * j0) = u32x2{pack2<DT>(va[0], va[1]), pack2<DT>(va[2], va[3])};
                *(lds_u32x2 *)(size_t)(i_hi + esz * j0) = u32x2{pack2<DT>(vc[0], vc[1]), pack2<DT>(vc[2], vc[3])};
            }
        }
        if constexpr (HALF) {
            wave_sync();
            // 8. coalesced row stores of this column block
            store(32u * jb, std::integral_constant<uint32_t, 32>{});
            wave_sync();  // the next block's park overwrites this one
        }
    }
    if constexpr (!HALF) {
        wave_sync();
        if constexpr (!EARLY) consumed();
        // 8. coalesced row stores (16 bytes per lane)
        store(0u, std::integral_constant<uint32_t, 64>{});
    }
    if (B.status[ti] != nullptr && lane == 0)
        ((int32_t HH_GLOBAL *)B.status[ti])[t] = ok ? HH_OK : HH_ERR_CORRUPTED_DATA;
}

template <int DT, bool DW, int NP>
__global__ __launch_bounds__(kThreads, kWavesPerSimd(DT, NP)) void hctt_decode_kernel(TileBatch Bk,
                                                                   const u32x4 *__restrict__ basis) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = (int)uniform((uint32_t)threadIdx.x >> 6);  // in a scalar register
    u32x4 *mtab = reinterpret_cast<u32x4 *>(smem + kMTabOff);
    for (int i = threadIdx.x; i < (int)(sizeof(TileBatch) / 4); i += kThreads)
        reinterpret_cast<uint32_t *>(smem + kBatchOff)[i] = reinterpret_cast<const uint32_t *>(&Bk)[i];
    for (int i = threadIdx.x; i < (int)(kMTabBytes / 16); i += kThreads) mtab[i] = basis[i];
    if (threadIdx.x == 0) *reinterpret_cast<u32x4 *>(smem + kZeroOff) = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
    const TileBatch &B = *reinterpret_cast<const TileBatch *>(smem + kBatchOff);
    const float one = Bk.one;                 // 1.0
    const int32_t n4 = (int32_t)(int8_t)Bk.neg4;  // -4, known to fit 24 bits
    const uint32_t wbase = kSharedBytes + wave * B.wave_lds;  // byte offset of this wave's area
    const uint32_t pbase = wbase + B.vo_bytes;                // staged tile bytes
    uint32_t *V = reinterpret_cast<uint32_t *>(smem + wbase);
    const uint8_t *pay = smem + pbase;

    // Tile bytes travel global -> registers (prefetched one tile ahead, 16 B
    // per lane per 1 KiB) -> LDS, so no global latency sits on the critical
    // path of a tile.
    const uint32_t ntiles = B.start[B.n];
    const uint32_t stride = gridDim.x * kWaves;
    u32x4 pf[NP];
    uint32_t gt = blockIdx.x * kWaves + wave;
    // tensor of the tile staged next (looked up once per tile, when its
    // bytes are fetched)
    uint32_t ti_next = 0;
    if (gt < ntiles) {
        ti_next = tensor_of(B, gt, lane);
        prefetch_tile<DW, NP>(B, gt, ti_next, lane, pf);
#pragma unroll
        for (int i = 0; i < NP; i++)
            *reinterpret_cast<u32x4 *>(smem + pbase + 16 * (lane + 64 * i)) = pf[i];
    }
    for (; gt < ntiles; gt += stride) {
        const uint32_t ti = ti_next;
        const uint32_t t = gt - uniform(B.start[ti]);

        // This tile's bytes are staged in LDS.  Fetch the next tile now; it is
        // staged at the end of this iteration, long after the loads landed
        // and before this tile's output stores are issued (the wait counter
        // is in order, so stores issued earlier would have to drain first).
        const bool has_next = gt + stride < ntiles;
        const uint32_t gn = has_next ? gt + stride : gt;
        ti_next = has_next ? tensor_of(B, gn, lane) : ti;
        prefetch_tile<DW, NP>(B, gn, ti_next, lane, pf);
        wave_sync();

        tile_body<DT, false, false, true>(B, ti, t, pay + tile_shift<DW>(B, ti, t), V, wbase, mtab, lane, one, n4, [&]() {
            // stage the next tile's bytes (the current ones are no longer needed)
#pragma unroll
            for (int i = 0; i < NP; i++)
                *reinterpret_cast<u32x4 *>(smem + pbase + 16 * (lane + 64 * i)) = pf[i];
        });
        wave_sync();
    }
}

// ---- LZ4 blocks and their tiles in one launch ------------------------------
//
// One persistent workgroup per CU (G of them) takes the launch's blocks g,
// g + G, g + 2 G, ... (its slots 0, 1, 2, ...) and all their tiles (each
// block holds whole tiles of one tensor: block j of tensor i tiles
// [j tpb_i, j tpb_i + tpb_i) of it, the last block the rest).  Every wave of the
// workgroup does both kinds of work, claimed from two LDS counters:
//   next_block  the slots' blocks are decoded in order, each by the wave
//               that claims it, with the LDS-ring decoder (lz4_ring.hpp, the
//               whole output kept in LDS: at most kFusedMax bytes) into a
//               ring of nbuf block buffers (slot q into buffer q mod nbuf);
//   next_tile   the slots' tiles are decoded in order (tile slot v: tile
//               v mod T of slot v / T, T the largest tpb_i, skipped past a
//               block's tiles), each by the wave that claims it, straight from the
//               block buffer with tile_body (the whole output tile parked in
//               LDS, then stored).
// A wave first claims the next block if its buffer is free (compare and
// swap: only a free buffer's block is ever claimed this way), else the next
// tile; a claimed tile whose block nobody has claimed yet makes its wave
// claim and decode the blocks up to it first (waiting for their buffers).
// A wave's LDS area is its tile's V table and output park, or its input
// stage while it decodes a block.  The tile bytes never reach HBM, and the
// LZ4 parse of a block runs while other waves already decode its first
// tiles.
//
// Two LDS words per buffer order the two kinds of work:
//   state[x]  (64 bits) 1 + the slot of the block the buffer holds, and
//             the bytes of it decoded so far (published after LZ4
//             sequences; the whole block only by its final store);
//   done[x]   how many of that block's tiles are still to be read (its
//             decoder sets the block's tile count before publishing slot
//             i; every tile read takes one off).  Slot i may take buffer x
//             once state[x] names slot i - nbuf (placed there by another
//             wave, possibly late) and done[x] is 0.
// A tile is decoded as soon as the published bytes cover it.  Two LDS
// bitmaps over the workgroup's slots record which are complete and which
// failed.  A failed block's decoder zeroes its buffer from the first tile it
// had not released (those tiles then fail their bitmap count).  After its
// last tile each wave waits until its stores are done and counts itself
// finished; once every block of the workgroup is complete, if one failed,
// the waves wait for each other and rewrite the failed blocks' tiles (tile
// j of a block by wave j mod W) as zeros with HH_ERR_CORRUPTED_DATA: every
// tile of a failed block ends up so, as with the two-launch path.  A block
// that decodes short (no error) leaves the rest of its buffer zeroed: those
// tiles fail their bitmap count.
//
// No wait can deadlock: a wave waits on a buffer only for slot i, whose
// buffer's previous slot i - nbuf has all its tiles claimed (they come
// before a claimed tile of slot i or later); a tile's wave waits for its
// block's bytes, whose decoder waits only on lower slots; every such chain
// descends to a slot whose buffer is free.  Every wait is bounded all the
// same (kSpinLimit polls, or the context's HH_OPT_FUSED_POLL_LIMIT, which
// tests set small to run this path); one that runs out raises the
// workgroup's abort word, every wave then leaves, and every block record of
// the workgroup reports HH_ERR_DEVICE (written by the last wave to leave).
//
// The input stage holds 8 KiB of a block's compressed bytes (a 16 KiB block
// is staged in two or three batches of loads): it fits a wave's tile area,
// which leaves the rest of the LDS to three block buffers.
constexpr uint32_t kFusedStageData = 8 * 1024;
using FusedRing = ring::RingDec<16384, kFusedStageData, true>;
using FusedSeq = seq::SeqDec<16384, kFusedStageData, true>;
constexpr uint32_t kFusedMax = 16384 - 32;
constexpr uint32_t kFusedBuf = 16384;  // a block buffer: the decoder's ring
// a decoder's input stage (the sequence-batched decoder's run table after it)
constexpr uint32_t kFusedStageRing = FusedRing::kSFront + kFusedStageData + FusedRing::kSPad;
constexpr uint32_t kFusedStageSeq = FusedSeq::kStageLds + FusedSeq::kTabLds;
constexpr uint32_t kFusedStage = kFusedStageRing > kFusedStageSeq ? kFusedStageRing : kFusedStageSeq;
static_assert(FusedRing::kSFront == FusedSeq::kSFront, "both decoders' stages start at the same offset");
constexpr int kFusedMaxWaves = 12;     // 3 per SIMD: 168 registers, tile_body's budget
constexpr uint32_t kFusedMaxBufs = 4;
constexpr uint32_t kFusedLdsMax = 160u * 1024u;
constexpr uint32_t kSpinLimit = 1u << 24;  // polls of about 64 cycles each
constexpr uint32_t kFusedMaxRange = 512;  // slots per workgroup (the bitmaps' size)
// tiles a wave claims with one atomic (2 measured 2 % slower on the
// Llama-3-8B layer: the block claims, checked once per claim, came later)
constexpr uint32_t kTileClaim = 1;

struct FusedBlocks {
    const uint8_t *in;
    uint64_t in_total;
    const uint64_t *in_off;  // indexed by global block number
    const uint32_t *in_len;
    hh_block_status *status;
    uint32_t blk_base;                    // global number of this launch's block 0
    uint32_t blk_start[kMaxTensors + 1];  // first block of each tensor, launch-relative
    uint32_t tpb[kMaxTensors];            // tiles per block of each tensor
    uint32_t tpb_max;
    uint32_t nbuf;                        // block buffers
    uint32_t buf_off;                     // LDS byte offset of the buffers
    uint32_t spin_limit;                  // polls before a wait gives up
};

// Workgroup LDS layout after the shared part: [block descriptor][state[8]
// (8 bytes each), done[8], abort, next_block, next_tile, finished, left,
// the complete and failed bitmaps][wave areas][block buffers].
constexpr uint32_t kFusedFOff = kSharedBytes;
constexpr uint32_t kFusedFlagsOff = kFusedFOff + ((sizeof(FusedBlocks) + 15u) & ~15u);
constexpr uint32_t kFusedStateOff = kFusedFlagsOff;
constexpr uint32_t kFusedDoneOff = kFusedStateOff + 8 * kFusedMaxBufs;
constexpr uint32_t kFusedAbortOff = kFusedDoneOff + 4 * kFusedMaxBufs;
constexpr uint32_t kFusedNextBlockOff = kFusedAbortOff + 4;
constexpr uint32_t kFusedNextTileOff = kFusedNextBlockOff + 4;
constexpr uint32_t kFusedFinishedOff = kFusedNextTileOff + 4;
constexpr uint32_t kFusedLeftOff = kFusedFinishedOff + 4;
constexpr uint32_t kFusedFinalOff = kFusedLeftOff + 4;
constexpr uint32_t kFusedFailOff = kFusedFinalOff + kFusedMaxRange / 8;
constexpr uint32_t kFusedFlagWords = (kFusedFailOff + kFusedMaxRange / 8 - kFusedFlagsOff) / 4;
constexpr uint32_t kFusedWaveOff = kFusedFlagsOff + ((4 * kFusedFlagWords + 15u) & ~15u);
// 16-bit outputs of tiles with k <= 2176 (every retention up to 0.53): 12
// waves with a whole-tile park each and three block buffers
static_assert(kFusedWaveOff + 12u * 64u * kParkPitch<HH_BF16> + 3u * kFusedBuf <= kFusedLdsMax,
              "twelve waves and three block buffers fit the LDS");

typedef uint32_t __attribute__((address_space(3))) lds_word;
typedef uint64_t __attribute__((address_space(3))) lds_dword;

// The lane number, computed where it is used from a mask the compiler cannot
// see through: values derived from it are then recomputed inside a loop
// instead of being hoisted and held (or spilled) across it.
__device__ __forceinline__ int opaque_lane() {
    uint32_t m = ~0u;
    asm volatile("" : "+s"(m));
    return (int)__builtin_amdgcn_mbcnt_hi(m, __builtin_amdgcn_mbcnt_lo(m, 0u));
}

__device__ __forceinline__ uint64_t lds_load_acq(uint32_t a, uint64_t) {
    return __hip_atomic_load((lds_dword *)(size_t)a, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint32_t lds_load_acq(uint32_t a, uint32_t) {
    return __hip_atomic_load((lds_word *)(size_t)a, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Polls the LDS word (32 or 64 bits, by T) at LDS address w until ok(value)
// holds (true, the value in v), or the abort word is raised or the poll
// limit runs out (false; the latter raises it).
template <typename T, typename Pred>
__device__ __forceinline__ bool fused_poll(uint32_t w, int lane, uint32_t limit, T &v, Pred &&ok) {
    for (uint32_t it = 0;; it++) {
        v = uniform(lds_load_acq(w, T{}));
        if (ok(v)) return true;
        const uint32_t ab = uniform(
            __hip_atomic_load((lds_word *)(size_t)kFusedAbortOff, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (ab != 0) return false;
        if (it >= limit) {
            if (lane == 0)
                __hip_atomic_store((lds_word *)(size_t)kFusedAbortOff, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// SEQ: the blocks are decoded by the sequence-batched decoder
// (lz4_seq.hpp) instead of the one-sequence ring decoder (lz4_ring.hpp).
template <int DT, bool SEQ>
__global__ __launch_bounds__(64 * kFusedMaxWaves) void hctt_lz4_fused_kernel(TileBatch Bk, FusedBlocks Fk,
                                                                              const u32x4 *__restrict__ basis) {
    extern __shared__ __align__(16) uint8_t smem[];
    // wave-uniform (scalar) wave number
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t nthr = blockDim.x;
    u32x4 *mtab = reinterpret_cast<u32x4 *>(smem + kMTabOff);
    for (uint32_t i = threadIdx.x; i < (uint32_t)(sizeof(TileBatch) / 4); i += nthr)
        reinterpret_cast<uint32_t *>(smem + kBatchOff)[i] = reinterpret_cast<const uint32_t *>(&Bk)[i];
    for (uint32_t i = threadIdx.x; i < (uint32_t)(sizeof(FusedBlocks) / 4); i += nthr)
        reinterpret_cast<uint32_t *>(smem + kFusedFOff)[i] = reinterpret_cast<const uint32_t *>(&Fk)[i];
    for (uint32_t i = threadIdx.x; i < kMTabBytes / 16; i += nthr) mtab[i] = basis[i];
    for (uint32_t i = threadIdx.x; i < kFusedFlagWords; i += nthr) reinterpret_cast<uint32_t *>(smem + kFusedFlagsOff)[i] = 0u;
    if (threadIdx.x == 0) *reinterpret_cast<u32x4 *>(smem + kZeroOff) = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();  // the only workgroup barrier
    const TileBatch &B = *reinterpret_cast<const TileBatch *>(smem + kBatchOff);
    // the LDS copy serves the indexed block table; pointers come from the
    // kernel arguments, where the compiler knows them to be global
    const FusedBlocks &F = *reinterpret_cast<const FusedBlocks *>(smem + kFusedFOff);
    const uint32_t nw = nthr >> 6, nbuf = Fk.nbuf;
    // slot q's buffer, q mod nbuf without a division (exact: q < 2^22)
    const float nbuf_inv = 1.0f / (float)nbuf;
    auto buf_of = [&](uint32_t q) { return q - nbuf * uniform((uint32_t)(((float)q + 0.5f) * nbuf_inv)); };
    auto state_w = [](uint32_t x) { return kFusedStateOff + 8u * x; };
    auto done_w = [](uint32_t x) { return kFusedDoneOff + 4u * x; };

    // block lb -> tensor, first tile, tile count
    auto locate = [&](uint32_t lb, uint32_t &ti, uint32_t &t0, uint32_t &nt, uint32_t &tb) {
        // lane j holds tensor j's first block, tiles per block, first and
        // last tile and tile bytes (one round of LDS reads); the tensor is
        // the count of first blocks after the first at or below lb (the
        // unused entries past blk_start[n] are all-ones), by a ballot, and
        // its fields come from lane ti (wave-uniform; every lane active)
        const uint32_t j = (uint32_t)opaque_lane() & (kMaxTensors - 1);
        const uint32_t sj = F.blk_start[j], pj = F.tpb[j], s0 = B.start[j], s1 = B.start[j + 1], bj = B.tb[j];
        ti = (uint32_t)__popcll(__builtin_amdgcn_ballot_w64(lb >= sj) & (((1ull << kMaxTensors) - 1ull) & ~1ull));
        const uint32_t tpb_i = (uint32_t)__builtin_amdgcn_readlane((int)pj, (int)ti);
        t0 = (lb - (uint32_t)__builtin_amdgcn_readlane((int)sj, (int)ti)) * tpb_i;
        nt = min(tpb_i, (uint32_t)__builtin_amdgcn_readlane((int)s1, (int)ti) -
                            (uint32_t)__builtin_amdgcn_readlane((int)s0, (int)ti) - t0);
        tb = (uint32_t)__builtin_amdgcn_readlane((int)bj, (int)ti);
    };
    // The workgroup's blocks: launch blocks g, g + G, g + 2 G, ... (G
    // workgroups), its q-th block lb(q) = g + q G, all of whose tiles it
    // decodes; slot q of a workgroup is decoded into buffer q mod nbuf.
    const uint32_t nblk = F.blk_start[B.n];
    const uint32_t g = blockIdx.x, G = gridDim.x;
    const uint32_t Q = nblk > g ? (nblk - g + G - 1u) / G : 0u;
    auto lb_of = [&](uint32_t q) { return g + q * G; };
    // bit q of a bitmap: LDS word address and mask
    auto bit_w = [&](uint32_t base, uint32_t q) { return base + 4u * (q >> 5); };
    auto bit_m = [&](uint32_t q) { return 1u << (q & 31u); };
    // Every wave leaves through here: its stores complete, it counts itself
    // out, and the last one out, if a wait gave up (the abort word), writes
    // HH_ERR_DEVICE into every block record and every tile status of the
    // workgroup's blocks (any of its tiles may be undecoded); the other
    // waves' records and statuses are complete by then, so none overwrites
    // it.
    auto leave = [&]() {
        const int l = opaque_lane();
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        uint32_t prev = 0;
        if (l == 0)
            prev = __hip_atomic_fetch_add((lds_word *)(size_t)kFusedLeftOff, 1u, __ATOMIC_ACQ_REL,
                                          __HIP_MEMORY_SCOPE_WORKGROUP);
        prev = uniform(prev);
        const uint32_t ab = uniform(
            __hip_atomic_load((lds_word *)(size_t)kFusedAbortOff, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (prev + 1u == nw && ab != 0u) {
            for (uint32_t q = (uint32_t)l; q < Q; q += 64u) {
                hh_block_status st;
                st.code = HH_ERR_DEVICE;
                st.detail = HH_CORRUPT_NONE;
                st.position = 0;
                st.required = 0;
                st.written = 0;
                ((hh_block_status *)Fk.status)[Fk.blk_base + lb_of(q)] = st;
            }
            for (uint32_t q = 0; q < Q; q++) {
                uint32_t ti, t0, nt, tbq;
                locate(lb_of(q), ti, t0, nt, tbq);
                int32_t *ts = B.status[ti];
                if (ts != nullptr)
                    for (uint32_t j = (uint32_t)l; j < nt; j += 64u) ts[t0 + j] = HH_ERR_DEVICE;
            }
        }
    };
    // this wave's LDS area: a tile's V table and output park, or the input
    // stage of the block it decodes
    const uint32_t wbase = kFusedWaveOff + wave * B.wave_lds;
    uint8_t *stage = smem + wbase + FusedRing::kSFront;
    uint32_t *V = reinterpret_cast<uint32_t *>(smem + wbase);

    // may slot q take its buffer now?  (once true, true until q is placed.)
    // A probe with both words read at once: decode() waits on them again
    // with acquire loads before it touches the buffer.  The state is read
    // first (one wave's LDS reads are performed in order, and the count is
    // set before the state names its slot).
    auto buf_free = [&](uint32_t q) {
        if (q < nbuf) return true;
        const uint32_t x = buf_of(q);
        const uint64_t sv =
            __hip_atomic_load((lds_dword *)(size_t)state_w(x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        asm volatile("" ::: "memory");
        const uint32_t rem =
            __hip_atomic_load((lds_word *)(size_t)done_w(x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return (uint32_t)(uniform(sv) >> 32) == q - nbuf + 1u && uniform(rem) == 0u;
    };
    // the next slot to claim (the word counts the slots claimed)
    auto next_block = [&]() {
        return uniform(
            __hip_atomic_load((lds_word *)(size_t)kFusedNextBlockOff, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    };
    // claims slot q if it is still the next one
    auto claim = [&](uint32_t q, int ln) {
        uint32_t e = q;
        if (ln == 0)
            __hip_atomic_compare_exchange_strong((lds_word *)(size_t)kFusedNextBlockOff, &e, q + 1u,
                                                 __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return uniform(e) == q;
    };
    // decodes slot q's block (claimed by this wave) into its buffer, after
    // waiting for the buffer; false when a wait ran out
    auto decode = [&](uint32_t q) {
        const int ln = opaque_lane();
        const uint32_t x = buf_of(q);
        if (q >= nbuf) {
            // the buffer's previous block (slot q - nbuf, possibly placed late
            // by another wave) must have been placed there, then read: its
            // count is only meaningful once its stamp is up
            uint32_t v;
            uint64_t sv;
            if (!fused_poll(state_w(x), ln, Fk.spin_limit, sv,
                            [&](uint64_t s) { return (uint32_t)(s >> 32) == q - nbuf + 1u; }) ||
                !fused_poll(done_w(x), ln, Fk.spin_limit, v, [&](uint32_t c) { return c == 0u; }))
                return false;
        }
        const uint32_t lb = lb_of(q);
        uint32_t ti, t0, nt, tbq;
        locate(lb, ti, t0, nt, tbq);
        const uint64_t stamp = (uint64_t)(q + 1u) << 32;
        if (ln == 0) {
            __hip_atomic_store((lds_word *)(size_t)done_w(x), nt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_store((lds_dword *)(size_t)state_w(x), stamp, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        const uint32_t tb = tbq;
        const uint32_t cap = nt * tb;
        uint8_t *rbuf = smem + Fk.buf_off + x * kFusedBuf;
        const uint32_t gb = Fk.blk_base + lb;
        int32_t code = HH_OK, detail = HH_CORRUPT_NONE;
        uint64_t pos = 0, req = 0;
        const uint64_t ioff = Fk.in_off[gb];
        const uint32_t ilen = Fk.in_len[gb];
        using Dec = typename std::conditional<SEQ, FusedSeq, FusedRing>::type;
        Dec d;
        if constexpr (SEQ) {
            d.ring = (seq::lds8 *)(size_t)(Fk.buf_off + x * kFusedBuf);
            d.stage = (seq::lds8 *)(size_t)(wbase + FusedSeq::kSFront);
            d.tab = (seq::lds32 *)(size_t)(wbase + FusedSeq::kStageLds);
        } else {
            d.ring = rbuf;
            d.stage = stage;
            d.wso = ring::kNoWin;
            d.w = 0;
        }
        d.gbuf = Fk.in;
        d.gsz = Fk.in_total;
        d.ioff = ioff;
        d.a0 = 0;
        d.obase = nullptr;
        d.cap = cap;
        d.sb = 0;
        d.at_end = false;
        d.op = 0;
        d.fl = 0;
        d.lane = ln;
        // bytes published so far (every lane's copies are issued: each copy
        // piece ends with a wave barrier).  The whole block is published only
        // by the final state store below: were the last tile released here,
        // the block could be counted done and its buffer refilled before
        // that store, which would then overwrite the new block's state.
        uint32_t published = 0;
        auto publish = [&](uint32_t op) {
            if (op >= published + tb && op < cap) {
                published = op;
                if (ln == 0)
                    __hip_atomic_store((lds_dword *)(size_t)state_w(x), stamp | op, __ATOMIC_RELEASE,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        };
        if (ioff > Fk.in_total || (uint64_t)ilen > Fk.in_total - ioff) {
            code = HH_ERR_INVALID_ARGUMENT;
        } else {
            if constexpr (SEQ)
                seq::decode_block(d, ilen, code, detail, pos, req, false, publish);
            else
                ring::parse_block(d, ilen, code, detail, pos, req, false, publish);
        }
        // a complete block: the bytes it did not produce read as zeros; a
        // failed one: zeros from its first tile not released (released
        // tiles are rewritten at the end)
        const uint32_t zfrom = code == HH_OK ? d.op : (published / tb) * tb;
        if (zfrom < cap) {
            wave_sync();
            wave_zero_fill(rbuf + zfrom, cap - zfrom, ln);
        }
        if (ln == 0) {
            hh_block_status st;
            st.code = code;
            st.detail = detail;
            st.position = pos;
            st.required = req;
            st.written = code == HH_OK ? d.op : 0u;
            ((hh_block_status *)Fk.status)[gb] = st;
        }
        wave_sync();  // every lane's buffer writes are issued before the release
        if (ln == 0) {
            if (code != HH_OK)
                __hip_atomic_fetch_or((lds_word *)(size_t)bit_w(kFusedFailOff, q), bit_m(q), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_fetch_or((lds_word *)(size_t)bit_w(kFusedFinalOff, q), bit_m(q), __ATOMIC_RELEASE,
                                  __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_store((lds_dword *)(size_t)state_w(x), stamp | cap, __ATOMIC_RELEASE,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        return true;
    };

    const float one = Bk.one;
    const int32_t n4 = (int32_t)(int8_t)Bk.neg4;
    const uint32_t tpb = Fk.tpb_max;
    // v / tpb without a division: (v + 1/2) / tpb lies at least 1/(2 tpb)
    // from an integer, and the float product's relative error (2^-23, 1/tpb
    // rounded) stays below that for v < 2^22 (v < kFusedMaxRange x 31 tiles
    // per block + the waves' last claims)
    const float tpb_inv = 1.0f / (float)tpb;
    // the block of the wave's last tile (a wave usually takes several tiles
    // of one block in a row): its tensor, first tile, tile count and tile
    // bytes, and the bytes of it seen published (the state's low word,
    // read with acquire by this wave)
    uint32_t cq = ~0u, cti = 0, ct0 = 0, cnt = 0, ctb = 0, cpub = 0;
    bool aborted = false;
    for (;;) {
        // the next block, when its buffer is free
        const uint32_t nq = next_block();
        if (nq < Q && buf_free(nq) && claim(nq, opaque_lane())) {
            if (!decode(nq)) {
                aborted = true;
                break;
            }
            continue;
        }
        // else the next kTileClaim tiles (one atomic): slot v / tpb, tile
        // v % tpb of its block (slots past the block's tiles are skipped).
        // The claims keep the counter's order, and a wave works on its first
        // tile before its second, so every wait still descends to lower
        // slots.
        const int ln = opaque_lane();
        uint32_t v = 0;
        if (ln == 0)
            v = __hip_atomic_fetch_add((lds_word *)(size_t)kFusedNextTileOff, kTileClaim, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
        v = uniform(v);
        bool past = false;
        for (uint32_t c = 0; c < kTileClaim; c++, v++) {
            const uint32_t q = uniform((uint32_t)(((float)v + 0.5f) * tpb_inv)), off = v - q * tpb;
            if (q >= Q) {
                past = true;
                break;
            }
            if (q != cq) {
                locate(lb_of(q), cti, ct0, cnt, ctb);
                cq = q;
                cpub = 0;
            }
            const uint32_t ti = cti, t0 = ct0, nt = cnt, tb = ctb;
            if (off >= nt) continue;
            // its block and every one before it claimed (by this wave if need
            // be; the count read above only grows)
            if (nq <= q) {
                for (;;) {
                    const uint32_t n2 = next_block();
                    if (n2 > q) break;
                    if (claim(n2, opaque_lane()) && !decode(n2)) {
                        aborted = true;
                        break;
                    }
                }
                if (aborted) break;
            }
            const int ln2 = opaque_lane();
            const uint32_t x = buf_of(q);
            const uint32_t need = (off + 1u) * tb;
            // the tile's bytes are there: published bytes only grow while the
            // buffer holds slot q, and it holds q until this tile is read
            if (cpub < need) {
                uint64_t sv;
                if (!fused_poll(state_w(x), ln2, Fk.spin_limit, sv, [&](uint64_t s) {
                        return (uint32_t)(s >> 32) == q + 1u && (uint32_t)s >= need;
                    })) {
                    aborted = true;
                    break;
                }
                cpub = (uint32_t)sv;
            }
            const uint8_t *rbuf = smem + Fk.buf_off + x * kFusedBuf;
            tile_body<DT, false, true>(B, ti, t0 + off, rbuf + off * tb, V, wbase, mtab, ln2, one, n4, [&]() {
                // the tile's LDS reads are complete (their values fed the V table)
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                if (ln2 == 0)
                    __hip_atomic_fetch_sub((lds_word *)(size_t)done_w(x), 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
            });
        }
        if (aborted || past) break;
    }
    if (aborted) {
        leave();
        return;
    }
    // this wave's tile stores are complete: count it finished
    const int ln = opaque_lane();
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    if (ln == 0)
        __hip_atomic_fetch_add((lds_word *)(size_t)kFusedFinishedOff, 1u, __ATOMIC_RELEASE,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    // every block of the workgroup complete; any failed?
    bool any_failed = false;
    for (uint32_t q = 0; q < Q; q++) {
        uint32_t w;
        if (!fused_poll(bit_w(kFusedFinalOff, q), ln, Fk.spin_limit, w,
                        [&](uint32_t b) { return (b & bit_m(q)) != 0u; })) {
            leave();
            return;
        }
        const uint32_t f = uniform(__hip_atomic_load((lds_word *)(size_t)bit_w(kFusedFailOff, q), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP));
        any_failed = any_failed || (f & bit_m(q)) != 0u;
    }
    if (!any_failed) {
        leave();
        return;
    }
    // rewrite the failed blocks' tiles (tile j of a block by wave j mod nw)
    // once every wave's own stores are complete
    {
        uint32_t c;
        if (!fused_poll(kFusedFinishedOff, ln, Fk.spin_limit, c, [&](uint32_t n) { return n == nw; })) {
            leave();
            return;
        }
    }
    constexpr uint32_t esz = DT == HH_F32 ? 4u : 2u;
    constexpr uint32_t per_row = 64u * esz / 16u;
    constexpr uint32_t rows_per = 64u / per_row;
    for (uint32_t q = 0; q < Q; q++) {
        const uint32_t f = uniform(__hip_atomic_load((lds_word *)(size_t)bit_w(kFusedFailOff, q), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP));
        if ((f & bit_m(q)) == 0u) continue;
        uint32_t bti, bt0, bnt, btb;
        locate(lb_of(q), bti, bt0, bnt, btb);
        const uint32_t cols = B.cols[bti], tpr = cols >> 6;
        uint8_t HH_GLOBAL *o = (uint8_t HH_GLOBAL *)B.out[bti];
        for (uint32_t j = wave; j < bnt; j += nw) {
            const uint32_t t = bt0 + j;
            const size_t base = (size_t)(64u * (t / tpr)) * cols + 64u * (t % tpr);
            for (uint32_t it = 0; it < 64u / rows_per; it++) {
                const uint32_t row = rows_per * it + (uint32_t)ln / per_row;
                *(u32x4 HH_GLOBAL *)(o + esz * (base + (size_t)row * cols) + 16u * ((uint32_t)ln % per_row)) =
                    u32x4{0u, 0u, 0u, 0u};
            }
            if (B.status[bti] != nullptr && ln == 0)
                ((int32_t HH_GLOBAL *)B.status[bti])[t] = HH_ERR_CORRUPTED_DATA;
        }
    }
    leave();
}

}  // namespace

hipError_t launch_hctt_decode(const hh_hctt_tensor *tensors, uint32_t n, int dtype,
                              const void *d_basis, int num_cus, hipStream_t s) {
    // each launch takes the next (up to) kMaxTensors non-empty tensors
    for (uint32_t i = 0; i < n;) {
        TileBatch B;
        std::memset(&B, 0, sizeof(B));
        uint32_t max_k = 0, total = 0;
        bool all_dw = true;
        for (; i < n && B.n < (uint32_t)kMaxTensors; i++) {
            const hh_hctt_tensor &T = tensors[i];
            const uint32_t nt = (T.rows / 64) * (T.cols / 64);
            if (nt == 0) continue;
            const uint32_t j = B.n++;
            const uint32_t tb = (uint32_t)hh_hctt_tile_bytes(T.k);
            B.tiles[j] = T.d_tiles;
            B.out[j] = T.d_out;
            B.status[j] = T.d_tile_status;
            B.start[j] = total;
            B.tpr_inv[j] = 1.0f / (float)(T.cols / 64);
            B.cols[j] = T.cols;
            B.k[j] = T.k;
            B.tb[j] = tb;
            const bool dword_ok = (tb & 3u) == 0 && ((uintptr_t)T.d_tiles & 3u) == 0;
            total += nt;
            max_k = T.k > max_k ? T.k : max_k;
            all_dw = all_dw && dword_ok;
        }
        if (B.n == 0) continue;
        B.start[B.n] = total;
        for (uint32_t j = B.n + 1; j <= (uint32_t)kMaxTensors; j++) B.start[j] = 0xffffffffu;
        B.one = 1.0f;
        B.neg4 = -4;
        // per wave: the V table (k words) shares space with the parked output
        // tile; the staged tile bytes follow (2 bytes of slack for the last
        // 16-bit nibble read)
        const uint32_t vbytes = 4 * ((max_k + 7u) & ~7u);  // whole 8-entry groups
        const uint32_t obytes = 64 * (dtype == HH_F32 ? kParkPitch<HH_F32> : kParkPitch<HH_BF16>);
        B.vo_bytes = ((vbytes > obytes ? vbytes : obytes) + 15u) & ~15u;
        uint32_t max_tb = 0;
        for (uint32_t j = 0; j < B.n; j++) max_tb = B.tb[j] > max_tb ? B.tb[j] : max_tb;
        // KiB of tile bytes prefetched per wave: the tile, up to 3 bytes of
        // alignment before it and the V build's 2-byte reads past its end
        const int np = max_tb + 8u <= 2048u ? 2 : 3;
        B.wave_lds = B.vo_bytes + 16u * 64u * (uint32_t)np;
        const uint32_t lds = kSharedBytes + B.wave_lds * kWaves;
        // workgroups per CU: what the registers allow, then the LDS
        uint32_t per_cu = (uint32_t)kWavesPerSimd(dtype, np);
        if (per_cu > (160u * 1024u) / lds) per_cu = (160u * 1024u) / lds;
        if (per_cu == 0) per_cu = 1;
        uint32_t grid = (uint32_t)(num_cus > 0 ? num_cus : 256) * per_cu;
        const uint32_t need = (total + kWaves - 1) / kWaves;
        if (grid > need) grid = need;
        const u32x4 *basis = reinterpret_cast<const u32x4 *>(d_basis);
        hipError_t e = hipSuccess;
#define HH_LAUNCH3(DTV, DWV, NPV)                                                                 \
    do {                                                                                          \
        e = hipFuncSetAttribute((const void *)hctt_decode_kernel<DTV, DWV, NPV>,                  \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);            \
        if (e != hipSuccess) return e;                                                            \
        hipLaunchKernelGGL((hctt_decode_kernel<DTV, DWV, NPV>), dim3(grid), dim3(kThreads), lds, \
                           s, B, basis);                                                          \
    } while (0)
#define HH_LAUNCH2(DTV, DWV)             \
    do {                                 \
        if (np == 2)                     \
            HH_LAUNCH3(DTV, DWV, 2);     \
        else                             \
            HH_LAUNCH3(DTV, DWV, 3);     \
    } while (0)
#define HH_LAUNCH(DTV)                  \
    do {                                \
        if (all_dw)                     \
            HH_LAUNCH2(DTV, true);      \
        else                            \
            HH_LAUNCH2(DTV, false);     \
    } while (0)
        switch (dtype) {
            case HH_F32: HH_LAUNCH(HH_F32); break;
            case HH_F16: HH_LAUNCH(HH_F16); break;
            case HH_BF16: HH_LAUNCH(HH_BF16); break;
            default: return hipErrorInvalidValue;
        }
#undef HH_LAUNCH
#undef HH_LAUNCH2
#undef HH_LAUNCH3
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}


hipError_t launch_hctt_lz4_fused(const hh_hctt_tensor *tensors, uint32_t n, const uint32_t *tpb, const uint8_t *d_in,
                                 uint64_t in_total, const uint64_t *d_in_off, const uint32_t *d_in_len,
                                 hh_block_status *d_status, int dtype, const void *d_basis, int num_cus,
                                 uint32_t poll_limit, bool seq_decoder, hipStream_t s) {
    uint32_t blk = 0;  // global block number of the next tensor's first block
    for (uint32_t i = 0; i < n;) {
        TileBatch B;
        FusedBlocks F;
        std::memset(&B, 0, sizeof(B));
        std::memset(&F, 0, sizeof(F));
        F.in = d_in;
        F.in_total = in_total;
        F.in_off = d_in_off;
        F.in_len = d_in_len;
        F.status = d_status;
        F.blk_base = blk;
        uint32_t max_k = 0, total = 0, nb = 0;
        for (; i < n && B.n < (uint32_t)kMaxTensors; i++) {
            const hh_hctt_tensor &T = tensors[i];
            const uint32_t nt = (T.rows / 64) * (T.cols / 64);
            if (nt == 0) continue;
            const uint32_t j = B.n++;
            B.out[j] = T.d_out;
            B.status[j] = T.d_tile_status;
            B.start[j] = total;
            B.tpr_inv[j] = 1.0f / (float)(T.cols / 64);
            B.cols[j] = T.cols;
            B.k[j] = T.k;
            B.tb[j] = (uint32_t)hh_hctt_tile_bytes(T.k);
            F.blk_start[j] = nb;
            F.tpb[j] = tpb[i];
            F.tpb_max = tpb[i] > F.tpb_max ? tpb[i] : F.tpb_max;
            total += nt;
            nb += (nt + tpb[i] - 1) / tpb[i];
            max_k = T.k > max_k ? T.k : max_k;
        }
        if (B.n == 0) continue;
        B.start[B.n] = total;
        F.blk_start[B.n] = nb;
        for (uint32_t j = B.n + 1; j <= (uint32_t)kMaxTensors; j++) B.start[j] = F.blk_start[j] = 0xffffffffu;
        B.one = 1.0f;
        B.neg4 = -4;
        // per wave: the V table shares space with the parked output tile, and
        // both with the input stage of a block the wave decodes
        const uint32_t vbytes = 4 * ((max_k + 7u) & ~7u);
        const uint32_t obytes = 64 * (dtype == HH_F32 ? kParkPitch<HH_F32> : kParkPitch<HH_BF16>);
        B.vo_bytes = ((vbytes > obytes ? vbytes : obytes) + 15u) & ~15u;
        B.wave_lds = B.vo_bytes > kFusedStage ? B.vo_bytes : (kFusedStage + 15u) & ~15u;
        // one workgroup per CU: kFusedMaxWaves waves (fewer when their areas
        // leave room for fewer than 3 block buffers)
        uint32_t nw = kFusedMaxWaves, nbuf = 0;
        for (;;) {
            const uint32_t used = kFusedWaveOff + nw * B.wave_lds;
            nbuf = used < kFusedLdsMax ? (kFusedLdsMax - used) / kFusedBuf : 0u;
            if (nbuf >= 3 || nw == 1) break;
            nw--;
        }
        if (nbuf < 2) return hipErrorInvalidValue;  // not reached: tiles are at most 3 KiB (k <= 4096)
        if (nbuf > kFusedMaxBufs) nbuf = kFusedMaxBufs;
        F.nbuf = nbuf;
        F.buf_off = kFusedWaveOff + nw * B.wave_lds;
        F.spin_limit = poll_limit >= 1 && poll_limit <= kSpinLimit ? poll_limit : kSpinLimit;
        const uint32_t lds = F.buf_off + nbuf * kFusedBuf;
        const uint32_t threads = 64u * nw;
        // workgroup g takes blocks g, g + grid, ...: at most kFusedMaxRange
        // of them (the bitmaps' size)
        uint32_t grid = (uint32_t)(num_cus > 0 ? num_cus : 256);
        if (grid > nb) grid = nb;
        if ((nb + grid - 1) / grid > kFusedMaxRange) grid = (nb + kFusedMaxRange - 1) / kFusedMaxRange;
        const u32x4 *basis = reinterpret_cast<const u32x4 *>(d_basis);
        hipError_t e = hipSuccess;
#define HH_LAUNCH_FUSED(DTV, SQ)                                                                            \
    do {                                                                                                    \
        e = hipFuncSetAttribute((const void *)hctt_lz4_fused_kernel<DTV, SQ>,                               \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                      \
        if (e != hipSuccess) return e;                                                                      \
        hipLaunchKernelGGL((hctt_lz4_fused_kernel<DTV, SQ>), dim3(grid), dim3(threads), lds, s, B, F, basis);   \
    } while (0)
        if (seq_decoder) {
            switch (dtype) {
                case HH_F32: HH_LAUNCH_FUSED(HH_F32, true); break;
                case HH_F16: HH_LAUNCH_FUSED(HH_F16, true); break;
                case HH_BF16: HH_LAUNCH_FUSED(HH_BF16, true); break;
                default: return hipErrorInvalidValue;
            }
        } else {
            switch (dtype) {
                case HH_F32: HH_LAUNCH_FUSED(HH_F32, false); break;
                case HH_F16: HH_LAUNCH_FUSED(HH_F16, false); break;
                case HH_BF16: HH_LAUNCH_FUSED(HH_BF16, false); break;
                default: return hipErrorInvalidValue;
            }
        }
#undef HH_LAUNCH_FUSED
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        blk += nb;
    }
    return hipSuccess;
}

uint32_t fused_block_max() { return kFusedMax; }

}  // namespace hh
