// Internal declarations shared by the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "../../include/haagenti_hip.h"

struct hh_context {
    int device = 0;
    hipStream_t stream = nullptr;
    int num_cus = 0;
    // 64x64 inverse-DCT basis, pre-split into f16 hi/lo MFMA fragments in
    // per-lane order (see hctt_decode.hip), uploaded once per context.
    void *d_basis = nullptr;
    // Device scratch used by the host-pointer and whole-tensor entry points
    // (grown on demand, kept until the context is destroyed).
    void *d_scratch = nullptr;
    size_t scratch_bytes = 0;
    // Whole-matrix DCT bases as f16 hi / lo planes (dct_gemm.hip), two
    // cached: kind 0 B_n, 1 B_n^T, 2 the even / odd split of B_n^T.
    struct Basis {
        uint32_t n = 0;
        int kind = 0;
        uint16_t *hl = nullptr;  // hi plane then lo plane
        uint64_t stamp = 0;
    };
    Basis dct_basis[2];
    uint64_t dct_stamp = 0;
    // scratch of the whole-matrix transforms: block maxima, scale constants
    // and the f16 planes of the input and of the intermediate product
    void *d_split = nullptr;
    size_t split_bytes = 0;
    // Device address of the library-owned tile-byte array of
    // hh_hctt_decode_lz4_batch_noalloc on this context's device, looked up
    // at context creation (capi_noalloc.hip), and the lookup's result.
    uint8_t *noalloc_scratch = nullptr;
    hipError_t noalloc_status = hipErrorNotInitialized;
    // hh_context_set_option settings: the LZ4 decoder (hh_lz4_decoder), the
    // poll limit of the fused decode's waits (0: the default)
    int32_t lz4_decoder = HH_LZ4_AUTO;
    uint32_t fused_poll_limit = 0;
    // how hh_pipeline_submit decodes a unit's tensors (hh_pipeline_route)
    int32_t pipeline_route = HH_PIPE_AUTO;
    // whole-matrix transform route (hh_dct_route), the FFT route's twiddle
    // tables (two lengths cached) and its two f32 matrices of scratch
    int32_t dct_route = HH_DCT_AUTO;
    struct FftTables {
        uint32_t n = 0;
        void *tab = nullptr;
        uint64_t stamp = 0;
    };
    FftTables fft_tab[2];
    void *d_fft = nullptr;
    size_t fft_bytes = 0;
};

namespace hh {

// Checks of one tensor of the tile decode (capi.hip): rows and cols
// multiples of 64 (cols at most 2^24), 1 <= k <= 4096, tile bytes for every
// tile, d_tiles set and d_out 16-byte aligned; *ntiles its tile count.
int32_t check_hctt_tensor(const hh_hctt_tensor &T, size_t *ntiles);
// hipError_t -> hh_status; grows ctx->d_scratch to at least `bytes`
// (capi.hip).
int32_t from_hip(hipError_t e);
int32_t ensure_scratch(hh_context *ctx, size_t bytes);
// Device address of the no-allocation entry point's array on `device`
// (which must be current), looked up once per device (capi_noalloc.hip).
hipError_t noalloc_scratch(int device, uint8_t **out);

// Makes a device current for the lifetime of the guard and restores the
// calling thread's previous current device afterwards, so an entry point
// leaves the caller's device selection as it found it.  `status` is the
// result of the switch (hipSuccess when nothing needed to change).
class DeviceGuard {
  public:
    explicit DeviceGuard(int device) {
        int cur = -1;
        status_ = hipGetDevice(&cur);
        if (status_ != hipSuccess) return;
        if (cur != device) {
            status_ = hipSetDevice(device);
            if (status_ == hipSuccess) prev_ = cur;
        }
    }
    ~DeviceGuard() {
        if (prev_ >= 0) (void)hipSetDevice(prev_);
    }
    DeviceGuard(const DeviceGuard &) = delete;
    DeviceGuard &operator=(const DeviceGuard &) = delete;
    hipError_t status() const { return status_; }

  private:
    hipError_t status_ = hipSuccess;
    int prev_ = -1;
};

// ---- device helpers -------------------------------------------------------

// f16 bit pattern -> f32, exact for every code, NaN payload kept
// (crates/haagenti/src/testing/quantization.rs:166-197).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t frac = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1fu) {
        bits = sign | 0x7f800000u | (frac << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (frac << 13);
    } else if (frac == 0) {
        bits = sign;
    } else {
        // subnormal: value = frac * 2^-24, normalise with a leading-zero count
        uint32_t lz = __clz(frac) - 21;          // shifts to bring bit 10 up
        uint32_t f = (frac << lz) & 0x3ffu;
        bits = sign | ((113u - lz) << 23) | (f << 13);
    }
    return __uint_as_float(bits);
}

// Zero-fills out[0, cap) from one wavefront (every lane calls it with its
// lane index): the output range of an LZ4 block whose decode failed, so no
// byte of an earlier use of the buffer survives there (a tile whose bitmap
// reads as zeros then fails its popcount check instead of decoding stale
// bytes).  Stores of the same wave to the same address land in order, so
// this overrides whatever the decoder wrote before the failure.
__device__ __forceinline__ void wave_zero_fill(uint8_t *out, uint32_t cap, int lane) {
    typedef uint32_t u32x4z __attribute__((ext_vector_type(4)));
    uint32_t head = (uint32_t)((16u - ((uintptr_t)out & 15u)) & 15u);
    if (head > cap) head = cap;
    if ((uint32_t)lane < head) out[lane] = 0;
    uint8_t *body = out + head;
    const uint32_t nch = (cap - head) >> 4, tail = (cap - head) & 15u;
    for (uint32_t c = (uint32_t)lane; c < nch; c += 64)
        reinterpret_cast<u32x4z *>(body)[c] = u32x4z{0u, 0u, 0u, 0u};
    if ((uint32_t)lane < tail) body[16u * nch + (uint32_t)lane] = 0;
}

// f32 -> bf16 round-to-nearest-even; NaN stays a (quiet) NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// f32 -> f16 round-to-nearest-even (hardware conversion, default round mode).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// ---- launchers (return hipSuccess or the launch error) ---------------------

hipError_t launch_dequant_int4(const uint8_t *d_q, size_t n, size_t nscale_groups,
                               int dtype, void *d_out, int num_cus, hipStream_t s);

// One batched LZ4 decode: block i reads in[in_off[i], +in_len[i]) (ranges
// outside [0, in_total) are reported as HH_ERR_INVALID_ARGUMENT) and writes
// at most out_cap[i] bytes at out + out_off[i]; a block whose output range
// leaves [0, out_total) is reported the same way and writes nothing.
struct Lz4Batch {
    const uint8_t *in;
    uint64_t in_total;
    const uint64_t *in_off;
    const uint32_t *in_len;
    uint8_t *out;
    uint64_t out_total;
    const uint64_t *out_off;
    const uint32_t *out_cap;
    uint32_t nblocks;
    hh_block_status *status;
    // tile layer entries: a block that decodes short (no error, fewer bytes
    // than its capacity) zeroes the rest of its capacity, so the tiles there
    // fail their bitmap count instead of reading what the buffer held
    uint32_t zero_tail = 0;
};

// Batched LZ4 with the decoder `decoder` (hh_lz4_decoder; HH_LZ4_AUTO is
// resolved by the caller): the sequence-batched decoder (lz4_seq.hip), the
// one-sequence-at-a-time LDS ring decoder (lz4_ring.hip) or the
// register-window decoder (lz4_decode.hip).
hipError_t launch_lz4_batch(const Lz4Batch &B, int32_t decoder, hipStream_t s);
// The context's decoder for an entry point whose default is `dflt`.
inline int32_t lz4_decoder_for(const hh_context *ctx, int32_t dflt) {
    return ctx->lz4_decoder == HH_LZ4_AUTO ? dflt : ctx->lz4_decoder;
}
// The automatic decoder of a launch whose LZ4 blocks hold the tiles of
// these tensors: tiles of retention below 25 % (k < 1024) compress into
// blocks of many short LZ4 sequences (runs of the sparse bitmaps), which the
// sequence-batched decoder copies many at a time; denser tiles leave a few
// long runs per block, which the one-sequence ring decoder copies faster.
inline int32_t lz4_decoder_for_tiles(const hh_context *ctx, const hh_hctt_tensor *tensors, uint32_t n) {
    bool sparse = false;
    for (uint32_t i = 0; i < n; i++) sparse = sparse || tensors[i].k < 1024u;
    return lz4_decoder_for(ctx, sparse ? HH_LZ4_SEQ : HH_LZ4_RING4);
}
hipError_t launch_lz4_seq(const Lz4Batch &B, uint32_t ring_kib, hipStream_t s);
hipError_t launch_lz4_ring(const Lz4Batch &B, uint32_t ring_kib, hipStream_t s);

hipError_t launch_xxh3_batch(const uint8_t *d_data, size_t data_len, const uint64_t *d_off,
                             const uint32_t *d_len, uint32_t n, uint64_t *d_out, hipStream_t s);
uint64_t xxh3_64_host(const uint8_t *data, size_t len);

// Build the MFMA basis fragments on the host (host_basis.cpp).
size_t basis_table_bytes();
void build_basis_table(void *host_buf);

// HCT3 whole-tensor decode (hct3_decode.hip).  Scatter: the set bits of the
// nbits-bit bitmap (64-bit words, 8-byte aligned) take coefficients (f16 or
// f32, little-endian at any byte address) in rank order while rank < ncoef; `first` writes every output (zeros where no
// value lands), otherwise only the assigned ones.  d_block_sums needs
// hct3_block_sums_bytes(nbits).
hipError_t launch_hct3_scatter(const uint64_t *d_bits, uint64_t nbits, uint32_t *d_block_sums,
                               const void *d_coef, uint32_t ncoef, int coef_f32, float *d_dense,
                               int first, hipStream_t s);
size_t hct3_block_sums_bytes(uint64_t nbits);
// Bitmap bytes at any device address -> zero-padded 64-bit words.
hipError_t launch_pack_bits(const uint8_t *d_src, uint64_t nbytes, uint64_t *d_words, hipStream_t s);
// In-place exclusive scan of n 32-bit counts (one workgroup).
hipError_t launch_scan_counts(uint32_t *d, uint32_t n, hipStream_t s);
hipError_t launch_f32_convert(const float *d_x, uint64_t n, int dtype, void *d_out, hipStream_t s);
// One HCT3 fragment in device memory: its bitmap bytes and its f16
// coefficient values (both at any byte address).
struct Hct3Frag {
    const uint8_t *bitmap;
    const uint8_t *coef;
    uint32_t ncoef;
};
// The h x w HCT3 decode straight to d_out (dtype): the fragments' values,
// scaled by a power of two from the largest of them, scattered in order
// into the operand plane of the even / odd split inverse DCT, then its two
// products.  d_stage holds hct3_block_sums_bytes(h w) rounded up to 16 plus
// the bitmap words.  HH_ERR_UNSUPPORTED (nothing enqueued) unless h and w
// are multiples of 512, d_out is aligned (16 bytes f32, 8 bytes 16-bit) and
// there are 1..16 fragments.
int32_t hct3_decode_eo(hh_context *ctx, const Hct3Frag *frags, uint32_t nfrags, uint32_t h, uint32_t w,
                       int32_t dtype, void *d_out, uint8_t *d_stage, hipStream_t s);
// One split-f16 MFMA product D = s_out * A Bt^T (dct_gemm.hip).  A (M x K)
// and Bt (N x K) are f16 hi / lo planes, row-major with k contiguous,
// dct_planes_rows(rows) x dct_planes_cols(K) with zeros past the matrix;
// b_lo null: Bt has no low half.  D: M x N (row stride ldd) in d_dtype, or
// with d_planes the hi / lo planes of the next product's Bt (its padded
// extent, zeros included; lo follows hi at dct_planes_rows(M) x
// dct_planes_cols(N) elements).
// lda / ldb: the planes' row strides when not dct_planes_cols(K) (0: that);
// rows m >= m_split (when not 0, a multiple of 256) read Bt from column
// b_koff on.
struct DctGemm {
    const uint16_t *a_hi, *a_lo, *b_hi, *b_lo;
    const float *out_scale;  // device scalar, or null for 1
    void *d;
    uint32_t ldd;
    int32_t d_dtype;
    bool d_planes;
    uint32_t M, N, K;
    uint32_t lda = 0, ldb = 0, m_split = 0, b_koff = 0;
};
hipError_t launch_dct_gemm(const DctGemm &p, hipStream_t s);
uint32_t dct_planes_rows(uint32_t n);
uint32_t dct_planes_cols(uint32_t n);
// hi / lo planes of B_n (P[m][k] = B_n[m][k]) or of B_n^T.
hipError_t launch_dct_basis_planes(uint16_t *hi, uint16_t *lo, uint32_t n, bool transposed, hipStream_t s);
// The even / odd split of B_n^T (n a multiple of 512): an n x n/2 plane
// pair, rows m < n/2 holding B_n[2k][m] and rows n/2 + m holding
// B_n[2k + 1][m] (k < n/2).
hipError_t launch_dct_basis_split_planes(uint16_t *hi, uint16_t *lo, uint32_t n, hipStream_t s);
// launch_operand_planes with the columns in even / odd order (column k to
// k / 2, or cols / 2 + k / 2 when odd; cols a multiple of 32).
hipError_t launch_operand_planes_eo(const float *x, uint32_t rows, uint32_t cols, uint32_t ld, const float *scale,
                                    uint16_t *hi, uint16_t *lo, hipStream_t s);
// The butterfly of an even / odd split product: y (2 mh x n f32, row stride
// n) holds E in rows [0, mh) and O in rows [mh, 2 mh); row m of the result
// is E_m + O_m and row 2 mh - 1 - m is E_m - O_m (m < mh).  eo_planes: the
// result as f16 hi / lo planes with its columns in even / odd order (the
// next product's Bt, 2 mh x n, lo at 2 mh n elements after hi); else the
// result times *scale (null: 1) in dtype, row stride ldd.
hipError_t launch_dct_butterfly(const float *y, uint32_t mh, uint32_t n, bool eo_planes, const float *scale,
                                int32_t dtype, void *out, uint32_t ldd, hipStream_t s);
// hi (and lo, unless null) planes of an f32 rows x cols matrix (row stride
// ld) times *scale.
hipError_t launch_operand_planes(const float *x, uint32_t rows, uint32_t cols, uint32_t ld, const float *scale,
                                 uint16_t *hi, uint16_t *lo, hipStream_t s);

// Orthonormal 2-D DCT-III (inverse) or DCT-II (forward) of a row-major
// rows x cols f32 matrix: two split-f16 MFMA products through d_tmp
// (rows*cols f32); d_out may not alias d_in or d_tmp.  f16_exact: every
// input value is an f16 value (the first product then skips the pass of the
// input's low f16 half).  cvt_out: a 16-bit output (cvt_dtype) the inverse
// may write directly from its last pass, reported in *converted (d_out then
// is not written).
int32_t dct2d_full(hh_context *ctx, bool inverse, const float *d_in, float *d_tmp, float *d_out,
                   uint32_t rows, uint32_t cols, hipStream_t s, bool f16_exact = false,
                   int32_t cvt_dtype = HH_F32, void *cvt_out = nullptr, bool *converted = nullptr);
void release_dct_resources(hh_context *ctx);

// FFT route of the whole-matrix transforms (dct_fft.hip).  fft_supported:
// n a multiple of 64 whose half factors into 2, 3, 5, 7 and fits in LDS.
// use_fft: the route the context's setting takes for a rows x cols matrix
// (HH_DCT_AUTO: both sides supported and the larger at least kFftAutoMin).
// fft_scratch: two f32 matrices of `total` elements from the context.
// dct2d_fft: the orthonormal 2-D DCT-II (forward) or DCT-III of the h x w
// d_in into d_out (out_dtype; 16-byte aligned f32 or 8-byte aligned 16-bit;
// the forward's d_in 16-byte aligned), with d_a and d_b (fft_scratch) as the
// intermediates; d_in may be d_a.
constexpr uint32_t kFftAutoMin = 1024;
bool fft_supported(uint32_t n);
bool use_fft(const hh_context *ctx, uint32_t rows, uint32_t cols);
int32_t fft_scratch(hh_context *ctx, uint64_t total, hipStream_t s, float **a, float **b);
int32_t dct2d_fft(hh_context *ctx, bool inverse, const float *d_in, float *d_a, float *d_b, uint32_t h,
                  uint32_t w, int32_t out_dtype, void *d_out, hipStream_t s);
void release_fft_resources(hh_context *ctx);
// The h x w HCT3 decode on the FFT route with the fragments scattered in
// order (HCT3 rules) straight into the first row pass's LDS; d_out as for
// dct2d_fft.  HH_ERR_UNSUPPORTED (nothing launched) when the shape or
// fragment count leaves that fused pass's limits (more than 16 fragments,
// a row's inputs past 8 per thread or past the LDS).
int32_t hct3_decode_fft(hh_context *ctx, const Hct3Frag *frags, uint32_t nfrags, uint32_t h, uint32_t w,
                        int32_t dtype, void *d_out, hipStream_t s);
// zstd::decode_all on the host (host_zstd.cpp): false on a malformed stream.
bool zstd_decode_all(const uint8_t *in, size_t len, std::vector<uint8_t> &out);

// Decodes n tensors (validated by the caller) in ceil(n/8) launches.
hipError_t launch_hctt_decode(const hh_hctt_tensor *tensors, uint32_t n, int dtype,
                              const void *d_basis, int num_cus, hipStream_t s);
// LZ4 blocks of whole tiles decoded and their tiles decoded from LDS in one
// launch per 8 tensors (hctt_decode.hip; validated by the caller: tensor i's
// blocks are the next ceil(ntiles_i / tpb[i]) of d_in_off / d_in_len, each
// tpb[i] * tile bytes <= fused_block_max()).
// poll_limit: polls before a wait gives up (0: the default 2^24);
// seq_decoder: blocks decoded by the sequence-batched decoder (else the
// one-sequence ring decoder).
hipError_t launch_hctt_lz4_fused(const hh_hctt_tensor *tensors, uint32_t n, const uint32_t *tpb, const uint8_t *d_in,
                                 uint64_t in_total, const uint64_t *d_in_off, const uint32_t *d_in_len,
                                 hh_block_status *d_status, int dtype, const void *d_basis, int num_cus,
                                 uint32_t poll_limit, bool seq_decoder, hipStream_t s);
uint32_t fused_block_max();

}  // namespace hh
