// XXH3-64 (seed 0, default secret): the checksum of HCT v2 containers.
//
// Reference call sites: crates/haagenti-hct/src/tensor.rs:729 (block
// checksums written by HctWriterV2), :794 (header checksum over bytes
// 0..56), :858 and :967 (HctReaderV2 validation); the function is
// xxhash-rust 0.8.15 `xxh3::xxh3_64`, an implementation of the published
// XXH3 algorithm (xxHash 0.8).  The default secret and the length classes
// (0-16, 17-128, 129-240, longer) are the algorithm's own and kept alike.
//
// Host: hh_xxh3_64 hashes one buffer.  Device: one wavefront per buffer.
// Inputs up to 240 bytes are hashed by lane 0 with the host code path.
// Longer inputs run the 64-byte-stripe accumulation on the whole wave: a
// 1 KiB block (16 stripes x 8 accumulator lanes) is 128 (stripe, lane)
// products, two per wave lane; the per-accumulator sums are reduced across
// the lanes and added, then the accumulators are scrambled as the algorithm
// does after every block.  The next block's bytes are loaded while the
// current one is reduced.  All sums are additions mod 2^64, so the order in
// which the wave adds a block's stripes does not change the result.
#include "hh_internal.hpp"

namespace hh {
namespace {

// The published algorithm's default 192-byte secret.
__host__ __device__ __forceinline__ const uint8_t *xxh3_secret();

constexpr uint32_t P32_1 = 0x9E3779B1u, P32_2 = 0x85EBCA77u, P32_3 = 0xC2B2AE3Du;
constexpr uint64_t P64_1 = 0x9E3779B185EBCA87ull, P64_2 = 0xC2B2AE3D27D4EB4Full,
                   P64_3 = 0x165667B19E3779F9ull, P64_4 = 0x85EBCA77C2B2AE63ull,
                   P64_5 = 0x27D4EB2F165667C5ull;
constexpr uint64_t PMX1 = 0x165667919E3779F9ull, PMX2 = 0x9FB21C651E98DF25ull;

#define HH_XXH3_SECRET_BYTES                                                                      \
    {0xb8, 0xfe, 0x6c, 0x39, 0x23, 0xa4, 0x4b, 0xbe, 0x7c, 0x01, 0x81, 0x2c, 0xf7, 0x21, 0xad, 0x1c, \
     0xde, 0xd4, 0x6d, 0xe9, 0x83, 0x90, 0x97, 0xdb, 0x72, 0x40, 0xa4, 0xa4, 0xb7, 0xb3, 0x67, 0x1f, \
     0xcb, 0x79, 0xe6, 0x4e, 0xcc, 0xc0, 0xe5, 0x78, 0x82, 0x5a, 0xd0, 0x7d, 0xcc, 0xff, 0x72, 0x21, \
     0xb8, 0x08, 0x46, 0x74, 0xf7, 0x43, 0x24, 0x8e, 0xe0, 0x35, 0x90, 0xe6, 0x81, 0x3a, 0x26, 0x4c, \
     0x3c, 0x28, 0x52, 0xbb, 0x91, 0xc3, 0x00, 0xcb, 0x88, 0xd0, 0x65, 0x8b, 0x1b, 0x53, 0x2e, 0xa3, \
     0x71, 0x64, 0x48, 0x97, 0xa2, 0x0d, 0xf9, 0x4e, 0x38, 0x19, 0xef, 0x46, 0xa9, 0xde, 0xac, 0xd8, \
     0xa8, 0xfa, 0x76, 0x3f, 0xe3, 0x9c, 0x34, 0x3f, 0xf9, 0xdc, 0xbb, 0xc7, 0xc7, 0x0b, 0x4f, 0x1d, \
     0x8a, 0x51, 0xe0, 0x4b, 0xcd, 0xb4, 0x59, 0x31, 0xc8, 0x9f, 0x7e, 0xc9, 0xd9, 0x78, 0x73, 0x64, \
     0xea, 0xc5, 0xac, 0x83, 0x34, 0xd3, 0xeb, 0xc3, 0xc5, 0x81, 0xa0, 0xff, 0xfa, 0x13, 0x63, 0xeb, \
     0x17, 0x0d, 0xdd, 0x51, 0xb7, 0xf0, 0xda, 0x49, 0xd3, 0x16, 0x55, 0x26, 0x29, 0xd4, 0x68, 0x9e, \
     0x2b, 0x16, 0xbe, 0x58, 0x7d, 0x47, 0xa1, 0xfc, 0x8f, 0xf8, 0xb8, 0xd1, 0x7a, 0xd0, 0x31, 0xce, \
     0x45, 0xcb, 0x3a, 0x8f, 0x95, 0x16, 0x04, 0x28, 0xaf, 0xd7, 0xfb, 0xca, 0xbb, 0x4b, 0x40, 0x7e}

__constant__ uint8_t d_secret[192] = HH_XXH3_SECRET_BYTES;
const uint8_t h_secret[192] = HH_XXH3_SECRET_BYTES;

__host__ __device__ __forceinline__ const uint8_t *xxh3_secret() {
#ifdef __HIP_DEVICE_COMPILE__
    return d_secret;
#else
    return h_secret;
#endif
}

// Little-endian reads that need no alignment (byte loads).
__host__ __device__ __forceinline__ uint64_t rd64(const uint8_t *p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; i--) v = (v << 8) | p[i];
    return v;
}
__host__ __device__ __forceinline__ uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__host__ __device__ __forceinline__ uint64_t rotl64(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }
__host__ __device__ __forceinline__ uint64_t bswap64(uint64_t v) {
    v = ((v & 0x00ff00ff00ff00ffull) << 8) | ((v >> 8) & 0x00ff00ff00ff00ffull);
    v = ((v & 0x0000ffff0000ffffull) << 16) | ((v >> 16) & 0x0000ffff0000ffffull);
    return (v << 32) | (v >> 32);
}
// low 64 ^ high 64 of the 128-bit product
__host__ __device__ __forceinline__ uint64_t fold128(uint64_t a, uint64_t b) {
#ifdef __HIP_DEVICE_COMPILE__
    return (a * b) ^ __umul64hi(a, b);
#else
    const unsigned __int128 m = (unsigned __int128)a * b;
    return (uint64_t)m ^ (uint64_t)(m >> 64);
#endif
}
__host__ __device__ __forceinline__ uint64_t avalanche3(uint64_t h) {
    h ^= h >> 37;
    h *= PMX1;
    return h ^ (h >> 32);
}
__host__ __device__ __forceinline__ uint64_t avalanche64(uint64_t h) {
    h ^= h >> 33;
    h *= P64_2;
    h ^= h >> 29;
    h *= P64_3;
    return h ^ (h >> 32);
}
__host__ __device__ __forceinline__ uint64_t mix16(const uint8_t *in, const uint8_t *sec) {
    return fold128(rd64(in) ^ rd64(sec), rd64(in + 8) ^ rd64(sec + 8));
}

// Inputs of at most 240 bytes (the algorithm's short and mid-size paths).
__host__ __device__ uint64_t xxh3_short(const uint8_t *in, size_t len) {
    const uint8_t *S = xxh3_secret();
    if (len == 0) return avalanche64(rd64(S + 56) ^ rd64(S + 64));
    if (len <= 3) {
        const uint32_t c = ((uint32_t)in[0] << 16) | ((uint32_t)in[len >> 1] << 24) | (uint32_t)in[len - 1] |
                           ((uint32_t)len << 8);
        return avalanche64((uint64_t)c ^ (uint64_t)(rd32(S) ^ rd32(S + 4)));
    }
    if (len <= 8) {
        uint64_t h = ((uint64_t)rd32(in + len - 4) + ((uint64_t)rd32(in) << 32)) ^ (rd64(S + 8) ^ rd64(S + 16));
        h ^= rotl64(h, 49) ^ rotl64(h, 24);
        h *= PMX2;
        h ^= (h >> 35) + len;
        h *= PMX2;
        return h ^ (h >> 28);
    }
    if (len <= 16) {
        const uint64_t lo = rd64(in) ^ (rd64(S + 24) ^ rd64(S + 32));
        const uint64_t hi = rd64(in + len - 8) ^ (rd64(S + 40) ^ rd64(S + 48));
        return avalanche3(len + bswap64(lo) + hi + fold128(lo, hi));
    }
    uint64_t acc = len * P64_1;
    if (len <= 128) {
        for (size_t i = 0; i <= (len - 1) / 32; i++) {  // from both ends inwards
            acc += mix16(in + 16 * i, S + 32 * i);
            acc += mix16(in + len - 16 * (i + 1), S + 32 * i + 16);
        }
        return avalanche3(acc);
    }
    for (int i = 0; i < 8; i++) acc += mix16(in + 16 * i, S + 16 * i);
    uint64_t tail = mix16(in + len - 16, S + 119);
    acc = avalanche3(acc);
    for (size_t i = 8; i < len / 16; i++) tail += mix16(in + 16 * i, S + 16 * (i - 8) + 3);
    return avalanche3(acc + tail);
}

__host__ __device__ __forceinline__ void stripe(uint64_t acc[8], const uint8_t *in, const uint8_t *sec) {
    for (int i = 0; i < 8; i++) {
        const uint64_t v = rd64(in + 8 * i), k = v ^ rd64(sec + 8 * i);
        acc[i ^ 1] += v;
        acc[i] += (k & 0xffffffffull) * (k >> 32);
    }
}
__host__ __device__ __forceinline__ uint64_t finalize(const uint64_t acc[8], size_t len) {
    const uint8_t *S = xxh3_secret();
    uint64_t r = len * P64_1;
    for (int i = 0; i < 4; i++)
        r += fold128(acc[2 * i] ^ rd64(S + 11 + 16 * i), acc[2 * i + 1] ^ rd64(S + 19 + 16 * i));
    return avalanche3(r);
}

uint64_t xxh3_host(const uint8_t *in, size_t len) {
    if (len <= 240) return xxh3_short(in, len);
    const uint8_t *S = xxh3_secret();
    uint64_t acc[8] = {P32_3, P64_1, P64_2, P64_3, P64_4, P32_2, P64_5, P32_1};
    const size_t nb = (len - 1) / 1024;
    for (size_t b = 0; b < nb; b++) {
        for (int s = 0; s < 16; s++) stripe(acc, in + 1024 * b + 64 * s, S + 8 * s);
        for (int i = 0; i < 8; i++) acc[i] = (acc[i] ^ (acc[i] >> 47) ^ rd64(S + 128 + 8 * i)) * P32_1;
    }
    const size_t ns = ((len - 1) - 1024 * nb) / 64;
    for (size_t s = 0; s < ns; s++) stripe(acc, in + 1024 * nb + 64 * s, S + 8 * s);
    stripe(acc, in + len - 64, S + 121);
    return finalize(acc, len);
}

// ---------------------------------------------------------------- device
constexpr int kWaves = 4;

// Eight input bytes at p (any alignment) from dword loads; bytes outside
// [lo, hi) read as zero (they only occur past the last stripe).
__device__ __forceinline__ uint64_t ld64(const uint8_t *p, const uint8_t *lo, const uint8_t *hi) {
    const uint8_t *a = (const uint8_t *)((uintptr_t)p & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
    uint32_t w[3];
    if (a >= lo && a + 12 <= hi) {
#pragma unroll
        for (int k = 0; k < 3; k++) w[k] = reinterpret_cast<const uint32_t *>(a)[k];
    } else {
#pragma unroll
        for (int k = 0; k < 3; k++) {
            uint32_t v = 0;
            for (int b = 0; b < 4; b++)
                if (a + 4 * k + b >= lo && a + 4 * k + b < hi) v |= (uint32_t)a[4 * k + b] << (8 * b);
            w[k] = v;
        }
    }
    const uint32_t x = __builtin_amdgcn_alignbyte(w[1], w[0], sh), y = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
    return (uint64_t)x | ((uint64_t)y << 32);
}

// Eight input bytes at abase + off + sh (abase 4-byte aligned and
// wave-uniform, off a multiple of 4, sh = the input's address mod 4), when
// every byte read lies inside the buffer: scalar base plus a 32-bit lane
// offset, no per-lane checks.
__device__ __forceinline__ uint64_t ld64_in(const uint8_t *abase, uint32_t off, uint32_t sh) {
    uint32_t w[3];
#pragma unroll
    for (int k = 0; k < 3; k++) w[k] = *reinterpret_cast<const uint32_t *>(abase + off + 4 * k);
    const uint32_t x = __builtin_amdgcn_alignbyte(w[1], w[0], sh), y = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
    return (uint64_t)x | ((uint64_t)y << 32);
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}

__global__ __launch_bounds__(64 * kWaves) void xxh3_batch_kernel(const uint8_t *__restrict__ data,
                                                                 uint64_t data_len,
                                                                 const uint64_t *__restrict__ off,
                                                                 const uint32_t *__restrict__ len,
                                                                 uint32_t n, uint64_t *__restrict__ out) {
    __shared__ uint8_t sec[192 + 16];
    for (int i = threadIdx.x; i < 192; i += blockDim.x) sec[i] = d_secret[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    // wave-uniform (scalar): the block's offset, length and base follow
    const uint32_t b = blockIdx.x * kWaves + (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (b >= n) return;
    const uint64_t o = off[b];
    const uint32_t L = len[b];
    if (o > data_len || L > data_len - o) {  // outside the buffer: report 0 (the caller checks ranges)
        if (lane == 0) out[b] = 0;
        return;
    }
    const uint8_t *in = data + o;
    const uint8_t *lo = data, *hi = data + data_len;
    if (L <= 240) {
        if (lane == 0) out[b] = xxh3_short(in, L);
        return;
    }
    // lane = 8 s + i: stripes s and s + 8 of a block, accumulator i
    const int i = lane & 7, s = lane >> 3;
    const uint64_t k0 = rd64(sec + 8 * s + 8 * i), k1 = rd64(sec + 8 * (s + 8) + 8 * i);
    const uint64_t ks = rd64(sec + 128 + 8 * i);  // scramble key
    const uint64_t init[8] = {P32_3, P64_1, P64_2, P64_3, P64_4, P32_2, P64_5, P32_1};
    uint64_t acc = init[i];
    // per-lane contribution of one block: its products go to accumulator i,
    // its input words to accumulator i ^ 1 (exchanged with the neighbour lane)
    auto reduce = [&](uint64_t prod, uint64_t val) {
        uint64_t t = prod + shfl_xor64(val, 1);
        t += shfl_xor64(t, 8);
        t += shfl_xor64(t, 16);
        t += shfl_xor64(t, 32);
        return t;
    };
    const uint32_t nb = (L - 1) / 1024;
    uint64_t v0 = 0, v1 = 0;
    if (nb > 0) {
        v0 = ld64(in + 64 * s + 8 * i, lo, hi);
        v1 = ld64(in + 64 * (s + 8) + 8 * i, lo, hi);
    }
    for (uint32_t blk = 0; blk < nb; blk++) {
        uint64_t n0 = 0, n1 = 0;
        if (blk + 1 < nb) {  // next block's words, loaded before this one is reduced
            const uint8_t *nbk = in + 1024 * (size_t)(blk + 1);
            const uint8_t *ab = (const uint8_t *)((uintptr_t)nbk & ~(uintptr_t)3);
            if (ab >= lo && ab + 1024 + 12 <= hi) {  // the block's words inside the buffer
                const uint32_t sh = (uint32_t)((uintptr_t)nbk & 3u);
                n0 = ld64_in(ab, 64u * s + 8u * i, sh);
                n1 = ld64_in(ab, 64u * (s + 8) + 8u * i, sh);
            } else {
                n0 = ld64(nbk + 64 * s + 8 * i, lo, hi);
                n1 = ld64(nbk + 64 * (s + 8) + 8 * i, lo, hi);
            }
        }
        const uint64_t x0 = v0 ^ k0, x1 = v1 ^ k1;
        const uint64_t prod = (x0 & 0xffffffffull) * (x0 >> 32) + (x1 & 0xffffffffull) * (x1 >> 32);
        acc += reduce(prod, v0 + v1);
        acc = (acc ^ (acc >> 47) ^ ks) * P32_1;
        v0 = n0;
        v1 = n1;
    }
    // last partial block: stripes [0, ns) of block nb, then the last stripe
    const uint32_t ns = ((L - 1) - 1024 * nb) / 64;
    uint64_t prod = 0, val = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int st = s + 8 * h;
        if ((uint32_t)st < ns) {
            const uint64_t v = ld64(in + 1024 * (size_t)nb + 64 * st + 8 * i, lo, hi);
            const uint64_t x = v ^ (h ? k1 : k0);
            prod += (x & 0xffffffffull) * (x >> 32);
            val += v;
        }
    }
    if (s == 0) {
        const uint64_t v = ld64(in + L - 64 + 8 * i, lo, hi);
        const uint64_t x = v ^ rd64(sec + 121 + 8 * i);
        prod += (x & 0xffffffffull) * (x >> 32);
        val += v;
    }
    acc += reduce(prod, val);
    uint64_t a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t alo = __builtin_amdgcn_readlane((uint32_t)acc, j);
        const uint32_t ahi = __builtin_amdgcn_readlane((uint32_t)(acc >> 32), j);
        a[j] = (uint64_t)alo | ((uint64_t)ahi << 32);
    }
    if (lane == 0) out[b] = finalize(a, L);
}

}  // namespace

hipError_t launch_xxh3_batch(const uint8_t *d_data, size_t data_len, const uint64_t *d_off,
                             const uint32_t *d_len, uint32_t n, uint64_t *d_out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(xxh3_batch_kernel, dim3((n + kWaves - 1) / kWaves), dim3(64 * kWaves), 0, s, d_data,
                       (uint64_t)data_len, d_off, d_len, n, d_out);
    return hipGetLastError();
}

uint64_t xxh3_64_host(const uint8_t *data, size_t len) { return xxh3_host(data, len); }

}  // namespace hh
