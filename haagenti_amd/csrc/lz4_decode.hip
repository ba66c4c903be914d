// Batched raw-LZ4 block decoder: one wavefront (64 lanes) per block.
//
// Semantics: crates/haagenti-lz4/src/block.rs:261-366 (decompress_block),
// including its error order and its early stop when the output reaches
// output_size.  Blocks are independent (offsets never reach before the
// block start), so a launch is just many waves.
//
// Per wave:
//  * Token parsing is wave-uniform (scalar registers).  The compressed
//    stream is read through a 256-byte register window (one dword per lane)
//    and bytes are picked out with v_readlane; the window at the byte after a
//    literal run is fetched before the run is copied, so its latency hides
//    behind the copy.
//  * Literal runs and non-overlapping matches are copied in destination-
//    aligned 16-byte chunks (one per lane, 1 KiB per wave instruction);
//    an unaligned source is realigned with v_alignbyte on 5 loaded dwords.
//  * Overlapping matches (offset < length) are periodic with period offset:
//    out[op + j] = out[op - offset + (j mod offset)], all of whose source
//    bytes precede op, so every lane copies independently.
//  * Every read is clamped to the caller's buffers and every write to the
//    block's output capacity; corrupt input yields a status, never an
//    out-of-bounds access.
//
// Matches read bytes the same wave wrote earlier in the same block; a wave's
// vector memory operations are performed in order, so no wait is needed
// between those stores and loads (a wavefront-scope fence keeps the compiler
// from reordering them).
#include "hh_internal.hpp"

namespace hh {
namespace {

constexpr int kWaves = 4;               // blocks per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kCopyUnroll = 4;

__device__ __forceinline__ void wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// Dword at 4-aligned address a; bytes outside [lo, hi) read as zero.
__device__ __forceinline__ uint32_t ld_dw(uintptr_t a, uintptr_t lo, uintptr_t hi) {
    if (a >= lo && a + 4 <= hi) return *reinterpret_cast<const uint32_t *>(a);
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const uintptr_t x = a + b;
        if (x >= lo && x < hi) v |= (uint32_t)(*reinterpret_cast<const uint8_t *>(x)) << (8 * b);
    }
    return v;
}

// dst[0..n) = src[0..n); [src, src+n) lies inside the readable [slo, shi).
__device__ __forceinline__ void wave_copy(uint8_t *dst, uintptr_t src, uint32_t n, uintptr_t slo,
                                          uintptr_t shi, int lane) {
    uint32_t head = (uint32_t)((16u - ((uintptr_t)dst & 15u)) & 15u);
    if (head > n) head = n;
    if (lane < (int)head) dst[lane] = *reinterpret_cast<const uint8_t *>(src + lane);
    dst += head;
    src += head;
    n -= head;
    const uint32_t nch = n >> 4;
    const uint32_t sh = (uint32_t)(src & 3u);
    const uintptr_t sal = src - sh;
    for (uint32_t c0 = 0; c0 < nch; c0 += 64 * kCopyUnroll) {
        uint4 o[kCopyUnroll];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; u++) {
            const uint32_t c = c0 + 64u * u + lane;
            if (c < nch) {
                const uintptr_t a = sal + 16u * (uintptr_t)c;
                uint32_t d0, d1, d2, d3, d4 = 0;
                if (a >= slo && a + 20 <= shi) {
                    const uint32_t *p = reinterpret_cast<const uint32_t *>(a);
                    d0 = p[0];
                    d1 = p[1];
                    d2 = p[2];
                    d3 = p[3];
                    if (sh) d4 = p[4];
                } else {
                    d0 = ld_dw(a, slo, shi);
                    d1 = ld_dw(a + 4, slo, shi);
                    d2 = ld_dw(a + 8, slo, shi);
                    d3 = ld_dw(a + 12, slo, shi);
                    if (sh) d4 = ld_dw(a + 16, slo, shi);
                }
                o[u].x = __builtin_amdgcn_alignbyte(d1, d0, sh);
                o[u].y = __builtin_amdgcn_alignbyte(d2, d1, sh);
                o[u].z = __builtin_amdgcn_alignbyte(d3, d2, sh);
                o[u].w = __builtin_amdgcn_alignbyte(d4, d3, sh);
            }
        }
#pragma unroll
        for (int u = 0; u < kCopyUnroll; u++) {
            const uint32_t c = c0 + 64u * u + lane;
            if (c < nch) reinterpret_cast<uint4 *>(dst)[c] = o[u];
        }
    }
    const uint32_t done = nch * 16u, tail = n - done;
    if (lane < (int)tail) dst[done + lane] = *reinterpret_cast<const uint8_t *>(src + done + lane);
}

// Periodic copy for offset < length: out[j] = out[j - off + ((j) mod off)]
// relative to the match start; sources all precede the destination.
__device__ __forceinline__ void wave_copy_periodic(uint8_t *dst, uint32_t off, uint32_t n,
                                                   int lane) {
    const uint8_t *src = dst - off;
    uint32_t m = (uint32_t)lane % off;
    const uint32_t step = 64u % off;
    for (uint32_t j0 = 0; j0 < n; j0 += 64 * 8) {
        uint8_t v[8];
        uint32_t mm = m;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t j = j0 + 64u * u + lane;
            if (j < n) v[u] = src[mm];
            mm += step;
            if (mm >= off) mm -= off;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t j = j0 + 64u * u + lane;
            if (j < n) dst[j] = v[u];
        }
        m = mm;
    }
}

__global__ __launch_bounds__(kThreads) void lz4_batch_kernel(
    const uint8_t *__restrict__ d_in, uint64_t in_total, const uint64_t *__restrict__ in_off,
    const uint32_t *__restrict__ in_len, uint8_t *d_out, const uint64_t *__restrict__ out_off,
    const uint32_t *__restrict__ out_cap, uint32_t nblocks, hh_block_status *__restrict__ status) {
    const int lane = threadIdx.x & 63;
    const uint32_t b = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (b >= nblocks) return;

    int32_t code = HH_OK, detail = HH_CORRUPT_NONE;
    uint64_t pos = 0, req = 0;
    uint32_t op = 0;

    const uint64_t ioff = in_off[b];
    const uint32_t ilen = in_len[b];
    uint8_t *out = d_out + out_off[b];
    const uint32_t cap = out_cap[b];

    if (ioff > in_total || (uint64_t)ilen > in_total - ioff) {
        code = HH_ERR_INVALID_ARGUMENT;
    } else {
        const uintptr_t glo = (uintptr_t)d_in, ghi = glo + in_total;
        const uintptr_t ilo = glo + ioff;
        const uintptr_t olo = (uintptr_t)out, ohi = olo + cap;

        uintptr_t wb = ilo & ~(uintptr_t)3;
        uint32_t w = ld_dw(wb + 4u * lane, glo, ghi);
        auto byte_at = [&](uint32_t p) -> uint32_t {
            const uintptr_t a = ilo + p;
            if (a < wb || a >= wb + 256) {
                wb = a & ~(uintptr_t)3;
                w = ld_dw(wb + 4u * lane, glo, ghi);
            }
            const uint32_t d = (uint32_t)(a - wb);
            return (__builtin_amdgcn_readlane(w, d >> 2) >> ((d & 3u) * 8u)) & 0xffu;
        };

        uint32_t ip = 0;
        while (ip < ilen) {
            const uint32_t token = byte_at(ip++);
            uint64_t ll = token >> 4;
            if (ll == 15) {
                for (;;) {
                    if (ip >= ilen) {
                        code = HH_ERR_UNEXPECTED_EOF;
                        pos = ip;
                        break;
                    }
                    const uint32_t x = byte_at(ip++);
                    ll += x;
                    if (x != 255) break;
                }
                if (code != HH_OK) break;
            }
            if (ll > 0) {
                if ((uint64_t)ip + ll > ilen) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ip;
                    break;
                }
                if ((uint64_t)op + ll > cap) {
                    code = HH_ERR_BUFFER_TOO_SMALL;
                    req = (uint64_t)op + ll;
                    break;
                }
                // prefetch the window that holds the next offset/token
                const uintptr_t na = ilo + ip + ll;
                wb = na & ~(uintptr_t)3;
                w = ld_dw(wb + 4u * lane, glo, ghi);
                wave_copy(out + op, ilo + ip, (uint32_t)ll, glo, ghi, lane);
                ip += (uint32_t)ll;
                op += (uint32_t)ll;
            }
            if (op >= cap) break;  // block.rs:309-311
            if ((uint64_t)ip + 2 > ilen) {
                code = HH_ERR_UNEXPECTED_EOF;
                pos = ip;
                break;
            }
            const uint32_t off = byte_at(ip) | (byte_at(ip + 1) << 8);
            ip += 2;
            if (off == 0) {
                code = HH_ERR_CORRUPTED_DATA;
                detail = HH_CORRUPT_ZERO_OFFSET;
                break;
            }
            if (off > op) {
                code = HH_ERR_CORRUPTED_DATA;
                detail = HH_CORRUPT_OFFSET_BEYOND;
                pos = op;
                break;
            }
            uint64_t ml = (token & 15u) + 4u;
            if ((token & 15u) == 15u) {
                for (;;) {
                    if (ip >= ilen) {
                        code = HH_ERR_UNEXPECTED_EOF;
                        pos = ip;
                        break;
                    }
                    const uint32_t x = byte_at(ip++);
                    ml += x;
                    if (x != 255) break;
                }
                if (code != HH_OK) break;
            }
            if ((uint64_t)op + ml > cap) {
                code = HH_ERR_BUFFER_TOO_SMALL;
                req = (uint64_t)op + ml;
                break;
            }
            wave_fence();
            if (off >= ml)
                wave_copy(out + op, olo + op - off, (uint32_t)ml, olo, ohi, lane);
            else
                wave_copy_periodic(out + op, off, (uint32_t)ml, lane);
            wave_fence();
            op += (uint32_t)ml;
        }
    }
    if (lane == 0) {
        hh_block_status st;
        st.code = code;
        st.detail = detail;
        st.position = pos;
        st.required = req;
        st.written = code == HH_OK ? op : 0;
        status[b] = st;
    }
}

}  // namespace

hipError_t launch_lz4_batch(const uint8_t *d_in, size_t in_total, const uint64_t *d_in_off,
                            const uint32_t *d_in_len, uint8_t *d_out, const uint64_t *d_out_off,
                            const uint32_t *d_out_cap, uint32_t nblocks, hh_block_status *d_status,
                            hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    const uint32_t grid = (nblocks + kWaves - 1) / kWaves;
    hipLaunchKernelGGL(lz4_batch_kernel, dim3(grid), dim3(kThreads), 0, s, d_in,
                       (uint64_t)in_total, d_in_off, d_in_len, d_out, d_out_off, d_out_cap, nblocks,
                       d_status);
    return hipGetLastError();
}

}  // namespace hh
