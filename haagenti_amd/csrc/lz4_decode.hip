// Batched raw-LZ4 block decoder: one wavefront (64 lanes) per block.
//
// Semantics: crates/haagenti-lz4/src/block.rs:261-366 (decompress_block),
// including its error order and its early stop when the output reaches
// output_size.  Blocks are independent (offsets never reach before the
// block start), so a launch is just many waves.
//
// Per wave:
//  * Token parsing is wave-uniform (scalar registers).  The compressed
//    stream is read through a 256-byte register window (one dword per lane);
//    single bytes are picked out with v_readlane, and a run of 255-valued
//    length-extension bytes is measured with one ballot per window instead of
//    byte by byte.  The window at the byte after a literal run is fetched
//    before the run is copied, so its latency hides behind the copy.
//  * Literal runs and non-overlapping matches are copied in destination-
//    aligned 16-byte chunks, one per lane (1 KiB per wave instruction), as a
//    software pipeline that keeps two groups of kCopyUnroll chunks in flight;
//    an unaligned source is realigned with v_alignbyte on 5 loaded dwords.
//    Only chunks whose reads could leave the caller's buffer take a clamped
//    byte-wise path.
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
#include <cstdlib>
#include <cstring>

#include "hh_internal.hpp"

namespace hh {
namespace {

constexpr int kWaves = 4;  // blocks per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kCopyUnroll = 4;

// Compiler-only ordering point between a match's stores and the next
// sequence's loads; the hardware already performs a wave's vector memory
// operations in order, so no wait instruction is emitted.
__device__ __forceinline__ void wave_fence() { __asm__ __volatile__("" ::: "memory"); }

// Dword at 4-aligned p; bytes outside [lo, hi) read as zero.
__device__ __forceinline__ uint32_t ld_dw_clamped(const uint8_t *__restrict__ p,
                                                  const uint8_t *__restrict__ lo,
                                                  const uint8_t *__restrict__ hi) {
    if (p >= lo && p + 4 <= hi) return *reinterpret_cast<const uint32_t *>(p);
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; b++)
        if (p + b >= lo && p + b < hi) v |= (uint32_t)p[b] << (8 * b);
    return v;
}

struct Chunk {
    uint32_t d[5];
};

__device__ __forceinline__ uint4 realign(const Chunk &c, uint32_t sh) {
    uint4 o;
    o.x = __builtin_amdgcn_alignbyte(c.d[1], c.d[0], sh);
    o.y = __builtin_amdgcn_alignbyte(c.d[2], c.d[1], sh);
    o.z = __builtin_amdgcn_alignbyte(c.d[3], c.d[2], sh);
    o.w = __builtin_amdgcn_alignbyte(c.d[4], c.d[3], sh);
    return o;
}

// dst[0..n) = src[0..n).  [src, src+n) lies inside the readable [lo, hi).
// dst and src may point into the same buffer (non-overlapping matches), so
// neither is declared __restrict__.
__device__ __forceinline__ void wave_copy(uint8_t *dst, const uint8_t *src, uint32_t n,
                                          const uint8_t *__restrict__ lo,
                                          const uint8_t *__restrict__ hi, int lane) {
    uint32_t head = (uint32_t)((16u - ((uintptr_t)dst & 15u)) & 15u);
    if (head > n) head = n;
    if (lane < (int)head) dst[lane] = src[lane];
    dst += head;
    src += head;
    n -= head;
    const uint32_t nch = n >> 4;
    const uint32_t sh = (uint32_t)((uintptr_t)src & 3u);
    const uint8_t *base = src - sh;  // 4-aligned
    const uint32_t *s32 = reinterpret_cast<const uint32_t *>(base);
    uint4 *d16 = reinterpret_cast<uint4 *>(dst);
    const uint32_t span = 20u;  // bytes a chunk's loads touch
    // chunks [c_lo, c_hi) are readable without clamping
    const uint32_t c_lo = base >= lo ? 0u : 1u;
    const int64_t room = (int64_t)(hi - base);
    uint32_t c_hi = room >= (int64_t)span ? (uint32_t)((room - span) / 16 + 1) : 0u;
    if (c_hi > nch) c_hi = nch;
    if (c_hi < c_lo) c_hi = c_lo;

    auto load = [&](uint32_t c, Chunk &k) {
        const uint32_t *p = s32 + 4 * (size_t)c;
        k.d[0] = p[0];
        k.d[1] = p[1];
        k.d[2] = p[2];
        k.d[3] = p[3];
        k.d[4] = p[4];  // unused when sh == 0 (alignbyte by 0)
    };
    auto load_clamped = [&](uint32_t c, Chunk &k) {
        const uint8_t *p = base + 16 * (size_t)c;
#pragma unroll
        for (int i = 0; i < 4; i++) k.d[i] = ld_dw_clamped(p + 4 * i, lo, hi);
        k.d[4] = ld_dw_clamped(p + 16, lo, hi);
    };

    // edge chunks before c_lo
    for (uint32_t c = lane; c < c_lo; c += 64) {
        Chunk k;
        load_clamped(c, k);
        d16[c] = realign(k, sh);
    }
    // pipelined body: groups of 64*U chunks, two groups in flight
    constexpr uint32_t G = 64u * kCopyUnroll;
    uint32_t c0 = c_lo;
    if (c0 + G <= c_hi) {
        Chunk a[kCopyUnroll];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; u++) load(c0 + 64u * u + lane, a[u]);
        for (uint32_t c1 = c0 + G; c1 + G <= c_hi; c1 += G) {
            Chunk b[kCopyUnroll];
#pragma unroll
            for (int u = 0; u < kCopyUnroll; u++) load(c1 + 64u * u + lane, b[u]);
#pragma unroll
            for (int u = 0; u < kCopyUnroll; u++) d16[c0 + 64u * u + lane] = realign(a[u], sh);
#pragma unroll
            for (int u = 0; u < kCopyUnroll; u++) a[u] = b[u];
            c0 = c1;
        }
#pragma unroll
        for (int u = 0; u < kCopyUnroll; u++) d16[c0 + 64u * u + lane] = realign(a[u], sh);
        c0 += G;
    }
    // remaining unclamped chunks, then clamped ones at the end of the buffer
    for (uint32_t c = c0 + lane; c < c_hi; c += 64) {
        Chunk k;
        load(c, k);
        d16[c] = realign(k, sh);
    }
    for (uint32_t c = (c_hi > c0 ? c_hi : c0) + lane; c < nch; c += 64) {
        Chunk k;
        load_clamped(c, k);
        d16[c] = realign(k, sh);
    }
    const uint32_t done = nch * 16u, tail = n - done;
    if (lane < (int)tail) dst[done + lane] = src[done + lane];
}

// Periodic copy for offset < length: dst[j] = dst[j - off + (j mod off)]
// relative to the match start; all sources precede the destination.
__device__ __forceinline__ void wave_copy_periodic(uint8_t *dst, uint32_t off,
                                                   uint32_t n, int lane) {
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

// 256-byte register window over the compressed stream.  Positions are
// byte offsets from the input buffer start (no integer-to-pointer casts, so
// every access stays a global-address-space access).
struct Window {
    const uint8_t *__restrict__ g;  // input buffer
    uint64_t gsz;                   // its size
    uint64_t wb;                    // 4-aligned window base (offset into g)
    uint32_t w;                     // this lane's dword of the window
    int lane;

    __device__ __forceinline__ void load_at(uint64_t a) {
        wb = a & ~(uint64_t)3;
        w = ld_dw_clamped(g + wb + 4 * lane, g, g + gsz);
    }
    __device__ __forceinline__ uint32_t byte(uint64_t a) {
        if (a < wb || a >= wb + 256) load_at(a);
        const uint32_t d = (uint32_t)(a - wb);
        return (__builtin_amdgcn_readlane(w, d >> 2) >> ((d & 3u) * 8u)) & 0xffu;
    }
    // Length extension starting at offset *pp (block.rs:277-289, 329-341):
    // adds 255 per 0xFF byte plus the first other byte.  Returns false at end
    // of input (the reference then reports UnexpectedEof at the input end).
    __device__ __forceinline__ bool extension(uint64_t &pp, uint64_t end, uint64_t &len) {
        uint64_t p = pp;
        for (;;) {
            if (p >= end) {
                pp = end;
                return false;
            }
            if (p < wb || p >= wb + 256) load_at(p);
            // terminator: first byte q >= p with (q >= end || byte != 255)
            const uint64_t q0 = wb + 4 * lane;
            uint32_t tmask = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint64_t q = q0 + b;
                const bool t = q >= p && (q >= end || ((w >> (8 * b)) & 0xffu) != 255u);
                tmask |= (uint32_t)t << b;
            }
            const uint64_t ball = __ballot(tmask != 0);
            if (ball) {
                const int tl = __ffsll((unsigned long long)ball) - 1;
                const uint32_t tm = __builtin_amdgcn_readlane(tmask, tl);
                const uint32_t tb = (uint32_t)(__ffs(tm) - 1);
                const uint64_t t = wb + 4 * (uint64_t)tl + tb;
                len += 255ull * (t - p);
                if (t >= end) {
                    pp = end;
                    return false;
                }
                len += (__builtin_amdgcn_readlane(w, tl) >> (8 * tb)) & 0xffu;
                pp = t + 1;
                return true;
            }
            len += 255ull * (wb + 256 - p);
            p = wb + 256;
        }
    }
};

__global__ __launch_bounds__(kThreads) void lz4_batch_kernel(Lz4Batch B) {
    const int lane = threadIdx.x & 63;
    const uint32_t b = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (b >= B.nblocks) return;
    const uint8_t *__restrict__ d_in = B.in;
    const uint64_t in_total = B.in_total;

    int32_t code = HH_OK, detail = HH_CORRUPT_NONE;
    uint64_t pos = 0, req = 0;
    uint32_t op = 0;

    const uint64_t ioff = B.in_off[b];
    const uint32_t ilen = B.in_len[b];
    const uint64_t oofs = B.out_off[b];
    const uint32_t cap = B.out_cap[b];
    const bool out_ok = oofs <= B.out_total && (uint64_t)cap <= B.out_total - oofs;
    uint8_t *out = B.out + oofs;

    if (ioff > in_total || (uint64_t)ilen > in_total - ioff || !out_ok) {
        code = HH_ERR_INVALID_ARGUMENT;
    } else {
        const uint8_t *__restrict__ glo = d_in;
        const uint8_t *__restrict__ ghi = d_in + in_total;
        const uint64_t end = ioff + ilen;  // offsets into d_in
        Window win;
        win.g = d_in;
        win.gsz = in_total;
        win.lane = lane;
        win.load_at(ioff);

        uint64_t ip = ioff;
        while (ip < end) {
            const uint32_t token = win.byte(ip++);
            uint64_t ll = token >> 4;
            if (ll == 15 && !win.extension(ip, end, ll)) {
                code = HH_ERR_UNEXPECTED_EOF;
                pos = ilen;
                break;
            }
            if (ll > 0) {
                if (end - ip < ll) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ip - ioff;
                    break;
                }
                if ((uint64_t)op + ll > cap) {
                    code = HH_ERR_BUFFER_TOO_SMALL;
                    req = (uint64_t)op + ll;
                    break;
                }
                win.load_at(ip + ll);  // prefetch the next offset/token window
                wave_copy(out + op, d_in + ip, (uint32_t)ll, glo, ghi, lane);
                ip += ll;
                op += (uint32_t)ll;
            }
            if (op >= cap) break;  // block.rs:309-311
            if (end - ip < 2) {
                code = HH_ERR_UNEXPECTED_EOF;
                pos = ip - ioff;
                break;
            }
            const uint32_t off = win.byte(ip) | (win.byte(ip + 1) << 8);
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
            if ((token & 15u) == 15u && !win.extension(ip, end, ml)) {
                code = HH_ERR_UNEXPECTED_EOF;
                pos = ilen;
                break;
            }
            if ((uint64_t)op + ml > cap) {
                code = HH_ERR_BUFFER_TOO_SMALL;
                req = (uint64_t)op + ml;
                break;
            }
            wave_fence();
            if (off >= ml)
                wave_copy(out + op, out + op - off, (uint32_t)ml, out, out + cap, lane);
            else
                wave_copy_periodic(out + op, off, (uint32_t)ml, lane);
            wave_fence();
            op += (uint32_t)ml;
        }
    }
    // a failed block's output reads as zeros (the reference returns no output)
    if (code != HH_OK && out_ok) {
        wave_fence();
        wave_zero_fill(out, cap, lane);
    } else if (code == HH_OK && B.zero_tail && op < cap) {
        wave_zero_fill(out + op, cap - op, lane);
    }
    if (lane == 0) {
        hh_block_status st;
        st.code = code;
        st.detail = detail;
        st.position = pos;
        st.required = req;
        st.written = code == HH_OK ? op : 0;
        B.status[b] = st;
    }
}

}  // namespace

hipError_t launch_lz4_batch(const Lz4Batch &B, int32_t decoder, hipStream_t s) {
    if (B.nblocks == 0) return hipSuccess;
    switch (decoder) {
        case HH_LZ4_AUTO:
        case HH_LZ4_SEQ: return launch_lz4_seq(B, 4u, s);
        case HH_LZ4_SEQ8: return launch_lz4_seq(B, 8u, s);
        case HH_LZ4_RING4: return launch_lz4_ring(B, 4u, s);
        case HH_LZ4_RING8: return launch_lz4_ring(B, 8u, s);
        case HH_LZ4_RING16: return launch_lz4_ring(B, 16u, s);
        case HH_LZ4_RING32: return launch_lz4_ring(B, 32u, s);
        default: break;
    }
    const uint32_t grid = (B.nblocks + kWaves - 1) / kWaves;
    hipLaunchKernelGGL(lz4_batch_kernel, dim3(grid), dim3(kThreads), 0, s, B);
    return hipGetLastError();
}

}  // namespace hh
