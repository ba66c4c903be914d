// Raw-LZ4 block decoding with each block's recent output in LDS, one
// wavefront per block; used by the batched LZ4 kernel (lz4_ring.hip) and the
// fused LZ4 -> tile kernel (hctt_decode.hip).
//
// Semantics: crates/haagenti-lz4/src/block.rs:261-366 (decompress_block),
// including its error order and its early stop when the output reaches
// output_size; the checks and the positions they report are those of the
// register-window decoder in lz4_decode.hip.
//
// Why LDS.  In LZ4 streams of weight data a match usually copies bytes that
// an earlier match of the same block produced moments before (runs of zero
// bytes are encoded as a chain of matches, each pointing at the previous
// run).  Decoding straight to global memory makes every such match a global
// store followed by a dependent global load, and on gfx950 a wave's vector
// memory operations share one in-order completion counter, so each of those
// loads also waits for every store issued before it.  Here each wave owns
//  * an output ring of R bytes in LDS.  Every decoded byte is written there
//    first; a match whose offset is at most kNear reads its source from the
//    ring.  The ring is flushed to the output in aligned 16-byte chunks once
//    kFlushAt bytes are pending; matches with larger offsets read the
//    flushed output (their source bytes are flushed first);
//  * an input stage of S bytes of the compressed stream, refilled with
//    coalesced 16-byte loads.  Tokens, lengths and offsets are read through
//    a 256-byte window over the stage (one dword per lane, bytes picked with
//    v_readlane, runs of 255-valued extension bytes measured with one ballot
//    per window), and literal runs are copied stage -> ring.
// So a block's global traffic is its compressed bytes read once, its output
// written once, and the sources of far matches.
//
// Ring bookkeeping (all positions are "virtual": output position + a0, the
// misalignment of the block's output address, so that 16-aligned virtual
// positions are 16-aligned addresses; the ring slot of position v is
// v mod R):
//  * copies are split into pieces of at most kP bytes (literals: kPL), each
//    followed by the flush check (a flush once kFlushAt = R - 2 max(kP, kPL)
//    bytes are pending), so a piece never overwrites a pending byte;
//  * a piece writes slots of positions at least R behind it, i.e. more than
//    kNear behind its start, which no near match reads.
// Every read is clamped to the caller's buffers and every write stays inside
// the block's output capacity; corrupt input yields a status, never an
// out-of-bounds access.
//
// With LDS = true the whole output stays in the ring (a block of at most
// R - 32 bytes: every match is a near one and nothing is flushed), for a
// consumer that reads it from LDS.
#pragma once

#include "hh_internal.hpp"

namespace hh {
namespace ring {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Compiler-only ordering point between flush stores and far-match loads of
// the same bytes; a wave's vector memory operations are performed in order.
__device__ __forceinline__ void mem_order() { __asm__ __volatile__("" ::: "memory"); }

// 16 bytes starting at byte sh of the 20 bytes d0..d4.
__device__ __forceinline__ u32x4 realign(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                                         uint32_t d4, uint32_t sh) {
    return u32x4{__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh),
                 __builtin_amdgcn_alignbyte(d3, d2, sh), __builtin_amdgcn_alignbyte(d4, d3, sh)};
}

// "no window": any stage offset minus it is >= 256 (see in_win)
constexpr uint32_t kNoWin = 0x80000000u;

template <uint32_t R, uint32_t S, bool LDS = false>
struct RingDec {
    static_assert((R & (R - 1)) == 0 && R >= 4096, "ring size is a power of two");
    static_assert(S % 1024 == 0 && S >= 1024, "stage is whole KiB");
    static constexpr uint32_t kRM = R - 1;
    static constexpr uint32_t kP = 992;             // largest piece: at most 63 chunks
    // literal pieces: kLitU chunks per lane (LDS mode has no flush
    // bookkeeping; a small ring keeps one so that flushes stay rare)
    static constexpr uint32_t kLitU = LDS ? 4 : R >= 8192 ? 2 : 1;
    static constexpr uint32_t kPL = 64u * 16u * kLitU - 16u;
    static constexpr uint32_t kNear = R - 32;       // offsets served from the ring
    static constexpr uint32_t kFlushAt = R - 2 * (kPL > kP ? kPL : kP);
    static constexpr uint32_t kSFront = 16;         // stage under-read (first chunk of a literal)
    static constexpr uint32_t kSPad = 272;          // window and realign over-read
    static constexpr uint32_t kLds = R + kSFront + S + kSPad;

    uint8_t *ring;
    uint8_t *stage;
    const uint8_t *gbuf;  // whole input buffer: reads are clamped to it
    uint64_t gsz;
    uint64_t ioff;        // block start in gbuf
    uint8_t *obase;       // 16-aligned, <= the block's output address
    uint32_t a0;          // output address - obase
    uint32_t cap;
    // Block-relative input position of stage byte 0, modulo 2^32 (it is up
    // to 15 before the block start when the block starts unaligned); every
    // use takes a difference x - sb, exact for x in or after the stage.
    uint32_t sb;
    bool at_end;          // the stage reaches the end of the input buffer
    uint32_t wso;         // stage offset of the window (4-aligned), or kNoWin
    uint32_t w;           // this lane's window dword
    uint32_t op;          // bytes decoded
    uint32_t fl;          // bytes flushed to the output
    int lane;

    // Loads the stage contents for the compressed bytes from x on of the
    // block at ioff_ (x block-relative) into registers: stage byte 0 is
    // 16-aligned in memory, at most 15 bytes before x.  Separate from
    // put_stage so that a caller can have the loads in flight meanwhile.
    static __device__ __forceinline__ void load_stage(const uint8_t *gbuf_, uint64_t gsz_, uint64_t ioff_,
                                                      uint32_t x, int lane_, u32x4 (&v)[S / 1024]) {
        const uintptr_t addr = (uintptr_t)(gbuf_ + ioff_ + x);
        const int64_t b0 = (int64_t)ioff_ + (int64_t)x - (int64_t)(addr & 15u);  // may be < 0
#pragma unroll
        for (uint32_t i = 0; i < S / 1024; i++) {
            const int64_t o = b0 + 16 * (int64_t)(lane_ + 64 * i);
            if (o >= 0 && o + 16 <= (int64_t)gsz_) {
                v[i] = *reinterpret_cast<const u32x4 *>(gbuf_ + o);
            } else {
                // edge chunk of the buffer: bytes outside it read as zero
                u32x4 d = u32x4{0u, 0u, 0u, 0u};
#pragma unroll 1
                for (int j = 0; j < 16; j++)
                    if (o + j >= 0 && o + j < (int64_t)gsz_) d[j >> 2] |= (uint32_t)gbuf_[o + j] << (8 * (j & 3));
                v[i] = d;
            }
        }
    }
    // Writes what load_stage(gbuf, gsz, ioff, x, lane, v) loaded into the
    // stage and sets the stage bookkeeping for it.
    __device__ __forceinline__ void put_stage(uint32_t x, const u32x4 (&v)[S / 1024]) {
        const uintptr_t addr = (uintptr_t)(gbuf + ioff + x);
        sb = x - (uint32_t)(addr & 15u);
        const int64_t b0 = (int64_t)ioff + (int64_t)x - (int64_t)(addr & 15u);
        at_end = (uint64_t)(b0 + S) >= gsz;
#pragma unroll
        for (uint32_t i = 0; i < S / 1024; i++)
            *reinterpret_cast<u32x4 *>(stage + 16 * (lane + 64 * i)) = v[i];
        wso = kNoWin;
        wave_sync();
    }
    // Stage the compressed bytes from x on.
    __device__ __forceinline__ void restage(uint32_t x) {
        u32x4 v[S / 1024];
        load_stage(gbuf, gsz, ioff, x, lane, v);
        put_stage(x, v);
    }

    // Window at x (block-relative).  The stage must hold x and the 255 bytes
    // after it, unless it already reaches the end of the input buffer (the
    // bytes past it are then never used: every parse read is below the
    // block end).
    __device__ __forceinline__ void win_at(uint32_t x) {
        uint32_t so = x - sb;
        if (so >= S || (so + 256 > S && !at_end)) {
            restage(x);
            so = x - sb;
        }
        wso = so & ~3u;
        w = *reinterpret_cast<const uint32_t *>(stage + wso + 4 * lane);
    }
    __device__ __forceinline__ bool in_win(uint32_t x) const { return x - sb - wso < 256u; }
    __device__ __forceinline__ uint32_t byte(uint32_t x) {
        if (!in_win(x)) win_at(x);
        const uint32_t d = x - sb - wso;
        return (__builtin_amdgcn_readlane(w, d >> 2) >> ((d & 3u) * 8u)) & 0xffu;
    }

    // Length extension starting at *pp (block.rs:277-289, 329-341): adds 255
    // per 0xFF byte plus the first other byte.  Returns false at the end of
    // the block input (the reference then reports UnexpectedEof).
    __device__ __forceinline__ bool extension(uint32_t &pp, uint32_t end, uint64_t &len) {
        uint32_t p = pp;
        for (;;) {
            if (p >= end) {
                pp = end;
                return false;
            }
            if (!in_win(p)) win_at(p);
            // window-relative positions (the window may start before the
            // block: the stage starts at a 16-aligned address)
            const uint32_t wb = sb + wso;  // block-relative, modulo 2^32
            const uint32_t pr = p - wb;    // < 256
            const uint32_t er = end - wb > 256u ? 256u : end - wb;  // > pr
            const uint32_t r0 = 4u * (uint32_t)lane;
            uint32_t tmask = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t r = r0 + b;
                const bool t = r >= pr && (r >= er || ((w >> (8 * b)) & 0xffu) != 255u);
                tmask |= (uint32_t)t << b;
            }
            const uint64_t ball = __ballot(tmask != 0);
            if (ball) {
                const int tl = __ffsll((unsigned long long)ball) - 1;
                const uint32_t tm = __builtin_amdgcn_readlane(tmask, tl);
                const uint32_t tb = (uint32_t)(__ffs(tm) - 1);
                const uint32_t tr = 4u * (uint32_t)tl + tb;
                len += 255ull * (tr - pr);
                if (tr >= er) {
                    pp = end;
                    return false;
                }
                len += (__builtin_amdgcn_readlane(w, tl) >> (8 * tb)) & 0xffu;
                pp = wb + tr + 1;
                return true;
            }
            len += 255ull * (256u - pr);
            p = wb + 256;
        }
    }

    // 8 bytes from x on (block-relative; bytes past the block end are
    // don't-care and never used by the callers).
    __device__ __forceinline__ uint64_t read8(uint32_t x) {
        uint32_t d = x - sb - wso;
        if (d > 244u) {
            win_at(x);
            d = x - sb - wso;
        }
        const uint32_t k = d >> 2, sh = 8u * (d & 3u);
        const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane(w, k);
        const uint64_t mi = (uint32_t)__builtin_amdgcn_readlane(w, k + 1);
        const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane(w, k + 2);
        const uint64_t v = (mi << 32) | lo;
        return sh == 0 ? v : (v >> sh) | (hi << (64u - sh));
    }

    // One copy piece of n bytes (n <= kP) to the ring at op, as one pass of
    // 16-byte chunks aligned in virtual positions: lane l writes chunk l of
    // the piece.  The first chunk keeps its bytes before the piece (read
    // back from the ring); bytes of the last chunk past the piece are
    // don't-care (the next piece overwrites them, nothing reads them first).
    // K selects the source of piece byte j:
    //   0: stage byte src + j (literal)
    //   1: ring byte src + j (match, src = op - off + a0, n <= off)
    //   2: output byte src + j (far match; the source is flushed, n <= off)
    //   3: ring byte src + (j mod off) (periodic match, src = op - off + a0)
    template <int K>
    __device__ __forceinline__ void piece(uint32_t src, uint32_t n, uint32_t off) {
        const uint32_t v = op + a0;
        const uint32_t c0 = v & ~15u;
        const uint32_t nch = ((v + n + 15u) >> 4) - (v >> 4);  // <= 63
        if (lane < (int)nch) {
            const uint32_t cv = c0 + 16u * (uint32_t)lane;
            u32x4 o;
            if constexpr (K == 3) {
                // (cv - v) mod off (cv - v >= -15, off < 16): x / off as
                // (x * magic) >> 16 with magic = floor(65536 / off) + 1,
                // exact for x < 4096 (x / off is never within 1/16 of an
                // integer from below); rcp(off) is exact or far enough from
                // an integer that the floor is exact
                const uint32_t x = cv + 16u * off - v;
                const uint32_t magic = (uint32_t)(65536.0f * __builtin_amdgcn_rcpf((float)off)) + 1u;
                uint32_t m = x - ((x * magic) >> 16) * off;
                uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int b = 0; b < 16; b++) {
                    d[b >> 2] |= (uint32_t)ring[(src + m) & kRM] << (8 * (b & 3));
                    m = m + 1 == off ? 0u : m + 1;
                }
                o = u32x4{d[0], d[1], d[2], d[3]};
            } else if constexpr (K <= 1) {
                const uint32_t sp = src + cv - v;  // source of chunk byte 0 (lane 0: up to 15 before src)
                const uint32_t sb4 = sp & ~3u, sh = sp & 3u;
                uint32_t d[5];
                if constexpr (K == 0) {
                    const uint32_t *q = reinterpret_cast<const uint32_t *>(stage + (int32_t)sb4);
#pragma unroll
                    for (int i = 0; i < 5; i++) d[i] = q[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 5; i++) d[i] = *reinterpret_cast<const uint32_t *>(ring + ((sb4 + 4u * i) & kRM));
                }
                o = realign(d[0], d[1], d[2], d[3], d[4], sh);
            } else {
                const uint32_t sp = src + cv - v;  // source of chunk byte 0 (lane 0: up to 15 before src)
                const uint32_t sh = sp & 3u;
                uint32_t d[5];
                {
                    // output bytes [a0, a0 + cap) only; the first chunk's
                    // source may start before the block's output
                    const int64_t lo = a0, hi = (int64_t)a0 + cap;
                    const int64_t q0 = ((int64_t)src + (int64_t)cv - (int64_t)v) & ~(int64_t)3;
                    if (q0 >= lo && q0 + 20 <= hi) {
                        const uint32_t *q = reinterpret_cast<const uint32_t *>(obase + q0);
#pragma unroll
                        for (int i = 0; i < 5; i++) d[i] = q[i];
                    } else {
#pragma unroll
                        for (int i = 0; i < 5; i++) d[i] = 0u;
#pragma unroll 1
                        for (int j = 0; j < 20; j++) {
                            const int64_t qq = q0 + j;
                            if (qq >= lo && qq < hi) {
                                const uint32_t x = (uint32_t)obase[qq] << (8 * (j & 3));
                                switch (j >> 2) {
                                    case 0: d[0] |= x; break;
                                    case 1: d[1] |= x; break;
                                    case 2: d[2] |= x; break;
                                    case 3: d[3] |= x; break;
                                    default: d[4] |= x; break;
                                }
                            }
                        }
                    }
                }
                o = realign(d[0], d[1], d[2], d[3], d[4], sh);
            }
            if (v & 15u) {  // the first chunk keeps its bytes before the piece
                const uint32_t keep = lane == 0 ? (v & 15u) : 0u;
                const u32x4 old = *reinterpret_cast<const u32x4 *>(ring + (cv & kRM));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t kb = keep > 4u * i ? keep - 4u * i : 0u;
                    const uint32_t m = kb >= 4u ? 0xffffffffu : (1u << (8u * kb)) - 1u;
                    o[i] = (old[i] & m) | (o[i] & ~m);
                }
            }
            *reinterpret_cast<u32x4 *>(ring + (cv & kRM)) = o;
        }
        op += n;
        wave_sync();
    }

    // A literal piece of n bytes (n <= kPL) from stage byte src to the ring
    // at op: lane l writes chunks l, l + 64, ... of the piece (16-byte chunks
    // aligned in virtual positions), all stage reads issued before the first
    // write.  Chunk rules as in piece<0>.
    __device__ __forceinline__ void piece_lit(uint32_t src, uint32_t n) {
        const uint32_t v = op + a0;
        const uint32_t c0 = v & ~15u;
        const uint32_t nch = ((v + n + 15u) >> 4) - (v >> 4);  // <= 64 kLitU
        uint32_t d[kLitU][5];
#pragma unroll
        for (uint32_t u = 0; u < kLitU; u++) {
            const uint32_t ci = (uint32_t)lane + 64u * u;
            const uint32_t sp = src + c0 + 16u * ci - v;  // source of chunk byte 0 (chunk 0: up to 15 before src)
            const uint32_t *q = reinterpret_cast<const uint32_t *>(stage + (int32_t)(sp & ~3u));
            if (ci < nch) {
#pragma unroll
                for (int i = 0; i < 5; i++) d[u][i] = q[i];
            }
        }
        u32x4 old = u32x4{0u, 0u, 0u, 0u};
        const uint32_t keep = lane == 0 ? (v & 15u) : 0u;
        if (keep) old = *reinterpret_cast<const u32x4 *>(ring + (c0 & kRM));
#pragma unroll
        for (uint32_t u = 0; u < kLitU; u++) {
            const uint32_t ci = (uint32_t)lane + 64u * u;
            if (ci < nch) {
                const uint32_t cv = c0 + 16u * ci;
                const uint32_t sp = src + cv - v;
                u32x4 o = realign(d[u][0], d[u][1], d[u][2], d[u][3], d[u][4], sp & 3u);
                if (u == 0 && keep) {  // the first chunk keeps its bytes before the piece
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t kb = keep > 4u * i ? keep - 4u * i : 0u;
                        const uint32_t m = kb >= 4u ? 0xffffffffu : (1u << (8u * kb)) - 1u;
                        o[i] = (old[i] & m) | (o[i] & ~m);
                    }
                }
                *reinterpret_cast<u32x4 *>(ring + (cv & kRM)) = o;
            }
        }
        op += n;
        wave_sync();
    }

    // Writes the pending bytes [fl, op) to the output: all of them when
    // `exact`, else up to the last 16-aligned address.
    __device__ __forceinline__ void flush(bool exact) {
        if constexpr (LDS) {  // the output stays in the ring
            fl = op;
            return;
        }
        const uint32_t vf = fl + a0, vo = op + a0;
        const uint32_t ve = exact ? vo : (vo & ~15u);
        if (ve <= vf) return;
        uint32_t h = (16u - (vf & 15u)) & 15u;
        if (h > ve - vf) h = ve - vf;
        if (lane < (int)h) obase[vf + lane] = ring[(vf + lane) & kRM];
        const uint32_t vb = vf + h;
        const uint32_t nch = (ve - vb) >> 4;
        for (uint32_t c = lane; c < nch; c += 64) {
            const uint32_t x = vb + 16u * c;
            *reinterpret_cast<u32x4 *>(obase + x) = *reinterpret_cast<const u32x4 *>(ring + (x & kRM));
        }
        const uint32_t vt = vb + 16u * nch;
        if (lane < (int)(ve - vt)) obase[vt + lane] = ring[(vt + lane) & kRM];
        fl = ve - a0;
        mem_order();
    }
    __device__ __forceinline__ void mem_sync() { mem_order(); }
    __device__ __forceinline__ void check_flush() {
        if constexpr (!LDS)
            if (op - fl >= kFlushAt) flush(false);
    }
};

// Parses and copies one block whose input is [0, ilen) (block-relative)
// into d; on return code / detail / pos / req hold the outcome (HH_OK or the
// reference's error record) and d.op the bytes decoded.  The caller flushes
// the rest of a successful block.  `staged`: the caller has already staged
// the input from 0 on (put_stage(0, ...)).  `progress(op)` runs after each
// sequence's copies (every lane; the output bytes before op are final).
struct NoProgress {
    __device__ __forceinline__ void operator()(uint32_t) const {}
};
template <uint32_t R, uint32_t S, bool LDS, typename Progress = NoProgress>
__device__ __forceinline__ void parse_block(RingDec<R, S, LDS> &d, uint32_t ilen, int32_t &code, int32_t &detail,
                                            uint64_t &pos, uint64_t &req, bool staged = false,
                                            Progress &&progress = Progress{}) {
    using D = RingDec<R, S, LDS>;
    const uint32_t end = ilen;
    uint32_t ip = 0;
    if (end > 0 && !staged) d.restage(0);
    while (ip < end) {
        // token and literal length (block.rs:270-289); the extension
        // bytes usually lie in the 7 bytes after the token
        const uint64_t t8 = d.read8(ip);
        const uint32_t token = (uint32_t)t8 & 0xffu;
        // lengths are 32-bit: one longer than the block input (only a
        // run of > 2^24 0xFF bytes makes it) fails the input-length check
        // below as the reference's 64-bit length does, so it is reported
        // right away
        uint32_t ll = token >> 4;
        ip++;
        if (ll == 15) {
            const uint64_t x = t8 >> 8;
            const uint64_t nz = ~x & 0x00ffffffffffffffull;  // bytes other than 0xFF
            if (nz != 0) {
                const uint32_t e = (uint32_t)__builtin_ctzll(nz) >> 3;
                if (ip + e >= end) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ilen;
                    return;
                }
                ll += 255u * e + (uint32_t)((x >> (8 * e)) & 0xffu);
                ip += e + 1;
            } else {
                uint64_t l64 = ll;
                if (end - ip < 7 || (l64 += 255ull * 7, ip += 7, !d.extension(ip, end, l64))) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ilen;
                    return;
                }
                if (l64 > 0xffffffffull) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ip;
                    return;
                }
                ll = (uint32_t)l64;
            }
        }
        if (ll > 0) {
            if (end - ip < ll) {
                code = HH_ERR_UNEXPECTED_EOF;
                pos = ip;
                return;
            }
            if (ll > d.cap - d.op) {  // op <= cap throughout
                code = HH_ERR_BUFFER_TOO_SMALL;
                req = (uint64_t)d.op + ll;
                return;
            }
            uint32_t rem = (uint32_t)ll;
            // read the window at the offset now when the stage already
            // holds it, so its LDS latency overlaps the literal copy
            const uint32_t so_end = ip - d.sb + rem;
            if (so_end + 256u <= S || (d.at_end && so_end < S)) d.win_at(ip + rem);
            while (rem > 0) {
                uint32_t so = ip - d.sb;
                if (so >= S) {
                    d.restage(ip);
                    so = ip - d.sb;
                }
                uint32_t n = rem < D::kPL ? rem : D::kPL;
                if (n > S - so) n = S - so;
                d.piece_lit(so, n);
                ip += n;
                rem -= n;
                d.check_flush();
            }
        }
        if (d.op >= d.cap) return;  // block.rs:309-311
        if (end - ip < 2) {
            code = HH_ERR_UNEXPECTED_EOF;
            pos = ip;
            return;
        }
        // offset and match length (block.rs:313-345)
        const uint64_t o8 = d.read8(ip);
        const uint32_t off = (uint32_t)o8 & 0xffffu;
        ip += 2;
        if (off == 0) {
            code = HH_ERR_CORRUPTED_DATA;
            detail = HH_CORRUPT_ZERO_OFFSET;
            return;
        }
        if (off > d.op) {
            code = HH_ERR_CORRUPTED_DATA;
            detail = HH_CORRUPT_OFFSET_BEYOND;
            pos = d.op;
            return;
        }
        uint32_t ml = (token & 15u) + 4u;
        if ((token & 15u) == 15u) {
            const uint64_t x = o8 >> 16;
            const uint64_t nz = ~x & 0x0000ffffffffffffull;
            if (nz != 0) {
                const uint32_t e = (uint32_t)__builtin_ctzll(nz) >> 3;
                if (ip + e >= end) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ilen;
                    return;
                }
                ml += 255u * e + (uint32_t)((x >> (8 * e)) & 0xffu);
                ip += e + 1;
            } else {
                uint64_t m64 = ml;
                if (end - ip < 6 || (m64 += 255ull * 6, ip += 6, !d.extension(ip, end, m64))) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ilen;
                    return;
                }
                if (m64 > 0xffffffffull) {  // more than any capacity
                    code = HH_ERR_BUFFER_TOO_SMALL;
                    req = (uint64_t)d.op + m64;
                    return;
                }
                ml = (uint32_t)m64;
            }
        }
        if (ml > d.cap - d.op) {
            code = HH_ERR_BUFFER_TOO_SMALL;
            req = (uint64_t)d.op + ml;
            return;
        }
        uint32_t rem = (uint32_t)ml;
        if (!LDS && off > D::kNear) {
            while (rem > 0) {
                d.flush(true);
                uint32_t n = rem < D::kP ? rem : D::kP;
                if (n > off) n = off;
                d.mem_sync();
                d.template piece<2>(d.op + d.a0 - off, n, off);
                rem -= n;
            }
        } else if (off < 16u && off < rem) {
            while (rem > 0) {
                const uint32_t n = rem < D::kP ? rem : D::kP;
                d.template piece<3>(d.op + d.a0 - off, n, off);
                rem -= n;
                d.check_flush();
            }
        } else {
            while (rem > 0) {
                uint32_t n = rem < D::kP ? rem : D::kP;
                if (n > off) n = off;
                d.template piece<1>(d.op + d.a0 - off, n, off);
                rem -= n;
                d.check_flush();
            }
        }
        progress(d.op);
    }
}

}  // namespace ring
}  // namespace hh
