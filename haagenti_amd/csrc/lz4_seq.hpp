// Raw-LZ4 block decoding, one wavefront per block, in batches of sequences:
// a scalar pass parses up to 64 sequences into lane-held descriptors, a wave
// prefix sum turns their lengths into output offsets, and the copies of the
// whole batch then run lane-parallel -- every literal run of the batch in one
// set of passes, then the matches, those that read only bytes final before
// them sharing a pass.  Used by the batched LZ4 kernel (lz4_seq.hip) and the
// fused LZ4 -> tile kernel (hctt_decode.hip).
//
// Semantics: crates/haagenti-lz4/src/block.rs:261-366 (decompress_block):
// the same checks in the same order, the same reported positions, the early
// stop once the output reaches output_size.  Every check is made by the
// parse, so a batch's copies never fail; a block that fails is not copied
// further (its caller zero-fills its output).
//
// LDS per wave:
//  * an output ring of R bytes holding the block's latest output.  A match
//    reads its source from the ring when the source was written at most R
//    bytes before the end of the current batch (nothing of the batch has
//    overwritten it), else from the output in global memory, which every
//    complete 16-byte chunk has reached by then (batches produce at most
//    R - 64 bytes and complete chunks are written out after each batch);
//  * an input stage of S bytes of the compressed stream, refilled with
//    16-byte loads; headers and literal runs are read there.  A batch ends
//    where the stage does; a literal run or match that crosses a batch end
//    continues in the next batch;
//  * a 64-word table that maps a pass's chunks to their runs.
// Copies write exactly their own bytes (16-byte chunks aligned in output
// position; partial dwords merged with LDS and/or atomics), so the runs of a
// pass may share chunks.  A match of length n at output position v with
// offset `off` writes byte t from position v - off + (t mod off): a periodic
// (overlapping) match reads only the `off` bytes before it, so all of its
// chunks are independent.  Matches of one pass read only bytes before the
// first of them.
//
// With LDS = true the whole block output stays in the ring (a block of at
// most R - 32 bytes; every match reads the ring, nothing is written out) for
// a consumer that reads it there; progress(op) runs after each batch with
// the output before op final.
#pragma once

#include "hh_internal.hpp"

namespace hh {
namespace seq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// LDS-qualified pointers: every ring, stage and table access is a ds_*
// instruction (a generic pointer lets the compiler merge a ring read with a
// global read into one flat load, which is not ordered after earlier ds_*
// writes of other lanes)
typedef __attribute__((address_space(3))) uint8_t lds8;
typedef __attribute__((address_space(3))) uint32_t lds32;
typedef __attribute__((address_space(3))) u32x4 ldsx4;

__device__ __forceinline__ uint32_t rfl(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint32_t rdl(uint32_t v, uint32_t l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ uint64_t ballot(bool b) { return __builtin_amdgcn_ballot_w64(b); }
__device__ __forceinline__ uint32_t bperm(uint32_t v, uint32_t l) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute((int)(l << 2), (int)v);
}

// Inclusive prefix sum / maximum over the 64 lanes: DPP row shifts (1, 2,
// 4, 8 within each row of 16 lanes) and the row broadcasts of lanes 15 and
// 31; lanes whose source lies outside the row keep the 0 passed as `old`.
__device__ __forceinline__ uint32_t scan_add(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);
    return v;
}
__device__ __forceinline__ uint32_t scan_max(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));
    return v;
}

// Orders the LDS accesses of the wave's lanes: what one lane wrote before it
// is what every lane reads after it (the compiler may otherwise keep a
// value a lane stored itself and miss another lane's atomic update).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 16 bytes starting at byte sh of the 20 bytes d0..d4.
__device__ __forceinline__ u32x4 realign(const uint32_t (&d)[5], uint32_t sh) {
    return u32x4{__builtin_amdgcn_alignbyte(d[1], d[0], sh), __builtin_amdgcn_alignbyte(d[2], d[1], sh),
                 __builtin_amdgcn_alignbyte(d[3], d[2], sh), __builtin_amdgcn_alignbyte(d[4], d[3], sh)};
}

// Byte mask of bytes [lo, hi) of dword i of a 16-byte chunk.
__device__ __forceinline__ uint32_t dword_mask(uint32_t lo, uint32_t hi, uint32_t i) {
    const int32_t a = (int32_t)lo - (int32_t)(4 * i), b = (int32_t)hi - (int32_t)(4 * i);
    const uint32_t ma = a <= 0 ? 0xffffffffu : a >= 4 ? 0u : (0xffffffffu << (8 * a));
    const uint32_t mb = b >= 4 ? 0xffffffffu : b <= 0 ? 0u : ((1u << (8 * b)) - 1u);
    return ma & mb;
}

// x mod m for 0 <= x < 2^24, 1 <= m < 2^17 (f32 quotient estimate, corrected).
__device__ __forceinline__ uint32_t umod(uint32_t x, uint32_t m) {
    uint32_t q = (uint32_t)((float)x * __builtin_amdgcn_rcpf((float)m));
    int32_t r = (int32_t)(x - q * m);
    r = r < 0 ? r + (int32_t)m : r;
    r = r >= (int32_t)m ? r - (int32_t)m : r;
    r = r < 0 ? r + (int32_t)m : r;
    return (uint32_t)r;
}

// Parse state between batches.
enum : uint32_t { kToken = 0, kLit = 1, kOff = 2, kMatch = 3 };

struct NoProgress {
    __device__ __forceinline__ void operator()(uint32_t) const {}
};

template <uint32_t R, uint32_t S, bool LDS>
struct SeqDec {
    static_assert((R & (R - 1)) == 0 && R >= 4096, "ring size is a power of two");
    static_assert(S % 1024 == 0 && S >= 1024, "stage is whole KiB");
    static constexpr uint32_t kRM = R - 1;
    static constexpr uint32_t kS = S;
    static constexpr uint32_t kOB = LDS ? R - 32 : R - 96;  // batch output budget
    static constexpr uint32_t kSFront = 16;                // stage under-read (first chunk of a literal)
    static constexpr uint32_t kSPad = 32;                  // stage over-read (headers, realign)
    static constexpr uint32_t kStageLds = kSFront + S + kSPad;
    static constexpr uint32_t kTabLds = 256;
    // ring, table, stage (the caller may place them elsewhere)
    static constexpr uint32_t kLds = R + kTabLds + kStageLds;

    lds8 *ring;
    lds32 *tab;           // 64 words
    lds8 *stage;          // kSFront bytes of slack before it, kSPad after
    const uint8_t *gbuf;  // whole input buffer: every read is clamped to it
    uint64_t gsz;
    uint64_t ioff;        // block start in gbuf
    uint8_t *obase;       // 16-aligned, <= the block's output address
    uint32_t a0;          // output address - obase
    uint32_t cap;
    // Block-relative input position of stage byte 0, modulo 2^32 (up to 15
    // before the block start when the block starts unaligned).
    uint32_t sb;
    bool at_end;          // the stage reaches the end of the input buffer
    uint32_t op;          // bytes decoded
    uint32_t fl;          // bytes written out
    int lane;

    // ---------------------------------------------------------------- stage
    // The stage holds input bytes [sb, sb + S) (block-relative; sb is
    // 16-aligned in memory, up to 15 bytes before the block when it starts
    // unaligned).  The next stage, starting 64 bytes before this one ends,
    // is loaded into registers (pv) as soon as this one is in place, so its
    // loads are in flight while the wave parses and copies.
    u32x4 pv[S / 1024];
    uint32_t pf;   // input position of the prefetched stage
    bool pf_on;    // pv holds (or is loading) the stage at pf
    // Loads into v the stage whose byte 0 is input byte s0 (16-aligned in
    // memory).  Inside the buffer: 16-byte loads; at its edges each dword is
    // read at an address clamped to the dwords holding buffer bytes (bytes
    // outside the buffer are never used).
    __device__ __forceinline__ void load_stage(uint32_t s0, u32x4 (&v)[S / 1024]) const {
        const int64_t b0 = (int64_t)ioff + (int64_t)(int32_t)s0;
        if (b0 >= 0 && b0 + (int64_t)S <= (int64_t)gsz) {
#pragma unroll
            for (uint32_t i = 0; i < S / 1024; i++)
                v[i] = *reinterpret_cast<const u32x4 *>(gbuf + b0 + 16 * (lane + 64 * i));
        } else {
            const int64_t lo = -(int64_t)((uintptr_t)gbuf & 3u);
            const int64_t hi = (int64_t)(((uintptr_t)gbuf + gsz - 1) & ~(uintptr_t)3) - (int64_t)(uintptr_t)gbuf;
#pragma unroll
            for (uint32_t i = 0; i < S / 1024; i++) {
#pragma unroll
                for (uint32_t j = 0; j < 4; j++) {
                    int64_t o = b0 + 16 * (lane + 64 * i) + 4 * j;
                    o = o < lo ? lo : o > hi ? hi : o;
                    v[i][j] = *reinterpret_cast<const uint32_t *>(gbuf + o);
                }
            }
        }
    }
    __device__ __forceinline__ void put_stage(uint32_t s0, const u32x4 (&v)[S / 1024]) {
        sb = s0;
        at_end = (int64_t)ioff + (int64_t)(int32_t)s0 + (int64_t)S >= (int64_t)gsz;
#pragma unroll
        for (uint32_t i = 0; i < S / 1024; i++)
            *reinterpret_cast<ldsx4 *>(stage + 16 * (lane + 64 * i)) = v[i];
        wave_sync();
    }
    // Starts the load of the stage after the current one.  Not in LDS mode,
    // whose caller runs other waves beside this one to hide the loads (and
    // needs the registers).
    static constexpr bool kPrefetch = !LDS;
    __device__ __forceinline__ void prefetch() {
        pf_on = kPrefetch && !at_end;
        if (pf_on) {
            pf = sb + S - 64u;
            load_stage(pf, pv);
        }
    }
    // Makes the stage hold input position x: from the prefetched stage when
    // it holds x with at least 1 KiB after it, else loaded now.
    __device__ __forceinline__ void restage(uint32_t x) {
        if constexpr (kPrefetch) {
            if (!(pf_on && x - pf <= S - 1024u)) {
                pf = x - (uint32_t)((uintptr_t)(gbuf + ioff + x) & 15u);
                load_stage(pf, pv);
            }
            put_stage(pf, pv);
            prefetch();
        } else {
            const uint32_t s0 = x - (uint32_t)((uintptr_t)(gbuf + ioff + x) & 15u);
            u32x4 v[S / 1024];
            load_stage(s0, v);
            put_stage(s0, v);
        }
    }
    // [x, x + 8) is in the stage (or the stage reaches the end of the buffer)
    __device__ __forceinline__ bool in_stage8(uint32_t x) const { return at_end || x - sb <= S - 8; }
    // stage bytes available for a literal run from x on
    __device__ __forceinline__ uint32_t lit_avail(uint32_t x) const { return at_end ? 0xffffffffu : sb + S - x; }

    // Header window: input bytes [hb, hb + hv) in scalar registers (hv <=
    // 16), read from the stage 16 at a time, so that a sequence's offset,
    // its match-length bytes and the next token usually come from one read.
    uint64_t hw0, hw1;
    uint32_t hb, hv;
    // 16 bytes from x on (x in the stage); the bytes past the stage's data
    // are not counted valid
    __device__ __forceinline__ void read16(uint32_t x) {
        const uint32_t so = x - sb;
        const lds32 *q = reinterpret_cast<const lds32 *>(stage + (so & ~3u));
        const uint32_t d0 = q[0], d1 = q[1], d2 = q[2], d3 = q[3], d4 = q[4];
        const uint32_t sh = so & 3u;
        const uint32_t w0 = rfl(__builtin_amdgcn_alignbyte(d1, d0, sh));
        const uint32_t w1 = rfl(__builtin_amdgcn_alignbyte(d2, d1, sh));
        const uint32_t w2 = rfl(__builtin_amdgcn_alignbyte(d3, d2, sh));
        const uint32_t w3 = rfl(__builtin_amdgcn_alignbyte(d4, d3, sh));
        hw0 = ((uint64_t)w1 << 32) | w0;
        hw1 = ((uint64_t)w3 << 32) | w2;
        hb = x;
        hv = at_end || S - so >= 16u ? 16u : S - so;
    }
    // 8 bytes from x on: from the window when it holds them, else from the
    // stage (the caller has checked in_stage8(x)).
    __device__ __forceinline__ bool in_win8(uint32_t x) const { return x - hb <= hv - 8u && hv >= 8u; }
    __device__ __forceinline__ uint64_t peek8(uint32_t x) const {  // in_win8(x)
        const uint32_t k = x - hb;  // 0..8
        const uint64_t a = hw0 >> (8 * (k & 7u)), b = (hw1 << 1) << (63 - 8 * (k & 7u));
        return k >= 8u ? hw1 : (a | b);
    }
    __device__ __forceinline__ uint64_t get8(uint32_t x) {
        if (!in_win8(x)) read16(x);
        return peek8(x);
    }
    // the raw stage read of 8 bytes (extension runs)
    __device__ __forceinline__ uint64_t read8(uint32_t x) {
        read16(x);
        return hw0;
    }

    // Length extension from *pp (block.rs:277-289, 329-341) once 7 (or 6)
    // 0xFF bytes have been seen: adds 255 per 0xFF byte plus the first other
    // byte.  Returns 0 when done, 1 at the end of the block input (the
    // reference reports UnexpectedEof), 2 when it needs bytes past the stage
    // while the batch holds copies that read the stage (the caller ends the
    // batch and parses the sequence again); with no such copies it restages.
    __device__ __forceinline__ int ext_slow(uint32_t &pp, uint32_t end, uint64_t &len, bool pend) {
        uint32_t p = pp;
        for (;;) {
            if (p >= end) return 1;
            if (!in_stage8(p)) {
                if (pend) return 2;
                restage(p);
            }
            const uint64_t x = read8(p);
            const uint64_t nz = ~x;
            if (nz == 0) {
                len += 255ull * 8;
                p += 8;
                continue;
            }
            const uint32_t e = (uint32_t)__builtin_ctzll(nz) >> 3;
            if (p + e >= end) return 1;
            len += 255ull * e + ((x >> (8 * e)) & 0xffu);
            pp = p + e + 1;
            return 0;
        }
    }

    // ---------------------------------------------------------------- copies
    // Writes bytes [lo, hi) of chunk o to the ring at virtual position cv
    // (16-aligned); bytes outside [lo, hi) are left as they are (a chunk's
    // partial dwords are merged with LDS and / or atomics, so two lanes may
    // share a chunk).
    __device__ __forceinline__ void mwrite(uint32_t cv, const u32x4 &o, uint32_t lo, uint32_t hi) {
        lds8 *dst = ring + (cv & kRM);
        if (lo == 0 && hi == 16) {
            *reinterpret_cast<ldsx4 *>(dst) = o;
        } else {
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t m = dword_mask(lo, hi, i);
                lds32 *w = reinterpret_cast<lds32 *>(dst + 4 * i);
                __hip_atomic_fetch_and(w, ~m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                __hip_atomic_fetch_or(w, o[i] & m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
    }

    // 16 bytes of output from virtual position sp on: from the ring when
    // their 20-byte window (from sp rounded down to 4) starts at or after
    // rlo (written at most R bytes before the batch end), else from the
    // written-out output.  The output's dwords are read at addresses clamped
    // to the dwords holding the block's output bytes, so a window reaching
    // outside them reads no memory outside them (those bytes are never used:
    // they lie before a match's source).
    __device__ __forceinline__ u32x4 src16(int32_t sp, int32_t rlo) const {
        const int32_t w = sp & ~3;
        uint32_t d[5];
        if (LDS || w >= rlo) {
#pragma unroll
            for (int i = 0; i < 5; i++) d[i] = *reinterpret_cast<const lds32 *>(ring + (((uint32_t)w + 4u * i) & kRM));
        } else {
            const int32_t lo = (int32_t)(a0 & ~3u), hi = (int32_t)((a0 + cap - 1u) & ~3u);
#pragma unroll
            for (int i = 0; i < 5; i++) {
                int32_t x = w + 4 * i;
                x = x < lo ? lo : x > hi ? hi : x;
                d[i] = *reinterpret_cast<const uint32_t *>(obase + x);
            }
        }
        return realign(d, (uint32_t)sp & 3u);
    }

    // Chunk c of the literal run of n bytes at virtual position v whose
    // bytes are at stage offset src.
    __device__ __forceinline__ void lit_chunk(uint32_t v, uint32_t n, uint32_t src, uint32_t c) {
        const uint32_t cv = (v & ~15u) + 16u * c;
        const uint32_t lo = v > cv ? v - cv : 0u;
        const uint32_t hi = v + n - cv < 16u ? v + n - cv : 16u;
        const int32_t sp = (int32_t)(src + cv - v);  // >= src - 15
        const lds32 *q = reinterpret_cast<const lds32 *>(stage + (sp & ~3));
        uint32_t d[5];
#pragma unroll
        for (int i = 0; i < 5; i++) d[i] = q[i];
        mwrite(cv, realign(d, (uint32_t)sp & 3u), lo, hi);
    }

    // Chunk c of the match of n bytes at virtual position v, offset off.
    // Byte t of the match comes from v - off + (t mod off).  K: 0 a plain
    // copy (off >= n), 1 periodic with off >= 16, 2 periodic with off < 16,
    // -1 chosen per chunk (the runs of a pass differ).
    template <int K>
    __device__ __forceinline__ void match_chunk(uint32_t v, uint32_t n, uint32_t off, uint32_t c, int32_t rlo) {
        const uint32_t cv = (v & ~15u) + 16u * c;
        const uint32_t lo = v > cv ? v - cv : 0u;
        const uint32_t hi = v + n - cv < 16u ? v + n - cv : 16u;
        const int32_t r0 = (int32_t)(cv - v);  // match-relative position of chunk byte 0, >= -15
        u32x4 o;
        const int k = K >= 0 ? K : (r0 + (int32_t)hi <= (int32_t)off ? 0 : off >= 16u ? 1 : 2);
        if (k == 0) {
            // every byte of the chunk lies in the first period
            o = src16((int32_t)(cv - off), rlo);
        } else if (k == 1) {
            // byte t from v - off + ((a + t) mod off), wrapping at most once:
            // bytes before the wrap from base on, the rest from base - off on
            const uint32_t a = umod((uint32_t)(r0 + (int32_t)off), off);
            const int32_t base = (int32_t)(v - off + a);
            o = src16(base, rlo);
            const u32x4 b = src16(base - (int32_t)off, rlo);
            const uint32_t kw = off - a < 16u ? off - a : 16u;  // bytes before the wrap
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t m = dword_mask(0, kw, i);
                o[i] = (o[i] & m) | (b[i] & ~m);
            }
        } else {
            // byte t from v - off + ((a + t) mod off), in the ring
            uint32_t m = umod((uint32_t)(r0 + 16 * (int32_t)off), off);
            const uint32_t sv = v - off;
            uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (uint32_t t = 0; t < 16; t++) {
                d[t >> 2] |= (uint32_t)ring[(sv + m) & kRM] << (8 * (t & 3));
                m = m + 1 == off ? 0u : m + 1;
            }
            o = u32x4{d[0], d[1], d[2], d[3]};
        }
        mwrite(cv, o, lo, hi);
    }

    // Lane l's run for flat chunk g0 + l, given each run's first flat chunk
    // `ex` (runs in lane order, ex non-decreasing): the last run i with
    // ex_i <= g0 + l.  Runs starting in [g0, g0 + 64) mark their first lane
    // in the table (largest index wins), a prefix maximum spreads them, and
    // the runs started before g0 (a prefix of the lanes) set the floor.
    __device__ __forceinline__ uint32_t lane_run(uint32_t ex, uint32_t g0) {
        const int32_t u = (int32_t)(ex - g0);
        const uint32_t before = (uint32_t)__builtin_popcountll(ballot(u < 0));
        tab[lane] = 0u;
        if (u >= 0 && u < 64) __hip_atomic_fetch_max(&tab[u], (uint32_t)lane + 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_WORKGROUP);
        wave_sync();
        uint32_t x = tab[lane];
        x = scan_max(x > before ? x : before);
        return x - 1u;
    }

    // Copies the runs of the lanes with cnt > 0 (v: virtual position, n:
    // length, s: source -- stage offset of a literal run, offset of a
    // match), all runs of a kind at once.
    template <bool MATCH>
    __device__ __forceinline__ void run_pass(uint32_t v, uint32_t n, uint32_t s, bool on, int32_t rlo) {
        const uint32_t cnt = on && n > 0 ? ((v + n + 15u) >> 4) - (v >> 4) : 0u;
        const uint32_t incl = scan_add(cnt);
        const uint32_t total = rdl(incl, 63);
        const uint32_t ex = incl - cnt;
        for (uint32_t g0 = 0; g0 < total; g0 += 64) {
            const uint32_t gl = g0 + 63 < total ? g0 + 63 : total - 1;
            // runs of the first and last chunk of the pass
            const uint32_t rf = 63u - (uint32_t)__builtin_clzll(ballot(ex <= g0));
            const uint32_t rl = 63u - (uint32_t)__builtin_clzll(ballot(ex <= gl));
            uint32_t rv, rn, rs, rex;
            if (rf == rl) {
                rv = rdl(v, rf);
                rn = rdl(n, rf);
                rs = rdl(s, rf);
                rex = rdl(ex, rf);
            } else {
                const uint32_t r = lane_run(ex, g0);
                rv = bperm(v, r);
                rn = bperm(n, r);
                rs = bperm(s, r);
                rex = bperm(ex, r);
            }
            const uint32_t g = g0 + (uint32_t)lane;
            if (g < total) {
                if constexpr (MATCH)
                    match_chunk<-1>(rv, rn, rs, g - rex, rlo);
                else
                    lit_chunk(rv, rn, rs, g - rex);
            }
            wave_sync();
        }
    }

    // Copies one parsed batch: lane i < nsl holds slot i (a literal run of
    // ll bytes at stage offset ls, then a match of ml bytes at offset mo);
    // the batch starts at output position op_b and ends at op.
    // ------------------------------------------------ serial copies (long runs)
    // One run at a time in output order, 64 chunks per pass: a chunk's
    // bytes before the run keep what the ring holds (read back), its bytes
    // past the run are don't-care (the next run's first chunk overwrites
    // them; the flush writes out complete chunks only, and a batch ends 32
    // bytes short of the ring slots a near source occupies).
    __device__ __forceinline__ void keep_front(uint32_t cv, uint32_t v, u32x4 &o) const {
        if (cv < v) {  // the run's first chunk: keep its bytes before v
            const u32x4 old = *reinterpret_cast<const ldsx4 *>(ring + (cv & kRM));
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t m = dword_mask(0, v - cv, i);
                o[i] = (old[i] & m) | (o[i] & ~m);
            }
        }
    }
    __device__ __forceinline__ void lit_serial(uint32_t v, uint32_t n, uint32_t src) {
        const uint32_t c0 = v & ~15u;
        const uint32_t nch = ((v + n + 15u) >> 4) - (v >> 4);
        for (uint32_t b = 0; b < nch; b += 64) {
            const uint32_t c = b + (uint32_t)lane;
            if (c < nch) {
                const uint32_t cv = c0 + 16u * c;
                const int32_t sp = (int32_t)(src + cv - v);
                const lds32 *q = reinterpret_cast<const lds32 *>(stage + (sp & ~3));
                uint32_t d[5];
#pragma unroll
                for (int i = 0; i < 5; i++) d[i] = q[i];
                u32x4 o = realign(d, (uint32_t)sp & 3u);
                keep_front(cv, v, o);
                *reinterpret_cast<ldsx4 *>(ring + (cv & kRM)) = o;
            }
            wave_sync();
        }
    }
    template <int K>
    __device__ __forceinline__ void match_serial(uint32_t v, uint32_t n, uint32_t off, int32_t rlo) {
        const uint32_t c0 = v & ~15u;
        const uint32_t nch = ((v + n + 15u) >> 4) - (v >> 4);
        for (uint32_t b = 0; b < nch; b += 64) {
            const uint32_t c = b + (uint32_t)lane;
            if (c < nch) {
                const uint32_t cv = c0 + 16u * c;
                const int32_t r0 = (int32_t)(cv - v);
                u32x4 o;
                if (K == 0) {
                    o = src16((int32_t)(cv - off), rlo);
                } else if (K == 1) {
                    const uint32_t a = umod((uint32_t)(r0 + (int32_t)off), off);
                    const int32_t base = (int32_t)(v - off + a);
                    o = src16(base, rlo);
                    const u32x4 bb = src16(base - (int32_t)off, rlo);
                    const uint32_t kw = off - a < 16u ? off - a : 16u;
#pragma unroll
                    for (uint32_t i = 0; i < 4; i++) {
                        const uint32_t m = dword_mask(0, kw, i);
                        o[i] = (o[i] & m) | (bb[i] & ~m);
                    }
                } else {
                    uint32_t m = umod((uint32_t)(r0 + 16 * (int32_t)off), off);
                    const uint32_t sv = v - off;
                    uint32_t dd[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                    for (uint32_t t = 0; t < 16; t++) {
                        dd[t >> 2] |= (uint32_t)ring[(sv + m) & kRM] << (8 * (t & 3));
                        m = m + 1 == off ? 0u : m + 1;
                    }
                    o = u32x4{dd[0], dd[1], dd[2], dd[3]};
                }
                keep_front(cv, v, o);
                *reinterpret_cast<ldsx4 *>(ring + (cv & kRM)) = o;
            }
            wave_sync();
        }
    }

    __device__ __forceinline__ void execute(uint32_t nsl, uint32_t op_b, uint32_t ls, uint32_t ll, uint32_t mo,
                                            uint32_t ml) {
        const bool live = (uint32_t)lane < nsl;
        ll = live ? ll : 0u;
        ml = live ? ml : 0u;
        const uint32_t len = ll + ml;
        const uint32_t vl = op_b + a0 + scan_add(len) - len;  // virtual start of the slot
        const uint32_t vm = vl + ll;
        const int32_t rlo = (int32_t)(op + a0) - (int32_t)R;
        if (op - op_b >= 256u * nsl) {
            // runs of 128 bytes or more on average: one run per pass
            for (uint32_t i = 0; i < nsl; i++) {
                const uint32_t v = rdl(vl, i), n = rdl(ll, i);
                if (n > 0) lit_serial(v, n, rdl(ls, i));
                const uint32_t m = rdl(ml, i);
                if (m > 0) {
                    const uint32_t off = rdl(mo, i);
                    // (ring slots up to 16 bytes past a run's end may hold its
                    // don't-care bytes: the ring serves windows from rlo + 32)
                    if (off >= m)
                        match_serial<0>(v + n, m, off, rlo + 32);
                    else if (off >= 16u)
                        match_serial<1>(v + n, m, off, rlo + 32);
                    else
                        match_serial<2>(v + n, m, off, rlo + 32);
                }
            }
            return;
        }
        // short runs: all literal runs of the batch at once, then the matches
        run_pass<false>(vl, ll, ls, live, rlo);
        // matches in order; a pass takes the next pending match and every
        // following one up to the first whose source reaches past the start
        // of that first match
        const int32_t src_hi = (int32_t)(vm - mo + (mo < ml ? mo : ml));
        uint64_t pend = ballot(live && ml > 0);
        while (pend) {
            const uint32_t j0 = (uint32_t)__builtin_ctzll(pend);
            const int32_t D = (int32_t)rdl(vm, j0);
            const uint64_t block = pend & ~ballot(src_hi <= D);
            const uint64_t upto = block >> j0 ? ((1ull << ((uint32_t)__builtin_ctzll(block >> j0) + j0)) - 1) : ~0ull;
            const uint64_t grp = pend & upto;
            if ((grp & (grp - 1)) == 0) {
                // one match: its chunks over the lanes
                const uint32_t v = rdl(vm, j0), n = rdl(ml, j0), off = rdl(mo, j0);
                const uint32_t nch = ((v + n + 15u) >> 4) - (v >> 4);
                for (uint32_t c0 = 0; c0 < nch; c0 += 64) {
                    const uint32_t c = c0 + (uint32_t)lane;
                    if (c < nch) {
                        if (off >= n)
                            match_chunk<0>(v, n, off, c, rlo);
                        else if (off >= 16u)
                            match_chunk<1>(v, n, off, c, rlo);
                        else
                            match_chunk<2>(v, n, off, c, rlo);
                    }
                    wave_sync();
                }
            } else {
                run_pass<true>(vm, ml, mo, ((grp >> lane) & 1ull) != 0, rlo);
            }
            pend &= ~grp;
        }
    }

    // Writes the output [fl, op) out: all of it when `exact`, else up to the
    // last 16-aligned virtual position.
    __device__ __forceinline__ void flush(bool exact) {
        if constexpr (LDS) {
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
            *reinterpret_cast<u32x4 *>(obase + x) = *reinterpret_cast<const ldsx4 *>(ring + (x & kRM));
        }
        const uint32_t vt = vb + 16u * nch;
        if (lane < (int)(ve - vt)) obase[vt + lane] = ring[(vt + lane) & kRM];
        fl = ve - a0;
        __asm__ __volatile__("" ::: "memory");
    }
};

// Decodes one block whose input is [0, ilen) (block-relative) into d; on
// return code / detail / pos / req hold the outcome (HH_OK or the
// reference's error record) and d.op the bytes decoded.  The caller writes
// out the rest of a successful block (d.flush(true)).  `staged`: the caller
// has already put the stage for input position 0 in place.
//
// A batch is parsed in two ways.  The fast loop only follows the chain of
// headers -- token, literal length, offset, match length -- and records
// each sequence in a lane, stopping where a header would leave the stage or
// a length extension is longer than 7 (6) bytes; the wave then checks all of
// the recorded sequences at once (input bounds, capacity, offsets, the
// batch budget) and keeps those before the first one that fails.  The
// general step parses the sequence after them one state at a time with
// every check in the reference's order: a run continued from the previous
// batch, a run cut by the stage end or the budget, long extensions, and
// every error, reported as the reference reports it.
template <uint32_t R, uint32_t S, bool LDS, typename Progress = NoProgress>
__device__ __forceinline__ void decode_block(SeqDec<R, S, LDS> &d, uint32_t ilen, int32_t &code, int32_t &detail,
                                             uint64_t &pos, uint64_t &req, bool staged = false,
                                             Progress &&progress = Progress{}) {
    using D = SeqDec<R, S, LDS>;
    const uint32_t end = ilen;
    const uint32_t cap = d.cap;
    const uint32_t lane = (uint32_t)d.lane;
    uint32_t ip = 0;
    uint32_t ms = kToken;
    uint32_t lit_rem = 0, m_rem = 0, m_off = 0, tml = 0;
    d.hv = 0;
    d.hb = 0;
    d.pf_on = false;
    if (end == 0) return;
    if (!staged)
        d.restage(0);
    else
        d.prefetch();
    for (;;) {
        // ---------------------------------------------------------- parse
        const uint32_t op_b = d.op;
        uint32_t op = d.op;
        uint32_t nsl = 0, bout = 0;
        // the batch's output may not pass lim (near match sources stay in
        // the ring)
        uint32_t lim = 0xffffffffu;
        bool done = false, restage = false;
        // slots in lanes (slot i in lane i): literal stage offset and length,
        // match offset and length, token position (fast loop only)
        uint32_t ls = 0, ll = 0, mo = 0, ml = 0, tp = 0;
        if (ms != kToken) nsl = 1;  // a run continued from the previous batch
        for (;;) {
            // ---- fast loop: header chain only
            if (ms == kToken) {
                const uint32_t f0 = nsl;
                // last position a header may start at: before the block end,
                // with 8 bytes in the stage
                const uint32_t hl = d.at_end ? end - 1u : (end - 1u < d.sb + (S - 8u) ? end - 1u : d.sb + (S - 8u));
                uint32_t fp = ip;
                // output end and near-match limit of the chain so far: the
                // loop stops before a sequence that would pass the batch's
                // budget or limit (the check after it then rarely fails)
                uint32_t fo = op;
                uint32_t fl = lim < op_b + D::kOB ? lim : op_b + D::kOB;
                bool full = false;
                while (nsl < 64u && fp <= hl) {
                    if (!d.in_win8(fp)) d.read16(fp);
                    const uint64_t t8 = d.peek8(fp);
                    const uint32_t token = (uint32_t)t8 & 0xffu;
                    uint32_t lit = token >> 4;
                    uint32_t p = fp + 1;
                    if (lit == 15u) {
                        const uint64_t x = t8 >> 8;
                        const uint32_t e = (uint32_t)__builtin_ctzll(~x | (1ull << 56)) >> 3;  // 7: none
                        if (e == 7u) break;
                        lit += 255u * e + (uint32_t)((x >> (8 * e)) & 0xffu);
                        p += e + 1;
                    }
                    const uint32_t le = p + lit;  // offset position
                    if (le > hl) break;
                    if (!d.in_win8(le)) d.read16(le);
                    const uint64_t o8 = d.peek8(le);
                    uint32_t mlen = (token & 15u) + 4u;
                    uint32_t q = le + 2;
                    if ((token & 15u) == 15u) {
                        const uint64_t x = o8 >> 16;
                        const uint32_t e = (uint32_t)__builtin_ctzll(~x | (1ull << 48)) >> 3;  // 6: none
                        if (e == 6u) break;
                        mlen += 255u * e + (uint32_t)((x >> (8 * e)) & 0xffu);
                        q += e + 1;
                    }
                    const uint32_t off = (uint32_t)o8 & 0xffffu;
                    const uint32_t fm = fo + lit;
                    uint32_t fl2 = fl;
                    if (!LDS && off <= R - 128u && off <= fm) {
                        const uint32_t l2 = fm - off + (R - 64u);
                        fl2 = l2 < fl2 ? l2 : fl2;
                    }
                    if (fm + mlen > fl2) {
                        full = true;
                        break;
                    }
                    const bool me = lane == nsl;
                    tp = me ? fp : tp;
                    ls = me ? p - d.sb : ls;
                    ll = me ? lit : ll;
                    mo = me ? off : mo;
                    ml = me ? mlen : ml;
                    nsl++;
                    fp = q;
                    fo = fm + mlen;
                    fl = fl2;
                }
                if (nsl > f0) {
                    // check slots f0 .. nsl - 1 at once; keep those before
                    // the first that fails (the general step parses it again)
                    const bool live = lane < nsl;
                    const uint32_t len = live ? ll + ml : 0u;
                    const uint32_t oe = op_b + scan_add(len);  // output end of each slot
                    const uint32_t om = oe - ml;               // output position of the match
                    const uint32_t qn = bperm(tp, lane + 1u);
                    const uint32_t q = lane + 1u == nsl ? fp : qn;  // input end of each slot
                    // near-match limit: prefix minimum over the fast slots
                    uint32_t nl = (!LDS && lane >= f0 && live && mo <= R - 128u) ? om - mo + (R - 64u) : 0xffffffffu;
                    nl = ~scan_max(~nl);
                    nl = nl < lim ? nl : lim;
                    const bool ok = q <= end && om < cap && mo != 0u && mo <= om && oe <= cap && oe - op_b <= D::kOB &&
                                    oe <= nl;
                    const uint64_t badm = ballot(!ok && lane >= f0 && live);
                    const uint32_t f = badm ? (uint32_t)__builtin_ctzll(badm) : nsl;
                    if (f > f0) {
                        op = rdl(oe, f - 1u);
                        lim = rdl(nl, f - 1u);
                        bout = op - op_b;
                    }
                    if (f < nsl) full = false;
                    ip = f < nsl ? rdl(tp, f) : fp;
                    nsl = f;
                    const bool keep = lane < f;
                    ls = keep ? ls : 0u;
                    ll = keep ? ll : 0u;
                    mo = keep ? mo : 0u;
                    ml = keep ? ml : 0u;
                }
                // the next sequence does not fit this batch: start the next
                // one with it (the general step splits only a sequence that
                // an empty batch cannot hold)
                if (full && bout > 0) break;
            }
            // ---- general step
            if (ms == kToken) {
                if (ip >= end) {
                    done = true;
                    break;
                }
                if (nsl == 64u) break;
                if (!d.in_win8(ip) && !d.in_stage8(ip)) {
                    restage = true;
                    break;
                }
                // token and literal length (block.rs:270-289); the extension
                // bytes usually lie in the 7 bytes after the token
                const uint64_t t8 = d.get8(ip);
                const uint32_t token = (uint32_t)t8 & 0xffu;
                uint32_t lit = token >> 4;
                uint32_t p = ip + 1;
                if (lit == 15) {
                    const uint64_t x = t8 >> 8;
                    const uint64_t nz = ~x & 0x00ffffffffffffffull;
                    if (nz != 0) {
                        const uint32_t e = (uint32_t)__builtin_ctzll(nz) >> 3;
                        if (p + e >= end) {
                            code = HH_ERR_UNEXPECTED_EOF;
                            pos = ilen;
                            return;
                        }
                        lit += 255u * e + (uint32_t)((x >> (8 * e)) & 0xffu);
                        p += e + 1;
                    } else {
                        uint64_t l64 = lit + 255ull * 7;
                        p += 7;
                        const int r = p >= end ? 1 : d.ext_slow(p, end, l64, bout != 0);
                        if (r == 1) {
                            code = HH_ERR_UNEXPECTED_EOF;
                            pos = ilen;
                            return;
                        }
                        if (r == 2) {  // parse this sequence again after the batch
                            restage = true;
                            break;
                        }
                        // a length beyond 32 bits exceeds the block input:
                        // the input-length check below fails for it too
                        if (l64 > 0xffffffffull) {
                            code = HH_ERR_UNEXPECTED_EOF;
                            pos = p;
                            return;
                        }
                        lit = (uint32_t)l64;
                    }
                }
                if (lit > 0) {
                    if (end - p < lit) {
                        code = HH_ERR_UNEXPECTED_EOF;
                        pos = p;
                        return;
                    }
                    if (lit > cap - op) {
                        code = HH_ERR_BUFFER_TOO_SMALL;
                        req = (uint64_t)op + lit;
                        return;
                    }
                }
                nsl++;  // the sequence's slot (zero in every lane)
                tml = token & 15u;
                ip = p;
                lit_rem = lit;
                ms = kLit;
            }
            if (ms == kLit) {
                if (lit_rem > 0) {
                    const uint32_t av = d.lit_avail(ip);
                    uint32_t n = lit_rem < av ? lit_rem : av;
                    if (n > D::kOB - bout) n = D::kOB - bout;
                    if (n > lim - op) n = lim - op;
                    if (n == 0) {
                        restage = av == 0;
                        break;
                    }
                    const bool me = lane == nsl - 1u;
                    ls = me ? ip - d.sb : ls;
                    ll = me ? n : ll;
                    ip += n;
                    op += n;
                    bout += n;
                    lit_rem -= n;
                    if (lit_rem > 0) {
                        restage = av == n;
                        break;
                    }
                }
                if (op >= cap) {  // block.rs:309-311
                    done = true;
                    break;
                }
                ms = kOff;
            }
            if (ms == kOff) {
                // offset and match length (block.rs:313-345)
                if (end - ip < 2) {
                    code = HH_ERR_UNEXPECTED_EOF;
                    pos = ip;
                    return;
                }
                if (!d.in_win8(ip) && !d.in_stage8(ip)) {
                    restage = true;
                    break;
                }
                const uint64_t o8 = d.get8(ip);
                const uint32_t off = (uint32_t)o8 & 0xffffu;
                uint32_t p = ip + 2;
                if (off == 0) {
                    code = HH_ERR_CORRUPTED_DATA;
                    detail = HH_CORRUPT_ZERO_OFFSET;
                    return;
                }
                if (off > op) {
                    code = HH_ERR_CORRUPTED_DATA;
                    detail = HH_CORRUPT_OFFSET_BEYOND;
                    pos = op;
                    return;
                }
                uint32_t mlen = tml + 4u;
                if (tml == 15u) {
                    const uint64_t x = o8 >> 16;
                    const uint64_t nz = ~x & 0x0000ffffffffffffull;
                    if (nz != 0) {
                        const uint32_t e = (uint32_t)__builtin_ctzll(nz) >> 3;
                        if (p + e >= end) {
                            code = HH_ERR_UNEXPECTED_EOF;
                            pos = ilen;
                            return;
                        }
                        mlen += 255u * e + (uint32_t)((x >> (8 * e)) & 0xffu);
                        p += e + 1;
                    } else {
                        uint64_t m64 = mlen + 255ull * 6;
                        p += 6;
                        const int r = p >= end ? 1 : d.ext_slow(p, end, m64, bout != 0);
                        if (r == 1) {
                            code = HH_ERR_UNEXPECTED_EOF;
                            pos = ilen;
                            return;
                        }
                        if (r == 2) {  // parse the offset again after the batch
                            restage = true;
                            break;
                        }
                        if (m64 > 0xffffffffull) {  // more than any capacity
                            code = HH_ERR_BUFFER_TOO_SMALL;
                            req = (uint64_t)op + m64;
                            return;
                        }
                        mlen = (uint32_t)m64;
                    }
                }
                if (mlen > cap - op) {
                    code = HH_ERR_BUFFER_TOO_SMALL;
                    req = (uint64_t)op + mlen;
                    return;
                }
                ip = p;
                m_rem = mlen;
                m_off = off;
                ms = kMatch;
            }
            // ms == kMatch: a match whose offset fits the ring reads it
            // there: the batch then ends before its output reaches R - 64
            // bytes past the match's source
            uint32_t lm = lim;
            if (!LDS && m_off <= R - 128u) {
                const uint32_t l2 = op - m_off + (R - 64u);
                lm = l2 < lm ? l2 : lm;
            }
            uint32_t n = m_rem;
            if (n > D::kOB - bout) n = D::kOB - bout;
            if (n > lm - op) n = lm - op;
            if (n == 0) break;
            lim = lm;
            {
                const bool me = lane == nsl - 1u;
                mo = me ? m_off : mo;
                ml = me ? n : ml;
            }
            op += n;
            bout += n;
            m_rem -= n;
            if (m_rem > 0) break;
            ms = kToken;
        }
        // ---------------------------------------------------------- copy
        // the next stage is put in place after the copies (which read the
        // current one) and before the batch's output is written out, so the
        // wait for its loads does not include those stores (a wave's memory
        // operations complete in order)
        d.op = op;
        if (bout > 0) d.execute(nsl, op_b, ls, ll, mo, ml);
        if (restage) d.restage(ip);
        if (bout > 0) {
            d.flush(false);
            progress(op);
        }
        if (done) return;
    }
}

}  // namespace seq
}  // namespace hh
