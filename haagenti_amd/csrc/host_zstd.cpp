// Zstandard frame decoder on the host (RFC 8878), for the zstd wrapper the
// turbo pipeline puts around HCT3 containers
// (crates/haagenti/src/pipeline/turbo.rs:389-391, zstd::encode_all level 1)
// and GpuDecompressor::try_zstd_decompress (crates/haagenti-cuda/src/
// decompress.rs:296-319, zstd::decode_all).  The reference links the zstd
// crate 0.13.3 (libzstd); this is a restatement of the published format:
//   frames: magic 0xFD2FB528, frame header, blocks (raw / RLE / compressed),
//           optional XXH64 content checksum; skippable frames are skipped;
//   compressed blocks: literals (raw, RLE, Huffman with 1 or 4 streams, or
//           the previous Huffman table), then sequences whose literal
//           lengths, match lengths and offsets are FSE-coded (predefined,
//           RLE, described or repeated tables), executed with the three
//           repeat offsets.
// Frames with a dictionary id are rejected (decode_all has no dictionary),
// as are windows above 2^27 bytes (libzstd's default decoding limit).
#include <cstdint>
#include <cstddef>
#include <climits>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/haagenti_hip.h"

namespace {

// ---------------------------------------------------------------- XXH64
constexpr uint64_t P1 = 11400714785074694791ull, P2 = 14029467366897019727ull, P3 = 1609587929392839161ull,
                   P4 = 9650029242287828579ull, P5 = 2870177450012600261ull;
inline uint64_t rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
inline uint64_t ld64(const uint8_t *p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}
inline uint32_t ld32(const uint8_t *p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
inline uint64_t round64(uint64_t acc, uint64_t in) { return rotl(acc + in * P2, 31) * P1; }
inline uint64_t merge64(uint64_t acc, uint64_t v) { return (acc ^ round64(0, v)) * P1 + P4; }

uint64_t xxh64(const uint8_t *p, size_t len, uint64_t seed) {
    const uint8_t *end = p + len;
    uint64_t h;
    if (len >= 32) {
        uint64_t v1 = seed + P1 + P2, v2 = seed + P2, v3 = seed, v4 = seed - P1;
        const uint8_t *limit = end - 32;
        do {
            v1 = round64(v1, ld64(p));
            v2 = round64(v2, ld64(p + 8));
            v3 = round64(v3, ld64(p + 16));
            v4 = round64(v4, ld64(p + 24));
            p += 32;
        } while (p <= limit);
        h = rotl(v1, 1) + rotl(v2, 7) + rotl(v3, 12) + rotl(v4, 18);
        h = merge64(h, v1);
        h = merge64(h, v2);
        h = merge64(h, v3);
        h = merge64(h, v4);
    } else {
        h = seed + P5;
    }
    h += (uint64_t)len;
    while (p + 8 <= end) {
        h ^= round64(0, ld64(p));
        h = rotl(h, 27) * P1 + P4;
        p += 8;
    }
    if (p + 4 <= end) {
        h ^= (uint64_t)ld32(p) * P1;
        h = rotl(h, 23) * P2 + P3;
        p += 4;
    }
    while (p < end) {
        h ^= (uint64_t)(*p) * P5;
        h = rotl(h, 11) * P1;
        p++;
    }
    h ^= h >> 33;
    h *= P2;
    h ^= h >> 29;
    h *= P3;
    h ^= h >> 32;
    return h;
}

// ---------------------------------------------------------------- bit readers
struct Fail {};  // thrown on corrupt input; caught at the entry point

// Forward little-endian bit reader (FSE table descriptions).
struct FwdBits {
    const uint8_t *p;
    size_t n;
    uint64_t bit = 0;
    uint32_t peek(int nb) const {  // nb <= 25
        uint32_t v = 0;
        for (int i = 0; i < nb; i++) {
            const uint64_t b = bit + i;
            if ((b >> 3) < n) v |= (uint32_t)((p[b >> 3] >> (b & 7)) & 1u) << i;
        }
        return v;
    }
    void skip(int nb) { bit += nb; }
    size_t bytes() const { return (size_t)((bit + 7) >> 3); }
};

// Backward bit reader: the stream's last byte holds a 1 marker bit above the
// data; reads take the highest unread bits, the most recent bit most
// significant; bits before the stream start read as zero.
struct BackBits {
    const uint8_t *p = nullptr;
    size_t n = 0;
    int64_t pos = 0;  // unread bits are [0, pos)
    void init(const uint8_t *src, size_t len) {
        if (len == 0 || src[len - 1] == 0) throw Fail{};
        p = src;
        n = len;
        pos = (int64_t)(len - 1) * 8 + (31 - __builtin_clz((unsigned)src[len - 1]));
    }
    uint64_t get(int64_t start, int nb) const {  // bits [start, start + nb), nb <= 56
        if (nb == 0) return 0;
        // the 8 bytes ending at the byte of the last bit hold all nb bits
        const int64_t base = ((start + nb - 1) >> 3) - 7;
        if (start >= 0 && base >= 0 && (size_t)base + 8 <= n)
            return (ld64(p + base) >> (start - base * 8)) & ((1ull << nb) - 1);
        uint64_t v = 0;
        const int64_t first = start >> 3, last = (start + nb - 1) >> 3;
        for (int64_t b = last; b >= first; b--) v = (v << 8) | (b >= 0 && (size_t)b < n ? p[b] : 0u);
        const int sh = (int)(start - first * 8);
        v >>= sh;
        return nb == 64 ? v : v & ((1ull << nb) - 1);
    }
    uint64_t read(int nb) {
        pos -= nb;
        return get(pos, nb);
    }
    uint64_t peek(int nb) const { return get(pos - nb, nb); }
    void skip(int nb) { pos -= nb; }
    bool overflow() const { return pos < 0; }
};

// ---------------------------------------------------------------- FSE
struct FseEntry {
    uint16_t symbol;
    uint8_t nbits;
    uint16_t base;  // next state = base + read(nbits)
};
struct FseTable {
    int log = 0;
    std::vector<FseEntry> t;
};

// Decoding table from normalized counts (-1 = "less than one").
void fse_build(FseTable &T, const int16_t *norm, int nsym, int log) {
    const uint32_t size = 1u << log;
    T.log = log;
    T.t.assign(size, FseEntry{0, 0, 0});
    std::vector<uint16_t> next(nsym);
    uint32_t high = size - 1;
    for (int s = 0; s < nsym; s++) {
        if (norm[s] == -1) {
            T.t[high--].symbol = (uint16_t)s;
            next[s] = 1;
        } else {
            next[s] = (uint16_t)(norm[s] < 0 ? 0 : norm[s]);
        }
    }
    const uint32_t step = (size >> 1) + (size >> 3) + 3, mask = size - 1;
    uint32_t pos = 0;
    for (int s = 0; s < nsym; s++)
        for (int i = 0; i < norm[s]; i++) {
            T.t[pos].symbol = (uint16_t)s;
            do pos = (pos + step) & mask;
            while (pos > high);
        }
    if (pos != 0) throw Fail{};
    for (uint32_t u = 0; u < size; u++) {
        const uint16_t s = T.t[u].symbol;
        const uint32_t ns = next[s]++;
        const int hb = 31 - __builtin_clz(ns);
        T.t[u].nbits = (uint8_t)(log - hb);
        T.t[u].base = (uint16_t)((ns << (log - hb)) - size);
    }
}

// FSE table description (normalized counts), returns bytes consumed.
size_t fse_read_ncount(FseTable &T, const uint8_t *src, size_t len, int max_sym, int max_log) {
    FwdBits br{src, len};
    const int log = (int)br.peek(4) + 5;
    br.skip(4);
    if (log > max_log) throw Fail{};
    std::vector<int16_t> norm(max_sym + 1, 0);
    int remaining = (1 << log) + 1, threshold = 1 << log, nb = log + 1, s = 0;
    bool prev0 = false;
    while (remaining > 1) {
        if (prev0) {
            // runs of zero probabilities: 2-bit repeat fields, 3 = keep going
            for (;;) {
                const uint32_t r = br.peek(2);
                br.skip(2);
                s += (int)r;
                if (r != 3) break;
            }
            if (s > max_sym) throw Fail{};
        }
        if (s > max_sym) throw Fail{};
        const int maxv = (2 * threshold - 1) - remaining;
        int count;
        const uint32_t low = br.peek(nb - 1);
        if ((int)low < maxv) {
            count = (int)low;
            br.skip(nb - 1);
        } else {
            count = (int)br.peek(nb);
            if (count >= threshold) count -= maxv;
            br.skip(nb);
        }
        count--;
        remaining -= count < 0 ? -count : count;
        norm[s++] = (int16_t)count;
        prev0 = count == 0;
        while (remaining < threshold) {
            nb--;
            threshold >>= 1;
        }
        if (br.bytes() > len) throw Fail{};
    }
    if (remaining != 1) throw Fail{};
    fse_build(T, norm.data(), s, log);
    return br.bytes();
}

// ---------------------------------------------------------------- Huffman
struct HufTable {
    int maxbits = 0;
    std::vector<uint8_t> sym, nbits;  // indexed by the top maxbits bits
};

void huf_build(HufTable &H, const uint8_t *w, int nsym) {
    // weights of the given symbols; the last one completes a power of two
    uint32_t total = 0;
    for (int i = 0; i < nsym; i++) {
        if (w[i] > 11) throw Fail{};
        if (w[i]) total += 1u << (w[i] - 1);
    }
    if (total == 0) throw Fail{};
    const int maxbits = 32 - __builtin_clz(total);  // floor(log2) + 1
    const uint32_t rest = (1u << maxbits) - total;
    if (rest == 0 || (rest & (rest - 1)) || maxbits > 11) throw Fail{};
    std::vector<uint8_t> weights(w, w + nsym);
    weights.push_back((uint8_t)(__builtin_ctz(rest) + 1));
    const int n = nsym + 1;
    H.maxbits = maxbits;
    H.sym.assign(1u << maxbits, 0);
    H.nbits.assign(1u << maxbits, 0);
    // table slots by increasing weight, symbols in increasing order within a weight
    uint32_t start[13] = {0}, count[13] = {0};
    for (int i = 0; i < n; i++) count[weights[i]]++;
    uint32_t cur = 0;
    for (int wt = 1; wt <= maxbits; wt++) {
        start[wt] = cur;
        cur += count[wt] << (wt - 1);
    }
    for (int i = 0; i < n; i++) {
        const int wt = weights[i];
        if (!wt) continue;
        const uint32_t len = 1u << (wt - 1);
        for (uint32_t j = 0; j < len; j++) {
            H.sym[start[wt] + j] = (uint8_t)i;
            H.nbits[start[wt] + j] = (uint8_t)(maxbits + 1 - wt);
        }
        start[wt] += len;
    }
}

// Huffman tree description, returns bytes consumed.
size_t huf_read_table(HufTable &H, const uint8_t *src, size_t len) {
    if (len < 1) throw Fail{};
    const uint8_t hb = src[0];
    uint8_t w[256];
    int nsym;
    size_t used;
    if (hb < 128) {
        // FSE-compressed weights: hb bytes, two interleaved states
        if ((size_t)hb + 1 > len || hb == 0) throw Fail{};
        FseTable T;
        const size_t nc = fse_read_ncount(T, src + 1, hb, 255, 6);
        if (nc >= hb) throw Fail{};
        BackBits br;
        br.init(src + 1 + nc, hb - nc);
        uint32_t s1 = (uint32_t)br.read(T.log), s2 = (uint32_t)br.read(T.log);
        nsym = 0;
        for (;;) {
            if (nsym >= 255) throw Fail{};
            w[nsym++] = (uint8_t)T.t[s1].symbol;
            s1 = T.t[s1].base + (uint32_t)br.read(T.t[s1].nbits);
            if (br.overflow()) {
                if (nsym >= 255) throw Fail{};
                w[nsym++] = (uint8_t)T.t[s2].symbol;
                break;
            }
            if (nsym >= 255) throw Fail{};
            w[nsym++] = (uint8_t)T.t[s2].symbol;
            s2 = T.t[s2].base + (uint32_t)br.read(T.t[s2].nbits);
            if (br.overflow()) {
                if (nsym >= 255) throw Fail{};
                w[nsym++] = (uint8_t)T.t[s1].symbol;
                break;
            }
        }
        used = 1 + (size_t)hb;
    } else {
        nsym = hb - 127;
        const size_t nb = (size_t)(nsym + 1) / 2;
        if (1 + nb > len) throw Fail{};
        for (int i = 0; i < nsym; i++) w[i] = (uint8_t)(i & 1 ? src[1 + i / 2] & 15 : src[1 + i / 2] >> 4);
        used = 1 + nb;
    }
    huf_build(H, w, nsym);
    return used;
}

void huf_stream(const HufTable &H, const uint8_t *src, size_t len, uint8_t *out, size_t n) {
    BackBits br;
    br.init(src, len);
    for (size_t i = 0; i < n; i++) {
        const uint32_t idx = (uint32_t)br.peek(H.maxbits);
        out[i] = H.sym[idx];
        br.skip(H.nbits[idx]);
    }
    if (br.pos != 0) throw Fail{};  // the stream is consumed exactly
}

// Up to four Huffman streams decoded in one loop, so that their symbol
// chains (each read depends on the previous symbol's length) overlap; each
// stream reads from a 64-bit window reloaded from memory while at least 7
// bytes precede its read position, and through BackBits near its start.
void huf_streams(const HufTable &H, int k, const uint8_t *const *src, const size_t *len, uint8_t *const *out,
                 const size_t *n) {
    BackBits br[4];
    size_t nmin = SIZE_MAX;
    for (int j = 0; j < k; j++) {
        br[j].init(src[j], len[j]);
        nmin = n[j] < nmin ? n[j] : nmin;
    }
    const int mb = H.maxbits;
    const uint8_t *sym = H.sym.data(), *nbits = H.nbits.data();
    size_t i = 0;
    // all streams in step while each has >= 8 readable bytes below its position
    for (; i < nmin; i++) {
        bool fast = true;
        for (int j = 0; j < k; j++) fast = fast && br[j].pos - mb >= 64;
        if (!fast) break;
        for (int j = 0; j < k; j++) {
            const int64_t start = br[j].pos - mb;
            const int64_t base = ((br[j].pos - 1) >> 3) - 7;
            const uint32_t idx = (uint32_t)((ld64(br[j].p + base) >> (start - base * 8)) & ((1ull << mb) - 1));
            out[j][i] = sym[idx];
            br[j].pos -= nbits[idx];
        }
    }
    for (int j = 0; j < k; j++) {
        for (size_t q = i; q < n[j]; q++) {
            const uint32_t idx = (uint32_t)br[j].peek(mb);
            out[j][q] = sym[idx];
            br[j].skip(nbits[idx]);
        }
        if (br[j].pos != 0) throw Fail{};
    }
}

// ---------------------------------------------------------------- sequences
const uint32_t kLLBase[36] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 18, 20, 22, 24, 28, 32, 40,
                              48, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768, 65536};
const uint8_t kLLBits[36] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 3, 3,
                             4, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16};
const uint32_t kMLBase[53] = {3,  4,  5,  6,  7,  8,  9,  10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20,
                              21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31, 32, 33, 34, 35, 37, 39, 41,
                              43, 47, 51, 59, 67, 83, 99, 131, 259, 515, 1027, 2051, 4099, 8195, 16387, 32771, 65539};
static_assert(sizeof(kLLBase) / sizeof(kLLBase[0]) == 36 && sizeof(kLLBits) == 36, "LL table");
static_assert(sizeof(kMLBase) / sizeof(kMLBase[0]) == 53, "ML table");
const uint8_t kMLBits[53] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                             0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 3, 3, 4, 4, 5, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16};
// predefined distributions (RFC 8878 section 3.1.1.3.2.2)
const int16_t kLLDefault[36] = {4, 3, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 1, 1, 1, 2, 2,
                                2, 2, 2, 2, 2, 2, 2, 3, 2, 1, 1, 1, 1, 1, -1, -1, -1, -1};
const int16_t kMLDefault[53] = {1, 4, 3, 2, 2, 2, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1,
                                1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, -1, -1, -1, -1, -1, -1, -1};
const int16_t kOFDefault[29] = {1, 1, 1, 1, 1, 1, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, -1, -1, -1, -1, -1};

struct FrameState {
    HufTable huf;
    bool have_huf = false;
    FseTable ll, of, ml;
    bool have_ll = false, have_of = false, have_ml = false;
    uint32_t rep[3] = {1, 4, 8};
    size_t frame_start = 0;  // output position where this frame began
    uint64_t window = 0;
};

// table for one of LL / OF / ML per its compression mode; returns bytes used
size_t seq_table(FseTable &T, bool &have, int mode, const uint8_t *src, size_t len, const int16_t *def,
                 int ndef, int deflog, int max_sym, int max_log) {
    switch (mode) {
        case 0:
            fse_build(T, def, ndef, deflog);
            have = true;
            return 0;
        case 1: {  // RLE: one symbol, every state decodes it with 0 bits
            if (len < 1 || src[0] > max_sym) throw Fail{};
            T.log = 0;
            T.t.assign(1, FseEntry{src[0], 0, 0});
            have = true;
            return 1;
        }
        case 2: {
            const size_t n = fse_read_ncount(T, src, len, max_sym, max_log);
            have = true;
            return n;
        }
        default:
            if (!have) throw Fail{};
            return 0;
    }
}

void decode_block(FrameState &F, const uint8_t *src, size_t len, std::vector<uint8_t> &out) {
    if (len < 1) throw Fail{};
    // ---- literals section
    const uint8_t b0 = src[0];
    const int ltype = b0 & 3, sf = (b0 >> 2) & 3;
    std::vector<uint8_t> lit;
    size_t p = 0;
    if (ltype == 0 || ltype == 1) {
        size_t regen, hdr;
        if ((sf & 1) == 0) {
            regen = b0 >> 3;
            hdr = 1;
        } else if (sf == 1) {
            if (len < 2) throw Fail{};
            regen = (b0 >> 4) + ((size_t)src[1] << 4);
            hdr = 2;
        } else {
            if (len < 3) throw Fail{};
            regen = (b0 >> 4) + ((size_t)src[1] << 4) + ((size_t)src[2] << 12);
            hdr = 3;
        }
        p = hdr;
        if (ltype == 0) {
            if (p + regen > len) throw Fail{};
            lit.assign(src + p, src + p + regen);
            p += regen;
        } else {
            if (p + 1 > len) throw Fail{};
            lit.assign(regen, src[p]);
            p += 1;
        }
    } else {
        size_t regen, comp, hdr;
        int streams;
        if (len < (size_t)(sf <= 1 ? 3 : sf == 2 ? 4 : 5)) throw Fail{};
        if (sf <= 1) {
            const uint32_t h = src[0] | (src[1] << 8) | (src[2] << 16);
            regen = (h >> 4) & 0x3ff;
            comp = (h >> 14) & 0x3ff;
            hdr = 3;
            streams = sf == 0 ? 1 : 4;
        } else if (sf == 2) {
            const uint32_t h = ld32(src);
            regen = (h >> 4) & 0x3fff;
            comp = (h >> 18) & 0x3fff;
            hdr = 4;
            streams = 4;
        } else {
            const uint64_t h = (uint64_t)ld32(src) | ((uint64_t)src[4] << 32);
            regen = (size_t)((h >> 4) & 0x3ffff);
            comp = (size_t)((h >> 22) & 0x3ffff);
            hdr = 5;
            streams = 4;
        }
        if (hdr + comp > len) throw Fail{};
        const uint8_t *c = src + hdr;
        size_t cl = comp;
        if (ltype == 2) {
            const size_t t = huf_read_table(F.huf, c, cl);
            F.have_huf = true;
            c += t;
            cl -= t;
        } else if (!F.have_huf) {
            throw Fail{};
        }
        lit.resize(regen);
        if (streams == 1) {
            huf_stream(F.huf, c, cl, lit.data(), regen);
        } else {
            if (cl < 6) throw Fail{};
            const size_t s1 = c[0] | (c[1] << 8), s2 = c[2] | (c[3] << 8), s3 = c[4] | (c[5] << 8);
            if (6 + s1 + s2 + s3 > cl) throw Fail{};
            const size_t s4 = cl - 6 - s1 - s2 - s3;
            const size_t q = (regen + 3) / 4;
            if (3 * q > regen) throw Fail{};
            const uint8_t *d = c + 6;
            const uint8_t *srcs[4] = {d, d + s1, d + s1 + s2, d + s1 + s2 + s3};
            const size_t lens[4] = {s1, s2, s3, s4};
            uint8_t *outs[4] = {lit.data(), lit.data() + q, lit.data() + 2 * q, lit.data() + 3 * q};
            const size_t ns[4] = {q, q, q, regen - 3 * q};
            huf_streams(F.huf, 4, srcs, lens, outs, ns);
        }
        p = hdr + comp;
    }
    // ---- sequences section
    if (p >= len) throw Fail{};
    size_t nseq = src[p];
    if (nseq < 128) {
        p += 1;
    } else if (nseq < 255) {
        if (p + 2 > len) throw Fail{};
        nseq = ((nseq - 128) << 8) + src[p + 1];
        p += 2;
    } else {
        if (p + 3 > len) throw Fail{};
        nseq = src[p + 1] + ((size_t)src[p + 2] << 8) + 0x7f00;
        p += 3;
    }
    size_t lp = 0;
    if (nseq == 0) {
        out.insert(out.end(), lit.begin(), lit.end());
        if (p != len) throw Fail{};
        return;
    }
    if (p >= len) throw Fail{};
    const uint8_t modes = src[p++];
    if (modes & 3) throw Fail{};
    p += seq_table(F.ll, F.have_ll, modes >> 6, src + p, len - p, kLLDefault, 36, 6, 35, 9);
    if (p > len) throw Fail{};
    p += seq_table(F.of, F.have_of, (modes >> 4) & 3, src + p, len - p, kOFDefault, 29, 5, 31, 8);
    if (p > len) throw Fail{};
    p += seq_table(F.ml, F.have_ml, (modes >> 2) & 3, src + p, len - p, kMLDefault, 53, 6, 52, 9);
    if (p >= len) throw Fail{};
    BackBits br;
    br.init(src + p, len - p);
    uint32_t sll = (uint32_t)br.read(F.ll.log), sof = (uint32_t)br.read(F.of.log), sml = (uint32_t)br.read(F.ml.log);
    for (size_t i = 0; i < nseq; i++) {
        const uint32_t llc = F.ll.t[sll].symbol, ofc = F.of.t[sof].symbol, mlc = F.ml.t[sml].symbol;
        if (llc > 35 || mlc > 52 || ofc > 31) throw Fail{};
        const uint64_t ofv = (1ull << ofc) + br.read((int)ofc);
        const uint64_t ml = kMLBase[mlc] + br.read(kMLBits[mlc]);
        const uint64_t ll = kLLBase[llc] + br.read(kLLBits[llc]);
        uint64_t off;
        if (ofv > 3) {
            off = ofv - 3;
            F.rep[2] = F.rep[1];
            F.rep[1] = F.rep[0];
            F.rep[0] = (uint32_t)off;
        } else {
            const uint32_t idx = (uint32_t)ofv + (ll == 0 ? 1u : 0u);  // 1..4
            if (idx == 1) {
                off = F.rep[0];
            } else if (idx == 2) {
                off = F.rep[1];
                F.rep[1] = F.rep[0];
                F.rep[0] = (uint32_t)off;
            } else {
                off = idx == 3 ? F.rep[2] : (uint64_t)F.rep[0] - 1;
                if (off == 0) throw Fail{};
                F.rep[2] = F.rep[1];
                F.rep[1] = F.rep[0];
                F.rep[0] = (uint32_t)off;
            }
        }
        // execute: literals, then the match
        if (lp + ll > lit.size()) throw Fail{};
        out.insert(out.end(), lit.begin() + lp, lit.begin() + lp + ll);
        lp += ll;
        const size_t produced = out.size() - F.frame_start;
        if (off > produced || off > F.window) throw Fail{};
        size_t from = out.size() - off;
        out.resize(out.size() + ml);
        uint8_t *o = out.data() + out.size() - ml;
        const uint8_t *q = out.data() + from;
        if (off >= ml) {
            std::memcpy(o, q, ml);
        } else {
            for (uint64_t j = 0; j < ml; j++) o[j] = q[j];  // overlapping: byte order matters
        }
        if (i + 1 < nseq) {
            sll = F.ll.t[sll].base + (uint32_t)br.read(F.ll.t[sll].nbits);
            sml = F.ml.t[sml].base + (uint32_t)br.read(F.ml.t[sml].nbits);
            sof = F.of.t[sof].base + (uint32_t)br.read(F.of.t[sof].nbits);
        }
        if (br.overflow()) throw Fail{};
    }
    if (br.pos != 0) throw Fail{};
    out.insert(out.end(), lit.begin() + lp, lit.end());
}

void decode_frames(const uint8_t *in, size_t len, std::vector<uint8_t> &out) {
    size_t p = 0;
    if (len == 0) throw Fail{};
    while (p < len) {
        if (len - p < 4) throw Fail{};
        const uint32_t magic = ld32(in + p);
        if ((magic & 0xfffffff0u) == 0x184d2a50u) {  // skippable frame
            if (len - p < 8) throw Fail{};
            const uint32_t sz = ld32(in + p + 4);
            if (len - p - 8 < sz) throw Fail{};
            p += 8 + (size_t)sz;
            continue;
        }
        if (magic != 0xfd2fb528u) throw Fail{};
        p += 4;
        if (p >= len) throw Fail{};
        const uint8_t fhd = in[p++];
        const int fcs_flag = fhd >> 6, single = (fhd >> 5) & 1, checksum = (fhd >> 2) & 1, did_flag = fhd & 3;
        if (fhd & 0x08) throw Fail{};  // reserved bit
        FrameState F;
        F.frame_start = out.size();
        uint64_t window = 0;
        if (!single) {
            if (p >= len) throw Fail{};
            const uint8_t wd = in[p++];
            const uint64_t wlog = 10 + (wd >> 3);
            const uint64_t base = 1ull << wlog;
            window = base + (base / 8) * (wd & 7);
        }
        const int did_size = did_flag == 0 ? 0 : did_flag == 1 ? 1 : did_flag == 2 ? 2 : 4;
        if (len - p < (size_t)did_size) throw Fail{};
        uint32_t did = 0;
        for (int i = 0; i < did_size; i++) did |= (uint32_t)in[p + i] << (8 * i);
        p += did_size;
        if (did != 0) throw Fail{};  // no dictionary available
        const int fcs_size = fcs_flag == 0 ? (single ? 1 : 0) : fcs_flag == 1 ? 2 : fcs_flag == 2 ? 4 : 8;
        if (len - p < (size_t)fcs_size) throw Fail{};
        uint64_t fcs = 0;
        for (int i = 0; i < fcs_size; i++) fcs |= (uint64_t)in[p + i] << (8 * i);
        if (fcs_size == 2) fcs += 256;
        p += fcs_size;
        // room for the declared content (bounded: the field is untrusted)
        if (fcs_size) {
            const uint64_t cap = 64ull * len + (1ull << 20);
            out.reserve(out.size() + (size_t)(fcs < cap ? fcs : cap));
        }
        if (single) window = fcs;
        if (!single && window > (1ull << 27)) throw Fail{};  // libzstd's default window limit
        F.window = window ? window : 1;
        const uint64_t block_max = window < (128u << 10) ? window : (128u << 10);
        for (;;) {
            if (len - p < 3) throw Fail{};
            const uint32_t bh = in[p] | (in[p + 1] << 8) | (in[p + 2] << 16);
            p += 3;
            const bool last = bh & 1;
            const int btype = (bh >> 1) & 3;
            const size_t bsize = bh >> 3;
            if (btype == 3) throw Fail{};
            if (btype == 1) {
                if (p >= len) throw Fail{};
                out.insert(out.end(), bsize, in[p]);
                p += 1;
            } else {
                if (len - p < bsize) throw Fail{};
                if (btype == 0) {
                    out.insert(out.end(), in + p, in + p + bsize);
                } else {
                    if (bsize > block_max && block_max) throw Fail{};
                    const size_t before = out.size();
                    decode_block(F, in + p, bsize, out);
                    if (out.size() - before > (128u << 10)) throw Fail{};
                }
                p += bsize;
            }
            if (last) break;
        }
        if (fcs_size && out.size() - F.frame_start != fcs) throw Fail{};
        if (checksum) {
            if (len - p < 4) throw Fail{};
            const uint32_t want = ld32(in + p);
            p += 4;
            const uint64_t h = xxh64(out.data() + F.frame_start, out.size() - F.frame_start, 0);
            if ((uint32_t)h != want) throw Fail{};
        }
    }
}

}  // namespace

namespace hh {
// zstd::decode_all: every frame of the stream, concatenated.  Returns false
// on a malformed stream.
bool zstd_decode_all(const uint8_t *in, size_t len, std::vector<uint8_t> &out) {
    out.clear();
    try {
        decode_frames(in, len, out);
        return true;
    } catch (const Fail &) {
        out.clear();
        return false;
    }
}
}  // namespace hh

extern "C" {

int32_t hh_zstd_decompress(const uint8_t *in, size_t in_len, uint8_t *out, size_t out_cap, size_t *written) {
    if ((!in && in_len) || !written) return HH_ERR_INVALID_ARGUMENT;
    std::vector<uint8_t> v;
    if (!hh::zstd_decode_all(in, in_len, v)) {
        *written = 0;
        return HH_ERR_CORRUPTED_DATA;
    }
    *written = v.size();
    if (v.size() > out_cap) return HH_ERR_BUFFER_TOO_SMALL;
    if (!v.empty()) std::memcpy(out, v.data(), v.size());
    return HH_OK;
}

uint64_t hh_xxh64(const uint8_t *data, size_t len, uint64_t seed) { return xxh64(data, len, seed); }

}  // extern "C"
