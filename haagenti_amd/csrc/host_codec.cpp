// Host-side producer (Compressor side of the Codec boundary): the LZ4 block
// compressor, the INT4 quantizer and the HCT-T tile encoder.  These make the
// inputs the GPU decoder consumes; they are not on the timed path.
//
//   LZ4      crates/haagenti-lz4/src/block.rs:73-147 (byte-identical output)
//   INT4     crates/haagenti/src/testing/quantization.rs:30-70, 136-163
//   HCT-T    per 64x64 tile: dct_2d (haagenti-core/src/dct.rs:282-308),
//            top-k by |c| with a stable order (compressive.rs:144-172),
//            quantize_int4 of the kept values in ascending index order.
//
// The tile DCT is the reference's f32 computation: dct_1d's Makhoul form
// (dct.rs:79-129; an n-point complex FFT of the even/odd-reordered input,
// then a quarter-wave twiddle) over the rows, then over the columns
// (dct_2d, dct.rs:282-308).  The 64-point FFT is an iterative radix-2
// decimation in time whose twiddles are cos/sin of the f64 angle rounded to
// f32 (rustfft's twiddle tables are made the same way); host code built
// without FMA contraction, so the coefficient bits, and with them the top-k
// selection, are fixed by this order of operations.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/haagenti_hip.h"

namespace {

// ------------------------------------------------------------------ LZ4

constexpr size_t kMinMatch = 4, kLastLiterals = 5, kMinInput = 13;
constexpr uint32_t kHashBits = 16;

inline uint32_t load32(const uint8_t *p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;  // little-endian host
}

inline uint32_t hash4(uint32_t v) { return (v * 2654435761u) >> (32 - kHashBits); }

class Lz4Writer {
  public:
    Lz4Writer(uint8_t *out, size_t cap) : out_(out), cap_(cap) {}
    size_t pos() const { return pos_; }
    size_t failed_need() const { return need_; }

    // One sequence; match_len == 0 means the final literal-only sequence.
    bool put(const uint8_t *lit, size_t ll, uint16_t offset, size_t match_len) {
        const size_t mx = match_len ? match_len - kMinMatch : 0;
        const size_t need = match_len ? 1 + ll / 255 + 1 + ll + 2 + mx / 255 + 1
                                      : 1 + ll / 255 + 1 + ll;
        if (pos_ + need > cap_) {
            need_ = pos_ + need;
            return false;
        }
        out_[pos_++] = (uint8_t)((std::min<size_t>(ll, 15) << 4) | (match_len ? std::min<size_t>(mx, 15) : 0));
        if (ll >= 15) put_len(ll - 15);
        std::memcpy(out_ + pos_, lit, ll);
        pos_ += ll;
        if (match_len) {
            out_[pos_++] = (uint8_t)offset;
            out_[pos_++] = (uint8_t)(offset >> 8);
            if (mx >= 15) put_len(mx - 15);
        }
        return true;
    }

  private:
    void put_len(size_t rem) {
        for (; rem >= 255; rem -= 255) out_[pos_++] = 255;
        out_[pos_++] = (uint8_t)rem;
    }
    uint8_t *out_;
    size_t cap_, pos_ = 0, need_ = 0;
};

int32_t lz4_compress(const uint8_t *in, size_t n, uint8_t *out, size_t cap, size_t *written) {
    Lz4Writer w(out, cap);
    auto finish = [&](bool ok) -> int32_t {
        if (written) *written = ok ? w.pos() : w.failed_need();
        return ok ? HH_OK : HH_ERR_BUFFER_TOO_SMALL;
    };
    if (n < kMinInput) return finish(w.put(in, n, 0, 0));
    // Positions are stored +1 so that zero means "empty"; the reference's
    // table stores raw positions and rejects match_pos == 0, which is the
    // same as never matching position 0.
    std::vector<uint32_t> table(size_t(1) << kHashBits, 0);
    const size_t match_limit = n - kLastLiterals;
    const size_t mf_limit = match_limit >= kMinMatch ? match_limit - kMinMatch : 0;
    size_t ip = 0, anchor = 0;
    while (ip < mf_limit) {
        const uint32_t cur = load32(in + ip);
        uint32_t &slot = table[hash4(cur)];
        const size_t cand = slot;  // position + 1, 0 = none
        slot = (uint32_t)(ip + 1);
        if (cand > 1) {
            const size_t mp = cand - 1;
            if (ip - mp <= 65535 && load32(in + mp) == cur) {
                size_t a = mp + kMinMatch, b = ip + kMinMatch;
                while (b < match_limit && in[a] == in[b]) {
                    a++;
                    b++;
                }
                const size_t ml = b - ip;
                if (!w.put(in + anchor, ip - anchor, (uint16_t)(ip - mp), ml)) return finish(false);
                ip += ml;
                anchor = ip;
                if (ip < mf_limit) table[hash4(load32(in + ip - 2))] = (uint32_t)(ip - 2 + 1);
                continue;
            }
        }
        ip++;
    }
    if (n > anchor && !w.put(in + anchor, n - anchor, 0, 0)) return finish(false);
    return finish(true);
}

// ------------------------------------------------------------------ INT4

uint16_t f32_to_f16_trunc(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int exp = (int)((b >> 23) & 0xffu);
    const uint32_t frac = b & 0x7fffffu;
    if (exp == 0) return (uint16_t)sign;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (frac >> 13));
    const int e16 = exp - 112;
    if (e16 >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e16 <= 0) return (uint16_t)sign;
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | (frac >> 13));
}

// Rust `(x).round() as i8` then clamp(-8, 7): half away from zero,
// saturating, NaN -> 0.
inline int quant_nibble(float x) {
    if (x != x) return 8;
    float r = std::round(x);
    int q = r >= 127.f ? 127 : (r <= -128.f ? -128 : (int)r);
    q = q < -8 ? -8 : (q > 7 ? 7 : q);
    return q + 8;
}

size_t quantize(const float *w, size_t n, uint8_t *out) {
    if (n == 0) return 0;
    const size_t groups = (n + 31) / 32;
    uint8_t *packed = out + 2 * groups;
    std::memset(packed, 0, (n + 1) / 2);
    for (size_t g = 0; g < groups; g++) {
        const size_t s = g * 32, e = std::min(n, s + 32);
        float mx = 0.f;
        for (size_t i = s; i < e; i++) mx = std::fmax(mx, std::fabs(w[i]));
        const float scale = mx > 1e-10f ? mx / 7.0f : 1.0f;
        const uint16_t h = f32_to_f16_trunc(scale);
        out[2 * g] = (uint8_t)h;
        out[2 * g + 1] = (uint8_t)(h >> 8);
        for (size_t i = s; i < e; i++) {
            const int nib = quant_nibble(w[i] / scale);
            packed[i >> 1] |= (uint8_t)(nib << ((i & 1) * 4));
        }
    }
    return 2 * groups + (n + 1) / 2;
}

// ------------------------------------------------------------------ HCT-T

// 64-point forward DCT-II (orthonormal) in f32, Makhoul's method.
class TileDct {
  public:
    TileDct() {
        for (int i = 0, j = 0; i < 64; i++) {  // bit-reversal permutation
            rev_[i] = (uint8_t)j;
            int bit = 32;
            for (; j & bit; bit >>= 1) j ^= bit;
            j ^= bit;
        }
        for (int k = 0; k <= 32; k++) {
            const double a = -2.0 * 3.14159265358979323846 * (double)k / 64.0;
            wr_[k] = (float)std::cos(a);
            wi_[k] = (float)std::sin(a);
        }
        const float pi = 3.14159265358979323846f;
        for (int k = 0; k < 64; k++) {
            const float angle = -pi * (float)k / (2.0f * 64.0f);
            cr_[k] = std::cos(angle);
            ci_[k] = std::sin(angle);
        }
        scale_ = std::sqrt(2.0f / 64.0f);
    }

    // out[k] = a_k sum_i in[i * stride] cos(pi k (2i + 1) / 128)
    void operator()(const float *in, size_t stride, float *out) const {
        float re[64], im[64], xr[64];
        // v = [x0, x2, ..., x62, x63, x61, ..., x1]
        for (int k = 0; k < 32; k++) {
            xr[k] = in[(size_t)(2 * k) * stride];
            xr[63 - k] = in[(size_t)(2 * k + 1) * stride];
        }
        for (int i = 0; i < 64; i++) {
            re[rev_[i]] = xr[i];
            im[rev_[i]] = 0.0f;
        }
        for (int len = 2, step = 32; len <= 64; len <<= 1, step >>= 1) {
            const int half = len >> 1;
            for (int i = 0; i < 64; i += len)
                for (int k = 0; k < half; k++) {
                    const float w_r = wr_[k * step], w_i = wi_[k * step];
                    const int a = i + k, b = i + k + half;
                    const float br = re[b] * w_r - im[b] * w_i;
                    const float bi = re[b] * w_i + im[b] * w_r;
                    const float ar = re[a], ai = im[a];
                    re[a] = ar + br;
                    im[a] = ai + bi;
                    re[b] = ar - br;
                    im[b] = ai - bi;
                }
        }
        for (int k = 0; k < 64; k++) out[k] = (re[k] * cr_[k] - im[k] * ci_[k]) * scale_;
        out[0] /= 1.41421356237309504880f;
    }

  private:
    uint8_t rev_[64];
    float wr_[33], wi_[33], cr_[64], ci_[64];
    float scale_;
};

const TileDct &tile_dct() {
    static const TileDct d;
    return d;
}

void encode_tile(const float *w, size_t ld, uint32_t k, uint8_t *out) {
    const TileDct &dct = tile_dct();
    float t[4096], c[4096];
    for (int i = 0; i < 64; i++) dct(w + (size_t)i * ld, 1, t + 64 * i);  // rows
    float col[64];
    for (int v = 0; v < 64; v++) {  // then columns
        dct(t + v, 64, col);
        for (int u = 0; u < 64; u++) c[64 * u + v] = col[u];
    }
    float mag[4096];
    for (int i = 0; i < 4096; i++) {
        const float a = std::fabs(c[i]);
        mag[i] = a != a ? -1.0f : a;  // NaN ranks last
    }
    // Stable descending order by magnitude: the k-th largest value is the
    // threshold; ties at the threshold go to the lowest indices.
    std::vector<float> sorted(mag, mag + 4096);
    std::nth_element(sorted.begin(), sorted.begin() + (k - 1), sorted.end(), std::greater<float>());
    const float thr = sorted[k - 1];
    uint32_t above = 0;
    for (int i = 0; i < 4096; i++) above += mag[i] > thr;
    uint32_t ties_left = k - above;
    uint8_t *bitmap = out;
    std::memset(bitmap, 0, 512);
    float vals[4096];
    uint32_t nv = 0;
    for (int i = 0; i < 4096; i++) {
        bool keep = mag[i] > thr;
        if (!keep && mag[i] == thr && ties_left) {
            keep = true;
            ties_left--;
        }
        if (keep) {
            bitmap[i >> 3] |= (uint8_t)(1u << (i & 7));
            vals[nv++] = c[i];
        }
    }
    quantize(vals, nv, out + 512);
}

}  // namespace

extern "C" {

size_t hh_lz4_max_compressed_size(size_t n) { return n + n / 255 + 16; }

int32_t hh_lz4_compress_block(const uint8_t *in, size_t in_len, uint8_t *out, size_t out_cap,
                              size_t *written) {
    if ((!in && in_len) || (!out && out_cap)) return HH_ERR_INVALID_ARGUMENT;
    if (in_len >= 0xffffffffu) return HH_ERR_UNSUPPORTED;
    return lz4_compress(in, in_len, out, out_cap, written);
}

size_t hh_int4_compressed_size(size_t n) { return n ? 2 * ((n + 31) / 32) + (n + 1) / 2 : 0; }

size_t hh_quantize_int4(const float *w, size_t n, uint8_t *out) {
    if (!w || !out) return 0;
    return quantize(w, n, out);
}

size_t hh_hctt_tile_bytes(uint32_t k) { return 512 + hh_int4_compressed_size(k); }

uint32_t hh_hctt_retain_count(float rho) {
    float r = rho != rho ? 0.05f : std::min(1.0f, std::max(0.05f, rho));
    const uint32_t k = (uint32_t)(4096.0f * r);
    return k < 1 ? 1 : k;
}

int32_t hh_hctt_encode(const float *w, uint32_t rows, uint32_t cols, uint32_t k, uint8_t *out,
                       int32_t threads) {
    if (!w || !out || rows % 64 || cols % 64 || k < 1 || k > 4096) return HH_ERR_INVALID_ARGUMENT;
    const size_t tpr = cols / 64, ntiles = (size_t)(rows / 64) * tpr;
    const size_t tb = hh_hctt_tile_bytes(k);
    unsigned nt = threads > 0 ? (unsigned)threads : std::max(1u, std::thread::hardware_concurrency());
    if (nt > ntiles) nt = (unsigned)std::max<size_t>(1, ntiles);
    std::atomic<size_t> next{0};
    auto work = [&]() {
        for (;;) {
            const size_t t = next.fetch_add(1);
            if (t >= ntiles) break;
            const size_t tr = t / tpr, tc = t % tpr;
            encode_tile(w + (tr * 64) * (size_t)cols + tc * 64, cols, k, out + t * tb);
        }
    };
    std::vector<std::thread> pool;
    for (unsigned i = 1; i < nt; i++) pool.emplace_back(work);
    work();
    for (auto &th : pool) th.join();
    return HH_OK;
}

}  // extern "C"
