/*
 * hh_oracle.c -- CPU restatement of the reference HCT decode path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load this library; the product never does.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so that a*b+c is not fused,
 * matching the reference's Rust float semantics; no -ffast-math).
 *
 * Citations are file:line in the reference repository.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   LZ4 compress/decompress  hand-derived byte vectors, hand-written streams
 *                            for every branch and error, round trips on the
 *                            reference's own test inputs (block.rs:379-450).
 *   INT4 + f16 helpers       hand-computed known answers (truncating scale,
 *                            half-away rounding), numpy's float16 decoder over
 *                            all 65,536 codes, brute force over 256 bytes.
 *   DCT / IDCT               spec known answers (sequential_4x4, constant_4x4),
 *                            f64 closed form, orthogonality, round trip, and
 *                            the reference's own C decoder (oracle/_ref).
 *   top-k / bitmap           brute force over small inputs, spec retained
 *                            indices, popcount == k.
 *   HCT-T tile decode        oracle/_ref hct_decode on the same bitmap +
 *                            coefficients, f64 truth within tolerance.
 *   HCT container            byte layout asserted by the reference's tests
 *                            (tensor.rs:1056-1091,1637-1722,2088-2207).
 *   XXH3-64                  the xxhash library's xxh3_64 on every length
 *                            0..2048 and longer random inputs (python
 *                            xxhash, tests/test_oracle_xxh3.py).
 *   HCT v2 container         the reference's v2 tests (tensor.rs:1250-1440,
 *                            1943-2060): round trips, corruption detection,
 *                            quantization metadata, v1 compatibility.
 */
#define _GNU_SOURCE
#include "hh_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define HHO_PI_F 3.14159265358979323846f
#define HHO_SQRT2_F 1.41421356237309504880f

/* ===================================================================== */
/* Small thread pool helper: run fn(i) for i in [0, n) on nthreads.      */
/* Mirrors the rayon par_iter fan-out of pipeline/turbo.rs:236-261.      */
/* ===================================================================== */

typedef void (*hho_task_fn)(void *ctx, size_t i);

typedef struct {
    hho_task_fn fn;
    void *ctx;
    size_t n;
    size_t next;
    pthread_mutex_t mu;
} hho_pool;

static void *hho_worker(void *arg) {
    hho_pool *p = (hho_pool *)arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        size_t i = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (i >= p->n) break;
        p->fn(p->ctx, i);
    }
    return NULL;
}

static int hho_resolve_threads(int nthreads) {
    if (nthreads > 0) return nthreads;
    long c = sysconf(_SC_NPROCESSORS_ONLN);
    return c > 0 ? (int)c : 1;
}

static void hho_parallel_for(size_t n, int nthreads, hho_task_fn fn, void *ctx) {
    int t = hho_resolve_threads(nthreads);
    if (t <= 1 || n <= 1) {
        for (size_t i = 0; i < n; i++) fn(ctx, i);
        return;
    }
    if ((size_t)t > n) t = (int)n;
    hho_pool p;
    p.fn = fn;
    p.ctx = ctx;
    p.n = n;
    p.next = 0;
    pthread_mutex_init(&p.mu, NULL);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)t);
    for (int i = 0; i < t; i++) pthread_create(&th[i], NULL, hho_worker, &p);
    for (int i = 0; i < t; i++) pthread_join(th[i], NULL);
    free(th);
    pthread_mutex_destroy(&p.mu);
}

static void set_err(hho_err *e, int kind, int sub, uint64_t pos, uint64_t req,
                    uint64_t prov) {
    if (!e) return;
    e->kind = kind;
    e->sub = sub;
    e->position = pos;
    e->required = req;
    e->provided = prov;
}

/* ===================================================================== */
/* LZ4 raw block -- crates/haagenti-lz4/src/block.rs                      */
/* ===================================================================== */

#define LZ4_MIN_MATCH 4u        /* block.rs:15 */
#define LZ4_HASH_SIZE (1u << 16) /* block.rs:21 */
#define LZ4_LAST_LITERALS 5u    /* block.rs:27 */
#define LZ4_MIN_INPUT 13u       /* block.rs:30 */

static inline uint32_t rd_u32le(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}

/* block.rs:33-37: (v * 2654435761 wrapping) >> 16, masked to 16 bits. */
static inline size_t lz4_hash(uint32_t v) {
    return (size_t)((uint32_t)(v * 2654435761u) >> 16) & (LZ4_HASH_SIZE - 1);
}

size_t hho_lz4_max_compressed_size(size_t n) { return n + n / 255 + 16; }

/* block.rs:212-251 */
static int lz4_write_last_literals(const uint8_t *in, uint8_t *out, size_t cap,
                                   size_t *pos, size_t lit_start,
                                   size_t lit_len, hho_err *err) {
    size_t p = *pos;
    size_t ll_tok = lit_len < 15 ? lit_len : 15;
    size_t needed = 1 + lit_len / 255 + 1 + lit_len;
    if (p + needed > cap) {
        set_err(err, HHO_BUFFER_TOO_SMALL, 0, 0, p + needed, cap);
        return HHO_BUFFER_TOO_SMALL;
    }
    out[p++] = (uint8_t)(ll_tok << 4);
    if (lit_len >= 15) {
        size_t rem = lit_len - 15;
        while (rem >= 255) {
            out[p++] = 255;
            rem -= 255;
        }
        out[p++] = (uint8_t)rem;
    }
    memcpy(out + p, in + lit_start, lit_len);
    p += lit_len;
    *pos = p;
    return HHO_OK;
}

/* block.rs:150-209 */
static int lz4_write_sequence(const uint8_t *in, uint8_t *out, size_t cap,
                              size_t *pos, size_t lit_start, size_t lit_len,
                              uint16_t offset, size_t match_len, hho_err *err) {
    size_t p = *pos;
    size_t ll_tok = lit_len < 15 ? lit_len : 15;
    size_t mlx = match_len - LZ4_MIN_MATCH;
    size_t ml_tok = mlx < 15 ? mlx : 15;
    size_t needed = 1 + lit_len / 255 + 1 + lit_len + 2 + mlx / 255 + 1;
    if (p + needed > cap) {
        set_err(err, HHO_BUFFER_TOO_SMALL, 0, 0, p + needed, cap);
        return HHO_BUFFER_TOO_SMALL;
    }
    out[p++] = (uint8_t)((ll_tok << 4) | ml_tok);
    if (lit_len >= 15) {
        size_t rem = lit_len - 15;
        while (rem >= 255) {
            out[p++] = 255;
            rem -= 255;
        }
        out[p++] = (uint8_t)rem;
    }
    memcpy(out + p, in + lit_start, lit_len);
    p += lit_len;
    out[p++] = (uint8_t)(offset & 0xff);
    out[p++] = (uint8_t)(offset >> 8);
    if (mlx >= 15) {
        size_t rem = mlx - 15;
        while (rem >= 255) {
            out[p++] = 255;
            rem -= 255;
        }
        out[p++] = (uint8_t)rem;
    }
    *pos = p;
    return HHO_OK;
}

/* block.rs:73-147 */
int hho_lz4_compress_block(const uint8_t *in, size_t n, uint8_t *out,
                           size_t cap, size_t *written, hho_err *err) {
    size_t op = 0;
    set_err(err, HHO_OK, 0, 0, 0, 0);
    if (n < LZ4_MIN_INPUT) { /* compress_literals_only, :253-256 */
        int rc = lz4_write_last_literals(in, out, cap, &op, 0, n, err);
        if (rc == HHO_OK && written) *written = op;
        return rc;
    }
    size_t *table = (size_t *)calloc(LZ4_HASH_SIZE, sizeof(size_t));
    size_t ip = 0, anchor = 0;
    size_t match_limit = n >= LZ4_LAST_LITERALS ? n - LZ4_LAST_LITERALS : 0;
    size_t mf_limit = match_limit >= LZ4_MIN_MATCH ? match_limit - LZ4_MIN_MATCH : 0;
    int rc = HHO_OK;
    while (ip < mf_limit) {
        size_t h = lz4_hash(rd_u32le(in + ip));
        size_t mp = table[h];
        table[h] = ip;
        if (mp > 0 && ip - mp <= 65535 && rd_u32le(in + mp) == rd_u32le(in + ip)) {
            /* count_match, :61-68 */
            size_t p1 = mp + LZ4_MIN_MATCH, p2 = ip + LZ4_MIN_MATCH, s = p2;
            while (p2 < match_limit && in[p1] == in[p2]) {
                p1++;
                p2++;
            }
            size_t ml = LZ4_MIN_MATCH + (p2 - s);
            size_t ll = ip - anchor;
            uint16_t off = (uint16_t)(ip - mp);
            rc = lz4_write_sequence(in, out, cap, &op, anchor, ll, off, ml, err);
            if (rc != HHO_OK) break;
            ip += ml;
            anchor = ip;
            if (ip < mf_limit) table[lz4_hash(rd_u32le(in + ip - 2))] = ip - 2;
        } else {
            ip += 1; /* ACCELERATION, :24 */
        }
    }
    free(table);
    if (rc != HHO_OK) return rc;
    size_t ll = n - anchor;
    if (ll > 0) {
        rc = lz4_write_last_literals(in, out, cap, &op, anchor, ll, err);
        if (rc != HHO_OK) return rc;
    }
    if (written) *written = op;
    return HHO_OK;
}

/* block.rs:261-366 */
int hho_lz4_decompress_block(const uint8_t *in, size_t in_len, uint8_t *out,
                             size_t out_len, size_t output_size,
                             size_t *written, hho_err *err) {
    size_t ip = 0, op = 0;
    set_err(err, HHO_OK, 0, 0, 0, 0);
    while (ip < in_len) {
        uint8_t token = in[ip++];
        size_t ll = token >> 4;
        size_t ml = token & 0x0f;
        if (ll == 15) {
            for (;;) {
                if (ip >= in_len) {
                    set_err(err, HHO_UNEXPECTED_EOF, 0, ip, 0, 0);
                    return HHO_UNEXPECTED_EOF;
                }
                uint8_t b = in[ip++];
                ll += b;
                if (b != 255) break;
            }
        }
        if (ll > 0) {
            if (ip + ll > in_len) {
                set_err(err, HHO_UNEXPECTED_EOF, 0, ip, 0, 0);
                return HHO_UNEXPECTED_EOF;
            }
            if (op + ll > out_len) {
                set_err(err, HHO_BUFFER_TOO_SMALL, 0, 0, op + ll, out_len);
                return HHO_BUFFER_TOO_SMALL;
            }
            memcpy(out + op, in + ip, ll);
            ip += ll;
            op += ll;
        }
        if (op >= output_size) break; /* :309-311 */
        if (ip + 2 > in_len) {
            set_err(err, HHO_UNEXPECTED_EOF, 0, ip, 0, 0);
            return HHO_UNEXPECTED_EOF;
        }
        size_t off = (size_t)in[ip] | ((size_t)in[ip + 1] << 8);
        ip += 2;
        if (off == 0) {
            set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_ZERO_OFFSET, 0, 0, 0);
            return HHO_CORRUPTED_DATA;
        }
        if (off > op) {
            set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_OFFSET_BEYOND, op, 0, 0);
            return HHO_CORRUPTED_DATA;
        }
        ml += LZ4_MIN_MATCH;
        if ((token & 0x0f) == 15) {
            for (;;) {
                if (ip >= in_len) {
                    set_err(err, HHO_UNEXPECTED_EOF, 0, ip, 0, 0);
                    return HHO_UNEXPECTED_EOF;
                }
                uint8_t b = in[ip++];
                ml += b;
                if (b != 255) break;
            }
        }
        size_t ms = op - off;
        if (op + ml > out_len) {
            set_err(err, HHO_BUFFER_TOO_SMALL, 0, 0, op + ml, out_len);
            return HHO_BUFFER_TOO_SMALL;
        }
        if (off >= ml) {
            memmove(out + op, out + ms, ml);
        } else {
            for (size_t i = 0; i < ml; i++) out[op + i] = out[ms + i];
        }
        op += ml;
    }
    if (written) *written = op;
    return HHO_OK;
}

typedef struct {
    const uint8_t *in;
    const uint64_t *in_off;
    const uint32_t *in_len;
    uint8_t *out;
    const uint64_t *out_off;
    const uint32_t *out_cap;
    int32_t *kinds;
    uint64_t *written;
} lz4_batch_ctx;

static void lz4_batch_task(void *vctx, size_t i) {
    lz4_batch_ctx *c = (lz4_batch_ctx *)vctx;
    size_t w = 0;
    hho_err e;
    int rc = hho_lz4_decompress_block(c->in + c->in_off[i], c->in_len[i],
                                      c->out + c->out_off[i], c->out_cap[i],
                                      c->out_cap[i], &w, &e);
    if (c->kinds) c->kinds[i] = rc;
    if (c->written) c->written[i] = rc == HHO_OK ? w : 0;
}

void hho_lz4_decompress_batch(const uint8_t *in, const uint64_t *in_off,
                              const uint32_t *in_len, uint8_t *out,
                              const uint64_t *out_off, const uint32_t *out_cap,
                              size_t nblocks, int32_t *kinds, uint64_t *written,
                              int nthreads) {
    lz4_batch_ctx c = {in, in_off, in_len, out, out_off, out_cap, kinds, written};
    hho_parallel_for(nblocks, nthreads, lz4_batch_task, &c);
}

/* ===================================================================== */
/* INT4 -- crates/haagenti/src/testing/quantization.rs                    */
/* ===================================================================== */

#define Q4_BLOCK 32u /* :10 */

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* :136-163 -- truncating conversion, subnormals flushed to signed zero. */
uint16_t hho_f32_to_f16_bits(float v) {
    uint32_t bits = f2u(v);
    uint32_t sign = (bits >> 31) & 1u;
    int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    uint32_t frac = bits & 0x7fffffu;
    if (exp == 0) return (uint16_t)(sign << 15);
    if (exp == 0xff) return (uint16_t)((sign << 15) | (0x1fu << 10) | (frac >> 13));
    int32_t ne = exp - 127 + 15;
    if (ne >= 31) return (uint16_t)((sign << 15) | (0x1fu << 10));
    if (ne <= 0) return (uint16_t)(sign << 15);
    return (uint16_t)((sign << 15) | ((uint32_t)ne << 10) | (frac >> 13));
}

/* :166-197 -- exact, NaN payload kept as frac << 13. */
float hho_f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t frac = h & 0x3ffu;
    if (exp == 0) {
        if (frac == 0) return u2f(sign << 31);
        int32_t e = -14;
        uint32_t f = frac;
        while ((f & 0x400u) == 0) {
            f <<= 1;
            e -= 1;
        }
        f &= 0x3ffu;
        uint32_t ne = (uint32_t)(e + 127) & 0xffu;
        return u2f((sign << 31) | (ne << 23) | (f << 13));
    }
    if (exp == 31) return u2f((sign << 31) | (0xffu << 23) | (frac << 13));
    uint32_t ne = (uint32_t)((int32_t)exp - 15 + 127);
    return u2f((sign << 31) | (ne << 23) | (frac << 13));
}

void hho_f16_bits_to_f32_bits(const uint16_t *h, size_t n, uint32_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = f2u(hho_f16_bits_to_f32(h[i]));
}

size_t hho_int4_compressed_size(size_t n) {
    if (n == 0) return 0;
    size_t nb = (n + Q4_BLOCK - 1) / Q4_BLOCK;
    return nb * 2 + (n + 1) / 2;
}

/* Rust `x as i8`: saturating, NaN -> 0. */
static inline int8_t sat_i8(float x) {
    if (x != x) return 0;
    if (x >= 127.0f) return 127;
    if (x <= -128.0f) return -128;
    return (int8_t)x;
}

/* :30-70 */
size_t hho_quantize_int4(const float *w, size_t n, uint8_t *out) {
    if (n == 0) return 0;
    size_t nb = (n + Q4_BLOCK - 1) / Q4_BLOCK;
    float *scales = (float *)malloc(nb * sizeof(float));
    size_t p = 0;
    for (size_t b = 0; b < nb; b++) {
        size_t s = b * Q4_BLOCK, e = s + Q4_BLOCK < n ? s + Q4_BLOCK : n;
        float max_abs = 0.0f;
        for (size_t i = s; i < e; i++) max_abs = fmaxf(max_abs, fabsf(w[i]));
        float scale = max_abs > 1e-10f ? max_abs / 7.0f : 1.0f;
        scales[b] = scale;
        uint16_t h = hho_f32_to_f16_bits(scale);
        out[p++] = (uint8_t)(h & 0xff);
        out[p++] = (uint8_t)(h >> 8);
    }
    /* nibbles: low nibble first (:59-67) */
    for (size_t i = 0; i < n; i += 2) {
        float s0 = scales[i / Q4_BLOCK];
        int q0 = sat_i8(roundf(w[i] / s0));
        if (q0 < -8) q0 = -8;
        if (q0 > 7) q0 = 7;
        uint8_t byte = (uint8_t)((q0 + 8) & 0x0f);
        if (i + 1 < n) {
            float s1 = scales[(i + 1) / Q4_BLOCK];
            int q1 = sat_i8(roundf(w[i + 1] / s1));
            if (q1 < -8) q1 = -8;
            if (q1 > 7) q1 = 7;
            byte |= (uint8_t)(((q1 + 8) & 0x0f) << 4);
        }
        out[p++] = byte;
    }
    free(scales);
    return p;
}

/* :82-131 */
size_t hho_dequantize_int4(const uint8_t *data, size_t len, size_t n, float *out) {
    if (n == 0) return 0;
    size_t nb = (n + Q4_BLOCK - 1) / Q4_BLOCK;
    size_t sb = nb * 2;
    if (len < sb) return 0;
    const uint8_t *packed = data + sb;
    size_t plen = len - sb;
    size_t cnt = 0, nib = 0;
    for (size_t b = 0; b < nb; b++) {
        float scale = hho_f16_bits_to_f32((uint16_t)(data[2 * b] | (data[2 * b + 1] << 8)));
        size_t bs = n - b * Q4_BLOCK < Q4_BLOCK ? n - b * Q4_BLOCK : Q4_BLOCK;
        for (size_t j = 0; j < bs; j++) {
            size_t bi = nib / 2;
            if (bi >= plen) break;
            uint8_t v = (nib & 1) ? (uint8_t)((packed[bi] >> 4) & 0x0f) : (uint8_t)(packed[bi] & 0x0f);
            int q = (int)v - 8;
            out[cnt++] = (float)q * scale;
            nib++;
        }
    }
    return cnt;
}

typedef struct {
    const uint8_t *data;
    size_t n, nb, plen;
    float *out;
    size_t groups_per_task;
} dq_ctx;

static void dq_task(void *vctx, size_t t) {
    dq_ctx *c = (dq_ctx *)vctx;
    size_t g0 = t * c->groups_per_task;
    size_t g1 = g0 + c->groups_per_task < c->nb ? g0 + c->groups_per_task : c->nb;
    const uint8_t *packed = c->data + c->nb * 2;
    for (size_t b = g0; b < g1; b++) {
        float scale = hho_f16_bits_to_f32((uint16_t)(c->data[2 * b] | (c->data[2 * b + 1] << 8)));
        size_t s = b * Q4_BLOCK, e = s + Q4_BLOCK < c->n ? s + Q4_BLOCK : c->n;
        for (size_t i = s; i < e; i++) {
            uint8_t v = (i & 1) ? (uint8_t)(packed[i / 2] >> 4) : (uint8_t)(packed[i / 2] & 0x0f);
            c->out[i] = (float)((int)v - 8) * scale;
        }
    }
}

size_t hho_dequantize_int4_mt(const uint8_t *data, size_t len, size_t n,
                              float *out, int nthreads) {
    if (n == 0) return 0;
    size_t nb = (n + Q4_BLOCK - 1) / Q4_BLOCK;
    if (len < nb * 2) return 0;
    size_t plen = len - nb * 2;
    if (plen * 2 < n) return hho_dequantize_int4(data, len, n, out); /* short */
    dq_ctx c = {data, n, nb, plen, out, 4096};
    size_t tasks = (nb + c.groups_per_task - 1) / c.groups_per_task;
    hho_parallel_for(tasks, nthreads, dq_task, &c);
    return n;
}

/* ===================================================================== */
/* FFT used by the Makhoul DCT (the reference uses rustfft 6.4.1 here:    */
/* forward X[k] = sum x[n] e^{-2 pi i kn/N}, inverse unnormalised with    */
/* e^{+...}).  Own radix-2 / mixed-radix Cooley-Tukey, twiddles computed  */
/* in f64 and rounded to f32 like rustfft's twiddle tables.               */
/* ===================================================================== */

typedef struct {
    float re, im;
} cf32;

#define HHO_MAX_LOG2 24
static cf32 *g_tw[2][HHO_MAX_LOG2 + 1];
static pthread_mutex_t g_tw_mu = PTHREAD_MUTEX_INITIALIZER;

static const cf32 *twiddles_pow2(int lg, int inverse) {
    cf32 *t = __atomic_load_n(&g_tw[inverse][lg], __ATOMIC_ACQUIRE);
    if (t) return t;
    pthread_mutex_lock(&g_tw_mu);
    t = g_tw[inverse][lg];
    if (!t) {
        size_t n = (size_t)1 << lg;
        t = (cf32 *)malloc(sizeof(cf32) * (n / 2 + 1));
        double sgn = inverse ? 1.0 : -1.0;
        for (size_t k = 0; k < n / 2 + 1; k++) {
            double a = sgn * 2.0 * M_PI * (double)k / (double)n;
            t[k].re = (float)cos(a);
            t[k].im = (float)sin(a);
        }
        __atomic_store_n(&g_tw[inverse][lg], t, __ATOMIC_RELEASE);
    }
    pthread_mutex_unlock(&g_tw_mu);
    return t;
}

static void fft_pow2(cf32 *x, size_t n, int lg, int inverse) {
    /* bit reversal */
    for (size_t i = 1, j = 0; i < n; i++) {
        size_t bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) {
            cf32 t = x[i];
            x[i] = x[j];
            x[j] = t;
        }
    }
    const cf32 *tw = twiddles_pow2(lg, inverse);
    for (size_t len = 2; len <= n; len <<= 1) {
        size_t half = len >> 1, step = n / len;
        for (size_t i = 0; i < n; i += len) {
            for (size_t k = 0; k < half; k++) {
                cf32 w = tw[k * step];
                cf32 a = x[i + k], b = x[i + k + half];
                cf32 bw = {b.re * w.re - b.im * w.im, b.re * w.im + b.im * w.re};
                x[i + k].re = a.re + bw.re;
                x[i + k].im = a.im + bw.im;
                x[i + k + half].re = a.re - bw.re;
                x[i + k + half].im = a.im - bw.im;
            }
        }
    }
}

static size_t smallest_factor(size_t n) {
    if (n % 2 == 0) return 2;
    for (size_t p = 3; p * p <= n; p += 2)
        if (n % p == 0) return p;
    return n;
}

/* Mixed-radix decimation in time for sizes that are not powers of two. */
static void fft_mixed(cf32 *x, size_t n, int inverse) {
    if (n <= 1) return;
    size_t p = smallest_factor(n), m = n / p;
    double sgn = inverse ? 1.0 : -1.0;
    cf32 *y = (cf32 *)malloc(sizeof(cf32) * n);
    if (p == n) { /* prime: direct DFT */
        for (size_t k = 0; k < n; k++) {
            double re = 0, im = 0;
            for (size_t j = 0; j < n; j++) {
                double a = sgn * 2.0 * M_PI * (double)((k * j) % n) / (double)n;
                float wr = (float)cos(a), wi = (float)sin(a);
                re += (double)(x[j].re * wr - x[j].im * wi);
                im += (double)(x[j].re * wi + x[j].im * wr);
            }
            y[k].re = (float)re;
            y[k].im = (float)im;
        }
        memcpy(x, y, sizeof(cf32) * n);
        free(y);
        return;
    }
    for (size_t r = 0; r < p; r++)
        for (size_t j = 0; j < m; j++) y[r * m + j] = x[j * p + r];
    for (size_t r = 0; r < p; r++) fft_mixed(y + r * m, m, inverse);
    for (size_t k = 0; k < m; k++) {
        for (size_t q = 0; q < p; q++) {
            float re = 0.f, im = 0.f;
            for (size_t r = 0; r < p; r++) {
                double a = sgn * 2.0 * M_PI * (double)((r * (k + m * q)) % n) / (double)n;
                float wr = (float)cos(a), wi = (float)sin(a);
                cf32 v = y[r * m + k];
                re += v.re * wr - v.im * wi;
                im += v.re * wi + v.im * wr;
            }
            x[k + m * q].re = re;
            x[k + m * q].im = im;
        }
    }
    free(y);
}

static void fft_any(cf32 *x, size_t n, int inverse) {
    if (n <= 1) return;
    if ((n & (n - 1)) == 0) {
        int lg = 0;
        while (((size_t)1 << lg) < n) lg++;
        if (lg <= HHO_MAX_LOG2) {
            fft_pow2(x, n, lg, inverse);
            return;
        }
    }
    fft_mixed(x, n, inverse);
}

/* ===================================================================== */
/* DCT -- crates/haagenti-core/src/dct.rs                                  */
/* ===================================================================== */

/* :133-146 */
void hho_dct_1d_direct(const float *in, float *out, size_t n) {
    float scale = sqrtf(2.0f / (float)n);
    for (size_t k = 0; k < n; k++) {
        float sum = 0.0f;
        for (size_t i = 0; i < n; i++)
            sum += in[i] * cosf(HHO_PI_F * (float)k * ((float)i + 0.5f) / (float)n);
        out[k] = sum * scale;
    }
    out[0] /= HHO_SQRT2_F;
}

/* :79-129 (Makhoul) */
void hho_dct_1d(const float *in, float *out, size_t n) {
    if (n == 0) return;
    if (n <= 32) {
        hho_dct_1d_direct(in, out, n);
        return;
    }
    cf32 *y = (cf32 *)calloc(n, sizeof(cf32));
    for (size_t k = 0; k < (n + 1) / 2; k++)
        if (2 * k < n) y[k].re = in[2 * k];
    for (size_t k = 0; k < n / 2; k++)
        if (2 * k + 1 < n) y[n - 1 - k].re = in[2 * k + 1];
    fft_any(y, n, 0);
    float scale = sqrtf(2.0f / (float)n);
    for (size_t k = 0; k < n; k++) {
        float angle = -HHO_PI_F * (float)k / (2.0f * (float)n);
        float c = cosf(angle), s = sinf(angle);
        /* (y * twiddle).re = y.re*c - y.im*s */
        float re = y[k].re * c - y[k].im * s;
        out[k] = re * scale;
    }
    out[0] /= HHO_SQRT2_F;
    free(y);
}

/* :263-277 */
void hho_idct_1d_direct(const float *in, float *out, size_t n) {
    float scale = sqrtf(2.0f / (float)n);
    for (size_t i = 0; i < n; i++) {
        float sum = in[0] / HHO_SQRT2_F;
        for (size_t k = 1; k < n; k++)
            sum += in[k] * cosf(HHO_PI_F * (float)k * ((float)i + 0.5f) / (float)n);
        out[i] = sum * scale;
    }
}

/* :154-259 (inverse Makhoul) */
void hho_idct_1d(const float *in, float *out, size_t n) {
    if (n == 0) return;
    if (n <= 32) {
        hho_idct_1d_direct(in, out, n);
        return;
    }
    float scale = sqrtf(2.0f / (float)n);
    float *c = (float *)malloc(sizeof(float) * n);
    c[0] = in[0] * HHO_SQRT2_F / scale;
    for (size_t k = 1; k < n; k++) c[k] = in[k] / scale;
    cf32 *y = (cf32 *)calloc(n, sizeof(cf32));
    y[0].re = c[0];
    if (n % 2 == 0) {
        size_t k = n / 2;
        float angle = -HHO_PI_F * (float)k / (2.0f * (float)n);
        y[k].re = c[k] / cosf(angle);
    }
    size_t limit = (n % 2 == 0) ? n / 2 : (n + 1) / 2;
    for (size_t k = 1; k < limit; k++) {
        float ak = -HHO_PI_F * (float)k / (2.0f * (float)n);
        float ank = -HHO_PI_F * (float)(n - k) / (2.0f * (float)n);
        float cos_k = cosf(ak), sin_k = sinf(ak);
        float cos_nk = cosf(ank), sin_nk = sinf(ank);
        float det = cos_k * sin_nk + sin_k * cos_nk;
        float yr = (c[k] * sin_nk + c[n - k] * sin_k) / det;
        float yi = (c[n - k] * cos_k - c[k] * cos_nk) / det;
        y[k].re = yr;
        y[k].im = yi;
        y[n - k].re = yr;
        y[n - k].im = -yi;
    }
    fft_any(y, n, 1);
    float inv_n = 1.0f / (float)n;
    for (size_t k = 0; k < (n + 1) / 2; k++)
        if (2 * k < n) out[2 * k] = y[k].re * inv_n;
    for (size_t k = 0; k < n / 2; k++)
        if (2 * k + 1 < n) out[2 * k + 1] = y[n - 1 - k].re * inv_n;
    free(y);
    free(c);
}

/* :282-308 rows, then columns */
void hho_dct_2d(const float *in, float *out, size_t width, size_t height) {
    float *tmp = (float *)malloc(sizeof(float) * width * height);
    float *cb = (float *)malloc(sizeof(float) * height);
    float *co = (float *)malloc(sizeof(float) * height);
    for (size_t y = 0; y < height; y++) hho_dct_1d(in + y * width, tmp + y * width, width);
    for (size_t x = 0; x < width; x++) {
        for (size_t y = 0; y < height; y++) cb[y] = tmp[y * width + x];
        hho_dct_1d(cb, co, height);
        for (size_t y = 0; y < height; y++) out[y * width + x] = co[y];
    }
    free(tmp);
    free(cb);
    free(co);
}

/* :311-337 columns first, then rows */
void hho_idct_2d(const float *in, float *out, size_t width, size_t height) {
    float *tmp = (float *)malloc(sizeof(float) * width * height);
    float *cb = (float *)malloc(sizeof(float) * height);
    float *co = (float *)malloc(sizeof(float) * height);
    for (size_t x = 0; x < width; x++) {
        for (size_t y = 0; y < height; y++) cb[y] = in[y * width + x];
        hho_idct_1d(cb, co, height);
        for (size_t y = 0; y < height; y++) tmp[y * width + x] = co[y];
    }
    for (size_t y = 0; y < height; y++) hho_idct_1d(tmp + y * width, out + y * width, width);
    free(tmp);
    free(cb);
    free(co);
}

/* hho_idct_2d on nthreads threads: the same 1-D transforms (columns
 * first, then rows), each independent, so the result is bit-identical. */
typedef struct {
    const float *in;
    float *tmp, *out;
    size_t w, h, nchunk;
    int pass;
} idct2_mt_ctx;

static void idct2_mt_task(void *vctx, size_t c) {
    idct2_mt_ctx *t = (idct2_mt_ctx *)vctx;
    if (t->pass == 0) {
        const size_t x0 = c * t->w / t->nchunk, x1 = (c + 1) * t->w / t->nchunk;
        float *cb = (float *)malloc(sizeof(float) * t->h);
        float *co = (float *)malloc(sizeof(float) * t->h);
        for (size_t x = x0; x < x1; x++) {
            for (size_t y = 0; y < t->h; y++) cb[y] = t->in[y * t->w + x];
            hho_idct_1d(cb, co, t->h);
            for (size_t y = 0; y < t->h; y++) t->tmp[y * t->w + x] = co[y];
        }
        free(cb);
        free(co);
    } else {
        const size_t y0 = c * t->h / t->nchunk, y1 = (c + 1) * t->h / t->nchunk;
        for (size_t y = y0; y < y1; y++) hho_idct_1d(t->tmp + y * t->w, t->out + y * t->w, t->w);
    }
}

void hho_idct_2d_mt(const float *in, float *out, size_t width, size_t height, int nthreads) {
    idct2_mt_ctx t = {in, (float *)malloc(sizeof(float) * width * height), out, width, height, 0, 0};
    t.nchunk = 256;
    t.pass = 0;
    hho_parallel_for(t.nchunk, nthreads, idct2_mt_task, &t);
    t.pass = 1;
    hho_parallel_for(t.nchunk, nthreads, idct2_mt_task, &t);
    free(t.tmp);
}

/* :342-361 */
void hho_dct_1d_f64(const double *in, double *out, size_t n) {
    if (n == 0) return;
    double scale = sqrt(2.0 / (double)n), scale_dc = sqrt(1.0 / (double)n);
    for (size_t k = 0; k < n; k++) {
        double sum = 0.0;
        for (size_t i = 0; i < n; i++) {
            double a = M_PI * (2.0 * (double)i + 1.0) * (double)k / (2.0 * (double)n);
            sum += in[i] * cos(a);
        }
        out[k] = sum * (k == 0 ? scale_dc : scale);
    }
}

/* :364-383 */
void hho_idct_1d_f64(const double *in, double *out, size_t n) {
    if (n == 0) return;
    double scale = sqrt(2.0 / (double)n), scale_dc = sqrt(1.0 / (double)n);
    for (size_t i = 0; i < n; i++) {
        double sum = in[0] * scale_dc;
        for (size_t k = 1; k < n; k++) {
            double a = M_PI * (2.0 * (double)i + 1.0) * (double)k / (2.0 * (double)n);
            sum += in[k] * cos(a) * scale;
        }
        out[i] = sum;
    }
}

/* :386-412 */
void hho_dct_2d_f64(const double *in, double *out, size_t w, size_t h) {
    double *tmp = (double *)malloc(sizeof(double) * w * h);
    double *cb = (double *)malloc(sizeof(double) * h);
    double *co = (double *)malloc(sizeof(double) * h);
    for (size_t y = 0; y < h; y++) hho_dct_1d_f64(in + y * w, tmp + y * w, w);
    for (size_t x = 0; x < w; x++) {
        for (size_t y = 0; y < h; y++) cb[y] = tmp[y * w + x];
        hho_dct_1d_f64(cb, co, h);
        for (size_t y = 0; y < h; y++) out[y * w + x] = co[y];
    }
    free(tmp);
    free(cb);
    free(co);
}

/* :415-441 */
void hho_idct_2d_f64(const double *in, double *out, size_t w, size_t h) {
    double *tmp = (double *)malloc(sizeof(double) * w * h);
    double *cb = (double *)malloc(sizeof(double) * h);
    double *co = (double *)malloc(sizeof(double) * h);
    for (size_t x = 0; x < w; x++) {
        for (size_t y = 0; y < h; y++) cb[y] = in[y * w + x];
        hho_idct_1d_f64(cb, co, h);
        for (size_t y = 0; y < h; y++) tmp[y * w + x] = co[y];
    }
    for (size_t y = 0; y < h; y++) hho_idct_1d_f64(tmp + y * w, out + y * w, w);
    free(tmp);
    free(cb);
    free(co);
}

/* crates/haagenti/src/hct_test_vectors.rs:43-75 */
void hho_reference_dct_2d(const float *in, float *out, size_t rows, size_t cols) {
    for (size_t u = 0; u < rows; u++) {
        for (size_t v = 0; v < cols; v++) {
            float sum = 0.0f;
            for (size_t i = 0; i < rows; i++) {
                for (size_t j = 0; j < cols; j++) {
                    float ci = cosf((float)(2 * i + 1) * (float)u * HHO_PI_F / (2.0f * (float)rows));
                    float cj = cosf((float)(2 * j + 1) * (float)v * HHO_PI_F / (2.0f * (float)cols));
                    sum += in[i * cols + j] * ci * cj;
                }
            }
            float au = u == 0 ? sqrtf(1.0f / (float)rows) : sqrtf(2.0f / (float)rows);
            float av = v == 0 ? sqrtf(1.0f / (float)cols) : sqrtf(2.0f / (float)cols);
            out[u * cols + v] = au * av * sum;
        }
    }
}

/* crates/haagenti/src/hct_test_vectors.rs:78-107 */
void hho_reference_idct_2d(const float *in, float *out, size_t rows, size_t cols) {
    for (size_t i = 0; i < rows; i++) {
        for (size_t j = 0; j < cols; j++) {
            float sum = 0.0f;
            for (size_t u = 0; u < rows; u++) {
                for (size_t v = 0; v < cols; v++) {
                    float au = u == 0 ? sqrtf(1.0f / (float)rows) : sqrtf(2.0f / (float)rows);
                    float av = v == 0 ? sqrtf(1.0f / (float)cols) : sqrtf(2.0f / (float)cols);
                    float ci = cosf((float)(2 * i + 1) * (float)u * HHO_PI_F / (2.0f * (float)rows));
                    float cj = cosf((float)(2 * j + 1) * (float)v * HHO_PI_F / (2.0f * (float)cols));
                    sum += au * av * in[u * cols + v] * ci * cj;
                }
            }
            out[i * cols + j] = sum;
        }
    }
}

/* ===================================================================== */
/* Retention + bitmap -- crates/haagenti/src/compressive.rs               */
/* ===================================================================== */

size_t hho_retain_count(size_t n, float rho) {
    /* :97 clamp(0.05, 1.0); :152 ((n as f32 * r) as usize).max(1) */
    float r = rho;
    if (r < 0.05f) r = 0.05f;
    if (r > 1.0f) r = 1.0f;
    if (r != r) r = 0.05f;
    float prod = (float)n * r;
    size_t k = prod >= 1.8446744e19f ? (size_t)-1 : (size_t)prod;
    return k < 1 ? 1 : k;
}

typedef struct {
    float mag;
    uint32_t idx;
} mag_idx;

/* Stable descending order by magnitude; equal magnitudes keep ascending
 * index order (what a stable sort of the enumerate() sequence yields). */
static int cmp_mag_desc(const void *a, const void *b) {
    const mag_idx *x = (const mag_idx *)a, *y = (const mag_idx *)b;
    int xn = x->mag != x->mag, yn = y->mag != y->mag;
    if (xn != yn) return xn - yn; /* NaN last */
    if (!xn) {
        if (x->mag > y->mag) return -1;
        if (x->mag < y->mag) return 1;
    }
    return (x->idx > y->idx) - (x->idx < y->idx);
}

static int cmp_u32(const void *a, const void *b) {
    uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    return (x > y) - (x < y);
}

void hho_topk_bitmap(const float *c, size_t n, size_t k, uint8_t *bitmap, uint32_t *idx) {
    mag_idx *v = (mag_idx *)malloc(sizeof(mag_idx) * n);
    for (size_t i = 0; i < n; i++) {
        v[i].mag = fabsf(c[i]);
        v[i].idx = (uint32_t)i;
    }
    qsort(v, n, sizeof(mag_idx), cmp_mag_desc);
    if (k > n) k = n;
    memset(bitmap, 0, (n + 7) / 8);
    for (size_t i = 0; i < k; i++) {
        bitmap[v[i].idx / 8] |= (uint8_t)(1u << (v[i].idx % 8));
        idx[i] = v[i].idx;
    }
    qsort(idx, k, sizeof(uint32_t), cmp_u32);
    free(v);
}

size_t hho_bitmap_index_map(const uint8_t *bitmap, size_t n, uint32_t *idx) {
    size_t m = 0;
    for (size_t i = 0; i < n; i++)
        if ((bitmap[i / 8] >> (i % 8)) & 1u) idx[m++] = (uint32_t)i;
    return m;
}

/* ===================================================================== */
/* HCT-T tiles (format composed of the reference rules above)             */
/* ===================================================================== */

#define TILE 64u
#define TILE_N (TILE * TILE)
#define TILE_BITMAP (TILE_N / 8)

size_t hho_hctt_tile_bytes(size_t k) { return TILE_BITMAP + hho_int4_compressed_size(k); }

void hho_hctt_encode_tile(const float *tile, size_t k, uint8_t *out) {
    float coeffs[TILE_N];
    uint32_t idx[TILE_N];
    float vals[TILE_N];
    hho_dct_2d(tile, coeffs, TILE, TILE);
    hho_topk_bitmap(coeffs, TILE_N, k, out, idx);
    for (size_t i = 0; i < k; i++) vals[i] = coeffs[idx[i]];
    hho_quantize_int4(vals, k, out + TILE_BITMAP);
}

static int hctt_scatter(const uint8_t *t, size_t k, float *coeffs) {
    uint32_t idx[TILE_N];
    float vals[TILE_N];
    size_t m = hho_bitmap_index_map(t, TILE_N, idx);
    if (m != k) return HHO_CORRUPTED_DATA; /* compressive.rs:630-636 */
    size_t got = hho_dequantize_int4(t + TILE_BITMAP, hho_int4_compressed_size(k), k, vals);
    memset(coeffs, 0, sizeof(float) * TILE_N);
    for (size_t i = 0; i < m; i++) /* compressive.rs:741-745 */
        if (idx[i] < TILE_N && i < got) coeffs[idx[i]] = vals[i];
    return HHO_OK;
}

int hho_hctt_decode_tile(const uint8_t *t, size_t k, float *out) {
    float coeffs[TILE_N];
    int rc = hctt_scatter(t, k, coeffs);
    if (rc != HHO_OK) return rc;
    hho_idct_2d(coeffs, out, TILE, TILE); /* compressive.rs:748-749 */
    return HHO_OK;
}

int hho_hctt_decode_tile_f64(const uint8_t *t, size_t k, double *out) {
    float coeffs[TILE_N];
    double cd[TILE_N];
    int rc = hctt_scatter(t, k, coeffs);
    if (rc != HHO_OK) return rc;
    for (size_t i = 0; i < TILE_N; i++) cd[i] = coeffs[i];
    hho_idct_2d_f64(cd, out, TILE, TILE);
    return HHO_OK;
}

typedef struct {
    const float *w;
    float *outf;
    const uint8_t *tin;
    uint8_t *tout;
    size_t rows, cols, k, tb;
    int rc;
} hctt_ctx;

static void hctt_enc_task(void *vctx, size_t t) {
    hctt_ctx *c = (hctt_ctx *)vctx;
    size_t tpr = c->cols / TILE, tr = t / tpr, tc = t % tpr;
    float tile[TILE_N];
    for (size_t r = 0; r < TILE; r++)
        memcpy(tile + r * TILE, c->w + (tr * TILE + r) * c->cols + tc * TILE, TILE * sizeof(float));
    hho_hctt_encode_tile(tile, c->k, c->tout + t * c->tb);
}

static void hctt_dec_task(void *vctx, size_t t) {
    hctt_ctx *c = (hctt_ctx *)vctx;
    size_t tpr = c->cols / TILE, tr = t / tpr, tc = t % tpr;
    float tile[TILE_N];
    if (hho_hctt_decode_tile(c->tin + t * c->tb, c->k, tile) != HHO_OK) {
        __atomic_store_n(&c->rc, HHO_CORRUPTED_DATA, __ATOMIC_RELAXED);
        return;
    }
    for (size_t r = 0; r < TILE; r++)
        memcpy(c->outf + (tr * TILE + r) * c->cols + tc * TILE, tile + r * TILE, TILE * sizeof(float));
}

void hho_hctt_encode_tensor(const float *w, size_t rows, size_t cols, size_t k,
                            uint8_t *out, int nthreads) {
    hctt_ctx c = {w, NULL, NULL, out, rows, cols, k, hho_hctt_tile_bytes(k), 0};
    hho_parallel_for((rows / TILE) * (cols / TILE), nthreads, hctt_enc_task, &c);
}

int hho_hctt_decode_tensor(const uint8_t *tiles, size_t rows, size_t cols, size_t k,
                           float *out, int nthreads) {
    hctt_ctx c = {NULL, out, tiles, NULL, rows, cols, k, hho_hctt_tile_bytes(k), HHO_OK};
    hho_parallel_for((rows / TILE) * (cols / TILE), nthreads, hctt_dec_task, &c);
    return c.rc;
}

/* ===================================================================== */
/* HCT v1 container -- crates/haagenti-hct/src/tensor.rs                   */
/* ===================================================================== */

#define HCT_HEADER 64u
#define HCT_INDEX_ENTRY 8u

static void wr_u16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
static void wr_u32(uint8_t *p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i));
}
static void wr_u64(uint8_t *p, uint64_t v) {
    for (int i = 0; i < 8; i++) p[i] = (uint8_t)(v >> (8 * i));
}
static uint64_t rd_u64le(const uint8_t *p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; i--) v = (v << 8) | p[i];
    return v;
}

size_t hho_hct_file_size(size_t nblocks, size_t total_compressed) {
    return HCT_HEADER + nblocks * HCT_INDEX_ENTRY + total_compressed;
}

/* :556-616 (compress_data + finish), header :294-322 */
size_t hho_hct_write_lz4(const uint8_t *data, size_t len, uint32_t block_size,
                         uint8_t dtype, const uint64_t *shape, int rank,
                         uint8_t *out, size_t out_cap) {
    if (block_size == 0 || rank < 0 || rank > 3) return 0;
    size_t nblocks = (len + block_size - 1) / block_size;
    size_t data_start = HCT_HEADER + nblocks * HCT_INDEX_ENTRY;
    if (data_start > out_cap) return 0;
    size_t pos = data_start;
    uint32_t offset = 0;
    for (size_t b = 0; b < nblocks; b++) {
        size_t s = b * block_size, e = s + block_size < len ? s + block_size : len;
        size_t cap = hho_lz4_max_compressed_size(e - s);
        if (pos + cap > out_cap) return 0;
        size_t w = 0;
        hho_err er;
        if (hho_lz4_compress_block(data + s, e - s, out + pos, cap, &w, &er) != HHO_OK) return 0;
        uint8_t *ie = out + HCT_HEADER + b * HCT_INDEX_ENTRY;
        wr_u32(ie, offset);
        wr_u32(ie + 4, (uint32_t)w);
        offset += (uint32_t)w;
        pos += w;
    }
    uint8_t *h = out;
    memset(h, 0, HCT_HEADER);
    memcpy(h, "HCTN", 4);
    wr_u32(h + 4, 1);     /* HCT_VERSION */
    h[8] = 0;             /* LZ4 */
    h[9] = dtype;
    wr_u16(h + 10, 0);    /* flags */
    wr_u64(h + 12, len);  /* original_size */
    wr_u64(h + 20, offset);
    wr_u32(h + 28, block_size);
    wr_u32(h + 32, (uint32_t)nblocks);
    h[36] = (uint8_t)rank;
    for (int i = 0; i < rank; i++) wr_u64(h + 37 + 8 * i, shape[i]);
    return pos;
}

/* :417-445 (new), :458-483 (read_block), :486-503 (decompress_block),
 * :506-515 (decompress_all) */
int hho_hct_read_all_lz4(const uint8_t *file, size_t file_len, uint8_t *out,
                         size_t out_cap, size_t *written, hho_err *err) {
    set_err(err, HHO_OK, 0, 0, 0, 0);
    if (file_len < HCT_HEADER) { /* read_exact of the header fails, :420-423 */
        set_err(err, HHO_ALGORITHM, 0, file_len, 0, 0);
        return HHO_ALGORITHM;
    }
    if (memcmp(file, "HCTN", 4) != 0) goto bad_header;
    uint32_t ver = (uint32_t)file[4] | ((uint32_t)file[5] << 8) |
                   ((uint32_t)file[6] << 16) | ((uint32_t)file[7] << 24);
    if (ver > 2 || file[8] > 1 || file[9] > 4) goto bad_header;
    if (file[36] > 3) goto bad_header; /* rank 4 overflows the 64-byte header */
    uint64_t original = rd_u64le(file + 12);
    uint32_t block_size = rd_u32le(file + 28);
    uint32_t nblocks = rd_u32le(file + 32);
    size_t index_end = HCT_HEADER + (size_t)nblocks * HCT_INDEX_ENTRY;
    if (index_end > file_len) { /* read_exact of the index fails, :428-431 */
        set_err(err, HHO_ALGORITHM, 0, file_len, 0, 0);
        return HHO_ALGORITHM;
    }
    size_t op = 0;
    for (uint32_t b = 0; b < nblocks; b++) {
        const uint8_t *ie = file + HCT_HEADER + (size_t)b * HCT_INDEX_ENTRY;
        uint32_t off = rd_u32le(ie), csz = rd_u32le(ie + 4);
        if (index_end + (size_t)off + csz > file_len) { /* read_block, :477-480 */
            set_err(err, HHO_ALGORITHM, 0, file_len, 0, 0);
            return HHO_ALGORITHM;
        }
        uint64_t expected;
        if (b == nblocks - 1) {
            uint64_t full = (uint64_t)(nblocks - 1) * block_size;
            if (full > original) {
                set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_SIZE, 0, 0, 0);
                return HHO_CORRUPTED_DATA;
            }
            expected = original - full;
        } else {
            expected = block_size;
        }
        if (op + expected > out_cap) {
            set_err(err, HHO_BUFFER_TOO_SMALL, 0, 0, op + expected, out_cap);
            return HHO_BUFFER_TOO_SMALL;
        }
        /* decompress_with_size: zero-filled output of the expected size */
        memset(out + op, 0, expected);
        size_t w = 0;
        int rc = hho_lz4_decompress_block(file + index_end + off, csz, out + op,
                                          expected, expected, &w, err);
        if (rc != HHO_OK) return rc;
        op += w; /* truncate(len) then extend: a short block shifts the rest */
    }
    if (written) *written = op;
    return HHO_OK;
bad_header:
    set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_HEADER, 0, 0, 0);
    return HHO_CORRUPTED_DATA;
}

/* ======================= XXH3-64, seed 0 ================================= */

/* Default secret of the published XXH3 algorithm (192 bytes). */
static const uint8_t XXH3_SECRET[192] = {
    0xb8, 0xfe, 0x6c, 0x39, 0x23, 0xa4, 0x4b, 0xbe, 0x7c, 0x01, 0x81, 0x2c, 0xf7, 0x21, 0xad, 0x1c,
    0xde, 0xd4, 0x6d, 0xe9, 0x83, 0x90, 0x97, 0xdb, 0x72, 0x40, 0xa4, 0xa4, 0xb7, 0xb3, 0x67, 0x1f,
    0xcb, 0x79, 0xe6, 0x4e, 0xcc, 0xc0, 0xe5, 0x78, 0x82, 0x5a, 0xd0, 0x7d, 0xcc, 0xff, 0x72, 0x21,
    0xb8, 0x08, 0x46, 0x74, 0xf7, 0x43, 0x24, 0x8e, 0xe0, 0x35, 0x90, 0xe6, 0x81, 0x3a, 0x26, 0x4c,
    0x3c, 0x28, 0x52, 0xbb, 0x91, 0xc3, 0x00, 0xcb, 0x88, 0xd0, 0x65, 0x8b, 0x1b, 0x53, 0x2e, 0xa3,
    0x71, 0x64, 0x48, 0x97, 0xa2, 0x0d, 0xf9, 0x4e, 0x38, 0x19, 0xef, 0x46, 0xa9, 0xde, 0xac, 0xd8,
    0xa8, 0xfa, 0x76, 0x3f, 0xe3, 0x9c, 0x34, 0x3f, 0xf9, 0xdc, 0xbb, 0xc7, 0xc7, 0x0b, 0x4f, 0x1d,
    0x8a, 0x51, 0xe0, 0x4b, 0xcd, 0xb4, 0x59, 0x31, 0xc8, 0x9f, 0x7e, 0xc9, 0xd9, 0x78, 0x73, 0x64,
    0xea, 0xc5, 0xac, 0x83, 0x34, 0xd3, 0xeb, 0xc3, 0xc5, 0x81, 0xa0, 0xff, 0xfa, 0x13, 0x63, 0xeb,
    0x17, 0x0d, 0xdd, 0x51, 0xb7, 0xf0, 0xda, 0x49, 0xd3, 0x16, 0x55, 0x26, 0x29, 0xd4, 0x68, 0x9e,
    0x2b, 0x16, 0xbe, 0x58, 0x7d, 0x47, 0xa1, 0xfc, 0x8f, 0xf8, 0xb8, 0xd1, 0x7a, 0xd0, 0x31, 0xce,
    0x45, 0xcb, 0x3a, 0x8f, 0x95, 0x16, 0x04, 0x28, 0xaf, 0xd7, 0xfb, 0xca, 0xbb, 0x4b, 0x40, 0x7e,
};
#define P32_1 0x9E3779B1u
#define P32_2 0x85EBCA77u
#define P32_3 0xC2B2AE3Du
#define P64_1 0x9E3779B185EBCA87ull
#define P64_2 0xC2B2AE3D27D4EB4Full
#define P64_3 0x165667B19E3779F9ull
#define P64_4 0x85EBCA77C2B2AE63ull
#define P64_5 0x27D4EB2F165667C5ull
#define PMX1 0x165667919E3779F9ull
#define PMX2 0x9FB21C651E98DF25ull

static uint64_t x_rd64(const uint8_t *p) { return rd_u64le(p); }
static uint32_t x_rd32(const uint8_t *p) { return rd_u32le(p); }
static uint64_t x_rotl(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }
static uint64_t x_fold(uint64_t a, uint64_t b) { /* low ^ high of the 128-bit product */
    unsigned __int128 m = (unsigned __int128)a * b;
    return (uint64_t)m ^ (uint64_t)(m >> 64);
}
static uint64_t x_avalanche(uint64_t h) { /* XXH3 avalanche */
    h ^= h >> 37;
    h *= PMX1;
    return h ^ (h >> 32);
}
static uint64_t x64_avalanche(uint64_t h) { /* XXH64 avalanche */
    h ^= h >> 33;
    h *= P64_2;
    h ^= h >> 29;
    h *= P64_3;
    return h ^ (h >> 32);
}
static uint64_t x_rrmxmx(uint64_t h, uint64_t len) {
    h ^= x_rotl(h, 49) ^ x_rotl(h, 24);
    h *= PMX2;
    h ^= (h >> 35) + len;
    h *= PMX2;
    return h ^ (h >> 28);
}
static uint64_t x_mix16(const uint8_t *in, const uint8_t *sec) {
    return x_fold(x_rd64(in) ^ x_rd64(sec), x_rd64(in + 8) ^ x_rd64(sec + 8));
}
/* one 64-byte stripe into the eight accumulators */
static void x_stripe(uint64_t acc[8], const uint8_t *in, const uint8_t *sec) {
    for (int i = 0; i < 8; i++) {
        uint64_t v = x_rd64(in + 8 * i), k = v ^ x_rd64(sec + 8 * i);
        acc[i ^ 1] += v;
        acc[i] += (k & 0xffffffffull) * (k >> 32);
    }
}

uint64_t hho_xxh3_64(const uint8_t *in, size_t len) {
    const uint8_t *S = XXH3_SECRET;
    if (len == 0) return x64_avalanche(x_rd64(S + 56) ^ x_rd64(S + 64));
    if (len <= 3) {
        uint32_t c = ((uint32_t)in[0] << 16) | ((uint32_t)in[len >> 1] << 24) |
                     (uint32_t)in[len - 1] | ((uint32_t)len << 8);
        return x64_avalanche((uint64_t)c ^ (uint64_t)(x_rd32(S) ^ x_rd32(S + 4)));
    }
    if (len <= 8) {
        uint64_t v = (uint64_t)x_rd32(in + len - 4) + ((uint64_t)x_rd32(in) << 32);
        return x_rrmxmx(v ^ (x_rd64(S + 8) ^ x_rd64(S + 16)), len);
    }
    if (len <= 16) {
        uint64_t lo = x_rd64(in) ^ (x_rd64(S + 24) ^ x_rd64(S + 32));
        uint64_t hi = x_rd64(in + len - 8) ^ (x_rd64(S + 40) ^ x_rd64(S + 48));
        return x_avalanche(len + __builtin_bswap64(lo) + hi + x_fold(lo, hi));
    }
    if (len <= 128) {
        uint64_t acc = len * P64_1;
        size_t r = (len - 1) / 32; /* pairs of 16-byte mixes from both ends */
        for (size_t i = 0; i <= r; i++) {
            acc += x_mix16(in + 16 * i, S + 32 * i);
            acc += x_mix16(in + len - 16 * (i + 1), S + 32 * i + 16);
        }
        return x_avalanche(acc);
    }
    if (len <= 240) {
        uint64_t acc = len * P64_1;
        for (int i = 0; i < 8; i++) acc += x_mix16(in + 16 * i, S + 16 * i);
        uint64_t tail = x_mix16(in + len - 16, S + 136 - 17);
        acc = x_avalanche(acc);
        for (size_t i = 8; i < len / 16; i++) tail += x_mix16(in + 16 * i, S + 16 * (i - 8) + 3);
        return x_avalanche(acc + tail);
    }
    /* long input: 1 KiB blocks of 16 stripes, scramble after each block */
    uint64_t acc[8] = {P32_3, P64_1, P64_2, P64_3, P64_4, P32_2, P64_5, P32_1};
    const size_t block = 64 * 16;
    size_t nb = (len - 1) / block;
    for (size_t b = 0; b < nb; b++) {
        for (int s = 0; s < 16; s++) x_stripe(acc, in + b * block + 64 * s, S + 8 * s);
        for (int i = 0; i < 8; i++) {
            uint64_t a = acc[i];
            a ^= a >> 47;
            a ^= x_rd64(S + 192 - 64 + 8 * i);
            acc[i] = a * P32_1;
        }
    }
    size_t ns = ((len - 1) - block * nb) / 64;
    for (size_t s = 0; s < ns; s++) x_stripe(acc, in + nb * block + 64 * s, S + 8 * s);
    x_stripe(acc, in + len - 64, S + 192 - 64 - 7);
    uint64_t r = len * P64_1;
    for (int i = 0; i < 4; i++)
        r += x_fold(acc[2 * i] ^ x_rd64(S + 11 + 16 * i), acc[2 * i + 1] ^ x_rd64(S + 11 + 16 * i + 8));
    return x_avalanche(r);
}

/* ======================= HCT v2 container ================================ */

#define HCT_INDEX_V2 16u

size_t hho_hct_write_v2_lz4(const uint8_t *data, size_t len, uint32_t block_size,
                            uint8_t dtype, const uint64_t *shape, int rank, uint16_t flags,
                            const uint8_t *quant8, uint8_t *out, size_t out_cap) {
    if (block_size == 0 || rank < 0 || rank > 3) return 0;
    size_t nblocks = (len + block_size - 1) / block_size;
    size_t qsz = (flags & HHO_FLAG_QUANTIZATION) ? 8 : 0;
    /* :809-814: the index is always written with 16-byte v2 entries; the
     * checksum field is 0 when block checksums are off (:726-733) */
    size_t data_start = HCT_HEADER + qsz + nblocks * HCT_INDEX_V2;
    if (data_start > out_cap) return 0;
    size_t pos = data_start;
    uint32_t offset = 0;
    for (size_t b = 0; b < nblocks; b++) {
        size_t s = b * block_size, e = s + block_size < len ? s + block_size : len;
        size_t cap = hho_lz4_max_compressed_size(e - s);
        if (pos + cap > out_cap) return 0;
        size_t w = 0;
        hho_err er;
        if (hho_lz4_compress_block(data + s, e - s, out + pos, cap, &w, &er) != HHO_OK) return 0;
        uint8_t *ie = out + HCT_HEADER + qsz + b * HCT_INDEX_V2;
        wr_u32(ie, offset);
        wr_u32(ie + 4, (uint32_t)w);
        wr_u64(ie + 8, (flags & HHO_FLAG_BLOCK_CHECKSUMS) ? hho_xxh3_64(out + pos, w) : 0);
        offset += (uint32_t)w;
        pos += w;
    }
    uint8_t *h = out;
    memset(h, 0, HCT_HEADER);
    memcpy(h, "HCTN", 4);
    wr_u32(h + 4, 2); /* HCT_VERSION_V2 */
    h[8] = 0;         /* LZ4 */
    h[9] = dtype;
    wr_u16(h + 10, flags);
    wr_u64(h + 12, len);
    wr_u64(h + 20, offset);
    wr_u32(h + 28, block_size);
    wr_u32(h + 32, (uint32_t)nblocks);
    h[36] = (uint8_t)rank;
    for (int i = 0; i < rank; i++) wr_u64(h + 37 + 8 * i, shape[i]);
    /* :792-795: XXH3 of bytes 0..56 stored at 56..64 (over dims[2]'s tail) */
    wr_u64(h + 56, hho_xxh3_64(h, 56));
    if (qsz) memcpy(h + HCT_HEADER, quant8, 8);
    return pos;
}

/* HctReaderV2::new (:841-920): header, header checksum, quantization
 * metadata, index entry size and data offset. */
static int v2_open(const uint8_t *file, size_t file_len, hho_err *err, uint64_t *original,
                   uint32_t *block_size, uint32_t *nblocks, size_t *index_at, size_t *entry,
                   size_t *data_at) {
    if (file_len < HCT_HEADER) {
        set_err(err, HHO_ALGORITHM, 0, file_len, 0, 0);
        return HHO_ALGORITHM;
    }
    if (memcmp(file, "HCTN", 4) != 0) goto bad_header;
    uint32_t ver = rd_u32le(file + 4);
    if (ver > 2 || file[8] > 1 || file[9] > 4 || file[36] > 3) goto bad_header;
    uint16_t flags = (uint16_t)(file[10] | (file[11] << 8));
    if (ver >= 2 && (flags & HHO_FLAG_HEADER_CHECKSUM) &&
        hho_xxh3_64(file, 56) != rd_u64le(file + 56)) {
        set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_HEADER_CHECKSUM, 0, 0, 0);
        return HHO_CORRUPTED_DATA;
    }
    size_t at = HCT_HEADER;
    if (flags & HHO_FLAG_QUANTIZATION) {
        if (file_len < at + 8) {
            set_err(err, HHO_ALGORITHM, 0, file_len, 0, 0);
            return HHO_ALGORITHM;
        }
        if (file[at] > 4) {
            set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_QUANT_SCHEME, 0, 0, 0);
            return HHO_CORRUPTED_DATA;
        }
        at += 8;
    }
    *entry = (ver >= 2 && (flags & HHO_FLAG_BLOCK_CHECKSUMS)) ? HCT_INDEX_V2 : HCT_INDEX_ENTRY;
    *original = rd_u64le(file + 12);
    *block_size = rd_u32le(file + 28);
    *nblocks = rd_u32le(file + 32);
    *index_at = at;
    *data_at = at + (size_t)*nblocks * *entry;
    if (*data_at > file_len) {
        set_err(err, HHO_ALGORITHM, 0, file_len, 0, 0);
        return HHO_ALGORITHM;
    }
    return HHO_OK;
bad_header:
    set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_HEADER, 0, 0, 0);
    return HHO_CORRUPTED_DATA;
}

/* read_block_validated (:937-977): range, then checksum when non-zero */
static int v2_block(const uint8_t *file, size_t file_len, size_t index_at, size_t entry,
                    size_t data_at, uint32_t b, hho_err *err, const uint8_t **blk, uint32_t *csz) {
    const uint8_t *ie = file + index_at + (size_t)b * entry;
    uint32_t off = rd_u32le(ie);
    *csz = rd_u32le(ie + 4);
    uint64_t sum = entry == HCT_INDEX_V2 ? rd_u64le(ie + 8) : 0;
    if (data_at + (size_t)off + *csz > file_len) {
        set_err(err, HHO_ALGORITHM, 0, file_len, 0, 0);
        return HHO_ALGORITHM;
    }
    *blk = file + data_at + off;
    if (sum != 0 && hho_xxh3_64(*blk, *csz) != sum) {
        set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_BLOCK_CHECKSUM, 0, 0, 0);
        return HHO_CORRUPTED_DATA;
    }
    return HHO_OK;
}

int hho_hct_read_all_v2_lz4(const uint8_t *file, size_t file_len, uint8_t *out,
                            size_t out_cap, size_t *written, hho_err *err,
                            int64_t *failed_block) {
    set_err(err, HHO_OK, 0, 0, 0, 0);
    if (failed_block) *failed_block = -1;
    uint64_t original;
    uint32_t block_size, nblocks;
    size_t index_at, entry, data_at;
    int rc = v2_open(file, file_len, err, &original, &block_size, &nblocks, &index_at, &entry,
                     &data_at);
    if (rc != HHO_OK) return rc;
    size_t op = 0;
    for (uint32_t b = 0; b < nblocks; b++) {
        if (failed_block) *failed_block = b;
        const uint8_t *blk;
        uint32_t csz;
        rc = v2_block(file, file_len, index_at, entry, data_at, b, err, &blk, &csz);
        if (rc != HHO_OK) return rc;
        uint64_t expected;
        if (b == nblocks - 1) { /* :988-994 */
            uint64_t full = (uint64_t)(nblocks - 1) * block_size;
            if (full > original) {
                set_err(err, HHO_CORRUPTED_DATA, HHO_CORRUPT_SIZE, 0, 0, 0);
                return HHO_CORRUPTED_DATA;
            }
            expected = original - full;
        } else {
            expected = block_size;
        }
        if (op + expected > out_cap) {
            set_err(err, HHO_BUFFER_TOO_SMALL, 0, 0, op + expected, out_cap);
            return HHO_BUFFER_TOO_SMALL;
        }
        memset(out + op, 0, expected);
        size_t w = 0;
        rc = hho_lz4_decompress_block(blk, csz, out + op, expected, expected, &w, err);
        if (rc != HHO_OK) return rc;
        op += w;
    }
    if (failed_block) *failed_block = -1;
    if (written) *written = op;
    return HHO_OK;
}

int hho_hct_validate_v2(const uint8_t *file, size_t file_len, hho_err *err,
                        int64_t *failed_block) {
    set_err(err, HHO_OK, 0, 0, 0, 0);
    if (failed_block) *failed_block = -1;
    uint64_t original;
    uint32_t block_size, nblocks;
    size_t index_at, entry, data_at;
    int rc = v2_open(file, file_len, err, &original, &block_size, &nblocks, &index_at, &entry,
                     &data_at);
    if (rc != HHO_OK) return rc;
    for (uint32_t b = 0; b < nblocks; b++) {
        const uint8_t *blk;
        uint32_t csz;
        rc = v2_block(file, file_len, index_at, entry, data_at, b, err, &blk, &csz);
        if (rc != HHO_OK) {
            if (failed_block) *failed_block = b;
            return rc;
        }
    }
    return HHO_OK;
}

typedef struct {
    const uint8_t *data;
    const uint64_t *off;
    const uint32_t *len;
    uint64_t *out;
} xxh_batch_ctx;
static void xxh_batch_task(void *vctx, size_t i) {
    xxh_batch_ctx *c = (xxh_batch_ctx *)vctx;
    c->out[i] = hho_xxh3_64(c->data + c->off[i], c->len[i]);
}
void hho_xxh3_64_batch(const uint8_t *data, const uint64_t *off, const uint32_t *len, size_t n,
                       uint64_t *out, int nthreads) {
    xxh_batch_ctx c = {data, off, len, out};
    hho_parallel_for(n, nthreads, xxh_batch_task, &c);
}

/* =====================================================================
 * HCT3 whole-tensor spectral decode
 * ===================================================================== */

static uint16_t rd16le(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32le(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* half::f16::from_f32 (round to nearest even; NaN stays NaN). */
uint16_t hho_f32_to_f16_rne(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return (uint16_t)sign;
        uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u, sh = 126 - e;
        uint32_t r = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (a - 0x38000000u) >> 13, rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

/* parse_hct_fragments + reconstruct_coefficients
 * (crates/haagenti-cuda/src/decompress.rs:322-427). */
int hho_hct3_coefficients(const uint8_t *data, size_t len, size_t total, float *dense) {
    if (len < 2) return HHO_INVALID_DATA;                 /* :324-326 */
    for (size_t i = 0; i < total; i++) dense[i] = 0.0f;   /* :405 */
    size_t nf = rd16le(data), off = 2, bm = (total + 7) / 8;
    for (size_t f = 0; f < nf; f++) {
        if (off + 16 > len) break;                        /* :335-337 */
        off += 12;                                        /* index, flags, checksum */
        size_t dl = rd32le(data + off);
        off += 4;
        if (off + dl > len) return HHO_INVALID_DATA;      /* :362-367 */
        const uint8_t *fd = data + off;
        off += dl;
        if (dl < 4) continue;                             /* :373-375 */
        if (dl < 4 + bm) continue;                        /* :380-383 */
        const uint8_t *bits = fd + 4, *cd = fd + 4 + bm;
        size_t nc = (dl - 4 - bm) / 2;                    /* chunks_exact(2), :388-394 */
        size_t ci = 0;
        for (size_t b = 0; b < bm; b++)                   /* :408-424 */
            for (int k = 0; k < 8; k++) {
                size_t e = b * 8 + (size_t)k;
                if (e >= total) break;
                if (((bits[b] >> k) & 1) && ci < nc) {
                    dense[e] = hho_f16_bits_to_f32(rd16le(cd + 2 * ci));
                    ci++;
                }
            }
    }
    return HHO_OK;
}

/* GpuDecompressor::decompress with the CPU transform: coefficients, then
 * idct_2d (dct.rs:311-337) over width = last dimension, height = the rest
 * (decompress.rs:430-442). */
int hho_hct3_decode(const uint8_t *data, size_t len, const uint64_t *shape, size_t rank, float *out) {
    size_t total = 1;
    for (size_t i = 0; i < rank; i++) total *= (size_t)shape[i];
    size_t w = rank == 0 ? 1 : (size_t)shape[rank - 1], h = w ? total / w : 0;
    float *dense = (float *)malloc(sizeof(float) * (total ? total : 1));
    int rc = hho_hct3_coefficients(data, len, total, dense);
    if (rc == HHO_OK && total) hho_idct_2d(dense, out, w, h);
    free(dense);
    return rc;
}

/* CompressiveSpectralEncoder::encode_2d_from_dct (compressive.rs:240-340):
 * fragment f is out[offsets[f] .. offsets[f+1]).  Returns the bytes
 * written (0 when cap is short). */
size_t hho_spectral_encode_from_dct(const float *dct, uint32_t width, uint32_t height, uint16_t nfrag,
                                    float retention, float essential_ratio, uint8_t *out, size_t cap,
                                    uint64_t *offsets) {
    size_t n = (size_t)width * height;
    float rr = retention < 0.05f ? 0.05f : retention > 1.0f ? 1.0f : retention;   /* :98 */
    float er = essential_ratio < 0.05f ? 0.05f : essential_ratio > 1.0f ? 1.0f : essential_ratio; /* :107 */
    size_t keep = (size_t)((float)n * rr);
    if (keep < 1) keep = 1;
    if (keep > n) keep = n;
    size_t ess = (size_t)((float)keep * er);
    if (ess < 1) ess = 1;
    size_t det = keep - ess;
    size_t dpf = nfrag > 1 ? (det + nfrag - 2) / (nfrag - 1) : det;
    uint8_t *bm = (uint8_t *)malloc((n + 7) / 8 + 1);
    uint32_t *idx = (uint32_t *)malloc(sizeof(uint32_t) * (keep ? keep : 1));
    hho_topk_bitmap(dct, n, keep, bm, idx);
    size_t need = 24 + (n + 7) / 8 + 2 * ess;
    for (size_t f = 1; f < nfrag; f++) {
        size_t s = ess + (f - 1) * dpf, e = s + dpf < keep ? s + dpf : keep;
        need += 8 + 2 * (e > s ? e - s : 0);
    }
    if (need > cap) {
        free(bm);
        free(idx);
        return 0;
    }
    uint8_t *p = out;
#define W32(v) do { uint32_t t_ = (uint32_t)(v); for (int i_ = 0; i_ < 4; i_++) *p++ = (uint8_t)(t_ >> (8 * i_)); } while (0)
#define W16(v) do { uint16_t t_ = (uint16_t)(v); *p++ = (uint8_t)t_; *p++ = (uint8_t)(t_ >> 8); } while (0)
    offsets[0] = 0;
    W32(0x48435433u);
    W32(width);
    W32(height);
    W32(keep);
    W32(ess);
    W32(dpf);
    memcpy(p, bm, (n + 7) / 8);
    p += (n + 7) / 8;
    for (size_t i = 0; i < ess; i++) W16(hho_f32_to_f16_rne(dct[idx[i]]));
    for (size_t f = 1; f < nfrag; f++) {
        offsets[f] = (uint64_t)(p - out);
        W16(f);
        W16(nfrag);
        size_t s = ess + (f - 1) * dpf, e = s + dpf < keep ? s + dpf : keep;
        W32(e > s ? e - s : 0);
        for (size_t i = s; i < e; i++) W16(hho_f32_to_f16_rne(dct[idx[i]]));
    }
#undef W32
#undef W16
    offsets[nfrag] = (uint64_t)(p - out);
    free(bm);
    free(idx);
    return (size_t)(p - out);
}

/* CompressiveSpectralDecoder::add_essentials (V2/V3, compressive.rs:438-651),
 * add_detail (:653-700) and reconstruct (:728-752).  Fragments after the
 * first with index 0 are ignored; a detail fragment whose own index field
 * is 0 is rejected (the reference's start position underflows). */
int hho_spectral_reconstruct(const uint8_t *const *frags, const size_t *lens, const uint16_t *fidx, uint32_t nf,
                             float *out, size_t out_cap, uint32_t *width, uint32_t *height, hho_err *err) {
    memset(err, 0, sizeof(*err));
    err->kind = HHO_CORRUPTED_DATA;
    if (nf == 0 || fidx[0] != 0) { err->sub = HHO_CORRUPT_HEADER; return err->kind; }
    const uint8_t *d = frags[0];
    size_t l = lens[0];
    if (l < 24) { err->sub = HHO_CORRUPT_SIZE; return err->kind; }
    uint32_t magic = rd32le(d);
    if (magic != 0x48435433u && magic != 0x48435432u) { err->kind = HHO_UNSUPPORTED; return err->kind; }
    int v3 = magic == 0x48435433u;
    size_t csz = v3 ? 2 : 4;
    uint32_t w = rd32le(d + 4), h = rd32le(d + 8), ntot = rd32le(d + 12), ness = rd32le(d + 16), dpf = rd32le(d + 20);
    *width = w;
    *height = h;
    size_t n = (size_t)w * h, bm = (n + 7) / 8;
    if (24 + bm > l) { err->sub = HHO_CORRUPT_SIZE; return err->kind; }
    uint32_t *map = (uint32_t *)malloc(sizeof(uint32_t) * (n ? n : 1));
    size_t cnt = hho_bitmap_index_map(d + 24, n, map);
    if (cnt != ntot) { free(map); err->sub = HHO_CORRUPT_BITMAP_COUNT; return err->kind; }
    float *coef = (float *)calloc(ntot ? ntot : 1, sizeof(float));
    size_t off = 24 + bm;
    for (uint32_t i = 0; i < ness; i++) {
        if (off + csz > l || i >= ntot) { free(map); free(coef); err->sub = HHO_CORRUPT_SIZE; return err->kind; }
        if (v3) coef[i] = hho_f16_bits_to_f32(rd16le(d + off));
        else memcpy(&coef[i], d + off, 4);
        off += csz;
    }
    for (uint32_t f = 1; f < nf; f++) {
        if (fidx[f] == 0) continue;
        const uint8_t *q = frags[f];
        size_t ql = lens[f];
        if (ql < 8) { free(map); free(coef); err->sub = HHO_CORRUPT_SIZE; return err->kind; }
        uint32_t fi = rd16le(q), count = rd32le(q + 4);
        if (fi == 0) { free(map); free(coef); err->sub = HHO_CORRUPT_HEADER; return err->kind; }
        size_t start = (size_t)ness + (size_t)(fi - 1) * dpf, o = 8;
        for (uint32_t i = 0; i < count; i++) {
            if (o + csz > ql) break;
            size_t ci = start + i;
            if (ci < ntot) {
                if (v3) coef[ci] = hho_f16_bits_to_f32(rd16le(q + o));
                else memcpy(&coef[ci], q + o, 4);
            }
            o += csz;
        }
    }
    if (out_cap < n) {
        free(map); free(coef);
        err->kind = HHO_BUFFER_TOO_SMALL;
        err->required = n;
        err->provided = out_cap;
        return err->kind;
    }
    float *dense = (float *)calloc(n ? n : 1, sizeof(float));
    for (size_t i = 0; i < ntot; i++) dense[map[i]] = coef[i];
    if (n) hho_idct_2d(dense, out, w, h);
    free(dense);
    free(map);
    free(coef);
    err->kind = HHO_OK;
    return HHO_OK;
}
