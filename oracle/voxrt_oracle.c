/* voxrt_oracle.c — scalar CPU restatement of voxrt's ternary x int8 GEMM path (the oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never the product path. Built with
 * -O2 -ffp-contract=off and no fast-math, so every float operation below is one IEEE-rounded step, exactly as the
 * Rust reference performs it (Rust never contracts a*b+c; `mul_add` is a correctly rounded fma, as is C's fmaf).
 */
#include "voxrt_oracle.h"
#include "par.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* Reference test generator: crates/voxrt/tests/kernels.rs:7-12 (also x86_kernels.rs:9-14). */
uint32_t or_lcg(uint64_t *state) {
    *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
    return (uint32_t)(*state >> 33);
}

/* trits.rs:7-27 — 5 base-3 digits per byte, least significant first, trit = digit - 1. The last byte of a row
 * with in_features % 5 != 0 holds fewer real digits; its pad digits are never decoded. */
void or_unpack_row(const uint8_t *packed, size_t in_features, int8_t *out) {
    size_t full = in_features / 5;
    for (size_t i = 0; i < full; i++) {
        unsigned v = packed[i];
        for (int d = 0; d < 5; d++) {
            out[i * 5 + d] = (int8_t)((int)(v % 3) - 1);
            v /= 3;
        }
    }
    size_t rem = in_features - full * 5;
    if (rem) {
        unsigned v = packed[full];
        for (size_t d = 0; d < rem; d++) {
            out[full * 5 + d] = (int8_t)((int)(v % 3) - 1);
            v /= 3;
        }
    }
}

/* trits.rs:30-41 — inverse of unpack_row; pad digits are 0 (u8 arithmetic, p wraps after the 5th digit). */
void or_pack_row(const int8_t *trits, size_t n, uint8_t *out) {
    for (size_t i = 0; i * 5 < n; i++) {
        uint8_t v = 0, p = 1;
        for (size_t j = i * 5; j < n && j < i * 5 + 5; j++) {
            v = (uint8_t)(v + (uint8_t)(trits[j] + 1) * p);
            p = (uint8_t)(p * 3);
        }
        out[i] = v;
    }
}

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* IEEE binary16 -> binary32, exact (the `half` crate's f16::to_f32, used by trits.rs:56 and packed.rs:126). */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        float v = ldexpf((float)m, -24); /* subnormal half: m * 2^-24, exact in binary32 */
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112) << 23) | (m << 13));
}

/* IEEE binary32 -> binary16, round to nearest even (half's f16::from_f32; used by the test generators,
 * tests/kernels.rs:25). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t e = (x >> 23) & 0xff, m = x & 0x7fffff;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00 | (m ? (0x200 | (m >> 13)) : 0));
    int32_t he = (int32_t)e - 127 + 15;
    if (he >= 31) return (uint16_t)(sign | 0x7c00);
    if (he <= 0) {
        if (he < -10) return sign;
        uint32_t mm = m | 0x800000; /* 24-bit significand */
        int shift = 14 - he;        /* 1 - he + 13 */
        uint32_t q = mm >> shift, rem = mm & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)he << 10) | (m >> 13), rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++; /* carry into the exponent is the correct result */
    return (uint16_t)(sign | q);
}

void or_f16_to_f32_n(const uint16_t *h, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(h[i]);
}

/* trits.rs:44-84 — w[r][c] = f16 scale[r][c / group] * trit[r][c]. */
void or_dequant_matrix(const uint8_t *qweight, const uint16_t *scales_f16, size_t out_features,
                       size_t in_features, size_t group, float *w) {
    size_t rb = (in_features + 4) / 5, ng = in_features / group;
    int8_t *t = (int8_t *)malloc(in_features);
    for (size_t r = 0; r < out_features; r++) {
        or_unpack_row(qweight + r * rb, in_features, t);
        for (size_t g = 0; g < ng; g++) {
            float s = or_f16_to_f32(scales_f16[r * ng + g]);
            for (size_t c = g * group; c < (g + 1) * group; c++) w[r * in_features + c] = s * (float)t[c];
        }
    }
    free(t);
}

/* packed.rs:96-100 (Layout::Rows) — the whole matrix unpacked to int8 rows. */
void or_unpack_matrix(const uint8_t *qweight, size_t out_features, size_t in_features, int8_t *w) {
    size_t rb = (in_features + 4) / 5;
    for (size_t r = 0; r < out_features; r++) or_unpack_row(qweight + r * rb, in_features, w + r * in_features);
}

/* packed.rs:527-535 quantize_group_portable — s = absmax/127 (1 for an all-zero group), inv = 1/s,
 * q = clamp(round_half_even(v*inv), -127, 127). Rust's f32::max ignores a NaN operand, as fmaxf does; a NaN code
 * casts to 0 in Rust (`as i8`). */
float or_quantize_group(const float *src, size_t n, int8_t *dst) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) amax = fmaxf(amax, fabsf(src[i]));
    float s = amax == 0.0f ? 1.0f : amax / 127.0f;
    float inv = 1.0f / s;
    for (size_t i = 0; i < n; i++) {
        float v = rintf(src[i] * inv);
        if (isnan(v)) { dst[i] = 0; continue; }
        if (v < -127.0f) v = -127.0f;
        if (v > 127.0f) v = 127.0f;
        dst[i] = (int8_t)v;
    }
    return s;
}

/* packed.rs:307-436 (QuantAct::quantize_layout, Rows/Quad16) — per (token, group) scale and codes, plus the code
 * sums `gsum` (packed.rs:349-360). q has n rows of inp bytes; scales and gsum are [n, inp/group]. */
/* ---- parallel-for (par.h) */
static int g_threads = 1;
int or_get_threads(void) { return g_threads; }
void or_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }

typedef struct {
    or_range_fn fn;
    void *ctx;
    size_t lo, hi;
} par_job;

static void *par_main(void *p) {
    par_job *j = (par_job *)p;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

void or_par_for(size_t n, or_range_fn fn, void *ctx) {
    size_t T = (size_t)g_threads;
    if (T > n) T = n;
    if (T <= 1) {
        if (n) fn(ctx, 0, n);
        return;
    }
    pthread_t th[256];
    par_job jobs[256];
    size_t chunk = (n + T - 1) / T;
    size_t used = 0;
    for (size_t i = 0; i < T; i++) {
        size_t lo = i * chunk, hi = lo + chunk < n ? lo + chunk : n;
        if (lo >= hi) break;
        jobs[i] = (par_job){fn, ctx, lo, hi};
        if (pthread_create(&th[i], NULL, par_main, &jobs[i]) != 0) { /* fall back to running inline */
            fn(ctx, lo, hi);
            th[i] = 0;
        }
        used = i + 1;
    }
    for (size_t i = 0; i < used; i++)
        if (th[i]) pthread_join(th[i], NULL);
}

typedef struct {
    const float *x;
    size_t inp, group;
    int8_t *q;
    float *scales;
    int32_t *gsum;
} quant_ctx;

static void quantize_rows(void *c_, size_t lo, size_t hi) {
    quant_ctx *c = (quant_ctx *)c_;
    size_t inp = c->inp, group = c->group, ng = inp / group;
    for (size_t t = lo; t < hi; t++)
        for (size_t g = 0; g < ng; g++) {
            int8_t *d = c->q + t * inp + g * group;
            c->scales[t * ng + g] = or_quantize_group(c->x + t * inp + g * group, group, d);
            if (c->gsum) {
                int32_t s = 0;
                for (size_t k = 0; k < group; k++) s += d[k];
                c->gsum[t * ng + g] = s;
            }
        }
}

void or_quantize(const float *x, size_t n, size_t inp, size_t group, int8_t *q, float *scales, int32_t *gsum) {
    quant_ctx c = {x, inp, group, q, scales, gsum};
    or_par_for(n, quantize_rows, &c);
}

/* tensor.rs:829-848 exp_poly — clamp to [-87, 88], n = round_half_even(x*log2 e), two-step Cody-Waite reduction
 * with fmas, degree-6 Horner polynomial by fma, times 2^n built in the exponent field. */
float or_exp_poly(float x) {
    if (x < -87.0f) x = -87.0f;
    if (x > 88.0f) x = 88.0f;
    float n = rintf(x * 1.44269504088896340736f);
    float r = fmaf(-n, 0.69314575f, x);
    r = fmaf(-n, 1.4286068e-6f, r);
    static const float c[6] = {1.0f / 120.0f, 1.0f / 24.0f, 1.0f / 6.0f, 0.5f, 1.0f, 1.0f};
    float p = 1.0f / 720.0f;
    for (int i = 0; i < 6; i++) p = fmaf(p, r, c[i]);
    return p * bits_f32((uint32_t)(((int32_t)n + 127) << 23));
}

/* tensor.rs:852-854 silu_fast, 856-860 sigmoid_fast. */
float or_silu_fast(float x) { return x / (1.0f + or_exp_poly(-x)); }
float or_sigmoid_fast(float x) { return 1.0f / (1.0f + or_exp_poly(-x)); }

/* kernels/mod.rs:41-48 Epilogue::apply — Store: v; Silu: silu_fast(v); AddScaled(s): fma(s, v, old). */
float or_ep_apply(int ep, float alpha, float old, float v) {
    switch (ep) {
    case OR_EP_SILU: return or_silu_fast(v);
    case OR_EP_ADD_SCALED: return fmaf(alpha, v, old);
    default: return v;
    }
}

/* kernels/mod.rs:166-210 gemm_scalar_range (Rows layouts) — for rows o in [r0, r1) and tokens t in [t0, t1):
 * S_g = sum_{c in g} w[o][c]*x[t][c] (exact int32), acc = fma((float)S_g, xs[t][g]*ws[o][g], acc) for g ascending
 * from acc = 0, then y[t*out + o] = ep(y_old, acc). Only that block of y is written. When group_sums is given,
 * S_g is also written to group_sums[(g*n + t)*out + o]. */
void or_gemm_scalar_range(const int8_t *w, const float *ws, size_t out, size_t inp, size_t group,
                          const int8_t *x, const float *xs, size_t n, float *y, size_t r0, size_t r1, size_t t0,
                          size_t t1, int ep, float alpha, int32_t *group_sums) {
    size_t ng = inp / group;
    for (size_t o = r0; o < r1; o++) {
        const int8_t *wr = w + o * inp;
        for (size_t t = t0; t < t1; t++) {
            const int8_t *xr = x + t * inp;
            float acc = 0.0f;
            for (size_t g = 0; g < ng; g++) {
                int32_t s = 0;
                for (size_t c = g * group; c < (g + 1) * group; c++) s += (int32_t)wr[c] * (int32_t)xr[c];
                float p = xs[t * ng + g] * ws[o * ng + g];
                acc = fmaf((float)s, p, acc);
                if (group_sums) group_sums[(g * n + t) * out + o] = s;
            }
            y[t * out + o] = or_ep_apply(ep, alpha, y[t * out + o], acc);
        }
    }
}

/* The same, split over output-row blocks on `threads` threads (blocks are disjoint in columns of y, as in
 * kernels/mod.rs:348-354), so the oracle finishes the larger parity cases in seconds. */
typedef struct {
    const int8_t *w; const float *ws; size_t out, inp, group; const int8_t *x; const float *xs; size_t n;
    float *y; int ep; float alpha; int32_t *gs; size_t chunk; size_t nblocks; size_t next;
    pthread_mutex_t mu;
} scalar_job;

static void *scalar_worker(void *arg) {
    scalar_job *j = (scalar_job *)arg;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        size_t b = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (b >= j->nblocks) return NULL;
        size_t r0 = b * j->chunk, r1 = r0 + j->chunk < j->out ? r0 + j->chunk : j->out;
        or_gemm_scalar_range(j->w, j->ws, j->out, j->inp, j->group, j->x, j->xs, j->n, j->y, r0, r1, 0, j->n, j->ep,
                             j->alpha, j->gs);
    }
}

void or_gemm_scalar_mt(const int8_t *w, const float *ws, size_t out, size_t inp, size_t group, const int8_t *x,
                       const float *xs, size_t n, float *y, int ep, float alpha, int32_t *group_sums, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    scalar_job j = {w, ws, out, inp, group, x, xs, n, y, ep, alpha, group_sums, 0, 0, 0, PTHREAD_MUTEX_INITIALIZER};
    j.chunk = (out + (size_t)threads * 4 - 1) / ((size_t)threads * 4);
    if (j.chunk == 0) j.chunk = 1;
    j.nblocks = (out + j.chunk - 1) / j.chunk;
    pthread_t th[64];
    for (int i = 0; i < threads; i++) pthread_create(&th[i], NULL, scalar_worker, &j);
    for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
    pthread_mutex_destroy(&j.mu);
}
