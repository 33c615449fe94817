/* avx2_baseline.c — restatement of voxrt's AVX2 ternary x int8 GEMM (the reference's second x86 CPU path).
 *
 * TEST INFRASTRUCTURE ONLY: timed by bench.py as a CPU figure and checked bit-for-bit against
 * or_gemm_scalar_range by the tests; never part of the product path.
 *
 * Follows crates/voxrt/src/kernels/x86.rs:163-290 (gemm_avx2_range, avx2_tile<T, TERN>) on the Quad16 weight plane
 * of packed.rs:22-33,132-161,275-282 (the same plane as the VNNI restatement):
 *   - token tiles of 4, then 2, then 1; per tile 16 rows as two 8-lane halves;
 *   - ternary weights: u = w + 1 in {0, 1, 2} times 4 broadcast activation bytes by vpmaddubsw, summed in int16
 *     over the whole group (|sum| <= 2*127*2 per quad and lane, so group <= 256 cannot overflow), widened to int32
 *     by vpmaddwd with ones, minus the activation code sum gsum;
 *   - int8 weights: |w| times sign(x, w) by vpmaddubsw, widened by vpmaddwd with ones each quad, int32 sums;
 *   - per group f = fma(cvt(S), xs * sw, f); the epilogue as store_block (x86.rs:22-38).
 */
#include "voxrt_oracle.h"

#include <immintrin.h>
#include <string.h>

int or_have_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

static inline void avx2_store_block(const float *vals, float *y, size_t out, size_t rbase, size_t r0, size_t r1,
                                    size_t t, int ep, float alpha) {
    size_t lo = r0 > rbase ? r0 : rbase, hi = r1 < rbase + 16 ? r1 : rbase + 16;
    for (size_t o = lo; o < hi; o++) y[t * out + o] = or_ep_apply(ep, alpha, y[t * out + o], vals[o - rbase]);
}

#define AVX2_TARGET __attribute__((target("avx2,fma")))
AVX2_TARGET static inline __attribute__((always_inline)) void avx2_tile(int T, int tern, const int8_t *wqp,
                                                                      const float *scales_q, size_t out, size_t inp,
                                                                      size_t group, const int8_t *x, const float *xs,
                                                                      const int32_t *gsum, float *y, size_t rb,
                                                                      size_t r0, size_t r1, size_t t, int ep,
                                                                      float alpha) {
    const size_t ng = inp / group, qpg = group / 4;
    const int8_t *wb = wqp + rb * (inp / 4) * 64;
    const float *sq = scales_q + rb * ng * 16;
    const __m256i one8 = _mm256_set1_epi8(1), one16 = _mm256_set1_epi16(1);
    __m256 f[4][2];
    for (int j = 0; j < T; j++) f[j][0] = f[j][1] = _mm256_setzero_ps();
    for (size_t gi = 0; gi < ng; gi++) {
        __m256i s[4][2];
        for (int j = 0; j < T; j++) s[j][0] = s[j][1] = _mm256_setzero_si256();
        for (size_t q = gi * qpg; q < (gi + 1) * qpg; q++) {
            const __m256i lo = _mm256_loadu_si256((const __m256i *)(wb + q * 64));
            const __m256i hi = _mm256_loadu_si256((const __m256i *)(wb + q * 64 + 32));
            for (int j = 0; j < T; j++) {
                int32_t xb4;
                memcpy(&xb4, x + (t + (size_t)j) * inp + q * 4, 4);
                const __m256i xb = _mm256_set1_epi32(xb4);
                if (tern) {
                    s[j][0] = _mm256_add_epi16(s[j][0], _mm256_maddubs_epi16(_mm256_add_epi8(lo, one8), xb));
                    s[j][1] = _mm256_add_epi16(s[j][1], _mm256_maddubs_epi16(_mm256_add_epi8(hi, one8), xb));
                } else {
                    const __m256i p0 = _mm256_maddubs_epi16(_mm256_abs_epi8(lo), _mm256_sign_epi8(xb, lo));
                    const __m256i p1 = _mm256_maddubs_epi16(_mm256_abs_epi8(hi), _mm256_sign_epi8(xb, hi));
                    s[j][0] = _mm256_add_epi32(s[j][0], _mm256_madd_epi16(p0, one16));
                    s[j][1] = _mm256_add_epi32(s[j][1], _mm256_madd_epi16(p1, one16));
                }
            }
        }
        const __m256 sw0 = _mm256_loadu_ps(sq + gi * 16), sw1 = _mm256_loadu_ps(sq + gi * 16 + 8);
        for (int j = 0; j < T; j++) {
            const size_t tok = t + (size_t)j;
            const __m256 sx = _mm256_set1_ps(xs[tok * ng + gi]);
            const __m256i corr = _mm256_set1_epi32(gsum[tok * ng + gi]);
            for (int h = 0; h < 2; h++) {
                const __m256i S = tern ? _mm256_sub_epi32(_mm256_madd_epi16(s[j][h], one16), corr) : s[j][h];
                f[j][h] = _mm256_fmadd_ps(_mm256_cvtepi32_ps(S), _mm256_mul_ps(sx, h ? sw1 : sw0), f[j][h]);
            }
        }
    }
    const int full = rb * 16 >= r0 && rb * 16 + 16 <= r1;
    float vals[16];
    for (int j = 0; j < T; j++) {
        float *dst = y + (t + (size_t)j) * out + rb * 16;
        if (full && ep == OR_EP_STORE) {
            _mm256_storeu_ps(dst, f[j][0]);
            _mm256_storeu_ps(dst + 8, f[j][1]);
        } else if (full && ep == OR_EP_ADD_SCALED) {
            const __m256 a = _mm256_set1_ps(alpha);
            _mm256_storeu_ps(dst, _mm256_fmadd_ps(a, f[j][0], _mm256_loadu_ps(dst)));
            _mm256_storeu_ps(dst + 8, _mm256_fmadd_ps(a, f[j][1], _mm256_loadu_ps(dst + 8)));
        } else {
            _mm256_storeu_ps(vals, f[j][0]);
            _mm256_storeu_ps(vals + 8, f[j][1]);
            avx2_store_block(vals, y, out, rb * 16, r0, r1, t + (size_t)j, ep, alpha);
        }
    }
}

/* x86.rs:163-197 gemm_avx2_range: rows [r0, r1) x tokens [t0, t1), token tiles of 4, 2 and 1. Returns -1 without
 * writing when ternary weights come with group > 256 (the int16 sums could overflow; the reference's kernel
 * selection, kernels/mod.rs:326-328, then picks another kernel), else 0. */
AVX2_TARGET int or_gemm_avx2_range(const int8_t *wq, const float *scales_q, size_t out, size_t inp, size_t group,
                                   int ternary, const int8_t *x, const float *xs, const int32_t *gsum, size_t n,
                                   float *y, size_t r0, size_t r1, size_t t0, size_t t1, int ep, float alpha) {
    (void)n;
    if (ternary && group > 256) return -1;
    for (size_t rb = r0 / 16; rb < (r1 + 15) / 16; rb++) {
        size_t t = t0;
        while (t < t1) {
            const size_t left = t1 - t;
            const int T = left >= 4 ? 4 : left >= 2 ? 2 : 1;
            if (ternary) {
                if (T == 4) avx2_tile(4, 1, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                else if (T == 2) avx2_tile(2, 1, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                else avx2_tile(1, 1, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
            } else {
                if (T == 4) avx2_tile(4, 0, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                else if (T == 2) avx2_tile(2, 0, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                else avx2_tile(1, 0, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
            }
            t += (size_t)T;
        }
    }
    return 0;
}
