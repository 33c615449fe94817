/* vnni_baseline.c — restatement of voxrt's AVX-512 VNNI ternary x int8 GEMM (the CPU baseline).
 *
 * TEST INFRASTRUCTURE ONLY: timed by bench.py's cpu_baseline leg on the host cores and checked bit-for-bit
 * against or_gemm_scalar_range by the tests; never part of the product path.
 *
 * Follows crates/voxrt/src/kernels/x86.rs:46-154 (gemm_vnni_range, vnni_tile<T,K>), the Quad16 weight plane of
 * packed.rs:22-33,132-161,275-282 and the row-block split of kernels/mod.rs:324-354 (gemm_ep), with a pthread
 * pool taking blocks from a shared counter in place of rayon's work stealing.
 */
#include "voxrt_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

int or_have_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("fma");
}

/* packed.rs:41 — rows padded to a multiple of 16. */
size_t or_quad16_bytes(size_t out, size_t inp) { return (out + 15) / 16 * 16 * inp; }

/* packed.rs:275-282 put_quad16 and packed.rs:143-149 scales_q: block (rb, quad q) = 64 bytes
 * [w[16rb][4q..4q+4], ..., w[16rb+15][4q..4q+4]]; scales_q[(rb*ng + g)*16 + r%16]; pad rows are zero. */
void or_quad16_pack(const int8_t *rows, size_t out, size_t inp, size_t group, const float *scales, int8_t *wq,
                    float *scales_q) {
    size_t ng = inp / group, nrb = (out + 15) / 16;
    memset(wq, 0, or_quad16_bytes(out, inp));
    memset(scales_q, 0, nrb * ng * 16 * sizeof(float));
    for (size_t r = 0; r < out; r++) {
        for (size_t q = 0; q < inp / 4; q++) memcpy(wq + ((r / 16) * (inp / 4) + q) * 64 + (r % 16) * 4, rows + r * inp + q * 4, 4);
        for (size_t g = 0; g < ng; g++) scales_q[((r / 16) * ng + g) * 16 + r % 16] = scales[r * ng + g];
    }
}

/* x86.rs:22-38 store_block: per-lane epilogue for rows inside [r0, r1). */
static inline void store_block(const float *vals, float *y, size_t out, size_t rbase, size_t r0, size_t r1,
                               size_t t, int ep, float alpha) {
    size_t lo = r0 > rbase ? r0 : rbase, hi = r1 < rbase + 16 ? r1 : rbase + 16;
    for (size_t o = lo; o < hi; o++) y[t * out + o] = or_ep_apply(ep, alpha, y[t * out + o], vals[o - rbase]);
}

/* x86.rs:89-154 vnni_tile<T, K>: T tokens x 16 rows; per group, K independent vpdpbusd accumulators per token over
 * (w ^ 0x80) (unsigned) times 4 broadcast activation bytes; S = acc - 128*gsum; f = fma(cvt(S), xs*sw, f). */
#define VNNI_TARGET __attribute__((target("avx512f,avx512bw,avx512vnni,fma")))
VNNI_TARGET static inline __attribute__((always_inline)) void vnni_tile(int T, int K, const int8_t *wqp, const float *scales_q, size_t out,
                                         size_t inp, size_t group, const int8_t *x, const float *xs,
                                         const int32_t *gsum, float *y, size_t rb, size_t r0, size_t r1, size_t t,
                                         int ep, float alpha) {
    size_t ng = inp / group, qpg = group / 4;
    const int8_t *wb = wqp + rb * (inp / 4) * 64;
    const float *sq = scales_q + rb * ng * 16;
    const __m512i flip = _mm512_set1_epi8((char)0x80);
    __m512 accf[8];
    for (int j = 0; j < T; j++) accf[j] = _mm512_setzero_ps();
    for (size_t gi = 0; gi < ng; gi++) {
        __m512i acc[8][4];
        for (int j = 0; j < T; j++)
            for (int k = 0; k < K; k++) acc[j][k] = _mm512_setzero_si512();
        for (size_t q = gi * qpg; q < (gi + 1) * qpg; q += (size_t)K) {
            for (int k = 0; k < K; k++) {
                __m512i wv = _mm512_xor_si512(_mm512_loadu_si512((const void *)(wb + (q + (size_t)k) * 64)), flip);
                for (int j = 0; j < T; j++) {
                    int32_t xb;
                    memcpy(&xb, x + (t + (size_t)j) * inp + (q + (size_t)k) * 4, 4);
                    acc[j][k] = _mm512_dpbusd_epi32(acc[j][k], wv, _mm512_set1_epi32(xb));
                }
            }
        }
        __m512 sw = _mm512_loadu_ps(sq + gi * 16);
        for (int j = 0; j < T; j++) {
            size_t tok = t + (size_t)j;
            __m512i a = _mm512_setzero_si512();
            for (int k = 0; k < K; k++) a = _mm512_add_epi32(a, acc[j][k]);
            __m512i corr = _mm512_set1_epi32(128 * gsum[tok * ng + gi]);
            __m512 s = _mm512_cvtepi32_ps(_mm512_sub_epi32(a, corr));
            __m512 p = _mm512_mul_ps(_mm512_set1_ps(xs[tok * ng + gi]), sw);
            accf[j] = _mm512_fmadd_ps(s, p, accf[j]);
        }
    }
    int full = rb * 16 >= r0 && rb * 16 + 16 <= r1;
    float vals[16];
    for (int j = 0; j < T; j++) {
        float *dst = y + (t + (size_t)j) * out + rb * 16;
        if (full && ep == OR_EP_STORE) {
            _mm512_storeu_ps(dst, accf[j]);
        } else if (full && ep == OR_EP_ADD_SCALED) {
            _mm512_storeu_ps(dst, _mm512_fmadd_ps(_mm512_set1_ps(alpha), accf[j], _mm512_loadu_ps(dst)));
        } else {
            _mm512_storeu_ps(vals, accf[j]);
            store_block(vals, y, out, rb * 16, r0, r1, t + (size_t)j, ep, alpha);
        }
    }
}

/* x86.rs:46-87 gemm_vnni_range: rows [r0, r1) x tokens [t0, t1); token tiles of 8, 4, then 2 and 1 with split
 * accumulators when group/4 is a multiple of 4. */
VNNI_TARGET void or_gemm_vnni_range(const int8_t *wq, const float *scales_q, size_t out, size_t inp, size_t group,
                                    const int8_t *x, const float *xs, const int32_t *gsum, size_t n, float *y,
                                    size_t r0, size_t r1, size_t t0, size_t t1, int ep, float alpha) {
    (void)n;
    int split = ((group / 4) % 4) == 0;
    for (size_t rb = r0 / 16; rb < (r1 + 15) / 16; rb++) {
        size_t t = t0;
        while (t < t1) {
            size_t left = t1 - t;
            if (left >= 8) {
                vnni_tile(8, 1, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                t += 8;
            } else if (left >= 4) {
                vnni_tile(4, 1, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                t += 4;
            } else if (left >= 2) {
                if (split)
                    vnni_tile(2, 2, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                else
                    vnni_tile(2, 1, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                t += 2;
            } else {
                if (split)
                    vnni_tile(1, 4, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                else
                    vnni_tile(1, 1, wq, scales_q, out, inp, group, x, xs, gsum, y, rb, r0, r1, t, ep, alpha);
                t += 1;
            }
        }
    }
}

/* kernels/mod.rs:324-354 gemm_ep: blocks = threads * mult (VOXRT_GEMM_BLOCKS, default 8), at most out/8, at least
 * 1; chunk = ceil(ceil(out/blocks)/16)*16 rows (Quad16 alignment); each block computes its rows for all tokens. */
typedef struct {
    const int8_t *wq; const float *sq; size_t out, inp, group; const int8_t *x; const float *xs; const int32_t *gsum;
    size_t n; float *y; int ep; float alpha; size_t chunk, nblocks; size_t next; pthread_mutex_t mu;
} vnni_job;

static void *vnni_worker(void *arg) {
    vnni_job *j = (vnni_job *)arg;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        size_t b = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (b >= j->nblocks) return NULL;
        size_t r0 = b * j->chunk, r1 = r0 + j->chunk < j->out ? r0 + j->chunk : j->out;
        or_gemm_vnni_range(j->wq, j->sq, j->out, j->inp, j->group, j->x, j->xs, j->gsum, j->n, j->y, r0, r1, 0,
                           j->n, j->ep, j->alpha);
    }
}

void or_gemm_ep_vnni(const int8_t *wq, const float *scales_q, size_t out, size_t inp, size_t group,
                     const int8_t *x, const float *xs, const int32_t *gsum, size_t n, float *y, int ep, float alpha,
                     int threads, size_t blocks_mult) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (blocks_mult == 0) blocks_mult = 8;
    size_t blocks = (size_t)threads * blocks_mult;
    if (blocks > out / 8) blocks = out / 8;
    if (blocks < 1) blocks = 1;
    size_t chunk = ((out + blocks - 1) / blocks + 15) / 16 * 16;
    vnni_job j = {wq, scales_q, out, inp, group, x, xs, gsum, n, y, ep, alpha, chunk, (out + chunk - 1) / chunk, 0, PTHREAD_MUTEX_INITIALIZER};
    if (threads == 1) {
        vnni_worker(&j);
    } else {
        pthread_t th[256];
        for (int i = 0; i < threads; i++) pthread_create(&th[i], NULL, vnni_worker, &j);
        for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
    }
    pthread_mutex_destroy(&j.mu);
}
