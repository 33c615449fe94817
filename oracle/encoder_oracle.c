/* encoder_oracle.c — CPU restatement of the encoder around the ternary x int8 GEMM (the oracle, continued).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP encoder kernels, never the product path.
 *
 * Restated here (each function cites the reference function it follows):
 *   LayerNorm and its fusion into the int8 quantizer, GLU, depthwise conv with folded BatchNorm and SiLU, the
 *   scaled row exponentials of the softmax, the relative position table, the f32 linear of the subsampling, the
 *   subsampling, the int8 attention core, one FastConformer layer and the whole encoder on the int8 path.
 * Every float operation is one IEEE-rounded step in the reference's order (-ffp-contract=off; Rust never
 * contracts, `mul_add` is fmaf).
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "par.h"
#include "voxrt_oracle.h"

static inline float hsum4(const float a[4]) { return (a[0] + a[1]) + (a[2] + a[3]); } /* tensor.rs:227-229 */

/* tensor.rs:331-363 (row_mean_var_portable): sums over 8-column steps into two 4-lane arrays, hsum4 of the
 * lane pairs, the tail in order; the squares by fma in the same pattern, the tail squares unfused. */
void or_row_mean_var(const float *x, size_t d, float *mean_out, float *var_out) {
    size_t n8 = d / 8 * 8;
    float s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0};
    for (size_t c = 0; c < n8; c += 8)
        for (int l = 0; l < 4; l++) {
            s0[l] += x[c + l];
            s1[l] += x[c + 4 + l];
        }
    float p[4];
    for (int l = 0; l < 4; l++) p[l] = s0[l] + s1[l];
    float sum = hsum4(p);
    for (size_t c = n8; c < d; c++) sum += x[c];
    float mean = sum / (float)d;
    float q0[4] = {0, 0, 0, 0}, q1[4] = {0, 0, 0, 0};
    for (size_t c = 0; c < n8; c += 8)
        for (int l = 0; l < 4; l++) {
            float a = x[c + l] - mean, e = x[c + 4 + l] - mean;
            q0[l] = fmaf(a, a, q0[l]);
            q1[l] = fmaf(e, e, q1[l]);
        }
    for (int l = 0; l < 4; l++) p[l] = q0[l] + q1[l];
    float sq = hsum4(p);
    for (size_t c = n8; c < d; c++) {
        float a = x[c] - mean;
        sq += a * a;
    }
    *mean_out = mean;
    *var_out = sq / (float)d;
}

/* tensor.rs:712-719 (layer_norm_row): eps 1e-5, biased variance, y = ((x - mean) * inv) * g + b unfused. */
static void layer_norm_row(const float *x, const float *g, const float *b, size_t d, float *y) {
    float mean, var;
    or_row_mean_var(x, d, &mean, &var);
    float inv = 1.0f / sqrtf(var + 1e-5f);
    for (size_t k = 0; k < d; k++) y[k] = (x[k] - mean) * inv * g[k] + b[k];
}

typedef struct {
    const float *x, *g, *b;
    size_t d, group;
    float *y;
    int8_t *q;
    float *scales;
    int32_t *gsum;
} ln_ctx;

static void ln_rows(void *c_, size_t lo, size_t hi) {
    ln_ctx *c = (ln_ctx *)c_;
    for (size_t i = lo; i < hi; i++) layer_norm_row(c->x + i * c->d, c->g, c->b, c->d, c->y + i * c->d);
}

/* tensor.rs:700-707 (layer_norm), parallel over rows as par_rows */
void or_layer_norm(const float *x, size_t n, size_t d, const float *g, const float *b, float *y) {
    ln_ctx c = {x, g, b, d, 0, y, NULL, NULL, NULL};
    or_par_for(n, ln_rows, &c);
}

/* ternary_linear.rs:132-155 (prepare_normed, Int8) through packed.rs:315-436 (QuantAct::from_rows): each token's
 * LayerNorm row is quantized per group as it is produced. Same outputs as or_quantize. */
static void lnq_rows(void *c_, size_t lo, size_t hi) {
    ln_ctx *c = (ln_ctx *)c_;
    size_t inp = c->d, group = c->group, ng = inp / group;
    float *row = malloc(inp * sizeof(float));
    for (size_t t = lo; t < hi; t++) {
        layer_norm_row(c->x + t * inp, c->g, c->b, inp, row);
        for (size_t gi = 0; gi < ng; gi++) {
            int8_t *dq = c->q + t * inp + gi * group;
            c->scales[t * ng + gi] = or_quantize_group(row + gi * group, group, dq);
            int32_t s = 0;
            for (size_t k = 0; k < group; k++) s += dq[k];
            if (c->gsum) c->gsum[t * ng + gi] = s;
        }
    }
    free(row);
}

void or_quantize_normed(const float *x, size_t n, size_t inp, size_t group, const float *g, const float *b,
                        int8_t *q, float *scales, int32_t *gsum) {
    ln_ctx c = {x, g, b, inp, group, NULL, q, scales, gsum};
    or_par_for(n, lnq_rows, &c);
}

/* tensor.rs:810-826 (exp_row_scaled_portable): max of v*scale; v = exp_poly(v*scale - max) (two roundings);
 * four lane sums over the quads, (l0 + l1) + (l2 + l3), then the tail in order. Returns the sum. */
float or_exp_row_scaled(float *row, size_t n, float scale) {
    float mx = -INFINITY;
    for (size_t j = 0; j < n; j++) {
        float v = row[j] * scale;
        mx = v > mx ? v : mx;
    }
    float lanes[4] = {0, 0, 0, 0};
    size_t n4 = n / 4 * 4;
    for (size_t j = 0; j < n4; j += 4)
        for (int l = 0; l < 4; l++) {
            float v = or_exp_poly(row[j + l] * scale - mx);
            row[j + l] = v;
            lanes[l] += v;
        }
    float sum = hsum4(lanes);
    for (size_t j = n4; j < n; j++) {
        float v = or_exp_poly(row[j] * scale - mx);
        row[j] = v;
        sum += v;
    }
    return sum;
}

/* encoder.rs:592-600 with tensor.rs:936-940 (glu_row_portable): out = a * sigmoid_fast(b), a = first half. */
typedef struct {
    const float *a, *w, *bias;
    size_t t, d, k;
    float *out;
} rows_ctx;

static void glu_rows(void *c_, size_t lo, size_t hi) {
    rows_ctx *c = (rows_ctx *)c_;
    size_t d = c->d;
    for (size_t i = lo; i < hi; i++)
        for (size_t k = 0; k < d; k++) c->out[i * d + k] = c->a[i * 2 * d + k] * or_sigmoid_fast(c->a[i * 2 * d + d + k]);
}

void or_glu(const float *gbuf, size_t n, size_t d, float *out) {
    rows_ctx c = {gbuf, NULL, NULL, n, d, 0, out};
    or_par_for(n, glu_rows, &c);
}

/* encoder.rs:548-573 (ConvModule::load): BatchNorm(eval) folded into the depthwise taps, tap-major [k][d]:
 * s = gamma / sqrt(var + 1e-5), w' = w * s, bias = beta - mean * s. dw is [d][k] (PyTorch [d, 1, k]). */
void or_fold_bn(const float *dw, const float *gamma, const float *beta, const float *mean, const float *var,
                size_t d, size_t k, float *dw_t, float *dw_bias) {
    for (size_t c = 0; c < d; c++) {
        float s = gamma[c] / sqrtf(var[c] + 1e-5f);
        for (size_t kk = 0; kk < k; kk++) dw_t[kk * d + c] = dw[c * k + kk] * s;
        dw_bias[c] = beta[c] - mean[c] * s;
    }
}

/* encoder.rs:602-624: row i = bias, + w[kk] * a[i + kk - pad] for each tap in order (unfused, taps outside
 * [0, t) skipped), then silu_fast per element (tensor.rs:962-973). */
static void dwconv_rows(void *c_, size_t lo, size_t hi) {
    rows_ctx *c = (rows_ctx *)c_;
    const float *a = c->a, *dw_t = c->w, *dw_bias = c->bias;
    size_t t = c->t, d = c->d, k = c->k, pad = (k - 1) / 2;
    float *out = c->out;
    for (size_t i = lo; i < hi; i++) {
        float *row = out + i * d;
        memcpy(row, dw_bias, d * sizeof(float));
        for (size_t kk = 0; kk < k; kk++) {
            size_t j = i + kk;
            if (j >= pad && j - pad < t) {
                const float *w = dw_t + kk * d, *aj = a + (j - pad) * d;
                for (size_t c = 0; c < d; c++) row[c] += w[c] * aj[c];
            }
        }
        for (size_t c = 0; c < d; c++) row[c] = or_silu_fast(row[c]);
    }
}

void or_dwconv_bn_silu(const float *a, size_t t, size_t d, size_t k, const float *dw_t, const float *dw_bias,
                       float *out) {
    rows_ctx c = {a, dw_t, dw_bias, t, d, k, out};
    or_par_for(t, dwconv_rows, &c);
}

/* encoder.rs:760-776 (rel_pos_table): [2t-1][d], positions t-1 .. -(t-1), (sin, cos) interleaved per frequency,
 * inv_i = 1 / powf(10000, 2i/d). The reference calls the libm crate's powf/sinf/cosf; these are the C library's,
 * which may differ from it by an ulp. */
void or_rel_pos_table(size_t t, size_t d, float *out) {
    size_t np = 2 * t - 1, half = d / 2;
    float *inv = malloc(half * sizeof(float));
    for (size_t i = 0; i < half; i++) inv[i] = 1.0f / powf(10000.0f, 2.0f * (float)i / (float)d);
    for (size_t r = 0; r < np; r++) {
        float pos = (float)((int64_t)t - 1 - (int64_t)r);
        for (size_t i = 0; i < half; i++) {
            float f = inv[i] * pos;
            out[r * d + 2 * i] = sinf(f);
            out[r * d + 2 * i + 1] = cosf(f);
        }
    }
    free(inv);
}

/* tensor.rs:78-95 (dot): 8 unfused lane sums, summed in order, then the tail in order. */
static float dot8(const float *a, const float *b, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t n8 = n / 8 * 8;
    for (size_t c = 0; c < n8; c += 8)
        for (int k = 0; k < 8; k++) acc[k] += a[c + k] * b[c + k];
    float s = acc[0];
    for (int k = 1; k < 8; k++) s += acc[k];
    for (size_t c = n8; c < n; c++) s += a[c] * b[c];
    return s;
}

/* tensor.rs:263-282 (dot_lanes8): fused lanes over 8-column steps, lane-wise a + b, hsum4, the tail in order. */
static float dot_lanes8(const float *x, const float *w, size_t n) {
    size_t n8 = n / 8 * 8;
    float a[4] = {0, 0, 0, 0}, bb[4] = {0, 0, 0, 0};
    for (size_t c = 0; c < n8; c += 8)
        for (int l = 0; l < 4; l++) {
            a[l] = fmaf(x[c + l], w[c + l], a[l]);
            bb[l] = fmaf(x[c + 4 + l], w[c + 4 + l], bb[l]);
        }
    float p[4];
    for (int l = 0; l < 4; l++) p[l] = a[l] + bb[l];
    float r = hsum4(p);
    for (size_t c = n8; c < n; c++) r += x[c] * w[c];
    return r;
}

typedef struct {
    const float *x, *w, *b;
    size_t in_f, out_f;
    float *y;
} lin_ctx;

static void linear_rows(void *c_, size_t lo, size_t hi);

/* tensor.rs:98-127 (linear): one token -> gemv_portable (tensor.rs:284-303: 4-row blocks by dot_lanes8, the
 * leftover rows by dot); otherwise tile_rows_portable (tensor.rs:233-261) for every token: four fused lanes over
 * 4-column steps, the tail unfused, y = (hsum4 + tail) + bias. */
void or_linear_f32(const float *x, size_t n, size_t in_f, const float *w, const float *b, size_t out_f, float *y) {
    if (n == 1) {
        size_t o4 = out_f / 4 * 4;
        for (size_t o = 0; o < out_f; o++) {
            const float *wr = w + o * in_f;
            float r = o < o4 ? dot_lanes8(x, wr, in_f) : dot8(x, wr, in_f);
            y[o] = r + (b ? b[o] : 0.0f);
        }
        return;
    }
    lin_ctx lc = {x, w, b, in_f, out_f, y};
    or_par_for(n, linear_rows, &lc);
}

static void linear_rows(void *c_, size_t lo, size_t hi) {
    lin_ctx *lc = (lin_ctx *)c_;
    const float *x = lc->x, *w = lc->w, *b = lc->b;
    size_t in_f = lc->in_f, out_f = lc->out_f;
    float *y = lc->y;
    size_t c4 = in_f / 4 * 4;
    for (size_t tk = lo; tk < hi; tk++) {
        const float *xr = x + tk * in_f;
        for (size_t o = 0; o < out_f; o++) {
            const float *wr = w + o * in_f;
            float acc[4] = {0, 0, 0, 0};
            for (size_t c = 0; c < c4; c += 4)
                for (int l = 0; l < 4; l++) acc[l] = fmaf(wr[c + l], xr[c + l], acc[l]);
            float tail = 0.0f;
            for (size_t c = c4; c < in_f; c++) tail += wr[c] * xr[c];
            y[tk * out_f + o] = hsum4(acc) + tail + (b ? b[o] : 0.0f);
        }
    }
}

/* subsampling.rs:25-28 */
static size_t out_len(size_t n, size_t k, size_t s, size_t p) { return (n + 2 * p - k) / s + 1; }

size_t or_subsampling_frames(size_t t, size_t k, size_t s) {
    size_t p = (k - 1) / 2, n = t;
    for (int i = 0; i < 3; i++) n = out_len(n, k, s, p);
    return n;
}

typedef struct {
    const float *in, *w, *b;
    size_t tin, fin, c, k, s, p, tout, fout;
    float *out;
} conv_ctx;

/* stage 0 rows [lo, hi) of the output time axis */
static void conv0_rows(void *c_, size_t lo, size_t hi) {
    conv_ctx *q = (conv_ctx *)c_;
    size_t c = q->c, k = q->k, s = q->s, p = q->p;
    for (size_t ot = lo; ot < hi; ot++)
        for (size_t of = 0; of < q->fout; of++) {
            float *o = q->out + (ot * q->fout + of) * c;
            memcpy(o, q->b, c * sizeof(float));
            for (size_t kt = 0; kt < k; kt++) {
                int64_t it = (int64_t)(ot * s + kt) - (int64_t)p;
                if (it < 0 || it >= (int64_t)q->tin) continue;
                for (size_t kf = 0; kf < k; kf++) {
                    int64_t i_f = (int64_t)(of * s + kf) - (int64_t)p;
                    if (i_f < 0 || i_f >= (int64_t)q->fin) continue;
                    float v = q->in[(size_t)it * q->fin + (size_t)i_f];
                    const float *wt = q->w + (kt * k + kf) * c;
                    for (size_t ch = 0; ch < c; ch++) o[ch] += wt[ch] * v;
                }
            }
            for (size_t ch = 0; ch < c; ch++) o[ch] = o[ch] > 0.0f ? o[ch] : 0.0f;
        }
}

/* depthwise stage rows [lo, hi) */
static void dw_rows(void *c_, size_t lo, size_t hi) {
    conv_ctx *q = (conv_ctx *)c_;
    size_t c = q->c, k = q->k, s = q->s, p = q->p;
    for (size_t ot = lo; ot < hi; ot++)
        for (size_t of = 0; of < q->fout; of++) {
            float *o = q->out + (ot * q->fout + of) * c;
            memcpy(o, q->b, c * sizeof(float));
            for (size_t kt = 0; kt < k; kt++) {
                int64_t it = (int64_t)(ot * s + kt) - (int64_t)p;
                if (it < 0 || it >= (int64_t)q->tin) continue;
                for (size_t kf = 0; kf < k; kf++) {
                    int64_t i_f = (int64_t)(of * s + kf) - (int64_t)p;
                    if (i_f < 0 || i_f >= (int64_t)q->fin) continue;
                    const float *xi = q->in + ((size_t)it * q->fin + (size_t)i_f) * c;
                    const float *wt = q->w + (kt * k + kf) * c;
                    for (size_t ch = 0; ch < c; ch++) o[ch] += wt[ch] * xi[ch];
                }
            }
        }
}

/* subsampling.rs:124-204 (Subsampling::forward), channels-last [T, F, C]:
 *   stage 0: 3x3 stride-s conv 1 -> C (bias first, taps kt-major then kf, unfused), ReLU;
 *   two stages of depthwise 3x3 stride-s (no activation), pointwise C -> C by the f32 linear (+ bias), ReLU;
 *   the [t3, f3*C] flatten through the final linear (columns already permuted to channels-last order).
 * Weights as loaded by subsampling.rs:32-104: conv0_w [k*k][C], dw_w [2][k*k][C], pw_w [2][C][C] (out, in),
 * lin_w [d][f3*C]. Returns the output frame count; out is [t3][d]. */
size_t or_subsampling(const float *feats, size_t t, size_t n_mels, size_t c, size_t k, size_t s, const float *conv0_w,
                      const float *conv0_b, const float *dw_w, const float *dw_b, const float *pw_w,
                      const float *pw_b, const float *lin_w, const float *lin_b, size_t d_model, float *out) {
    size_t p = (k - 1) / 2;
    size_t t1 = out_len(t, k, s, p), f1 = out_len(n_mels, k, s, p);
    float *x = calloc(t1 * f1 * c, sizeof(float));
    conv_ctx cc0 = {feats, conv0_w, conv0_b, t, n_mels, c, k, s, p, t1, f1, x};
    or_par_for(t1, conv0_rows, &cc0);
    size_t tc = t1, fc = f1;
    for (int stage = 0; stage < 2; stage++) {
        size_t t2 = out_len(tc, k, s, p), f2 = out_len(fc, k, s, p);
        const float *w = dw_w + (size_t)stage * k * k * c, *b = dw_b + (size_t)stage * c;
        float *y = calloc(t2 * f2 * c, sizeof(float));
        conv_ctx cd = {x, w, b, tc, fc, c, k, s, p, t2, f2, y};
        or_par_for(t2, dw_rows, &cd);
        size_t n_pos = t2 * f2;
        float *z = malloc(n_pos * c * sizeof(float));
        or_linear_f32(y, n_pos, c, pw_w + (size_t)stage * c * c, pw_b + (size_t)stage * c, c, z);
        for (size_t i = 0; i < n_pos * c; i++) z[i] = z[i] > 0.0f ? z[i] : 0.0f;
        free(y);
        free(x);
        x = z;
        tc = t2;
        fc = f2;
    }
    or_linear_f32(x, tc, fc * c, lin_w, lin_b, d_model, out);
    free(x);
    return tc;
}

/* ---------------------------------------------------------------------------------------- int8 attention core */

static int32_t idot(const int8_t *a, const int8_t *b, size_t n) {
    int32_t s = 0;
    for (size_t c = 0; c < n; c++) s += (int32_t)a[c] * (int32_t)b[c];
    return s;
}

typedef struct {
    const float *qkv, *rel_k, *bias_u, *bias_v;
    size_t t, d, h;
    float scaling;
    float *ctx;
} attn_ctx;

static void attn_heads(void *c_, size_t lo, size_t hi) {
    attn_ctx *A = (attn_ctx *)c_;
    const float *qkv = A->qkv, *rel_k = A->rel_k;
    size_t t = A->t, d = A->d, h = A->h;
    float *ctx = A->ctx;
    size_t dh = d / h, np = 2 * t - 1, t2 = (t + 1) / 2 * 2, np2 = (np + 1) / 2 * 2, t16 = (t + 15) / 16 * 16;
    size_t d3 = 3 * d;
    int8_t *qu = malloc(t * dh), *qv = malloc(t * dh), *kq = malloc(t2 * dh), *rq = malloc(np2 * dh);
    int8_t *vq = malloc(dh * t16), *pq = malloc(t16);
    float *qus = malloc(t * 4), *qvs = malloc(t * 4), *ks = malloc(t2 * 4), *rs = malloc(np2 * 4), *vs = malloc(dh * 4);
    float *tmp = malloc((t16 > dh ? t16 : dh) * sizeof(float)), *row = malloc(t16 * sizeof(float));
    for (size_t head = lo; head < hi; head++) {
        const float *bu = A->bias_u + head * dh, *bv = A->bias_v + head * dh;
        for (size_t i = 0; i < t; i++) {
            const float *qi = qkv + i * d3 + head * dh;
            for (size_t c = 0; c < dh; c++) tmp[c] = qi[c] + bu[c];
            qus[i] = or_quantize_group(tmp, dh, qu + i * dh);
            for (size_t c = 0; c < dh; c++) tmp[c] = qi[c] + bv[c];
            qvs[i] = or_quantize_group(tmp, dh, qv + i * dh);
        }
        for (size_t j = 0; j < t2; j++) {
            if (j < t)
                memcpy(tmp, qkv + j * d3 + d + head * dh, dh * sizeof(float));
            else
                memset(tmp, 0, dh * sizeof(float));
            ks[j] = or_quantize_group(tmp, dh, kq + j * dh);
        }
        for (size_t p = 0; p < np2; p++) {
            if (p < np)
                memcpy(tmp, rel_k + p * d + head * dh, dh * sizeof(float));
            else
                memset(tmp, 0, dh * sizeof(float));
            rs[p] = or_quantize_group(tmp, dh, rq + p * dh);
        }
        for (size_t c = 0; c < dh; c++) {
            for (size_t i = 0; i < t16; i++) tmp[i] = i < t ? qkv[i * d3 + 2 * d + head * dh + c] : 0.0f;
            vs[c] = or_quantize_group(tmp, t16, vq + c * t16);
        }
        for (size_t i = 0; i < t; i++) {
            for (size_t j = 0; j < t; j++) {
                size_t p = t - 1 - i + j;
                float s1 = fmaf((float)idot(qu + i * dh, kq + j * dh, dh), qus[i] * ks[j], 0.0f);
                float s2 = fmaf((float)idot(qv + i * dh, rq + p * dh, dh), qvs[i] * rs[p], 0.0f);
                row[j] = s1 + s2;
            }
            float inv = 1.0f / or_exp_row_scaled(row, t, A->scaling);
            for (size_t j = t; j < t16; j++) row[j] = 0.0f;
            float ps = or_quantize_group(row, t16, pq);
            ps = ps * inv;
            for (size_t c = 0; c < dh; c++)
                ctx[i * d + head * dh + c] = fmaf((float)idot(pq, vq + c * t16, t16), ps * vs[c], 0.0f);
        }
    }
    free(qu); free(qv); free(kq); free(rq); free(vq); free(pq);
    free(qus); free(qvs); free(ks); free(rs); free(vs); free(tmp); free(row);
}

/* encoder.rs:317-534 (attn_core_int8) for all heads. qkv [t][3d] (q | k | v), rel_k [2t-1][d]; ctx [t][d].
 * Per head: q + bias_u and q + bias_v quantized per token (one group = dh), keys [t2][dh], relative positions
 * [np2][dh] and vT [dh][t16] quantized per row (one group each; rows past the end are zero); the content score
 * S1[i][j] and the position score S2[i][p] are single-group int8 GEMM outputs fma((float)S, xs * ws, 0)
 * (kernels/mod.rs:166-210); score = S1[i][j] + S2[i][t-1-i+j]; exp_row_scaled with `scaling`; the row of
 * exponentials, zero-padded to t16, is quantized in one group and its scale multiplied by 1/sum; ctx is the
 * single-group int8 GEMM of those probabilities with vT. Heads run in parallel. */
void or_attn_core_int8(const float *qkv, const float *rel_k, size_t t, size_t d, size_t h, const float *bias_u,
                       const float *bias_v, float scaling, float *ctx) {
    attn_ctx A = {qkv, rel_k, bias_u, bias_v, t, d, h, scaling, ctx};
    or_par_for(h, attn_heads, &A);
}

/* ------------------------------------------------------------------------------------------ encoder (int8) */

/* One ternary linear on the int8 path: quantized activations (q, scales, gsum as or_quantize), y = ep(y, x.w^T).
 * The AVX-512 VNNI restatement when the host has it (bit-identical to the scalar kernel), else the scalar one. */
typedef struct {
    const int8_t *w;
    const float *ws;
    size_t out, inp, group;
    int8_t *wq;
    float *sq;
    int own;
} tlin;

static void tlin_init(tlin *l, const int8_t *w, const float *ws, size_t out, size_t inp, size_t group,
                      const int8_t *wq_pre, const float *sq_pre) {
    l->w = w;
    l->ws = ws;
    l->out = out;
    l->inp = inp;
    l->group = group;
    l->wq = NULL;
    l->sq = NULL;
    l->own = 0;
    if (wq_pre && sq_pre && or_have_vnni()) { /* packed at load time, as TernaryLinear::load does */
        l->wq = (int8_t *)wq_pre;
        l->sq = (float *)sq_pre;
        return;
    }
    if (or_have_vnni()) {
        l->own = 1;
        l->wq = malloc(or_quad16_bytes(out, inp));
        l->sq = malloc((out + 15) / 16 * 16 * (inp / group) * sizeof(float));
        or_quad16_pack(w, out, inp, group, ws, l->wq, l->sq);
    }
}

static void tlin_free(tlin *l) {
    if (l->own) {
        free(l->wq);
        free(l->sq);
    }
}

typedef struct {
    int8_t *q;
    float *s;
    int32_t *g;
    size_t n, inp, group;
} qact;

static void qact_alloc(qact *a, size_t n, size_t inp, size_t group) {
    a->q = malloc(n * inp);
    a->s = malloc(n * (inp / group) * sizeof(float));
    a->g = malloc(n * (inp / group) * sizeof(int32_t));
    a->n = n;
    a->inp = inp;
    a->group = group;
}

static void qact_free(qact *a) {
    free(a->q);
    free(a->s);
    free(a->g);
}

static void tlin_gemm(const tlin *l, const qact *a, float *y, int ep, float alpha, int threads) {
    if (l->wq)
        or_gemm_ep_vnni(l->wq, l->sq, l->out, l->inp, l->group, a->q, a->s, a->g, a->n, y, ep, alpha, threads, 8);
    else
        or_gemm_scalar_mt(l->w, l->ws, l->out, l->inp, l->group, a->q, a->s, a->n, y, ep, alpha, NULL, threads);
}

/* Parameter table of one layer (pointer array, in this order):
 *   0..8   ternary trits [out][inp] of ff1.linear1, ff1.linear2, q|k|v (stacked), o_proj, relative_k_proj,
 *          pointwise_conv1, pointwise_conv2, ff2.linear1, ff2.linear2
 *   9..17  their scales f32 [out][inp/group], same order
 *   18..27 LayerNorm (g, b) of norm_feed_forward1, norm_self_att, norm_conv, norm_feed_forward2, norm_out
 *   28, 29 bias_u, bias_v [heads][dh]
 *   30, 31 depthwise taps [k][d] and bias [d] with BatchNorm folded (or_fold_bn)
 *   32..49 optional (NULL: packed per call) Quad16 weights and scales of the 9 linears (or_quad16_pack), as pairs */
enum { P_W = 0, P_S = 9, P_LN = 18, P_BU = 28, P_BV = 29, P_DW = 30, P_DWB = 31, P_Q16 = 32, P_COUNT = 50 };

/* encoder.rs:706-756 (ConformerLayer::forward_profiled), int8 path, in place on x [t][d]:
 *   x += 0.5 * ff1.w2(quant(silu(ff1.w1(ln_quant(x)))))            (encoder.rs:79-94)
 *   x += o_proj(quant(attn_core(w_qkv(ln_quant(x)), w_pos(quant(pos)))))   (encoder.rs:138-191)
 *   x += pw2(quant(silu(bn(dw(glu(pw1(ln_quant(x))))))))            (encoder.rs:576-628)
 *   x += 0.5 * ff2(...) ; x = LN_out(x).  pos_emb is [2t-1][d]. */
static void feed_forward(float *x, size_t t, size_t d, size_t ff, size_t group, const tlin *w1, const tlin *w2,
                         const float *g, const float *b, qact *a_d, qact *a_ff, float *hbuf, int threads) {
    or_quantize_normed(x, t, d, group, g, b, a_d->q, a_d->s, a_d->g);
    memset(hbuf, 0, t * ff * sizeof(float));
    tlin_gemm(w1, a_d, hbuf, OR_EP_SILU, 0.0f, threads);
    or_quantize(hbuf, t, ff, group, a_ff->q, a_ff->s, a_ff->g);
    tlin_gemm(w2, a_ff, x, OR_EP_ADD_SCALED, 0.5f, threads);
}

void or_conformer_layer(float *x, size_t t, const float *pos_emb, const void *const *p, size_t d, size_t heads,
                        size_t ff, size_t kconv, size_t group, int threads) {
    size_t outs[9] = {ff, d, 3 * d, d, d, 2 * d, d, ff, d}, inps[9] = {d, ff, d, d, d, d, d, d, ff};
    tlin L[9];
    for (int i = 0; i < 9; i++)
        tlin_init(&L[i], (const int8_t *)p[P_W + i], (const float *)p[P_S + i], outs[i], inps[i], group,
                  (const int8_t *)p[P_Q16 + 2 * i], (const float *)p[P_Q16 + 2 * i + 1]);
    const float *ln_g[5], *ln_b[5];
    for (int i = 0; i < 5; i++) {
        ln_g[i] = (const float *)p[P_LN + 2 * i];
        ln_b[i] = (const float *)p[P_LN + 2 * i + 1];
    }
    size_t np = 2 * t - 1, dh = d / heads;
    qact a_d, a_ff, a_pos;
    qact_alloc(&a_d, t, d, group);
    qact_alloc(&a_ff, t, ff, group);
    qact_alloc(&a_pos, np, d, group);
    float *hbuf = malloc(t * ff * sizeof(float)), *qkv = malloc(t * 3 * d * sizeof(float));
    float *rel_k = malloc(np * d * sizeof(float)), *ctx = malloc(t * d * sizeof(float));
    float *g2 = malloc(t * 2 * d * sizeof(float)), *ga = malloc(t * d * sizeof(float));
    float *hb = malloc(t * d * sizeof(float)), *tmp = malloc(t * d * sizeof(float));
    /* feed-forward 1 (encoder.rs:79-94): x += 0.5 * w2(quant(silu(w1(ln_quant(x))))) */
    feed_forward(x, t, d, ff, group, &L[0], &L[1], ln_g[0], ln_b[0], &a_d, &a_ff, hbuf, threads);
    /* attention (encoder.rs:138-191): x += o_proj(quant(attn_core(w_qkv(ln_quant(x)), w_pos(quant(pos))))) */
    or_quantize_normed(x, t, d, group, ln_g[1], ln_b[1], a_d.q, a_d.s, a_d.g);
    memset(qkv, 0, t * 3 * d * sizeof(float));
    tlin_gemm(&L[2], &a_d, qkv, OR_EP_STORE, 0.0f, threads);
    or_quantize(pos_emb, np, d, group, a_pos.q, a_pos.s, a_pos.g);
    memset(rel_k, 0, np * d * sizeof(float));
    tlin_gemm(&L[4], &a_pos, rel_k, OR_EP_STORE, 0.0f, threads);
    or_attn_core_int8(qkv, rel_k, t, d, heads, (const float *)p[P_BU], (const float *)p[P_BV],
                      1.0f / sqrtf((float)dh), ctx);
    or_quantize(ctx, t, d, group, a_d.q, a_d.s, a_d.g);
    tlin_gemm(&L[3], &a_d, x, OR_EP_ADD_SCALED, 1.0f, threads);
    /* convolution module (encoder.rs:576-628): x += pw2(quant(silu(bn(dw(glu(pw1(ln_quant(x)))))))) */
    or_quantize_normed(x, t, d, group, ln_g[2], ln_b[2], a_d.q, a_d.s, a_d.g);
    memset(g2, 0, t * 2 * d * sizeof(float));
    tlin_gemm(&L[5], &a_d, g2, OR_EP_STORE, 0.0f, threads);
    or_glu(g2, t, d, ga);
    or_dwconv_bn_silu(ga, t, d, kconv, (const float *)p[P_DW], (const float *)p[P_DWB], hb);
    or_quantize(hb, t, d, group, a_d.q, a_d.s, a_d.g);
    tlin_gemm(&L[6], &a_d, x, OR_EP_ADD_SCALED, 1.0f, threads);
    /* feed-forward 2, then norm_out (encoder.rs:744-755) */
    feed_forward(x, t, d, ff, group, &L[7], &L[8], ln_g[3], ln_b[3], &a_d, &a_ff, hbuf, threads);
    or_layer_norm(x, t, d, ln_g[4], ln_b[4], tmp);
    memcpy(x, tmp, t * d * sizeof(float));
    qact_free(&a_d);
    qact_free(&a_ff);
    qact_free(&a_pos);
    free(hbuf); free(qkv); free(rel_k); free(ctx); free(g2); free(ga); free(hb); free(tmp);
    for (int i = 0; i < 9; i++) tlin_free(&L[i]);
}
