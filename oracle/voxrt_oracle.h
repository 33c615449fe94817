/* voxrt_oracle.h — CPU restatement of voxrt's ternary x int8 GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels in voxrt_amd/: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, never the product path.
 *
 * Every function restates one reference function (Rust, crates/voxrt/src/...), cited at its definition. The
 * floating-point steps are written out one IEEE operation at a time (no contraction: build with
 * -ffp-contract=off), so the results are bit-identical to the reference's scalar kernel.
 *
 * Pinning (what checks each function, besides restating its formula):
 *   or_unpack_row / or_pack_row / or_dequant_matrix : the reference's stored fixtures
 *       (crates/voxrt/tests/fixtures, copied to tests/golden/fixtures), the known answer 196 -> [0,1,-1,0,1],
 *       ragged round trips, every byte < 243.
 *   or_f16_to_f32 / or_f32_to_f16 : numpy's IEEE binary16 conversion on all 65536 codes / many f32 values.
 *   or_quantize_group / or_quantize : brute-force numpy restatement with np.rint (half-to-even) on .5 ties.
 *   or_gemm_scalar_range : numpy int64 matmul of the group sums; fp32 fold recomputed with np.float32 FMA-free
 *       steps plus math.fma; the known answer all +1 trits x 127 -> 4096*127 (tests/kernels.rs:176-200).
 *   or_exp_poly : relative error < 3e-7 against exp in double (tensor.rs:1018-1030).
 *   or_lcg : the numpy jump-ahead generator (voxrt_amd/synth.py) must reproduce its stream exactly.
 *   or_gemm_vnni_range (CPU baseline) : bit-identical to or_gemm_scalar_range on the x86_kernels.rs grid.
 *   or_gemm_avx2_range (CPU, AVX2)     : bit-identical to or_gemm_scalar_range on the same grid.
 *
 * Encoder side (encoder_oracle.c):
 *   or_row_mean_var / or_layer_norm : float64 LayerNorm within 1e-5; constant rows give exactly b; a numpy float32
 *       walk of the same lane order on rows with tails.
 *   or_quantize_normed : equals or_quantize(or_layer_norm(x)) element for element.
 *   or_exp_row_scaled : every element within 3e-7 of exp in float64, the arg-max element exactly 1, the sum within
 *       1e-6 of the float64 sum.
 *   or_glu / or_dwconv_bn_silu / or_fold_bn : float64 a*sigmoid(b); float64 depthwise conv with the unfolded
 *       BatchNorm and SiLU (torch conv1d).
 *   or_rel_pos_table : float64 sin/cos within 1e-6 (ulp-level agreement with the libm crate is parity unpinned).
 *   or_linear_f32 : float64 matmul within 1e-5 relative; a numpy float32 walk of the lane order.
 *   or_subsampling : torch float64 conv2d / depthwise conv2d / linear on the [T, F] input (NCHW) within 1e-4.
 *   or_attn_core_int8 : exact int32 score sums (int64 matmul), float64 relative-position softmax attention within
 *       the int8 quantization error, the position band checked by a one-hot relative table.
 *   or_conformer_layer : equals the composition of the pinned pieces above, called one by one.
 */
#ifndef VOXRT_ORACLE_H
#define VOXRT_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_EP_STORE = 0, OR_EP_SILU = 1, OR_EP_ADD_SCALED = 2 };

uint32_t or_lcg(uint64_t *state);
void or_unpack_row(const uint8_t *packed, size_t in_features, int8_t *out);
void or_pack_row(const int8_t *trits, size_t n, uint8_t *out);
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
void or_f16_to_f32_n(const uint16_t *h, size_t n, float *out);
void or_dequant_matrix(const uint8_t *qweight, const uint16_t *scales_f16, size_t out_features,
                       size_t in_features, size_t group, float *w);
void or_unpack_matrix(const uint8_t *qweight, size_t out_features, size_t in_features, int8_t *w);
float or_quantize_group(const float *src, size_t n, int8_t *dst);
void or_quantize(const float *x, size_t n, size_t inp, size_t group, int8_t *q, float *scales, int32_t *gsum);
float or_exp_poly(float x);
float or_silu_fast(float x);
float or_sigmoid_fast(float x);
float or_ep_apply(int ep, float alpha, float old, float v);
void or_gemm_scalar_range(const int8_t *w, const float *ws, size_t out, size_t inp, size_t group,
                          const int8_t *x, const float *xs, size_t n, float *y, size_t r0, size_t r1, size_t t0,
                          size_t t1, int ep, float alpha, int32_t *group_sums);
void or_gemm_scalar_mt(const int8_t *w, const float *ws, size_t out, size_t inp, size_t group, const int8_t *x,
                       const float *xs, size_t n, float *y, int ep, float alpha, int32_t *group_sums, int threads);

/* CPU baseline: AVX-512 VNNI restatement on the Quad16 layout (kernels/x86.rs:46-154) */
int or_have_vnni(void);
size_t or_quad16_bytes(size_t out, size_t inp);
void or_quad16_pack(const int8_t *rows, size_t out, size_t inp, size_t group, const float *scales, int8_t *wq,
                    float *scales_q);
void or_gemm_vnni_range(const int8_t *wq, const float *scales_q, size_t out, size_t inp, size_t group,
                        const int8_t *x, const float *xs, const int32_t *gsum, size_t n, float *y, size_t r0,
                        size_t r1, size_t t0, size_t t1, int ep, float alpha);
void or_gemm_ep_vnni(const int8_t *wq, const float *scales_q, size_t out, size_t inp, size_t group,
                     const int8_t *x, const float *xs, const int32_t *gsum, size_t n, float *y, int ep, float alpha,
                     int threads, size_t blocks_mult);

/* Second CPU path: AVX2 restatement on the same Quad16 plane (kernels/x86.rs:163-290); -1 for ternary with
 * group > 256, else 0 */
int or_have_avx2(void);
int or_gemm_avx2_range(const int8_t *wq, const float *scales_q, size_t out, size_t inp, size_t group, int ternary,
                       const int8_t *x, const float *xs, const int32_t *gsum, size_t n, float *y, size_t r0, size_t r1,
                       size_t t0, size_t t1, int ep, float alpha);

/* Thread count of the oracle's parallel loops (default 1; results do not depend on it). */
int or_get_threads(void);
void or_set_threads(int n);

/* Encoder side (encoder_oracle.c) */
void or_row_mean_var(const float *x, size_t d, float *mean, float *var);
void or_layer_norm(const float *x, size_t n, size_t d, const float *g, const float *b, float *y);
void or_quantize_normed(const float *x, size_t n, size_t inp, size_t group, const float *g, const float *b,
                        int8_t *q, float *scales, int32_t *gsum);
float or_exp_row_scaled(float *row, size_t n, float scale);
void or_glu(const float *gbuf, size_t n, size_t d, float *out);
void or_fold_bn(const float *dw, const float *gamma, const float *beta, const float *mean, const float *var,
                size_t d, size_t k, float *dw_t, float *dw_bias);
void or_dwconv_bn_silu(const float *a, size_t t, size_t d, size_t k, const float *dw_t, const float *dw_bias,
                       float *out);
void or_rel_pos_table(size_t t, size_t d, float *out);
void or_linear_f32(const float *x, size_t n, size_t in_f, const float *w, const float *b, size_t out_f, float *y);
size_t or_subsampling_frames(size_t t, size_t k, size_t s);
size_t or_subsampling(const float *feats, size_t t, size_t n_mels, size_t c, size_t k, size_t s, const float *conv0_w,
                      const float *conv0_b, const float *dw_w, const float *dw_b, const float *pw_w,
                      const float *pw_b, const float *lin_w, const float *lin_b, size_t d_model, float *out);
void or_attn_core_int8(const float *qkv, const float *rel_k, size_t t, size_t d, size_t h, const float *bias_u,
                       const float *bias_v, float scaling, float *ctx);
void or_conformer_layer(float *x, size_t t, const float *pos_emb, const void *const *params, size_t d, size_t heads,
                        size_t ff, size_t kconv, size_t group, int threads);

#ifdef __cplusplus
}
#endif
#endif
