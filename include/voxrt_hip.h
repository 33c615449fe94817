/* voxrt_hip.h — C ABI of the MI355X (gfx950) ternary x int8 GEMM path.
 *
 * The entry points mirror voxrt's runtime kernel-dispatch surface (crates/voxrt/src/kernels/mod.rs and
 * crates/voxrt/src/packed.rs), so a GPU backend binds beside its scalar/AVX2/VNNI/NEON kernels:
 *
 *   vx_detect / vx_init               <- kernels::detect (kernels/mod.rs:85-109)
 *   vx_shutdown                       <- (none: drains the device at the end of a session)
 *   vx_tmat_upload_packed             <- TernaryMatrix::from_packed_layout (packed.rs:73-130)
 *   vx_tmat_upload_packed_f32         <- the same with f32 scales (a per-output-channel fp32 scale, as in the
 *                                        338 x 1024 x 4096 single-GEMM workload)
 *   vx_tmat_upload_trits              <- a TernaryMatrix in the Rows layout (packed.rs:48-60: trits + f32 scales)
 *   vx_tmat_upload_i8                 <- TernaryMatrix::from_i8_rows (packed.rs:164-201)
 *   vx_tmat_free / vx_tmat_info       <- drop / the out, inp, group, ternary fields (packed.rs:48-60)
 *   vx_quantize                       <- QuantAct::quantize_layout (packed.rs:307-436, quantize_group 527-535)
 *   vx_gemm_ep                        <- kernels::gemm_ep / gemm (kernels/mod.rs:319-362)
 *   vx_gemm_ep_quantize               <- FeedForward::forward_fused's up-projection + prepare (encoder.rs:87-89)
 *   vx_gemm_rows_range                <- kernels::gemm_rows_range (kernels/mod.rs:257-282)
 *   vx_gemm_single                    <- kernels::gemm_single (kernels/mod.rs:285-316)
 *   vx_quantize_normed                <- TernaryLinear::prepare_normed (ternary_linear.rs:132-155)
 *   vx_layer_norm                     <- tensor::layer_norm (tensor.rs:700-719)
 *   vx_glu_dwconv_silu, vx_fold_bn    <- ConvModule::forward_fused / load (encoder.rs:548-573, 590-624)
 *   vx_glu_dwconv_silu_quantize       <- the same conv rows + pw2.prepare(hb) (encoder.rs:605-625)
 *   vx_linear_f32                     <- tensor::linear (tensor.rs:98-127)
 *   vx_subsampling*                   <- Subsampling::forward / out_frames (subsampling.rs:114-204)
 *   vx_rel_pos_table                  <- encoder::rel_pos_table (encoder.rs:760-776)
 *   vx_attention_core*                <- attn_core_int8 (encoder.rs:317-534)
 *   vx_encoder_*                      <- GpuEncoder::{load, forward, forward_feats} (metal/mod.rs:446-603) on the
 *                                        CPU int8 Encoder's operation order (encoder.rs:706-857)
 *   vx_encoder_set_profiling / _take_profile <- VOXRT_PROFILE's per-sublayer Profile (encoder.rs:645-653,823-854)
 *   vx_encoder_memory                 <- (none: the workspace size and graph count, for hosts that bound memory)
 *   vx_last_error                     <- voxrt_last_error (crates/voxrt-ffi/src/lib.rs:61-74)
 *   vx_check_activations              <- (none: device self-check of exp_poly/silu_fast/sigmoid_fast)
 *   vx_set_kernel_override            <- VOXRT_KERNEL's role for the GPU kernels (kernels/mod.rs:126-149): forcing
 *                                        a kernel family, tile or grid for tests and tuning
 *
 * Conventions (as voxrt-ffi): every call returns a vx_status; on failure a message is kept in a thread-local
 * buffer read by vx_last_error(). No exception crosses the ABI. Weight uploads take HOST pointers (the load-time
 * repack of the reference runs on the device). Activation, scale, output and bias pointers are DEVICE pointers on
 * the current HIP device; `stream` is a hipStream_t (NULL = the default stream); every GEMM / quantize call is
 * ordered on that stream and returns before the work completes. Calls on different streams that write disjoint
 * outputs may run concurrently; a vx_tmat is immutable after upload and may be shared by any number of calls.
 *
 * Shape rules: inp % group == 0, group % 64 == 0 (one i8 MFMA step is 64 columns). A call over zero tokens
 * (n = 0, t = 0, or an empty row or token range) does nothing and returns VX_OK; its activation, output and
 * parameter pointers may then be NULL (the reference's kernels loop over zero tokens).
 */
#ifndef VOXRT_HIP_H
#define VOXRT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum vx_status {
    VX_OK = 0,
    VX_ERR_INVALID = 1,     /* a NULL pointer, a bad shape or an unsupported group */
    VX_ERR_NO_DEVICE = 2,   /* no HIP device, or the current device is not gfx950 */
    VX_ERR_HIP = 3,         /* a HIP runtime call failed (the message names it) */
    VX_ERR_OOM = 4          /* device allocation failed */
} vx_status;

/* kernels/mod.rs:14-21 Epilogue: STORE y = v; SILU y = silu_fast(v); ADD_SCALED y = fma(alpha, v, y). */
typedef enum vx_epilogue { VX_EP_STORE = 0, VX_EP_SILU = 1, VX_EP_ADD_SCALED = 2 } vx_epilogue;

/* Opaque device-resident weight matrix [out, inp] in the MFMA layout (TernaryMatrix, packed.rs:48-60). */
typedef struct vx_tmat vx_tmat;

/* Thread-local text of the last failure on this thread ("" if none). */
const char *vx_last_error(void);

/* 1 if the current process sees at least one gfx950 device, else 0 (kernels::detect). */
int vx_detect(void);

/* Make `device` current for this thread and check that it is gfx950. */
vx_status vx_init(int device);

/* Force a GEMM kernel choice for the whole process (tests and tuning; the library reads no environment variable):
 * name "gemm" with value direct | splitk | lds | big | splitg | small | stream, "tile" and "small_tile" with "MTxNT"
 * (16*MT tokens x 16*NT rows), "stream_grid" with a workgroup count (a multiple of 8). A forced kernel that cannot
 * run a shape is not used for it. NULL or "" clears the override of that name. Not for concurrent use with GEMM
 * calls that should not see it. */
vx_status vx_set_kernel_override(const char *name, const char *value);

/* Wait for all work on the current device and report any error it left. No counterpart in voxrt (its GPU
 * context lives until the process drops it); for hosts that end a device session explicitly. The library keeps no
 * global device memory: weight and encoder handles are released by their _free calls. */
vx_status vx_shutdown(void);

/* from_packed_layout: qweight = thrush-ternary-v2 rows uint8 [out, ceil(inp/5)] (5 trits per byte, least
 * significant base-3 digit first, trit = digit - 1), scales_f16 = IEEE binary16 [out, inp/group]. */
vx_status vx_tmat_upload_packed(const uint8_t *qweight, const uint16_t *scales_f16, int64_t out, int64_t inp,
                                int64_t group, vx_tmat **w);

/* As vx_tmat_upload_packed with float32 scales [out, inp/group]. */
vx_status vx_tmat_upload_packed_f32(const uint8_t *qweight, const float *scales, int64_t out, int64_t inp,
                                    int64_t group, vx_tmat **w);

/* A ternary matrix already unpacked to trits: int8 rows [out, inp] in {-1, 0, +1} (TernaryMatrix::w in the Rows
 * layout) with float32 scales [out, inp/group]. Uploaded as a ternary matrix (the 2-bit layout, as from the model
 * file's rows); any other value is refused with VX_ERR_INVALID. */
vx_status vx_tmat_upload_trits(const int8_t *trits, const float *scales, int64_t out, int64_t inp, int64_t group,
                               vx_tmat **w);

/* from_i8_rows: arbitrary int8 rows [out, inp] with float32 scales [out, inp/group] (not ternary). */
vx_status vx_tmat_upload_i8(const int8_t *rows, const float *scales, int64_t out, int64_t inp, int64_t group,
                            vx_tmat **w);

void vx_tmat_free(vx_tmat *w);

vx_status vx_tmat_info(const vx_tmat *w, int64_t *out, int64_t *inp, int64_t *group, int *ternary);

/* Padded token count of the transposed activation tables: n rounded up to a multiple of 16. */
#define VX_NPAD(n) ((((n) + 15) / 16) * 16)

/* quantize_layout on the device: per (token, group) s = absmax/127 (1 when all zero), codes
 * clamp(rint(x * (1/s)), -127, 127); x float32 [n, inp] -> q int8 [n, inp], scales_t float32 [inp/group, np] and
 * gsum_t int32 [inp/group, np] with np = VX_NPAD(n): the scales and code sums transposed (QuantAct::scales_t,
 * packed.rs:294), pad tokens zero. gsum (sum of the codes of each group) is what ternary GEMMs need. */
vx_status vx_quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t,
                      int32_t *gsum_t, void *stream);

/* gemm_ep: y[t*out + o] = ep(y_old, sum_g fma-fold of S_g * (xs[t][g] * ws[o][g])) for all t < n, o < out, then
 * y += bias[o] when bias is not NULL. xq int8 [n, inp]; xs_t float32 [inp/group, VX_NPAD(n)] and xgsum_t int32
 * [inp/group, VX_NPAD(n)] as written by vx_quantize (xgsum_t is required for ternary weights); y float32
 * [n, out]. When group_sums is not NULL the exact int32 group sums S_g are also written to
 * group_sums[(g*n + t)*out + o] (int32 [inp/group, n, out]). */
vx_status vx_gemm_ep(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t, int64_t n,
                     float *y, const float *bias, int ep, float alpha, int32_t *group_sums, void *stream);

/* gemm_ep + prepare fused: the FFN up-projection followed by the down-projection's activation quantization
 * (FeedForward::forward_fused, encoder.rs:87-89: w1.forward_prepared_ep(a, t, hbuf, Epilogue::Silu), then
 * w2.prepare(hbuf, t) = QuantAct::quantize_layout, packed.rs:307-436). y = ep(x . w^T) (+ bias) with ep Store or
 * Silu, quantized in `group`-column groups into q int8 [n, out], scales_t float32 and gsum_t int32
 * [out/group, VX_NPAD(n)] (pad tokens zero), bit for bit as vx_gemm_ep followed by vx_quantize. y_tmp float32
 * [n, out] is scratch: with 128-column groups and n <= 1024 the GEMM quantizes in its epilogue and y_tmp is not
 * touched (it may then be NULL); other shapes write y there and quantize it. */
vx_status vx_gemm_ep_quantize(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t,
                              int64_t n, float *y_tmp, const float *bias, int ep, int64_t group, int8_t *q,
                              float *scales_t, int32_t *gsum_t, void *stream);

/* gemm_rows_range: as vx_gemm_ep without bias, writing only rows o in [r0, r1) and tokens t in [t0, t1) of
 * y [n, out]; nothing else in y is read or written. */
vx_status vx_gemm_rows_range(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t,
                             int64_t n, float *y, int64_t r0, int64_t r1, int64_t t0, int64_t t1, int ep, float alpha,
                             void *stream);

/* gemm_single: y[n, out] = x . w^T, then y += bias (when not NULL), unfused (kernels/mod.rs:285-316); the decoder's
 * single-token GEMV. Same operands as vx_gemm_ep. */
vx_status vx_gemm_single(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t, int64_t n,
                         float *y, const float *bias, void *stream);

/* prepare_normed: vx_quantize of LayerNorm(x) (eps 1e-5, biased variance, the reference's summation order;
 * y = ((x - mean) * inv) * gamma + beta) without writing the normalized rows. gamma, beta float32 [inp]. */
vx_status vx_quantize_normed(const float *x, int64_t n, int64_t inp, int64_t group, const float *gamma,
                             const float *beta, int8_t *q, float *scales_t, int32_t *gsum_t, void *stream);

/* layer_norm: y [n, d] = LayerNorm(x [n, d]) with gamma, beta [d]. y may not alias x. */
vx_status vx_layer_norm(const float *x, int64_t n, int64_t d, const float *gamma, const float *beta, float *y,
                        void *stream);

/* The conv module between its pointwise convolutions: g [t, 2d] (pointwise_conv1 output) -> out [t, d] =
 * silu(bias + sum over taps kk of w_t[kk][c] * glu(g)[i + kk - (k-1)/2][c]), glu = a * sigmoid(b) over the two
 * halves of g, taps outside [0, t) skipped. w_t [k][d] and bias [d] are the BatchNorm-folded taps of vx_fold_bn. */
vx_status vx_glu_dwconv_silu(const float *g, int64_t t, int64_t d, int64_t k, const float *w_t, const float *bias,
                             float *out, void *stream);

/* glu_dwconv_silu + prepare fused (ConvModule::forward_fused, encoder.rs:605-625: the depthwise conv rows, then
 * pw2.prepare(hb)): the rows of vx_glu_dwconv_silu quantized in 128-channel groups (group must be 128, d a
 * multiple of 256) into q int8 [t, d], scales_t float32 and gsum_t int32 [d/128, VX_NPAD(t)] (pad tokens zero),
 * bit for bit as vx_glu_dwconv_silu followed by vx_quantize. */
vx_status vx_glu_dwconv_silu_quantize(const float *g, int64_t t, int64_t d, int64_t k, const float *w_t,
                                      const float *bias, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t,
                                      void *stream);

/* HOST: fold BatchNorm(eval) into the depthwise taps: dw [d][k] (PyTorch [d,1,k]) -> w_t [k][d], bias [d]. */
vx_status vx_fold_bn(const float *dw, const float *gamma, const float *beta, const float *mean, const float *var,
                     int64_t d, int64_t k, float *w_t, float *bias);

/* linear: y [n, out_f] = x [n, in_f] . w [out_f, in_f]^T (+ b [out_f] when not NULL), then max(y, 0) when relu. */
vx_status vx_linear_f32(const float *x, int64_t n, int64_t in_f, const float *w, const float *b, int64_t out_f,
                        float *y, int relu, void *stream);

/* Subsampling output frames for t input frames (three stride-s convolutions of kernel k, padding (k-1)/2). */
int64_t vx_subsampling_frames(int64_t t, int64_t k, int64_t s);
/* Device scratch (float32 elements) that vx_subsampling needs for t frames of nm mel bins and c channels. */
int64_t vx_subsampling_scratch_floats(int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s);
/* Subsampling::forward on device buffers: feats [t, nm] -> out [t3, d_model]. Weights as the reference loads them:
 * conv0_w [k*k, c], conv0_b [c], dw_w [2, k*k, c], dw_b [2, c], pw_w [2, c, c] (out, in), pw_b [2, c],
 * lin_w [d_model, f3*c] (channels-last columns), lin_b [d_model]. */
vx_status vx_subsampling(const float *feats, int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s,
                         const float *conv0_w, const float *conv0_b, const float *dw_w, const float *dw_b,
                         const float *pw_w, const float *pw_b, const float *lin_w, const float *lin_b, int64_t d_model,
                         float *scratch, float *out, int64_t *t_out, void *stream);

/* HOST: the relative position table [2t-1, d] (positions t-1 .. -(t-1), sin/cos interleaved per frequency). */
vx_status vx_rel_pos_table(int64_t t, int64_t d, float *out);

/* DEVICE SELF-CHECK (no counterpart in voxrt): evaluates the library's exp_poly, silu_fast and sigmoid_fast
 * (tensor.rs:829-860) on the device for all 2^32 float inputs and compares each bit for bit with the IEEE form of
 * the same formula (NaN equals NaN). mismatch[0..2] receive the mismatch counts of exp, SiLU and sigmoid; all
 * three are 0 on a correct build. Synchronous, about 0.1 s. */
vx_status vx_check_activations(uint64_t *mismatch);

/* Device workspace bytes of vx_attention_core for t frames, model width d and h heads. */
int64_t vx_attention_ws_bytes(int64_t t, int64_t d, int64_t h);
/* The int8 attention core of one layer for all heads (head dim 128, 1 <= t <= 1024): qkv [t, 3d] (q | k | v),
 * rel_k [2t-1, d] (relative_k_proj of the position table), bias_u / bias_v [h, 128], scaling = 1/sqrt(128);
 * ctx [t, d]. ws: vx_attention_ws_bytes device bytes. */
vx_status vx_attention_core(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                            const float *bias_u, const float *bias_v, float scaling, void *ws, float *ctx,
                            void *stream);

/* NO COUNTERPART IN THE REFERENCE. vx_attention_core without the ws argument, for callers that cannot allocate
 * device memory (code under graph capture, serving loops or harnesses that forbid hipMalloc): the workspace is a
 * fixed 8 MiB array in the library, one per GPU, held until the process ends (its address is looked up by vx_init,
 * or by the first call on a device). Calls whose vx_attention_ws_bytes(t, d, h) exceeds 8 MiB are refused with
 * VX_ERR_INVALID (t <= 1024 with d = 1024 and 8 heads fits). Nothing is allocated. All calls on one GPU share the
 * array: calls that overlap on one GPU (other streams, other threads) race; serialize them. */
vx_status vx_attention_core_noalloc(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                                    const float *bias_u, const float *bias_v, float scaling, float *ctx,
                                    void *stream);

/* attention core + prepare fused (Attention::forward_fused, encoder.rs:180-183: attn_core_int8 into ctx, then
 * wo.prepare(ctx)): as vx_attention_core, but ctx is written as the o-projection's int8 activations in 128-column
 * groups, one per head (group must be 128): q int8 [t, d], scales_t float32 and gsum_t int32 [h, VX_NPAD(t)]
 * (pad tokens zero), bit for bit as vx_attention_core followed by vx_quantize. */
vx_status vx_attention_core_quantize(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                                     const float *bias_u, const float *bias_v, float scaling, void *ws, int64_t group,
                                     int8_t *q, float *scales_t, int32_t *gsum_t, void *stream);

/* ---------------------------------------------------------------------------------------------- encoder */

/* Shape of a FastConformer encoder (reference/config.json encoder_config): d = heads * 128. */
typedef struct vx_encoder_config {
    int64_t d, heads, ff, kconv, group, n_layers;
    int64_t n_mels, sub_channels, sub_kernel, sub_stride; /* subsampling (0 if unused) */
} vx_encoder_config;

/* One layer's weights, HOST pointers, as the model file holds them. Linears in this order: feed_forward1.linear1,
 * feed_forward1.linear2, q|k|v (q_proj, k_proj, v_proj rows stacked), o_proj, relative_k_proj, pointwise_conv1,
 * pointwise_conv2, feed_forward2.linear1, feed_forward2.linear2: thrush-ternary-v2 qweight uint8 [out, ceil(inp/5)]
 * and f16 scales [out, inp/group]. LayerNorms in this order: norm_feed_forward1, norm_self_att, norm_conv,
 * norm_feed_forward2, norm_out ([d] each). bias_u, bias_v [heads, 128]. dw = depthwise_conv.weight [d, k] and the
 * BatchNorm (eval) statistics [d], folded at load. */
typedef struct vx_layer_params {
    const uint8_t *qweight[9];
    const uint16_t *scales_f16[9];
    const float *ln_gamma[5], *ln_beta[5];
    const float *bias_u, *bias_v;
    const float *dw, *bn_gamma, *bn_beta, *bn_mean, *bn_var;
} vx_layer_params;

/* Subsampling weights, HOST pointers, in the layout of vx_subsampling. */
typedef struct vx_subsampling_params {
    const float *conv0_w, *conv0_b, *dw_w, *dw_b, *pw_w, *pw_b, *lin_w, *lin_b;
} vx_subsampling_params;

typedef struct vx_encoder vx_encoder;

vx_status vx_encoder_create(const vx_encoder_config *cfg, vx_encoder **enc);
/* Upload layer `layer`'s weights (every layer must be set before a forward). */
vx_status vx_encoder_set_layer(vx_encoder *enc, int64_t layer, const vx_layer_params *p);
vx_status vx_encoder_set_subsampling(vx_encoder *enc, const vx_subsampling_params *p);
/* 1 (default): the layer stack of each (frames, segments) pair is captured once into a hipGraph (on a private stream:
 * nothing runs during the capture) and launched on the caller's stream, NULL included; the 8 most recently used
 * graphs are kept. 0: kernels are launched one by one. */
vx_status vx_encoder_use_graphs(vx_encoder *enc, int on);

/* Wall-clock device time per sublayer type, summed over layers and over the forwards since the last take
 * (encoder.rs:645-653 Profile; attn includes attn_core). */
typedef struct vx_encoder_profile {
    double total_ms, subsampling_ms, ff_ms, attn_ms, attn_core_ms, conv_ms, norm_ms;
    int64_t forwards;
} vx_encoder_profile;
/* 1: every forward launches its kernels one by one with device events between the sublayers and waits for them
 * (a timing mode, as VOXRT_PROFILE=1 is for the reference's encoder); 0 (default): off. */
vx_status vx_encoder_set_profiling(vx_encoder *enc, int on);
/* The sums since the previous take (then reset). */
vx_status vx_encoder_take_profile(vx_encoder *enc, vx_encoder_profile *out);
/* Device bytes of the encoder's workspace (weights not counted) and the number of graphs kept. */
vx_status vx_encoder_memory(vx_encoder *enc, int64_t *workspace_bytes, int64_t *graphs);

/* Memory and concurrency of the forward calls (GpuEncoder's Mutex-guarded workspace, metal/mod.rs:449-460,641-645):
 * one device workspace serves every frame count and segment count; it grows to 1.25x a call's need when a call needs
 * more (after the device has finished the previous forward) and never shrinks. Calls on one encoder may come from
 * any threads and streams: they are serialized on the host, and each forward's work waits on the device for the
 * previous forward's, so they never share the workspace at the same time. The encoder belongs to the device that
 * was current at vx_encoder_create (or at its first weight upload, when none was then). */

/* The layer stack (GpuEncoder::forward): x [t, d] (device, the subsampling output) -> out [t, d] (may alias x);
 * 1 <= t <= 1024. */
vx_status vx_encoder_forward(vx_encoder *enc, const float *x, float *out, int64_t t, void *stream);
/* Subsampling + layers (GpuEncoder::forward_feats): feats [t_in, n_mels] (device) -> out [t_out, d] (device, sized
 * for vx_subsampling_frames(t_in, sub_kernel, sub_stride) rows). */
vx_status vx_encoder_forward_feats(vx_encoder *enc, const float *feats, int64_t t_in, float *out, int64_t *t_out,
                                   void *stream);
/* Batched forms: nseg segments of equal length in one pass, x / feats / out laid out [nseg][t][...]. Each segment's
 * output equals its own vx_encoder_forward(_feats) bit for bit: token-row work (LayerNorm, quantizers, GEMMs)
 * runs over all nseg * t rows at once, while the depthwise convolution, the attention and the subsampling stay
 * inside each segment. The reference encodes one VAD segment per call (Transcriber::transcribe_long,
 * transcriber.rs:356-386); these entry points have no counterpart there and serve callers that hold several
 * segments of one length at once. nseg * t <= 65535. */
vx_status vx_encoder_forward_batch(vx_encoder *enc, const float *x, float *out, int64_t nseg, int64_t t, void *stream);
vx_status vx_encoder_forward_feats_batch(vx_encoder *enc, const float *feats, int64_t nseg, int64_t t_in, float *out,
                                         int64_t *t_out, void *stream);
void vx_encoder_free(vx_encoder *enc);

#ifdef __cplusplus
}
#endif
#endif
