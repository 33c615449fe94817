// vx_abi.hip — the extern "C" entry points of libvoxrt_hip (declared in include/voxrt_hip.h).
//
// Every entry point catches what the C++ layer throws and turns it into a vx_status plus a thread-local message
// (the convention of crates/voxrt-ffi/src/lib.rs:61-74,97-107), so no exception crosses the ABI.
#include <cstring>
#include <string>

#include "vx_internal.h"

namespace vx {
vx_tmat *upload_packed(const uint8_t *qweight, const void *scales, bool scales_f16, int64_t out, int64_t inp,
                       int64_t group);
vx_tmat *upload_i8(const int8_t *rows, const float *scales, int64_t out, int64_t inp, int64_t group);
vx_tmat *upload_trits(const int8_t *trits, const float *scales, int64_t out, int64_t inp, int64_t group);
void free_tmat(vx_tmat *h);
void quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t,
              hipStream_t stream);
void gemm(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y,
          const float *bias, int ep, float alpha, int32_t *gs, int64_t r0, int64_t r1, int64_t t0, int64_t t1,
          hipStream_t st, int64_t cap_rows = 0);
void quantize_ln(const float *x, int64_t n, int64_t inp, int64_t group, const float *g, const float *b, int8_t *q,
                 float *scales_t, int32_t *gsum_t, hipStream_t stream);
void gemm_quant(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y_tmp,
                const float *bias, int ep, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t, hipStream_t st,
                int64_t cap_rows = 0);
void layer_norm(const float *x, int64_t n, int64_t d, const float *g, const float *b, float *y, hipStream_t stream);
void glu_dwconv_silu(const float *g, int64_t t, int64_t d, int64_t k, const float *w_t, const float *bias, float *out,
                     hipStream_t st);
void glu_dwconv_silu_quant_seg(const float *g, int64_t nseg, int64_t t, int64_t d, int64_t k, const float *w_t,
                               const float *bias, int8_t *q, float *scales_t, int32_t *gsum_t, hipStream_t st);
void linear_f32(const float *x, int64_t n, int64_t in_f, const float *w, const float *b, int64_t out_f, float *y,
                bool relu, hipStream_t st);
int64_t subsampling(const float *feats, int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s, const float *conv0_w,
                    const float *conv0_b, const float *dw_w, const float *dw_b, const float *pw_w, const float *pw_b,
                    const float *lin_w, const float *lin_b, int64_t d_model, float *scratch, float *out,
                    hipStream_t st);
int64_t subsampling_frames(int64_t t, int64_t k, int64_t s);
int64_t subsampling_scratch_floats(int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s);
void fold_bn(const float *dw, const float *gamma, const float *beta, const float *mean, const float *var, int64_t d,
             int64_t k, float *dw_t, float *dw_bias);
void rel_pos_table(int64_t t, int64_t d, float *out);
void check_activations(uint64_t *mismatch_host);
size_t attn_ws_bytes(int64_t t, int64_t d, int64_t h);
void attention_core(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h, const float *bias_u,
                    const float *bias_v, float scaling, void *ws, float *ctx, hipStream_t st);
void attention_core_noalloc(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                            const float *bias_u, const float *bias_v, float scaling, float *ctx, hipStream_t st);
void *static_attn_ws();
void attention_core_seg(const float *qkv, const float *rel_k, int64_t nseg, int64_t t, int64_t d, int64_t h,
                        const float *bias_u, const float *bias_v, float scaling, void *ws, float *ctx,
                        hipStream_t st, int8_t *q, float *scales_t, int32_t *gsum_t, int64_t rel_ld,
                        const int8_t *rq_pre, const float *rs_pre);
void set_kernel_override(const char *name, const char *value);
vx_encoder *encoder_create(const vx_encoder_config *cfg);
void encoder_free(vx_encoder *e);
void encoder_use_graphs(vx_encoder *e, bool on);
void encoder_set_layer(vx_encoder *e, int64_t li, const vx_layer_params *p);
void encoder_set_subsampling(vx_encoder *e, const vx_subsampling_params *p);
void encoder_forward(vx_encoder *e, const float *x, float *out, int64_t t, hipStream_t st);
void encoder_set_profiling(vx_encoder *e, bool on);
void encoder_take_profile(vx_encoder *e, vx_encoder_profile *out);
void encoder_memory(vx_encoder *e, int64_t *workspace_bytes, int64_t *graphs);
void encoder_forward_batch(vx_encoder *e, const float *x, float *out, int64_t nseg, int64_t t, hipStream_t st);
void encoder_forward_feats_batch(vx_encoder *e, const float *feats, int64_t nseg, int64_t t_in, float *out,
                                 int64_t *t_out, hipStream_t st);
void encoder_forward_feats(vx_encoder *e, const float *feats, int64_t t_in, float *out, int64_t *t_out,
                           hipStream_t st);
}  // namespace vx

namespace {

thread_local std::string g_last_error;

template <class F>
vx_status guarded(F &&f) {
    try {
        f();
        g_last_error.clear();
        return VX_OK;
    } catch (const vx::Error &e) {
        g_last_error = e.what();
        return e.code;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return VX_ERR_HIP;
    } catch (...) {
        g_last_error = "unknown error";
        return VX_ERR_HIP;
    }
}

bool is_gfx950(int device) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

const vx::TMat *unwrap(const vx_tmat *w) { return &w->m; }

}  // namespace

extern "C" {

const char *vx_last_error(void) { return g_last_error.c_str(); }

int vx_detect(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    for (int d = 0; d < n; d++)
        if (is_gfx950(d)) return 1;
    return 0;
}

vx_status vx_init(int device) {
    return guarded([&] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
            (void)hipGetLastError();
            throw vx::Error(VX_ERR_NO_DEVICE, "no HIP device visible");
        }
        if (device < 0 || device >= n) throw vx::Error(VX_ERR_INVALID, "device index out of range");
        if (!is_gfx950(device)) throw vx::Error(VX_ERR_NO_DEVICE, "device is not gfx950 (MI355X)");
        vx::hip_check(hipSetDevice(device), "hipSetDevice");
        (void)vx::static_attn_ws();  // the device address of the workspace-free attention core's array
    });
}

vx_status vx_set_kernel_override(const char *name, const char *value) {
    return guarded([&] { vx::set_kernel_override(name, value); });
}

vx_status vx_shutdown(void) {
    return guarded([&] { vx::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}

vx_status vx_tmat_upload_packed(const uint8_t *qweight, const uint16_t *scales_f16, int64_t out, int64_t inp,
                                int64_t group, vx_tmat **w) {
    return guarded([&] {
        vx::require(w != nullptr, "output handle pointer must not be NULL");
        *w = nullptr;
        *w = vx::upload_packed(qweight, scales_f16, true, out, inp, group);
    });
}

vx_status vx_tmat_upload_packed_f32(const uint8_t *qweight, const float *scales, int64_t out, int64_t inp,
                                    int64_t group, vx_tmat **w) {
    return guarded([&] {
        vx::require(w != nullptr, "output handle pointer must not be NULL");
        *w = nullptr;
        *w = vx::upload_packed(qweight, scales, false, out, inp, group);
    });
}

vx_status vx_tmat_upload_trits(const int8_t *trits, const float *scales, int64_t out, int64_t inp, int64_t group,
                               vx_tmat **w) {
    return guarded([&] {
        vx::require(w != nullptr, "output handle pointer must not be NULL");
        *w = nullptr;
        *w = vx::upload_trits(trits, scales, out, inp, group);
    });
}

vx_status vx_tmat_upload_i8(const int8_t *rows, const float *scales, int64_t out, int64_t inp, int64_t group,
                            vx_tmat **w) {
    return guarded([&] {
        vx::require(w != nullptr, "output handle pointer must not be NULL");
        *w = nullptr;
        *w = vx::upload_i8(rows, scales, out, inp, group);
    });
}

void vx_tmat_free(vx_tmat *w) { vx::free_tmat(w); }

vx_status vx_tmat_info(const vx_tmat *w, int64_t *out, int64_t *inp, int64_t *group, int *ternary) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        const vx::TMat *m = unwrap(w);
        if (out) *out = m->out;
        if (inp) *inp = m->inp;
        if (group) *group = m->group;
        if (ternary) *ternary = m->ternary ? 1 : 0;
    });
}

vx_status vx_quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t,
                      int32_t *gsum_t, void *stream) {
    return guarded([&] { vx::quantize(x, n, inp, group, q, scales_t, gsum_t, (hipStream_t)stream); });
}

vx_status vx_gemm_ep(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t, int64_t n,
                     float *y, const float *bias, int ep, float alpha, int32_t *group_sums, void *stream) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        const vx::TMat *m = unwrap(w);
        vx::gemm(m, xq, xs_t, xgsum_t, n, y, bias, ep, alpha, group_sums, 0, m->out, 0, n, (hipStream_t)stream);
    });
}

vx_status vx_gemm_ep_quantize(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t,
                              int64_t n, float *y_tmp, const float *bias, int ep, int64_t group, int8_t *q,
                              float *scales_t, int32_t *gsum_t, void *stream) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        vx::gemm_quant(unwrap(w), xq, xs_t, xgsum_t, n, y_tmp, bias, ep, group, q, scales_t, gsum_t,
                       (hipStream_t)stream);
    });
}

vx_status vx_gemm_rows_range(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t,
                             int64_t n, float *y, int64_t r0, int64_t r1, int64_t t0, int64_t t1, int ep, float alpha,
                             void *stream) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        vx::gemm(unwrap(w), xq, xs_t, xgsum_t, n, y, nullptr, ep, alpha, nullptr, r0, r1, t0, t1,
                 (hipStream_t)stream);
    });
}

vx_status vx_gemm_single(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t, int64_t n,
                         float *y, const float *bias, void *stream) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        const vx::TMat *m = unwrap(w);
        vx::gemm(m, xq, xs_t, xgsum_t, n, y, bias, VX_EP_STORE, 0.0f, nullptr, 0, m->out, 0, n, (hipStream_t)stream);
    });
}

vx_status vx_quantize_normed(const float *x, int64_t n, int64_t inp, int64_t group, const float *gamma,
                             const float *beta, int8_t *q, float *scales_t, int32_t *gsum_t, void *stream) {
    return guarded([&] {
        vx::require(n == 0 || (gamma && beta), "gamma and beta must not be NULL");
        vx::quantize_ln(x, n, inp, group, gamma, beta, q, scales_t, gsum_t, (hipStream_t)stream);
    });
}

vx_status vx_layer_norm(const float *x, int64_t n, int64_t d, const float *gamma, const float *beta, float *y,
                        void *stream) {
    return guarded([&] {
        vx::require(n == 0 || x != y, "vx_layer_norm: y must not alias x");
        vx::layer_norm(x, n, d, gamma, beta, y, (hipStream_t)stream);
    });
}

vx_status vx_glu_dwconv_silu(const float *g, int64_t t, int64_t d, int64_t k, const float *w_t, const float *bias,
                             float *out, void *stream) {
    return guarded([&] { vx::glu_dwconv_silu(g, t, d, k, w_t, bias, out, (hipStream_t)stream); });
}

vx_status vx_glu_dwconv_silu_quantize(const float *g, int64_t t, int64_t d, int64_t k, const float *w_t,
                                      const float *bias, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t,
                                      void *stream) {
    return guarded([&] {
        vx::require(group == 128, "glu_dwconv_quantize: 128-channel groups");
        vx::glu_dwconv_silu_quant_seg(g, 1, t, d, k, w_t, bias, q, scales_t, gsum_t, (hipStream_t)stream);
    });
}

vx_status vx_fold_bn(const float *dw, const float *gamma, const float *beta, const float *mean, const float *var,
                     int64_t d, int64_t k, float *w_t, float *bias) {
    return guarded([&] {
        vx::require(dw && gamma && beta && mean && var && w_t && bias, "vx_fold_bn: NULL pointer");
        vx::require(d > 0 && k > 0, "vx_fold_bn: bad shape");
        vx::fold_bn(dw, gamma, beta, mean, var, d, k, w_t, bias);
    });
}

vx_status vx_linear_f32(const float *x, int64_t n, int64_t in_f, const float *w, const float *b, int64_t out_f,
                        float *y, int relu, void *stream) {
    return guarded([&] { vx::linear_f32(x, n, in_f, w, b, out_f, y, relu != 0, (hipStream_t)stream); });
}

int64_t vx_subsampling_frames(int64_t t, int64_t k, int64_t s) { return vx::subsampling_frames(t, k, s); }

int64_t vx_subsampling_scratch_floats(int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s) {
    return vx::subsampling_scratch_floats(t, nm, c, k, s);
}

vx_status vx_subsampling(const float *feats, int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s,
                         const float *conv0_w, const float *conv0_b, const float *dw_w, const float *dw_b,
                         const float *pw_w, const float *pw_b, const float *lin_w, const float *lin_b, int64_t d_model,
                         float *scratch, float *out, int64_t *t_out, void *stream) {
    return guarded([&] {
        const int64_t t3 = vx::subsampling(feats, t, nm, c, k, s, conv0_w, conv0_b, dw_w, dw_b, pw_w, pw_b, lin_w,
                                           lin_b, d_model, scratch, out, (hipStream_t)stream);
        if (t_out) *t_out = t3;
    });
}

vx_status vx_rel_pos_table(int64_t t, int64_t d, float *out) {
    return guarded([&] {
        vx::require(out != nullptr && t >= 1 && d > 0 && d % 2 == 0, "vx_rel_pos_table: bad arguments");
        vx::rel_pos_table(t, d, out);
    });
}

vx_status vx_check_activations(uint64_t *mismatch) {
    return guarded([&] {
        vx::require(mismatch != nullptr, "vx_check_activations: mismatch must not be NULL");
        vx::check_activations(mismatch);
    });
}

int64_t vx_attention_ws_bytes(int64_t t, int64_t d, int64_t h) {
    if (t < 1 || h < 1 || d != h * 128) return -1;
    return (int64_t)vx::attn_ws_bytes(t, d, h);
}

vx_status vx_attention_core(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                            const float *bias_u, const float *bias_v, float scaling, void *ws, float *ctx,
                            void *stream) {
    return guarded([&] {
        vx::attention_core(qkv, rel_k, t, d, h, bias_u, bias_v, scaling, ws, ctx, (hipStream_t)stream);
    });
}

vx_status vx_attention_core_noalloc(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                                    const float *bias_u, const float *bias_v, float scaling, float *ctx, void *stream) {
    return guarded([&] {
        vx::attention_core_noalloc(qkv, rel_k, t, d, h, bias_u, bias_v, scaling, ctx, (hipStream_t)stream);
    });
}

vx_status vx_attention_core_quantize(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                                     const float *bias_u, const float *bias_v, float scaling, void *ws, int64_t group,
                                     int8_t *q, float *scales_t, int32_t *gsum_t, void *stream) {
    return guarded([&] {
        vx::require(group == 128, "attention quantized output: 128-column groups (one per head)");
        vx::require(q && scales_t && gsum_t, "q, scales_t and gsum_t must not be NULL");
        vx::attention_core_seg(qkv, rel_k, 1, t, d, h, bias_u, bias_v, scaling, ws, nullptr, (hipStream_t)stream, q,
                               scales_t, gsum_t, d, nullptr, nullptr);
    });
}

vx_status vx_encoder_create(const vx_encoder_config *cfg, vx_encoder **enc) {
    return guarded([&] {
        vx::require(enc != nullptr, "output handle pointer must not be NULL");
        *enc = nullptr;
        *enc = vx::encoder_create(cfg);
    });
}

vx_status vx_encoder_set_layer(vx_encoder *enc, int64_t layer, const vx_layer_params *p) {
    return guarded([&] { vx::encoder_set_layer(enc, layer, p); });
}

vx_status vx_encoder_set_subsampling(vx_encoder *enc, const vx_subsampling_params *p) {
    return guarded([&] { vx::encoder_set_subsampling(enc, p); });
}

vx_status vx_encoder_use_graphs(vx_encoder *enc, int on) {
    return guarded([&] { vx::encoder_use_graphs(enc, on != 0); });
}

vx_status vx_encoder_set_profiling(vx_encoder *enc, int on) {
    return guarded([&] { vx::encoder_set_profiling(enc, on != 0); });
}

vx_status vx_encoder_take_profile(vx_encoder *enc, vx_encoder_profile *out) {
    return guarded([&] { vx::encoder_take_profile(enc, out); });
}

vx_status vx_encoder_memory(vx_encoder *enc, int64_t *workspace_bytes, int64_t *graphs) {
    return guarded([&] { vx::encoder_memory(enc, workspace_bytes, graphs); });
}

vx_status vx_encoder_forward(vx_encoder *enc, const float *x, float *out, int64_t t, void *stream) {
    return guarded([&] { vx::encoder_forward(enc, x, out, t, (hipStream_t)stream); });
}

vx_status vx_encoder_forward_feats(vx_encoder *enc, const float *feats, int64_t t_in, float *out, int64_t *t_out,
                                   void *stream) {
    return guarded([&] { vx::encoder_forward_feats(enc, feats, t_in, out, t_out, (hipStream_t)stream); });
}

vx_status vx_encoder_forward_batch(vx_encoder *enc, const float *x, float *out, int64_t nseg, int64_t t, void *stream) {
    return guarded([&] { vx::encoder_forward_batch(enc, x, out, nseg, t, (hipStream_t)stream); });
}

vx_status vx_encoder_forward_feats_batch(vx_encoder *enc, const float *feats, int64_t nseg, int64_t t_in, float *out,
                                         int64_t *t_out, void *stream) {
    return guarded([&] { vx::encoder_forward_feats_batch(enc, feats, nseg, t_in, out, t_out, (hipStream_t)stream); });
}

void vx_encoder_free(vx_encoder *enc) { vx::encoder_free(enc); }

}  // extern "C"
