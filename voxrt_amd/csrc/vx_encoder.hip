// vx_encoder.hip — the FastConformer encoder on one GPU, int8 path (the reference's CPU Encoder::forward with
// Precision::Int8, encoder.rs:800-857, and its GPU encoder surface GpuEncoder::{load, forward, forward_feats},
// metal/mod.rs:446-603).
//
// Load: every ternary linear is uploaded once (vx_tmat, repacked on the device), q|k|v stacked into one matrix
// (TernaryLinear::load_stacked, ternary_linear.rs:59-98), BatchNorm folded into the depthwise taps on the host
// (encoder.rs:548-573), LayerNorm and bias vectors copied to HBM.
//
// Forward for t frames (a workspace per distinct t is kept; the relative position table of t is computed on the
// host once, uploaded and quantized once, since every layer's relative_k_proj consumes the same table):
//   per layer, in place on the residual stream x [t][d] (ConformerLayer::forward_profiled, encoder.rs:706-756):
//     ff1:  q = LNquant(x); h = silu(W1 q); x = fma(0.5, W2 quant(h), x)   (W1's GEMM writes quant(h) itself)
//     attn: q = LNquant(x); qkv = Wqkv q; rel = Wpos quant(pos); ctx = core(qkv, rel); x = fma(1, Wo quant(ctx), x)
//           (the core writes quant(ctx) itself)
//     conv: q = LNquant(x); g = Wpw1 q; hb = silu(dwconv_bn(glu(g))); x = fma(1, Wpw2 quant(hb), x)
//           (the depthwise-conv kernel writes quant(hb) itself)
//     ff2 as ff1; x' = LN_out(x) into the other half of a ping-pong pair.
//   All of it is stream-ordered kernels on device buffers; with graphs on, the layer stack of each t is captured
//   once into a hipGraph and replayed (no memset nodes are recorded: every buffer is written by a kernel).
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <vector>

#include "vx_internal.h"

namespace vx {
vx_tmat *upload_packed(const uint8_t *qweight, const void *scales, bool scales_f16, int64_t out, int64_t inp,
                       int64_t group);
void free_tmat(vx_tmat *h);
void gemm(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y,
          const float *bias, int ep, float alpha, int32_t *gs, int64_t r0, int64_t r1, int64_t t0, int64_t t1,
          hipStream_t st);
void quantize_ln(const float *x, int64_t n, int64_t inp, int64_t group, const float *g, const float *b, int8_t *q,
                 float *scales_t, int32_t *gsum_t, hipStream_t stream);
void gemm_quant(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y_tmp,
                const float *bias, int ep, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t, hipStream_t st);
void layer_norm(const float *x, int64_t n, int64_t d, const float *g, const float *b, float *y, hipStream_t stream);
void layer_norm_quantize_ln(const float *x, int64_t n, int64_t d, const float *g, const float *b, float *y,
                            int64_t group, const float *g2, const float *b2, int8_t *q, float *scales_t,
                            int32_t *gsum_t, hipStream_t stream);
void glu_dwconv_silu_seg(const float *g, int64_t nseg, int64_t t, int64_t d, int64_t k, const float *w_t,
                         const float *bias, float *out, hipStream_t st);
void glu_dwconv_silu_quant_seg(const float *g, int64_t nseg, int64_t t, int64_t d, int64_t k, const float *w_t,
                               const float *bias, int8_t *q, float *scales_t, int32_t *gsum_t, hipStream_t st);
int64_t subsampling_seg(const float *feats, int64_t nseg, int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s,
                        const float *conv0_w, const float *conv0_b, const float *dw_w, const float *dw_b,
                        const float *pw_w, const float *pw_b, const float *lin_w, const float *lin_b,
                        int64_t d_model, float *scratch, float *out, hipStream_t st);
int64_t subsampling_frames(int64_t t, int64_t k, int64_t s);
int64_t subsampling_scratch_floats(int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s);
void fold_bn(const float *dw, const float *gamma, const float *beta, const float *mean, const float *var, int64_t d,
             int64_t k, float *dw_t, float *dw_bias);
void rel_pos_table(int64_t t, int64_t d, float *out);
size_t attn_ws_bytes_seg(int64_t t, int64_t d, int64_t h, int64_t nseg);
void attention_core_seg(const float *qkv, const float *rel_k, int64_t nseg, int64_t t, int64_t d, int64_t h,
                        const float *bias_u, const float *bias_v, float scaling, void *ws, float *ctx,
                        hipStream_t st, int8_t *q, float *scales_t, int32_t *gsum_t, int64_t rel_ld);

namespace {

// Device allocation owned by the encoder.
struct DevBuf {
    void *p = nullptr;
    DevBuf() = default;
    explicit DevBuf(size_t bytes) {
        const hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
        if (e != hipSuccess) {
            p = nullptr;
            throw Error(VX_ERR_OOM, std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e));
        }
    }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p(o.p) { o.p = nullptr; }
    DevBuf &operator=(DevBuf &&o) noexcept {
        std::swap(p, o.p);
        return *this;
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    template <class T>
    T *as() const {
        return (T *)p;
    }
};

DevBuf upload(const void *host, size_t bytes) {
    require(host != nullptr, "encoder parameter pointer must not be NULL");
    DevBuf b(bytes);
    hip_check(hipMemcpy(b.p, host, bytes, hipMemcpyHostToDevice), "encoder parameter upload");
    return b;
}

struct QBuf {  // one quantized activation block: q [n][inp], scales_t / gsum_t [inp/group][npad(n)]
    DevBuf q, s, g;
    void alloc(int64_t n, int64_t inp, int64_t group) {
        const int64_t np = (n + 15) / 16 * 16;
        q = DevBuf((size_t)(n * inp));
        s = DevBuf((size_t)(inp / group * np * 4));
        g = DevBuf((size_t)(inp / group * np * 4));
    }
};

}  // namespace

struct EncLayer {
    vx_tmat *lin[9] = {};
    std::vector<uint8_t> pos_q;   // relative_k_proj packed rows and f16 scales (host), for the stacked projection
    std::vector<uint16_t> pos_s;
    DevBuf ln_g[5], ln_b[5], bias_u, bias_v, dw_t, dw_bias;
    bool set = false;
    ~EncLayer() {
        for (auto *w : lin) free_tmat(w);
    }
};

struct EncWs {  // everything one forward of nseg segments of t frames touches
    int64_t t = 0, nseg = 1, np = 0;
    DevBuf x[2], hbuf, qkv, rel_k, ctx, g2, hb, pos, attn, sub_scratch, feats;
    QBuf a, f, posq;
    int64_t t_in = 0;
    hipGraphExec_t exec = nullptr;
    hipStream_t exec_stream = nullptr;
    ~EncWs() {
        if (exec) (void)hipGraphExecDestroy(exec);
    }
};

}  // namespace vx

struct vx_encoder {
    vx_encoder_config cfg;
    std::vector<std::unique_ptr<vx::EncLayer>> layers;
    // the relative_k_proj matrices of all layers stacked along the output rows (layer l: rows [l*d, (l+1)*d)),
    // built from the layers' host copies before the first forward after a change
    vx_tmat *pos_all = nullptr;
    bool pos_dirty = true;
    ~vx_encoder() {
        if (pos_all) vx::free_tmat(pos_all);
    }
    vx::DevBuf sub_w[8];
    bool sub_set = false;
    bool graphs = true;
    std::map<std::pair<int64_t, int64_t>, std::unique_ptr<vx::EncWs>> ws;  // by (frames, segments)
};

namespace vx {

namespace {

const int kLinOut[9] = {0, 1, 2, 1, 1, 3, 1, 0, 1};  // 0: ff, 1: d, 2: 3d, 3: 2d
const int kLinInp[9] = {1, 0, 1, 1, 1, 1, 1, 1, 0};  // 0: ff, 1: d

int64_t dim_of(const vx_encoder_config &c, int code) {
    switch (code) {
        case 0: return c.ff;
        case 1: return c.d;
        case 2: return 3 * c.d;
        default: return 2 * c.d;
    }
}

// Workspace of nseg segments of t frames: the token-row buffers hold nseg * t rows; the relative position table,
// its projection and the quantized table depend on t only and are shared by the segments.
EncWs &workspace(vx_encoder *e, int64_t t, int64_t nseg) {
    auto it = e->ws.find({t, nseg});
    if (it != e->ws.end()) return *it->second;
    const vx_encoder_config &c = e->cfg;
    auto w = std::make_unique<EncWs>();
    w->t = t;
    w->nseg = nseg;
    w->np = 2 * t - 1;
    const int64_t n = nseg * t;
    const size_t f4 = sizeof(float);
    for (auto &x : w->x) x = DevBuf((size_t)(n * c.d) * f4);
    w->hbuf = DevBuf((size_t)(n * c.ff) * f4);
    w->qkv = DevBuf((size_t)(n * 3 * c.d) * f4);
    w->rel_k = DevBuf((size_t)(w->np * c.n_layers * c.d) * f4);  // [np][n_layers * d]: every layer's projection
    w->ctx = DevBuf((size_t)(n * c.d) * f4);
    w->g2 = DevBuf((size_t)(n * 2 * c.d) * f4);
    w->hb = DevBuf((size_t)(n * c.d) * f4);
    w->attn = DevBuf(attn_ws_bytes_seg(t, c.d, c.heads, nseg));
    w->a.alloc(n, c.d, c.group);
    w->f.alloc(n, c.ff, c.group);
    w->posq.alloc(w->np, c.d, c.group);
    // the relative position table of t frames, quantized once (its quantization is input-independent)
    std::vector<float> pos((size_t)(w->np * c.d));
    rel_pos_table(t, c.d, pos.data());
    w->pos = upload(pos.data(), pos.size() * f4);
    quantize_ln(w->pos.as<float>(), w->np, c.d, c.group, nullptr, nullptr, w->posq.q.as<int8_t>(),
                w->posq.s.as<float>(), w->posq.g.as<int32_t>(), nullptr);
    hip_check(hipDeviceSynchronize(), "position table quantization");
    EncWs &ref = *w;
    e->ws[{t, nseg}] = std::move(w);
    return ref;
}

void gemm_full(const vx_tmat *w, const QBuf &a, int64_t n, float *y, int ep, float alpha, hipStream_t st) {
    gemm(&w->m, a.q.as<int8_t>(), a.s.as<float>(), a.g.as<int32_t>(), n, y, nullptr, ep, alpha, nullptr, 0, w->m.out,
         0, n, st);
}

// The layer stack on ws.x[0] (result in ws.x[n_layers % 2]). The token-row work runs over all nseg * t rows at
// once; the depthwise convolution and the attention stay inside each segment.
void run_layers(vx_encoder *e, EncWs &w, hipStream_t st) {
    const vx_encoder_config &c = e->cfg;
    const int64_t t = w.nseg * w.t, d = c.d, G = c.group;
    const float scaling = 1.0f / std::sqrt((float)(d / c.heads));
    // relative_k_proj of the position table for all layers in one GEMM (it depends on t and the weights only):
    // rel_k [np][n_layers * d], layer l's block at columns [l*d, (l+1)*d)
    const int64_t rel_ld = (int64_t)e->layers.size() * d;
    gemm_full(e->pos_all, w.posq, w.np, w.rel_k.as<float>(), VX_EP_STORE, 0.0f, st);
    for (size_t li = 0; li < e->layers.size(); li++) {
        EncLayer &L = *e->layers[li];
        float *x = w.x[li % 2].as<float>(), *xn = w.x[(li + 1) % 2].as<float>();
        auto lnq = [&](int norm) {
            quantize_ln(x, t, d, G, L.ln_g[norm].as<float>(), L.ln_b[norm].as<float>(), w.a.q.as<int8_t>(),
                        w.a.s.as<float>(), w.a.g.as<int32_t>(), st);
        };
        auto quant = [&](const float *src, int64_t inp, QBuf &dst) {
            quantize_ln(src, t, inp, G, nullptr, nullptr, dst.q.as<int8_t>(), dst.s.as<float>(), dst.g.as<int32_t>(),
                        st);
        };
        auto ffn = [&](int norm, int w1, int w2) {
            if (norm == 0 && li > 0) {
                // this layer's norm_feed_forward1 -> quantize ran with the previous layer's norm_out
            } else {
                lnq(norm);
            }
            // h = silu(W1 q) quantized for W2 in one call (up to 1024 rows the GEMM quantizes in its epilogue and
            // h never reaches memory; above, hbuf carries it)
            gemm_quant(&L.lin[w1]->m, w.a.q.as<int8_t>(), w.a.s.as<float>(), w.a.g.as<int32_t>(), t, w.hbuf.as<float>(),
                       nullptr, VX_EP_SILU, G, w.f.q.as<int8_t>(), w.f.s.as<float>(), w.f.g.as<int32_t>(), st);
            gemm_full(L.lin[w2], w.f, t, x, VX_EP_ADD_SCALED, 0.5f, st);
        };
        ffn(0, 0, 1);
        // attention
        lnq(1);
        gemm_full(L.lin[2], w.a, t, w.qkv.as<float>(), VX_EP_STORE, 0.0f, st);
        if (G == 128) {  // a head's 128 channels are one group: the core writes the o-projection's activations
            attention_core_seg(w.qkv.as<float>(), w.rel_k.as<float>() + li * d, w.nseg, w.t, d, c.heads,
                               L.bias_u.as<float>(), L.bias_v.as<float>(), scaling, w.attn.p, nullptr, st,
                               w.a.q.as<int8_t>(), w.a.s.as<float>(), w.a.g.as<int32_t>(), rel_ld);
        } else {
            attention_core_seg(w.qkv.as<float>(), w.rel_k.as<float>() + li * d, w.nseg, w.t, d, c.heads,
                               L.bias_u.as<float>(), L.bias_v.as<float>(), scaling, w.attn.p, w.ctx.as<float>(), st,
                               nullptr, nullptr, nullptr, rel_ld);
            quant(w.ctx.as<float>(), d, w.a);
        }
        gemm_full(L.lin[3], w.a, t, x, VX_EP_ADD_SCALED, 1.0f, st);
        // convolution module
        lnq(2);
        gemm_full(L.lin[5], w.a, t, w.g2.as<float>(), VX_EP_STORE, 0.0f, st);
        if (G == 128 && d % 256 == 0) {  // the conv rows quantized for pw2 in the same kernel
            glu_dwconv_silu_quant_seg(w.g2.as<float>(), w.nseg, w.t, d, c.kconv, L.dw_t.as<float>(),
                                      L.dw_bias.as<float>(), w.a.q.as<int8_t>(), w.a.s.as<float>(), w.a.g.as<int32_t>(),
                                      st);
        } else {
            glu_dwconv_silu_seg(w.g2.as<float>(), w.nseg, w.t, d, c.kconv, L.dw_t.as<float>(), L.dw_bias.as<float>(),
                                w.hb.as<float>(), st);
            quant(w.hb.as<float>(), d, w.a);
        }
        gemm_full(L.lin[6], w.a, t, x, VX_EP_ADD_SCALED, 1.0f, st);
        ffn(3, 7, 8);
        if (li + 1 < e->layers.size()) {  // norm_out, then the next layer's first LayerNorm -> quantize
            EncLayer &Ln = *e->layers[li + 1];
            layer_norm_quantize_ln(x, t, d, L.ln_g[4].as<float>(), L.ln_b[4].as<float>(), xn, G,
                                   Ln.ln_g[0].as<float>(), Ln.ln_b[0].as<float>(), w.a.q.as<int8_t>(),
                                   w.a.s.as<float>(), w.a.g.as<int32_t>(), st);
        } else {
            layer_norm(x, t, d, L.ln_g[4].as<float>(), L.ln_b[4].as<float>(), xn, st);
        }
    }
}

void check_ready(vx_encoder *e) {
    for (size_t i = 0; i < e->layers.size(); i++)
        if (!e->layers[i]->set) throw Error(VX_ERR_INVALID, "encoder layer " + std::to_string(i) + " has no weights");
    if (e->pos_dirty) {  // stack the layers' relative_k_proj matrices (TernaryLinear::load_stacked's row order)
        const vx_encoder_config &c = e->cfg;
        std::vector<uint8_t> q;
        std::vector<uint16_t> s;
        for (auto &L : e->layers) {
            q.insert(q.end(), L->pos_q.begin(), L->pos_q.end());
            s.insert(s.end(), L->pos_s.begin(), L->pos_s.end());
        }
        vx_tmat *all = upload_packed(q.data(), s.data(), true, (int64_t)e->layers.size() * c.d, c.d, c.group);
        if (e->pos_all) free_tmat(e->pos_all);
        e->pos_all = all;
        e->pos_dirty = false;
    }
}

// x (device [nseg][t][d]) -> the encoder output (device [nseg][t][d]), both caller buffers (they may alias).
void forward_layers(vx_encoder *e, const float *x_in, float *x_out, int64_t t, int64_t nseg, hipStream_t st) {
    check_ready(e);
    require(t >= 1 && t <= 1024, "encoder: 1 <= t <= 1024 frames");
    require(nseg >= 1 && nseg * t <= 65535, "encoder: 1 <= segments, segments * t <= 65535");
    EncWs &w = workspace(e, t, nseg);
    const size_t bytes = (size_t)(nseg * t * e->cfg.d) * sizeof(float);
    hip_check(hipMemcpyAsync(w.x[0].p, x_in, bytes, hipMemcpyDeviceToDevice, st), "encoder input copy");
    if (e->graphs && st != nullptr) {  // the legacy NULL stream cannot be captured
        if (!w.exec || w.exec_stream != st) {
            if (w.exec) {
                (void)hipGraphExecDestroy(w.exec);
                w.exec = nullptr;
            }
            // one eager pass first (one-time work such as kernel attribute setup happens outside the capture)
            run_layers(e, w, st);
            hipGraph_t g = nullptr;
            hip_check(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "encoder graph capture begin");
            try {
                run_layers(e, w, st);
            } catch (...) {
                (void)hipStreamEndCapture(st, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            hip_check(hipStreamEndCapture(st, &g), "encoder graph capture end");
            const hipError_t ie = hipGraphInstantiate(&w.exec, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            hip_check(ie, "encoder graph instantiate");
            w.exec_stream = st;
            // the eager pass consumed the input copy: restore it
            hip_check(hipMemcpyAsync(w.x[0].p, x_in, bytes, hipMemcpyDeviceToDevice, st), "encoder input copy");
        }
        hip_check(hipGraphLaunch(w.exec, st), "encoder graph launch");
    } else {
        run_layers(e, w, st);
    }
    hip_check(hipMemcpyAsync(x_out, w.x[e->layers.size() % 2].p, bytes, hipMemcpyDeviceToDevice, st),
              "encoder output copy");
}

}  // namespace
}  // namespace vx

namespace vx {

vx_encoder *encoder_create(const vx_encoder_config *cfg) {
    require(cfg != nullptr, "NULL config");
    const vx_encoder_config &c = *cfg;
    require(c.d > 0 && c.heads > 0 && c.d == c.heads * 128, "encoder: d must be heads * 128");
    require(c.ff > 0 && c.kconv > 0 && c.kconv % 2 == 1 && c.n_layers > 0, "encoder: bad ff / kconv / layers");
    require(c.group > 0 && c.group % 64 == 0 && c.d % c.group == 0 && c.ff % c.group == 0,
            "encoder: group must divide d and ff and be a multiple of 64");
    auto e = std::make_unique<vx_encoder>();
    e->cfg = c;
    for (int64_t i = 0; i < c.n_layers; i++) e->layers.push_back(std::make_unique<EncLayer>());
    return e.release();
}

void encoder_free(vx_encoder *e) { delete e; }

void encoder_use_graphs(vx_encoder *e, bool on) {
    require(e != nullptr, "NULL encoder");
    e->graphs = on;
}

}  // namespace vx

namespace vx {

void encoder_set_layer(vx_encoder *e, int64_t li, const vx_layer_params *p) {
    require(e && p, "NULL argument");
    require(li >= 0 && li < (int64_t)e->layers.size(), "layer index out of range");
    const vx_encoder_config &c = e->cfg;
    auto L = std::make_unique<EncLayer>();
    for (int i = 0; i < 9; i++)
        L->lin[i] = upload_packed(p->qweight[i], p->scales_f16[i], true, dim_of(c, kLinOut[i]), dim_of(c, kLinInp[i]),
                                  c.group);
    const size_t dv = (size_t)c.d * sizeof(float);
    for (int i = 0; i < 5; i++) {
        L->ln_g[i] = upload(p->ln_gamma[i], dv);
        L->ln_b[i] = upload(p->ln_beta[i], dv);
    }
    L->bias_u = upload(p->bias_u, dv);
    L->bias_v = upload(p->bias_v, dv);
    std::vector<float> wt((size_t)(c.kconv * c.d)), bias((size_t)c.d);
    require(p->dw && p->bn_gamma && p->bn_beta && p->bn_mean && p->bn_var, "depthwise / BatchNorm parameter is NULL");
    fold_bn(p->dw, p->bn_gamma, p->bn_beta, p->bn_mean, p->bn_var, c.d, c.kconv, wt.data(), bias.data());
    L->dw_t = upload(wt.data(), wt.size() * sizeof(float));
    L->dw_bias = upload(bias.data(), dv);
    const size_t pq = (size_t)(c.d * ((c.d + 4) / 5)), ps = (size_t)(c.d * (c.d / c.group));
    L->pos_q.assign(p->qweight[4], p->qweight[4] + pq);
    L->pos_s.assign(p->scales_f16[4], p->scales_f16[4] + ps);
    e->pos_dirty = true;
    L->set = true;
    e->layers[(size_t)li] = std::move(L);
    for (auto &kv : e->ws)
        if (kv.second->exec) {
            (void)hipGraphExecDestroy(kv.second->exec);
            kv.second->exec = nullptr;
        }
}

void encoder_set_subsampling(vx_encoder *e, const vx_subsampling_params *p) {
    require(e && p, "NULL argument");
    const vx_encoder_config &c = e->cfg;
    require(c.n_mels > 0 && c.sub_channels > 0 && c.sub_kernel > 0 && c.sub_stride > 0, "encoder: no subsampling shape");
    const int64_t C = c.sub_channels, k = c.sub_kernel;
    int64_t f3 = c.n_mels;
    for (int i = 0; i < 3; i++) f3 = (f3 + 2 * ((k - 1) / 2) - k) / c.sub_stride + 1;
    const size_t f4 = sizeof(float);
    const void *src[8] = {p->conv0_w, p->conv0_b, p->dw_w, p->dw_b, p->pw_w, p->pw_b, p->lin_w, p->lin_b};
    const size_t n[8] = {(size_t)(k * k * C), (size_t)C, (size_t)(2 * k * k * C), (size_t)(2 * C), (size_t)(2 * C * C),
                         (size_t)(2 * C), (size_t)(c.d * f3 * C), (size_t)c.d};
    for (int i = 0; i < 8; i++) e->sub_w[i] = upload(src[i], n[i] * f4);
    e->sub_set = true;
}

void encoder_forward_feats_batch(vx_encoder *e, const float *feats, int64_t nseg, int64_t t_in, float *out,
                                 int64_t *t_out, hipStream_t st) {
    require(e && feats && out, "NULL argument");
    require(e->sub_set, "encoder: subsampling weights not set");
    const vx_encoder_config &c = e->cfg;
    const int64_t t = subsampling_frames(t_in, c.sub_kernel, c.sub_stride);
    require(t >= 1 && t <= 1024, "encoder: 1 <= subsampled frames <= 1024");
    require(nseg >= 1 && nseg * t <= 65535, "encoder: 1 <= segments, segments * frames <= 65535");
    EncWs &w = workspace(e, t, nseg);
    const int64_t scratch = subsampling_scratch_floats(t_in, c.n_mels, c.sub_channels, c.sub_kernel, c.sub_stride);
    if (w.t_in < t_in) {
        w.sub_scratch = DevBuf((size_t)(nseg * scratch) * sizeof(float));
        w.t_in = t_in;
    }
    subsampling_seg(feats, nseg, t_in, c.n_mels, c.sub_channels, c.sub_kernel, c.sub_stride, e->sub_w[0].as<float>(),
                    e->sub_w[1].as<float>(), e->sub_w[2].as<float>(), e->sub_w[3].as<float>(),
                    e->sub_w[4].as<float>(), e->sub_w[5].as<float>(), e->sub_w[6].as<float>(),
                    e->sub_w[7].as<float>(), c.d, w.sub_scratch.as<float>(), out, st);
    forward_layers(e, out, out, t, nseg, st);
    if (t_out) *t_out = t;
}

void encoder_forward_feats(vx_encoder *e, const float *feats, int64_t t_in, float *out, int64_t *t_out,
                           hipStream_t st) {
    encoder_forward_feats_batch(e, feats, 1, t_in, out, t_out, st);
}

void encoder_forward_batch(vx_encoder *e, const float *x, float *out, int64_t nseg, int64_t t, hipStream_t st) {
    require(e && x && out, "NULL argument");
    forward_layers(e, x, out, t, nseg, st);
}

void encoder_forward(vx_encoder *e, const float *x, float *out, int64_t t, hipStream_t st) {
    encoder_forward_batch(e, x, out, 1, t, st);
}

}  // namespace vx
