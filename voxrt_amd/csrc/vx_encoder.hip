// vx_encoder.hip — the FastConformer encoder on one GPU, int8 path (the reference's CPU Encoder::forward with
// Precision::Int8, encoder.rs:800-857, and its GPU encoder surface GpuEncoder::{load, forward, forward_feats},
// metal/mod.rs:446-603).
//
// Load: every ternary linear is uploaded once (vx_tmat, repacked on the device), q|k|v stacked into one matrix
// (TernaryLinear::load_stacked, ternary_linear.rs:59-98), BatchNorm folded into the depthwise taps on the host
// (encoder.rs:548-573), LayerNorm and bias vectors copied to HBM.
//
// Forward for t frames:
//   per layer, in place on the residual stream x [t][d] (ConformerLayer::forward_profiled, encoder.rs:706-756):
//     ff1:  q = LNquant(x); h = silu(W1 q); x = fma(0.5, W2 quant(h), x)   (W1's GEMM writes quant(h) itself)
//     attn: q = LNquant(x); qkv = Wqkv q; rel = Wpos quant(pos); ctx = core(qkv, rel); x = fma(1, Wo quant(ctx), x)
//           (the core writes quant(ctx) itself)
//     conv: q = LNquant(x); g = Wpw1 q; hb = silu(dwconv_bn(glu(g))); x = fma(1, Wpw2 quant(hb), x)
//           (the depthwise-conv kernel writes quant(hb) itself)
//     ff2 as ff1; x' = LN_out(x) into the other half of a ping-pong pair.
//
// Memory and concurrency (GpuEncoder keeps one workspace behind a Mutex and grows it by 25 %, metal/mod.rs:449-460,
// 641-645): one workspace serves every frame count and segment count; it grows, to 1.25x what a call needs, only
// when a call needs more, after the previous forward has finished on the device. Each (frames, segments) pair's
// layer stack is captured once into a hipGraph on a private capture stream (nothing runs during a capture) and
// launched on the caller's stream; at most kMaxGraphs are kept, the least recently used dropped, and all of them
// when the workspace moves. Calls on one encoder are serialized by a mutex, and each forward's first command waits
// for the previous forward's completion event, so calls from several threads and streams never share the workspace
// on the device. The relative position table of every t is a slice of one table of kMaxFrames frames (row r of
// t's table holds position t-1-r, which is row r + kMaxFrames - t of the big one, value for value): it is built on
// the host once per encoder, and each forward quantizes its slice.
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "vx_internal.h"

namespace vx {
vx_tmat *upload_packed(const uint8_t *qweight, const void *scales, bool scales_f16, int64_t out, int64_t inp,
                       int64_t group);
void free_tmat(vx_tmat *h);
void gemm(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y,
          const float *bias, int ep, float alpha, int32_t *gs, int64_t r0, int64_t r1, int64_t t0, int64_t t1,
          hipStream_t st, int64_t cap_rows = 0);
void quantize_ln(const float *x, int64_t n, int64_t inp, int64_t group, const float *g, const float *b, int8_t *q,
                 float *scales_t, int32_t *gsum_t, hipStream_t stream);
void gemm_quant(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y_tmp,
                const float *bias, int ep, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t, hipStream_t st,
                int64_t cap_rows = 0);
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
void attention_prime();
int cu_count();
void attention_core_seg(const float *qkv, const float *rel_k, int64_t nseg, int64_t t, int64_t d, int64_t h,
                        const float *bias_u, const float *bias_v, float scaling, void *ws, float *ctx,
                        hipStream_t st, int8_t *q, float *scales_t, int32_t *gsum_t, int64_t rel_ld,
                        const int8_t *rq_pre, const float *rs_pre);
int64_t attn_rel_rows(int64_t t, int64_t h);
void attention_rel_quantize(const float *rel_k, int64_t nl, int64_t t, int64_t d, int64_t h, int64_t rel_ld,
                            int8_t *rq, float *rs, hipStream_t st);

constexpr int64_t kMaxFrames = 1024;  // frames per segment (the attention core's limit)
constexpr int64_t kMaxRows = 65535;   // segments * frames in one call
constexpr size_t kMaxGraphs = 8;      // captured layer stacks kept per encoder

namespace {

// Device allocation owned by the encoder.
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    explicit DevBuf(size_t n) {
        const hipError_t e = hipMalloc(&p, n ? n : 1);
        if (e != hipSuccess) {
            p = nullptr;
            throw Error(VX_ERR_OOM, std::string("hipMalloc(") + std::to_string(n) + "): " + hipGetErrorString(e));
        }
        bytes = n;
    }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p(o.p), bytes(o.bytes) {
        o.p = nullptr;
        o.bytes = 0;
    }
    DevBuf &operator=(DevBuf &&o) noexcept {
        std::swap(p, o.p);
        std::swap(bytes, o.bytes);
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
    size_t bytes() const { return q.bytes + s.bytes + g.bytes; }
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

// The one workspace of an encoder. Capacities: token rows (segments * frames) of the row buffers, position rows
// (2 * frames - 1) of the position buffers, attention workspace bytes, subsampling scratch floats.
struct EncWs {
    int64_t rows = 0, np = 0;
    size_t attn_bytes = 0;
    int64_t sub_floats = 0;
    DevBuf x[2], hbuf, qkv, rel_k, relq, rels, ctx, g2, hb, attn, sub_scratch;
    QBuf a, f, posq;
    size_t bytes() const {
        return x[0].bytes + x[1].bytes + hbuf.bytes + qkv.bytes + rel_k.bytes + relq.bytes + rels.bytes + ctx.bytes +
               g2.bytes + hb.bytes + attn.bytes + sub_scratch.bytes + a.bytes() + f.bytes() + posq.bytes();
    }
};

struct GraphSlot {
    hipGraphExec_t exec = nullptr;
    uint64_t used = 0;
};

// Device events around the sublayers of a profiled forward: (event, category the time since the previous one
// belongs to).
enum ProfCat { kProfFf, kProfAttn, kProfAttnCore, kProfConv, kProfNorm, kProfSub, kProfCats };

struct ProfMarks {
    std::vector<std::pair<hipEvent_t, int>> ev;
    hipStream_t st = nullptr;
    void mark(int cat) {
        hipEvent_t e = nullptr;
        hip_check(hipEventCreate(&e), "profile event");
        ev.emplace_back(e, cat);
        hip_check(hipEventRecord(e, st), "profile event record");
    }
    ~ProfMarks() {
        for (auto &p : ev) (void)hipEventDestroy(p.first);
    }
};

}  // namespace vx

struct vx_encoder {
    vx_encoder_config cfg;
    int device = -1;
    std::vector<std::unique_ptr<vx::EncLayer>> layers;
    // the relative_k_proj matrices of all layers stacked along the output rows (layer l: rows [l*d, (l+1)*d)),
    // built from the layers' host copies before the first forward after a change
    vx_tmat *pos_all = nullptr;
    bool pos_dirty = true;
    vx::DevBuf pos_table;  // float32 [2 * kMaxFrames - 1][d]: positions kMaxFrames-1 .. -(kMaxFrames-1)
    vx::DevBuf sub_w[8];
    bool sub_set = false;
    bool graphs = true;
    bool profiling = false;
    vx_encoder_profile prof{};
    vx::EncWs ws;
    std::map<std::pair<int64_t, int64_t>, vx::GraphSlot> graph_cache;  // by (frames, segments)
    uint64_t clock = 0;
    hipStream_t capture_stream = nullptr;
    hipEvent_t done = nullptr;  // recorded on the caller's stream at the end of every forward
    bool done_recorded = false;
    std::mutex mu;
    ~vx_encoder() {
        if (done_recorded) (void)hipEventSynchronize(done);
        for (auto &kv : graph_cache)
            if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
        if (pos_all) vx::free_tmat(pos_all);
        if (capture_stream) (void)hipStreamDestroy(capture_stream);
        if (done) (void)hipEventDestroy(done);
    }
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

// Waits until every forward enqueued so far has finished on the device (before buffers or graphs they use go).
void wait_idle(vx_encoder *e) {
    if (e->done_recorded) hip_check(hipEventSynchronize(e->done), "encoder: wait for the previous forward");
}

void drop_graphs(vx_encoder *e) {
    wait_idle(e);
    for (auto &kv : e->graph_cache)
        if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
    e->graph_cache.clear();
}

int64_t grown(int64_t need, int64_t limit) { return std::min(limit, need + need / 4); }

// Makes the workspace hold a forward of nseg segments of t frames (and sub_floats of subsampling scratch): buffers
// that are too small are replaced by ones 1.25x the need, after the device has finished with the old ones.
void ensure_workspace(vx_encoder *e, int64_t t, int64_t nseg, int64_t sub_floats) {
    const vx_encoder_config &c = e->cfg;
    EncWs &w = e->ws;
    const int64_t rows = nseg * t, np = 2 * t - 1;
    const size_t attn = attn_ws_bytes_seg(t, c.d, c.heads, nseg);
    const bool g_rows = rows > w.rows, g_np = np > w.np, g_attn = attn > w.attn_bytes, g_sub = sub_floats > w.sub_floats;
    if (!(g_rows || g_np || g_attn || g_sub)) return;
    drop_graphs(e);  // waits for the device; the graphs hold the old addresses
    const size_t f4 = sizeof(float);
    if (g_rows) {
        const int64_t n = grown(rows, kMaxRows);
        // the old buffers go first, so the peak is the new size, not old + new
        for (DevBuf *b : {&w.x[0], &w.x[1], &w.hbuf, &w.qkv, &w.ctx, &w.g2, &w.hb}) *b = DevBuf();
        w.a = QBuf();
        w.f = QBuf();
        for (auto &x : w.x) x = DevBuf((size_t)(n * c.d) * f4);
        w.hbuf = DevBuf((size_t)(n * c.ff) * f4);
        w.qkv = DevBuf((size_t)(n * 3 * c.d) * f4);
        w.ctx = DevBuf((size_t)(n * c.d) * f4);
        w.g2 = DevBuf((size_t)(n * 2 * c.d) * f4);
        w.hb = DevBuf((size_t)(n * c.d) * f4);
        w.a.alloc(n, c.d, c.group);
        w.f.alloc(n, c.ff, c.group);
        w.rows = n;
    }
    if (g_np) {
        const int64_t n = grown(np, 2 * kMaxFrames - 1);
        w.rel_k = DevBuf();
        w.relq = DevBuf();
        w.rels = DevBuf();
        w.posq = QBuf();
        w.rel_k = DevBuf((size_t)(n * c.n_layers * c.d) * f4);  // [np][n_layers * d]: every layer's projection
        // every layer's relative rows quantized for the attention: [n_layers][heads][rp][128] int8 and
        // [n_layers][heads][rp] scales, rp = up16(np) + 16 at this capacity
        const int64_t rrows = c.heads * ((n + 15) / 16 * 16 + 16);
        w.relq = DevBuf((size_t)(c.n_layers * rrows * (c.d / c.heads)));
        w.rels = DevBuf((size_t)(c.n_layers * rrows) * f4);
        w.posq.alloc(n, c.d, c.group);
        w.np = n;
    }
    if (g_attn) {
        const size_t n = attn + attn / 4;
        w.attn = DevBuf();
        w.attn = DevBuf(n);
        w.attn_bytes = n;
    }
    if (g_sub) {
        const int64_t n = sub_floats + sub_floats / 4;
        w.sub_scratch = DevBuf();
        w.sub_scratch = DevBuf((size_t)n * f4);
        w.sub_floats = n;
    }
}

// cap: the rows that a and y hold in the workspace (at least n), which lets the streaming kernel run a last
// partial tile
void gemm_full(const vx_tmat *w, const QBuf &a, int64_t n, float *y, int ep, float alpha, int64_t cap,
               hipStream_t st) {
    gemm(&w->m, a.q.as<int8_t>(), a.s.as<float>(), a.g.as<int32_t>(), n, y, nullptr, ep, alpha, nullptr, 0, w->m.out,
         0, n, st, cap);
}

// The layer stack of nseg segments of t frames on ws.x[0] (result in ws.x[n_layers % 2]). The token-row work runs
// over all nseg * t rows at once; the depthwise convolution and the attention stay inside each segment. With
// marks, an event is recorded after each sublayer (profiled forwards).
void run_layers(vx_encoder *e, int64_t t_seg, int64_t nseg, hipStream_t st, ProfMarks *marks) {
    const vx_encoder_config &c = e->cfg;
    EncWs &w = e->ws;
    const int64_t t = nseg * t_seg, np = 2 * t_seg - 1, d = c.d, G = c.group;
    const float scaling = 1.0f / std::sqrt((float)(d / c.heads));
    auto mark = [&](int cat) {
        if (marks) marks->mark(cat);
    };
    // t's position table: rows [kMaxFrames - t, kMaxFrames + t - 1) of the encoder's table, quantized once per
    // forward; then relative_k_proj of it for all layers in one GEMM (it depends on t and the weights only):
    // rel_k [np][n_layers * d], layer l's block at columns [l*d, (l+1)*d)
    quantize_ln(e->pos_table.as<float>() + (kMaxFrames - t_seg) * d, np, d, G, nullptr, nullptr, w.posq.q.as<int8_t>(),
                w.posq.s.as<float>(), w.posq.g.as<int32_t>(), st);
    const int64_t rel_ld = (int64_t)e->layers.size() * d, nl = (int64_t)e->layers.size();
    gemm_full(e->pos_all, w.posq, np, w.rel_k.as<float>(), VX_EP_STORE, 0.0f, w.np, st);
    // and the attention's quantization of those rows, for all layers in one launch
    const int64_t rrows = attn_rel_rows(t_seg, c.heads), dh = d / c.heads;
    attention_rel_quantize(w.rel_k.as<float>(), nl, t_seg, d, c.heads, rel_ld, w.relq.as<int8_t>(),
                           w.rels.as<float>(), st);
    mark(kProfAttn);
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
                       nullptr, VX_EP_SILU, G, w.f.q.as<int8_t>(), w.f.s.as<float>(), w.f.g.as<int32_t>(), st, w.rows);
            gemm_full(L.lin[w2], w.f, t, x, VX_EP_ADD_SCALED, 0.5f, w.rows, st);
            mark(kProfFf);
        };
        ffn(0, 0, 1);
        // attention
        lnq(1);
        gemm_full(L.lin[2], w.a, t, w.qkv.as<float>(), VX_EP_STORE, 0.0f, w.rows, st);
        mark(kProfAttn);
        if (G == 128) {  // a head's 128 channels are one group: the core writes the o-projection's activations
            attention_core_seg(w.qkv.as<float>(), w.rel_k.as<float>() + li * d, nseg, t_seg, d, c.heads,
                               L.bias_u.as<float>(), L.bias_v.as<float>(), scaling, w.attn.p, nullptr, st,
                               w.a.q.as<int8_t>(), w.a.s.as<float>(), w.a.g.as<int32_t>(), rel_ld,
                               w.relq.as<int8_t>() + li * rrows * dh, w.rels.as<float>() + li * rrows);
            mark(kProfAttnCore);
        } else {
            attention_core_seg(w.qkv.as<float>(), w.rel_k.as<float>() + li * d, nseg, t_seg, d, c.heads,
                               L.bias_u.as<float>(), L.bias_v.as<float>(), scaling, w.attn.p, w.ctx.as<float>(), st,
                               nullptr, nullptr, nullptr, rel_ld, w.relq.as<int8_t>() + li * rrows * dh,
                               w.rels.as<float>() + li * rrows);
            mark(kProfAttnCore);
            quant(w.ctx.as<float>(), d, w.a);
        }
        gemm_full(L.lin[3], w.a, t, x, VX_EP_ADD_SCALED, 1.0f, w.rows, st);
        mark(kProfAttn);
        // convolution module
        lnq(2);
        gemm_full(L.lin[5], w.a, t, w.g2.as<float>(), VX_EP_STORE, 0.0f, w.rows, st);
        if (G == 128 && d % 256 == 0) {  // the conv rows quantized for pw2 in the same kernel
            glu_dwconv_silu_quant_seg(w.g2.as<float>(), nseg, t_seg, d, c.kconv, L.dw_t.as<float>(),
                                      L.dw_bias.as<float>(), w.a.q.as<int8_t>(), w.a.s.as<float>(), w.a.g.as<int32_t>(),
                                      st);
        } else {
            glu_dwconv_silu_seg(w.g2.as<float>(), nseg, t_seg, d, c.kconv, L.dw_t.as<float>(), L.dw_bias.as<float>(),
                                w.hb.as<float>(), st);
            quant(w.hb.as<float>(), d, w.a);
        }
        gemm_full(L.lin[6], w.a, t, x, VX_EP_ADD_SCALED, 1.0f, w.rows, st);
        mark(kProfConv);
        ffn(3, 7, 8);
        if (li + 1 < e->layers.size()) {  // norm_out, then the next layer's first LayerNorm -> quantize
            EncLayer &Ln = *e->layers[li + 1];
            layer_norm_quantize_ln(x, t, d, L.ln_g[4].as<float>(), L.ln_b[4].as<float>(), xn, G,
                                   Ln.ln_g[0].as<float>(), Ln.ln_b[0].as<float>(), w.a.q.as<int8_t>(),
                                   w.a.s.as<float>(), w.a.g.as<int32_t>(), st);
        } else {
            layer_norm(x, t, d, L.ln_g[4].as<float>(), L.ln_b[4].as<float>(), xn, st);
        }
        mark(kProfNorm);
    }
}

// Weights ready for a forward: every layer set, the stacked position projection and the position table built.
void check_ready(vx_encoder *e) {
    for (size_t i = 0; i < e->layers.size(); i++)
        if (!e->layers[i]->set) throw Error(VX_ERR_INVALID, "encoder layer " + std::to_string(i) + " has no weights");
    const vx_encoder_config &c = e->cfg;
    if (e->pos_dirty) {  // stack the layers' relative_k_proj matrices (TernaryLinear::load_stacked's row order)
        std::vector<uint8_t> q;
        std::vector<uint16_t> s;
        for (auto &L : e->layers) {
            q.insert(q.end(), L->pos_q.begin(), L->pos_q.end());
            s.insert(s.end(), L->pos_s.begin(), L->pos_s.end());
        }
        vx_tmat *all = upload_packed(q.data(), s.data(), true, (int64_t)e->layers.size() * c.d, c.d, c.group);
        drop_graphs(e);
        if (e->pos_all) free_tmat(e->pos_all);
        e->pos_all = all;
        e->pos_dirty = false;
    }
    if (!e->pos_table.p) {
        std::vector<float> pos((size_t)((2 * kMaxFrames - 1) * c.d));
        rel_pos_table(kMaxFrames, c.d, pos.data());
        e->pos_table = upload(pos.data(), pos.size() * sizeof(float));
    }
}

// The encoder's device made current (the device current at creation; the one current at the first upload when
// none was then).
void make_current(vx_encoder *e) {
    int dev = -1;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (e->device < 0) e->device = dev;
    if (dev != e->device) hip_check(hipSetDevice(e->device), "hipSetDevice (the encoder's device)");
}

// The hipGraph of the layer stack of (t, nseg) on the current workspace, captured on the private capture stream if
// it is not cached (the capture records the launches; nothing runs).
hipGraphExec_t graph_for(vx_encoder *e, int64_t t, int64_t nseg) {
    const auto key = std::make_pair(t, nseg);
    auto it = e->graph_cache.find(key);
    if (it != e->graph_cache.end()) {
        it->second.used = ++e->clock;
        return it->second.exec;
    }
    if (e->graph_cache.size() >= kMaxGraphs) {  // drop the least recently used
        auto lru = e->graph_cache.begin();
        for (auto i = e->graph_cache.begin(); i != e->graph_cache.end(); ++i)
            if (i->second.used < lru->second.used) lru = i;
        wait_idle(e);
        (void)hipGraphExecDestroy(lru->second.exec);
        e->graph_cache.erase(lru);
    }
    if (!e->capture_stream)
        hip_check(hipStreamCreateWithFlags(&e->capture_stream, hipStreamNonBlocking), "encoder capture stream");
    // one-time per-device set-up that must not happen inside a capture
    attention_prime();
    (void)cu_count();
    hipGraph_t g = nullptr;
    hip_check(hipStreamBeginCapture(e->capture_stream, hipStreamCaptureModeThreadLocal), "encoder graph capture");
    try {
        run_layers(e, t, nseg, e->capture_stream, nullptr);
    } catch (...) {
        (void)hipStreamEndCapture(e->capture_stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    hip_check(hipStreamEndCapture(e->capture_stream, &g), "encoder graph capture end");
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    hip_check(ie, "encoder graph instantiate");
    e->graph_cache[key] = GraphSlot{exec, ++e->clock};
    return exec;
}

// Orders this forward after the previous one (which may have been on another stream).
void begin_forward(vx_encoder *e, hipStream_t st) {
    if (!e->done) hip_check(hipEventCreateWithFlags(&e->done, hipEventDisableTiming), "encoder event");
    if (e->done_recorded) hip_check(hipStreamWaitEvent(st, e->done, 0), "encoder: order after the previous forward");
}

void end_forward(vx_encoder *e, hipStream_t st) {
    hip_check(hipEventRecord(e->done, st), "encoder completion event");
    e->done_recorded = true;
}

// Accumulates a profiled forward's sublayer times (the events it recorded) into e->prof.
void add_profile(vx_encoder *e, ProfMarks &m, hipEvent_t start) {
    if (m.ev.empty()) return;
    hip_check(hipEventSynchronize(m.ev.back().first), "profile wait");
    double cat[kProfCats] = {};
    hipEvent_t prev = start;
    for (auto &p : m.ev) {
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, prev, p.first), "profile elapsed time");
        cat[p.second] += ms;
        prev = p.first;
    }
    float total = 0.0f;
    hip_check(hipEventElapsedTime(&total, start, m.ev.back().first), "profile elapsed time");
    vx_encoder_profile &P = e->prof;
    P.total_ms += total;
    P.subsampling_ms += cat[kProfSub];
    P.ff_ms += cat[kProfFf];
    P.attn_ms += cat[kProfAttn] + cat[kProfAttnCore];
    P.attn_core_ms += cat[kProfAttnCore];
    P.conv_ms += cat[kProfConv];
    P.norm_ms += cat[kProfNorm];
    P.forwards += 1;
}

// x (device [nseg][t][d]) -> the encoder output (device [nseg][t][d]), both caller buffers (they may alias).
// feats (device [nseg][t_in][n_mels]) when not NULL: the subsampling runs first, into x_out, which then feeds the
// layers. The caller holds e->mu.
void forward_locked(vx_encoder *e, const float *feats, int64_t t_in, const float *x_in, float *x_out, int64_t t,
                    int64_t nseg, hipStream_t st) {
    make_current(e);
    check_ready(e);
    require(t >= 1 && t <= kMaxFrames, "encoder: 1 <= t <= 1024 frames");
    require(nseg >= 1 && nseg * t <= kMaxRows, "encoder: 1 <= segments, segments * t <= 65535");
    const vx_encoder_config &c = e->cfg;
    const int64_t sub_floats =
        feats ? nseg * subsampling_scratch_floats(t_in, c.n_mels, c.sub_channels, c.sub_kernel, c.sub_stride) : 0;
    ensure_workspace(e, t, nseg, sub_floats);
    EncWs &w = e->ws;
    begin_forward(e, st);
    ProfMarks marks;
    marks.st = st;
    hipEvent_t start = nullptr;
    if (e->profiling) {
        hip_check(hipEventCreate(&start), "profile event");
        hip_check(hipEventRecord(start, st), "profile event record");
    }
    try {
        if (feats) {
            subsampling_seg(feats, nseg, t_in, c.n_mels, c.sub_channels, c.sub_kernel, c.sub_stride,
                            e->sub_w[0].as<float>(), e->sub_w[1].as<float>(), e->sub_w[2].as<float>(),
                            e->sub_w[3].as<float>(), e->sub_w[4].as<float>(), e->sub_w[5].as<float>(),
                            e->sub_w[6].as<float>(), e->sub_w[7].as<float>(), c.d, w.sub_scratch.as<float>(), x_out,
                            st);
            if (e->profiling) marks.mark(kProfSub);
            x_in = x_out;
        }
        const size_t bytes = (size_t)(nseg * t * c.d) * sizeof(float);
        hip_check(hipMemcpyAsync(w.x[0].p, x_in, bytes, hipMemcpyDeviceToDevice, st), "encoder input copy");
        if (e->profiling) {
            run_layers(e, t, nseg, st, &marks);
        } else if (e->graphs) {
            hip_check(hipGraphLaunch(graph_for(e, t, nseg), st), "encoder graph launch");
        } else {
            run_layers(e, t, nseg, st, nullptr);
        }
        hip_check(hipMemcpyAsync(x_out, w.x[e->layers.size() % 2].p, bytes, hipMemcpyDeviceToDevice, st),
                  "encoder output copy");
    } catch (...) {
        end_forward(e, st);
        if (start) (void)hipEventDestroy(start);
        throw;
    }
    end_forward(e, st);
    if (e->profiling) {
        try {
            add_profile(e, marks, start);
        } catch (...) {
            (void)hipEventDestroy(start);
            throw;
        }
        (void)hipEventDestroy(start);
    }
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
    if (hipGetDevice(&e->device) != hipSuccess) {  // no device yet: bound at the first upload
        (void)hipGetLastError();
        e->device = -1;
    }
    for (int64_t i = 0; i < c.n_layers; i++) e->layers.push_back(std::make_unique<EncLayer>());
    return e.release();
}

void encoder_free(vx_encoder *e) { delete e; }

void encoder_use_graphs(vx_encoder *e, bool on) {
    require(e != nullptr, "NULL encoder");
    std::lock_guard<std::mutex> lock(e->mu);
    e->graphs = on;
}

void encoder_set_profiling(vx_encoder *e, bool on) {
    require(e != nullptr, "NULL encoder");
    std::lock_guard<std::mutex> lock(e->mu);
    e->profiling = on;
}

void encoder_take_profile(vx_encoder *e, vx_encoder_profile *out) {
    require(e != nullptr && out != nullptr, "NULL argument");
    std::lock_guard<std::mutex> lock(e->mu);
    *out = e->prof;
    e->prof = vx_encoder_profile{};
}

void encoder_memory(vx_encoder *e, int64_t *workspace_bytes, int64_t *graphs) {
    require(e != nullptr, "NULL encoder");
    std::lock_guard<std::mutex> lock(e->mu);
    if (workspace_bytes) *workspace_bytes = (int64_t)e->ws.bytes();
    if (graphs) *graphs = (int64_t)e->graph_cache.size();
}

void encoder_set_layer(vx_encoder *e, int64_t li, const vx_layer_params *p) {
    require(e && p, "NULL argument");
    std::lock_guard<std::mutex> lock(e->mu);
    require(li >= 0 && li < (int64_t)e->layers.size(), "layer index out of range");
    make_current(e);
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
    // the captured graphs hold the old layer's weight addresses; the old layer may still be in use on the device
    drop_graphs(e);
    e->pos_dirty = true;
    L->set = true;
    e->layers[(size_t)li] = std::move(L);
}

void encoder_set_subsampling(vx_encoder *e, const vx_subsampling_params *p) {
    require(e && p, "NULL argument");
    std::lock_guard<std::mutex> lock(e->mu);
    make_current(e);
    const vx_encoder_config &c = e->cfg;
    require(c.n_mels > 0 && c.sub_channels > 0 && c.sub_kernel > 0 && c.sub_stride > 0, "encoder: no subsampling shape");
    const int64_t C = c.sub_channels, k = c.sub_kernel;
    int64_t f3 = c.n_mels;
    for (int i = 0; i < 3; i++) f3 = (f3 + 2 * ((k - 1) / 2) - k) / c.sub_stride + 1;
    const size_t f4 = sizeof(float);
    const void *src[8] = {p->conv0_w, p->conv0_b, p->dw_w, p->dw_b, p->pw_w, p->pw_b, p->lin_w, p->lin_b};
    const size_t n[8] = {(size_t)(k * k * C), (size_t)C, (size_t)(2 * k * k * C), (size_t)(2 * C), (size_t)(2 * C * C),
                         (size_t)(2 * C), (size_t)(c.d * f3 * C), (size_t)c.d};
    DevBuf next[8];
    for (int i = 0; i < 8; i++) next[i] = upload(src[i], n[i] * f4);
    wait_idle(e);  // a forward still on the device may read the old weights
    for (int i = 0; i < 8; i++) e->sub_w[i] = std::move(next[i]);
    e->sub_set = true;
}

void encoder_forward_feats_batch(vx_encoder *e, const float *feats, int64_t nseg, int64_t t_in, float *out,
                                 int64_t *t_out, hipStream_t st) {
    require(e && feats && out, "NULL argument");
    std::lock_guard<std::mutex> lock(e->mu);
    require(e->sub_set, "encoder: subsampling weights not set");
    const vx_encoder_config &c = e->cfg;
    const int64_t t = subsampling_frames(t_in, c.sub_kernel, c.sub_stride);
    require(t >= 1 && t <= kMaxFrames, "encoder: 1 <= subsampled frames <= 1024");
    forward_locked(e, feats, t_in, nullptr, out, t, nseg, st);
    if (t_out) *t_out = t;
}

void encoder_forward_feats(vx_encoder *e, const float *feats, int64_t t_in, float *out, int64_t *t_out,
                           hipStream_t st) {
    encoder_forward_feats_batch(e, feats, 1, t_in, out, t_out, st);
}

void encoder_forward_batch(vx_encoder *e, const float *x, float *out, int64_t nseg, int64_t t, hipStream_t st) {
    require(e && x && out, "NULL argument");
    std::lock_guard<std::mutex> lock(e->mu);
    forward_locked(e, nullptr, 0, x, out, t, nseg, st);
}

void encoder_forward(vx_encoder *e, const float *x, float *out, int64_t t, hipStream_t st) {
    encoder_forward_batch(e, x, out, 1, t, st);
}

}  // namespace vx
