// vx_attn.hip — the int8 relative-position attention core of one layer (attn_core_int8, encoder.rs:317-534), all
// heads in two launches, equal to the CPU path bit for bit.
//
// Reference semantics, per head h (dh = 128 columns of q | k | v):
//   qu = q + bias_u, qv = q + bias_v, quantized per token in one group of dh (QuantAct::from_rows);
//   keys, relative positions (rows of the relative_k_proj output) and vT (one row per channel over the tokens,
//   zero-padded to t16) quantized per row in one group (TernaryMatrix::from_f32_rows, packed.rs:203-249);
//   S1[i][j] = fma((float)(qu_i . k_j), s_qu[i] * s_k[j], 0), S2[i][p] = fma((float)(qv_i . r_p), s_qv[i] * s_r[p], 0)
//   (single-group folds of kernels/mod.rs:166-210); score = S1[i][j] + S2[i][t-1-i+j];
//   e = exp_row_scaled(score, 1/sqrt(dh)) (tensor.rs:810-826: max of score*scale, exp_poly(score*scale - max), four
//   lane sums over quads, hsum4, the tail in order); the row e (zero-padded to t16) quantized in one group, its scale
//   multiplied by 1/sum; ctx[i][h*dh + c] = fma((float)(p_i . v_c), s_p[i] * s_v[c], 0).
//
// Kernels:
//   attn_prep_kernel  : the row items (one wavefront per 128-wide row: q+bias_u, q+bias_v, k (tokens), relative
//                       rows; quantize) and the vT rows (a workgroup per 16 channels of a head: the columns of v
//                       over the tokens, quantized) in one launch.
//   attn_core_kernel  : one workgroup per (head, 16 query rows). Content scores for all keys through
//                       v_mfma_i32_16x16x64_i8 into LDS, the position band [t-1-i_max, 2t-2-i0] through the same MFMA
//                       added to them in place; softmax in LDS (the four running sums per row on four lanes, so the
//                       order is the reference's); the probabilities quantized into LDS; P . vT through the same
//                       MFMA; ctx written in place in [t][d].
#include <atomic>
#include <string>

#include "vx_internal.h"

namespace vx {

constexpr int kDh = 128;

struct AttnWs {  // device workspace, see attn_ws_bytes
    int8_t *qu, *qv, *kq, *rq, *vq;
    float *qus, *qvs, *ks, *rs, *vs;
};

// round up helpers
__host__ __device__ inline int up16(int x) { return (x + 15) / 16 * 16; }
__host__ __device__ inline int up64(int x) { return (x + 63) / 64 * 64; }

struct AttnDims {
    int t, d, h, np, tp, rp, tv;
    int nseg = 1;  // segments of t frames each: qkv and ctx are [nseg][t][...], the relative rows are shared
    int rel_ld = 0;  // row pitch (floats) of rel_k: d, or wider when rel_k is one layer's block of a stacked output
    __host__ __device__ AttnDims(int t_, int d_, int h_) : t(t_), d(d_), h(h_) {
        np = 2 * t - 1;
        tp = up16(t);       // token rows (queries, keys)
        rp = up16(np) + 16; // relative rows, one spare block for the band alignment
        tv = up64(t);       // K extent of the context product
    }
};

__device__ inline int8_t q_code(float x, float inv) {
    float v = __builtin_rintf(x * inv);
    if (!(v == v)) return 0;
    v = v < -127.0f ? -127.0f : v;
    v = v > 127.0f ? 127.0f : v;
    return (int8_t)(int)v;
}

// max over the wavefront of non-negative values (every lane active)
__device__ inline float wave_max(float m) { return lane_group_max<64>(m); }

// Quantize the 128 values a (two per lane: columns 2*lane, 2*lane+1) into dst[128]; returns the scale.
__device__ inline float quant128(float a0, float a1, int lane, int8_t *dst) {
    const float m = wave_max(fmaxf(fabsf(a0), fabsf(a1)));
    const float s = m == 0.0f ? 1.0f : m / 127.0f;
    const float inv = 1.0f / s;
    const int8_t c0 = q_code(a0, inv), c1 = q_code(a1, inv);
    *(int16_t *)(dst + 2 * lane) = (int16_t)((uint16_t)(uint8_t)c0 | ((uint16_t)(uint8_t)c1 << 8));
    return s;
}

// Relative row r of h * rp (head-major): row p of rel_k's block of head h quantized into rq [h][rp][dh], rs [h][rp];
// rows past 2t-1 (the band's spare block) are zeros.
__device__ inline void attn_rel_item(int r, const float *__restrict__ rel_k, const AttnDims &D, int8_t *rq,
                                     float *rs) {
    const int lane = threadIdx.x & 63;
    if (r >= D.h * D.rp) return;
    const int h = r / D.rp, p = r % D.rp;
    float a0 = 0.0f, a1 = 0.0f;
    if (p < D.np) {
        const float2 v = *(const float2 *)(rel_k + (int64_t)p * D.rel_ld + h * kDh + 2 * lane);
        a0 = v.x;
        a1 = v.y;
    }
    const float s = quant128(a0, a1, lane, rq + ((int64_t)h * D.rp + p) * kDh);
    if (lane == 0) rs[h * D.rp + p] = s;
}

// Work items: [0, nseg*h*tp) query/key rows (segment-major, then head-major), then h*rp relative rows (shared).
__device__ inline void attn_rows_item(int item, const float *__restrict__ qkv, const float *__restrict__ rel_k,
                                      const float *__restrict__ bias_u, const float *__restrict__ bias_v,
                                      const AttnDims &D, const AttnWs &W) {
    const int lane = threadIdx.x & 63;
    const int d3 = 3 * D.d;
    if (item < D.nseg * D.h * D.tp) {
        const int seg = item / (D.h * D.tp), hi = item % (D.h * D.tp);
        const int h = hi / D.tp, i = hi % D.tp;
        qkv += (int64_t)seg * D.t * d3;
        const int64_t so = (int64_t)seg * D.h * D.tp;  // this segment's rows of the per-token tables
        const int64_t o = (so + (int64_t)h * D.tp + i) * kDh;
        float q0 = 0.0f, q1 = 0.0f, k0 = 0.0f, k1 = 0.0f;
        if (i < D.t) {
            const float2 qq = *(const float2 *)(qkv + (int64_t)i * d3 + h * kDh + 2 * lane);
            const float2 kk = *(const float2 *)(qkv + (int64_t)i * d3 + D.d + h * kDh + 2 * lane);
            q0 = qq.x;
            q1 = qq.y;
            k0 = kk.x;
            k1 = kk.y;
        }
        const float2 bu = *(const float2 *)(bias_u + h * kDh + 2 * lane);
        const float2 bv = *(const float2 *)(bias_v + h * kDh + 2 * lane);
        const bool live = i < D.t;
        const float su = quant128(live ? q0 + bu.x : 0.0f, live ? q1 + bu.y : 0.0f, lane, W.qu + o);
        const float sv = quant128(live ? q0 + bv.x : 0.0f, live ? q1 + bv.y : 0.0f, lane, W.qv + o);
        const float sk = quant128(k0, k1, lane, W.kq + o);
        if (lane == 0) {
            W.qus[so + h * D.tp + i] = su;
            W.qvs[so + h * D.tp + i] = sv;
            W.ks[so + h * D.tp + i] = sk;
        }
        return;
    }
    attn_rel_item(item - D.nseg * D.h * D.tp, rel_k, D, W.rq, W.rs);
}

// One wavefront per (segment, head, channel): vT row = v[i][h*dh + c] for i < t, zero to tv; one group.
__device__ inline void attn_vt_item(int item, const float *__restrict__ qkv, const AttnDims &D, const AttnWs &W) {
    const int lane = threadIdx.x & 63;
    if (item >= D.nseg * D.h * kDh) return;
    const int seg = item / (D.h * kDh), hc = item % (D.h * kDh);
    const int h = hc / kDh, c = hc % kDh;
    const float *col = qkv + (int64_t)seg * D.t * 3 * D.d + 2 * D.d + h * kDh + c;
    const int64_t ld = 3 * (int64_t)D.d;
    float m = 0.0f;
    for (int i = lane; i < D.t; i += 64) m = fmaxf(m, fabsf(col[i * ld]));
    m = wave_max(m);
    const float s = m == 0.0f ? 1.0f : m / 127.0f;
    const float inv = 1.0f / s;
    int8_t *dst = W.vq + ((int64_t)item) * D.tv;
    for (int i = lane; i < D.tv; i += 64) dst[i] = i < D.t ? q_code(col[i * ld], inv) : (int8_t)0;
    if (lane == 0) W.vs[item] = s;
}

// The vT rows of 16 channels of one (segment, head), a 256-thread workgroup (for batches of segments; one segment
// keeps the wavefront per channel above, whose 64x more workgroups hide the strided reads better: T = 338 / 750
// prep + core 19.9 / 48.0 us against 24.0 / 56.1 us, while 32 x 125 tokens gain 0.27 ms per encoder forward): thread (c, p) = (tid % 16, tid / 16)
// reads channel c of tokens p, p + 16, ... (16 lanes read 64 contiguous bytes of a token row), the channel's amax
// over the tokens meets in LDS, then thread (c, p) writes the codes of tokens 64 k + 4 p .. + 3 as one dword
// (zero past t). One group per vT row: amax, s = amax / 127 (1 when zero), inv = 1 / s, codes rint(x * inv).
__device__ inline void attn_vt16_block(int blk, const float *__restrict__ qkv, const AttnDims &D, const AttnWs &W,
                                       float (*smax)[16]) {
    const int head = blk % D.h, rest = blk / D.h, seg = rest / (kDh / 16), cb = rest % (kDh / 16);
    const int c = threadIdx.x & 15, p = threadIdx.x >> 4;
    const int64_t ld = 3 * (int64_t)D.d;
    const float *col = qkv + (int64_t)seg * D.t * ld + 2 * D.d + head * kDh + cb * 16 + c;
    float m = 0.0f;
    for (int i = p; i < D.t; i += 16) m = fmaxf(m, fabsf(col[i * ld]));
    smax[p][c] = m;
    __syncthreads();
    m = smax[0][c];
#pragma unroll
    for (int q = 1; q < 16; q++) m = fmaxf(m, smax[q][c]);
    const float s = m == 0.0f ? 1.0f : m / 127.0f;
    const float inv = 1.0f / s;
    const int item = (seg * D.h + head) * kDh + cb * 16 + c;
    uint32_t *dst = (uint32_t *)(W.vq + (int64_t)item * D.tv);
    for (int i0 = 4 * p; i0 < D.tv; i0 += 64) {
        uint32_t w4 = 0;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (i0 + j < D.t) w4 |= (uint32_t)(uint8_t)q_code(col[(i0 + j) * ld], inv) << (8 * j);
        dst[i0 / 4] = w4;
    }
    if (p == 0) W.vs[item] = s;
}

// The relative rows of nl layers in one launch (their projections depend on t and the weights only): layer blockIdx.y
// reads columns [l*d, (l+1)*d) of rel_k (row pitch D.rel_ld) and writes rq + l * h*rp*dh, rs + l * h*rp. A wavefront
// quantizes kRelPerWave consecutive rows r = h * rp + p, their loads issued together (one row per wavefront made
// 135K wavefronts for 24 layers at T = 338, whose launch and single load each dominated).
constexpr int kRelPerWave = 8;
__global__ __launch_bounds__(256) void attn_rel_kernel(const float *__restrict__ rel_k, AttnDims D, int8_t *rq,
                                                      float *rs) {
    const int l = blockIdx.y, lane = threadIdx.x & 63, nr = D.h * D.rp;
    const int r0 = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * kRelPerWave;
    if (r0 >= nr) return;  // uniform per wavefront
    rel_k += (int64_t)l * D.d;
    rq += (int64_t)l * nr * kDh;
    rs += (int64_t)l * nr;
    float2 v[kRelPerWave];
#pragma unroll
    for (int j = 0; j < kRelPerWave; j++) {
        const int r = r0 + j, h = r / D.rp, p = r % D.rp;
        v[j] = r < nr && p < D.np ? *(const float2 *)(rel_k + (int64_t)p * D.rel_ld + h * kDh + 2 * lane)
                                  : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < kRelPerWave; j++) {
        const int r = r0 + j;
        if (r >= nr) break;  // uniform per wavefront
        const float s = quant128(v[j].x, v[j].y, lane, rq + (int64_t)r * kDh);
        if (lane == 0) rs[r] = s;
    }
}

// The per-row quantizations and the vT rows in one launch: the first `rows_blocks` workgroups take the row items
// (four wavefronts, one item each), the others four vT rows (vt16 = 0) or 16 (vt16 = 1) each.
__global__ __launch_bounds__(256) void attn_prep_kernel(const float *__restrict__ qkv, const float *__restrict__ rel_k,
                                                       const float *__restrict__ bias_u,
                                                       const float *__restrict__ bias_v, AttnDims D, AttnWs W,
                                                       int rows_blocks, int vt16) {
    // Head-major workgroups go to the XCD of their head (workgroup b runs on XCD b % 8, the core's workgroups of head
    // h on XCD h % 8 with eight heads): the token rows of (segment, head) are tp/4 workgroups b with b % h == head,
    // the relative rows (when quantized here) follow in order, the vT blocks start at rows_blocks (a multiple of 64)
    // with the same head rule.
    const int wv = threadIdx.x >> 6, b = blockIdx.x;
    const int tok_blocks = D.nseg * D.h * (D.tp / 4);
    if (b < tok_blocks) {
        const int head = b % D.h, rest = b / D.h, seg = rest / (D.tp / 4), chunk = rest % (D.tp / 4);
        attn_rows_item(((seg * D.h + head) * D.tp) + chunk * 4 + wv, qkv, rel_k, bias_u, bias_v, D, W);
    } else if (b < rows_blocks) {
        attn_rows_item(b * 4 + wv, qkv, rel_k, bias_u, bias_v, D, W);  // relative rows (and padding)
    } else if (vt16) {
        __shared__ float smax[16][16];
        attn_vt16_block(b - rows_blocks, qkv, D, W, smax);
    } else {
        const int v = b - rows_blocks, head = v % D.h, rest = v / D.h, seg = rest / (kDh / 4), chunk = rest % (kDh / 4);
        attn_vt_item((seg * D.h + head) * kDh + chunk * 4 + wv, qkv, D, W);
    }
}

// LDS plan of attn_core_kernel (bytes): scores [16][s1w] f32 (content scores, then the band added in place, then the
// exponentials), pq [16][tv] int8, row stats (kRowv words: [0,16) max, [16,32) 1/sum, [32,48) probability scale,
// [64,192) and [192,320) the quantized output's per-wavefront row maxima and code sums).
constexpr int kCoreWaves = 8, kRowv = 320;
__host__ __device__ inline int s1w_of(int t) { return up16(t) + 4; }
__host__ __device__ inline size_t core_lds_bytes(int t) {
    return (size_t)16 * s1w_of(t) * 4 + (size_t)16 * up64(t) + kRowv * 4;
}

// ctx written as the o-projection's int8 activations (Attention::forward_fused, encoder.rs:180-183: attn_core_int8
// into ctx, then wo.prepare(ctx) = QuantAct::quantize_layout, packed.rs:307-436): a head's 128 channels are one
// 128-column group, so each query row's group is complete inside the workgroup.
struct AttnQOut {
    int8_t *q;     // [nseg * t][d]
    float *s;      // scales_t [h][np]
    int32_t *g;    // gsum_t [h][np]
    int np;        // npad(nseg * t)
};

// Eight wavefronts: the key and band blocks are dealt out over them, each query row's softmax runs on 32 lanes (four
// consecutive columns per lane), and each wavefront owns one 16-channel block of the context. Every global operand
// is requested before the phase that needs it starts: the band rows with the keys, the vT rows of the context
// product right after the content scores. The workgroup's vector-memory instructions are few because each costs the
// address unit 16 cycles whatever its width: KPF (the blocks a wave takes per batch) is the smallest depth that
// covers the keys and the band in one batch (up to 4; loops take the rest), the query scales are one 16-byte load,
// and one load per batch brings the scales of all its blocks, handed to the lanes that use them by ds_bpermute.
template <bool QOUT, int KPF>
__global__ __launch_bounds__(64 * kCoreWaves, 2) void attn_core_kernel(AttnDims D, AttnWs W, float scaling,
                                                                       float *__restrict__ ctx, AttnQOut Q) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int s1w = s1w_of(D.t);
    float *s1 = (float *)smem;
    int8_t *pq = (int8_t *)(s1 + 16 * s1w);
    float *rowv = (float *)(pq + 16 * D.tv);
    // wave is uniform across the wavefront; readfirstlane lets the compiler know it, so the loops over a wave's
    // blocks are scalar loops and the loads issued ahead of them are not drained at their heads
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // workgroup id = query block * h + head: with eight heads one head's workgroups run on one XCD (workgroup b runs
    // on XCD b % 8) and share its keys, band rows and vT in that XCD's L2
    const int h = blockIdx.x % D.h, qb = blockIdx.x / D.h, i0 = qb * 16;
    const int t = D.t;
    // segment blockIdx.z: its per-token tables and its rows of ctx (the relative rows are shared)
    {
        const int64_t seg = blockIdx.z, so = seg * D.h * D.tp;
        W.qu += so * kDh;
        W.qv += so * kDh;
        W.kq += so * kDh;
        W.qus += so;
        W.qvs += so;
        W.ks += so;
        W.vq += seg * D.h * kDh * D.tv;
        W.vs += seg * D.h * kDh;
        if (!QOUT) ctx += seg * D.t * D.d;
    }
    const int64_t row0 = (int64_t)blockIdx.z * D.t;  // this segment's first token row
    const int imax = min(i0 + 15, t - 1);
    const int nrows = imax - i0 + 1;             // valid query rows of the block
    const int pb0 = (t - 1 - imax) & ~15;        // first position block of the band
    const int pend = 2 * t - 2 - i0;             // last position used by the block
    const int npb = (pend - pb0) / 16 + 1;       // position blocks
    const int nkb = up16(t) / 16;                // key blocks

    // query fragments (A operand, 16x16x64 layout: lane l = row l%16, 16 bytes at 16*(l/16) of each 64-step)
    const int arow = lane & 15, aq = lane >> 4;
    const int8_t *qu = W.qu + ((int64_t)h * D.tp + i0 + arow) * kDh + 16 * aq;
    const int8_t *qv = W.qv + ((int64_t)h * D.tp + i0 + arow) * kDh + 16 * aq;
    const v4i au0 = *(const v4i *)qu, au1 = *(const v4i *)(qu + 64);
    const v4i av0 = *(const v4i *)qv, av1 = *(const v4i *)(qv + 64);
    // D element e of lane l: row 4*(l/16) + e, column l%16
    const int drow = 4 * aq, dcol = arow;
    const float vsv = W.vs[h * kDh + wave * 16 + dcol];  // the context block's vT scale, for the epilogue
    const float4 qu4 = *(const float4 *)&W.qus[h * D.tp + i0 + drow];
    const float4 qv4 = *(const float4 *)&W.qvs[h * D.tp + i0 + drow];
    const float qus[4] = {qu4.x, qu4.y, qu4.z, qu4.w}, qvs[4] = {qv4.x, qv4.y, qv4.z, qv4.w};
    constexpr int kPF = KPF, NW = kCoreWaves;
    // Key and band operands of kPF of this wave's blocks b0, b0+8, ... (past the last block: a repeat of it, not
    // used). The first batch of each is issued in straight-line code before any score is computed: a loop here would
    // make the compiler drain every load issued before it (a loop that uses registers loaded ahead of it gets a full
    // vmcnt wait at its head).
    v4i k0v[kPF], k1v[kPF], r0[kPF], r1[kPF];
    float ksv[kPF], rsv[kPF];
    // lane 16p + c of a scale load holds the scale of block p's key (position) c; block p's lanes take theirs
    auto spread = [&](float v, float (&out)[kPF]) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < kPF; p++) out[p] = __int_as_float(__shfl(__float_as_int(v), 16 * p + dcol, 64));
    };
    float ks_l = 0.0f, rs_l = 0.0f;  // this lane's scale of a batch (see spread)
    auto load_keys = [&](int kb0) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < kPF; p++) {
            const int kb = min(kb0 + NW * p, nkb - 1);
            const int8_t *kr = W.kq + ((int64_t)h * D.tp + kb * 16 + arow) * kDh + 16 * aq;
            k0v[p] = *(const v4i *)kr;
            k1v[p] = *(const v4i *)(kr + 64);
        }
        ks_l = W.ks[h * D.tp + min(kb0 + NW * min(lane >> 4, kPF - 1), nkb - 1) * 16 + dcol];
    };
    auto load_band = [&](int q0) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < kPF; p++) {
            const int p0 = pb0 + min(q0 + NW * p, npb - 1) * 16;
            const int8_t *rr = W.rq + ((int64_t)h * D.rp + p0 + arow) * kDh + 16 * aq;
            r0[p] = *(const v4i *)rr;
            r1[p] = *(const v4i *)(rr + 64);
        }
        rs_l = W.rs[h * D.rp + pb0 + min(q0 + NW * min(lane >> 4, kPF - 1), npb - 1) * 16 + dcol];
    };
    // content scores: key block kb -> s1[row][16*kb + col]
    auto score_keys = [&](int kb0) __attribute__((always_inline)) {
        spread(ks_l, ksv);
#pragma unroll
        for (int p = 0; p < kPF; p++) {
            const int kb = kb0 + NW * p;
            if (kb < nkb) {
                v4i acc = {0, 0, 0, 0};
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(au0, k0v[p], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(au1, k1v[p], acc, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++)
                    s1[(drow + e) * s1w + kb * 16 + dcol] = __builtin_fmaf((float)acc[e], qus[e] * ksv[p], 0.0f);
            }
        }
    };
    // position band: block pb, column col is position p = pb0 + 16*pb + col, i.e. key j = p - (t-1-i) of query
    // row i; score = S1 + S2 is formed in place (each (row, key) of the block is one (block, column) of the band)
    auto score_band = [&](int q0) __attribute__((always_inline)) {
        spread(rs_l, rsv);
#pragma unroll
        for (int p = 0; p < kPF; p++) {
            const int pb = q0 + NW * p;
            if (pb < npb) {
                v4i acc = {0, 0, 0, 0};
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av0, r0[p], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av1, r1[p], acc, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = drow + e;
                    const int j = pb0 + pb * 16 + dcol - (t - 1 - (i0 + r));
                    if (r < nrows && j >= 0 && j < t)
                        s1[r * s1w + j] = s1[r * s1w + j] + __builtin_fmaf((float)acc[e], qvs[e] * rsv[p], 0.0f);
                }
            }
        }
    };
    load_keys(wave);
    load_band(wave);
    score_keys(wave);
    for (int kb0 = wave + NW * kPF; kb0 < nkb; kb0 += NW * kPF) {  // t > 512
        load_keys(kb0);
        score_keys(kb0);
    }
    // the context product's vT operands (channel block `wave`, the first kVPre K steps of 64 tokens)
    constexpr int kVPre = 6;
    const int8_t *vr0 = W.vq + ((int64_t)h * kDh + wave * 16 + arow) * D.tv + 16 * aq;
    v4i vb[kVPre];
#pragma unroll
    for (int p = 0; p < kVPre; p++) vb[p] = *(const v4i *)(vr0 + min(64 * p, D.tv - 64));
    __syncthreads();  // s1 holds the content scores
    score_band(wave);
    for (int q0 = wave + NW * kPF; q0 < npb; q0 += NW * kPF) {  // t > 504
        load_band(q0);
        score_band(q0);
    }
    __syncthreads();
    // per row (32 lanes, wave w rows 2w, 2w+1; lane l32 columns 4*l32 + 128*k .. +3): the row max of
    // score * scaling, then exp_poly(score * scaling - max) in place
    {
        const int r = wave * 2 + (lane >> 5), l32 = lane & 31;
        float *sr = s1 + r * s1w;
        float m = -INFINITY;
        if (r < nrows)
            for (int j = 4 * l32; j < t; j += 128) {
                const float4 f = *(const float4 *)(sr + j);
                m = fmaxf(m, f.x * scaling);
                if (j + 1 < t) m = fmaxf(m, f.y * scaling);
                if (j + 2 < t) m = fmaxf(m, f.z * scaling);
                if (j + 3 < t) m = fmaxf(m, f.w * scaling);
            }
        m = lane_group_max<32>(m);
        if (r < nrows)
            for (int j = 4 * l32; j < t; j += 128) {
                float4 f = *(const float4 *)(sr + j);
                f.x = exp_poly(f.x * scaling - m);
                f.y = exp_poly(f.y * scaling - m);
                f.z = exp_poly(f.z * scaling - m);
                f.w = exp_poly(f.w * scaling - m);
                *(float4 *)(sr + j) = f;  // columns past t (inside the row's pitch) are never read as scores
            }
    }
    __syncthreads();
    // row sums in the reference's order: lane 4r + l keeps the running sum of columns j = 4q + l
    if (wave == 0) {
        const int r = lane >> 2, l = lane & 3;
        const int t4 = t / 4 * 4;
        float acc = 0.0f;
        if (r < nrows) {
#pragma unroll 8
            for (int j = l; j < t4; j += 4) acc += s1[r * s1w + j];
        }
        const int base = lane & ~3;
        const float l0 = __shfl(acc, base, 64), l1 = __shfl(acc, base + 1, 64), l2 = __shfl(acc, base + 2, 64),
                    l3 = __shfl(acc, base + 3, 64);
        float sum = (l0 + l1) + (l2 + l3);
        if (r < nrows)
            for (int j = t4; j < t; j++) sum += s1[r * s1w + j];
        if (l == 0) rowv[16 + r] = 1.0f / sum;
    }
    // probability quantization on waves 4-7 while wave 0 runs the row sums: amax per row (16 lanes per row), four
    // codes per lane and step into pq, zero to tv
    {
        const int r = (wave - 4) * 4 + (lane >> 4), l16 = lane & 15;
        float s = 1.0f;
        if (wave >= 4) {
            const float *sr = s1 + r * s1w;
            float m = 0.0f;
            if (r < nrows)
                for (int j = 4 * l16; j < t; j += 64) {
                    const float4 f = *(const float4 *)(sr + j);
                    m = fmaxf(m, fabsf(f.x));
                    if (j + 1 < t) m = fmaxf(m, fabsf(f.y));
                    if (j + 2 < t) m = fmaxf(m, fabsf(f.z));
                    if (j + 3 < t) m = fmaxf(m, fabsf(f.w));
                }
            m = lane_group_max<16>(m);
            s = m == 0.0f ? 1.0f : m / 127.0f;
            const float inv = 1.0f / s;
            for (int j = 4 * l16; j < D.tv; j += 64) {
                uint32_t w4 = 0;
                if (r < nrows && j < t) {
                    const float4 f = *(const float4 *)(sr + j);
                    const uint32_t c0 = (uint8_t)q_code(f.x, inv);
                    const uint32_t c1 = j + 1 < t ? (uint8_t)q_code(f.y, inv) : 0u;
                    const uint32_t c2 = j + 2 < t ? (uint8_t)q_code(f.z, inv) : 0u;
                    const uint32_t c3 = j + 3 < t ? (uint8_t)q_code(f.w, inv) : 0u;
                    w4 = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
                }
                *(uint32_t *)(pq + r * D.tv + j) = w4;
            }
        }
        __syncthreads();  // the 1/sum of wave 0 is visible after this barrier
        if (wave >= 4 && l16 == 0) rowv[32 + r] = s * rowv[16 + r];
    }
    __syncthreads();
    // context: channel block `wave`; K over tv in 64-steps; A = pq rows from LDS, B = vT rows (the first kVPre
    // steps loaded above, the loads of kPF later steps issued before their MFMAs)
    float val[4];
    v4i pacc = {0, 0, 0, 0};
    {
        const int8_t *pr = pq + arow * D.tv + 16 * aq;
#pragma unroll
        for (int p = 0; p < kVPre; p++)
            if (64 * p < D.tv) pacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i *)(pr + 64 * p), vb[p], pacc, 0, 0, 0);
        for (int k0 = 64 * kVPre; k0 < D.tv; k0 += 64 * kPF) {
            v4i b[kPF];
#pragma unroll
            for (int p = 0; p < kPF; p++) b[p] = *(const v4i *)(vr0 + min(k0 + 64 * p, D.tv - 64));
#pragma unroll
            for (int p = 0; p < kPF; p++) {
                if (k0 + 64 * p < D.tv) {
                    const v4i a = *(const v4i *)(pr + k0 + 64 * p);
                    pacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[p], pacc, 0, 0, 0);
                }
            }
        }
    }
    {
        const int c = wave * 16 + dcol;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int r = drow + e;
            val[e] = __builtin_fmaf((float)pacc[e], rowv[32 + r] * vsv, 0.0f);
            if (!QOUT && r < nrows) ctx[(int64_t)(i0 + r) * D.d + h * kDh + c] = val[e];
        }
    }
    if constexpr (QOUT) {
        // quantize_group of each query row over the head's 128 channels: one per lane, 16 lanes per wave, 8 waves
        float *qmax = rowv + 64;         // [wave][row]
        int *qsum = (int *)(rowv + 192);
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float m = lane_group_max<16>(fabsf(val[e]));
            if (dcol == 0) qmax[wave * 16 + drow + e] = m;
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int r = drow + e;
            float m = qmax[r];
#pragma unroll
            for (int w = 1; w < NW; w++) m = fmaxf(m, qmax[w * 16 + r]);
            sc[e] = m == 0.0f ? 1.0f : m / 127.0f;
            const float inv = 1.0f / sc[e];
            const int8_t c0 = q_code(val[e], inv);
            if (r < nrows) Q.q[(row0 + i0 + r) * D.d + h * kDh + wave * 16 + dcol] = c0;
            const int sum = lane_group_sum<16>((int)c0);
            if (dcol == 0) qsum[wave * 16 + r] = sum;
        }
        __syncthreads();
        if (wave == 0 && dcol == 0) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = drow + e;
                if (r < nrows) {
                    const int64_t gi = (int64_t)h * Q.np + row0 + i0 + r;
                    int g = 0;
#pragma unroll
                    for (int w = 0; w < NW; w++) g += qsum[w * 16 + r];
                    Q.s[gi] = sc[e];
                    Q.g[gi] = g;
                }
            }
        }
        // pad tokens [nseg * t, np) of this head's group: zero scale and code sum
        if (qb == D.tp / 16 - 1 && blockIdx.z == gridDim.z - 1) {
            const int64_t n = (int64_t)gridDim.z * D.t;
            if (tid < Q.np - n) {
                Q.s[(int64_t)h * Q.np + n + tid] = 0.0f;
                Q.g[(int64_t)h * Q.np + n + tid] = 0;
            }
        }
    }
}

size_t attn_ws_bytes_seg(int64_t t, int64_t d, int64_t h, int64_t nseg) {
    const AttnDims D((int)t, (int)d, (int)h);
    const size_t rows = (size_t)(nseg * h) * D.tp, rrows = (size_t)h * D.rp;
    size_t b = 0;
    auto add = [&](size_t n) { b += (n + 255) / 256 * 256; };
    add(rows * kDh);       // qu
    add(rows * kDh);       // qv
    add(rows * kDh);       // kq
    add(rrows * kDh);      // rq
    add((size_t)(nseg * h) * kDh * D.tv);  // vq
    add(rows * 4);         // qus
    add(rows * 4);         // qvs
    add(rows * 4);         // ks
    add(rrows * 4);        // rs
    add((size_t)(nseg * h) * kDh * 4);     // vs
    return b;
}

size_t attn_ws_bytes(int64_t t, int64_t d, int64_t h) { return attn_ws_bytes_seg(t, d, h, 1); }

// The dynamic-LDS limit of the core kernels (above the 64 KiB default), raised once per device; thread-safe, devices
// past 63 every call. Callers that capture launches into a graph call it before the capture.
void attention_prime() {
    static std::atomic<bool> lds_raised[64];
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    const bool cached = dev >= 0 && dev < 64;
    if (cached && lds_raised[dev].load(std::memory_order_acquire)) return;
    const void *kernels[] = {(const void *)attn_core_kernel<false, 1>, (const void *)attn_core_kernel<false, 2>,
                             (const void *)attn_core_kernel<false, 3>, (const void *)attn_core_kernel<false, 4>,
                             (const void *)attn_core_kernel<true, 1>,  (const void *)attn_core_kernel<true, 2>,
                             (const void *)attn_core_kernel<true, 3>,  (const void *)attn_core_kernel<true, 4>};
    for (const void *k : kernels)
        hip_check(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024), "attention LDS limit");
    if (cached) lds_raised[dev].store(true, std::memory_order_release);
}

// ctx [nseg][t][d] from qkv [nseg][t][3d] (q | k | v) and the shared rel_k [2t-1][d] of t frames: each segment's
// attention on its own tokens; ws is attn_ws_bytes_seg(t, d, h, nseg) device bytes.
// With q (and scales_t, gsum_t) not NULL, ctx is not written: the o-projection's activations are, in 128-column
// groups (one per head): q int8 [nseg * t][d], scales_t and gsum_t [h][npad(nseg * t)].
void attention_core_seg(const float *qkv, const float *rel_k, int64_t nseg, int64_t t, int64_t d, int64_t h,
                        const float *bias_u, const float *bias_v, float scaling, void *ws, float *ctx,
                        hipStream_t st, int8_t *q, float *scales_t, int32_t *gsum_t, int64_t rel_ld,
                        const int8_t *rq_pre, const float *rs_pre) {
    const bool qout = q != nullptr, pre = rq_pre != nullptr;
    require(qkv && (rel_k || pre) && bias_u && bias_v && ws && (ctx || qout) && (!qout || (scales_t && gsum_t)) &&
                (!pre || rs_pre),
            "attention: NULL pointer");
    require(h > 0 && d == h * kDh, "attention: the head dimension must be 128");
    require(t >= 1 && t <= 1024, "attention: 1 <= t <= 1024 frames");
    require(nseg >= 1 && nseg <= 65535 && nseg * t * 3 * d < (1ll << 31), "attention: 1 <= segments, size < 2^31");
    AttnDims D((int)t, (int)d, (int)h);
    D.nseg = (int)nseg;
    require(rel_ld >= d && (2 * t - 1) * rel_ld < (1ll << 31), "attention: bad rel_k row pitch");
    D.rel_ld = (int)rel_ld;
    uint8_t *p = (uint8_t *)ws;
    auto take = [&](size_t n) {
        uint8_t *r = p;
        p += (n + 255) / 256 * 256;
        return r;
    };
    const size_t rows = (size_t)(nseg * h) * D.tp, rrows = (size_t)h * D.rp;
    AttnWs W;
    W.qu = (int8_t *)take(rows * kDh);
    W.qv = (int8_t *)take(rows * kDh);
    W.kq = (int8_t *)take(rows * kDh);
    W.rq = (int8_t *)take(rrows * kDh);
    W.vq = (int8_t *)take((size_t)(nseg * h) * kDh * D.tv);
    W.qus = (float *)take(rows * 4);
    W.qvs = (float *)take(rows * 4);
    W.ks = (float *)take(rows * 4);
    W.rs = (float *)take(rrows * 4);
    W.vs = (float *)take((size_t)(nseg * h) * kDh * 4);
    if (pre) {  // the relative rows were quantized by attention_rel_quantize
        W.rq = const_cast<int8_t *>(rq_pre);
        W.rs = const_cast<float *>(rs_pre);
    }
    const int items = (int)(rows + (pre ? 0 : rrows));
    const int rows_blocks = ((items + 3) / 4 + 63) / 64 * 64;
    const int vt16 = nseg * h * (kDh / 16) >= 512 ? 1 : 0;
    const int vt_blocks = (int)(vt16 ? nseg * h * (kDh / 16) : (nseg * h * kDh + 3) / 4);
    attn_prep_kernel<<<(unsigned)(rows_blocks + vt_blocks), 256, 0, st>>>(qkv, rel_k, bias_u, bias_v, D, W,
                                                                         rows_blocks, vt16);
    hip_check(hipGetLastError(), "attention rows / vT kernel launch");
    const size_t lds = core_lds_bytes((int)t);
    attention_prime();
    AttnQOut Q{q, scales_t, gsum_t, (int)((nseg * t + 15) / 16 * 16)};
    const dim3 grid((unsigned)(D.tp / 16 * h), 1, (unsigned)nseg);
    // blocks per wave and batch: the smallest depth whose one batch covers the keys (nkb blocks) and the widest band
    // (at most (t + 29) / 16 + 1 position blocks), at most 4
    const int nblk = std::max((int)(D.tp / 16), (int)((t + 29) / 16 + 1));
    const int kpf = std::min(4, (nblk + kCoreWaves - 1) / kCoreWaves);
    auto launch = [&](auto kernel) { kernel<<<grid, 64 * kCoreWaves, lds, st>>>(D, W, scaling, ctx, Q); };
    switch (kpf + (qout ? 4 : 0)) {
        case 1: launch(attn_core_kernel<false, 1>); break;
        case 2: launch(attn_core_kernel<false, 2>); break;
        case 3: launch(attn_core_kernel<false, 3>); break;
        case 4: launch(attn_core_kernel<false, 4>); break;
        case 5: launch(attn_core_kernel<true, 1>); break;
        case 6: launch(attn_core_kernel<true, 2>); break;
        case 7: launch(attn_core_kernel<true, 3>); break;
        default: launch(attn_core_kernel<true, 4>); break;
    }
    hip_check(hipGetLastError(), "attention core kernel launch");
}

// The relative rows of nl layers quantized once, for attention_core_seg's rq_pre / rs_pre: layer l's rows are
// columns [l*d, (l+1)*d) of rel_k [2t-1][rel_ld]; per layer rq holds attn_rel_rows(t, h) rows of dh int8 ([h][rp][dh])
// and rs attn_rel_rows(t, h) floats ([h][rp]).
int64_t attn_rel_rows(int64_t t, int64_t h) { return h * AttnDims((int)t, (int)(h * kDh), (int)h).rp; }

void attention_rel_quantize(const float *rel_k, int64_t nl, int64_t t, int64_t d, int64_t h, int64_t rel_ld,
                            int8_t *rq, float *rs, hipStream_t st) {
    require(rel_k && rq && rs, "attention relative rows: NULL pointer");
    require(h > 0 && d == h * kDh && t >= 1 && t <= 1024 && nl >= 1 && nl <= 65535, "attention relative rows: shape");
    require(rel_ld >= nl * d && (2 * t - 1) * rel_ld < (1ll << 31), "attention relative rows: bad rel_k row pitch");
    AttnDims D((int)t, (int)d, (int)h);
    D.rel_ld = (int)rel_ld;
    const dim3 grid((unsigned)((h * D.rp + 4 * kRelPerWave - 1) / (4 * kRelPerWave)), (unsigned)nl);
    attn_rel_kernel<<<grid, 256, 0, st>>>(rel_k, D, rq, rs);
    hip_check(hipGetLastError(), "attention relative rows kernel launch");
}

// ---------------------------------------------------------------- the attention core without a caller workspace
//
// For callers that cannot allocate device memory (code under graph capture, serving loops that forbid it): the
// workspace is this file-scope array, one copy per GPU, held until the process ends. Its size bounds the calls:
// attn_ws_bytes(t, d, h) <= kStaticAttnWsBytes (t <= 1024 frames with d = 1024, 8 heads, needs 6.4 MiB). All calls
// on one GPU share its array, which keeps the previous call's contents: the preparation kernel writes every byte
// the core kernel then reads, so nothing needs clearing, and calls that overlap on one GPU race.
constexpr size_t kStaticAttnWsBytes = 8u << 20;
static __device__ __align__(256) uint8_t scratch[kStaticAttnWsBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void *> scratch_addr[kMaxDevices];
}  // namespace

// The device address of `scratch` on the current device (the host-side name is only a stand-in): looked up once per
// device with hipGetSymbolAddress and kept.
void *static_attn_ws() {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < kMaxDevices, "attention without a workspace: device index above 63");
    void *p = scratch_addr[dev].load(std::memory_order_acquire);
    if (!p) {
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(attention scratch)");
        require(p != nullptr, "hipGetSymbolAddress(attention scratch) returned NULL");
        scratch_addr[dev].store(p, std::memory_order_release);
    }
    return p;
}

void attention_core_noalloc(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h,
                            const float *bias_u, const float *bias_v, float scaling, float *ctx, hipStream_t st) {
    require(h > 0 && d == h * kDh, "attention: the head dimension must be 128");
    require(t >= 1 && t <= 1024, "attention: 1 <= t <= 1024 frames");
    const size_t need = attn_ws_bytes(t, d, h);
    require(need <= kStaticAttnWsBytes, "attention without a workspace: t = " + std::to_string(t) + ", " +
                                            std::to_string(h) + " heads need " + std::to_string(need) +
                                            " bytes of workspace, above the fixed " +
                                            std::to_string(kStaticAttnWsBytes) + " (use vx_attention_core)");
    attention_core_seg(qkv, rel_k, 1, t, d, h, bias_u, bias_v, scaling, static_attn_ws(), ctx, st, nullptr, nullptr,
                       nullptr, d, nullptr, nullptr);
}

// ctx [t][d] from qkv [t][3d] (q | k | v) and rel_k [2t-1][d]; ws is attn_ws_bytes(t, d, h) device bytes.
void attention_core(const float *qkv, const float *rel_k, int64_t t, int64_t d, int64_t h, const float *bias_u,
                    const float *bias_v, float scaling, void *ws, float *ctx, hipStream_t st) {
    attention_core_seg(qkv, rel_k, 1, t, d, h, bias_u, bias_v, scaling, ws, ctx, st, nullptr, nullptr, nullptr, d,
                       nullptr, nullptr);
}

}  // namespace vx
