// vx_glue.hip — the encoder's f32 glue around the int8 GEMMs, in the reference's operation order so that the
// results equal the CPU path bit for bit:
//
//   conv module (encoder.rs:576-628): GLU over channels (a * sigmoid_fast(b), tensor.rs:936-940), the depthwise
//     time convolution with BatchNorm folded into its taps (encoder.rs:548-573), SiLU — one fused kernel;
//   the f32 linear of the subsampling (tensor.rs:98-127: four fused lanes per output over 4-column steps, the
//     tail unfused, (hsum4 + tail) + bias; one token goes through gemv_portable, tensor.rs:284-303);
//   the subsampling convolutions (subsampling.rs:124-204): 3x3 stride-2 conv 1 -> C with ReLU and the depthwise
//     3x3 stride-2 convs, channels-last [T, F, C];
//   host helpers: the BatchNorm fold and the relative position table (encoder.rs:760-776, computed with the C
//     library's powf/sinf/cosf).
#include <cmath>
#include <vector>

#include "vx_gemm.h"

namespace vx {

// ---------------------------------------------------------------------------------------- conv module

// out[i][c] = silu(bias[c] + sum over taps kk of w[kk][c] * glu(g[i + kk - pad][c])), taps outside [0, t) skipped,
// each product and sum rounded separately (encoder.rs:604-624). g is the pointwise_conv1 output [t][2d]; the GLU
// value of a tap is recomputed per output (it is a pure function of g), so no [t][d] intermediate is stored.
// Row blockIdx.y of [nseg][t] rows: the taps stay inside its segment (rows outside are the zero padding).
__global__ __launch_bounds__(256) void glu_dwconv_silu_kernel(const float *__restrict__ g, int t, int d, int k,
                                                             const float *__restrict__ w_t,
                                                             const float *__restrict__ bias, float *__restrict__ out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int row = blockIdx.y, i = row % t, base = row - i;
    if (c >= d) return;
    const int pad = (k - 1) / 2;
    float acc = bias[c];
    for (int kk = 0; kk < k; kk++) {
        const int j = i + kk - pad;
        if (j < 0 || j >= t) continue;
        const float *gj = g + (int64_t)(base + j) * 2 * d;
        const float a = gj[c] * sigmoid_fast(gj[d + c]);
        acc = acc + w_t[(int64_t)kk * d + c] * a;
    }
    out[(int64_t)row * d + c] = silu_fast(acc);
}

// nseg segments of t frames each: g [nseg][t][2d] -> out [nseg][t][d].
void glu_dwconv_silu_seg(const float *g, int64_t nseg, int64_t t, int64_t d, int64_t k, const float *w_t,
                         const float *bias, float *out, hipStream_t st) {
    require(t == 0 || (g && w_t && bias && out), "glu_dwconv: NULL pointer");
    require(nseg >= 1 && t >= 0 && d > 0 && k > 0 && k % 2 == 1 && nseg * t * 2 * d < (1ll << 31) &&
                nseg * t <= 65535,
            "glu_dwconv: bad shape");
    if (t == 0) return;
    glu_dwconv_silu_kernel<<<dim3((unsigned)((d + 255) / 256), (unsigned)(nseg * t)), 256, 0, st>>>(
        g, (int)t, (int)d, (int)k, w_t, bias, out);
    hip_check(hipGetLastError(), "glu_dwconv kernel launch");
}

// As glu_dwconv_silu_kernel, with the result quantized for pointwise_conv2 (ConvModule::forward_fused,
// encoder.rs:605-625: the conv rows, then pw2.prepare(hb) = QuantAct::quantize_layout, packed.rs:307-436) in
// 128-channel groups, so hb never reaches memory. A block is 256 channels of one row: two groups of two wavefronts
// each; a group's amax and code sum meet in LDS (a max and an integer sum are exact in any order). Rows [n, np)
// are the pad tokens: their scales and code sums are written as zero.
__global__ __launch_bounds__(256) void glu_dwconv_silu_quant_kernel(const float *__restrict__ g, int t, int n, int np,
                                                                   int d, int k, const float *__restrict__ w_t,
                                                                   const float *__restrict__ bias,
                                                                   int8_t *__restrict__ q, float *__restrict__ st,
                                                                   int32_t *__restrict__ gt) {
    __shared__ float smax[4];
    __shared__ int ssum[4];
    const int c = blockIdx.x * 256 + threadIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.y;
    const int64_t gi = (int64_t)(c / 128) * np + row;
    if (row >= n) {  // uniform per block
        if ((threadIdx.x & 127) == 0) {
            st[gi] = 0.0f;
            gt[gi] = 0;
        }
        return;
    }
    const int i = row % t, base = row - i, pad = (k - 1) / 2;
    float acc = bias[c];
    for (int kk = 0; kk < k; kk++) {
        const int j = i + kk - pad;
        if (j < 0 || j >= t) continue;
        const float *gj = g + (int64_t)(base + j) * 2 * d;
        const float a = gj[c] * sigmoid_fast(gj[d + c]);
        acc = acc + w_t[(int64_t)kk * d + c] * a;
    }
    const float v = silu_fast(acc);
    float m = fabsf(v);
    m = lane_group_max<64>(m);
    if (lane == 0) smax[wv] = m;
    __syncthreads();
    m = fmaxf(smax[wv & ~1], smax[wv | 1]);
    const float s = m == 0.0f ? 1.0f : m / 127.0f;
    const float inv = 1.0f / s;
    const int8_t code = code_of(v, inv);
    q[(int64_t)row * d + c] = code;
    int sum = code;
    sum = lane_group_sum<64>(sum);
    if (lane == 0) ssum[wv] = sum;
    __syncthreads();
    if ((threadIdx.x & 127) == 0) {
        st[gi] = s;
        gt[gi] = ssum[wv] + ssum[wv + 1];
    }
}

// The same for kernel size 9, a workgroup per (128 channels, kGluRows rows): thread c computes the GLU of channel c
// once for the rows r0 - 4 .. r0 + kGluRows + 3 (the taps of its rows; a row of another segment or past the last is
// never used) and keeps them in registers, then for each of its rows the taps in order (acc = bias; acc = acc + w *
// a, unfused, taps outside the row's segment skipped), SiLU, and the row's 128-channel group quantized (amax and
// code sums by DPP within each wavefront, the two wavefronts combined through LDS). Taller tiles recompute fewer GLU
// rows (window kGluRows + 8) but launch fewer workgroups: 2 rows where that gives fewer than 2048 workgroups
// (T = 338 / 750: 6.4 / 9.9 -> 6.35 / 8.1 us against the per-row kernel), else the tallest of 4 and 8 that keeps
// 2048 (32 x 125 rows: 42.6 -> 21.5 us).
template <int kGluRows>
__global__ __launch_bounds__(128) void glu_dwconv9_silu_quant_kernel(const float *__restrict__ g, int t, int n, int np,
                                                                    int d, const float *__restrict__ w_t,
                                                                    const float *__restrict__ bias,
                                                                    int8_t *__restrict__ q, float *__restrict__ st,
                                                                    int32_t *__restrict__ gt) {
    constexpr int K = 9, PAD = 4, W = kGluRows + 2 * PAD;
    __shared__ float smax[2][kGluRows];
    __shared__ int ssum[2][kGluRows];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c = blockIdx.x * 128 + threadIdx.x, r0 = blockIdx.y * kGluRows;
    float a[W];
#pragma unroll
    for (int r = 0; r < W; r++) {
        const int R = r0 - PAD + r;  // uniform per workgroup
        a[r] = 0.0f;
        if (R >= 0 && R < n) {
            const float *gr = g + (int64_t)R * 2 * d;
            a[r] = gr[c] * sigmoid_fast(gr[d + c]);
        }
    }
    float wk[K];
#pragma unroll
    for (int kk = 0; kk < K; kk++) wk[kk] = w_t[(int64_t)kk * d + c];
    const float b = bias[c];
    float v[kGluRows];
#pragma unroll
    for (int i = 0; i < kGluRows; i++) {
        const int R = r0 + i, ti = R % t;
        float acc = b;
#pragma unroll
        for (int kk = 0; kk < K; kk++) {
            const int j = ti + kk - PAD;
            if (j >= 0 && j < t) acc = acc + wk[kk] * a[i + kk];
        }
        v[i] = silu_fast(acc);
    }
    float m[kGluRows];
#pragma unroll
    for (int i = 0; i < kGluRows; i++) m[i] = lane_group_max<64>(fabsf(v[i]));
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < kGluRows; i++) smax[wv][i] = m[i];
    __syncthreads();
    float s[kGluRows];
#pragma unroll
    for (int i = 0; i < kGluRows; i++) {
        const float mm = fmaxf(smax[0][i], smax[1][i]);
        s[i] = mm == 0.0f ? 1.0f : mm / 127.0f;
        const float inv = 1.0f / s[i];
        const int8_t code = code_of(v[i], inv);
        if (r0 + i < n) q[(int64_t)(r0 + i) * d + c] = code;
        const int sum = lane_group_sum<64>((int)code);
        if (lane == 0) ssum[wv][i] = sum;
    }
    __syncthreads();
    if (threadIdx.x < kGluRows) {
        const int i = threadIdx.x, R = r0 + i;
        const int64_t gi = (int64_t)blockIdx.x * np + R;
        if (R < n) {
            const float mm = fmaxf(smax[0][i], smax[1][i]);
            st[gi] = mm == 0.0f ? 1.0f : mm / 127.0f;
            gt[gi] = ssum[0][i] + ssum[1][i];
        } else if (R < np) {  // pad tokens: zero scale and code sum
            st[gi] = 0.0f;
            gt[gi] = 0;
        }
    }
}

// nseg segments of t frames: g [nseg][t][2d] -> the QuantAct of the conv rows in 128-channel groups: q int8
// [nseg * t][d], scales_t and gsum_t [d / 128][npad(nseg * t)].
void glu_dwconv_silu_quant_seg(const float *g, int64_t nseg, int64_t t, int64_t d, int64_t k, const float *w_t,
                               const float *bias, int8_t *q, float *scales_t, int32_t *gsum_t, hipStream_t st) {
    require(t == 0 || (g && w_t && bias && q && scales_t && gsum_t), "glu_dwconv_quantize: NULL pointer");
    require(nseg >= 1 && t >= 0 && d > 0 && d % 256 == 0 && k > 0 && k % 2 == 1 && nseg * t * 2 * d < (1ll << 31) &&
                nseg * t <= 65535,
            "glu_dwconv_quantize: bad shape (d a multiple of 256)");
    if (t == 0) return;
    const int64_t n = nseg * t, np = (n + 15) / 16 * 16;
    if (k == 9) {
        const int64_t cg = d / 128;
        const int rows = cg * (np / 8) >= 2048 ? 8 : cg * (np / 4) >= 2048 ? 4 : 2;
        auto launch = [&](auto kernel) {
            kernel<<<dim3((unsigned)cg, (unsigned)(np / rows)), 128, 0, st>>>(g, (int)t, (int)n, (int)np, (int)d, w_t,
                                                                          bias, q, scales_t, gsum_t);
        };
        if (rows == 8)
            launch(glu_dwconv9_silu_quant_kernel<8>);
        else if (rows == 4)
            launch(glu_dwconv9_silu_quant_kernel<4>);
        else
            launch(glu_dwconv9_silu_quant_kernel<2>);
    } else
        glu_dwconv_silu_quant_kernel<<<dim3((unsigned)(d / 256), (unsigned)np), 256, 0, st>>>(
            g, (int)t, (int)n, (int)np, (int)d, (int)k, w_t, bias, q, scales_t, gsum_t);
    hip_check(hipGetLastError(), "glu_dwconv_quantize kernel launch");
}

void glu_dwconv_silu(const float *g, int64_t t, int64_t d, int64_t k, const float *w_t, const float *bias, float *out,
                     hipStream_t st) {
    require(t <= 65535, "glu_dwconv: t <= 65535");
    if (t == 0) return;
    glu_dwconv_silu_seg(g, 1, t, d, k, w_t, bias, out, st);
}

// ---------------------------------------------------------------------------------------- f32 linear

// y[n][out] = x[n][in] . w[out][in]^T + b, each output with the reference tile's lane order: acc[l] =
// fma(w[c + l], x[c + l], acc[l]) over 4-column steps, tail = sum of unfused w*x in order, y = (hsum4 + tail) + b,
// optional ReLU. The four running sums of one output are sequential by definition, so the parallelism is across
// outputs. A 256-thread block owns 64 outputs x 16 tokens: lane l of every wavefront owns output o0 + l, wavefront
// w tokens 4w .. 4w+3 (16 running sums per thread). Per 4-column step a lane reads its own weight quad from LDS
// and the 4 token quads as LDS broadcasts, so LDS traffic stays below the FMA issue rate.
constexpr int LO = 64, LTT = 16, LK = 64, LKP = LK + 4;

template <bool RELU>
__global__ __launch_bounds__(256) void linear_f32_kernel(const float *__restrict__ x, int n, int in_f,
                                                        const float *__restrict__ w, const float *__restrict__ b,
                                                        int out_f, float *__restrict__ y) {
    __shared__ __attribute__((aligned(16))) float xs[LTT][LKP];
    __shared__ __attribute__((aligned(16))) float ws[LO][LKP];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.y * LTT, o0 = blockIdx.x * LO;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int l = 0; l < 4; l++) acc[i][l] = 0.0f;
    const int c4 = in_f / 4 * 4;
    const bool vec = (in_f % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    auto ld4 = [&](const float *base, int row, int nrows, int col) {
        if (row >= nrows || col >= c4) return make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float *q = base + (int64_t)row * in_f + col;
        return vec ? *(const float4 *)q : make_float4(q[0], q[1], q[2], q[3]);
    };
    // software pipeline: the next slab's quads are loaded into registers while the current slab is consumed
    const int q = tid & 15, r = tid >> 4;
    float4 pw[4], px;
    auto fetch = [&](int k0) {
#pragma unroll
        for (int h = 0; h < 4; h++) pw[h] = ld4(w, o0 + r + 16 * h, out_f, k0 + q * 4);
        px = ld4(x, t0 + r, n, k0 + q * 4);
    };
    if (c4 > 0) fetch(0);
    for (int k0 = 0; k0 < c4; k0 += LK) {
#pragma unroll
        for (int h = 0; h < 4; h++) *(float4 *)&ws[r + 16 * h][q * 4] = pw[h];
        *(float4 *)&xs[r][q * 4] = px;
        __syncthreads();
        if (k0 + LK < c4) fetch(k0 + LK);
        // one 4-column step: this lane's weight quad, the four token quads (LDS broadcasts), 16 chained FMAs
        auto step4 = [&](int kk) __attribute__((always_inline)) {
            const float4 wa = *(const float4 *)&ws[lane][kk];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 xa = *(const float4 *)&xs[4 * wv + i][kk];
                acc[i][0] = __builtin_fmaf(wa.x, xa.x, acc[i][0]);
                acc[i][1] = __builtin_fmaf(wa.y, xa.y, acc[i][1]);
                acc[i][2] = __builtin_fmaf(wa.z, xa.z, acc[i][2]);
                acc[i][3] = __builtin_fmaf(wa.w, xa.w, acc[i][3]);
            }
        };
        if (c4 - k0 >= LK) {
            // a whole slab: unrolled, so the LDS reads of later steps issue while earlier steps' FMAs run
#pragma unroll
            for (int kk = 0; kk < LK; kk += 4) step4(kk);
        } else {
            for (int kk = 0; kk < c4 - k0; kk += 4) step4(kk);
        }
        __syncthreads();
    }
    const int o = o0 + lane;
    if (o >= out_f) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = t0 + 4 * wv + i;
        if (t >= n) continue;
        float tail = 0.0f;
        for (int col = c4; col < in_f; col++) tail += w[(int64_t)o * in_f + col] * x[(int64_t)t * in_f + col];
        float v = ((acc[i][0] + acc[i][1]) + (acc[i][2] + acc[i][3])) + tail;
        v = v + (b ? b[o] : 0.0f);
        if (RELU) v = v > 0.0f ? v : 0.0f;
        y[(int64_t)t * out_f + o] = v;
    }
}

// The same sums on the fp32 matrix cores. v_mfma_f32_16x16x1f32 computes four independent 16 x 16 blocks of
// D = A (x) B + C with K = 1, each element one fused multiply-add with a single rounding; it equals fmaf bit for bit
// (checked on the device against fmaf over random and special operands: denormals, infinities, NaN, exact
// cancellation, signed zeros). Block c of one instruction is running sum c of the reference's lanes, so one
// instruction is one 4-column step for 16 tokens x 16 outputs:
//   lane l supplies A = x[token l % 16][4s + l / 16] and B = w[output l % 16][4s + l / 16];
//   D register r of lane l is running sum r / 4 of token 4 * (l / 16) + r % 4 and output l % 16.
// The slabs of x and w are staged in LDS de-interleaved by running sum, [c][row][step] with a row pitch of KS/4 + 4
// floats (16 consecutive rows of one c start in distinct bank quads), so one 16-byte read gives a lane four steps.
// Two LDS buffers and two register sets: slab s + 2 is fetched into registers while slab s is multiplied, slab s + 1
// is written to the other buffer after it, one barrier per slab, so a fetch has two slabs of MFMAs to arrive.
// Only the steps below in_f / 4 are issued (padding is never accumulated: fma(0, 0, -0) would be +0); the
// unfused tail and (hsum4 + tail) + bias follow in the epilogue. A workgroup of four wavefronts (2 x 2) owns
// (32 WT) tokens x (32 WO) outputs, a wavefront WT x WO blocks of 16 x 16.
template <bool RELU, int WT, int WO, int KS>
__global__ __launch_bounds__(256) void linear_f32_mfma_kernel(const float *__restrict__ x, int n, int in_f,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ b, int out_f,
                                                             float *__restrict__ y) {
    constexpr int BM = 32 * WT, BN = 32 * WO, SP = KS / 4 + 4;      // SP: row pitch (floats)
    constexpr int QX = BM * KS / 16 / 256, QW = BN * KS / 16 / 256;  // 16-column pieces per thread
    static_assert(QX >= 1 && QW >= 1, "a thread stages at least one piece of each operand");
    __shared__ __attribute__((aligned(16))) float sx[2][4][BM][SP], sw[2][4][BN][SP];
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.y * BM, o0 = blockIdx.x * BN;
    const int l16 = lane & 15, lc = lane >> 4;                           // row in a block, running sum
    const int wt0 = (wv & 1) * 16 * WT, wo0 = (wv >> 1) * 16 * WO;       // the wavefront's blocks in the tile
    const int c4 = in_f / 4 * 4, nsteps = c4 / 4, nslab = (c4 + KS - 1) / KS;

    v16f acc[WT][WO];
#pragma unroll
    for (int i = 0; i < WT; i++)
#pragma unroll
        for (int j = 0; j < WO; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    // staging: piece p of an operand is row p / (KS / 16), columns 16 (p % (KS / 16)) .. + 15 of the slab, loaded as
    // four quads and written as four quads of consecutive steps, one per running sum. Quads at or past c4 are
    // loaded from column c4 - 4 (in bounds, no branch around the load, so the loads of a fetch stay in flight
    // together) and written as zeros.
    float4 px[2][QX][4], pq[2][QW][4];
    auto fetch = [&](int set, int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < QX; q++) {
            const int p = tid + 256 * q, r = p / (KS / 16), c = k0 + 16 * (p % (KS / 16));
            const float *src = x + (int64_t)min(t0 + r, n - 1) * in_f;
#pragma unroll
            for (int j = 0; j < 4; j++) px[set][q][j] = *(const float4 *)(src + min(c + 4 * j, c4 - 4));
        }
#pragma unroll
        for (int q = 0; q < QW; q++) {
            const int p = tid + 256 * q, r = p / (KS / 16), c = k0 + 16 * (p % (KS / 16));
            const float *src = w + (int64_t)min(o0 + r, out_f - 1) * in_f;
#pragma unroll
            for (int j = 0; j < 4; j++) pq[set][q][j] = *(const float4 *)(src + min(c + 4 * j, c4 - 4));
        }
    };
    // stash unit u < 4 (QX + QW): running-sum plane u % 4 of piece (u / 4) of x, then of w; register set `set` ->
    // LDS buffer `set`
    constexpr int NU = 4 * (QX + QW);
    auto stash_unit = [&](int set, int k0, int u) __attribute__((always_inline)) {
        const bool isx = u < 4 * QX;
        const int q = (isx ? u : u - 4 * QX) / 4, c = u % 4;
        const int p = tid + 256 * q, r = p / (KS / 16), s = 4 * (p % (KS / 16)), col = k0 + 4 * s;
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 v = isx ? px[set][q][j] : pq[set][q][j];
            const float comp = c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
            e[j] = col + 4 * j < c4 ? comp : 0.0f;
        }
        *(float4 *)(isx ? &sx[set][c][r][s] : &sw[set][c][r][s]) = make_float4(e[0], e[1], e[2], e[3]);
    };
    auto stash = [&](int set, int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NU; u++) stash_unit(set, k0, u);
    };
    // the steps of slab sl from LDS buffer `buf`, and the stash of register set `sset` (slab at column sk0) into the
    // other buffer: in a whole slab its units follow the MFMAs of each quad, so that they issue while those run
    auto compute = [&](int buf, int sl, int sset, int sk0) __attribute__((always_inline)) {
        const int sn = min(KS / 4, nsteps - sl * (KS / 4));  // steps in this slab
        auto quad = [&](int s4) __attribute__((always_inline)) {  // steps s4 .. s4 + 3
            float4 xa[WT], wa[WO];
#pragma unroll
            for (int i = 0; i < WT; i++) xa[i] = *(const float4 *)&sx[buf][lc][wt0 + 16 * i + l16][s4];
#pragma unroll
            for (int j = 0; j < WO; j++) wa[j] = *(const float4 *)&sw[buf][lc][wo0 + 16 * j + l16][s4];
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < WT; i++)
#pragma unroll
                    for (int j = 0; j < WO; j++) {
                        const float av = e == 0 ? xa[i].x : e == 1 ? xa[i].y : e == 2 ? xa[i].z : xa[i].w;
                        const float bv = e == 0 ? wa[j].x : e == 1 ? wa[j].y : e == 2 ? wa[j].z : wa[j].w;
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x1f32(av, bv, acc[i][j], 0, 0, 0);
                    }
        };
        auto single = [&](int s) __attribute__((always_inline)) {  // one step (a slab's last partial quad)
#pragma unroll
            for (int i = 0; i < WT; i++)
#pragma unroll
                for (int j = 0; j < WO; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x1f32(sx[buf][lc][wt0 + 16 * i + l16][s],
                                                                    sw[buf][lc][wo0 + 16 * j + l16][s], acc[i][j],
                                                                    0, 0, 0);
        };
        int s = 0;
        if (sn == KS / 4) {
            // a whole slab: unrolled, the LDS reads of quad q + RA issued before the MFMAs of quad q (two quads
            // ahead for one block per wavefront, one for four blocks, whose quad has 16 MFMAs)
            constexpr int NQ = KS / 16, RA = WT * WO >= 4 ? 1 : 2;
            float4 xr[RA + 1][WT], wr[RA + 1][WO];
            auto rd = [&](int slot, int s4) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < WT; i++) xr[slot][i] = *(const float4 *)&sx[buf][lc][wt0 + 16 * i + l16][s4];
#pragma unroll
                for (int j = 0; j < WO; j++) wr[slot][j] = *(const float4 *)&sw[buf][lc][wo0 + 16 * j + l16][s4];
            };
#pragma unroll
            for (int q = 0; q < RA; q++) rd(q, 4 * q);
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                if (q + RA < NQ) rd((q + RA) % (RA + 1), 4 * (q + RA));
                __builtin_amdgcn_sched_barrier(0);  // the scheduler would sink the reads to their MFMAs
                const int sl3 = q % (RA + 1);
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int i = 0; i < WT; i++)
#pragma unroll
                        for (int j = 0; j < WO; j++) {
                            const float4 xa = xr[sl3][i], wa = wr[sl3][j];
                            const float av = e == 0 ? xa.x : e == 1 ? xa.y : e == 2 ? xa.z : xa.w;
                            const float bv = e == 0 ? wa.x : e == 1 ? wa.y : e == 2 ? wa.z : wa.w;
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x1f32(av, bv, acc[i][j], 0, 0, 0);
                        }
                constexpr int UPQ = (NU + NQ - 1) / NQ;
#pragma unroll
                for (int u = q * UPQ; u < (q + 1) * UPQ; u++)
                    if (u < NU) stash_unit(sset, sk0, u);
            }
        } else {
            for (; s + 4 <= sn; s += 4) quad(s);
            for (; s < sn; s++) single(s);
            stash(sset, sk0);
        }
    };
    // slab k lives in register set k % 2 and LDS buffer k % 2. The fetches and stashes past the last slab repeat
    // it (in bounds, never multiplied), so every slab issues the same loads and the counter waits stay exact.
    fetch(0, 0);
    fetch(1, min(1, nslab - 1) * KS);
    __builtin_amdgcn_sched_barrier(0);
    stash(0, 0);
    __syncthreads();
    auto slab = [&](auto Pc, int sl) __attribute__((always_inline)) {
        constexpr int P = decltype(Pc)::value;            // sl % 2
        fetch(P, min(sl + 2, nslab - 1) * KS);            // set P held slab sl, in LDS since the last barrier
        __builtin_amdgcn_sched_barrier(0);
        compute(P, sl, P ^ 1, min(sl + 1, nslab - 1) * KS);  // buffer P ^ 1 was last read before the last barrier
        __syncthreads();
    };
    int sl = 0;
    for (; sl + 1 < nslab; sl += 2) {
        slab(IC<0>{}, sl);
        slab(IC<1>{}, sl + 1);
    }
    if (sl < nslab) slab(IC<0>{}, sl);
    // epilogue: lane l holds, for output o0 + wo0 + 16 j + l % 16, tokens t0 + wt0 + 16 i + 4 (l / 16) + e
#pragma unroll
    for (int j = 0; j < WO; j++) {
        const int o = o0 + wo0 + 16 * j + l16;
        if (o >= out_f) continue;
        const float bo = b ? b[o] : 0.0f;
#pragma unroll
        for (int i = 0; i < WT; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = t0 + wt0 + 16 * i + 4 * lc + e;
                if (t >= n) continue;
                float tail = 0.0f;
                for (int col = c4; col < in_f; col++) tail += w[(int64_t)o * in_f + col] * x[(int64_t)t * in_f + col];
                float v = ((acc[i][j][e] + acc[i][j][4 + e]) + (acc[i][j][8 + e] + acc[i][j][12 + e])) + tail;
                v = v + bo;
                if (RELU) v = v > 0.0f ? v : 0.0f;
                y[(int64_t)t * out_f + o] = v;
            }
    }
}

// One token: gemv_portable (tensor.rs:284-303): rows below out_f/4*4 by dot_lanes8 (fused lanes over 8-column
// steps, lane-wise a + b, hsum4, tail unfused), the others by dot (8 unfused lane sums summed in order, tail).
template <bool RELU>
__global__ void gemv_f32_kernel(const float *__restrict__ x, int in_f, const float *__restrict__ w,
                                const float *__restrict__ b, int out_f, float *__restrict__ y) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= out_f) return;
    const float *wr = w + (int64_t)o * in_f;
    const int n8 = in_f / 8 * 8, o4 = out_f / 4 * 4;
    float r;
    if (o < o4) {
        float a[4] = {0, 0, 0, 0}, bb[4] = {0, 0, 0, 0};
        for (int c = 0; c < n8; c += 8)
            for (int l = 0; l < 4; l++) {
                a[l] = __builtin_fmaf(x[c + l], wr[c + l], a[l]);
                bb[l] = __builtin_fmaf(x[c + 4 + l], wr[c + 4 + l], bb[l]);
            }
        float p[4];
        for (int l = 0; l < 4; l++) p[l] = a[l] + bb[l];
        r = (p[0] + p[1]) + (p[2] + p[3]);
        for (int c = n8; c < in_f; c++) r += x[c] * wr[c];
    } else {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int c = 0; c < n8; c += 8)
            for (int l = 0; l < 8; l++) acc[l] += x[c + l] * wr[c + l];
        r = acc[0];
        for (int l = 1; l < 8; l++) r += acc[l];
        for (int c = n8; c < in_f; c++) r += x[c] * wr[c];
    }
    float v = r + (b ? b[o] : 0.0f);
    if (RELU) v = v > 0.0f ? v : 0.0f;
    y[o] = v;
}

void linear_f32(const float *x, int64_t n, int64_t in_f, const float *w, const float *b, int64_t out_f, float *y,
                bool relu, hipStream_t st) {
    require(n == 0 || (x && w && y), "linear_f32: NULL pointer");
    require(n >= 0 && in_f > 0 && out_f > 0 && n * in_f < (1ll << 31) && n * out_f < (1ll << 31) &&
                out_f * in_f < (1ll << 31),
            "linear_f32: bad shape");
    if (n == 0) return;
    if (n == 1) {
        auto k = relu ? gemv_f32_kernel<true> : gemv_f32_kernel<false>;
        k<<<(unsigned)((out_f + 255) / 256), 256, 0, st>>>(x, (int)in_f, w, b, (int)out_f, y);
    } else {
        // the matrix-core kernel where its 16-byte loads are aligned: 64 x 64 tiles when they give 256 workgroups
        // (the subsampling's pointwise convolutions), else 32 x 32 (its final linear); else the LDS-broadcast kernel
        const bool aligned = in_f % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                             reinterpret_cast<uintptr_t>(w) % 16 == 0;
        int kind = overrides().linear.load(std::memory_order_relaxed);
        auto wgs = [&](int bm, int bn) { return ((n + bm - 1) / bm) * ((out_f + bn - 1) / bn); };
        if (kind == 0) kind = wgs(64, 64) >= 256 ? 122 : 111;
        if (aligned && kind > 0) {
            const int wt = kind / 10 % 10, wo = kind % 10;
            const dim3 grid((unsigned)((out_f + 32 * wo - 1) / (32 * wo)), (unsigned)((n + 32 * wt - 1) / (32 * wt)));
#define VX_LINM(WT, WO, KS)                                                                                       \
    (relu ? linear_f32_mfma_kernel<true, WT, WO, KS> : linear_f32_mfma_kernel<false, WT, WO, KS>)<<<grid, 256, 0, \
                                                                                                   st>>>(         \
        x, (int)n, (int)in_f, w, b, (int)out_f, y)
            // slabs of 64 columns for 64 x 64 tiles (two workgroups of 80 KB LDS per CU), else 128
            if (wt == 2 && wo == 2)
                VX_LINM(2, 2, 64);
            else if (wt == 2)
                VX_LINM(2, 1, 128);
            else
                VX_LINM(1, 1, 128);
#undef VX_LINM
        } else {
            auto k = relu ? linear_f32_kernel<true> : linear_f32_kernel<false>;
            k<<<dim3((unsigned)((out_f + LO - 1) / LO), (unsigned)((n + LTT - 1) / LTT)), 256, 0, st>>>(
                x, (int)n, (int)in_f, w, b, (int)out_f, y);
        }
    }
    hip_check(hipGetLastError(), "linear_f32 kernel launch");
}

// ---------------------------------------------------------------------------------------- subsampling convs

__host__ __device__ inline int conv_out_len(int n, int k, int s, int p) { return (n + 2 * p - k) / s + 1; }

// stage 0 (subsampling.rs:130-160): out[ot][of][ch] = relu(b[ch] + sum over (kt, kf) in order of w[kt*k+kf][ch] *
// feats[ot*s + kt - p][of*s + kf - p]), out-of-range taps skipped. A block is one output time row: the k input rows
// it reads are staged in LDS (zero where out of range, never read there), each thread keeps one channel's taps.
constexpr int kMaxMels = 256, kMaxK = 3;
__global__ __launch_bounds__(256) void conv0_kernel(const float *__restrict__ feats, int t, int nm, int k, int s,
                                                   const float *__restrict__ w, const float *__restrict__ b, int c,
                                                   int t1, int f1, float *__restrict__ out) {
    __shared__ float rows[kMaxK][kMaxMels];
    const int ot = blockIdx.x % t1, seg = blockIdx.x / t1, p = (k - 1) / 2;
    feats += (int64_t)seg * t * nm;  // segment seg of [nseg][t][nm] -> [nseg][t1][f1][c]
    out += (int64_t)seg * t1 * f1 * c;
    for (int e = threadIdx.x; e < k * nm; e += blockDim.x) {
        const int kt = e / nm, f = e % nm, it = ot * s + kt - p;
        rows[kt][f] = (it >= 0 && it < t) ? feats[(int64_t)it * nm + f] : 0.0f;
    }
    __syncthreads();
    for (int ch = threadIdx.x; ch < c; ch += blockDim.x) {
        float wk[kMaxK * kMaxK];
#pragma unroll
        for (int i = 0; i < kMaxK * kMaxK; i++) {
            const int kt = i / kMaxK, kf = i % kMaxK;
            wk[i] = (kt < k && kf < k) ? w[(kt * k + kf) * c + ch] : 0.0f;
        }
        const float bc = b[ch];
        for (int of = 0; of < f1; of++) {
            float o = bc;
#pragma unroll
            for (int kt = 0; kt < kMaxK; kt++) {
                if (kt >= k) break;
                const int it = ot * s + kt - p;
                if (it < 0 || it >= t) continue;
#pragma unroll
                for (int kf = 0; kf < kMaxK; kf++) {
                    if (kf >= k) break;
                    const int i_f = of * s + kf - p;
                    if (i_f < 0 || i_f >= nm) continue;
                    o = o + wk[kt * kMaxK + kf] * rows[kt][i_f];
                }
            }
            out[((int64_t)ot * f1 + of) * c + ch] = o > 0.0f ? o : 0.0f;
        }
    }
}

// depthwise stage (subsampling.rs:163-190): y[ot][of][ch] = b[ch] + sum over (kt, kf) of w[kt*k+kf][ch] *
// x[ot*s+kt-p][of*s+kf-p][ch], no activation.
__global__ __launch_bounds__(256) void dwconv2d_kernel(const float *__restrict__ x, int tc, int fc, int k, int s,
                                                      const float *__restrict__ w, const float *__restrict__ b, int c,
                                                      int t2, int f2, float *__restrict__ y) {
    const int seg = blockIdx.x / (t2 * f2), pos = blockIdx.x % (t2 * f2);
    const int ot = pos / f2, of = pos % f2, p = (k - 1) / 2;
    x += (int64_t)seg * tc * fc * c;  // segment seg of [nseg][tc][fc][c] -> [nseg][t2][f2][c]
    y += (int64_t)seg * t2 * f2 * c;
    for (int ch = threadIdx.x; ch < c; ch += blockDim.x) {
        float o = b[ch];
        for (int kt = 0; kt < k; kt++) {
            const int it = ot * s + kt - p;
            if (it < 0 || it >= tc) continue;
            for (int kf = 0; kf < k; kf++) {
                const int i_f = of * s + kf - p;
                if (i_f < 0 || i_f >= fc) continue;
                o = o + w[(kt * k + kf) * c + ch] * x[((int64_t)it * fc + i_f) * c + ch];
            }
        }
        y[(int64_t)pos * c + ch] = o;
    }
}

// dwconv2d_kernel for the model's 3x3 stride-2 stages: a block is one output time row of one segment, a thread one
// channel; its nine weights stay in registers and it walks the output frequencies, each reading the two new input
// columns of the three rows (the first column is the previous output's last), so an output costs 6 loads instead
// of 18. Taps in the same order (kt outer, kf inner, out-of-range ones skipped), each o = o + w * x unfused.
__global__ __launch_bounds__(256) void dwconv2d_k3s2_kernel(const float *__restrict__ x, int tc, int fc,
                                                           const float *__restrict__ w, const float *__restrict__ b,
                                                           int c, int t2, int f2, float *__restrict__ y) {
    const int seg = blockIdx.x / t2, ot = blockIdx.x % t2;
    x += (int64_t)seg * tc * fc * c;
    y += ((int64_t)seg * t2 + ot) * f2 * c;
    for (int ch = threadIdx.x; ch < c; ch += blockDim.x) {
        float wk[9];
#pragma unroll
        for (int e = 0; e < 9; e++) wk[e] = w[e * c + ch];
        const float bias = b[ch];
        bool rv[3];
        const float *xr[3];
#pragma unroll
        for (int kt = 0; kt < 3; kt++) {
            const int it = 2 * ot + kt - 1;
            rv[kt] = it >= 0 && it < tc;
            xr[kt] = x + (int64_t)(rv[kt] ? it : 0) * fc * c + ch;
        }
        float prev[3] = {0.0f, 0.0f, 0.0f};  // column 2 of - 1 (of = 0: column -1, out of range)
        for (int of = 0; of < f2; of++) {
            const int f1 = 2 * of, f2c = 2 * of + 1;
            const bool v0 = of > 0, v2 = f2c < fc;  // column 2 of - 1 and 2 of + 1 in range (2 of < fc always)
            float cur1[3], cur2[3];
#pragma unroll
            for (int kt = 0; kt < 3; kt++) {
                cur1[kt] = rv[kt] ? xr[kt][(int64_t)f1 * c] : 0.0f;
                cur2[kt] = rv[kt] && v2 ? xr[kt][(int64_t)f2c * c] : 0.0f;
            }
            float o = bias;
#pragma unroll
            for (int kt = 0; kt < 3; kt++) {
                if (!rv[kt]) continue;
                if (v0) o = o + wk[kt * 3] * prev[kt];
                o = o + wk[kt * 3 + 1] * cur1[kt];
                if (v2) o = o + wk[kt * 3 + 2] * cur2[kt];
            }
#pragma unroll
            for (int kt = 0; kt < 3; kt++) prev[kt] = cur2[kt];
            y[(int64_t)of * c + ch] = o;
        }
    }
}

// Stage 0 and the first depthwise stage in one pass, without the stage-0 tensor in memory, for the model's shape (3x3
// kernels, stride 2, NM mel bins: F1 = NM / 2 stage-0 frequencies, F2 = F1 / 2 depthwise outputs). A block is one
// output time row ot2 of the depthwise stage, a thread one channel: it streams the stage-0 values of its channel
// over the input rows it = 2 ot2 + kt - 1 (kt ascending, in range) and, within a row, the frequencies in ascending
// order, each recomputed exactly as conv0_kernel does (taps in order, ReLU), and adds each into the depthwise
// outputs it feeds (of2 with 2 of2 + kf - 1 = i_f). For every depthwise output this visits its in-range taps in the
// reference's order (kt outer, kf inner), so the sums equal conv0_kernel followed by dwconv2d_kernel bit for bit.
// The three input rows of each stage-0 row are staged in LDS.
template <int NM>
__global__ __launch_bounds__(256) void conv0_dw_kernel(const float *__restrict__ feats, int t,
                                                      const float *__restrict__ w0, const float *__restrict__ b0,
                                                      const float *__restrict__ w1, const float *__restrict__ b1,
                                                      int c, int t1, int t2, float *__restrict__ y) {
    constexpr int F1 = NM / 2, F2 = F1 / 2;
    static_assert(NM % 4 == 0, "two stride-2 halvings without a remainder");
    __shared__ float rows[3][3][NM];  // [stage-0 row kt][its input row kt0][mel bin]
    const int ot2 = blockIdx.x % t2, seg = blockIdx.x / t2;
    feats += (int64_t)seg * t * NM;
    y += (int64_t)seg * t2 * F2 * c;
    for (int e = threadIdx.x; e < 9 * NM; e += blockDim.x) {
        const int kt = e / (3 * NM), kt0 = (e / NM) % 3, f = e % NM;
        const int it = 2 * ot2 + kt - 1, ii = 2 * it + kt0 - 1;
        rows[kt][kt0][f] = (it >= 0 && it < t1 && ii >= 0 && ii < t) ? feats[(int64_t)ii * NM + f] : 0.0f;
    }
    __syncthreads();
    for (int ch = threadIdx.x; ch < c; ch += blockDim.x) {
        float wa[9], wb[9];
#pragma unroll
        for (int i = 0; i < 9; i++) {
            wa[i] = w0[i * c + ch];
            wb[i] = w1[i * c + ch];
        }
        const float bc0 = b0[ch];
        float acc[F2];
#pragma unroll
        for (int o = 0; o < F2; o++) acc[o] = b1[ch];
        for (int kt = 0; kt < 3; kt++) {
            const int it = 2 * ot2 + kt - 1;
            if (it < 0 || it >= t1) continue;
            bool in_row[3];
#pragma unroll
            for (int kt0 = 0; kt0 < 3; kt0++) {
                const int ii = 2 * it + kt0 - 1;
                in_row[kt0] = ii >= 0 && ii < t;
            }
            const float *r0 = rows[kt][0], *r1 = rows[kt][1], *r2 = rows[kt][2];
#pragma unroll
            for (int i_f = 0; i_f < F1; i_f++) {
                // the stage-0 value (it, i_f) of this channel: taps (kt0, kf0) in order, bins 2 i_f + kf0 - 1
                float o = bc0;
#pragma unroll
                for (int kt0 = 0; kt0 < 3; kt0++) {
                    if (!in_row[kt0]) continue;
                    const float *r = kt0 == 0 ? r0 : kt0 == 1 ? r1 : r2;
#pragma unroll
                    for (int kf0 = 0; kf0 < 3; kf0++) {
                        const int fi = 2 * i_f + kf0 - 1;
                        if (fi < 0 || fi >= NM) continue;
                        o = o + wa[kt0 * 3 + kf0] * r[fi];
                    }
                }
                o = o > 0.0f ? o : 0.0f;
                // into the depthwise outputs it feeds, in ascending kf
                if (i_f % 2 == 1 && (i_f + 1) / 2 < F2) acc[(i_f + 1) / 2] = acc[(i_f + 1) / 2] + wb[kt * 3 + 0] * o;
                if (i_f % 2 == 0) acc[i_f / 2] = acc[i_f / 2] + wb[kt * 3 + 1] * o;
                if (i_f % 2 == 1) acc[(i_f - 1) / 2] = acc[(i_f - 1) / 2] + wb[kt * 3 + 2] * o;
            }
        }
#pragma unroll
        for (int o = 0; o < F2; o++) y[((int64_t)ot2 * F2 + o) * c + ch] = acc[o];
    }
}

// The whole subsampling (subsampling.rs:124-204) of nseg segments of t frames each on device buffers: feats
// [nseg][t][nm] -> out [nseg][t3][d_model]; scratch must hold 2 * nseg * t1 * f1 * c floats. Returns t3.
int64_t subsampling_seg(const float *feats, int64_t nseg, int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s,
                        const float *conv0_w, const float *conv0_b, const float *dw_w, const float *dw_b,
                        const float *pw_w, const float *pw_b, const float *lin_w, const float *lin_b,
                        int64_t d_model, float *scratch, float *out, hipStream_t st) {
    require(feats && conv0_w && conv0_b && dw_w && dw_b && pw_w && pw_b && lin_w && lin_b && scratch && out,
            "subsampling: NULL pointer");
    require(t > 0 && nm > 0 && nm <= kMaxMels && c > 0 && k > 0 && k <= kMaxK && s > 0 && c <= 1024,
            "subsampling: bad shape (k <= 3, n_mels <= 256)");
    const int p = (int)(k - 1) / 2;
    const int t1 = conv_out_len((int)t, (int)k, (int)s, p), f1 = conv_out_len((int)nm, (int)k, (int)s, p);
    require(nseg >= 1 && nseg * t1 * f1 * c < (1ll << 31), "subsampling: input too long");
    float *a = scratch, *bbuf = scratch + nseg * t1 * f1 * c;
    // the model's shape (3x3, stride 2, 128 mel bins) runs stage 0 inside the first depthwise stage
    const bool fused = k == 3 && s == 2 && nm == 128;
    if (!fused) {
        conv0_kernel<<<(unsigned)(nseg * t1), 256, 0, st>>>(feats, (int)t, (int)nm, (int)k, (int)s, conv0_w,
                                                                    conv0_b, (int)c, t1, f1, a);
        hip_check(hipGetLastError(), "conv0 kernel launch");
    }
    int tc = t1, fc = f1;
    for (int stage = 0; stage < 2; stage++) {
        const int t2 = conv_out_len(tc, (int)k, (int)s, p), f2 = conv_out_len(fc, (int)k, (int)s, p);
        if (stage == 0 && fused) {
            conv0_dw_kernel<128><<<(unsigned)(nseg * t2), 256, 0, st>>>(feats, (int)t, conv0_w, conv0_b, dw_w, dw_b,
                                                                         (int)c, t1, t2, bbuf);
            hip_check(hipGetLastError(), "conv0 + dwconv2d kernel launch");
        } else {
            if (k == 3 && s == 2)
                dwconv2d_k3s2_kernel<<<(unsigned)(nseg * t2), 256, 0, st>>>(a, tc, fc, dw_w + (int64_t)stage * 9 * c,
                                                                             dw_b + (int64_t)stage * c, (int)c, t2,
                                                                             f2, bbuf);
            else
                dwconv2d_kernel<<<(unsigned)(nseg * t2 * f2), 256, 0, st>>>(a, tc, fc, (int)k, (int)s,
                                                                              dw_w + (int64_t)stage * k * k * c,
                                                                              dw_b + (int64_t)stage * c, (int)c, t2,
                                                                              f2, bbuf);
            hip_check(hipGetLastError(), "dwconv2d kernel launch");
        }
        linear_f32(bbuf, nseg * t2 * f2, c, pw_w + (int64_t)stage * c * c, pw_b + (int64_t)stage * c, c, a, true,
                   st);
        tc = t2;
        fc = f2;
    }
    linear_f32(a, nseg * tc, (int64_t)fc * c, lin_w, lin_b, d_model, out, false, st);
    return tc;
}

int64_t subsampling(const float *feats, int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s, const float *conv0_w,
                    const float *conv0_b, const float *dw_w, const float *dw_b, const float *pw_w, const float *pw_b,
                    const float *lin_w, const float *lin_b, int64_t d_model, float *scratch, float *out,
                    hipStream_t st) {
    return subsampling_seg(feats, 1, t, nm, c, k, s, conv0_w, conv0_b, dw_w, dw_b, pw_w, pw_b, lin_w, lin_b, d_model,
                           scratch, out, st);
}

int64_t subsampling_frames(int64_t t, int64_t k, int64_t s) {
    const int p = (int)(k - 1) / 2;
    int n = (int)t;
    for (int i = 0; i < 3; i++) n = conv_out_len(n, (int)k, (int)s, p);
    return n;
}

int64_t subsampling_scratch_floats(int64_t t, int64_t nm, int64_t c, int64_t k, int64_t s) {
    const int p = (int)(k - 1) / 2;
    return 2 * (int64_t)conv_out_len((int)t, (int)k, (int)s, p) * conv_out_len((int)nm, (int)k, (int)s, p) * c;
}

// ---------------------------------------------------------------------------------------- host helpers

// encoder.rs:548-573: s = gamma / sqrt(var + 1e-5); w_t[kk][c] = dw[c][kk] * s; bias = beta - mean * s.
void fold_bn(const float *dw, const float *gamma, const float *beta, const float *mean, const float *var, int64_t d,
             int64_t k, float *dw_t, float *dw_bias) {
    for (int64_t c = 0; c < d; c++) {
        const float s = gamma[c] / std::sqrt(var[c] + 1e-5f);
        for (int64_t kk = 0; kk < k; kk++) dw_t[kk * d + c] = dw[c * k + kk] * s;
        dw_bias[c] = beta[c] - mean[c] * s;
    }
}

// encoder.rs:760-776 on the host, float arithmetic with the C library's powf / sinf / cosf.
void rel_pos_table(int64_t t, int64_t d, float *out) {
    const int64_t np = 2 * t - 1, half = d / 2;
    std::vector<float> inv((size_t)half);
    for (int64_t i = 0; i < half; i++) inv[(size_t)i] = 1.0f / ::powf(10000.0f, 2.0f * (float)i / (float)d);
    for (int64_t r = 0; r < np; r++) {
        const float pos = (float)(t - 1 - r);
        for (int64_t i = 0; i < half; i++) {
            const float f = inv[(size_t)i] * pos;
            out[r * d + 2 * i] = ::sinf(f);
            out[r * d + 2 * i + 1] = ::cosf(f);
        }
    }
}

// Device self-check of the activation functions: exp_poly, silu_fast and sigmoid_fast against their IEEE forms
// (exp_poly_ieee; x / (1 + exp_poly_ieee(-x)) and 1 / (...) with the IEEE division) over all 2^32 float inputs.
// NaN results count as equal to NaN; every other result must match bit for bit (the sign of zero included).
__global__ __launch_bounds__(256) void check_activations_kernel(unsigned long long *mismatch) {
    const uint64_t nthr = (uint64_t)gridDim.x * 256;
    unsigned long long c[3] = {0, 0, 0};
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < (1ull << 32); i += nthr) {
        const float x = __uint_as_float((uint32_t)i);
        const float got[3] = {exp_poly(x), silu_fast(x), sigmoid_fast(x)};
        const float want[3] = {exp_poly_ieee(x), silu_ieee(x), sigmoid_ieee(x)};
#pragma unroll
        for (int f = 0; f < 3; f++)
            c[f] += !((got[f] != got[f] && want[f] != want[f]) || __float_as_uint(got[f]) == __float_as_uint(want[f]));
    }
#pragma unroll
    for (int f = 0; f < 3; f++)
        if (c[f]) atomicAdd(&mismatch[f], c[f]);
}

void check_activations(uint64_t *mismatch_host) {
    unsigned long long *dev = nullptr;
    hip_check(hipMalloc(&dev, 3 * sizeof(unsigned long long)), "hipMalloc");
    hipError_t e = hipMemset(dev, 0, 3 * sizeof(unsigned long long));
    if (e == hipSuccess) {
        check_activations_kernel<<<16384, 256>>>(dev);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(mismatch_host, dev, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    (void)hipFree(dev);
    hip_check(e, "check_activations");
}

}  // namespace vx
