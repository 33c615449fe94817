// vx_gemm_small.hip — small-token ternary x int8 GEMM (a few hundred tokens: one utterance's frames) on gfx950 i8
// MFMA, bit-exact to voxrt's scalar kernel (crates/voxrt/src/kernels/mod.rs:166-210):
//
//   acc = 0; for each group g ascending: acc = fma((float)S_g, xs[t][g] * ws[o][g], acc); y = ep(acc) (+ bias)
//
// At a few hundred tokens the work of one GEMM is a few microseconds of the whole chip, so the kernel is built for
// latency: all workgroups of the grid are resident at once (several small ones per CU, which hide each other's
// memory latency), every workgroup issues all of its loads up front (the K steps of its four wavefronts in a
// register ring, the scales, the bias and, for AddScaled, the old outputs), and nothing between the first load and
// the last store waits for memory twice.
//
// A workgroup owns a (16 * MT) token x (16 * NT) output-row tile; its four wavefronts split K:
//   * one group (G = K): wavefront w takes K steps [w * nk / 4, (w + 1) * nk / 4);
//   * 128-column groups: chunk c holds groups 4c .. 4c + 3 and wavefront w takes group 4c + w (two steps).
// Operands of v_mfma_i32_16x16x64_i8: A = weight codes (trit + 1) widened to int8 (rows = output rows), B = activations
// (columns = tokens), both over K columns 16 * (l / 16) .. + 15 of the step for lane l. D element e of lane l is
// output row 4 * (l / 16) + e of token l % 16, so a lane's four sums of a block leave with one 16-byte LDS write.
// The int32 sums of the four wavefronts meet in LDS (exact in any order); then each thread owns 8 consecutive
// output rows of (16 * MT * NT / 32) tokens: for one group it adds the four partial sums and folds once; with
// groups it folds the chunk's four group sums in ascending group order after every chunk.
//
// Group-sum output (one group, Store): the exact int32 sums S (the fold's operand) are also stored, to the
// group_sums buffer [1][n][out], beside y.
//
// With 8, 16 or 32 128-column groups a second kernel, tgemm_small_ws_kernel, splits each workgroup into producer
// wavefronts (the MFMA chains) and consumer wavefronts (the fold, one chunk behind), so the fold of one chunk
// overlaps the loads and MFMAs of the next; it is the default for those shapes except the fused quantized output.
//
// Quantized output (16 x 128 tiles): instead of y, the epilogue writes the next GEMM's activations. The 16 fold
// threads of a token hold its 128 outputs of one 128-column group after the epilogue and bias, so the group's
// quantization (QuantAct::quantize_group, packed.rs:527-535: amax, s = amax / 127 or 1, inv = 1 / s, codes
// clamp(rint(x * inv)), code sum) reduces over those 16 lanes, and the f32 outputs never reach memory.
#include <algorithm>
#include <cstdio>
#include <cstring>

#include "vx_gemm.h"

namespace vx {
namespace {

constexpr int kMaxG = 32;  // groups staged in LDS (K <= 4096 with 128-column groups); kernels for K <= 1024 stage 8

// MT x NT blocks of 16 x 16; GROUPED: 128-column groups (else one group); D: K steps per wavefront in flight.
// MAXG: groups the LDS scale tables hold (8 or 32; sized so that a small K leaves room for more workgroups per CU).
// 16 x 128 tiles with a ring of at most 4 steps (one group, or a quantized output) are held to 168 registers, so
// that three workgroups fit per CU and a T = 338 grid of 704 tiles runs in one round.
template <int MT, int NT, bool GROUPED, int D, int EP, bool BIAS, bool QOUT, int MAXG, bool GSO = false>
__global__ __launch_bounds__(256, (MT == 1 && NT == 8 && D <= 4 && (!GROUPED || QOUT)) ? 3 : 1) void tgemm_small_kernel(
    const GemmArgs a, const int n_mt, const int per_xcd, const int ntiles) {
    static_assert(!GSO || (!GROUPED && !QOUT && EP == VX_EP_STORE), "group sums: one group, Store epilogue");
    constexpr int BM = 16 * MT, BN = 16 * NT, BNP = BN + 4;  // BNP: LDS row pitch (16-byte shift per token row)
    constexpr int TPR = BN / 8;                               // fold threads per token row
    constexpr int RPP = 256 / TPR;                            // token rows per fold pass
    constexpr int R = (BM + RPP - 1) / RPP;                   // fold passes (the last one partial if BM % RPP)
    constexpr int QX = GROUPED ? (MAXG * BM + 255) / 256 : 1, QW = GROUPED ? (MAXG * BN + 255) / 256 : 1;
    static_assert(!QOUT || (BN == 128 && BM % RPP == 0 && EP != VX_EP_ADD_SCALED),
                  "a quantized output group is one token row of a 128-row tile");
    // NRED = 2: with 32-group tables (K > 1024, eight or more chunks) the chunks alternate between two reduction
    // planes, so a chunk's fold needs no barrier after it (the next chunk writes the other plane, and the barrier
    // after that write orders it after every thread's reads of the plane it overwrites two chunks later); only for
    // tiles whose two planes and tables fit in LDS next to each other (at most 88 KB)
    constexpr int NRED = (GROUPED && MAXG > 8 && BM * BNP <= 2176) ? 2 : 1;
    __shared__ __attribute__((aligned(16))) int red[NRED][4][BM * BNP];
    __shared__ __attribute__((aligned(16))) float sxs[GROUPED ? MAXG * BM : 1], sws[GROUPED ? MAXG * BN : 1];
    __shared__ __attribute__((aligned(16))) int sgs[GROUPED ? MAXG * BM : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lq = lane >> 4;
    // workgroup b runs on XCD b % 8; the tiles of one XCD are a contiguous range of the tile order, in which
    // consecutive tiles share output rows (the weight tile) and walk the token tiles
    const int b = (int)blockIdx.x, tile = (b & 7) * per_xcd + (b >> 3);
    if (tile >= ntiles) return;  // the grid is a multiple of 8
    const int tm = tile % n_mt, tn = tile / n_mt;
    const int m0 = (int)a.m_base + tm * BM, n0 = tn * BN;
    const int inp = (int)a.inp, nk = inp / 64, nsteps = nk / 4, ng = (int)a.ng, np = (int)a.np;

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto grs = make_rsrc(a.xg, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);
    const auto yrs = make_rsrc(a.y, a.y_bytes);
    const auto brs = make_rsrc(a.bias, BIAS ? (uint32_t)(a.out * 4) : 0u);
    const auto gsrs = make_rsrc(a.gs, GSO ? a.y_bytes : 0u);  // [1][n][out] int32, the same layout as y

    // fold ownership: token rows tt0 + r * RPP of the tile, output rows c0 .. c0 + 7
    const int tt0 = tid / TPR, c0 = (tid % TPR) * 8, o0 = n0 + c0;
    const uint32_t out4 = (uint32_t)a.out * 4;

    // loads that only the fold and the epilogue need, issued before the K loop
    float xsr[GROUPED ? 1 : R];
    int gsr[GROUPED ? 1 : R];
    v4i wlo = v4i{0, 0, 0, 0}, whi = v4i{0, 0, 0, 0};
    if constexpr (!GROUPED) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            xsr[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, (uint32_t)(m0 + tt0 + r * RPP) * 4, 0, 0));
            gsr[r] = (int)__builtin_amdgcn_raw_buffer_load_b32(grs, (uint32_t)(m0 + tt0 + r * RPP) * 4, 0, 0);
        }
        wlo = __builtin_amdgcn_raw_buffer_load_b128(wsrs, (uint32_t)o0 * 4, 0, 0);
        whi = __builtin_amdgcn_raw_buffer_load_b128(wsrs, (uint32_t)o0 * 4 + 16, 0, 0);
    }
    v4i blo = v4i{0, 0, 0, 0}, bhi = v4i{0, 0, 0, 0};
    if constexpr (BIAS) {
        blo = __builtin_amdgcn_raw_buffer_load_b128(brs, (uint32_t)o0 * 4, 0, 0);
        bhi = __builtin_amdgcn_raw_buffer_load_b128(brs, (uint32_t)o0 * 4 + 16, 0, 0);
    }
    v4i olo[EP == VX_EP_ADD_SCALED ? R : 1], ohi[EP == VX_EP_ADD_SCALED ? R : 1];
    if constexpr (EP == VX_EP_ADD_SCALED) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t so = (uint32_t)(m0 + tt0 + r * RPP) * out4 + (uint32_t)o0 * 4;
            olo[r] = __builtin_amdgcn_raw_buffer_load_b128(yrs, so, 0, 0);
            ohi[r] = __builtin_amdgcn_raw_buffer_load_b128(yrs, so + 16, 0, 0);
        }
    }
    // groups: the token scales, code sums and weight scales of every group of the tile, loaded here and written to
    // LDS at the first chunk's fold (entries past the last group read zeros and are never used)
    uint32_t qx[QX], qg[QX], qw[QW];
    if constexpr (GROUPED) {
#pragma unroll
        for (int q = 0; q < QX; q++) {
            const int i = tid + 256 * q, g = i / BM, k = i % BM;
            const uint32_t off = g < ng ? (uint32_t)(g * np + m0 + k) * 4 : kOff;
            qx[q] = __builtin_amdgcn_raw_buffer_load_b32(srs, off, 0, 0);
            qg[q] = __builtin_amdgcn_raw_buffer_load_b32(grs, off, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < QW; q++) {
            const int i = tid + 256 * q, g = i / BN, k = i % BN;
            qw[q] = __builtin_amdgcn_raw_buffer_load_b32(wsrs, g < ng ? (uint32_t)(g * (int)a.out_pad + n0 + k) * 4 : kOff,
                                                         0, 0);
        }
    }

    // the K loop: step i of this wavefront is global step kb_of(i); activations of token m0 + 16 mb + l16 (a token
    // past n reads zeros: its offset lies past the end of xq), weight codes one dword per lane and block
    uint32_t va[MT];
#pragma unroll
    for (int mb = 0; mb < MT; mb++) va[mb] = (uint32_t)(m0 + 16 * mb + l16) * (uint32_t)inp + 16 * lq;
    auto kb_of = [&](int i) __attribute__((always_inline)) {
        return GROUPED ? ((i >> 1) * 4 + wave) * 2 + (i & 1) : wave * nsteps + i;
    };
    v4i ra[D][MT];
    uint32_t rb[D][NT];
    auto issue = [&](int i, int slot) __attribute__((always_inline)) {
        const int kb = kb_of(i);
#pragma unroll
        for (int mb = 0; mb < MT; mb++) ra[slot][mb] = __builtin_amdgcn_raw_buffer_load_b128(xrs, va[mb], kb * 64, 0);
#pragma unroll
        for (int nb = 0; nb < NT; nb++)
            rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)lane * 4, ((n0 / 16 + nb) * nk + kb) * 256, 0);
    };

    // the weight operand is the code trit + 1, so a group's sum over its columns is S_g + sum(x codes) of the token
    // and group, and the fold subtracts the quantizer's gsum (exact in int32)
    v4i acc[MT][NT];
#pragma unroll
    for (int mb = 0; mb < MT; mb++)
#pragma unroll
        for (int nb = 0; nb < NT; nb++) acc[mb][nb] = v4i{0, 0, 0, 0};
    float accf[R][8];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int j = 0; j < 8; j++) accf[r][j] = 0.0f;
    v4i gso[GSO ? R : 1][2];  // the exact sums of the group-sum output

    // int32 sums of this wavefront -> its LDS plane (one 16-byte write per block)
    auto to_lds = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int nb = 0; nb < NT; nb++)
                *(v4i *)&red[buf][wave][(16 * mb + l16) * BNP + 16 * nb + 4 * lq] = acc[mb][nb];
    };

    // step i of this wavefront from ring slot `slot`; with groups D is even, so the step's position in its group
    // is the slot's parity (known at compile time)
    auto compute = [&](int slot, int i) __attribute__((always_inline)) {
        v4i bw[NT];
#pragma unroll
        for (int nb = 0; nb < NT; nb++) bw[nb] = widen_codes(rb[slot][nb]);
        const bool first = GROUPED && (slot & 1) == 0;  // a group's chain starts from zero
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int nb = 0; nb < NT; nb++)
                acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[nb], ra[slot][mb],
                                                                     first ? v4i{0, 0, 0, 0} : acc[mb][nb], 0, 0, 0);
        if constexpr (GROUPED) {
            if ((slot & 1) == 1) {  // chunk (i >> 1) complete: fold groups 4c .. 4c + 3 in ascending order
                if (i == 1) {
#pragma unroll
                    for (int q = 0; q < QX; q++)
                        if (tid + 256 * q < MAXG * BM) {
                            sxs[tid + 256 * q] = __uint_as_float(qx[q]);
                            sgs[tid + 256 * q] = (int)qg[q];
                        }
#pragma unroll
                    for (int q = 0; q < QW; q++)
                        if (tid + 256 * q < MAXG * BN) sws[tid + 256 * q] = __uint_as_float(qw[q]);
                }
                const int c = i >> 1;
                const int buf = NRED == 2 ? (c & 1) : 0;
                to_lds(buf);
                __syncthreads();
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const int g = 4 * c + w;
                    const float4 wa = *(const float4 *)&sws[g * BN + c0];
                    const float4 wb = *(const float4 *)&sws[g * BN + c0 + 4];
                    const float wsv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const int tt = tt0 + r * RPP;
                        if (BM % RPP != 0 && tt >= BM) continue;
                        const float xs = sxs[g * BM + tt];
                        const int gsum = sgs[g * BM + tt];
                        const v4i lo = *(const v4i *)&red[buf][w][tt * BNP + c0];
                        const v4i hi = *(const v4i *)&red[buf][w][tt * BNP + c0 + 4];
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            accf[r][j] = __builtin_fmaf((float)(lo[j] - gsum), xs * wsv[j], accf[r][j]);
                            accf[r][4 + j] = __builtin_fmaf((float)(hi[j] - gsum), xs * wsv[4 + j], accf[r][4 + j]);
                        }
                    }
                }
                if constexpr (NRED == 1) __syncthreads();
            }
        }
    };

    // nsteps is a multiple of D (the host picks D): prologue, steady state, drain
#pragma unroll
    for (int i = 0; i < D; i++) issue(i, i);
    for (int s0 = 0; s0 < nsteps - D; s0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            compute(i, s0 + i);
            issue(s0 + i + D, i);
        }
    }
#pragma unroll
    for (int i = 0; i < D; i++) compute(i, nsteps - D + i);

    if constexpr (!GROUPED) {
        to_lds(0);
        __syncthreads();
        const float wsv[8] = {__int_as_float(wlo[0]), __int_as_float(wlo[1]), __int_as_float(wlo[2]),
                              __int_as_float(wlo[3]), __int_as_float(whi[0]), __int_as_float(whi[1]),
                              __int_as_float(whi[2]), __int_as_float(whi[3])};
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int tt = tt0 + r * RPP;
            if (BM % RPP != 0 && tt >= BM) continue;
            int S[8];
#pragma unroll
            for (int j = 0; j < 8; j++) S[j] = -gsr[r];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const v4i lo = *(const v4i *)&red[0][w][tt * BNP + c0];
                const v4i hi = *(const v4i *)&red[0][w][tt * BNP + c0 + 4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    S[j] += lo[j];
                    S[4 + j] += hi[j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; j++) accf[r][j] = __builtin_fmaf((float)S[j], xsr[r] * wsv[j], 0.0f);
            if constexpr (GSO) {
                gso[r][0] = v4i{S[0], S[1], S[2], S[3]};
                gso[r][1] = v4i{S[4], S[5], S[6], S[7]};
            }
        }
    }

    // epilogue (kernels/mod.rs:41-48), bias after it; tokens outside [t0, t1) are not written
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int t = m0 + tt0 + r * RPP;
        v4i lo, hi;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = accf[r][j];
            float res = v;
            if constexpr (EP == VX_EP_SILU) res = silu_fast(v);
            if constexpr (EP == VX_EP_ADD_SCALED)
                res = __builtin_fmaf(a.alpha, v, __int_as_float(j < 4 ? olo[r][j] : ohi[r][j - 4]));
            if constexpr (BIAS) res = res + __int_as_float(j < 4 ? blo[j] : bhi[j - 4]);
            if (j < 4)
                lo[j] = __float_as_int(res);
            else
                hi[j - 4] = __float_as_int(res);
        }
        if constexpr (QOUT) {
            // quantize_group over the token's 128 outputs: 8 per lane on 16 adjacent lanes
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) m = fmaxf(m, fmaxf(fabsf(__int_as_float(lo[j])), fabsf(__int_as_float(hi[j]))));
            m = lane_group_max<16>(m);
            const float s = m == 0.0f ? 1.0f : m / 127.0f;
            const float inv = 1.0f / s;
            uint32_t w0 = 0, w1 = 0;
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int8_t c0 = code_of(__int_as_float(lo[j]), inv), c1 = code_of(__int_as_float(hi[j]), inv);
                sum += (int)c0 + (int)c1;
                w0 |= (uint32_t)(uint8_t)c0 << (8 * j);
                w1 |= (uint32_t)(uint8_t)c1 << (8 * j);
            }
            sum = lane_group_sum<16>(sum);
            const int64_t gi = (int64_t)(o0 / 128) * a.np + t;
            if (t < a.n) {
                *(uint2 *)(a.qo + (int64_t)t * a.out + o0) = make_uint2(w0, w1);
                if ((tid & 15) == 0) {
                    a.qs[gi] = s;
                    a.qg[gi] = sum;
                }
            } else if (t < a.np && (tid & 15) == 0) {  // pad tokens: zero scale and code sum
                a.qs[gi] = 0.0f;
                a.qg[gi] = 0;
            }
        } else if (t >= a.t0 && t < a.t1 && (BM % RPP == 0 || tt0 + r * RPP < BM)) {
            const uint32_t so = (uint32_t)t * out4 + (uint32_t)o0 * 4;
            store_b128_sep(lo, yrs, so, 0);
            store_b128_sep(hi, yrs, so + 16, 0);
            if constexpr (GSO) {
                store_b128_sep(gso[r][0], gsrs, so, 0);
                store_b128_sep(gso[r][1], gsrs, so + 16, 0);
            }
        }
    }
}

// 128-column groups with producer and consumer wavefronts: eight wavefronts per workgroup, two per SIMD.
//   * producers (wavefronts 0-3): in chunk c, wavefront p computes group 4c + p over its two 64-column steps (the
//     same operands, ring and MFMA roles as tgemm_small_kernel), the chain seeded with -gsum of its token and
//     group so that it ends at S_g exactly, and writes the int32 sums to an LDS plane;
//   * consumers (wavefronts 4-7): after the barrier that ends chunk c they fold its four groups in ascending order,
//     acc = fma((float)S_g, xs * ws, acc), while the producers already run chunk c + 1, so on each SIMD the fold's
//     VALU work overlaps the other wavefront's MFMAs and memory waits; then the epilogue.
// NPL = 2: chunk c uses plane c % 2, one barrier per chunk (chunk c + 2 overwrites the plane of chunk c only after
// the barrier that ends chunk c + 1, which each consumer reaches after folding chunk c). NPL = 1 (half the LDS):
// the producers also wait, before writing chunk c, for a second barrier that the consumers reach after folding
// chunk c - 1.
template <int MT, int NT, int D, int EP, bool BIAS, bool QOUT, int MAXG, int NPL>
__global__ __launch_bounds__(512, NPL == 1 ? 2 : 1) void tgemm_small_ws_kernel(const GemmArgs a, const int n_mt,
                                                                               const int per_xcd, const int ntiles) {
    constexpr int BM = 16 * MT, BN = 16 * NT, BNP = BN + 4;
    constexpr int TPR = BN / 8, RPP = 256 / TPR, R = (BM + RPP - 1) / RPP;
    static_assert(D % 2 == 0, "a group is two ring steps");
    static_assert(!QOUT || (BN == 128 && BM % RPP == 0 && EP != VX_EP_ADD_SCALED),
                  "a quantized output group is one token row of a 128-row tile");
    __shared__ __attribute__((aligned(16))) int red[NPL][4][BM * BNP];
    __shared__ __attribute__((aligned(16))) float sxs[MAXG * BM], sws[MAXG * BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = (int)blockIdx.x, tile = (b & 7) * per_xcd + (b >> 3);
    if (tile >= ntiles) return;  // the whole workgroup: the grid is a multiple of 8
    const int tm = tile % n_mt, tn = tile / n_mt;
    const int m0 = (int)a.m_base + tm * BM, n0 = tn * BN;
    const int inp = (int)a.inp, nk = inp / 64, ng = (int)a.ng, np = (int)a.np, nch = ng / 4;

    if (wave < 4) {
        // ---- producer: groups 4c + wave, c = 0 .. nch - 1; ring step i is step (i & 1) of group 4 (i >> 1) + wave
        const int l16 = lane & 15, lq = lane >> 4;
        const auto xrs = make_rsrc(a.xq, a.xq_bytes);
        const auto wrs = make_rsrc(a.w, a.w_bytes);
        const auto grs = make_rsrc(a.xg, a.xs_bytes);
        uint32_t va[MT], vg[MT];
#pragma unroll
        for (int mb = 0; mb < MT; mb++) {
            va[mb] = (uint32_t)(m0 + 16 * mb + l16) * (uint32_t)inp + 16 * lq;
            vg[mb] = (uint32_t)(m0 + 16 * mb + l16) * 4;
        }
        const int nsteps = 2 * nch;
        v4i ra[D][MT];
        uint32_t rb[D][NT], rg[D / 2][MT];
        auto issue = [&](int i, int slot) __attribute__((always_inline)) {
            const int g = 4 * (i >> 1) + wave, kb = 2 * g + (i & 1);
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
                ra[slot][mb] = __builtin_amdgcn_raw_buffer_load_b128(xrs, va[mb], kb * 64, 0);
#pragma unroll
            for (int nb = 0; nb < NT; nb++)
                rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)lane * 4, ((n0 / 16 + nb) * nk + kb) * 256, 0);
            if ((slot & 1) == 0) {
#pragma unroll
                for (int mb = 0; mb < MT; mb++)
                    rg[slot / 2][mb] = __builtin_amdgcn_raw_buffer_load_b32(grs, vg[mb], g * np * 4, 0);
            }
        };
        v4i acc[MT][NT];
        auto compute = [&](int slot, int i) __attribute__((always_inline)) {
            v4i bw[NT];
#pragma unroll
            for (int nb = 0; nb < NT; nb++) bw[nb] = widen_codes(rb[slot][nb]);
            if ((slot & 1) == 0) {
                // the weight operand is the code trit + 1: seeded with -gsum, the chain ends at sum(trit * x)
#pragma unroll
                for (int mb = 0; mb < MT; mb++) {
                    const int s = -(int)rg[slot / 2][mb];
                    const v4i seed = v4i{s, s, s, s};
#pragma unroll
                    for (int nb = 0; nb < NT; nb++)
                        acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[nb], ra[slot][mb], seed, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int mb = 0; mb < MT; mb++)
#pragma unroll
                    for (int nb = 0; nb < NT; nb++)
                        acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[nb], ra[slot][mb], acc[mb][nb], 0, 0, 0);
                const int c = i >> 1;
                if (NPL == 1 && c > 0) __syncthreads();  // the consumers have folded chunk c - 1
                const int buf = NPL == 2 ? (c & 1) : 0;
#pragma unroll
                for (int mb = 0; mb < MT; mb++)
#pragma unroll
                    for (int nb = 0; nb < NT; nb++)
                        *(v4i *)&red[buf][wave][(16 * mb + l16) * BNP + 16 * nb + 4 * lq] = acc[mb][nb];
                __syncthreads();  // chunk c is in its plane
            }
        };
        // the ring in program order (the scheduler would otherwise group the loads by kind and wait for most of
        // the ring before the first step)
#pragma unroll
        for (int i = 0; i < D; i++) {
            issue(i, i);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int s0 = 0; s0 < nsteps - D; s0 += D) {
#pragma unroll
            for (int i = 0; i < D; i++) {
                compute(i, s0 + i);
                __builtin_amdgcn_sched_barrier(0);
                issue(s0 + i + D, i);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int i = 0; i < D; i++) {
            compute(i, nsteps - D + i);
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }

    // ---- consumer: thread ct owns token rows tt0 + r * RPP of the tile and output rows c0 .. c0 + 7
    const int ct = tid - 256;
    const int tt0 = ct / TPR, c0 = (ct % TPR) * 8, o0 = n0 + c0;
    const uint32_t out4 = (uint32_t)a.out * 4;
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);
    const auto yrs = make_rsrc(a.y, a.y_bytes);
    const auto brs = make_rsrc(a.bias, BIAS ? (uint32_t)(a.out * 4) : 0u);
    // the token and weight scales of every group of the tile (entries past the last group read zeros, unused)
#pragma unroll
    for (int q = 0; q < (MAXG * BM + 255) / 256; q++) {
        const int i = ct + 256 * q, g = i / BM, k = i % BM;
        if (i < MAXG * BM)
            sxs[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                srs, g < ng ? (uint32_t)(g * np + m0 + k) * 4 : kOff, 0, 0));
    }
#pragma unroll
    for (int q = 0; q < (MAXG * BN + 255) / 256; q++) {
        const int i = ct + 256 * q, g = i / BN, k = i % BN;
        if (i < MAXG * BN)
            sws[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                wsrs, g < ng ? (uint32_t)(g * (int)a.out_pad + n0 + k) * 4 : kOff, 0, 0));
    }
    v4i blo = v4i{0, 0, 0, 0}, bhi = v4i{0, 0, 0, 0};
    if constexpr (BIAS) {
        blo = __builtin_amdgcn_raw_buffer_load_b128(brs, (uint32_t)o0 * 4, 0, 0);
        bhi = __builtin_amdgcn_raw_buffer_load_b128(brs, (uint32_t)o0 * 4 + 16, 0, 0);
    }
    v4i olo[EP == VX_EP_ADD_SCALED ? R : 1], ohi[EP == VX_EP_ADD_SCALED ? R : 1];
    if constexpr (EP == VX_EP_ADD_SCALED) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t so = (uint32_t)(m0 + tt0 + r * RPP) * out4 + (uint32_t)o0 * 4;
            olo[r] = __builtin_amdgcn_raw_buffer_load_b128(yrs, so, 0, 0);
            ohi[r] = __builtin_amdgcn_raw_buffer_load_b128(yrs, so + 16, 0, 0);
        }
    }
    float accf[R][8];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int j = 0; j < 8; j++) accf[r][j] = 0.0f;
    for (int c = 0; c < nch; c++) {
        if (NPL == 1 && c > 0) __syncthreads();  // chunk c - 1 folded: the producers may overwrite the plane
        __syncthreads();                          // chunk c is in its plane (the first one also orders the tables)
        const int buf = NPL == 2 ? (c & 1) : 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const int g = 4 * c + w;
            const float4 wa = *(const float4 *)&sws[g * BN + c0];
            const float4 wb = *(const float4 *)&sws[g * BN + c0 + 4];
            const float wsv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int tt = tt0 + r * RPP;
                if (BM % RPP != 0 && tt >= BM) continue;
                const float xs = sxs[g * BM + tt];
                const v4i lo = *(const v4i *)&red[buf][w][tt * BNP + c0];
                const v4i hi = *(const v4i *)&red[buf][w][tt * BNP + c0 + 4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    accf[r][j] = __builtin_fmaf((float)lo[j], xs * wsv[j], accf[r][j]);
                    accf[r][4 + j] = __builtin_fmaf((float)hi[j], xs * wsv[4 + j], accf[r][4 + j]);
                }
            }
        }
    }

    // epilogue (kernels/mod.rs:41-48), bias after it; tokens outside [t0, t1) are not written
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int t = m0 + tt0 + r * RPP;
        v4i lo, hi;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = accf[r][j];
            float res = v;
            if constexpr (EP == VX_EP_SILU) res = silu_fast(v);
            if constexpr (EP == VX_EP_ADD_SCALED)
                res = __builtin_fmaf(a.alpha, v, __int_as_float(j < 4 ? olo[r][j] : ohi[r][j - 4]));
            if constexpr (BIAS) res = res + __int_as_float(j < 4 ? blo[j] : bhi[j - 4]);
            if (j < 4)
                lo[j] = __float_as_int(res);
            else
                hi[j - 4] = __float_as_int(res);
        }
        if constexpr (QOUT) {
            // quantize_group over the token's 128 outputs: 8 per lane on 16 adjacent lanes
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) m = fmaxf(m, fmaxf(fabsf(__int_as_float(lo[j])), fabsf(__int_as_float(hi[j]))));
            m = lane_group_max<16>(m);
            const float s = m == 0.0f ? 1.0f : m / 127.0f;
            const float inv = 1.0f / s;
            uint32_t w0 = 0, w1 = 0;
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int8_t q0 = code_of(__int_as_float(lo[j]), inv), q1 = code_of(__int_as_float(hi[j]), inv);
                sum += (int)q0 + (int)q1;
                w0 |= (uint32_t)(uint8_t)q0 << (8 * j);
                w1 |= (uint32_t)(uint8_t)q1 << (8 * j);
            }
            sum = lane_group_sum<16>(sum);
            const int64_t gi = (int64_t)(o0 / 128) * a.np + t;
            if (t < a.n) {
                *(uint2 *)(a.qo + (int64_t)t * a.out + o0) = make_uint2(w0, w1);
                if ((ct & 15) == 0) {
                    a.qs[gi] = s;
                    a.qg[gi] = sum;
                }
            } else if (t < a.np && (ct & 15) == 0) {  // pad tokens: zero scale and code sum
                a.qs[gi] = 0.0f;
                a.qg[gi] = 0;
            }
        } else if (t >= a.t0 && t < a.t1 && (BM % RPP == 0 || tt0 + r * RPP < BM)) {
            const uint32_t so = (uint32_t)t * out4 + (uint32_t)o0 * 4;
            store_b128_sep(lo, yrs, so, 0);
            store_b128_sep(hi, yrs, so + 16, 0);
        }
    }
}

// deepest ring of K steps whose operands (MT activation and NT weight registers per step) fit in 128 registers
constexpr int max_ring(int mt, int nt) { return 128 / (4 * mt + nt) >= 8 ? 8 : 128 / (4 * mt + nt) >= 4 ? 4 : 2; }

struct SmallPlan {
    int mt = 0, nt = 0, d = 0, tiles = 0;
};

bool tile_ok(const GemmArgs &a, int mt, int nt) {
    static const int tiles[][2] = {{1, 8}, {2, 4}, {2, 8}, {3, 2}, {3, 4}, {3, 8}};
    for (const auto &t : tiles)
        if (t[0] == mt && t[1] == nt) return a.out % (16 * nt) == 0;
    return false;
}

// Tile choice, from measurements of the encoder's shapes at 125, 338 and 750 tokens: with one group, 16 x 128 tiles
// (several small workgroups per CU hide each other's memory latency); with 128-column
// groups 32 x 64 tiles below 512 tokens, except for the wide projections from K = 1024 (N >= 3072: q|k|v, FFN up) at
// 256 tokens or more, where the split-K kernel over groups is as fast or faster.
SmallPlan plan_small(const GemmArgs &a, bool grouped, int force_mt, int force_nt) {
    const int64_t ntok = a.t1 - a.m_base, nk = a.inp / 64;
    SmallPlan best;
    if (force_mt) {
        if (tile_ok(a, force_mt, force_nt)) best.mt = force_mt, best.nt = force_nt;
    } else if (!grouped) {
        if (tile_ok(a, 1, 8))
            best.mt = 1, best.nt = 8;
        else if (tile_ok(a, 2, 4))
            best.mt = 2, best.nt = 4;
        else if (tile_ok(a, 3, 2))
            best.mt = 3, best.nt = 2;
    } else if (ntok < 512 && !(a.inp <= 1024 && a.out >= 3072 && ntok >= 256)) {
        if (tile_ok(a, 2, 4))
            best.mt = 2, best.nt = 4;
        else if (tile_ok(a, 3, 2))
            best.mt = 3, best.nt = 2;
    }
    if (best.mt) best.tiles = (int)((ntok + 16 * best.mt - 1) / (16 * best.mt) * (a.out / (16 * best.nt)));
    if (best.mt == 0) return best;
    // ring depth: a power of two dividing the wavefront's steps, at most 128 registers of operands in flight
    const int steps = (int)(nk / 4), dmax = max_ring(best.mt, best.nt);
    best.d = 1;
    while (best.d * 2 <= dmax && steps % (best.d * 2) == 0) best.d *= 2;
    if (grouped && best.d < 2) best.mt = 0;  // a group is two steps
    return best;
}

template <int MT, int NT, bool GROUPED, int D, int MAXG>
void launch_small_g(const GemmArgs &a, int grid, int n_mt, int per_xcd, int ntiles, hipStream_t st) {
    const bool bias = a.bias != nullptr;
    if constexpr (MT == 1 && NT == 8) {
        if (a.qo) {
#define VX_SMALLQ(EP)                                                                                             \
    (bias ? tgemm_small_kernel<MT, NT, GROUPED, D, EP, true, true, MAXG>                                          \
          : tgemm_small_kernel<MT, NT, GROUPED, D, EP, false, true, MAXG>)
            auto k = a.ep == VX_EP_SILU ? VX_SMALLQ(VX_EP_SILU) : VX_SMALLQ(VX_EP_STORE);
#undef VX_SMALLQ
            k<<<grid, 256, 0, st>>>(a, n_mt, per_xcd, ntiles);
            return;
        }
    }
    if constexpr (!GROUPED) {
        if (a.gs) {  // group sums (one group): Store only
            auto k = bias ? tgemm_small_kernel<MT, NT, false, D, VX_EP_STORE, true, false, MAXG, true>
                          : tgemm_small_kernel<MT, NT, false, D, VX_EP_STORE, false, false, MAXG, true>;
            k<<<grid, 256, 0, st>>>(a, n_mt, per_xcd, ntiles);
            return;
        }
    }
#define VX_SMALL(EP)                                                                                              \
    (bias ? tgemm_small_kernel<MT, NT, GROUPED, D, EP, true, false, MAXG>                                         \
          : tgemm_small_kernel<MT, NT, GROUPED, D, EP, false, false, MAXG>)
    auto k = a.ep == VX_EP_SILU ? VX_SMALL(VX_EP_SILU) : a.ep == VX_EP_ADD_SCALED ? VX_SMALL(VX_EP_ADD_SCALED)
                                                                                  : VX_SMALL(VX_EP_STORE);
#undef VX_SMALL
    k<<<grid, 256, 0, st>>>(a, n_mt, per_xcd, ntiles);
}

// the scale tables for 8 groups when K <= 1024 (the LDS then admits more workgroups per CU), else for 32
template <int MT, int NT, bool GROUPED, int D>
void launch_small_ep(const GemmArgs &a, int grid, int n_mt, int per_xcd, int ntiles, hipStream_t st) {
    if constexpr (GROUPED && D <= 4) {
        if (a.ng <= 8) return launch_small_g<MT, NT, GROUPED, D, 8>(a, grid, n_mt, per_xcd, ntiles, st);
    }
    launch_small_g<MT, NT, GROUPED, D, GROUPED ? kMaxG : 1>(a, grid, n_mt, per_xcd, ntiles, st);
}

template <int MT, int NT, bool GROUPED>
void launch_small_d(const GemmArgs &a, int d, int grid, int n_mt, int per_xcd, int ntiles, hipStream_t st) {
    if constexpr (max_ring(MT, NT) >= 8)
        if (d == 8) return launch_small_ep<MT, NT, GROUPED, 8>(a, grid, n_mt, per_xcd, ntiles, st);
    if (d == 4)
        launch_small_ep<MT, NT, GROUPED, 4>(a, grid, n_mt, per_xcd, ntiles, st);
    else if (d == 2)
        launch_small_ep<MT, NT, GROUPED, 2>(a, grid, n_mt, per_xcd, ntiles, st);
    else if constexpr (!GROUPED)
        launch_small_ep<MT, NT, GROUPED, 1>(a, grid, n_mt, per_xcd, ntiles, st);
}

template <bool GROUPED>
void launch_small(const GemmArgs &a, const SmallPlan &p, int grid, int n_mt, int per_xcd, int ntiles, hipStream_t st) {
#define VX_TILE(M, N)                                                                                             \
    if (p.mt == M && p.nt == N) return launch_small_d<M, N, GROUPED>(a, p.d, grid, n_mt, per_xcd, ntiles, st);
    VX_TILE(1, 8) VX_TILE(2, 4) VX_TILE(2, 8) VX_TILE(3, 2) VX_TILE(3, 4) VX_TILE(3, 8)
#undef VX_TILE
}

template <int MT, int NT, int NPL, int D, int MAXG>
void launch_ws_g(const GemmArgs &a, int grid, int n_mt, int per_xcd, int ntiles, hipStream_t st) {
    const bool bias = a.bias != nullptr;
    if constexpr (NT == 8) {  // 128-row tiles: the quantized output
#define VX_WSQ(EP)                                                                                                \
    (bias ? tgemm_small_ws_kernel<MT, NT, D, EP, true, true, MAXG, NPL>                                           \
          : tgemm_small_ws_kernel<MT, NT, D, EP, false, true, MAXG, NPL>)
        auto k = a.ep == VX_EP_SILU ? VX_WSQ(VX_EP_SILU) : VX_WSQ(VX_EP_STORE);
#undef VX_WSQ
        k<<<grid, 512, 0, st>>>(a, n_mt, per_xcd, ntiles);
    } else {
#define VX_WS(EP)                                                                                                 \
    (bias ? tgemm_small_ws_kernel<MT, NT, D, EP, true, false, MAXG, NPL>                                          \
          : tgemm_small_ws_kernel<MT, NT, D, EP, false, false, MAXG, NPL>)
        auto k = a.ep == VX_EP_SILU ? VX_WS(VX_EP_SILU) : a.ep == VX_EP_ADD_SCALED ? VX_WS(VX_EP_ADD_SCALED)
                                                                                   : VX_WS(VX_EP_STORE);
#undef VX_WS
        k<<<grid, 512, 0, st>>>(a, n_mt, per_xcd, ntiles);
    }
}

// The producer/consumer kernel for 8 groups (K = 1024, a ring of 2 steps per producer) or 16 / 32 groups (a ring
// of 4): 32 x 64 tiles with two LDS planes for y, 16 x 128 or 32 x 128 tiles with one plane for the quantized output
// (the next GEMM's activations, 8 groups only, a ring of 4). Launches nothing and returns false for other shapes or a
// forced tile it is not built for.
bool launch_ws(const GemmArgs &a, bool qout, int fm, int fn, hipStream_t st) {
    if (a.ng != 8 && a.ng != 16 && a.ng != 32) return false;
    int mt = qout ? 1 : 2, nt = qout ? 8 : 4;
    if (fm) {
        if (qout ? !((fm == 1 || fm == 2) && fn == 8) : !((fm == 1 || fm == 2) && fn == 4)) return false;
        mt = fm;
        nt = fn;
    }
    if (a.out % (16 * nt) != 0 || (qout && a.ng != 8)) return false;
    const int64_t ntok = a.t1 - a.m_base;
    // 16 x 64 tiles for Store (q|k|v, pw1 at T = 338: 7.56 / 5.56 -> 7.06 / 5.22 us with 32 x 64 tiles), and for
    // AddScaled where 32 x 64 tiles would leave more than half the CUs idle (T = 125: FFN-down 9.13 -> 8.45 us) or
    // give every CU more than one and a half (T = 750: FFN-down, o-proj 13.38 / 5.71 -> 12.28 / 5.36 us); in
    // between (T = 338) the 32-token tile is faster (FFN-down 8.63 against 9.86 us)
    if (!qout && !fm) {
        const int64_t t32 = ((ntok + 31) / 32) * (a.out / (16 * nt));
        if (a.ep != VX_EP_ADD_SCALED || t32 < cu_count() / 2 || 2 * t32 >= 3 * (int64_t)cu_count()) mt = 1;
    }
    const int n_mt = (int)((ntok + 16 * mt - 1) / (16 * mt)), tiles = n_mt * (int)(a.out / (16 * nt));
    const int per_xcd = (tiles + 7) / 8, grid = 8 * per_xcd;
    if (qout) {
        if (mt == 1)
            launch_ws_g<1, 8, 1, 4, 8>(a, grid, n_mt, per_xcd, tiles, st);
        else
            launch_ws_g<2, 8, 1, 4, 8>(a, grid, n_mt, per_xcd, tiles, st);
    } else if (a.ng == 8) {
        // shallow rings: the loads of the whole workgroup at its start queue behind each other, so a deep ring
        // delays the first chunk; inside the encoder (operands not in L2) K = 4096 keeps two chunks in flight
        // (encoder T = 338 / 750: rings 4 and 8 -> 2 and 4, 3.049 / 4.852 -> 3.024 / 4.663 ms; alone, o-proj at
        // T = 338: 4.48 -> 4.24 us)
        if (mt == 1)
            launch_ws_g<1, 4, 2, 2, 8>(a, grid, n_mt, per_xcd, tiles, st);
        else
            launch_ws_g<2, 4, 2, 2, 8>(a, grid, n_mt, per_xcd, tiles, st);
    } else {
        if (mt == 1)
            launch_ws_g<1, 4, 2, 4, kMaxG>(a, grid, n_mt, per_xcd, tiles, st);
        else
            launch_ws_g<2, 4, 2, 4, kMaxG>(a, grid, n_mt, per_xcd, tiles, st);
    }
    return true;
}

}  // namespace

bool gemm_small(const GemmArgs &a, hipStream_t st) {
    const bool grouped = a.ng > 1;
    if (a.qo) {  // quantized output: 16 x 128 tiles, Store or SiLU, whole tokens from 0
        if (a.out % 128 != 0 || a.ep == VX_EP_ADD_SCALED || a.m_base != 0 || a.t0 != 0 || a.t1 != a.n) return false;
        if (a.gs != nullptr || a.r0 != 0 || a.r1 != a.out || a.n > 1024) return false;
        if (grouped ? (a.spg != 2 || a.ng % 4 != 0 || a.ng > kMaxG) : (a.inp / 64) % 4 != 0) return false;
        SmallPlan p;
        p.mt = 1;
        p.nt = 8;
        p.tiles = (int)((a.n + 15) / 16 * (a.out / 128));
        const int steps = (int)(a.inp / 64 / 4);
        p.d = 1;
        while (p.d * 2 <= max_ring(1, 8) && steps % (p.d * 2) == 0) p.d *= 2;
        if (grouped && p.d < 2) return false;
        const int n_mt = (int)((a.n + 15) / 16), per_xcd = (p.tiles + 7) / 8;
        // up to 128 tokens the producer/consumer kernel (FFN-up at T = 125: 5.51 -> 5.06 us; from 338 tokens the
        // four-wavefront kernel is faster, 8.27 / 14.3 against 10.1 / 17.9 us at T = 338 / 750)
        const int wsq = overrides().small_ws.load(std::memory_order_relaxed);
        if (grouped && (wsq == 1 || (wsq == 0 && a.n <= 128))) {
            const int ft = overrides().small_tile.load(std::memory_order_relaxed);
            if (launch_ws(a, true, ft >> 4, ft & 15, st)) {
                hip_check(hipGetLastError(), "tgemm_small_ws launch");
                return true;
            }
        }
        if (grouped)
            launch_small<true>(a, p, 8 * per_xcd, n_mt, per_xcd, p.tiles, st);
        else
            launch_small<false>(a, p, 8 * per_xcd, n_mt, per_xcd, p.tiles, st);
        hip_check(hipGetLastError(), "tgemm_small launch");
        return true;
    }
    // group sums only with one group and the Store epilogue (other cases: the kernels of vx_gemm.hip)
    if (a.gs != nullptr && (grouped || a.ep != VX_EP_STORE)) return false;
    if (a.y_bytes == 0 || !a.vec_ok) return false;
    if (a.r0 != 0 || a.r1 != a.out || a.n_base != 0) return false;
    if (grouped ? (a.spg != 2 || a.ng % 4 != 0 || a.ng > kMaxG) : (a.inp / 64) % 4 != 0) return false;
    // a "small" override forces this kernel ("stream" keeps it for the tokens after the streaming kernel's tiles; any
    // other kernel override turns it off); a "small_tile" override forces a tile (tests and tuning)
    const int forced = overrides().gemm.load(std::memory_order_relaxed);
    if (forced != kForceNone && forced != kForceSmall && forced != kForceStream) return false;
    const int ft = overrides().small_tile.load(std::memory_order_relaxed);
    const int fm = ft >> 4, fn = ft & 15;
    // up to 1024 tokens; longer token ranges go to the kernels built for throughput
    if (a.t1 - a.m_base > 1024 && forced != kForceSmall) return false;
    // the producer/consumer kernel by default for 8, 16 or 32 groups: the fold of one chunk overlaps the next
    // chunk's loads and MFMAs (FFN-down, T = 125 / 338 / 750: 11.1 / 11.5 / 18.6 -> 9.2 / 9.3 / 16.9 us; o-proj
    // T = 338 / 750: 4.69 / 6.46 -> 4.44 / 5.85 us; q|k|v T = 338 / 750: 8.08 / 13.09 -> 7.06 / 10.83 us, where the
    // four-wavefront kernel or split-K over groups ran); other group counts keep those kernels
    const int ws = overrides().small_ws.load(std::memory_order_relaxed);
    if (grouped && (ws == 1 || (ws == 0 && !(fm && fn))) && launch_ws(a, false, fm, fn, st)) {
        hip_check(hipGetLastError(), "tgemm_small_ws launch");
        return true;
    }
    const SmallPlan p = plan_small(a, grouped, fm, fn);
    if (p.mt == 0) return false;
    const int64_t ntok = a.t1 - a.m_base;
    const int n_mt = (int)((ntok + 16 * p.mt - 1) / (16 * p.mt));
    const int per_xcd = (p.tiles + 7) / 8;  // grid 8 * per_xcd; workgroups past the last tile return at once
    if (grouped)
        launch_small<true>(a, p, 8 * per_xcd, n_mt, per_xcd, p.tiles, st);
    else
        launch_small<false>(a, p, 8 * per_xcd, n_mt, per_xcd, p.tiles, st);
    hip_check(hipGetLastError(), "tgemm_small launch");
    return true;
}

}  // namespace vx
