// vx_gemm.hip — ternary (or int8) x int8 GEMM on CDNA4 i8 MFMA, bit-exact to voxrt's scalar kernel
// (crates/voxrt/src/kernels/mod.rs:166-210).
//
//   y[t, o] = ep(y_old, acc),  acc = fold over groups g ascending of fma((float)S_g, xs[t, g] * ws[o, g], acc)
//   S_g     = sum_{c in group g} w[o, c] * x[t, c]   (exact int32)
//
// Work decomposition. A workgroup of 4 wavefronts owns a tile of BM = 16*MT tokens x BN = 4*16*NT output rows;
// wavefront w owns the BN/4 rows [16*NT*w, 16*NT*(w+1)) of it and all BM tokens. The K dimension is walked in
// 64-column steps. Each step's operands travel through a register ring D steps deep (loads for step kb + D are
// issued while step kb computes): the BM x 64 int8 activation tile, this wavefront's weight operands (one dword of
// 2-bit codes per lane per 16x64 block) and, on a group's first step, the group's activation scales, activation
// code sums and weight scales. One step ahead of use the activation tile is written to LDS (double buffered,
// XOR-swizzled 16-byte chunks so a 16-lane phase of ds_read_b128 touches 64 distinct banks) and the group's
// scales to a two-slot LDS table; one barrier per step. The weight codes (trit + 1 in {0, 1, 2}) are widened to
// int8 with four shift/and operations and v_mfma_i32_16x16x64_i8 accumulates sum x * (trit + 1) in int32;
// seeding its C operand with -sum(x) of the group (the quantizer's gsum) makes the accumulator exactly S_g at no
// extra instruction. At the end of each group the int32 sums are folded into the fp32 accumulators in the
// reference's operation order (a single group, G = K, skips the fp32 accumulator: acc = fma(S, p, 0)); the
// epilogue applies Store / SiLU / AddScaled (+ bias).
//
// MFMA operand layouts (16x16x64, wave64): lane l supplies row l%16 of A and column l%16 of B over the same 16
// columns of the 64-column step (lane group l/16); D element e of lane l is D[4*(l/16) + e][l%16].
// A = activations (rows = tokens), B = weights (columns = output rows), so a lane's outputs are 4 tokens of one
// output row and 16 consecutive lanes store 64 contiguous bytes of y.
//
// Ragged edges: every read-only operand goes through a raw buffer descriptor whose range ends at the operand's
// size, so loads past the last token (or past the padded weight rows) return zero without branches; stores are
// guarded by the [t0, t1) x [r0, r1) window.
#include <cstring>

#include "vx_gemm.h"

namespace vx {

// int32 group sums of group g to gs[(g*n + t)*out + o] inside the [t0, t1) x [r0, r1) window
template <int MT, int NT>
__device__ inline void store_group_sums(const GemmArgs &a, const v4i (&acc)[MT][NT], int g, int m0, int nw0, int aj,
                                        int arow) {
#pragma unroll
    for (int mb = 0; mb < MT; mb++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int64_t t = m0 + mb * 16 + 4 * aj + e;
            if (t < a.t0 || t >= a.t1) continue;
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                const int64_t o = nw0 + nb * 16 + arow;
                if (o >= a.r0 && o < a.r1) a.gs[((int64_t)g * a.n + t) * a.out + o] = acc[mb][nb][e];
            }
        }
}

// Epilogue (kernels/mod.rs:41-48; the bias is added after it as in gemm_ep, kernels/mod.rs:355-361), one
// 16-token block at a time: the old outputs and the bias are loaded in one batch, then each output in the
// [t0, t1) x [r0, r1) window is written once. A single group folds here: acc = fma(S, xs * ws, 0).
template <int MT, int NT, bool SINGLE, class XS>
__device__ inline void epilogue(const GemmArgs &a, const v4i (&acc)[MT][NT],
                                const float (&accf)[SINGLE ? 1 : MT][SINGLE ? 1 : NT][4], const XS &xsf,
                                const float (&wsf)[SINGLE ? NT : 1], int m0, int nw0, int aj, int arow) {
    float bia[NT];
    const bool add = a.ep == VX_EP_ADD_SCALED;
#pragma unroll
    for (int nb = 0; nb < NT; nb++) {
        const int64_t o = nw0 + nb * 16 + arow;
        bia[nb] = (a.bias && o >= a.r0 && o < a.r1) ? a.bias[o] : 0.0f;
    }
#pragma unroll
    for (int mb = 0; mb < MT; mb++) {
        float old[4][NT];
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                const int64_t t = m0 + mb * 16 + 4 * aj + e, o = nw0 + nb * 16 + arow;
                old[e][nb] = (add && t >= a.t0 && t < a.t1 && o >= a.r0 && o < a.r1) ? a.y[t * a.out + o] : 0.0f;
            }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int64_t t = m0 + mb * 16 + 4 * aj + e;
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                const int64_t o = nw0 + nb * 16 + arow;
                if (t < a.t0 || t >= a.t1 || o < a.r0 || o >= a.r1) continue;
                float v;
                if constexpr (SINGLE)
                    v = __builtin_fmaf((float)acc[mb][nb][e], __int_as_float(xsf[mb][e]) * wsf[nb], 0.0f);
                else
                    v = accf[mb][nb][e];
                float r = ep_apply(a.ep, a.alpha, old[e][nb], v);
                if (a.bias) r = r + bia[nb];
                a.y[t * a.out + o] = r;
            }
        }
    }
}

template <int MT, int NT, bool TERN, bool GS, bool SINGLE, int D>
__global__ __launch_bounds__(256) void tgemm_kernel(const GemmArgs a) {
    constexpr int BM = MT * 16;
    constexpr int BN = NT * 16 * 4;
    constexpr int ACH = (BM * 4 + 255) / 256;  // 16-byte activation chunks per thread per stage
    constexpr int SW = 2 * BM + BN;            // scale words of one group: xs[BM], gsum[BM], ws[BN]
    __shared__ __attribute__((aligned(16))) int8_t lds_a[2][BM * 64];
    __shared__ float lds_s[2][SW];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int arow = lane & 15, aj = lane >> 4;
    // 32-bit index arithmetic: the host guarantees every operand is below 4 GiB
    const int m0 = (int)a.m_base + (int)blockIdx.y * BM;
    const int nblk0 = (int)a.n_base + (int)blockIdx.x * BN;
    const int nw0 = nblk0 + wave * NT * 16;
    const int nk = (int)(a.inp / 64), inp = (int)a.inp, ng = (int)a.ng, spg = (int)a.spg, np = (int)a.np;
    const int out_pad = (int)a.out_pad;

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    // the scale operand of this wavefront's role (see issue): activation scales, code sums or weight scales
    const auto rsrc = make_rsrc(wave == 0 ? (const void *)a.xs : (wave == 1 ? (const void *)a.xg : (const void *)a.ws_t),
                                wave < 2 ? a.xs_bytes : a.ws_bytes);

    // Register ring of D stages in flight: stage kb = the 64-column step kb of the activation tile, the weight
    // operands of this wavefront and, on the first step of a group, that group's scales and code sums. Loads are
    // issued D steps before use and consumed in issue order, so the in-order vmcnt wait only ever waits for the
    // oldest stage.
    typedef typename std::conditional<TERN, uint32_t, v4i>::type BReg;
    v4i ra[D][ACH];
    BReg rb[D][NT];
    uint32_t rs[SINGLE ? 1 : D][2];

    // (group, step within the group) of a stage, advanced by counting instead of dividing
    struct Pos {
        int g, s;
    };
    auto advance = [&](Pos p) {
        p.s++;
        if (p.s == spg) {
            p.s = 0;
            p.g++;
        }
        return p;
    };

    // Every lane issues the same loads on every step (a load that is not wanted gets an offset past the end of
    // its buffer and returns zero without touching memory): with a fixed load count per step the compiler's
    // in-order vmcnt waits can name exactly the stage that is consumed instead of draining the whole ring.
    constexpr uint32_t kOff = 0xFFFFFFF0u;
    auto scale_off = [&](int j, int g) {
        uint32_t off = kOff;
        if (wave < 2) {
            if (j == 0 && lane < BM && (wave == 0 || TERN)) off = (uint32_t)((g * np + m0 + lane) * 4);
        } else {
            const int c = (wave - 2) * (BN / 2) + j * 64 + lane;
            if (j * 64 + lane < BN / 2) off = (uint32_t)((g * out_pad + nblk0 + c) * 4);
        }
        return off;
    };
    auto issue = [&](int kb, Pos p, int slot) {
        const bool live = kb < nk;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = tid + i * 256;
            const uint32_t off = (uint32_t)((m0 + (c >> 2)) * inp + kb * 64 + (c & 3) * 16);
            ra[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, live && c < BM * 4 ? off : kOff, 0, 0);
        }
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            const uint32_t blk = (uint32_t)((nw0 / 16 + nb) * nk + kb);
            if constexpr (TERN)
                rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, live ? (blk * 64 + lane) * 4 : kOff, 0, 0);
            else
                rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b128(wrs, live ? (blk * 64 + lane) * 16 : kOff, 0, 0);
        }
        // scale words of the group, one role per wavefront (so the buffer descriptor stays uniform): wave 0 the
        // activation scales of the BM tokens, wave 1 their code sums, waves 2 and 3 one half each of the BN
        // weight scales; every wavefront issues the same two loads (a single group loads them once, in the
        // prologue, outside the ring)
        if constexpr (!SINGLE) {
            const bool gl = live && p.s == 0;
#pragma unroll
            for (int j = 0; j < 2; j++)
                rs[slot][j] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, gl ? scale_off(j, p.g) : kOff, 0, 0);
        }
    };

    // ring slot -> LDS: the activation tile (XOR-swizzled 16-byte chunks) and, on a group start, the scales
    auto store = [&](int slot, int kb, Pos p) {
        const int buf = kb & 1;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = tid + i * 256;
            if (c < BM * 4) {
                const int row = c >> 2, ch = (c & 3) ^ ((row >> 2) & 3);
                *(v4i *)&lds_a[buf][row * 64 + ch * 16] = ra[slot][i];
            }
        }
        if (p.s == 0) {
            float *dst = lds_s[p.g & 1];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float v = __builtin_bit_cast(float, rs[SINGLE ? 0 : slot][j]);
                if (wave < 2) {
                    if (j == 0 && lane < BM) dst[wave * BM + lane] = v;
                } else if (j * 64 + lane < BN / 2) {
                    dst[2 * BM + (wave - 2) * (BN / 2) + j * 64 + lane] = v;
                }
            }
        }
    };

    v4i acc[MT][NT];
    float accf[SINGLE ? 1 : MT][SINGLE ? 1 : NT][4];  // fp32 accumulators (a single group folds in the epilogue)
    if constexpr (!SINGLE) {
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int nb = 0; nb < NT; nb++)
#pragma unroll
                for (int e = 0; e < 4; e++) accf[mb][nb][e] = 0.0f;
    }

    // fold group g into the fp32 accumulators: acc_f = fma((float)S_g, xs[t][g] * ws[o][g], acc_f)
    auto fold = [&](int g) {
        const float *sx = lds_s[g & 1];
        float xsv[MT][4], wsv[NT];
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int e = 0; e < 4; e++) xsv[mb][e] = sx[mb * 16 + 4 * aj + e];
#pragma unroll
        for (int nb = 0; nb < NT; nb++) wsv[nb] = sx[2 * BM + wave * NT * 16 + nb * 16 + arow];
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int nb = 0; nb < NT; nb++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float p = xsv[mb][e] * wsv[nb];
                    if constexpr (!SINGLE) accf[mb][nb][e] = __builtin_fmaf((float)acc[mb][nb][e], p, accf[mb][nb][e]);
                }
        if constexpr (GS) store_group_sums<MT, NT>(a, acc, g, m0, nw0, aj, arow);
    };

    auto compute = [&](int kb, Pos p, int slot) {
        const int buf = kb & 1;
        v4i av[MT], bv[NT];
#pragma unroll
        for (int mb = 0; mb < MT; mb++) {
            const int row = mb * 16 + arow, ch = aj ^ ((row >> 2) & 3);
            av[mb] = *(const v4i *)&lds_a[buf][row * 64 + ch * 16];
        }
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            if constexpr (TERN)
                bv[nb] = widen_codes(rb[slot][nb]);
            else
                bv[nb] = rb[slot][nb];
        }
        if (p.s == 0) {
            // seed C with -sum(x) of the group (ternary codes are trit + 1), so the accumulator ends at S_g
            const float *sx = lds_s[p.g & 1];
            v4i cinit[MT];
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    cinit[mb][e] = TERN ? -__builtin_bit_cast(int, sx[BM + mb * 16 + 4 * aj + e]) : 0;
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mb], bv[nb], cinit[mb], 0, 0, 0);
        } else {
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mb], bv[nb], acc[mb][nb], 0, 0, 0);
        }
        if (!SINGLE && p.s == spg - 1) fold(p.g);
    };

    // D divides nk (the host picks it), so every unrolled step below is a real one
    Pos pc = {0, 0}, ps = {0, 0}, pi = {0, 0};
    if constexpr (SINGLE) {
#pragma unroll
        for (int j = 0; j < 2; j++) rs[0][j] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, scale_off(j, 0), 0, 0);
    }
#pragma unroll
    for (int i = 0; i < D; i++) {
        issue(i, pi, i);
        pi = advance(pi);
    }
    store(0, 0, ps);
    ps = advance(ps);
    __syncthreads();
    for (int kb0 = 0; kb0 < nk; kb0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            const int kb = kb0 + i;
            compute(kb, pc, i);
            pc = advance(pc);
            if (kb + 1 < nk) store((i + 1) % D, kb + 1, ps);
            ps = advance(ps);
            issue(kb + D, pi, i);
            pi = advance(pi);
            __syncthreads();
        }
    }
    // a single group folds in the epilogue with the scales staged in LDS slot 0
    v4i xsf[MT];
    float wsf[SINGLE ? NT : 1];
    if constexpr (SINGLE) {
        const float *sx = lds_s[0];
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int e = 0; e < 4; e++) xsf[mb][e] = __builtin_bit_cast(int, sx[mb * 16 + 4 * aj + e]);
#pragma unroll
        for (int nb = 0; nb < NT; nb++) wsf[SINGLE ? nb : 0] = sx[2 * BM + wave * NT * 16 + nb * 16 + arow];
        if constexpr (GS) store_group_sums<MT, NT>(a, acc, 0, m0, nw0, aj, arow);
    }
    epilogue<MT, NT, SINGLE>(a, acc, accf, xsf, wsf, m0, nw0, aj, arow);
}

// ---------------------------------------------------------------------------------------------------------------
// Direct kernel: every wavefront owns a 16*MT x 16*NT output tile and streams its own operands from memory into
// registers (the four wavefronts of a workgroup share their activation rows through the L1 cache). There is no
// LDS staging and no barrier in the K loop, so a wavefront's only wait is for the data of the stage it consumes:
// the register ring keeps D stages of KS 64-column steps in flight, up to the whole K for the small-token shapes
// where the kernel is bound by memory latency rather than by MFMA or HBM throughput. A stage is one quantization
// group (KS = group / 64) and carries the group's activation scales and code sums for the lane's 4 tokens
// (16-byte loads from the transposed [ng][np] layout) and the weight scales of its NT rows; a single group
// (G = K) loads its code sums once before the loop and its scales once after it.
template <int MT, int NT, bool TERN, bool GS, bool SINGLE, int KS, int D>
__global__ __launch_bounds__(256) void tgemm_direct_kernel(const GemmArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int arow = lane & 15, aj = lane >> 4;
    const int m0 = (int)a.m_base + (int)blockIdx.y * (MT * 16);
    const int nw0 = (int)a.n_base + (int)blockIdx.x * (NT * 64) + wave * NT * 16;
    const int inp = (int)a.inp, nk = inp / 64, nst = nk / KS, np = (int)a.np, out_pad = (int)a.out_pad;

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto grs = make_rsrc(a.xg, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);

    typedef typename std::conditional<TERN, uint32_t, v4i>::type BReg;
    constexpr int SD = SINGLE ? 1 : D;  // per-stage scale registers exist only for multi-group GEMMs
    v4i ra[D][KS][MT];
    BReg rb[D][KS][NT];
    v4i rx[SD][MT], rg[SD][MT];  // activation scales / code sums of the lane's 4 tokens per 16-token block
    float rw[SD][NT];            // weight scale of the lane's output row per 16-row block

    constexpr uint32_t kOff = 0xFFFFFFF0u;
    // token offset of the lane's 4 scale entries of block mb in the [ng][np] tables
    auto tok4 = [&](int mb) { return m0 + mb * 16 + 4 * aj; };
    auto issue = [&](int s, int slot) {
        const bool live = s < nst;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int kb = s * KS + ks;
#pragma unroll
            for (int mb = 0; mb < MT; mb++) {
                const uint32_t off = (uint32_t)((m0 + mb * 16 + arow) * inp + kb * 64 + 16 * aj);
                ra[slot][ks][mb] = __builtin_amdgcn_raw_buffer_load_b128(xrs, live ? off : kOff, 0, 0);
            }
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                const uint32_t blk = (uint32_t)((nw0 / 16 + nb) * nk + kb);
                if constexpr (TERN)
                    rb[slot][ks][nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, live ? (blk * 64 + lane) * 4 : kOff,
                                                                            0, 0);
                else
                    rb[slot][ks][nb] = __builtin_amdgcn_raw_buffer_load_b128(
                        wrs, live ? (blk * 64 + lane) * 16 : kOff, 0, 0);
            }
        }
        if constexpr (!SINGLE) {
            const int g = s;  // one group per stage
#pragma unroll
            for (int mb = 0; mb < MT; mb++) {
                const uint32_t off = (uint32_t)((g * np + tok4(mb)) * 4);
                rx[slot][mb] = __builtin_amdgcn_raw_buffer_load_b128(srs, live ? off : kOff, 0, 0);
                if constexpr (TERN) rg[slot][mb] = __builtin_amdgcn_raw_buffer_load_b128(grs, live ? off : kOff, 0, 0);
            }
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                const uint32_t off = (uint32_t)((g * out_pad + nw0 + nb * 16 + arow) * 4);
                rw[slot][nb] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wsrs, live ? off : kOff, 0, 0));
            }
        }
    };

    v4i acc[MT][NT];
    float accf[SINGLE ? 1 : MT][SINGLE ? 1 : NT][4];
    if constexpr (!SINGLE) {
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int nb = 0; nb < NT; nb++)
#pragma unroll
                for (int e = 0; e < 4; e++) accf[mb][nb][e] = 0.0f;
    }

    // single group: the code sums seed the accumulators once (loaded before the ring, so they are the oldest)
    v4i g0[SINGLE ? MT : 1];
    if constexpr (SINGLE) {
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
            g0[mb] = TERN ? __builtin_amdgcn_raw_buffer_load_b128(grs, (uint32_t)(tok4(mb) * 4), 0, 0) : v4i{0, 0, 0, 0};
    }

    auto compute = [&](int s, int slot) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            v4i bv[NT];
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                if constexpr (TERN)
                    bv[nb] = widen_codes(rb[slot][ks][nb]);
                else
                    bv[nb] = rb[slot][ks][nb];
            }
            const bool first = ks == 0 && (!SINGLE || s == 0);
            if (first) {
                // seed C with -sum(x) of the group (ternary codes are trit + 1), so the accumulator ends at S_g
#pragma unroll
                for (int mb = 0; mb < MT; mb++) {
                    const v4i gsum = SINGLE ? g0[SINGLE ? mb : 0] : rg[SINGLE ? 0 : slot][mb];
                    const v4i cinit = TERN ? -gsum : v4i{0, 0, 0, 0};
#pragma unroll
                    for (int nb = 0; nb < NT; nb++)
                        acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ra[slot][ks][mb], bv[nb], cinit, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int mb = 0; mb < MT; mb++)
#pragma unroll
                    for (int nb = 0; nb < NT; nb++)
                        acc[mb][nb] =
                            __builtin_amdgcn_mfma_i32_16x16x64_i8(ra[slot][ks][mb], bv[nb], acc[mb][nb], 0, 0, 0);
            }
        }
        if constexpr (!SINGLE) {
            // fold group s: acc_f = fma((float)S_g, xs[t][g] * ws[o][g], acc_f)
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float p = __int_as_float(rx[slot][mb][e]) * rw[slot][nb];
                        accf[mb][nb][e] = __builtin_fmaf((float)acc[mb][nb][e], p, accf[mb][nb][e]);
                    }
            if constexpr (GS) store_group_sums<MT, NT>(a, acc, s, m0, nw0, aj, arow);
        }
    };

#pragma unroll
    for (int i = 0; i < D; i++) issue(i, i);
    for (int s0 = 0; s0 < nst; s0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            const int s = s0 + i;
            if (s < nst) compute(s, i);
            issue(s + D, i);
        }
    }

    // single group: its scales, loaded after the loop
    v4i xsf[SINGLE ? MT : 1];
    float wsf[SINGLE ? NT : 1];
    if constexpr (SINGLE) {
#pragma unroll
        for (int mb = 0; mb < MT; mb++) xsf[mb] = __builtin_amdgcn_raw_buffer_load_b128(srs, (uint32_t)(tok4(mb) * 4), 0, 0);
#pragma unroll
        for (int nb = 0; nb < NT; nb++)
            wsf[nb] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                    wsrs, (uint32_t)((nw0 + nb * 16 + arow) * 4), 0, 0));
        if constexpr (GS) store_group_sums<MT, NT>(a, acc, 0, m0, nw0, aj, arow);
    }
    epilogue<MT, NT, SINGLE>(a, acc, accf, xsf, wsf, m0, nw0, aj, arow);
}


// ---------------------------------------------------------------------------------------------------------------
// Split-K kernel (one group, G = K; the small-token shapes). The four wavefronts of a workgroup share one
// 16*MT x 16*NT output tile and each walks a quarter of the K steps with up to all of its stages in flight (a
// register ring D stages deep; the per-step offsets travel in scalar registers, so a step costs no vector address
// arithmetic, and the loop is peeled so that no load is conditional). Their int32 partial sums meet in LDS, where
// the sum is exact in any order (wave 0 seeds its MFMA chain with -sum(x) of the tokens, the others with zero).
// Then each thread owns 8 consecutive outputs of one token: S -> acc = fma(S, xs * ws, 0), the epilogue, and two
// 16-byte stores.
template <int MT, int NT, bool TERN, bool GS, int D>
__global__ __launch_bounds__(256) void tgemm_splitk_kernel(const GemmArgs a) {
    constexpr int BM = 16 * MT, BN = 16 * NT, BNP = BN + 4;  // BNP: LDS row pitch (bank-conflict-free writes)
    static_assert(BM * BN == 256 * 8, "each thread folds 8 outputs");
    __shared__ __attribute__((aligned(16))) int red[4][BM * BNP];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int arow = lane & 15, aj = lane >> 4;
    const int m0 = (int)a.m_base + (int)blockIdx.y * BM;
    const int n0 = (int)a.n_base + (int)blockIdx.x * BN;
    const int inp = (int)a.inp, nk = inp / 64, nkw = nk / 4, kb0 = wave * nkw;

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto grs = make_rsrc(a.xg, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);

    // lane-constant offsets; a token past n lands past the end of xq and reads zeros
    int va[MT];
#pragma unroll
    for (int mb = 0; mb < MT; mb++) va[mb] = (m0 + mb * 16 + arow) * inp + 16 * aj;
    constexpr int BBYTES = TERN ? 4 : 16;  // weight operand bytes per lane per 16x64 block
    const int vb = lane * BBYTES;

    typedef typename std::conditional<TERN, uint32_t, v4i>::type BReg;
    v4i ra[D][MT];
    BReg rb[D][NT];
    auto issue = [&](int kb, int slot) {
#pragma unroll
        for (int mb = 0; mb < MT; mb++) ra[slot][mb] = __builtin_amdgcn_raw_buffer_load_b128(xrs, va[mb], kb * 64, 0);
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            const int soff = ((n0 / 16 + nb) * nk + kb) * 64 * BBYTES;
            if constexpr (TERN)
                rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, vb, soff, 0);
            else
                rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b128(wrs, vb, soff, 0);
        }
    };

    // wave 0 seeds its chain with -gsum of the lane's 4 tokens per block; the other waves with zero
    v4i cinit[MT];
#pragma unroll
    for (int mb = 0; mb < MT; mb++) {
        cinit[mb] = v4i{0, 0, 0, 0};
        if (TERN && wave == 0)
            cinit[mb] = -(v4i)__builtin_amdgcn_raw_buffer_load_b128(grs, (m0 + mb * 16 + 4 * aj) * 4, 0, 0);
    }

    v4i acc[MT][NT];
    auto compute = [&](int slot, bool first) {
        v4i bv[NT];
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            if constexpr (TERN)
                bv[nb] = widen_codes(rb[slot][nb]);
            else
                bv[nb] = rb[slot][nb];
        }
        if (first) {
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ra[slot][mb], bv[nb], cinit[mb], 0, 0, 0);
        } else {
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ra[slot][mb], bv[nb], acc[mb][nb], 0, 0, 0);
        }
    };

    // D divides nkw (the host picks it): prologue, steady state, drain
#pragma unroll
    for (int i = 0; i < D; i++) issue(kb0 + i, i);
    for (int s0 = 0; s0 < nkw - D; s0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            compute(i, s0 + i == 0);
            issue(kb0 + s0 + i + D, i);
        }
    }
#pragma unroll
    for (int i = 0; i < D; i++) compute(i, nkw - D + i == 0);

    // partial sums -> LDS
#pragma unroll
    for (int mb = 0; mb < MT; mb++)
#pragma unroll
        for (int nb = 0; nb < NT; nb++)
#pragma unroll
            for (int e = 0; e < 4; e++) red[wave][(mb * 16 + 4 * aj + e) * BNP + nb * 16 + arow] = acc[mb][nb][e];
    __syncthreads();

    // thread -> token tt of the tile, rows c0 .. c0+7
    const int tt = tid / (BN / 8), c0 = (tid % (BN / 8)) * 8;
    int S[8];
#pragma unroll
    for (int j = 0; j < 8; j++) S[j] = 0;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const v4i lo = *(const v4i *)&red[w][tt * BNP + c0];
        const v4i hi = *(const v4i *)&red[w][tt * BNP + c0 + 4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            S[j] += lo[j];
            S[4 + j] += hi[j];
        }
    }
    const int t = m0 + tt, o0 = n0 + c0;
    if (t < a.t0 || t >= a.t1) return;
    const float xs = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, t * 4, 0, 0));
    const v4i wlo = __builtin_amdgcn_raw_buffer_load_b128(wsrs, o0 * 4, 0, 0);
    const v4i whi = __builtin_amdgcn_raw_buffer_load_b128(wsrs, o0 * 4 + 16, 0, 0);
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v[j] = __builtin_fmaf((float)S[j], xs * __int_as_float(wlo[j]), 0.0f);
        v[4 + j] = __builtin_fmaf((float)S[4 + j], xs * __int_as_float(whi[j]), 0.0f);
    }
    float *yrow = a.y + (int64_t)t * a.out;
    if (a.vec_ok && o0 >= a.r0 && o0 + 8 <= a.r1) {
        float old[8] = {0, 0, 0, 0, 0, 0, 0, 0}, bia[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (a.ep == VX_EP_ADD_SCALED) {
            const float4 p = *(const float4 *)(yrow + o0), q = *(const float4 *)(yrow + o0 + 4);
            old[0] = p.x, old[1] = p.y, old[2] = p.z, old[3] = p.w, old[4] = q.x, old[5] = q.y, old[6] = q.z,
            old[7] = q.w;
        }
        if (a.bias) {
            const float4 p = *(const float4 *)(a.bias + o0), q = *(const float4 *)(a.bias + o0 + 4);
            bia[0] = p.x, bia[1] = p.y, bia[2] = p.z, bia[3] = p.w, bia[4] = q.x, bia[5] = q.y, bia[6] = q.z,
            bia[7] = q.w;
        }
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            r[j] = ep_apply(a.ep, a.alpha, old[j], v[j]);
            if (a.bias) r[j] = r[j] + bia[j];
        }
        store16_sep((float4 *)(yrow + o0), make_float4(r[0], r[1], r[2], r[3]));
        store16_sep((float4 *)(yrow + o0 + 4), make_float4(r[4], r[5], r[6], r[7]));
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int o = o0 + j;
            if (o < a.r0 || o >= a.r1) continue;
            float r = ep_apply(a.ep, a.alpha, a.ep == VX_EP_ADD_SCALED ? yrow[o] : 0.0f, v[j]);
            if (a.bias) r = r + a.bias[o];
            yrow[o] = r;
        }
    }
    if constexpr (GS) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int o = o0 + j;
            if (o >= a.r0 && o < a.r1) a.gs[(int64_t)t * a.out + o] = S[j];
        }
    }
}


// Split-K over groups (several groups, G = 64 * SPG): chunk c of the K dimension holds groups 4c .. 4c+3 and wave w
// computes group 4c + w, its MFMA chain seeded with the group's -sum(x codes) so it ends at S_g. After every chunk
// the four group sums of each output meet in LDS and are folded in ascending group order into the fp32
// accumulators, acc = fma((float)S_g, xs[t][g] * ws[o][g], acc) — the reference's fold, so the result is the
// scalar kernel's bit for bit. Small-M shapes get 4x the wavefronts of the one-wave-per-tile kernels this way.
template <int MT, int NT, bool TERN, bool GS, int SPG, int D>
__global__ __launch_bounds__(256) void tgemm_splitk_groups_kernel(const GemmArgs a) {
    constexpr int BM = 16 * MT, BN = 16 * NT, BNP = BN + 4;
    static_assert(BM * BN == 256 * 8, "each thread folds 8 outputs");
    static_assert(D % SPG == 0, "the ring depth covers whole groups");
    __shared__ __attribute__((aligned(16))) int red[4][BM * BNP];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int arow = lane & 15, aj = lane >> 4;
    const int m0 = (int)a.m_base + (int)blockIdx.y * BM;
    const int n0 = (int)a.n_base + (int)blockIdx.x * BN;
    const int inp = (int)a.inp, nk = inp / 64, ng = (int)a.ng, nchunk = ng / 4, nsw = nchunk * SPG;
    const int np = (int)a.np;

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto grs = make_rsrc(a.xg, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);

    int va[MT];
#pragma unroll
    for (int mb = 0; mb < MT; mb++) va[mb] = (m0 + mb * 16 + arow) * inp + 16 * aj;
    constexpr int BBYTES = TERN ? 4 : 16;
    const int vb = lane * BBYTES;

    typedef typename std::conditional<TERN, uint32_t, v4i>::type BReg;
    v4i ra[D][MT];
    BReg rb[D][NT];
    // this wave's k-step s lies in chunk s / SPG: global step ((s / SPG) * 4 + wave) * SPG + s % SPG
    auto kb_of = [&](int st) { return ((st / SPG) * 4 + wave) * SPG + st % SPG; };
    auto issue = [&](int st, int slot) {
        const int kb = kb_of(st);
#pragma unroll
        for (int mb = 0; mb < MT; mb++) ra[slot][mb] = __builtin_amdgcn_raw_buffer_load_b128(xrs, va[mb], kb * 64, 0);
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            const int soff = ((n0 / 16 + nb) * nk + kb) * 64 * BBYTES;
            if constexpr (TERN)
                rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, vb, soff, 0);
            else
                rb[slot][nb] = __builtin_amdgcn_raw_buffer_load_b128(wrs, vb, soff, 0);
        }
    };

    // fold state: thread -> token tt of the tile, rows c0 .. c0+7
    const int tt = tid / (BN / 8), c0 = (tid % (BN / 8)) * 8;
    const int t = m0 + tt, o0 = n0 + c0;
    float accf[8];
#pragma unroll
    for (int j = 0; j < 8; j++) accf[j] = 0.0f;

    v4i acc[MT][NT];
    auto compute = [&](int slot, int st) {
        v4i bv[NT];
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            if constexpr (TERN)
                bv[nb] = widen_codes(rb[slot][nb]);
            else
                bv[nb] = rb[slot][nb];
        }
        if (st % SPG == 0) {  // first step of a group: seed with -gsum of the group (ternary) or zero
            const int g = (st / SPG) * 4 + wave;
#pragma unroll
            for (int mb = 0; mb < MT; mb++) {
                v4i c = v4i{0, 0, 0, 0};
                if constexpr (TERN)
                    c = -(v4i)__builtin_amdgcn_raw_buffer_load_b128(grs, (g * np + m0 + mb * 16 + 4 * aj) * 4, 0, 0);
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ra[slot][mb], bv[nb], c, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ra[slot][mb], bv[nb], acc[mb][nb], 0, 0, 0);
        }
        if (st % SPG == SPG - 1) {  // group complete: the chunk's four group sums meet in LDS, then the fold
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int nb = 0; nb < NT; nb++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        red[wave][(mb * 16 + 4 * aj + e) * BNP + nb * 16 + arow] = acc[mb][nb][e];
            __syncthreads();
            const int chunk = st / SPG;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const int g = chunk * 4 + w;
                const v4i lo = *(const v4i *)&red[w][tt * BNP + c0];
                const v4i hi = *(const v4i *)&red[w][tt * BNP + c0 + 4];
                const float xs = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, (g * np + t) * 4, 0, 0));
                const v4i wlo = __builtin_amdgcn_raw_buffer_load_b128(wsrs, (g * (int)a.out_pad + o0) * 4, 0, 0);
                const v4i whi = __builtin_amdgcn_raw_buffer_load_b128(wsrs, (g * (int)a.out_pad + o0) * 4 + 16, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    accf[j] = __builtin_fmaf((float)lo[j], xs * __int_as_float(wlo[j]), accf[j]);
                    accf[4 + j] = __builtin_fmaf((float)hi[j], xs * __int_as_float(whi[j]), accf[4 + j]);
                }
                if constexpr (GS) {
                    if (t >= a.t0 && t < a.t1)
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const int o = o0 + j;
                            if (o >= a.r0 && o < a.r1) a.gs[((int64_t)g * a.n + t) * a.out + o] = j < 4 ? lo[j] : hi[j - 4];
                        }
                }
            }
            __syncthreads();
        }
    };

    // D divides nsw and is a multiple of SPG (the host picks it): prologue, steady state, drain
#pragma unroll
    for (int i = 0; i < D; i++) issue(i, i);
    for (int s0 = 0; s0 < nsw - D; s0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            compute(i, s0 + i);
            issue(s0 + i + D, i);
        }
    }
#pragma unroll
    for (int i = 0; i < D; i++) compute(i, nsw - D + i);

    if (t < a.t0 || t >= a.t1) return;
    const float *v = accf;
    float *yrow = a.y + (int64_t)t * a.out;
    if (a.vec_ok && o0 >= a.r0 && o0 + 8 <= a.r1) {
        float old[8] = {0, 0, 0, 0, 0, 0, 0, 0}, bia[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (a.ep == VX_EP_ADD_SCALED) {
            const float4 p = *(const float4 *)(yrow + o0), q = *(const float4 *)(yrow + o0 + 4);
            old[0] = p.x, old[1] = p.y, old[2] = p.z, old[3] = p.w, old[4] = q.x, old[5] = q.y, old[6] = q.z,
            old[7] = q.w;
        }
        if (a.bias) {
            const float4 p = *(const float4 *)(a.bias + o0), q = *(const float4 *)(a.bias + o0 + 4);
            bia[0] = p.x, bia[1] = p.y, bia[2] = p.z, bia[3] = p.w, bia[4] = q.x, bia[5] = q.y, bia[6] = q.z,
            bia[7] = q.w;
        }
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            r[j] = ep_apply(a.ep, a.alpha, old[j], v[j]);
            if (a.bias) r[j] = r[j] + bia[j];
        }
        store16_sep((float4 *)(yrow + o0), make_float4(r[0], r[1], r[2], r[3]));
        store16_sep((float4 *)(yrow + o0 + 4), make_float4(r[4], r[5], r[6], r[7]));
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int o = o0 + j;
            if (o < a.r0 || o >= a.r1) continue;
            float r = ep_apply(a.ep, a.alpha, a.ep == VX_EP_ADD_SCALED ? yrow[o] : 0.0f, v[j]);
            if (a.bias) r = r + a.bias[o];
            yrow[o] = r;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Large-token kernel (one group, G = K; K a multiple of 512). Built for MFMA throughput:
//  * v_mfma_i32_32x32x32_i8: a wavefront owns a 128 x 64 output tile (4 x 2 blocks of 32 x 32, 128 int32
//    accumulators); D element v of lane l is row (v/4)*8 + (l/32)*4 + v%4, column l%32 of its block.
//  * the workgroup's 128 x 64 activation tile of each K step reaches LDS by buffer_load ... lds (no registers),
//    16 rows x 64 contiguous bytes per instruction, in a chunk-swizzled row layout that keeps the fragment reads
//    free of bank conflicts. Four LDS slots: steps kb+1 .. kb+3 are in flight while kb computes, and the
//    fragments of kb+1 are read while the MFMAs of kb run.
//  * each wavefront gathers its weight codes (one dword per lane per 32 x 32 block half) from the 16-row block
//    layout into a 4-deep register ring; all per-step offsets are scalar.
//  * one explicit vmcnt wait and one barrier per step; the loads of a step are issued in a fixed order, so the
//    wait count is a constant (10: the B loads of step kb-2+4 and the 6 loads of step kb-1 may be pending).
//  * the accumulators start at -sum(x codes) of their token, so they end at S; the fold fma(S, xs * ws, 0) and
//    the epilogue are specialised on the epilogue kind and the bias, with buffer stores for whole tiles.
template <int EP, bool BIAS>
__global__ __launch_bounds__(256, 2) void tgemm_big_kernel(const GemmArgs a) {
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ __attribute__((aligned(1024))) int8_t sa0[8192];
    __shared__ __attribute__((aligned(1024))) int8_t sa1[8192];
    __shared__ __attribute__((aligned(1024))) int8_t sa2[8192];
    __shared__ __attribute__((aligned(1024))) int8_t sa3[8192];
    auto slot = [&](int i) -> int8_t * { return i == 0 ? sa0 : i == 1 ? sa1 : i == 2 ? sa2 : sa3; };

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, lh = lane >> 5;
    const int m0 = (int)a.m_base + (int)blockIdx.y * 128;
    const int nw0 = (int)a.n_base + (int)blockIdx.x * 256 + wave * 64;
    const int inp = (int)a.inp, nk = inp / 64;
    constexpr uint32_t kOff = 0xFFFFFFF0u;

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);

    // Activation tile of a step in LDS: 8 blocks of 16 token rows x 64 bytes; row i of a block holds its four
    // 16-byte chunks c at position c ^ swz(i), swz(i) = ((i >> 1) ^ (i >> 2)) & 3, so that the fragment reads
    // below (32 rows, one chunk each) hit distinct banks for every 8 (and every 16) consecutive lanes. One DMA
    // instruction fills one block (lane l -> row l/4, position l%4), i.e. 16 rows x 64 contiguous bytes: this wave
    // moves blocks 2*wave and 2*wave+1.
    uint32_t vdma[2];
    {
        const int i = lane >> 2, c = (lane & 3) ^ (((i >> 1) ^ (i >> 2)) & 3);
#pragma unroll
        for (int q = 0; q < 2; q++) vdma[q] = (uint32_t)((m0 + (2 * wave + q) * 16 + i) * inp + c * 16);
    }
    // fragment reads: lane l takes row 32*rb + l%32 (block 2*rb + (l%32)/16, row l%16), chunk 2*kh + l/32
    uint32_t vfr[2];
    {
        const int i = lane & 15, sw = ((i >> 1) ^ (i >> 2)) & 3;
#pragma unroll
        for (int kh = 0; kh < 2; kh++) vfr[kh] = (uint32_t)((l32 >> 4) * 1024 + i * 64 + 16 * ((2 * kh + lh) ^ sw));
    }
    // weight gather: block half (cb, kh) of lane l = row nw0 + 32cb + l%32, columns 32kh + 16*(l/32) .. +15,
    // i.e. 16-row block (nw0 + 32cb)/16 + (l%32)/16, lane' = 16*(2kh + l/32) + l%16 of the 16x64 layout
    constexpr int BB = 4;  // bytes of weight codes per lane per 16 x 64 block
    uint32_t vb[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            const int nb16 = (nw0 + 32 * cb) / 16 + (l32 >> 4);
            vb[cb][kh] = (uint32_t)((nb16 * nk * 64 + 16 * (2 * kh + lh) + (lane & 15)) * BB);
        }

    uint32_t rb[4][2][2];
    // `live` is a compile-time constant at every call: loads past the last step keep the issue order (and so
    // the constant wait count) with an out-of-range offset, which reads zeros and touches no memory
    auto dma = [&](int kb, int sl, bool live) {
#pragma unroll
        for (int q = 0; q < 2; q++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_void *)(slot(sl) + (2 * wave + q) * 1024), 16,
                                                     live ? vdma[q] : kOff, kb * 64, 0, 0);
    };
    auto bload = [&](int kb, int ring, bool live) {
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int kh = 0; kh < 2; kh++)
                rb[ring][cb][kh] = __builtin_amdgcn_raw_buffer_load_b32(wrs, live ? vb[cb][kh] : kOff, kb * 64 * BB, 0);
    };
    // fragments of one step: [khalf][rowblock]
    v4i fr[2][2][4];
    auto read_frags = [&](int sl, int set) {
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int r = 0; r < 4; r++) fr[set][kh][r] = *(const v4i *)(slot(sl) + vfr[kh] + r * 2048);
    };
    // accumulators seeded with -sum(x codes) of their token (codes are trit + 1), so they end at S
    typedef int v16i __attribute__((ext_vector_type(16)));
    v16i acc[4][2];
    {
        const auto grs = make_rsrc(a.xg, a.xs_bytes);
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int vq = 0; vq < 4; vq++) {
                const v4i g4 = __builtin_amdgcn_raw_buffer_load_b128(grs, (uint32_t)((m0 + r * 32 + vq * 8 + lh * 4) * 4), 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[r][0][vq * 4 + e] = acc[r][1][vq * 4 + e] = -g4[e];
            }
    }

    // Per wave the loads are issued as  bload(0) dma(0) bload(1) dma(1) ... dma(j) bload(j+1) ...; at the top of
    // step kb the activation DMA of step kb+1 is complete once at most bload(kb+2), dma(kb+2), bload(kb+3) (10
    // loads) are outstanding.
    constexpr int kWait = 10 | (7 << 4) | (15 << 8);  // vmcnt(10); expcnt, lgkmcnt not waited
    constexpr int kWait0 = 16 | (7 << 4) | (15 << 8);  // vmcnt(16): dma(0) complete in the prologue
    auto step = [&](int kb, int i, bool dma_live, bool b_live, bool next) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kWait);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        dma(kb + 3, (i + 3) & 3, dma_live);
        if (next) read_frags((i + 1) & 3, (i + 1) & 1);
        // keep the fragment reads of step kb+1 ahead of the MFMAs of step kb (two fragment sets live)
        __builtin_amdgcn_sched_barrier(0);
        v4i bv[2][2];
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int kh = 0; kh < 2; kh++) bv[cb][kh] = widen_codes(rb[i][cb][kh]);
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int cb = 0; cb < 2; cb++)
                    acc[r][cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fr[i & 1][kh][r], bv[cb][kh], acc[r][cb], 0, 0,
                                                                        0);
        __builtin_amdgcn_sched_barrier(0);
        bload(kb + 4, i, b_live);
        __builtin_amdgcn_sched_barrier(0);
    };

    bload(0, 0, true);
    dma(0, 0, true);
    bload(1, 1, true);
    dma(1, 1, true);
    bload(2, 2, true);
    dma(2, 2, true);
    bload(3, 3, true);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWait0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(0, 0);
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0 << 8) | 0x3f);  // lgkmcnt(0): nothing of the prologue left
    __builtin_amdgcn_sched_barrier(0);

    // nk is a multiple of 8: all steps but the last four load steps kb+3 and kb+4
    for (int kb0 = 0; kb0 < nk - 4; kb0 += 4) {
#pragma unroll
        for (int i = 0; i < 4; i++) step(kb0 + i, i, true, true, true);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) step(nk - 4 + i, i, i == 0, false, i < 3);
    __builtin_amdgcn_s_waitcnt(0);

    // epilogue: the accumulators hold S (seeded with -gsum), y = ep(fma((float)S, xs * ws, 0)) (+ bias)
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);
    float wsv[2], bia[2] = {0.0f, 0.0f};
#pragma unroll
    for (int cb = 0; cb < 2; cb++) {
        const int o = nw0 + cb * 32 + l32;
        wsv[cb] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wsrs, (uint32_t)(o * 4), 0, 0));
        if constexpr (BIAS) bia[cb] = (o >= a.r0 && o < a.r1) ? a.bias[o] : 0.0f;
    }
    const bool full = m0 >= a.t0 && m0 + 128 <= a.t1 && nw0 >= a.r0 && nw0 + 64 <= a.r1;
    if (full) {
        // whole wave tile inside the window: buffer stores, the row offset in a scalar register
        const auto yrs = make_rsrc(a.y, a.y_bytes);
        const uint32_t out4 = (uint32_t)a.out * 4;
        const uint32_t vy = (uint32_t)(lh * 4) * out4 + (uint32_t)(nw0 + l32) * 4;
        v4i xs4a[4][4];  // all 16 token-scale quads in one batch (the fragment registers are free by now)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int vq = 0; vq < 4; vq++)
                xs4a[r][vq] = __builtin_amdgcn_raw_buffer_load_b128(
                    srs, (uint32_t)((m0 + r * 32 + vq * 8 + lh * 4) * 4), 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int vq = 0; vq < 4; vq++) {
                const v4i xs4 = xs4a[r][vq];
                float old[4][2];
                if constexpr (EP == VX_EP_ADD_SCALED) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
#pragma unroll
                        for (int cb = 0; cb < 2; cb++)
                            old[e][cb] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                yrs, vy + cb * 128, (uint32_t)(m0 + r * 32 + vq * 8 + e) * out4, 0));
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float xsv = __int_as_float(xs4[e]);
                    const uint32_t so = (uint32_t)(m0 + r * 32 + vq * 8 + e) * out4;
#pragma unroll
                    for (int cb = 0; cb < 2; cb++) {
                        const float v = __builtin_fmaf((float)acc[r][cb][vq * 4 + e], xsv * wsv[cb], 0.0f);
                        float res = v;
                        if constexpr (EP == VX_EP_SILU) res = silu_fast(v);
                        if constexpr (EP == VX_EP_ADD_SCALED) res = __builtin_fmaf(a.alpha, v, old[e][cb]);
                        if constexpr (BIAS) res = res + bia[cb];
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(res), yrs, vy + cb * 128, so, 0);
                    }
                }
            }
    } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int vq = 0; vq < 4; vq++) {
                const int t4 = m0 + r * 32 + vq * 8 + lh * 4;
                const v4i xs4 = __builtin_amdgcn_raw_buffer_load_b128(srs, (uint32_t)(t4 * 4), 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int64_t t = t4 + e;
                    if (t < a.t0 || t >= a.t1) continue;
                    const float xsv = __int_as_float(xs4[e]);
#pragma unroll
                    for (int cb = 0; cb < 2; cb++) {
                        const int64_t o = nw0 + cb * 32 + l32;
                        if (o < a.r0 || o >= a.r1) continue;
                        const float v = __builtin_fmaf((float)acc[r][cb][vq * 4 + e], xsv * wsv[cb], 0.0f);
                        float *py = a.y + t * a.out + o;
                        float res = v;
                        if constexpr (EP == VX_EP_SILU) res = silu_fast(v);
                        if constexpr (EP == VX_EP_ADD_SCALED) res = __builtin_fmaf(a.alpha, v, *py);
                        if constexpr (BIAS) res = res + bia[cb];
                        *py = res;
                    }
                }
            }
    }
}

namespace {

// Launch geometry: grid.x covers the output rows [n_base, r1) in BN = 64*NT steps, grid.y the tokens
// [m_base, t1) in BM = 16*MT steps (n_base and m_base are r0 and t0 rounded down to 16).
template <int MT, int NT>
dim3 grid_of(const GemmArgs &a) {
    return dim3((unsigned)((a.r1 - a.n_base + 64 * NT - 1) / (64 * NT)),
                (unsigned)((a.t1 - a.m_base + 16 * MT - 1) / (16 * MT)));
}

// Ring depth of the direct kernel: as many stages as fit in 60 outstanding loads (the vmcnt counter holds 63) and
// about 120 registers, at most 16.
constexpr int direct_depth(int mt, int nt, bool tern, bool single, int ks) {
    const int loads = ks * (mt + nt) + (single ? 0 : (tern ? 2 : 1) * mt + nt);
    const int regs = ks * (4 * mt + (tern ? 1 : 4) * nt) + (single ? 0 : 8 * mt + nt);
    int d = 60 / loads;
    if (d * regs > 120) d = 120 / regs;
    if (d > 16) d = 16;
    return d < 1 ? 1 : d;
}

template <int MT, int NT, bool TERN, bool GS>
void launch_direct(const GemmArgs &a, bool single, hipStream_t st) {
    const dim3 grid = grid_of<MT, NT>(a);
    if (single) {
        constexpr int D = direct_depth(MT, NT, TERN, true, 1);
        tgemm_direct_kernel<MT, NT, TERN, GS, true, 1, D><<<grid, 256, 0, st>>>(a);
    } else if (a.spg == 2) {
        constexpr int D = direct_depth(MT, NT, TERN, false, 2);
        tgemm_direct_kernel<MT, NT, TERN, GS, false, 2, D><<<grid, 256, 0, st>>>(a);
    } else {
        constexpr int D = direct_depth(MT, NT, TERN, false, 1);
        tgemm_direct_kernel<MT, NT, TERN, GS, false, 1, D><<<grid, 256, 0, st>>>(a);
    }
}

template <int MT, int NT, bool TERN, bool GS>
void launch_lds(const GemmArgs &a, bool single, int d, hipStream_t st) {
    const dim3 grid = grid_of<MT, NT>(a);
    if (d == 8) {
        if (single)
            tgemm_kernel<MT, NT, TERN, GS, true, 8><<<grid, 256, 0, st>>>(a);
        else
            tgemm_kernel<MT, NT, TERN, GS, false, 8><<<grid, 256, 0, st>>>(a);
    } else {
        // any group and step count (one stage in flight)
        tgemm_kernel<MT, NT, TERN, GS, false, 1><<<grid, 256, 0, st>>>(a);
    }
}

enum Kind { kDirect, kSplitK, kLds, kBig, kSplitG };

struct Plan {
    Kind kind;
    int mt, nt;
};

int64_t wgs_of(const GemmArgs &a, int bm, int bn) {
    return ((a.r1 - a.n_base + bn - 1) / bn) * ((a.t1 - a.m_base + bm - 1) / bm);
}

// Kernel and tile per shape. One group (G = K) with up to 1024 tokens and K a multiple of 256 takes the split-K
// kernel; the large-token ternary shapes whose K is a multiple of 512 the LDS-staged kernel; everything else the
// direct kernel (one group, or 64 or 128 columns per group) or, for other group sizes, the LDS-staged kernel with
// one stage in flight. vx_set_kernel_override("gemm" / "tile") forces a kernel and a tile (tests, tuning).
Plan plan_for(const GemmArgs &a, bool tern, bool gs, bool single) {
    const bool direct_ok = single || a.spg == 1 || a.spg == 2;
    const bool splitk_ok = single && (a.inp / 64) % 4 == 0;
    const bool lds_fast_ok = tern && !gs && (a.inp / 64) % 8 == 0;
    const bool big_ok = tern && single && !gs && (a.inp / 64) % 8 == 0 && a.y_bytes != 0;
    const bool splitg_ok = !single && a.spg == 2 && a.ng % 4 == 0;
    const int64_t m = a.t1 - a.m_base;
    Kind kind = (splitg_ok && m <= 1024) ? kSplitG
                : !direct_ok ? kLds
                : (splitk_ok && m <= 1024) ? kSplitK
                : (big_ok && m > 1024)     ? kBig
                : (lds_fast_ok && m > 1024) ? kLds
                                            : kDirect;
    const int forced = overrides().gemm.load(std::memory_order_relaxed);
    if (forced == kForceLds && lds_fast_ok) kind = kLds;
    if (forced == kForceDirect && direct_ok) kind = kDirect;
    if (forced == kForceSplitK && splitk_ok) kind = kSplitK;
    if (forced == kForceBig && big_ok) kind = kBig;
    if (forced == kForceSplitG && splitg_ok) kind = kSplitG;
    const int ft = overrides().tile.load(std::memory_order_relaxed), fmt = ft >> 4, fnt = ft & 15;
    if (kind == kBig) return Plan{kBig, 8, 4};
    if (kind == kSplitG) {
        static const Plan gtiles[] = {{kSplitG, 1, 8}, {kSplitG, 2, 4}, {kSplitG, 4, 2}};
        for (const Plan &t : gtiles)
            if (fmt == t.mt && fnt == t.nt) return t;
        return gtiles[0];
    }
    static const Plan dtiles[] = {{kDirect, 4, 4}, {kDirect, 2, 4}, {kDirect, 2, 2}, {kDirect, 1, 2}, {kDirect, 1, 1}};
    static const Plan ltiles[] = {{kLds, 4, 4}, {kLds, 4, 2}, {kLds, 2, 4}};
    static const Plan stiles[] = {{kSplitK, 2, 4}, {kSplitK, 1, 8}, {kSplitK, 4, 2}};
    const Plan *tiles = kind == kDirect ? dtiles : kind == kLds ? ltiles : stiles;
    const int ntiles = kind == kDirect ? 5 : 3;
    for (int i = 0; i < ntiles; i++)
        if (tiles[i].mt == fmt && tiles[i].nt == fnt) return tiles[i];
    if (kind == kLds) return m >= 4096 ? ltiles[1] : ltiles[2];
    if (kind == kSplitK) return stiles[0];
    for (int i = 0; i < ntiles; i++)
        if (wgs_of(a, 16 * tiles[i].mt, 64 * tiles[i].nt) >= 1024) return tiles[i];
    return tiles[ntiles - 1];
}

template <int MT, int NT, bool TERN, bool GS>
void launch_splitg(const GemmArgs &a, hipStream_t st) {
    const dim3 grid((unsigned)((a.r1 - a.n_base + 16 * NT - 1) / (16 * NT)),
                    (unsigned)((a.t1 - a.m_base + 16 * MT - 1) / (16 * MT)));
    const int nsw = (int)(a.ng / 4) * 2;  // k-steps per wave (two per group)
    if (nsw % 4 == 0)
        tgemm_splitk_groups_kernel<MT, NT, TERN, GS, 2, 4><<<grid, 256, 0, st>>>(a);
    else
        tgemm_splitk_groups_kernel<MT, NT, TERN, GS, 2, 2><<<grid, 256, 0, st>>>(a);
}

template <int MT, int NT, bool TERN, bool GS>
void launch_splitk(const GemmArgs &a, hipStream_t st) {
    const dim3 grid((unsigned)((a.r1 - a.n_base + 16 * NT - 1) / (16 * NT)),
                    (unsigned)((a.t1 - a.m_base + 16 * MT - 1) / (16 * MT)));
    // ring depth: every step of the wave's quarter of K when it fits in about 100 registers, else 8 (or fewer)
    const int nkw = (int)(a.inp / 64) / 4;
    constexpr int REGS = 4 * MT + (TERN ? 1 : 4) * NT;
    constexpr int DMAX = 100 / REGS >= 16 ? 16 : (100 / REGS >= 8 ? 8 : 4);
    if (DMAX >= 16 && nkw % 16 == 0)
        tgemm_splitk_kernel<MT, NT, TERN, GS, (DMAX >= 16 ? 16 : 1)><<<grid, 256, 0, st>>>(a);
    else if (DMAX >= 8 && nkw % 8 == 0)
        tgemm_splitk_kernel<MT, NT, TERN, GS, (DMAX >= 8 ? 8 : 1)><<<grid, 256, 0, st>>>(a);
    else if (nkw % 4 == 0)
        tgemm_splitk_kernel<MT, NT, TERN, GS, 4><<<grid, 256, 0, st>>>(a);
    else if (nkw % 2 == 0)
        tgemm_splitk_kernel<MT, NT, TERN, GS, 2><<<grid, 256, 0, st>>>(a);
    else
        tgemm_splitk_kernel<MT, NT, TERN, GS, 1><<<grid, 256, 0, st>>>(a);
}

#define VX_DISPATCH_TERN_GS(FN, ...)                   \
    do {                                               \
        if (tern) {                                    \
            if (gs)                                    \
                FN<MT, NT, true, true>(__VA_ARGS__);   \
            else                                       \
                FN<MT, NT, true, false>(__VA_ARGS__);  \
        } else {                                       \
            if (gs)                                    \
                FN<MT, NT, false, true>(__VA_ARGS__);  \
            else                                       \
                FN<MT, NT, false, false>(__VA_ARGS__); \
        }                                              \
    } while (0)

template <int MT, int NT>
void run_splitg(const GemmArgs &a, bool tern, bool gs, hipStream_t st) {
    VX_DISPATCH_TERN_GS(launch_splitg, a, st);
}

template <int MT, int NT>
void run_splitk(const GemmArgs &a, bool tern, bool gs, hipStream_t st) {
    VX_DISPATCH_TERN_GS(launch_splitk, a, st);
}

template <int MT, int NT>
void run_direct(const GemmArgs &a, bool tern, bool gs, bool single, hipStream_t st) {
    VX_DISPATCH_TERN_GS(launch_direct, a, single, st);
}

template <int MT, int NT>
void run_lds(const GemmArgs &a, bool tern, bool gs, bool single, int d, hipStream_t st) {
    VX_DISPATCH_TERN_GS(launch_lds, a, single, d, st);
}

}  // namespace

// Checks the operands of a GEMM call and fills its launch arguments (y may be NULL only for a quantized output).
static GemmArgs gemm_args(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n,
                          float *y, const float *bias, int ep, float alpha, int32_t *gs, int64_t r0, int64_t r1,
                          int64_t t0, int64_t t1, bool y_needed) {
    require(w != nullptr, "weight matrix must not be NULL");
    require(n == 0 || (xq && xs_t && (y || !y_needed)), "xq, xs_t and y must not be NULL");
    require(n == 0 || !w->ternary || xg_t, "ternary weights need the activation code sums (xgsum_t)");
    require(ep == VX_EP_STORE || ep == VX_EP_SILU || ep == VX_EP_ADD_SCALED, "unknown epilogue");
    require(n >= 0, "n must be >= 0");
    require(0 <= r0 && r0 <= r1 && r1 <= w->out, "row range outside [0, out]");
    require(0 <= t0 && t0 <= t1 && t1 <= n, "token range outside [0, n]");
    const int64_t np = (n + 15) / 16 * 16;
    require((np + 256) * w->inp < (1ll << 31) && np * w->ng * 4 < (1ll << 31), "activation operand above 2 GiB");
    GemmArgs a{};
    a.w = w->wdev;
    a.ws_t = w->scales_t;
    a.xq = xq;
    a.xs = xs_t;
    a.xg = xg_t;
    a.y = y;
    a.bias = bias;
    a.gs = gs;
    a.n = n;
    a.np = np;
    a.out = w->out;
    a.inp = w->inp;
    a.ng = w->ng;
    a.out_pad = w->out_pad;
    a.spg = w->group / 64;
    a.r0 = r0;
    a.r1 = r1;
    a.t0 = t0;
    a.t1 = t1;
    a.n_base = r0 / 16 * 16;
    a.m_base = t0 / 16 * 16;
    const int64_t wbytes = (w->out_pad / 16) * (w->inp / 64) * 64 * (w->ternary ? 4 : 16);
    require(wbytes < (1ll << 31), "weight plane above 2 GiB");
    a.w_bytes = (uint32_t)wbytes;
    a.ws_bytes = (uint32_t)(w->ng * w->out_pad * 4);
    a.xq_bytes = (uint32_t)(n * w->inp);
    a.xs_bytes = (uint32_t)(w->ng * np * 4);
    a.y_bytes = n * w->out * 4 < (1ll << 31) ? (uint32_t)(n * w->out * 4) : 0u;  // 0: no buffer stores
    a.ep = ep;
    a.alpha = alpha;
    a.vec_ok = (w->out % 4 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
               (!bias || reinterpret_cast<uintptr_t>(bias) % 16 == 0);
    return a;
}

// cap_rows: the rows that xq and y hold (0: n). With 128-column groups above 1024 tokens, buffers that hold the last
// partial 128-token tile let the streaming kernel run it too (its rows past n are read and written inside those
// buffers and not used), instead of a small-token launch for the remainder (32 x 125 tokens: 10.9 ms a forward
// against 12.0).
void gemm(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y,
          const float *bias, int ep, float alpha, int32_t *gs, int64_t r0, int64_t r1, int64_t t0, int64_t t1,
          hipStream_t st, int64_t cap_rows) {
    GemmArgs a = gemm_args(w, xq, xs_t, xg_t, n, y, bias, ep, alpha, gs, r0, r1, t0, t1, true);
    if (r0 == r1 || t0 == t1) return;
    const bool tern = w->ternary, g = gs != nullptr, single = w->ng == 1;
    // the streaming and small-token kernels also write the group sums of one group with the Store epilogue
    const bool fast_ok = !g || (single && ep == VX_EP_STORE);
    // whole 128-token tiles of a full-width ternary GEMM (one group or 128-column groups): the streaming kernels;
    // the remaining tokens (fewer than 128) go through the kernels below
    if (tern && fast_ok && r0 == 0 && r1 == w->out && t0 == 0 && n >= 128) {
        const int64_t up = (n + 127) / 128 * 128;
        const int64_t full = (!single && t1 == n && n > 1024 && cap_rows >= up) ? up : n / 128 * 128;
        if (full < (1ll << 30) && (single ? gemm_stream(a, (int)full, st) : gemm_stream_groups(a, (int)full, st))) {
            if (full >= n) return;
            a.t0 = full;
            a.m_base = full;
        }
    }
    if (tern && fast_ok && gemm_small(a, st)) return;
    const Plan p = plan_for(a, tern, g, single);
    if (p.kind == kBig) {
        const dim3 grid((unsigned)((a.r1 - a.n_base + 255) / 256), (unsigned)((a.t1 - a.m_base + 127) / 128));
        auto k = a.ep == VX_EP_SILU ? (a.bias ? tgemm_big_kernel<VX_EP_SILU, true> : tgemm_big_kernel<VX_EP_SILU, false>)
                 : a.ep == VX_EP_ADD_SCALED
                     ? (a.bias ? tgemm_big_kernel<VX_EP_ADD_SCALED, true> : tgemm_big_kernel<VX_EP_ADD_SCALED, false>)
                     : (a.bias ? tgemm_big_kernel<VX_EP_STORE, true> : tgemm_big_kernel<VX_EP_STORE, false>);
        k<<<grid, 256, 0, st>>>(a);
    } else if (p.kind == kSplitG) {
        if (p.mt == 2 && p.nt == 4)
            run_splitg<2, 4>(a, tern, g, st);
        else if (p.mt == 1 && p.nt == 8)
            run_splitg<1, 8>(a, tern, g, st);
        else
            run_splitg<4, 2>(a, tern, g, st);
    } else if (p.kind == kSplitK) {
        if (p.mt == 2 && p.nt == 4)
            run_splitk<2, 4>(a, tern, g, st);
        else if (p.mt == 1 && p.nt == 8)
            run_splitk<1, 8>(a, tern, g, st);
        else
            run_splitk<4, 2>(a, tern, g, st);
    } else if (p.kind == kDirect) {
        if (p.mt == 4 && p.nt == 4)
            run_direct<4, 4>(a, tern, g, single, st);
        else if (p.mt == 2 && p.nt == 4)
            run_direct<2, 4>(a, tern, g, single, st);
        else if (p.mt == 2 && p.nt == 2)
            run_direct<2, 2>(a, tern, g, single, st);
        else if (p.mt == 1 && p.nt == 2)
            run_direct<1, 2>(a, tern, g, single, st);
        else
            run_direct<1, 1>(a, tern, g, single, st);
    } else {
        const int d = (tern && !g && (a.inp / 64) % 8 == 0) ? 8 : 1;
        if (p.mt == 4 && p.nt == 4)
            run_lds<4, 4>(a, tern, g, single, d, st);
        else if (p.mt == 4 && p.nt == 2)
            run_lds<4, 2>(a, tern, g, single, d, st);
        else
            run_lds<2, 4>(a, tern, g, single, d, st);
    }
    hip_check(hipGetLastError(), "tgemm launch");
}

void quantize_ln(const float *x, int64_t n, int64_t inp, int64_t group, const float *g, const float *b, int8_t *q,
                 float *scales_t, int32_t *gsum_t, hipStream_t stream);

KernelOverrides &overrides() {
    static KernelOverrides o;
    return o;
}

// vx_set_kernel_override: name "gemm" (direct, splitk, lds, big, splitg, small, stream), "tile" and "small_tile"
// ("MTxNT"), "stream_grid" (workgroups, a multiple of 8), "small_ws" ("on" / "off": the grouped small-token kernel
// with producer and consumer wavefronts), "linear" (the f32 linear: "lds", or the
// matrix-core kernel's tile, "mfma1x1" / "mfma2x1" / "mfma2x2"), "stream_tile" (token blocks of 16 per wavefront of
// the 128-column-group streaming kernel: 4 or 8); NULL or "" clears the name's override.
void set_kernel_override(const char *name, const char *value) {
    require(name != nullptr, "override name must not be NULL");
    const std::string n(name), v(value ? value : "");
    KernelOverrides &o = overrides();
    auto tile_code = [&](const std::string &t) {
        int mt = 0, nt = 0;
        require(sscanf(t.c_str(), "%dx%d", &mt, &nt) == 2 && mt > 0 && mt < 16 && nt > 0 && nt < 16,
                "a tile override is MTxNT with 0 < MT, NT < 16");
        return mt * 16 + nt;
    };
    if (n == "gemm") {
        static const char *kinds[] = {"", "direct", "splitk", "lds", "big", "splitg", "small", "stream"};
        for (int k = 0; k < 8; k++)
            if (v == kinds[k]) {
                o.gemm.store(k, std::memory_order_relaxed);
                return;
            }
        throw Error(VX_ERR_INVALID, "unknown gemm override '" + v + "'");
    } else if (n == "tile") {
        o.tile.store(v.empty() ? 0 : tile_code(v), std::memory_order_relaxed);
    } else if (n == "small_tile") {
        o.small_tile.store(v.empty() ? 0 : tile_code(v), std::memory_order_relaxed);
    } else if (n == "small_ws") {
        require(v.empty() || v == "on" || v == "off", "small_ws is \"on\", \"off\" or empty");
        o.small_ws.store(v.empty() ? 0 : v == "on" ? 1 : 2, std::memory_order_relaxed);
    } else if (n == "stream_tile") {
        const int tb = v.empty() ? 0 : atoi(v.c_str());
        require(tb == 0 || tb == 4 || tb == 8, "stream_tile is 4, 8 or empty");
        o.stream_tb.store(tb, std::memory_order_relaxed);
    } else if (n == "linear") {
        const int k = v.empty() ? 0 : v == "lds" ? -1 : v == "mfma1x1" ? 111 : v == "mfma2x1" ? 121
                                                        : v == "mfma2x2" ? 122 : -2;
        require(k != -2, "linear is \"lds\", \"mfma1x1\", \"mfma2x1\", \"mfma2x2\" or empty");
        o.linear.store(k, std::memory_order_relaxed);
    } else if (n == "stream_grid") {
        const int g = v.empty() ? 0 : atoi(v.c_str());
        require(g == 0 || (g >= 8 && g % 8 == 0), "stream_grid is a positive multiple of 8");
        o.stream_grid.store(g, std::memory_order_relaxed);
    } else {
        throw Error(VX_ERR_INVALID, "unknown override name '" + n + "'");
    }
}

// The FFN up-projection with the down-projection's quantization fused (encoder.rs:87-89: forward_prepared_ep with
// Silu into hbuf, then prepare(hbuf) = QuantAct::quantize_layout, packed.rs:307-436): y = ep(x . w^T) (+ bias),
// quantized in `group`-column groups into q [n][out], scales_t and gsum_t [out/group][npad(n)]. With 128-column
// groups and up to 1024 tokens the small-token kernel quantizes in its epilogue and y never reaches memory; other
// shapes run the GEMM into y_tmp and then the quantizer. The codes equal those of the two-step chain bit for bit.
void gemm_quant(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y_tmp,
                const float *bias, int ep, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t, hipStream_t st,
                int64_t cap_rows) {
    require(n == 0 || (q && scales_t && gsum_t), "q, scales_t and gsum_t must not be NULL");
    require(ep == VX_EP_STORE || ep == VX_EP_SILU, "a quantized output takes the Store or Silu epilogue");
    require(w != nullptr && group > 0 && w->out % group == 0, "out must be a positive multiple of group");
    GemmArgs a = gemm_args(w, xq, xs_t, xg_t, n, y_tmp, bias, ep, 0.0f, nullptr, 0, w->out, 0, n, false);
    if (n == 0) return;
    if (w->ternary && group == 128) {
        a.qo = q;
        a.qs = scales_t;
        a.qg = gsum_t;
        if (gemm_small(a, st)) return;
    }
    require(y_tmp != nullptr, "y_tmp must not be NULL for this shape (the GEMM output goes through it)");
    gemm(w, xq, xs_t, xg_t, n, y_tmp, bias, ep, 0.0f, nullptr, 0, w->out, 0, n, st, cap_rows);
    quantize_ln(y_tmp, n, w->out, group, nullptr, nullptr, q, scales_t, gsum_t, st);
}

}  // namespace vx
