// vx_gemm.hip — ternary (or int8) x int8 GEMM on CDNA4 i8 MFMA, bit-exact to voxrt's scalar kernel
// (crates/voxrt/src/kernels/mod.rs:166-210).
//
//   y[t, o] = ep(y_old, acc),  acc = fold over groups g ascending of fma((float)S_g, xs[t, g] * ws[o, g], acc)
//   S_g     = sum_{c in group g} w[o, c] * x[t, c]   (exact int32)
//
// Work decomposition. A workgroup of 4 wavefronts owns a tile of BM = 16*MT tokens x BN = 4*16*NT output rows;
// wavefront w owns the BN/4 rows [16*NT*w, 16*NT*(w+1)) of it and all BM tokens. Per 64-column step the
// workgroup stages the BM x 64 int8 activation tile in LDS (double buffered, XOR-swizzled 16-byte chunks so a
// 16-lane phase of ds_read_b128 touches 64 distinct banks) and each wavefront streams its own weight operands
// straight from HBM into registers: one dword of 2-bit codes per lane per 16x64 block, widened to int8 codes
// (trit + 1 in {0, 1, 2}) with four shift/and operations. v_mfma_i32_16x16x64_i8 accumulates
// sum x * (trit + 1) in int32; seeding its C operand with -sum(x) of the group (the quantizer's gsum) makes the
// accumulator exactly S_g at no extra instruction. At the end of each group the int32 sums are folded into the
// fp32 accumulators with the reference's operation order; the epilogue applies Store / SiLU / AddScaled (+ bias).
//
// MFMA operand layouts (16x16x64, wave64): lane l supplies row l%16 of A and column l%16 of B over the same 16
// columns of the 64-column step (lane group l/16); D element e of lane l is D[4*(l/16) + e][l%16].
// A = activations (rows = tokens), B = weights (columns = output rows), so a lane's outputs are 4 tokens of one
// output row and 16 consecutive lanes store 64 contiguous bytes of y.
//
// Ragged edges: every read-only operand goes through a raw buffer descriptor whose range ends at the operand's
// size, so loads past the last token (or past the padded weight rows) return zero without branches; stores are
// guarded by the [t0, t1) x [r0, r1) window.
#include "vx_internal.h"

namespace vx {

struct GemmArgs {
    const void *w;          // ternary: uint32 codes; int8: 16-byte chunks (see TMat)
    const float *ws_t;      // [ng][out_pad]
    const int8_t *xq;       // [n][inp]
    const float *xs;        // [n][ng]
    const int32_t *xg;      // [n][ng] (ternary only)
    float *y;               // [n][out]
    const float *bias;      // [out] or NULL
    int32_t *gs;            // [ng][n][out] or NULL
    int64_t n, out, inp, ng, out_pad, spg;
    int64_t r0, r1, t0, t1, n_base;
    uint32_t w_bytes, ws_bytes, xq_bytes, xs_bytes;
    int ep;
    float alpha;
};

__device__ inline v4i widen_codes(uint32_t p) {
    v4i r;
    r.x = (int)(p & 0x03030303u);
    r.y = (int)((p >> 2) & 0x03030303u);
    r.z = (int)((p >> 4) & 0x03030303u);
    r.w = (int)((p >> 6) & 0x03030303u);
    return r;
}

template <int MT, int NT, bool TERN, bool GS>
__global__ __launch_bounds__(256) void tgemm_kernel(const GemmArgs a) {
    constexpr int BM = MT * 16;
    constexpr int BN = NT * 16 * 4;
    constexpr int ACH = (BM * 4 + 255) / 256;  // 16-byte activation chunks per thread per step
    __shared__ __attribute__((aligned(16))) int8_t lds[2][BM * 64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m0 = a.t0 + (int64_t)blockIdx.y * BM;
    const int64_t nw0 = a.n_base + (int64_t)blockIdx.x * BN + wave * NT * 16;
    const int64_t nk = a.inp / 64;
    const int64_t ng = a.ng;

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto grs = make_rsrc(a.xg, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);

    // activation chunk c of a step: row c >> 2, 16-byte column chunk c & 3
    v4i apre[ACH];
    auto load_a = [&](int64_t kb) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = tid + i * 256;
            if (c < BM * 4) {
                const uint32_t off = (uint32_t)((m0 + (c >> 2)) * a.inp + kb * 64 + (c & 3) * 16);
                apre[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
            }
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int c = tid + i * 256;
            if (c < BM * 4) {
                const int row = c >> 2, ch = (c & 3) ^ ((row >> 2) & 3);
                *(v4i *)&lds[buf][row * 64 + ch * 16] = apre[i];
            }
        }
    };

    // weight operand of block nb of this wavefront at step kb
    typedef typename std::conditional<TERN, uint32_t, v4i>::type BReg;
    BReg bcur[NT], bpre[NT];
    auto load_b = [&](int64_t kb, BReg *dst) {
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            const int64_t blk = (nw0 / 16 + nb) * nk + kb;
            if constexpr (TERN)
                dst[nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)((blk * 64 + lane) * 4), 0, 0);
            else
                dst[nb] = __builtin_amdgcn_raw_buffer_load_b128(wrs, (uint32_t)((blk * 64 + lane) * 16), 0, 0);
        }
    };

    v4i acc[MT][NT];
    float accf[MT][NT][4];
#pragma unroll
    for (int mb = 0; mb < MT; mb++)
#pragma unroll
        for (int nb = 0; nb < NT; nb++)
#pragma unroll
            for (int e = 0; e < 4; e++) accf[mb][nb][e] = 0.0f;

    load_a(0);
    load_b(0, bcur);
    store_a(0);
    __syncthreads();

    const int arow = lane & 15, aj = lane >> 4;
    int64_t kb = 0;
    for (int64_t g = 0; g < ng; g++) {
        v4i cinit[MT];
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if constexpr (TERN) {
                    const int64_t t = m0 + mb * 16 + 4 * aj + e;
                    cinit[mb][e] = -(int)__builtin_amdgcn_raw_buffer_load_b32(grs, (uint32_t)((t * ng + g) * 4), 0, 0);
                } else {
                    cinit[mb][e] = 0;
                }
            }
        for (int64_t s = 0; s < a.spg; s++, kb++) {
            const int buf = (int)(kb & 1);
            if (kb + 1 < nk) {
                load_a(kb + 1);
                load_b(kb + 1, bpre);
            }
            v4i av[MT], bv[NT];
#pragma unroll
            for (int mb = 0; mb < MT; mb++) {
                const int row = mb * 16 + arow, ch = aj ^ ((row >> 2) & 3);
                av[mb] = *(const v4i *)&lds[buf][row * 64 + ch * 16];
            }
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                if constexpr (TERN)
                    bv[nb] = widen_codes(bcur[nb]);
                else
                    bv[nb] = bcur[nb];
            }
            if (s == 0) {
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
            if (kb + 1 < nk) {
                store_a(buf ^ 1);
#pragma unroll
                for (int nb = 0; nb < NT; nb++) bcur[nb] = bpre[nb];
            }
            __syncthreads();
        }
        // fold group g: acc_f = fma((float)S_g, xs[t][g] * ws[o][g], acc_f)
        float xsv[MT][4], wsv[NT];
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t t = m0 + mb * 16 + 4 * aj + e;
                xsv[mb][e] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(srs, (uint32_t)((t * ng + g) * 4), 0, 0));
            }
#pragma unroll
        for (int nb = 0; nb < NT; nb++) {
            const int64_t o = nw0 + nb * 16 + arow;
            wsv[nb] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(wsrs, (uint32_t)((g * a.out_pad + o) * 4), 0, 0));
        }
#pragma unroll
        for (int mb = 0; mb < MT; mb++)
#pragma unroll
            for (int nb = 0; nb < NT; nb++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float p = xsv[mb][e] * wsv[nb];
                    accf[mb][nb][e] = __builtin_fmaf((float)acc[mb][nb][e], p, accf[mb][nb][e]);
                }
        if constexpr (GS) {
#pragma unroll
            for (int mb = 0; mb < MT; mb++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int64_t t = m0 + mb * 16 + 4 * aj + e;
                    if (t >= a.t1) continue;
#pragma unroll
                    for (int nb = 0; nb < NT; nb++) {
                        const int64_t o = nw0 + nb * 16 + arow;
                        if (o >= a.r0 && o < a.r1) a.gs[(g * a.n + t) * a.out + o] = acc[mb][nb][e];
                    }
                }
        }
    }

    // epilogue (kernels/mod.rs:41-48; bias added after it as in gemm_ep, kernels/mod.rs:355-361)
#pragma unroll
    for (int mb = 0; mb < MT; mb++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int64_t t = m0 + mb * 16 + 4 * aj + e;
            if (t >= a.t1) continue;
#pragma unroll
            for (int nb = 0; nb < NT; nb++) {
                const int64_t o = nw0 + nb * 16 + arow;
                if (o < a.r0 || o >= a.r1) continue;
                float *p = a.y + t * a.out + o;
                float r = ep_apply(a.ep, a.alpha, a.ep == VX_EP_ADD_SCALED ? *p : 0.0f, accf[mb][nb][e]);
                if (a.bias) r = r + a.bias[o];
                *p = r;
            }
        }
}

namespace {

struct Tile {
    int mt, nt;
};

// Largest tile that still gives at least two workgroups per CU (256 CUs); the smallest one otherwise.
Tile choose_tile(int64_t m, int64_t nrows) {
    static const Tile tiles[] = {{4, 4}, {4, 2}, {2, 4}, {2, 2}, {1, 2}, {1, 1}};
    const char *env = getenv("VX_TILE");
    if (env && *env) {
        int mt = 0, nt = 0;
        if (sscanf(env, "%dx%d", &mt, &nt) == 2)
            for (const Tile &t : tiles)
                if (t.mt == mt && t.nt == nt) return t;
    }
    for (const Tile &t : tiles) {
        int64_t wgs = ((m + 16 * t.mt - 1) / (16 * t.mt)) * ((nrows + 64 * t.nt - 1) / (64 * t.nt));
        if (wgs >= 512) return t;
    }
    return tiles[sizeof(tiles) / sizeof(tiles[0]) - 1];
}

template <int MT, int NT>
void launch_tile(const GemmArgs &a, bool tern, bool gs, hipStream_t st) {
    constexpr int BM = MT * 16, BN = NT * 64;
    dim3 grid((unsigned)((a.r1 - a.n_base + BN - 1) / BN), (unsigned)((a.t1 - a.t0 + BM - 1) / BM));
    if (tern) {
        if (gs)
            tgemm_kernel<MT, NT, true, true><<<grid, 256, 0, st>>>(a);
        else
            tgemm_kernel<MT, NT, true, false><<<grid, 256, 0, st>>>(a);
    } else {
        if (gs)
            tgemm_kernel<MT, NT, false, true><<<grid, 256, 0, st>>>(a);
        else
            tgemm_kernel<MT, NT, false, false><<<grid, 256, 0, st>>>(a);
    }
}

}  // namespace

void gemm(const TMat *w, const int8_t *xq, const float *xs, const int32_t *xg, int64_t n, float *y,
          const float *bias, int ep, float alpha, int32_t *gs, int64_t r0, int64_t r1, int64_t t0, int64_t t1,
          hipStream_t st) {
    require(w != nullptr, "weight matrix must not be NULL");
    require(xq && xs && y, "xq, xs and y must not be NULL");
    require(!w->ternary || xg, "ternary weights need the activation code sums (xgsum)");
    require(ep == VX_EP_STORE || ep == VX_EP_SILU || ep == VX_EP_ADD_SCALED, "unknown epilogue");
    require(n >= 0, "n must be >= 0");
    require(0 <= r0 && r0 <= r1 && r1 <= w->out, "row range outside [0, out]");
    require(0 <= t0 && t0 <= t1 && t1 <= n, "token range outside [0, n]");
    require((n + 256) * w->inp < (1ll << 32) && n * w->ng * 4 < (1ll << 32), "activation operand above 4 GiB");
    if (r0 == r1 || t0 == t1) return;
    GemmArgs a;
    a.w = w->wdev;
    a.ws_t = w->scales_t;
    a.xq = xq;
    a.xs = xs;
    a.xg = xg;
    a.y = y;
    a.bias = bias;
    a.gs = gs;
    a.n = n;
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
    const int64_t wbytes = (w->out_pad / 16) * (w->inp / 64) * 64 * (w->ternary ? 4 : 16);
    require(wbytes < (1ll << 32), "weight plane above 4 GiB");
    a.w_bytes = (uint32_t)wbytes;
    a.ws_bytes = (uint32_t)(w->ng * w->out_pad * 4);
    a.xq_bytes = (uint32_t)(n * w->inp);
    a.xs_bytes = (uint32_t)(n * w->ng * 4);
    a.ep = ep;
    a.alpha = alpha;
    const Tile t = choose_tile(t1 - t0, r1 - a.n_base);
    const bool tern = w->ternary, g = gs != nullptr;
    if (t.mt == 4 && t.nt == 4)
        launch_tile<4, 4>(a, tern, g, st);
    else if (t.mt == 4 && t.nt == 2)
        launch_tile<4, 2>(a, tern, g, st);
    else if (t.mt == 2 && t.nt == 4)
        launch_tile<2, 4>(a, tern, g, st);
    else if (t.mt == 2 && t.nt == 2)
        launch_tile<2, 2>(a, tern, g, st);
    else if (t.mt == 1 && t.nt == 2)
        launch_tile<1, 2>(a, tern, g, st);
    else
        launch_tile<1, 1>(a, tern, g, st);
    hip_check(hipGetLastError(), "tgemm_kernel launch");
}

}  // namespace vx
