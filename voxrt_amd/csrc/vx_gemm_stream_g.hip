// vx_gemm_stream_g.hip — persistent large-token ternary x int8 GEMM with 128-column groups (G = 128, the model
// format) on gfx950 i8 MFMA, bit-exact to voxrt's scalar kernel (crates/voxrt/src/kernels/mod.rs:166-210):
//
//   acc = 0; for each group g ascending: acc = fma((float)S_g, xs[t][g] * ws[o][g], acc); y = ep(acc) (+ bias)
//
// Tiles, XCD grouping, MFMA operand roles and the load pipeline are those of the one-group streaming kernel
// (vx_gemm_stream.hip): 128-token (or 64-token, two workgroups per CU) x 256-row tiles, wavefront w owns rows
// [64w, 64w + 64) and all the tile's tokens,
// v_mfma_i32_16x16x64_i8 with A = weight codes and B = activations, the activation tile and the weight codes of
// step s + 6 brought to LDS by buffer_load ... lds, one constant vmcnt wait and one barrier per step.
//
// Groups: a group is two 64-column steps. The weight codes (trit + 1) are widened to the signed trits themselves
// (one byte permute per dword maps 0, 1, 2 to -1, 0, +1), every MFMA chain starts from zero on the group's first
// step, and after its second step the int32 accumulator is exactly S_g; each block's four sums are folded into
// the fp32 accumulators in the reference's operation order a few MFMAs after its last one. The token scales and
// weight scales of a group reach LDS with the loads of its two steps (four group slots). The epilogue (Store, SiLU
// or AddScaled, then bias) of a tile runs after its last step.
#include <algorithm>
#include <cstring>

#include "vx_gemm.h"

namespace vx {
namespace {

constexpr int kPDg = 6;  // steps of loads in flight
// Per step TB / 4 + 2 vector-memory instructions per wavefront (TB / 4 activation DMA, 1 weight DMA, 1 scale DMA)
// issued together. When step s begins, the loads of step s+1 (issued at step s+1-kPDg) must be complete: the
// instructions issued after them are those of steps s+2-kPDg .. s-1.
__host__ __device__ constexpr int vmem_per_step(int tb) { return tb / 4 + 2; }
__host__ __device__ constexpr int wait_g(int tb) { return vmem_per_step(tb) * (kPDg - 2); }

// 16 weight codes (trit + 1, 2 bits each, in the MFMA operand order) -> 16 signed trits: byte b of component d is
// code 4d + b; v_perm_b32 with the codes as byte selectors picks -1, 0, +1 from the table 0x000100FF.
__device__ inline v4i widen_trits(uint32_t p) {
    v4i r;
    r.x = (int)__builtin_amdgcn_perm(0u, 0x000100FFu, p & 0x03030303u);
    r.y = (int)__builtin_amdgcn_perm(0u, 0x000100FFu, (p >> 2) & 0x03030303u);
    r.z = (int)__builtin_amdgcn_perm(0u, 0x000100FFu, (p >> 4) & 0x03030303u);
    r.w = (int)__builtin_amdgcn_perm(0u, 0x000100FFu, (p >> 6) & 0x03030303u);
    return r;
}

// TB: token blocks of 16 per wavefront, the tile's token rows are 16 TB. TB = 8: one workgroup per CU (128-token
// tiles); TB = 4: 64-token tiles, half the accumulators and LDS, two workgroups (two wavefronts per SIMD) per CU, so
// that one wavefront's fold issues while the other's MFMAs run.
template <int EP, bool BIAS, int TB>
__global__ __launch_bounds__(256, TB == 4 ? 2 : 1) void tgemm_stream_groups_kernel(const GemmArgs a,
                                                                                    const StreamGeom g) {
    typedef __attribute__((address_space(3))) void lds_void;
    constexpr int BM = 16 * TB, NAD = TB / 4;  // tile token rows; activation DMAs (16 rows each) per wavefront
    // one LDS object per slot, so that the compiler sees that a DMA into one slot does not alias reads of another
    __shared__ __attribute__((aligned(1024))) int8_t sa0[BM * 64], sa1[BM * 64], sa2[BM * 64], sa3[BM * 64],
        sa4[BM * 64], sa5[BM * 64], sa6[BM * 64], sa7[BM * 64];
    __shared__ __attribute__((aligned(1024))) uint32_t sw0[1024], sw1[1024], sw2[1024], sw3[1024], sw4[1024],
        sw5[1024], sw6[1024], sw7[1024];
    // per group slot: token scales (256 tokens from the tile's first, 128 used), weight scales (256 rows)
    __shared__ __attribute__((aligned(16))) float xs0[256], xs1[256], xs2[256], xs3[256], ws0[256], ws1[256],
        ws2[256], ws3[256];
    auto sact = [&](int i) __attribute__((always_inline)) -> int8_t * {
        return i == 0 ? sa0 : i == 1 ? sa1 : i == 2 ? sa2 : i == 3 ? sa3 : i == 4 ? sa4 : i == 5 ? sa5 : i == 6 ? sa6 : sa7;
    };
    auto swt = [&](int i) __attribute__((always_inline)) -> uint32_t * {
        return i == 0 ? sw0 : i == 1 ? sw1 : i == 2 ? sw2 : i == 3 ? sw3 : i == 4 ? sw4 : i == 5 ? sw5 : i == 6 ? sw6 : sw7;
    };
    auto sxs = [&](int q) __attribute__((always_inline)) -> float * { return q == 0 ? xs0 : q == 1 ? xs1 : q == 2 ? xs2 : xs3; };
    auto sws = [&](int q) __attribute__((always_inline)) -> float * { return q == 0 ? ws0 : q == 1 ? ws1 : q == 2 ? ws2 : ws3; };

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lq = lane >> 4;
    const int inp = (int)a.inp, nk = g.nk;
    const uint32_t out4 = (uint32_t)a.out * 4, np4 = (uint32_t)a.np * 4, opad4 = (uint32_t)a.out_pad * 4;

    const int xcd = blockIdx.x & 7, wi = blockIdx.x >> 3, nwx = gridDim.x >> 3;
    auto tile_at = [&](int j) __attribute__((always_inline)) -> int {
        const int s = wi + j * nwx, t = xcd * g.per_xcd + s;
        return (s < g.per_xcd && t < g.ntiles) ? t : -1;
    };

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);
    const auto yrs = make_rsrc(a.y, a.y_bytes);

    uint32_t vdma[NAD];
    {
        const int i = lane >> 2, c = (lane & 3) ^ ((i >> 2) & 3);
#pragma unroll
        for (int q = 0; q < NAD; q++) vdma[q] = (uint32_t)(((NAD * wave + q) * 16 + i) * inp + c * 16);
    }
    const uint32_t vfr = (uint32_t)(l16 * 64 + ((lq ^ ((l16 >> 2) & 3)) * 16));
    const uint32_t vwd = (uint32_t)((lane >> 4) * nk * 256 + (lane & 15) * 16);
    const uint32_t vyl = (uint32_t)l16 * out4 + (uint32_t)lq * 16;
    const uint32_t vq4 = (uint32_t)(64 * wave + lane) * 4;  // this wavefront's quarter of a scale table

    // --- tile state ---------------------------------------------------------------------------------------------
    int jt = 0;
    int cur = tile_at(0);
    if (cur < 0) return;  // a workgroup of the last XCD past its last tile
    int m0 = (cur / g.n_nt) * BM, n0 = (cur % g.n_nt) * kBN;
    uint32_t sa_cur = (uint32_t)m0 * inp, sw_cur = (uint32_t)((n0 / 16 + wave * 4) * nk) * 256;
    uint32_t sa_nxt = 0, sw_nxt = 0, vdma_nxt[NAD], vw_nxt = kOff;
#pragma unroll
    for (int q = 0; q < NAD; q++) vdma_nxt[q] = kOff;
    int nxt = -1, nm0 = 0, nn0 = 0;
    bool has_nxt = false;
    auto set_next = [&]() __attribute__((always_inline)) {
        nxt = tile_at(jt + 1);
        has_nxt = nxt >= 0;
        nm0 = has_nxt ? (nxt / g.n_nt) * BM : 0;
        nn0 = has_nxt ? (nxt % g.n_nt) * kBN : 0;
        sa_nxt = (uint32_t)nm0 * inp;
        sw_nxt = (uint32_t)((nn0 / 16 + wave * 4) * nk) * 256;
#pragma unroll
        for (int q = 0; q < NAD; q++) vdma_nxt[q] = has_nxt ? vdma[q] : kOff;
        vw_nxt = has_nxt ? vwd : kOff;
    };

    // the loads of step k of a tile (token base tm0, row base tn0, scalar offsets sa / sw), into slot k % 8:
    // activations, weight codes, and the scales of group k / 2 (even k: token scales; odd k: weight scales)
    // (slot, the group slot q = (k / 2) % 4 and the parity of k are compile-time at every call: tile steps run in
    // blocks of 8 aligned to multiples of 8)
    auto loads = [&](int slot, int q, int odd, int k, bool live, const uint32_t *vd, uint32_t sa, uint32_t vw,
                     uint32_t sw, int tm0, int tn0) {
#pragma unroll
        for (int q = 0; q < NAD; q++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_void *)(sact(slot) + (NAD * wave + q) * 1024), 16,
                                                     vd[q], sa + (uint32_t)k * 64, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void *)(swt(slot) + wave * 256), 16, vw,
                                                 sw + (uint32_t)k * 256, 0, 0);
        // the group's scales, each wavefront one quarter of the 256-entry table (4 bytes per lane)
        const int gg = k >> 1;
        if (!odd) {
            const uint32_t vt = live ? (uint32_t)gg * np4 + (uint32_t)tm0 * 4 + vq4 : kOff;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (lds_void *)(sxs(q) + 64 * wave), 4, vt, 0, 0, 0);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wsrs, (lds_void *)(sws(q) + 64 * wave), 4, live ? vq4 : kOff,
                                                     (uint32_t)gg * opad4 + (uint32_t)tn0 * 4, 0, 0);
        }
    };

    v4i fr[2][TB];
    uint32_t rw[4];
    auto read_frags = [&](int slot, int set) __attribute__((always_inline)) {
#pragma unroll
        for (int tb = 0; tb < TB; tb++) fr[set][tb] = *(const v4i *)(sact(slot) + tb * 1024 + vfr);
    };
    auto read_weights = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int ob = 0; ob < 4; ob++) rw[ob] = swt(slot)[wave * 256 + ob * 64 + lane];
    };
    v4i bw[2][4];
    auto widen = [&](int set) __attribute__((always_inline)) {
#pragma unroll
        for (int ob = 0; ob < 4; ob++) bw[set][ob] = widen_trits(rw[ob]);
    };

    v4i acc[TB][4];
    float accf[TB][4][4];

    // one K step of the current tile. SLOT = i % 8; H = i % 2 (0: the group's first step, 1: its second);
    // FIRST: group 0 (the fp32 fold starts from zero); NEXT: this step's loads are the next tile's step i+6-nk
    auto step = [&](auto SLOTc, auto FIRSTc, auto NEXTc, int i) __attribute__((always_inline)) {
        constexpr int SLOT = decltype(SLOTc)::value, H = SLOT & 1;
        constexpr bool FIRST = decltype(FIRSTc)::value != 0, NEXT = decltype(NEXTc)::value != 0;
        constexpr int q = SLOT >> 1;                          // group slot of this step (i % 8 == SLOT)
        constexpr int qn = ((SLOT + kPDg) >> 1) & 3;          // group slot of the step whose loads issue now
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(wait_g(TB)));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // LDS reads that this step's VALU work waits for
        float xsv[TB];
        float4 wsv[4];
        if constexpr (H == 1) {
#pragma unroll
            for (int tb = 0; tb < TB; tb++) xsv[tb] = sxs(q)[tb * 16 + l16];
#pragma unroll
            for (int ob = 0; ob < 4; ob++) wsv[ob] = *(const float4 *)&sws(q)[wave * 64 + ob * 16 + lq * 4];
        }
        read_weights((SLOT + 1) & 7);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NEXT)
            loads((SLOT + kPDg) & 7, qn, (SLOT + kPDg) & 1, i + kPDg - nk, has_nxt, vdma_nxt, sa_nxt, vw_nxt, sw_nxt,
                  nm0, nn0);
        else
            loads((SLOT + kPDg) & 7, qn, (SLOT + kPDg) & 1, i + kPDg, true, vdma, sa_cur, vwd, sw_cur, m0, n0);
        __builtin_amdgcn_sched_barrier(0);
        read_frags((SLOT + 1) & 7, (SLOT + 1) & 1);
        constexpr int fs = SLOT & 1;
        // the group's sums of block (tb, ob) are final after its second-step MFMA: fold them into the fp32
        // accumulators (kernels/mod.rs:186-188), four MFMAs later in program order
        auto fold = [&](int tb, int ob) __attribute__((always_inline)) {
            const float wsa[4] = {wsv[ob].x, wsv[ob].y, wsv[ob].z, wsv[ob].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float p = xsv[tb] * wsa[e];
                accf[tb][ob][e] = __builtin_fmaf((float)acc[tb][ob][e], p, FIRST ? 0.0f : accf[tb][ob][e]);
            }
        };
        static_for<0, 4 * TB>([&](auto B) __attribute__((always_inline)) {
            constexpr int b = decltype(B)::value, tb = b >> 2, ob = b & 3;
            if constexpr (H == 0) {
                acc[tb][ob] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[fs][ob], fr[fs][tb], v4i{0, 0, 0, 0}, 0, 0, 0);
            } else {
                acc[tb][ob] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[fs][ob], fr[fs][tb], acc[tb][ob], 0, 0, 0);
                if constexpr (b >= 4) fold((b - 4) >> 2, (b - 4) & 3);
            }
        });
        if constexpr (H == 1)
            static_for<4 * TB - 4, 4 * TB>([&](auto B) __attribute__((always_inline)) {
                fold(decltype(B)::value >> 2, decltype(B)::value & 3);
            });
        widen(fs ^ 1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // the epilogue of the current tile from the fp32 accumulators (kernels/mod.rs:41-48, bias after it)
    auto epilogue = [&]() __attribute__((always_inline)) {
        const uint32_t sy = (uint32_t)m0 * out4 + (uint32_t)(n0 + wave * 64) * 4;
        const auto brs = make_rsrc(a.bias, BIAS ? (uint32_t)(a.out * 4) : 0u);
#pragma unroll
        for (int ob = 0; ob < 4; ob++) {
            v4i b4 = v4i{0, 0, 0, 0};
            if constexpr (BIAS)
                b4 = __builtin_amdgcn_raw_buffer_load_b128(brs, (uint32_t)(n0 + wave * 64 + ob * 16 + lq * 4) * 4, 0,
                                                           0);
#pragma unroll
            for (int tb = 0; tb < TB; tb++) {
                const uint32_t so = sy + (uint32_t)(tb * 16) * out4 + (uint32_t)(ob * 64);
                v4i old = v4i{0, 0, 0, 0};
                if constexpr (EP == VX_EP_ADD_SCALED) old = __builtin_amdgcn_raw_buffer_load_b128(yrs, vyl, so, 0);
                v4i r;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v = accf[tb][ob][e];
                    float res = v;
                    if constexpr (EP == VX_EP_SILU) res = silu_fast(v);
                    if constexpr (EP == VX_EP_ADD_SCALED) res = __builtin_fmaf(a.alpha, v, __int_as_float(old[e]));
                    if constexpr (BIAS) res = res + __int_as_float(b4[e]);
                    r[e] = __float_as_int(res);
                }
                store_b128_sep(r, yrs, vyl, so);
            }
        }
    };

    // prologue: the loads of steps 0 .. kPDg-1 of the first tile
#pragma unroll
    for (int i = 0; i < kPDg; i++) {
        loads(i, (i >> 1) & 3, i & 1, i, true, vdma, sa_cur, vwd, sw_cur, m0, n0);
        __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(vmem_per_step(TB) * (kPDg - 1)));  // the loads of step 0 complete
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(0, 0);
    read_weights(0);
    widen(0);

    for (;;) {
        set_next();
        // steps 0..7 (groups 0..3; group 0 starts the fold), then 8-step blocks, the last one loading the next
        // tile's first steps; nk is a multiple of 8 and at least 16
        static_for<0, 8>([&](auto P) __attribute__((always_inline)) {
            constexpr int p = decltype(P)::value;
            step(IC<p>{}, IC<(p < 2)>{}, IC<0>{}, p);
        });
        for (int i0 = 8; i0 < nk - 8; i0 += 8) {
            static_for<0, 8>([&](auto P) __attribute__((always_inline)) {
                constexpr int p = decltype(P)::value;
                step(IC<p>{}, IC<0>{}, IC<0>{}, i0 + p);
            });
        }
        static_for<0, 8>([&](auto P) __attribute__((always_inline)) {
            constexpr int p = decltype(P)::value;
            step(IC<p>{}, IC<0>{}, IC<(p >= 8 - kPDg)>{}, nk - 8 + p);
        });
        epilogue();
        if (nxt < 0) break;
        cur = nxt;
        m0 = nm0;
        n0 = nn0;
        sa_cur = sa_nxt;
        sw_cur = sw_nxt;
        jt++;
    }
    __builtin_amdgcn_s_waitcnt(0);
}

template <int EP, int TB>
void launch_groups(const GemmArgs &a, const StreamGeom &g, int grid, bool bias, hipStream_t st) {
    if (bias)
        tgemm_stream_groups_kernel<EP, true, TB><<<grid, 256, 0, st>>>(a, g);
    else
        tgemm_stream_groups_kernel<EP, false, TB><<<grid, 256, 0, st>>>(a, g);
}

template <int TB>
void launch_groups_ep(const GemmArgs &a, const StreamGeom &g, int grid, bool bias, hipStream_t st) {
    if (a.ep == VX_EP_SILU)
        launch_groups<VX_EP_SILU, TB>(a, g, grid, bias, st);
    else if (a.ep == VX_EP_ADD_SCALED)
        launch_groups<VX_EP_ADD_SCALED, TB>(a, g, grid, bias, st);
    else
        launch_groups<VX_EP_STORE, TB>(a, g, grid, bias, st);
}

}  // namespace

bool gemm_stream_groups(const GemmArgs &a, int tokens_full, hipStream_t st) {
    const int64_t nk = a.inp / 64;
    if (a.spg != 2 || a.ng < 2 || a.gs != nullptr || a.y_bytes == 0) return false;  // 128-column groups
    if (a.inp % 512 != 0 || nk < 16) return false;
    if (a.out % kBN != 0 || a.r0 != 0 || a.r1 != a.out || a.t0 != 0 || tokens_full % kBM != 0) return false;
    const int forced = overrides().gemm.load(std::memory_order_relaxed);
    if (forced != kForceNone && forced != kForceStream) return false;
    // 64-token tiles with two workgroups per CU (at 8192 tokens: FFN-up 76 -> 65 us, FFN-down 64 -> 53 us against
    // 128-token tiles with one), or 128-token tiles ("stream_tile" override: 4 or 8 token blocks per wavefront)
    int tb = 4;
    const int ft = overrides().stream_tb.load(std::memory_order_relaxed);
    if (ft == 4 || ft == 8) tb = ft;
    const int bm = 16 * tb;
    StreamGeom g;
    g.n_nt = (int)(a.out / kBN);
    g.ntiles = (tokens_full / bm) * g.n_nt;
    g.per_xcd = (g.ntiles + 7) / 8;
    g.nk = (int)nk;
    g.ng = (int)a.ng;
    const int cus = cu_count(), wpc = tb == 4 ? 2 : 1;  // workgroups per CU
    // too few tiles of this kernel's height. Above 1024 tokens (no small-token kernel) a quarter of the CUs is
    // enough: at 1500 / 4000 tokens and 1024 outputs its 88 / 248 tiles beat the LDS-staged kernel (o-proj 19.7 /
    // 22.5 -> 17.3 / 19.0 us, FFN-down 49.9 / 54.3 -> 44.1 / 47.6 us)
    if (g.ntiles < (a.t1 > 1024 ? cus / 4 : cus / 2) && forced == kForceNone) return false;
    int per_x = std::min(wpc * cus / 8, g.per_xcd);
    const int fg = overrides().stream_grid.load(std::memory_order_relaxed);  // workgroups: tests and tuning
    if (fg >= 8) per_x = std::min(fg / 8, g.per_xcd);
    const int grid = 8 * per_x;
    GemmArgs b = a;
    b.t1 = tokens_full;
    const bool bias = a.bias != nullptr;
    if (tb == 4)
        launch_groups_ep<4>(b, g, grid, bias, st);
    else
        launch_groups_ep<8>(b, g, grid, bias, st);
    hip_check(hipGetLastError(), "tgemm_stream_groups launch");
    return true;
}

}  // namespace vx
