// vx_gemm_stream.hip — persistent large-token ternary x int8 GEMM (one group, G = K) on gfx950 i8 MFMA, bit-exact
// to voxrt's scalar kernel (crates/voxrt/src/kernels/mod.rs:166-210): y[t, o] = ep(fma((float)S, xs[t] * ws[o], 0)).
//
// One workgroup of 4 wavefronts per CU (two per CU for the SiLU epilogue with K = 1024, each with half the LDS ring)
// walks a sequence of 128-token x 256-row output tiles; wavefront w owns the tile's rows [64w, 64w + 64). The tiles of XCD x (workgroup b runs on XCD b % 8) are a contiguous range of the
// row-major tile order, so the workgroups of one XCD work on the same token rows at the same time and its L2 cache
// serves their activation tiles and the weight plane.
//
// Operands of v_mfma_i32_16x16x64_i8 (wave64): A = weights (rows = output rows), B = activations (columns = tokens).
// Lane l supplies output row l%16 (one dword of 2-bit codes widened to 16 int8 codes, straight from the weight
// layout) and token l%16 (16 bytes from LDS), both over K columns 16*(l/16) .. +15 of the 64-column step. D element
// e of lane l is output 4*(l/16) + e of token l%16: four consecutive outputs of one token, stored with one 16-byte
// store, and 16 lanes write 16 token rows x 64 contiguous bytes.
//
// Ternary trick: the codes are trit + 1 in {0, 1, 2}; the accumulator ends at S + sum(x codes of the token) and the
// epilogue subtracts the quantizer's gsum, which is exact in int32.
//
// Pipeline, per 64-column K step s (the steps of all tiles of the workgroup form one stream, so the loads of the
// next tile's first steps are in flight while a tile finishes):
//   * the 128 x 64 activation tile and the weight codes of step s + 6 reach LDS by buffer_load ... lds (8 slots):
//     activations 16 rows x 64 contiguous bytes per instruction, chunk c of row i at position c ^ ((i >> 2) & 3), so
//     a 16-lane fragment read touches all 64 banks once; weight codes one instruction per wavefront (its four
//     256-byte blocks), read back one dword per lane and block and widened to int8 one step ahead of use;
//   * one explicit vmcnt wait and one barrier per step. Every step issues the same vector-memory instructions in
//     the same order (dummy stores and loads, whose offsets lie past the buffer end, keep the count fixed), so the
//     wait count is a constant of the step's position in the tile;
//   * within a step: the LDS reads that its VALU work waits for (epilogue scales, next step's weight codes) come
//     first, two rows of MFMAs run while the step's loads issue, and the next step's fragment reads and the VALU
//     work are interleaved with the remaining MFMAs;
//   * Store with K = 1024: two accumulator sets alternate between tiles; while the MFMAs of tile j accumulate into
//     one, the epilogue of tile j - 1 (subtract gsum, fold fma((float)S, xs * ws, 0), bias) is computed from the
//     other, two output blocks per step over the first 16 steps, and its 16-byte stores leave between the MFMAs, so
//     the f32 output stream overlaps the next tile's MFMA work. SiLU, AddScaled (which reads y) and K > 1024 use
//     one accumulator set and write each tile's epilogue after its last step (measured faster for those).
// Token scales, gsum, weight scales and bias of a tile are brought to LDS by DMA six steps before the tile ends.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <utility>

#include "vx_gemm.h"

namespace vx {
namespace {

// Two workgroups per CU (two wavefronts per SIMD) for the SiLU epilogue with K = 1024: its epilogue's VALU work
// (about 24 instructions per output) then overlaps the other workgroup's MFMAs. Measured at 8192 tokens: FFN-up
// SiLU 62.7-64.5 -> 53.4-56.7 us; the Store epilogue (40 -> 46 us) and K = 4096 (35 -> 42 us) are slower so.
constexpr bool occ2_of(int ep, bool k16) { return ep == VX_EP_SILU && k16; }

// Loads run kPD steps ahead of use. When step s begins, the loads of step s+1 (the first instructions of step
// s+1-kPD) must be complete: the vector-memory instructions issued after them are 2 stores of that step and 5 per
// later step (3 DMA + 2 stores), plus the 4 scale DMAs issued after the loads of tile step nk-kPD.
constexpr int kEarly = 2;  // token rows of MFMAs issued before a step's loads (the matrix pipe stays busy)
constexpr int kValuPerDs = 2;    // VALU instructions placed beside each fragment read (with its MFMA)
constexpr int kValuPerMfma = 3;  // VALU instructions after each remaining MFMA (one MFMA is 16 cycles)
__device__ constexpr int wait_of(int pd, int i, int nk) { return 2 + 5 * (pd - 2) + ((i >= nk - pd + 1) ? 4 : 0); }

template <int EP, bool BIAS, bool K16, bool OCC2, bool GSO>
__global__ __launch_bounds__(256, OCC2 ? 2 : 1) void tgemm_stream_kernel(const GemmArgs a, const StreamGeom g) {
    // GSO: the exact int32 sums S are stored too, to the group-sum buffer [1][n][out] (Store epilogue; each tile's
    // epilogue after its last step)
    static_assert(!GSO || (EP == VX_EP_STORE && !OCC2), "group sums: Store epilogue");
    // OCC2: two workgroups per CU (two wavefronts per SIMD), each with half the LDS ring and one accumulator set, so
    // that one workgroup's epilogue, waits and barriers overlap the other's MFMAs
    constexpr int kPD = OCC2 ? 3 : 6;  // steps the loads run ahead
    constexpr int NS = OCC2 ? 4 : 8;   // LDS slots
    // DRAIN: every tile's epilogue after its last step, one accumulator set. Measured at 8192 tokens: faster for
    // SiLU (its VALU work made the steps of the next tile VALU-bound: 67 -> 62 us for FFN-up) and for K > 1024
    // (FFN-down 32.7 -> 31.4 us); the Store epilogue with K = 1024 keeps the two-blocks-per-step overlap
    // (40 us against 43).
    constexpr bool DRAIN = OCC2 || GSO || EP != VX_EP_STORE || !K16;
    typedef __attribute__((address_space(3))) void lds_void;
    // one LDS object per activation slot and per scale table: the compiler then sees that a DMA into one slot
    // does not alias the fragment reads of another and adds no vmcnt wait of its own before them
    __shared__ __attribute__((aligned(1024))) int8_t sa0[8192], sa1[8192], sa2[8192], sa3[8192], sa4[8192],
        sa5[8192], sa6[8192], sa7[8192];
    // weight codes of a step: per wave 4 blocks of 16 rows x 64 columns (256 bytes each)
    __shared__ __attribute__((aligned(1024))) uint32_t sw0[1024], sw1[1024], sw2[1024], sw3[1024], sw4[1024],
        sw5[1024], sw6[1024], sw7[1024];
    // per tile parity: token scales, gsum, weight scales, bias (256 entries each)
    __shared__ __attribute__((aligned(16))) float xs0[256], xs1[256], gs0[256], gs1[256], ws0[256], ws1[256],
        bi0[256], bi1[256];
    auto sact = [&](int i) -> int8_t * {
        if constexpr (NS == 4) return i == 0 ? sa0 : i == 1 ? sa1 : i == 2 ? sa2 : sa3;
        return i == 0 ? sa0 : i == 1 ? sa1 : i == 2 ? sa2 : i == 3 ? sa3 : i == 4 ? sa4 : i == 5 ? sa5 : i == 6 ? sa6 : sa7;
    };
    auto swt = [&](int i) -> uint32_t * {
        if constexpr (NS == 4) return i == 0 ? sw0 : i == 1 ? sw1 : i == 2 ? sw2 : sw3;
        return i == 0 ? sw0 : i == 1 ? sw1 : i == 2 ? sw2 : i == 3 ? sw3 : i == 4 ? sw4 : i == 5 ? sw5 : i == 6 ? sw6 : sw7;
    };
    auto ssc = [&](int par, int kind) -> float * {
        return kind == 0 ? (par ? xs1 : xs0) : kind == 1 ? (par ? gs1 : gs0) : kind == 2 ? (par ? ws1 : ws0)
                                                                              : (par ? bi1 : bi0);
    };

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lq = lane >> 4;
    const int inp = (int)a.inp, nk = g.nk;
    const uint32_t out4 = (uint32_t)a.out * 4;

    const int xcd = blockIdx.x & 7, wi = blockIdx.x >> 3, nwx = gridDim.x >> 3;
    auto tile_at = [&](int j) -> int {
        const int s = wi + j * nwx, t = xcd * g.per_xcd + s;
        return (s < g.per_xcd && t < g.ntiles) ? t : -1;
    };

    const auto xrs = make_rsrc(a.xq, a.xq_bytes);
    const auto wrs = make_rsrc(a.w, a.w_bytes);
    const auto srs = make_rsrc(a.xs, a.xs_bytes);
    const auto grs = make_rsrc(a.xg, a.xs_bytes);
    const auto wsrs = make_rsrc(a.ws_t, a.ws_bytes);
    const auto brs = make_rsrc(a.bias, BIAS ? (uint32_t)(a.out * 4) : 0u);
    const auto yrs = make_rsrc(a.y, a.y_bytes);
    const auto gsrs = make_rsrc(a.gs, GSO ? a.y_bytes : 0u);

    // activation DMA: this wave fills token blocks 2w, 2w+1 of the tile; lane l -> row l/4 of the block, LDS
    // position l%4, global chunk (l%4) ^ ((row >> 2) & 3). The tile's token base travels in the scalar offset
    // (whole tiles only, so every row exists).
    uint32_t vdma[2];
    {
        const int i = lane >> 2, c = (lane & 3) ^ ((i >> 2) & 3);
#pragma unroll
        for (int q = 0; q < 2; q++) vdma[q] = (uint32_t)(((2 * wave + q) * 16 + i) * inp + c * 16);
    }
    // fragment read: token l%16 of a 16-token block, K chunk l/16 at its swizzled position
    const uint32_t vfr = (uint32_t)(l16 * 64 + ((lq ^ ((l16 >> 2) & 3)) * 16));
    // weight DMA: lane l fetches 16 bytes of block l/16 of the wave's four 16 x 64 blocks of a step
    const uint32_t vwd = (uint32_t)((lane >> 4) * nk * 256 + (lane & 15) * 16);
    const uint32_t vyl = (uint32_t)l16 * out4 + (uint32_t)lq * 16;

    // --- tile state -----------------------------------------------------------------------------------------
    int jt = 0;
    int cur = tile_at(0);
    if (cur < 0) return;  // a workgroup of the last XCD past its last tile
    auto mt_of = [&](int t) { return t / g.n_nt; };
    auto nt_of = [&](int t) { return t % g.n_nt; };
    int m0 = mt_of(cur) * kBM, n0 = nt_of(cur) * kBN;
    // scalar offsets of the current and the next tile
    uint32_t sa_cur = (uint32_t)m0 * inp, sw_cur = (uint32_t)((n0 / 16 + wave * 4) * nk) * 256;
    uint32_t sa_nxt = 0, sw_nxt = 0, vdma_nxt[2] = {kOff, kOff}, vw_nxt = kOff;
    int nxt = -1, nm0 = 0, nn0 = 0;
    auto set_next = [&]() {
        nxt = tile_at(jt + 1);
        const bool has = nxt >= 0;
        nm0 = has ? mt_of(nxt) * kBM : 0;
        nn0 = has ? nt_of(nxt) * kBN : 0;
        sa_nxt = (uint32_t)nm0 * inp;
        sw_nxt = (uint32_t)((nn0 / 16 + wave * 4) * nk) * 256;
        vdma_nxt[0] = has ? vdma[0] : kOff;
        vdma_nxt[1] = has ? vdma[1] : kOff;
        vw_nxt = has ? vwd : kOff;
    };
    // pending tile (its epilogue runs during the current tile)
    uint32_t sy_p = 0, vy_p = kOff;

    // the loads of one step: its activation tile (two DMA per wave) and this wave's weight codes (one DMA)
    auto dma = [&](int slot, int kb, const uint32_t (&vd)[2], uint32_t sa, uint32_t vw, uint32_t sw) {
#pragma unroll
        for (int q = 0; q < 2; q++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_void *)(sact(slot) + (2 * wave + q) * 1024), 16,
                                                     vd[q], sa + (uint32_t)kb * 64, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void *)(swt(slot) + wave * 256), 16, vw,
                                                 sw + (uint32_t)kb * 256, 0, 0);
    };
    // scales of the current tile to LDS parity `par`: 256 floats each (token scales and gsum of tokens
    // m0 .. m0+255, of which 128 are used; weight scales and bias of rows n0 .. n0+255)
    auto scale_dma = [&](int par, bool live) {
        const uint32_t vt = live ? (uint32_t)m0 * 4 + (uint32_t)lane * 16 : kOff;
        const uint32_t vo = live ? (uint32_t)n0 * 4 + (uint32_t)lane * 16 : kOff;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (lds_void *)ssc(par, 0), 16, vt, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(grs, (lds_void *)ssc(par, 1), 16, vt, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wsrs, (lds_void *)ssc(par, 2), 16, vo, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (lds_void *)ssc(par, 3), 16, BIAS ? vo : kOff, 0, 0, 0);
    };
    constexpr int NFS = OCC2 ? 1 : 2;  // fragment sets: OCC2 reads the next step's fragment of a token block
                                       // into the registers its last MFMA of this step has just read
    v4i fr[NFS][8];
    uint32_t rw[4];
    auto read_frags = [&](int slot, int set) {
#pragma unroll
        for (int tb = 0; tb < 8; tb++) fr[set % NFS][tb] = *(const v4i *)(sact(slot) + tb * 1024 + vfr);
    };
    auto read_weights = [&](int slot) {
#pragma unroll
        for (int ob = 0; ob < 4; ob++) rw[ob] = swt(slot)[wave * 256 + ob * 64 + lane];
    };
    v4i bw[2][4];  // widened weight operands of this step and the next
    auto widen = [&](int set) {
#pragma unroll
        for (int ob = 0; ob < 4; ob++) bw[set][ob] = widen_codes(rw[ob]);
    };

    // epilogue of output block (tb, ob) of a tile whose accumulators are `acc` and scales are in LDS parity
    // `par`: 4 consecutive outputs of one token per lane, one 16-byte store (dropped when vy is past the end).
    // The LDS reads (block_scales) come first, so that the VALU work waits only for them.
    struct BlockScales {
        float xs;
        int gsum;
        float4 ws, bia;
    };
    auto block_scales = [&](int par, int tb, int ob) {
        BlockScales c;
        c.xs = ssc(par, 0)[tb * 16 + l16];
        c.gsum = __float_as_int(ssc(par, 1)[tb * 16 + l16]);
        c.ws = *(const float4 *)&ssc(par, 2)[wave * 64 + ob * 16 + lq * 4];
        c.bia = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (BIAS) c.bia = *(const float4 *)&ssc(par, 3)[wave * 64 + ob * 16 + lq * 4];
        return c;
    };
    // Two stores that write nothing (offsets past the buffer end) where a step has no output blocks to store, so
    // that every step issues the same vector-memory instructions. Their offsets differ: two identical stores would
    // be merged into one by the compiler, and the wait counts, which assume two, would no longer cover the loads.
    auto dummy_stores = [&]() {
        const v4i z{0, 0, 0, 0};
        store_b128_sep(z, yrs, kOff, 0);
        store_b128_sep(z, yrs, kOff - 16, 0);
    };
    auto out_block = [&](const v4i (&acc)[8][4], const BlockScales &c, int tb, int ob, uint32_t vy, uint32_t sy) {
        const float xs = c.xs;
        const int gsum = c.gsum;
        const float4 ws = c.ws, bia = c.bia;
        const uint32_t so = sy + (uint32_t)(tb * 16) * out4 + (uint32_t)(ob * 64);
        float4 old = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (EP == VX_EP_ADD_SCALED) {
            const v4i o4 = __builtin_amdgcn_raw_buffer_load_b128(yrs, vy, so, 0);
            old = make_float4(__int_as_float(o4[0]), __int_as_float(o4[1]), __int_as_float(o4[2]),
                              __int_as_float(o4[3]));
        }
        const float wsv[4] = {ws.x, ws.y, ws.z, ws.w}, bv[4] = {bia.x, bia.y, bia.z, bia.w},
                    ov[4] = {old.x, old.y, old.z, old.w};
        v4i r, sums;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            sums[e] = acc[tb][ob][e] - gsum;
            const float v = __builtin_fmaf((float)sums[e], xs * wsv[e], 0.0f);
            float res = v;
            if constexpr (EP == VX_EP_SILU) res = silu_fast(v);
            if constexpr (EP == VX_EP_ADD_SCALED) res = __builtin_fmaf(a.alpha, v, ov[e]);
            if constexpr (BIAS) res = res + bv[e];
            r[e] = __float_as_int(res);
        }
        store_b128_sep(r, yrs, vy, so);
        if constexpr (GSO) store_b128_sep(sums, gsrs, vy, so);
    };

    // one K step. i: tile step (runtime in the middle loop); SLOT = i % 8 (LDS slot);
    // CH: output-block pair of the pending tile stored in this step (-1: two dummy stores); NEXT: the loads of
    // this step are the next tile's steps I+4-nk; SCALE: this is step nk-4 (the tile's scales go to LDS)
    auto step = [&](auto Wc, auto SLOTc, auto CHc, auto NEXTc, auto SCALEc, auto PARc, int i, v4i(&acc)[8][4],
                    const v4i(&accp)[8][4]) {
        constexpr int W = decltype(Wc)::value, SLOT = decltype(SLOTc)::value, CH = decltype(CHc)::value;
        constexpr bool NEXT = decltype(NEXTc)::value != 0, SCALE = decltype(SCALEc)::value != 0;
        constexpr int PAR = decltype(PARc)::value;
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(W));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // LDS reads that this step's VALU work waits for: the pending block pair's scales, next step's weights
        constexpr bool CHUNK = CH >= 0 && !DRAIN;
        BlockScales sc0, sc1;
        if constexpr (CHUNK) {
            sc0 = block_scales(PAR ^ 1, CH / 2, 2 * (CH % 2));
            sc1 = block_scales(PAR ^ 1, CH / 2, 2 * (CH % 2) + 1);
        }
        read_weights((SLOT + 1) % NS);
        constexpr int fs = SLOT & 1;
        auto mfma_row = [&](int tb) {
#pragma unroll
            for (int ob = 0; ob < 4; ob++) {
                if constexpr (CH == 0)  // tile step 0: the chains start from zero
                    acc[tb][ob] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[fs][ob], fr[fs % NFS][tb], v4i{0, 0, 0, 0}, 0, 0, 0);
                else
                    acc[tb][ob] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[fs][ob], fr[fs % NFS][tb], acc[tb][ob], 0, 0, 0);
            }
        };
        // the first kEarly token rows of MFMAs go before this step's loads, so that the matrix pipe is busy while
        // the loads issue
        static_for<0, kEarly>([&](auto T) { mfma_row(decltype(T)::value); });
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NEXT)
            dma((SLOT + kPD) % NS, i + kPD - nk, vdma_nxt, sa_nxt, vw_nxt, sw_nxt);
        else
            dma((SLOT + kPD) % NS, i + kPD, vdma, sa_cur, vwd, sw_cur);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (SCALE) scale_dma(PAR, true);
        read_frags((SLOT + 1) % NS, (SLOT + 1) & 1);
        static_for<kEarly, 8>([&](auto T) { mfma_row(decltype(T)::value); });
        if constexpr (CHUNK) {
            out_block(accp, sc0, CH / 2, 2 * (CH % 2), vy_p, sy_p);
            out_block(accp, sc1, CH / 2, 2 * (CH % 2) + 1, vy_p, sy_p);
        } else {
            dummy_stores();
        }
        widen(fs ^ 1);
        // issue order: the 8 fragment reads of the next step each after an MFMA with 2 VALU, then 3 VALU after
        // each of the remaining MFMAs (epilogue and widening work hides under the matrix pipe)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, kValuPerDs, 0);
        }
#pragma unroll
        for (int k = 0; k < 24 - 4 * kEarly; k++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // OCC2 step: the same loads, one fragment set. After the four MFMAs of token block tb, the next step's fragment
    // of tb is read into the same registers; the next step's weights are widened beside the MFMAs.
    auto step2 = [&](auto Wc, auto SLOTc, auto CHc, auto NEXTc, auto SCALEc, auto PARc, int i, v4i(&acc)[8][4]) {
        constexpr int W = decltype(Wc)::value, SLOT = decltype(SLOTc)::value, CH = decltype(CHc)::value;
        constexpr bool NEXT = decltype(NEXTc)::value != 0, SCALE = decltype(SCALEc)::value != 0;
        constexpr int PAR = decltype(PARc)::value;
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(W));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        read_weights((SLOT + 1) % NS);
        constexpr int fs = SLOT & 1;
        constexpr int nslot = (SLOT + 1) % NS;
        auto mfma_row = [&](int tb) {
#pragma unroll
            for (int ob = 0; ob < 4; ob++) {
                if constexpr (CH == 0)
                    acc[tb][ob] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[fs][ob], fr[0][tb], v4i{0, 0, 0, 0}, 0, 0, 0);
                else
                    acc[tb][ob] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bw[fs][ob], fr[0][tb], acc[tb][ob], 0, 0, 0);
            }
            fr[0][tb] = *(const v4i *)(sact(nslot) + tb * 1024 + vfr);
        };
        static_for<0, kEarly>([&](auto T) { mfma_row(decltype(T)::value); });
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NEXT)
            dma((SLOT + kPD) % NS, i + kPD - nk, vdma_nxt, sa_nxt, vw_nxt, sw_nxt);
        else
            dma((SLOT + kPD) % NS, i + kPD, vdma, sa_cur, vwd, sw_cur);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (SCALE) scale_dma(PAR, true);
        dummy_stores();
        __builtin_amdgcn_sched_barrier(0);
        static_for<kEarly, 8>([&](auto T) { mfma_row(decltype(T)::value); });
        widen(fs ^ 1);
#pragma unroll
        for (int k = 0; k < 4 * (8 - kEarly); k++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // whole epilogue of a tile at once (after its last step): AddScaled tiles, and the last tile of the sequence
    auto drain = [&](auto PARc, const v4i(&acc)[8][4]) {
        constexpr int PAR = decltype(PARc)::value;
        // the tile's scale DMAs (step nk-kPD) are complete once the later vector-memory instructions may pend
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 + 5 * (kPD - 1)));
        __builtin_amdgcn_s_barrier();
        const uint32_t sy = (uint32_t)m0 * out4 + (uint32_t)(n0 + wave * 64) * 4;
#pragma unroll
        for (int tb = 0; tb < 8; tb++)
#pragma unroll
            for (int ob = 0; ob < 4; ob++) {
                out_block(acc, block_scales(PAR, tb, ob), tb, ob, vyl, sy);
                if constexpr (OCC2) __builtin_amdgcn_sched_barrier(0);  // one block's registers at a time
            }
    };

    auto stepx = [&](auto Wc, auto SLOTc, auto CHc, auto NEXTc, auto SCALEc, auto PARc, int i, v4i(&acc)[8][4],
                     const v4i(&accp)[8][4]) {
        if constexpr (OCC2)
            step2(Wc, SLOTc, CHc, NEXTc, SCALEc, PARc, i, acc);
        else
            step(Wc, SLOTc, CHc, NEXTc, SCALEc, PARc, i, acc, accp);
    };

    // one tile: steps 0..nk-1 into `acc` (tile parity PAR), the pending tile's epilogue from `accp`
    auto run_tile = [&](auto PARc, v4i(&acc)[8][4], const v4i(&accp)[8][4]) {
        constexpr int PAR = decltype(PARc)::value;
        set_next();
        if constexpr (K16) {
            static_for<0, 16>([&](auto I) {
                constexpr int i = decltype(I)::value;
                stepx(IC<wait_of(kPD, i, 16)>{}, IC<i % NS>{}, IC<i>{}, IC<(i >= 16 - kPD)>{}, IC<i == 16 - kPD>{},
                      IC<PAR>{}, i, acc, accp);
            });
        } else {
            static_for<0, 16>([&](auto I) {
                constexpr int i = decltype(I)::value;
                stepx(IC<wait_of(kPD, 0, 64)>{}, IC<i % NS>{}, IC<i>{}, IC<0>{}, IC<0>{}, IC<PAR>{}, i, acc, accp);
            });
            // steps 16 .. nk-9 in groups of 8 (slot positions stay compile-time: nk % 8 == 0)
            for (int i0 = 16; i0 < nk - 8; i0 += 8) {
                static_for<0, 8>([&](auto P) {
                    constexpr int p = decltype(P)::value;
                    stepx(IC<wait_of(kPD, 0, 64)>{}, IC<p % NS>{}, IC<-1>{}, IC<0>{}, IC<0>{}, IC<PAR>{}, i0 + p, acc,
                          accp);
                });
            }
            static_for<0, 8>([&](auto P) {
                constexpr int p = decltype(P)::value;
                stepx(IC<wait_of(kPD, 56 + p, 64)>{}, IC<p % NS>{}, IC<-1>{}, IC<(p >= 8 - kPD)>{}, IC<p == 8 - kPD>{},
                      IC<PAR>{}, nk - 8 + p, acc, accp);
            });
        }
        // this tile becomes the pending one (or is written now: AddScaled, or the last tile)
        if (DRAIN || nxt < 0) {
            drain(IC<PAR>{}, acc);
            vy_p = kOff;
        } else {
            vy_p = vyl;
            sy_p = (uint32_t)m0 * out4 + (uint32_t)(n0 + wave * 64) * 4;
        }
        cur = nxt;
        m0 = nm0;
        n0 = nn0;
        sa_cur = sa_nxt;
        sw_cur = sw_nxt;
        jt++;
    };

    // prologue: the instruction pattern of tile steps nk-4 .. nk-1 of a virtual previous tile (dummy scale DMAs
    // and stores), loading steps 0..3 of the first tile
    {
#pragma unroll
        for (int i = 0; i < kPD; i++) {
            dma(i, i, vdma, sa_cur, vwd, sw_cur);
            __builtin_amdgcn_sched_barrier(0);
            if (i == 0) scale_dma(1, false);
            dummy_stores();
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 + 2 + 5 * (kPD - 1)));  // the loads of step 0 complete
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        read_frags(0, 0);
        read_weights(0);
        widen(0);
    }

    v4i acc0[8][4], acc1[8][4];
    for (;;) {
        run_tile(IC<0>{}, acc0, acc1);
        if (cur < 0) break;
        if constexpr (DRAIN)
            run_tile(IC<1>{}, acc0, acc1);
        else
            run_tile(IC<1>{}, acc1, acc0);
        if (cur < 0) break;
    }
    __builtin_amdgcn_s_waitcnt(0);
}

template <int EP, bool BIAS>
void launch_stream(const GemmArgs &a, const StreamGeom &g, int grid, hipStream_t st) {
    if constexpr (EP == VX_EP_STORE) {
        if (a.gs) {
            if (g.nk == 16)
                tgemm_stream_kernel<EP, BIAS, true, false, true><<<grid, 256, 0, st>>>(a, g);
            else
                tgemm_stream_kernel<EP, BIAS, false, false, true><<<grid, 256, 0, st>>>(a, g);
            return;
        }
    }
    if (g.nk == 16)
        tgemm_stream_kernel<EP, BIAS, true, occ2_of(EP, true), false><<<grid, 256, 0, st>>>(a, g);
    else
        tgemm_stream_kernel<EP, BIAS, false, occ2_of(EP, false), false><<<grid, 256, 0, st>>>(a, g);
}

}  // namespace

// CU count of the current device, cached per device (a host thread may switch devices between calls)
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    const bool cached = dev >= 0 && dev < 64;
    int n = cached ? cache[dev].load(std::memory_order_relaxed) : 0;
    if (n == 0) {
        int c = 0;
        hip_check(hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
        n = c > 0 ? c : 256;
        if (cached) cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

bool gemm_stream(const GemmArgs &a, int tokens_full, hipStream_t st) {
    const int64_t nk = a.inp / 64;
    if (a.ng != 1 || (a.gs != nullptr && a.ep != VX_EP_STORE) || a.y_bytes == 0) return false;
    if (a.inp % 64 != 0 || nk < 16 || nk % 8 != 0 || (nk != 16 && nk < 24)) return false;
    if (a.out % kBN != 0 || a.r0 != 0 || a.r1 != a.out || a.t0 != 0 || tokens_full % kBM != 0) return false;
    const int forced = overrides().gemm.load(std::memory_order_relaxed);
    if (forced != kForceNone && forced != kForceStream) return false;
    StreamGeom g;
    g.n_nt = (int)(a.out / kBN);
    g.ntiles = (tokens_full / kBM) * g.n_nt;
    g.per_xcd = (g.ntiles + 7) / 8;
    g.nk = (int)nk;
    g.ng = 1;
    const int cus = cu_count();
    if (g.ntiles < cus && forced == kForceNone) return false;  // too few tiles to fill the chip: the other kernels
    int per_x = std::min((occ2_of(a.ep, nk == 16) && !a.gs ? 2 : 1) * cus / 8, g.per_xcd);
    const int fg = overrides().stream_grid.load(std::memory_order_relaxed);  // workgroups: tests and tuning
    if (fg >= 8) per_x = std::min(fg / 8, g.per_xcd);
    const int grid = 8 * per_x;
    // XCD x's workgroup i starts at tile x*per_xcd + i; on the last XCD that tile may not exist (fewer tiles), and
    // such a workgroup returns at once
    GemmArgs b = a;
    b.t1 = tokens_full;
    const bool bias = a.bias != nullptr;
    switch (a.ep) {
        case VX_EP_SILU:
            bias ? launch_stream<VX_EP_SILU, true>(b, g, grid, st) : launch_stream<VX_EP_SILU, false>(b, g, grid, st);
            break;
        case VX_EP_ADD_SCALED:
            bias ? launch_stream<VX_EP_ADD_SCALED, true>(b, g, grid, st)
                 : launch_stream<VX_EP_ADD_SCALED, false>(b, g, grid, st);
            break;
        default:
            bias ? launch_stream<VX_EP_STORE, true>(b, g, grid, st) : launch_stream<VX_EP_STORE, false>(b, g, grid, st);
    }
    hip_check(hipGetLastError(), "tgemm_stream launch");
    return true;
}

}  // namespace vx
