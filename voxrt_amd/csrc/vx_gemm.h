// vx_gemm.h — GEMM launch arguments and operand helpers shared by the GEMM kernels (vx_gemm.hip,
// vx_gemm_stream.hip, vx_gemm_stream_g.hip, vx_gemm_small.hip).
#pragma once

#include <atomic>
#include <type_traits>

#include "vx_internal.h"

namespace vx {

struct GemmArgs {
    const void *w;          // ternary: uint32 codes; int8: 16-byte chunks (see TMat)
    const float *ws_t;      // [ng][out_pad]
    const int8_t *xq;       // [n][inp]
    const float *xs;        // scales_t [ng][np]
    const int32_t *xg;      // gsum_t [ng][np] (ternary only)
    float *y;               // [n][out]
    const float *bias;      // [out] or NULL
    int32_t *gs;            // [ng][n][out] or NULL
    int64_t n, np, out, inp, ng, out_pad, spg;
    int64_t r0, r1, t0, t1, n_base, m_base;
    uint32_t w_bytes, ws_bytes, xq_bytes, xs_bytes, y_bytes;
    int ep;
    float alpha;
    int vec_ok;  // y (and bias) rows are 16-byte aligned: out % 4 == 0 and 16-byte aligned base pointers
    // quantized output (the next GEMM's activations, 128-column groups): codes [n][out], scales_t and gsum_t
    // [out/128][np]; NULL qo: y is written
    int8_t *qo;
    float *qs;
    int32_t *qg;
};

__device__ inline v4i widen_codes(uint32_t p) {
    v4i r;
    r.x = (int)(p & 0x03030303u);
    r.y = (int)((p >> 2) & 0x03030303u);
    r.z = (int)((p >> 4) & 0x03030303u);
    r.w = (int)((p >> 6) & 0x03030303u);
    return r;
}

// --- streaming large-token kernels (vx_gemm_stream.hip: one group; vx_gemm_stream_g.hip: 128-column groups) ---

constexpr int kBM = 128, kBN = 256;  // workgroup tile: tokens x output rows
constexpr uint32_t kOff = 0xFFFFFFF0u;

struct StreamGeom {
    int n_nt;     // tiles along the output rows
    int ntiles;   // tiles in all
    int per_xcd;  // tiles per XCD (a contiguous range of the tile order)
    int nk;       // 64-column K steps (a multiple of 8, at least 16)
    int ng;       // groups
};

// s_waitcnt immediate on gfx9: vmcnt in bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left unwaited.
constexpr int waitcnt_vm(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int I>
using IC = std::integral_constant<int, I>;

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(IC<B>{});
        static_for<B + 1, E>(f);
    }
}

// Kernel choices forced by vx_set_kernel_override (tests and tuning; nothing is forced by default and no environment
// variable is read): the GEMM kernel family, the tile of the split-K / direct / LDS kernels and of the small-token
// kernel (16 * mt tokens x 16 * nt rows, encoded mt * 16 + nt), and the streaming kernels' grid (workgroups).
enum ForcedKernel { kForceNone, kForceDirect, kForceSplitK, kForceLds, kForceBig, kForceSplitG, kForceSmall, kForceStream };
struct KernelOverrides {
    std::atomic<int> gemm{kForceNone}, tile{0}, small_tile{0}, stream_grid{0};
    std::atomic<int> small_ws{0};  // grouped small-token kernel with producer/consumer wavefronts: 0 auto, 1 on, 2 off
    std::atomic<int> stream_tb{0}; // 128-column-group streaming kernel: token blocks per wavefront (4 or 8), 0 auto
    std::atomic<int> linear{0};    // f32 linear: 0 auto, -1 the LDS-broadcast kernel, 1WT*10+WO the matrix-core
                                   // kernel with WT x WO blocks per wavefront (111, 121, 122)
};
KernelOverrides &overrides();

// The streaming kernels run the GEMM and return true when the shape and window fit them (whole 128-token x
// 256-row tiles of a full-width ternary GEMM), else return false and launch nothing.
bool gemm_stream(const GemmArgs &a, int tokens_full, hipStream_t st);
bool gemm_stream_groups(const GemmArgs &a, int tokens_full, hipStream_t st);
int cu_count();  // compute units of the current device

// The small-token kernel (vx_gemm_small.hip): one or two rounds of workgroups for a whole-width ternary GEMM of a
// few hundred tokens. Returns false and launches nothing when the shape or window does not fit it.
bool gemm_small(const GemmArgs &a, hipStream_t st);

}  // namespace vx
