// vx_gemm.h — GEMM launch arguments and operand helpers shared by the GEMM kernels (vx_gemm.hip,
// vx_gemm_stream.hip).
#pragma once

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
};

__device__ inline v4i widen_codes(uint32_t p) {
    v4i r;
    r.x = (int)(p & 0x03030303u);
    r.y = (int)((p >> 2) & 0x03030303u);
    r.z = (int)((p >> 4) & 0x03030303u);
    r.w = (int)((p >> 6) & 0x03030303u);
    return r;
}

// Streaming large-token kernel (vx_gemm_stream.hip): runs the GEMM and returns true when the shape and window
// fit it (whole 128-token x 256-row tiles, one group, ternary weights), else returns false and launches nothing.
bool gemm_stream(const GemmArgs &a, int tokens_full, hipStream_t st);

}  // namespace vx
