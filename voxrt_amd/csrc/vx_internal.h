// vx_internal.h — shared host and device definitions of libvoxrt_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "../../include/voxrt_hip.h"

namespace vx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Device weight matrix. Ternary matrices hold 2-bit codes (trit + 1) in the MFMA operand order; int8 matrices
// hold the bytes themselves in the same block order. Rows are padded with zero weights and zero scales to a
// multiple of kRowPad plus one more kRowPad, so every workgroup column tile (at most kRowPad rows, starting at or
// below the last real row) reads inside the allocation even when its row offset travels in a scalar register,
// which the buffer range check does not cover.
constexpr int kRowPad = 256;

struct TMat {
    int64_t out = 0, inp = 0, group = 0, ng = 0, out_pad = 0;
    bool ternary = false;
    // ternary: uint32 [out_pad/16][inp/64][64]: lane l = 16*j + n holds the 16 codes of row 16*nb + n at columns
    //          64*kb + 16*j + 4*d + b, code at bit 8*b + 2*d.
    // int8:    int8 [out_pad/16][inp/64][64][16]: lane l = 16*j + n holds row 16*nb + n, columns 64*kb + 16*j + i.
    void *wdev = nullptr;
    float *scales_t = nullptr;  // float32 [ng][out_pad]
};

// Error carrying a status code; converted to (status, vx_last_error text) at the ABI boundary.
struct Error : std::runtime_error {
    vx_status code;
    Error(vx_status c, const std::string &m) : std::runtime_error(m), code(c) {}
};

inline void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error(VX_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

inline void require(bool ok, const std::string &msg) {
    if (!ok) throw Error(VX_ERR_INVALID, msg);
}

// --- device helpers -------------------------------------------------------------------------------------------

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    // gfx9 buffer descriptor, raw (stride 0): loads at byte offsets >= bytes return zero.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// A 16-byte buffer store whose data registers are not written again by the next instructions: two wait states
// (s_nop 1) pinned right after it. A VMEM store of more than 8 bytes may read its data registers after it issues;
// with the VALU write of one of them right behind the store (which the compiler emits), the store can send the new
// value when the memory pipeline is busy (seen with two streaming workgroups per CU: the fourth dword of stored
// outputs replaced by the next output's intermediate).
__device__ inline void store_b128_sep(v4i v, __amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, voff, soff, 0);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 1");
    __builtin_amdgcn_sched_barrier(0);
}

// The same separation for a 16-byte global store through a plain pointer (float4, uint4).
template <typename T> __device__ inline void store16_sep(T *p, T v) {
    static_assert(sizeof(T) == 16, "16-byte stores only");
    *p = v;
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 1");
    __builtin_amdgcn_sched_barrier(0);
}

__device__ inline float bits_f32(uint32_t u) { return __uint_as_float(u); }

// Butterfly reduction over aligned groups of L lanes (L a power of two up to 64; every lane of the wavefront
// active), for order-independent operations only (max, integer sums). Distances 1 and 2 are DPP quad permutations;
// distance 4 and 8 are the half-row and row mirrors: once every lane of an aligned d-group holds the group's value,
// the mirror pairs each lane with a lane of the other d-group of its 2d-group. 16 and 32 go through ds_bpermute.
template <int L, typename Op> __device__ inline int lane_group_reduce(int v, Op op) {
    static_assert(L >= 1 && L <= 64 && (L & (L - 1)) == 0, "L must be a power of two up to 64");
    if constexpr (L > 1) v = op(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    if constexpr (L > 2) v = op(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    if constexpr (L > 4) v = op(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false));  // row_half_mirror
    if constexpr (L > 8) v = op(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false));  // row_mirror
    if constexpr (L > 16) v = op(v, __shfl_xor(v, 16, 64));
    if constexpr (L > 32) v = op(v, __shfl_xor(v, 32, 64));
    return v;
}

template <int L> __device__ inline int lane_group_sum(int v) {
    return lane_group_reduce<L>(v, [](int a, int b) { return a + b; });
}

// max of non-negative floats (amax of |x|): compared as floats, so the result is the float max of the group
template <int L> __device__ inline float lane_group_max(float m) {
    return __int_as_float(lane_group_reduce<L>(__float_as_int(m), [](int a, int b) {
        return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
    }));
}

// The reference's hsum4 of eight running sums held in lanes 0-7: (s0+s4 + s1+s5) + (s2+s6 + s3+s7), read out with
// v_readlane so the result is uniform across the wavefront.
__device__ inline float hsum8_lanes(float s) {
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), j));
    const float p0 = a[0] + a[4], p1 = a[1] + a[5], p2 = a[2] + a[6], p3 = a[3] + a[7];
    return (p0 + p1) + (p2 + p3);
}

// Note: reinterpret an element of an ext_vector_type through __int_as_float(v[e]), never
// __builtin_bit_cast(float, v[e]): this clang lowers the latter to element 0 whatever e is.

// exp_poly (crates/voxrt/src/tensor.rs:829-848): clamp to [-87, 88], n = rint(x * log2 e), two fma reduction
// steps, degree-6 Horner by fma, times 2^n. Each step is one IEEE operation (the library is built with
// -ffp-contract=off), so the result equals the reference bit for bit. exp_poly_ieee is that sequence as written;
// exp_poly computes the same function in fewer instructions: the NaN-propagating v_maximum3/v_minimum3 clamp
// (two instructions where two compare-and-select pairs were), and v_ldexp_f32 in place of building 2^n and
// multiplying. Both forms are exact, so they agree on every input; vx_check_activations compares them over all
// 2^32 inputs.
__device__ inline float exp_poly_tail(float x) {
    float n = __builtin_rintf(x * 1.44269504088896340736f);
    float r = __builtin_fmaf(-n, 0.69314575f, x);
    r = __builtin_fmaf(-n, 1.4286068e-6f, r);
    float p = 1.0f / 720.0f;
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_amdgcn_ldexpf(p, (int)n);
}
__device__ inline float exp_poly(float x) {
    return exp_poly_tail(__builtin_elementwise_minimum(__builtin_elementwise_maximum(x, -87.0f), 88.0f));
}
__device__ inline float exp_poly_ieee(float x) {
    x = x < -87.0f ? -87.0f : x;
    x = x > 88.0f ? 88.0f : x;
    float n = __builtin_rintf(x * 1.44269504088896340736f);
    float r = __builtin_fmaf(-n, 0.69314575f, x);
    r = __builtin_fmaf(-n, 1.4286068e-6f, r);
    float p = 1.0f / 720.0f;
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return p * bits_f32((uint32_t)(((int32_t)n + 127) << 23));
}

// silu_fast / sigmoid_fast (tensor.rs:852-860): x / (1 + exp_poly(-x)) and 1 / (1 + exp_poly(-x)), correctly
// rounded as the reference's IEEE division, without a branch (a branch would split the GEMM epilogues' scheduled
// regions). The divisor d = 1 + exp_poly(-x) lies in [1, 1.7e38]. y = v_rcp_f32(d / 4) / 4 estimates 1/d (the
// estimate of 4/d is normal over that whole range; 1/d alone would flush to zero for d >= 2^126). SiLU: q = x*y,
// then one correction by the exact residual fma(-d, q, x) (Markstein's step). The residual is clamped below at
// -FLT_MAX, which changes nothing for finite x and turns the inf - inf of x = +-inf into a finite correction of
// q = +-inf; copysign(., x) restores the -0 of x = -0 (SiLU has the sign of x). Sigmoid: one Newton step
// y + y * fma(-d, y, 1). vx_check_activations compares both with the IEEE forms over all 2^32 inputs.
__device__ inline float silu_ieee(float x) { return x / (1.0f + exp_poly_ieee(-x)); }
__device__ inline float sigmoid_ieee(float x) { return 1.0f / (1.0f + exp_poly_ieee(-x)); }
__device__ inline float recip_est(float d) { return __builtin_amdgcn_rcpf(d * 0.25f) * 0.25f; }
__device__ inline float silu_fast(float x) {
    // the clamp by one v_med3_f32: it differs from the NaN-propagating form only for x = NaN, where q0 = x * y
    // makes the quotient NaN whatever d is
    const float d = 1.0f + exp_poly_tail(__builtin_amdgcn_fmed3f(-x, -87.0f, 88.0f));
    const float y = recip_est(d);
    const float q0 = x * y;
    const float r = __builtin_fmaxf(__builtin_fmaf(-d, q0, x), -3.40282347e38f);
    return __builtin_copysignf(__builtin_fmaf(r, y, q0), x);
}
__device__ inline float sigmoid_fast(float x) {
    const float d = 1.0f + exp_poly(-x);
    const float y0 = recip_est(d);
    return __builtin_fmaf(__builtin_fmaf(-d, y0, 1.0f), y0, y0);
}

// One quantized code (quantize_group_portable, packed.rs:527-535): clamp(rint(x * inv), -127, 127) with
// round-half-to-even; NaN -> 0 as Rust's `as i8`.
__device__ inline int8_t code_of(float x, float inv) {
    float v = __builtin_rintf(x * inv);
    if (!(v == v)) return 0;
    v = v < -127.0f ? -127.0f : v;
    v = v > 127.0f ? 127.0f : v;
    return (int8_t)(int)v;
}

// Epilogue::apply (kernels/mod.rs:41-48).
__device__ inline float ep_apply(int ep, float alpha, float old, float v) {
    if (ep == VX_EP_SILU) return silu_fast(v);
    if (ep == VX_EP_ADD_SCALED) return __builtin_fmaf(alpha, v, old);
    return v;
}

}  // namespace vx

// The public opaque handle (include/voxrt_hip.h) is a shell around the matrix.
struct vx_tmat {
    vx::TMat m;
};
