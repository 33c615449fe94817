/* voxrt_hip.h — C ABI of the MI355X (gfx950) ternary x int8 GEMM path.
 *
 * The entry points mirror voxrt's runtime kernel-dispatch surface (crates/voxrt/src/kernels/mod.rs and
 * crates/voxrt/src/packed.rs), so a GPU backend binds beside its scalar/AVX2/VNNI/NEON kernels:
 *
 *   vx_detect / vx_init               <- kernels::detect (kernels/mod.rs:85-109)
 *   vx_tmat_upload_packed             <- TernaryMatrix::from_packed_layout (packed.rs:73-130)
 *   vx_tmat_upload_packed_f32         <- the same with f32 scales (BASELINE config 0's per-channel fp32 scale)
 *   vx_tmat_upload_i8                 <- TernaryMatrix::from_i8_rows (packed.rs:164-201)
 *   vx_tmat_free / vx_tmat_info       <- drop / the out, inp, group, ternary fields (packed.rs:48-60)
 *   vx_quantize                       <- QuantAct::quantize_layout (packed.rs:307-436, quantize_group 527-535)
 *   vx_gemm_ep                        <- kernels::gemm_ep / gemm (kernels/mod.rs:319-362)
 *   vx_gemm_rows_range                <- kernels::gemm_rows_range (kernels/mod.rs:257-282)
 *   vx_last_error                     <- voxrt_last_error (crates/voxrt-ffi/src/lib.rs:61-74)
 *
 * Conventions (as voxrt-ffi): every call returns a vx_status; on failure a message is kept in a thread-local
 * buffer read by vx_last_error(). No exception crosses the ABI. Weight uploads take HOST pointers (the load-time
 * repack of the reference runs on the device). Activation, scale, output and bias pointers are DEVICE pointers on
 * the current HIP device; `stream` is a hipStream_t (NULL = the default stream); every GEMM / quantize call is
 * ordered on that stream and returns before the work completes. Calls on different streams that write disjoint
 * outputs may run concurrently; a vx_tmat is immutable after upload and may be shared by any number of calls.
 *
 * Shape rules: inp % group == 0, group % 64 == 0 (one i8 MFMA step is 64 columns).
 */
#ifndef VOXRT_HIP_H
#define VOXRT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum vx_status {
    VX_OK = 0,
    VX_ERR_INVALID = 1,     /* a NULL pointer, a bad shape or an unsupported group */
    VX_ERR_NO_DEVICE = 2,   /* no HIP device, or the current device is not gfx950 */
    VX_ERR_HIP = 3,         /* a HIP runtime call failed (the message names it) */
    VX_ERR_OOM = 4          /* device allocation failed */
} vx_status;

/* kernels/mod.rs:14-21 Epilogue: STORE y = v; SILU y = silu_fast(v); ADD_SCALED y = fma(alpha, v, y). */
typedef enum vx_epilogue { VX_EP_STORE = 0, VX_EP_SILU = 1, VX_EP_ADD_SCALED = 2 } vx_epilogue;

/* Opaque device-resident weight matrix [out, inp] in the MFMA layout (TernaryMatrix, packed.rs:48-60). */
typedef struct vx_tmat vx_tmat;

/* Thread-local text of the last failure on this thread ("" if none). */
const char *vx_last_error(void);

/* 1 if the current process sees at least one gfx950 device, else 0 (kernels::detect). */
int vx_detect(void);

/* Make `device` current for this thread and check that it is gfx950. */
vx_status vx_init(int device);

/* from_packed_layout: qweight = thrush-ternary-v2 rows uint8 [out, ceil(inp/5)] (5 trits per byte, least
 * significant base-3 digit first, trit = digit - 1), scales_f16 = IEEE binary16 [out, inp/group]. */
vx_status vx_tmat_upload_packed(const uint8_t *qweight, const uint16_t *scales_f16, int64_t out, int64_t inp,
                                int64_t group, vx_tmat **w);

/* As vx_tmat_upload_packed with float32 scales [out, inp/group]. */
vx_status vx_tmat_upload_packed_f32(const uint8_t *qweight, const float *scales, int64_t out, int64_t inp,
                                    int64_t group, vx_tmat **w);

/* from_i8_rows: arbitrary int8 rows [out, inp] with float32 scales [out, inp/group] (not ternary). */
vx_status vx_tmat_upload_i8(const int8_t *rows, const float *scales, int64_t out, int64_t inp, int64_t group,
                            vx_tmat **w);

void vx_tmat_free(vx_tmat *w);

vx_status vx_tmat_info(const vx_tmat *w, int64_t *out, int64_t *inp, int64_t *group, int *ternary);

/* Padded token count of the transposed activation tables: n rounded up to a multiple of 16. */
#define VX_NPAD(n) ((((n) + 15) / 16) * 16)

/* quantize_layout on the device: per (token, group) s = absmax/127 (1 when all zero), codes
 * clamp(rint(x * (1/s)), -127, 127); x float32 [n, inp] -> q int8 [n, inp], scales_t float32 [inp/group, np] and
 * gsum_t int32 [inp/group, np] with np = VX_NPAD(n): the scales and code sums transposed (QuantAct::scales_t,
 * packed.rs:294), pad tokens zero. gsum (sum of the codes of each group) is what ternary GEMMs need. */
vx_status vx_quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t,
                      int32_t *gsum_t, void *stream);

/* gemm_ep: y[t*out + o] = ep(y_old, sum_g fma-fold of S_g * (xs[t][g] * ws[o][g])) for all t < n, o < out, then
 * y += bias[o] when bias is not NULL. xq int8 [n, inp]; xs_t float32 [inp/group, VX_NPAD(n)] and xgsum_t int32
 * [inp/group, VX_NPAD(n)] as written by vx_quantize (xgsum_t is required for ternary weights); y float32
 * [n, out]. When group_sums is not NULL the exact int32 group sums S_g are also written to
 * group_sums[(g*n + t)*out + o] (int32 [inp/group, n, out]). */
vx_status vx_gemm_ep(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t, int64_t n,
                     float *y, const float *bias, int ep, float alpha, int32_t *group_sums, void *stream);

/* gemm_rows_range: as vx_gemm_ep without bias, writing only rows o in [r0, r1) and tokens t in [t0, t1) of
 * y [n, out]; nothing else in y is read or written. */
vx_status vx_gemm_rows_range(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t,
                             int64_t n, float *y, int64_t r0, int64_t r1, int64_t t0, int64_t t1, int ep, float alpha,
                             void *stream);

#ifdef __cplusplus
}
#endif
#endif
