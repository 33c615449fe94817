//! Raw bindings to libvoxrt_hip, the MI355X (gfx950) ternary x int8 GEMM path: the declarations of
//! include/voxrt_hip.h, one for one, plus the four HIP runtime calls a host needs to stage buffers
//! (hipMalloc, hipFree, hipMemcpy, hipDeviceSynchronize from libamdhip64).
//!
//! Conventions (include/voxrt_hip.h): every call returns a `VxStatus`; on failure `vx_last_error()` holds a
//! thread-local message. Weight uploads take host pointers; activations, scales, outputs and biases are device
//! pointers; `stream` is a `hipStream_t` (null: the default stream).
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub type VxStatus = c_int;
pub const VX_OK: VxStatus = 0;
pub const VX_ERR_INVALID: VxStatus = 1;
pub const VX_ERR_NO_DEVICE: VxStatus = 2;
pub const VX_ERR_HIP: VxStatus = 3;
pub const VX_ERR_OOM: VxStatus = 4;

pub const VX_EP_STORE: c_int = 0;
pub const VX_EP_SILU: c_int = 1;
pub const VX_EP_ADD_SCALED: c_int = 2;

/// Padded token count of the transposed activation tables (`VX_NPAD`).
pub const fn vx_npad(n: usize) -> usize {
    n.div_ceil(16) * 16
}

#[repr(C)]
pub struct vx_tmat {
    _private: [u8; 0],
}

#[repr(C)]
pub struct vx_encoder {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct vx_encoder_config {
    pub d: i64,
    pub heads: i64,
    pub ff: i64,
    pub kconv: i64,
    pub group: i64,
    pub n_layers: i64,
    pub n_mels: i64,
    pub sub_channels: i64,
    pub sub_kernel: i64,
    pub sub_stride: i64,
}

/// One layer's weights as host pointers, in the model file's layouts (see `vx_layer_params` in voxrt_hip.h for the
/// order of the nine linears and five LayerNorms).
#[repr(C)]
pub struct vx_layer_params {
    pub qweight: [*const u8; 9],
    pub scales_f16: [*const u16; 9],
    pub ln_gamma: [*const f32; 5],
    pub ln_beta: [*const f32; 5],
    pub bias_u: *const f32,
    pub bias_v: *const f32,
    pub dw: *const f32,
    pub bn_gamma: *const f32,
    pub bn_beta: *const f32,
    pub bn_mean: *const f32,
    pub bn_var: *const f32,
}

#[repr(C)]
pub struct vx_subsampling_params {
    pub conv0_w: *const f32,
    pub conv0_b: *const f32,
    pub dw_w: *const f32,
    pub dw_b: *const f32,
    pub pw_w: *const f32,
    pub pw_b: *const f32,
    pub lin_w: *const f32,
    pub lin_b: *const f32,
}

#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct vx_encoder_profile {
    pub total_ms: f64,
    pub subsampling_ms: f64,
    pub ff_ms: f64,
    pub attn_ms: f64,
    pub attn_core_ms: f64,
    pub conv_ms: f64,
    pub norm_ms: f64,
    pub forwards: i64,
}

extern "C" {
    pub fn vx_last_error() -> *const c_char;
    pub fn vx_detect() -> c_int;
    pub fn vx_init(device: c_int) -> VxStatus;
    pub fn vx_set_kernel_override(name: *const c_char, value: *const c_char) -> VxStatus;
    pub fn vx_shutdown() -> VxStatus;

    pub fn vx_tmat_upload_packed(
        qweight: *const u8,
        scales_f16: *const u16,
        out: i64,
        inp: i64,
        group: i64,
        w: *mut *mut vx_tmat,
    ) -> VxStatus;
    pub fn vx_tmat_upload_packed_f32(
        qweight: *const u8,
        scales: *const f32,
        out: i64,
        inp: i64,
        group: i64,
        w: *mut *mut vx_tmat,
    ) -> VxStatus;
    pub fn vx_tmat_upload_trits(
        trits: *const i8,
        scales: *const f32,
        out: i64,
        inp: i64,
        group: i64,
        w: *mut *mut vx_tmat,
    ) -> VxStatus;
    pub fn vx_tmat_upload_i8(
        rows: *const i8,
        scales: *const f32,
        out: i64,
        inp: i64,
        group: i64,
        w: *mut *mut vx_tmat,
    ) -> VxStatus;
    pub fn vx_tmat_free(w: *mut vx_tmat);
    pub fn vx_tmat_info(
        w: *const vx_tmat,
        out: *mut i64,
        inp: *mut i64,
        group: *mut i64,
        ternary: *mut c_int,
    ) -> VxStatus;

    pub fn vx_quantize(
        x: *const f32,
        n: i64,
        inp: i64,
        group: i64,
        q: *mut i8,
        scales_t: *mut f32,
        gsum_t: *mut i32,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_quantize_normed(
        x: *const f32,
        n: i64,
        inp: i64,
        group: i64,
        gamma: *const f32,
        beta: *const f32,
        q: *mut i8,
        scales_t: *mut f32,
        gsum_t: *mut i32,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_gemm_ep(
        w: *const vx_tmat,
        xq: *const i8,
        xs_t: *const f32,
        xgsum_t: *const i32,
        n: i64,
        y: *mut f32,
        bias: *const f32,
        ep: c_int,
        alpha: f32,
        group_sums: *mut i32,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_gemm_ep_quantize(
        w: *const vx_tmat,
        xq: *const i8,
        xs_t: *const f32,
        xgsum_t: *const i32,
        n: i64,
        y_tmp: *mut f32,
        bias: *const f32,
        ep: c_int,
        group: i64,
        q: *mut i8,
        scales_t: *mut f32,
        gsum_t: *mut i32,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_gemm_rows_range(
        w: *const vx_tmat,
        xq: *const i8,
        xs_t: *const f32,
        xgsum_t: *const i32,
        n: i64,
        y: *mut f32,
        r0: i64,
        r1: i64,
        t0: i64,
        t1: i64,
        ep: c_int,
        alpha: f32,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_gemm_single(
        w: *const vx_tmat,
        xq: *const i8,
        xs_t: *const f32,
        xgsum_t: *const i32,
        n: i64,
        y: *mut f32,
        bias: *const f32,
        stream: *mut c_void,
    ) -> VxStatus;

    pub fn vx_encoder_create(cfg: *const vx_encoder_config, enc: *mut *mut vx_encoder) -> VxStatus;
    pub fn vx_encoder_set_layer(enc: *mut vx_encoder, layer: i64, p: *const vx_layer_params) -> VxStatus;
    pub fn vx_encoder_set_subsampling(enc: *mut vx_encoder, p: *const vx_subsampling_params) -> VxStatus;
    pub fn vx_encoder_use_graphs(enc: *mut vx_encoder, on: c_int) -> VxStatus;
    pub fn vx_encoder_set_profiling(enc: *mut vx_encoder, on: c_int) -> VxStatus;
    pub fn vx_encoder_take_profile(enc: *mut vx_encoder, out: *mut vx_encoder_profile) -> VxStatus;
    pub fn vx_encoder_memory(enc: *mut vx_encoder, workspace_bytes: *mut i64, graphs: *mut i64) -> VxStatus;
    pub fn vx_encoder_forward(
        enc: *mut vx_encoder,
        x: *const f32,
        out: *mut f32,
        t: i64,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_encoder_forward_feats(
        enc: *mut vx_encoder,
        feats: *const f32,
        t_in: i64,
        out: *mut f32,
        t_out: *mut i64,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_encoder_forward_batch(
        enc: *mut vx_encoder,
        x: *const f32,
        out: *mut f32,
        nseg: i64,
        t: i64,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_encoder_forward_feats_batch(
        enc: *mut vx_encoder,
        feats: *const f32,
        nseg: i64,
        t_in: i64,
        out: *mut f32,
        t_out: *mut i64,
        stream: *mut c_void,
    ) -> VxStatus;
    pub fn vx_encoder_free(enc: *mut vx_encoder);
    pub fn vx_subsampling_frames(t: i64, k: i64, s: i64) -> i64;
}

// The HIP runtime calls used to stage host buffers (libamdhip64; hipError_t is an int, 0 = success).
pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

extern "C" {
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> c_int;
    pub fn hipFree(ptr: *mut c_void) -> c_int;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> c_int;
    pub fn hipDeviceSynchronize() -> c_int;
}

/// The thread-local message of the last failed call, as an owned string.
pub fn last_error() -> String {
    // SAFETY: vx_last_error returns a NUL-terminated thread-local buffer that outlives this call.
    unsafe {
        let p = vx_last_error();
        if p.is_null() {
            String::new()
        } else {
            std::ffi::CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}
