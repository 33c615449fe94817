//! `Kernel::Hip`: voxrt's ternary x int8 GEMM on an AMD Instinct MI355X (gfx950) through libvoxrt_hip, beside the
//! scalar, AVX2, AVX-512 VNNI and NEON kernels of `kernels`. This file is crates/voxrt/src/kernels/hip.rs of a voxrt
//! built with the `hip` feature (the edits that wire it into kernels/mod.rs, packed.rs and Cargo.toml are listed in
//! INTEGRATION.md).
//!
//! Same contract as the CPU kernels (kernels/mod.rs:151-362): `y[t, o] = ep(y, fold)` with the fold
//! `acc = fma(S_g, s_x[t,g] * s_w[o,g], acc)` over the groups in ascending order, so the results are bit-identical
//! to every other kernel's. The weights live on the device: a `TernaryMatrix` keeps its device copy in its `hip`
//! field, uploaded the first time a HIP GEMM reads it (ternary matrices in the 2-bit MFMA layout, int8 ones as
//! 16-byte chunks). The activations and outputs of these entry points are host slices, as the CPU kernels take
//! them, so each call stages them through device buffers; the device-resident path for whole encoder forwards is
//! `hip_encoder::HipEncoder`.
use std::os::raw::c_void;
use std::sync::{Mutex, OnceLock};

use voxrt_hip_sys as sys;

use super::Epilogue;
use crate::packed::{Layout, QuantAct, TernaryMatrix};

/// `true` when a gfx950 device is visible and the library initialises on device 0 (checked once per process), the
/// HIP counterpart of `detect()`'s CPU feature tests.
pub fn available() -> bool {
    static OK: OnceLock<bool> = OnceLock::new();
    // SAFETY: plain C calls without pointer arguments.
    *OK.get_or_init(|| unsafe { sys::vx_detect() == 1 && sys::vx_init(0) == sys::VX_OK })
}

/// The CPU kernels cannot fail; a device failure in the middle of a forward is reported the way their debug
/// assertions are, with a panic naming the call and the library's message.
fn check(st: sys::VxStatus, what: &str) {
    if st != sys::VX_OK {
        panic!("voxrt: HIP {what} failed (status {st}): {}", sys::last_error());
    }
}

/// A weight matrix on the device (an opaque `vx_tmat`), immutable after upload.
pub struct DeviceMatrix {
    h: *mut sys::vx_tmat,
}

// SAFETY: a vx_tmat is never written after upload and may be read by any number of concurrent calls.
unsafe impl Send for DeviceMatrix {}
unsafe impl Sync for DeviceMatrix {}

impl Drop for DeviceMatrix {
    fn drop(&mut self) {
        // SAFETY: h came from a successful upload and is freed once.
        unsafe { sys::vx_tmat_free(self.h) }
    }
}

impl DeviceMatrix {
    /// Uploads a matrix in the `Rows` layout (`Kernel::Hip.layout()`): ternary rows as trits, others as int8.
    pub fn upload(w: &TernaryMatrix) -> Self {
        assert_eq!(w.layout, Layout::Rows, "Kernel::Hip reads matrices in the Rows layout");
        let mut h = std::ptr::null_mut();
        let (out, inp, group) = (w.out as i64, w.inp as i64, w.group as i64);
        // SAFETY: w.w holds out * inp bytes and w.scales out * inp / group floats (TernaryMatrix, packed.rs:48-60).
        let st = unsafe {
            if w.ternary {
                sys::vx_tmat_upload_trits(w.w.as_ptr(), w.scales.as_ptr(), out, inp, group, &mut h)
            } else {
                sys::vx_tmat_upload_i8(w.w.as_ptr(), w.scales.as_ptr(), out, inp, group, &mut h)
            }
        };
        check(st, "weight upload");
        Self { h }
    }
}

/// The device copy of `w`, uploaded on first use.
fn device(w: &TernaryMatrix) -> &DeviceMatrix {
    w.hip.get_or_init(|| DeviceMatrix::upload(w))
}

/// A grow-only device buffer of the staging area.
struct DevBuf {
    p: *mut c_void,
    cap: usize,
}

impl DevBuf {
    const fn new() -> Self {
        Self { p: std::ptr::null_mut(), cap: 0 }
    }

    fn ensure(&mut self, bytes: usize) -> *mut c_void {
        if bytes > self.cap {
            // SAFETY: p is null or a live allocation of this buffer; the device is idle for it (every staged call
            // ends with a synchronous copy).
            unsafe {
                if !self.p.is_null() {
                    sys::hipFree(self.p);
                    self.p = std::ptr::null_mut();
                    self.cap = 0;
                }
                let want = bytes.max(self.cap + self.cap / 4);
                let mut p = std::ptr::null_mut();
                if sys::hipMalloc(&mut p, want) != 0 {
                    panic!("voxrt: hipMalloc({want}) failed");
                }
                self.p = p;
                self.cap = want;
            }
        }
        self.p
    }

    fn upload<T>(&mut self, host: &[T]) -> *mut c_void {
        let bytes = std::mem::size_of_val(host);
        let p = self.ensure(bytes.max(1));
        // SAFETY: p holds at least `bytes`; host is a live slice of that size.
        let st = unsafe { sys::hipMemcpy(p, host.as_ptr() as *const c_void, bytes, sys::HIP_MEMCPY_HOST_TO_DEVICE) };
        assert_eq!(st, 0, "voxrt: hipMemcpy to the device failed");
        p
    }

    fn download<T>(&self, host: &mut [T]) {
        let bytes = std::mem::size_of_val(host);
        // SAFETY: self.p holds at least `bytes` (it was ensured for this call); the copy is synchronous and so also
        // waits for the kernel that wrote it (both on the default stream).
        let st = unsafe { sys::hipMemcpy(host.as_mut_ptr() as *mut c_void, self.p, bytes, sys::HIP_MEMCPY_DEVICE_TO_HOST) };
        assert_eq!(st, 0, "voxrt: hipMemcpy to the host failed");
    }
}

/// Device buffers for the operands of one staged call. The CPU kernels are called concurrently (rayon blocks, the
/// attention tasks); staged HIP calls take this lock one at a time.
struct Staging {
    xq: DevBuf,
    xs: DevBuf,
    xg: DevBuf,
    y: DevBuf,
    bias: DevBuf,
}

// SAFETY: the raw device pointers are only used under the mutex.
unsafe impl Send for Staging {}

static STAGING: Mutex<Staging> = Mutex::new(Staging {
    xq: DevBuf::new(),
    xs: DevBuf::new(),
    xg: DevBuf::new(),
    y: DevBuf::new(),
    bias: DevBuf::new(),
});

/// The device activation operand of `x` (Rows layout): its codes, and its scales and code sums transposed to
/// `[inp/group][npad16(n)]` with zero pad tokens (the sums are the `gsum` that `QuantAct` fills for `Quad16`).
fn stage_act(st: &mut Staging, x: &QuantAct) -> (*const i8, *const f32, *const i32) {
    assert!(matches!(x.layout, Layout::Rows | Layout::Rows8), "Kernel::Hip reads activations in the Rows layout");
    let ng = x.inp / x.group;
    let np = sys::vx_npad(x.n);
    let mut s = vec![0f32; ng * np];
    let mut g = vec![0i32; ng * np];
    for t in 0..x.n {
        let row = &x.x[t * x.inp..(t + 1) * x.inp];
        for (gi, codes) in row.chunks_exact(x.group).enumerate() {
            s[gi * np + t] = x.scales[t * ng + gi];
            g[gi * np + t] = codes.iter().map(|&c| c as i32).sum();
        }
    }
    let xq = st.xq.upload(&x.x[..x.n * x.inp]) as *const i8;
    let xs = st.xs.upload(&s) as *const f32;
    let xg = st.xg.upload(&g) as *const i32;
    (xq, xs, xg)
}

fn ep_code(ep: Epilogue) -> (i32, f32) {
    match ep {
        Epilogue::Store => (sys::VX_EP_STORE, 0.0),
        Epilogue::Silu => (sys::VX_EP_SILU, 0.0),
        Epilogue::AddScaled(s) => (sys::VX_EP_ADD_SCALED, s),
    }
}

/// `gemm_ep` (kernels/mod.rs:319-362) on the device: the whole `[n, out]` product in one launch (no row blocks),
/// the bias added after the epilogue.
pub fn gemm_ep(w: &TernaryMatrix, x: &QuantAct, y: &mut [f32], bias: Option<&[f32]>, ep: Epilogue) {
    debug_assert_eq!(x.inp, w.inp);
    debug_assert_eq!(x.group, w.group);
    debug_assert_eq!(y.len(), x.n * w.out);
    if x.n == 0 {
        return;
    }
    let dm = device(w);
    let mut st = STAGING.lock().unwrap_or_else(|e| e.into_inner());
    let (xq, xs, xg) = stage_act(&mut st, x);
    // AddScaled reads the old outputs
    let dy = (if matches!(ep, Epilogue::AddScaled(_)) {
        st.y.upload(y)
    } else {
        st.y.ensure(std::mem::size_of_val(y))
    }) as *mut f32;
    let db = match bias {
        Some(b) => {
            debug_assert_eq!(b.len(), w.out);
            st.bias.upload(b) as *const f32
        }
        None => std::ptr::null(),
    };
    let (kind, alpha) = ep_code(ep);
    // SAFETY: every device pointer was staged above with the sizes the call reads and writes.
    let r = unsafe {
        sys::vx_gemm_ep(dm.h, xq, xs, xg, x.n as i64, dy, db, kind, alpha, std::ptr::null_mut(), std::ptr::null_mut())
    };
    check(r, "gemm_ep");
    st.y.download(y);
}

/// `gemm_rows_range` (kernels/mod.rs:257-282): rows `[r0, r1)` x tokens `[t0, t1)` of `y[n, out]`; the rest of `y`
/// is left as it was (the staged copy of `y` goes up and comes back whole).
#[allow(clippy::too_many_arguments)]
pub fn gemm_rows_range(
    w: &TernaryMatrix,
    x: &QuantAct,
    y: &mut [f32],
    r0: usize,
    r1: usize,
    t0: usize,
    t1: usize,
    ep: Epilogue,
) {
    debug_assert!(t1 <= x.n && r1 <= w.out);
    if r0 == r1 || t0 == t1 {
        return;
    }
    let dm = device(w);
    let mut st = STAGING.lock().unwrap_or_else(|e| e.into_inner());
    let (xq, xs, xg) = stage_act(&mut st, x);
    let dy = st.y.upload(&y[..x.n * w.out]) as *mut f32;
    let (kind, alpha) = ep_code(ep);
    // SAFETY: as in gemm_ep; the kernel writes only the window.
    let r = unsafe {
        sys::vx_gemm_rows_range(
            dm.h,
            xq,
            xs,
            xg,
            x.n as i64,
            dy,
            r0 as i64,
            r1 as i64,
            t0 as i64,
            t1 as i64,
            kind,
            alpha,
            std::ptr::null_mut(),
        )
    };
    check(r, "gemm_rows_range");
    st.y.download(&mut y[..x.n * w.out]);
}

/// `gemm_single` (kernels/mod.rs:285-316): `y[n, out] = x . w^T`, then `y += bias`, unfused.
pub fn gemm_single(w: &TernaryMatrix, x: &QuantAct, y: &mut [f32], bias: Option<&[f32]>) {
    if x.n == 0 {
        return;
    }
    let dm = device(w);
    let mut st = STAGING.lock().unwrap_or_else(|e| e.into_inner());
    let (xq, xs, xg) = stage_act(&mut st, x);
    let ylen = x.n * w.out;
    let dy = st.y.ensure(ylen * 4) as *mut f32;
    let db = bias.map_or(std::ptr::null(), |b| st.bias.upload(b) as *const f32);
    // SAFETY: as in gemm_ep.
    let r = unsafe { sys::vx_gemm_single(dm.h, xq, xs, xg, x.n as i64, dy, db, std::ptr::null_mut()) };
    check(r, "gemm_single");
    st.y.download(&mut y[..ylen]);
}
