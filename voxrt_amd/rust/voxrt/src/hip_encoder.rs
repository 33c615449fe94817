//! The int8 encoder on an AMD Instinct MI355X (gfx950): `Device::Gpu` for a voxrt built with the `hip` feature, the
//! counterpart of `metal::GpuEncoder` (metal/mod.rs:446-603) on the CPU int8 `Encoder`'s operation order
//! (encoder.rs:706-857). This file is crates/voxrt/src/hip_encoder.rs; INTEGRATION.md lists the lines that select it
//! in transcriber.rs.
//!
//! Loading reads the model file's own tensors (thrush-ternary-v2, HF names): each ternary linear's packed rows and
//! f16 scales go to the device as they are (the 2-bit repack runs there; q | k | v stacked, as
//! `TernaryLinear::load_stacked` does), the LayerNorm, relative-position bias and BatchNorm vectors widened to f32
//! (`tensor::load_f32`), the depthwise taps with their BatchNorm statistics (folded at upload), and the subsampling
//! convolutions in the layouts `Subsampling::load` gives them (subsampling.rs:31-90). A forward keeps every
//! activation on the device from the log-mel features to the encoder output: one upload of the features and one
//! download of the result per call. The library serializes calls on one encoder and keeps one growing workspace, so
//! the encoder is `Send + Sync`.
use std::os::raw::c_void;
use std::sync::Mutex;

use voxrt_hip_sys as sys;

use crate::format::ModelFile;
use crate::tensor::load_f32_shaped;
use crate::{Error, Result};

pub struct HipEncoder {
    enc: *mut sys::vx_encoder,
    d: usize,
    n_mels: usize,
    sub_kernel: usize,
    sub_stride: usize,
    io: Mutex<Io>,
}

// SAFETY: the library serializes the calls on one vx_encoder; the staging buffers are behind `io`.
unsafe impl Send for HipEncoder {}
unsafe impl Sync for HipEncoder {}

impl Drop for HipEncoder {
    fn drop(&mut self) {
        // SAFETY: enc came from vx_encoder_create and is freed once.
        unsafe { sys::vx_encoder_free(self.enc) }
    }
}

fn status(st: sys::VxStatus, what: &str) -> Result<()> {
    if st == sys::VX_OK {
        Ok(())
    } else {
        Err(Error::Format(format!("hip: {what}: {}", sys::last_error())))
    }
}

/// Raw bytes of a tensor with the expected dtype and shape.
fn raw<'a>(m: &'a ModelFile, name: &str, dtype: safetensors::Dtype, shape: &[usize]) -> Result<&'a [u8]> {
    let (info, bytes) = m.tensor(name)?;
    if info.dtype != dtype || info.shape != shape {
        return Err(Error::Format(format!(
            "{name}: {:?} {:?}, expected {dtype:?} {shape:?}",
            info.dtype, info.shape
        )));
    }
    Ok(bytes)
}

/// The packed rows and f16 scale bits of one or several modules with one input, stacked along the output rows.
fn packed_linear(m: &ModelFile, names: &[String], group: usize) -> Result<(Vec<u8>, Vec<u16>, usize, usize)> {
    let (mut q, mut s, mut out, mut inp) = (Vec::new(), Vec::new(), 0usize, 0usize);
    for name in names {
        let module = m
            .ternary
            .quantized_modules
            .iter()
            .find(|x| &x.name == name)
            .ok_or_else(|| Error::Format(format!("{name}: not a quantized module")))?;
        if module.group_size != group || (inp != 0 && module.in_features != inp) || module.has_bias {
            return Err(Error::Format(format!("{name}: group, input width or bias differs from the encoder's")));
        }
        inp = module.in_features;
        let o = module.out_features;
        q.extend_from_slice(raw(m, &format!("{name}.qweight"), safetensors::Dtype::U8, &[o, inp.div_ceil(5)])?);
        let sb = raw(m, &format!("{name}.scales"), safetensors::Dtype::F16, &[o, inp / group])?;
        s.extend(sb.chunks_exact(2).map(|c| u16::from_le_bytes([c[0], c[1]])));
        out += o;
    }
    Ok((q, s, out, inp))
}

/// Conv taps [C, 1, k, k] -> [k*k, C] (the layout Subsampling::load gives them).
fn taps(m: &ModelFile, name: &str, c: usize, k: usize) -> Result<Vec<f32>> {
    let w = load_f32_shaped(m, name, &[c, 1, k, k])?;
    let mut t = vec![0f32; k * k * c];
    for ch in 0..c {
        for j in 0..k * k {
            t[j * c + ch] = w[ch * k * k + j];
        }
    }
    Ok(t)
}

impl HipEncoder {
    /// `GpuEncoder::load`: every layer and the subsampling uploaded; an error when no gfx950 device is usable (the
    /// transcriber then stays on the CPU).
    pub fn load(m: &ModelFile) -> Result<Self> {
        if !crate::kernels::hip::available() {
            return Err(Error::Format("hip: no gfx950 (MI355X) device".into()));
        }
        let e = &m.config.encoder_config;
        let (d, heads, ff, k) = (e.hidden_size, e.num_attention_heads, e.intermediate_size, e.conv_kernel_size);
        let group = m.config.ternary_group_size;
        let cfg = sys::vx_encoder_config {
            d: d as i64,
            heads: heads as i64,
            ff: ff as i64,
            kconv: k as i64,
            group: group as i64,
            n_layers: e.num_hidden_layers as i64,
            n_mels: e.num_mel_bins as i64,
            sub_channels: e.subsampling_conv_channels as i64,
            sub_kernel: e.subsampling_conv_kernel_size as i64,
            sub_stride: e.subsampling_conv_stride as i64,
        };
        let mut enc = std::ptr::null_mut();
        // SAFETY: cfg is a live struct; enc receives the handle.
        status(unsafe { sys::vx_encoder_create(&cfg, &mut enc) }, "encoder create")?;
        let me = Self {
            enc,
            d,
            n_mels: e.num_mel_bins,
            sub_kernel: e.subsampling_conv_kernel_size,
            sub_stride: e.subsampling_conv_stride,
            io: Mutex::new(Io::default()),
        };
        for i in 0..e.num_hidden_layers {
            me.load_layer(m, i, d, heads, ff, k, group)?;
        }
        me.load_subsampling(m)?;
        Ok(me)
    }

    #[allow(clippy::too_many_arguments)]
    fn load_layer(&self, m: &ModelFile, i: usize, d: usize, heads: usize, ff: usize, k: usize, group: usize) -> Result<()> {
        let p = format!("encoder.layers.{i}");
        let one = |n: &str| vec![format!("{p}.{n}")];
        let lin: [Vec<String>; 9] = [
            one("feed_forward1.linear1"),
            one("feed_forward1.linear2"),
            vec![format!("{p}.self_attn.q_proj"), format!("{p}.self_attn.k_proj"), format!("{p}.self_attn.v_proj")],
            one("self_attn.o_proj"),
            one("self_attn.relative_k_proj"),
            one("conv.pointwise_conv1"),
            one("conv.pointwise_conv2"),
            one("feed_forward2.linear1"),
            one("feed_forward2.linear2"),
        ];
        let want = [(ff, d), (d, ff), (3 * d, d), (d, d), (d, d), (2 * d, d), (d, d), (ff, d), (d, ff)];
        let mut packed = Vec::with_capacity(9);
        for (names, &(o, inp)) in lin.iter().zip(want.iter()) {
            let (q, s, out, got_inp) = packed_linear(m, names, group)?;
            if out != o || got_inp != inp {
                return Err(Error::Format(format!("{}: [{out}, {got_inp}], expected [{o}, {inp}]", names[0])));
            }
            packed.push((q, s));
        }
        let norms = ["norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"];
        let mut ln = Vec::with_capacity(5);
        for n in norms {
            ln.push((
                load_f32_shaped(m, &format!("{p}.{n}.weight"), &[d])?,
                load_f32_shaped(m, &format!("{p}.{n}.bias"), &[d])?,
            ));
        }
        let dh = d / heads;
        let bias_u = load_f32_shaped(m, &format!("{p}.self_attn.bias_u"), &[heads, dh])?;
        let bias_v = load_f32_shaped(m, &format!("{p}.self_attn.bias_v"), &[heads, dh])?;
        let dw = load_f32_shaped(m, &format!("{p}.conv.depthwise_conv.weight"), &[d, 1, k])?;
        let bn: Vec<Vec<f32>> = ["weight", "bias", "running_mean", "running_var"]
            .iter()
            .map(|n| load_f32_shaped(m, &format!("{p}.conv.norm.{n}"), &[d]))
            .collect::<Result<_>>()?;
        let lp = sys::vx_layer_params {
            qweight: std::array::from_fn(|j| packed[j].0.as_ptr()),
            scales_f16: std::array::from_fn(|j| packed[j].1.as_ptr()),
            ln_gamma: std::array::from_fn(|j| ln[j].0.as_ptr()),
            ln_beta: std::array::from_fn(|j| ln[j].1.as_ptr()),
            bias_u: bias_u.as_ptr(),
            bias_v: bias_v.as_ptr(),
            dw: dw.as_ptr(),
            bn_gamma: bn[0].as_ptr(),
            bn_beta: bn[1].as_ptr(),
            bn_mean: bn[2].as_ptr(),
            bn_var: bn[3].as_ptr(),
        };
        // SAFETY: every pointer refers to a host vector of the size the configuration implies, alive for the call.
        status(unsafe { sys::vx_encoder_set_layer(self.enc, i as i64, &lp) }, "layer upload")
    }

    fn load_subsampling(&self, m: &ModelFile) -> Result<()> {
        let e = &m.config.encoder_config;
        let (c, k, d) = (e.subsampling_conv_channels, e.subsampling_conv_kernel_size, e.hidden_size);
        let f = e.num_mel_bins / e.subsampling_factor;
        let pre = "encoder.subsampling.layers";
        let conv0_w = taps(m, &format!("{pre}.0.weight"), c, k)?;
        let conv0_b = load_f32_shaped(m, &format!("{pre}.0.bias"), &[c])?;
        let mut dw_w = taps(m, &format!("{pre}.2.weight"), c, k)?;
        dw_w.extend(taps(m, &format!("{pre}.5.weight"), c, k)?);
        let mut dw_b = load_f32_shaped(m, &format!("{pre}.2.bias"), &[c])?;
        dw_b.extend(load_f32_shaped(m, &format!("{pre}.5.bias"), &[c])?);
        let mut pw_w = load_f32_shaped(m, &format!("{pre}.3.weight"), &[c, c, 1, 1])?;
        pw_w.extend(load_f32_shaped(m, &format!("{pre}.6.weight"), &[c, c, 1, 1])?);
        let mut pw_b = load_f32_shaped(m, &format!("{pre}.3.bias"), &[c])?;
        pw_b.extend(load_f32_shaped(m, &format!("{pre}.6.bias"), &[c])?);
        // the final linear's columns from the HF flatten order c*F + f to channels-last f*C + c
        let lw = load_f32_shaped(m, "encoder.subsampling.linear.weight", &[d, c * f])?;
        let mut lin_w = vec![0f32; d * f * c];
        for o in 0..d {
            for ch in 0..c {
                for fi in 0..f {
                    lin_w[o * f * c + fi * c + ch] = lw[o * c * f + ch * f + fi];
                }
            }
        }
        let lin_b = load_f32_shaped(m, "encoder.subsampling.linear.bias", &[d])?;
        let sp = sys::vx_subsampling_params {
            conv0_w: conv0_w.as_ptr(),
            conv0_b: conv0_b.as_ptr(),
            dw_w: dw_w.as_ptr(),
            dw_b: dw_b.as_ptr(),
            pw_w: pw_w.as_ptr(),
            pw_b: pw_b.as_ptr(),
            lin_w: lin_w.as_ptr(),
            lin_b: lin_b.as_ptr(),
        };
        // SAFETY: as in load_layer.
        status(unsafe { sys::vx_encoder_set_subsampling(self.enc, &sp) }, "subsampling upload")
    }

    /// Encoder frames for `t` log-mel frames (`Subsampling::out_frames`).
    pub fn out_frames(&self, t: usize) -> usize {
        // SAFETY: pure function.
        unsafe { sys::vx_subsampling_frames(t as i64, self.sub_kernel as i64, self.sub_stride as i64) as usize }
    }

    /// `GpuEncoder::forward_feats`: log-mel `feats [t, n_mels]` -> `(encoder_out [t_e, d], t_e)`.
    pub fn forward_feats(&self, feats: &[f32], t: usize) -> (Vec<f32>, usize) {
        assert_eq!(feats.len(), t * self.n_mels);
        let te = self.out_frames(t);
        let mut out = vec![0f32; te * self.d];
        let mut io = self.io.lock().unwrap_or_else(|e| e.into_inner());
        let df = io.feats.upload(feats);
        let dout = io.out.ensure(out.len() * 4);
        let mut got = 0i64;
        // SAFETY: df holds the features, dout te * d floats.
        let st = unsafe {
            sys::vx_encoder_forward_feats(self.enc, df as *const f32, t as i64, dout as *mut f32, &mut got, std::ptr::null_mut())
        };
        if st != sys::VX_OK {
            panic!("voxrt: HIP encoder forward failed: {}", sys::last_error());
        }
        debug_assert_eq!(got as usize, te);
        io.out.download(&mut out);
        (out, te)
    }

    /// Device time per sublayer type of every later forward (the reference's `VOXRT_PROFILE`): on or off.
    pub fn set_profiling(&self, on: bool) -> Result<()> {
        // SAFETY: plain call on a live handle.
        status(unsafe { sys::vx_encoder_set_profiling(self.enc, on as i32) }, "profiling")
    }

    /// The sums since the previous call: (total, subsampling, ff, attn, attn core, conv, norm) in ms, forwards.
    pub fn take_profile(&self) -> Result<sys::vx_encoder_profile> {
        let mut p = sys::vx_encoder_profile::default();
        // SAFETY: p is a live struct.
        status(unsafe { sys::vx_encoder_take_profile(self.enc, &mut p) }, "profile")?;
        Ok(p)
    }
}

/// Device staging of one forward's input and output (grow-only).
#[derive(Default)]
struct Io {
    feats: Buf,
    out: Buf,
}

struct Buf {
    p: *mut c_void,
    cap: usize,
}

impl Default for Buf {
    fn default() -> Self {
        Self { p: std::ptr::null_mut(), cap: 0 }
    }
}

impl Drop for Buf {
    fn drop(&mut self) {
        if !self.p.is_null() {
            // SAFETY: p is this buffer's allocation; the forwards that used it have completed (synchronous copies).
            unsafe { sys::hipFree(self.p) };
        }
    }
}

impl Buf {
    fn ensure(&mut self, bytes: usize) -> *mut c_void {
        if bytes > self.cap {
            let want = bytes.max(self.cap + self.cap / 4);
            // SAFETY: the old allocation is not in use (every forward ends with a synchronous copy).
            unsafe {
                if !self.p.is_null() {
                    sys::hipFree(self.p);
                }
                self.p = std::ptr::null_mut();
                self.cap = 0;
                if sys::hipMalloc(&mut self.p, want) != 0 {
                    panic!("voxrt: hipMalloc({want}) failed");
                }
            }
            self.cap = want;
        }
        self.p
    }

    fn upload(&mut self, host: &[f32]) -> *mut c_void {
        let bytes = std::mem::size_of_val(host);
        let p = self.ensure(bytes.max(4));
        // SAFETY: p holds at least `bytes`.
        let st = unsafe { sys::hipMemcpy(p, host.as_ptr() as *const c_void, bytes, sys::HIP_MEMCPY_HOST_TO_DEVICE) };
        assert_eq!(st, 0, "voxrt: hipMemcpy to the device failed");
        p
    }

    fn download(&self, host: &mut [f32]) {
        let bytes = std::mem::size_of_val(host);
        // SAFETY: p holds at least `bytes`; the copy is synchronous and follows the forward on the default stream.
        let st = unsafe { sys::hipMemcpy(host.as_mut_ptr() as *mut c_void, self.p, bytes, sys::HIP_MEMCPY_DEVICE_TO_HOST) };
        assert_eq!(st, 0, "voxrt: hipMemcpy to the host failed");
    }
}
