"""Host-side mirror of voxrt's kernel-dispatch surface over the C ABI of libvoxrt_hip.so.

Names, argument meaning and error behaviour follow the reference:
  Epilogue                    kernels/mod.rs:14-21  (Store, Silu, AddScaled(s))
  Kernel, detect, kernel      kernels/mod.rs:52-149 (Kernel.Hip added beside the CPU backends)
  TernaryMatrix               packed.rs:48-60       (from_packed, from_packed_f32, from_i8_rows; device resident)
  QuantAct                    packed.rs:286-298     (quantize: int8 codes, scales and gsum on the device)
  gemm / gemm_ep              kernels/mod.rs:319-362
  gemm_rows_range             kernels/mod.rs:257-282
  gemm_single                 kernels/mod.rs:285-316
  QuantAct.quantize_normed    ternary_linear.rs:132-155 (LayerNorm fused into the quantizer)

Activations and outputs are torch tensors on the current HIP device (torch is the device-memory and stream
plumbing here); every call is ordered on torch's current stream. The HIP library must be built: nothing here falls
back to a CPU path.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvoxrt_hip.so")

VX_OK, VX_ERR_INVALID, VX_ERR_NO_DEVICE, VX_ERR_HIP, VX_ERR_OOM = 0, 1, 2, 3, 4
EP_STORE, EP_SILU, EP_ADD_SCALED = 0, 1, 2


class HipError(RuntimeError):
    """A failed C-ABI call: `status` is the vx_status, the message is vx_last_error()."""

    def __init__(self, status: int, message: str):
        super().__init__(f"vx status {status}: {message}")
        self.status = status


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python voxrt_amd/build.py` (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        P, I64, I, F = C.c_void_p, C.c_int64, C.c_int, C.c_float
        sig = {
            "vx_last_error": (C.c_char_p, []),
            "vx_detect": (I, []),
            "vx_init": (I, [I]),
            "vx_shutdown": (I, []),
            "vx_set_kernel_override": (I, [C.c_char_p, C.c_char_p]),
            "vx_tmat_upload_packed": (I, [P, P, I64, I64, I64, C.POINTER(P)]),
            "vx_tmat_upload_packed_f32": (I, [P, P, I64, I64, I64, C.POINTER(P)]),
            "vx_tmat_upload_i8": (I, [P, P, I64, I64, I64, C.POINTER(P)]),
            "vx_tmat_upload_trits": (I, [P, P, I64, I64, I64, C.POINTER(P)]),
            "vx_tmat_free": (None, [P]),
            "vx_tmat_info": (I, [P, C.POINTER(I64), C.POINTER(I64), C.POINTER(I64), C.POINTER(I)]),
            "vx_quantize": (I, [P, I64, I64, I64, P, P, P, P]),
            "vx_gemm_ep": (I, [P, P, P, P, I64, P, P, I, F, P, P]),
            "vx_gemm_ep_quantize": (I, [P, P, P, P, I64, P, P, I, I64, P, P, P, P]),
            "vx_gemm_rows_range": (I, [P, P, P, P, I64, P, I64, I64, I64, I64, I, F, P]),
            "vx_gemm_single": (I, [P, P, P, P, I64, P, P, P]),
            "vx_quantize_normed": (I, [P, I64, I64, I64, P, P, P, P, P, P]),
            "vx_layer_norm": (I, [P, I64, I64, P, P, P, P]),
            "vx_glu_dwconv_silu": (I, [P, I64, I64, I64, P, P, P, P]),
            "vx_glu_dwconv_silu_quantize": (I, [P, I64, I64, I64, P, P, I64, P, P, P, P]),
            "vx_fold_bn": (I, [P, P, P, P, P, I64, I64, P, P]),
            "vx_linear_f32": (I, [P, I64, I64, P, P, I64, P, I, P]),
            "vx_subsampling_frames": (I64, [I64, I64, I64]),
            "vx_subsampling_scratch_floats": (I64, [I64, I64, I64, I64, I64]),
            "vx_subsampling": (I, [P, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, P, I64, P, P,
                                   C.POINTER(I64), P]),
            "vx_rel_pos_table": (I, [I64, I64, P]),
            "vx_attention_ws_bytes": (I64, [I64, I64, I64]),
            "vx_check_activations": (I, [P]),
            "vx_attention_core": (I, [P, P, I64, I64, I64, P, P, F, P, P, P]),
            "vx_attention_core_noalloc": (I, [P, P, I64, I64, I64, P, P, F, P, P]),
            "vx_attention_core_quantize": (I, [P, P, I64, I64, I64, P, P, F, P, I64, P, P, P, P]),
            "vx_encoder_create": (I, [P, C.POINTER(P)]),
            "vx_encoder_set_layer": (I, [P, I64, P]),
            "vx_encoder_set_subsampling": (I, [P, P]),
            "vx_encoder_use_graphs": (I, [P, I]),
            "vx_encoder_forward": (I, [P, P, P, I64, P]),
            "vx_encoder_forward_feats": (I, [P, P, I64, P, C.POINTER(I64), P]),
            "vx_encoder_forward_batch": (I, [P, P, P, I64, I64, P]),
            "vx_encoder_forward_feats_batch": (I, [P, P, I64, I64, P, C.POINTER(I64), P]),
            "vx_encoder_free": (None, [P]),
            "vx_encoder_set_profiling": (I, [P, I]),
            "vx_encoder_take_profile": (I, [P, P]),
            "vx_encoder_memory": (I, [P, C.POINTER(I64), C.POINTER(I64)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != VX_OK:
        raise HipError(status, lib().vx_last_error().decode(errors="replace"))


class Kernel(enum.Enum):
    """kernels/mod.rs:52-60 plus the MI355X backend."""
    Scalar = "scalar"
    Avx2 = "avx2"
    Avx512Vnni = "vnni"
    NeonDotprod = "sdot"
    NeonI8mm = "i8mm"
    Hip = "hip"


def detect() -> Kernel:
    """Kernel.Hip when a gfx950 device is visible, else Kernel.Scalar (the CPU kernels live in the reference)."""
    return Kernel.Hip if lib().vx_detect() else Kernel.Scalar


def kernel() -> Kernel:
    """VOXRT_KERNEL=hip forces the HIP backend when it can run (an override the machine cannot run falls back to
    detection, kernels/mod.rs:126-149)."""
    want = os.environ.get("VOXRT_KERNEL", "")
    best = detect()
    if want == "hip" and best == Kernel.Hip:
        return Kernel.Hip
    return best


def set_kernel_override(name: str, value) -> None:
    """Force a GEMM kernel choice (vx_set_kernel_override): gemm=direct|splitk|lds|big|splitg|small|stream,
    tile / small_tile="MTxNT", stream_grid=<workgroups>; None or "" clears it. For tests and tuning."""
    check(lib().vx_set_kernel_override(name.encode(), None if value in (None, "") else str(value).encode()))


class kernel_override:
    """Context manager: kernel_override(gemm="stream", stream_grid=8) forces those choices inside the block."""

    def __init__(self, **kw):
        self.kw = kw

    def __enter__(self):
        for k, v in self.kw.items():
            set_kernel_override(k, v)
        return self

    def __exit__(self, *exc):
        for k in self.kw:
            set_kernel_override(k, None)
        return False


@dataclass(frozen=True)
class Epilogue:
    kind: int
    alpha: float = 0.0

    @staticmethod
    def AddScaled(s: float) -> "Epilogue":
        return Epilogue(EP_ADD_SCALED, float(s))


Epilogue.Store = Epilogue(EP_STORE)
Epilogue.Silu = Epilogue(EP_SILU)


def _np_ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


def _stream(stream=None):
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _dev_ptr(t, dtype, name, shape=None):
    """Device address of a contiguous tensor of `dtype`; with `shape`, the tensor must have exactly that shape (the
    kernels read and write every element of the shape the call implies, so a smaller tensor would be overrun)."""
    import torch

    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if t.dtype != dtype or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous {dtype} tensor")
    if shape is not None and tuple(t.shape) != tuple(int(v) for v in shape):
        raise ValueError(f"{name} must have shape {tuple(int(v) for v in shape)}, not {tuple(t.shape)}")
    return C.c_void_p(t.data_ptr())


def _act_ptrs(x: "QuantAct"):
    """The three device operands of a QuantAct, each checked against its n, inp and group."""
    import torch

    ng = x.inp // x.group
    return (_dev_ptr(x.x, torch.int8, "x", (x.n, x.inp)),
            _dev_ptr(x.scales_t, torch.float32, "scales_t", (ng, npad(x.n))),
            _dev_ptr(x.gsum_t, torch.int32, "gsum_t", (ng, npad(x.n))))


class TernaryMatrix:
    """Device-resident weight matrix [out, inp] (packed.rs:48-60); repacked into the MFMA layout at upload."""

    def __init__(self, handle: C.c_void_p, out: int, inp: int, group: int, ternary: bool):
        self._h = handle
        self.out, self.inp, self.group, self.ternary = out, inp, group, ternary

    @classmethod
    def from_packed(cls, qweight, scales_f16, out: int, inp: int, group: int) -> "TernaryMatrix":
        """thrush-ternary-v2 rows uint8 [out, ceil(inp/5)] + IEEE binary16 scales [out, inp/group]
        (TernaryMatrix::from_packed_layout, packed.rs:73-130)."""
        q = np.ascontiguousarray(qweight, np.uint8)
        s = np.ascontiguousarray(np.asarray(scales_f16).view(np.uint16) if np.asarray(scales_f16).dtype != np.uint16
                                 else scales_f16, np.uint16)
        if q.size != out * ((inp + 4) // 5) or s.size != out * (inp // max(group, 1)):
            raise ValueError("qweight/scales sizes do not match out, inp, group")
        h = C.c_void_p()
        check(lib().vx_tmat_upload_packed(_np_ptr(q), _np_ptr(s), out, inp, group, C.byref(h)))
        return cls(h, out, inp, group, True)

    @classmethod
    def from_packed_f32(cls, qweight, scales, out: int, inp: int, group: int) -> "TernaryMatrix":
        """As from_packed with float32 scales [out, inp/group]."""
        q = np.ascontiguousarray(qweight, np.uint8)
        s = np.ascontiguousarray(scales, np.float32)
        if q.size != out * ((inp + 4) // 5) or s.size != out * (inp // max(group, 1)):
            raise ValueError("qweight/scales sizes do not match out, inp, group")
        h = C.c_void_p()
        check(lib().vx_tmat_upload_packed_f32(_np_ptr(q), _np_ptr(s), out, inp, group, C.byref(h)))
        return cls(h, out, inp, group, True)

    @classmethod
    def from_trits(cls, trits, scales, out: int, inp: int, group: int) -> "TernaryMatrix":
        """An unpacked ternary matrix: int8 rows [out, inp] in {-1, 0, +1} with float32 scales [out, inp/group]
        (TernaryMatrix in the Rows layout, packed.rs:48-60), uploaded as ternary (2-bit layout)."""
        r = np.ascontiguousarray(trits, np.int8)
        s = np.ascontiguousarray(scales, np.float32)
        if r.size != out * inp or s.size != out * (inp // max(group, 1)):
            raise ValueError("trits/scales sizes do not match out, inp, group")
        h = C.c_void_p()
        check(lib().vx_tmat_upload_trits(_np_ptr(r), _np_ptr(s), out, inp, group, C.byref(h)))
        return cls(h, out, inp, group, True)

    @classmethod
    def from_i8_rows(cls, rows, scales, out: int, inp: int, group: int) -> "TernaryMatrix":
        """Arbitrary int8 rows [out, inp] with float32 scales [out, inp/group] (packed.rs:164-201)."""
        r = np.ascontiguousarray(rows, np.int8)
        s = np.ascontiguousarray(scales, np.float32)
        if r.size != out * inp or s.size != out * (inp // max(group, 1)):
            raise ValueError("rows/scales sizes do not match out, inp, group")
        h = C.c_void_p()
        check(lib().vx_tmat_upload_i8(_np_ptr(r), _np_ptr(s), out, inp, group, C.byref(h)))
        return cls(h, out, inp, group, False)

    def groups(self) -> int:
        return self.inp // self.group

    def free(self) -> None:
        if self._h is not None and self._h.value:
            lib().vx_tmat_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def npad(n: int) -> int:
    """Padded token count of the transposed activation tables (VX_NPAD)."""
    return (n + 15) // 16 * 16


class QuantAct:
    """Quantised activations on the device (packed.rs:286-298): codes int8 [n, inp], and the per-(token, group)
    scales and code sums transposed, scales_t float32 [ng, npad(n)] and gsum_t int32 [ng, npad(n)]
    (QuantAct::scales_t, packed.rs:294; pad tokens zero)."""

    def __init__(self, q, scales_t, gsum_t, n: int, inp: int, group: int):
        self.x, self.scales_t, self.gsum_t = q, scales_t, gsum_t
        self.n, self.inp, self.group = n, inp, group

    @property
    def scales(self):
        """[n, ng] view of the scales (QuantAct::scales)."""
        return self.scales_t[:, : self.n].t()

    @property
    def gsum(self):
        """[n, ng] view of the code sums (QuantAct::gsum)."""
        return self.gsum_t[:, : self.n].t()

    @classmethod
    def quantize_normed(cls, x, gamma, beta, group: int, stream=None) -> "QuantAct":
        """QuantAct::from_rows over LayerNorm rows (TernaryLinear::prepare_normed, ternary_linear.rs:132-155)."""
        import torch

        if x.dim() != 2:
            raise ValueError("x must be [n, inp]")
        n, inp = x.shape
        if group <= 0 or inp % group:
            raise ValueError("inp must be a multiple of group")
        q = torch.empty((n, inp), dtype=torch.int8, device=x.device)
        s = torch.empty((inp // group, npad(n)), dtype=torch.float32, device=x.device)
        g = torch.empty((inp // group, npad(n)), dtype=torch.int32, device=x.device)
        check(lib().vx_quantize_normed(_dev_ptr(x, torch.float32, "x"), n, inp, group,
                                       _dev_ptr(gamma, torch.float32, "gamma", (inp,)),
                                       _dev_ptr(beta, torch.float32, "beta", (inp,)),
                                       _dev_ptr(q, torch.int8, "q"), _dev_ptr(s, torch.float32, "scales_t"),
                                       _dev_ptr(g, torch.int32, "gsum_t"), _stream(stream)))
        return cls(q, s, g, n, inp, group)

    @classmethod
    def quantize(cls, x, group: int, stream=None) -> "QuantAct":
        """QuantAct::quantize_layout (packed.rs:307-436) on a float32 device tensor [n, inp]."""
        import torch

        if x.dim() != 2:
            raise ValueError("x must be [n, inp]")
        n, inp = x.shape
        if group <= 0 or inp % group:
            raise ValueError("inp must be a multiple of group")
        q = torch.empty((n, inp), dtype=torch.int8, device=x.device)
        s = torch.empty((inp // group, npad(n)), dtype=torch.float32, device=x.device)
        g = torch.empty((inp // group, npad(n)), dtype=torch.int32, device=x.device)
        check(lib().vx_quantize(_dev_ptr(x, torch.float32, "x"), n, inp, group, _dev_ptr(q, torch.int8, "q"),
                                _dev_ptr(s, torch.float32, "scales_t"), _dev_ptr(g, torch.int32, "gsum_t"),
                                _stream(stream)))
        return cls(q, s, g, n, inp, group)


def gemm_ep(w: TernaryMatrix, x: QuantAct, y, bias=None, ep: Epilogue = Epilogue.Store, group_sums=None,
            stream=None) -> None:
    """y[n, out] = ep(y, x . w^T) (+ bias) (kernels/mod.rs:324-362); optional exact int32 group sums
    [inp/group, n, out]."""
    import torch

    if x.inp != w.inp or x.group != w.group:
        raise ValueError("activation and weight shapes or groups differ")
    check(lib().vx_gemm_ep(w._h, *_act_ptrs(x), x.n, _dev_ptr(y, torch.float32, "y", (x.n, w.out)),
                           _dev_ptr(bias, torch.float32, "bias", (w.out,)), ep.kind, ep.alpha,
                           _dev_ptr(group_sums, torch.int32, "group_sums", (w.groups(), x.n, w.out)),
                           _stream(stream)))


def gemm_ep_quantize(w: TernaryMatrix, x: QuantAct, bias=None, ep: Epilogue = Epilogue.Silu, group: int = 128,
                     y_tmp=None, stream=None) -> QuantAct:
    """The FFN up-projection with the next GEMM's quantization fused (encoder.rs:87-89: forward_prepared_ep into
    hbuf, then prepare(hbuf)): QuantAct of ep(x . w^T) (+ bias) in `group`-column groups, equal to gemm_ep followed
    by QuantAct.quantize. y_tmp float32 [n, out] is scratch for shapes the fused epilogue does not take (allocated
    here when None)."""
    import torch

    if x.inp != w.inp or x.group != w.group:
        raise ValueError("activation and weight shapes or groups differ")
    if ep.kind not in (Epilogue.Store.kind, Epilogue.Silu.kind):
        raise ValueError("a quantized output takes the Store or Silu epilogue")
    if group <= 0 or w.out % group:
        raise ValueError("out must be a multiple of group")
    dev = x.x.device
    n = x.n
    if y_tmp is None and not (group == 128 and n <= 1024 and w.out % 128 == 0):
        y_tmp = torch.empty((n, w.out), dtype=torch.float32, device=dev)
    q = torch.empty((n, w.out), dtype=torch.int8, device=dev)
    s = torch.empty((w.out // group, npad(n)), dtype=torch.float32, device=dev)
    g = torch.empty((w.out // group, npad(n)), dtype=torch.int32, device=dev)
    check(lib().vx_gemm_ep_quantize(w._h, *_act_ptrs(x), n, _dev_ptr(y_tmp, torch.float32, "y_tmp", (n, w.out)),
                                    _dev_ptr(bias, torch.float32, "bias", (w.out,)), ep.kind, group,
                                    _dev_ptr(q, torch.int8, "q"), _dev_ptr(s, torch.float32, "scales_t"),
                                    _dev_ptr(g, torch.int32, "gsum_t"), _stream(stream)))
    return QuantAct(q, s, g, n, w.out, group)


def gemm(w: TernaryMatrix, x: QuantAct, y, bias=None, stream=None) -> None:
    gemm_ep(w, x, y, bias, Epilogue.Store, stream=stream)


def gemm_rows_range(w: TernaryMatrix, x: QuantAct, y, r0: int, r1: int, t0: int, t1: int,
                    ep: Epilogue = Epilogue.Store, stream=None) -> None:
    """Rows [r0, r1) x tokens [t0, t1) of y[n, out] only (kernels/mod.rs:257-282)."""
    import torch

    if x.inp != w.inp or x.group != w.group:
        raise ValueError("activation and weight shapes or groups differ")
    check(lib().vx_gemm_rows_range(w._h, *_act_ptrs(x), x.n, _dev_ptr(y, torch.float32, "y", (x.n, w.out)), r0, r1,
                                   t0, t1, ep.kind, ep.alpha, _stream(stream)))


def gemm_single(w: TernaryMatrix, x: QuantAct, y, bias=None, stream=None) -> None:
    """y[n, out] = x . w^T, then y += bias (kernels/mod.rs:285-316; the decoder's single-token GEMV)."""
    import torch

    if x.inp != w.inp or x.group != w.group:
        raise ValueError("activation and weight shapes or groups differ")
    check(lib().vx_gemm_single(w._h, *_act_ptrs(x), x.n, _dev_ptr(y, torch.float32, "y", (x.n, w.out)),
                               _dev_ptr(bias, torch.float32, "bias", (w.out,)), _stream(stream)))


def check_activations() -> tuple:
    """Device self-check: mismatch counts (exp, SiLU, sigmoid) of the library's activation functions against the
    IEEE forms of tensor.rs:829-860 over all 2^32 float inputs; (0, 0, 0) on a correct build."""
    out = (C.c_uint64 * 3)()
    check(lib().vx_check_activations(C.cast(out, C.c_void_p)))
    return tuple(int(v) for v in out)
