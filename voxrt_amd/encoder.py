"""Host-side mirror of voxrt's encoder surface on the MI355X path, over the C ABI of libvoxrt_hip.so.

  TernaryLinear          crates/voxrt/src/ternary_linear.rs:30-184 (load_stacked, prepare, prepare_normed,
                         forward_prepared_ep, forward) on device tensors, Int8 precision
  layer_norm             tensor.rs:700-719
  glu_dwconv_silu        encoder.rs:590-624 (the conv module between its pointwise convolutions)
  fold_bn                encoder.rs:548-573
  linear_f32             tensor.rs:98-127
  Subsampling            subsampling.rs:10-204 (forward, out_frames)
  rel_pos_table          encoder.rs:760-776
  attention_core         encoder.rs:317-534 (attn_core_int8, all heads)
  Encoder                GpuEncoder::{load, forward, forward_feats} (metal/mod.rs:446-603) with the CPU int8
                         Encoder's operation order (encoder.rs:706-857); one grow-only workspace, a bounded cache
                         of hipGraphs by (frames, segments); VOXRT_PROFILE=1 prints the per-sublayer profile of
                         every forward to stderr (encoder.rs:823-854)

Device tensors are torch tensors on the current HIP device; calls are ordered on torch's current stream. Nothing
here has a CPU fallback: every op is a HIP kernel of the library.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

from . import kernels as K
from .kernels import Epilogue, QuantAct, TernaryMatrix, check, lib

LAYER_LINEARS = ("ff1_w1", "ff1_w2", "qkv", "o", "pos", "pw1", "pw2", "ff2_w1", "ff2_w2")
LAYER_NORMS = ("ff1", "attn", "conv", "ff2", "out")


def _f32(t, name, shape=None):
    import torch

    return K._dev_ptr(t, torch.float32, name, shape)


def _dims(t, nd, name):
    if t.dim() != nd:
        raise ValueError(f"{name} must have {nd} dimensions, not {t.dim()}")
    return tuple(int(v) for v in t.shape)


class TernaryLinear:
    """A ternary linear layer on the int8 path (ternary_linear.rs:30-184); weights device resident."""

    def __init__(self, w: TernaryMatrix):
        self.w = w

    @classmethod
    def load_stacked(cls, parts, group: int = 128) -> "TernaryLinear":
        """Modules with the same input stacked along the output dimension (q|k|v): parts = [(qweight uint8
        [out_i, ceil(inp/5)], scales_f16 uint16 [out_i, inp/group]), ...] (ternary_linear.rs:59-98)."""
        qs = [np.ascontiguousarray(q, np.uint8) for q, _ in parts]
        ss = [np.ascontiguousarray(np.asarray(s).view(np.uint16), np.uint16) for _, s in parts]
        out = sum(q.shape[0] for q in qs)
        inp = ss[0].shape[1] * group
        if any(s.shape[1] * group != inp for s in ss) or any(q.shape[1] != (inp + 4) // 5 for q in qs):
            raise ValueError("cannot stack, shapes differ")
        return cls(TernaryMatrix.from_packed(np.concatenate(qs), np.concatenate(ss), out, inp, group))

    @classmethod
    def load(cls, qweight, scales_f16, group: int = 128) -> "TernaryLinear":
        return cls.load_stacked([(qweight, scales_f16)], group)

    @property
    def out_features(self) -> int:
        return self.w.out

    @property
    def in_features(self) -> int:
        return self.w.inp

    def prepare(self, x) -> QuantAct:
        """Quantize an input [n, in] once (ternary_linear.rs:118-130)."""
        return QuantAct.quantize(x, self.w.group)

    def prepare_normed(self, x, gamma, beta) -> QuantAct:
        """Fused LayerNorm -> int8 input (ternary_linear.rs:132-155)."""
        return QuantAct.quantize_normed(x, gamma, beta, self.w.group)

    def forward_prepared_ep(self, a: QuantAct, y, ep: Epilogue = Epilogue.Store) -> None:
        K.gemm_ep(self.w, a, y, None, ep)

    def forward_prepared(self, a: QuantAct, y) -> None:
        self.forward_prepared_ep(a, y, Epilogue.Store)

    def forward(self, x, y) -> None:
        self.forward_prepared(self.prepare(x), y)


def layer_norm(x, gamma, beta, y=None):
    import torch

    n, d = _dims(x, 2, "x")
    y = torch.empty_like(x) if y is None else y
    check(lib().vx_layer_norm(_f32(x, "x"), n, d, _f32(gamma, "gamma", (d,)), _f32(beta, "beta", (d,)),
                              _f32(y, "y", (n, d)), K._stream()))
    return y


def fold_bn(dw, gamma, beta, mean, var):
    """HOST: BatchNorm(eval) folded into the depthwise taps: dw [d, k] -> (w_t [k, d], bias [d])."""
    dw = np.ascontiguousarray(dw, np.float32)
    d, k = dw.shape
    w_t = np.empty((k, d), np.float32)
    bias = np.empty(d, np.float32)
    arrs = [np.ascontiguousarray(a, np.float32) for a in (gamma, beta, mean, var)]
    check(lib().vx_fold_bn(K._np_ptr(dw), *[K._np_ptr(a) for a in arrs], d, k, K._np_ptr(w_t), K._np_ptr(bias)))
    return w_t, bias


def glu_dwconv_silu(g, w_t, bias, out=None):
    """g [t, 2d] -> silu(dwconv_bn(glu(g))) [t, d]; w_t [k, d], bias [d] from fold_bn (device tensors)."""
    import torch

    t, d2 = _dims(g, 2, "g")
    d, k = d2 // 2, _dims(w_t, 2, "w_t")[0]
    out = torch.empty((t, d), dtype=torch.float32, device=g.device) if out is None else out
    check(lib().vx_glu_dwconv_silu(_f32(g, "g", (t, 2 * d)), t, d, k, _f32(w_t, "w_t", (k, d)),
                                   _f32(bias, "bias", (d,)), _f32(out, "out", (t, d)), K._stream()))
    return out


def glu_dwconv_silu_quantize(g, w_t, bias, group=128):
    """glu_dwconv_silu followed by pw2.prepare (encoder.rs:605-625) in one kernel: the QuantAct of the conv rows in
    128-channel groups."""
    import torch

    t, d2 = _dims(g, 2, "g")
    d, k = d2 // 2, _dims(w_t, 2, "w_t")[0]
    if group <= 0 or d % group:
        raise ValueError("d must be a multiple of group")
    q = torch.empty((t, d), dtype=torch.int8, device=g.device)
    s = torch.empty((d // group, K.npad(t)), dtype=torch.float32, device=g.device)
    gs = torch.empty((d // group, K.npad(t)), dtype=torch.int32, device=g.device)
    check(lib().vx_glu_dwconv_silu_quantize(_f32(g, "g", (t, 2 * d)), t, d, k, _f32(w_t, "w_t", (k, d)),
                                            _f32(bias, "bias", (d,)), group,
                                            K._dev_ptr(q, torch.int8, "q"), _f32(s, "scales_t"),
                                            K._dev_ptr(gs, torch.int32, "gsum_t"), K._stream()))
    return K.QuantAct(q, s, gs, t, d, group)


def linear_f32(x, w, b=None, relu=False, y=None):
    import torch

    n, in_f = _dims(x, 2, "x")
    out_f = _dims(w, 2, "w")[0]
    y = torch.empty((n, out_f), dtype=torch.float32, device=x.device) if y is None else y
    check(lib().vx_linear_f32(_f32(x, "x"), n, in_f, _f32(w, "w", (out_f, in_f)), _f32(b, "b", (out_f,)), out_f,
                              _f32(y, "y", (n, out_f)), int(relu), K._stream()))
    return y


def rel_pos_table(t: int, d: int) -> np.ndarray:
    """HOST: [2t-1, d] relative position table (encoder.rs:760-776)."""
    out = np.empty((2 * t - 1, d), np.float32)
    check(lib().vx_rel_pos_table(t, d, K._np_ptr(out)))
    return out


def attention_ws_bytes(t: int, d: int, heads: int) -> int:
    return int(lib().vx_attention_ws_bytes(t, d, heads))


def _attention_ws(t, d, heads, ws, device):
    """The attention core's device workspace: a new one, or the caller's uint8 tensor if it is large enough."""
    import torch

    nb = attention_ws_bytes(t, d, heads)
    if nb < 0:
        raise ValueError("attention: d must be heads * 128")
    if ws is None:
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=device)
    K._dev_ptr(ws, torch.uint8, "ws")
    if ws.numel() < nb:
        raise ValueError(f"ws must hold at least {nb} bytes")
    return C.c_void_p(ws.data_ptr())


def attention_core(qkv, rel_k, heads, bias_u, bias_v, ctx=None, ws=None):
    """The int8 attention core of one layer (attn_core_int8, encoder.rs:317-534): qkv [t, 3d], rel_k [2t-1, d],
    bias_u / bias_v [heads, 128] -> ctx [t, d]."""
    import torch

    t, d3 = _dims(qkv, 2, "qkv")
    d = d3 // 3
    ctx = torch.empty((t, d), dtype=torch.float32, device=qkv.device) if ctx is None else ctx
    ws = _attention_ws(t, d, heads, ws, qkv.device)
    scaling = float(np.float32(1.0) / np.sqrt(np.float32(d // heads)))
    dh = d // heads
    check(lib().vx_attention_core(_f32(qkv, "qkv", (t, 3 * d)), _f32(rel_k, "rel_k", (2 * t - 1, d)), t, d, heads,
                                  _f32(bias_u, "bias_u", (heads, dh)), _f32(bias_v, "bias_v", (heads, dh)), scaling,
                                  ws, _f32(ctx, "ctx", (t, d)), K._stream()))
    return ctx


def attention_core_quantize(qkv, rel_k, heads, bias_u, bias_v, group=128, ws=None):
    """attention_core followed by wo.prepare (encoder.rs:180-183) in one kernel: the QuantAct of ctx in 128-column
    groups, one per head."""
    import torch

    t, d3 = _dims(qkv, 2, "qkv")
    d = d3 // 3
    if group <= 0 or d % group:
        raise ValueError("d must be a multiple of group")
    ws = _attention_ws(t, d, heads, ws, qkv.device)
    dh = d // heads
    scaling = float(np.float32(1.0) / np.sqrt(np.float32(d // heads)))
    q = torch.empty((t, d), dtype=torch.int8, device=qkv.device)
    s = torch.empty((d // group, K.npad(t)), dtype=torch.float32, device=qkv.device)
    gs = torch.empty((d // group, K.npad(t)), dtype=torch.int32, device=qkv.device)
    check(lib().vx_attention_core_quantize(_f32(qkv, "qkv", (t, 3 * d)), _f32(rel_k, "rel_k", (2 * t - 1, d)), t,
                                           d, heads, _f32(bias_u, "bias_u", (heads, dh)),
                                           _f32(bias_v, "bias_v", (heads, dh)), scaling, ws, group, K._dev_ptr(q, torch.int8, "q"),
                                           _f32(s, "scales_t"), K._dev_ptr(gs, torch.int32, "gsum_t"), K._stream()))
    return K.QuantAct(q, s, gs, t, d, group)


SUB_KEYS = ("conv0_w", "conv0_b", "dw_w", "dw_b", "pw_w", "pw_b", "lin_w", "lin_b")


class Subsampling:
    """dw-striding Conv2d subsampling, 8x in time (subsampling.rs:10-204), device resident."""

    def __init__(self, params: dict, n_mels: int, device):
        import torch

        self.k, self.s = int(params["k"]), int(params["s"])
        self.c = params["conv0_b"].shape[0]
        self.d = params["lin_b"].shape[0]
        self.n_mels = n_mels
        self.host = {k: np.ascontiguousarray(params[k], np.float32) for k in SUB_KEYS}
        self.dev = {k: torch.from_numpy(v).to(device) for k, v in self.host.items()}

    def out_frames(self, t: int) -> int:
        return int(lib().vx_subsampling_frames(t, self.k, self.s))

    def forward(self, feats):
        import torch

        t, nm = _dims(feats, 2, "feats")
        if nm != self.n_mels:
            raise ValueError(f"feats must have {self.n_mels} mel columns")
        t3 = self.out_frames(t)
        out = torch.empty((t3, self.d), dtype=torch.float32, device=feats.device)
        scratch = torch.empty(int(lib().vx_subsampling_scratch_floats(t, nm, self.c, self.k, self.s)),
                              dtype=torch.float32, device=feats.device)
        got = C.c_int64()
        check(lib().vx_subsampling(_f32(feats, "feats"), t, nm, self.c, self.k, self.s,
                                   *[_f32(self.dev[k], k) for k in SUB_KEYS], self.d, _f32(scratch, "scratch"),
                                   _f32(out, "out"), C.byref(got), K._stream()))
        return out


class _Config(C.Structure):
    _fields_ = [(n, C.c_int64) for n in ("d", "heads", "ff", "kconv", "group", "n_layers", "n_mels", "sub_channels",
                                          "sub_kernel", "sub_stride")]


class _LayerParams(C.Structure):
    _fields_ = [("qweight", C.c_void_p * 9), ("scales_f16", C.c_void_p * 9), ("ln_gamma", C.c_void_p * 5),
                ("ln_beta", C.c_void_p * 5), ("bias_u", C.c_void_p), ("bias_v", C.c_void_p), ("dw", C.c_void_p),
                ("bn_gamma", C.c_void_p), ("bn_beta", C.c_void_p), ("bn_mean", C.c_void_p), ("bn_var", C.c_void_p)]


class _SubParams(C.Structure):
    _fields_ = [(k, C.c_void_p) for k in SUB_KEYS]


class _Profile(C.Structure):
    _fields_ = [(n, C.c_double) for n in ("total_ms", "subsampling_ms", "ff_ms", "attn_ms", "attn_core_ms", "conv_ms",
                                          "norm_ms")] + [("forwards", C.c_int64)]


class Encoder:
    """The FastConformer encoder on one GPU, int8 path (vx_encoder_*)."""

    def __init__(self, d=1024, heads=8, ff=4096, kconv=9, group=128, n_layers=24, n_mels=128, sub_channels=256,
                 sub_kernel=3, sub_stride=2):
        cfg = _Config(d, heads, ff, kconv, group, n_layers, n_mels, sub_channels, sub_kernel, sub_stride)
        h = C.c_void_p()
        check(lib().vx_encoder_create(C.byref(cfg), C.byref(h)))
        self._h = h
        self.d, self.heads, self.ff, self.kconv, self.group, self.n_layers = d, heads, ff, kconv, group, n_layers
        self.n_mels, self.sub_channels, self.sub_kernel, self.sub_stride = n_mels, sub_channels, sub_kernel, sub_stride
        self._print_profile = os.environ.get("VOXRT_PROFILE") is not None
        if self._print_profile:
            self.set_profiling(True)

    def set_layer(self, i: int, p: dict) -> None:
        """p: {"linears": {name: (qweight, scales_f16)}, "norms": {name: (g, b)}, "bias_u", "bias_v", "dw" [d, k],
        "bn": {"gamma", "beta", "mean", "var"}} as synth.synth_layer produces (the model file's tensors)."""
        keep = []

        def ptr(a, dtype, shape, name):
            a = np.asarray(a)
            if dtype == np.uint16 and a.dtype == np.float16:
                a = a.view(np.uint16)
            a = np.ascontiguousarray(a, dtype)
            if a.shape != tuple(shape):
                raise ValueError(f"layer {i}: {name} must have shape {tuple(shape)}, not {a.shape}")
            keep.append(a)
            return a.ctypes.data

        d, ff, G = self.d, self.ff, self.group
        dims = {"ff1_w1": (ff, d), "ff1_w2": (d, ff), "qkv": (3 * d, d), "o": (d, d), "pos": (d, d),
                "pw1": (2 * d, d), "pw2": (d, d), "ff2_w1": (ff, d), "ff2_w2": (d, ff)}
        lp = _LayerParams()
        for i_, n in enumerate(LAYER_LINEARS):
            q, s = p["linears"][n]
            out, inp = dims[n]
            lp.qweight[i_] = ptr(q, np.uint8, (out, (inp + 4) // 5), f"{n} qweight")
            lp.scales_f16[i_] = ptr(s, np.uint16, (out, inp // G), f"{n} scales")
        for i_, n in enumerate(LAYER_NORMS):
            g, b = p["norms"][n]
            lp.ln_gamma[i_] = ptr(g, np.float32, (d,), f"norm {n} weight")
            lp.ln_beta[i_] = ptr(b, np.float32, (d,), f"norm {n} bias")
        hd = (self.heads, d // self.heads)
        lp.bias_u, lp.bias_v = ptr(p["bias_u"], np.float32, hd, "bias_u"), ptr(p["bias_v"], np.float32, hd, "bias_v")
        lp.dw = ptr(p["dw"], np.float32, (d, self.kconv), "dw")
        bn = p["bn"]
        lp.bn_gamma, lp.bn_beta = ptr(bn["gamma"], np.float32, (d,), "bn gamma"), ptr(bn["beta"], np.float32, (d,), "bn beta")
        lp.bn_mean, lp.bn_var = ptr(bn["mean"], np.float32, (d,), "bn mean"), ptr(bn["var"], np.float32, (d,), "bn var")
        check(lib().vx_encoder_set_layer(self._h, i, C.byref(lp)))

    def set_subsampling(self, params: dict) -> None:
        arrs = {k: np.ascontiguousarray(params[k], np.float32) for k in SUB_KEYS}
        k, c, d = self.sub_kernel, self.sub_channels, self.d
        f3 = self.n_mels
        for _ in range(3):
            f3 = (f3 + 2 * ((k - 1) // 2) - k) // self.sub_stride + 1
        want = {"conv0_w": (k * k, c), "conv0_b": (c,), "dw_w": (2, k * k, c), "dw_b": (2, c), "pw_w": (2, c, c),
                "pw_b": (2, c), "lin_w": (d, f3 * c), "lin_b": (d,)}
        for key, shape in want.items():
            if arrs[key].shape != shape:
                raise ValueError(f"subsampling {key} must have shape {shape}, not {arrs[key].shape}")
        sp = _SubParams(*[arrs[k].ctypes.data for k in SUB_KEYS])
        check(lib().vx_encoder_set_subsampling(self._h, C.byref(sp)))

    def use_graphs(self, on: bool) -> None:
        check(lib().vx_encoder_use_graphs(self._h, int(on)))

    def set_profiling(self, on: bool) -> None:
        """Per-sublayer device timing of every forward (kernels launched one by one, events between sublayers)."""
        check(lib().vx_encoder_set_profiling(self._h, int(on)))

    def take_profile(self) -> dict:
        """Milliseconds per sublayer type summed over layers and over the forwards since the last take."""
        p = _Profile()
        check(lib().vx_encoder_take_profile(self._h, C.byref(p)))
        return {n: getattr(p, n) for n, _ in _Profile._fields_}

    def memory(self) -> tuple:
        """(workspace device bytes, graphs kept)."""
        b, g = C.c_int64(), C.c_int64()
        check(lib().vx_encoder_memory(self._h, C.byref(b), C.byref(g)))
        return int(b.value), int(g.value)

    def _after_forward(self, t: int) -> None:
        if self._print_profile:  # the reference's eprintln! line (encoder.rs:845-854), device times
            p = self.take_profile()
            print(f"encoder profile (Int8, HIP, T_e={t}): total {p['total_ms'] / 1e3:.3f}s · subsampling "
                  f"{p['subsampling_ms'] / 1e3:.3f} · ff {p['ff_ms'] / 1e3:.3f} · attn {p['attn_ms'] / 1e3:.3f} (core "
                  f"{p['attn_core_ms'] / 1e3:.3f}) · conv {p['conv_ms'] / 1e3:.3f} · norm {p['norm_ms'] / 1e3:.3f}",
                  file=sys.stderr)

    def forward(self, x, out=None):
        """The layer stack on x [t, d] (the subsampling output); returns out [t, d]."""
        import torch

        t, _ = _dims(x, 2, "x")
        out = torch.empty_like(x) if out is None else out
        check(lib().vx_encoder_forward(self._h, _f32(x, "x", (t, self.d)), _f32(out, "out", (t, self.d)), t,
                                       K._stream()))
        self._after_forward(t)
        return out

    def out_frames(self, t_in: int) -> int:
        return int(lib().vx_subsampling_frames(t_in, self.sub_kernel, self.sub_stride))

    def forward_feats(self, feats, out=None):
        """Subsampling + layers: feats [t_in, n_mels] -> [t_out, d]."""
        import torch

        t_in, _ = _dims(feats, 2, "feats")
        t3 = self.out_frames(t_in)
        out = torch.empty((t3, self.d), dtype=torch.float32, device=feats.device) if out is None else out
        got = C.c_int64()
        check(lib().vx_encoder_forward_feats(self._h, _f32(feats, "feats", (t_in, self.n_mels)), t_in,
                                             _f32(out, "out", (t3, self.d)), C.byref(got), K._stream()))
        self._after_forward(t3)
        return out

    def forward_batch(self, x, out=None):
        """The layer stack on nseg segments of equal length at once: x [nseg, t, d] -> out [nseg, t, d]; each
        segment's output equals forward() of that segment alone, bit for bit."""
        import torch

        nseg, t, _ = _dims(x, 3, "x")
        out = torch.empty_like(x) if out is None else out
        check(lib().vx_encoder_forward_batch(self._h, _f32(x, "x", (nseg, t, self.d)),
                                             _f32(out, "out", (nseg, t, self.d)), nseg, t, K._stream()))
        self._after_forward(t)
        return out

    def forward_feats_batch(self, feats, out=None):
        """Subsampling + layers on nseg segments of equal length: feats [nseg, t_in, n_mels] -> [nseg, t_out, d],
        each segment equal to forward_feats() of that segment alone."""
        import torch

        nseg, t_in, _ = _dims(feats, 3, "feats")
        t3 = self.out_frames(t_in)
        out = torch.empty((nseg, t3, self.d), dtype=torch.float32, device=feats.device) if out is None else out
        got = C.c_int64()
        check(lib().vx_encoder_forward_feats_batch(self._h, _f32(feats, "feats", (nseg, t_in, self.n_mels)), nseg,
                                                   t_in, _f32(out, "out", (nseg, t3, self.d)), C.byref(got),
                                                   K._stream()))
        self._after_forward(t3)
        return out

    def free(self) -> None:
        if self._h is not None and self._h.value:
            lib().vx_encoder_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
