"""ctypes view of liboracle.so — the CPU restatement of voxrt's ternary x int8 GEMM path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker (and the timed CPU baseline). The product path (voxrt_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

EP_STORE, EP_SILU, EP_ADD_SCALED = 0, 1, 2

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C oracle`)")
        L = C.CDLL(LIB_PATH)
        P, S, F, I = C.c_void_p, C.c_size_t, C.c_float, C.c_int
        sig = {
            "or_lcg": (C.c_uint32, [C.POINTER(C.c_uint64)]),
            "or_unpack_row": (None, [P, S, P]),
            "or_pack_row": (None, [P, S, P]),
            "or_f16_to_f32": (F, [C.c_uint16]),
            "or_f32_to_f16": (C.c_uint16, [F]),
            "or_f16_to_f32_n": (None, [P, S, P]),
            "or_dequant_matrix": (None, [P, P, S, S, S, P]),
            "or_unpack_matrix": (None, [P, S, S, P]),
            "or_quantize_group": (F, [P, S, P]),
            "or_quantize": (None, [P, S, S, S, P, P, P]),
            "or_exp_poly": (F, [F]),
            "or_silu_fast": (F, [F]),
            "or_sigmoid_fast": (F, [F]),
            "or_ep_apply": (F, [I, F, F, F]),
            "or_gemm_scalar_range": (None, [P, P, S, S, S, P, P, S, P, S, S, S, S, I, F, P]),
            "or_gemm_scalar_mt": (None, [P, P, S, S, S, P, P, S, P, I, F, P, I]),
            "or_have_vnni": (I, []),
            "or_quad16_bytes": (S, [S, S]),
            "or_quad16_pack": (None, [P, S, S, S, P, P, P]),
            "or_gemm_vnni_range": (None, [P, P, S, S, S, P, P, P, S, P, S, S, S, S, I, F]),
            "or_gemm_ep_vnni": (None, [P, P, S, S, S, P, P, P, S, P, I, F, I, S]),
            "or_have_avx2": (I, []),
            "or_gemm_avx2_range": (I, [P, P, S, S, S, I, P, P, P, S, P, S, S, S, S, I, F]),
            "or_get_threads": (I, []),
            "or_set_threads": (None, [I]),
            "or_row_mean_var": (None, [P, S, P, P]),
            "or_layer_norm": (None, [P, S, S, P, P, P]),
            "or_quantize_normed": (None, [P, S, S, S, P, P, P, P, P]),
            "or_exp_row_scaled": (F, [P, S, F]),
            "or_glu": (None, [P, S, S, P]),
            "or_fold_bn": (None, [P, P, P, P, P, S, S, P, P]),
            "or_dwconv_bn_silu": (None, [P, S, S, S, P, P, P]),
            "or_rel_pos_table": (None, [S, S, P]),
            "or_linear_f32": (None, [P, S, S, P, P, S, P]),
            "or_subsampling_frames": (S, [S, S, S]),
            "or_subsampling": (S, [P, S, S, S, S, S, P, P, P, P, P, P, P, P, S, P]),
            "or_attn_core_int8": (None, [P, P, S, S, S, P, P, F, P]),
            "or_conformer_layer": (None, [P, S, P, P, S, S, S, S, S, I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def lcg_outputs(seed: int, n: int) -> np.ndarray:
    s = C.c_uint64(seed)
    return np.array([lib().or_lcg(C.byref(s)) for _ in range(n)], np.uint32)


def unpack_rows(packed: np.ndarray, inp: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8)
    out = np.empty((packed.shape[0], inp), np.int8)
    lib().or_unpack_matrix(_p(packed), packed.shape[0], inp, _p(out))
    return out


def pack_row(trits: np.ndarray) -> np.ndarray:
    trits = np.ascontiguousarray(trits, np.int8)
    out = np.empty((trits.size + 4) // 5, np.uint8)
    lib().or_pack_row(_p(trits), trits.size, _p(out))
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_n(_p(h), h.size, _p(out))
    return out


def dequant_matrix(qweight: np.ndarray, scales_f16: np.ndarray, out: int, inp: int, group: int) -> np.ndarray:
    q = np.ascontiguousarray(qweight, np.uint8)
    s = np.ascontiguousarray(scales_f16, np.uint16)
    w = np.empty((out, inp), np.float32)
    lib().or_dequant_matrix(_p(q), _p(s), out, inp, group, _p(w))
    return w


def quantize(x: np.ndarray, group: int):
    """QuantAct::quantize_layout (Rows + gsum): int8 [n, inp], scales [n, ng], gsum [n, ng]."""
    x = np.ascontiguousarray(x, np.float32)
    n, inp = x.shape
    ng = inp // group
    q = np.empty((n, inp), np.int8)
    s = np.empty((n, ng), np.float32)
    g = np.empty((n, ng), np.int32)
    lib().or_quantize(_p(x), n, inp, group, _p(q), _p(s), _p(g))
    return q, s, g


def gemm_scalar_range(w, ws, x, xs, group, y, r0, r1, t0, t1, ep=EP_STORE, alpha=0.0, group_sums=None):
    """kernels/mod.rs:166-210 on int8 rows w [out, inp] with f32 scales ws [out, ng]; updates y [n, out] in place."""
    out, inp = w.shape
    n = x.shape[0]
    lib().or_gemm_scalar_range(_p(w), _p(ws), out, inp, group, _p(x), _p(xs), n, _p(y), r0, r1, t0, t1, ep,
                               alpha, _p(group_sums))


def gemm(w, ws, x, xs, group, y=None, ep=EP_STORE, alpha=0.0, want_group_sums=False, threads=None):
    """The whole [n, out] product on `threads` threads (defaults to all cores); returns y (and the group sums
    [ng, n, out] when asked)."""
    out, inp = w.shape
    n = x.shape[0]
    if y is None:
        y = np.zeros((n, out), np.float32)
    gs = np.empty((inp // group, n, out), np.int32) if want_group_sums else None
    lib().or_gemm_scalar_mt(_p(w), _p(ws), out, inp, group, _p(x), _p(xs), n, _p(y), ep, alpha, _p(gs),
                            threads or os.cpu_count() or 1)
    return (y, gs) if want_group_sums else y


def quad16_pack(rows: np.ndarray, scales: np.ndarray, group: int):
    rows = np.ascontiguousarray(rows, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    out, inp = rows.shape
    wq = np.empty(lib().or_quad16_bytes(out, inp), np.int8)
    sq = np.empty(((out + 15) // 16) * (inp // group) * 16, np.float32)
    lib().or_quad16_pack(_p(rows), out, inp, group, _p(scales), _p(wq), _p(sq))
    return wq, sq


def gemm_vnni_range(wq, sq, out, inp, group, x, xs, gsum, y, r0, r1, t0, t1, ep=EP_STORE, alpha=0.0):
    n = x.shape[0]
    lib().or_gemm_vnni_range(_p(wq), _p(sq), out, inp, group, _p(x), _p(xs), _p(gsum), n, _p(y), r0, r1, t0, t1,
                             ep, alpha)


def gemm_avx2_range(wq, sq, out, inp, group, ternary, x, xs, gsum, y, r0, r1, t0, t1, ep=EP_STORE, alpha=0.0):
    """The AVX2 restatement (x86.rs:163-290); returns -1 (nothing written) for ternary weights with group > 256."""
    n = x.shape[0]
    return lib().or_gemm_avx2_range(_p(wq), _p(sq), out, inp, group, int(bool(ternary)), _p(x), _p(xs), _p(gsum), n,
                                    _p(y), r0, r1, t0, t1, ep, alpha)


def gemm_ep_vnni(wq, sq, out, inp, group, x, xs, gsum, y, ep=EP_STORE, alpha=0.0, threads=1, blocks_mult=8):
    n = x.shape[0]
    lib().or_gemm_ep_vnni(_p(wq), _p(sq), out, inp, group, _p(x), _p(xs), _p(gsum), n, _p(y), ep, alpha, threads,
                          blocks_mult)


# ------------------------------------------------------------------------------------------------ encoder side

def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def row_mean_var(x):
    x = _f32(x)
    m, v = C.c_float(), C.c_float()
    lib().or_row_mean_var(_p(x), x.size, C.byref(m), C.byref(v))
    return m.value, v.value


def layer_norm(x, g, b):
    x, g, b = _f32(x), _f32(g), _f32(b)
    n, d = x.shape
    y = np.empty_like(x)
    lib().or_layer_norm(_p(x), n, d, _p(g), _p(b), _p(y))
    return y


def quantize_normed(x, g, b, group):
    x, g, b = _f32(x), _f32(g), _f32(b)
    n, inp = x.shape
    ng = inp // group
    q = np.empty((n, inp), np.int8)
    s = np.empty((n, ng), np.float32)
    gs = np.empty((n, ng), np.int32)
    lib().or_quantize_normed(_p(x), n, inp, group, _p(g), _p(b), _p(q), _p(s), _p(gs))
    return q, s, gs


def exp_row_scaled(row, scale):
    """Returns (exponentials, sum); the input is not modified."""
    r = _f32(row).copy()
    s = lib().or_exp_row_scaled(_p(r), r.size, scale)
    return r, s


def glu(gbuf):
    gbuf = _f32(gbuf)
    n, d2 = gbuf.shape
    out = np.empty((n, d2 // 2), np.float32)
    lib().or_glu(_p(gbuf), n, d2 // 2, _p(out))
    return out


def fold_bn(dw, gamma, beta, mean, var):
    dw = _f32(dw)
    d, k = dw.shape
    dw_t = np.empty((k, d), np.float32)
    bias = np.empty(d, np.float32)
    lib().or_fold_bn(_p(dw), _p(_f32(gamma)), _p(_f32(beta)), _p(_f32(mean)), _p(_f32(var)), d, k, _p(dw_t),
                     _p(bias))
    return dw_t, bias


def dwconv_bn_silu(a, dw_t, dw_bias):
    a, dw_t, dw_bias = _f32(a), _f32(dw_t), _f32(dw_bias)
    t, d = a.shape
    out = np.empty_like(a)
    lib().or_dwconv_bn_silu(_p(a), t, d, dw_t.shape[0], _p(dw_t), _p(dw_bias), _p(out))
    return out


def rel_pos_table(t, d):
    out = np.empty((2 * t - 1, d), np.float32)
    lib().or_rel_pos_table(t, d, _p(out))
    return out


def linear_f32(x, w, b=None):
    x, w = _f32(x), _f32(w)
    n, in_f = x.shape
    out_f = w.shape[0]
    y = np.empty((n, out_f), np.float32)
    lib().or_linear_f32(_p(x), n, in_f, _p(w), _p(None if b is None else _f32(b)), out_f, _p(y))
    return y


def subsampling_frames(t, k=3, s=2):
    return lib().or_subsampling_frames(t, k, s)


def subsampling(feats, sp):
    """sp: dict with conv0_w [k*k, C], conv0_b [C], dw_w [2, k*k, C], dw_b [2, C], pw_w [2, C, C], pw_b [2, C],
    lin_w [d, f3*C], lin_b [d], k, s."""
    feats = _f32(feats)
    t, n_mels = feats.shape
    c = sp["conv0_b"].shape[0]
    d = sp["lin_b"].shape[0]
    t3 = subsampling_frames(t, sp["k"], sp["s"])
    out = np.empty((t3, d), np.float32)
    keep = [_f32(sp[k]) for k in ("conv0_w", "conv0_b", "dw_w", "dw_b", "pw_w", "pw_b", "lin_w", "lin_b")]
    lib().or_subsampling(_p(feats), t, n_mels, c, sp["k"], sp["s"], *[_p(a) for a in keep], d, _p(out))
    return out


def attn_core_int8(qkv, rel_k, heads, bias_u, bias_v, scaling=None):
    qkv, rel_k = _f32(qkv), _f32(rel_k)
    t, d3 = qkv.shape
    d = d3 // 3
    if scaling is None:
        scaling = float(np.float32(1.0) / np.sqrt(np.float32(d // heads)))
    ctx = np.empty((t, d), np.float32)
    lib().or_attn_core_int8(_p(qkv), _p(rel_k), t, d, heads, _p(_f32(bias_u)), _p(_f32(bias_v)), scaling, _p(ctx))
    return ctx


LAYER_LINEARS = ("ff1_w1", "ff1_w2", "qkv", "o", "pos", "pw1", "pw2", "ff2_w1", "ff2_w2")
LAYER_NORMS = ("ff1", "attn", "conv", "ff2", "out")


def conformer_layer(x, pos_emb, lp, heads, kconv=9, group=128, threads=None):
    """One layer in place on a copy of x [t, d]; lp: dict with the 9 ternary linears as (trits int8 [out, inp],
    scales f32 [out, inp/group]) under LAYER_LINEARS, norms {name: (g, b)}, bias_u, bias_v, dw_t, dw_bias."""
    x = _f32(x).copy()
    t, d = x.shape
    ff = lp["ff1_w1"][0].shape[0]
    keep = [np.ascontiguousarray(lp[n][0], np.int8) for n in LAYER_LINEARS]
    keep += [_f32(lp[n][1]) for n in LAYER_LINEARS]
    for n in LAYER_NORMS:
        keep += [_f32(lp["norms"][n][0]), _f32(lp["norms"][n][1])]
    keep += [_f32(lp["bias_u"]), _f32(lp["bias_v"]), _f32(lp["dw_t"]), _f32(lp["dw_bias"])]
    addrs = [a.ctypes.data for a in keep]
    q16 = lp.get("quad16")  # {name: (wq, sq)} packed once (pack_layer_quad16), else packed per call
    for n in LAYER_LINEARS:
        if q16 is not None:
            keep += [q16[n][0], q16[n][1]]
            addrs += [q16[n][0].ctypes.data, q16[n][1].ctypes.data]
        else:
            addrs += [None, None]
    ptrs = (C.c_void_p * len(addrs))(*addrs)
    pos_emb = _f32(pos_emb)
    lib().or_conformer_layer(_p(x), t, _p(pos_emb), ptrs, d, heads, ff, kconv, group,
                             threads or os.cpu_count() or 1)
    return x


def set_threads(n: int) -> None:
    """Thread count of the oracle's parallel loops (results are the same for any count)."""
    lib().or_set_threads(int(n))


def pack_layer_quad16(lp, group=128):
    """Quad16 copies of a layer's 9 linears for the VNNI GEMM (TernaryLinear::load's repack), done once."""
    lp["quad16"] = {n: quad16_pack(lp[n][0], lp[n][1], group) for n in LAYER_LINEARS}
    return lp
