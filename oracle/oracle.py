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


def gemm_ep_vnni(wq, sq, out, inp, group, x, xs, gsum, y, ep=EP_STORE, alpha=0.0, threads=1, blocks_mult=8):
    n = x.shape[0]
    lib().or_gemm_ep_vnni(_p(wq), _p(sq), out, inp, group, _p(x), _p(xs), _p(gsum), n, _p(y), ep, alpha, threads,
                          blocks_mult)
