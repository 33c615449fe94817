"""Synthetic inputs for the ternary x int8 GEMM workloads (numpy, host side).

The random stream is the 64-bit LCG of the reference's kernel tests (crates/voxrt/tests/kernels.rs:7-12):
``s = s * 6364136223846793005 + 1442695040888963407 (mod 2**64)``, output ``s >> 33``. ``lcg_stream`` produces
``n`` consecutive outputs at once by jump-ahead: with ``s_k = A_k * s_0 + C_k`` the coefficient pairs double as
``A_{m+j} = A_j A_m`` and ``C_{m+j} = A_j C_m + C_j``, so the whole stream costs O(n) vector work in log2(n)
rounds instead of an n-step Python loop.

Workload distributions: trits with P(0)=0.4, P(-1)=P(+1)=0.3 (``u = lcg % 10``: 0-3 -> 0, 4-6 -> -1, 7-9 -> +1),
per-output-channel scales ``f16(0.01 + 0.04 U)``, activations N(0,1) by Box-Muller in float64 cast to float32.
"""
from __future__ import annotations

import numpy as np

LCG_A = np.uint64(6364136223846793005)
LCG_C = np.uint64(1442695040888963407)


def lcg_stream(seed: int, n: int) -> tuple[np.ndarray, int]:
    """The next ``n`` outputs (uint32) of the LCG started at ``seed``, and the state after them."""
    if n <= 0:
        return np.zeros(0, np.uint32), seed
    with np.errstate(over="ignore"):
        a = np.empty(n, np.uint64)
        c = np.empty(n, np.uint64)
        a[0], c[0] = LCG_A, LCG_C
        m = 1
        while m < n:
            j = min(m, n - m)
            a[m:m + j] = a[:j] * a[m - 1]
            c[m:m + j] = a[:j] * c[m - 1] + c[:j]
            m += j
        s = a * np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + c
    return (s >> np.uint64(33)).astype(np.uint32), int(s[-1])


class Lcg:
    """Sequential consumer of the stream: ``take(n)`` returns the next n outputs."""

    def __init__(self, seed: int):
        self.state = seed & 0xFFFFFFFFFFFFFFFF

    def take(self, n: int) -> np.ndarray:
        out, self.state = lcg_stream(self.state, n)
        return out


def pack_rows(trits: np.ndarray) -> np.ndarray:
    """thrush-ternary-v2 packing of int8 trit rows [out, inp] -> uint8 [out, ceil(inp/5)]: 5 base-3 digits per
    byte, least significant first, digit = trit + 1, pad digits 0 (crates/voxrt/src/trits.rs:30-41)."""
    out, inp = trits.shape
    nb = (inp + 4) // 5
    d = np.zeros((out, nb * 5), np.uint16)
    d[:, :inp] = trits.astype(np.int16) + 1
    d = d.reshape(out, nb, 5)
    return (d[..., 0] + 3 * d[..., 1] + 9 * d[..., 2] + 27 * d[..., 3] + 81 * d[..., 4]).astype(np.uint8)


def unpack_rows(packed: np.ndarray, inp: int) -> np.ndarray:
    """Inverse of ``pack_rows`` (trits.rs:7-27)."""
    v = packed.astype(np.int16)
    digits = np.empty(packed.shape + (5,), np.int8)
    for i in range(5):
        digits[..., i] = v % 3 - 1
        v //= 3
    return digits.reshape(packed.shape[0], -1)[:, :inp].copy()


def workload_seed(config: int, role: int) -> int:
    """Seed of one input of a workload: 'voxr' in the top 32 bits, then the config and the role."""
    return 0x766F787200000000 | (config << 8) | role


def synth_trits(seed: int, out: int, inp: int) -> np.ndarray:
    u = Lcg(seed).take(out * inp) % 10
    t = np.zeros(out * inp, np.int8)
    t[(u >= 4) & (u <= 6)] = -1
    t[u >= 7] = 1
    return t.reshape(out, inp)


def synth_channel_scales_f16(seed: int, out: int, ng: int) -> np.ndarray:
    """One f16 scale per output channel, uniform in [0.01, 0.05], replicated over the ng groups: uint16 [out, ng]."""
    u = (Lcg(seed).take(out).astype(np.float64) + 0.5) / 2147483648.0
    s = (0.01 + 0.04 * u).astype(np.float32).astype(np.float16)
    return np.repeat(s[:, None], ng, axis=1).view(np.uint16).copy()


def synth_normal(seed: int, n: int) -> np.ndarray:
    """n float32 samples of N(0,1), Box-Muller in float64 over pairs of LCG uniforms."""
    m = (n + 1) // 2
    u = (Lcg(seed).take(2 * m).astype(np.float64) + 0.5) / 2147483648.0
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n].astype(np.float32)


def ref_random_matrix(rng: Lcg, out: int, inp: int, group: int = 128):
    """The reference tests' random ternary matrix (tests/kernels.rs:14-33): per row, ``inp`` trits
    ``lcg % 3 - 1`` then ``inp/128`` f16 scales ``0.01 + (lcg % 100) * 0.001``. Returns the packed rows, the f16
    scale codes [out, inp/group] and the trits."""
    ng = inp // group
    draws = rng.take(out * (inp + ng)).reshape(out, inp + ng)
    trits = (draws[:, :inp] % 3).astype(np.int8) - 1
    k = (draws[:, inp:] % 100).astype(np.float32)
    s = (np.float32(0.01) + k * np.float32(0.001)).astype(np.float32)
    return pack_rows(trits), s.astype(np.float16).view(np.uint16), trits


def ref_acts(rng: Lcg, n: int, inp: int, div: float = 100.0, off: float = 10.0) -> np.ndarray:
    """The reference tests' activations ``(lcg % 2001) as f32 / div - off`` (tests/kernels.rs:42-44)."""
    k = (rng.take(n * inp) % 2001).astype(np.float32)
    return (k / np.float32(div) - np.float32(off)).astype(np.float32).reshape(n, inp)


# ------------------------------------------------------------------------------- encoder parameters (synthetic)
#
# Random FastConformer weights for the encoder workloads (no checkpoint is available): ternary linears in the
# thrush-ternary-v2 format (packed trits + f16 scales per (row, 128-column group)), LayerNorm, relative-position
# biases, depthwise conv with BatchNorm statistics, and the subsampling convolutions. numpy's PCG64 seeded per
# (layer, tensor), so every run and both sides of a parity test see the same weights.

LAYER_LINEARS = ("ff1_w1", "ff1_w2", "qkv", "o", "pos", "pw1", "pw2", "ff2_w1", "ff2_w2")
LAYER_NORMS = ("ff1", "attn", "conv", "ff2", "out")


def _rng(layer: int, tensor: int) -> np.random.Generator:
    return np.random.default_rng([0x766F7872, layer, tensor])


def synth_ternary_linear(layer: int, tensor: int, out: int, inp: int, group: int = 128):
    """(packed uint8 [out, ceil(inp/5)], f16 scale codes uint16 [out, inp/group]); trits with P(0)=0.4,
    P(+-1)=0.3 and scales uniform in [0.01, 0.05]."""
    r = _rng(layer, tensor)
    u = r.integers(0, 10, size=(out, inp), dtype=np.int8)
    trits = np.zeros((out, inp), np.int8)
    trits[(u >= 4) & (u <= 6)] = -1
    trits[u >= 7] = 1
    s = r.uniform(0.01, 0.05, size=(out, inp // group)).astype(np.float16).view(np.uint16)
    return pack_rows(trits), s


def synth_layer(layer: int, d: int = 1024, ff: int = 4096, heads: int = 8, kconv: int = 9, group: int = 128):
    """One FastConformer layer's parameters as the model file holds them (before BatchNorm folding)."""
    shapes = {"ff1_w1": (ff, d), "ff1_w2": (d, ff), "qkv": (3 * d, d), "o": (d, d), "pos": (d, d),
              "pw1": (2 * d, d), "pw2": (d, d), "ff2_w1": (ff, d), "ff2_w2": (d, ff)}
    p = {"linears": {n: synth_ternary_linear(layer, i, *shapes[n], group) for i, n in enumerate(LAYER_LINEARS)}}
    r = _rng(layer, 100)
    f32 = np.float32
    p["norms"] = {n: ((1.0 + 0.1 * r.standard_normal(d)).astype(f32), (0.1 * r.standard_normal(d)).astype(f32))
                  for n in LAYER_NORMS}
    dh = d // heads
    p["bias_u"] = (0.1 * r.standard_normal((heads, dh))).astype(f32)
    p["bias_v"] = (0.1 * r.standard_normal((heads, dh))).astype(f32)
    p["dw"] = (r.standard_normal((d, kconv)) / 3.0).astype(f32)
    p["bn"] = {"gamma": (1.0 + 0.1 * r.standard_normal(d)).astype(f32), "beta": (0.1 * r.standard_normal(d)).astype(f32),
               "mean": (0.1 * r.standard_normal(d)).astype(f32), "var": r.uniform(0.5, 1.5, d).astype(f32)}
    return p


def synth_subsampling(d: int = 1024, c: int = 256, k: int = 3, n_mels: int = 128):
    """Subsampling weights in the layout the reference loads them to (subsampling.rs:32-104): conv0_w [k*k, C],
    dw_w [2, k*k, C], pw_w [2, C, C] (out, in), lin_w [d, f3*C] with channels-last columns."""
    r = _rng(1000, 0)
    f32 = np.float32
    f3 = n_mels
    for _ in range(3):
        f3 = (f3 - 1) // 2 + 1
    return {"k": k, "s": 2,
            "conv0_w": (r.standard_normal((k * k, c)) / 3.0).astype(f32), "conv0_b": (0.1 * r.standard_normal(c)).astype(f32),
            "dw_w": (r.standard_normal((2, k * k, c)) / 3.0).astype(f32), "dw_b": (0.1 * r.standard_normal((2, c))).astype(f32),
            "pw_w": (r.standard_normal((2, c, c)) / np.sqrt(c)).astype(f32), "pw_b": (0.1 * r.standard_normal((2, c))).astype(f32),
            "lin_w": (r.standard_normal((d, f3 * c)) / np.sqrt(f3 * c)).astype(f32), "lin_b": (0.1 * r.standard_normal(d)).astype(f32)}
