"""The benchmark workloads themselves, checked against the oracle at their real shapes through the C ABI.

- The linear set of one FastConformer layer at T = 338 (encoder.rs:79-94,138-293,582-630): the nine GEMMs of the
  bench's step, each with its own epilogue, with one group per row (G = K: per-output-channel scales, the single-GEMM
  workload's per-channel x per-token dequant) and with the model's 128-column groups (f16 scale per (row, group)).
  The calls go through vx_gemm_ep without a group-sum buffer, so the instantiations the bench times run here on
  their real grids. Every output is compared with the oracle's scalar kernel (kernels/mod.rs:166-210), bit for bit.
- The batched short-clip GEMMs: 64 clips of 2-15 s concatenated to 6987 rows, the FFN, q|k|v and pw1 shapes with
  one group and with 128-column groups, every output against the same scalar kernel.
- The 24-layer encoder from log-mel features (Encoder::forward, encoder.rs:816-856): one 60 s segment
  (6000 frames -> T = 750) and 32 segments of 10 s (1000 frames -> T = 125 each) in one batched pass, against the
  oracle's subsampling and 24 conformer layers, bit for bit.
"""
import os
import sys

import numpy as np
import pytest

from voxrt_amd import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


@pytest.fixture(scope="module")
def dev():
    import torch

    import voxrt_amd as vx

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    assert vx.detect() == vx.Kernel.Hip, "no gfx950 device"
    vx.kernels.check(vx.lib().vx_init(0))
    return torch.device("cuda:0")


def _bits_equal(got, want, what):
    g = np.ascontiguousarray(got, np.float32).view(np.uint32).ravel()
    w = np.ascontiguousarray(want, np.float32).view(np.uint32).ravel()
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ, first at {bad[0]}: got "
                           f"{np.asarray(got).ravel()[bad[0]]!r} want {np.asarray(want).ravel()[bad[0]]!r}")


def _layer_set():
    from bench import layer_shapes

    return layer_shapes(338)


@pytest.mark.parametrize("group", ["K", 128, "128ws"])
@pytest.mark.parametrize("idx", range(9), ids=[s[0] for s in _layer_set()])
def test_layer_linear_set_t338(dev, orc, idx, group):
    """One GEMM of the T = 338 layer set with the bench's operands (same seeds, trits, scales and activations),
    its epilogue over a random previous y for AddScaled: every output equal to the oracle. "128ws": the model's
    groups with the producer/consumer small-token kernel switched on."""
    import torch

    import voxrt_amd as vx

    name, m, k, n, ep, alpha = _layer_set()[idx]
    ws_on = group == "128ws"
    group = 128 if ws_on else group
    G = k if group == "K" else group
    ng = k // G
    role = 8 * idx
    trits = synth.synth_trits(synth.workload_seed(1, role), n, k)
    if G == k:  # the single-GEMM workload's per-output-channel scale (f16-representable, as the bench uses)
        s16 = synth.synth_channel_scales_f16(synth.workload_seed(1, role + 1), n, 1)
    else:  # the model format: one f16 scale per (row, 128-column group)
        s16 = synth.synth_ternary_linear(idx, 0, n, k, G)[1]
    x = synth.synth_normal(synth.workload_seed(1, role + 2), m * k).reshape(m, k)
    y0 = synth.synth_normal(synth.workload_seed(1, role + 3), m * n).reshape(m, n) if ep == 2 else \
        np.zeros((m, n), np.float32)
    w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n, k, G)
    xa = vx.QuantAct.quantize(torch.from_numpy(x).to(dev), G)
    y = torch.from_numpy(y0).to(dev)
    epi = {0: vx.Epilogue.Store, 1: vx.Epilogue.Silu}.get(ep) or vx.Epilogue.AddScaled(alpha)
    with vx.kernels.kernel_override(**({"small_ws": "on"} if ws_on else {})):
        vx.gemm_ep(w, xa, y, None, epi)
    torch.cuda.synchronize()
    q, xs, _ = orc.quantize(x, G)
    ws = orc.f16_to_f32(s16).reshape(n, ng)
    want = orc.gemm(trits, ws, q, xs, G, y=y0.copy(), ep=ep, alpha=alpha)
    _bits_equal(y.cpu().numpy(), want, f"{name} {m}x{k}x{n} G={G}")
    w.free()


def test_single_gemm_f32_channel_scales(dev, orc):
    """The single-GEMM workload as stated: M=338, K=1024, N=4096, one fp32 scale per output channel uniform in
    [0.01, 0.05] (not f16-rounded: uploaded with vx_tmat_upload_packed_f32), per-token int8 activations by absmax,
    fp32 output, every output equal to the oracle."""
    import torch

    import voxrt_amd as vx

    m, k, n = 338, 1024, 4096
    trits = synth.synth_trits(synth.workload_seed(0, 0), n, k)
    u = (synth.Lcg(synth.workload_seed(0, 1)).take(n).astype(np.float64) + 0.5) / 2147483648.0
    ws = (0.01 + 0.04 * u).astype(np.float32).reshape(n, 1)
    x = synth.synth_normal(synth.workload_seed(0, 2), m * k).reshape(m, k)
    w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n, k, k)
    xa = vx.QuantAct.quantize(torch.from_numpy(x).to(dev), k)
    y = torch.zeros((m, n), dtype=torch.float32, device=dev)
    vx.gemm_ep(w, xa, y)
    torch.cuda.synchronize()
    q, xs, _ = orc.quantize(x, k)
    _bits_equal(y.cpu().numpy(), orc.gemm(trits, ws, q, xs, k), "338x1024x4096 f32 channel scales")
    w.free()


# ------------------------------------------------------------------------- batched short clips (M = 6987)

@pytest.fixture(scope="module")
def clip_acts():
    """The batched short-clip workload's activations: 64 clips of 25 + lcg % 164 frames (2-15 s) concatenated,
    M = 6987 rows of N(0,1) for K = 1024 and K = 4096, with the bench's seeds."""
    lens = 25 + synth.Lcg(synth.workload_seed(2, 0)).take(64) % 164
    m = int(lens.sum())
    return {k: synth.synth_normal(synth.workload_seed(2, k >> 10), m * k).reshape(m, k) for k in (1024, 4096)}


@pytest.mark.parametrize("group", ["K", 128])
@pytest.mark.parametrize("name,k,n", [("ff_w1", 1024, 4096), ("ff_w2", 4096, 1024), ("qkv", 1024, 3072),
                                      ("pw1", 1024, 2048)])
def test_clip_batch_linears(dev, orc, clip_acts, name, k, n, group):
    """The batched short-clip workload (encoder GEMMs over 64 concatenated clips, Store as the bench times them)
    at its real row count, 6987 = 54 whole 128-token tiles on the large-token kernels plus 75 rows on the
    small-token kernels; one group per row and the model's 128-column groups: every output equal to the oracle."""
    import torch

    import voxrt_amd as vx

    x = clip_acts[k]
    m = x.shape[0]
    assert m == 6987
    G = k if group == "K" else group
    ng = k // G
    idx = ("ff_w1", "ff_w2", "qkv", "pw1").index(name)
    trits = synth.synth_trits(synth.workload_seed(2, 16 + 4 * idx), n, k)
    s16 = synth.synth_channel_scales_f16(synth.workload_seed(2, 17 + 4 * idx), n, ng) if G == k else \
        synth.synth_ternary_linear(idx, 1, n, k, G)[1]
    w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n, k, G)
    xa = vx.QuantAct.quantize(torch.from_numpy(x).to(dev), G)
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    vx.gemm_ep(w, xa, y, None, vx.Epilogue.Store)
    torch.cuda.synchronize()
    q, xs, _ = orc.quantize(x, G)
    want = orc.gemm(trits, orc.f16_to_f32(s16).reshape(n, ng), q, xs, G, threads=min(16, os.cpu_count() or 1))
    _bits_equal(y.cpu().numpy(), want, f"clip batch {name} {m}x{k}x{n} G={G}")
    w.free()


# ------------------------------------------------------------------------------------ the 24-layer encoder

@pytest.fixture(scope="module")
def model24(orc):
    """24 synthetic layers (the model's shapes and format) and the subsampling, with the oracle's unpacked copies."""
    layers = [synth.synth_layer(i) for i in range(24)]
    sp = synth.synth_subsampling()
    lps = []
    for p in layers:
        lp = {n: (orc.unpack_rows(q, s.shape[1] * 128), orc.f16_to_f32(s)) for n, (q, s) in p["linears"].items()}
        lp["norms"] = p["norms"]
        lp["bias_u"], lp["bias_v"] = p["bias_u"], p["bias_v"]
        lp["dw_t"], lp["dw_bias"] = orc.fold_bn(p["dw"], **p["bn"])
        orc.pack_layer_quad16(lp)
        lps.append(lp)
    return layers, sp, lps


def _oracle_encoder(orc, feats, sp, lps):
    x = orc.subsampling(feats, sp)
    pos = orc.rel_pos_table(x.shape[0], 1024)
    for lp in lps:
        x = orc.conformer_layer(x, pos, lp, heads=8)
    return x


@pytest.fixture(scope="module")
def enc24(dev, model24):
    from voxrt_amd import encoder as E

    layers, sp, _ = model24
    enc = E.Encoder(n_layers=24)
    for i, p in enumerate(layers):
        enc.set_layer(i, p)
    enc.set_subsampling(sp)
    yield enc
    enc.free()


def test_encoder_24_layers_60s_segment(dev, orc, model24, enc24):
    """One 60 s segment: 6000 log-mel frames -> T = 750 through subsampling and all 24 layers (graph replayed
    twice), equal to the oracle bit for bit."""
    import torch

    feats = np.random.default_rng(60).standard_normal((6000, 128)).astype(np.float32)
    want = _oracle_encoder(orc, feats, model24[1], model24[2])
    assert want.shape == (750, 1024)
    fd = torch.from_numpy(feats).to(dev)
    for rep in range(2):
        got = enc24.forward_feats(fd).cpu().numpy()
        _bits_equal(got, want, f"24-layer encoder, T=750 (pass {rep})")


def test_encoder_24_layers_32x10s_batch(dev, orc, model24, enc24):
    """32 segments of 10 s (1000 frames -> T = 125 each) in one batched pass through subsampling and all 24 layers:
    every segment equal to the oracle's encoder of that segment alone, bit for bit."""
    import torch

    feats = np.random.default_rng(10).standard_normal((32, 1000, 128)).astype(np.float32)
    got = enc24.forward_feats_batch(torch.from_numpy(feats).to(dev)).cpu().numpy()
    assert got.shape == (32, 125, 1024)
    for s in range(32):
        _bits_equal(got[s], _oracle_encoder(orc, feats[s], model24[1], model24[2]), f"32x10 s batch, segment {s}")
