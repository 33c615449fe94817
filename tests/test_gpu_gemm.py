"""HIP ternary x int8 GEMM == the oracle, bit for bit (int32 group sums and fp32 outputs), through the C ABI.

Restates the reference's kernel-exactness tests for the HIP backend: crates/voxrt/tests/kernels.rs
(simd_equals_scalar_exactly, epilogues_are_identical_across_kernels, accumulation_cannot_overflow,
row_token_ranges_equal_scalar_exactly with its NaN canary) and tests/x86_kernels.rs (ternary and int8 grids, four
row/token ranges x three epilogues, saturation extremes, the f32-rows operand), plus the quantizer, the stored
fixtures through the device repack, and the benchmark shapes.
"""
import json
import os

import numpy as np
import pytest

from voxrt_amd import synth

pytestmark = pytest.mark.gpu

FIX = os.path.join(os.path.dirname(__file__), "golden", "fixtures")


@pytest.fixture(scope="module")
def dev():
    import torch

    import voxrt_amd as vx

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    assert vx.detect() == vx.Kernel.Hip, "no gfx950 device"
    vx.kernels.check(vx.lib().vx_init(0))
    return torch.device("cuda:0")


def _t(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _assert_bits_equal(got, want, what):
    g, w = _bits(got), _bits(want)
    bad = np.flatnonzero(g.ravel() != w.ravel())
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: got {got.ravel()[bad[0]]!r} want {want.ravel()[bad[0]]!r}"


def _device_gemm(vx, dev, w, x_f32, group, y_init=None, ep=None, want_gs=False):
    import torch

    ep = ep or vx.Epilogue.Store
    xa = vx.QuantAct.quantize(_t(x_f32, dev), group)
    n = x_f32.shape[0]
    y = _t(y_init, dev) if y_init is not None else torch.zeros((n, w.out), dtype=torch.float32, device=dev)
    gs = torch.full((w.inp // group, n, w.out), -7, dtype=torch.int32, device=dev) if want_gs else None
    vx.gemm_ep(w, xa, y, None, ep, gs)
    torch.cuda.synchronize()
    return xa, y.cpu().numpy(), (gs.cpu().numpy() if want_gs else None)


def _ep_of(vx, ep_kind, alpha):
    return {0: vx.Epilogue.Store, 1: vx.Epilogue.Silu}.get(ep_kind) or vx.Epilogue.AddScaled(alpha)


# ------------------------------------------------------------------------------------------ quantizer

def test_quantize_equals_oracle(dev, orc):
    import voxrt_amd as vx

    rng = synth.Lcg(3)
    for n, inp, group in [(1, 128, 128), (17, 256, 128), (338, 1024, 1024), (338, 1024, 128), (5, 4096, 128),
                          (3, 384, 384), (8, 640, 128), (33, 4096, 4096), (40, 2048, 256), (21, 1024, 64),
                          (9, 3072, 1024)]:
        x = synth.ref_acts(rng, n, inp)
        x[0, :group] = 0.0  # an all-zero group
        x[-1, 1::7] = np.float32(0.5) * (np.arange(x[-1, 1::7].size) % 5).astype(np.float32)  # ties after scaling
        qa = vx.QuantAct.quantize(_t(x, dev), group)
        q, s, g = orc.quantize(x, group)
        np.testing.assert_array_equal(qa.x.cpu().numpy(), q)
        st, gt = qa.scales_t.cpu().numpy(), qa.gsum_t.cpu().numpy()
        assert st.shape == (inp // group, (n + 15) // 16 * 16)
        _assert_bits_equal(np.ascontiguousarray(st[:, :n].T), s, f"scales n={n} inp={inp} g={group}")
        np.testing.assert_array_equal(gt[:, :n].T, g)
        assert (st[:, n:] == 0).all() and (gt[:, n:] == 0).all(), "pad tokens must be zero"


# ------------------------------------------------------------------------------------------ kernels.rs

@pytest.mark.parametrize("out,inp", [(7, 128), (9, 256), (64, 1024), (130, 4096)])
def test_hip_equals_scalar_exactly(dev, orc, out, inp):
    """kernels.rs:35-53 (simd_equals_scalar_exactly) for the HIP kernel, plus the int32 group sums."""
    import voxrt_amd as vx

    rng = synth.Lcg(42 + out)
    qw, s16, trits = synth.ref_random_matrix(rng, out, inp)
    w = vx.TernaryMatrix.from_packed(qw, s16, out, inp, 128)
    ws = orc.f16_to_f32(s16)
    for n in [1, 3, 4, 5, 17]:
        x = synth.ref_acts(rng, n, inp)
        q, xs, _ = orc.quantize(x, 128)
        want, want_gs = orc.gemm(trits, ws, q, xs, 128, want_group_sums=True)
        _, got, got_gs = _device_gemm(vx, dev, w, x, 128, want_gs=True)
        np.testing.assert_array_equal(got_gs, want_gs, err_msg=f"group sums out={out} inp={inp} n={n}")
        _assert_bits_equal(got, want, f"y out={out} inp={inp} n={n}")


def test_epilogues_are_identical(dev, orc):
    """kernels.rs:91-112: Store, Silu, AddScaled(0.5) on a pre-filled y."""
    import voxrt_amd as vx

    rng = synth.Lcg(5)
    out, inp, n = 64, 1024, 13
    qw, s16, trits = synth.ref_random_matrix(rng, out, inp)
    w = vx.TernaryMatrix.from_packed(qw, s16, out, inp, 128)
    ws = orc.f16_to_f32(s16)
    x = synth.ref_acts(rng, n, inp)
    q, xs, _ = orc.quantize(x, 128)
    base = ((np.arange(n * out) % 7) - 3).astype(np.float32).reshape(n, out)
    for ep_kind, alpha in [(0, 0.0), (1, 0.0), (2, 0.5)]:
        want = orc.gemm(trits, ws, q, xs, 128, y=base.copy(), ep=ep_kind, alpha=alpha)
        _, got, _ = _device_gemm(vx, dev, w, x, 128, y_init=base, ep=_ep_of(vx, ep_kind, alpha))
        _assert_bits_equal(got, want, f"epilogue {ep_kind}")


def test_accumulation_cannot_overflow(dev):
    """kernels.rs:176-200: all +1 trits, x = 127, K = 4096, unit scales -> 4096 * 127."""
    import voxrt_amd as vx

    inp = 4096
    qw = synth.pack_rows(np.ones((1, inp), np.int8))
    s16 = np.full((1, inp // 128), np.float16(1.0)).view(np.uint16)
    w = vx.TernaryMatrix.from_packed(qw, s16, 1, inp, 128)
    _, y, gs = _device_gemm(vx, dev, w, np.full((1, inp), 127.0, np.float32), 128, want_gs=True)
    assert y[0, 0] == 4096 * 127.0
    assert (gs == 128 * 127).all()


def test_bias_is_added_after_epilogue(dev, orc):
    """gemm_ep adds the bias after the epilogue (kernels/mod.rs:355-361)."""
    import torch

    import voxrt_amd as vx

    rng = synth.Lcg(17)
    out, inp, n = 96, 256, 9
    qw, s16, trits = synth.ref_random_matrix(rng, out, inp)
    w = vx.TernaryMatrix.from_packed(qw, s16, out, inp, 128)
    x = synth.ref_acts(rng, n, inp)
    bias = (rng.take(out) % 100).astype(np.float32) / np.float32(10.0)
    q, xs, _ = orc.quantize(x, 128)
    want = orc.gemm(trits, orc.f16_to_f32(s16), q, xs, 128, ep=1)
    want = (want + bias[None, :]).astype(np.float32)
    xa = vx.QuantAct.quantize(_t(x, dev), 128)
    y = torch.zeros((n, out), dtype=torch.float32, device=dev)
    vx.gemm_ep(w, xa, y, _t(bias, dev), vx.Epilogue.Silu)
    _assert_bits_equal(y.cpu().numpy(), want, "bias")


@pytest.mark.parametrize("out,inp,n", [(14, 128, 11), (34, 128, 19), (8, 256, 8), (6, 128, 3)])
def test_row_token_ranges_with_nan_canary(dev, orc, out, inp, n):
    """kernels.rs:202-269: int8 (from_f32_rows) weights, every (row range, token range) equals the scalar kernel
    and nothing outside the block is written."""
    import torch

    import voxrt_amd as vx

    rng = synth.Lcg(7 + out)
    wf = synth.ref_acts(rng, out, inp)
    wq, wsc, _ = orc.quantize(wf, 128)  # from_f32_rows = per (row, group) absmax quantization
    w = vx.TernaryMatrix.from_i8_rows(wq, wsc, out, inp, 128)
    x = synth.ref_acts(rng, n, inp)
    q, xs, _ = orc.quantize(x, 128)
    want = orc.gemm(wq, wsc, q, xs, 128)
    xa = vx.QuantAct.quantize(_t(x, dev), 128)
    for r0, r1 in [(0, out), (2, out), (0, (out // 2) & ~1), (4, min(6, out))]:
        for t0, t1 in [(0, n), (0, min(n, 8)), (min(8, n) & ~1, n), (min(2, n), min(n, 5))]:
            if r0 >= r1 or t0 >= t1:
                continue
            y = torch.full((n, out), float("nan"), dtype=torch.float32, device=dev)
            vx.gemm_rows_range(w, xa, y, r0, r1, t0, t1)
            got = y.cpu().numpy()
            inside = np.zeros((n, out), bool)
            inside[t0:t1, r0:r1] = True
            assert (np.isnan(got) == ~inside).all(), f"stray write rows {r0}..{r1} toks {t0}..{t1}"
            _assert_bits_equal(got[inside], want[inside], f"rows {r0}..{r1} toks {t0}..{t1}")


# ------------------------------------------------------------------------------------------ x86_kernels.rs

def _check_ranges(vx, dev, orc, rng, w, rows, ws, group, x):
    import torch

    out, inp = rows.shape
    n = x.shape[0]
    q, xs, _ = orc.quantize(x, group)
    xa = vx.QuantAct.quantize(_t(x, dev), group)
    ranges = [(0, out, 0, n), (min(1, out), out, 0, n), (0, min(out, 17), n // 2, n),
              (out // 3, out - out // 4, 0, (n + 1) // 2)]
    for ep_kind, alpha in [(0, 0.0), (1, 0.0), (2, 0.37)]:
        for r0, r1, t0, t1 in ranges:
            if r0 >= r1 or t0 >= t1:
                continue
            init = ((rng.take(n * out) % 100).astype(np.float32) * np.float32(0.01)).reshape(n, out)
            want = init.copy()
            orc.gemm_scalar_range(rows, ws, q, xs, group, want, r0, r1, t0, t1, ep_kind, alpha)
            y = _t(init, dev)
            vx.gemm_rows_range(w, xa, y, r0, r1, t0, t1, _ep_of(vx, ep_kind, alpha))
            _assert_bits_equal(y.cpu().numpy(), want, f"out={out} inp={inp} g={group} n={n} {r0}..{r1} {t0}..{t1} ep={ep_kind}")


def test_x86_grid_ternary(dev, orc):
    """x86_kernels.rs:140-152 grid on the HIP kernel."""
    import voxrt_amd as vx

    rng = synth.Lcg(3)
    for out, inp in [(7, 128), (16, 256), (33, 1024), (130, 4096)]:
        qw, s16, trits = synth.ref_random_matrix(rng, out, inp)
        w = vx.TernaryMatrix.from_packed(qw, s16, out, inp, 128)
        for n in [1, 2, 3, 4, 5, 8, 9, 17]:
            _check_ranges(vx, dev, orc, rng, w, trits, orc.f16_to_f32(s16), 128, synth.ref_acts(rng, n, inp))


def test_x86_grid_int8(dev, orc):
    """x86_kernels.rs:154-172: arbitrary int8 weights, groups 128 / 384 / 1024."""
    import voxrt_amd as vx

    rng = synth.Lcg(5)
    for out, inp, group in [(7, 128, 128), (40, 640, 128), (128, 384, 384), (19, 1024, 1024)]:
        rows = ((rng.take(out * inp) % 255).astype(np.int32) - 127).astype(np.int8).reshape(out, inp)
        ws = (np.float32(0.001) + (rng.take(out * (inp // group)) % 1000).astype(np.float32) * np.float32(1e-5))
        ws = ws.astype(np.float32).reshape(out, inp // group)
        w = vx.TernaryMatrix.from_i8_rows(rows, ws, out, inp, group)
        for n in [1, 2, 5, 8, 11]:
            _check_ranges(vx, dev, orc, rng, w, rows, ws, group, synth.ref_acts(rng, n, inp))


def test_x86_extremes_do_not_saturate(dev, orc):
    """x86_kernels.rs:174-185."""
    import voxrt_amd as vx

    rng = synth.Lcg(9)
    trits = np.ones((32, 1024), np.int8)
    s16 = (np.float32(0.01) + (rng.take(32 * 8) % 100).astype(np.float32) * np.float32(0.001)).astype(np.float16)
    s16 = s16.view(np.uint16).reshape(32, 8)
    w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, 32, 1024, 128)
    x = np.where(np.arange(5 * 1024) % 2 == 0, 5.0, -5.0).astype(np.float32).reshape(5, 1024)
    _check_ranges(vx, dev, orc, rng, w, trits, orc.f16_to_f32(s16), 128, x)
    rows = np.where(np.arange(32 * 1024) % 2 == 0, 127, -127).astype(np.int8).reshape(32, 1024)
    ws = np.full((32, 1), 0.002, np.float32)
    w8 = vx.TernaryMatrix.from_i8_rows(rows, ws, 32, 1024, 1024)
    _check_ranges(vx, dev, orc, rng, w8, rows, ws, 1024, x)


# ------------------------------------------------------------------------------------------ fixtures

def test_fixture_rows_through_device_repack(dev, orc):
    """The reference's stored model rows (fixtures_trits.rs) uploaded in their on-disk format: the GEMM against
    one-hot activations returns the stored dequantised weights exactly, and random activations match the oracle."""
    import torch

    import voxrt_amd as vx

    meta = json.load(open(os.path.join(FIX, "ternary_fixtures.json")))
    for tag, m in meta.items():
        rows, inf, g = m["rows"], m["in_features"], m["group_size"]
        q = np.fromfile(os.path.join(FIX, f"{tag}.qweight.bin"), np.uint8).reshape(rows, -1)
        s = np.fromfile(os.path.join(FIX, f"{tag}.scales.f16.bin"), np.uint16).reshape(rows, -1)
        want_w = np.fromfile(os.path.join(FIX, f"{tag}.weight.f32.bin"), np.float32).reshape(rows, inf)
        trits = np.fromfile(os.path.join(FIX, f"{tag}.trits.i8.bin"), np.int8).reshape(rows, inf)
        w = vx.TernaryMatrix.from_packed(q, s, rows, inf, g)
        # one-hot token c has code 127 at column c and scale 1/127*... use x = 127 * e_c: s = 1, code 127
        eye = np.zeros((inf, inf), np.float32)
        eye[np.arange(inf), np.arange(inf)] = 127.0
        xa = vx.QuantAct.quantize(_t(eye, dev), g)
        y = torch.zeros((inf, rows), dtype=torch.float32, device=dev)
        vx.gemm(w, xa, y)
        got = y.cpu().numpy().T / np.float32(127.0)
        _assert_bits_equal(got.astype(np.float32), want_w, f"{tag} one-hot")
        rng = synth.Lcg(77)
        x = synth.ref_acts(rng, 19, inf)
        qq, xs, _ = orc.quantize(x, g)
        want = orc.gemm(trits, orc.f16_to_f32(s), qq, xs, g)
        _, got, _ = _device_gemm(vx, dev, w, x, g)
        _assert_bits_equal(got, want, f"{tag} random")


# ------------------------------------------------------------------------------------------ workload shapes

def _workload(orc, m, k, n_out, group, seed_cfg=0):
    trits = synth.synth_trits(synth.workload_seed(seed_cfg, 1), n_out, k)
    s16 = synth.synth_channel_scales_f16(synth.workload_seed(seed_cfg, 2), n_out, k // group)
    x = synth.synth_normal(synth.workload_seed(seed_cfg, 3), m * k).reshape(m, k)
    return trits, s16, x


@pytest.mark.parametrize("group", [1024, 128])
def test_ffn_up_t338_bit_exact(dev, orc, group):
    """The FFN up-projection of one layer at T=338 (M=338, K=1024, N=4096): per-channel scales with G=K (fp32
    scale upload) and the model's G=128 (f16 scales): int32 sums and fp32 outputs bit-exact."""
    import voxrt_amd as vx

    m, k, n_out = 338, 1024, 4096
    trits, s16, x = _workload(orc, m, k, n_out, group)
    ws = orc.f16_to_f32(s16)
    qw = synth.pack_rows(trits)
    w = vx.TernaryMatrix.from_packed_f32(qw, ws, n_out, k, group) if group == k else \
        vx.TernaryMatrix.from_packed(qw, s16, n_out, k, group)
    q, xs, _ = orc.quantize(x, group)
    want, want_gs = orc.gemm(trits, ws, q, xs, group, want_group_sums=True)
    _, got, got_gs = _device_gemm(vx, dev, w, x, group, want_gs=True)
    np.testing.assert_array_equal(got_gs, want_gs)
    _assert_bits_equal(got, want, f"T=338 FFN-up G={group}")


@pytest.mark.parametrize("k,n_out", [(1024, 4096), (4096, 1024)])
@pytest.mark.parametrize("per_channel", [False, True])
def test_batched_m8192_all_rows(dev, orc, k, n_out, per_channel):
    """M=8192 (the batched regime, the up- and down-projection shapes): every output of the 8192 tokens against
    the oracle's scalar kernel, bit-exact; G=128 (f16 scales) and per-channel G=K (fp32 scales, the large-token
    kernel). The oracle takes about a second per case on 16 host threads."""
    import os

    import voxrt_amd as vx

    m = 8192
    group = k if per_channel else 128
    trits, s16, x = _workload(orc, m, k, n_out, group, seed_cfg=2)
    ws = orc.f16_to_f32(s16)
    qw = synth.pack_rows(trits)
    w = vx.TernaryMatrix.from_packed_f32(qw, ws, n_out, k, group) if per_channel else \
        vx.TernaryMatrix.from_packed(qw, s16, n_out, k, group)
    _, got, _ = _device_gemm(vx, dev, w, x, group)
    q, xs, _ = orc.quantize(x, group)
    want = orc.gemm(trits, ws, q, xs, group, threads=min(16, os.cpu_count() or 1))
    _assert_bits_equal(got, want, f"M=8192 K={k} N={n_out} G={group}")


@pytest.mark.parametrize("m,k,n_out", [(1300, 512, 300), (2048, 1024, 512)])
def test_large_token_kernel_epilogues_and_bias(dev, orc, m, k, n_out):
    """More than 1024 tokens with one group (G = K) takes the large-token kernel: ragged tiles (1300 x 300) and
    whole tiles (2048 x 512), each epilogue with and without bias, bit-exact against the oracle."""
    import torch

    import voxrt_amd as vx

    trits, s16, x = _workload(orc, m, k, n_out, k, seed_cfg=3)
    ws = orc.f16_to_f32(s16)
    w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n_out, k, k)
    q, xs, _ = orc.quantize(x, k)
    xa = vx.QuantAct.quantize(_t(x, dev), k)
    rng = synth.Lcg(31)
    base = ((rng.take(m * n_out) % 200).astype(np.float32) * np.float32(0.01) - np.float32(1.0)).reshape(m, n_out)
    bias = (rng.take(n_out) % 100).astype(np.float32) / np.float32(10.0)
    for ep_kind, alpha in [(0, 0.0), (1, 0.0), (2, 0.5)]:
        want = orc.gemm(trits, ws, q, xs, k, y=base.copy(), ep=ep_kind, alpha=alpha)
        for with_bias in (False, True):
            y = _t(base, dev)
            vx.gemm_ep(w, xa, y, _t(bias, dev) if with_bias else None, _ep_of(vx, ep_kind, alpha))
            exp = (want + bias[None, :]).astype(np.float32) if with_bias else want
            _assert_bits_equal(y.cpu().numpy(), exp, f"{m}x{k}x{n_out} ep={ep_kind} bias={with_bias}")


def test_large_token_kernel_ranges_with_nan_canary(dev, orc):
    """Row and token windows on the large-token kernel: every element inside equals the oracle and nothing
    outside is written (a NaN canary), including windows that start and end inside a tile."""
    import torch

    import voxrt_amd as vx

    m, k, n_out = 1500, 512, 600
    trits, s16, x = _workload(orc, m, k, n_out, k, seed_cfg=4)
    ws = orc.f16_to_f32(s16)
    w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n_out, k, k)
    q, xs, _ = orc.quantize(x, k)
    want = orc.gemm(trits, ws, q, xs, k)
    xa = vx.QuantAct.quantize(_t(x, dev), k)
    for r0, r1, t0, t1 in [(0, n_out, 0, m), (5, 590, 3, 1497), (256, 512, 0, 1300), (17, 300, 200, 1400)]:
        y = torch.full((m, n_out), float("nan"), dtype=torch.float32, device=dev)
        vx.gemm_rows_range(w, xa, y, r0, r1, t0, t1)
        got = y.cpu().numpy()
        inside = np.zeros((m, n_out), bool)
        inside[t0:t1, r0:r1] = True
        assert (np.isnan(got) == ~inside).all(), f"stray write rows {r0}..{r1} toks {t0}..{t1}"
        _assert_bits_equal(got[inside], want[inside], f"rows {r0}..{r1} toks {t0}..{t1}")


@pytest.mark.parametrize("m,k,n_out,grid", [(1536 + 37, 1024, 1024, 8), (1024, 4096, 1024, 8), (338, 1024, 4096, 0)])
def test_group_sums_on_the_fast_kernels(dev, orc, m, k, n_out, grid):
    """The single-GEMM workload's literal output, int32 accumulators plus fp32 dequant (one group, Store), from the
    streaming kernel (forced grids: several tiles per workgroup; K = 1024 and 4096) and from the small-token kernel
    (the last 37 tokens; all of M = 338): every int32 sum and every fp32 output equal to the oracle, with and
    without bias."""
    import torch

    import voxrt_amd as vx

    trits, s16, x = _workload(orc, m, k, n_out, k, seed_cfg=6)
    ws = orc.f16_to_f32(s16)
    w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n_out, k, k)
    q, xs, _ = orc.quantize(x, k)
    xa = vx.QuantAct.quantize(_t(x, dev), k)
    want, want_gs = orc.gemm(trits, ws, q, xs, k, want_group_sums=True)
    bias = (synth.Lcg(43).take(n_out) % 100).astype(np.float32) / np.float32(10.0)
    with vx.kernels.kernel_override(**({"gemm": "stream", "stream_grid": grid} if grid else {})):
        for with_bias in (False, True):
            y = torch.full((m, n_out), float("nan"), dtype=torch.float32, device=dev)
            gs = torch.full((1, m, n_out), -7, dtype=torch.int32, device=dev)
            vx.gemm_ep(w, xa, y, _t(bias, dev) if with_bias else None, vx.Epilogue.Store, gs)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(gs.cpu().numpy(), want_gs, err_msg=f"group sums {m}x{k}x{n_out}")
            exp = (want + bias[None, :]).astype(np.float32) if with_bias else want
            _assert_bits_equal(y.cpu().numpy(), exp, f"y with group sums {m}x{k}x{n_out} bias={with_bias}")
    w.free()


@pytest.mark.parametrize("m,k,n_out,grid", [(1536, 1024, 2048, 16), (1536 + 37, 1024, 1024, 8),
                                            (1024, 4096, 1024, 8), (2048, 1024, 3072, 0)])
def test_stream_kernel_every_output(dev, orc, m, k, n_out, grid):
    """The streaming large-token kernel (whole 128 x 256 tiles, G = K), forced on shapes the oracle checks in
    full: several tiles per workgroup (a small grid), so each tile's epilogue runs while the next tile computes;
    K = 4096 (the general step loop); a ragged token count whose last 37 rows go through another kernel; each
    epilogue with and without bias, every output bit-exact."""
    import torch

    import voxrt_amd as vx

    trits, s16, x = _workload(orc, m, k, n_out, k, seed_cfg=5)
    ws = orc.f16_to_f32(s16)
    w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n_out, k, k)
    q, xs, _ = orc.quantize(x, k)
    xa = vx.QuantAct.quantize(_t(x, dev), k)
    rng = synth.Lcg(41)
    base = ((rng.take(m * n_out) % 200).astype(np.float32) * np.float32(0.01) - np.float32(1.0)).reshape(m, n_out)
    bias = (rng.take(n_out) % 100).astype(np.float32) / np.float32(10.0)
    with vx.kernels.kernel_override(gemm="stream", stream_grid=grid or None):
        for ep_kind, alpha in [(0, 0.0), (1, 0.0), (2, 0.5)]:
            want = orc.gemm(trits, ws, q, xs, k, y=base.copy(), ep=ep_kind, alpha=alpha)
            for with_bias in (False, True):
                y = _t(base, dev)
                vx.gemm_ep(w, xa, y, _t(bias, dev) if with_bias else None, _ep_of(vx, ep_kind, alpha))
                exp = (want + bias[None, :]).astype(np.float32) if with_bias else want
                _assert_bits_equal(y.cpu().numpy(), exp, f"stream {m}x{k}x{n_out} grid={grid} ep={ep_kind} "
                                                         f"bias={with_bias}")


@pytest.mark.parametrize("tile", ["8", "4"])
@pytest.mark.parametrize("m,k,n_out,grid", [(1536, 1024, 2048, 16), (1536 + 37, 1024, 1024, 8),
                                            (1024, 4096, 1024, 8), (2048, 1024, 3072, 0)])
def test_stream_groups_kernel_every_output(dev, orc, m, k, n_out, grid, tile):
    """The streaming kernel for 128-column groups (the model format: f16 scales per row and group, per-token and
    group activation scales), forced on shapes the oracle checks in full: several tiles per workgroup, K = 4096
    (32 groups), a ragged token count whose last 37 rows go through another kernel; 128-token tiles (one
    workgroup per CU) and 64-token tiles (two); each epilogue with and without bias, every output bit-exact."""
    import voxrt_amd as vx

    group = 128
    trits, s16, x = _workload(orc, m, k, n_out, group, seed_cfg=6)
    ws = orc.f16_to_f32(s16)
    w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n_out, k, group)
    q, xs, _ = orc.quantize(x, group)
    xa = vx.QuantAct.quantize(_t(x, dev), group)
    rng = synth.Lcg(43)
    base = ((rng.take(m * n_out) % 200).astype(np.float32) * np.float32(0.01) - np.float32(1.0)).reshape(m, n_out)
    bias = (rng.take(n_out) % 100).astype(np.float32) / np.float32(10.0)
    with vx.kernels.kernel_override(gemm="stream", stream_grid=grid or None, stream_tile=tile):
        for ep_kind, alpha in [(0, 0.0), (1, 0.0), (2, 0.5)]:
            want = orc.gemm(trits, ws, q, xs, group, y=base.copy(), ep=ep_kind, alpha=alpha)
            for with_bias in (False, True):
                y = _t(base, dev)
                vx.gemm_ep(w, xa, y, _t(bias, dev) if with_bias else None, _ep_of(vx, ep_kind, alpha))
                exp = (want + bias[None, :]).astype(np.float32) if with_bias else want
                _assert_bits_equal(y.cpu().numpy(), exp, f"stream groups {m}x{k}x{n_out} grid={grid} "
                                                         f"ep={ep_kind} bias={with_bias}")


@pytest.mark.parametrize("path", ["stream4", "stream8", "small", "small_ws"])
def test_grouped_fold_with_zero_and_negative_scales(dev, orc, path):
    """128-column groups whose products xs * ws are exact zeros of either sign or negative: weight scales of -0.0,
    +0.0 and negative values, all-zero token rows (scale 1, codes 0) and a zero group inside a row, with old outputs
    of -0.0 and +0.0 under AddScaled (whose result shows the sign of a zero fold). The kernels that form xs * ws on
    the fp32 matrix cores (+0 for an exact zero product where the multiply gives -0) equal the oracle bit for bit."""
    import voxrt_amd as vx

    m, k, n_out, group = 300, 1024, 1024, 128
    ng = k // group
    trits, s16, x = _workload(orc, m, k, n_out, group, seed_cfg=11)
    ws = orc.f16_to_f32(s16).reshape(n_out, ng).copy()
    ws[0:16, 3] = -0.0
    ws[16:32, 5] = 0.0
    ws[32:48, :] = -ws[32:48, :]
    ws[48, :] = -0.0
    ws[49, :] = 0.0
    x = x.copy()
    x[[5, 77, 200, 299], :] = 0.0
    x[10, 2 * group:3 * group] = 0.0
    w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n_out, k, group)
    q, xs, _ = orc.quantize(x, group)
    xa = vx.QuantAct.quantize(_t(x, dev), group)
    base = np.zeros((m, n_out), np.float32)
    base[::2, ::3] = -0.0
    base[1::2, 1::5] = np.float32(0.25)
    ov = {"stream4": dict(gemm="stream", stream_tile="4"), "stream8": dict(gemm="stream", stream_tile="8"),
          "small": dict(gemm="small", small_ws="off"), "small_ws": dict(gemm="small", small_ws="on")}[path]
    with vx.kernels.kernel_override(**ov):
        for ep_kind, alpha in [(0, 0.0), (2, 0.5)]:
            want = orc.gemm(trits, ws, q, xs, group, y=base.copy(), ep=ep_kind, alpha=alpha)
            y = _t(base, dev)
            vx.gemm_ep(w, xa, y, None, _ep_of(vx, ep_kind, alpha))
            _assert_bits_equal(y.cpu().numpy(), want, f"signed-zero scales {path} ep={ep_kind}")


@pytest.mark.parametrize("tile,group,m,k", [
    ("1x8", 0, 100, 1024), ("2x4", 0, 100, 256), ("2x8", 0, 53, 4096), ("3x2", 0, 100, 4096),
    ("3x4", 0, 338, 512), ("3x8", 0, 100, 1024), ("1x8", 0, 70, 2048), ("2x8", 0, 100, 2048),
    ("1x8", 128, 100, 1024), ("2x4", 128, 53, 512), ("2x8", 128, 100, 4096), ("3x2", 128, 100, 4096),
    ("3x4", 128, 338, 1024), ("3x8", 128, 100, 1024), ("1x8", 128, 70, 2048), ("2x4", 128, 100, 1024)])
def test_small_kernel_every_output(dev, orc, tile, group, m, k):
    """The small-token kernel (one round of workgroups, K split over the four wavefronts, int32 partial sums
    reduced in LDS), forced with each of its tiles on ragged token counts: one group (G = K, K = 256 .. 4096, ring
    depths 1 .. 8) and 128-column groups (the model format, 4 .. 32 groups folded chunk by chunk); each epilogue
    with and without bias, every output bit-exact."""
    import voxrt_amd as vx

    n_out = 256
    g = k if group == 0 else group
    trits, s16, x = _workload(orc, m, k, n_out, g, seed_cfg=7)
    ws = orc.f16_to_f32(s16)
    if group == 0:
        w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n_out, k, k)
    else:
        w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n_out, k, group)
    q, xs, _ = orc.quantize(x, g)
    xa = vx.QuantAct.quantize(_t(x, dev), g)
    rng = synth.Lcg(47)
    base = ((rng.take(m * n_out) % 200).astype(np.float32) * np.float32(0.01) - np.float32(1.0)).reshape(m, n_out)
    bias = (rng.take(n_out) % 100).astype(np.float32) / np.float32(10.0)
    with vx.kernels.kernel_override(gemm="small", small_tile=tile):
        for ep_kind, alpha in [(0, 0.0), (1, 0.0), (2, 0.5)]:
            want = orc.gemm(trits, ws, q, xs, g, y=base.copy(), ep=ep_kind, alpha=alpha)
            for with_bias in (False, True):
                y = _t(base, dev)
                vx.gemm_ep(w, xa, y, _t(bias, dev) if with_bias else None, _ep_of(vx, ep_kind, alpha))
                exp = (want + bias[None, :]).astype(np.float32) if with_bias else want
                _assert_bits_equal(y.cpu().numpy(), exp, f"small tile={tile} G={g} {m}x{k}x{n_out} ep={ep_kind} "
                                                         f"bias={with_bias}")


@pytest.mark.parametrize("tile", ["2x4", "1x4"])
@pytest.mark.parametrize("m,k", [(100, 1024), (338, 4096), (70, 2048), (338, 1024), (17, 4096)])
def test_small_ws_kernel_every_output(dev, orc, m, k, tile):
    """The grouped small-token kernel with producer and consumer wavefronts (chains seeded with -gsum, int32 sums
    through two LDS planes, the fold one chunk behind), forced on ragged token counts with 8, 16 and 32 groups
    (rings of 2 and 4 steps) and with 32- and 16-token tiles: each epilogue with and without bias, every output
    bit-exact."""
    import voxrt_amd as vx

    n_out, g = 256, 128
    trits, s16, x = _workload(orc, m, k, n_out, g, seed_cfg=11)
    ws = orc.f16_to_f32(s16)
    w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n_out, k, g)
    q, xs, _ = orc.quantize(x, g)
    xa = vx.QuantAct.quantize(_t(x, dev), g)
    rng = synth.Lcg(61)
    base = ((rng.take(m * n_out) % 200).astype(np.float32) * np.float32(0.01) - np.float32(1.0)).reshape(m, n_out)
    bias = (rng.take(n_out) % 100).astype(np.float32) / np.float32(10.0)
    with vx.kernels.kernel_override(gemm="small", small_ws="on", small_tile=tile):
        for ep_kind, alpha in [(0, 0.0), (1, 0.0), (2, 0.5)]:
            want = orc.gemm(trits, ws, q, xs, g, y=base.copy(), ep=ep_kind, alpha=alpha)
            for with_bias in (False, True):
                y = _t(base, dev)
                vx.gemm_ep(w, xa, y, _t(bias, dev) if with_bias else None, _ep_of(vx, ep_kind, alpha))
                exp = (want + bias[None, :]).astype(np.float32) if with_bias else want
                _assert_bits_equal(y.cpu().numpy(), exp, f"small_ws G=128 {m}x{k}x{n_out} tile={tile} "
                                                         f"ep={ep_kind} bias={with_bias}")


@pytest.mark.parametrize("tile", ["1x8", "2x8"])
@pytest.mark.parametrize("m,n_out,ep_kind,with_bias", [(338, 4096, 1, False), (70, 384, 0, True), (5, 256, 1, True)])
def test_small_ws_quantized_output(dev, orc, tile, m, n_out, ep_kind, with_bias):
    """The producer/consumer kernel writing the next GEMM's activations (one plane, two barriers per chunk): codes,
    scales and code sums equal the oracle's GEMM -> quantize chain bit for bit, pad tokens zero."""
    import torch

    import voxrt_amd as vx

    k, g = 1024, 128
    trits, s16, x = _workload(orc, m, k, n_out, g, seed_cfg=12)
    ws = orc.f16_to_f32(s16)
    w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n_out, k, g)
    q, xs, _ = orc.quantize(x, g)
    xa = vx.QuantAct.quantize(_t(x, dev), g)
    bias = (synth.Lcg(67).take(n_out) % 100).astype(np.float32) / np.float32(10.0) - np.float32(5.0)
    want = orc.gemm(trits, ws, q, xs, g, ep=ep_kind)
    if with_bias:
        want = (want + bias[None, :]).astype(np.float32)
    wq, wsc, wgs = orc.quantize(want, 128)
    with vx.kernels.kernel_override(small_ws="on", small_tile=tile):
        got = vx.gemm_ep_quantize(w, xa, _t(bias, dev) if with_bias else None, _ep_of(vx, ep_kind, 0.0), 128)
    torch.cuda.synchronize()
    tag = f"small_ws {tile} {m}x{k}x{n_out} ep={ep_kind} bias={with_bias}"
    np.testing.assert_array_equal(got.x.cpu().numpy(), wq, err_msg=f"codes {tag}")
    st, gt = got.scales_t.cpu().numpy(), got.gsum_t.cpu().numpy()
    _assert_bits_equal(st[:, :m].T.copy(), wsc, f"scales {tag}")
    np.testing.assert_array_equal(gt[:, :m].T, wgs, err_msg=f"gsum {tag}")
    assert not st[:, m:].any() and not gt[:, m:].any(), f"pad tokens not zero {tag}"


@pytest.mark.parametrize("m,k,n_out,group,ep_kind,with_bias", [
    (338, 1024, 4096, 128, 1, False),   # the encoder's FFN up-projection at T = 338 (fused epilogue)
    (338, 1024, 4096, 0, 1, True),      # one group (G = K), bias after SiLU
    (70, 1024, 384, 128, 0, True),      # ragged tokens, three output groups, Store
    (125, 4096, 256, 128, 1, False),    # 32 input groups (ring depth 8)
    (1100, 1024, 512, 128, 1, True)])   # above 1024 tokens: GEMM into y_tmp, then the quantizer
def test_gemm_ep_quantize_equals_two_step(dev, orc, m, k, n_out, group, ep_kind, with_bias):
    """gemm_ep_quantize (the FFN up-projection with the down-projection's quantization fused) equals the reference
    chain forward_prepared_ep(Silu) -> QuantAct::quantize_layout of the oracle: int8 codes, scales and code sums
    bit for bit, pad tokens of the transposed scales and sums zero."""
    import torch

    import voxrt_amd as vx

    g = k if group == 0 else group
    trits, s16, x = _workload(orc, m, k, n_out, g, seed_cfg=8)
    ws = orc.f16_to_f32(s16)
    if group == 0:
        w = vx.TernaryMatrix.from_packed_f32(synth.pack_rows(trits), ws, n_out, k, k)
    else:
        w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n_out, k, group)
    q, xs, _ = orc.quantize(x, g)
    xa = vx.QuantAct.quantize(_t(x, dev), g)
    bias = (synth.Lcg(53).take(n_out) % 100).astype(np.float32) / np.float32(10.0) - np.float32(5.0)
    want = orc.gemm(trits, ws, q, xs, g, ep=ep_kind)
    if with_bias:
        want = (want + bias[None, :]).astype(np.float32)
    wq, wsc, wgs = orc.quantize(want, 128)
    got = vx.gemm_ep_quantize(w, xa, _t(bias, dev) if with_bias else None, _ep_of(vx, ep_kind, 0.0), 128)
    torch.cuda.synchronize()
    tag = f"{m}x{k}x{n_out} G={g} ep={ep_kind} bias={with_bias}"
    np.testing.assert_array_equal(got.x.cpu().numpy(), wq, err_msg=f"codes {tag}")
    st, gt = got.scales_t.cpu().numpy(), got.gsum_t.cpu().numpy()
    _assert_bits_equal(st[:, :m].T.copy(), wsc, f"scales {tag}")
    np.testing.assert_array_equal(gt[:, :m].T, wgs, err_msg=f"gsum {tag}")
    assert not st[:, m:].any() and not gt[:, m:].any(), f"pad tokens not zero {tag}"


def test_zero_tokens_is_a_no_op(dev):
    """A batch of zero tokens (the reference's kernels loop over nothing): quantize, gemm_ep with every epilogue,
    the fused GEMM -> quantize, gemm_single and the empty row / token ranges of gemm_rows_range return without
    touching y, also with the NULL data pointers of empty torch tensors."""
    import torch

    import voxrt_amd as vx

    rng = synth.Lcg(77)
    out, inp = 256, 1024
    qw, s16, _ = synth.ref_random_matrix(rng, out, inp)
    w = vx.TernaryMatrix.from_packed(qw, s16, out, inp, 128)
    x0 = vx.QuantAct.quantize(torch.empty((0, inp), dtype=torch.float32, device=dev), 128)
    assert x0.n == 0
    y0 = torch.empty((0, out), dtype=torch.float32, device=dev)
    for ep in (vx.Epilogue.Store, vx.Epilogue.Silu, vx.Epilogue.AddScaled(0.5)):
        vx.gemm_ep(w, x0, y0, None, ep)
    qa = vx.gemm_ep_quantize(w, x0)
    assert qa.n == 0
    vx.gemm_single(w, x0, y0)
    # empty ranges of a non-empty batch leave y as it was
    x = vx.QuantAct.quantize(torch.from_numpy(synth.ref_acts(rng, 5, inp)).to(dev), 128)
    y = torch.full((5, out), 3.0, dtype=torch.float32, device=dev)
    vx.gemm_rows_range(w, x, y, 7, 7, 0, 5)
    vx.gemm_rows_range(w, x, y, 0, out, 2, 2)
    torch.cuda.synchronize()
    assert bool((y == 3.0).all())


def test_wrappers_refuse_tensors_of_the_wrong_shape(dev):
    """Every device tensor handed to the C ABI is checked against the shape the call implies (the kernels read or
    write all of it): a bias, y, group-sum buffer or activation table that is too small raises ValueError before
    any launch, and y is left untouched."""
    import torch

    import voxrt_amd as vx
    from voxrt_amd import encoder as E

    rng = synth.Lcg(78)
    out, inp, n = 256, 1024, 5
    qw, s16, _ = synth.ref_random_matrix(rng, out, inp)
    w = vx.TernaryMatrix.from_packed(qw, s16, out, inp, 128)
    x = vx.QuantAct.quantize(_t(synth.ref_acts(rng, n, inp), dev), 128)
    y = torch.full((n, out), 3.0, dtype=torch.float32, device=dev)
    short = torch.zeros(out - 4, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="bias"):
        vx.gemm_ep(w, x, y, short)
    with pytest.raises(ValueError, match="group_sums"):
        vx.gemm_ep(w, x, y, None, vx.Epilogue.Store, torch.zeros((8, n, out - 1), dtype=torch.int32, device=dev))
    with pytest.raises(ValueError, match="y must have shape"):
        vx.gemm_rows_range(w, x, y[:4], 0, out, 0, 4)
    with pytest.raises(ValueError, match="bias"):
        vx.gemm_single(w, x, y, short)
    bad = vx.QuantAct(x.x, x.scales_t[:, :8].contiguous(), x.gsum_t, n, inp, 128)
    with pytest.raises(ValueError, match="scales_t"):
        vx.gemm_ep(w, bad, y)
    with pytest.raises(ValueError, match="gamma"):
        vx.QuantAct.quantize_normed(_t(synth.ref_acts(rng, n, inp), dev), short, short, 128)
    with pytest.raises(ValueError, match="rel_k"):
        E.attention_core(torch.zeros((9, 3 * 256), device=dev), torch.zeros((16, 256), device=dev), 2,
                         torch.zeros((2, 128), device=dev), torch.zeros((2, 128), device=dev))
    enc = E.Encoder(d=256, heads=2, ff=512, n_layers=1)
    with pytest.raises(ValueError, match="x must have shape"):
        enc.forward(torch.zeros((9, 255), device=dev))
    enc.free()
    torch.cuda.synchronize()
    assert bool((y == 3.0).all())
    w.free()


def test_trit_rows_upload_equals_packed_upload(dev, orc):
    """A matrix uploaded from unpacked trits (vx_tmat_upload_trits, the Rows layout a CPU-side TernaryMatrix holds)
    is the same device matrix as the one uploaded from the model file's packed rows: equal outputs, bit for bit,
    for 128-column groups and for one group, including a K whose last byte holds pad digits."""
    import torch

    import voxrt_amd as vx

    rng = synth.Lcg(91)
    for out, inp, group in [(256, 1024, 128), (384, 640, 640)]:
        qw, s16, trits = synth.ref_random_matrix(rng, out, inp, 128)
        ws = orc.f16_to_f32(s16)
        if group != 128:
            ws = ws[:, :1].copy()
        x = synth.ref_acts(rng, 45, inp)
        a = vx.TernaryMatrix.from_packed_f32(qw, ws, out, inp, group)
        b = vx.TernaryMatrix.from_trits(trits, ws, out, inp, group)
        xa = vx.QuantAct.quantize(_t(x, dev), group)
        ya = torch.zeros((45, out), dtype=torch.float32, device=dev)
        yb = torch.zeros((45, out), dtype=torch.float32, device=dev)
        vx.gemm_ep(a, xa, ya, None, vx.Epilogue.Silu)
        vx.gemm_ep(b, xa, yb, None, vx.Epilogue.Silu)
        torch.cuda.synchronize()
        _assert_bits_equal(yb.cpu().numpy(), ya.cpu().numpy(), f"trit upload {out}x{inp} G={group}")
        q, xs, _ = orc.quantize(x, group)
        _assert_bits_equal(yb.cpu().numpy(), orc.gemm(trits, ws, q, xs, group, ep=orc.EP_SILU), "against the oracle")
        a.free()
        b.free()
