"""The oracle pinned against the reference's stored vectors, known answers and independent closed forms.

Restates crates/voxrt/tests/fixtures_trits.rs, the unit tests of trits.rs:90-109 and tensor.rs:1017-1030,
tests/kernels.rs (accumulation_cannot_overflow, quantised_path_tracks_f32_path) and tests/x86_kernels.rs (the VNNI
CPU baseline equals the scalar kernel bit for bit).
"""
import json
import os

import numpy as np
import pytest

from voxrt_amd import synth

FIX = os.path.join(os.path.dirname(__file__), "golden", "fixtures")


def _fx(name, dtype):
    return np.fromfile(os.path.join(FIX, name), dtype=dtype)


# ---------------------------------------------------------------- codec (trits.rs, fixtures_trits.rs)

def test_fixtures_trits_and_dequant(orc):
    """fixtures_trits.rs:13-47: unpack and dequant equal the stored rows exactly; zero fraction matches."""
    meta = json.load(open(os.path.join(FIX, "ternary_fixtures.json")))
    assert len(meta) == 3
    for tag, m in meta.items():
        rows, inf, g = m["rows"], m["in_features"], m["group_size"]
        q = _fx(f"{tag}.qweight.bin", np.uint8).reshape(rows, (inf + 4) // 5)
        s = _fx(f"{tag}.scales.f16.bin", np.uint16).reshape(rows, inf // g)
        want_t = _fx(f"{tag}.trits.i8.bin", np.int8).reshape(rows, inf)
        want_w = _fx(f"{tag}.weight.f32.bin", np.float32).reshape(rows, inf)
        got_t = orc.unpack_rows(q, inf)
        np.testing.assert_array_equal(got_t, want_t, err_msg=tag)
        got_w = orc.dequant_matrix(q, s, rows, inf, g)
        assert got_w.view(np.uint32).tolist() == want_w.view(np.uint32).tolist(), tag
        zf = float((got_t == 0).mean())
        assert abs(zf - m["zero_fraction_rows"]) < 1e-9, tag
        # the numpy host codec (used to pack synthetic weights) agrees with the stored rows too
        np.testing.assert_array_equal(synth.unpack_rows(q, inf), want_t)
        np.testing.assert_array_equal(synth.pack_rows(want_t), q)


def test_lsd_first_known_answer(orc):
    """trits.rs:103-109: digits (1,2,0,1,2) -> 196 -> trits [0, 1, -1, 0, 1]."""
    np.testing.assert_array_equal(orc.unpack_rows(np.array([[196]], np.uint8), 5)[0], [0, 1, -1, 0, 1])
    np.testing.assert_array_equal(orc.pack_row(np.array([0, 1, -1, 0, 1], np.int8)), [196])


@pytest.mark.parametrize("n", [1, 4, 5, 6, 127, 128, 1024, 4096])
def test_roundtrip_ragged_widths(orc, n):
    """trits.rs:90-101 (same trit pattern), plus every byte < 243 and the numpy packer agreeing."""
    trits = ((np.arange(n) * 7 + 3) % 3 - 1).astype(np.int8)
    packed = orc.pack_row(trits)
    assert packed.size == (n + 4) // 5 and (packed < 243).all()
    np.testing.assert_array_equal(orc.unpack_rows(packed[None, :], n)[0], trits)
    np.testing.assert_array_equal(synth.pack_rows(trits[None, :])[0], packed)


# ---------------------------------------------------------------- f16 (half crate, IEEE binary16)

def test_f16_to_f32_all_codes(orc):
    codes = np.arange(65536, dtype=np.uint16)
    got = orc.f16_to_f32(codes)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_f32_to_f16_round_to_nearest_even(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        (rng.random(20000).astype(np.float32) * np.float32(1e-4)),  # subnormal halves
        np.arange(65505, dtype=np.float32)[::7],
        # exact ties between neighbouring halves
        ((np.arange(1, 2000, dtype=np.float64) * 2 + 1) * 2.0 ** -11).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 6e-8, 3e-8, 2.9e-8], np.float32),
    ])
    lib = orc.lib()
    got = np.array([lib.or_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------- quantizer (packed.rs:453-536)

def _quantize_np(x, group):
    """Independent numpy statement: absmax/127 scale (1 if all zero), codes rint(x * (1/s)) clamped to +-127."""
    n, inp = x.shape
    xg = x.reshape(n, inp // group, group)
    amax = np.abs(xg).max(axis=2)
    s = np.where(amax == 0, np.float32(1.0), amax / np.float32(127.0)).astype(np.float32)
    inv = (np.float32(1.0) / s).astype(np.float32)
    q = np.clip(np.rint(xg * inv[:, :, None]), -127, 127).astype(np.int8)
    return q.reshape(n, inp), s, q.astype(np.int32).sum(axis=2)


@pytest.mark.parametrize("n", [1, 7, 8, 15, 16, 17, 128, 133, 384, 4096])
def test_quantize_group_ties_and_generator(orc, n):
    """packed.rs:604-632's generator: exact .5 ties at every 5th element; numpy rint is half-to-even."""
    seed = 3
    src = np.empty(n, np.float32)
    with np.errstate(over="ignore"):
        for i in range(n):
            seed = (seed * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
            src[i] = np.float32(i + 0.5) * np.float32(0.1) if i % 5 == 0 else np.float32(seed >> 40) / np.float32(1e6) - np.float32(8.0)
    q, s, g = orc.quantize(src[None, :], n)
    wq, ws, wg = _quantize_np(src[None, :], n)
    np.testing.assert_array_equal(q, wq)
    assert s.view(np.uint32)[0, 0] == ws.view(np.uint32)[0, 0]
    np.testing.assert_array_equal(g, wg)


def test_quantize_special_groups(orc):
    x = np.zeros((3, 256), np.float32)
    x[1, :128] = 5.0
    x[1, 128:] = -5.0
    x[2, 7] = 1e-30
    q, s, g = orc.quantize(x, 128)
    np.testing.assert_array_equal(s[0], [1.0, 1.0])  # all-zero group -> scale 1, codes 0
    assert (q[0] == 0).all()
    assert (q[1, :128] == 127).all() and (q[1, 128:] == -127).all()
    assert g[1, 0] == 128 * 127 and g[1, 1] == -128 * 127
    assert q[2, 7] == 127 and g[2, 0] == 127


# ---------------------------------------------------------------- exp_poly / SiLU (tensor.rs:829-860)

def test_exp_poly_close_to_exp(orc):
    """tensor.rs:1017-1030: relative error < 3e-7 against exp in double on the clamped input."""
    xs = np.concatenate([np.arange(-2000, 2000, dtype=np.float32) * np.float32(0.05),
                         np.array([-87.0, -100.0, 88.0, 1e3, 0.0, -0.0], np.float32)])
    lib = orc.lib()
    for x in xs:
        got = lib.or_exp_poly(float(x))
        want = np.exp(np.float64(np.clip(x, -87.0, 88.0)))
        assert abs((got - want) / want) < 3e-7, (x, got, want)


def test_silu_and_sigmoid_close(orc):
    lib = orc.lib()
    for x in np.linspace(-30, 30, 2001, dtype=np.float32):
        want = float(x) / (1.0 + np.exp(-np.float64(x)))
        assert abs(lib.or_silu_fast(float(x)) - want) <= 1e-6 * max(1.0, abs(want))
        assert abs(lib.or_sigmoid_fast(float(x)) - 1.0 / (1.0 + np.exp(-np.float64(x)))) <= 1e-6


# ---------------------------------------------------------------- GEMM (kernels/mod.rs:166-210)

def _rand_case(rng, out, inp, n, group=128):
    qw, s16, trits = synth.ref_random_matrix(rng, out, inp, group)
    x = synth.ref_acts(rng, n, inp)
    return trits, s16.view(np.float16).astype(np.float32), x


def test_group_sums_equal_integer_matmul(orc):
    """Group sums are exact integer dot products (brute force in int64)."""
    rng = synth.Lcg(42)
    for out, inp, n in [(7, 128, 1), (9, 256, 17), (64, 1024, 5), (130, 4096, 3)]:
        trits, ws, x = _rand_case(rng, out, inp, n)
        q, xs, _ = orc.quantize(x, 128)
        y, gs = orc.gemm(trits, ws, q, xs, 128, want_group_sums=True)
        ng = inp // 128
        want = np.einsum("tgc,ogc->gto", q.reshape(n, ng, 128).astype(np.int64),
                         trits.reshape(out, ng, 128).astype(np.int64))
        np.testing.assert_array_equal(gs, want)


def test_single_group_closed_form(orc):
    """G = K: acc = fma(S, p, 0) is one correctly rounded product, so y = f32(S * f32(xs*ws)) computed exactly in
    float64 (|S| < 2^21 and p has 24 bits, so S*p is exact there) and rounded once."""
    rng = synth.Lcg(11)
    for out, inp, n in [(33, 1024, 9), (19, 1024, 4), (64, 4096, 3)]:
        qw, _, trits = synth.ref_random_matrix(rng, out, inp, inp)
        ws = rng.take(out).astype(np.float32) / np.float32(4e10) + np.float32(0.01)
        ws = ws.reshape(out, 1)
        x = synth.ref_acts(rng, n, inp)
        q, xs, _ = orc.quantize(x, inp)
        y, gs = orc.gemm(trits, ws, q, xs, inp, want_group_sums=True)
        S = q.astype(np.int64) @ trits.astype(np.int64).T
        np.testing.assert_array_equal(gs[0], S)
        p = (xs.reshape(n, 1) * ws.reshape(1, out)).astype(np.float32)
        want = (S.astype(np.float64) * p.astype(np.float64)).astype(np.float32)
        np.testing.assert_array_equal(y.view(np.uint32), want.view(np.uint32))


def test_grouped_fold_close_to_exact(orc):
    """G = 128: the fp32 fold stays within 1e-6 relative of the exact (float64) sum of S_g * xs * ws over
    groups; a dropped group, a wrong scale index or a sign error moves it by orders of magnitude more."""
    rng = synth.Lcg(5)
    out, inp, n = 64, 1024, 13
    trits, ws, x = _rand_case(rng, out, inp, n)
    q, xs, _ = orc.quantize(x, 128)
    y, gs = orc.gemm(trits, ws, q, xs, 128, want_group_sums=True)
    exact = np.einsum("gto,tg,og->to", gs.astype(np.float64), xs.astype(np.float64), ws.astype(np.float64))
    scale = np.abs(exact).max()
    assert np.abs(y - exact).max() <= 1e-6 * scale


def test_accumulation_cannot_overflow(orc):
    """tests/kernels.rs:176-200: all +1 trits, x = 127, K = 4096, unit scales -> y = 4096 * 127."""
    inp = 4096
    trits = np.ones((1, inp), np.int8)
    ws = np.ones((1, inp // 128), np.float32)
    q, xs, _ = orc.quantize(np.full((1, inp), 127.0, np.float32), 128)
    assert (xs == 1.0).all()
    y = orc.gemm(trits, ws, q, xs, 128)
    assert y[0, 0] == 4096 * 127.0


def test_quantised_path_tracks_f32_path(orc):
    """tests/kernels.rs:149-174: int8 per-group-128 within 1e-2 relative of the f32 dequantised product."""
    rng = synth.Lcg(7)
    out, inp, n = 256, 1024, 16
    qw, s16, trits = synth.ref_random_matrix(rng, out, inp)
    wf = orc.dequant_matrix(qw, s16, out, inp, 128)
    x = synth.ref_acts(rng, n, inp, div=1000.0, off=1.0)
    yf = x.astype(np.float64) @ wf.astype(np.float64).T
    q, xs, _ = orc.quantize(x, 128)
    yq = orc.gemm(trits, orc.f16_to_f32(s16), q, xs, 128)
    assert np.abs(yf - yq).max() / np.abs(yf).max() < 1e-2


def test_epilogues(orc):
    """Store / Silu / AddScaled write ep(old, acc) (kernels/mod.rs:41-48) and nothing outside the block."""
    rng = synth.Lcg(9)
    out, inp, n = 40, 256, 11
    trits, ws, x = _rand_case(rng, out, inp, n)
    q, xs, _ = orc.quantize(x, 128)
    base = ((np.arange(n * out) % 7) - 3).astype(np.float32).reshape(n, out)
    y0 = orc.gemm(trits, ws, q, xs, 128)
    lib = orc.lib()
    for ep, alpha in [(orc.EP_STORE, 0.0), (orc.EP_SILU, 0.0), (orc.EP_ADD_SCALED, 0.5)]:
        y = np.full((n, out), np.nan, np.float32)
        y[2:9, 3:30] = base[2:9, 3:30]
        orc.gemm_scalar_range(trits, ws, q, xs, 128, y, 3, 30, 2, 9, ep, alpha)
        for t in range(n):
            for o in range(out):
                inside = 2 <= t < 9 and 3 <= o < 30
                assert np.isnan(y[t, o]) != inside
                if inside:
                    want = lib.or_ep_apply(ep, alpha, float(base[t, o]), float(y0[t, o]))
                    assert np.float32(want).view(np.uint32) == y[t, o].view(np.uint32)


# ---------------------------------------------------------------- LCG (tests/kernels.rs:7-12)

@pytest.mark.parametrize("seed", [0, 1, 42, 0x766F787200000105])
def test_numpy_lcg_equals_sequential(orc, seed):
    np.testing.assert_array_equal(synth.lcg_stream(seed, 1000)[0], orc.lcg_outputs(seed, 1000))


def test_workload_generators_distribution():
    t = synth.synth_trits(synth.workload_seed(0, 1), 512, 1024)
    frac0, fracm, fracp = (t == 0).mean(), (t == -1).mean(), (t == 1).mean()
    assert abs(frac0 - 0.4) < 0.01 and abs(fracm - 0.3) < 0.01 and abs(fracp - 0.3) < 0.01
    s = synth.synth_channel_scales_f16(synth.workload_seed(0, 2), 4096, 8).view(np.float16).astype(np.float32)
    assert s.min() >= 0.0099 and s.max() <= 0.0501 and (s == s[:, :1]).all()
    z = synth.synth_normal(synth.workload_seed(0, 3), 100000)
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1.0) < 0.02


# ---------------------------------------------------------------- CPU baseline (x86_kernels.rs)

def _ternary_q16(orc, rng, out, inp, extreme=False):
    if extreme:
        trits = np.ones((out, inp), np.int8)
        draws = rng.take(out * (inp // 128)).reshape(out, inp // 128)
    else:
        d = rng.take(out * (inp + inp // 128)).reshape(out, inp + inp // 128)
        trits = (d[:, :inp] % 3).astype(np.int8) - 1
        draws = d[:, inp:]
    s = (np.float32(0.01) + (draws % 100).astype(np.float32) * np.float32(0.001)).astype(np.float16).astype(np.float32)
    return trits, s


def _int8_q16(rng, out, inp, group, extreme=False):
    if extreme:
        rows = np.where(np.arange(out * inp) % 2 == 0, 127, -127).astype(np.int8).reshape(out, inp)
    else:
        rows = ((rng.take(out * inp) % 255).astype(np.int32) - 127).astype(np.int8).reshape(out, inp)
    s = (np.float32(0.001) + (rng.take(out * (inp // group)) % 1000).astype(np.float32) * np.float32(1e-5))
    return rows, s.astype(np.float32).reshape(out, inp // group)


def _acts(rng, n, inp, extreme=False):
    if extreme:
        return np.where(np.arange(n * inp) % 2 == 0, 5.0, -5.0).astype(np.float32).reshape(n, inp)
    return synth.ref_acts(rng, n, inp)


def _check_vnni(orc, rng, rows, ws, group, xf, kernel=None):
    out, inp = rows.shape
    n = xf.shape[0]
    q, xs, gsum = orc.quantize(xf, group)
    wq, sq = orc.quad16_pack(rows, ws, group)
    ranges = [(0, out, 0, n), (min(1, out), out, 0, n), (0, min(out, 17), n // 2, n),
              (out // 3, out - out // 4, 0, (n + 1) // 2)]
    for ep, alpha in [(orc.EP_STORE, 0.0), (orc.EP_SILU, 0.0), (orc.EP_ADD_SCALED, 0.37)]:
        for r0, r1, t0, t1 in ranges:
            if r0 >= r1 or t0 >= t1:
                continue
            init = ((rng.take(n * out) % 100).astype(np.float32) * np.float32(0.01)).reshape(n, out)
            want = init.copy()
            orc.gemm_scalar_range(rows, ws, q, xs, group, want, r0, r1, t0, t1, ep, alpha)
            got = init.copy()
            if kernel is None:
                orc.gemm_vnni_range(wq, sq, out, inp, group, q, xs, gsum, got, r0, r1, t0, t1, ep, alpha)
            else:
                assert kernel(wq, sq, out, inp, group, q, xs, gsum, got, r0, r1, t0, t1, ep, alpha) == 0
            assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), (out, inp, group, n, r0, r1, t0, t1, ep)


def _need_vnni(orc):
    if not orc.lib().or_have_vnni():
        pytest.skip("no AVX-512 VNNI on this host")


def test_vnni_ternary_equals_scalar_exactly(orc):
    """x86_kernels.rs:140-152."""
    _need_vnni(orc)
    rng = synth.Lcg(3)
    for out, inp in [(7, 128), (16, 256), (33, 1024), (130, 4096)]:
        trits, ws = _ternary_q16(orc, rng, out, inp)
        for n in [1, 2, 3, 4, 5, 8, 9, 17]:
            _check_vnni(orc, rng, trits, ws, 128, _acts(rng, n, inp))


def test_vnni_ternary_one_group_equals_scalar_exactly(orc):
    """Ternary weights with one group per row (G = K, the per-channel scales of the GPU's full-size checks):
    the VNNI restatement equals the scalar kernel bit for bit."""
    _need_vnni(orc)
    rng = synth.Lcg(7)
    for out, inp in [(16, 1024), (37, 4096)]:
        trits = ((rng.take(out * inp) % 3).astype(np.int8) - 1).reshape(out, inp)
        ws = (rng.take(out) % 4000 + 100).astype(np.float32) * np.float32(1e-5)
        for n in [1, 3, 8, 13]:
            _check_vnni(orc, rng, trits, ws.reshape(out, 1), inp, _acts(rng, n, inp))


def test_vnni_int8_equals_scalar_exactly(orc):
    """x86_kernels.rs:154-172 (groups 128, 384, 1024)."""
    _need_vnni(orc)
    rng = synth.Lcg(5)
    for out, inp, group in [(7, 128, 128), (40, 640, 128), (128, 384, 384), (19, 1024, 1024)]:
        rows, ws = _int8_q16(rng, out, inp, group)
        for n in [1, 2, 5, 8, 11]:
            _check_vnni(orc, rng, rows, ws, group, _acts(rng, n, inp))


def test_vnni_extremes_do_not_saturate(orc):
    """x86_kernels.rs:174-185."""
    _need_vnni(orc)
    rng = synth.Lcg(9)
    trits, ws = _ternary_q16(orc, rng, 32, 1024, extreme=True)
    _check_vnni(orc, rng, trits, ws, 128, _acts(rng, 5, 1024, extreme=True))
    rows, ws = _int8_q16(rng, 32, 1024, 1024, extreme=True)
    _check_vnni(orc, rng, rows, ws, 1024, _acts(rng, 5, 1024, extreme=True))


def test_vnni_threaded_gemm_ep_equals_scalar(orc):
    """gemm_ep's row-block split (kernels/mod.rs:324-354) on several threads changes nothing."""
    _need_vnni(orc)
    rng = synth.Lcg(21)
    out, inp, n = 4096, 1024, 37
    trits = synth.synth_trits(synth.workload_seed(0, 1), out, inp)
    ws = np.repeat(synth.synth_channel_scales_f16(synth.workload_seed(0, 2), out, 1).view(np.float16).astype(np.float32), 8, axis=1)
    x = synth.synth_normal(synth.workload_seed(0, 3), n * inp).reshape(n, inp)
    q, xs, gsum = orc.quantize(x, 128)
    want = orc.gemm(trits, ws, q, xs, 128)
    wq, sq = orc.quad16_pack(trits, ws, 128)
    got = np.zeros((n, out), np.float32)
    orc.gemm_ep_vnni(wq, sq, out, inp, 128, q, xs, gsum, got, threads=4)
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


# the AVX2 path (x86.rs:163-290) on the same grids (x86_kernels.rs runs both kernels through one check)

def _need_avx2(orc):
    if not orc.lib().or_have_avx2():
        pytest.skip("no AVX2/FMA on this host")


def _avx2(orc, ternary):
    return lambda *a: orc.gemm_avx2_range(*a[:5], ternary, *a[5:])


def test_avx2_ternary_equals_scalar_exactly(orc):
    """x86_kernels.rs:140-152 for gemm_avx2_range (ternary weights, int16 sums per group)."""
    _need_avx2(orc)
    rng = synth.Lcg(3)
    for out, inp in [(7, 128), (16, 256), (33, 1024), (130, 4096)]:
        trits, ws = _ternary_q16(orc, rng, out, inp)
        for n in [1, 2, 3, 4, 5, 8, 9, 17]:
            _check_vnni(orc, rng, trits, ws, 128, _acts(rng, n, inp), _avx2(orc, True))


def test_avx2_int8_equals_scalar_exactly(orc):
    """x86_kernels.rs:154-172 for gemm_avx2_range (int8 weights, groups 128, 384, 1024)."""
    _need_avx2(orc)
    rng = synth.Lcg(5)
    for out, inp, group in [(7, 128, 128), (40, 640, 128), (128, 384, 384), (19, 1024, 1024)]:
        rows, ws = _int8_q16(rng, out, inp, group)
        for n in [1, 2, 5, 8, 11]:
            _check_vnni(orc, rng, rows, ws, group, _acts(rng, n, inp), _avx2(orc, False))


def test_avx2_extremes_do_not_saturate(orc):
    """x86_kernels.rs:174-185 for gemm_avx2_range: all-ones trits and +-127 weights against +-127 codes, where
    vpmaddubsw would saturate if the pairs were not bounded."""
    _need_avx2(orc)
    rng = synth.Lcg(9)
    trits, ws = _ternary_q16(orc, rng, 32, 1024, extreme=True)
    _check_vnni(orc, rng, trits, ws, 128, _acts(rng, 5, 1024, extreme=True), _avx2(orc, True))
    trits, ws = _ternary_q16(orc, rng, 16, 512, extreme=True)
    ws = np.repeat(ws[:, :1], 2, axis=1)
    _check_vnni(orc, rng, trits, ws, 256, _acts(rng, 3, 512, extreme=True), _avx2(orc, True))
    rows, ws = _int8_q16(rng, 32, 1024, 1024, extreme=True)
    _check_vnni(orc, rng, rows, ws, 1024, _acts(rng, 5, 1024, extreme=True), _avx2(orc, False))


def test_avx2_ternary_needs_group_at_most_256(orc):
    """Ternary int16 group sums bound the AVX2 path to group <= 256 (x86.rs:173-174, kernels/mod.rs:326-328): a
    larger group is refused and y is left untouched."""
    _need_avx2(orc)
    rng = synth.Lcg(11)
    trits, ws = _ternary_q16(orc, rng, 16, 1024)
    ws1 = ws[:, :1].copy()
    q, xs, gsum = orc.quantize(_acts(rng, 2, 1024), 1024)
    wq, sq = orc.quad16_pack(trits, ws1, 1024)
    y = np.full((2, 16), 7.0, np.float32)
    assert orc.gemm_avx2_range(wq, sq, 16, 1024, 1024, True, q, xs, gsum, y, 0, 16, 0, 2) == -1
    assert (y == 7.0).all()
