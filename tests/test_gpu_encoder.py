"""The encoder-side HIP kernels and the whole encoder == the oracle, bit for bit, through the C ABI.

Restates, for the HIP path, the reference's per-piece exactness (the int8 encoder's fused LayerNorm quantizer,
ternary_linear.rs:132-155; glue of encoder.rs and tensor.rs; the int8 attention core, encoder.rs:317-534; the f32
subsampling, subsampling.rs:124-204) and its GPU-encoder test (metal_encoder.rs: GPU encoder vs CPU encoder on the
same input; here bit-exact against the CPU int8 restatement instead of a tolerance), plus the single-token GEMV of
kernels.rs:271-316 (gemv_equals_scalar_exactly).
"""
import numpy as np
import pytest

from voxrt_amd import synth

pytestmark = pytest.mark.gpu


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


def _bits_equal(got, want, what):
    g = np.ascontiguousarray(got, np.float32).view(np.uint32).ravel()
    w = np.ascontiguousarray(want, np.float32).view(np.uint32).ravel()
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ, first at {bad[0]}: got "
                           f"{np.asarray(got).ravel()[bad[0]]!r} want {np.asarray(want).ravel()[bad[0]]!r}")


def _x(seed, *shape, scale=1.0):
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)


@pytest.mark.parametrize("n,inp,group", [(1, 1024, 128), (37, 1024, 128), (338, 1024, 128), (5, 1024, 1024),
                                         (9, 2048, 64), (3, 192, 64), (1500, 1024, 128)])
def test_quantize_normed_equals_oracle(dev, orc, n, inp, group):
    """LayerNorm -> quantize, bit for bit; 1500 rows take the variant that reads the statistics column in quarters."""
    import voxrt_amd as vx

    x = _x(n + inp, n, inp, scale=2.0) + np.float32(0.3)
    g = _x(1, inp) * np.float32(0.2) + np.float32(1.0)
    b = _x(2, inp) * np.float32(0.2)
    want_q, want_s, want_g = orc.quantize_normed(x, g, b, group)
    a = vx.QuantAct.quantize_normed(_t(x, dev), _t(g, dev), _t(b, dev), group)
    np.testing.assert_array_equal(a.x.cpu().numpy(), want_q)
    _bits_equal(a.scales.cpu().numpy(), want_s, "scales")
    np.testing.assert_array_equal(a.gsum.cpu().numpy(), want_g)


@pytest.mark.parametrize("n,d", [(1, 1024), (65, 1024), (7, 1027), (3, 20)])
def test_layer_norm_equals_oracle(dev, orc, n, d):
    from voxrt_amd import encoder as E

    x = _x(d, n, d, scale=3.0)
    g = _x(3, d) * np.float32(0.1) + np.float32(1.0)
    b = _x(4, d) * np.float32(0.1)
    got = E.layer_norm(_t(x, dev), _t(g, dev), _t(b, dev)).cpu().numpy()
    _bits_equal(got, orc.layer_norm(x, g, b), f"layer_norm n={n} d={d}")


def test_fold_bn_equals_oracle(orc):
    from voxrt_amd import encoder as E

    d, k = 1024, 9
    dw = _x(5, d, k, scale=0.3)
    gamma, beta, mean = _x(6, d) * 0.1 + 1, _x(7, d) * 0.1, _x(8, d) * 0.1
    var = np.random.default_rng(9).uniform(0.5, 1.5, d).astype(np.float32)
    w1, b1 = E.fold_bn(dw, gamma, beta, mean, var)
    w2, b2 = orc.fold_bn(dw, gamma, beta, mean, var)
    _bits_equal(w1, w2, "taps")
    _bits_equal(b1, b2, "bias")


@pytest.mark.parametrize("t,d", [(1, 64), (4, 64), (338, 1024), (750, 1024)])
def test_glu_dwconv_silu_equals_oracle(dev, orc, t, d):
    from voxrt_amd import encoder as E

    g = _x(t + d, t, 2 * d, scale=2.0)
    dw = _x(10, d, 9, scale=0.3)
    gamma, beta, mean = _x(11, d) * 0.1 + 1, _x(12, d) * 0.1, _x(13, d) * 0.1
    var = np.random.default_rng(14).uniform(0.5, 1.5, d).astype(np.float32)
    w_t, bias = orc.fold_bn(dw, gamma, beta, mean, var)
    want = orc.dwconv_bn_silu(orc.glu(g), w_t, bias)
    got = E.glu_dwconv_silu(_t(g, dev), _t(w_t, dev), _t(bias, dev)).cpu().numpy()
    _bits_equal(got, want, f"glu/dwconv t={t} d={d}")


@pytest.mark.parametrize("n,in_f,out_f,relu", [(1, 37, 9, False), (1, 4096, 1024, False), (6, 256, 40, True),
                                               (13, 4099, 5, False), (700, 256, 256, True), (94, 4096, 1024, False)])
def test_linear_f32_equals_oracle(dev, orc, n, in_f, out_f, relu):
    from voxrt_amd import encoder as E

    x, w, b = _x(15, n, in_f), _x(16, out_f, in_f, scale=0.05), _x(17, out_f)
    want = orc.linear_f32(x, w, b)
    if relu:
        want = np.where(want > 0, want, np.float32(0)).astype(np.float32)
    got = E.linear_f32(_t(x, dev), _t(w, dev), _t(b, dev), relu=relu).cpu().numpy()
    _bits_equal(got, want, f"linear {n}x{in_f}x{out_f}")


@pytest.mark.parametrize("kernel", ["lds", "mfma1x1", "mfma2x1", "mfma2x2"])
@pytest.mark.parametrize("n,in_f,out_f,relu", [(6, 256, 40, True), (700, 256, 256, True), (94, 4096, 1024, False),
                                               (33, 4100, 70, False), (338, 4096, 1024, False), (5, 4, 3, False),
                                               (77, 302, 19, True)])
def test_linear_f32_each_kernel(dev, orc, kernel, n, in_f, out_f, relu):
    """Both f32 linear kernels, forced: the LDS-broadcast one and the matrix-core one (K = 1 MFMA per 4-column step,
    one block per running sum) with each tile (partial output tiles, partial 128-column slabs, a partial last quad
    of steps, a tail, the subsampling's final linear), bit-exact."""
    import voxrt_amd as vx
    from voxrt_amd import encoder as E

    x, w, b = _x(19, n, in_f), _x(20, out_f, in_f, scale=0.05), _x(21, out_f)
    want = orc.linear_f32(x, w, b)
    if relu:
        want = np.where(want > 0, want, np.float32(0)).astype(np.float32)
    with vx.kernels.kernel_override(linear=kernel):
        got = E.linear_f32(_t(x, dev), _t(w, dev), _t(b, dev), relu=relu).cpu().numpy()
    _bits_equal(got, want, f"linear kernel={kernel} {n}x{in_f}x{out_f}")


@pytest.mark.parametrize("kernel", ["mfma1x1", "mfma2x2"])
def test_linear_f32_matrix_cores_on_special_operands(dev, orc, kernel):
    """The matrix-core f32 linear relies on the K = 1 MFMA rounding like fmaf (one rounding, denormals kept, signed
    zeros and exact cancellation as IEEE): operands made of denormals, zeros of both signs, values that cancel
    exactly, huge and tiny magnitudes, infinities and NaN, against the oracle's fmaf chains, bit for bit."""
    import voxrt_amd as vx
    from voxrt_amd import encoder as E

    rng = np.random.default_rng(23)
    n, in_f, out_f = 70, 512, 96
    bits = rng.integers(0, 2**32, size=(n + out_f) * in_f, dtype=np.uint64).astype(np.uint32)
    kind = rng.integers(0, 6, size=bits.size)
    mant_sign = bits & np.uint32(0x807FFFFF)
    exps = np.where(kind == 0, 0,                                   # denormals and signed zeros
           np.where(kind == 1, 1 + (bits >> 24) % 8,                # tiny normals
           np.where(kind == 2, 120 + (bits >> 24) % 16,             # ordinary
           np.where(kind == 3, 230 + (bits >> 24) % 24, 127))))     # huge / ones
    vals = (mant_sign | (exps.astype(np.uint32) << 23)).view(np.float32)
    vals[kind == 5] = np.where(bits[kind == 5] & 1, np.float32(-0.0), np.float32(0.0))
    x = vals[:n * in_f].reshape(n, in_f).copy()
    w = vals[n * in_f:].reshape(out_f, in_f).copy()
    x[3, :] = -x[4, :]                                              # exact cancellation between rows
    x[5, 7], w[9, 11] = np.inf, np.nan
    b = rng.standard_normal(out_f).astype(np.float32)
    b[::5] = -0.0
    want = orc.linear_f32(x, w, b)
    with vx.kernels.kernel_override(linear=kernel):
        got = E.linear_f32(_t(x, dev), _t(w, dev), _t(b, dev)).cpu().numpy()
    g, wv = got.view(np.uint32), want.view(np.uint32)
    same = (g == wv) | (np.isnan(got) & np.isnan(want))
    assert same.all(), f"{(~same).sum()} differ, first {np.argwhere(~same)[0]}"


@pytest.mark.parametrize("t,n_mels,c,d", [(41, 40, 16, 96), (2704, 128, 256, 1024), (9, 128, 16, 32),
                                          (130, 128, 40, 64), (137, 128, 300, 64), (141, 128, 24, 32)])
def test_subsampling_equals_oracle(dev, orc, t, n_mels, c, d):
    """128 mel bins run the first stage fused into the first depthwise stage: 3 to 676 output rows, even and odd
    row counts, and more channels than threads (300)."""
    from voxrt_amd import encoder as E

    sp = synth.synth_subsampling(d=d, c=c, n_mels=n_mels)
    feats = _x(18, t, n_mels)
    want = orc.subsampling(feats, sp)
    sub = E.Subsampling(sp, n_mels, dev)
    got = sub.forward(_t(feats, dev)).cpu().numpy()
    assert got.shape == want.shape == (sub.out_frames(t), d)
    _bits_equal(got, want, f"subsampling t={t}")


def test_rel_pos_table_equals_oracle(orc):
    from voxrt_amd import encoder as E

    for t in (1, 9, 338):
        _bits_equal(E.rel_pos_table(t, 1024), orc.rel_pos_table(t, 1024), f"pos table t={t}")


@pytest.mark.parametrize("t,heads", [(1, 1), (5, 2), (29, 2), (338, 8), (750, 8)])
def test_attention_core_equals_oracle(dev, orc, t, heads):
    from voxrt_amd import encoder as E

    d = heads * 128
    qkv = _x(19 + t, t, 3 * d)
    rel = _x(20 + t, 2 * t - 1, d)
    bu, bv = _x(21, heads, 128, scale=0.3), _x(22, heads, 128, scale=0.3)
    want = orc.attn_core_int8(qkv, rel, heads, bu, bv)
    got = E.attention_core(_t(qkv, dev), _t(rel, dev), heads, _t(bu, dev), _t(bv, dev)).cpu().numpy()
    _bits_equal(got, want, f"attention t={t} heads={heads}")


def test_gemm_single_equals_scalar(dev, orc):
    """kernels.rs:271-316: int8 rows (lcg % 255 as i8), scales (lcg % 100)/1000 + 0.001, x = (lcg % 2001)/100 - 10,
    bias (lcg % 100)/10, one token; y == scalar kernel + bias, bit for bit."""
    import torch

    import voxrt_amd as vx

    rng = synth.Lcg(99)
    for out, inp in [(8194, 640), (2560, 640), (13, 128), (8, 256), (3, 128)]:
        rows = (rng.take(out * inp) % 255).astype(np.uint8).view(np.int8).reshape(out, inp)
        scales = ((rng.take(out * inp // 128) % 100).astype(np.float32) / np.float32(1000.0)
                  + np.float32(0.001)).astype(np.float32).reshape(out, inp // 128)
        x = ((rng.take(inp) % 2001).astype(np.float32) / np.float32(100.0) - np.float32(10.0)).reshape(1, inp)
        bias = ((rng.take(out) % 100).astype(np.float32) / np.float32(10.0)).astype(np.float32)
        q, xs, _ = orc.quantize(x, 128)
        want = (orc.gemm(rows, scales, q, xs, 128) + bias[None, :]).astype(np.float32)
        w = vx.TernaryMatrix.from_i8_rows(rows, scales, out, inp, 128)
        xa = vx.QuantAct.quantize(_t(x, dev), 128)
        y = torch.zeros((1, out), dtype=torch.float32, device=dev)
        vx.kernels.gemm_single(w, xa, y, _t(bias, dev))
        _bits_equal(y.cpu().numpy(), want, f"gemv out={out} inp={inp}")


def _oracle_layer(orc, p):
    d = p["norms"]["out"][0].size
    lp = {}
    for n, (q, s) in p["linears"].items():
        inp = s.shape[1] * 128
        lp[n] = (orc.unpack_rows(q, inp), orc.f16_to_f32(s))
    lp["norms"] = p["norms"]
    lp["bias_u"], lp["bias_v"] = p["bias_u"], p["bias_v"]
    lp["dw_t"], lp["dw_bias"] = orc.fold_bn(p["dw"], **p["bn"])
    assert lp["dw_t"].shape[1] == d
    return lp


@pytest.mark.parametrize("graphs", [False, True])
def test_encoder_layers_equal_oracle(dev, orc, graphs):
    """Two full-width layers (d=1024, 8 heads, FFN 4096, conv kernel 9) at t=64: the device layer stack equals the
    CPU int8 layer restatement bit for bit; with graphs, three replays in a row agree with it too."""
    from voxrt_amd import encoder as E

    t, L = 64, 2
    params = [synth.synth_layer(i) for i in range(L)]
    enc = E.Encoder(n_layers=L)
    enc.use_graphs(graphs)
    for i, p in enumerate(params):
        enc.set_layer(i, p)
    x = _x(23, t, 1024)
    want = x.copy()
    pos = orc.rel_pos_table(t, 1024)
    for p in params:
        want = orc.conformer_layer(want, pos, _oracle_layer(orc, p), heads=8)
    xd = _t(x, dev)
    for rep in range(3 if graphs else 1):
        got = enc.forward(xd).cpu().numpy()
        _bits_equal(got, want, f"encoder layers (graphs={graphs}, pass {rep})")
    enc.free()


def test_encoder_feats_equal_oracle(dev, orc):
    """Subsampling + one layer from log-mel features (t_in = 200 -> 25 frames), bit-exact."""
    from voxrt_amd import encoder as E

    t_in = 200
    p = synth.synth_layer(5)
    sp = synth.synth_subsampling()
    enc = E.Encoder(n_layers=1)
    enc.set_layer(0, p)
    enc.set_subsampling(sp)
    feats = _x(24, t_in, 128)
    x = orc.subsampling(feats, sp)
    t = x.shape[0]
    want = orc.conformer_layer(x, orc.rel_pos_table(t, 1024), _oracle_layer(orc, p), heads=8)
    got = enc.forward_feats(_t(feats, dev)).cpu().numpy()
    assert got.shape == (t, 1024) == (enc.out_frames(t_in), 1024)
    _bits_equal(got, want, "encoder from features")
    enc.free()


def test_encoder_batch_equals_oracle(dev, orc):
    """Three segments of t=29 frames in one batched pass through two full-width layers (graphs on, two replays):
    every segment equals the CPU int8 layer restatement of that segment alone, bit for bit (the batched GEMMs see
    87 rows, the attention and the depthwise convolution stay inside each segment)."""
    from voxrt_amd import encoder as E

    nseg, t, L = 3, 29, 2
    params = [synth.synth_layer(10 + i) for i in range(L)]
    enc = E.Encoder(n_layers=L)
    for i, p in enumerate(params):
        enc.set_layer(i, p)
    x = _x(31, nseg, t, 1024)
    pos = orc.rel_pos_table(t, 1024)
    want = []
    for s in range(nseg):
        y = x[s].copy()
        for p in params:
            y = orc.conformer_layer(y, pos, _oracle_layer(orc, p), heads=8)
        want.append(y)
    xd = _t(x, dev)
    for rep in range(2):
        got = enc.forward_batch(xd).cpu().numpy()
        assert got.shape == (nseg, t, 1024)
        for s in range(nseg):
            _bits_equal(got[s], want[s], f"batched encoder segment {s} (pass {rep})")
    enc.free()


def test_encoder_feats_batch_equals_oracle(dev, orc):
    """Four segments of 120 log-mel frames (15 frames after subsampling) through subsampling and one layer in one
    batched pass: each segment equals the oracle's subsampling + layer of that segment, bit for bit."""
    from voxrt_amd import encoder as E

    nseg, t_in = 4, 120
    p = synth.synth_layer(6)
    sp = synth.synth_subsampling()
    enc = E.Encoder(n_layers=1)
    enc.set_layer(0, p)
    enc.set_subsampling(sp)
    feats = _x(32, nseg, t_in, 128)
    got = enc.forward_feats_batch(_t(feats, dev)).cpu().numpy()
    lp = _oracle_layer(orc, p)
    for s in range(nseg):
        x = orc.subsampling(feats[s], sp)
        t = x.shape[0]
        want = orc.conformer_layer(x, orc.rel_pos_table(t, 1024), lp, heads=8)
        assert got.shape == (nseg, t, 1024)
        _bits_equal(got[s], want, f"batched features segment {s}")
    enc.free()


def test_encoder_batch_of_32_equals_single_segments(dev):
    """32 segments of 125 frames (the 32 x 10 s workload: 4000 rows, so the GEMMs take the large-token kernels)
    through one layer: each segment of the batched pass equals the single-segment pass of that segment."""
    import torch

    from voxrt_amd import encoder as E

    nseg, t = 32, 125
    enc = E.Encoder(n_layers=1)
    enc.set_layer(0, synth.synth_layer(7))
    x = _t(_x(33, nseg, t, 1024), dev)
    got = enc.forward_batch(x).cpu().numpy()
    for s in (0, 1, 17, 31):
        one = enc.forward(x[s].contiguous()).cpu().numpy()
        _bits_equal(got[s], one, f"batch of 32, segment {s}")
    torch.cuda.synchronize()
    enc.free()


@pytest.mark.parametrize("t,k", [(1, 9), (29, 9), (338, 9), (750, 9), (29, 7), (338, 5)])
def test_glu_dwconv_silu_quantize_equals_oracle(dev, orc, t, k):
    """The conv rows quantized for pointwise_conv2 in the same kernel (encoder.rs:605-625) equal the oracle's
    dwconv_bn_silu(glu(g)) quantized in 128-channel groups: codes, scales and code sums bit for bit, pad tokens
    zero. Kernel size 9 (the model's) runs the 8-row tiled kernel, other sizes the per-row kernel."""
    import torch

    from voxrt_amd import encoder as E

    d = 1024
    g = _x(t + 7, t, 2 * d, scale=2.0)
    dw = _x(20, d, k, scale=0.3)
    gamma, beta, mean = _x(21, d) * 0.1 + 1, _x(22, d) * 0.1, _x(23, d) * 0.1
    var = np.random.default_rng(24).uniform(0.5, 1.5, d).astype(np.float32)
    w_t, bias = orc.fold_bn(dw, gamma, beta, mean, var)
    wq, ws, wg = orc.quantize(orc.dwconv_bn_silu(orc.glu(g), w_t, bias), 128)
    got = E.glu_dwconv_silu_quantize(_t(g, dev), _t(w_t, dev), _t(bias, dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.x.cpu().numpy(), wq, err_msg=f"codes t={t}")
    st, gt = got.scales_t.cpu().numpy(), got.gsum_t.cpu().numpy()
    _bits_equal(st[:, :t].T.copy(), ws, f"scales t={t}")
    np.testing.assert_array_equal(gt[:, :t].T, wg, err_msg=f"gsum t={t}")
    assert not st[:, t:].any() and not gt[:, t:].any(), f"pad tokens not zero t={t}"


@pytest.mark.parametrize("t,heads", [(1, 8), (29, 8), (338, 8), (750, 2)])
def test_attention_core_quantize_equals_oracle(dev, orc, t, heads):
    """The attention core writing the o-projection's activations (encoder.rs:180-183) equals the oracle's
    attn_core_int8 quantized in 128-column groups: codes, scales and code sums bit for bit, pad tokens zero."""
    import torch

    from voxrt_amd import encoder as E

    d = heads * 128
    qkv = _x(29 + t, t, 3 * d)
    rel = _x(30 + t, 2 * t - 1, d)
    bu, bv = _x(31, heads, 128, scale=0.3), _x(32, heads, 128, scale=0.3)
    wq, ws, wg = orc.quantize(orc.attn_core_int8(qkv, rel, heads, bu, bv), 128)
    got = E.attention_core_quantize(_t(qkv, dev), _t(rel, dev), heads, _t(bu, dev), _t(bv, dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.x.cpu().numpy(), wq, err_msg=f"codes t={t}")
    st, gt = got.scales_t.cpu().numpy(), got.gsum_t.cpu().numpy()
    _bits_equal(st[:, :t].T.copy(), ws, f"scales t={t}")
    np.testing.assert_array_equal(gt[:, :t].T, wg, err_msg=f"gsum t={t}")
    assert not st[:, t:].any() and not gt[:, t:].any(), f"pad tokens not zero t={t}"


def test_encoder_from_model_directory(dev, orc, tmp_path):
    """An encoder loaded from a model directory (thrush-ternary-v2 files, HF tensor names; voxrt_amd.model) equals
    the oracle encoder on the same file's parameters: subsampling and two layers from features, bit for bit."""
    from modeldir import synth_model, write_model_dir
    from voxrt_amd import encoder as E
    from voxrt_amd import model as M

    layers, sp = synth_model(d=1024, heads=8, ff=4096, n_layers=2, n_mels=128, c=256)
    path = write_model_dir(str(tmp_path / "model"), layers, sp, d=1024, heads=8, ff=4096, n_mels=128, c=256)
    m = M.ModelFile(path)
    assert m.validate() == []
    enc = M.load_encoder(m)
    feats = _x(77, 203, 128)
    got = enc.forward_feats(_t(feats, dev)).cpu().numpy()
    enc.free()
    x = orc.subsampling(feats, M.subsampling_params(m))
    t = x.shape[0]
    pos = orc.rel_pos_table(t, 1024)
    for i in range(2):
        x = orc.conformer_layer(x, pos, _oracle_layer(orc, M.layer_params(m, i)), heads=8)
    _bits_equal(got, x, "encoder from a model directory")


def _small_encoder(n_layers=2, d=256, heads=2, ff=1024):
    from voxrt_amd import encoder as E

    params = [synth.synth_layer(40 + i, d=d, ff=ff, heads=heads) for i in range(n_layers)]
    enc = E.Encoder(d=d, heads=heads, ff=ff, n_layers=n_layers)
    for i, p in enumerate(params):
        enc.set_layer(i, p)
    return enc, params


def _oracle_stack(orc, x, params, heads):
    pos = orc.rel_pos_table(x.shape[0], x.shape[1])
    for p in params:
        x = orc.conformer_layer(x, pos, _oracle_layer(orc, p), heads=heads)
    return x


def test_encoder_workspace_is_bounded_over_many_lengths(dev, orc):
    """20 distinct frame counts in a row (VAD-like segment lengths, the longest fifth): one workspace serves them
    all. It stops growing once the longest has run, at most 8 graphs are kept, and every output equals the oracle
    bit for bit (GpuEncoder's single growing workspace, metal/mod.rs:449-460,641-645)."""
    enc, params = _small_encoder()
    lengths = [25, 188, 60, 125, 750, 33, 97, 140, 301, 64, 1, 17, 480, 199, 2, 77, 256, 49, 600, 333]
    assert len(set(lengths)) == 20
    sizes = []
    for i, t in enumerate(lengths):
        x = _x(300 + t, t, 256)
        got = enc.forward(_t(x, dev)).cpu().numpy()
        _bits_equal(got, _oracle_stack(orc, x, params, 2), f"t={t}")
        ws, graphs = enc.memory()
        sizes.append(ws)
        assert graphs <= 8, graphs
    top = lengths.index(750)
    assert all(s == sizes[top] for s in sizes[top:]), sizes
    assert sizes[top] > 0 and max(sizes) == sizes[top]
    enc.free()


def test_encoder_calls_from_two_threads_on_two_streams(dev, orc):
    """Two host threads, each on its own stream, call one encoder four times each with different lengths: the calls
    are serialized and ordered on the device, so every output equals the one-at-a-time result."""
    import threading

    import torch

    enc, params = _small_encoder()
    jobs = {0: [(29, 1), (64, 2), (29, 3), (101, 4)], 1: [(64, 5), (29, 6), (77, 7), (64, 8)]}
    inputs = {seed: _x(400 + seed, t, 256) for lst in jobs.values() for t, seed in lst}
    want = {seed: _oracle_stack(orc, inputs[seed], params, 2) for seed in inputs}
    got, errors = {}, []

    def worker(k):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for t, seed in jobs[k]:
                    got[seed] = enc.forward(_t(inputs[seed], dev))
            s.synchronize()
        except Exception as e:  # reported by the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(k,)) for k in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    torch.cuda.synchronize()
    for seed, w in want.items():
        _bits_equal(got[seed].cpu().numpy(), w, f"threaded call {seed}")
    enc.free()


def test_encoder_profile_sums_sublayers(dev, orc):
    """With profiling on (the reference's VOXRT_PROFILE), a forward reports device time per sublayer type; the types
    add up to the total and the output is the same as without profiling."""
    enc, params = _small_encoder()
    x = _x(500, 88, 256)
    want = _oracle_stack(orc, x, params, 2)
    enc.set_profiling(True)
    got = enc.forward(_t(x, dev)).cpu().numpy()
    p = enc.take_profile()
    _bits_equal(got, want, "profiled forward")
    assert p["forwards"] == 1
    parts = [p[k] for k in ("subsampling_ms", "ff_ms", "attn_ms", "conv_ms", "norm_ms")]
    assert all(v > 0 for v in parts[1:]) and p["attn_core_ms"] > 0
    assert abs(sum(parts) - p["total_ms"]) <= 0.02 * p["total_ms"] + 1e-3
    assert enc.take_profile()["forwards"] == 0
    enc.set_profiling(False)
    _bits_equal(enc.forward(_t(x, dev)).cpu().numpy(), want, "after profiling")
    enc.free()
