"""The oracle's encoder composition pinned by checks that do not restate it.

``or_conformer_layer`` (oracle/encoder_oracle.c, restating encoder.rs:79-94,138-191,576-628,706-756) is the one
oracle function whose pieces are pinned one by one but whose composition — which LayerNorm feeds which linear, the
residual scales, the q|k|v split, the relative-position band, the GLU halves, the sublayer order — would otherwise
be checked only against a second restatement. Here it is checked:

1. in closed form: with every ternary weight zero, each sublayer adds exactly zero, so the layer is
   ``layer_norm(x, norm_out)`` bit for bit;
2. against an independent implementation of the same model: Hugging Face transformers' Parakeet encoder
   (tests/hf_parakeet.py), run in float64 with the dequantized weights, one sublayer at a time and whole;
3. with planted mistakes: the same composition rebuilt from the oracle's pinned pieces with one plausible misreading
   each (a residual scale, a LayerNorm, the q/k order, the position direction, the u/v biases, the GLU halves, the
   sublayer order, norm_out) must land outside the tolerance that the oracle itself meets.

The tolerance is the int8 activation quantization of the reference's int8 path (per-(token, 128-column group)
absmax codes, packed.rs:523-536) against float64: about 0.5 % of the output's range for one layer, 2 % after 24.
"""
import numpy as np
import pytest

from voxrt_amd import synth

hf = pytest.importorskip("hf_parakeet")


def _x(seed, *shape, scale=1.0):
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)


def _rel(got, want):
    """(max |got - want| / max |want|, mean |got - want| / mean |want|)."""
    diff = np.abs(np.asarray(got, np.float64) - want)
    return diff.max() / np.abs(want).max(), diff.mean() / np.abs(want).mean()


def _zero_linears(p, names):
    """A copy of layer p whose listed linears hold only zero trits (scales unchanged)."""
    q = dict(p)
    q["linears"] = dict(p["linears"])
    for n in names:
        packed, s16 = p["linears"][n]
        inp = s16.shape[1] * 128
        q["linears"][n] = (synth.pack_rows(np.zeros((packed.shape[0], inp), np.int8)), s16)
    return q


def _layer(seed, d=1024, heads=8, ff=4096):
    """A synthetic layer with relative-position biases of unit size, so that bias_u and bias_v weigh as much as
    the query they are added to (synth_layer's 0.1 would let a u/v swap hide inside the quantization error)."""
    p = synth.synth_layer(seed, d=d, ff=ff, heads=heads)
    r = np.random.default_rng(seed + 500)
    p["bias_u"] = r.standard_normal(p["bias_u"].shape).astype(np.float32)
    p["bias_v"] = r.standard_normal(p["bias_v"].shape).astype(np.float32)
    return p


def _oracle_params(orc, p):
    lp = {}
    for n, (q, s) in p["linears"].items():
        lp[n] = (orc.unpack_rows(q, s.shape[1] * 128), orc.f16_to_f32(s))
    lp["norms"] = p["norms"]
    lp["bias_u"], lp["bias_v"] = p["bias_u"], p["bias_v"]
    lp["dw_t"], lp["dw_bias"] = orc.fold_bn(p["dw"], **p["bn"])
    return lp


SUBLAYER_LINEARS = {"ff1": ("ff1_w1", "ff1_w2"), "attn": ("qkv", "o", "pos"), "conv": ("pw1", "pw2"),
                    "ff2": ("ff2_w1", "ff2_w2")}
ALL_LINEARS = tuple(n for v in SUBLAYER_LINEARS.values() for n in v)


def test_zero_trits_leave_only_norm_out(orc):
    """Every sublayer's last linear is an AddScaled GEMM of zero trits: fma(alpha, 0, x) = x, so the residual
    stream passes through untouched and the layer equals layer_norm(x, norm_out) exactly."""
    d, heads, ff, t = 256, 2, 1024, 23
    p = _zero_linears(_layer(1, d, heads, ff), ALL_LINEARS)
    x = _x(2, t, d, scale=2.0)
    got = orc.conformer_layer(x, orc.rel_pos_table(t, d), _oracle_params(orc, p), heads=heads)
    want = orc.layer_norm(x, *p["norms"]["out"])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.fixture(scope="module")
def layer0():
    return _layer(0)


@pytest.mark.parametrize("only", ["ff1", "attn", "conv", "ff2"])
def test_one_sublayer_against_hf(orc, layer0, only):
    """One sublayer live, the others' linears zero: the oracle layer equals HF's block within the int8
    quantization error, and the same sublayer with its residual scale doubled or halved does not."""
    t = 48
    keep = set(SUBLAYER_LINEARS[only])
    p = _zero_linears(layer0, [n for n in ALL_LINEARS if n not in keep])
    x = _x(3, t, 1024)
    pos = orc.rel_pos_table(t, 1024)
    got = orc.conformer_layer(x, pos, _oracle_params(orc, p), heads=8)
    want = hf.layers_forward(hf.encoder([p]), x)
    mx, mean = _rel(got, want)
    assert mx < 0.01 and mean < 0.006, (only, mx, mean)
    wrong = _compose(orc, x, pos, _oracle_params(orc, p), 8, f"{only}_scale")
    assert _rel(wrong, want)[1] > 0.02, only


def _compose(orc, x, pos, lp, heads, mistake=None):
    """The layer rebuilt from the oracle's pinned pieces (quantize_normed, gemm, quantize, attn_core_int8, glu,
    dwconv_bn_silu, layer_norm), with one planted mistake when `mistake` names one."""
    d = x.shape[1]

    def lin(name, q, s, y=None, ep=0, alpha=0.0):
        w, ws = lp[name]
        return orc.gemm(w, ws, q, s, 128, y=y, ep=ep, alpha=alpha)

    def norm(name):
        if mistake == "attn_conv_norms_swapped" and name in ("attn", "conv"):
            name = "conv" if name == "attn" else "attn"
        if mistake == "ff2_reads_ff1_norm" and name == "ff2":
            name = "ff1"
        return lp["norms"][name]

    def scale(sub, right):
        return (2.0 * right if right < 1.0 else 0.5 * right) if mistake == f"{sub}_scale" else right

    def ffn(x, w1, w2, nm):
        q, s, _ = orc.quantize_normed(x, *norm(nm), 128)
        q2, s2, _ = orc.quantize(lin(w1, q, s, ep=orc.EP_SILU), 128)
        return lin(w2, q2, s2, y=x.copy(), ep=orc.EP_ADD_SCALED, alpha=scale(nm, 0.5))

    def attn(x):
        q, s, _ = orc.quantize_normed(x, *norm("attn"), 128)
        qkv = lin("qkv", q, s)
        if mistake == "q_k_swapped":
            qkv = np.concatenate([qkv[:, d:2 * d], qkv[:, :d], qkv[:, 2 * d:]], 1)
        qp, sp, _ = orc.quantize(pos[::-1].copy() if mistake == "positions_reversed" else pos, 128)
        bu, bv = (lp["bias_v"], lp["bias_u"]) if mistake == "bias_u_v_swapped" else (lp["bias_u"], lp["bias_v"])
        qc, sc, _ = orc.quantize(orc.attn_core_int8(qkv, lin("pos", qp, sp), heads, bu, bv), 128)
        return lin("o", qc, sc, y=x.copy(), ep=orc.EP_ADD_SCALED, alpha=scale("attn", 1.0))

    def conv(x):
        q, s, _ = orc.quantize_normed(x, *norm("conv"), 128)
        g2 = lin("pw1", q, s)
        if mistake == "glu_halves_swapped":
            g2 = np.concatenate([g2[:, d:], g2[:, :d]], 1)
        qh, sh, _ = orc.quantize(orc.dwconv_bn_silu(orc.glu(g2), lp["dw_t"], lp["dw_bias"]), 128)
        return lin("pw2", qh, sh, y=x.copy(), ep=orc.EP_ADD_SCALED, alpha=scale("conv", 1.0))

    x = ffn(x, "ff1_w1", "ff1_w2", "ff1")
    x = attn(conv(x)) if mistake == "conv_before_attn" else conv(attn(x))
    x = ffn(x, "ff2_w1", "ff2_w2", "ff2")
    return x if mistake == "no_norm_out" else orc.layer_norm(x, *norm("out"))


MISTAKES = ["ff1_scale", "ff2_scale", "attn_scale", "conv_scale", "attn_conv_norms_swapped", "ff2_reads_ff1_norm",
            "q_k_swapped", "positions_reversed", "bias_u_v_swapped", "glu_halves_swapped", "conv_before_attn",
            "no_norm_out"]


def test_layer_against_hf_and_planted_mistakes(orc, layer0):
    """The whole layer: the oracle is within the quantization error of HF's float64 block; the composition rebuilt
    from the pinned pieces equals the oracle bit for bit; each planted mistake lands at least twice as far."""
    t = 64
    x = _x(4, t, 1024)
    pos = orc.rel_pos_table(t, 1024)
    lp = _oracle_params(orc, layer0)
    want = hf.layers_forward(hf.encoder([layer0]), x)
    got = orc.conformer_layer(x, pos, lp, heads=8)
    mx, mean = _rel(got, want)
    assert mx < 0.01 and mean < 0.008, (mx, mean)
    np.testing.assert_array_equal(_compose(orc, x, pos, lp, 8).view(np.uint32), got.view(np.uint32))
    far = {m: _rel(_compose(orc, x, pos, lp, 8, m), want)[1] for m in MISTAKES}
    near = [m for m, e in far.items() if e < 2 * mean or e < 0.016]
    assert not near, {m: far[m] for m in near}


def test_rel_pos_table_against_hf(orc):
    """HF's float32 table (positions t-1 .. -(t-1), sin/cos interleaved per frequency): the oracle's table (the C
    library's powf/sinf/cosf where the reference calls the libm crate's) agrees to float32 rounding."""
    for t in (1, 9, 338, 750):
        got, want = orc.rel_pos_table(t, 1024), hf.rel_pos_table(t, 1024)
        assert got.shape == want.shape == (2 * t - 1, 1024)
        assert np.abs(got.astype(np.float64) - want).max() < 4e-6 * max(1, t / 64), t


def test_subsampling_against_hf(orc):
    """The f32 subsampling (subsampling.rs:109-204) against HF's Conv2D stack in float64 (NCHW, channel-major
    flatten): rounding-level agreement."""
    sp = synth.synth_subsampling()
    enc = hf.encoder([], sp)
    feats = _x(5, 203, 128)
    got = orc.subsampling(feats, sp)
    want = hf.subsample(enc, feats)
    assert got.shape == want.shape == (orc.subsampling_frames(203), 1024)
    assert _rel(got, want)[0] < 1e-5


@pytest.mark.slow
def test_encoder_24_layers_from_features_against_hf(orc):
    """The oracle's subsampling + 24 conformer layers (one 10 s segment: 1000 mel frames -> 125) against HF's
    ParakeetEncoder in float64 on the same parameters: within 3 % of the output's range (the int8 quantization of
    24 layers; measured 2.0 % and 1.5 % mean), and every layer's output within 3.5 % (mean 2 %) on the way."""
    layers = [synth.synth_layer(i) for i in range(24)]
    sp = synth.synth_subsampling()
    enc = hf.encoder(layers, sp)
    feats = _x(6, 1000, 128)
    x = orc.subsampling(feats, sp)
    t = x.shape[0]
    assert t == 125
    pos = orc.rel_pos_table(t, 1024)
    outs = hf.layer_outputs(enc, feats)
    for i, p in enumerate(layers):
        x = orc.conformer_layer(x, pos, _oracle_params(orc, p), heads=8)
        mx, mean = _rel(x, outs[i])
        assert mx < 0.035 and mean < 0.02, (i, mx, mean)
    mx, mean = _rel(x, hf.forward_feats(enc, feats))
    assert mx < 0.03 and mean < 0.02, (mx, mean)
