"""Pins the encoder half of the oracle (oracle/encoder_oracle.c) against independent float64 computations, closed
forms and compositions, before the HIP encoder kernels are compared with it.

Reference behaviour followed: crates/voxrt/src/tensor.rs (row_mean_var_portable 331-363, layer_norm_row 712-719,
exp_row_scaled_portable 810-826, glu_row_portable 936-940, silu_row 962-973, linear/tile_rows_portable 98-127,
233-261), encoder.rs (fold 548-573, dwconv 602-624, rel_pos_table 760-776, attn_core_int8 317-534, layer
706-756), subsampling.rs:109-204; the bounds come from the reference's own tests (exp_poly error < 3e-7 at
tensor.rs:1018-1030; encoder goldens at 1e-4 / 1e-3, golden_encoder.rs:14-76).
"""
import numpy as np
import pytest
import torch

from voxrt_amd import synth


def _x(seed, *shape, scale=1.0):
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)


def _numpy_mean_var_f32(x):
    """The lane order of row_mean_var_portable walked in numpy float32 (an independent loop, not the C code)."""
    f = np.float32
    d = x.size
    n8 = d // 8 * 8
    s0 = np.zeros(4, f)
    s1 = np.zeros(4, f)
    for c in range(0, n8, 8):
        s0 = (s0 + x[c:c + 4]).astype(f)
        s1 = (s1 + x[c + 4:c + 8]).astype(f)
    p = (s0 + s1).astype(f)
    s = f(f(p[0] + p[1]) + f(p[2] + p[3]))
    for v in x[n8:]:
        s = f(s + v)
    mean = f(s / f(d))
    q0 = np.zeros(4, np.float64)
    q1 = np.zeros(4, np.float64)
    qs0, qs1 = np.zeros(4, f), np.zeros(4, f)
    for c in range(0, n8, 8):
        a = (x[c:c + 4] - mean).astype(f)
        e = (x[c + 4:c + 8] - mean).astype(f)
        # fma: exact product plus accumulator, one rounding (float64 holds a*a exactly for float32 a)
        qs0 = (a.astype(np.float64) * a + qs0.astype(np.float64)).astype(f)
        qs1 = (e.astype(np.float64) * e + qs1.astype(np.float64)).astype(f)
    p = (qs0 + qs1).astype(f)
    sq = f(f(p[0] + p[1]) + f(p[2] + p[3]))
    for v in x[n8:]:
        a = f(v - mean)
        sq = f(sq + f(a * a))
    del q0, q1
    return mean, f(sq / f(d))


@pytest.mark.parametrize("d", [8, 20, 1024, 1027])
def test_row_mean_var_lane_order(orc, d):
    x = _x(d, d, scale=3.0) + np.float32(0.5)
    m, v = orc.row_mean_var(x)
    m2, v2 = _numpy_mean_var_f32(x)
    assert np.float32(m) == m2 and np.float32(v) == v2
    xd = x.astype(np.float64)
    assert abs(m - xd.mean()) < 1e-5 * (1 + abs(xd.mean())) and abs(v - xd.var()) < 1e-5 * xd.var()


def test_layer_norm_against_float64_and_constant_rows(orc):
    x = _x(1, 9, 1024, scale=2.0)
    g = _x(2, 1024) * np.float32(0.1) + np.float32(1.0)
    b = _x(3, 1024) * np.float32(0.1)
    y = orc.layer_norm(x, g, b)
    xd = x.astype(np.float64)
    want = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * g + b
    assert np.abs(y - want).max() < 2e-5
    const = np.full((2, 1024), 3.25, np.float32)
    np.testing.assert_array_equal(orc.layer_norm(const, g, b), np.broadcast_to(b, (2, 1024)))


def test_quantize_normed_is_quantize_of_layer_norm(orc):
    x = _x(4, 37, 1024, scale=1.5)
    g = _x(5, 1024) * np.float32(0.2) + np.float32(1.0)
    b = _x(6, 1024) * np.float32(0.2)
    for group in (128, 1024):
        q, s, gs = orc.quantize_normed(x, g, b, group)
        q2, s2, gs2 = orc.quantize(orc.layer_norm(x, g, b), group)
        np.testing.assert_array_equal(q, q2)
        np.testing.assert_array_equal(s, s2)
        np.testing.assert_array_equal(gs, gs2)


@pytest.mark.parametrize("n", [1, 7, 338, 750])
def test_exp_row_scaled(orc, n):
    row = _x(n, n, scale=20.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(128.0))
    e, s = orc.exp_row_scaled(row, float(scale))
    sc = (row * scale).astype(np.float32)
    mx = sc.max()
    want = np.exp((sc - mx).astype(np.float32).astype(np.float64))
    assert np.abs(e / want - 1).max() < 3e-7
    assert e[np.argmax(sc)] == 1.0
    assert abs(s - want.sum()) < 1e-6 * want.sum()


def test_glu(orc):
    gb = _x(7, 11, 2 * 64, scale=4.0)
    out = orc.glu(gb)
    a, b = gb[:, :64].astype(np.float64), gb[:, 64:].astype(np.float64)
    want = a / (1 + np.exp(-b))
    assert np.abs(out - want).max() < 1e-6 * (1 + np.abs(want).max())


def test_dwconv_bn_silu_against_torch_conv1d(orc):
    t, d, k = 23, 64, 9
    a = _x(8, t, d)
    dw = _x(9, d, k, scale=0.3)
    gamma, beta, mean = _x(10, d) * 0.1 + 1, _x(11, d) * 0.1, _x(12, d) * 0.1
    var = np.random.default_rng(13).uniform(0.5, 1.5, d).astype(np.float32)
    dw_t, bias = orc.fold_bn(dw, gamma, beta, mean, var)
    got = orc.dwconv_bn_silu(a, dw_t, bias)
    xt = torch.from_numpy(a.astype(np.float64)).T[None]  # [1, d, t]
    conv = torch.nn.functional.conv1d(xt, torch.from_numpy(dw.astype(np.float64))[:, None, :], padding=(k - 1) // 2,
                                      groups=d)[0].T.numpy()
    bn = (conv - mean) / np.sqrt(var.astype(np.float64) + 1e-5) * gamma + beta
    want = bn / (1 + np.exp(-bn))
    assert np.abs(got - want).max() < 2e-5 * (1 + np.abs(want).max())


def test_rel_pos_table(orc):
    t, d = 9, 64
    tab = orc.rel_pos_table(t, d)
    pos = (t - 1 - np.arange(2 * t - 1))[:, None].astype(np.float64)
    inv = 1.0 / 10000.0 ** (2 * np.arange(d // 2) / d)
    assert np.abs(tab[:, 0::2] - np.sin(pos * inv)).max() < 2e-6 * t
    assert np.abs(tab[:, 1::2] - np.cos(pos * inv)).max() < 2e-6 * t
    np.testing.assert_array_equal(tab[t - 1, 0::2], 0.0)  # position 0: sin 0, cos 1
    np.testing.assert_array_equal(tab[t - 1, 1::2], 1.0)


@pytest.mark.parametrize("n,in_f,out_f", [(1, 37, 9), (6, 256, 40), (13, 4099, 5)])
def test_linear_f32(orc, n, in_f, out_f):
    x, w, b = _x(14, n, in_f), _x(15, out_f, in_f, scale=0.05), _x(16, out_f)
    y = orc.linear_f32(x, w, b)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.abs(y - want).max() < 1e-5 * (1 + np.abs(want).max())
    if n > 1:  # the lane order walked in numpy float32 for one output
        f = np.float32
        c4 = in_f // 4 * 4
        acc = np.zeros(4, np.float64)
        accf = np.zeros(4, f)
        for c in range(0, c4, 4):
            accf = (w[1, c:c + 4].astype(np.float64) * x[2, c:c + 4] + accf).astype(f)
        tail = f(0)
        for c in range(c4, in_f):
            tail = f(tail + f(w[1, c] * x[2, c]))
        del acc
        assert y[2, 1] == f(f(f(f(accf[0] + accf[1]) + f(accf[2] + accf[3])) + tail) + b[1])


def test_subsampling_against_torch(orc):
    sp = synth.synth_subsampling(d=96, c=16, n_mels=40)
    t = 41
    feats = _x(17, t, 40)
    got = orc.subsampling(feats, sp)
    k, c = 3, 16
    D = torch.float64
    x = torch.from_numpy(feats.astype(np.float64))[None, None]  # [1, 1, T, F]
    w0 = torch.from_numpy(sp["conv0_w"].astype(np.float64)).T.reshape(c, 1, k, k)
    x = torch.relu(torch.nn.functional.conv2d(x, w0, torch.from_numpy(sp["conv0_b"]).to(D), stride=2, padding=1))
    for st in range(2):
        wd = torch.from_numpy(sp["dw_w"][st].astype(np.float64)).T.reshape(c, 1, k, k)
        x = torch.nn.functional.conv2d(x, wd, torch.from_numpy(sp["dw_b"][st]).to(D), stride=2, padding=1, groups=c)
        wp = torch.from_numpy(sp["pw_w"][st].astype(np.float64))[:, :, None, None]
        x = torch.relu(torch.nn.functional.conv2d(x, wp, torch.from_numpy(sp["pw_b"][st]).to(D)))
    t3, f3 = x.shape[2], x.shape[3]
    flat = x[0].permute(1, 2, 0).reshape(t3, f3 * c)  # channels-last flatten f*C + c
    want = (flat @ torch.from_numpy(sp["lin_w"].astype(np.float64)).T + torch.from_numpy(sp["lin_b"]).to(D)).numpy()
    assert got.shape == (orc.subsampling_frames(t), 96) == want.shape
    assert np.abs(got - want).max() < 1e-4 * (1 + np.abs(want).max())


def _attn_f64(qkv, rel_k, heads, bu, bv):
    t, d3 = qkv.shape
    d = d3 // 3
    dh = d // heads
    q, k, v = (qkv[:, i * d:(i + 1) * d].astype(np.float64) for i in range(3))
    out = np.zeros((t, d))
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        s1 = (q[:, sl] + bu[h]) @ k[:, sl].T
        s2f = (q[:, sl] + bv[h]) @ rel_k[:, sl].astype(np.float64).T  # [t, 2t-1]
        idx = (t - 1 - np.arange(t))[:, None] + np.arange(t)[None, :]
        s2 = np.take_along_axis(s2f, idx, 1)
        sc = (s1 + s2) / np.sqrt(dh)
        p = np.exp(sc - sc.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[:, sl] = p @ v[:, sl]
    return out


def test_attention_core_against_float64_softmax(orc):
    t, d, heads = 29, 128, 2
    qkv = _x(18, t, 3 * d)
    rel = _x(19, 2 * t - 1, d)
    bu, bv = _x(20, heads, d // heads, scale=0.3), _x(21, heads, d // heads, scale=0.3)
    got = orc.attn_core_int8(qkv, rel, heads, bu, bv)
    want = _attn_f64(qkv, rel, heads, bu, bv)
    # int8 operands (1/127 relative steps) through a softmax and an int8 context product
    assert np.abs(got - want).max() < 0.05 * np.abs(want).max()
    assert np.abs(got - want).mean() < 0.03 * np.abs(want).mean()


def test_attention_position_band_by_one_hot_table(orc):
    """Keys and biases zero and a relative table whose row p is e_0 * (p == target): every query then puts all its
    weight on the one key j with t-1-i+j == target, so the context equals v[j] — a wrong band offset or sign
    selects a different key."""
    t, d, heads = 12, 64, 1
    rng = np.random.default_rng(22)
    qkv = np.zeros((t, 3 * d), np.float32)
    qkv[:, 0] = 60.0  # q: large first component
    qkv[:, 2 * d:] = rng.integers(-100, 100, (t, d)).astype(np.float32) / np.float32(8.0)
    target = t - 1 + 3  # relative offset +3: key j = i + 3
    rel = np.zeros((2 * t - 1, d), np.float32)
    rel[target, 0] = 1.0
    z = np.zeros((heads, d), np.float32)
    got = orc.attn_core_int8(qkv, rel, heads, z, z)
    for i in range(t - 3):
        want = qkv[i + 3, 2 * d:]
        assert np.abs(got[i] - want).max() < 0.02 * np.abs(want).max(), i


# The conformer layer's composition is pinned in tests/test_oracle_hf.py (zero-weight closed form, Hugging Face's
# float64 Parakeet encoder, planted mistakes).
