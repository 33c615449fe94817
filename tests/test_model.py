"""The model-file loader (voxrt_amd.model): format checks and validation as format.rs does them, and the
load-time transforms (q|k|v stacking, f16 widening, subsampling layouts) against the tensors written to a
synthetic model directory and against torch on the file's own (HF) layout."""
import json
import os

import numpy as np
import pytest
import torch

from modeldir import synth_model, write_model_dir
from voxrt_amd import model as M


@pytest.fixture(scope="module")
def mdir(tmp_path_factory):
    layers, sp = synth_model()
    path = write_model_dir(str(tmp_path_factory.mktemp("model")), layers, sp)
    return path, layers, sp


def test_open_validate_and_tensors(mdir):
    path, layers, _ = mdir
    m = M.ModelFile(path)
    assert m.validate() == []
    dt, shape, q = m.tensor("encoder.layers.1.self_attn.o_proj.qweight")
    assert dt == "U8" and shape == (256, 52)
    np.testing.assert_array_equal(q, layers[1]["linears"]["o"][0])
    dt, shape, s = m.tensor("encoder.layers.0.feed_forward1.linear2.scales")
    assert dt == "F16" and shape == (256, 8)
    np.testing.assert_array_equal(np.asarray(s).view(np.uint16), layers[0]["linears"]["ff1_w2"][1])
    assert m.tensor_infos()["encoder.layers.0.conv.depthwise_conv.weight"] == ("F16", (256, 1, 9))
    with pytest.raises(M.FormatError, match="missing tensor"):
        m.tensor("encoder.layers.9.norm_out.weight")


def _rewrite(src, dst, edit_tensors=None, edit_ternary=None):
    from safetensors.numpy import load_file, save_file

    os.makedirs(dst, exist_ok=True)
    t = load_file(os.path.join(src, "model.safetensors"))
    if edit_tensors:
        edit_tensors(t)
    save_file(t, os.path.join(dst, "model.safetensors"))
    with open(os.path.join(src, "config.json")) as f:
        cfg = f.read()
    with open(os.path.join(dst, "config.json"), "w") as f:
        f.write(cfg)
    with open(os.path.join(src, "ternary.json")) as f:
        tj = json.load(f)
    if edit_ternary:
        edit_ternary(tj)
    with open(os.path.join(dst, "ternary.json"), "w") as f:
        json.dump(tj, f)
    return dst


def test_validate_reports_what_format_rs_reports(mdir, tmp_path):
    path = mdir[0]

    def edit(t):
        del t["encoder.layers.0.norm_out.bias"]
        t["encoder.layers.1.self_attn.bias_u"] = t["encoder.layers.1.self_attn.bias_u"].astype(np.float32)
        t["encoder.subsampling.linear.bias"] = np.zeros(7, np.float32)
        t["encoder.layers.0.self_attn.o_proj.weight"] = np.zeros((2, 2), np.float32)

    m = M.ModelFile(_rewrite(path, str(tmp_path / "bad"), edit))
    problems = m.validate()
    assert "missing encoder.layers.0.norm_out.bias" in problems
    assert "encoder.layers.1.self_attn.bias_u: got F32 [2, 128], expected F16 [2, 128]" in problems
    assert "encoder.subsampling.linear.bias: got F32 [7], expected F32 [256]" in problems
    assert "encoder.layers.0.self_attn.o_proj.weight present alongside qweight" == problems[-1]
    assert len(problems) == 4


def test_format_and_naming_are_checked(mdir, tmp_path):
    path = mdir[0]
    bad = _rewrite(path, str(tmp_path / "fmt"), edit_ternary=lambda tj: tj.update(format="thrush-ternary-v1"))
    with pytest.raises(M.FormatError, match="unsupported format"):
        M.ModelFile(bad)
    bad = _rewrite(path, str(tmp_path / "names"), edit_ternary=lambda tj: tj.update(names="nemo"))
    with pytest.raises(M.FormatError, match="unsupported tensor naming"):
        M.ModelFile(bad)
    # a header whose offsets do not match the tensor sizes
    broken = str(tmp_path / "hdr")
    _rewrite(path, broken)
    with open(os.path.join(broken, "model.safetensors"), "r+b") as f:
        n = int.from_bytes(f.read(8), "little")
        hdr = json.loads(f.read(n))
        name = "encoder.subsampling.linear.bias"
        hdr[name]["shape"] = [255]
        raw = json.dumps(hdr, separators=(",", ":")).encode().ljust(n)
        assert len(raw) == n
        f.seek(8)
        f.write(raw)
    with pytest.raises(M.FormatError, match="data offsets"):
        M.ModelFile(broken)


def test_layer_params_are_the_file_tensors(mdir):
    path, layers, _ = mdir
    m = M.ModelFile(path)
    for i, want in enumerate(layers):
        got = M.layer_params(m, i)
        for n, (q, s) in want["linears"].items():
            np.testing.assert_array_equal(got["linears"][n][0], q, err_msg=n)
            np.testing.assert_array_equal(got["linears"][n][1], s, err_msg=n)
        for n, (g, b) in want["norms"].items():
            np.testing.assert_array_equal(got["norms"][n][0], g)
            np.testing.assert_array_equal(got["norms"][n][1], b)
        for key in ("bias_u", "bias_v", "dw"):
            np.testing.assert_array_equal(got[key], want[key], err_msg=key)
        for key in ("gamma", "beta", "mean", "var"):
            np.testing.assert_array_equal(got["bn"][key], want["bn"][key])


def test_qkv_is_stacked_in_q_k_v_order(mdir):
    path = mdir[0]
    m = M.ModelFile(path)
    q, s = M.packed_linear(m, ["encoder.layers.0.self_attn.q_proj", "encoder.layers.0.self_attn.k_proj",
                               "encoder.layers.0.self_attn.v_proj"])
    for j, n in enumerate(("q_proj", "k_proj", "v_proj")):
        np.testing.assert_array_equal(q[j * 256:(j + 1) * 256], m.tensor(f"encoder.layers.0.self_attn.{n}.qweight")[2])
    with pytest.raises(M.FormatError, match="cannot stack"):
        M.packed_linear(m, ["encoder.layers.0.self_attn.q_proj", "encoder.layers.0.feed_forward1.linear2"])


def test_module_group_must_match_the_encoder_group(mdir, tmp_path):
    """Each linear's own group_size (ternary_linear.rs:70-76) is checked against the encoder's group before any
    scale table reaches the device: a module declaring 64-column groups is refused, whatever its tensors hold."""
    path = mdir[0]
    m = M.ModelFile(path)
    assert M.layer_params(m, 0, 128)["linears"]["o"][1].shape == (256, 2)

    def edit(tj):
        for mod in tj["quantized_modules"]:
            if mod["name"] == "encoder.layers.1.self_attn.o_proj":
                mod["group_size"] = 64

    bad = M.ModelFile(_rewrite(path, str(tmp_path / "grp"), edit_ternary=edit))
    M.layer_params(bad, 0, 128)
    with pytest.raises(M.FormatError, match="group_size 64 differs"):
        M.layer_params(bad, 1, 128)


def test_subsampling_params_against_torch_on_the_file_layout(mdir, orc):
    """The loader's subsampling (taps to [k*k, C], the final linear's columns to channels-last) through the oracle
    equals torch float64 on the file's own tensors: NCHW convolutions and the HF flatten order c*F + f."""
    path, _, sp_want = mdir
    m = M.ModelFile(path)
    sp = M.subsampling_params(m)
    for key in ("conv0_w", "conv0_b", "dw_w", "dw_b", "pw_w", "pw_b", "lin_w", "lin_b"):
        np.testing.assert_array_equal(sp[key], sp_want[key], err_msg=key)
    t, c, k = 57, 32, 3
    feats = np.random.default_rng(5).standard_normal((t, 32)).astype(np.float32)
    got = orc.subsampling(feats, sp)
    D = torch.float64
    w = {n: torch.from_numpy(m.load_f32(n).astype(np.float64)) for n in m.tensor_infos() if n.startswith("encoder.subsampling")}
    pre = "encoder.subsampling.layers"
    x = torch.from_numpy(feats.astype(np.float64))[None, None]
    x = torch.relu(torch.nn.functional.conv2d(x, w[f"{pre}.0.weight"], w[f"{pre}.0.bias"], stride=2, padding=1))
    for dwi, pwi in ((2, 3), (5, 6)):
        x = torch.nn.functional.conv2d(x, w[f"{pre}.{dwi}.weight"], w[f"{pre}.{dwi}.bias"], stride=2, padding=1,
                                       groups=c)
        x = torch.relu(torch.nn.functional.conv2d(x, w[f"{pre}.{pwi}.weight"], w[f"{pre}.{pwi}.bias"]))
    flat = x[0].permute(1, 0, 2).reshape(x.shape[2], -1)  # HF: [T3, C, F3] flattened c*F + f
    want = (flat @ w["encoder.subsampling.linear.weight"].T + w["encoder.subsampling.linear.bias"]).numpy()
    assert got.shape == want.shape
    assert np.abs(got - want).max() < 1e-4 * (1 + np.abs(want).max())
    assert w["encoder.subsampling.layers.0.weight"].dtype == D
