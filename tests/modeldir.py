"""Writes a small synthetic model directory in the thrush-ternary-v2 format (config.json, ternary.json and
model.safetensors with the reference's HF tensor names, dtypes and shapes, format.rs:153-305) from the synthetic
encoder parameters, so the model-file loader can be tested without real weights. The file is written by the
safetensors package, independently of the loader's own header parser."""
import json
import os

import numpy as np
from safetensors.numpy import save_file

from voxrt_amd import synth


def round_f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def synth_model(d=256, heads=2, ff=1024, kconv=9, group=128, n_layers=2, n_mels=32, c=32):
    """The encoder parameters (layer dicts as Encoder.set_layer takes them, the subsampling dict) with every tensor
    the file stores as F16 already rounded to f16, so loading it gives these values back exactly."""
    layers = []
    for i in range(n_layers):
        p = synth.synth_layer(i, d=d, ff=ff, heads=heads, kconv=kconv, group=group)
        p["bias_u"], p["bias_v"], p["dw"] = round_f16(p["bias_u"]), round_f16(p["bias_v"]), round_f16(p["dw"])
        layers.append(p)
    sp = synth.synth_subsampling(d=d, c=c, n_mels=n_mels)
    for key in ("conv0_w", "dw_w", "pw_w", "lin_w"):
        sp[key] = round_f16(sp[key])
    return layers, sp


def write_model_dir(path, layers, sp, d=256, heads=2, ff=1024, kconv=9, group=128, n_mels=32, c=32):
    os.makedirs(path, exist_ok=True)
    n_layers, k = len(layers), sp["k"]
    f_out = n_mels // 8
    h, vocab, durations = 64, 10, [0, 1, 2, 3, 4]
    config = {"encoder_config": {"hidden_size": d, "intermediate_size": ff, "num_hidden_layers": n_layers,
                                 "num_attention_heads": heads, "num_mel_bins": n_mels, "conv_kernel_size": kconv,
                                 "subsampling_conv_channels": c, "subsampling_conv_kernel_size": k,
                                 "subsampling_conv_stride": sp["s"], "subsampling_factor": 8,
                                 "max_position_embeddings": 5000, "scale_input": False},
              "blank_token_id": vocab - 1, "decoder_hidden_size": h, "num_decoder_layers": 1, "durations": durations,
              "max_symbols_per_step": 10, "vocab_size": vocab, "ternary_group_size": group, "ternary_modules": []}
    t = {}
    modules = []
    f16, f32 = np.float16, np.float32

    def ternary(name, q, s16, out, inp):
        t[f"{name}.qweight"] = np.ascontiguousarray(q, np.uint8)
        t[f"{name}.scales"] = np.ascontiguousarray(np.asarray(s16, np.uint16).view(f16))
        modules.append({"name": name, "out_features": out, "in_features": inp, "group_size": group,
                        "as_conv1d": "pointwise" in name, "has_bias": False, "zero_fraction": 0.4})

    for i, p in enumerate(layers):
        pre = f"encoder.layers.{i}"
        L = p["linears"]
        ternary(f"{pre}.feed_forward1.linear1", *L["ff1_w1"], ff, d)
        ternary(f"{pre}.feed_forward1.linear2", *L["ff1_w2"], d, ff)
        q, s = L["qkv"]
        for j, n in enumerate(("q_proj", "k_proj", "v_proj")):
            ternary(f"{pre}.self_attn.{n}", q[j * d:(j + 1) * d], s[j * d:(j + 1) * d], d, d)
        ternary(f"{pre}.self_attn.o_proj", *L["o"], d, d)
        ternary(f"{pre}.self_attn.relative_k_proj", *L["pos"], d, d)
        ternary(f"{pre}.conv.pointwise_conv1", *L["pw1"], 2 * d, d)
        ternary(f"{pre}.conv.pointwise_conv2", *L["pw2"], d, d)
        ternary(f"{pre}.feed_forward2.linear1", *L["ff2_w1"], ff, d)
        ternary(f"{pre}.feed_forward2.linear2", *L["ff2_w2"], d, ff)
        for key, n in (("ff1", "norm_feed_forward1"), ("attn", "norm_self_att"), ("conv", "norm_conv"),
                       ("ff2", "norm_feed_forward2"), ("out", "norm_out")):
            g, b = p["norms"][key]
            t[f"{pre}.{n}.weight"], t[f"{pre}.{n}.bias"] = np.asarray(g, f32), np.asarray(b, f32)
        bn = p["bn"]
        t[f"{pre}.conv.norm.weight"], t[f"{pre}.conv.norm.bias"] = bn["gamma"].astype(f32), bn["beta"].astype(f32)
        t[f"{pre}.conv.norm.running_mean"], t[f"{pre}.conv.norm.running_var"] = bn["mean"].astype(f32), bn["var"].astype(f32)
        t[f"{pre}.conv.depthwise_conv.weight"] = p["dw"].reshape(d, 1, kconv).astype(f16)
        t[f"{pre}.self_attn.bias_u"] = p["bias_u"].astype(f16)
        t[f"{pre}.self_attn.bias_v"] = p["bias_v"].astype(f16)
    # subsampling in the HF layout: conv taps [C, 1, k, k], pointwise [C, C, 1, 1], linear columns c*F + f
    sub = "encoder.subsampling.layers"

    def conv(w):  # [k*k, C] -> [C, 1, k, k]
        return np.ascontiguousarray(w.T.reshape(c, 1, k, k)).astype(f16)

    t[f"{sub}.0.weight"], t[f"{sub}.0.bias"] = conv(sp["conv0_w"]), sp["conv0_b"].astype(f32)
    for st, (dwi, pwi) in enumerate(((2, 3), (5, 6))):
        t[f"{sub}.{dwi}.weight"], t[f"{sub}.{dwi}.bias"] = conv(sp["dw_w"][st]), sp["dw_b"][st].astype(f32)
        t[f"{sub}.{pwi}.weight"] = sp["pw_w"][st].reshape(c, c, 1, 1).astype(f16)
        t[f"{sub}.{pwi}.bias"] = sp["pw_b"][st].astype(f32)
    lw = sp["lin_w"].reshape(d, f_out, c).transpose(0, 2, 1).reshape(d, c * f_out)
    t["encoder.subsampling.linear.weight"] = np.ascontiguousarray(lw).astype(f16)
    t["encoder.subsampling.linear.bias"] = sp["lin_b"].astype(f32)
    # the rest of the file (decoder, joint, VAD head): zeros of the right shapes
    nj = vocab + len(durations)
    for name, dt, shape in [("encoder_projector.weight", f16, (h, d)), ("encoder_projector.bias", f32, (h,)),
                            ("decoder.embedding.weight", f16, (vocab, h)),
                            ("decoder.lstm.weight_ih_l0", f16, (4 * h, h)), ("decoder.lstm.weight_hh_l0", f16, (4 * h, h)),
                            ("decoder.lstm.bias_ih_l0", f32, (4 * h,)), ("decoder.lstm.bias_hh_l0", f32, (4 * h,)),
                            ("decoder.decoder_projector.weight", f16, (h, h)),
                            ("decoder.decoder_projector.bias", f32, (h,)), ("joint.head.weight", f16, (nj, h)),
                            ("joint.head.bias", f32, (nj,)), ("vad_head.proj.weight", f16, (8, d, 1)),
                            ("vad_head.proj.bias", f16, (8,)), ("vad_head.ctx.weight", f16, (8, 8, 5)),
                            ("vad_head.ctx.bias", f16, (8,)), ("vad_head.out.weight", f16, (1, 8, 1)),
                            ("vad_head.out.bias", f16, (1,))]:
        t[name] = np.zeros(shape, dt)
    ternary_json = {"format": "thrush-ternary-v2", "names": "hf", "quant": {"mode": "ternary", "group_size": group},
                    "vad_head": {"d_model": d, "hidden": 8, "kernel": 5, "frame_seconds": 0.08},
                    "quantized_modules": modules, "n_quantized_params": 0, "n_dense_params": 0}
    config["ternary_modules"] = [m["name"] for m in modules]
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(config, f)
    with open(os.path.join(path, "ternary.json"), "w") as f:
        json.dump(ternary_json, f)
    save_file(t, os.path.join(path, "model.safetensors"))
    return path
