"""Model-directory loader for the GPU encoder: the thrush-ternary-v2 model format (crates/voxrt/src/format.rs) and the
load-time parameter transforms of the int8 encoder (tensor.rs:9-37, encoder.rs:108-134,546-574,677-692,
ternary_linear.rs:59-98, subsampling.rs:31-90), so real weights replace the synthetic ones once a model directory is
supplied.

A model directory holds config.json, ternary.json and model.safetensors. The safetensors file is memory-mapped and
its header parsed here (8-byte little-endian header length, a JSON header of name -> dtype, shape, data_offsets,
then the data); nothing in the file is executed. Ternary modules keep their packed form (qweight u8 [out, ceil(in/5)],
scales f16 [out, in/group]): the 2-bit repack happens on the device when the encoder uploads them.
"""
from __future__ import annotations

import json
import os

import numpy as np

FORMAT = "thrush-ternary-v2"  # format.rs:71

_DTYPES = {"U8": np.uint8, "I8": np.int8, "F16": np.float16, "F32": np.float32, "BF16": None, "I32": np.int32,
           "I64": np.int64, "F64": np.float64, "U16": np.uint16, "I16": np.int16, "U32": np.uint32, "BOOL": np.bool_}


class FormatError(ValueError):
    """A model directory that does not follow the format (format.rs's Error::Format)."""


class ModelFile:
    """ModelFile (format.rs:73-150): parsed config.json and ternary.json plus the memory-mapped safetensors file."""

    def __init__(self, directory: str):
        self.dir = directory
        with open(os.path.join(directory, "config.json")) as f:
            self.config = json.load(f)
        with open(os.path.join(directory, "ternary.json")) as f:
            self.ternary = json.load(f)
        if self.ternary.get("format") != FORMAT:
            raise FormatError(f"unsupported format {self.ternary.get('format')!r}, expected {FORMAT}")
        if self.ternary.get("names") != "hf":
            raise FormatError(f"unsupported tensor naming {self.ternary.get('names')!r}")
        path = os.path.join(directory, "model.safetensors")
        self._map = np.memmap(path, dtype=np.uint8, mode="r")
        if self._map.size < 8:
            raise FormatError("model.safetensors: truncated header")
        n = int(np.frombuffer(self._map[:8].tobytes(), "<u8")[0])
        if n <= 0 or 8 + n > self._map.size:
            raise FormatError("model.safetensors: bad header length")
        try:
            header = json.loads(self._map[8:8 + n].tobytes().decode("utf-8"))
        except (UnicodeDecodeError, ValueError) as e:
            raise FormatError(f"model.safetensors: header does not parse ({e})") from None
        header.pop("__metadata__", None)
        base = 8 + n
        self._infos = {}
        for name, v in header.items():
            dt, shape, (b0, b1) = v["dtype"], tuple(int(s) for s in v["shape"]), v["data_offsets"]
            if dt not in _DTYPES:
                raise FormatError(f"{name}: unknown dtype {dt}")
            size = int(np.prod(shape, dtype=np.int64)) if shape else 1
            width = 2 if dt == "BF16" else np.dtype(_DTYPES[dt]).itemsize
            if not (0 <= b0 <= b1 and base + b1 <= self._map.size and b1 - b0 == size * width):
                raise FormatError(f"{name}: data offsets do not match its dtype and shape")
            self._infos[name] = (dt, shape, base + b0, base + b1)

    def tensor_infos(self) -> dict:
        """name -> (dtype, shape) (format.rs:121-136)."""
        return {n: (v[0], v[1]) for n, v in sorted(self._infos.items())}

    def tensor(self, name: str):
        """(dtype, shape, array) of one tensor, the array a read-only view of the mapped file (format.rs:138-150)."""
        if name not in self._infos:
            raise FormatError(f"missing tensor {name}")
        dt, shape, b0, b1 = self._infos[name]
        raw = self._map[b0:b1]
        arr = raw if dt == "BF16" else raw.view(np.dtype(_DTYPES[dt]).newbyteorder("<"))
        return dt, shape, arr.reshape(shape) if dt != "BF16" else arr

    def load_f32(self, name: str, shape=None) -> np.ndarray:
        """load_f32 / load_f32_shaped (tensor.rs:9-37): an F32 or F16 tensor as float32, its shape checked."""
        dt, s, arr = self.tensor(name)
        if dt not in ("F32", "F16"):
            raise FormatError(f"{name}: cannot load {dt} as f32")
        if shape is not None and tuple(s) != tuple(shape):
            raise FormatError(f"{name}: shape {list(s)}, expected {list(shape)}")
        return np.asarray(arr, dtype=np.float32).reshape(s)

    def module(self, name: str) -> dict:
        for q in self.ternary.get("quantized_modules", []):
            if q["name"] == name:
                return q
        raise FormatError(f"{name} is not a ternary module")

    def validate(self) -> list:
        """Every expected tensor exists with the right dtype and shape; the list of problems (format.rs:153-305)."""
        infos = self.tensor_infos()
        problems, extra = [], []

        def expect(name, dtype, shape):
            i = infos.get(name)
            if i is None:
                problems.append(f"missing {name}")
            elif i[0] != dtype or list(i[1]) != list(shape):
                problems.append(f"{name}: got {i[0]} {list(i[1])}, expected {dtype} {list(shape)}")

        c = self.config
        e = c["encoder_config"]
        d, h = e["hidden_size"], c["decoder_hidden_size"]
        for m in self.ternary.get("quantized_modules", []):
            expect(f"{m['name']}.qweight", "U8", [m["out_features"], -(-m["in_features"] // 5)])
            expect(f"{m['name']}.scales", "F16", [m["out_features"], m["in_features"] // m["group_size"]])
            if m["has_bias"]:
                expect(f"{m['name']}.bias", "F32", [m["out_features"]])
            if f"{m['name']}.weight" in infos:
                extra.append(f"{m['name']}.weight present alongside qweight")
        ch, k = e["subsampling_conv_channels"], e["subsampling_conv_kernel_size"]
        for idx, shape in [(0, [ch, 1, k, k]), (2, [ch, 1, k, k]), (3, [ch, ch, 1, 1]), (5, [ch, 1, k, k]),
                           (6, [ch, ch, 1, 1])]:
            expect(f"encoder.subsampling.layers.{idx}.weight", "F16", shape)
            expect(f"encoder.subsampling.layers.{idx}.bias", "F32", [ch])
        sub_out = e["num_mel_bins"] // e["subsampling_factor"]
        expect("encoder.subsampling.linear.weight", "F16", [d, ch * sub_out])
        expect("encoder.subsampling.linear.bias", "F32", [d])
        heads = e["num_attention_heads"]
        for i in range(e["num_hidden_layers"]):
            p = f"encoder.layers.{i}"
            for n in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out",
                      "conv.norm"):
                expect(f"{p}.{n}.weight", "F32", [d])
                expect(f"{p}.{n}.bias", "F32", [d])
            expect(f"{p}.conv.norm.running_mean", "F32", [d])
            expect(f"{p}.conv.norm.running_var", "F32", [d])
            expect(f"{p}.conv.depthwise_conv.weight", "F16", [d, 1, e["conv_kernel_size"]])
            expect(f"{p}.self_attn.bias_u", "F16", [heads, d // heads])
            expect(f"{p}.self_attn.bias_v", "F16", [heads, d // heads])
        expect("encoder_projector.weight", "F16", [h, d])
        expect("encoder_projector.bias", "F32", [h])
        expect("decoder.embedding.weight", "F16", [c["vocab_size"], h])
        for layer in range(c["num_decoder_layers"]):
            expect(f"decoder.lstm.weight_ih_l{layer}", "F16", [4 * h, h])
            expect(f"decoder.lstm.weight_hh_l{layer}", "F16", [4 * h, h])
            expect(f"decoder.lstm.bias_ih_l{layer}", "F32", [4 * h])
            expect(f"decoder.lstm.bias_hh_l{layer}", "F32", [4 * h])
        expect("decoder.decoder_projector.weight", "F16", [h, h])
        expect("decoder.decoder_projector.bias", "F32", [h])
        nj = c["vocab_size"] + len(c["durations"])
        expect("joint.head.weight", "F16", [nj, h])
        expect("joint.head.bias", "F32", [nj])
        v = self.ternary["vad_head"]
        expect("vad_head.proj.weight", "F16", [v["hidden"], v["d_model"], 1])
        expect("vad_head.proj.bias", "F16", [v["hidden"]])
        expect("vad_head.ctx.weight", "F16", [v["hidden"], v["hidden"], v["kernel"]])
        expect("vad_head.ctx.bias", "F16", [v["hidden"]])
        expect("vad_head.out.weight", "F16", [1, v["hidden"], 1])
        expect("vad_head.out.bias", "F16", [1])
        return problems + extra


def packed_linear(m: ModelFile, names, group: int | None = None) -> tuple:
    """TernaryLinear::load / load_stacked (ternary_linear.rs:59-98): the packed rows and f16 scales of one module,
    or of several with the same input stacked along the output dimension (q | k | v), in the model file's own
    layout: (qweight uint8 [out, ceil(in/5)], scales as uint16 bits [out, in/group]). Each module's own group_size
    (ternary_linear.rs:70-76) is read from ternary.json; when `group` is given every module must use it (the GPU
    encoder holds one group for all its linears)."""
    qs, ss, inp = [], [], None
    for name in names:
        q = m.module(name)
        if group is not None and q["group_size"] != group:
            raise FormatError(f"{name}: group_size {q['group_size']} differs from the encoder's group {group}")
        if inp is not None and (q["in_features"] != inp or q["group_size"] != group):
            raise FormatError(f"{name}: cannot stack, shapes differ")
        if q["has_bias"]:
            raise FormatError(f"{name}: a bias on an encoder linear is not supported")
        inp, group = q["in_features"], q["group_size"]
        dq, sq, aq = m.tensor(f"{name}.qweight")
        ds, shs, asc = m.tensor(f"{name}.scales")
        if dq != "U8" or ds != "F16" or tuple(sq) != (q["out_features"], -(-inp // 5)) or \
                tuple(shs) != (q["out_features"], inp // group):
            raise FormatError(f"{name}: qweight / scales do not match ternary.json")
        qs.append(np.asarray(aq))
        ss.append(np.asarray(asc).view(np.uint16))
    return np.ascontiguousarray(np.concatenate(qs)), np.ascontiguousarray(np.concatenate(ss))


def layer_params(m: ModelFile, i: int, group: int | None = None) -> dict:
    """ConformerLayer::load (encoder.rs:677-692) with FeedForward / Attention / ConvModule::load
    (encoder.rs:70-76,108-134,546-574): the parameters of layer i in the form Encoder.set_layer takes (the BatchNorm
    fold into the depthwise taps happens at upload, as ConvModule::load does)."""
    e = m.config["encoder_config"]
    d, heads, k = e["hidden_size"], e["num_attention_heads"], e["conv_kernel_size"]
    p = f"encoder.layers.{i}"
    lin = {
        "ff1_w1": [f"{p}.feed_forward1.linear1"], "ff1_w2": [f"{p}.feed_forward1.linear2"],
        "qkv": [f"{p}.self_attn.q_proj", f"{p}.self_attn.k_proj", f"{p}.self_attn.v_proj"],
        "o": [f"{p}.self_attn.o_proj"], "pos": [f"{p}.self_attn.relative_k_proj"],
        "pw1": [f"{p}.conv.pointwise_conv1"], "pw2": [f"{p}.conv.pointwise_conv2"],
        "ff2_w1": [f"{p}.feed_forward2.linear1"], "ff2_w2": [f"{p}.feed_forward2.linear2"],
    }
    norms = {"ff1": "norm_feed_forward1", "attn": "norm_self_att", "conv": "norm_conv", "ff2": "norm_feed_forward2",
             "out": "norm_out"}
    return {
        "linears": {n: packed_linear(m, names, group) for n, names in lin.items()},
        "norms": {n: (m.load_f32(f"{p}.{v}.weight", [d]), m.load_f32(f"{p}.{v}.bias", [d])) for n, v in norms.items()},
        "bias_u": m.load_f32(f"{p}.self_attn.bias_u", [heads, d // heads]),
        "bias_v": m.load_f32(f"{p}.self_attn.bias_v", [heads, d // heads]),
        "dw": m.load_f32(f"{p}.conv.depthwise_conv.weight", [d, 1, k]).reshape(d, k),
        "bn": {"gamma": m.load_f32(f"{p}.conv.norm.weight", [d]), "beta": m.load_f32(f"{p}.conv.norm.bias", [d]),
               "mean": m.load_f32(f"{p}.conv.norm.running_mean", [d]),
               "var": m.load_f32(f"{p}.conv.norm.running_var", [d])},
    }


def subsampling_params(m: ModelFile) -> dict:
    """Subsampling::load (subsampling.rs:31-90): conv taps to [k*k, C], pointwise weights [out, in], the final
    linear's columns from the HF flatten order c*F + f to channels-last f*C + c."""
    e = m.config["encoder_config"]
    c, k, s = e["subsampling_conv_channels"], e["subsampling_conv_kernel_size"], e["subsampling_conv_stride"]
    f_out, d = e["num_mel_bins"] // e["subsampling_factor"], e["hidden_size"]
    pre = "encoder.subsampling.layers"

    def taps(name):
        return np.ascontiguousarray(m.load_f32(name, [c, 1, k, k]).reshape(c, k * k).T)

    lw = m.load_f32("encoder.subsampling.linear.weight", [d, c * f_out])
    lin_w = np.ascontiguousarray(lw.reshape(d, c, f_out).transpose(0, 2, 1).reshape(d, f_out * c))
    return {
        "k": k, "s": s,
        "conv0_w": taps(f"{pre}.0.weight"), "conv0_b": m.load_f32(f"{pre}.0.bias", [c]),
        "dw_w": np.stack([taps(f"{pre}.2.weight"), taps(f"{pre}.5.weight")]),
        "dw_b": np.stack([m.load_f32(f"{pre}.2.bias", [c]), m.load_f32(f"{pre}.5.bias", [c])]),
        "pw_w": np.stack([m.load_f32(f"{pre}.3.weight", [c, c, 1, 1]).reshape(c, c),
                          m.load_f32(f"{pre}.6.weight", [c, c, 1, 1]).reshape(c, c)]),
        "pw_b": np.stack([m.load_f32(f"{pre}.3.bias", [c]), m.load_f32(f"{pre}.6.bias", [c])]),
        "lin_w": lin_w, "lin_b": m.load_f32("encoder.subsampling.linear.bias", [d]),
    }


def load_encoder(m: ModelFile):
    """Encoder::load_with(Precision::Int8) (encoder.rs:791-800) onto the GPU: every layer and the subsampling
    uploaded through the C ABI (weights repacked on the device)."""
    from .encoder import Encoder

    e = m.config["encoder_config"]
    group = m.config["ternary_group_size"]
    enc = Encoder(d=e["hidden_size"], heads=e["num_attention_heads"], ff=e["intermediate_size"],
                  kconv=e["conv_kernel_size"], group=group, n_layers=e["num_hidden_layers"], n_mels=e["num_mel_bins"],
                  sub_channels=e["subsampling_conv_channels"], sub_kernel=e["subsampling_conv_kernel_size"],
                  sub_stride=e["subsampling_conv_stride"])
    try:
        for i in range(e["num_hidden_layers"]):
            enc.set_layer(i, layer_params(m, i, group))
        enc.set_subsampling(subsampling_params(m))
    except Exception:
        enc.free()
        raise
    return enc
