"""An independent float64 statement of the FastConformer encoder: Hugging Face transformers' own Parakeet encoder
(``transformers.models.parakeet.modeling_parakeet``, installed in the image; not the reference's code) built with
the synthetic parameters the oracle and the GPU encoder run on.

The reference's int8 encoder restates that model (its golden vectors were dumped from it,
reference-py/dump_golden.py:19-79), so it fixes what a restatement could misread and a second restatement would
repeat: which LayerNorm feeds which sublayer, the 0.5 / 1.0 residual scales, the q|k|v split, the relative-position
shift and its sign, the GLU halves, the BatchNorm and the order of the sublayers. It runs in float64 with the
dequantized ternary weights (trit * f16 scale); the int8 path differs from it only by its activation quantization.

The model's parameters map as the model file stores them (format.rs, HF names; the same layouts as
tests/modeldir.py writes): q|k|v rows split into q_proj / k_proj / v_proj, pointwise convolutions as [out, in, 1],
the depthwise taps [d, 1, k] with the raw BatchNorm statistics (HF folds nothing), subsampling convolutions in NCHW
and the final linear's columns channel-major (c * F + f).
"""
from __future__ import annotations

import numpy as np
import torch
from transformers.initialization import no_init_weights
from transformers.models.parakeet.configuration_parakeet import ParakeetEncoderConfig
from transformers.models.parakeet.modeling_parakeet import ParakeetEncoder, ParakeetEncoderRelPositionalEncoding

from voxrt_amd import synth


def _dequant(q, s16, out, inp, group=128):
    trits = synth.unpack_rows(np.asarray(q, np.uint8), inp).astype(np.float64)
    scales = np.asarray(s16, np.uint16).view(np.float16).astype(np.float64)
    return trits * np.repeat(scales, group, axis=1)[:, :inp]


def config(d=1024, heads=8, ff=4096, kconv=9, n_layers=1, n_mels=128, c=256):
    return ParakeetEncoderConfig(hidden_size=d, num_hidden_layers=n_layers, num_attention_heads=heads,
                                 intermediate_size=ff, hidden_act="silu", attention_bias=False,
                                 convolution_bias=False, conv_kernel_size=kconv, subsampling_factor=8,
                                 subsampling_conv_channels=c, num_mel_bins=n_mels, subsampling_conv_kernel_size=3,
                                 subsampling_conv_stride=2, dropout=0.0, dropout_positions=0.0, layerdrop=0.0,
                                 activation_dropout=0.0, attention_dropout=0.0, scale_input=False)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float64))


def load_layer(block, p, d, ff, group=128):
    """Copies one synthetic layer (synth.synth_layer's dict) into an HF ParakeetEncoderBlock."""
    L = p["linears"]
    sd = {
        "feed_forward1.linear1.weight": _dequant(*L["ff1_w1"], ff, d, group),
        "feed_forward1.linear2.weight": _dequant(*L["ff1_w2"], d, ff, group),
        "self_attn.o_proj.weight": _dequant(*L["o"], d, d, group),
        "self_attn.relative_k_proj.weight": _dequant(*L["pos"], d, d, group),
        "conv.pointwise_conv1.weight": _dequant(*L["pw1"], 2 * d, d, group)[:, :, None],
        "conv.pointwise_conv2.weight": _dequant(*L["pw2"], d, d, group)[:, :, None],
        "feed_forward2.linear1.weight": _dequant(*L["ff2_w1"], ff, d, group),
        "feed_forward2.linear2.weight": _dequant(*L["ff2_w2"], d, ff, group),
        "self_attn.bias_u": p["bias_u"], "self_attn.bias_v": p["bias_v"],
        "conv.depthwise_conv.weight": np.asarray(p["dw"])[:, None, :],
        "conv.norm.weight": p["bn"]["gamma"], "conv.norm.bias": p["bn"]["beta"],
        "conv.norm.running_mean": p["bn"]["mean"], "conv.norm.running_var": p["bn"]["var"],
    }
    qkv = _dequant(*L["qkv"], 3 * d, d, group)
    for j, n in enumerate(("q_proj", "k_proj", "v_proj")):
        sd[f"self_attn.{n}.weight"] = qkv[j * d:(j + 1) * d]
    for key, n in (("ff1", "norm_feed_forward1"), ("attn", "norm_self_att"), ("conv", "norm_conv"),
                   ("ff2", "norm_feed_forward2"), ("out", "norm_out")):
        sd[f"{n}.weight"], sd[f"{n}.bias"] = p["norms"][key]
    own = block.state_dict()
    missing = [k for k in own if k not in sd and not k.endswith("num_batches_tracked")]
    assert not missing, f"unmapped HF parameters: {missing}"
    block.load_state_dict({k: _t(v) for k, v in sd.items()}, strict=False)


def load_subsampling(sub, sp, d, n_mels, c):
    """Copies the synthetic subsampling weights (channels-last layouts of subsampling.rs) into HF's Conv2D stack."""
    k = sp["k"]
    f_out = n_mels
    for _ in range(3):
        f_out = (f_out - 1) // 2 + 1

    def conv(w):  # [k*k, C] -> [C, 1, k, k]
        return np.asarray(w).T.reshape(c, 1, k, k)

    sd = {"layers.0.weight": conv(sp["conv0_w"]), "layers.0.bias": sp["conv0_b"]}
    for st, (dwi, pwi) in enumerate(((2, 3), (5, 6))):
        sd[f"layers.{dwi}.weight"], sd[f"layers.{dwi}.bias"] = conv(sp["dw_w"][st]), sp["dw_b"][st]
        sd[f"layers.{pwi}.weight"] = np.asarray(sp["pw_w"][st]).reshape(c, c, 1, 1)
        sd[f"layers.{pwi}.bias"] = sp["pw_b"][st]
    sd["linear.weight"] = np.asarray(sp["lin_w"]).reshape(d, f_out, c).transpose(0, 2, 1).reshape(d, c * f_out)
    sd["linear.bias"] = sp["lin_b"]
    sub.load_state_dict({kk: _t(v) for kk, v in sd.items()}, strict=True)


def encoder(layers, sp=None, d=1024, heads=8, ff=4096, kconv=9, n_mels=128, c=256):
    """An HF ParakeetEncoder in float64, eval mode, holding the given synthetic layers (and subsampling)."""
    with no_init_weights():  # every parameter is overwritten below
        enc = ParakeetEncoder(config(d, heads, ff, kconv, len(layers), n_mels, c))
    enc = enc.double().eval()
    for blk, p in zip(enc.layers, layers):
        load_layer(blk, p, d, ff)
    if sp is not None:
        load_subsampling(enc.subsampling, sp, d, n_mels, c)
    return enc


def pos_emb(enc, t):
    """HF's relative position table for t frames ([2t-1, d], positions t-1 .. -(t-1), sin/cos interleaved)."""
    return enc.encode_positions(torch.zeros((1, t, enc.config.hidden_size), dtype=torch.float64))


@torch.no_grad()
def layers_forward(enc, x, upto=None):
    """The layer stack on x [t, d] (no subsampling): the output after `upto` layers (all by default)."""
    h = _t(x)[None]
    pe = pos_emb(enc, h.shape[1])
    for blk in enc.layers[:upto]:
        h = blk(h, attention_mask=None, position_embeddings=pe)
    return h[0].numpy()


@torch.no_grad()
def forward_feats(enc, feats):
    """Subsampling + layers from log-mel features [t_in, n_mels]."""
    return enc(input_features=_t(feats)[None]).last_hidden_state[0].numpy()


@torch.no_grad()
def layer_outputs(enc, feats):
    """Subsampling + layers from features, every layer's output in order ([t, d] each)."""
    h = enc.subsampling(_t(feats)[None])
    pe = pos_emb(enc, h.shape[1])
    outs = []
    for blk in enc.layers:
        h = blk(h, attention_mask=None, position_embeddings=pe)
        outs.append(h[0].numpy())
    return outs


@torch.no_grad()
def subsample(enc, feats):
    return enc.subsampling(_t(feats)[None])[0].numpy()


def rel_pos_table(t, d=1024):
    """HF's table in its own float32 arithmetic ([2t-1, d])."""
    m = ParakeetEncoderRelPositionalEncoding(config(d=d))
    return m(torch.zeros((1, t, d), dtype=torch.float32))[0].numpy()
