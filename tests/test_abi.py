"""The C-ABI library loads and exports every entry point of include/voxrt_hip.h; host-side argument checks fail
with the documented status and message (no GPU work: these run on a CPU-only host)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import voxrt_amd as vx
from voxrt_amd import kernels

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(vx_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    names = _declared_symbols()
    assert {"vx_gemm_ep", "vx_gemm_rows_range", "vx_quantize", "vx_tmat_upload_packed"} <= names
    L = vx.lib()
    for n in sorted(names):
        assert hasattr(L, n), f"{n} declared in include/ but not exported"


def test_detect_without_device_reports_scalar():
    if os.environ.get("HIP_VISIBLE_DEVICES", None) == "" or not vx.lib().vx_detect():
        assert vx.detect() == vx.Kernel.Scalar


def test_upload_rejects_bad_shapes():
    q = np.zeros((4, (128 + 4) // 5), np.uint8)
    s = np.zeros((4, 4), np.uint16)
    with pytest.raises(vx.HipError) as e:
        vx.TernaryMatrix.from_packed(q, s, 4, 128, 32)  # group not a multiple of 64
    assert e.value.status == kernels.VX_ERR_INVALID and "group" in str(e.value)
    h = C.c_void_p()
    st = vx.lib().vx_tmat_upload_packed(None, None, 4, 128, 128, C.byref(h))
    assert st == kernels.VX_ERR_INVALID and b"NULL" in vx.lib().vx_last_error()
    st = vx.lib().vx_tmat_upload_i8(None, None, 4, 100, 50, C.byref(h))
    assert st == kernels.VX_ERR_INVALID


def test_gemm_rejects_null_arguments():
    st = vx.lib().vx_gemm_ep(None, None, None, None, 1, None, None, 0, 0.0, None, None)
    assert st == kernels.VX_ERR_INVALID and b"NULL" in vx.lib().vx_last_error()
    st = vx.lib().vx_quantize(None, 1, 128, 128, None, None, None, None)
    assert st == kernels.VX_ERR_INVALID


def test_last_error_is_cleared_by_success():
    assert vx.lib().vx_tmat_info(None, None, None, None, None) == kernels.VX_ERR_INVALID
    assert vx.lib().vx_last_error() != b""
    # a successful call (an empty quantize is a no-op) clears it
    assert vx.lib().vx_quantize(C.c_void_p(8), 0, 128, 128, C.c_void_p(8), C.c_void_p(8), C.c_void_p(8), None) == 0
    assert vx.lib().vx_last_error() == b""


def test_epilogue_values_match_header():
    hdr = open(os.path.join(ROOT, "include", "voxrt_hip.h")).read()
    assert "VX_EP_STORE = 0" in hdr and "VX_EP_SILU = 1" in hdr and "VX_EP_ADD_SCALED = 2" in hdr
    assert vx.Epilogue.Store.kind == 0 and vx.Epilogue.Silu.kind == 1 and vx.Epilogue.AddScaled(0.5).kind == 2


def test_zero_tokens_take_null_pointers():
    """n = 0 / t = 0 is a no-op that returns VX_OK with NULL data pointers and touches no device (as the
    reference's kernels loop over zero tokens); with one token the same NULL pointers are refused."""
    L = vx.lib()
    assert L.vx_quantize(None, 0, 128, 128, None, None, None, None) == 0
    assert L.vx_quantize_normed(None, 0, 128, 128, None, None, None, None, None, None) == 0
    assert L.vx_layer_norm(None, 0, 1024, None, None, None, None) == 0
    assert L.vx_linear_f32(None, 0, 64, None, None, 32, None, 0, None) == 0
    assert L.vx_glu_dwconv_silu(None, 0, 256, 9, None, None, None, None) == 0
    assert L.vx_quantize(None, 1, 128, 128, None, None, None, None) == kernels.VX_ERR_INVALID
    assert L.vx_layer_norm(None, 1, 1024, None, None, None, None) == kernels.VX_ERR_INVALID


def test_encoder_parameters_are_checked_on_the_host():
    """Encoder.set_layer / set_subsampling compare every host array with the shape the configuration implies
    before the C side copies that many bytes (a short array would be over-read)."""
    from voxrt_amd import encoder as E
    from voxrt_amd import synth

    p = synth.synth_layer(0, d=256, ff=512, heads=2)
    enc = E.Encoder(d=256, heads=2, ff=512, n_layers=1, n_mels=32, sub_channels=16)
    try:
        for name, edit, msg in [
            ("o", lambda q: (q[0][:-1], q[1]), "o qweight"),
            ("ff1_w2", lambda q: (q[0], q[1][:, :-1]), "ff1_w2 scales"),
        ]:
            bad = dict(p, linears=dict(p["linears"]))
            bad["linears"][name] = edit(p["linears"][name])
            with pytest.raises(ValueError, match=msg):
                enc.set_layer(0, bad)
        with pytest.raises(ValueError, match="bias_u"):
            enc.set_layer(0, dict(p, bias_u=p["bias_u"][:1]))
        with pytest.raises(ValueError, match="dw"):
            enc.set_layer(0, dict(p, dw=p["dw"][:, :8]))
        sp = synth.synth_subsampling(d=256, c=16, n_mels=32)
        with pytest.raises(ValueError, match="lin_w"):
            enc.set_subsampling(dict(sp, lin_w=sp["lin_w"][:, :-1]))
    finally:
        enc.free()


def test_kernel_override_is_explicit_and_checked():
    """Kernel choices are forced only through vx_set_kernel_override (the library reads no environment variable):
    known names and values are taken and cleared, anything else is refused with VX_ERR_INVALID."""
    import subprocess

    L = vx.lib()
    for name, value in [("gemm", b"stream"), ("gemm", b"small"), ("tile", b"2x4"), ("small_tile", b"1x8"),
                        ("stream_grid", b"16"), ("small_ws", b"on"), ("small_ws", b"off"), ("linear", b"lds"),
                        ("linear", b"mfma2x2"), ("stream_tile", b"4")]:
        assert L.vx_set_kernel_override(name.encode(), value) == 0
        assert L.vx_set_kernel_override(name.encode(), None) == 0
    for name, value in [(b"gemm", b"fastest"), (b"tile", b"2by4"), (b"stream_grid", b"12"), (b"grid", b"8"),
                        (b"small_ws", b"yes"), (b"linear", b"3"),
                        (b"stream_tile", b"6")]:
        assert L.vx_set_kernel_override(name, value) == kernels.VX_ERR_INVALID
    with kernels.kernel_override(gemm="direct", tile="1x2"):
        pass
    so = os.path.join(ROOT, "voxrt_amd", "libvoxrt_hip.so")
    strings = subprocess.run(["strings", so], capture_output=True, text=True).stdout
    assert "VX_GEMM" not in strings and "VX_STREAM_GRID" not in strings and "VX_SMALL_TILE" not in strings


def test_trit_upload_refuses_non_trits():
    """vx_tmat_upload_trits checks every value on the host before any device work: a 2 is refused."""
    rows = np.zeros((4, 128), np.int8)
    rows[2, 77] = 2
    scales = np.ones((4, 1), np.float32)
    h = C.c_void_p()
    st = vx.lib().vx_tmat_upload_trits(rows.ctypes.data, scales.ctypes.data, 4, 128, 128, C.byref(h))
    assert st == kernels.VX_ERR_INVALID and b"-1, 0 or +1 (row 2)" in vx.lib().vx_last_error()


def _c_params(text):
    """{function: parameter count} of the vx_ functions a C header declares."""
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(vx_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_rust_bindings_declare_every_entry_point_with_its_arity():
    """The Rust -sys crate (voxrt_amd/rust/voxrt-hip-sys/src/lib.rs, not compiled here: no cargo) declares every
    function of include/voxrt_hip.h with the same number of parameters, and the Rust build script compiles exactly
    the sources the Python build compiles."""
    hdr = _c_params(open(os.path.join(ROOT, "include", "voxrt_hip.h")).read())
    rs = open(os.path.join(ROOT, "voxrt_amd", "rust", "voxrt-hip-sys", "src", "lib.rs")).read()
    decl = {}
    for m in re.finditer(r"pub fn (vx_[a-z0-9_]+)\s*\((.*?)\)\s*(->[^;]*)?;", rs, flags=re.S):
        args = re.sub(r"//[^\n]*", "", m.group(2)).strip().rstrip(",")
        decl[m.group(1)] = 0 if not args else args.count(",") + 1
    missing = sorted(set(hdr) - set(decl) - {"vx_npad"})
    optional = {"vx_fold_bn", "vx_glu_dwconv_silu", "vx_glu_dwconv_silu_quantize", "vx_layer_norm", "vx_linear_f32",
                "vx_subsampling", "vx_subsampling_scratch_floats", "vx_rel_pos_table", "vx_check_activations",
                "vx_attention_ws_bytes", "vx_attention_core", "vx_attention_core_quantize",
                "vx_attention_core_noalloc"}
    assert not [n for n in missing if n not in optional], missing
    for name, n in decl.items():
        assert name in hdr, f"{name} is not in the header"
        assert hdr[name] == n, f"{name}: {n} parameters in Rust, {hdr[name]} in C"
    build_rs = open(os.path.join(ROOT, "voxrt_amd", "rust", "voxrt-hip-sys", "build.rs")).read()
    from voxrt_amd import build as B

    assert sorted(re.findall(r'"(vx_[a-z_]+\.hip)"', build_rs)) == sorted(B.SOURCES)
    for flag in ("-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero", "-packed-fp32-ops", "--offload-arch="):
        assert flag in build_rs
