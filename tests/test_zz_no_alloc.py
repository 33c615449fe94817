"""vx_attention_core_noalloc (the attention core with the library's fixed workspace, for callers that cannot
allocate) against vx_attention_core with a caller workspace, through the C ABI: bit for bit on two calls in a row,
the second smaller, the first call's workspace contents still in the array; and sizes above the fixed array are
refused."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _x(seed, *shape, scale=1.0):
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)


def test_attention_without_workspace_equals_with_workspace():
    import torch

    import voxrt_amd as vx
    from voxrt_amd import kernels as K

    assert torch.cuda.is_available()
    K.check(vx.lib().vx_init(0))
    dev = torch.device("cuda:0")
    L = vx.lib()
    for t, heads in [(750, 8), (97, 8)]:  # the second call smaller than the first
        d = heads * 128
        qkv = torch.from_numpy(_x(600 + t, t, 3 * d)).to(dev)
        rel = torch.from_numpy(_x(601 + t, 2 * t - 1, d)).to(dev)
        bu = torch.from_numpy(_x(602, heads, 128, scale=0.3)).to(dev)
        bv = torch.from_numpy(_x(603, heads, 128, scale=0.3)).to(dev)
        scaling = float(np.float32(1.0) / np.sqrt(np.float32(128)))
        ws = torch.full((int(L.vx_attention_ws_bytes(t, d, heads)),), 0x5A, dtype=torch.uint8, device=dev)
        want = torch.full((t, d), float("nan"), dtype=torch.float32, device=dev)
        got = torch.full((t, d), float("nan"), dtype=torch.float32, device=dev)
        st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        K.check(L.vx_attention_core(C.c_void_p(qkv.data_ptr()), C.c_void_p(rel.data_ptr()), t, d, heads,
                                    C.c_void_p(bu.data_ptr()), C.c_void_p(bv.data_ptr()), scaling,
                                    C.c_void_p(ws.data_ptr()), C.c_void_p(want.data_ptr()), st))
        K.check(L.vx_attention_core_noalloc(C.c_void_p(qkv.data_ptr()), C.c_void_p(rel.data_ptr()), t, d, heads,
                                            C.c_void_p(bu.data_ptr()), C.c_void_p(bv.data_ptr()), scaling,
                                            C.c_void_p(got.data_ptr()), st))
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert not np.isnan(w).any()
        bad = np.flatnonzero(g.view(np.uint32) != w.view(np.uint32))
        assert bad.size == 0, f"t={t}: {bad.size} outputs differ"
    # above the fixed array: 16 heads at t = 1024 need about 12.8 MiB
    st = L.vx_attention_core_noalloc(C.c_void_p(8), C.c_void_p(8), 1024, 2048, 16, C.c_void_p(8), C.c_void_p(8),
                                     0.1, C.c_void_p(8), None)
    assert st == K.VX_ERR_INVALID and b"above the fixed" in L.vx_last_error()
