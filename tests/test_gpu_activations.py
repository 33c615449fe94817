"""The activation functions of the library (exp_poly, silu_fast, sigmoid_fast; tensor.rs:829-860) evaluated on the
device for every one of the 2^32 float inputs: each equals the IEEE form of the reference's formula bit for bit
(the division correctly rounded, the sign of zero kept; NaN for NaN). The SiLU/sigmoid epilogues of the GEMM, GLU
and conv kernels use these functions, and their parity tests compare them with the oracle on sampled inputs."""
import pytest

pytestmark = pytest.mark.gpu


def test_activations_equal_ieee_forms_on_all_inputs():
    import torch

    import voxrt_amd as vx

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    assert vx.detect() == vx.Kernel.Hip, "no gfx950 device"
    vx.kernels.check(vx.lib().vx_init(0))
    assert vx.kernels.check_activations() == (0, 0, 0)


def test_shutdown_drains_the_device():
    import voxrt_amd as vx

    vx.kernels.check(vx.lib().vx_init(0))
    vx.kernels.check(vx.lib().vx_shutdown())
