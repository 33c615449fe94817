"""voxrt_amd — the MI355X (gfx950) ternary x int8 GEMM path of voxrt behind a C ABI (include/voxrt_hip.h)."""
from .kernels import (EP_ADD_SCALED, EP_SILU, EP_STORE, Epilogue, HipError, Kernel, QuantAct, TernaryMatrix,
                      detect, gemm, gemm_ep, gemm_ep_quantize, gemm_rows_range, gemm_single, kernel, lib)

__all__ = ["Epilogue", "HipError", "Kernel", "QuantAct", "TernaryMatrix", "detect", "gemm", "gemm_ep",
           "gemm_ep_quantize", "gemm_rows_range", "gemm_single", "kernel", "lib", "EP_STORE", "EP_SILU", "EP_ADD_SCALED"]
