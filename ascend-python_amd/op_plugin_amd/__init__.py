"""op_plugin_amd -- MI355X (gfx950) quantized-inference ops behind the torch_npu op names.

Importing this package loads ``_npu_ops.so``, which registers

* ``torch.ops.npu.npu_dynamic_quant(input, *, smooth_scales=None) -> (int8 y, fp32 scale)``
* ``torch.ops.npu.npu_quant_matmul(x1, x2, scale, *, offset=None, pertoken_scale=None,
  bias=None, output_dtype=None) -> Tensor``  (W8A8)
* ``torch.ops.npu.npu_weight_quant_batchmatmul(x, weight, antiquant_scale,
  antiquant_offset=None, quant_scale=None, quant_offset=None, bias=None,
  antiquant_group_size=0) -> Tensor``  (W4A16 / W8A16)
* ``torch.ops.npu.npu_convert_weight_to_int4pack(weight, inner_k_tiles=0) -> Tensor``
  (``inner_k_tiles=4``: straight to the NZ layout)
* ``torch.ops.npu.npu_format_cast(self, acl_format) -> Tensor``: an int4-packed or int8 weight between ND (2)
  and FRACTAL_NZ (29), the MFMA-tiled layouts ``npu_weight_quant_batchmatmul`` streams fastest
* ``torch.ops.npu.quantize_per_tensor(self, scale, zero_point, dtype)``,
  ``torch.ops.npu.quantize_per_channel(self, scales, zero_points, axis, dtype)`` and
  ``torch.ops.npu.dequantize(self)``: the reference's static quantization ops (plain int8 / uint8 / int32
  results for torch.qint8 / quint8 / qint32; dequantize is their cast to float32)
* ``torch.ops.npu.npu_rms_norm(self, gamma, epsilon=1e-6) -> (y, fp32 rstd)``
* ``torch.ops.npu.npu_swiglu(self, dim=-1) -> Tensor``
* ``torch.ops.npu.npu_rms_norm_dynamic_quant(self, gamma, epsilon=1e-6) -> (int8 q, fp32 scale, fp32 rstd)``
  and ``torch.ops.npu.npu_swiglu_dynamic_quant(self, dim=-1) -> (int8 q, fp32 scale)``: RMSNorm / SwiGLU
  fused with npu_dynamic_quant of their 16-bit output (bit-identical to the unfused chain)
* ``torch.ops.npu.npu_quant_matmul_swiglu(x1, x2, scale, *, pertoken_scale=None, output_dtype=None) -> h``: the
  quantized MLP block's gate-up projection with the SwiGLU in the GEMM's epilogue, h =
  npu_swiglu(npu_quant_matmul(x1, x2, scale, pertoken_scale=..., output_dtype=...)) bit for bit (x2 [K, 2I] or
  its int8 NZ cast; no bias)
* ``torch.ops.npu.npu_quant_matmul_swiglu_quant(x1, x2, scale, *, pertoken_scale=None, output_dtype=None) -> (q,
  scale)``: the same followed by npu_dynamic_quant of h, bit for bit; the GEMM's epilogue stores each row's
  partial absmax, so the quantizer reads h once with no row reduction

and exposes the same callables here, so code written as
``torch_npu.npu_quant_matmul(...)`` runs as ``op_plugin_amd.npu_quant_matmul(...)``
(the reference tests call ops this way, e.g.
test/test_custom_ops/test_npu_rms_norm.py:20).  The kernels are the HIP code of
``libqk_hip.so``; there is no fallback: if the native library is missing, the
import fails.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqk_hip.so")
OPS_PATH = os.path.join(_HERE, "_npu_ops.so")

if not (os.path.exists(LIB_PATH) and os.path.exists(OPS_PATH)):
    raise ImportError(
        "op_plugin_amd: native libraries are not built (expected "
        f"{LIB_PATH} and {OPS_PATH}); run `python ascend-python_amd/build.py` or "
        "`__graft_entry__.build()` first")

if not hasattr(torch.ops.npu, "npu_quant_matmul"):
    torch.ops.load_library(OPS_PATH)

npu_dynamic_quant = torch.ops.npu.npu_dynamic_quant
npu_quant_matmul = torch.ops.npu.npu_quant_matmul
npu_weight_quant_batchmatmul = torch.ops.npu.npu_weight_quant_batchmatmul
npu_convert_weight_to_int4pack = torch.ops.npu.npu_convert_weight_to_int4pack
npu_format_cast = torch.ops.npu.npu_format_cast
quantize_per_tensor = torch.ops.npu.quantize_per_tensor
quantize_per_channel = torch.ops.npu.quantize_per_channel
dequantize = torch.ops.npu.dequantize
npu_rms_norm = torch.ops.npu.npu_rms_norm
npu_swiglu = torch.ops.npu.npu_swiglu
npu_rms_norm_dynamic_quant = torch.ops.npu.npu_rms_norm_dynamic_quant
npu_swiglu_dynamic_quant = torch.ops.npu.npu_swiglu_dynamic_quant
npu_quant_matmul_swiglu = torch.ops.npu.npu_quant_matmul_swiglu
npu_quant_matmul_swiglu_quant = torch.ops.npu.npu_quant_matmul_swiglu_quant

# qk_abi.h constants
QK_F16, QK_BF16, QK_F32, QK_I8, QK_I32, QK_U8, QK_I4_NZ, QK_I8_NZ, QK_I8_NK = 1, 2, 3, 4, 5, 6, 16, 17, 18
ACL_FORMAT_ND, ACL_FORMAT_FRACTAL_NZ = 2, 29
QK_OK, QK_ERR_ARG, QK_ERR_UNSUPPORTED, QK_ERR_WORKSPACE, QK_ERR_LAUNCH = 0, -1, -2, -3, -4
QK_NOALLOC_SCRATCH_BYTES = 16 << 20

ABI_SYMBOLS = (
    "qk_last_error", "qk_abi_version", "qk_debug_set_plan", "qk_dynamic_quant", "qk_quant_matmul_workspace_size",
    "qk_quant_matmul", "qk_quant_matmul_nz_workspace_size", "qk_quant_matmul_nz", "qk_weight_quant_bmm_workspace_size",
    "qk_weight_quant_bmm", "qk_weight_quant_bmm_noalloc", "qk_int4_pack", "qk_weight_format_cast",
    "qk_quantize_per_tensor", "qk_quantize_per_channel", "qk_dequantize", "qk_rms_norm", "qk_rms_norm_quant",
    "qk_swiglu", "qk_swiglu_quant", "qk_quant_matmul_swiglu", "qk_quant_matmul_swiglu_quant_workspace_size",
    "qk_quant_matmul_swiglu_quant",
)

_abi = None


def abi() -> ctypes.CDLL:
    """ctypes handle on libqk_hip.so with argtypes set (the C ABI of include/qk_abi.h)."""
    global _abi
    if _abi is None:
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
        L.qk_last_error.restype = ctypes.c_char_p
        L.qk_last_error.argtypes = []
        L.qk_abi_version.restype = I
        L.qk_debug_set_plan.argtypes = [ctypes.c_char_p]
        L.qk_dynamic_quant.argtypes = [P, I, I64, I64, P, P, P, P]
        L.qk_quant_matmul_workspace_size.argtypes = [I64, I64, I64, I, ctypes.POINTER(SZ)]
        L.qk_quant_matmul.argtypes = [P, I64, P, I64, I64, I64, I64, I64, P, I64, P, I64, P, P, I, P, I, P, SZ, P]
        L.qk_quant_matmul_nz_workspace_size.argtypes = [I64, I64, I64, I, ctypes.POINTER(SZ)]
        L.qk_quant_matmul_nz.argtypes = [P, I64, P, I64, I64, I64, P, I64, P, I64, P, P, I, P, I, P, SZ, P]
        L.qk_weight_quant_bmm_workspace_size.argtypes = [I64, I64, I64, I, I64, ctypes.POINTER(SZ)]
        L.qk_weight_quant_bmm.argtypes = [P, I, P, I, P, P, I, I64, I64, I64, I64, P, I, P, I, P, SZ, P]
        L.qk_weight_quant_bmm_noalloc.argtypes = [P, I, P, I, P, P, I, I64, I64, I64, I64, P, I, P, I, P]
        L.qk_int4_pack.argtypes = [P, I, I64, I64, P, P]
        L.qk_weight_format_cast.argtypes = [P, I, P, I, I, I64, I64, P]
        L.qk_quantize_per_tensor.argtypes = [P, I, I64, ctypes.c_float, I64, P, I, P]
        L.qk_quantize_per_channel.argtypes = [P, I, I64, I64, I64, P, P, P, I, P]
        L.qk_dequantize.argtypes = [P, I, I64, P, P]
        F = ctypes.c_float
        L.qk_rms_norm.argtypes = [P, I, P, I64, I64, F, P, P, P]
        L.qk_rms_norm_quant.argtypes = [P, I, P, I64, I64, F, P, P, P, P]
        L.qk_swiglu.argtypes = [P, I, I64, I64, P, P]
        L.qk_swiglu_quant.argtypes = [P, I, I64, I64, P, P, P]
        L.qk_quant_matmul_swiglu.argtypes = [P, I64, P, I, I64, I64, I64, I64, P, I64, P, P, I, P]
        L.qk_quant_matmul_swiglu_quant_workspace_size.argtypes = [I64, I64, P]
        L.qk_quant_matmul_swiglu_quant.argtypes = [P, I64, P, I, I64, I64, I64, I64, P, I64, P, I, P, P, P, SZ, P]
        for name in ABI_SYMBOLS:
            getattr(L, name).restype = I if name != "qk_last_error" else ctypes.c_char_p
        _abi = L
    return _abi


def get_npu_format(t: torch.Tensor) -> int:
    """Storage format of a tensor, as torch_npu.get_npu_format reports it: FRACTAL_NZ (29) for a weight that
    npu_format_cast(w, 29) or npu_convert_weight_to_int4pack(w, inner_k_tiles=4) returned (the format is recorded
    with its storage, not inferred from the shape), ND (2) for every other tensor."""
    return int(torch.ops.npu.get_npu_format(t))


def last_error() -> str:
    return abi().qk_last_error().decode()


def debug_set_plan(spec: str = "") -> None:
    """Force kernel choices of the planners (tests and tuning only; "" restores the planners' choices).

    Spec grammar: see PlanOverride in csrc/kernels/common.h, e.g. "w4_gemm=force" or
    "w4_stream=8:4:2,skinny_splits=4"."""
    rc = abi().qk_debug_set_plan(spec.encode())
    if rc != 0:
        raise ValueError(last_error())


__all__ = [
    "npu_dynamic_quant", "npu_quant_matmul", "npu_weight_quant_batchmatmul",
    "npu_convert_weight_to_int4pack", "npu_format_cast", "get_npu_format", "quantize_per_tensor",
    "quantize_per_channel", "dequantize", "npu_rms_norm", "npu_swiglu", "npu_rms_norm_dynamic_quant",
    "npu_swiglu_dynamic_quant", "npu_quant_matmul_swiglu", "npu_quant_matmul_swiglu_quant", "abi", "last_error", "debug_set_plan", "LIB_PATH", "OPS_PATH",
]
