"""The quantized Llama-style MLP block built from the torch.ops.npu ops (the cfg5 workload).

    y1, s1  = RMSNorm(x; gamma, eps) -> per-token int8        npu_rms_norm_dynamic_quant
    y2, s2  = per-token int8 of h = SwiGLU(W8A8(y1, W_gate_up; s1, s_gate_up))
                                                               npu_quant_matmul_swiglu_quant   h: [T, I]
    out     = W8A8(y2, W_down; s2, s_down) -> bf16             npu_quant_matmul   [T, H]

The gate-up GEMM applies the SwiGLU in its epilogue (its output is the [T, I] activation instead of the
[T, 2I] gate-up product: half the bytes written, and the SwiGLU pass no longer reads them) and stores each
row's absmax per 128 columns, so quantizing h is one elementwise pass with no row reduction.  With
``fused=False`` the same block runs as the unfused chain (npu_rms_norm, npu_dynamic_quant, npu_quant_matmul
to [T, 2I], npu_swiglu, npu_dynamic_quant); both give identical bits.  The first half of the gate_up output
is the gate (silu(gate) * up).
"""
from __future__ import annotations

import torch

from . import (npu_dynamic_quant, npu_quant_matmul, npu_quant_matmul_swiglu_quant, npu_rms_norm,
               npu_rms_norm_dynamic_quant, npu_swiglu)


def quant_mlp(x: torch.Tensor, gamma: torch.Tensor, w_gate_up: torch.Tensor, s_gate_up: torch.Tensor,
              w_down: torch.Tensor, s_down: torch.Tensor, eps: float = 1e-6, fused: bool = True,
              out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """x [T, H] fp16/bf16, gamma [H], w_gate_up int8 [H, 2I] (or a transposed [2I, H] view, or the int8 NZ
    weight npu_format_cast(w, 29) writes), s_gate_up fp32 [2I], w_down int8 [I, H] (likewise), s_down fp32 [H]
    -> [T, H]."""
    if fused:
        y1, s1, _ = npu_rms_norm_dynamic_quant(x, gamma, eps)
    else:
        y, _ = npu_rms_norm(x, gamma, eps)
        y1, s1 = npu_dynamic_quant(y)
    if fused:
        y2, s2 = npu_quant_matmul_swiglu_quant(y1, w_gate_up, s_gate_up, pertoken_scale=s1, output_dtype=out_dtype)
    else:
        h = npu_swiglu(npu_quant_matmul(y1, w_gate_up, s_gate_up, pertoken_scale=s1, output_dtype=out_dtype))
        y2, s2 = npu_dynamic_quant(h)
    return npu_quant_matmul(y2, w_down, s_down, pertoken_scale=s2, output_dtype=out_dtype)
