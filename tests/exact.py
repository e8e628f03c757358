"""Whole-output references for the large configurations (test helper, CPU only).

W8A8: the int32 accumulator of int8 x int8 from a float64 GEMM.  Every product
is an integer of magnitude at most 128 * 128 = 16384 and every partial sum an
integer below 2^53 (K < 2^39), so each float64 addition is exact and the
result equals the int32 accumulator bit for bit, whatever order the BLAS adds
in.  The float64 GEMM runs on all host cores, so a cfg4-sized accumulator
(4096 x 8192 x 8192) takes seconds where the C oracle's scalar loop takes tens.
Callers pin it against the C oracle (qo_w8a8_acc) on a sub-block in the same
test and then apply the oracle's epilogue (qo_quant_matmul_epilogue) to the
whole accumulator.

W4A16 / W8A16: x @ ((w + offset) * scale) in float64 with the group scales
expanded along K -- the dequant-matmul that tests/test_oracle.py
(test_w4a16_matches_float64_dequant) pins the C oracle against.
"""
from __future__ import annotations

import os

import numpy as np
import torch


def _threads():
    torch.set_num_threads(max(1, os.cpu_count() or 1))


def w8a8_acc(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """a int8 [M,K], w int8 [K,N] -> exact int32 [M,N]."""
    _threads()
    acc = torch.from_numpy(np.ascontiguousarray(a)).double() @ torch.from_numpy(np.ascontiguousarray(w)).double()
    assert acc.abs().max().item() < 2.0**31
    return acc.to(torch.int32).numpy()


def pin_acc(oracle, a: np.ndarray, w: np.ndarray, acc: np.ndarray, rows) -> None:
    """The float64 accumulator equals the C oracle's on the given rows (all columns)."""
    ref = oracle.w8a8_acc(a[rows], w)
    assert np.array_equal(acc[rows], ref), "float64 accumulator differs from qo_w8a8_acc"


def wq_dequant_matmul(x: torch.Tensor, w_values: torch.Tensor, scale: torch.Tensor, offset, group: int,
                      bias=None) -> torch.Tensor:
    """x [M,K] fp16/bf16, w_values int [K,N] (the unpacked weights), scale/offset [K/G,N] or [N] -> float64 [M,N]."""
    _threads()
    K = x.shape[-1]
    G = group if group > 0 else K
    s = scale.double().reshape(-1, scale.shape[-1])
    o = None if offset is None else offset.double().reshape(-1, offset.shape[-1])
    wf = w_values.double()
    if o is not None:
        wf = wf + o.repeat_interleave(G, 0)
    wf = wf * s.repeat_interleave(G, 0)
    out = x.double() @ wf
    if bias is not None:
        out = out + bias.double()
    return out
