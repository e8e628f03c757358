"""Seeded synthetic inputs for the five benchmark configurations.

Every tensor is drawn on the CPU from one ``torch.Generator().manual_seed(seed)``
per configuration in a fixed order (x -> outlier channels -> W -> w_scale ->
bias / antiquant scale -> antiquant offset), so the GPU kernels and the CPU
oracle see identical bits.  Uniform int8 in [-127,127] is
``randint(-127, 128)``; int4 in [-8,7] is ``randint(-8, 8)``; ``U[a,b]`` is
``a + (b-a) * rand``.
"""
from __future__ import annotations

import dataclasses

import torch


@dataclasses.dataclass(frozen=True)
class W8A8Case:
    M: int
    N: int
    K: int
    x_dtype: torch.dtype = torch.float16
    bias: bool = True
    outlier_frac: float = 0.0


@dataclasses.dataclass(frozen=True)
class W4A16Case:
    M: int
    N: int
    K: int
    group: int = 128
    x_dtype: torch.dtype = torch.bfloat16
    offset: bool = True


# BASELINE.json "configs", in order.
CFG1 = W8A8Case(M=128, N=4096, K=4096)                                        # CPU reference config
CFG2 = tuple(W8A8Case(M=m, N=28672, K=8192, bias=False, outlier_frac=0.01) for m in (1, 4, 16))
CFG3 = tuple(W4A16Case(M=m, N=11008, K=4096) for m in (16, 2048))
CFG4 = W8A8Case(M=4096, N=8192, K=8192)                                       # prefill, headline
CFG5 = dict(tokens=512, hidden=4096, intermediate=14336, eps=1e-6)


def _uniform(g: torch.Generator, shape, lo: float, hi: float) -> torch.Tensor:
    return lo + (hi - lo) * torch.rand(shape, generator=g, dtype=torch.float32)


def w8a8_inputs(case: W8A8Case, seed: int = 0) -> dict:
    """x [M,K] (fp16/bf16), w int8 [K,N], w_scale fp32 [N], bias bf16 [N] or None."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((case.M, case.K), generator=g, dtype=torch.float32)
    if case.outlier_frac > 0:
        n_out = max(1, round(case.outlier_frac * case.K))
        idx = torch.randperm(case.K, generator=g)[:n_out]
        x[:, idx] *= 20.0
    x = x.to(case.x_dtype)
    w = torch.randint(-127, 128, (case.K, case.N), generator=g, dtype=torch.int8)
    w_scale = _uniform(g, (case.N,), 1e-3, 1e-2)
    bias = (0.1 * torch.randn((case.N,), generator=g, dtype=torch.float32)).to(torch.bfloat16) \
        if case.bias else None
    return dict(x=x, w=w, w_scale=w_scale, bias=bias)


def int4_pack_cpu(w: torch.Tensor) -> torch.Tensor:
    """int8 [K,N] in [-8,7] -> int32 [K,N/8], nibble i of word j = w[:, 8j+i].

    Vectorised host-side packing used to prepare synthetic inputs; the device
    op ``npu_convert_weight_to_int4pack`` does the same on the GPU."""
    K, N = w.shape
    assert N % 8 == 0
    nib = (w.to(torch.int64) & 0xF).reshape(K, N // 8, 8)
    shifts = torch.arange(8, dtype=torch.int64) * 4
    words = (nib << shifts).sum(dim=-1)
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32)


def w4a16_inputs(case: W4A16Case, seed: int = 0) -> dict:
    """x [M,K] bf16, w int8 values [K,N] in [-8,7], w_packed int32 [K,N/8],
    scale fp16 [K/G,N] in U[5e-3,2e-2], offset fp16 [K/G,N] in U[-1,1]."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((case.M, case.K), generator=g, dtype=torch.float32).to(case.x_dtype)
    w = torch.randint(-8, 8, (case.K, case.N), generator=g, dtype=torch.int8)
    ng = case.K // case.group if case.group > 0 else 1
    scale = _uniform(g, (ng, case.N), 5e-3, 2e-2).to(torch.float16)
    offset = _uniform(g, (ng, case.N), -1.0, 1.0).to(torch.float16) if case.offset else None
    return dict(x=x, w=w, w_packed=int4_pack_cpu(w), scale=scale, offset=offset)


def mlp_inputs(tokens: int, hidden: int, intermediate: int, seed: int = 0) -> dict:
    """cfg5: x bf16 [T,H], gamma bf16 [H] ~ N(1,0.02), gate_up int8 [H,2I],
    down int8 [I,H], per-channel fp32 scales in U[1e-3,1e-2]."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((tokens, hidden), generator=g, dtype=torch.float32).to(torch.bfloat16)
    gamma = (1.0 + 0.02 * torch.randn((hidden,), generator=g, dtype=torch.float32)).to(torch.bfloat16)
    w_gu = torch.randint(-127, 128, (hidden, 2 * intermediate), generator=g, dtype=torch.int8)
    s_gu = _uniform(g, (2 * intermediate,), 1e-3, 1e-2)
    w_d = torch.randint(-127, 128, (intermediate, hidden), generator=g, dtype=torch.int8)
    s_d = _uniform(g, (hidden,), 1e-3, 1e-2)
    return dict(x=x, gamma=gamma, w_gu=w_gu, s_gu=s_gu, w_d=w_d, s_d=s_d)


def bits(t: torch.Tensor):
    """uint16 numpy view of an fp16/bf16 CPU tensor (what the oracle consumes)."""
    import numpy as np
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a, dtype: torch.dtype) -> torch.Tensor:
    import numpy as np
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)
