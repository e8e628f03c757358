"""Seeded random shapes and argument mixes through the row-major weight paths (the reference's default ND
format) of npu_quant_matmul and npu_weight_quant_batchmatmul, against the oracle.

The draws span every planner of both ops: decode streams with and without K splits, the mid-M kernels, whole
256 x 256 prefill tiles with and without a K split, ragged M / N / K and the generic kernels for shapes the
tiled kernels do not take. Bars as in the other parity tests: W8A8 int32 accumulators and every output dtype
bit-exact against the exact accumulator plus the oracle's epilogue; W4A16 / W8A16 within rtol / atol 1e-2 of
the float64 oracle.
"""
import numpy as np
import pytest
import torch

import exact
from op_plugin_amd import workloads as W

pytestmark = pytest.mark.gpu

F16, BF16, F32, I8, I32 = 1, 2, 3, 4, 5
CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32, torch.int8: I8, torch.int32: I32}
DTYPE = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "i8": torch.int8, "i32": torch.int32}
DEV = "cuda"


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    return op_plugin_amd


def say(msg):
    print(f"[case] {msg}", flush=True)


# ----------------------------------------------------------------------------- npu_quant_matmul

def _qmm_draws(seed, n):
    """(M, N, K, layout, out, bias, pertoken, per_tensor, offset) draws: a third whole 256 x 256 tiles
    (M >= 256), a third 16-column / 64-row multiples, a third arbitrary sizes; the argument mix restricted to
    what the op accepts (per-token scales only with float outputs, an offset only with int8 output, integer
    outputs with an int32 bias or none)."""
    rng = np.random.default_rng(seed)
    ms = [1, 2, 3, 4, 7, 8, 15, 16, 17, 24, 32, 33, 48, 63, 64, 65, 96, 100, 127, 128, 129, 192, 255, 256, 257,
          384, 511, 512, 600]
    out = []
    for i in range(n):
        kind = i % 3
        M = int(rng.choice(ms))
        if kind == 0:  # the prefill tiles: M of two or more 256-row tiles or a ragged last one
            M = int(rng.choice([256, 257, 384, 511, 512, 600, 768]))
            N, K = 256 * int(rng.integers(1, 13)), 256 * int(rng.integers(1, 17))
        elif kind == 1:
            N, K = 16 * int(rng.integers(1, 160)), 64 * int(rng.integers(1, 64))
        else:
            N, K = int(rng.integers(1, 700)), int(rng.integers(1, 1500))
        layout = str(rng.choice(["kn", "nk"]))
        o = str(rng.choice(["bf16", "f16", "f32", "i8", "i32"]))
        if o in ("i8", "i32"):
            bias = str(rng.choice(["none", "i32"]))
            pertoken = False
        else:
            bias = str(rng.choice(["none", "bf16", "f16", "f32", "i32"]))
            pertoken = bool(rng.integers(0, 2))
        per_tensor = bool(rng.integers(0, 4) == 0)
        offset = o == "i8" and bool(rng.integers(0, 2))
        out.append((M, N, K, layout, o, bias, pertoken, per_tensor, offset))
    return out


@pytest.mark.parametrize("M,N,K,layout,out,bias,pertoken,per_tensor,offset", _qmm_draws(20261202, 45))
def test_quant_matmul_random(ops, oracle, M, N, K, layout, out, bias, pertoken, per_tensor, offset):
    say(f"quant_matmul random M={M} N={N} K={K} {layout} out={out} bias={bias} pertoken={pertoken} "
        f"per_tensor={per_tensor} offset={offset}")
    g = torch.Generator().manual_seed(M * 131 + N * 17 + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    wd = w.to(DEV) if layout == "kn" else w.t().contiguous().to(DEV).t()  # [K,N] view of an [N,K] tensor
    # int8 output: scales that keep most outputs inside the int8 range, so rounding is exercised, not clamping
    lo, hi = (1e-5, 1e-4) if out == "i8" else (1e-3, 1e-2)
    s = lo + (hi - lo) * torch.rand(1 if per_tensor else N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g) if pertoken else None
    off = torch.randn(1 if per_tensor else N, generator=g) if offset else None
    b = None
    if bias == "i32":
        b = torch.randint(-1000, 1000, (N,), generator=g, dtype=torch.int32)
    elif bias != "none":
        b = torch.randn(N, generator=g).to(DTYPE[bias])
    got = ops.npu_quant_matmul(a.to(DEV), wd, s.to(DEV), offset=None if off is None else off.to(DEV),
                               pertoken_scale=None if pt is None else pt.to(DEV),
                               bias=None if b is None else b.to(DEV), output_dtype=DTYPE[out]).cpu()
    assert got.shape == (M, N) and got.dtype == DTYPE[out]

    an, wn = a.numpy(), w.numpy()
    acc = exact.w8a8_acc(an, wn)
    exact.pin_acc(oracle, an, wn, acc, np.r_[0:1, M - 1:M])
    if out == "i32" and b is None:
        ref = acc
    else:
        bias_np = None if b is None else (b.numpy() if b.dtype in (torch.int32, torch.float32) else W.bits(b))
        ref = oracle.quant_matmul_epilogue(acc, s.numpy(), offset=None if off is None else off.numpy(),
                                           pertoken=None if pt is None else pt.numpy(), bias=bias_np,
                                           bias_dtype=CODE[b.dtype] if b is not None else BF16, out_dtype=CODE[DTYPE[out]])
    got_np = got.numpy() if out in ("f32", "i8", "i32") else W.bits(got)
    bad = np.argwhere(got_np != ref)
    assert bad.size == 0, f"{len(bad)} outputs differ, first at {tuple(bad[0])}"


# ----------------------------------------------------------------------------- npu_weight_quant_batchmatmul

def _wq_draws(seed, n):
    """(M, N, K, group, bits, offset, x, scale, bias) draws with the oracle's scalar loop in well under a second
    (M * N * K <= 4e7): int4 weights need N % 8 == 0, groups of 32 to 512 rows or per channel."""
    rng = np.random.default_rng(seed)
    ms = [1, 2, 3, 5, 8, 9, 16, 17, 31, 32, 33, 64, 65, 100, 128, 129, 200, 256, 300]
    out = []
    for i in range(n):
        bits = 4 if i % 3 else 8
        M = int(rng.choice(ms))
        group = int(rng.choice([32, 64, 128, 256, 512, 0]))
        kq = group if group else 32
        K = kq * int(rng.integers(1, max(2, 4096 // kq + 1)))
        step = 8 if bits == 4 else int(rng.choice([1, 8, 16]))
        nmax = max(1, min(12000 // step, int(4e7 // (M * K * step))))
        N = step * int(rng.integers(1, nmax + 1))
        offset = bool(rng.integers(0, 2))
        x = str(rng.choice(["bf16", "f16"]))
        sc = str(rng.choice(["bf16", "f16"]))
        bias = str(rng.choice(["none", "same", "f32"]))
        out.append((M, N, K, group, bits, offset, x, sc, bias))
    return out


@pytest.mark.parametrize("M,N,K,group,bits,offset,x,sc,bias", _wq_draws(1202, 45))
def test_weight_quant_bmm_random(ops, oracle, M, N, K, group, bits, offset, x, sc, bias):
    say(f"weight_quant_bmm random M={M} N={N} K={K} group={group} int{bits} offset={offset} x={x} scale={sc} "
        f"bias={bias}")
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K + bits)
    xd, sd = DTYPE[x], DTYPE[sc]
    xt = torch.randn((M, K), generator=g).to(xd)
    ng = K // group if group else 1
    if bits == 4:
        w = torch.randint(-8, 8, (K, N), generator=g, dtype=torch.int8)
        wt = W.int4_pack_cpu(w)
        s = (5e-3 + 1.5e-2 * torch.rand((ng, N), generator=g)).to(sd)
        o = (2 * torch.rand((ng, N), generator=g) - 1).to(sd) if offset else None
    else:
        wt = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
        s = (5e-4 + 2.5e-3 * torch.rand((ng, N), generator=g)).to(sd)
        o = (8 * torch.rand((ng, N), generator=g) - 4).to(sd) if offset else None
    if group == 0:
        s = s.reshape(-1)
        o = None if o is None else o.reshape(-1)
    b = None if bias == "none" else torch.randn(N, generator=g).to(xd if bias == "same" else torch.float32)
    got = ops.npu_weight_quant_batchmatmul(xt.to(DEV), wt.to(DEV), s.to(DEV), None if o is None else o.to(DEV),
                                           bias=None if b is None else b.to(DEV), antiquant_group_size=group)
    assert got.shape == (M, N) and got.dtype == xd
    bias_np = None if b is None else (b.numpy() if b.dtype == torch.float32 else W.bits(b))
    ref = oracle.weight_quant_bmm(W.bits(xt), CODE[xd], wt.numpy(), W.bits(s), None if o is None else W.bits(o),
                                  CODE[sd], group, bias=bias_np, bias_dtype=CODE[b.dtype] if b is not None else BF16,
                                  out_dtype=CODE[xd])
    torch.testing.assert_close(got.cpu().float(), W.from_bits(ref, xd).float(), rtol=1e-2, atol=1e-2)
