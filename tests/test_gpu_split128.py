"""The W8A8 K split on 128-row tiles (qmm_dma<.., 128> + qmm_reduce_tiled).

Shapes with few 256 x 256 tiles (cfg5's down projection, 512 x 4096 x 14336: 32 tiles) are split along K to fill
the 256 CUs.  On 128-row tiles the same shape needs half the splits, so half the int32 partials are written and
read back.  The int32 sums are exact whatever the split, so the outputs must equal the 256-row split's bit for bit
(debug override qmm_bm128=0) and the oracle's: int32 outputs against the exact accumulator, bf16 outputs against
qo_quant_matmul_epilogue on that accumulator.
"""
import ctypes

import numpy as np
import pytest
import torch

import exact
from op_plugin_amd import workloads as W

pytestmark = pytest.mark.gpu

BF16, I32 = 2, 5
DEV = "cuda"
NZ = 29


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    return op_plugin_amd


@pytest.fixture
def plan(ops):
    yield ops.debug_set_plan
    ops.debug_set_plan("")


def say(msg):
    print(f"[case] {msg}", flush=True)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _inputs(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    s = 1e-4 + 1e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    b = torch.randn(N, generator=g).to(torch.bfloat16)
    return a, w, s, pt, b


def _weight(ops, w, layout):
    """The same [K,N] weight as the op reads it: NZ (cast once), [K,N] rows, or an [N,K] tensor's transpose."""
    wd = w.to(DEV)
    if layout == "nz":
        return ops.npu_format_cast(wd, NZ)
    if layout == "nk":
        return wd.t().contiguous().t()
    return wd


SHAPES = [
    (512, 4096, 14336),  # cfg5 down projection: 4 splits of 64 tiles instead of 8 of 32
    (300, 4096, 8192),   # ragged M: the last 128-row tile holds 44 rows
]


@pytest.mark.parametrize("layout", ["nz", "kn", "nk"])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_split128_bits_and_oracle(ops, oracle, plan, M, N, K, layout):
    say(f"quant_matmul 128-row split {M}x{N}x{K} weight={layout}")
    a, w, s, pt, b = _inputs(M, N, K, seed=M + K)
    ad, sd, ptd, bd = a.to(DEV), s.to(DEV), pt.to(DEV), b.to(DEV)
    wd = _weight(ops, w, layout)
    acc_gpu = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    out = ops.npu_quant_matmul(ad, wd, sd, pertoken_scale=ptd, bias=bd, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    plan("qmm_bm128=0")
    acc_256 = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    out_256 = ops.npu_quant_matmul(ad, wd, sd, pertoken_scale=ptd, bias=bd, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(acc_gpu, acc_256), "int32 sums differ between the 128-row and 256-row splits"
    assert torch.equal(out.view(torch.int16), out_256.view(torch.int16))
    acc = exact.w8a8_acc(a.numpy(), w.numpy())
    exact.pin_acc(oracle, a.numpy(), w.numpy(), acc, np.r_[0:2, M - 2:M])
    got = acc_gpu.cpu().numpy()
    bad = np.argwhere(got != acc)
    assert bad.size == 0, f"{len(bad)} int32 sums differ from the exact accumulator, first at {tuple(bad[0])}"
    ref = oracle.quant_matmul_epilogue(acc, s.numpy(), pertoken=pt.numpy(), bias=W.bits(b), bias_dtype=BF16,
                                       out_dtype=BF16)
    assert np.array_equal(W.bits(out.cpu()), ref)


@pytest.mark.parametrize("nz", [False, True])
def test_abi_split128_exact_workspace_ff(ops, oracle, nz):
    """Through the C ABI with exactly the queried workspace, pre-filled with 0xFF, twice: the partials of every
    row (the ragged tile's padding rows included) are written before they are read."""
    M, N, K = 300, 4096, 8192
    say(f"ABI 128-row split {M}x{N}x{K} nz={nz}, 0xFF workspace")
    L = ops.abi()
    n = ctypes.c_size_t(0)
    query = L.qk_quant_matmul_nz_workspace_size if nz else L.qk_quant_matmul_workspace_size
    assert query(M, N, K, BF16, ctypes.byref(n)) == 0
    a, w, s, pt, b = _inputs(M, N, K, seed=77)
    ad, sd, ptd, bd = a.to(DEV), s.to(DEV), pt.to(DEV), b.to(DEV)
    wd = ops.npu_format_cast(w.to(DEV), NZ) if nz else w.to(DEV)
    wsbuf = torch.full((n.value,), 0xFF, dtype=torch.uint8, device=DEV)
    outs = []
    for _ in range(2):
        out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
        if nz:
            rc = L.qk_quant_matmul_nz(ad.data_ptr(), K, wd.data_ptr(), M, N, K, sd.data_ptr(), N, None, 0,
                                      ptd.data_ptr(), bd.data_ptr(), BF16, out.data_ptr(), BF16, wsbuf.data_ptr(),
                                      n.value, _stream())
        else:
            rc = L.qk_quant_matmul(ad.data_ptr(), K, wd.data_ptr(), N, 1, M, N, K, sd.data_ptr(), N, None, 0,
                                   ptd.data_ptr(), bd.data_ptr(), BF16, out.data_ptr(), BF16, wsbuf.data_ptr(),
                                   n.value, _stream())
        assert rc == 0, ops.last_error()
        torch.cuda.synchronize()
        outs.append(out)
    rows = np.r_[0:3, 127:130, 255:258, M - 4:M]
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(), pertoken=pt[rows].numpy(), bias=W.bits(b),
                              bias_dtype=BF16, out_dtype=BF16)
    assert np.array_equal(W.bits(outs[0].cpu())[rows], ref)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
