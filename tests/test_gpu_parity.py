"""GPU parity: the HIP kernels against the CPU oracle on the same seeded inputs.

Bar: int8 quantized activations, their scales and int32 accumulators
bit-exact; W8A8 bf16/fp16 outputs bit-exact as well (the epilogue's float32
operations are fixed by the op contract) and, as the stated bar, within
rtol 1e-2 / atol 1e-2; W4A16 outputs within rtol 1e-2 / atol 1e-2 of the
float64 oracle.  Full-size shapes the oracle cannot finish in seconds are
checked on a row subset plus exact checksums of the whole int32 output.
"""
import ctypes

import numpy as np
import pytest
import torch

import exact
from op_plugin_amd import workloads as W

pytestmark = pytest.mark.gpu

F16, BF16, F32, I8, I32 = 1, 2, 3, 4, 5
CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32, torch.int8: I8, torch.int32: I32}
DEV = "cuda"


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    return op_plugin_amd


def say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture
def plan(ops):
    """Force planner choices for one test (the library's debug override); restored afterwards."""
    yield ops.debug_set_plan
    ops.debug_set_plan("")


def to_bits(t):
    return W.bits(t.cpu())


def bf16_close(got_bits, ref_bits, dtype=torch.bfloat16, rtol=1e-2, atol=1e-2):
    g = W.from_bits(got_bits, dtype).float()
    r = W.from_bits(ref_bits, dtype).float()
    torch.testing.assert_close(g, r, rtol=rtol, atol=atol)


# ----------------------------------------------------------------------------- npu_dynamic_quant

DQ_CASES = [
    ("cfg1", W.CFG1, None),
    ("cfg2_m16", W.CFG2[2], None),
    ("cfg4", W.CFG4, None),
]


@pytest.mark.parametrize("name,case,_", DQ_CASES)
def test_dynamic_quant_configs(ops, oracle, name, case, _):
    say(f"dynamic_quant {name} {case.M}x{case.K}")
    x = W.w8a8_inputs(case)["x"]
    y, s = ops.npu_dynamic_quant(x.to(DEV))
    torch.cuda.synchronize()
    ry, rs = oracle.dynamic_quant(W.bits(x), CODE[x.dtype])
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(y.cpu().numpy(), ry)


@pytest.mark.parametrize("K", [4096, 14336])
def test_dynamic_quant_cfg5_bf16(ops, oracle, K):
    say(f"dynamic_quant cfg5 bf16 512x{K}")
    g = torch.Generator().manual_seed(K)
    x = torch.randn((512, K), generator=g).to(torch.bfloat16)
    y, s = ops.npu_dynamic_quant(x.to(DEV))
    ry, rs = oracle.dynamic_quant(W.bits(x), BF16)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(y.cpu().numpy(), ry)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K", [1, 7, 8, 24, 1000, 2056, 40000])
def test_dynamic_quant_edge_cases(ops, oracle, dtype, K):
    say(f"dynamic_quant edge {dtype} K={K}")
    g = torch.Generator().manual_seed(K)
    x = torch.randn((6, K), generator=g)
    x[1] = 0.0                                   # zero row
    x[2] = 0.0
    x[2, K // 2] = -3.0                          # single nonzero
    x[3] = x[3] * 1e-30 if dtype == torch.bfloat16 else x[3] * 1e-6   # tiny (subnormal range)
    if K >= 8:                                   # exact ties around scale 1.0
        x[4, :8] = torch.tensor([127.0, 0.5, 1.5, 2.5, -2.5, 3.5, 126.5, -126.5])
        x[4, 8:] = 0.0
    x = x.to(dtype)
    y, s = ops.npu_dynamic_quant(x.to(DEV))
    ry, rs = oracle.dynamic_quant(W.bits(x), CODE[dtype])
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(y.cpu().numpy(), ry)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K", [8, 1000, 1001, 8192])
def test_dynamic_quant_non_finite_and_half_max(ops, oracle, dtype, K):
    """Rows at +-65504 (NPU_HALF_MAX, op_plugin/utils/OpConstants.h:25), rows holding NaN or +-Inf, an all-NaN row,
    and for bf16 rows at the bf16 limit: bit-exact against the oracle's stated non-finite contract (NaN elements
    do not enter the absmax; a NaN quotient gives -128; a row with an infinity has s = +Inf).  K = 1001 takes the
    generic kernel, the others the vector kernel."""
    say(f"dynamic_quant non-finite / half-max {dtype} K={K}")
    g = torch.Generator().manual_seed(K + 1)
    x = torch.randn((9, K), generator=g)
    nan, inf = float("nan"), float("inf")
    x[0, 0], x[0, K // 2] = 65504.0, -65504.0                  # fp16 limits with ordinary values
    x[1] = 0.0
    x[1, K - 1] = -65504.0                                      # a lone -65504
    x[2, 1 % K] = nan                                           # one NaN in an ordinary row
    x[3, ::3] = nan                                             # many NaNs
    x[4, K - 1] = inf                                           # +Inf: s = +Inf
    x[5, 0] = -inf
    x[5, K // 2] = inf
    x[5, K // 3] = nan
    x[6] = nan                                                  # all NaN: s = 0, y = 0
    x[7, 3 % K] = 3.3895e38 if dtype == torch.bfloat16 else 65504.0   # the dtype's largest finite value
    x[8, :8] = torch.tensor([127.0, nan, 126.5, -0.5, 1.5, -inf if K > 8 else 2.0, 0.0, -2.5])
    x = x.to(dtype)
    y, s = ops.npu_dynamic_quant(x.to(DEV))
    ry, rs = oracle.dynamic_quant(W.bits(x), CODE[dtype])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(y.cpu().numpy(), ry)
    assert ry[6].tolist() == [0] * K and rs[6] == 0.0
    assert ry[2, 1 % K] == -128 and rs[4] == np.inf


def test_dynamic_quant_smooth_and_batch_dims(ops, oracle):
    say("dynamic_quant smooth scales, 3-D input")
    g = torch.Generator().manual_seed(11)
    x = torch.randn((2, 3, 512), generator=g).to(torch.float16)
    sm = 0.5 + torch.rand(512, generator=g)
    y, s = ops.npu_dynamic_quant(x.to(DEV), smooth_scales=sm.to(DEV))
    assert y.shape == (2, 3, 512) and s.shape == (2, 3)
    ry, rs = oracle.dynamic_quant(W.bits(x), F16, sm.numpy())
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(y.cpu().numpy(), ry)


def test_dynamic_quant_empty(ops):
    say("dynamic_quant empty")
    y, s = ops.npu_dynamic_quant(torch.empty((0, 64), dtype=torch.float16, device=DEV))
    assert y.shape == (0, 64) and s.shape == (0,)


# ----------------------------------------------------------------------------- npu_quant_matmul

@pytest.mark.parametrize("M,N,K", [(1, 128, 64), (4, 256, 128), (16, 96, 512), (33, 200, 1024),
                                   (128, 384, 4096), (257, 136, 192), (64, 8, 16), (5, 7, 13)])
@pytest.mark.parametrize("transposed", [False, True])
def test_quant_matmul_int32_exact(ops, oracle, M, N, K, transposed):
    say(f"quant_matmul int32 M={M} N={N} K={K} transposed={transposed}")
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    wd = w.to(DEV)
    if transposed:
        wd = w.t().contiguous().to(DEV).t()      # [K,N] view of an [N,K] tensor
    one = torch.ones(1, device=DEV)
    out = ops.npu_quant_matmul(a.to(DEV), wd, one, output_dtype=torch.int32)
    ref = oracle.w8a8_acc(a.numpy(), w.numpy())
    assert np.array_equal(out.cpu().numpy(), ref)


def _w8a8_full_path(ops, oracle, case, seed=0, nz=False):
    """dynamic quant -> W8A8 -> bf16 on a whole config, every output element bit-exact against the oracle:
    the quantized rows and scales from qo_dynamic_quant, the accumulator from a float64 GEMM (exact; pinned
    against qo_w8a8_acc on its first and last rows here), the epilogue from qo_quant_matmul_epilogue.
    nz: the weight is cast once to the int8 NZ layout (npu_format_cast(w, 29)) and the op reads that.
    Returns the quantized activations (device), the weight the op read (device) and the exact accumulator."""
    d = W.w8a8_inputs(case, seed)
    x, w, ws, b = d["x"], d["w"], d["w_scale"], d["bias"]
    xq, xs = ops.npu_dynamic_quant(x.to(DEV))
    wd = w.to(DEV)
    if nz:
        wd = ops.npu_format_cast(wd, 29)
        assert ops.get_npu_format(wd) == 29
    out = ops.npu_quant_matmul(xq, wd, ws.to(DEV), pertoken_scale=xs,
                               bias=None if b is None else b.to(DEV), output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    rq, rs = oracle.dynamic_quant(W.bits(x), CODE[x.dtype])
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(xs.cpu().numpy(), rs)
    wn = w.numpy()
    acc = exact.w8a8_acc(rq, wn)
    exact.pin_acc(oracle, rq, wn, acc, np.r_[0:2, case.M - 2:case.M] if case.M > 4 else np.arange(case.M))
    ref = oracle.quant_matmul_epilogue(acc, ws.numpy(), pertoken=rs, bias=None if b is None else W.bits(b),
                                       bias_dtype=BF16, out_dtype=BF16)
    got = to_bits(out)
    bf16_close(got, ref)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{len(bad)} bf16 outputs differ in bits, first at {tuple(bad[0])}"
    return xq, wd, acc


@pytest.mark.parametrize("nz", [False, True])
def test_quant_matmul_cfg1(ops, oracle, nz):
    say(f"quant_matmul cfg1 full path 128x4096x4096 nz={nz}")
    _w8a8_full_path(ops, oracle, W.CFG1, nz=nz)


@pytest.mark.parametrize("idx", [0, 1, 2])
def test_quant_matmul_cfg2_decode(ops, oracle, idx):
    c = W.CFG2[idx]
    say(f"quant_matmul cfg2 M={c.M} 8192x28672")
    _w8a8_full_path(ops, oracle, c)


@pytest.mark.parametrize("nz", [False, True])
def test_quant_matmul_cfg4_prefill(ops, oracle, nz):
    """Full 4096x8192x8192 on the [K,N] weight and on its int8 NZ cast (the weight bench.py's headline line
    times): every quantized activation, scale and bf16 output bit-exact against the oracle, and the int32
    output (the raw accumulators) equal to the exact accumulator element for element."""
    c = W.CFG4
    say(f"quant_matmul cfg4 prefill 4096x8192x8192 (whole output) nz={nz}")
    xq, wd, acc_ref = _w8a8_full_path(ops, oracle, c, nz=nz)
    acc = ops.npu_quant_matmul(xq, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    assert np.array_equal(acc.cpu().numpy(), acc_ref)


@pytest.mark.parametrize("M,N,K,kn", [
    (512, 28672, 4096, True),    # cfg5 gate_up: 224 tiles of 256x256, no split
    (512, 4096, 14336, True),    # cfg5 down: 32 tiles, K split 8 ways (int32 partials + in-order reduce)
    (512, 4096, 14336, False),   # the same through an [N, K] weight view
    (512, 1024, 8192, True),     # 8 tiles, K split 16 ways
    (100, 2048, 4096, True),     # small M: 128-row stream tiles, K split
    (128, 4096, 4096, False),    # cfg1 shape through an [N, K] weight view
])
def test_quant_matmul_big_tiles_and_split_k(ops, oracle, M, N, K, kn):
    """Every int32 accumulator through exact row and column checksums; a row subset of the bf16
    output (per-token and per-channel scales, bf16 bias) bit-exact against the oracle."""
    say(f"quant_matmul M={M} N={N} K={K} {'[K,N]' if kn else '[N,K] view'}")
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    wd = w.to(DEV) if kn else w.t().contiguous().to(DEV).t()
    ad = a.to(DEV)
    acc = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    a64, w64, acc64 = a.to(torch.int64), w.to(torch.int64), acc.cpu().to(torch.int64)
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    b = torch.randn(N, generator=g).to(torch.bfloat16)
    out = ops.npu_quant_matmul(ad, wd, s.to(DEV), pertoken_scale=pt.to(DEV), bias=b.to(DEV),
                               output_dtype=torch.bfloat16)
    rows = np.r_[0:8, M - 8:M]
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(), pertoken=pt[rows].numpy(), bias=W.bits(b),
                              bias_dtype=BF16, out_dtype=BF16)
    assert np.array_equal(to_bits(out)[rows], ref)


@pytest.mark.parametrize("M,N,K,kn,out_dtype,bias_dtype", [
    (17, 64, 256, False, torch.bfloat16, torch.bfloat16),    # [N,K]: 16 x 64 blocks, one K stage, a 1-row last block
    (48, 4096, 512, False, torch.float16, torch.float32),    # 16-row blocks, [N,K] weight view
    (128, 4096, 4096, True, torch.bfloat16, torch.bfloat16),  # cfg1: 16 x 128 blocks ([K,N]), 16 K stages
    (200, 4096, 1024, True, torch.float32, torch.int32),     # 16 x 128 blocks, last block 8 rows
    (256, 2048, 768, False, torch.int8, torch.int32),        # 32-row blocks, 3 K stages (fewer than the ring)
    (96, 1024, 2304, True, torch.int32, None),               # 16-row blocks, 9 K stages
    (256, 4096, 512, True, torch.bfloat16, torch.bfloat16),  # [K,N]: 32 x 128 blocks
    (64, 192, 256, True, torch.float16, None),               # [K,N] with N % 128 != 0: 64-column blocks
    (64, 4096, 8192, True, torch.int8, torch.int32),         # [K,N]: 16 x 128 blocks, K split in two
    (1, 28672, 1024, False, torch.bfloat16, torch.bfloat16), # decode rows on an [N,K] weight: one row of 16
    (7, 4096, 2048, False, torch.float16, None),             # 7 of 16 rows
])
def test_quant_matmul_mid_m(ops, oracle, M, N, K, kn, out_dtype, bias_dtype):
    """M <= 256 with N % 64 == 0 and K % 256 == 0 (a [K,N] weight from M = 33): the no-split mid-M
    kernel (waves splitting each K stage, exact int32 reduction in LDS; for a [K,N] weight, with the L2
    prefetch wave).  Every int32 accumulator through exact row and column checksums;
    first, middle and last rows of the fused output bit-exact against the oracle."""
    say(f"quant_matmul mid-M M={M} N={N} K={K} {'[K,N]' if kn else '[N,K] view'} out={out_dtype} bias={bias_dtype}")
    g = torch.Generator().manual_seed(M * 3 + N + K)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    ad = a.to(DEV)
    wd = w.to(DEV) if kn else w.t().contiguous().to(DEV).t()
    acc = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    a64, w64, acc64 = a.to(torch.int64), w.to(torch.int64), acc.cpu().to(torch.int64)
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    integer_out = out_dtype in (torch.int8, torch.int32)
    s = (1e-4 + 1e-3 * torch.rand(N, generator=g)) if out_dtype is torch.int8 else 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    off = torch.randn(N, generator=g) if out_dtype is torch.int8 else None
    b = None
    if bias_dtype is torch.int32:
        b = torch.randint(-1000, 1000, (N,), generator=g, dtype=torch.int32)
    elif bias_dtype is not None:
        b = torch.randn(N, generator=g).to(bias_dtype)
    kw = dict(bias=None if b is None else b.to(DEV), output_dtype=out_dtype)
    if out_dtype is torch.int8:
        kw["offset"] = off.to(DEV)
    elif not integer_out:
        kw["pertoken_scale"] = pt.to(DEV)
    out = ops.npu_quant_matmul(ad, wd, s.to(DEV), **kw).cpu()
    rows = np.unique(np.clip(np.r_[0:4, M // 2 - 2:M // 2 + 2, M - 4:M], 0, M - 1))
    bias_np = None if b is None else (b.numpy() if b.dtype in (torch.int32, torch.float32) else W.bits(b))
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(),
                              pertoken=None if integer_out else pt[rows].numpy(),
                              offset=None if off is None else off.numpy(), bias=bias_np,
                              bias_dtype=CODE[b.dtype] if b is not None else BF16, out_dtype=CODE[out_dtype])
    got = out[rows]
    got_np = got.numpy() if out_dtype in (torch.float32, torch.int32, torch.int8) else W.bits(got)
    bad = np.argwhere(got_np != ref)
    assert bad.size == 0, (f"{len(bad)} mismatches, first at (row {rows[bad[0][0]]}, col {bad[0][1]}): "
                           f"{got_np[tuple(bad[0])]} vs {ref[tuple(bad[0])]}")


def test_quant_matmul_mid_m_against_split_plan(ops, plan):
    """The mid-M kernel and the split stream it replaced (debug override qmm_mid=0) give the same bf16 bits."""
    say("quant_matmul mid-M vs split stream, M=100 N=2048 K=4096")
    g = torch.Generator().manual_seed(11)
    M, N, K = 100, 2048, 4096
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(DEV)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8).to(DEV)
    s = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(DEV)
    pt = (1e-2 * torch.rand(M, generator=g)).to(DEV)
    b = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
    mid = ops.npu_quant_matmul(a, w, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
    plan("qmm_mid=0")
    split = ops.npu_quant_matmul(a, w, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
    assert torch.equal(mid.view(torch.int16), split.view(torch.int16))


def test_abi_quant_matmul_mid_m_split_workspace(ops, oracle):
    """M = 64 on a [K,N] weight plans a K split finished in-kernel (16 x 128 blocks, device-coherent partials
    and a tagged counter per tile in the workspace).  The ABI refuses a call without the queried workspace; on a
    0xFF-filled one every tile is finished once: bit-exact against the oracle on a row subset, and the same
    on a second call over the same workspace."""
    say("ABI qk_quant_matmul mid-M split, 0xFF workspace")
    L = ops.abi()
    M, N, K = 64, 4096, 4096
    n = ctypes.c_size_t(0)
    assert L.qk_quant_matmul_workspace_size(M, N, K, BF16, ctypes.byref(n)) == 0
    assert n.value > 0, "the [K,N] plan splits K"
    g = torch.Generator().manual_seed(13)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    b = torch.randn(N, generator=g).to(torch.bfloat16)
    ad, wd, sd, ptd, bd = a.to(DEV), w.to(DEV), s.to(DEV), pt.to(DEV), b.to(DEV)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    rc = L.qk_quant_matmul(ad.data_ptr(), K, wd.data_ptr(), N, 1, M, N, K, sd.data_ptr(), N, None, 0,
                           ptd.data_ptr(), bd.data_ptr(), BF16, out.data_ptr(), BF16, None, 0, _stream())
    assert rc != 0 and "workspace" in ops.last_error()
    wsbuf = torch.full((n.value,), 0xFF, dtype=torch.uint8, device=DEV)
    outs = []
    for rep in range(2):  # twice on the same workspace: the counters must be reusable
        out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
        rc = L.qk_quant_matmul(ad.data_ptr(), K, wd.data_ptr(), N, 1, M, N, K, sd.data_ptr(), N, None, 0,
                               ptd.data_ptr(), bd.data_ptr(), BF16, out.data_ptr(), BF16, wsbuf.data_ptr(),
                               n.value, _stream())
        assert rc == 0, ops.last_error()
        torch.cuda.synchronize()
        outs.append(out)
    rows = np.r_[0:4, 30:34, M - 4:M]
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(), pertoken=pt[rows].numpy(), bias=W.bits(b),
                              bias_dtype=BF16, out_dtype=BF16)
    assert np.array_equal(to_bits(outs[0])[rows], ref)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_abi_quant_matmul_mid_m_unaligned_rows(ops, oracle):
    """A mid-M shape whose x1 rows are not 16-byte aligned (lda = K + 8) cannot take the direct-to-LDS
    kernel: the library falls back to the tiled kernels (no workspace) with the same results."""
    say("ABI qk_quant_matmul mid-M, lda = K + 8")
    L = ops.abi()
    M, N, K = 64, 128, 512
    g = torch.Generator().manual_seed(12)
    a_wide = torch.randint(-127, 128, (M, K + 8), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    ad, wd, sd = a_wide.to(DEV), w.to(DEV), s.to(DEV)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    n = ctypes.c_size_t(0)
    assert L.qk_quant_matmul_workspace_size(M, N, K, BF16, ctypes.byref(n)) == 0
    wsbuf = torch.empty(max(n.value, 1), dtype=torch.uint8, device=DEV)
    rc = L.qk_quant_matmul(ad.data_ptr(), K + 8, wd.data_ptr(), N, 1, M, N, K, sd.data_ptr(), N, None, 0, None, None,
                           0, out.data_ptr(), BF16, wsbuf.data_ptr(), n.value, _stream())
    assert rc == 0, ops.last_error()
    torch.cuda.synchronize()
    ref = oracle.quant_matmul(a_wide[:, :K].contiguous().numpy(), w.numpy(), s.numpy(), out_dtype=BF16)
    assert np.array_equal(to_bits(out), ref)


@pytest.mark.parametrize("K,out_dtype,bias_dtype,kn", [
    (256, torch.bfloat16, torch.bfloat16, True),   # 192 whole 256x256 tiles, direct-to-LDS kernel (one ring)
    (256, torch.float16, torch.float32, False),
    (256, torch.float32, torch.int32, True),
    (512, torch.int32, None, False),
    (512, torch.int8, torch.int32, True),
    (384, torch.bfloat16, torch.bfloat16, True),   # K not a multiple of 256: register-staged kernel
    (384, torch.float16, None, False),
])
def test_quant_matmul_prefill_kernel_epilogues(ops, oracle, K, out_dtype, bias_dtype, kn):
    """Full-tile shapes with enough tiles to run unsplit: int32 checksums of every accumulator, and
    rows of each output dtype / bias dtype bit-exact against the oracle (both weight layouts)."""
    M, N = 512, 24576
    say(f"quant_matmul prefill tiles M={M} N={N} K={K} out={out_dtype} bias={bias_dtype} kn={kn}")
    g = torch.Generator().manual_seed(K + (7 if kn else 0))
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    ad = a.to(DEV)
    wd = w.to(DEV) if kn else w.t().contiguous().to(DEV).t()
    acc = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    a64, w64, acc64 = a.to(torch.int64), w.to(torch.int64), acc.cpu().to(torch.int64)
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    s = (1e-4 + 1e-3 * torch.rand(N, generator=g)) if out_dtype is torch.int8 else 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    off = torch.randn(N, generator=g) if out_dtype is torch.int8 else None
    b = None
    if bias_dtype is torch.int32:
        b = torch.randint(-1000, 1000, (N,), generator=g, dtype=torch.int32)
    elif bias_dtype is not None:
        b = torch.randn(N, generator=g).to(bias_dtype)
    kw = dict(bias=None if b is None else b.to(DEV), output_dtype=out_dtype)
    integer_out = out_dtype in (torch.int8, torch.int32)   # no per-token scale on integer outputs
    if out_dtype is torch.int8:
        kw["offset"] = off.to(DEV)
    elif not integer_out:
        kw["pertoken_scale"] = pt.to(DEV)
    out = ops.npu_quant_matmul(ad, wd, s.to(DEV), **kw).cpu()
    rows = np.r_[0:4, 250:262, M - 4:M]
    bias_np = None if b is None else (b.numpy() if b.dtype in (torch.int32, torch.float32) else W.bits(b))
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(),
                              pertoken=None if integer_out else pt[rows].numpy(),
                              offset=None if off is None else off.numpy(), bias=bias_np,
                              bias_dtype=CODE[b.dtype] if b is not None else BF16, out_dtype=CODE[out_dtype])
    got = out[rows]
    got_np = got.numpy() if out_dtype in (torch.float32, torch.int32, torch.int8) else W.bits(got)
    bad = np.argwhere(got_np != ref)
    assert bad.size == 0, (f"{len(bad)} mismatches, first at (row {rows[bad[0][0]]}, col {bad[0][1]}): "
                           f"{got_np[tuple(bad[0])]} vs {ref[tuple(bad[0])]}")


@pytest.mark.parametrize("M,N,K,kn,out_dtype,bias_dtype", [
    (300, 8192, 1024, True, torch.bfloat16, torch.bfloat16),  # 64 tiles, K split 2, last row tile 44 rows
    (1000, 8192, 4096, True, torch.bfloat16, torch.bfloat16), # 128 tiles, K split 2, last row tile 232 rows
    (257, 4096, 2048, True, torch.int8, torch.int32),         # 32 tiles, K split 4, one row in the last tile
    (600, 8192, 2048, False, torch.int32, None),              # [N,K] view, 96 tiles, K split 2
    (4000, 4096, 1024, False, torch.float16, torch.float32),  # [N,K] view, 256 tiles unsplit, 160-row last tile
    (3900, 8192, 512, True, torch.float32, torch.int32),      # 512 tiles unsplit (one ring), 60-row last tile
])
def test_quant_matmul_prefill_ragged_m(ops, oracle, M, N, K, kn, out_dtype, bias_dtype):
    """M not a multiple of 256 on the 256 x 256 direct-to-LDS kernel (rows past M load as zeros and are not
    stored), unsplit and with K splits: every int32 accumulator through exact row and column checksums, and
    the last row tile's rows (the ragged ones), with first and middle rows, bit-exact against the oracle."""
    say(f"quant_matmul ragged M={M} N={N} K={K} {'[K,N]' if kn else '[N,K] view'} out={out_dtype} bias={bias_dtype}")
    g = torch.Generator().manual_seed(M * 5 + N + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    ad = a.to(DEV)
    wd = w.to(DEV) if kn else w.t().contiguous().to(DEV).t()
    acc = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    a64, w64, acc64 = a.to(torch.int64), w.to(torch.int64), acc.cpu().to(torch.int64)
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    integer_out = out_dtype in (torch.int8, torch.int32)
    s = (1e-4 + 1e-3 * torch.rand(N, generator=g)) if out_dtype is torch.int8 else 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    off = torch.randn(N, generator=g) if out_dtype is torch.int8 else None
    b = None
    if bias_dtype is torch.int32:
        b = torch.randint(-1000, 1000, (N,), generator=g, dtype=torch.int32)
    elif bias_dtype is not None:
        b = torch.randn(N, generator=g).to(bias_dtype)
    kw = dict(bias=None if b is None else b.to(DEV), output_dtype=out_dtype)
    if out_dtype is torch.int8:
        kw["offset"] = off.to(DEV)
    elif not integer_out:
        kw["pertoken_scale"] = pt.to(DEV)
    out = ops.npu_quant_matmul(ad, wd, s.to(DEV), **kw).cpu()
    last = (M - 1) // 256 * 256
    rows = np.unique(np.r_[0:2, M // 2 - 1:M // 2 + 1, last:min(last + 4, M), max(last, M - 6):M])
    bias_np = None if b is None else (b.numpy() if b.dtype in (torch.int32, torch.float32) else W.bits(b))
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(),
                              pertoken=None if integer_out else pt[rows].numpy(),
                              offset=None if off is None else off.numpy(), bias=bias_np,
                              bias_dtype=CODE[b.dtype] if b is not None else BF16, out_dtype=CODE[out_dtype])
    got = out[rows]
    got_np = got.numpy() if out_dtype in (torch.float32, torch.int32, torch.int8) else W.bits(got)
    bad = np.argwhere(got_np != ref)
    assert bad.size == 0, (f"{len(bad)} mismatches, first at (row {rows[bad[0][0]]}, col {bad[0][1]}): "
                           f"{got_np[tuple(bad[0])]} vs {ref[tuple(bad[0])]}")


def test_quant_matmul_prefill_ragged_m_register_staged(ops, plan):
    """With the direct-to-LDS kernel switched off (debug override qmm_dma=0) a ragged M that the planner splits
    runs unsplit on the register-staged 256 x 256 kernel: the same bf16 bits as the split direct-to-LDS run."""
    say("quant_matmul ragged M=300 N=8192 K=1024, qmm_dma on vs off")
    g = torch.Generator().manual_seed(21)
    M, N, K = 300, 8192, 1024
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8).to(DEV)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8).to(DEV)
    s = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(DEV)
    pt = (1e-2 * torch.rand(M, generator=g)).to(DEV)
    b = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
    dma = ops.npu_quant_matmul(a, w, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
    plan("qmm_dma=0")
    reg = ops.npu_quant_matmul(a, w, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
    assert torch.equal(dma.view(torch.int16), reg.view(torch.int16))


@pytest.mark.parametrize("M", [1500, 2000])
@pytest.mark.parametrize("layout", ["kn", "nk", "nz"])
def test_quant_matmul_split_where_128_row_tiles_fill_the_cus(ops, oracle, M, layout):
    """N = K = 4096 with M = 1500 / 2000: 96 / 128 tiles of 256 rows (split in two), while 128-row tiles alone
    (192 / 256) would fill the CUs unsplit, which their split-only kernel does not run.  The 256-row split runs:
    exact int32 row and column checksums, a bf16 row subset bit-exact against the oracle, and no read past
    x's last row (the NZ launch once sized its 256-row grid by the 128-row tile count)."""
    N = K = 4096
    say(f"quant_matmul M={M} N={N} K={K} {layout}: 256-row split where 128-row tiles fill the CUs")
    g = torch.Generator().manual_seed(M + 17)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    wd = w.to(DEV)
    if layout == "nk":
        wd = w.t().contiguous().to(DEV).t()
    elif layout == "nz":
        wd = ops.npu_format_cast(wd, ops.ACL_FORMAT_FRACTAL_NZ)
    ad = a.to(DEV)
    acc = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
    a64, w64, acc64 = a.to(torch.int64), w.to(torch.int64), acc.cpu().to(torch.int64)
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    out = ops.npu_quant_matmul(ad, wd, s.to(DEV), pertoken_scale=pt.to(DEV), output_dtype=torch.bfloat16)
    rows = np.r_[0:8, M - 8:M]
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(), pertoken=pt[rows].numpy(), out_dtype=BF16)
    assert np.array_equal(to_bits(out)[rows], ref)


@pytest.mark.parametrize("M,N,K,nz,spec", [
    (128, 11008, 4096, False, ""),           # the cost model's 128-row K splits (4)
    (100, 11008, 4096, False, ""),           # the same with a ragged row tile (28 rows past M)
    (128, 4096, 14336, False, ""),           # a deep weight (8 splits)
    (64, 4096, 4096, False, "qmm_small=2"),  # forced: 2 splits, half a row tile
    (48, 4096, 8192, False, "qmm_small=8"),  # forced: 8 splits
    (128, 4096, 14336, True, ""),            # NZ blocks: the cost model's 8 splits
    (100, 11008, 4096, True, "qmm_small=4"), # NZ blocks, forced: 4 splits, a ragged row tile
])
def test_quant_matmul_small_m_split_tiles(ops, oracle, plan, M, N, K, nz, spec):
    """[K,N] and int8 NZ weights with 32 < M <= 128 on 128-row tiles with K splits (exact int32 partials, then
    the tiled reduce) where the cost model favours them over the mid-M kernel: every int32 accumulator passes
    exact row and column checksums, a row subset of the bf16 output (per-token and per-channel scales, bf16 bias)
    equals the oracle bit for bit, and both outputs equal the mid-M kernel's (qmm_small=0)."""
    say(f"quant_matmul small M on split tiles M={M} N={N} K={K} {'NZ' if nz else '[K,N]'} {spec or 'planner'}")
    g = torch.Generator().manual_seed(M + N + K + 1)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    ad, wd = a.to(DEV), w.to(DEV)
    if nz:
        wd = ops.npu_format_cast(wd, ops.ACL_FORMAT_FRACTAL_NZ)
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    b = torch.randn(N, generator=g).to(torch.bfloat16)
    outs = []
    for sp in (spec, "qmm_small=0"):
        plan(sp)
        acc = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
        out = ops.npu_quant_matmul(ad, wd, s.to(DEV), pertoken_scale=pt.to(DEV), bias=b.to(DEV),
                                   output_dtype=torch.bfloat16)
        outs.append((acc, out))
    a64, w64, acc64 = a.to(torch.int64), w.to(torch.int64), outs[0][0].cpu().to(torch.int64)
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    rows = np.r_[0:8, M - 8:M]
    ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(), pertoken=pt[rows].numpy(), bias=W.bits(b),
                              bias_dtype=BF16, out_dtype=BF16)
    assert np.array_equal(to_bits(outs[0][1])[rows], ref)
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1].view(torch.int16), outs[1][1].view(torch.int16))


@pytest.mark.parametrize("M,N,K", [(8192, 8192, 512), (2304, 8192, 1024), (4000, 8192, 512)])
@pytest.mark.parametrize("layout", ["kn", "nk", "nz"])
def test_quant_matmul_prefill_reverse_rounds(ops, plan, M, N, K, layout):
    """The direct-to-LDS prefill kernel walks K backwards in every other round of one workgroup per CU (1024
    tiles: four rounds; 288 tiles: one and a bit; M = 4000: two rounds, the last row tile 160 rows).  Every int32 accumulator passes exact row and column
    checksums, and the int32 and bf16 outputs equal those of the run with every round forwards (qmm_rev=0)."""
    say(f"quant_matmul M={M} N={N} K={K} {layout}, K backwards in odd rounds vs forwards")
    g = torch.Generator().manual_seed(M + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    wd = w.to(DEV)
    if layout == "nk":
        wd = w.t().contiguous().to(DEV).t()
    elif layout == "nz":
        wd = ops.npu_format_cast(wd, ops.ACL_FORMAT_FRACTAL_NZ)
    ad = a.to(DEV)
    s = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(DEV)
    pt = (1e-2 * torch.rand(M, generator=g)).to(DEV)
    outs = []
    for spec in ("", "qmm_rev=0"):
        plan(spec)
        acc = ops.npu_quant_matmul(ad, wd, torch.ones(1, device=DEV), output_dtype=torch.int32)
        out = ops.npu_quant_matmul(ad, wd, s, pertoken_scale=pt, output_dtype=torch.bfloat16)
        outs.append((acc, out))
    acc64 = outs[0][0].to(torch.int64)
    a64, w64 = a.to(torch.int64), w.to(torch.int64)
    assert torch.equal(acc64.sum(0).cpu(), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1).cpu(), a64 @ w64.sum(1))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1].view(torch.int16), outs[1][1].view(torch.int16))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bias_dtype", [None, torch.bfloat16, torch.float32, torch.int32])
@pytest.mark.parametrize("per_tensor", [False, True])
def test_quant_matmul_epilogue_variants(ops, oracle, out_dtype, bias_dtype, per_tensor):
    say(f"quant_matmul epilogue out={out_dtype} bias={bias_dtype} per_tensor={per_tensor}")
    g = torch.Generator().manual_seed(3)
    M, N, K = 48, 160, 320
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    s = 1e-3 + 9e-3 * torch.rand(1 if per_tensor else N, generator=g)
    pt = 1e-2 * torch.rand(M, generator=g)
    b = None
    if bias_dtype is torch.int32:
        b = torch.randint(-1000, 1000, (N,), generator=g, dtype=torch.int32)
    elif bias_dtype is not None:
        b = torch.randn(N, generator=g).to(bias_dtype)
    out = ops.npu_quant_matmul(a.to(DEV), w.to(DEV), s.to(DEV), pertoken_scale=pt.to(DEV),
                               bias=None if b is None else b.to(DEV), output_dtype=out_dtype)
    bias_np = None if b is None else (b.numpy() if b.dtype in (torch.int32, torch.float32) else W.bits(b))
    ref = oracle.quant_matmul(a.numpy(), w.numpy(), s.numpy(), pertoken=pt.numpy(), bias=bias_np,
                              bias_dtype=CODE[b.dtype] if b is not None else BF16, out_dtype=CODE[out_dtype])
    got = out.cpu()
    got_np = got.numpy() if out_dtype == torch.float32 else W.bits(got)
    assert np.array_equal(got_np, ref)


def test_quant_matmul_int8_output(ops, oracle):
    say("quant_matmul int8 output with offset and int32 bias")
    g = torch.Generator().manual_seed(4)
    M, N, K = 20, 64, 256
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
    s = 1e-4 + 1e-3 * torch.rand(N, generator=g)
    off = torch.randn(N, generator=g)
    b = torch.randint(-500, 500, (N,), generator=g, dtype=torch.int32)
    out = ops.npu_quant_matmul(a.to(DEV), w.to(DEV), s.to(DEV), offset=off.to(DEV), bias=b.to(DEV),
                               output_dtype=torch.int8)
    ref = oracle.quant_matmul(a.numpy(), w.numpy(), s.numpy(), offset=off.numpy(), bias=b.numpy(),
                              bias_dtype=I32, out_dtype=I8)
    assert np.array_equal(out.cpu().numpy(), ref)


def test_quant_matmul_batched_x1_and_transposed_weight(ops, oracle):
    say("quant_matmul 3-D x1, nn.Linear-layout weight")
    g = torch.Generator().manual_seed(5)
    a = torch.randint(-127, 128, (2, 24, 256), generator=g, dtype=torch.int8)
    w_nk = torch.randint(-127, 128, (192, 256), generator=g, dtype=torch.int8)
    s = 1e-3 + 9e-3 * torch.rand(192, generator=g)
    out = ops.npu_quant_matmul(a.to(DEV), w_nk.to(DEV).t(), s.to(DEV), output_dtype=torch.bfloat16)
    assert out.shape == (2, 24, 192)
    ref = oracle.quant_matmul(a.reshape(48, 256).numpy(), w_nk.t().numpy(), s.numpy(), out_dtype=BF16)
    assert np.array_equal(to_bits(out).reshape(48, 192), ref)


def test_quant_matmul_errors(ops):
    say("quant_matmul argument errors")
    a = torch.zeros((4, 64), dtype=torch.int8, device=DEV)
    w = torch.zeros((64, 32), dtype=torch.int8, device=DEV)
    with pytest.raises(RuntimeError, match="must equal"):
        ops.npu_quant_matmul(a, w[:32], torch.ones(32, device=DEV), output_dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="scale must be"):
        ops.npu_quant_matmul(a, w, torch.ones(7, device=DEV), output_dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="int8"):
        ops.npu_quant_matmul(a.float(), w, torch.ones(32, device=DEV))


# ----------------------------------------------------------------------------- npu_weight_quant_batchmatmul

def _w4_ref(oracle, d, group, bias=None, x_dtype=torch.bfloat16, s_dtype=torch.float16):
    return oracle.weight_quant_bmm(W.bits(d["x"]), CODE[x_dtype], d["w_packed"].numpy(), W.bits(d["scale"]),
                                   None if d["offset"] is None else W.bits(d["offset"]), CODE[s_dtype], group,
                                   bias=None if bias is None else W.bits(bias), bias_dtype=CODE.get(
                                       None if bias is None else bias.dtype, BF16),
                                   out_dtype=CODE[x_dtype])


def _w4_run(ops, d, group, bias=None):
    return ops.npu_weight_quant_batchmatmul(
        d["x"].to(DEV), d["w_packed"].to(DEV), d["scale"].to(DEV),
        None if d["offset"] is None else d["offset"].to(DEV), bias=None if bias is None else bias.to(DEV),
        antiquant_group_size=group)


def test_w4a16_cfg3_decode(ops, oracle):
    c = W.CFG3[0]
    say(f"w4a16 cfg3 M={c.M} 4096x11008")
    d = W.w4a16_inputs(c)
    out = _w4_run(ops, d, 128)
    bf16_close(to_bits(out), _w4_ref(oracle, d, 128))


def test_w4a16_cfg3_prefill(ops, oracle):
    """cfg3 M=2048, every output element within rtol/atol 1e-2 of the float64 dequant-matmul (pinned against
    the C oracle on a row subset here)."""
    c = W.CFG3[1]
    say(f"w4a16 cfg3 M={c.M} 4096x11008 (whole output)")
    d = W.w4a16_inputs(c)
    out = _w4_run(ops, d, 128)
    ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], 128)
    rows = np.r_[0:4, 2044:2048]
    pin = _w4_ref(oracle, dict(d, x=d["x"][rows]), 128)
    pin_diff = (W.from_bits(pin, torch.bfloat16).float() - ref64[rows].float()).abs()
    assert pin_diff.max().item() <= 2.0**-7 * ref64[rows].abs().max().item()
    torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype", [
    (1, 64, 128, 128, True, torch.bfloat16),
    (3, 136, 256, 32, True, torch.bfloat16),
    (16, 256, 512, 64, False, torch.bfloat16),
    (17, 128, 384, 128, True, torch.float16),
    (40, 200, 256, 0, True, torch.bfloat16),
    (5, 24, 96, 0, False, torch.float16),
    (2, 16, 100, 0, True, torch.bfloat16),       # K % 32 != 0: generic kernel
    (16, 1024, 4160, 64, True, torch.bfloat16),  # K % 256 != 0: no decode kernel; the register-staged prefill kernel
    (3, 512, 320, 64, False, torch.float16),
    # stream kernel (M <= 16, K a multiple of 512): ragged strips, clamped rows, every group size
    (7, 1000, 1024, 32, True, torch.float16),
    (16, 520, 2048, 64, True, torch.bfloat16),
    (9, 4096, 4096, 0, True, torch.bfloat16),
    (2, 8, 512, 128, False, torch.float16),
    (1, 11008, 4096, 128, True, torch.bfloat16),
    (13, 2056, 1536, 256, True, torch.float16),
    # past 256 rows a row-major weight is cast to NZ in the workspace when the NZ prefill kernel takes the shape
    (300, 8192, 1024, 128, True, torch.bfloat16),
])
def test_w4a16_shapes(ops, oracle, M, N, K, group, offset, x_dtype):
    say(f"w4a16 M={M} N={N} K={K} group={group} offset={offset} {x_dtype}")
    case = W.W4A16Case(M=M, N=N, K=K, group=group, x_dtype=x_dtype, offset=offset)
    d = W.w4a16_inputs(case, seed=M + N + K)
    if x_dtype == torch.float16:
        d = dict(d, scale=d["scale"], offset=d["offset"])
    if group == 0:
        d = dict(d, scale=d["scale"].reshape(-1), offset=None if d["offset"] is None else d["offset"].reshape(-1))
    b = torch.randn(N).to(x_dtype)
    out = _w4_run(ops, d, group, bias=b)
    ref = _w4_ref(oracle, d, group, bias=b, x_dtype=x_dtype)
    bf16_close(to_bits(out), ref, dtype=x_dtype)


def test_int4_pack_device(ops, oracle):
    say("npu_convert_weight_to_int4pack")
    g = torch.Generator().manual_seed(8)
    w = torch.randint(-8, 8, (64, 96), generator=g, dtype=torch.int32)
    p = ops.npu_convert_weight_to_int4pack(w.to(DEV))
    assert np.array_equal(p.cpu().numpy(), oracle.int4_pack(w.numpy().astype(np.int8)))


# ----------------------------------------------------------------------------- through the C ABI

def _stream():
    return torch.cuda.current_stream().cuda_stream


def test_abi_quant_matmul_matches_op(ops, oracle):
    """Drive qk_quant_matmul directly with device pointers (the drop-in boundary)."""
    say("ABI qk_quant_matmul")
    L = ops.abi()
    g = torch.Generator().manual_seed(12)
    M, N, K = 32, 256, 512
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(DEV)
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8).to(DEV)
    s = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(DEV)
    pt = (1e-2 * torch.rand(M, generator=g)).to(DEV)
    b = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    import ctypes
    ws = ctypes.c_size_t(0)
    assert L.qk_quant_matmul_workspace_size(M, N, K, BF16, ctypes.byref(ws)) == 0
    wsbuf = torch.zeros(max(1, ws.value), dtype=torch.uint8, device=DEV)   # split-K counters start at zero
    rc = L.qk_quant_matmul(a.data_ptr(), K, w.data_ptr(), N, 1, M, N, K, s.data_ptr(), N, None, 0, pt.data_ptr(),
                           b.data_ptr(), BF16, out.data_ptr(), BF16, wsbuf.data_ptr(), ws.value, _stream())
    assert rc == 0, ops.last_error()
    ref = ops.npu_quant_matmul(a, w, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    # a bad stride pair is refused with a message, nothing launched
    rc = L.qk_quant_matmul(a.data_ptr(), K, w.data_ptr(), 2, 2, M, N, K, s.data_ptr(), N, None, 0, None, None, 0,
                           out.data_ptr(), BF16, None, 0, _stream())
    assert rc == -1 and "transposed view" in ops.last_error()


@pytest.mark.parametrize("cfg", ["16:4:2", "16:4:4", "8:4:2", "8:4:4", "8:8:2", "8:8:3"])
def test_w4a16_stream_configs(ops, oracle, plan, cfg):
    """Every wave count / K-blocks per wave / prefetch depth of the decode stream kernel (forced through the
    planner override)."""
    plan(f"w4_stream={cfg}")
    for (M, N, K, group) in [(5, 1096, 2048, 128), (16, 264, 4096, 32)]:
        say(f"w4a16 stream cfg={cfg} M={M} N={N} K={K} group={group}")
        case = W.W4A16Case(M=M, N=N, K=K, group=group, x_dtype=torch.bfloat16, offset=True)
        d = W.w4a16_inputs(case, seed=7 * M + K)
        b = torch.randn(N).to(torch.bfloat16)
        out = _w4_run(ops, d, group, bias=b)
        bf16_close(to_bits(out), _w4_ref(oracle, d, group, bias=b))


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (16, 11008, 4096, 128, True, torch.bfloat16, False),   # cfg3 decode: 43 strips x 4 K splits
    (5, 1104, 2048, 128, True, torch.float16, True),       # last strip of 80 columns (10 words), 2 splits
    (9, 272, 1024, 0, False, torch.bfloat16, True),        # per channel, one split, last strip of 16 columns
    (16, 1096, 2048, 128, True, torch.bfloat16, False),    # N % 16 != 0: the half-line strips run instead
])
def test_w4a16_stream_whole_line(ops, oracle, plan, M, N, K, group, offset, x_dtype, bias):
    """The decode stream with whole 128-byte weight rows per wave (8-wave strips, each lane two adjacent
    packed words: the plan for M > 4 and N % 16 == 0): within rtol/atol 1e-2 of the oracle, and bit for bit
    the half-line strips' output (the same K ranges, folded in the same order)."""
    say(f"w4a16 whole-line stream M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    case = W.W4A16Case(M=M, N=N, K=K, group=group, x_dtype=x_dtype, offset=offset)
    d = W.w4a16_inputs(case, seed=3 * M + N)
    if group == 0:
        d = dict(d, scale=d["scale"].reshape(-1), offset=None if d["offset"] is None else d["offset"].reshape(-1))
    b = torch.randn(N).to(x_dtype) if bias else None
    out = _w4_run(ops, d, group, bias=b)
    plan("w4_stream_wpl=16")
    half = _w4_run(ops, d, group, bias=b)
    plan("")
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), half.view(torch.int16))
    bf16_close(to_bits(out), _w4_ref(oracle, d, group, bias=b, x_dtype=x_dtype), dtype=x_dtype)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (16, 11008, 4096, 128, True, torch.bfloat16, False),   # cfg3's shape: whole rows, 43 strips x 4 K splits
    (1, 1040, 2048, 128, True, torch.float16, True),       # whole rows, last strip of 16 columns, 2 splits
    (7, 1032, 1024, 128, False, torch.bfloat16, True),     # N % 16 == 8: half rows, last strip of 8 columns
    (4, 24576, 8192, 128, True, torch.bfloat16, False),    # 768 workgroups of whole rows: half rows instead
    (5, 1036, 2048, 128, True, torch.bfloat16, False),     # N % 8 == 4: quarter rows (16-wave strips)
])
def test_w8a16_stream_row_widths(ops, oracle, plan, M, N, K, group, offset, x_dtype, bias):
    """The int8 decode stream on a row-major [K, N] weight with 4 (whole 256-byte rows per wave), 2 (half rows)
    or 1 (quarter rows) dwords per lane, as planned for the shape: within rtol/atol 1e-2 of the oracle; and every
    row width forced on the shape (where it applies) within the same bar."""
    say(f"w8a16 stream row widths M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn((M, K), generator=g).to(x_dtype)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    sc = (5e-4 + 2.5e-3 * torch.rand((K // group, N), generator=g)).to(torch.float16)
    off = (8 * torch.rand((K // group, N), generator=g) - 4).to(torch.float16) if offset else None
    b = torch.randn(N, generator=g).to(x_dtype) if bias else None
    ref = oracle.weight_quant_bmm(W.bits(x), CODE[x_dtype], w.numpy(), W.bits(sc),
                                  None if off is None else W.bits(off), F16, group,
                                  bias=None if b is None else W.bits(b), bias_dtype=CODE[x_dtype],
                                  out_dtype=CODE[x_dtype])
    args = (x.to(DEV), w.to(DEV), sc.to(DEV), None if off is None else off.to(DEV))
    for spec in ("", "w4_stream_wpl=16", "w4_stream_wpl=32", "w4_stream_wpl=64"):
        plan(spec)
        out = ops.npu_weight_quant_batchmatmul(*args, bias=None if b is None else b.to(DEV), antiquant_group_size=group)
        bf16_close(to_bits(out), ref, dtype=x_dtype)
    plan("")


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype", [
    (300, 520, 512, 128, True, torch.bfloat16),     # ragged M and N
    (256, 256, 256, 64, False, torch.float16),      # full tiles
    (512, 1024, 1024, 32, True, torch.bfloat16),    # full tiles, 32-row groups
    (70, 136, 64, 0, True, torch.bfloat16),         # one K stage, per-channel scale
    (260, 264, 2048, 0, False, torch.float16),      # per-channel over a long K
    # whole tiles and groups of whole 64-row stages: the DMA pipeline
    (256, 128, 64, 64, True, torch.bfloat16),       # a single stage (no full triple of stages)
    (512, 256, 320, 64, True, torch.float16),       # five stages (two after the last triple)
    (256, 384, 1024, 0, True, torch.bfloat16),      # per-channel scale, 16 stages per group
    (768, 640, 512, 256, False, torch.bfloat16),    # 256-row groups, several tile rows
])
def test_w4a16_prefill_kernel(ops, oracle, plan, M, N, K, group, offset, x_dtype):
    """The large-M kernels (exact int4 MFMA operands + group fold), forced onto small shapes."""
    plan("w4_gemm=force")
    say(f"w4a16 prefill kernel M={M} N={N} K={K} group={group} offset={offset} {x_dtype}")
    case = W.W4A16Case(M=M, N=N, K=K, group=group, x_dtype=x_dtype, offset=offset)
    d = W.w4a16_inputs(case, seed=M + 3 * N + K)
    if group == 0:
        d = dict(d, scale=d["scale"].reshape(-1), offset=None if d["offset"] is None else d["offset"].reshape(-1))
    b = torch.randn(N).to(x_dtype)
    out = _w4_run(ops, d, group, bias=b)
    bf16_close(to_bits(out), _w4_ref(oracle, d, group, bias=b, x_dtype=x_dtype), dtype=x_dtype)


def test_w4a16_prefill_dma_sweep(ops, oracle, plan):
    """Seeded random whole-tile shapes through the DMA prefill kernel (int4 and int8 weights, fp16 and bf16,
    group sizes 64..K, with and without offset and bias), each against the oracle on a row sample."""
    plan("w4_gemm=force")
    rng = np.random.default_rng(2024)
    for t in range(10):
        M = 256 * int(rng.integers(1, 4))
        N = 128 * int(rng.integers(1, 9))
        K = 64 * int(rng.integers(1, 33))
        gs = [g for g in (64, 128, 192, 256, 512) if K % g == 0] + [0]
        group = int(rng.choice(gs))
        x_dtype = torch.bfloat16 if t % 2 == 0 else torch.float16
        offset = bool(t % 3)
        w8 = t % 4 == 3
        say(f"w4a16 dma sweep {t}: M={M} N={N} K={K} group={group} offset={offset} {x_dtype} int8={w8}")
        b = torch.randn(N).to(x_dtype) if t % 2 else None
        rows = np.r_[0:8, M - 8:M]
        if w8:
            d = _w8_inputs(M, N, K, group, offset, x_dtype, seed=100 + t)
            out = ops.npu_weight_quant_batchmatmul(d["x"].to(DEV), d["w"].to(DEV), d["scale"].to(DEV),
                                                   None if d["offset"] is None else d["offset"].to(DEV),
                                                   bias=None if b is None else b.to(DEV), antiquant_group_size=group)
            ref = oracle.weight_quant_bmm(W.bits(d["x"][rows]), CODE[x_dtype], d["w"].numpy(), W.bits(d["scale"]),
                                          None if d["offset"] is None else W.bits(d["offset"]), F16, group,
                                          bias=None if b is None else W.bits(b), bias_dtype=CODE[x_dtype],
                                          out_dtype=CODE[x_dtype])
        else:
            case = W.W4A16Case(M=M, N=N, K=K, group=group, x_dtype=x_dtype, offset=offset)
            d = W.w4a16_inputs(case, seed=100 + t)
            if group == 0:
                d = dict(d, scale=d["scale"].reshape(-1),
                         offset=None if d["offset"] is None else d["offset"].reshape(-1))
            out = _w4_run(ops, d, group, bias=b)
            ref = _w4_ref(oracle, dict(d, x=d["x"][rows]), group, bias=b, x_dtype=x_dtype)
        bf16_close(to_bits(out)[rows], ref, dtype=x_dtype)


@pytest.mark.parametrize("mode", ["dma", "nodma"])
def test_w4a16_prefill_pipelines(ops, oracle, plan, mode):
    """Both prefill pipelines on one whole-tile shape with 128 tiles: the DMA kernel (default, group sums
    from the pre-pass) and the register-staged kernel (w4_gemm=nodma), each against the oracle."""
    if mode == "nodma":
        plan("w4_gemm=nodma")
    M, N, K, group = 2048, 2048, 384, 128
    say(f"w4a16 prefill {mode} M={M} N={N} K={K} group={group}")
    case = W.W4A16Case(M=M, N=N, K=K, group=group, x_dtype=torch.bfloat16, offset=True)
    d = W.w4a16_inputs(case, seed=31)
    b = torch.randn(N).to(torch.bfloat16)
    out = _w4_run(ops, d, group, bias=b)
    rows = np.r_[0:8, 700:708, 2040:2048]
    sub = dict(d, x=d["x"][rows])
    bf16_close(to_bits(out)[rows], _w4_ref(oracle, sub, group, bias=b))


# ----------------------------------------------------------------------------- W8A16 (int8 weights)

def _w8_inputs(M, N, K, group, offset, x_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g).to(x_dtype)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    ng = K // group if group > 0 else 1
    scale = (5e-4 + 2.5e-3 * torch.rand((ng, N), generator=g)).to(torch.float16)
    off = (8 * torch.rand((ng, N), generator=g) - 4).to(torch.float16) if offset else None
    if group == 0:
        scale = scale.reshape(-1)
        off = None if off is None else off.reshape(-1)
    return dict(x=x, w=w, scale=scale, offset=off)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,force", [
    (16, 11008, 4096, 128, True, torch.bfloat16, None),   # decode weight stream, the cfg3 shape with int8 weights
    (1, 4096, 4096, 128, True, torch.float16, None),
    (7, 2048, 1024, 64, False, torch.bfloat16, None),
    (16, 1024, 2048, 32, True, torch.float16, None),
    (16, 768, 512, 0, True, torch.bfloat16, None),        # per-channel scales
    (300, 512, 512, 128, True, torch.bfloat16, "force"),   # prefill kernel, ragged M
    (256, 384, 256, 64, False, torch.float16, "force"),
    (2048, 11008, 4096, 128, True, torch.bfloat16, None),  # prefill at the cfg3 shape (row subset)
    (5, 24, 96, 0, True, torch.bfloat16, None),            # generic kernel
    (40, 4096, 2048, 128, True, torch.bfloat16, None),     # 16 < M <= 128: the decode stream on 16-row slices
    (128, 2048, 1024, 64, False, torch.float16, None),     # eight slices (64-row groups: no NZ decode plan)
    (100, 4096, 2048, 128, True, torch.bfloat16, None),    # 64 < M <= 128: cast to NZ, NZ decode on two row chunks
    (200, 8192, 1024, 128, True, torch.bfloat16, None),    # M > 128: cast to NZ, NZ prefill kernel
    (200, 2048, 1024, 128, True, torch.bfloat16, None),    # too few NZ prefill tiles: cast, NZ decode on row chunks
    (300, 2048, 1024, 128, True, torch.bfloat16, None),    # M > 256 with too few NZ tiles: the register-staged kernel
])
def test_w8a16(ops, oracle, plan, M, N, K, group, offset, x_dtype, force):
    """npu_weight_quant_batchmatmul with int8 weights [K, N] (W8A16) against the float64 oracle."""
    if force:
        plan(f"w4_gemm={force}")
    say(f"w8a16 M={M} N={N} K={K} group={group} offset={offset} {x_dtype} {force or ''}")
    d = _w8_inputs(M, N, K, group, offset, x_dtype, seed=M + 5 * N + K)
    b = torch.randn(N).to(x_dtype)
    out = ops.npu_weight_quant_batchmatmul(d["x"].to(DEV), d["w"].to(DEV), d["scale"].to(DEV),
                                           None if d["offset"] is None else d["offset"].to(DEV), bias=b.to(DEV),
                                           antiquant_group_size=group)
    if M > 300:   # the whole output against the float64 dequant-matmul, pinned to the oracle on 8 rows
        ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], group, bias=b)
        torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)
    rows = np.arange(M) if M <= 300 else np.r_[0:4, M - 4:M]
    ref = oracle.weight_quant_bmm(W.bits(d["x"][rows]), CODE[x_dtype], d["w"].numpy(), W.bits(d["scale"]),
                                  None if d["offset"] is None else W.bits(d["offset"]), F16, group,
                                  bias=W.bits(b), bias_dtype=CODE[x_dtype], out_dtype=CODE[x_dtype])
    bf16_close(to_bits(out)[rows], ref, dtype=x_dtype)


def test_abi_dynamic_quant_and_w4a16(ops, oracle):
    say("ABI qk_dynamic_quant / qk_weight_quant_bmm")
    L = ops.abi()
    g = torch.Generator().manual_seed(13)
    x = torch.randn((8, 1024), generator=g).to(torch.float16).to(DEV)
    y = torch.empty((8, 1024), dtype=torch.int8, device=DEV)
    s = torch.empty(8, dtype=torch.float32, device=DEV)
    assert L.qk_dynamic_quant(x.data_ptr(), F16, 8, 1024, None, y.data_ptr(), s.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    ry, rs = oracle.dynamic_quant(W.bits(x.cpu()), F16)
    assert np.array_equal(y.cpu().numpy(), ry) and np.array_equal(s.cpu().numpy(), rs)

    case = W.W4A16Case(M=4, N=128, K=256)
    d = W.w4a16_inputs(case, seed=1)
    xd, wd, sd, od = (d[k].to(DEV) for k in ("x", "w_packed", "scale", "offset"))
    out = torch.empty((4, 128), dtype=torch.bfloat16, device=DEV)
    rc = L.qk_weight_quant_bmm(xd.data_ptr(), BF16, wd.data_ptr(), I32, sd.data_ptr(), od.data_ptr(), F16, 4, 128,
                               256, 128, None, 0, out.data_ptr(), BF16, None, 0, _stream())
    assert rc == 0, ops.last_error()
    torch.cuda.synchronize()
    bf16_close(to_bits(out), _w4_ref(oracle, d, 128))


def _fill(buf, how, seed=0):
    if how == "zeros":
        buf.zero_()
    elif how == "ff":
        buf.fill_(0xFF)
    elif how == "random":
        g = torch.Generator(device=buf.device).manual_seed(seed)
        buf.copy_(torch.randint(0, 256, buf.shape, generator=g, device=buf.device, dtype=torch.int32).to(torch.uint8))
    # "empty": whatever the caching allocator hands out


@pytest.mark.parametrize("how", ["zeros", "ff", "random", "empty"])
def test_abi_split_workspace_any_contents(ops, oracle, how):
    """Split-K calls through the ABI on a workspace of arbitrary contents, as EXEC_NPU_CMD hands out
    fresh uninitialised scratch (op_plugin/utils/op_api_common.h:547-551): zero-, 0xFF- and randomly filled
    and uninitialised, one workspace reused by several split shapes in a row (cfg3 M=16 twice, W4A16 at
    M=5 and M=1, W8A16 at M=16), every result against the oracle."""
    say(f"ABI qk_weight_quant_bmm split workspace ({how})")
    import ctypes
    L = ops.abi()
    cases = [(W.W4A16Case(M=16, N=11008, K=4096), I32), (W.W4A16Case(M=5, N=2048, K=2048), I32),
             (W.W4A16Case(M=1, N=4096, K=8192), I32), (W.W4A16Case(M=16, N=4096, K=4096), I8),
             (W.W4A16Case(M=16, N=11008, K=4096), I32)]
    need = []
    for c, wdt in cases:
        n = ctypes.c_size_t(0)
        assert L.qk_weight_quant_bmm_workspace_size(c.M, c.N, c.K, wdt, 128, ctypes.byref(n)) == 0
        need.append(n.value)
    assert min(need) > 0, "the shapes must split K"
    wsbuf = torch.empty(max(need), dtype=torch.uint8, device=DEV)
    _fill(wsbuf, how, seed=5)
    for i, (c, wdt) in enumerate(cases):
        say(f"  M={c.M} N={c.N} K={c.K} weight={'int4' if wdt == I32 else 'int8'}")
        if wdt == I32:
            d = W.w4a16_inputs(c, seed=20 + i)
            wt = d["w_packed"]
        else:
            d = _w8_inputs(c.M, c.N, c.K, 128, True, torch.bfloat16, seed=20 + i)
            wt = d["w"]
        xd, wd, sd, od = d["x"].to(DEV), wt.to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
        out = torch.empty((c.M, c.N), dtype=torch.bfloat16, device=DEV)
        rc = L.qk_weight_quant_bmm(xd.data_ptr(), BF16, wd.data_ptr(), wdt, sd.data_ptr(), od.data_ptr(), F16, c.M,
                                   c.N, c.K, 128, None, 0, out.data_ptr(), BF16, wsbuf.data_ptr(), wsbuf.numel(),
                                   _stream())
        assert rc == 0, ops.last_error()
        torch.cuda.synchronize()
        ref = oracle.weight_quant_bmm(W.bits(d["x"]), BF16, wt.numpy(), W.bits(d["scale"]), W.bits(d["offset"]),
                                      F16, 128, out_dtype=BF16)
        bf16_close(to_bits(out), ref)


def test_weight_quant_op_workspace_is_uninitialised_scratch(ops, oracle):
    """The torch op takes a fresh uninitialised workspace per call from the caching allocator; a block that
    previously held 0xFF bytes must not disturb the split-K decode (the allocator hands the freed block back)."""
    say("npu_weight_quant_batchmatmul on recycled 0xFF scratch")
    c = W.CFG3[0]
    d = W.w4a16_inputs(c, seed=3)
    ref = _w4_ref(oracle, d, 128)
    import ctypes
    n = ctypes.c_size_t(0)
    assert ops.abi().qk_weight_quant_bmm_workspace_size(c.M, c.N, c.K, I32, 128, ctypes.byref(n)) == 0
    for rep in range(3):
        junk = torch.full((n.value,), 0xFF, dtype=torch.uint8, device=DEV)
        del junk                                   # the next same-size allocation on this stream reuses it
        out = _w4_run(ops, d, 128)
        bf16_close(to_bits(out), ref)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.int8, torch.int32])
def test_quant_matmul_k_zero(ops, oracle, out_dtype):
    """K = 0: every accumulator is 0, so the output is the epilogue of 0 (plus bias)."""
    say(f"quant_matmul K=0 out={out_dtype}")
    M, N = 6, 40
    g = torch.Generator().manual_seed(9)
    a = torch.empty((2, 3, 0), dtype=torch.int8)
    w = torch.empty((0, N), dtype=torch.int8)
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    kw = dict(output_dtype=out_dtype)
    if out_dtype is torch.bfloat16:
        b = torch.randn(N, generator=g).to(torch.bfloat16)
        pt = torch.rand(M, generator=g)
        kw.update(bias=b.to(DEV), pertoken_scale=pt.to(DEV))
        ref = oracle.quant_matmul_epilogue(np.zeros((M, N), np.int32), s.numpy(), pertoken=pt.numpy(),
                                           bias=W.bits(b), bias_dtype=BF16, out_dtype=BF16)
    elif out_dtype is torch.int8:
        off = 3 * torch.randn(N, generator=g)
        kw.update(offset=off.to(DEV))
        ref = oracle.quant_matmul_epilogue(np.zeros((M, N), np.int32), s.numpy(), offset=off.numpy(), out_dtype=I8)
    else:
        b = torch.randint(-1000, 1000, (N,), generator=g, dtype=torch.int32)
        kw.update(bias=b.to(DEV))
        ref = oracle.quant_matmul_epilogue(np.zeros((M, N), np.int32), np.ones(1, np.float32), bias=b.numpy(),
                                           bias_dtype=I32, out_dtype=I32)
    out = ops.npu_quant_matmul(a.to(DEV), w.to(DEV), s.to(DEV), **kw)
    assert out.shape == (2, 3, N)
    got = out.cpu().reshape(M, N)
    got_np = W.bits(got) if out_dtype is torch.bfloat16 else got.numpy()
    assert np.array_equal(got_np, ref)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("group", [0, 128])
def test_weight_quant_k_zero(ops, oracle, bias, group):
    """K = 0: the sum over K is empty, so the output is the bias (or zero)."""
    say(f"weight_quant_batchmatmul K=0 group={group} bias={bias}")
    M, N = 3, 64
    x = torch.empty((M, 0), dtype=torch.bfloat16, device=DEV)
    w = torch.empty((0, N // 8), dtype=torch.int32, device=DEV)
    sc = torch.ones((N,) if group == 0 else (0, N), dtype=torch.float16, device=DEV)
    b = torch.randn(N).to(torch.bfloat16) if bias else None
    out = ops.npu_weight_quant_batchmatmul(x, w, sc, bias=None if b is None else b.to(DEV),
                                           antiquant_group_size=group)
    want = (b.float() if bias else torch.zeros(N)).to(torch.bfloat16).expand(M, N)
    assert torch.equal(out.cpu().view(torch.int16), want.contiguous().view(torch.int16))


def test_abi_w8a8_split_workspace_reuse(ops, oracle):
    """W8A8 split-K calls through the ABI (skinny stream and 256x256 tiles with int32 partials and the
    split reduce): one 0xFF-filled workspace reused by calls of different shapes and output types, each
    result against the oracle (int32 fully through checksums, 16-bit and int8 on a row subset)."""
    say("ABI qk_quant_matmul split workspace reuse")
    import ctypes
    L = ops.abi()
    cases = [(16, 4096, 8192, BF16), (512, 4096, 14336, BF16), (16, 2048, 4096, I8), (512, 1024, 8192, I32),
             (16, 4096, 8192, F16)]
    need = []
    for (M, N, K, od) in cases:
        n = ctypes.c_size_t(0)
        assert L.qk_quant_matmul_workspace_size(M, N, K, od, ctypes.byref(n)) == 0
        need.append(n.value)
    assert min(need) > 0, "every shape must split K"
    wsbuf = torch.full((max(need),), 0xFF, dtype=torch.uint8, device=DEV)
    tdt = {BF16: torch.bfloat16, F16: torch.float16, I8: torch.int8, I32: torch.int32}
    for ci, (M, N, K, od) in enumerate(cases):
        say(f"  M={M} N={N} K={K} out={od}")
        g = torch.Generator().manual_seed(40 + ci)
        a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
        s = 1e-4 + 1e-3 * torch.rand(N, generator=g) if od == I8 else 1e-3 + 9e-3 * torch.rand(N, generator=g)
        off = torch.randn(N, generator=g) if od == I8 else None
        pt = 1e-2 * torch.rand(M, generator=g) if od in (BF16, F16) else None
        b = torch.randint(-500, 500, (N,), generator=g, dtype=torch.int32) if od in (I8, I32) else \
            torch.randn(N, generator=g).to(torch.bfloat16)
        bdt = I32 if od in (I8, I32) else BF16
        if od == I32:
            s = torch.ones(1)
        ad, wd, sd, bd = a.to(DEV), w.to(DEV), s.to(DEV), b.to(DEV)
        offd = off.to(DEV) if off is not None else None
        ptd = pt.to(DEV) if pt is not None else None
        out = torch.empty((M, N), dtype=tdt[od], device=DEV)
        rc = L.qk_quant_matmul(ad.data_ptr(), K, wd.data_ptr(), N, 1, M, N, K, sd.data_ptr(), sd.numel(),
                               offd.data_ptr() if offd is not None else None, N if offd is not None else 0,
                               ptd.data_ptr() if ptd is not None else None, bd.data_ptr(), bdt, out.data_ptr(), od,
                               wsbuf.data_ptr(), wsbuf.numel(), _stream())
        assert rc == 0, ops.last_error()
        torch.cuda.synchronize()
        if od == I32:
            a64, w64 = a.to(torch.int64), w.to(torch.int64)
            acc64 = out.cpu().to(torch.int64) - b.to(torch.int64)
            assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
            assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
            continue
        rows = np.r_[0:8, M - 8:M]
        ref = oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(),
                                  offset=off.numpy() if off is not None else None,
                                  pertoken=pt[rows].numpy() if pt is not None else None,
                                  bias=b.numpy() if bdt == I32 else W.bits(b), bias_dtype=bdt, out_dtype=od)
        got = out.cpu().numpy()[rows] if od == I8 else to_bits(out)[rows]
        assert np.array_equal(got, ref)
