"""GPU parity of npu_quant_matmul (W8A8) on int8 weights in the NZ layout.

The weight is cast once with npu_format_cast(w, 29) (int8 [N/16, K/64, 64, 16]), as the reference casts
matmul weights to FRACTAL_NZ before its matmuls (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:303-316).
Every case checks the NZ call:
* bit for bit against the same call on the row-major weight (the path the other parity tests pin);
* its exact int32 accumulators through row and column checksums against int64 sums on the CPU;
* the fused output bit-exact against the oracle on first, middle and last rows.
Shapes are chosen to reach each kernel of the NZ dispatch: the decode stream (M <= 16), the mid-M kernel
on NZ blocks, the 256 x 256 prefill kernel on NZ blocks (with and without a K split) and the unpack-to-[K,N]
fallback.
"""
import ctypes

import numpy as np
import pytest
import torch

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


def _bits(t):
    return t.numpy() if t.dtype in (torch.float32, torch.int32, torch.int8) else W.bits(t)


def _epilogue_args(g, M, N, out_dtype, bias_dtype):
    integer_out = out_dtype in (torch.int8, torch.int32)
    s = (1e-4 + 1e-3 * torch.rand(N, generator=g)) if out_dtype is torch.int8 else 1e-3 + 9e-3 * torch.rand(N, generator=g)
    pt = None if integer_out else 1e-2 * torch.rand(M, generator=g)
    off = torch.randn(N, generator=g) if out_dtype is torch.int8 else None
    b = None
    if bias_dtype is torch.int32:
        b = torch.randint(-1000, 1000, (N,), generator=g, dtype=torch.int32)
    elif bias_dtype is not None:
        b = torch.randn(N, generator=g).to(bias_dtype)
    return s, pt, off, b


def _call(ops, ad, wd, s, pt, off, b, out_dtype):
    kw = dict(bias=None if b is None else b.to(DEV), output_dtype=out_dtype)
    if off is not None:
        kw["offset"] = off.to(DEV)
    if pt is not None:
        kw["pertoken_scale"] = pt.to(DEV)
    return ops.npu_quant_matmul(ad, wd, s.to(DEV), **kw)


def _oracle_rows(oracle, a, w, rows, s, pt, off, b, out_dtype):
    bias_np = None if b is None else (b.numpy() if b.dtype in (torch.int32, torch.float32) else W.bits(b))
    return oracle.quant_matmul(a[rows].numpy(), w.numpy(), s.numpy(), pertoken=None if pt is None else pt[rows].numpy(),
                               offset=None if off is None else off.numpy(), bias=bias_np,
                               bias_dtype=CODE[b.dtype] if b is not None else BF16, out_dtype=CODE[out_dtype])


def _check(ops, oracle, M, N, K, out_dtype, bias_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    ad, wd = a.to(DEV), w.to(DEV)
    wnz = ops.npu_format_cast(wd, 29)
    assert tuple(wnz.shape) == (N // 16, K // 64, 64, 16) and ops.get_npu_format(wnz) == 29
    acc = ops.npu_quant_matmul(ad, wnz, torch.ones(1, device=DEV), output_dtype=torch.int32)
    a64, w64, acc64 = a.to(torch.int64), w.to(torch.int64), acc.cpu().to(torch.int64)
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    s, pt, off, b = _epilogue_args(g, M, N, out_dtype, bias_dtype)
    out = _call(ops, ad, wnz, s, pt, off, b, out_dtype).cpu()
    nd = _call(ops, ad, wd, s, pt, off, b, out_dtype).cpu()
    assert out.dtype == out_dtype and out.shape == (M, N)
    assert np.array_equal(_bits(out), _bits(nd)), "NZ and row-major weights disagree"
    rows = np.unique(np.clip(np.r_[0:3, M // 2 - 1:M // 2 + 1, M - 3:M], 0, M - 1))
    ref = _oracle_rows(oracle, a, w, rows, s, pt, off, b, out_dtype)
    got = _bits(out[rows])
    bad = np.argwhere(got != ref)
    assert bad.size == 0, (f"{len(bad)} mismatches, first at (row {rows[bad[0][0]]}, col {bad[0][1]}): "
                           f"{got[tuple(bad[0])]} vs {ref[tuple(bad[0])]}")


@pytest.mark.parametrize("M,N,K,out_dtype,bias_dtype", [
    # decode stream (M <= 16): n-blocks per workgroup 1 / 7 / 3, K blocks fewer than the waves, one row
    (1, 4096, 1024, torch.bfloat16, torch.bfloat16),
    (16, 28672, 1024, torch.bfloat16, torch.bfloat16),
    (4, 11008, 2048, torch.float16, torch.float32),
    (7, 2064, 64, torch.int8, torch.int32),
    (3, 16, 128, torch.float32, None),
    (16, 4096, 4160, torch.int32, torch.int32),
    # mid-M kernel on NZ blocks (16 < M <= 256, N % 64 == 0, K % 256 == 0)
    (17, 4096, 512, torch.bfloat16, torch.bfloat16),
    (128, 4096, 4096, torch.bfloat16, torch.bfloat16),
    (200, 2048, 1024, torch.float32, torch.int32),
    (256, 2048, 768, torch.int8, torch.int32),
    # prefill kernel on NZ blocks: whole 256 x 256 tiles, unsplit and with a K split of 2 / 4
    (4096, 4096, 1024, torch.bfloat16, torch.bfloat16),
    (2048, 2048, 1024, torch.float16, None),
    (1024, 1024, 2048, torch.bfloat16, torch.bfloat16),
    # the same on a ragged M: 160-row last tile unsplit; 232-row last tile with a K split of 4
    (4000, 4096, 1024, torch.float16, torch.float32),
    (1000, 4096, 2048, torch.bfloat16, torch.bfloat16),
    # unpack-to-[K,N] fallback: K not a multiple of 256 above the mid-M range, N % 64 != 0 with K % 256 != 0
    (300, 1024, 192, torch.bfloat16, torch.bfloat16),
    (40, 4112, 320, torch.int32, None),
])
def test_quant_matmul_nz(ops, oracle, M, N, K, out_dtype, bias_dtype):
    say(f"quant_matmul NZ M={M} N={N} K={K} out={out_dtype} bias={bias_dtype}")
    _check(ops, oracle, M, N, K, out_dtype, bias_dtype, seed=M * 7 + N + 3 * K)


def test_quant_matmul_nz_random_shapes(ops):
    """Seeded random shapes across the NZ dispatch (decode stream, mid-M, 256 x 256 tiles with and without a K
    split, unpack fallback): every int32 accumulator against the exact product (float64 BLAS is exact here:
    |sums| < 2^53), and the bf16 output with per-token scale and bias bit for bit against the row-major weight."""
    rng = np.random.default_rng(20261202)
    shapes = [(int(m), 16 * int(n), 64 * int(k)) for m, n, k in zip(
        rng.choice([1, 2, 5, 9, 16, 17, 31, 64, 100, 128, 200, 256, 257, 300, 512, 768], 18),
        rng.integers(1, 200, 18), rng.integers(1, 40, 18))]
    shapes += [(512, 1024, 1024), (768, 512, 2048), (256, 4096, 256)]  # whole 256 x 256 tiles
    for M, N, K in shapes:
        say(f"quant_matmul NZ random M={M} N={N} K={K}")
        g = torch.Generator().manual_seed(M * 31 + N * 7 + K)
        a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
        w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
        ad, wd = a.to(DEV), w.to(DEV)
        wnz = ops.npu_format_cast(wd, 29)
        acc = ops.npu_quant_matmul(ad, wnz, torch.ones(1, device=DEV), output_dtype=torch.int32).cpu()
        assert torch.equal(acc.double(), a.double() @ w.double()), (M, N, K)
        s = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(DEV)
        pt = (1e-2 * torch.rand(M, generator=g)).to(DEV)
        b = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
        out = ops.npu_quant_matmul(ad, wnz, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
        nd = ops.npu_quant_matmul(ad, wd, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
        assert torch.equal(out.view(torch.int16), nd.view(torch.int16)), (M, N, K)


@pytest.mark.parametrize("idx", [0, 1, 2])
def test_quant_matmul_nz_cfg2(ops, oracle, idx):
    """cfg2 decode shapes (M = 1, 4, 16; K=8192, N=28672; activations with 1 % outlier channels, dynamically
    quantized): the NZ decode stream bit for bit against the row-major weight and, on every row, against the
    oracle, bf16 output."""
    c = W.CFG2[idx]
    say(f"quant_matmul NZ cfg2 M={c.M}")
    d = W.w8a8_inputs(c, seed=idx)
    xq, pt = ops.npu_dynamic_quant(d["x"].to(DEV))
    w = d["w"].to(DEV)
    wnz = ops.npu_format_cast(w, 29)
    s = d["w_scale"].to(DEV)
    out = ops.npu_quant_matmul(xq, wnz, s, pertoken_scale=pt, output_dtype=torch.bfloat16)
    nd = ops.npu_quant_matmul(xq, w, s, pertoken_scale=pt, output_dtype=torch.bfloat16)
    assert torch.equal(out.view(torch.int16), nd.view(torch.int16))
    ref = oracle.quant_matmul(xq.cpu().numpy(), d["w"].numpy(), d["w_scale"].numpy(), pertoken=pt.cpu().numpy(),
                              out_dtype=BF16)
    assert np.array_equal(W.bits(out.cpu()), ref)


def test_quant_matmul_nz_cfg4(ops):
    """cfg4 prefill shape (M=4096, K=N=8192): every int32 accumulator through exact row and column checksums,
    and the bf16 output bit for bit against the row-major weight's."""
    say("quant_matmul NZ cfg4 M=4096 N=8192 K=8192")
    g = torch.Generator(device=DEV).manual_seed(4)
    M, N, K = 4096, 8192, 8192
    a = torch.randint(-128, 128, (M, K), generator=g, device=DEV, dtype=torch.int8)
    w = torch.randint(-128, 128, (K, N), generator=g, device=DEV, dtype=torch.int8)
    wnz = ops.npu_format_cast(w, 29)
    acc = ops.npu_quant_matmul(a, wnz, torch.ones(1, device=DEV), output_dtype=torch.int32)
    # exact in float64: |partial sums| < 2^53
    a64, w64, acc64 = a.double(), w.double(), acc.double()
    assert torch.equal(acc64.sum(0), a64.sum(0) @ w64)
    assert torch.equal(acc64.sum(1), a64 @ w64.sum(1))
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g, device=DEV)
    pt = 1e-2 * torch.rand(M, generator=g, device=DEV)
    b = torch.randn(N, generator=g, device=DEV).to(torch.bfloat16)
    out = ops.npu_quant_matmul(a, wnz, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
    nd = ops.npu_quant_matmul(a, w, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
    assert torch.equal(out.view(torch.int16), nd.view(torch.int16))


def test_quant_matmul_nz_k0(ops):
    """K = 0: an empty NZ weight gives the epilogue of zero sums (bias alone for a float output)."""
    say("quant_matmul NZ K=0")
    N = 64
    a = torch.empty((5, 0), dtype=torch.int8, device=DEV)
    wnz = ops.npu_format_cast(torch.empty((0, N), dtype=torch.int8, device=DEV), 29)
    assert wnz.shape == (N // 16, 0, 64, 16) and ops.get_npu_format(wnz) == 29
    b = torch.randn(N, device=DEV).to(torch.bfloat16)
    out = ops.npu_quant_matmul(a, wnz, torch.ones(N, device=DEV), bias=b, output_dtype=torch.bfloat16)
    assert torch.equal(out, b.float().expand(5, N).to(torch.bfloat16))


def test_quant_matmul_nz_refusals(ops):
    """The op refuses an NZ weight whose K does not match x1."""
    a = torch.zeros((4, 128), dtype=torch.int8, device=DEV)
    wnz = torch.zeros((4, 1, 64, 16), dtype=torch.int8, device=DEV)
    with pytest.raises(RuntimeError, match="weight's K"):
        ops.npu_quant_matmul(a, wnz, torch.ones(1, device=DEV), output_dtype=torch.int32)


def test_abi_quant_matmul_nz(ops, oracle):
    """qk_quant_matmul_nz through the C ABI: the workspace query; a refused call without the workspace, with a
    misaligned x1 and with K % 64 != 0; on 0xFF-filled workspaces the split prefill path (counters and
    partials) and the unpack fallback give the row-major call's bits, twice in a row over the same
    workspace."""
    L = ops.abi()
    for (M, N, K, what) in [(1024, 1024, 2048, "prefill split"), (300, 1024, 192, "unpack fallback"),
                            (16, 28672, 1024, "decode")]:
        say(f"ABI qk_quant_matmul_nz {what} M={M} N={N} K={K}")
        g = torch.Generator().manual_seed(M + N + K)
        a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8).to(DEV)
        w = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8).to(DEV)
        wnz = ops.npu_format_cast(w, 29)
        s = (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(DEV)
        pt = (1e-2 * torch.rand(M, generator=g)).to(DEV)
        b = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
        ref = ops.npu_quant_matmul(a, w, s, pertoken_scale=pt, bias=b, output_dtype=torch.bfloat16)
        need = ctypes.c_size_t(0)
        assert L.qk_quant_matmul_nz_workspace_size(M, N, K, BF16, ctypes.byref(need)) == 0
        out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
        stream = torch.cuda.current_stream().cuda_stream

        def call(ws, nbytes, x=a, k=K):
            return L.qk_quant_matmul_nz(x.data_ptr(), k, wnz.data_ptr(), M, N, k, s.data_ptr(), N, None, 0,
                                        pt.data_ptr(), b.data_ptr(), BF16, out.data_ptr(), BF16,
                                        ws, nbytes, stream)
        if need.value:
            assert call(None, 0) == ops.QK_ERR_WORKSPACE
        ws = torch.full((max(need.value, 256),), 0xFF, dtype=torch.uint8, device=DEV)
        for _ in range(2):
            out.fill_(0)
            assert call(ws.data_ptr(), need.value) == 0, ops.last_error()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    # refusals: misaligned x1, K % 64 != 0 (nothing is launched)
    buf = torch.zeros(64 * 130, dtype=torch.int8, device=DEV)
    wz = torch.zeros(64 * 16 * 2, dtype=torch.int8, device=DEV)
    o = torch.empty((2, 64), dtype=torch.bfloat16, device=DEV)
    sc = torch.ones(64, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    assert L.qk_quant_matmul_nz(buf.data_ptr() + 1, 128, wz.data_ptr(), 2, 64, 128, sc.data_ptr(), 64, None, 0, None,
                                None, 0, o.data_ptr(), BF16, None, 0, stream) == ops.QK_ERR_ARG
    assert L.qk_quant_matmul_nz(buf.data_ptr(), 96, wz.data_ptr(), 2, 64, 96, sc.data_ptr(), 64, None, 0, None,
                                None, 0, o.data_ptr(), BF16, None, 0, stream) == ops.QK_ERR_ARG
