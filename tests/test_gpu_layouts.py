"""GPU parity of the weight layouts the ops take besides [K, N] rows and NZ blocks, against the CPU oracle.

* The storage format is a property of the storage, not of the shape: a tensor of the NZ shape that
  npu_format_cast did not write is an ND (batched) weight, as the reference reads the format from the storage
  descriptor (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:57-66).
* An int8 W8A16 weight passed as the transposed view of an [N, K] tensor (the nn.Linear layout) is read in
  place, as the reference flags a transposed mat2 (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:40-53,
  op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:39-40): the decode kernel reads the rows directly (no
  workspace, so no copy), other shapes transpose into the call's workspace.
* Weights with batch dims follow the reference's matmul broadcast rule
  (op_plugin/ops/base_ops/opapi/MatmulKernelNpuOpApi.cpp:45-73): every output slice is checked against the
  oracle on its own x and weight slices (W8A8 bit-exact, W4A16 / W8A16 within rtol / atol 1e-2).
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


def _close(out, ref_bits, dtype):
    torch.testing.assert_close(out.cpu().float(), W.from_bits(ref_bits, dtype).float(), rtol=1e-2, atol=1e-2)


def _w8(M, N, K, group, offset, x_dtype, seed):
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


def _w8_ref(oracle, d, group, x_dtype, bias=None):
    return oracle.weight_quant_bmm(W.bits(d["x"]), CODE[x_dtype], d["w"].numpy(), W.bits(d["scale"]),
                                   None if d["offset"] is None else W.bits(d["offset"]), F16, group,
                                   bias=None if bias is None else W.bits(bias), bias_dtype=CODE[x_dtype],
                                   out_dtype=CODE[x_dtype])


def _wq(ops, x, w, d, group, bias=None):
    return ops.npu_weight_quant_batchmatmul(x, w, d["scale"].to(DEV), None if d["offset"] is None else
                                            d["offset"].to(DEV), bias=bias, antiquant_group_size=group)


# ----------------------------------------------------------------------------- storage format

def test_nz_format_is_recorded_with_the_storage(ops, oracle):
    """A 4-D int8 tensor of the NZ shape that npu_format_cast did not write is ND: a batch of [64, 16] weights
    (checked bit for bit against the oracle slice by slice); the cast one is NZ; a copy of it is ND until cast."""
    say("storage format: recorded NZ vs an NZ-shaped ND tensor")
    g = torch.Generator().manual_seed(3)
    a = torch.randint(-128, 128, (5, 64), generator=g, dtype=torch.int8)
    raw = torch.randint(-128, 128, (4, 1, 64, 16), generator=g, dtype=torch.int8)
    rd = raw.to(DEV)
    assert ops.get_npu_format(rd) == 2
    acc = ops.npu_quant_matmul(a.to(DEV), rd, torch.ones(1, device=DEV), output_dtype=torch.int32).cpu()
    assert acc.shape == (4, 1, 5, 16)
    for i in range(4):
        assert np.array_equal(acc[i, 0].numpy(), oracle.w8a8_acc(a.numpy(), raw[i, 0].numpy()))
    w = torch.randint(-128, 128, (64, 64), generator=g, dtype=torch.int8)
    nz = ops.npu_format_cast(w.to(DEV), 29)
    assert nz.shape == (4, 1, 64, 16) and ops.get_npu_format(nz) == 29
    out = ops.npu_quant_matmul(a.to(DEV), nz, torch.ones(1, device=DEV), output_dtype=torch.int32).cpu()
    assert out.shape == (5, 64) and np.array_equal(out.numpy(), oracle.w8a8_acc(a.numpy(), w.numpy()))
    cl = nz.clone()
    assert ops.get_npu_format(cl) == 2               # a copy is ND until its [K, N] form is cast again
    with pytest.raises(RuntimeError, match="ND weight"):
        ops.npu_format_cast(cl, 29)


# ----------------------------------------------------------------------------- W8A16 on an [N, K] view

@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (16, 11008, 4096, 128, True, torch.bfloat16, False),   # the cfg3 shape, int8 weights: decode kernel in place
    (1, 4096, 4096, 128, True, torch.float16, True),       # decode, one row
    (40, 768, 1024, 0, True, torch.bfloat16, True),        # decode, per channel, three row blocks
    (300, 1024, 2048, 128, True, torch.bfloat16, False),   # prefill: transposed into the workspace
    (8, 80, 192, 64, False, torch.float16, False),         # K % 128 != 0: transposed, row-major decode kernels
    (100, 1024, 2048, 128, True, torch.bfloat16, True),    # 64 < M <= 128: the decode kernel on two row chunks
])
def test_w8a16_nk_view(ops, oracle, M, N, K, group, offset, x_dtype, bias):
    """The transposed view of an int8 [N, K] weight against the oracle, and bit for bit against the same call on
    the weight cast to NZ (decode shapes: the same kernel with the rows read in place) or on the [K, N] copy (the
    shapes that transpose into the workspace)."""
    say(f"w8a16 [N,K] view M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    d = _w8(M, N, K, group, offset, x_dtype, seed=M + N + K + 5)
    b = torch.randn(N, generator=torch.Generator().manual_seed(9)).to(x_dtype).to(DEV) if bias else None
    w_nk = d["w"].t().contiguous().to(DEV)          # [N, K] storage
    view = w_nk.t()                                  # [K, N] view, strides (1, K)
    assert view.stride() == (1, K)
    x = d["x"].to(DEV)
    out = _wq(ops, x, view, d, group, b)
    _close(out, _w8_ref(oracle, d, group, x_dtype, bias=None if b is None else b.cpu()), x_dtype)
    L = ops.abi()
    ws = ctypes.c_size_t(1)
    assert L.qk_weight_quant_bmm_workspace_size(M, N, K, ops.QK_I8_NK, group, ctypes.byref(ws)) == 0
    # the decode kernel (M <= 64, or two row chunks up to 128) reads the rows in place
    decode = M <= 128 and K % 128 == 0 and N % 16 == 0 and (group == 0 or group % 128 == 0)
    if decode:
        assert ws.value == 0, "the decode kernel reads the [N, K] rows in place: no workspace, no copy"
        same = _wq(ops, x, ops.npu_format_cast(d["w"].to(DEV), 29), d, group, b)
    else:
        assert ws.value >= K * N, "the transposed weight lives in the workspace"
        same = _wq(ops, x, d["w"].to(DEV), d, group, b)
    assert torch.equal(out.view(torch.int16), same.view(torch.int16))


def test_w8a16_nk_view_through_abi(ops, oracle):
    """QK_I8_NK through the C ABI at a decode shape (no workspace) and a prefill shape (0xFF-filled workspace),
    twice each."""
    L = ops.abi()
    stream = torch.cuda.current_stream().cuda_stream
    for M, N, K in [(16, 2048, 1024), (200, 512, 1024)]:
        say(f"ABI qk_weight_quant_bmm QK_I8_NK M={M} N={N} K={K}")
        d = _w8(M, N, K, 128, True, torch.bfloat16, seed=M + 77)
        x, sc, off = d["x"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
        w_nk = d["w"].t().contiguous().to(DEV)
        need = ctypes.c_size_t(0)
        assert L.qk_weight_quant_bmm_workspace_size(M, N, K, ops.QK_I8_NK, 128, ctypes.byref(need)) == 0
        ws = torch.full((max(need.value, 256),), 0xFF, dtype=torch.uint8, device=DEV)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        ref = _w8_ref(oracle, d, 128, torch.bfloat16)
        for _ in range(2):
            out.fill_(0)
            rc = L.qk_weight_quant_bmm(x.data_ptr(), BF16, w_nk.data_ptr(), ops.QK_I8_NK, sc.data_ptr(),
                                       off.data_ptr(), F16, M, N, K, 128, None, 0, out.data_ptr(), BF16,
                                       ws.data_ptr() if need.value else None, need.value, stream)
            assert rc == 0, ops.last_error()
            torch.cuda.synchronize()
            _close(out, ref, torch.bfloat16)


def test_w8a16_nz_k_multiple_of_64(ops, oracle):
    """An int8 NZ weight with K % 128 != 0 (K = 192: three 64-row blocks), which npu_format_cast writes for any
    K % 64 == 0: npu_weight_quant_batchmatmul unpacks it in the workspace and runs the row-major kernels."""
    say("w8a16 NZ K=192")
    for M in (4, 96):
        d = _w8(M, 80, 192, 64, True, torch.bfloat16, seed=M + 192)
        nz = ops.npu_format_cast(d["w"].to(DEV), 29)
        assert ops.get_npu_format(nz) == 29 and nz.shape == (5, 3, 64, 16)
        out = _wq(ops, d["x"].to(DEV), nz, d, 64)
        _close(out, _w8_ref(oracle, d, 64, torch.bfloat16), torch.bfloat16)


# ----------------------------------------------------------------------------- batched weights

def _qmm_ref(oracle, a, w, s, pt, b, out_dtype):
    return oracle.quant_matmul(a.numpy(), w.numpy(), s.numpy(), pertoken=None if pt is None else pt.numpy(),
                               bias=None if b is None else W.bits(b), bias_dtype=BF16, out_dtype=CODE[out_dtype])


@pytest.mark.parametrize("xb,wb,M,N,K,transposed", [
    ((2,), (3, 1), 40, 96, 320, False),      # broadcast both ways: out [3, 2, 40, 96]
    ((), (3,), 33, 512, 256, True),          # 2-D x over a batch of [N, K]-view weights
    ((2,), (2,), 256, 512, 1024, False),     # whole 256 x 256 tiles per slice
])
def test_quant_matmul_batched_weights(ops, oracle, xb, wb, M, N, K, transposed):
    """npu_quant_matmul with a batch of weights: the output batch is the broadcast of x1's and x2's batch dims;
    every slice bit-exact against the oracle (per-token scale of the x1 slice's rows, per-channel scale, bf16
    bias and output)."""
    say(f"quant_matmul batched x1 batch {xb} x2 batch {wb} M={M} N={N} K={K} transposed={transposed}")
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randint(-128, 128, (*xb, M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (*wb, K, N), generator=g, dtype=torch.int8)
    s = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    rows = int(np.prod(xb)) * M if xb else M
    pt = 1e-2 * torch.rand(rows, generator=g)
    b = torch.randn(N, generator=g).to(torch.bfloat16)
    wd = w.transpose(-1, -2).contiguous().to(DEV).transpose(-1, -2) if transposed else w.to(DEV)
    out = ops.npu_quant_matmul(a.to(DEV), wd, s.to(DEV), pertoken_scale=pt.to(DEV), bias=b.to(DEV),
                               output_dtype=torch.bfloat16).cpu()
    batch = list(torch.broadcast_shapes(torch.Size(xb), torch.Size(wb)))
    assert list(out.shape) == batch + [M, N]
    for idx in np.ndindex(*batch):
        xi = tuple(i if n > 1 else 0 for i, n in zip(idx[len(idx) - len(xb):], xb))
        wi = tuple(i if n > 1 else 0 for i, n in zip(idx[len(idx) - len(wb):], wb))
        xlin = int(np.ravel_multi_index(xi, xb)) if xb else 0
        ref = _qmm_ref(oracle, a[xi], w[wi], s, pt[xlin * M:(xlin + 1) * M], b, torch.bfloat16)
        assert np.array_equal(W.bits(out[idx]), ref), idx


@pytest.mark.parametrize("int4,scale_batched", [(True, True), (False, False), (True, False)])
def test_weight_quant_bmm_batched_weights(ops, oracle, int4, scale_batched):
    """npu_weight_quant_batchmatmul with a batch of weights ([B, K, N/8] int4 or [B, K, N] int8) and scales
    with or without the weight's batch dims; x 3-D with the same batch, or 2-D broadcast over it; every slice
    within rtol / atol 1e-2 of the oracle."""
    B, M, N, K, G = 3, 16, 512, 512, 128
    say(f"weight_quant_bmm batched int4={int4} scale_batched={scale_batched}")
    g = torch.Generator().manual_seed(int(int4) * 2 + int(scale_batched))
    wv = torch.randint(-8, 8, (B, K, N), generator=g, dtype=torch.int8) if int4 else \
        torch.randint(-128, 128, (B, K, N), generator=g, dtype=torch.int8)
    wq = torch.stack([W.int4_pack_cpu(wv[i]) for i in range(B)]) if int4 else wv
    sshape = (B, K // G, N) if scale_batched else (K // G, N)
    sc = (5e-3 + 1.5e-2 * torch.rand(sshape, generator=g)).to(torch.float16)
    off = (2 * torch.rand(sshape, generator=g) - 1).to(torch.float16)
    for x in (torch.randn((B, M, K), generator=g).to(torch.bfloat16), torch.randn((M, K), generator=g).to(torch.bfloat16)):
        out = ops.npu_weight_quant_batchmatmul(x.to(DEV), wq.to(DEV), sc.to(DEV), off.to(DEV),
                                               antiquant_group_size=G).cpu()
        assert out.shape == (B, M, N)
        for i in range(B):
            xs = x[i] if x.dim() == 3 else x
            si, oi = (sc[i], off[i]) if scale_batched else (sc, off)
            ref = oracle.weight_quant_bmm(W.bits(xs), BF16, wq[i].numpy(), W.bits(si), W.bits(oi), F16, G,
                                          out_dtype=BF16)
            _close(out[i], ref, torch.bfloat16)
