"""GPU parity of the quantized MLP block's neighbours (RMSNorm, SwiGLU, their fused dynamic
quantization) and of the whole cfg5 block, against the CPU oracle on the same seeded inputs.

Bar: RMSNorm / SwiGLU outputs are floating point, within rtol 1e-2 / atol 1e-2 of the float64
oracle (and in practice within one unit in the last place); rstd within 1e-6 relative.  The fused
kernels' int8 rows and scales are bit-exact against the oracle's dynamic quantization of the same
kernel's unfused 16-bit output, so the fusion itself changes no bit.  The block is checked on all
512 rows against the oracle chain.
"""
import ctypes

import numpy as np
import pytest
import torch

import exact
from op_plugin_amd import workloads as W

pytestmark = pytest.mark.gpu

F16, BF16 = 1, 2
CODE = {torch.float16: F16, torch.bfloat16: BF16}
DEV = "cuda"


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    return op_plugin_amd


def say(msg):
    print(f"[case] {msg}", flush=True)


def close(got, ref_bits, dtype, rtol=1e-2, atol=1e-2):
    g = got.cpu().float()
    r = W.from_bits(ref_bits, dtype).float().reshape(g.shape)
    torch.testing.assert_close(g, r, rtol=rtol, atol=atol)
    # diagnostic bar: the fp32 kernel and the float64 oracle differ by at most one rounding step
    # (signed zeros compare equal: results far below the 16-bit range may come out as -0 or +0)
    gb = W.bits(got.cpu()).astype(np.int32)
    rb = np.asarray(ref_bits).astype(np.int32).reshape(g.shape)
    gb[(gb & 0x7fff) == 0] = 0
    rb[(rb & 0x7fff) == 0] = 0
    assert np.abs(gb - rb).max() <= 1


RMS_CASES = [
    (512, 4096, torch.bfloat16),   # cfg5
    (7, 1000, torch.float16),      # vector path, partial last vector of threads
    (5, 1001, torch.bfloat16),     # D % 8 != 0: generic path
    (3, 8, torch.float16),
    (2, 32768, torch.bfloat16),    # largest vector-path row
    (1, 40000, torch.float16),     # beyond the vector path
]


def rms_inputs(rows, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (3 * torch.randn((rows, D), generator=g)).to(dtype)
    gamma = (1.0 + 0.02 * torch.randn((D,), generator=g)).to(dtype)
    return x, gamma


@pytest.mark.parametrize("rows,D,dtype", RMS_CASES)
def test_rms_norm(ops, oracle, rows, D, dtype):
    say(f"rms_norm rows={rows} D={D} {dtype}")
    x, gamma = rms_inputs(rows, D, dtype, rows + D)
    y, rstd = ops.npu_rms_norm(x.to(DEV), gamma.to(DEV), 1e-6)
    ry, rr = oracle.rms_norm(W.bits(x), CODE[dtype], W.bits(gamma), 1e-6)
    close(y, ry, dtype)
    assert rstd.shape == (rows, 1)
    np.testing.assert_allclose(rstd.cpu().numpy(), rr, rtol=1e-6)


def test_rms_norm_special_rows(ops, oracle):
    say("rms_norm zero row, huge row, 3-D input with 2-D gamma")
    x = torch.zeros((4, 64), dtype=torch.bfloat16)
    x[1] = 3e38   # sum of squares overflows fp32: rstd 0, y 0 (the float64 oracle gets a tiny nonzero)
    x[2, 5] = 1.0
    gamma = torch.ones(64, dtype=torch.bfloat16)
    y, rstd = ops.npu_rms_norm(x.to(DEV), gamma.to(DEV), 1e-6)
    ry, rr = oracle.rms_norm(W.bits(x), BF16, W.bits(gamma), 1e-6)
    r0 = rstd.cpu()
    # zero row: rstd = 1/sqrt(eps) (fp32 arithmetic on eps = float(1e-6): one ulp below the float64 value)
    np.testing.assert_allclose(r0[0].numpy(), rr[0], rtol=1e-6)
    assert torch.all(y[0].cpu() == 0)
    assert r0[1, 0] == 0 and torch.all(y[1].cpu() == 0)   # fp32 sum of squares overflows
    np.testing.assert_allclose(r0[2].numpy(), rr[2], rtol=1e-6)
    torch.testing.assert_close(y[2].cpu().float(), W.from_bits(ry[2], torch.bfloat16).float())
    x3, g2 = rms_inputs(6, 64, torch.float16, 3)
    y3, r3 = ops.npu_rms_norm(x3.reshape(3, 2, 64).to(DEV), g2.to(DEV), 1e-6)
    assert y3.shape == (3, 2, 64) and r3.shape == (3, 2, 1)
    ry3, _ = oracle.rms_norm(W.bits(x3), F16, W.bits(g2), 1e-6)
    close(y3.reshape(6, 64), ry3, torch.float16)


@pytest.mark.parametrize("rows,D,dtype", RMS_CASES)
def test_rms_norm_dynamic_quant(ops, oracle, rows, D, dtype):
    say(f"rms_norm_dynamic_quant rows={rows} D={D} {dtype}")
    x, gamma = rms_inputs(rows, D, dtype, 7 * rows + D)
    xd, gd = x.to(DEV), gamma.to(DEV)
    q, s, rstd = ops.npu_rms_norm_dynamic_quant(xd, gd, 1e-6)
    y, rstd_u = ops.npu_rms_norm(xd, gd, 1e-6)
    rq, rs = oracle.dynamic_quant(W.bits(y.cpu()), CODE[dtype])
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert torch.equal(rstd, rstd_u)


SWIGLU_CASES = [
    (512, 14336, torch.bfloat16),  # cfg5
    (3, 1000, torch.float16),
    (4, 1003, torch.bfloat16),     # I % 8 != 0: generic path
    (2, 20480, torch.bfloat16),    # beyond the vector path
]


def swiglu_inputs(rows, I, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    h = (4 * torch.randn((rows, 2 * I), generator=g)).to(dtype)
    h[0, :8] = torch.tensor([-100.0, 100.0, 0.0, -0.0, 20.0, -20.0, 1e-3, -88.0]).to(dtype)   # saturating silu
    return h


@pytest.mark.parametrize("rows,I,dtype", SWIGLU_CASES)
def test_swiglu(ops, oracle, rows, I, dtype):
    say(f"swiglu rows={rows} I={I} {dtype}")
    h = swiglu_inputs(rows, I, dtype, rows + I)
    y = ops.npu_swiglu(h.to(DEV))
    assert y.shape == (rows, I)
    close(y, oracle.swiglu(W.bits(h), CODE[dtype]), dtype)


@pytest.mark.parametrize("rows,I,dtype", SWIGLU_CASES)
def test_swiglu_dynamic_quant(ops, oracle, rows, I, dtype):
    say(f"swiglu_dynamic_quant rows={rows} I={I} {dtype}")
    h = swiglu_inputs(rows, I, dtype, 5 * rows + I).to(DEV)
    q, s = ops.npu_swiglu_dynamic_quant(h)
    rq, rs = oracle.dynamic_quant(W.bits(ops.npu_swiglu(h).cpu()), CODE[dtype])
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))


def test_swiglu_3d_and_empty(ops, oracle):
    say("swiglu 3-D input, empty rows")
    h = swiglu_inputs(6, 64, torch.float16, 11)
    y = ops.npu_swiglu(h.reshape(2, 3, 128).to(DEV), dim=2)
    assert y.shape == (2, 3, 64)
    close(y.reshape(6, 64), oracle.swiglu(W.bits(h), F16), torch.float16)
    assert ops.npu_swiglu(torch.empty((0, 16), dtype=torch.bfloat16, device=DEV)).shape == (0, 8)


def test_abi_rms_norm_and_swiglu(ops, oracle):
    say("ABI qk_rms_norm_quant / qk_swiglu")
    L = ops.abi()
    x, gamma = rms_inputs(4, 256, torch.bfloat16, 9)
    xd, gd = x.to(DEV), gamma.to(DEV)
    q = torch.empty((4, 256), dtype=torch.int8, device=DEV)
    s = torch.empty(4, dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    assert L.qk_rms_norm_quant(xd.data_ptr(), BF16, gd.data_ptr(), 4, 256, ctypes.c_float(1e-6), q.data_ptr(),
                               s.data_ptr(), None, stream) == 0, ops.last_error()
    ry, _ = oracle.rms_norm(W.bits(x), BF16, W.bits(gamma), 1e-6)
    torch.cuda.synchronize()
    # the oracle's own chain (float64 RMSNorm then quant) agrees up to the one-ulp RMSNorm difference
    rq, _ = oracle.dynamic_quant(ry, BF16)
    assert np.abs(q.cpu().numpy().astype(np.int32) - rq.astype(np.int32)).max() <= 1
    h = swiglu_inputs(3, 64, torch.float16, 2).to(DEV)
    y = torch.empty((3, 64), dtype=torch.float16, device=DEV)
    assert L.qk_swiglu(h.data_ptr(), F16, 3, 64, y.data_ptr(), stream) == 0, ops.last_error()
    torch.cuda.synchronize()
    close(y, oracle.swiglu(W.bits(h.cpu()), F16), torch.float16)


def test_quant_mlp_block_cfg5(ops, oracle):
    """cfg5 end to end: fused and unfused chains give identical bits, and all 512 rows match the oracle
    chain (RMSNorm -> quant -> W8A8 -> SwiGLU -> quant -> W8A8) within 1e-2.  The two GEMMs of the chain
    take their exact int32 accumulators from float64 GEMMs (pinned against qo_w8a8_acc on two rows each)
    and the oracle's epilogue."""
    from op_plugin_amd.mlp import quant_mlp
    c = W.CFG5
    say(f"quant_mlp cfg5 T={c['tokens']} H={c['hidden']} I={c['intermediate']} (all rows)")
    d = W.mlp_inputs(c["tokens"], c["hidden"], c["intermediate"], seed=0)
    dev = {k: v.to(DEV) for k, v in d.items()}
    out = quant_mlp(dev["x"], dev["gamma"], dev["w_gu"], dev["s_gu"], dev["w_d"], dev["s_d"], eps=c["eps"])
    out_u = quant_mlp(dev["x"], dev["gamma"], dev["w_gu"], dev["s_gu"], dev["w_d"], dev["s_d"], eps=c["eps"],
                      fused=False)
    assert out.shape == (c["tokens"], c["hidden"]) and out.dtype == torch.bfloat16
    assert torch.equal(out, out_u)
    pin = np.r_[0, c["tokens"] - 1]
    y, _ = oracle.rms_norm(W.bits(d["x"]), BF16, W.bits(d["gamma"]), c["eps"])
    q1, s1 = oracle.dynamic_quant(y, BF16)
    acc1 = exact.w8a8_acc(q1, d["w_gu"].numpy())
    exact.pin_acc(oracle, q1, d["w_gu"].numpy(), acc1, pin)
    h = oracle.quant_matmul_epilogue(acc1, d["s_gu"].numpy(), pertoken=s1, out_dtype=BF16)
    q2, s2 = oracle.dynamic_quant(oracle.swiglu(h, BF16), BF16)
    acc2 = exact.w8a8_acc(q2, d["w_d"].numpy())
    exact.pin_acc(oracle, q2, d["w_d"].numpy(), acc2, pin)
    ref = oracle.quant_matmul_epilogue(acc2, d["s_d"].numpy(), pertoken=s2, out_dtype=BF16)
    torch.testing.assert_close(out.cpu().float(), W.from_bits(ref, torch.bfloat16).float(), rtol=1e-2, atol=1e-2)
