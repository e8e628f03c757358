"""GPU parity of the static quantization ops against the CPU oracle, bit for bit.

quantize_per_tensor / quantize_per_channel (schemas op_plugin/config/v2r2/op_plugin_functions.yaml:1231, 1233)
return the plain int8 / uint8 / int32 tensors of the reference's NPU ops; dequantize
(op_plugin/config/v1r11/op_plugin_functions.yaml:127) casts them to float32.  The oracle is pinned against
torch.quantize_per_tensor / quantize_per_channel in tests/test_oracle.py.
"""
import numpy as np
import pytest
import torch

from op_plugin_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
F16, BF16, F32, I8, I32, U8 = 1, 2, 3, 4, 5, 6
XCODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
QT = {torch.qint8: I8, torch.quint8: U8, torch.qint32: I32}


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    return op_plugin_amd


def say(msg):
    print(f"[case] {msg}", flush=True)


def _xnp(x):
    return x.numpy() if x.dtype == torch.float32 else W.bits(x)


def _inputs(shape, dtype, seed, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * 4
    flat = x.view(-1)
    k = min(256, flat.numel())
    j = torch.randint(-100, 100, (k,), generator=g).float()
    flat[:k] = (j + 0.5) * scale                      # exact ties (for scales whose reciprocal is exact)
    if flat.numel() > k + 4:
        flat[k:k + 4] = torch.tensor([1e6, -1e6, 0.0, 300.0])
    return x.to(dtype)


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qdt", [torch.qint8, torch.quint8, torch.qint32])
@pytest.mark.parametrize("n,scale,zp", [(4096, 0.0625, 0), (4096 + 3, 0.0173, 3), (1000, 2.0, 17), (8, 0.5, 100)])
def test_quantize_per_tensor(ops, oracle, xdt, qdt, n, scale, zp):
    if qdt == torch.qint8:
        zp = min(zp, 127)
    say(f"quantize_per_tensor n={n} scale={scale} zp={zp} {xdt} -> {qdt}")
    x = _inputs((n,), xdt, seed=n + zp, scale=scale)
    got = ops.quantize_per_tensor(x.to(DEV), scale, zp, qdt)
    ref = oracle.quantize(_xnp(x), XCODE[xdt], np.array([np.float32(scale)]), np.array([zp]), None, QT[qdt])
    assert got.dtype == {torch.qint8: torch.int8, torch.quint8: torch.uint8, torch.qint32: torch.int32}[qdt]
    assert np.array_equal(got.cpu().numpy(), ref)


def test_quantize_per_tensor_strided_and_empty(ops, oracle):
    say("quantize_per_tensor on a non-contiguous view, an offset view and an empty tensor")
    x = _inputs((64, 48), torch.float16, seed=3)
    for v in (x.t(), x[:, 1:]):
        got = ops.quantize_per_tensor(v.to(DEV), 0.03, -4, torch.qint8)
        ref = oracle.quantize(W.bits(v.contiguous()), F16, np.array([np.float32(0.03)]), np.array([-4]), None, I8)
        assert np.array_equal(got.cpu().numpy(), ref)
    assert ops.quantize_per_tensor(torch.empty(0, 5, device=DEV), 0.1, 0, torch.qint8).shape == (0, 5)


@pytest.mark.parametrize("shape,axis", [((6, 40, 8), 0), ((6, 40, 8), 1), ((6, 40, 8), -1), ((128, 4096), 1),
                                        ((4096, 64), 0), ((3, 5, 7), 1), ((17,), 0)])
@pytest.mark.parametrize("qdt", [torch.qint8, torch.quint8, torch.qint32])
def test_quantize_per_channel(ops, oracle, shape, axis, qdt):
    say(f"quantize_per_channel shape={shape} axis={axis} -> {qdt}")
    x = _inputs(shape, torch.bfloat16, seed=sum(shape) + axis)
    C = x.shape[axis]
    g = torch.Generator().manual_seed(C)
    sc = torch.rand(C, generator=g, dtype=torch.float64) * 0.1 + 1e-3
    lo = 0 if qdt == torch.quint8 else -20
    zp = torch.randint(lo, 20, (C,), generator=g, dtype=torch.int64)
    got = ops.quantize_per_channel(x.to(DEV), sc.to(DEV), zp.to(DEV), axis, qdt)
    ref = oracle.quantize(W.bits(x), BF16, sc.float().numpy(), zp.numpy(), axis, QT[qdt])
    assert np.array_equal(got.cpu().numpy(), ref)


def test_quantize_per_channel_cfg4_shape(ops, oracle):
    """A cfg4-sized activation [4096, 8192] fp16, quantized per channel along the last axis (float32 scales,
    int32 zero points), whole output bit-exact."""
    say("quantize_per_channel fp16 [4096, 8192] axis -1")
    d = W.w8a8_inputs(W.CFG4)
    g = torch.Generator().manual_seed(5)
    sc = torch.rand(8192, generator=g) * 0.05 + 1e-3
    zp = torch.randint(-10, 10, (8192,), generator=g, dtype=torch.int32)
    got = ops.quantize_per_channel(d["x"].to(DEV), sc.to(DEV), zp.to(DEV), -1, torch.qint8)
    ref = oracle.quantize(W.bits(d["x"]), F16, sc.numpy(), zp.numpy().astype(np.int64), -1, I8)
    assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("dt,code", [(torch.int8, I8), (torch.uint8, U8), (torch.int32, I32)])
def test_dequantize(ops, oracle, dt, code):
    say(f"dequantize {dt}")
    g = torch.Generator().manual_seed(7)
    info = torch.iinfo(dt)
    q = torch.randint(info.min, info.max, (5003,), generator=g, dtype=torch.int64).to(dt)
    got = ops.dequantize(q.to(DEV))
    assert got.dtype == torch.float32
    assert np.array_equal(got.cpu().numpy(), oracle.dequantize(q.numpy(), code))
    # a round trip through the per-tensor quantizer with scale 1 returns the integers
    xq = ops.quantize_per_tensor(got, 1.0, 0, {torch.int8: torch.qint8, torch.uint8: torch.quint8,
                                                torch.int32: torch.qint32}[dt])
    if dt != torch.int32:
        assert torch.equal(xq.cpu(), q)


def test_abi_static_quant(ops, oracle):
    say("ABI qk_quantize_per_tensor / qk_quantize_per_channel / qk_dequantize")
    L = ops.abi()
    s = torch.cuda.current_stream().cuda_stream
    x = _inputs((32, 64), torch.float32, seed=11)
    xd = x.to(DEV)
    q = torch.empty(32, 64, dtype=torch.int8, device=DEV)
    assert L.qk_quantize_per_tensor(xd.data_ptr(), F32, x.numel(), 0.05, 2, q.data_ptr(), I8, s) == 0, ops.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), oracle.quantize(x.numpy(), F32, [0.05], [2], None, I8))
    sc = torch.linspace(0.01, 0.2, 64, device=DEV)
    zp = torch.arange(64, device=DEV, dtype=torch.int64) - 32
    assert L.qk_quantize_per_channel(xd.data_ptr(), F32, 32, 64, 1, sc.data_ptr(), zp.data_ptr(), q.data_ptr(), I8,
                                     s) == 0, ops.last_error()
    f = torch.empty(32, 64, device=DEV)
    assert L.qk_dequantize(q.data_ptr(), I8, q.numel(), f.data_ptr(), s) == 0
    torch.cuda.synchronize()
    ref = oracle.quantize(x.numpy(), F32, sc.cpu().numpy(), zp.cpu().numpy(), 1, I8)
    assert np.array_equal(q.cpu().numpy(), ref)
    assert np.array_equal(f.cpu().numpy(), ref.astype(np.float32))
