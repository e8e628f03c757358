"""qk_weight_quant_bmm_noalloc: the weight-quant matmul with no workspace argument, whose scratch is a
library-held device array.  Checked through the C ABI against qk_weight_quant_bmm (same kernels, caller
workspace) on two calls in a row, the second with a smaller input, plus the refusal of a shape whose
scratch exceeds the array."""
import ctypes

import numpy as np
import pytest
import torch

from op_plugin_amd import workloads as W

pytestmark = pytest.mark.gpu

F16, BF16, I32 = 1, 2, 5
DEV = "cuda"


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    L = op_plugin_amd.abi()
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    L.qk_weight_quant_bmm_noalloc.argtypes = [P, I, P, I, P, P, I, I64, I64, I64, I64, P, I, P, I, P]
    L.qk_weight_quant_bmm_noalloc.restype = I
    return op_plugin_amd


def _call(ops, d, c, noalloc, bias=None):
    L = ops.abi()
    stream = torch.cuda.current_stream().cuda_stream
    xd, wd, sd, od = d["x"].to(DEV), d["w_packed"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
    bd = None if bias is None else bias.to(DEV)
    out = torch.empty((c.M, c.N), dtype=torch.bfloat16, device=DEV)
    common = (xd.data_ptr(), BF16, wd.data_ptr(), I32, sd.data_ptr(), od.data_ptr(), F16, c.M, c.N, c.K, c.group,
              None if bd is None else bd.data_ptr(), BF16 if bd is not None else 0, out.data_ptr(), BF16)
    if noalloc:
        rc = L.qk_weight_quant_bmm_noalloc(*common, stream)
    else:
        n = ctypes.c_size_t(0)
        assert L.qk_weight_quant_bmm_workspace_size(c.M, c.N, c.K, I32, c.group, ctypes.byref(n)) == 0
        ws = torch.empty(max(1, n.value), dtype=torch.uint8, device=DEV)
        rc = L.qk_weight_quant_bmm(*common, ws.data_ptr(), n.value, stream)
    assert rc == 0, ops.last_error()
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_workspace_entry(ops, oracle):
    """Two calls in a row, the second smaller (both split K, so both use the scratch array), each equal bit
    for bit to qk_weight_quant_bmm and within 1e-2 of the oracle."""
    cases = [W.W4A16Case(M=16, N=11008, K=4096), W.W4A16Case(M=5, N=2048, K=2048)]
    for i, c in enumerate(cases):
        print(f"[case] noalloc call {i}: M={c.M} N={c.N} K={c.K}", flush=True)
        d = W.w4a16_inputs(c, seed=60 + i)
        b = torch.randn(c.N, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16)
        n = ctypes.c_size_t(0)
        assert ops.abi().qk_weight_quant_bmm_workspace_size(c.M, c.N, c.K, I32, c.group, ctypes.byref(n)) == 0
        assert 0 < n.value <= 16 << 20, "the shape must use the scratch array"
        got = _call(ops, d, c, noalloc=True, bias=b)
        want = _call(ops, d, c, noalloc=False, bias=b)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        ref = oracle.weight_quant_bmm(W.bits(d["x"]), BF16, d["w_packed"].numpy(), W.bits(d["scale"]),
                                      W.bits(d["offset"]), F16, c.group, bias=W.bits(b), bias_dtype=BF16,
                                      out_dtype=BF16)
        torch.testing.assert_close(got.cpu().float(), W.from_bits(ref, torch.bfloat16).float(), rtol=1e-2, atol=1e-2)


def test_noalloc_refuses_oversized_scratch(ops):
    """A shape whose workspace exceeds the library's scratch is refused before any launch."""
    print("[case] noalloc oversized refusal", flush=True)
    M, N, K = 16, 1 << 17, 8192
    n = ctypes.c_size_t(0)
    assert ops.abi().qk_weight_quant_bmm_workspace_size(M, N, K, I32, 128, ctypes.byref(n)) == 0
    assert n.value > 16 << 20
    fake = ctypes.c_void_p(256)   # never dereferenced: the size check fails first
    rc = ops.abi().qk_weight_quant_bmm_noalloc(fake, BF16, fake, I32, fake, None, F16, M, N, K, 128, None, 0, fake,
                                               BF16, None)
    assert rc == -2 and "scratch" in ops.last_error()
