"""GPU parity of the NZ (MFMA-tiled) int4 weight path against the CPU oracle.

* npu_format_cast / npu_convert_weight_to_int4pack(inner_k_tiles=4) on the
  device: bit-exact against the oracle's NZ restatement, both directions.
* npu_weight_quant_batchmatmul on NZ weights: within rtol 1e-2 / atol 1e-2
  of the float64 oracle on the same seeded inputs (the bar of the row-major
  path), through the NZ decode kernel (M <= 64), the NZ prefill kernel (M > 64
  with enough 128 x 256 tiles; int4 and int8 weights) and through the
  unpack-to-ND fallback (short groups, K with no even wave split, few prefill
  tiles, forced off).
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


@pytest.fixture
def plan(ops):
    yield ops.debug_set_plan
    ops.debug_set_plan("")


def say(msg):
    print(f"[case] {msg}", flush=True)


def _ref(oracle, d, group, bias=None, x_dtype=torch.bfloat16):
    return oracle.weight_quant_bmm(W.bits(d["x"]), CODE[x_dtype], d["w_packed"].numpy(), W.bits(d["scale"]),
                                   None if d["offset"] is None else W.bits(d["offset"]), F16, group,
                                   bias=None if bias is None else W.bits(bias), bias_dtype=CODE[x_dtype],
                                   out_dtype=CODE[x_dtype])


def _close(out, ref_bits, dtype):
    torch.testing.assert_close(out.cpu().float(), W.from_bits(ref_bits, dtype).float(), rtol=1e-2, atol=1e-2)


def _inputs(M, N, K, group, offset, x_dtype, seed):
    d = W.w4a16_inputs(W.W4A16Case(M=M, N=N, K=K, group=group, x_dtype=x_dtype, offset=offset), seed=seed)
    if group == 0:
        d = dict(d, scale=d["scale"].reshape(-1), offset=None if d["offset"] is None else d["offset"].reshape(-1))
    return d


def _run(ops, d, group, nz, bias=None):
    return ops.npu_weight_quant_batchmatmul(
        d["x"].to(DEV), nz, d["scale"].to(DEV), None if d["offset"] is None else d["offset"].to(DEV),
        bias=None if bias is None else bias.to(DEV), antiquant_group_size=group)


def test_format_cast_device_matches_oracle(ops, oracle):
    say("npu_format_cast ND <-> NZ, K=384 N=80")
    g = torch.Generator().manual_seed(11)
    w = torch.randint(-8, 8, (384, 80), generator=g, dtype=torch.int8)
    nd = oracle.int4_pack(w.numpy())
    ref = oracle.w4_nz_pack(nd)
    got = ops.npu_format_cast(torch.from_numpy(nd).to(DEV), 29)
    assert ops.get_npu_format(got) == 29
    assert np.array_equal(got.cpu().numpy(), ref)
    back = ops.npu_format_cast(got, 2)
    assert np.array_equal(back.cpu().numpy(), nd)
    direct = ops.npu_convert_weight_to_int4pack(w.to(torch.int32).to(DEV), inner_k_tiles=4)
    assert np.array_equal(direct.cpu().numpy(), ref)


def test_format_cast_cfg3_round_trip(ops, oracle):
    say("npu_format_cast cfg3 weight [4096, 1376] round trip")
    d = W.w4a16_inputs(W.CFG3[0])
    nd = d["w_packed"].to(DEV)
    nz = ops.npu_format_cast(nd, 29)
    assert nz.shape == (688, 32, 64, 4)
    assert torch.equal(ops.npu_format_cast(nz, 2), nd)
    # spot blocks against the oracle on a column slice (the oracle restates any slice of 16-column blocks)
    ref = oracle.w4_nz_pack(d["w_packed"][:, :64].numpy())
    assert np.array_equal(nz[:32].cpu().numpy(), ref)


def test_w4a16_nz_cfg3_decode(ops, oracle):
    c = W.CFG3[0]
    say(f"w4a16 NZ cfg3 M={c.M} 4096x11008 (whole output)")
    d = W.w4a16_inputs(c)
    nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)
    out = _run(ops, d, 128, nz)
    _close(out, _ref(oracle, d, 128), torch.bfloat16)
    nd_out = _run(ops, d, 128, d["w_packed"].to(DEV))
    torch.testing.assert_close(out.float(), nd_out.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (1, 11008, 4096, 128, True, torch.bfloat16, False),
    (4, 11008, 4096, 128, True, torch.bfloat16, True),
    (16, 256, 512, 128, False, torch.bfloat16, False),      # 4 waves, one superblock each
    (7, 1008, 1024, 256, True, torch.float16, True),        # fp16, 256-row groups
    (16, 4096, 4096, 0, True, torch.bfloat16, True),        # per channel
    (33, 512, 2048, 128, True, torch.bfloat16, False),      # three 16-row blocks, clamped rows
    (64, 144, 8192, 128, True, torch.bfloat16, True),       # four superblocks per wave (two in flight)
    (2, 48, 14336, 128, True, torch.bfloat16, False),       # seven superblocks per wave
    (3, 16, 128, 128, True, torch.float16, False),          # one wave, one block
    (5, 4112, 640, 128, False, torch.bfloat16, True),       # 257 blocks: some workgroups own one fewer
    # fallbacks: the weight is unpacked to ND in the workspace and the row-major kernels run
    (16, 256, 2176, 128, True, torch.bfloat16, False),      # 17 superblocks: no even wave split
    (8, 512, 1024, 64, True, torch.bfloat16, True),         # 64-row groups
    (100, 256, 1024, 128, True, torch.float16, False),      # M > 64
])
def test_w4a16_nz_shapes(ops, oracle, M, N, K, group, offset, x_dtype, bias):
    say(f"w4a16 NZ M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    d = _inputs(M, N, K, group, offset, x_dtype, seed=M + N + K)
    b = torch.randn(N, generator=torch.Generator().manual_seed(5)).to(x_dtype) if bias else None
    nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)
    out = _run(ops, d, group, nz, bias=b)
    _close(out, _ref(oracle, d, group, bias=b, x_dtype=x_dtype), x_dtype)


@pytest.mark.parametrize("spec", ["w4nz_wg=344", "w4nz_wg=688", "w4nz_wg=100", "w4nz=off"])
def test_w4a16_nz_plans(ops, oracle, plan, spec):
    """The cfg3 M=16 shape with other workgroup counts (344 and 688 give 2 and 1 blocks per workgroup; 100
    asks for 7, capped at the 4 a wave of two superblocks holds, so 172 workgroups) and with the NZ kernel
    switched off (unpack + row-major stream)."""
    c = W.CFG3[0]
    say(f"w4a16 NZ cfg3 M=16 plan {spec}")
    plan(spec)
    d = W.w4a16_inputs(c, seed=4)
    nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)
    out = _run(ops, d, 128, nz)
    _close(out, _ref(oracle, d, 128), torch.bfloat16)


def test_w4a16_nz_prefill_fallback(ops, oracle):
    """M = 512 on NZ weights: unpacked to ND, then the DMA prefill kernel (forced onto this small shape)."""
    say("w4a16 NZ prefill M=512 N=1024 K=1024")
    ops.debug_set_plan("w4_gemm=force")
    try:
        d = _inputs(512, 1024, 1024, 128, True, torch.bfloat16, seed=21)
        nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)
        out = _run(ops, d, 128, nz)
    finally:
        ops.debug_set_plan("")
    _close(out, _ref(oracle, d, 128), torch.bfloat16)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (2048, 11008, 4096, 128, True, torch.bfloat16, False),   # cfg3 prefill: 16 x 43 tiles
    (320, 8192, 1024, 256, False, torch.float16, True),      # two steps per group, last row tile half full
    (512, 6144, 768, 0, True, torch.bfloat16, False),        # per channel: one group of 768 rows
    (1000, 4096, 2048, 128, True, torch.bfloat16, True),     # last row tile of 104 rows
])
def test_w4a16_nz_prefill_kernel(ops, oracle, M, N, K, group, offset, x_dtype, bias):
    """The NZ prefill kernel (M > 64, at least 96 tiles of 128 x 256): every output element within
    rtol/atol 1e-2 of the float64 dequant-matmul, which is pinned against the C oracle on four rows; and
    against the row-major path on the same weight."""
    say(f"w4a16 NZ prefill M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    d = _inputs(M, N, K, group, offset, x_dtype, seed=M + N + K + 1)
    b = torch.randn(N, generator=torch.Generator().manual_seed(6)).to(x_dtype) if bias else None
    nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)
    out = _run(ops, d, group, nz, bias=b)
    ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], group, bias=b)
    rows = np.r_[0:2, M - 2:M]
    pin = _ref(oracle, dict(d, x=d["x"][rows]), group, bias=b, x_dtype=x_dtype)
    pin_diff = (W.from_bits(pin, x_dtype).float() - ref64[rows].float()).abs()
    assert pin_diff.max().item() <= 2.0**-7 * ref64[rows].abs().max().item() + 1e-3
    torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)
    nd_out = _run(ops, d, group, d["w_packed"].to(DEV), bias=b)
    torch.testing.assert_close(out.float(), nd_out.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (1024, 2048, 1024, 128, True, torch.bfloat16, True),     # 8 x 8 tiles, one step per group
    (1100, 2048, 2048, 256, False, torch.float16, False),    # two steps per group, last row tile of 76 rows
    (1024, 2560, 1024, 0, True, torch.bfloat16, True),       # per channel
])
def test_w4a16_row_major_cast_to_nz(ops, oracle, plan, M, N, K, group, offset, x_dtype, bias):
    """M >= 1024 on a row-major int4 weight: the call casts the weight to NZ in its workspace (which the size query
    reports) and runs the NZ prefill kernel on the copy. Every output within rtol/atol 1e-2 of the float64
    dequant-matmul (pinned against the C oracle on four rows) and of the row-major prefill kernel (the cast
    switched off by the debug override)."""
    say(f"w4a16 row-major cast to NZ M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    L = ops.abi()
    ws = ctypes.c_size_t(0)
    assert L.qk_weight_quant_bmm_workspace_size(M, N, K, ops.QK_I32, group, ctypes.byref(ws)) == 0
    assert ws.value >= 4096 + K * N // 2, "the workspace holds the cast weight"
    d = _inputs(M, N, K, group, offset, x_dtype, seed=M + N + K + 2)
    b = torch.randn(N, generator=torch.Generator().manual_seed(7)).to(x_dtype) if bias else None
    wd = d["w_packed"].to(DEV)
    out = _run(ops, d, group, wd, bias=b)
    ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], group, bias=b)
    rows = np.r_[0:2, M - 2:M]
    pin = _ref(oracle, dict(d, x=d["x"][rows]), group, bias=b, x_dtype=x_dtype)
    pin_diff = (W.from_bits(pin, x_dtype).float() - ref64[rows].float()).abs()
    assert pin_diff.max().item() <= 2.0**-7 * ref64[rows].abs().max().item() + 1e-3
    torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)
    plan("w4nz=off")
    rm = _run(ops, d, group, wd, bias=b)
    torch.testing.assert_close(out.float(), rm.float(), rtol=1e-2, atol=1e-2)


def test_abi_noalloc_row_major_beyond_cast(ops, oracle):
    """The no-allocation entry point at M = 1024 on cfg3's row-major int4 weight, whose NZ copy (22.5 MB) does not
    fit its 16 MB scratch: it sizes its scratch without the cast and runs the row-major prefill kernel, within
    rtol/atol 1e-2 of the op (which casts) and of the float64 dequant-matmul."""
    M, N, K = 1024, 11008, 4096
    say(f"ABI qk_weight_quant_bmm_noalloc row-major int4 M={M} N={N} K={K}")
    L = ops.abi()
    d = _inputs(M, N, K, 128, True, torch.bfloat16, seed=21)
    x, w, sc, off = d["x"].to(DEV), d["w_packed"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    rc = L.qk_weight_quant_bmm_noalloc(x.data_ptr(), BF16, w.data_ptr(), ops.QK_I32, sc.data_ptr(), off.data_ptr(),
                                       F16, M, N, K, 128, None, 0, out.data_ptr(), BF16,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ops.last_error()
    op_out = _run(ops, d, 128, w)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float(), op_out.float(), rtol=1e-2, atol=1e-2)
    ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], 128)
    torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M", [1024, 2048])
def test_w4a16_cfg3_cast_path_runs_and_matches_row_major_bits(ops, oracle, plan, M):
    """cfg3's shape (N=11008, K=4096, 128-row groups, offset, bf16, no bias) at M >= 1024 on the row-major int4
    weight, through the C ABI with a 0xA5-filled workspace: after the call the workspace holds the weight cast to
    NZ (bit for bit what npu_format_cast writes), which shows the cast and the NZ prefill kernel ran; its output
    equals bit for bit the row-major prefill kernel's (the cast switched off), whose 256 x 128 tiles add each
    group's raw sums in the same k order and fold them alike; and it is within rtol / atol 1e-2 of the float64
    dequant-matmul."""
    N, K = 11008, 4096
    say(f"w4a16 cfg3 M={M}: per-call cast to NZ ran, bits equal to the row-major kernel")
    L = ops.abi()
    d = _inputs(M, N, K, 128, True, torch.bfloat16, seed=M + 3)
    x, w, sc, off = d["x"].to(DEV), d["w_packed"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
    need = ctypes.c_size_t(0)
    assert L.qk_weight_quant_bmm_workspace_size(M, N, K, ops.QK_I32, 128, ctypes.byref(need)) == 0
    ws = torch.full((need.value,), 0xA5, dtype=torch.uint8, device=DEV)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    rc = L.qk_weight_quant_bmm(x.data_ptr(), BF16, w.data_ptr(), ops.QK_I32, sc.data_ptr(), off.data_ptr(), F16,
                               M, N, K, 128, None, 0, out.data_ptr(), BF16, ws.data_ptr(), need.value,
                               torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ops.last_error()
    nz = ops.npu_format_cast(w, 29)
    torch.cuda.synchronize()
    cast_region = ws[4096:4096 + K * N // 2]
    assert torch.equal(cast_region, nz.view(torch.uint8).reshape(-1)), "the workspace does not hold the NZ cast"
    on_nz = _run(ops, d, 128, nz)  # the same kernel on the weight cast once
    assert torch.equal(out.view(torch.int16), on_nz.view(torch.int16))
    plan("w4nz=off")
    rm = _run(ops, d, 128, w)
    plan("")
    assert torch.equal(out.view(torch.int16), rm.view(torch.int16))
    ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], 128)
    torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)


def test_abi_noalloc_row_major_cast_fits_scratch(ops, oracle):
    """The no-allocation entry point at M = 1024 on a row-major int4 weight whose NZ copy (1 MB) fits its 16 MB
    scratch: the cast and the NZ prefill kernel run inside the library's array. Two calls in a row (the second on
    other inputs, so stale scratch would show), each equal bit for bit to qk_weight_quant_bmm on an allocated
    workspace and within rtol / atol 1e-2 of the float64 dequant-matmul."""
    M, N, K = 1024, 2048, 1024
    L = ops.abi()
    s = torch.cuda.current_stream().cuda_stream
    for seed in (31, 32):
        say(f"ABI qk_weight_quant_bmm_noalloc row-major int4 M={M} N={N} K={K} seed={seed}")
        d = _inputs(M, N, K, 128, True, torch.bfloat16, seed=seed)
        x, w, sc, off = d["x"].to(DEV), d["w_packed"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
        need = ctypes.c_size_t(0)
        assert L.qk_weight_quant_bmm_workspace_size(M, N, K, ops.QK_I32, 128, ctypes.byref(need)) == 0
        assert 4096 + K * N // 2 <= need.value <= ops.QK_NOALLOC_SCRATCH_BYTES
        ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
        ref = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        assert L.qk_weight_quant_bmm(x.data_ptr(), BF16, w.data_ptr(), ops.QK_I32, sc.data_ptr(), off.data_ptr(),
                                     F16, M, N, K, 128, None, 0, ref.data_ptr(), BF16, ws.data_ptr(), need.value,
                                     s) == 0, ops.last_error()
        assert L.qk_weight_quant_bmm_noalloc(x.data_ptr(), BF16, w.data_ptr(), ops.QK_I32, sc.data_ptr(),
                                             off.data_ptr(), F16, M, N, K, 128, None, 0, out.data_ptr(), BF16,
                                             s) == 0, ops.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], 128)
        torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)


def test_abi_nz_and_noalloc(ops, oracle):
    """qk_weight_quant_bmm with QK_I4_NZ through the C ABI (no workspace needed), and the no-allocation entry
    point on the same NZ weight, against the oracle."""
    say("ABI qk_weight_quant_bmm QK_I4_NZ M=16 N=2048 K=4096")
    L = ops.abi()
    d = _inputs(16, 2048, 4096, 128, True, torch.bfloat16, seed=9)
    nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)
    x, sc, off = d["x"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
    ws = ctypes.c_size_t(1)
    assert L.qk_weight_quant_bmm_workspace_size(16, 2048, 4096, ops.QK_I4_NZ, 128, ctypes.byref(ws)) == 0
    assert ws.value == 0
    ref = _ref(oracle, d, 128)
    s = torch.cuda.current_stream().cuda_stream
    for entry in ("ws", "noalloc"):
        out = torch.empty(16, 2048, dtype=torch.bfloat16, device=DEV)
        if entry == "ws":
            rc = L.qk_weight_quant_bmm(x.data_ptr(), BF16, nz.data_ptr(), ops.QK_I4_NZ, sc.data_ptr(),
                                       off.data_ptr(), F16, 16, 2048, 4096, 128, None, 0, out.data_ptr(), BF16,
                                       None, 0, s)
        else:
            rc = L.qk_weight_quant_bmm_noalloc(x.data_ptr(), BF16, nz.data_ptr(), ops.QK_I4_NZ, sc.data_ptr(),
                                               off.data_ptr(), F16, 16, 2048, 4096, 128, None, 0, out.data_ptr(),
                                               BF16, s)
        assert rc == 0, ops.last_error()
        torch.cuda.synchronize()
        _close(out, ref, torch.bfloat16)


# ----------------------------------------------------------------------------- int8 NZ (W8A16)

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


def test_format_cast_int8_device_matches_oracle(ops, oracle):
    say("npu_format_cast int8 ND <-> NZ, K=192 N=80")
    g = torch.Generator().manual_seed(12)
    w = torch.randint(-128, 128, (192, 80), generator=g, dtype=torch.int8)
    got = ops.npu_format_cast(w.to(DEV), 29)
    assert got.shape == (5, 3, 64, 16) and ops.get_npu_format(got) == 29
    assert np.array_equal(got.cpu().numpy(), oracle.w8_nz_pack(w.numpy()))
    assert torch.equal(ops.npu_format_cast(got, 2).cpu(), w)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (16, 11008, 4096, 128, True, torch.bfloat16, False),   # the cfg3 shape with int8 weights
    (1, 4096, 4096, 128, True, torch.float16, True),
    (16, 768, 512, 0, True, torch.bfloat16, True),         # per channel
    (33, 512, 1024, 256, False, torch.bfloat16, False),    # three row blocks, 256-row groups
    (4, 144, 8192, 128, True, torch.float16, False),       # four superblocks per wave: one block per workgroup
    (3, 48, 384, 128, True, torch.bfloat16, True),         # three waves
    # fallbacks (unpacked to ND in the workspace)
    (7, 2048, 1024, 64, False, torch.bfloat16, False),     # 64-row groups
    (80, 256, 512, 128, True, torch.float16, False),       # M > 64: the decode kernel on two row chunks
    (128, 2048, 1024, 128, True, torch.bfloat16, True),    # two full 64-row chunks
    (200, 256, 512, 128, True, torch.float16, False),      # 128 < M <= 256, too few prefill tiles: four row chunks
    (300, 256, 512, 128, True, torch.bfloat16, False),     # M > 256: unpacked to ND
])
def test_w8a16_nz_shapes(ops, oracle, M, N, K, group, offset, x_dtype, bias):
    say(f"w8a16 NZ M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    d = _w8(M, N, K, group, offset, x_dtype, seed=M + N + K)
    b = torch.randn(N, generator=torch.Generator().manual_seed(6)).to(x_dtype) if bias else None
    nz = ops.npu_format_cast(d["w"].to(DEV), 29)
    out = ops.npu_weight_quant_batchmatmul(
        d["x"].to(DEV), nz, d["scale"].to(DEV), None if d["offset"] is None else d["offset"].to(DEV),
        bias=None if b is None else b.to(DEV), antiquant_group_size=group)
    _close(out, _w8_ref(oracle, d, group, x_dtype, bias=b), x_dtype)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (2048, 11008, 4096, 128, True, torch.bfloat16, False),   # the cfg3 prefill shape with int8 weights
    (320, 8192, 1024, 64, False, torch.float16, True),       # 64-row groups: one step per group; ragged rows
    (512, 6144, 768, 0, True, torch.bfloat16, False),        # per channel: one group of 768 rows
    (1000, 4096, 2048, 256, True, torch.bfloat16, True),     # four steps per group, last row tile of 104 rows
])
def test_w8a16_nz_prefill_kernel(ops, oracle, M, N, K, group, offset, x_dtype, bias):
    """The NZ prefill kernel on int8 NZ weights (64-row steps, one 1 KB block per 16 columns per step): every
    output element within rtol/atol 1e-2 of the float64 dequant-matmul, which is pinned against the C oracle on
    four rows; and against the row-major int8 path on the same weight."""
    say(f"w8a16 NZ prefill M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    d = _w8(M, N, K, group, offset, x_dtype, seed=M + N + K + 3)
    b = torch.randn(N, generator=torch.Generator().manual_seed(8)).to(x_dtype) if bias else None
    nz = ops.npu_format_cast(d["w"].to(DEV), 29)
    out = ops.npu_weight_quant_batchmatmul(
        d["x"].to(DEV), nz, d["scale"].to(DEV), None if d["offset"] is None else d["offset"].to(DEV),
        bias=None if b is None else b.to(DEV), antiquant_group_size=group)
    ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], group, bias=b)
    rows = np.r_[0:2, M - 2:M]
    pin = _w8_ref(oracle, dict(d, x=d["x"][rows]), group, x_dtype, bias=b)
    pin_diff = (W.from_bits(pin, x_dtype).float() - ref64[rows].float()).abs()
    assert pin_diff.max().item() <= 2.0**-7 * ref64[rows].abs().max().item() + 1e-3
    torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M,N,K,group,offset,x_dtype,bias", [
    (1024, 2048, 1024, 128, True, torch.bfloat16, True),     # 8 x 8 tiles, two steps per group
    (1100, 2048, 2048, 64, False, torch.float16, False),     # one step per group, last row tile of 76 rows
])
def test_w8a16_row_major_cast_to_nz(ops, oracle, plan, M, N, K, group, offset, x_dtype, bias):
    """M >= 1024 on a row-major int8 [K, N] weight: the call casts the weight to NZ in its workspace (which the
    size query reports) and runs the NZ prefill kernel on the copy; within rtol/atol 1e-2 of the float64
    dequant-matmul and of the row-major prefill kernel (the cast switched off by the debug override)."""
    say(f"w8a16 row-major cast to NZ M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    L = ops.abi()
    ws = ctypes.c_size_t(0)
    assert L.qk_weight_quant_bmm_workspace_size(M, N, K, ops.QK_I8, group, ctypes.byref(ws)) == 0
    assert ws.value >= 4096 + K * N, "the workspace holds the cast weight"
    d = _w8(M, N, K, group, offset, x_dtype, seed=M + N + K + 4)
    b = torch.randn(N, generator=torch.Generator().manual_seed(9)).to(x_dtype) if bias else None
    args = (d["x"].to(DEV), d["w"].to(DEV), d["scale"].to(DEV), None if d["offset"] is None else d["offset"].to(DEV))
    out = ops.npu_weight_quant_batchmatmul(*args, bias=None if b is None else b.to(DEV), antiquant_group_size=group)
    ref64 = exact.wq_dequant_matmul(d["x"], d["w"], d["scale"], d["offset"], group, bias=b)
    torch.testing.assert_close(out.cpu().float(), ref64.float(), rtol=1e-2, atol=1e-2)
    plan("w4nz=off")
    rm = ops.npu_weight_quant_batchmatmul(*args, bias=None if b is None else b.to(DEV), antiquant_group_size=group)
    torch.testing.assert_close(out.float(), rm.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("w8,M,N,K,group,offset,x_dtype,bias", [
    (False, 2048, 11008, 4096, 128, True, torch.bfloat16, False),   # cfg3: 688 tiles, one step per group
    (False, 1024, 11008, 4096, 256, False, torch.float16, True),    # 344 tiles, two steps per group
    (False, 2100, 4096, 1024, 128, True, torch.bfloat16, True),     # 272 tiles, last row tile of 52 rows
    (True, 2048, 11008, 4096, 128, True, torch.bfloat16, False),    # int8: two 64-row steps per group
    (True, 1100, 8192, 2048, 64, False, torch.float16, True),       # int8: one step per group, 76-row last tile
])
def test_nz_prefill_stream_k_bits(ops, plan, w8, M, N, K, group, offset, x_dtype, bias):
    """Shapes whose tiles leave part of the last round of CUs idle run the NZ prefill kernel as stream-K (one
    workgroup per CU, equal shares of all tiles' groups; the size query reports the partial slots). A split
    tile's second segment continues from the first one's folded accumulator, or runs the whole tile when it
    arrives first, so the output is bit for bit the kernel's with whole tiles per workgroup (debug override
    nzg_sk=0) -- also when every tail segment runs first and so takes the whole-tile path (nzg_sk=tailfirst),
    and with or without the whole-tile rounds the plan runs before the stream-K share (nzg_sk_dp=0: stream-K
    throughout; shapes of two rounds and more run one round of whole tiles first by default).
    Through the C ABI with a 0xA5-filled workspace: the partial slots were written, the output is the op's."""
    say(f"NZ prefill stream-K {'int8' if w8 else 'int4'} M={M} N={N} K={K} group={group} offset={offset} "
        f"{x_dtype} bias={bias}")
    L = ops.abi()
    if w8:
        d = _w8(M, N, K, group, offset, x_dtype, seed=M + N + K + 11)
        w, wdt = ops.npu_format_cast(d["w"].to(DEV), 29), ops.QK_I8_NZ
    else:
        d = _inputs(M, N, K, group, offset, x_dtype, seed=M + N + K + 11)
        w, wdt = ops.npu_format_cast(d["w_packed"].to(DEV), 29), ops.QK_I4_NZ
    b = torch.randn(N, generator=torch.Generator().manual_seed(12)).to(x_dtype).to(DEV) if bias else None
    x, sc = d["x"].to(DEV), d["scale"].to(DEV)
    off = None if d["offset"] is None else d["offset"].to(DEV)
    need = ctypes.c_size_t(0)
    assert L.qk_weight_quant_bmm_workspace_size(M, N, K, wdt, group, ctypes.byref(need)) == 0
    base = 4096 + (K // group) * M * 4
    assert need.value >= base + (1 << 20), "the size query reports the stream-K partial slots"

    def run():
        return ops.npu_weight_quant_batchmatmul(x, w, sc, off, bias=b, antiquant_group_size=group)

    sk = run()
    plan("nzg_sk=0")
    whole = run()
    plan("nzg_sk=tailfirst")
    tails_first = run()
    plan("nzg_sk_dp=0")
    sk_throughout = run()
    plan("")
    torch.cuda.synchronize()
    assert torch.equal(sk.view(torch.int16), whole.view(torch.int16)), "stream-K differs from whole tiles"
    assert torch.equal(tails_first.view(torch.int16), whole.view(torch.int16)), "the whole-tile fallback differs"
    assert torch.equal(sk_throughout.view(torch.int16), whole.view(torch.int16)), "stream-K throughout differs"

    ws = torch.full((need.value,), 0xA5, dtype=torch.uint8, device=DEV)
    out = torch.empty(M, N, dtype=x_dtype, device=DEV)
    XD = CODE[x_dtype]
    rc = L.qk_weight_quant_bmm(x.data_ptr(), XD, w.data_ptr(), wdt, sc.data_ptr(),
                               None if off is None else off.data_ptr(), F16, M, N, K, group,
                               None if b is None else b.data_ptr(), 0 if b is None else XD, out.data_ptr(), XD,
                               ws.data_ptr(), need.value, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ops.last_error()
    torch.cuda.synchronize()
    slots = ws[need.value - (1 << 20):]
    assert bool((slots != 0xA5).any()), "no stream-K partial slot was written"
    assert torch.equal(out.view(torch.int16), whole.view(torch.int16))
    # the no-allocation entry point: the partial slots do not fit its scratch, so whole tiles, the same bits
    assert need.value > ops.QK_NOALLOC_SCRATCH_BYTES
    na = torch.empty(M, N, dtype=x_dtype, device=DEV)
    rc = L.qk_weight_quant_bmm_noalloc(x.data_ptr(), XD, w.data_ptr(), wdt, sc.data_ptr(),
                                       None if off is None else off.data_ptr(), F16, M, N, K, group,
                                       None if b is None else b.data_ptr(), 0 if b is None else XD, na.data_ptr(), XD,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ops.last_error()
    torch.cuda.synchronize()
    assert torch.equal(na.view(torch.int16), whole.view(torch.int16))


def test_abi_w8_nz(ops, oracle):
    say("ABI qk_weight_quant_bmm QK_I8_NZ M=16 N=1024 K=2048")
    L = ops.abi()
    d = _w8(16, 1024, 2048, 128, True, torch.bfloat16, seed=13)
    nz = ops.npu_format_cast(d["w"].to(DEV), 29)
    x, sc, off = d["x"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
    ws = ctypes.c_size_t(1)
    assert L.qk_weight_quant_bmm_workspace_size(16, 1024, 2048, ops.QK_I8_NZ, 128, ctypes.byref(ws)) == 0
    assert ws.value == 0
    out = torch.empty(16, 1024, dtype=torch.bfloat16, device=DEV)
    rc = L.qk_weight_quant_bmm(x.data_ptr(), BF16, nz.data_ptr(), ops.QK_I8_NZ, sc.data_ptr(), off.data_ptr(), F16,
                               16, 1024, 2048, 128, None, 0, out.data_ptr(), BF16, None, 0,
                               torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ops.last_error()
    torch.cuda.synchronize()
    _close(out, _w8_ref(oracle, d, 128, torch.bfloat16), torch.bfloat16)


# ----------------------------------------------------------------------------- seeded random decode shapes

def _random_decode_shapes(seed, n):
    """M <= 64 decode shapes the NZ decode kernel plans for: K = 128 * S superblocks (S from 1 to 64, so 1 to 4
    superblocks per wave and 1 to 16 waves), groups of 128 / 256 / 512 rows or per channel, N any multiple of 16
    (sized so the C oracle finishes in well under a second)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        S = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16, 24, 32, 48, 64]))
        K = 128 * S
        group = int(rng.choice([g for g in (128, 256, 512) if K % g == 0] + [0]))
        M = int(rng.integers(1, 65))
        nmax = max(2, min(400, int(6e7 // (M * K * 16))))
        N = 16 * int(rng.integers(1, nmax + 1))
        out.append((M, N, K, group, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("M,N,K,group,offset,fp16,bias", _random_decode_shapes(2026, 12))
def test_w4a16_nz_decode_random_shapes(ops, oracle, M, N, K, group, offset, fp16, bias):
    """The NZ decode kernel (x rows by direct-to-LDS loads, non-temporal weight stream) on seeded random shapes
    against the oracle, within rtol / atol 1e-2."""
    x_dtype = torch.float16 if fp16 else torch.bfloat16
    say(f"w4a16 NZ decode random M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    d = _inputs(M, N, K, group, offset, x_dtype, seed=M * 7 + N + K)
    b = torch.randn(N, generator=torch.Generator().manual_seed(N)).to(x_dtype) if bias else None
    nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)
    out = _run(ops, d, group, nz, bias=b)
    _close(out, _ref(oracle, d, group, bias=b, x_dtype=x_dtype), x_dtype)


@pytest.mark.parametrize("M,N,K,group,offset,fp16,bias", _random_decode_shapes(7, 8))
def test_w8a16_nz_decode_random_shapes(ops, oracle, M, N, K, group, offset, fp16, bias):
    """The same kernel on int8 NZ weights (two 1 KB blocks per 128 rows) on seeded random shapes."""
    x_dtype = torch.float16 if fp16 else torch.bfloat16
    say(f"w8a16 NZ decode random M={M} N={N} K={K} group={group} offset={offset} {x_dtype} bias={bias}")
    d = _w8(M, N, K, group, offset, x_dtype, seed=M * 5 + N + K)
    b = torch.randn(N, generator=torch.Generator().manual_seed(N + 1)).to(x_dtype) if bias else None
    nz = ops.npu_format_cast(d["w"].to(DEV), 29)
    out = ops.npu_weight_quant_batchmatmul(
        d["x"].to(DEV), nz, d["scale"].to(DEV), None if d["offset"] is None else d["offset"].to(DEV),
        bias=None if b is None else b.to(DEV), antiquant_group_size=group)
    _close(out, _w8_ref(oracle, d, group, x_dtype, bias=b), x_dtype)
