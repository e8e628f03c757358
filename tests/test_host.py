"""Host-side checks that need no GPU: the C ABI library loads and exports every
symbol include/qk_abi.h declares, invalid arguments are refused before any
launch, and the torch.ops.npu schemas infer shapes and raise the documented
errors (Meta tensors run the same checks as the GPU implementations)."""
import ctypes
import os
import re

import pytest
import torch

import op_plugin_amd as q

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
F16, BF16, F32, I8, I32 = 1, 2, 3, 4, 5


def _declared_functions():
    src = open(os.path.join(ROOT, "include", "qk_abi.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(qk_\w+)\s*\(", src, flags=re.M)))


def test_abi_exports_every_declared_symbol():
    names = _declared_functions()
    assert len(names) >= 8
    L = ctypes.CDLL(q.LIB_PATH)
    for n in names:
        assert hasattr(L, n), f"{n} declared in qk_abi.h but not exported"
    assert set(names) == set(q.ABI_SYMBOLS)
    assert q.abi().qk_abi_version() == 6


def test_debug_plan_override_parsing():
    """The planners' one debug override: accepted specs, and refusal (with the override unchanged) of
    specs it does not understand.  Nothing is launched."""
    for spec in ("", "w4_stream=16:4:4", "w4_stream=off", "w4_gemm=force,skinny_splits=4", "qmm_dma=0", "qmm_mid=0",
                 "mid_bm=32,mid_split=2", "mid_bn=64", "qmm_bm128=0",
                 "w4_splits=8,w4_gemm=nodma", "w4nz=off", "w4nz_wg=172", "w4nz_nit=4", "nzg_sk=0",
                 "nzg_sk=tailfirst", "nzg_sk=1,nzg_sk_dp=0", "skinny_pf=2", "w4_stream_wpl=32", "w4_stream_wpl=64",
                 "qmm_rev=0", "qmm_rev=1", "qmm_small=0", "qmm_small=8"):
        q.debug_set_plan(spec)
    for bad in ("w4_stream=12:4:2", "w4_gemm=maybe", "skinny_splits=3", "nonsense", "qmm_dma=2", "w4nz=on",
                "w4nz_wg=0", "qmm_bm128=2", "nzg_sk=2", "nzg_sk_dp=-1", "skinny_pf=4", "w4_stream_wpl=8",
                "qmm_rev=2", "qmm_small=3"):
        with pytest.raises(ValueError, match="not understood"):
            q.debug_set_plan(bad)
    q.debug_set_plan("")


def test_w8a8_split_plan_workspace_sizes():
    """The K-split plans' workspaces (host arithmetic only).  cfg5's down projection (512 x 4096 x 14336) has 32
    tiles of 256 x 256, split 8 ways to fill the CUs; on 128-row tiles it has 64, split 4 ways: half the int32
    partials.  The NZ weight always runs the 128-row split; a row-major weight may fall back to the 256-row one
    (another kernel) and asks room for either."""
    L = q.abi()
    ws = ctypes.c_size_t(0)
    M, N, K = 512, 4096, 14336
    ctr = 4096  # QK_SPLIT_COUNTER_BYTES
    try:
        assert L.qk_quant_matmul_nz_workspace_size(M, N, K, BF16, ctypes.byref(ws)) == 0
        assert ws.value == ctr + 4 * M * N * 4
        assert L.qk_quant_matmul_workspace_size(M, N, K, BF16, ctypes.byref(ws)) == 0
        assert ws.value == ctr + 8 * M * N * 4
        # a ragged M pads the 128-row tiles' partials to whole tiles: 300 rows -> 3 tiles, 4 splits
        assert L.qk_quant_matmul_nz_workspace_size(300, 4096, 8192, BF16, ctypes.byref(ws)) == 0
        assert ws.value == ctr + 4 * 384 * 4096 * 4
        # M = 128 on a wide [K,N] weight (11008 x 4096) runs 128-row tiles with 4 K splits (the cost model's
        # choice over qmm_mid); cfg1 (4096 x 4096) stays on qmm_mid, which needs no workspace
        assert L.qk_quant_matmul_workspace_size(128, 11008, 4096, BF16, ctypes.byref(ws)) == 0
        assert ws.value == ctr + 4 * 128 * 11008 * 4
        assert L.qk_quant_matmul_workspace_size(128, 4096, 4096, BF16, ctypes.byref(ws)) == 0
        assert ws.value == 0
        # on NZ blocks (whose mid-M kernel streams better) 128 x 4096 x 14336 takes 8 splits, 128 x 11008 x 4096
        # stays on the mid-M kernel
        assert L.qk_quant_matmul_nz_workspace_size(128, 4096, 14336, BF16, ctypes.byref(ws)) == 0
        assert ws.value == ctr + 8 * 128 * 4096 * 4
        assert L.qk_quant_matmul_nz_workspace_size(128, 11008, 4096, BF16, ctypes.byref(ws)) == 0
        assert ws.value == 0
        q.debug_set_plan("qmm_small=0")
        assert L.qk_quant_matmul_workspace_size(128, 11008, 4096, BF16, ctypes.byref(ws)) == 0
        assert ws.value == 0
        assert L.qk_quant_matmul_nz_workspace_size(128, 4096, 14336, BF16, ctypes.byref(ws)) == 0
        assert ws.value == 0
        q.debug_set_plan("qmm_bm128=0")
        assert L.qk_quant_matmul_nz_workspace_size(M, N, K, BF16, ctypes.byref(ws)) == 0
        assert ws.value == ctr + 8 * M * N * 4
        assert L.qk_quant_matmul_nz_workspace_size(300, 4096, 8192, BF16, ctypes.byref(ws)) == 0
        assert ws.value == ctr + 8 * 300 * 4096 * 4
    finally:
        q.debug_set_plan("")


def test_abi_refuses_bad_arguments_without_launch():
    L = q.abi()
    assert L.qk_dynamic_quant(None, 9, 4, 16, None, None, None, None) == q.QK_ERR_ARG
    assert "float16 or bfloat16" in q.last_error()
    assert L.qk_dynamic_quant(None, F16, 4, 16, None, None, None, None) == q.QK_ERR_ARG
    assert "null pointer" in q.last_error()
    assert L.qk_dynamic_quant(None, F16, 0, 16, None, None, None, None) == q.QK_OK
    assert q.last_error() == ""
    fake = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    rc = L.qk_quant_matmul(fake, 64, fake, 2, 2, 4, 32, 64, fake, 32, None, 0, None, None, 0, fake, BF16, None, 0, None)
    assert rc == q.QK_ERR_ARG and "transposed view" in q.last_error()
    rc = L.qk_quant_matmul(fake, 64, fake, 32, 1, 4, 32, 64, fake, 7, None, 0, None, None, 0, fake, BF16, None, 0, None)
    assert rc == q.QK_ERR_ARG and "scale" in q.last_error()
    rc = L.qk_quant_matmul(fake, 200000, fake, 32, 1, 4, 32, 200000, fake, 32, None, 0, None, None, 0, fake, BF16,
                           None, 0, None)
    assert rc == q.QK_ERR_UNSUPPORTED and "int32-exact" in q.last_error()
    rc = L.qk_quant_matmul(fake, 64, fake, 32, 1, 4, 32, 64, fake, 32, fake, 32, None, None, 0, fake, BF16, None, 0,
                           None)
    assert rc == q.QK_ERR_ARG and "offset" in q.last_error()
    rc = L.qk_weight_quant_bmm(fake, BF16, fake, I32, fake, None, F16, 4, 12, 128, 128, None, 0, fake, BF16, None, 0,
                               None)
    assert rc == q.QK_ERR_ARG and "N % 8" in q.last_error()
    rc = L.qk_weight_quant_bmm(fake, BF16, fake, I32, fake, None, F16, 4, 16, 100, 128, None, 0, fake, BF16, None, 0,
                               None)
    assert rc == q.QK_ERR_ARG and "multiple of antiquant_group_size" in q.last_error()
    ws = ctypes.c_size_t(123)
    assert L.qk_weight_quant_bmm_workspace_size(16, 11008, 4096, I32, 128, ctypes.byref(ws)) == 0
    assert L.qk_int4_pack(fake, I8, 4, 12, fake, None) == q.QK_ERR_ARG
    assert L.qk_quantize_per_tensor(fake, I32, 4, 0.1, 0, fake, I8, None) == q.QK_ERR_ARG
    assert L.qk_quantize_per_tensor(fake, F32, 4, -1.0, 0, fake, I8, None) == q.QK_ERR_ARG
    assert L.qk_quantize_per_tensor(fake, F32, 4, 0.1, 0, fake, F16, None) == q.QK_ERR_ARG
    assert L.qk_quantize_per_channel(fake, F32, 2, 3, 4, None, None, fake, I8, None) == q.QK_ERR_ARG
    assert L.qk_quantize_per_channel(None, F32, 0, 3, 4, None, None, None, I8, None) == q.QK_OK
    assert L.qk_dequantize(fake, F32, 4, fake, None) == q.QK_ERR_ARG
    assert L.qk_dequantize(None, I8, 4, None, None) == q.QK_ERR_ARG and "null pointer" in q.last_error()
    # NZ weights: shape rules, supported casts, overlap
    rc = L.qk_weight_quant_bmm(fake, BF16, fake, q.QK_I4_NZ, fake, None, F16, 4, 24, 128, 128, None, 0, fake, BF16,
                               None, 0, None)
    assert rc == q.QK_ERR_ARG and "N % 16" in q.last_error()
    nd, nz = q.ACL_FORMAT_ND, q.ACL_FORMAT_FRACTAL_NZ
    assert L.qk_weight_format_cast(fake, nd, fake, nz, F16, 128, 16, None) == q.QK_ERR_UNSUPPORTED
    assert L.qk_weight_format_cast(fake, nd, fake, nz, I8, 96, 16, None) == q.QK_ERR_ARG
    assert L.qk_weight_format_cast(fake, nd, fake, 3, I32, 128, 16, None) == q.QK_ERR_UNSUPPORTED
    assert L.qk_weight_format_cast(fake, nd, fake, nz, I32, 100, 16, None) == q.QK_ERR_ARG
    assert L.qk_weight_format_cast(ctypes.c_void_p(4096), nd, ctypes.c_void_p(4096 + 512), nz, I32, 128, 16,
                                   None) == q.QK_ERR_ARG and "overlap" in q.last_error()
    assert L.qk_weight_format_cast(None, nz, None, nd, I32, 0, 16, None) == q.QK_OK
    assert L.qk_weight_quant_bmm_workspace_size(16, 11008, 4096, q.QK_I4_NZ, 128, ctypes.byref(ws)) == 0
    assert ws.value == 0   # the NZ decode kernel needs no workspace
    assert L.qk_weight_quant_bmm_workspace_size(16, 11008, 4096, q.QK_I4_NZ, 64, ctypes.byref(ws)) == 0
    assert ws.value >= 4096 + 4096 * 11008 // 2   # short groups: the ND weight is rebuilt in the workspace
    assert L.qk_rms_norm(fake, 9, fake, 4, 64, 1e-6, fake, None, None) == q.QK_ERR_ARG
    assert "float16 or bfloat16" in q.last_error()
    assert L.qk_rms_norm(fake, BF16, fake, 4, 0, 1e-6, fake, None, None) == q.QK_ERR_ARG and "D > 0" in q.last_error()
    assert L.qk_rms_norm(fake, BF16, fake, 4, 64, -1.0, fake, None, None) == q.QK_ERR_ARG
    assert L.qk_rms_norm(None, BF16, fake, 4, 64, 1e-6, fake, None, None) == q.QK_ERR_ARG
    assert L.qk_rms_norm(None, BF16, None, 0, 64, 1e-6, None, None, None) == q.QK_OK
    assert L.qk_rms_norm_quant(fake, BF16, fake, 4, 64, 1e-6, fake, None, None, None) == q.QK_ERR_ARG
    assert L.qk_rms_norm_quant(fake, 3, fake, 4, 64, 1e-6, fake, fake, None, None) == q.QK_ERR_ARG
    assert "float16 or bfloat16 (got" in q.last_error()   # float32 x: the fused quantization takes 16-bit rows
    assert L.qk_swiglu(fake, F16, -1, 8, fake, None) == q.QK_ERR_ARG
    assert L.qk_swiglu(None, F16, 3, 8, None, None) == q.QK_ERR_ARG and "null pointer" in q.last_error()
    assert L.qk_swiglu_quant(fake, BF16, 3, 0, fake, fake, None) == q.QK_ERR_ARG and "empty" in q.last_error()
    # the gate-up GEMM with the SwiGLU fused (x2 [K, 2I] rows: format ND, stride 2I)
    nd = q.ACL_FORMAT_ND
    assert L.qk_quant_matmul_swiglu(fake, 256, fake, nd, 512, 4, 256, 256, fake, 512, None, fake, F32,
                                    None) == q.QK_ERR_ARG and "float16 or bfloat16" in q.last_error()
    assert L.qk_quant_matmul_swiglu(fake, 256, fake, 5, 512, 4, 256, 256, fake, 512, None, fake, BF16,
                                    None) == q.QK_ERR_ARG and "x2_format" in q.last_error()
    assert L.qk_quant_matmul_swiglu(fake, 256, fake, nd, 300, 4, 256, 256, fake, 512, None, fake, BF16,
                                    None) == q.QK_ERR_ARG and "x2_stride_k" in q.last_error()
    assert L.qk_quant_matmul_swiglu(fake, 256, fake, nd, 512, 4, 256, 256, fake, 7, None, fake, BF16,
                                    None) == q.QK_ERR_ARG and "scale" in q.last_error()
    assert L.qk_quant_matmul_swiglu(None, 256, None, nd, 512, 0, 256, 256, None, 512, None, None, BF16,
                                    None) == q.QK_OK
    assert L.qk_quant_matmul_swiglu_quant_workspace_size(512, 14336, ctypes.byref(ws)) == q.QK_OK
    assert ws.value == 512 * 14336 * 2 + 512 * 112 * 4   # h, then the per-tile row absmax
    need = ws.value
    args = (fake, 4096, fake, nd, 28672, 512, 14336, 4096, fake, 28672, fake, BF16, fake, fake)
    assert L.qk_quant_matmul_swiglu_quant(*args, fake, need - 256, None) == q.QK_ERR_WORKSPACE
    assert L.qk_quant_matmul_swiglu_quant(*args, None, need, None) == q.QK_ERR_WORKSPACE
    assert L.qk_quant_matmul_swiglu_quant(*args[:11], F32, *args[12:], ctypes.c_void_p(4096), need,
                                          None) == q.QK_ERR_ARG and "float16 or bfloat16" in q.last_error()
    assert L.qk_quant_matmul_swiglu_quant(*args[:12], None, fake, ctypes.c_void_p(4096), need,
                                          None) == q.QK_ERR_ARG and "null output" in q.last_error()
    assert L.qk_quant_matmul_swiglu_quant(None, 4096, None, nd, 28672, 0, 14336, 4096, None, 28672, None, BF16, None,
                                          None, None, 0, None) == q.QK_OK


def _m(shape, dtype):
    return torch.empty(shape, dtype=dtype, device="meta")


def test_schemas_registered():
    for name in ("npu_dynamic_quant", "npu_quant_matmul", "npu_weight_quant_batchmatmul",
                 "npu_convert_weight_to_int4pack", "npu_format_cast", "quantize_per_tensor", "quantize_per_channel",
                 "dequantize", "npu_rms_norm", "npu_swiglu", "npu_rms_norm_dynamic_quant",
                 "npu_swiglu_dynamic_quant", "npu_quant_matmul_swiglu", "npu_quant_matmul_swiglu_quant"):
        assert hasattr(torch.ops.npu, name)
    s = str(torch.ops.npu.npu_quant_matmul.default._schema)
    assert "pertoken_scale" in s and "ScalarType? output_dtype" in s


def test_meta_shapes():
    y, s = q.npu_dynamic_quant(_m((2, 3, 64), torch.bfloat16))
    assert y.shape == (2, 3, 64) and y.dtype == torch.int8 and s.shape == (2, 3) and s.dtype == torch.float32
    out = q.npu_quant_matmul(_m((2, 5, 64), torch.int8), _m((64, 48), torch.int8), _m((48,), torch.float32),
                             pertoken_scale=_m((10,), torch.float32), bias=_m((48,), torch.bfloat16),
                             output_dtype=torch.bfloat16)
    assert out.shape == (2, 5, 48) and out.dtype == torch.bfloat16
    assert q.npu_quant_matmul(_m((4, 64), torch.int8), _m((64, 8), torch.int8), _m((1,), torch.float32)).dtype \
        == torch.int8
    out = q.npu_weight_quant_batchmatmul(_m((16, 4096), torch.bfloat16), _m((4096, 1376), torch.int32),
                                         _m((32, 11008), torch.float16), _m((32, 11008), torch.float16),
                                         antiquant_group_size=128)
    assert out.shape == (16, 11008) and out.dtype == torch.bfloat16
    assert q.npu_convert_weight_to_int4pack(_m((64, 96), torch.int32)).shape == (64, 12)
    assert q.npu_convert_weight_to_int4pack(_m((256, 96), torch.int32), inner_k_tiles=4).shape == (6, 2, 64, 4)
    nzw = q.npu_format_cast(_m((4096, 1376), torch.int32), 29)
    assert nzw.shape == (688, 32, 64, 4) and q.get_npu_format(nzw) == 29
    assert q.npu_format_cast(nzw, 2).shape == (4096, 1376) and q.npu_format_cast(nzw, 29) is nzw
    w8z = q.npu_format_cast(_m((4096, 11008), torch.int8), 29)
    assert w8z.shape == (688, 64, 64, 16) and q.get_npu_format(w8z) == 29
    assert q.npu_weight_quant_batchmatmul(_m((16, 4096), torch.bfloat16), w8z, _m((32, 11008), torch.float16),
                                          antiquant_group_size=128).shape == (16, 11008)
    out = q.npu_quant_matmul(_m((3, 7, 4096), torch.int8), w8z, _m((11008,), torch.float32),
                             pertoken_scale=_m((21,), torch.float32), output_dtype=torch.bfloat16)   # W8A8, NZ weight
    assert out.shape == (3, 7, 11008) and out.dtype == torch.bfloat16
    assert q.quantize_per_tensor(_m((3, 8), torch.float16), 0.1, 2, torch.quint8).dtype == torch.uint8
    qq = q.quantize_per_channel(_m((3, 8), torch.bfloat16), _m((8,), torch.float64), _m((8,), torch.int64), -1,
                                torch.qint32)
    assert qq.shape == (3, 8) and qq.dtype == torch.int32
    assert q.dequantize(_m((2, 2), torch.uint8)).dtype == torch.float32
    out = q.npu_weight_quant_batchmatmul(_m((16, 4096), torch.bfloat16), nzw, _m((32, 11008), torch.float16),
                                         _m((32, 11008), torch.float16), antiquant_group_size=128)
    assert out.shape == (16, 11008) and out.dtype == torch.bfloat16
    y, rstd = q.npu_rms_norm(_m((2, 7, 4096), torch.bfloat16), _m((4096,), torch.bfloat16))
    assert y.shape == (2, 7, 4096) and y.dtype == torch.bfloat16 and rstd.shape == (2, 7, 1) \
        and rstd.dtype == torch.float32
    y, rstd = q.npu_rms_norm(_m((3, 4, 8), torch.float16), _m((4, 8), torch.float16))   # 2-D gamma
    assert y.shape == (3, 4, 8) and rstd.shape == (3, 1, 1)
    y, rstd = q.npu_rms_norm(_m((1024, 12288), torch.float32), _m((12288,), torch.float32))
    assert y.dtype == torch.float32 and rstd.shape == (1024, 1)
    qq, sc, rstd = q.npu_rms_norm_dynamic_quant(_m((512, 4096), torch.bfloat16), _m((4096,), torch.bfloat16))
    assert qq.dtype == torch.int8 and qq.shape == (512, 4096) and sc.shape == (512,) and rstd.shape == (512, 1)
    assert q.npu_swiglu(_m((512, 28672), torch.bfloat16)).shape == (512, 14336)
    qq, sc = q.npu_swiglu_dynamic_quant(_m((2, 5, 64), torch.float16), dim=2)
    assert qq.shape == (2, 5, 32) and qq.dtype == torch.int8 and sc.shape == (2, 5)
    h = q.npu_quant_matmul_swiglu(_m((2, 256, 4096), torch.int8), _m((4096, 28672), torch.int8),
                                  _m((28672,), torch.float32), pertoken_scale=_m((512,), torch.float32))
    assert h.shape == (2, 256, 14336) and h.dtype == torch.bfloat16
    w8gu = q.npu_format_cast(_m((4096, 28672), torch.int8), 29)
    h = q.npu_quant_matmul_swiglu(_m((512, 4096), torch.int8), w8gu, _m((1,), torch.float32),
                                  output_dtype=torch.float16)
    assert h.shape == (512, 14336) and h.dtype == torch.float16
    qq, qs = q.npu_quant_matmul_swiglu_quant(_m((2, 256, 4096), torch.int8), w8gu, _m((28672,), torch.float32))
    assert qq.shape == (2, 256, 14336) and qq.dtype == torch.int8 and qs.shape == (2, 256) and qs.dtype == torch.float32


def test_storage_format_is_recorded_not_inferred():
    """get_npu_format reads the format recorded with a tensor's storage by npu_format_cast /
    npu_convert_weight_to_int4pack(inner_k_tiles=4), as the reference reads its storage descriptor
    (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:57-66): a tensor of the same shape made any other way is ND,
    and a view that does not cover the storage as cast is ND."""
    nz = q.npu_format_cast(_m((256, 64), torch.int8), 29)
    assert nz.shape == (4, 4, 64, 16) and q.get_npu_format(nz) == 29
    assert q.get_npu_format(nz.view(4, 4, 64, 16)) == 29          # the same storage, viewed whole
    assert q.get_npu_format(_m((4, 4, 64, 16), torch.int8)) == 2  # the shape alone is not the format
    assert q.get_npu_format(nz[1:]) == 2                          # part of the storage
    assert q.get_npu_format(nz.reshape(16, 64, 16)) == 2          # other sizes
    w4 = q.npu_convert_weight_to_int4pack(_m((256, 32), torch.int32), inner_k_tiles=4)
    assert q.get_npu_format(w4) == 29 and q.get_npu_format(q.npu_format_cast(w4, 2)) == 2
    assert q.get_npu_format(torch.zeros(2, 2)) == 2               # any device
    # a raw 4-D int8 tensor of the NZ shape is a batch of [64, 16] weights, not an NZ weight
    out = q.npu_quant_matmul(_m((5, 64), torch.int8), _m((4, 1, 64, 16), torch.int8), _m((1,), torch.float32),
                             output_dtype=torch.int32)
    assert out.shape == (4, 1, 5, 16)


def test_meta_batched_weights():
    """Weights with batch dims follow the reference's matmul output rule
    (op_plugin/ops/base_ops/opapi/MatmulKernelNpuOpApi.cpp:45-73): a 2-D x is broadcast over the weight's batch,
    and the batch dims of x and weight broadcast against each other."""
    f32, i8, i32, bf16, f16 = torch.float32, torch.int8, torch.int32, torch.bfloat16, torch.float16
    assert q.npu_quant_matmul(_m((5, 64), i8), _m((3, 64, 48), i8), _m((48,), f32),
                              pertoken_scale=_m((5,), f32), output_dtype=bf16).shape == (3, 5, 48)
    assert q.npu_quant_matmul(_m((2, 5, 64), i8), _m((3, 1, 64, 48), i8), _m((1,), f32),
                              output_dtype=i32).shape == (3, 2, 5, 48)
    assert q.npu_quant_matmul(_m((2, 5, 64), i8), _m((2, 48, 64), i8).transpose(-1, -2), _m((48,), f32),
                              pertoken_scale=_m((10,), f32), output_dtype=f16).shape == (2, 5, 48)
    out = q.npu_weight_quant_batchmatmul(_m((2, 16, 4096), bf16), _m((2, 4096, 1376), i32), _m((2, 32, 11008), f16),
                                         _m((2, 32, 11008), f16), antiquant_group_size=128)
    assert out.shape == (2, 16, 11008) and out.dtype == bf16
    assert q.npu_weight_quant_batchmatmul(_m((16, 256), f16), _m((4, 256, 64), i8), _m((64,), f16)).shape \
        == (4, 16, 64)


@pytest.mark.parametrize("call,msg", [
    (lambda: q.npu_dynamic_quant(_m((4, 8), torch.float32)), "float16 or bfloat16"),
    (lambda: q.npu_quant_matmul_swiglu(_m((4, 64), torch.int8), _m((64, 9), torch.int8), _m((9,), torch.float32)),
     "even"),
    (lambda: q.npu_quant_matmul_swiglu(_m((4, 64), torch.int8), _m((32, 8), torch.int8), _m((8,), torch.float32)),
     "must equal"),
    (lambda: q.npu_quant_matmul_swiglu(_m((4, 64), torch.int8), _m((64, 8), torch.int8), _m((8,), torch.float32),
                                       output_dtype=torch.float32), "bfloat16 or float16"),
    (lambda: q.npu_dynamic_quant(_m((4, 8), torch.float16), smooth_scales=_m((7,), torch.float32)), "smooth_scales"),
    (lambda: q.npu_quant_matmul(_m((4, 64), torch.int8), _m((32, 8), torch.int8), _m((8,), torch.float32)),
     "must equal"),
    (lambda: q.npu_quant_matmul(_m((4, 64), torch.int8), _m((64, 8), torch.int8), _m((8,), torch.float32),
                                pertoken_scale=_m((3,), torch.float32), output_dtype=torch.bfloat16), "pertoken_scale"),
    (lambda: q.npu_quant_matmul(_m((4, 64), torch.int8), _m((64, 8), torch.int8), _m((8,), torch.float32),
                                pertoken_scale=_m((4,), torch.float32)), "pertoken_scale needs"),
    (lambda: q.npu_quant_matmul(_m((4, 64), torch.int8), _m((64, 8), torch.int8), _m((8,), torch.float32),
                                bias=_m((8,), torch.bfloat16), output_dtype=torch.int32), "int32 bias"),
    (lambda: q.npu_weight_quant_batchmatmul(_m((2, 100), torch.bfloat16), _m((100, 2), torch.int32),
                                            _m((1, 16), torch.float16), antiquant_group_size=64), "multiple"),
    (lambda: q.npu_weight_quant_batchmatmul(_m((2, 128), torch.bfloat16), _m((128, 2), torch.int32),
                                            _m((2, 16), torch.float16), antiquant_group_size=128), "antiquant_scale"),
    (lambda: q.npu_weight_quant_batchmatmul(_m((2, 128), torch.bfloat16), _m((128, 2), torch.int32),
                                            _m((1, 16), torch.float16), quant_scale=_m((16,), torch.float32),
                                            antiquant_group_size=128), "not supported"),
    (lambda: q.npu_convert_weight_to_int4pack(_m((4, 12), torch.int32)), "multiple of 8"),
    (lambda: q.npu_convert_weight_to_int4pack(_m((128, 16), torch.int32), inner_k_tiles=2), "inner_k_tiles"),
    (lambda: q.npu_convert_weight_to_int4pack(_m((64, 16), torch.int32), inner_k_tiles=4), "K % 128"),
    (lambda: q.npu_format_cast(_m((100, 2), torch.int32), 29), "K % 128"),
    (lambda: q.quantize_per_tensor(_m((4,), torch.int32), 0.1, 0, torch.qint8), "float32, float16 or bfloat16"),
    (lambda: q.quantize_per_tensor(_m((4,), torch.float32), 0.0, 0, torch.qint8), "positive"),
    (lambda: q.quantize_per_tensor(_m((4,), torch.float32), 0.1, 0, torch.float16), "torch.qint8"),
    (lambda: q.quantize_per_channel(_m((4, 3), torch.float32), _m((3,), torch.float32), _m((3,), torch.int64), 2,
                                    torch.qint8), "axis out of range"),
    (lambda: q.quantize_per_channel(_m((4, 3), torch.float32), _m((4,), torch.float32), _m((4,), torch.int64), 1,
                                    torch.qint8), "as many elements"),
    (lambda: q.quantize_per_channel(_m((4, 3), torch.float32), _m((3,), torch.float32), _m((2,), torch.int64), 1,
                                    torch.qint8), "same length"),
    (lambda: q.quantize_per_channel(_m((4, 3), torch.float32), _m((3, 1), torch.float32), _m((3,), torch.int64), 1,
                                    torch.qint8), "1-D"),
    (lambda: q.dequantize(_m((4,), torch.float32)), "int8, uint8 or int32"),
    (lambda: q.npu_format_cast(_m((128, 2), torch.int32), 3), "only ND"),
    (lambda: q.npu_format_cast(_m((128, 16), torch.float16), 29), "int4-packed"),
    (lambda: q.npu_format_cast(_m((96, 16), torch.int8), 29), "K % 64"),
    (lambda: q.npu_weight_quant_batchmatmul(_m((2, 256), torch.bfloat16),
                                            q.npu_format_cast(_m((128, 2), torch.int32), 29),
                                            _m((1, 16), torch.float16), antiquant_group_size=128), "weight's K"),
    (lambda: q.npu_quant_matmul(_m((4, 128), torch.int8), q.npu_format_cast(_m((64, 64), torch.int8), 29),
                                _m((1,), torch.float32)), "weight's K"),
    (lambda: q.npu_quant_matmul(_m((4, 64), torch.int8), _m((1, 1, 1, 1, 1, 64, 4), torch.int8),
                                _m((1,), torch.float32)), "x2 must be"),
    (lambda: q.npu_quant_matmul(_m((2, 4, 64), torch.int8), _m((3, 64, 8), torch.int8), _m((1,), torch.float32)),
     "do not broadcast"),
    (lambda: q.npu_weight_quant_batchmatmul(_m((2, 4, 128), torch.bfloat16), _m((3, 128, 2), torch.int32),
                                            _m((1, 16), torch.float16), antiquant_group_size=128), "do not broadcast"),
    (lambda: q.npu_weight_quant_batchmatmul(_m((2, 4, 128), torch.bfloat16), _m((2, 128, 2), torch.int32),
                                            _m((3, 1, 16), torch.float16), antiquant_group_size=128),
     "antiquant_scale must be"),
    (lambda: q.npu_rms_norm(_m((4, 64), torch.bfloat16), _m((64,), torch.float16)), "dtype of self"),
    (lambda: q.npu_rms_norm(_m((4, 64), torch.bfloat16), _m((32,), torch.bfloat16)), "trailing dims"),
    (lambda: q.npu_rms_norm_dynamic_quant(_m((4, 8, 8), torch.bfloat16), _m((8, 8), torch.bfloat16)), "1-D gamma"),
    (lambda: q.npu_rms_norm_dynamic_quant(_m((4, 8), torch.float32), _m((8,), torch.float32)), "float16 or bfloat16"),
    (lambda: q.npu_swiglu(_m((4, 63), torch.bfloat16)), "even"),
    (lambda: q.npu_swiglu(_m((4, 64), torch.bfloat16), dim=0), "last dimension"),
    (lambda: q.npu_swiglu(_m((4, 64), torch.float32)), "float16 or bfloat16"),
])
def test_meta_errors(call, msg):
    with pytest.raises(RuntimeError, match=msg):
        call()


def test_product_path_has_no_cpu_kernel():
    """The ops have no CPU implementation: a CPU tensor is refused, never computed on the host."""
    with pytest.raises(NotImplementedError):
        q.npu_dynamic_quant(torch.zeros((2, 8), dtype=torch.float16))


def test_fast_quantizer_rule():
    """The kernels' quantizer (csrc/kernels/common.h, row_quant / quant_row) replaces rint(RN(v / s)) by
    rint(RN(v * RN(1/s))) wherever that product lies farther than 2^-14 from a half-integer, and divides
    otherwise.  Checked here in float32 against the IEEE division on rows of widely varying magnitude, a third
    of them holding exact ties (k + 0.5) * s, where a reciprocal-multiply alone goes wrong."""
    import numpy as np

    rng = np.random.default_rng(1)
    f32 = np.float32
    slow = 0
    for trial in range(24):
        v = (rng.standard_normal(16384) * 2.0 ** int(rng.integers(-60, 60))).astype(f32)
        s = f32(f32(np.max(np.abs(v))) / f32(127))
        if trial % 3 == 0:
            v[:1000] = ((rng.integers(-126, 126, 1000).astype(f32) + f32(0.5)) * s).astype(f32)
            s = f32(f32(np.max(np.abs(v))) / f32(127))
        ref = np.clip(np.rint((v / s).astype(f32)), -128, 127)
        t = (v * f32(f32(1) / s)).astype(f32)
        fast = np.abs((t - (np.floor(t) + f32(0.5)).astype(f32)).astype(f32)) > f32(2.0 ** -14)
        got = np.where(fast, np.clip(np.rint(t), -128, 127), ref)
        assert np.array_equal(got, ref), trial
        slow += int(np.sum(~fast))
    assert slow >= 8 * 1000  # the tie rows took the division path


def test_quant8_magic_rounding_rule():
    """quant8 (csrc/kernels/common.h) rounds t = RN(v * RN(1/s)) to an integer by adding 1.5 * 2^23 in float32
    and takes the low byte of the sum's bits as the int8; a group of eight with an element within 2^-14 of a
    half-integer (or NaN) is redone with the exact rule.  Emulated here in numpy float32 (IEEE, round to nearest
    even) on rows of widely varying magnitude with planted exact ties, against clamp(rint(RN(v / s)))."""
    import numpy as np

    rng = np.random.default_rng(5)
    f32 = np.float32
    magic = f32(12582912.0)
    redone = 0
    for trial in range(24):
        v = (rng.standard_normal(16384) * 2.0 ** int(rng.integers(-60, 60))).astype(f32)
        if trial % 3 == 0:
            s0 = f32(f32(np.max(np.abs(v))) / f32(127))
            v[:1000] = ((rng.integers(-127, 127, 1000).astype(f32) + f32(0.5)) * s0).astype(f32)
        if trial % 4 == 1:
            v[5] = -v[np.argmax(np.abs(v))]  # the absmax element with both signs: t = +-127 exactly
        s = f32(f32(np.max(np.abs(v))) / f32(127))
        ref = np.clip(np.rint((v / s).astype(f32)), -128, 127).astype(np.int64)
        t = (v * f32(f32(1) / s)).astype(f32)
        mf = (t + magic).astype(f32)
        d = (t - (mf - magic).astype(f32)).astype(f32)
        safe = np.abs(d) < f32(0.5 - 2.0 ** -14)
        byte = (mf.view(np.uint32) & 0xFF).astype(np.int64)
        fast = np.where(byte > 127, byte - 256, byte)
        group_safe = safe.reshape(-1, 8).all(axis=1).repeat(8)
        assert np.all(np.abs(t) <= 127 * (1 + 2.0 ** -22))
        assert np.array_equal(fast[group_safe], ref[group_safe]), trial
        redone += int(np.sum(~group_safe))
    assert redone >= 8 * 1000  # the tie rows' groups took the exact path


def test_split_counter_protocol_model():
    """The split-K arrival counter of splitk_last (csrc/kernels/common.h), stepped on the CPU: nsplit arrivals,
    each a fetch-and-add of D = tag * 2^16 + 1 and, on a stale word, a compare-and-swap loop, interleaved at
    random on initial words that a workspace may hold (zero, 0xFF fill, small integers, random bits, stale
    multiples of D).  Every interleaving must count the arrivals 1..nsplit exactly once and leave the word zero."""
    import random
    MASK = (1 << 64) - 1
    KC = (1 << 16) - 1
    rng = random.Random(7)
    for trial in range(3000):
        nsplit = rng.choice([2, 3, 4, 8, 16])
        tag = rng.randrange(1, (1 << 48) - 1)
        d = ((tag << 16) | 1) & MASK

        def valid(w):
            return (w & KC) < nsplit and w == ((w & KC) * d) & MASK

        word = rng.choice([0, MASK, rng.randrange(0, 1 << 20), rng.getrandbits(64), (-rng.randrange(1, 40) * d) & MASK,
                           ((nsplit + rng.randrange(0, 5)) * d) & MASK, (tag << 16) & MASK])
        # per arrival: stage 0 = fetch-and-add pending, 1 = CAS pending (expected value held), 2 = done
        stage = [0] * nsplit
        expect = [0] * nsplit
        counts = []
        last = []
        while any(s != 2 for s in stage):
            a = rng.choice([i for i in range(nsplit) if stage[i] != 2])
            if stage[a] == 0:
                old = word
                word = (word + d) & MASK
                if valid(old):
                    n = (old & KC) + 1
                else:
                    expect[a] = (old + d) & MASK
                    stage[a] = 1
                    continue
            else:
                nw = ((expect[a] + d) & MASK) if valid(expect[a]) else d
                if word != expect[a]:
                    expect[a] = word  # failed compare-and-swap: retry with the actual value
                    continue
                word = nw
                n = nw & KC
            stage[a] = 2
            counts.append(n)
            if n == nsplit:
                word = 0
                last.append(a)
        assert sorted(counts) == list(range(1, nsplit + 1)), (trial, counts)
        assert len(last) == 1 and word == 0
