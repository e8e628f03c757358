"""The committed golden fixtures (tests/golden/golden_seed0.npz, written by tests/golden/make_golden.py from torch /
numpy closed forms, independently of the C oracle and of the HIP kernels): the oracle on the CPU and the HIP path
through the registered ops on the GPU, each against the same expected outputs.

Bars (the north star's): int8 activations, scales, int32 accumulators, int4 packs and static-quant outputs
bit-exact; bf16 outputs within rtol / atol 1e-2.
"""
import os

import numpy as np
import pytest
import torch

from op_plugin_amd import workloads as W

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_seed0.npz")
F16, BF16, F32, I8, I32, U8 = 1, 2, 3, 4, 5, 6
DEV = "cuda"


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def _bf16(bits) -> torch.Tensor:
    return W.from_bits(np.ascontiguousarray(bits), torch.bfloat16).float()


def _close16(got_bits, exp_bits):
    torch.testing.assert_close(_bf16(got_bits), _bf16(exp_bits), rtol=1e-2, atol=1e-2)


# ----------------------------------------------------------------------------- oracle (CPU)

def test_golden_file_is_data_only(gold):
    assert len(gold) == 31 and all(v.dtype != object for v in gold.values())


@pytest.mark.parametrize("case,code", [("dq_f16", F16), ("dq_bf16", BF16)])
def test_oracle_dynamic_quant_golden(oracle, gold, case, code):
    y, s = oracle.dynamic_quant(gold[f"{case}_x"], code)
    assert np.array_equal(s, gold[f"{case}_scale"])
    assert np.array_equal(y, gold[f"{case}_y"])


def test_oracle_quant_matmul_golden(oracle, gold):
    acc = oracle.w8a8_acc(gold["qmm_x1"], gold["qmm_x2"])
    assert np.array_equal(acc, gold["qmm_acc"])
    out = oracle.quant_matmul_epilogue(acc, gold["qmm_scale"], pertoken=gold["qmm_pertoken"], bias=gold["qmm_bias"],
                                       bias_dtype=BF16, out_dtype=BF16)
    _close16(out, gold["qmm_out"])


def test_oracle_int4_pack_and_w4a16_golden(oracle, gold):
    assert np.array_equal(oracle.int4_pack(gold["w4_values"]), gold["w4_packed"])
    out = oracle.weight_quant_bmm(gold["w4_x"], BF16, gold["w4_packed"], gold["w4_scale"], gold["w4_offset"], F16, 128)
    _close16(out, gold["w4_out"])


def test_oracle_rms_norm_and_swiglu_golden(oracle, gold):
    y, rstd = oracle.rms_norm(gold["rms_x"], BF16, gold["rms_gamma"], 1e-6)
    _close16(y, gold["rms_y"])
    np.testing.assert_allclose(rstd, gold["rms_rstd"], rtol=1e-6)
    _close16(oracle.swiglu(gold["swiglu_h"], BF16), gold["swiglu_y"])


def test_oracle_static_quant_golden(oracle, gold):
    assert np.array_equal(oracle.quantize(gold["qpt_x"], F32, [0.05], [3], None, I8), gold["qpt_q"])
    assert np.array_equal(oracle.quantize(gold["qpc_x"], F32, gold["qpc_scale"], gold["qpc_zp"], 1, U8),
                          gold["qpc_q"])


# ----------------------------------------------------------------------------- HIP path (GPU)

@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    return op_plugin_amd


def _dev(bits, dtype):
    return W.from_bits(np.ascontiguousarray(bits), dtype).to(DEV)


@pytest.mark.gpu
@pytest.mark.parametrize("case,dtype", [("dq_f16", torch.float16), ("dq_bf16", torch.bfloat16)])
def test_gpu_dynamic_quant_golden(ops, gold, case, dtype):
    print(f"[case] golden {case}", flush=True)
    y, s = ops.npu_dynamic_quant(_dev(gold[f"{case}_x"], dtype))
    assert np.array_equal(s.cpu().numpy(), gold[f"{case}_scale"])
    assert np.array_equal(y.cpu().numpy(), gold[f"{case}_y"])


@pytest.mark.gpu
def test_gpu_quant_matmul_golden(ops, gold):
    print("[case] golden quant_matmul", flush=True)
    x1 = torch.from_numpy(gold["qmm_x1"]).to(DEV)
    x2 = torch.from_numpy(gold["qmm_x2"]).to(DEV)
    acc = ops.npu_quant_matmul(x1, x2, torch.ones(1, device=DEV), output_dtype=torch.int32)
    assert np.array_equal(acc.cpu().numpy(), gold["qmm_acc"])
    out = ops.npu_quant_matmul(x1, x2, torch.from_numpy(gold["qmm_scale"]).to(DEV),
                               pertoken_scale=torch.from_numpy(gold["qmm_pertoken"]).to(DEV),
                               bias=_dev(gold["qmm_bias"], torch.bfloat16), output_dtype=torch.bfloat16)
    _close16(W.bits(out.cpu()), gold["qmm_out"])


@pytest.mark.gpu
def test_gpu_int4_pack_and_w4a16_golden(ops, gold):
    print("[case] golden int4 pack + w4a16", flush=True)
    packed = ops.npu_convert_weight_to_int4pack(torch.from_numpy(gold["w4_values"].astype(np.int32)).to(DEV))
    assert np.array_equal(packed.cpu().numpy(), gold["w4_packed"])
    out = ops.npu_weight_quant_batchmatmul(_dev(gold["w4_x"], torch.bfloat16), packed,
                                           _dev(gold["w4_scale"], torch.float16), _dev(gold["w4_offset"], torch.float16),
                                           antiquant_group_size=128)
    _close16(W.bits(out.cpu()), gold["w4_out"])


@pytest.mark.gpu
def test_gpu_rms_norm_and_swiglu_golden(ops, gold):
    print("[case] golden rms_norm + swiglu", flush=True)
    y, rstd = ops.npu_rms_norm(_dev(gold["rms_x"], torch.bfloat16), _dev(gold["rms_gamma"], torch.bfloat16), 1e-6)
    _close16(W.bits(y.cpu()), gold["rms_y"])
    np.testing.assert_allclose(rstd.cpu().numpy(), gold["rms_rstd"], rtol=1e-6)
    y = ops.npu_swiglu(_dev(gold["swiglu_h"], torch.bfloat16))
    _close16(W.bits(y.cpu()), gold["swiglu_y"])


@pytest.mark.gpu
def test_gpu_static_quant_golden(ops, gold):
    print("[case] golden static quant", flush=True)
    q = ops.quantize_per_tensor(torch.from_numpy(gold["qpt_x"]).to(DEV), 0.05, 3, torch.qint8)
    assert np.array_equal(q.cpu().numpy(), gold["qpt_q"])
    q = ops.quantize_per_channel(torch.from_numpy(gold["qpc_x"]).to(DEV), torch.from_numpy(gold["qpc_scale"]).to(DEV),
                                 torch.from_numpy(gold["qpc_zp"]).to(DEV), 1, torch.quint8)
    assert np.array_equal(q.cpu().numpy(), gold["qpc_q"])
