"""Writes tests/golden/golden_seed0.npz: seeded inputs of every op on the path with their expected outputs.

The reference holds no golden vectors for this path (its ops live in closed CANN), so the expected outputs here
are computed independently of this repository's C oracle (oracle/qk_oracle.c) and of its HIP kernels, from the
closed forms of the op contracts with torch / numpy library routines:

* npu_dynamic_quant: s = absmax / 127 as an IEEE float32 division, y = clamp(torch.round(x / s)) (round half to
  even), zero rows give s = 0, y = 0 -- bit-exact.
* npu_quant_matmul: the int32 accumulator by numpy int64 matmul (exact); the bf16 output from the accumulator by
  the float64 epilogue acc * pertoken * scale + bias, rounded once to bf16 (the op's float32 operation order can
  differ from it by an ulp before that rounding: the bar for it is rtol / atol 1e-2).
* npu_convert_weight_to_int4pack: nibble i (bits 4i..4i+3, two's complement) of word j is column 8j + i -- exact.
* npu_weight_quant_batchmatmul (W4A16): x @ ((w + offset) * scale) in float64, groups of 128 along K, rounded
  to bf16 -- rtol / atol 1e-2.
* npu_rms_norm: the closed form of the reference's own test (test/test_custom_ops/test_npu_rms_norm.py:10-17)
  in float32: x * rsqrt(mean(x^2) + eps) * gamma, rstd = rsqrt(mean(x^2) + eps).
* npu_swiglu: silu(a) * b in float64 (a the first half), rounded to bf16.
* quantize_per_tensor / quantize_per_channel: torch's CPU quantizer (.int_repr()) -- exact.

Run from the repo root: ``python tests/golden/make_golden.py``.  The file is small (< 200 KB) and is read with
numpy.load(allow_pickle=False).
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_seed0.npz")


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def dynamic_quant(x: torch.Tensor):
    xf = x.float()
    s = xf.abs().amax(dim=-1) / 127.0
    y = torch.where(s[:, None] > 0, torch.round(xf / torch.where(s > 0, s, 1.0)[:, None]),
                    torch.zeros_like(xf))
    return torch.clamp(y, -128, 127).to(torch.int8), s


def main() -> None:
    g = torch.Generator().manual_seed(0)
    d: dict[str, np.ndarray] = {}

    # npu_dynamic_quant, fp16 rows: random with 1% outlier channels x20, a zero row, a row of exact ties
    x = torch.randn((6, 520), generator=g)
    x[:, torch.randperm(520, generator=g)[:5]] *= 20
    x[3] = 0.0
    x[4] = torch.arange(520, dtype=torch.float32) % 255 - 127  # absmax 127: scale exactly 1
    x[4, 1:9] = torch.tensor([0.5, 1.5, 2.5, -2.5, 3.5, 126.5, -126.5, -0.5])
    x16 = x.to(torch.float16)
    y, s = dynamic_quant(x16)
    d.update(dq_f16_x=bits16(x16), dq_f16_y=y.numpy(), dq_f16_scale=s.numpy())
    # bf16 rows of K = 4096
    xb = torch.randn((4, 4096), generator=g).to(torch.bfloat16)
    y, s = dynamic_quant(xb)
    d.update(dq_bf16_x=bits16(xb), dq_bf16_y=y.numpy(), dq_bf16_scale=s.numpy())

    # npu_quant_matmul (W8A8): int8 activations from a dynamic quant of fp16 rows, per-token and per-channel
    # scales, bf16 bias
    M, K, N = 16, 384, 128
    xq, pt = dynamic_quant(torch.randn((M, K), generator=g).to(torch.float16))
    w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int64).to(torch.int8)
    sc = (1e-3 + 9e-3 * torch.rand(N, generator=g)).float()
    bias = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
    acc = xq.numpy().astype(np.int64) @ w.numpy().astype(np.int64)
    out = torch.from_numpy(acc).double() * pt.double()[:, None] * sc.double()[None, :] + bias.double()[None, :]
    d.update(qmm_x1=xq.numpy(), qmm_x2=w.numpy(), qmm_scale=sc.numpy(), qmm_pertoken=pt.numpy(),
             qmm_bias=bits16(bias), qmm_acc=acc.astype(np.int32), qmm_out=bits16(out.to(torch.bfloat16)))

    # npu_convert_weight_to_int4pack and npu_weight_quant_batchmatmul (W4A16, group 128, with offset)
    M, K, N, G = 4, 256, 128, 128
    w4 = torch.randint(-8, 8, (K, N), generator=g, dtype=torch.int64)
    nib = (w4.numpy() & 0xF).astype(np.uint32).reshape(K, N // 8, 8)
    packed = np.zeros((K, N // 8), np.uint32)
    for i in range(8):
        packed |= nib[:, :, i] << np.uint32(4 * i)
    xw = torch.randn((M, K), generator=g).to(torch.bfloat16)
    ws = (5e-3 + 1.5e-2 * torch.rand((K // G, N), generator=g)).to(torch.float16)
    wo = (2 * torch.rand((K // G, N), generator=g) - 1).to(torch.float16)
    wf = (w4.double() + wo.double().repeat_interleave(G, 0)) * ws.double().repeat_interleave(G, 0)
    out = xw.double() @ wf
    d.update(w4_values=w4.numpy().astype(np.int8), w4_packed=packed.view(np.int32), w4_x=bits16(xw),
             w4_scale=bits16(ws), w4_offset=bits16(wo), w4_out=bits16(out.to(torch.bfloat16)))

    # npu_rms_norm (bf16), eps 1e-6: the reference test's closed form in float32
    xr = torch.randn((4, 1024), generator=g).to(torch.bfloat16)
    gr = (1 + 0.02 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    xf = xr.float()
    rstd = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    d.update(rms_x=bits16(xr), rms_gamma=bits16(gr), rms_y=bits16((xf * rstd * gr.float()).to(torch.bfloat16)),
             rms_rstd=rstd.numpy())

    # npu_swiglu (bf16): silu of the first half times the second
    h = torch.randn((4, 1024), generator=g).to(torch.bfloat16)
    a, b = h.double().chunk(2, dim=-1)
    d.update(swiglu_h=bits16(h), swiglu_y=bits16((F.silu(a) * b).to(torch.bfloat16)))

    # quantize_per_tensor (qint8, scale 0.05, zero point 3) with planted exact ties and clamped values
    xt = torch.randn(256, generator=g) * 4
    xt[:32] = (torch.randint(-100, 100, (32,), generator=g).float() + 0.5) * 0.05
    xt[32:36] = torch.tensor([1e6, -1e6, 0.0, 300.0])
    d.update(qpt_x=xt.numpy(), qpt_q=torch.quantize_per_tensor(xt, 0.05, 3, torch.qint8).int_repr().numpy())
    # quantize_per_channel (quint8, axis 1)
    xc = torch.randn((4, 32, 3), generator=g) * 3
    csc = torch.rand(32, generator=g, dtype=torch.float64) * 0.1 + 1e-3
    czp = torch.randint(0, 20, (32,), generator=g, dtype=torch.int64)
    d.update(qpc_x=xc.numpy(), qpc_scale=csc.float().numpy(), qpc_zp=czp.numpy(),
             qpc_q=torch.quantize_per_channel(xc, csc.float().double(), czp, 1, torch.quint8).int_repr().numpy())

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT}: {len(d)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
