"""CPU oracle for the quantized-inference hot path -- TEST INFRASTRUCTURE ONLY.

ctypes front end of ``qk_oracle.c``.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` import this module; the product
package never does, and it raises if asked to run without its HIP extension.

Every function takes and returns numpy arrays (uint16 bit patterns for
fp16/bf16, so no conversion happens outside the C restatement).  The closed
forms, the reference files they follow, and what pins each function are in
the header of ``qk_oracle.c``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libqk_oracle.so")

F16, BF16, F32, I8, I32, U8 = 1, 2, 3, 4, 5, 6

_lib = None


def build(force: bool = False) -> str:
    """Compile libqk_oracle.so with the committed Makefile (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.qo_dynamic_quant.argtypes = [P, I, I64, I64, P, P, P]
        L.qo_w8a8_acc.argtypes = [P, I64, P, I64, I64, I64, I64, I64, P]
        L.qo_quant_matmul_epilogue.argtypes = [P, I64, I64, P, I64, P, I64, P, P, I, P, I]
        L.qo_int4_pack.argtypes = [P, I64, I64, P]
        L.qo_int4_unpack.argtypes = [P, I64, I64, P]
        L.qo_w4_nz_pack.argtypes = [P, I64, I64, P]
        L.qo_w4_nz_unpack.argtypes = [P, I64, I64, P]
        L.qo_w8_nz_pack.argtypes = [P, I64, I64, P]
        L.qo_w8_nz_unpack.argtypes = [P, I64, I64, P]
        L.qo_weight_quant_bmm.argtypes = [P, I, P, I, P, P, I, I64, I64, I64, I64, P, I, P, I, P]
        L.qo_rms_norm.argtypes = [P, I, P, I64, I64, ctypes.c_double, P, P]
        L.qo_rms_norm_f32.argtypes = [P, P, I64, I64, ctypes.c_double, P, P]
        L.qo_swiglu.argtypes = [P, I, I64, I64, P]
        L.qo_cvt_array.argtypes = [P, I, P, I, I64]
        L.qo_quantize.argtypes = [P, I, I64, I64, I64, P, P, P, I]
        L.qo_dequantize.argtypes = [P, I, I64, P]
        L.qo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.qo_f32_to_bf16.restype = ctypes.c_uint16
        L.qo_f32_to_f16.argtypes = [ctypes.c_float]
        L.qo_f32_to_f16.restype = ctypes.c_uint16
        L.qo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.qo_f16_to_f32.restype = ctypes.c_float
        L.qo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.qo_bf16_to_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- conversions

def convert(a: np.ndarray, in_dtype: int, out_dtype: int) -> np.ndarray:
    """Elementwise cast through the C routines.  fp16/bf16 travel as uint16 bit
    patterns, float32 as float32."""
    src = np.ascontiguousarray(a, dtype=np.float32 if in_dtype == F32 else np.uint16)
    out = np.empty(src.shape, dtype=np.float32 if out_dtype == F32 else np.uint16)
    lib().qo_cvt_array(_p(src), in_dtype, _p(out), out_dtype, src.size)
    return out


# ---------------------------------------------------------------- hot-path ops

def dynamic_quant(x_bits: np.ndarray, x_dtype: int, smooth: np.ndarray | None = None):
    """x_bits: uint16 [..., K] (fp16 or bf16 patterns) -> (int8 [..., K], float32 [...])."""
    x = _c(x_bits, np.uint16)
    K = x.shape[-1]
    rows = x.size // K if K else 0
    y = np.empty(x.shape, dtype=np.int8)
    s = np.empty(x.shape[:-1], dtype=np.float32)
    sm = _c(smooth, np.float32)
    lib().qo_dynamic_quant(_p(x), x_dtype, rows, K, _p(sm), _p(y), _p(s))
    return y, s


def w8a8_acc(a: np.ndarray, w: np.ndarray, w_transposed: bool = False) -> np.ndarray:
    """Exact int32 accumulator.  a int8 [M,K]; w int8 [K,N], or [N,K] when w_transposed."""
    a = _c(a, np.int8)
    w = _c(w, np.int8)
    M, K = a.shape
    if w_transposed:
        N = w.shape[0]
        sk, sn = 1, K
    else:
        N = w.shape[1]
        sk, sn = N, 1
    acc = np.empty((M, N), dtype=np.int32)
    lib().qo_w8a8_acc(_p(a), K, _p(w), sk, sn, M, N, K, _p(acc))
    return acc


def quant_matmul_epilogue(acc, scale, offset=None, pertoken=None, bias=None, bias_dtype=BF16,
                          out_dtype=BF16):
    acc = _c(acc, np.int32)
    M, N = acc.shape
    scale = _c(scale, np.float32).ravel()
    offset = _c(offset, np.float32)
    offset = None if offset is None else offset.ravel()
    pertoken = _c(pertoken, np.float32)
    pertoken = None if pertoken is None else pertoken.ravel()
    if bias is not None:
        bias = np.ascontiguousarray(bias).ravel()
    out_np = {BF16: np.uint16, F16: np.uint16, F32: np.float32, I8: np.int8, I32: np.int32}[out_dtype]
    out = np.empty((M, N), dtype=out_np)
    lib().qo_quant_matmul_epilogue(_p(acc), M, N, _p(scale), scale.size, _p(offset),
                                   0 if offset is None else offset.size, _p(pertoken), _p(bias),
                                   bias_dtype, _p(out), out_dtype)
    return out


def quant_matmul(x1, x2, scale, offset=None, pertoken=None, bias=None, bias_dtype=BF16,
                 out_dtype=BF16, x2_transposed=False):
    """Full W8A8 path: exact int32 accumulation, then the fused epilogue."""
    acc = w8a8_acc(x1, x2, x2_transposed)
    return quant_matmul_epilogue(acc, scale, offset, pertoken, bias, bias_dtype, out_dtype)


def int4_pack(w: np.ndarray) -> np.ndarray:
    w = _c(w, np.int8)
    K, N = w.shape
    out = np.empty((K, N // 8), dtype=np.int32)
    lib().qo_int4_pack(_p(w), K, N, _p(out))
    return out


def int4_unpack(packed: np.ndarray) -> np.ndarray:
    packed = _c(packed, np.int32)
    K, NW = packed.shape
    out = np.empty((K, NW * 8), dtype=np.int8)
    lib().qo_int4_unpack(_p(packed), K, NW * 8, _p(out))
    return out


def w4_nz_pack(packed: np.ndarray) -> np.ndarray:
    """int32 [K, N/8] (ND int4) -> int32 [N/16, K/128, 64, 4] (MFMA-tiled NZ layout)."""
    nd = _c(packed, np.int32)
    K, NW = nd.shape
    N = NW * 8
    out = np.empty((N // 16, K // 128, 64, 4), dtype=np.int32)
    lib().qo_w4_nz_pack(_p(nd), K, N, _p(out))
    return out


def w4_nz_unpack(nz: np.ndarray) -> np.ndarray:
    """int32 [N/16, K/128, 64, 4] -> int32 [K, N/8] (ND int4)."""
    t = _c(nz, np.int32)
    N, K = t.shape[0] * 16, t.shape[1] * 128
    out = np.empty((K, N // 8), dtype=np.int32)
    lib().qo_w4_nz_unpack(_p(t), K, N, _p(out))
    return out


def w8_nz_pack(w: np.ndarray) -> np.ndarray:
    """int8 [K, N] -> int8 [N/16, K/64, 64, 16] (the int8 NZ layout)."""
    nd = _c(w, np.int8)
    K, N = nd.shape
    out = np.empty((N // 16, K // 64, 64, 16), dtype=np.int8)
    lib().qo_w8_nz_pack(_p(nd), K, N, _p(out))
    return out


def w8_nz_unpack(nz: np.ndarray) -> np.ndarray:
    t = _c(nz, np.int8)
    N, K = t.shape[0] * 16, t.shape[1] * 64
    out = np.empty((K, N), dtype=np.int8)
    lib().qo_w8_nz_unpack(_p(t), K, N, _p(out))
    return out


def weight_quant_bmm(x_bits, x_dtype, weight, scale_bits, offset_bits, scale_dtype, group,
                     bias=None, bias_dtype=BF16, out_dtype=BF16):
    """x_bits uint16 [M,K]; weight int32 [K,N/8] (int4 packed) or int8 [K,N];
    scale/offset uint16 [K/group, N] (or [1,N] / [N] when group == 0)."""
    x = _c(x_bits, np.uint16)
    M, K = x.shape
    if weight.dtype == np.int32:
        w = _c(weight, np.int32)
        N = w.shape[1] * 8
        wdt = I32
    else:
        w = _c(weight, np.int8)
        N = w.shape[1]
        wdt = I8
    sc = _c(scale_bits, np.uint16)
    off = _c(offset_bits, np.uint16)
    if bias is not None:
        bias = np.ascontiguousarray(bias).ravel()
    out = np.empty((M, N), dtype=np.uint16)
    work = np.empty((M + 1) * N, dtype=np.float64)
    lib().qo_weight_quant_bmm(_p(x), x_dtype, _p(w), wdt, _p(sc), _p(off), scale_dtype, M, N, K,
                              group, _p(bias), bias_dtype, _p(out), out_dtype, _p(work))
    return out


_QNP = {I8: np.int8, U8: np.uint8, I32: np.int32}


def quantize(x, x_dtype, scales, zero_points, axis=None, q_dtype=I8):
    """quantize_per_tensor (axis None; scales / zero_points of one element) or quantize_per_channel along
    `axis`.  x: float32 array (x_dtype F32) or uint16 bit patterns (F16 / BF16)."""
    xa = np.ascontiguousarray(x, dtype=np.float32 if x_dtype == F32 else np.uint16)
    sc = np.ascontiguousarray(scales, dtype=np.float32).ravel()
    zp = np.ascontiguousarray(zero_points, dtype=np.int64).ravel()
    if axis is None:
        outer, C, inner = 1, 1, xa.size
    else:
        axis %= xa.ndim
        C = xa.shape[axis]
        outer = int(np.prod(xa.shape[:axis], dtype=np.int64))
        inner = int(np.prod(xa.shape[axis + 1:], dtype=np.int64))
    out = np.empty(xa.shape, dtype=_QNP[q_dtype])
    lib().qo_quantize(_p(xa), x_dtype, outer, C, inner, _p(sc), _p(zp), _p(out), q_dtype)
    return out


def dequantize(q, q_dtype):
    qa = np.ascontiguousarray(q, dtype=_QNP[q_dtype])
    out = np.empty(qa.shape, dtype=np.float32)
    lib().qo_dequantize(_p(qa), q_dtype, qa.size, _p(out))
    return out


def rms_norm(x_bits, x_dtype, gamma_bits, eps=1e-6):
    x = _c(x_bits, np.uint16)
    D = x.shape[-1]
    rows = x.size // D
    y = np.empty(x.shape, dtype=np.uint16)
    rstd = np.empty(x.shape[:-1] + (1,), dtype=np.float32)
    lib().qo_rms_norm(_p(x), x_dtype, _p(_c(gamma_bits, np.uint16)), rows, D, eps, _p(y), _p(rstd))
    return y, rstd


def rms_norm_f32(x, gamma, eps=1e-6):
    """float32 RMSNorm (the reference's golden case): y float32 like x, rstd [..., 1] float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.size // D
    y = np.empty(x.shape, dtype=np.float32)
    rstd = np.empty(x.shape[:-1] + (1,), dtype=np.float32)
    lib().qo_rms_norm_f32(_p(x), _p(np.ascontiguousarray(gamma, dtype=np.float32)), rows, D, eps, _p(y), _p(rstd))
    return y, rstd


def swiglu(h_bits, dtype_code):
    h = _c(h_bits, np.uint16)
    I2 = h.shape[-1]
    rows = h.size // I2
    out = np.empty(h.shape[:-1] + (I2 // 2,), dtype=np.uint16)
    lib().qo_swiglu(_p(h), dtype_code, rows, I2 // 2, _p(out))
    return out
