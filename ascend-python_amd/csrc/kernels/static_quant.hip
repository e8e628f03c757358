// quantize_per_tensor / quantize_per_channel / dequantize for gfx950.
//
// The reference's NPU quantize ops return plain integer tensors (QInt8 -> int8,
// QUInt8 -> uint8, QInt32 -> int32;
// op_plugin/ops/base_ops/aclops/QuantizePerTensorKernelNpu.cpp:50-82,
// op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:69-92) and its
// dequantize is a cast of those integers to float32
// (op_plugin/ops/v1r11/opapi/DequantizeKernelNpuOpApi.cpp:22-24).  Element rule
// (torch's affine quantizer for the same schema):
//   q = clamp(RN(rint(x * RN(1 / scale)) + float(zero_point)), qmin, qmax),
// a NaN giving qmin.  x is viewed as [outer][C][inner]; per tensor is C == 1.
// HBM-bound: each thread converts 8 consecutive elements (one 16-byte load of
// 16-bit x, two of fp32 x; one 8- or 32-byte store).
#include "common.h"

namespace qk {
namespace {

constexpr int kSqThreads = 256;

template <int QDT>
__device__ __forceinline__ void store_q(void* q, int64_t i, float z) {
    if constexpr (QDT == QK_I8) {
        static_cast<int8_t*>(q)[i] = (int8_t)(int)fminf(fmaxf(z, -128.0f), 127.0f);
    } else if constexpr (QDT == QK_U8) {
        static_cast<uint8_t*>(q)[i] = (uint8_t)(int)fminf(fmaxf(z, 0.0f), 255.0f);
    } else {
        // float32 holds -2^31 exactly; 2^31 and above saturate to INT32_MAX; NaN -> INT32_MIN
        const int32_t v = z >= 2147483648.0f ? 2147483647 : (z >= -2147483648.0f ? (int32_t)z : (int32_t)0x80000000u);
        static_cast<int32_t*>(q)[i] = v;
    }
}

template <int XDT>
__device__ __forceinline__ float load_x(const void* x, int64_t i) {
    if constexpr (XDT == QK_F32) return static_cast<const float*>(x)[i];
    else return load_half_bits(static_cast<const uint16_t*>(x)[i], XDT);
}

// one rounding for the product, rint (ties to even), then the zero point added in float32
__device__ __forceinline__ float quant_value(float v, float r, float zp) { return __builtin_rintf(v * r) + zp; }

// VEC: the 8-element vector path (x and q 16-byte aligned, inner % 8 == 0 so one channel per group of 8);
// otherwise one element per thread.  per_channel == false: scale0 / zp0 for every element.
template <int XDT, int QDT, bool VEC>
__global__ __launch_bounds__(kSqThreads) void quantize_kernel(const void* __restrict__ x, int64_t n, int64_t C,
                                                              int64_t inner, const float* __restrict__ scales,
                                                              const int64_t* __restrict__ zps, float scale0,
                                                              int64_t zp0, void* __restrict__ q) {
    const bool per_channel = scales != nullptr;
    const float r0 = 1.0f / scale0;  // correctly rounded (the library is built with IEEE division)
    const float z0 = (float)zp0;
    const int64_t step = (int64_t)gridDim.x * kSqThreads;
    if constexpr (VEC) {
        const int64_t groups = n >> 3;
        for (int64_t gi = (int64_t)blockIdx.x * kSqThreads + threadIdx.x; gi < groups; gi += step) {
            const int64_t i0 = gi << 3;
            float r = r0, z = z0;
            if (per_channel) {
                const int64_t c = (i0 / inner) % C;
                r = 1.0f / scales[c];
                z = (float)zps[c];
            }
            float v[8];
            if constexpr (XDT == QK_F32) {
                const f32x4 a = reinterpret_cast<const f32x4*>(x)[2 * gi];
                const f32x4 b = reinterpret_cast<const f32x4*>(x)[2 * gi + 1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = a[e];
                    v[4 + e] = b[e];
                }
            } else {
                const u32x4 a = reinterpret_cast<const u32x4*>(x)[gi];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[2 * e] = load_half_bits(a[e] & 0xffffu, XDT);
                    v[2 * e + 1] = load_half_bits(a[e] >> 16, XDT);
                }
            }
            float zq[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) zq[e] = quant_value(v[e], r, z);
            if constexpr (QDT == QK_I32) {
                i32x4 lo, hi;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = zq[e], b = zq[4 + e];
                    lo[e] = a >= 2147483648.0f ? 2147483647 : (a >= -2147483648.0f ? (int32_t)a : (int32_t)0x80000000u);
                    hi[e] = b >= 2147483648.0f ? 2147483647 : (b >= -2147483648.0f ? (int32_t)b : (int32_t)0x80000000u);
                }
                reinterpret_cast<i32x4*>(q)[2 * gi] = lo;
                reinterpret_cast<i32x4*>(q)[2 * gi + 1] = hi;
            } else {
                u32x2 o = {0u, 0u};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t b = QDT == QK_I8 ? (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(zq[e], -128.0f), 127.0f)
                                                    : (uint32_t)(uint8_t)(int)fminf(fmaxf(zq[e], 0.0f), 255.0f);
                    o[e >> 2] |= b << (8 * (e & 3));
                }
                reinterpret_cast<u32x2*>(q)[gi] = o;
            }
        }
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kSqThreads + threadIdx.x; i < n; i += step) {
            float r = r0, z = z0;
            if (per_channel) {
                const int64_t c = (i / inner) % C;
                r = 1.0f / scales[c];
                z = (float)zps[c];
            }
            store_q<QDT>(q, i, quant_value(load_x<XDT>(x, i), r, z));
        }
    }
}

template <int QDT>
__global__ __launch_bounds__(kSqThreads) void dequantize_kernel(const void* __restrict__ q, int64_t n,
                                                                float* __restrict__ out) {
    const int64_t step = (int64_t)gridDim.x * kSqThreads;
    for (int64_t i = (int64_t)blockIdx.x * kSqThreads + threadIdx.x; i < n; i += step) {
        if constexpr (QDT == QK_I8) out[i] = (float)static_cast<const int8_t*>(q)[i];
        else if constexpr (QDT == QK_U8) out[i] = (float)static_cast<const uint8_t*>(q)[i];
        else out[i] = (float)static_cast<const int32_t*>(q)[i];  // round to nearest even past 2^24
    }
}

int64_t grid_of(int64_t work) {
    int64_t b = (work + kSqThreads - 1) / kSqThreads;
    return b < 1 ? 1 : (b > 65536 ? 65536 : b);
}

template <int XDT, int QDT>
hipError_t launch_q(const void* x, int64_t n, int64_t C, int64_t inner, const float* scales, const int64_t* zps,
                    float scale0, int64_t zp0, void* q, hipStream_t stream) {
    const bool vec = n % 8 == 0 && ((uintptr_t)x | (uintptr_t)q) % 16 == 0 && (scales == nullptr || inner % 8 == 0);
    if (vec)
        quantize_kernel<XDT, QDT, true><<<dim3((uint32_t)grid_of(n / 8)), dim3(kSqThreads), 0, stream>>>(
            x, n, C, inner, scales, zps, scale0, zp0, q);
    else
        quantize_kernel<XDT, QDT, false><<<dim3((uint32_t)grid_of(n)), dim3(kSqThreads), 0, stream>>>(
            x, n, C, inner, scales, zps, scale0, zp0, q);
    return hipGetLastError();
}

template <int XDT>
hipError_t launch_q_x(const void* x, int64_t n, int64_t C, int64_t inner, const float* scales, const int64_t* zps,
                      float scale0, int64_t zp0, void* q, int q_dtype, hipStream_t stream) {
    switch (q_dtype) {
    case QK_I8: return launch_q<XDT, QK_I8>(x, n, C, inner, scales, zps, scale0, zp0, q, stream);
    case QK_U8: return launch_q<XDT, QK_U8>(x, n, C, inner, scales, zps, scale0, zp0, q, stream);
    default: return launch_q<XDT, QK_I32>(x, n, C, inner, scales, zps, scale0, zp0, q, stream);
    }
}

}  // namespace

hipError_t launch_quantize(const void* x, int x_dtype, int64_t outer, int64_t C, int64_t inner, const float* scales,
                           const int64_t* zps, float scale0, int64_t zp0, void* q, int q_dtype, hipStream_t stream) {
    const int64_t n = outer * C * inner;
    if (n == 0) return hipSuccess;
    switch (x_dtype) {
    case QK_F32: return launch_q_x<QK_F32>(x, n, C, inner, scales, zps, scale0, zp0, q, q_dtype, stream);
    case QK_F16: return launch_q_x<QK_F16>(x, n, C, inner, scales, zps, scale0, zp0, q, q_dtype, stream);
    default: return launch_q_x<QK_BF16>(x, n, C, inner, scales, zps, scale0, zp0, q, q_dtype, stream);
    }
}

hipError_t launch_dequantize(const void* q, int q_dtype, int64_t n, float* out, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const dim3 grid((uint32_t)grid_of(n)), block(kSqThreads);
    switch (q_dtype) {
    case QK_I8: dequantize_kernel<QK_I8><<<grid, block, 0, stream>>>(q, n, out); break;
    case QK_U8: dequantize_kernel<QK_U8><<<grid, block, 0, stream>>>(q, n, out); break;
    default: dequantize_kernel<QK_I32><<<grid, block, 0, stream>>>(q, n, out); break;
    }
    return hipGetLastError();
}

}  // namespace qk
