// npu_dynamic_quant for gfx950: per-row symmetric int8 quantization.
//
// One 256-thread workgroup (4 wave64) per row.  The row is read once with
// 128-bit loads (8 halves per lane per load) and kept in registers; the
// absmax is reduced across the wave with xor-shuffles and across the four
// waves through LDS; the quantized row is written with 64-bit stores.  The
// arithmetic is exactly the op contract: s = amax / 127 (IEEE division),
// y = clamp(rint(x / s)) with ties to even, a zero row giving s = 0, y = 0.
// HBM-bound: 2 B read + 1 B written per element, 4 B per row for the scale.
#include "common.h"

namespace qk {
namespace {

constexpr int kThreads = 256;

// Vector path: K % 8 == 0, 16-byte aligned rows, K <= 8 * 256 * VPT.
template <int DT, int VPT, bool SMOOTH>
__global__ __launch_bounds__(kThreads) void dyn_quant_vec(const uint16_t* __restrict__ x, int64_t K,
                                                          const float* __restrict__ smooth,
                                                          int8_t* __restrict__ y, float* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * K);
    const int nv = (int)(K >> 3);
    float v[VPT][8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < nv) {
            u32x4 d = xr[idx];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[i][2 * e] = load_half_bits(d[e] & 0xffffu, DT);
                v[i][2 * e + 1] = load_half_bits(d[e] >> 16, DT);
            }
            if (SMOOTH) {
                const f32x4* sm = reinterpret_cast<const f32x4*>(smooth + (int64_t)idx * 8);
                f32x4 s0 = sm[0], s1 = sm[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[i][e] = v[i][e] * s0[e];
                    v[i][4 + e] = v[i][4 + e] * s1[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
        }
    }
    amax = block_absmax(amax);
    const float s = amax / 127.0f;
    if (threadIdx.x == 0) scale[row] = s;
    u32x2* yr = reinterpret_cast<u32x2*>(y + row * K);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < nv) {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                lo |= ((uint32_t)quant1(v[i][e], s) & 0xffu) << (8 * e);
                hi |= ((uint32_t)quant1(v[i][4 + e], s) & 0xffu) << (8 * e);
            }
            u32x2 o;
            o[0] = lo;
            o[1] = hi;
            yr[idx] = o;
        }
    }
}

// Generic path: any K, any alignment; reads the row twice.
template <int DT>
__global__ __launch_bounds__(kThreads) void dyn_quant_generic(const uint16_t* __restrict__ x, int64_t K,
                                                              const float* __restrict__ smooth,
                                                              int8_t* __restrict__ y, float* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * K;
    float amax = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += kThreads) {
        float v = load_half_bits(xr[k], DT);
        if (smooth) v = v * smooth[k];
        amax = fmaxf(amax, fabsf(v));
    }
    amax = block_absmax(amax);
    const float s = amax / 127.0f;
    if (threadIdx.x == 0) scale[row] = s;
    for (int64_t k = threadIdx.x; k < K; k += kThreads) {
        float v = load_half_bits(xr[k], DT);
        if (smooth) v = v * smooth[k];
        y[row * K + k] = (int8_t)quant1(v, s);
    }
}

template <int DT, int VPT>
hipError_t launch_vec(const uint16_t* x, int64_t rows, int64_t K, const float* smooth, int8_t* y, float* scale,
                      hipStream_t stream) {
    if (smooth)
        dyn_quant_vec<DT, VPT, true><<<dim3((uint32_t)rows), dim3(kThreads), 0, stream>>>(x, K, smooth, y, scale);
    else
        dyn_quant_vec<DT, VPT, false><<<dim3((uint32_t)rows), dim3(kThreads), 0, stream>>>(x, K, smooth, y, scale);
    return hipGetLastError();
}

template <int DT>
hipError_t dispatch(const uint16_t* x, int64_t rows, int64_t K, const float* smooth, int8_t* y, float* scale,
                    hipStream_t stream) {
    const bool aligned = (K % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 8 == 0) &&
                         (!smooth || (uintptr_t)smooth % 16 == 0);
    const int64_t per_thread = (K / 8 + kThreads - 1) / kThreads;
    if (aligned && K > 0 && per_thread <= 16) {
        if (per_thread <= 1) return launch_vec<DT, 1>(x, rows, K, smooth, y, scale, stream);
        if (per_thread <= 2) return launch_vec<DT, 2>(x, rows, K, smooth, y, scale, stream);
        if (per_thread <= 4) return launch_vec<DT, 4>(x, rows, K, smooth, y, scale, stream);
        if (per_thread <= 8) return launch_vec<DT, 8>(x, rows, K, smooth, y, scale, stream);
        return launch_vec<DT, 16>(x, rows, K, smooth, y, scale, stream);
    }
    dyn_quant_generic<DT><<<dim3((uint32_t)rows), dim3(kThreads), 0, stream>>>(x, K, smooth, y, scale);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dynamic_quant(const void* x, int x_dtype, int64_t rows, int64_t K, const float* smooth,
                                int8_t* y, float* scale, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    const uint16_t* xh = static_cast<const uint16_t*>(x);
    if (x_dtype == QK_BF16) return dispatch<QK_BF16>(xh, rows, K, smooth, y, scale, stream);
    return dispatch<QK_F16>(xh, rows, K, smooth, y, scale, stream);
}

}  // namespace qk
