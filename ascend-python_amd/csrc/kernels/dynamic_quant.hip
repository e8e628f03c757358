// npu_dynamic_quant for gfx950: per-row symmetric int8 quantization.
//
// One 256- or 512-thread workgroup per row.  The row is read once with
// 128-bit loads (8 halves per lane per load) and kept in registers; the
// absmax is reduced across each wave with DPP and lane reads and across the
// waves through LDS; the quantized row is written with 64-bit stores.  The
// arithmetic is exactly the op contract: s = amax / 127 (IEEE division),
// y = clamp(rint(x / s)) with ties to even, a zero row giving s = 0, y = 0.
// HBM-bound: 2 B read + 1 B written per element, 4 B per row for the scale.
#include <cstdlib>

#include "common.h"

namespace qk {
namespace {

constexpr int kThreads = 256;

// Vector path: K % 8 == 0, 16-byte aligned rows, K <= 8 * NT * VPT.  One NT-thread workgroup per row: the
// row is read once with 16-byte loads, all issued before the first reduction, and stays packed in registers
// (each value is widened where it is used, in the absmax and again in the quantizer, which keeps the register
// count, and so the number of rows in flight per CU, high).  The absmax is reduced across each wave with DPP
// row rotations and lane reads and across the waves through LDS.
template <int DT, int NT, int VPT, bool SMOOTH>
__global__ __launch_bounds__(NT) void dyn_quant_vec(const uint16_t* __restrict__ x, int64_t K,
                                                    const float* __restrict__ smooth, int8_t* __restrict__ y,
                                                    float* __restrict__ scale) {
    constexpr int NW = NT / 64;
    __shared__ float red[NW];
    const int nv = (int)(K >> 3);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = blockIdx.x;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * K);
    u32x4 raw[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) raw[i] = __builtin_nontemporal_load(xr + idx);  // read once
    }
    float sm[SMOOTH ? VPT : 1][8];
    if constexpr (SMOOTH) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int idx = threadIdx.x + i * NT;
            if (idx < nv) {
                const f32x4* sp = reinterpret_cast<const f32x4*>(smooth + (int64_t)idx * 8);
                const f32x4 s0 = sp[0], s1 = sp[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sm[i][e] = s0[e];
                    sm[i][4 + e] = s1[e];
                }
            }
        }
    }
    auto value = [&](int i, int e) {
        const uint32_t d = raw[i][e >> 1];
        float v = load_half_bits((e & 1) ? (d >> 16) : (d & 0xffffu), DT);
        if constexpr (SMOOTH) v = v * sm[i][e];
        return v;
    };
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) {
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(value(i, e)));
        }
    }
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, red[w]);
    const float s = m / 127.0f;
    if (threadIdx.x == 0) scale[row] = s;
    const RowQuant rq = row_quant(s);
    u32x2* yr = reinterpret_cast<u32x2*>(y + row * K);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) {
            float vf[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) vf[e] = value(i, e);
            __builtin_nontemporal_store(quant8(vf, rq), yr + idx);  // written once (measured 24.5 -> 23.1 us at cfg4)
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
    const RowQuant rq = row_quant(s);
    for (int64_t k = threadIdx.x; k < K; k += kThreads) {
        float v = load_half_bits(xr[k], DT);
        if (smooth) v = v * smooth[k];
        y[row * K + k] = (int8_t)quant_row(v, rq);
    }
}

// The quantizer for a row whose absmax arrives as `parts` partial maxima (amax_part[row * parts + j], each the
// largest |x| of one column slice, taken with fmaxf from +0 as above): each wave takes the largest of the
// row's partials itself (one or two loads per lane and a DPP / readlane reduction: no LDS, no barrier) and
// quantizes its vectors.  The same s and y as dyn_quant_vec, whose absmax is the same maximum.  Workgroup
// bid: row bid / chunks, vectors (bid % chunks) * 256 * VPT + ...; the workgroup of chunk 0 stores the scale.
template <int DT, int VPT>
__global__ __launch_bounds__(kThreads) void dyn_quant_premax(const uint16_t* __restrict__ x, int64_t K, int chunks,
                                                             const float* __restrict__ amax_part, int parts,
                                                             int8_t* __restrict__ y, float* __restrict__ scale) {
    const int64_t row = blockIdx.x / chunks;
    const int chunk = blockIdx.x % chunks;
    const int nv = (int)(K >> 3);
    const int base = chunk * (kThreads * VPT) + threadIdx.x;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * K);
    u32x4 raw[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i)
        if (base + i * kThreads < nv) raw[i] = __builtin_nontemporal_load(xr + base + i * kThreads);  // read once
    const int lane = threadIdx.x & 63;
    float amax = 0.0f;
    for (int j = lane; j < parts; j += 64) amax = fmaxf(amax, amax_part[row * parts + j]);
    const float s = wave_max(amax) / 127.0f;
    if (chunk == 0 && threadIdx.x == 0) scale[row] = s;
    const RowQuant rq = row_quant(s);
    u32x2* yr = reinterpret_cast<u32x2*>(y + row * K);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = base + i * kThreads;
        if (idx < nv) {
            float vf[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t d = raw[i][e >> 1];
                vf[e] = load_half_bits((e & 1) ? (d >> 16) : (d & 0xffffu), DT);
            }
            __builtin_nontemporal_store(quant8(vf, rq), yr + idx);  // written once
        }
    }
}

// One row per workgroup.  512 threads where a row has at least 1024 vectors (cfg4, K = 8192: 20.5-20.8 us against
// 21.2-21.5 with 256 threads and 26.8 with 1024, one box); 256 below that.
template <int DT, int NT, int VPT>
hipError_t launch_vec(const uint16_t* x, int64_t rows, int64_t K, const float* smooth, int8_t* y, float* scale,
                      hipStream_t stream) {
    const dim3 grid((uint32_t)rows), block(NT);
    if (smooth)
        dyn_quant_vec<DT, NT, VPT, true><<<grid, block, 0, stream>>>(x, K, smooth, y, scale);
    else
        dyn_quant_vec<DT, NT, VPT, false><<<grid, block, 0, stream>>>(x, K, smooth, y, scale);
    return hipGetLastError();
}

template <int DT>
hipError_t dispatch(const uint16_t* x, int64_t rows, int64_t K, const float* smooth, int8_t* y, float* scale,
                    hipStream_t stream) {
    const bool aligned = (K % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 8 == 0) &&
                         (!smooth || (uintptr_t)smooth % 16 == 0);
    const int64_t nv = K / 8;
    if (aligned && K > 0 && rows < ((int64_t)1 << 31) && nv <= 512 * 16) {
        if (nv < 1024) {
            if (nv <= 256) return launch_vec<DT, 256, 1>(x, rows, K, smooth, y, scale, stream);
            if (nv <= 512) return launch_vec<DT, 256, 2>(x, rows, K, smooth, y, scale, stream);
            return launch_vec<DT, 256, 4>(x, rows, K, smooth, y, scale, stream);
        }
        if (nv <= 1024) return launch_vec<DT, 512, 2>(x, rows, K, smooth, y, scale, stream);
        if (nv <= 2048) return launch_vec<DT, 512, 4>(x, rows, K, smooth, y, scale, stream);
        if (nv <= 4096) return launch_vec<DT, 512, 8>(x, rows, K, smooth, y, scale, stream);
        return launch_vec<DT, 512, 16>(x, rows, K, smooth, y, scale, stream);
    }
    dyn_quant_generic<DT><<<dim3((uint32_t)rows), dim3(kThreads), 0, stream>>>(x, K, smooth, y, scale);
    return hipGetLastError();
}

template <int DT>
hipError_t dispatch_premax(const uint16_t* x, int64_t rows, int64_t K, const float* amax_part, int parts, int8_t* y,
                           float* scale, hipStream_t stream) {
    const int64_t nv = K / 8;
    const int vpt = nv % (2 * kThreads) == 0 ? 2 : 1;  // whole chunks of two vectors per thread where they fit
    const int64_t chunks = (nv + (int64_t)kThreads * vpt - 1) / ((int64_t)kThreads * vpt);
    if (chunks * rows >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    const dim3 grid((uint32_t)(chunks * rows)), block(kThreads);
    if (vpt == 2)
        dyn_quant_premax<DT, 2><<<grid, block, 0, stream>>>(x, K, (int)chunks, amax_part, parts, y, scale);
    else
        dyn_quant_premax<DT, 1><<<grid, block, 0, stream>>>(x, K, (int)chunks, amax_part, parts, y, scale);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dynamic_quant_premax(const void* x, int x_dtype, int64_t rows, int64_t K, const float* amax_part,
                                       int parts, int8_t* y, float* scale, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (K <= 0 || K % 8 != 0 || K >= ((int64_t)1 << 31) || parts <= 0 || (uintptr_t)x % 16 != 0 ||
        (uintptr_t)y % 8 != 0 || !amax_part)
        return hipErrorInvalidValue;
    const uint16_t* xh = static_cast<const uint16_t*>(x);
    if (x_dtype == QK_BF16) return dispatch_premax<QK_BF16>(xh, rows, K, amax_part, parts, y, scale, stream);
    return dispatch_premax<QK_F16>(xh, rows, K, amax_part, parts, y, scale, stream);
}

hipError_t launch_dynamic_quant(const void* x, int x_dtype, int64_t rows, int64_t K, const float* smooth,
                                int8_t* y, float* scale, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    const uint16_t* xh = static_cast<const uint16_t*>(x);
    if (x_dtype == QK_BF16) return dispatch<QK_BF16>(xh, rows, K, smooth, y, scale, stream);
    return dispatch<QK_F16>(xh, rows, K, smooth, y, scale, stream);
}

}  // namespace qk
