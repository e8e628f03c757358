// RMSNorm and SwiGLU for the quantized MLP block, each alone or fused with
// npu_dynamic_quant, on gfx950 (RMSNorm also in float32, unfused).
//
// One workgroup per row: 512 threads (8 wave64) for the 16-bit vector paths
// of rows longer than 2048 elements (more waves per SIMD hide the row's load
// latency behind the other waves' arithmetic: measured 6.1 -> 5.2 us for the
// cfg5 RMSNorm+quant, 16 -> 12 us with the SwiGLU below), 256 threads
// otherwise.  The row is read once with 128-bit loads and kept in registers;
// row reductions (sum of squares, absmax) go through xor-shuffles inside a
// wave and LDS across the waves.  All arithmetic is fp32 and the 16-bit
// results are rounded to nearest even:
//   rms_norm:  rstd = 1 / sqrt(sum(x^2) / D + eps)  (IEEE division and square
//              root),  y = (x * rstd) * gamma                 (op contract:
//              op_plugin/ops/base_ops/opapi/RmsNormKernelOpApi.cpp:24-35,
//              golden test/test_custom_ops/test_npu_rms_norm.py:10-17)
//   swiglu:    y = a / (1 + exp(-a)) * b  with  a, b = h.chunk(2, -1), the
//              first half the gate (the halving of npu_geglu,
//              op_plugin/ops/v1r11/opapi/GeGluKernelNpuOpApi.cpp:29-38),
//              evaluated as (a * rcp(1 + exp2(-a * log2(e)))) * b on the
//              hardware exp2 and reciprocal (a few fp32 ulps from the exact
//              value, far below one 16-bit ulp; the 16-bit result stays
//              within one rounding step of the float64 oracle)
// The fused variants quantize the 16-bit y exactly as npu_dynamic_quant would
// quantize it after a round trip through HBM (s = absmax / 127, clamp(rint(y
// / s))), so fused and unfused paths give identical int8 rows; the fusion
// saves writing and re-reading y.  HBM-bound: RMSNorm+quant reads 2 B and
// writes 1 B per element, SwiGLU+quant reads 4 B and writes 1 B per output.
#include "common.h"

namespace qk {
namespace {

constexpr int kThreads = 256;

// Row reductions over the NW waves of a workgroup (DPP inside a wave; wave sums added in wave order).
template <int NW>
__device__ __forceinline__ float block_sum(float v) {
    __shared__ float red_sum[NW];
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red_sum[wave] = v;
    __syncthreads();
    if constexpr (NW == 4) return (red_sum[0] + red_sum[1]) + (red_sum[2] + red_sum[3]);
    float r = red_sum[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r += red_sum[w];
    return r;
}

template <int NW>
__device__ __forceinline__ float block_absmax_w(float amax) {
    __shared__ float red_amax[NW];
    amax = wave_max(amax);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red_amax[wave] = amax;
    __syncthreads();
    float r = red_amax[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = fmaxf(r, red_amax[w]);
    return r;
}

template <int DT>
__device__ __forceinline__ uint32_t to16(float f) {
    return DT == QK_BF16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f);
}

__device__ __forceinline__ void unpack8(u32x4 d, int dt, float v[8]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[2 * e] = load_half_bits(d[e] & 0xffffu, dt);
        v[2 * e + 1] = load_half_bits(d[e] >> 16, dt);
    }
}

// y (8 values, already rounded to 16 bits and widened back) -> 16-bit store, or
// (second pass) int8 under the row scale
template <int DT>
__device__ __forceinline__ u32x4 pack16(const uint32_t yb[8]) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = yb[2 * e] | (yb[2 * e + 1] << 16);
    return o;
}

__device__ __forceinline__ u32x2 packq(const float (&yf)[8], const RowQuant& rq) { return quant8(yf, rq); }

// ---------------------------------------------------------------- RMSNorm
// Vector path: D % 8 == 0, 16-byte aligned rows, D <= 8 * NT * VPT.
template <int DT, int NT, int VPT, bool QUANT>
__global__ __launch_bounds__(NT) void rms_norm_vec(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ gamma, int64_t D, float eps,
                                                         uint16_t* __restrict__ y, int8_t* __restrict__ q,
                                                         float* __restrict__ scale, float* __restrict__ rstd) {
    const int64_t row = blockIdx.x;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * D);
    const u32x4* gr = reinterpret_cast<const u32x4*>(gamma);
    const int nv = (int)(D >> 3);
    float v[VPT][8];
    u32x4 graw[VPT];
    float ss = 0.0f;
    // gamma's loads go out with the row's (they are L2 hits after the first rows), so the output pass does
    // not wait for a second round trip after the row reduction
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) graw[i] = gr[idx];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) {
            unpack8(__builtin_nontemporal_load(xr + idx), DT, v[i]);  // read once
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[i][e], v[i][e], ss);
        }
    }
    ss = block_sum<NT / 64>(ss);
    const float rs = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    // rstd is stored after the last barrier: a store ahead of a barrier makes its wave wait for the store's
    // completion there, and every other wave with it
    float amax = 0.0f;
    uint32_t yb[VPT][8];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) {
            float g[8];
            unpack8(graw[i], DT, g);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                yb[i][e] = to16<DT>((v[i][e] * rs) * g[e]);
                v[i][e] = load_half_bits(yb[i][e], DT);  // y as a later read of it would see it
                amax = fmaxf(amax, fabsf(v[i][e]));
            }
            if (!QUANT) __builtin_nontemporal_store(pack16<DT>(yb[i]), reinterpret_cast<u32x4*>(y + row * D) + idx);
        }
    }
    if (!QUANT) {
        if (threadIdx.x == 0 && rstd) rstd[row] = rs;
        return;
    }
    amax = block_absmax_w<NT / 64>(amax);
    const float s = amax / 127.0f;
    if (threadIdx.x == 0) {
        scale[row] = s;
        if (rstd) rstd[row] = rs;
    }
    const RowQuant rq = row_quant(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) __builtin_nontemporal_store(packq(v[i], rq), reinterpret_cast<u32x2*>(q + row * D) + idx);
    }
}

// Any D and alignment: the row is read again for the output pass.
template <int DT, bool QUANT>
__global__ __launch_bounds__(kThreads) void rms_norm_generic(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ gamma, int64_t D, float eps,
                                                             uint16_t* __restrict__ y, int8_t* __restrict__ q,
                                                             float* __restrict__ scale, float* __restrict__ rstd) {
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * D;
    float ss = 0.0f;
    for (int64_t d = threadIdx.x; d < D; d += kThreads) {
        const float v = load_half_bits(xr[d], DT);
        ss = __builtin_fmaf(v, v, ss);
    }
    ss = block_sum<4>(ss);
    const float rs = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    if (threadIdx.x == 0 && rstd) rstd[row] = rs;
    auto yat = [&](int64_t d) {
        return to16<DT>((load_half_bits(xr[d], DT) * rs) * load_half_bits(gamma[d], DT));
    };
    if (!QUANT) {
        for (int64_t d = threadIdx.x; d < D; d += kThreads) y[row * D + d] = (uint16_t)yat(d);
        return;
    }
    float amax = 0.0f;
    for (int64_t d = threadIdx.x; d < D; d += kThreads) amax = fmaxf(amax, fabsf(load_half_bits(yat(d), DT)));
    amax = block_absmax(amax);
    const float s = amax / 127.0f;
    if (threadIdx.x == 0) scale[row] = s;
    const RowQuant rq = row_quant(s);
    for (int64_t d = threadIdx.x; d < D; d += kThreads)
        q[row * D + d] = (int8_t)quant_row(load_half_bits(yat(d), DT), rq);
}

// ---------------------------------------------------------------- RMSNorm, float32
// The reference's golden case (fp32 x, gamma, y).  y = (x * rstd) * gamma stays
// fp32.  Vector path: D % 4 == 0, 16-byte aligned rows, D <= 4 * 256 * VPT.
template <int VPT>
__global__ __launch_bounds__(kThreads) void rms_norm_f32_vec(const float* __restrict__ x,
                                                             const float* __restrict__ gamma, int64_t D, float eps,
                                                             float* __restrict__ y, float* __restrict__ rstd) {
    const int64_t row = blockIdx.x;
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * D);
    const f32x4* gr = reinterpret_cast<const f32x4*>(gamma);
    const int nv = (int)(D >> 2);
    f32x4 v[VPT];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < nv) {
            v[i] = xr[idx];
#pragma unroll
            for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(v[i][e], v[i][e], ss);
        }
    }
    ss = block_sum<4>(ss);
    const float rs = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    if (threadIdx.x == 0 && rstd) rstd[row] = rs;
    f32x4* yr = reinterpret_cast<f32x4*>(y + row * D);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * kThreads;
        if (idx < nv) {
            const f32x4 g = gr[idx];
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = (v[i][e] * rs) * g[e];
            yr[idx] = o;
        }
    }
}

__global__ __launch_bounds__(kThreads) void rms_norm_f32_generic(const float* __restrict__ x,
                                                                 const float* __restrict__ gamma, int64_t D,
                                                                 float eps, float* __restrict__ y,
                                                                 float* __restrict__ rstd) {
    const int64_t row = blockIdx.x;
    const float* xr = x + row * D;
    float ss = 0.0f;
    for (int64_t d = threadIdx.x; d < D; d += kThreads) ss = __builtin_fmaf(xr[d], xr[d], ss);
    ss = block_sum<4>(ss);
    const float rs = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    if (threadIdx.x == 0 && rstd) rstd[row] = rs;
    for (int64_t d = threadIdx.x; d < D; d += kThreads) y[row * D + d] = (xr[d] * rs) * gamma[d];
}

// ---------------------------------------------------------------- SwiGLU (silu_mul: common.h)

template <int DT, int NT, int VPT, bool QUANT>
__global__ __launch_bounds__(NT) void swiglu_vec(const uint16_t* __restrict__ h, int64_t I,
                                                       uint16_t* __restrict__ y, int8_t* __restrict__ q,
                                                       float* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const u32x4* ar = reinterpret_cast<const u32x4*>(h + row * 2 * I);
    const u32x4* br = reinterpret_cast<const u32x4*>(h + row * 2 * I + I);
    const int nv = (int)(I >> 3);
    float v[VPT][8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) {
            float a[8], b[8];
            unpack8(__builtin_nontemporal_load(ar + idx), DT, a);  // read once
            unpack8(__builtin_nontemporal_load(br + idx), DT, b);
            uint32_t yb[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                yb[e] = to16<DT>(silu_mul(a[e], b[e]));
                v[i][e] = load_half_bits(yb[e], DT);
                amax = fmaxf(amax, fabsf(v[i][e]));
            }
            if (!QUANT) __builtin_nontemporal_store(pack16<DT>(yb), reinterpret_cast<u32x4*>(y + row * I) + idx);
        }
    }
    if (!QUANT) return;
    amax = block_absmax_w<NT / 64>(amax);
    const float s = amax / 127.0f;
    if (threadIdx.x == 0) scale[row] = s;
    const RowQuant rq = row_quant(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = threadIdx.x + i * NT;
        if (idx < nv) __builtin_nontemporal_store(packq(v[i], rq), reinterpret_cast<u32x2*>(q + row * I) + idx);
    }
}

template <int DT, bool QUANT>
__global__ __launch_bounds__(kThreads) void swiglu_generic(const uint16_t* __restrict__ h, int64_t I,
                                                           uint16_t* __restrict__ y, int8_t* __restrict__ q,
                                                           float* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const uint16_t* hr = h + row * 2 * I;
    auto yat = [&](int64_t i) {
        return to16<DT>(silu_mul(load_half_bits(hr[i], DT), load_half_bits(hr[I + i], DT)));
    };
    if (!QUANT) {
        for (int64_t i = threadIdx.x; i < I; i += kThreads) y[row * I + i] = (uint16_t)yat(i);
        return;
    }
    float amax = 0.0f;
    for (int64_t i = threadIdx.x; i < I; i += kThreads) amax = fmaxf(amax, fabsf(load_half_bits(yat(i), DT)));
    amax = block_absmax(amax);
    const float s = amax / 127.0f;
    if (threadIdx.x == 0) scale[row] = s;
    const RowQuant rq = row_quant(s);
    for (int64_t i = threadIdx.x; i < I; i += kThreads) q[row * I + i] = (int8_t)quant_row(load_half_bits(yat(i), DT), rq);
}

// ---------------------------------------------------------------- dispatch
template <int DT, int NT, int VPT>
hipError_t rms_vec(const uint16_t* x, const uint16_t* g, int64_t rows, int64_t D, float eps, uint16_t* y, int8_t* q,
                   float* scale, float* rstd, hipStream_t stream) {
    const dim3 grid((uint32_t)rows), block(NT);
    if (q) rms_norm_vec<DT, NT, VPT, true><<<grid, block, 0, stream>>>(x, g, D, eps, y, q, scale, rstd);
    else rms_norm_vec<DT, NT, VPT, false><<<grid, block, 0, stream>>>(x, g, D, eps, y, q, scale, rstd);
    return hipGetLastError();
}

template <int DT>
hipError_t rms_dispatch(const uint16_t* x, const uint16_t* g, int64_t rows, int64_t D, float eps, uint16_t* y,
                        int8_t* q, float* scale, float* rstd, hipStream_t stream) {
    const bool aligned = D % 8 == 0 && ((uintptr_t)x | (uintptr_t)g) % 16 == 0 &&
                         (q ? (uintptr_t)q % 8 == 0 : (uintptr_t)y % 16 == 0);
    const int64_t nv = D / 8;  // 16-byte vectors per row
    if (aligned && D > 0 && nv <= 256) return rms_vec<DT, 256, 1>(x, g, rows, D, eps, y, q, scale, rstd, stream);
    if (aligned && D > 0 && nv <= 8 * 512) {
        const int64_t per_thread = (nv + 511) / 512;
        if (per_thread <= 1) return rms_vec<DT, 512, 1>(x, g, rows, D, eps, y, q, scale, rstd, stream);
        if (per_thread <= 2) return rms_vec<DT, 512, 2>(x, g, rows, D, eps, y, q, scale, rstd, stream);
        if (per_thread <= 4) return rms_vec<DT, 512, 4>(x, g, rows, D, eps, y, q, scale, rstd, stream);
        return rms_vec<DT, 512, 8>(x, g, rows, D, eps, y, q, scale, rstd, stream);
    }
    const dim3 grid((uint32_t)rows), block(kThreads);
    if (q) rms_norm_generic<DT, true><<<grid, block, 0, stream>>>(x, g, D, eps, y, q, scale, rstd);
    else rms_norm_generic<DT, false><<<grid, block, 0, stream>>>(x, g, D, eps, y, q, scale, rstd);
    return hipGetLastError();
}

hipError_t rms_f32_dispatch(const float* x, const float* g, int64_t rows, int64_t D, float eps, float* y,
                            float* rstd, hipStream_t stream) {
    const dim3 grid((uint32_t)rows), block(kThreads);
    const bool aligned = D % 4 == 0 && ((uintptr_t)x | (uintptr_t)g | (uintptr_t)y) % 16 == 0;
    const int64_t per_thread = (D / 4 + kThreads - 1) / kThreads;
    if (aligned && per_thread <= 16) {
        if (per_thread <= 4) rms_norm_f32_vec<4><<<grid, block, 0, stream>>>(x, g, D, eps, y, rstd);
        else if (per_thread <= 8) rms_norm_f32_vec<8><<<grid, block, 0, stream>>>(x, g, D, eps, y, rstd);
        else rms_norm_f32_vec<16><<<grid, block, 0, stream>>>(x, g, D, eps, y, rstd);
    } else {
        rms_norm_f32_generic<<<grid, block, 0, stream>>>(x, g, D, eps, y, rstd);
    }
    return hipGetLastError();
}

template <int DT, int NT, int VPT>
hipError_t swi_vec(const uint16_t* h, int64_t rows, int64_t I, uint16_t* y, int8_t* q, float* scale,
                   hipStream_t stream) {
    const dim3 grid((uint32_t)rows), block(NT);
    if (q) swiglu_vec<DT, NT, VPT, true><<<grid, block, 0, stream>>>(h, I, y, q, scale);
    else swiglu_vec<DT, NT, VPT, false><<<grid, block, 0, stream>>>(h, I, y, q, scale);
    return hipGetLastError();
}

template <int DT>
hipError_t swi_dispatch(const uint16_t* h, int64_t rows, int64_t I, uint16_t* y, int8_t* q, float* scale,
                        hipStream_t stream) {
    const bool aligned = I % 8 == 0 && (uintptr_t)h % 16 == 0 && (q ? (uintptr_t)q % 8 == 0 : (uintptr_t)y % 16 == 0);
    const int64_t nv = I / 8;  // 16-byte vectors of each half row
    if (aligned && I > 0 && nv <= 256) return swi_vec<DT, 256, 1>(h, rows, I, y, q, scale, stream);
    if (aligned && I > 0 && nv <= 4 * 512) {
        const int64_t per_thread = (nv + 511) / 512;
        if (per_thread <= 1) return swi_vec<DT, 512, 1>(h, rows, I, y, q, scale, stream);
        if (per_thread <= 2) return swi_vec<DT, 512, 2>(h, rows, I, y, q, scale, stream);
        return swi_vec<DT, 512, 4>(h, rows, I, y, q, scale, stream);
    }
    const dim3 grid((uint32_t)rows), block(kThreads);
    if (q) swiglu_generic<DT, true><<<grid, block, 0, stream>>>(h, I, y, q, scale);
    else swiglu_generic<DT, false><<<grid, block, 0, stream>>>(h, I, y, q, scale);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_rms_norm(const void* x, int dt, const void* gamma, int64_t rows, int64_t D, float eps, void* y,
                           int8_t* q, float* scale, float* rstd, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (dt == QK_F32)  // unfused only: the fused quantization takes 16-bit rows
        return q ? hipErrorInvalidValue
                 : rms_f32_dispatch(static_cast<const float*>(x), static_cast<const float*>(gamma), rows, D, eps,
                                    static_cast<float*>(y), rstd, stream);
    const uint16_t* xh = static_cast<const uint16_t*>(x);
    const uint16_t* gh = static_cast<const uint16_t*>(gamma);
    uint16_t* yh = static_cast<uint16_t*>(y);
    if (dt == QK_BF16) return rms_dispatch<QK_BF16>(xh, gh, rows, D, eps, yh, q, scale, rstd, stream);
    return rms_dispatch<QK_F16>(xh, gh, rows, D, eps, yh, q, scale, rstd, stream);
}

hipError_t launch_swiglu(const void* h, int dt, int64_t rows, int64_t I, void* y, int8_t* q, float* scale,
                         hipStream_t stream) {
    if (rows == 0 || I == 0) return hipSuccess;
    const uint16_t* hh = static_cast<const uint16_t*>(h);
    uint16_t* yh = static_cast<uint16_t*>(y);
    if (dt == QK_BF16) return swi_dispatch<QK_BF16>(hh, rows, I, yh, q, scale, stream);
    return swi_dispatch<QK_F16>(hh, rows, I, yh, q, scale, stream);
}

}  // namespace qk
