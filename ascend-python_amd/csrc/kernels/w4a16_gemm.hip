// npu_weight_quant_batchmatmul (W4A16 / W8A16) for gfx950.
//
// out[m,n] = sum_g scale[g,n] * ( sum_{k in g} x[m,k]*w[k,n] + offset[g,n] * xs[m,g] ),
// xs[m,g] = sum_{k in g} x[m,k]: the group-wise antiquant (w + offset) * scale
// applied to the partial sums instead of to each weight, so the dequantized
// weight is never rounded to 16 bits and the MFMA consumes the raw integers.
//
// int4 unpack ("magic exponent", a published int->float trick): a nibble u
// placed in the low mantissa bits of a bf16 0x4300 (=128) / fp16 0x6400
// (=1024) reads as 128+u / 1024+u exactly.  With the two's-complement nibble
// flipped to offset binary (u = w+8) the MFMA operand is v = w + BASE
// (BASE = 136 for bf16, 1032 for fp16), and the bias is removed per group:
//   sum_k x*w = sum_k x*v - BASE * xs,
// where xs comes from one extra MFMA against a vector of ones.  Per group each
// accumulator then takes  acc += s*A_g + s*(offset - BASE)*xs.
//
// Column mapping: lane l of a wave reads packed word column wc = wc0 + (l&15)
// for 8 consecutive k rows; nibble j of those 8 words is the B operand of MFMA
// tile j, so tile j column c is output column 8*(wc0+c)+j and each lane ends
// up owning 8 consecutive output columns (one 16-byte store).
#include "common.h"

namespace qk {
namespace {

constexpr int kThreads = 256;

template <int DT>
struct Mfma;

template <>
struct Mfma<QK_BF16> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    static constexpr uint32_t MAGIC = 0x43004300u;  // bf16 pair (128, 128)
    static constexpr uint32_t ONES = 0x3f803f80u;   // bf16 pair (1, 1)
    static constexpr float BASE = 136.0f;
    static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0,
                                                       0, 0);
    }
};

template <>
struct Mfma<QK_F16> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    static constexpr uint32_t MAGIC = 0x64006400u;  // fp16 pair (1024, 1024)
    static constexpr uint32_t ONES = 0x3c003c00u;   // fp16 pair (1, 1)
    static constexpr float BASE = 1032.0f;
    static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0,
                                                      0, 0);
    }
};

__device__ __forceinline__ void store_out8(void* out, int out_dtype, int64_t off, const float v[8]) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        uint32_t lo, hi;
        if (out_dtype == QK_BF16) {
            lo = f32_to_bf16_bits(v[2 * e]);
            hi = f32_to_bf16_bits(v[2 * e + 1]);
        } else {
            lo = f32_to_f16_bits(v[2 * e]);
            hi = f32_to_f16_bits(v[2 * e + 1]);
        }
        o[e] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + off) = o;
}

// Workgroup tile: 16 rows x 128 columns (16 packed word columns); the four
// waves split the K groups round-robin and are reduced through LDS in a fixed
// order, so results are deterministic.
template <int DT, bool HAS_OFF>
__global__ __launch_bounds__(kThreads) void w4_tile16(WqbmmArgs p) {
    typedef Mfma<DT> MM;
    __shared__ float red[4][16][128 + 4];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int fr = lane & 15;
    const int kg = lane >> 4;  // which 8-row slice of a 32-row MFMA block
    const int64_t NW = p.N >> 3;
    const int64_t wc = (int64_t)blockIdx.x * 16 + fr;
    const int64_t m0 = (int64_t)blockIdx.y * 16;
    const int64_t G = p.group;
    const int64_t ngroups = p.K / G;
    const bool col_ok = wc < NW;
    const bool row_ok = (m0 + fr) < p.M;
    const uint16_t* xrow = static_cast<const uint16_t*>(p.x) + (m0 + fr) * p.K;
    const uint32_t* W = static_cast<const uint32_t*>(p.w);
    const uint16_t* S = static_cast<const uint16_t*>(p.scale);
    const uint16_t* O = static_cast<const uint16_t*>(p.offset);
    const u32x4 ones = {MM::ONES, MM::ONES, MM::ONES, MM::ONES};

    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    for (int64_t g = wave; g < ngroups; g += 4) {
        f32x4 ag[8], xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; ++j) ag[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        for (int64_t kb = 0; kb < G; kb += 32) {
            const int64_t k = g * G + kb + 8 * kg;
            u32x4 a = {0u, 0u, 0u, 0u};
            if (row_ok) a = *reinterpret_cast<const u32x4*>(xrow + k);
            uint32_t w[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) w[r] = col_ok ? W[(k + r) * NW + wc] : 0x88888888u;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                u32x4 b;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t lo = (w[2 * q] >> (4 * j)) & 0xfu;
                    const uint32_t hi = (w[2 * q + 1] >> (4 * j)) & 0xfu;
                    b[q] = ((lo | (hi << 16)) ^ 0x00080008u) | MM::MAGIC;
                }
                ag[j] = MM::mma(a, b, ag[j]);
            }
            xs = MM::mma(a, ones, xs);
        }
        if (col_ok) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t n = 8 * wc + j;
                const float s = load_half_bits(S[g * p.N + n], p.s_dtype);
                const float off = HAS_OFF ? load_half_bits(O[g * p.N + n], p.s_dtype) : 0.0f;
                const float sb = s * (off - MM::BASE);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[j][r] = __builtin_fmaf(s, ag[j][r], __builtin_fmaf(sb, xs[r], acc[j][r]));
            }
        }
    }

#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][4 * kg + r][8 * fr + j] = acc[j][r];
    __syncthreads();

    const int t = threadIdx.x;
    const int row = t >> 4;
    const int c8 = (t & 15) * 8;
    const int64_t m = m0 + row;
    const int64_t n = (int64_t)blockIdx.x * 128 + c8;
    if (m < p.M && n < p.N) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float s = red[0][row][c8 + e];
            s += red[1][row][c8 + e];
            s += red[2][row][c8 + e];
            s += red[3][row][c8 + e];
            if (p.bias_dtype) s += load_scalar(p.bias, n + e, p.bias_dtype);
            v[e] = s;
        }
        store_out8(p.out, p.out_dtype, m * p.N + n, v);
    }
}

// Any shape: one thread per output, fp32 sums per group then the same
// group-wise scale/offset algebra as the tiled kernel.
__global__ __launch_bounds__(kThreads) void wq_generic(WqbmmArgs p) {
    const int64_t total = p.M * p.N;
    const int64_t G = p.group > 0 ? p.group : p.K;
    const int64_t ngroups = G > 0 ? (p.K + G - 1) / G : 0;
    const uint16_t* X = static_cast<const uint16_t*>(p.x);
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t m = idx / p.N, n = idx % p.N;
        float acc = 0.0f;
        for (int64_t g = 0; g < ngroups; ++g) {
            float sw = 0.0f, xs = 0.0f;
            const int64_t kend = (g + 1) * G < p.K ? (g + 1) * G : p.K;
            for (int64_t k = g * G; k < kend; ++k) {
                const float xv = load_half_bits(X[m * p.K + k], p.x_dtype);
                int wv;
                if (p.w_dtype == QK_I32) {
                    const uint32_t word = static_cast<const uint32_t*>(p.w)[k * (p.N >> 3) + (n >> 3)];
                    wv = (int)((word >> (4 * (n & 7))) & 0xfu);
                    wv = wv >= 8 ? wv - 16 : wv;
                } else {
                    wv = static_cast<const int8_t*>(p.w)[k * p.N + n];
                }
                sw = __builtin_fmaf(xv, (float)wv, sw);
                xs += xv;
            }
            const float s = load_half_bits(static_cast<const uint16_t*>(p.scale)[g * p.N + n], p.s_dtype);
            const float off =
                p.offset ? load_half_bits(static_cast<const uint16_t*>(p.offset)[g * p.N + n], p.s_dtype) : 0.0f;
            acc = __builtin_fmaf(s, __builtin_fmaf(off, xs, sw), acc);
        }
        if (p.bias_dtype) acc += load_scalar(p.bias, n, p.bias_dtype);
        uint16_t* o = static_cast<uint16_t*>(p.out);
        o[m * p.N + n] = (uint16_t)(p.out_dtype == QK_BF16 ? f32_to_bf16_bits(acc) : f32_to_f16_bits(acc));
    }
}

template <int DT>
hipError_t launch_tile16(const WqbmmArgs& p, hipStream_t stream) {
    dim3 grid((uint32_t)((p.N / 8 + 15) / 16), (uint32_t)((p.M + 15) / 16));
    if (p.offset)
        w4_tile16<DT, true><<<grid, dim3(kThreads), 0, stream>>>(p);
    else
        w4_tile16<DT, false><<<grid, dim3(kThreads), 0, stream>>>(p);
    return hipGetLastError();
}

__global__ void int4_pack_kernel(const void* w, int w_dtype, int64_t K, int64_t N, int32_t* packed) {
    const int64_t NW = N >> 3;
    const int64_t total = K * NW;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = idx / NW, j = idx % NW;
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t e = k * N + 8 * j + i;
            const int32_t v = w_dtype == QK_I8 ? (int32_t) static_cast<const int8_t*>(w)[e]
                                               : static_cast<const int32_t*>(w)[e];
            word |= ((uint32_t)v & 0xfu) << (4 * i);
        }
        packed[idx] = (int32_t)word;
    }
}

}  // namespace

size_t weight_quant_bmm_workspace(int64_t, int64_t, int64_t, int, int64_t) { return 0; }

hipError_t launch_weight_quant_bmm(const WqbmmArgs& a, void*, size_t, hipStream_t stream) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    WqbmmArgs p = a;
    if (p.group == 0) p.group = p.K;  // per channel == one group spanning K
    const bool tile_ok = p.w_dtype == QK_I32 && p.K > 0 && p.group % 32 == 0 &&
                         p.K % p.group == 0 && ((uintptr_t)p.x % 16 == 0) && ((uintptr_t)p.out % 16 == 0) &&
                         ((uintptr_t)p.w % 4 == 0);
    if (tile_ok) return p.x_dtype == QK_BF16 ? launch_tile16<QK_BF16>(p, stream) : launch_tile16<QK_F16>(p, stream);
    const int64_t total = p.M * p.N;
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    wq_generic<<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(p);
    return hipGetLastError();
}

hipError_t launch_int4_pack(const void* w, int w_dtype, int64_t K, int64_t N, int32_t* packed, hipStream_t stream) {
    const int64_t total = K * (N >> 3);
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    int4_pack_kernel<<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(w, w_dtype, K, N, packed);
    return hipGetLastError();
}

}  // namespace qk
