// npu_weight_quant_batchmatmul (W4A16 / W8A16) for gfx950.
//
// out[m,n] = sum_g scale[g,n] * ( sum_{k in g} x[m,k]*w[k,n] + offset[g,n] * xs[m,g] ),
// xs[m,g] = sum_{k in g} x[m,k]: the group-wise antiquant (w + offset) * scale
// applied to partial sums instead of to each weight, so the dequantized weight
// is never rounded to 16 bits and the MFMA consumes the raw integers.  The
// identity is linear in the partial sums, so any K range that stays inside one
// group (a "piece") can be scaled on its own.
//
// int4 unpack ("magic exponent", a published int->float trick): a nibble u
// placed in the low mantissa bits of a bf16 0x4300 (=128) / fp16 0x6400
// (=1024) reads as 128+u / 1024+u exactly.  With the two's-complement nibble
// flipped to offset binary (u = w+8) the MFMA operand is v = w + BASE
// (BASE = 136 for bf16, 1032 for fp16), and the bias is removed per piece:
//   sum_k x*w = sum_k x*v - BASE * xs,
// where xs comes from one extra MFMA against a vector of ones.  Each piece
// then adds  s*A + s*(offset - BASE)*xs  to the accumulator.
//
// Decode kernel (w4_skinny): HBM weight stream for M <= 64.  A workgroup owns
// a strip of WCS packed word columns (8*WCS output columns) over all of K; its
// waves take 128-row chunks of K round-robin, stream them with every load of
// the next chunk in flight while the current one is unpacked and multiplied,
// and are reduced through LDS in a fixed order (deterministic, no workspace).
// MFMA column c of a wave maps to word column (c % WCS) and nibble
// t*(16/WCS) + c/WCS of tile t, so every weight word is unpacked by exactly
// the lanes that need it.
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

// B operand of one MFMA tile: nibble `j` (byte bj = j/2, shift 4*(j&1)) of 8
// offset-binary words, rows 0..7 -> bf16/fp16 lanes 0..7 (pairs per dword).
template <uint32_t MAGIC>
__device__ __forceinline__ u32x4 unpack_tile(const uint32_t w[8], uint32_t sel, uint32_t shift) {
    u32x4 b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t pair = __builtin_amdgcn_perm(w[2 * q + 1], w[2 * q], sel) >> shift;
        b[q] = (pair & 0x000f000fu) | MAGIC;
    }
    return b;
}

constexpr int CHUNK = 128;  // K rows a wave streams per step (4 MFMA K-blocks)

template <int DT, int WCS, int MB, int NWAVE, bool HAS_OFF>
__global__ __launch_bounds__(NWAVE * 64) void w4_skinny(WqbmmArgs p) {
    typedef Mfma<DT> MM;
    constexpr int T = WCS / 2;        // MFMA tiles per wave (16 columns each)
    constexpr int JSTEP = 16 / WCS;   // nibble stride between tiles
    constexpr int NCOL = 8 * WCS;     // output columns of the strip
    constexpr int ROWS = 16 * MB;
    __shared__ float red[NWAVE][ROWS][NCOL + 1];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c = lane & 15;
    const int kg = lane >> 4;
    const int64_t NW = p.N >> 3;
    // 1-D grid: strips sharing 128-byte weight lines land on one XCD
    const int nstrip = (int)((NW + WCS - 1) / WCS);
    const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int strip = bid % nstrip;
    const int64_t wc = (int64_t)strip * WCS + (c % WCS);
    const bool col_ok = wc < NW;
    const int64_t m0 = (int64_t)(bid / nstrip) * ROWS;
    const int64_t G = p.group;
    const int64_t piece = G < CHUNK ? G : CHUNK;
    const int64_t nchunk = p.K / CHUNK;
    const uint32_t* W = static_cast<const uint32_t*>(p.w);
    const uint16_t* X = static_cast<const uint16_t*>(p.x);
    const uint16_t* S = static_cast<const uint16_t*>(p.scale);
    const uint16_t* O = static_cast<const uint16_t*>(p.offset);
    const u32x4 ones = {MM::ONES, MM::ONES, MM::ONES, MM::ONES};

    int jt[T];
    uint32_t sel[T], shf[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        jt[t] = t * JSTEP + c / WCS;
        const uint32_t bj = (uint32_t)jt[t] >> 1;
        sel[t] = bj | ((4u + bj) << 16) | 0x0c000c00u;
        shf[t] = 4u * ((uint32_t)jt[t] & 1u);
    }
    bool row_ok[MB];
    const uint16_t* xrow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int64_t m = m0 + 16 * mb + c;
        row_ok[mb] = m < p.M;
        xrow[mb] = X + (row_ok[mb] ? m : 0) * p.K;
    }

    f32x4 acc[MB][T];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[mb][t] = (f32x4){0.f, 0.f, 0.f, 0.f};

    uint32_t wbuf[2][4][8];
    u32x4 xbuf[2][4][MB];

    auto load_chunk = [&](int64_t ch, uint32_t (&wv)[4][8], u32x4 (&xv)[4][MB]) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const int64_t k = ch * CHUNK + kb * 32 + 8 * kg;
#pragma unroll
            for (int r = 0; r < 8; ++r) wv[kb][r] = col_ok ? W[(k + r) * NW + wc] : 0u;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                xv[kb][mb] = row_ok[mb] ? *reinterpret_cast<const u32x4*>(xrow[mb] + k) : (u32x4){0u, 0u, 0u, 0u};
        }
    };

    auto compute_chunk = [&](int64_t ch, uint32_t (&wv)[4][8], u32x4 (&xv)[4][MB]) {
        f32x4 ag[MB][T], xs[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            xs[mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < T; ++t) ag[mb][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            uint32_t w8[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) w8[r] = wv[kb][r] ^ 0x88888888u;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const u32x4 b = unpack_tile<MM::MAGIC>(w8, sel[t], shf[t]);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) ag[mb][t] = MM::mma(xv[kb][mb], b, ag[mb][t]);
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) xs[mb] = MM::mma(xv[kb][mb], ones, xs[mb]);
            const int64_t kend = ch * CHUNK + (kb + 1) * 32;
            if (kend % piece == 0) {   // end of a piece: fold it into the accumulators
                const int64_t g = (kend - 1) / G;
                if (col_ok) {
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        const int64_t n = 8 * wc + jt[t];
                        const float s = load_half_bits(S[g * p.N + n], p.s_dtype);
                        const float off = HAS_OFF ? load_half_bits(O[g * p.N + n], p.s_dtype) : 0.0f;
                        const float sb = s * (off - MM::BASE);
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                acc[mb][t][r] = __builtin_fmaf(s, ag[mb][t][r], __builtin_fmaf(sb, xs[mb][r], acc[mb][t][r]));
                    }
                }
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    xs[mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int t = 0; t < T; ++t) ag[mb][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    };

    int64_t ch = wave;
    if (ch < nchunk) load_chunk(ch, wbuf[0], xbuf[0]);
    while (ch < nchunk) {
        const int64_t nx = ch + NWAVE;
        if (nx < nchunk) load_chunk(nx, wbuf[1], xbuf[1]);
        compute_chunk(ch, wbuf[0], xbuf[0]);
        if (nx >= nchunk) break;
        const int64_t nx2 = nx + NWAVE;
        if (nx2 < nchunk) load_chunk(nx2, wbuf[0], xbuf[0]);
        compute_chunk(nx, wbuf[1], xbuf[1]);
        ch = nx2;
    }

    // deterministic cross-wave reduction: LDS, summed in wave order
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][16 * mb + 4 * kg + r][8 * (c % WCS) + jt[t]] = acc[mb][t][r];
    __syncthreads();
    uint16_t* out = static_cast<uint16_t*>(p.out);
    const int64_t n0 = (int64_t)strip * NCOL;
    for (int i = threadIdx.x; i < ROWS * NCOL; i += NWAVE * 64) {
        const int row = i / NCOL, col = i % NCOL;
        const int64_t m = m0 + row, n = n0 + col;
        if (m >= p.M || n >= p.N) continue;
        float v = red[0][row][col];
#pragma unroll
        for (int w = 1; w < NWAVE; ++w) v += red[w][row][col];
        if (p.bias_dtype) v += load_scalar(p.bias, n, p.bias_dtype);
        out[m * p.N + n] = (uint16_t)(p.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
    }
}

// Any shape: one thread per output, fp32 sums per group then the same
// group-wise scale/offset algebra as the tiled kernels.
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

template <int DT, int WCS, int MB, int NWAVE>
hipError_t launch_skinny(const WqbmmArgs& p, hipStream_t stream) {
    constexpr int ROWS = 16 * MB;
    const int64_t NW = p.N / 8;
    const int64_t nblk = ((NW + WCS - 1) / WCS) * ((p.M + ROWS - 1) / ROWS);
    if (nblk >= (int64_t)1 << 31) return hipErrorInvalidValue;
    dim3 grid((uint32_t)nblk);
    if (p.offset)
        w4_skinny<DT, WCS, MB, NWAVE, true><<<grid, dim3(NWAVE * 64), 0, stream>>>(p);
    else
        w4_skinny<DT, WCS, MB, NWAVE, false><<<grid, dim3(NWAVE * 64), 0, stream>>>(p);
    return hipGetLastError();
}

template <int DT>
hipError_t dispatch_skinny(const WqbmmArgs& p, hipStream_t stream) {
    if (p.M <= 16) return launch_skinny<DT, 4, 1, 8>(p, stream);
    return launch_skinny<DT, 4, 2, 8>(p, stream);
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
    // pieces of min(group, 128) rows must tile the 128-row chunks
    const bool group_ok = p.group % 32 == 0 && (p.group % CHUNK == 0 || CHUNK % p.group == 0);
    const bool fast = p.w_dtype == QK_I32 && p.K > 0 && p.K % CHUNK == 0 && p.K % p.group == 0 && group_ok &&
                      ((uintptr_t)p.x % 16 == 0) && ((uintptr_t)p.w % 4 == 0);
    if (fast) return p.x_dtype == QK_BF16 ? dispatch_skinny<QK_BF16>(p, stream) : dispatch_skinny<QK_F16>(p, stream);
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
