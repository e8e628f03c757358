// npu_quant_matmul (W8A8) for gfx950.
//
// acc[m,n] = sum_k x1[m,k] * x2[k,n] on int8 MFMA (v_mfma_i32_16x16x64_i8,
// int32 accumulation, exact), then the fused epilogue of QmmEpilogue
// (per-token x per-channel scale, bias, RNE cast) in registers before the
// single store of each output element.
//
// Tiled kernel: a 256-thread workgroup (4 wave64 in a 2x2 grid) owns a
// BM x BN output tile and walks K in steps of 64 bytes.  Both operands are
// staged in LDS k-contiguous ([row][k], rows padded to 80 B so the 16-lane
// 128-bit fragment reads hit distinct banks); the next K step is fetched into
// registers while the current one is multiplied.  A weight given as
// [K,N]-contiguous is transposed 4x4 bytes at a time with v_perm_b32 on its
// way into LDS, so both storage orders feed the same MFMA fragments.
#include "common.h"

namespace qk {
namespace {

constexpr int kThreads = 256;
constexpr int BK = 64;        // K bytes per step == K of one i8 MFMA
constexpr int LDS_ROW = 80;   // padded row stride (bytes) of the LDS tiles

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// r[i] holds 4 bytes (4 consecutive n) of k-row i; returns o[j] = 4 bytes
// (4 consecutive k) of column j.
__device__ __forceinline__ void transpose4x4(const uint32_t r[4], uint32_t o[4]) {
    const uint32_t t0 = perm(r[1], r[0], 0x05010400u);
    const uint32_t t1 = perm(r[1], r[0], 0x07030602u);
    const uint32_t t2 = perm(r[3], r[2], 0x05010400u);
    const uint32_t t3 = perm(r[3], r[2], 0x07030602u);
    o[0] = perm(t2, t0, 0x05040100u);
    o[1] = perm(t2, t0, 0x07060302u);
    o[2] = perm(t3, t1, 0x05040100u);
    o[3] = perm(t3, t1, 0x07060302u);
}

template <int BM, int BN, bool B_KN>
struct TileLoader {
    // A and [N,K] B: 16-byte chunks (row, kc), 4 per row.
    static constexpr int A_CHUNKS = BM * 4;
    static constexpr int A_PER_T = (A_CHUNKS + kThreads - 1) / kThreads;
    static constexpr int B_CHUNKS = BN * 4;
    static constexpr int B_PER_T = (B_CHUNKS + kThreads - 1) / kThreads;
    // [K,N] B: units of 4 k-rows x 8 n bytes.
    static constexpr int B_UNITS = 16 * (BN / 8);
    static constexpr int BU_PER_T = (B_UNITS + kThreads - 1) / kThreads;

    i32x4 a[A_PER_T];
    i32x4 b[B_PER_T];
    u32x2 bu[BU_PER_T][4];

    __device__ __forceinline__ void load(const QmmArgs& p, int64_t m0, int64_t n0, int64_t k0) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int c = tid + i * kThreads;
            const int r = c >> 2, kc = c & 3;
            const int64_t m = m0 + r, k = k0 + 16 * kc;
            i32x4 v = {0, 0, 0, 0};
            if (c < A_CHUNKS && m < p.M && k < p.K) v = *reinterpret_cast<const i32x4*>(p.a + m * p.lda + k);
            a[i] = v;
        }
        if (!B_KN) {
#pragma unroll
            for (int i = 0; i < B_PER_T; ++i) {
                const int c = tid + i * kThreads;
                const int r = c >> 2, kc = c & 3;
                const int64_t n = n0 + r, k = k0 + 16 * kc;
                i32x4 v = {0, 0, 0, 0};
                if (c < B_CHUNKS && n < p.N && k < p.K) v = *reinterpret_cast<const i32x4*>(p.b + n * p.sbn + k);
                b[i] = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < BU_PER_T; ++i) {
                const int u = tid + i * kThreads;
                const int o = u % (BN / 8), q = u / (BN / 8);
                const int64_t n = n0 + 8 * o;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int64_t k = k0 + 4 * q + rr;
                    u32x2 v = {0u, 0u};
                    if (u < B_UNITS && n < p.N && k < p.K)
                        v = *reinterpret_cast<const u32x2*>(p.b + k * p.sbk + n);
                    bu[i][rr] = v;
                }
            }
        }
    }

    __device__ __forceinline__ void store(int8_t* As, int8_t* Bs) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int c = tid + i * kThreads;
            if (c < A_CHUNKS) *reinterpret_cast<i32x4*>(As + (c >> 2) * LDS_ROW + 16 * (c & 3)) = a[i];
        }
        if (!B_KN) {
#pragma unroll
            for (int i = 0; i < B_PER_T; ++i) {
                const int c = tid + i * kThreads;
                if (c < B_CHUNKS) *reinterpret_cast<i32x4*>(Bs + (c >> 2) * LDS_ROW + 16 * (c & 3)) = b[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < BU_PER_T; ++i) {
                const int u = tid + i * kThreads;
                if (u >= B_UNITS) continue;
                const int o = u % (BN / 8), q = u / (BN / 8);
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    uint32_t r[4], t[4];
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) r[rr] = bu[i][rr][d];
                    transpose4x4(r, t);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        *reinterpret_cast<uint32_t*>(Bs + (8 * o + 4 * d + j) * LDS_ROW + 4 * q) = t[j];
                }
            }
        }
    }
};

template <int BM, int BN, bool B_KN>
__global__ __launch_bounds__(kThreads) void qmm_tiled(QmmArgs p) {
    constexpr int WM = BM / 2, WN = BN / 2;    // wave tile
    constexpr int TM = WM / 16, TN = WN / 16;  // MFMA tiles per wave
    __shared__ __attribute__((aligned(16))) int8_t As[BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) int8_t Bs[BN * LDS_ROW];

    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15;       // fragment row / column
    const int fk = (lane >> 4) * 16;  // fragment k offset (bytes)

    i32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (i32x4){0, 0, 0, 0};

    TileLoader<BM, BN, B_KN> ld;
    ld.load(p, m0, n0, 0);
    for (int64_t k0 = 0; k0 < p.K; k0 += BK) {
        ld.store(As, Bs);
        __syncthreads();
        if (k0 + BK < p.K) ld.load(p, m0, n0, k0 + BK);
        i32x4 af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[i] = *reinterpret_cast<const i32x4*>(As + (wm * WM + 16 * i + fr) * LDS_ROW + fk);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bf[j] = *reinterpret_cast<const i32x4*>(Bs + (wn * WN + 16 * j + fr) * LDS_ROW + fk);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        __syncthreads();
    }

    // D layout of a 16x16 MFMA tile: lane holds column (lane & 15), rows 4*(lane>>4) + r.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * WM + 16 * i + 4 * (lane >> 4) + r;
                const int64_t n = n0 + wn * WN + 16 * j + fr;
                if (m < p.M && n < p.N) qmm_store(p.epi, m, n, acc[i][j][r]);
            }
}

// Any shape / stride / alignment: one thread per output element.
__global__ __launch_bounds__(kThreads) void qmm_generic(QmmArgs p) {
    const int64_t total = p.M * p.N;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t m = idx / p.N, n = idx % p.N;
        const int8_t* a = p.a + m * p.lda;
        const int8_t* b = p.b + n * p.sbn;
        int32_t s = 0;
        for (int64_t k = 0; k < p.K; ++k) s += (int32_t)a[k] * (int32_t)b[k * p.sbk];
        qmm_store(p.epi, m, n, s);
    }
}

template <int BM, int BN, bool B_KN>
hipError_t launch_tiled(const QmmArgs& p, hipStream_t stream) {
    dim3 grid((uint32_t)((p.N + BN - 1) / BN), (uint32_t)((p.M + BM - 1) / BM));
    qmm_tiled<BM, BN, B_KN><<<grid, dim3(kThreads), 0, stream>>>(p);
    return hipGetLastError();
}

template <bool B_KN>
hipError_t launch_by_m(const QmmArgs& p, hipStream_t stream) {
    if (p.M <= 32) return launch_tiled<32, 128, B_KN>(p, stream);
    if (p.M <= 64) return launch_tiled<64, 128, B_KN>(p, stream);
    return launch_tiled<128, 128, B_KN>(p, stream);
}

}  // namespace

size_t quant_matmul_workspace(int64_t, int64_t, int64_t) { return 0; }

hipError_t launch_quant_matmul(const QmmArgs& p, void*, size_t, hipStream_t stream) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    const bool a_ok = (p.K % 16 == 0) && (p.lda % 16 == 0) && ((uintptr_t)p.a % 16 == 0);
    const bool b_nk = (p.sbk == 1) && (p.sbn % 16 == 0) && ((uintptr_t)p.b % 16 == 0);
    const bool b_kn = (p.sbn == 1) && (p.sbk % 8 == 0) && (p.N % 8 == 0) && ((uintptr_t)p.b % 8 == 0);
    if (p.K > 0 && a_ok && b_kn) return launch_by_m<true>(p, stream);
    if (p.K > 0 && a_ok && b_nk) return launch_by_m<false>(p, stream);
    const int64_t total = p.M * p.N;
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    qmm_generic<<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(p);
    return hipGetLastError();
}

}  // namespace qk
