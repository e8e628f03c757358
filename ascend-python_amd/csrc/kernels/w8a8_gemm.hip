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
#include <climits>

#include "common.h"

namespace qk {
namespace {

constexpr int kThreads = 256;
constexpr int BK = 64;        // K bytes per step == K of one i8 MFMA
constexpr int LDS_ROW = 80;   // padded row stride (bytes) of the LDS tiles

// Weight layouts of the direct-to-LDS kernels: the transposed view of an [N,K] tensor, a [K,N] tensor, and
// the int8 NZ layout [N/16][K/64][64][16] (1 KB blocks of 16 columns x 64 rows, lane l of a block holding
// rows 16(l/16)..+15 of column l%16: one v_mfma_i32_16x16x64_i8 B operand per block).
constexpr int kLayNK = 0, kLayKN = 1, kLayNZ = 2;
constexpr int kOutSwiGLU = 64;  // qmm_dma's OUT for the fused gate-up + SwiGLU form (+ the output dtype)

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

// ---------------------------------------------------------------------------
// Prefill kernel: 256x256 output tile per 256-thread workgroup (wave tile
// 128x128 = 8x8 MFMA tiles, 256 int32 accumulators per lane), K in 64-byte
// steps, two LDS stages (64 KB) so one barrier per step, next step's global
// loads in flight during the current step's MFMAs.
//
// LDS layouts (16-byte chunks XOR-swizzled so fragment reads and tile writes
// are bank-conflict free):
//   A and [N,K] B : [row][64 k-bytes], chunk c of row r at r*64 + 16*(c ^ ((r>>2)&3))
//   [K,N] B       : [k][256 n-bytes],  chunk c of row k at k*256 + 16*(c ^ h(k)),
//                   h(k) = (k&7) | ((k>>4)&1)<<3
// A [K,N] weight is kept in its natural layout and the MFMA B fragment (16
// consecutive k of one column per lane) is read with two ds_read_b64_tr_b8:
// in each 16-lane group, lane i receives byte (i&7) of the 8-byte rows
// addressed by lanes 2b + (i>>3), b = 0..7 -- so lanes 2b / 2b+1 address row
// k0+b at columns 0..7 / 8..15 of the tile and every lane gets its column's
// 8 consecutive k bytes per read.
// Workgroups are renumbered so each XCD (ids congruent mod 8) owns a compact
// block of output tiles (8 tile-rows x 8 tile-cols share its L2).
namespace big {
constexpr int BM = 256, BN = 256, BK = 128;  // BK: K bytes per LDS stage (two MFMA k-steps)
constexpr int A_BYTES = BM * BK;
constexpr int CPR = BK / 16;                  // 16-byte chunks per [row][k] row

// [row][k] tiles (A, [N,K] weight): 128-byte rows, chunk c XOR-swizzled by
// (r>>1)&7 so 16 consecutive rows at one chunk cover all banks.
__device__ __forceinline__ int rk_off(int r, int c) { return r * BK + 16 * (c ^ ((r >> 1) & 7)); }
// [k][n] tiles ([K,N] weight): 256-byte rows padded to 272 B plus 128 B per
// 16-row block, so the 8 rows one 16-lane group of a transpose read touches
// fall in distinct banks and the next group (16 rows on) in the other half;
// the column offset stays a compile-time constant for the reads.
__device__ __forceinline__ int kn_off(int k, int c16) { return k * 272 + 128 * (k >> 4) + 16 * c16; }
constexpr int KN_BYTES = 127 * 272 + 128 * 7 + 256 + 144;  // kn_off(127, 16) rounded up to 256
constexpr int B_BYTES = KN_BYTES > BN * BK ? KN_BYTES : BN * BK;
constexpr int STAGE = A_BYTES + B_BYTES;

typedef int32_t v2i __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2i lds_tr8(const int8_t* p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(p));
}

// One output element from preloaded per-column / per-row operands; the same
// float operations, in the same order, as qmm_store (bi = 0 / bf = +0 / pt = 1
// when the op has no int32 bias / float bias / per-token scale).
template <int OUT>
__device__ __forceinline__ void store_elem(void* out, int64_t o, int32_t acc, float s, float bf, int32_t bi, float pt,
                                           float off) {
    acc = (int32_t)((uint32_t)acc + (uint32_t)bi);
    if constexpr (OUT == QK_I32) {
        ((int32_t*)out)[o] = acc;
    } else if constexpr (OUT == QK_I8) {
        float t = __builtin_rintf(__builtin_fmaf((float)acc, s, off));
        t = fminf(fmaxf(t, -128.0f), 127.0f);
        ((int8_t*)out)[o] = (int8_t)(int)t;
    } else {
        const float v = __builtin_fmaf((float)acc * pt, s, bf);
        if constexpr (OUT == QK_BF16) ((uint16_t*)out)[o] = (uint16_t)f32_to_bf16_bits(v);
        else if constexpr (OUT == QK_F16) ((uint16_t*)out)[o] = (uint16_t)f32_to_f16_bits(v);
        else ((float*)out)[o] = v;
    }
}
}  // namespace big

// The epilogue's per-column (scale, offset, bias) and per-row (per-token
// scale) operands of one lane: columns n0 + wn*128 + 16j + (lane&15), rows
// m0 + wm*16*TM + 16i + 4(lane>>4) + r.  bias holds the int32 bias, or the
// fp32 bits of a float bias (0 = +0.0f when there is none).  Loaded apart from
// the epilogue so a kernel can issue the loads long before the tile ends.
template <int TM>
struct EpiOps {
    float sc[8], of[8];
    uint32_t bias[8];
    float pt[TM][4];
};

// SWI (the gate-up GEMM with SwiGLU fused): wave column half wn = 0 holds the gate columns n0 .., wn = 1 the up
// columns n_up .., of the same outputs.
template <int TM, bool SWI = false>
__device__ __forceinline__ void load_epi_ops(const QmmArgs& p, EpiOps<TM>& o, int64_t m0, int64_t n0, int wm,
                                             int wn, int lane, int64_t n_up = 0) {
    const QmmEpilogue& e = p.epi;
    const int fr = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int64_t n = (SWI ? (wn == 0 ? n0 : n_up) : n0 + wn * 128) + 16 * j + fr;
        const bool ok = n < p.N;
        o.sc[j] = (ok && e.scale) ? e.scale[e.scale_per_ch ? n : 0] : 0.0f;
        o.of[j] = (ok && e.offset) ? e.offset[e.offset_per_ch ? n : 0] : 0.0f;
        o.bias[j] = 0u;
        if (ok && e.bias_dtype == QK_I32) o.bias[j] = (uint32_t)((const int32_t*)e.bias)[n];
        else if (ok && e.bias_dtype) o.bias[j] = __builtin_bit_cast(uint32_t, load_scalar(e.bias, n, e.bias_dtype));
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = m0 + wm * 16 * TM + 16 * i + 4 * g + r;
            o.pt[i][r] = (e.pertoken && m < p.M) ? e.pertoken[m] : 1.0f;  // multiplying by 1.0 is exact
        }
}

// The end of a 256x256 tile: exact int32 partials of a K split (FULL only), or
// the fused epilogue; FULL 16-bit tiles are staged through LDS (smem must
// hold BM x (2*BN + 16) bytes) so the global stores are 16-byte and
// row-contiguous.  acc[i][j] holds rows wm*WMR + 16i + 4(lane>>4) + r, column
// wn*128 + 16j + (lane&15) of the tile (the MFMA 16x16 output layout).
template <int OUT, int TM, int NT, bool FULL>
__device__ __forceinline__ void big_epilogue(const QmmArgs& p, const i32x4 (&acc)[TM][8], const EpiOps<TM>& ops,
                                             int8_t* smem, int64_t m0, int64_t n0, int wm, int wn, int lane, int tid,
                                             int split, int nsplit, int32_t* __restrict__ partial) {
    using namespace big;
    constexpr int WMR = 16 * TM;
    const int fr = lane & 15, g = lane >> 4;
    if (FULL && nsplit > 1) {  // exact int32 partial sums of this K range
        int32_t* dst = partial + (int64_t)split * p.M * p.N;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * WMR + 16 * i + 4 * g + r;
                if (m >= p.M) continue;  // the last row tile of a ragged M
                const int64_t ro = m * p.N + n0 + wn * 128 + fr;
#pragma unroll
                for (int j = 0; j < 8; ++j) dst[ro + 16 * j] = acc[i][j][r];
            }
        return;
    }

    // ---- epilogue
    const QmmEpilogue& e = p.epi;
    const bool ibias = e.bias_dtype == QK_I32;
    const float* sc = ops.sc;
    const float* of = ops.of;
    float bf[8];
    int32_t bi[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        bi[j] = ibias ? (int32_t)ops.bias[j] : 0;
        bf[j] = ibias ? 0.0f : __builtin_bit_cast(float, ops.bias[j]);
    }
    if constexpr (FULL && (OUT == QK_BF16 || OUT == QK_F16)) {
        // 16-bit outputs of a full tile are staged through LDS (the operand
        // stages are free now) so the global stores are whole 512-byte rows of
        // 16 bytes per lane instead of 32-byte pieces of 4 rows.
        constexpr int ROWB = 2 * BN + 16;  // padded LDS row (bytes)
        __syncthreads();
        uint16_t* ot = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = wm * WMR + 16 * i + 4 * g + r;
                const float pt = ops.pt[i][r];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int32_t a = (int32_t)((uint32_t)acc[i][j][r] + (uint32_t)bi[j]);
                    const float v = __builtin_fmaf((float)a * pt, sc[j], bf[j]);
                    ot[row * (ROWB / 2) + wn * 128 + 16 * j + fr] =
                        (uint16_t)(OUT == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
                }
            }
        }
        __syncthreads();
        constexpr int CPRO = 2 * BN / 16;  // 16-byte chunks per output row
        constexpr int TR = 4 * WMR;        // tile rows (four wave rows)
        static_assert(TR * CPRO % NT == 0, "whole chunks per thread");
#pragma unroll
        for (int it = 0; it < TR * CPRO / NT; ++it) {
            const int q = tid + it * NT;
            const int row = q / CPRO, c = q % CPRO;
            if (m0 + row >= p.M) break;  // rows past a ragged M (q grows with the row)
            const i32x4 v = *reinterpret_cast<const i32x4*>(smem + row * ROWB + 16 * c);
            // written once and not read again here: non-temporal, past the operand lines in the L2
            __builtin_nontemporal_store(v, reinterpret_cast<i32x4*>(static_cast<uint16_t*>(e.out) + (m0 + row) * e.ldo +
                                                                    n0 + 8 * c));
        }
        return;
    }
    // Fully unrolled with compile-time register indices (a runtime-indexed
    // accumulator would be demoted to scratch and spilled every K step).
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = m0 + wm * WMR + 16 * i + 4 * g + r;
            const bool row_ok = m < p.M;
            const float pt = ops.pt[i][r];
            const int64_t ro = m * e.ldo + n0 + wn * 128 + fr;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool ok = row_ok && (n0 + wn * 128 + 16 * j + fr) < p.N;
                if (ok) big::store_elem<OUT>(e.out, ro + 16 * j, acc[i][j][r], sc[j], bf[j], bi[j], pt, of[j]);
            }
        }
    }
}

// The gate-up GEMM's fused SwiGLU epilogue (256 x 256 tiles whose column halves are the gate and the up columns of
// 128 outputs): each half is rounded to the output type exactly as big_epilogue rounds it and staged through
// LDS; then each thread takes 8 outputs of one row (16 bytes of gate, 16 of up) and stores
// h = silu(gate) * up rounded to the same type -- the values the SwiGLU kernel computes from the gate-up
// output in HBM.  h has ldo = N / 2 columns; rows past M are not stored.  With amax (not null) the tile also
// stores, per row, the largest |h| of its 128 outputs (fmaxf from +0, so NaN outputs are passed over, as the
// dynamic quantizer's absmax passes them over) at amax[row * (I / 128) + tn]: the column tiles' partial absmax,
// from which the row scale of npu_dynamic_quant(h) follows without a reduction over h.
template <int ODT, int TM, int NT>
__device__ __forceinline__ void swiglu_epilogue(const QmmArgs& p, const i32x4 (&acc)[TM][8], const EpiOps<TM>& ops,
                                                int8_t* smem, int64_t m0, int64_t n0, int wm, int wn, int lane,
                                                int tid, float* __restrict__ amax, int tn) {
    using namespace big;
    constexpr int WMR = 16 * TM;
    constexpr int ROWB = 2 * BN + 16;  // padded LDS row (bytes): gate columns, then up columns
    const int fr = lane & 15, g = lane >> 4;
    const QmmEpilogue& e = p.epi;
    auto to16 = [](float v) { return ODT == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v); };
    __syncthreads();
    uint16_t* ot = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = wm * WMR + 16 * i + 4 * g + r;
            const float pt = ops.pt[i][r];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = __builtin_fmaf((float)acc[i][j][r] * pt, ops.sc[j], 0.0f);  // no bias: + 0
                ot[row * (ROWB / 2) + wn * 128 + 16 * j + fr] = (uint16_t)to16(v);
            }
        }
    }
    __syncthreads();
    constexpr int CH = BN / 16;  // 16-byte chunks of an h row (128 outputs): lanes 16k .. 16k+15 hold one row
    static_assert(BM * CH % NT == 0 && NT % CH == 0 && CH == 16, "whole rows per 16-lane group");
#pragma unroll
    for (int it = 0; it < BM * CH / NT; ++it) {
        const int q = tid + it * NT;
        const int row = q / CH, c = q % CH;
        const bool in = m0 + row < p.M;  // rows past a ragged M are computed, not stored
        const u32x4 gv = *reinterpret_cast<const u32x4*>(smem + row * ROWB + 16 * c);
        const u32x4 uv = *reinterpret_cast<const u32x4*>(smem + row * ROWB + BN + 16 * c);
        u32x4 hv;
        float mx = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t lo = to16(silu_mul(load_half_bits(gv[w] & 0xffffu, ODT), load_half_bits(uv[w] & 0xffffu, ODT)));
            const uint32_t hi = to16(silu_mul(load_half_bits(gv[w] >> 16, ODT), load_half_bits(uv[w] >> 16, ODT)));
            hv[w] = lo | (hi << 16);
            mx = fmaxf(mx, fmaxf(load_half_bits(lo & 0x7fffu, ODT), load_half_bits(hi & 0x7fffu, ODT)));
        }
        if (in)
            __builtin_nontemporal_store(hv, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(e.out) + (m0 + row) * e.ldo +
                                                                     n0 + 8 * c));  // written once
        if (amax) {  // the row's 16 lanes (a DPP row; every lane active here): max over the 128 outputs
            mx = row16_max(mx);
            if (in && c == 0) amax[(m0 + row) * (p.N / BN) + tn] = mx;
        }
    }
}

// NW = 4: 2x2 waves of 128x128 (one wave per SIMD); NW = 8: 4x2 waves of
// 64x128 (two waves per SIMD, so one wave's MFMAs cover the other's waits).
// FULL: every tile is inside M, N and K is a multiple of BK, so loads need no
// predicates and use one 32-bit per-lane offset from a uniform base (no 64-bit
// address registers live across the loop).
// nsplit > 1 (FULL only): workgroup bid/tiles takes the K range
// [split * K/nsplit, (split+1) * K/nsplit) and writes its exact int32 sums to
// partial[split][M][N]; qmm_reduce adds the splits and applies the epilogue.
template <bool B_KN, int OUT, int NW, bool FULL>
__global__ __launch_bounds__(64 * NW) void qmm_big(QmmArgs p, int tiles_m, int tiles_n, int nsplit,
                                                   int32_t* __restrict__ partial) {
    using namespace big;
    constexpr int NT = 64 * NW;              // threads
    constexpr int WMR = BM / (NW / 2);       // wave tile rows
    constexpr int TM = WMR / 16;             // MFMA row tiles per wave
    constexpr int NLD = BM * CPR / NT;       // 16-byte loads per thread per operand per stage
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * STAGE];
    static_assert(BM * (2 * BN + 16) <= 2 * STAGE, "output tile does not fit the LDS stages");

    // XCD-aware renumbering + grouped tile order (splits outermost)
    const int tiles = tiles_m * tiles_n;
    const int bid_all = xcd_swizzle(blockIdx.x, tiles * nsplit);
    const int split = bid_all / tiles;
    const int bid = bid_all - split * tiles;
    const int64_t k_len = p.K / nsplit;
    const int64_t k_base = (int64_t)split * k_len;
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const int grp = bid / per_group;
    const int first_m = grp * GM;
    const int gm = min(tiles_m - first_m, GM);
    const int tm = first_m + (bid % per_group) % gm;
    const int tn = (bid % per_group) / gm;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, g = lane >> 4;

    // ---- global -> register prefetch (NLD x 16 B of A and of B per thread)
    i32x4 ra[NLD], rb[NLD];
    // FULL path: lane offsets (rows advance NT/CPR per load; [K,N] rows NT/16)
    const uint32_t a_lane = (uint32_t)(tid / CPR) * (uint32_t)p.lda + 16u * (uint32_t)(tid % CPR);
    const uint32_t b_lane = B_KN ? (uint32_t)(tid >> 4) * (uint32_t)p.sbk + 16u * (uint32_t)(tid & 15)
                                 : (uint32_t)(tid / CPR) * (uint32_t)p.sbn + 16u * (uint32_t)(tid % CPR);
    auto gload = [&](int64_t k0) {
        k0 += k_base;
        if constexpr (FULL) {
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                const int8_t* abase = p.a + (m0 + (int64_t)i * (NT / CPR)) * p.lda + k0;
                ra[i] = *reinterpret_cast<const i32x4*>(abase + a_lane);
                const int8_t* bbase = B_KN ? p.b + (k0 + (int64_t)i * (NT / 16)) * p.sbk + n0
                                           : p.b + (n0 + (int64_t)i * (NT / CPR)) * p.sbn + k0;
                rb[i] = *reinterpret_cast<const i32x4*>(bbase + b_lane);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int q = tid + NT * i;
            const int r = q / CPR, c = q % CPR;
            const int64_t m = m0 + r, k = k0 + 16 * c;
            ra[i] = (m < p.M && k < p.K) ? *reinterpret_cast<const i32x4*>(p.a + m * p.lda + k) : (i32x4){0, 0, 0, 0};
            if (!B_KN) {
                const int64_t n = n0 + r;
                rb[i] = (n < p.N && k < p.K) ? *reinterpret_cast<const i32x4*>(p.b + n * p.sbn + k)
                                             : (i32x4){0, 0, 0, 0};
            } else {
                const int kr = q >> 4, c16 = q & 15;
                const int64_t kk = k0 + kr, n = n0 + 16 * c16;
                rb[i] = (kk < p.K && n < p.N) ? *reinterpret_cast<const i32x4*>(p.b + kk * p.sbk + n)
                                              : (i32x4){0, 0, 0, 0};
            }
        }
    };
    auto lstore = [&](int st) {
        int8_t* As = smem + st * STAGE;
        int8_t* Bs = As + A_BYTES;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int q = tid + NT * i;
            *reinterpret_cast<i32x4*>(As + rk_off(q / CPR, q % CPR)) = ra[i];
            if (!B_KN) *reinterpret_cast<i32x4*>(Bs + rk_off(q / CPR, q % CPR)) = rb[i];
            else *reinterpret_cast<i32x4*>(Bs + kn_off(q >> 4, q & 15)) = rb[i];
        }
    };

    i32x4 acc[TM][8];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = (i32x4){0, 0, 0, 0};

    // per-lane fragment addressing (constant over K)
    // transpose read: lanes 2b / 2b+1 of each 16-lane group address row
    // k0 + b, columns 0..7 / 8..15 of the tile (the +8 rows half is kn_off + 8*272)
    const int tr_k = 16 * g + (fr >> 1);
    const int tr_base = kn_off(tr_k, 0) + 8 * (fr & 1);

    const int64_t nk = (k_len + big::BK - 1) / big::BK;
    gload(0);
    lstore(0);
    if (nk > 1) gload(big::BK);
    for (int64_t it = 0; it < nk; ++it) {
        __syncthreads();
        const int st = (int)(it & 1);
        const int8_t* As = smem + st * STAGE;
        const int8_t* Bs = As + A_BYTES;
        auto frags = [&](int kk, i32x4 (&af)[TM], i32x4 (&bfr)[8]) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const i32x4*>(As + rk_off(wm * WMR + 16 * i + fr, 4 * kk + g));
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (!B_KN) {
                    bfr[j] = *reinterpret_cast<const i32x4*>(Bs + rk_off(wn * 128 + 16 * j + fr, 4 * kk + g));
                } else {
                    // rows 64kk + tr_k (+8): kn_off is affine in k inside a 16-row block
                    const int8_t* t = Bs + tr_base + kn_off(64 * kk, wn * 8 + j);
                    const v2i lo = lds_tr8(t);
                    const v2i hi = lds_tr8(t + 8 * 272);
                    bfr[j] = (i32x4){lo[0], lo[1], hi[0], hi[1]};
                }
            }
        };
        auto mma = [&](const i32x4 (&af)[TM], const i32x4 (&bfr)[8]) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bfr[j], acc[i][j], 0, 0, 0);
        };
        i32x4 af0[TM], bf0[8], af1[TM], bf1[8];
        frags(0, af0, bf0);
        // stage it+1 (already in registers) goes to the other buffer, then fetch it+2
        if constexpr (NW == 4) {  // one wave per SIMD: overlap its own LDS reads
            if (it + 1 < nk) {
                lstore(st ^ 1);
                if (it + 2 < nk) gload((it + 2) * big::BK);
            }
            frags(1, af1, bf1);
            mma(af0, bf0);
            mma(af1, bf1);
        } else {
            // the first half's MFMAs run before the wait on stage it+1's loads,
            // which so get a step and a half to arrive; the SIMD's other wave
            // covers the LDS latency of the second half
            mma(af0, bf0);
            if (it + 1 < nk) {
                lstore(st ^ 1);
                if (it + 2 < nk) gload((it + 2) * big::BK);
            }
            frags(1, af1, bf1);
            mma(af1, bf1);
        }
    }

    EpiOps<TM> ops;
    if (!(FULL && nsplit > 1)) load_epi_ops<TM>(p, ops, m0, n0, wm, wn, lane);
    big_epilogue<OUT, TM, NT, FULL>(p, acc, ops, smem, m0, n0, wm, wn, lane, tid, split, nsplit, partial);
}

// ---------------------------------------------------------------------------
// Prefill kernel with direct global->LDS loads (the aligned shapes whose K
// range is a multiple of 256): the same 256x256 tile and 4x2 waves of 64x128
// as qmm_big, but the operands never pass through registers.  Each
// buffer_load_dwordx4 ... lds writes one wave's 64 x 16 bytes to 1 KB of LDS
// at m0, so the swizzle is applied on the global side: lane l of an
// instruction fetches the chunk that belongs at LDS byte 16*l.  The MFMAs step
// through K 64 bytes at a time.  The weight sits in a ring of four 64-K stages
// (16 KB each); A sits in a ring of three 128-K slots (32 KB each), so every
// A DMA fetches whole 128-byte lines (a 64-K stage of A would fetch each line
// in two halves, at two different times).  The eight waves form two groups
// (rows 0-127 and 128-255 of the tile, one wave of each per SIMD) that run
// half a stage apart: while one group issues its MFMAs the other reads its
// next fragments and issues DMAs (group 0 A, group 1 the weight), with two
// barriers per stage.  vmcnt counts a wave's DMA instructions in order.
//   [row][128 B] A slots:                chunk c of row r at r*128 + 16*(c ^ ((r>>1)&7))
//   [row][64 B] weight stages ([N,K]):   chunk c of row r at r*64 + 16*(c ^ ((r>>1)&3))
//   [k][256 B]  weight stages ([K,N]):   chunk c of row k at k*256 + 16*(c ^ h(k)),
//                                         h(k) = (k&7) | ((k>>4)&1)<<3
//   NZ weight stages:                    the column block's 16 NZ blocks of one K block, 1 KB each, as
//                                         they are (fragment reads of 64 lanes x 16 contiguous bytes)
// All four are free of LDS bank conflicts for the fragment reads (b128 row
// reads; transpose reads for [K,N]; NZ by construction), the first three
// measured with SQ_LDS_BANK_CONFLICT.
namespace dm {
constexpr int BM = 256, BN = 256, BK = 64, NST = 4, NW = 8, NT = 64 * NW;
constexpr int TM = 4;                   // 64-row wave tiles: 4 x 8 MFMA tiles
constexpr int B_ST = BN * BK;           // one weight stage (16 KB)
constexpr int A_KB = 128, NSA = 3;      // A slots: 128 K-bytes each, three of them
constexpr int A_SL = BM * A_KB;         // one A slot (32 KB)
constexpr int A_BASE = NST * B_ST;      // A slots follow the weight stages
constexpr int OUT_BYTES = BM * (2 * BN + 16);
constexpr int RING = NST * B_ST + NSA * A_SL;  // 160 KB: all of the CU's LDS
constexpr int SMEM = RING > OUT_BYTES ? RING : OUT_BYTES;

}  // namespace dm

// BMX = 128 (K splits only): 128-row tiles, so a shape with few 256-row tiles needs half the K splits (and half
// the int32 partials) to fill the CUs.  Waves then own 32 x 128 (two row tiles), an A slot is 16 KB, and each
// split stores its exact sums in the MFMA output layout, one whole KB per store instruction:
// partial[split][tile][wave][TM*8 fragments][64 lanes] x 16 bytes (qmm_reduce_tiled reads it back).
// OUT = kOutSwiGLU + QK_BF16 / QK_F16: the gate-up GEMM with SwiGLU fused (swiglu_epilogue).  The weight has
// N = 2I columns, gate then up; tile tn covers outputs 128 tn .. +127, its B columns the gate columns
// 128 tn .. and the up columns I + 128 tn .. (NZ blocks or [K,N] column chunks addressed apart); no split.
// There `partial`, when not null, receives the tiles' per-row partial absmax of h (fp32 [M][I / 128]).
// rev_from (> 0; the CU count, or INT_MAX for none): workgroups in odd rounds of rev_from walk their K range
// backwards.  A second-round workgroup takes the next column tiles of the same row blocks on its XCD, so it
// starts on the K stages the first round read last, which are still in that XCD's L2.
template <int BL, int OUT, int BMX = 256>
__global__ __launch_bounds__(dm::NT) void qmm_dma(QmmArgs p, int tiles_m, int tiles_n, int nsplit,
                                                  int32_t* __restrict__ partial, int rev_from) {
    using namespace dm;
    constexpr bool B_KN = BL == kLayKN, B_NZ = BL == kLayNZ;
    constexpr bool SWI = OUT >= kOutSwiGLU;
    constexpr int ODT = SWI ? OUT - kOutSwiGLU : OUT;
    static_assert(BMX == 256 || (BMX == 128 && OUT == QK_I32), "128-row tiles run as K splits only");
    static_assert(!SWI || (BMX == 256 && BL != kLayNK && (ODT == QK_BF16 || ODT == QK_F16)), "fused SwiGLU form");
    constexpr int BM = BMX;          // tile rows
    constexpr int TM = BM / 64;      // MFMA row tiles per wave (the wave tile is BM/4 x 128)
    constexpr int A_SL = BM * A_KB;  // one A slot
    constexpr int NA = BM / 64;      // A DMAs per wave per half range
    constexpr int RING = NST * B_ST + NSA * A_SL;
    __shared__ __attribute__((aligned(1024))) int8_t smem[BM == 256 ? SMEM : RING];

    const int tiles = tiles_m * tiles_n;
    const int bid_all = xcd_swizzle(blockIdx.x, tiles * nsplit);
    const int split = bid_all / tiles;
    const int bid = bid_all - split * tiles;
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const int grp = bid / per_group;
    const int first_m = grp * GM;
    const int gm = min(tiles_m - first_m, GM);
    const int tm = first_m + (bid % per_group) % gm;
    const int tn = (bid % per_group) / gm;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * (SWI ? BN / 2 : BN);
    const int64_t n_up = SWI ? p.N / 2 + n0 : 0;  // SWI: the tile's first up column
    const int64_t k_len = p.K / nsplit;
    const uint32_t k_base = (uint32_t)(split * k_len);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int pg = wave >> 2;  // ping-pong group: waves 0-3 own rows 0-127, waves 4-7 rows 128-255
    const int gw = wave & 3;   // wave within its group
    const int fr = lane & 15, g = lane >> 4;

    // buffer views of this tile's operand rows (sizes checked on the host to fit 32 bits)
    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem;
    // A rows past M (the last row tile of a ragged M) fall outside the range and read as zeros: the row offset
    // of every A load is in its voff, which the range check covers
    const int64_t rows_valid = p.M - m0 < BM ? p.M - m0 : BM;
    const __amdgpu_buffer_rsrc_t rsA = make_rsrc(p.a + m0 * p.lda, (uint32_t)(rows_valid * p.lda));
    // an NZ column block: BN/16 consecutive n-blocks of K/64 1 KB blocks, BN * K contiguous bytes
    // SWI: the whole NZ weight (blocks addressed per wave), or the [K,N] rows from the gate columns on, whose
    // chunks 8..15 are moved to the up columns (I - 128 bytes further)
    const __amdgpu_buffer_rsrc_t rsB = B_NZ   ? (SWI ? make_rsrc(p.b, (uint32_t)(p.N * p.K))
                                                     : make_rsrc(p.b + n0 * p.K, (uint32_t)(BN * p.K)))
                                       : B_KN ? make_rsrc(p.b + n0, (uint32_t)((p.K - 1) * p.sbk + (SWI ? p.N / 2 + BN / 2 : BN)))
                                              : make_rsrc(p.b + n0 * p.sbn, (uint32_t)(BN * p.sbn));
    const uint32_t kblocks = (uint32_t)(p.K >> 6);
    const uint32_t lda = (uint32_t)p.lda, ldb = (uint32_t)(B_KN ? p.sbk : p.sbn);
    // A [row][128 B]: one instruction = 8 rows 8b..8b+7; lane l -> row l>>3, LDS chunk l&7, and
    // (r>>1)&7 = 4*(b&1) + (l>>4)
    const uint32_t va0 = (uint32_t)(lane >> 3) * lda + 16u * (uint32_t)((lane & 7) ^ (lane >> 4));
    const uint32_t va1 = (uint32_t)(lane >> 3) * lda + 16u * (uint32_t)((lane & 7) ^ (4 + (lane >> 4)));
    // [N,K] weight [row][64 B]: one instruction = 16 rows; lane l -> row l>>2, LDS chunk l&3
    const uint32_t vrk_b = (uint32_t)(lane >> 2) * ldb + 16u * (uint32_t)((lane & 3) ^ ((lane >> 3) & 3));
    // [k][256 B]: one instruction = 4 rows 4b..4b+3 (b = 4*gw + i); lane l -> row l>>4, LDS chunk l&15, and
    // h = 4*(b&1) + (l>>4) + 8*((b>>2)&1), (b>>2)&1 = gw&1
    const int hb = 8 * (gw & 1);
    auto kn_col = [&](int cc) {  // byte column of chunk cc (SWI: chunks 8..15 are up columns)
        return 16u * (uint32_t)cc + (SWI && cc >= 8 ? (uint32_t)(p.N / 2 - BN / 2) : 0u);
    };
    const uint32_t vkn0 = (uint32_t)(lane >> 4) * ldb + kn_col((lane & 15) ^ ((lane >> 4) + hb));
    const uint32_t vkn1 = (uint32_t)(lane >> 4) * ldb + kn_col((lane & 15) ^ (4 + (lane >> 4) + hb));

    const int nk = (int)(k_len / dm::BK);  // a multiple of NST (checked on the host)
    const int nr = nk / 2;                 // A slots' worth of K
    // every other round of rev_from workgroups (the second, fourth, ...) walks K backwards: int32 sums are
    // exact in any order
    const bool rev = (((int)blockIdx.x / rev_from) & 1) != 0;
    // group 1 issues the weight: stage kt into buffer st, four instructions per wave (a stage past the end
    // fetches the last one again into its free buffer, so every stage issues the same number of DMAs)
    auto issue_b = [&](int kt, int st) {
        const int ks = kt < nk ? kt : nk - 1;
        const uint32_t k0 = k_base + (uint32_t)(rev ? nk - 1 - ks : ks) * dm::BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 4 * gw + i;
            if constexpr (B_NZ) {  // n-block b of the column block, K block k0/64: one contiguous 1 KB block
                const uint32_t nb = SWI ? (uint32_t)(b < 8 ? n0 / 16 + b : n_up / 16 + (b - 8)) : (uint32_t)b;
                dma16(rsB, sbase + st * B_ST + b * 1024, (nb * kblocks + (k0 >> 6)) * 1024u + 16u * lane, 0u);
            }
            else if constexpr (B_KN)
                dma16(rsB, sbase + st * B_ST + b * 1024, (i & 1) ? vkn1 : vkn0, (k0 + 4u * b) * ldb);
            else
                dma16(rsB, sbase + st * B_ST + b * 1024, vrk_b, (uint32_t)(16 * b) * ldb + k0);
        }
    };
    // group 0 issues A: rows 128h..128h+127 of range r (K bytes 128r..128r+127 of this split) into slot
    // r % 3 (past the last range, the last range again)
    auto issue_a = [&](int r, int h) {
        const int rs0 = r < nr ? r : nr - 1;
        const int rs = rev ? nr - 1 - rs0 : rs0;
        const uint32_t lds = sbase + A_BASE + (uint32_t)(r % NSA) * A_SL;
        const uint32_t k0 = k_base + (uint32_t)rs * A_KB;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int b = 4 * NA * h + NA * gw + i;  // rows 8b .. 8b+7 (b & 1 == i & 1)
            dma16(rsA, lds + b * 1024, ((i & 1) ? va1 : va0) + (uint32_t)(8 * b) * lda, k0);
        }
    };

    // fragment read offsets: A for the low / high 64 K-bytes of a slot (slot s adds s * 32 KB); the
    // weight for stage 0 (stage st adds st * 16 KB)
    const int a_rd0 = A_BASE + (wm * (BM / 4) + fr) * A_KB + 16 * (g ^ ((fr >> 1) & 7));
    const int a_rd1 = A_BASE + (wm * (BM / 4) + fr) * A_KB + 16 * ((4 + g) ^ ((fr >> 1) & 7));
    const int b_rd = (wn * 128 + fr) * 64 + 16 * (g ^ ((fr >> 1) & 3));
    // transpose reads: lanes 2b / 2b+1 of each 16-lane group address k row 16g + b (and +8), columns
    // 0..7 / 8..15 of the 16-column tile, whose chunk index is XOR-ed by h(k)
    const int t_rd = (16 * g + (fr >> 1)) * 256 + 128 * (wn ^ (g & 1)) + 8 * (fr & 1);
    const int xr = fr >> 1;

    i32x4 af[TM], bfr[8];
    auto frags = [&](int kt, int st) {
        const int ard = (((kt & 1) != 0) != rev ? a_rd1 : a_rd0) + ((kt >> 1) % NSA) * A_SL;
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const i32x4*>(smem + ard + i * 16 * A_KB);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (B_NZ) {
                bfr[j] = *reinterpret_cast<const i32x4*>(smem + st * B_ST + (8 * wn + j) * 1024 + 16 * lane);
            } else if constexpr (!B_KN) {
                bfr[j] = *reinterpret_cast<const i32x4*>(smem + b_rd + st * B_ST + j * 1024);
            } else {
                const int8_t* t = smem + t_rd + st * B_ST + 16 * (j ^ xr);
                const big::v2i lo = big::lds_tr8(t);
                const big::v2i hi = big::lds_tr8(t + 8 * 256);
                bfr[j] = (i32x4){lo[0], lo[1], hi[0], hi[1]};
            }
        }
    };

    i32x4 acc[TM][8];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = (i32x4){0, 0, 0, 0};
    auto mma = [&]() {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bfr[j], acc[i][j], 0, 0, 0);
    };
    // a barrier nothing is scheduled across (the compiler would otherwise hoist MFMAs above it)
    auto bar = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    };
    constexpr int LGKM0 = 0xc07f;  // s_waitcnt lgkmcnt(0) alone

    // Ping-pong: the two groups run half a stage apart, so while one issues its 32 MFMAs the other reads
    // fragments and issues DMAs, and every SIMD (one wave of each group) always has MFMAs to run.
    //   half-step 2t:   group 0 multiplies stage t;  group 1 reads stage t, issues weight stage t+3
    //   half-step 2t+1: group 0 reads stage t+1, issues half (t+1)&1 of A range (t+5)>>1;  group 1 multiplies t
    // A range R goes out at t = 2R-5 and 2R-4: after its slot's last reader (range R-3, group 1 at half-step
    // 4R-10) and four half-steps before its first reader (group 0 at half-step 4R-1).  Weight stage s goes out
    // at half-step 2s-6, after its buffer's last reader (stage s-4, group 1 at 2s-8).  Each wave issues four
    // DMAs per stage; waiting for all but the last two stages' (vmcnt(8)) before the barrier that ends
    // half-step 2t lands everything stage t+1 needs (its A range went out at loop index t-3 at the latest,
    // its weight at t-2).
    // Both groups pass the same barriers in the same order.
    if (pg == 0) {  // loop indices -5..-1: A ranges 0, 1 and the first half of range 2
        issue_a(0, 0);
        issue_a(0, 1);
        issue_a(1, 0);
        issue_a(1, 1);
        issue_a(2, 0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * NA));  // range 0 (stages 0 and 1)
    } else {        // loop indices -3..-1: weight stages 0..2
        issue_b(0, 0);
        issue_b(1, 1);
        issue_b(2, 2);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));   // stage 0
    }
    bar();
    if (pg == 0) {
        frags(0, 0);
        __builtin_amdgcn_s_waitcnt(LGKM0);
    }
    bar();
    // Some stages before the tile ends, each wave touches the cache lines of its epilogue operands
    // (per-column scale and bias, per-row per-token scale) so the epilogue's loads of them hit the L2.
    // The loaded word is only kept live to the end (no wait inside the loop).
    float warm = 0.0f;
    auto warm_up = [&]() {
        if (nsplit != 1) return;
        const QmmEpilogue& e = p.epi;
        const int64_t n = n0 + 4 * lane, m = m0 + 4 * lane;  // 64 lanes x 16 B: 256 columns or rows
        if (wave == 0 && e.scale && e.scale_per_ch) warm = e.scale[n];
        else if (wave == 1 && e.pertoken && m < p.M) warm = e.pertoken[m];
        else if (wave == 2 && e.bias_dtype) {
            const int es = (e.bias_dtype == QK_F32 || e.bias_dtype == QK_I32) ? 4 : 2;
            if (16 * lane < 256 * es) warm = *(const float*)((const char*)e.bias + n0 * es + 16 * lane);
        }
    };
    if (pg == 0) {
        for (int t0 = 0; t0 < nk; t0 += NST) {
            if (t0 == nk - NST) warm_up();
#pragma unroll
            for (int u = 0; u < NST; ++u) {
                const int t = t0 + u;
                mma();
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NA));
                bar();
                if (t + 1 < nk) frags(t + 1, (u + 1) & 3);
                issue_a((t + 5) >> 1, (t + 1) & 1);
                __builtin_amdgcn_s_waitcnt(LGKM0);
                bar();
            }
        }
    } else {
        for (int t0 = 0; t0 < nk; t0 += NST) {
#pragma unroll
            for (int u = 0; u < NST; ++u) {
                const int t = t0 + u;
                frags(t, u);
                issue_b(t + 3, (u + 3) & 3);
                __builtin_amdgcn_s_waitcnt(LGKM0);
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
                bar();
                mma();
                bar();
            }
        }
    }
    // the trailing DMAs (past the last stage) land before the LDS is reused or released
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    asm volatile("" ::"v"(warm));
    if constexpr (BM == 128) {  // the split's exact sums in the MFMA layout, one KB per store, read once
        i32x4* dst = reinterpret_cast<i32x4*>(partial) + (((int64_t)split * tiles + bid) * 8 + wave) * (TM * 8 * 64) + lane;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) __builtin_nontemporal_store(acc[i][j], dst + (i * 8 + j) * 64);
    } else if constexpr (SWI) {
        EpiOps<TM> ops;
        load_epi_ops<TM, true>(p, ops, m0, n0, wm, wn, lane, n_up);
        swiglu_epilogue<ODT, TM, NT>(p, acc, ops, smem, m0, n0, wm, wn, lane, tid, reinterpret_cast<float*>(partial),
                                     tn);
    } else {
        EpiOps<TM> ops;
        if (nsplit == 1) load_epi_ops<TM>(p, ops, m0, n0, wm, wn, lane);
        big_epilogue<OUT, TM, NT, true>(p, acc, ops, smem, m0, n0, wm, wn, lane, tid, split, nsplit, partial);
    }
}

// ---------------------------------------------------------------------------
// Skinny kernel (decode and small M <= 128): an HBM weight stream.  A workgroup owns
// 16*MT rows x 256 columns and one K split; its 4 waves take 64 columns
// each.  Stages of 128 k-rows go through LDS (the weight in its natural
// layout, B fragments by ds_read_b64_tr_b8 for [K,N]) with the next PF
// stages' global loads in flight in registers.  With several splits each writes exact int32
// partial sums and qmm_reduce adds them (order-free, exact) before the same
// epilogue as every other path.
namespace sk {
constexpr int BN = 256, BK = 128;
}

template <bool B_KN, int MT, bool FINAL, int PF = 1>
__global__ __launch_bounds__(kThreads) void qmm_skinny(QmmArgs p, int tiles_n, int nsplit, int32_t* partial) {
    using big::rk_off;
    using big::kn_off;
    constexpr int BM = 16 * MT;
    constexpr int A_BYTES = BM * sk::BK, B_BYTES = big::B_BYTES, STAGE = A_BYTES + B_BYTES;
    constexpr int A_CHUNKS = BM * 8;                 // 16-byte chunks per stage
    constexpr int A_PER_T = (A_CHUNKS + kThreads - 1) / kThreads;
    constexpr int B_PER_T = sk::BN * 8 / kThreads;   // 8
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * STAGE];

    const int blk = blockIdx.x;
    const int tn = blk % tiles_n;
    const int split = (blk / tiles_n) % nsplit;
    const int tm = blk / (tiles_n * nsplit);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * sk::BN;
    const int64_t ks = p.K / nsplit, kbeg = (int64_t)split * ks;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15, g = lane >> 4;

    // PF register slots: stage s is loaded into slot s % PF, PF stages ahead of the one in LDS
    i32x4 ra[PF][A_PER_T], rb[PF][B_PER_T];
    auto gload = [&](int64_t k0, int sl) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int q = tid + kThreads * i;
            const int r = q >> 3, c = q & 7;
            const int64_t m = m0 + r;
            ra[sl][i] = (q < A_CHUNKS && m < p.M) ? *reinterpret_cast<const i32x4*>(p.a + m * p.lda + k0 + 16 * c)
                                                  : (i32x4){0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            const int q = tid + kThreads * i;
            // one row tile (M <= 16) reads each weight byte once: non-temporal, so the weight streams past
            // the L2 instead of evicting the x rows that every workgroup reads again
            auto wload = [](const int8_t* src) {
                const i32x4* v = reinterpret_cast<const i32x4*>(src);
                if constexpr (MT == 1) return __builtin_nontemporal_load(v);
                else return *v;
            };
            if (!B_KN) {
                const int r = q >> 3, c = q & 7;
                const int64_t n = n0 + r;
                rb[sl][i] = n < p.N ? wload(p.b + n * p.sbn + k0 + 16 * c) : (i32x4){0, 0, 0, 0};
            } else {
                const int kr = q >> 4, c16 = q & 15;
                const int64_t n = n0 + 16 * c16;
                rb[sl][i] = n < p.N ? wload(p.b + (k0 + kr) * p.sbk + n) : (i32x4){0, 0, 0, 0};
            }
        }
    };
    auto lstore = [&](int st, int sl) {
        int8_t* As = smem + st * STAGE;
        int8_t* Bs = As + A_BYTES;
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int q = tid + kThreads * i;
            if (q < A_CHUNKS) *reinterpret_cast<i32x4*>(As + rk_off(q >> 3, q & 7)) = ra[sl][i];
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            const int q = tid + kThreads * i;
            if (!B_KN) *reinterpret_cast<i32x4*>(Bs + rk_off(q >> 3, q & 7)) = rb[sl][i];
            else *reinterpret_cast<i32x4*>(Bs + kn_off(q >> 4, q & 15)) = rb[sl][i];
        }
    };

    i32x4 acc[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (i32x4){0, 0, 0, 0};
    const int tr_base = kn_off(16 * g + (fr >> 1), 0) + 8 * (fr & 1);

    const int64_t nk = ks / sk::BK;
    gload(kbeg, 0);
    lstore(0, 0);
#pragma unroll
    for (int u = 1; u <= PF; ++u)
        if (u < nk) gload(kbeg + u * sk::BK, u % PF);
    for (int64_t it0 = 0; it0 < nk; it0 += PF)
#pragma unroll
    for (int u = 0; u < PF; ++u) {  // it0 is a multiple of PF, so stage it + 1 sits in slot (u + 1) % PF
        const int64_t it = it0 + u;
        if (it >= nk) break;
        __syncthreads();
        const int st = (int)(it & 1);
        const int8_t* As = smem + st * STAGE;
        const int8_t* Bs = As + A_BYTES;
        i32x4 af[2][MT], bf[2][4];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int i = 0; i < MT; ++i) af[kk][i] = *reinterpret_cast<const i32x4*>(As + rk_off(16 * i + fr, 4 * kk + g));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (!B_KN) {
                    bf[kk][j] = *reinterpret_cast<const i32x4*>(Bs + rk_off(64 * wave + 16 * j + fr, 4 * kk + g));
                } else {
                    const int8_t* t = Bs + tr_base + kn_off(64 * kk, 4 * wave + j);
                    const big::v2i lo = big::lds_tr8(t);
                    const big::v2i hi = big::lds_tr8(t + 8 * 272);
                    bf[kk][j] = (i32x4){lo[0], lo[1], hi[0], hi[1]};
                }
            }
        }
        if (it + 1 < nk) {
            lstore(st ^ 1, (u + 1) % PF);
            if (it + 1 + PF < nk) gload(kbeg + (it + 1 + PF) * sk::BK, (u + 1) % PF);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[kk][i], bf[kk][j], acc[i][j], 0, 0, 0);
    }

#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + 16 * i + 4 * g + r;
                const int64_t n = n0 + 64 * wave + 16 * j + fr;
                if (m >= p.M || n >= p.N) continue;
                if (FINAL) qmm_store(p.epi, m, n, acc[i][j][r]);
                else partial[((int64_t)split * p.M + m) * p.N + n] = acc[i][j][r];
            }
}

// ---------------------------------------------------------------------------
// Mid-M kernel (M <= 256, every K in one workgroup, no split partials):
// a BM x BN output tile per workgroup of NW waves (BM = 16, 32 or 64; BN = 64,
// or 128 for a [K,N] weight so each of its k rows is one whole 128-byte line),
// so a few thousand output columns already give hundreds of workgroups.  K
// goes in stages of 256 bytes through a ring of NST LDS stages filled by
// direct global->LDS loads (buffer_load_dwordx4 ... lds), NST-1 stages in
// flight; every wave issues a share of each stage's 1 KB load instructions
// (a CU's fill rate from L2 grows with the number of waves issuing them).
// Wave w multiplies K bytes 64(w%4)..64(w%4)+63 of every stage for column
// group w/4 (BN/(NW/4) columns) into its own accumulators, and the four K
// partials of each column group are added (exact int32) through LDS before
// the epilogue.  Rows past M read as zeros (buffer range checks) and are not
// stored.
//   A stage [BM rows][256 B]:      chunk c of row r at r*256 + 16*(c ^ (r & 15))
//   [N,K] weight [BN n][256 B]:    as A
//   [K,N] weight [256 k][BN B]:    chunk c of row k at k*BN + 16*(c ^ h(k)),
//       BN = 64:  h(k) = ((k>>2)&1) | ((k>>4)&1)<<1
//       BN = 128: h(k) = ((k>>1)&3) | ((k>>4)&1)<<2
//   NZ weight [BN/16 n-blocks][4 K blocks][1 KB]: the weight's own 1 KB
//       blocks, copied as they are (16 columns x 64 rows; lane l's 16 bytes
//       are rows 16(l/16)..+15 of column l%16, its MFMA B operand)
// so the 16 rows of a fragment read (A, [N,K]) and the 16 k rows that two
// 16-lane groups of one ds_read_b64_tr_b8 address ([K,N]) fall in distinct
// banks, and an NZ fragment read is 64 lanes x 16 contiguous bytes.
namespace md {
constexpr int KS = 256;
template <int BM, int BN, int NW, int RES>
struct Cfg {  // RES: LDS bytes kept apart from the ring
    static constexpr int NT = 64 * NW;
    static constexpr int A_BYTES = BM * KS;
    static constexpr int B_BYTES = BN * KS;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int NST = ((160 * 1024 - RES) / STAGE) > 8 ? 8 : ((160 * 1024 - RES) / STAGE);
    static constexpr int A_DMA = BM / 4;              // 1 KB DMA instructions per stage (4 rows of A each)
    static constexpr int DMA = A_DMA + BN / 4;        // + the weight's
    static constexpr int PW_LO = DMA / NW;            // instructions per wave per stage: waves below
    static constexpr int PW_HI = PW_LO + 1;           // DMA % NW issue PW_HI, the others PW_LO
    static constexpr int NG = NW / 4;                 // column groups
    static constexpr int NTJ = BN / 16 / NG;          // MFMA column tiles per wave
    static constexpr int RED_ROW = BN + 4;            // int32 reduction rows, padded
    static constexpr int RED_BYTES = 4 * BM * RED_ROW * 4;
    static_assert(NW % 4 == 0 && NTJ >= 1 && NTJ * 16 * NG == BN, "waves cover the columns");
    static_assert(NST >= 3, "at least two stages in flight");
    static_assert(RED_BYTES <= NST * STAGE, "the reduction fits the ring");
};
template <int BN>
__device__ __forceinline__ int hkn(int k) {
    if constexpr (BN == 64) return ((k >> 2) & 1) | (((k >> 4) & 1) << 1);
    else return ((k >> 1) & 3) | (((k >> 4) & 1) << 2);
}
}  // namespace md

// 8 consecutive outputs of one row: the same float operations, in the same order, as qmm_store.
template <int OUT>
__device__ __forceinline__ void store8(const QmmEpilogue& e, int64_t m, int64_t n, const uint32_t (&s)[8]) {
    float pt = 1.0f;
    if (e.pertoken) pt = e.pertoken[m];
    uint32_t q[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int64_t c = n + t;
        int32_t acc = (int32_t)s[t];
        float bf = 0.0f;
        if (e.bias_dtype == QK_I32) acc = (int32_t)((uint32_t)acc + (uint32_t)((const int32_t*)e.bias)[c]);
        else if (e.bias_dtype) bf = load_scalar(e.bias, c, e.bias_dtype);
        const float sc = e.scale ? e.scale[e.scale_per_ch ? c : 0] : 0.0f;
        if constexpr (OUT == QK_I32) {
            q[t] = (uint32_t)acc;
        } else if constexpr (OUT == QK_I8) {
            const float off = e.offset ? e.offset[e.offset_per_ch ? c : 0] : 0.0f;
            float v = __builtin_rintf(__builtin_fmaf((float)acc, sc, off));
            v = fminf(fmaxf(v, -128.0f), 127.0f);
            q[t] = (uint32_t)(uint8_t)(int8_t)(int)v;
        } else {
            const float v = __builtin_fmaf((float)acc * pt, sc, bf);
            if constexpr (OUT == QK_BF16) q[t] = f32_to_bf16_bits(v);
            else if constexpr (OUT == QK_F16) q[t] = f32_to_f16_bits(v);
            else q[t] = __builtin_bit_cast(uint32_t, v);
        }
    }
    const int64_t o = m * e.ldo + n;
    if constexpr (OUT == QK_BF16 || OUT == QK_F16) {
        *reinterpret_cast<i32x4*>(static_cast<uint16_t*>(e.out) + o) =
            (i32x4){(int32_t)(q[0] | q[1] << 16), (int32_t)(q[2] | q[3] << 16), (int32_t)(q[4] | q[5] << 16),
                    (int32_t)(q[6] | q[7] << 16)};
    } else if constexpr (OUT == QK_I8) {
        *reinterpret_cast<u32x2*>(static_cast<int8_t*>(e.out) + o) =
            (u32x2){q[0] | q[1] << 8 | q[2] << 16 | q[3] << 24, q[4] | q[5] << 8 | q[6] << 16 | q[7] << 24};
    } else {
        i32x4* d = reinterpret_cast<i32x4*>(static_cast<int32_t*>(e.out) + o);
        d[0] = (i32x4){(int32_t)q[0], (int32_t)q[1], (int32_t)q[2], (int32_t)q[3]};
        d[1] = (i32x4){(int32_t)q[4], (int32_t)q[5], (int32_t)q[6], (int32_t)q[7]};
    }
}

// SPLIT: the grid holds nsplit workgroups per tile, each over K / nsplit; each stores its exact int32 tile
// sums device-coherently to partial[tile][split], and the last to arrive (splitk_last) adds the splits in
// split order and applies the epilogue.
template <int BL, int BM, int BN, int NW, int PD, int OUT, bool SPLIT>
__global__ __launch_bounds__(64 * NW + (PD > 0 ? 64 : 0)) void qmm_mid(QmmArgs p, int tiles_m, int nsplit,
                                                                     int32_t* __restrict__ partial,
                                                                     uint64_t* __restrict__ ctr, uint64_t tag) {
    constexpr bool B_KN = BL == kLayKN, B_NZ = BL == kLayNZ;
    static_assert(!B_NZ || PD == 0, "NZ blocks stream as whole lines without the prefetch wave");
    constexpr int SCRATCH = PD > 0 ? 1024 : 0;  // the prefetch wave's landing block
    using C = md::Cfg<BM, BN, NW, SCRATCH>;
    constexpr int NST = C::NST, TMI = BM / 16, NTJ = C::NTJ, NT = C::NT;
    static_assert(NST * C::STAGE + SCRATCH <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) int8_t smem[NST * C::STAGE + SCRATCH];

    // logical id: consecutive ids (one XCD) share a column block, so the weight's lines are fetched once
    // per XCD; the splits of a tile, then the row blocks of a column block, run side by side
    const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int split = SPLIT ? bid % nsplit : 0;
    const int tile = SPLIT ? bid / nsplit : bid;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int rows = (int)((p.M - m0) < BM ? (p.M - m0) : BM);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kq = wave & 3, cg = wave >> 2;  // K quarter of each stage, column group
    const int fr = lane & 15, g = lane >> 4;

    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem;
    const uint32_t lda = (uint32_t)p.lda, ldb = (uint32_t)(B_KN ? p.sbk : p.sbn);
    const __amdgpu_buffer_rsrc_t rsA = make_rsrc(p.a + m0 * p.lda, (uint32_t)((rows - 1) * p.lda + p.K));
    // an NZ column block is BN/16 consecutive n-blocks of K/64 blocks each: BN * K contiguous bytes
    const __amdgpu_buffer_rsrc_t rsB = B_NZ   ? make_rsrc(p.b + n0 * p.K, (uint32_t)(BN * p.K))
                                       : B_KN ? make_rsrc(p.b + n0, (uint32_t)((p.K - 1) * p.sbk + BN))
                                              : make_rsrc(p.b + n0 * p.sbn, (uint32_t)((BN - 1) * p.sbn + p.K));
    const uint32_t kblocks = (uint32_t)(p.K >> 6);  // NZ: 1 KB blocks per n-block
    // NZ DMA: instruction b copies block (n-block b/4 of the column block, K block 4*stage + b%4); the whole
    // offset goes in voff
    auto voff_nz = [&](int b, uint32_t k0) {
        return ((uint32_t)(b >> 2) * kblocks + (k0 >> 6) + (uint32_t)(b & 3)) * 1024u + 16u * (uint32_t)lane;
    };
    // [row][256 B] DMA (A, [N,K] weight): an instruction covers rows 4b..4b+3; lane l -> row 4b + (l>>4),
    // LDS chunk l&15, global chunk (l&15) ^ (row&15)
    auto voff_rk = [&](int b, uint32_t ld) {
        const int row = 4 * b + (lane >> 4);
        return (uint32_t)row * ld + 16u * (uint32_t)((lane & 15) ^ (row & 15));
    };
    // [k][BN B] DMA ([K,N] weight): an instruction covers 1024/BN k rows; lane l -> row b*(1024/BN) + l/(BN/16),
    // LDS chunk l%(BN/16), global chunk (l%(BN/16)) ^ h(row)
    auto voff_kn = [&](int b) {
        constexpr int CPR = BN / 16;
        const int row = b * (1024 / BN) + lane / CPR;
        return (uint32_t)row * ldb + 16u * (uint32_t)((lane % CPR) ^ md::hkn<BN>(row));
    };
    const int nk = (int)(p.K / md::KS / (SPLIT ? nsplit : 1));  // stages of this workgroup's K range
    const uint32_t kbeg = (uint32_t)(split * nk * md::KS);
    const bool hi = wave < C::DMA % NW;  // this wave issues PW_HI instructions per stage
    auto issue = [&](int s) {  // stage s into buffer s % NST: instructions wave, wave+NW, ...
        const uint32_t lds = sbase + (uint32_t)(s % NST) * C::STAGE;
        const uint32_t k0 = kbeg + (uint32_t)s * md::KS;
#pragma unroll
        for (int u = 0; u < C::PW_HI; ++u) {
            const int q = wave + NW * u;
            if (q >= C::DMA) break;
            if (q < C::A_DMA) {
                dma16(rsA, lds + q * 1024, voff_rk(q, lda), k0);
            } else {
                const int b = q - C::A_DMA;
                if constexpr (B_NZ) dma16(rsB, lds + C::A_BYTES + b * 1024, voff_nz(b, k0), 0u);
                else if constexpr (B_KN) dma16(rsB, lds + C::A_BYTES + b * 1024, voff_kn(b), k0 * ldb);
                else dma16(rsB, lds + C::A_BYTES + b * 1024, voff_rk(b, ldb), k0);
            }
        }
    };

    i32x4 acc[TMI][NTJ];
#pragma unroll
    for (int i = 0; i < TMI; ++i)
#pragma unroll
        for (int j = 0; j < NTJ; ++j) acc[i][j] = (i32x4){0, 0, 0, 0};

    const int ck = 4 * kq + g;  // this lane's 16-byte K chunk of a stage row
    // PD > 0: wave NW only runs ahead of the ring, loading stage s + PD of this workgroup's rows of A
    // and its share (1 / tiles_m) of the weight block into one scratch KB of LDS nobody reads, so the
    // ring's own loads of those lines later hit the L2.  It waits on nothing but its own loads at the end.
    // The A rows are prefetched only by the workgroups of the first column block an XCD runs (the first
    // tiles_m logical ids of each XCD's range), the weight block's rows split over its tiles_m row blocks.  The lead pd keeps the wave's outstanding loads under the 63 vmcnt can count,
    // so it never stalls at an issue while the other waves wait for it at a barrier.
    const bool pf_wave = PD > 0 && wave == NW;
    const int per_xcd = (int)(gridDim.x >> 3);
    const bool pf_a = per_xcd > 0 && (bid % per_xcd) < tiles_m;
    const int pf_cnt = (pf_a ? C::A_DMA : 0) + (BN / 4 + tiles_m - 1) / tiles_m;
    const int pd = min(PD, 56 / pf_cnt);
    auto prefetch = [&](int s) {
        const uint32_t lds = sbase + (uint32_t)(NST * C::STAGE);
        const uint32_t k0 = kbeg + (uint32_t)s * md::KS;
        if (pf_a)
            for (int q = 0; q < C::A_DMA; ++q) dma16(rsA, lds, voff_rk(q, lda), k0);
        for (int b = tm; b < BN / 4; b += tiles_m) {
            if constexpr (B_KN) dma16(rsB, lds, voff_kn(b), k0 * ldb);
            else dma16(rsB, lds, voff_rk(b, ldb), k0);
        }
    };
    if (pf_wave) {
        for (int s = NST - 1; s < NST - 1 + pd && s < nk; ++s) prefetch(s);
    } else {
        for (int s = 0; s < NST - 1 && s < nk; ++s) issue(s);
    }
    for (int s = 0; s < nk; ++s) {
        // stage s has landed once at most the later stages' instructions are outstanding
        if (pf_wave) {
        } else if (s + NST - 2 < nk) {
            if (hi) __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * C::PW_HI));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm((NST - 2) * C::PW_LO));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // stage s visible to every wave; every wave is done with stage s-1
        __builtin_amdgcn_sched_barrier(0);
        if (pf_wave) {
            if (s + NST - 1 + pd < nk) prefetch(s + NST - 1 + pd);
            continue;
        }
        if (s + NST - 1 < nk) issue(s + NST - 1);  // into the buffer of stage s-1
        const int8_t* As = smem + (s % NST) * C::STAGE;
        const int8_t* Bs = As + C::A_BYTES;
        i32x4 af[TMI], bf[NTJ];
#pragma unroll
        for (int i = 0; i < TMI; ++i) {
            const int r = 16 * i + fr;
            af[i] = *reinterpret_cast<const i32x4*>(As + r * md::KS + 16 * (ck ^ (r & 15)));
        }
#pragma unroll
        for (int jj = 0; jj < NTJ; ++jj) {
            const int j = cg * NTJ + jj;  // column tile of the block
            if constexpr (B_NZ) {
                bf[jj] = *reinterpret_cast<const i32x4*>(Bs + (4 * j + kq) * 1024 + 16 * lane);
            } else if constexpr (!B_KN) {
                const int r = 16 * j + fr;
                bf[jj] = *reinterpret_cast<const i32x4*>(Bs + r * md::KS + 16 * (ck ^ (r & 15)));
            } else {
                // lanes 2b / 2b+1 of each 16-lane group address k row 64kq + 16g + b (and +8), columns
                // 16j..16j+7 / 16j+8..16j+15
                const int k = 64 * kq + 16 * g + (fr >> 1);
                const big::v2i lo = big::lds_tr8(Bs + k * BN + 16 * (j ^ md::hkn<BN>(k)) + 8 * (fr & 1));
                const big::v2i hi8 = big::lds_tr8(Bs + (k + 8) * BN + 16 * (j ^ md::hkn<BN>(k + 8)) + 8 * (fr & 1));
                bf[jj] = (i32x4){lo[0], lo[1], hi8[0], hi8[1]};
            }
        }
#pragma unroll
        for (int i = 0; i < TMI; ++i)
#pragma unroll
            for (int jj = 0; jj < NTJ; ++jj)
                acc[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[jj], acc[i][jj], 0, 0, 0);
    }

    // the four K partials of each column group -> LDS (the ring is free once every wave is past its
    // last reads)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    int32_t* red = reinterpret_cast<int32_t*>(smem);
    if (!pf_wave) {
#pragma unroll
        for (int i = 0; i < TMI; ++i)
#pragma unroll
            for (int jj = 0; jj < NTJ; ++jj)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    red[(kq * BM + 16 * i + 4 * g + r) * C::RED_ROW + 16 * (cg * NTJ + jj) + fr] = acc[i][jj][r];
    }
    __syncthreads();
    // thread tid finishes 8 consecutive outputs of one row (tiles have at most 8 * NT outputs): the exact
    // int32 sum of the four K partials, then (this split's share of) the epilogue
    static_assert(BM * BN / 8 <= NT, "one group of 8 outputs per thread");
    const int row = tid / (BN / 8), c8 = 8 * (tid % (BN / 8));
    const bool has = !pf_wave && tid < BM * BN / 8 && row < rows;
    uint32_t s8[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) s8[t] = 0u;
    if (has) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int32_t* src = red + (w * BM + row) * C::RED_ROW + c8;
            const i32x4 a = *reinterpret_cast<const i32x4*>(src);
            const i32x4 b = *reinterpret_cast<const i32x4*>(src + 4);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s8[t] += (uint32_t)a[t];
                s8[4 + t] += (uint32_t)b[t];
            }
        }
    }
    if constexpr (!SPLIT) {
        if (has) store8<OUT>(p.epi, m0 + row, n0 + c8, s8);
    } else {
        // partial[tile][split][BM][BN], written through the L2 (device-coherent) and read back by the last split
        const __amdgpu_buffer_rsrc_t prs =
            make_rsrc(partial, (uint32_t)((int64_t)gridDim.x * BM * BN * 4));
        const uint32_t own_off = (uint32_t)((((int64_t)tile * nsplit + split) * BM + row) * BN + c8) * 4u;
        if (has) {
            __builtin_amdgcn_raw_buffer_store_b128((u32x4){s8[0], s8[1], s8[2], s8[3]}, prs, own_off, 0, kCoherent);
            __builtin_amdgcn_raw_buffer_store_b128((u32x4){s8[4], s8[5], s8[6], s8[7]}, prs, own_off + 16u, 0,
                                                   kCoherent);
        }
        if (!splitk_last(ctr + tile, (uint32_t)nsplit, tag)) return;
        if (has) {
            uint32_t t8[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) t8[t] = 0u;
            for (int sp = 0; sp < nsplit; ++sp) {  // in split order (integer sums: any order is exact)
                u32x4 lo, hi;
                if (sp == split) {
                    lo = (u32x4){s8[0], s8[1], s8[2], s8[3]};
                    hi = (u32x4){s8[4], s8[5], s8[6], s8[7]};
                } else {
                    const uint32_t off = (uint32_t)((((int64_t)tile * nsplit + sp) * BM + row) * BN + c8) * 4u;
                    lo = __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kCoherent);
                    hi = __builtin_amdgcn_raw_buffer_load_b128(prs, off + 16u, 0, kCoherent);
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    t8[t] += lo[t];
                    t8[4 + t] += hi[t];
                }
            }
            store8<OUT>(p.epi, m0 + row, n0 + c8, t8);
        }
    }
}

// ---------------------------------------------------------------------------
// Decode on an int8 NZ weight (M <= 16): an HBM weight stream with no split
// partials.  Workgroup wg owns n-blocks [b0, b1) (16 columns each, NB at most)
// over all of K; wave w takes K blocks (64 rows) w, w + NW, w + 2NW, ... of
// all of them.  Per K block a lane loads 16 bytes of x (lane (m, g): x[m,
// 64kb + 16g .. +16], the A operand of v_mfma_i32_16x16x64_i8) and 16 bytes of
// each of the NB weight blocks (its B operand as stored), PF K blocks ahead.
// Loads past a wave's last K block are given an out-of-range buffer offset,
// so they return zeros without touching memory and the loop needs no tail.
// The waves' exact int32 sums are added through LDS, and each thread applies
// the epilogue to 8 consecutive outputs of one row.  Rows past M load row
// M-1 and are not stored.
namespace nzd {
// measured at M=16, K=8192, N=28672: 2 to 5 K blocks in flight, 4 to 16 waves and direct-to-LDS loads in place of
// register loads all stream 5.0-5.3 TB/s; two blocks in flight were the fastest by a few percent
constexpr int NW = 8, NT = 64 * NW, PF = 2, NBMAX = 8;
constexpr int PITCH = 320;  // int32 per 16x16 tile: row r at 16*(r + r/4), so a wave's stores hit 64 banks
constexpr uint32_t kOff = 0x80000000u;  // an offset past every buffer range
}  // namespace nzd

template <int NB>
__global__ __launch_bounds__(nzd::NT) void qmm_nzd(QmmArgs p, int nwg) {
    using namespace nzd;
    __shared__ __attribute__((aligned(16))) int32_t red[NW][NB][PITCH];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int wg = blockIdx.x;
    const int M = (int)p.M;
    const int64_t NBT = p.N >> 4;
    const uint32_t KB = (uint32_t)(p.K >> 6);
    const int b0 = (int)((int64_t)wg * NBT / nwg), nb = (int)((int64_t)(wg + 1) * NBT / nwg) - b0;
    const int m = c < M ? c : M - 1;

    // 31-bit ranges by the C ABI's limits (M <= 16, ldx1 < 2^24, K <= 131071): (M-1)*lda + K and NB*K*16
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.a, (uint32_t)((M - 1) * p.lda + p.K));
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.b + (int64_t)b0 * p.K * 16, (uint32_t)(nb * p.K * 16));
    const uint32_t x_lane = (uint32_t)m * (uint32_t)p.lda + 16u * (uint32_t)g, w_lane = 16u * (uint32_t)lane;
    uint32_t blk[NB];  // a workgroup with fewer blocks repeats its last one (not stored)
#pragma unroll
    for (int b = 0; b < NB; ++b) blk[b] = (uint32_t)(b < nb ? b : nb - 1) * KB * 1024u;

    const int nkb = KB > (uint32_t)wave ? (int)((KB - 1 - (uint32_t)wave) / NW) + 1 : 0;
    i32x4 xa[PF], wv[PF][NB];
    auto issue = [&](int it, int sl) {
        const uint32_t kb = (uint32_t)(wave + it * NW);
        const bool in = it < nkb;
        __builtin_amdgcn_sched_barrier(0);
        xa[sl] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, in ? x_lane + 64u * kb : kOff, 0, 0));
#pragma unroll
        for (int b = 0; b < NB; ++b)
            wv[sl][b] = __builtin_bit_cast(
                i32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, in ? blk[b] + kb * 1024u + w_lane : kOff, 0,
                                                             kNonTemporal));
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int u = 0; u < PF; ++u) issue(u, u);

    i32x4 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = (i32x4){0, 0, 0, 0};
    for (int it0 = 0; it0 < nkb; it0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {  // slot u holds K block it0 + u (zeros past the wave's last one)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[u], wv[u][b], acc[b], 0, 0, 0);
            issue(it0 + u + PF, u);
        }
    }
    // the (zero) loads issued past the end land before the wave leaves
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

    // lane (c, g) holds rows 4g..4g+3 of column c of each block
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][b][16 * (5 * g + r) + c] = acc[b][r];
    __syncthreads();

    // thread t < 32*NB: block t/32, row (t/2)%16, columns 8*(t%2)..+7; exact int32 sums over the waves
    const int t = threadIdx.x;
    if (t >= 32 * NB) return;
    const int b = t >> 5, row = (t >> 1) & 15, c8 = 8 * (t & 1);
    if (b >= nb || row >= M) return;
    const int at = 16 * (row + (row >> 2)) + c8;
    uint32_t s8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s8[e] = 0u;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const i32x4 lo = *reinterpret_cast<const i32x4*>(&red[w][b][at]);
        const i32x4 hi = *reinterpret_cast<const i32x4*>(&red[w][b][at + 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s8[e] += (uint32_t)lo[e];
            s8[4 + e] += (uint32_t)hi[e];
        }
    }
    const int64_t n = ((int64_t)b0 + b) * 16 + c8;
    switch (p.epi.out_dtype) {
    case QK_BF16: store8<QK_BF16>(p.epi, row, n, s8); break;
    case QK_F16: store8<QK_F16>(p.epi, row, n, s8); break;
    case QK_F32: store8<QK_F32>(p.epi, row, n, s8); break;
    case QK_I8: store8<QK_I8>(p.epi, row, n, s8); break;
    default: store8<QK_I32>(p.epi, row, n, s8); break;
    }
}

// Exact int32 sum of the split partials, then the common epilogue.
__global__ __launch_bounds__(kThreads) void qmm_reduce(QmmArgs p, int nsplit, const int32_t* __restrict__ partial) {
    const int64_t total = p.M * p.N;
    if (p.N % 4 == 0) {  // 4 outputs of one row per thread, every split's 16-byte load in flight together
        const int64_t total4 = total >> 2;
        const i32x4* src = reinterpret_cast<const i32x4*>(partial);
        for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total4;
             idx += (int64_t)gridDim.x * kThreads) {
            i32x4 part[16];
            const int ns = nsplit < 16 ? nsplit : 16;
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (k < ns) part[k] = __builtin_nontemporal_load(src + (int64_t)k * total4 + idx);  // read once
            uint32_t s[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (k < ns)
#pragma unroll
                    for (int t = 0; t < 4; ++t) s[t] += (uint32_t)part[k][t];
            for (int k = 16; k < nsplit; ++k) {
                const i32x4 v = src[(int64_t)k * total4 + idx];
#pragma unroll
                for (int t = 0; t < 4; ++t) s[t] += (uint32_t)v[t];
            }
            const int64_t o = idx * 4, m = o / p.N, n = o % p.N;
            const QmmEpilogue& e = p.epi;
            if (e.out_dtype == QK_BF16 || e.out_dtype == QK_F16) {
                // qmm_store's operations for 4 columns of one row, one 8-byte store
                const float pt = e.pertoken ? e.pertoken[m] : 1.0f;
                uint32_t h[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    int32_t acc = (int32_t)s[t];
                    float bf = 0.0f;
                    if (e.bias_dtype == QK_I32) acc = (int32_t)((uint32_t)acc + (uint32_t)((const int32_t*)e.bias)[n + t]);
                    else if (e.bias_dtype) bf = load_scalar(e.bias, n + t, e.bias_dtype);
                    float v = (float)acc;
                    if (e.pertoken) v = v * pt;
                    v = __builtin_fmaf(v, e.scale[e.scale_per_ch ? n + t : 0], bf);
                    h[t] = e.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
                }
                uint16_t* dst = static_cast<uint16_t*>(e.out) + m * e.ldo + n;
                if (((uintptr_t)dst & 7) == 0)
                    *reinterpret_cast<u32x2*>(dst) = (u32x2){h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
                else
#pragma unroll
                    for (int t = 0; t < 4; ++t) dst[t] = (uint16_t)h[t];
                continue;
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) qmm_store(p.epi, m, n + t, (int32_t)s[t]);
        }
        return;
    }
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        uint32_t s = 0;
        for (int k = 0; k < nsplit; ++k) s += (uint32_t)partial[(int64_t)k * total + idx];
        qmm_store(p.epi, idx / p.N, idx % p.N, (int32_t)s);
    }
}

// The splits of qmm_dma<.., 128> (partial[split][tile][wave][16 fragments][64 lanes] x int32x4): one thread per
// 16-byte piece of a tile -- rows 4g..4g+3 of one column of one 16 x 16 fragment -- adds the NS splits' pieces in
// split order and applies qmm_store's operations to its four outputs.  All of a thread's loads (the column's
// scale and bias bits, the four rows' per-token scales, every split's piece) go out before the first use, in
// straight-line code: with qmm_store's per-element loads and a run-time split count, the compiler waited on
// each load in turn and the kernel took 33 us for 36 MB.  Rows past M (a ragged last row tile) are not stored.
template <int NS>
__global__ __launch_bounds__(kThreads) void qmm_reduce_tiled(QmmArgs p, int tiles_m, int tiles_n,
                                                             const i32x4* __restrict__ partial) {
    constexpr int BM = 128, TM = 2, PIECES = 8 * TM * 8 * 64;  // pieces per tile
    const int64_t per_split = (int64_t)tiles_m * tiles_n * PIECES;
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const QmmEpilogue& e = p.epi;
    const bool half = e.out_dtype == QK_BF16 || e.out_dtype == QK_F16;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < per_split;
         idx += (int64_t)gridDim.x * kThreads) {
        const int lane = (int)(idx & 63), f = (int)((idx >> 6) % (TM * 8)), wave = (int)((idx / (64 * TM * 8)) & 7);
        const int bid = (int)(idx / PIECES);
        const int grp = bid / per_group, first_m = grp * GM;
        const int gm = min(tiles_m - first_m, GM);
        const int tm = first_m + (bid % per_group) % gm, tn = (bid % per_group) / gm;
        const int64_t m = (int64_t)tm * BM + (wave >> 1) * (BM / 4) + 16 * (f >> 3) + 4 * (lane >> 4);
        const int64_t n = (int64_t)tn * 256 + (wave & 1) * 128 + 16 * (f & 7) + (lane & 15);
        if (!half) {
            uint32_t s[4] = {0u, 0u, 0u, 0u};
            for (int k = 0; k < NS; ++k) {
                const i32x4 v = partial[(int64_t)k * per_split + idx];
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] += (uint32_t)v[r];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (m + r < p.M) qmm_store(e, m + r, n, (int32_t)s[r]);
            continue;
        }
        // branch-free loads (a branch between two loads made the compiler wait on the first): an absent bias
        // or per-token scale reads the scale array's first word instead, and the value is not used
        const float sc = e.scale[e.scale_per_ch ? n : 0];
        const bool b4 = e.bias_dtype == QK_I32 || e.bias_dtype == QK_F32;
        const uint16_t* bp = e.bias_dtype ? reinterpret_cast<const uint16_t*>(e.bias) + (b4 ? 2 * n : n)
                                          : reinterpret_cast<const uint16_t*>(e.scale);
        const uint32_t blo = bp[0], bhi = bp[b4 ? 1 : 0];
        const float* ptp = e.pertoken ? e.pertoken : e.scale;
        float pt[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pt[r] = ptp[e.pertoken ? (m + r < p.M ? m + r : p.M - 1) : 0];
        i32x4 part[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) part[k] = __builtin_nontemporal_load(partial + (int64_t)k * per_split + idx);
        uint32_t s[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < NS; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] += (uint32_t)part[k][r];
        const uint32_t braw = b4 ? (blo | (bhi << 16)) : blo;
        const uint32_t bi = e.bias_dtype == QK_I32 ? braw : 0u;
        const float bf = e.bias_dtype == QK_F32    ? __uint_as_float(braw)
                         : e.bias_dtype == QK_F16  ? f16_bits_to_f32((uint16_t)braw)
                         : e.bias_dtype == QK_BF16 ? bf16_bits_to_f32((uint16_t)braw)
                                                   : 0.0f;
        uint16_t* dst = static_cast<uint16_t*>(e.out) + m * e.ldo + n;
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // qmm_store's operations, in its order
            float v = (float)(int32_t)(s[r] + bi);
            if (e.pertoken) v = v * pt[r];
            v = __builtin_fmaf(v, sc, bf);
            const uint32_t h = e.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
            if (m + r < p.M) dst[r * e.ldo] = (uint16_t)h;
        }
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

// Whole 256-column tiles and K ranges, 32-bit per-lane offsets (the 64-bit bases stay uniform) and 16-byte
// aligned output rows: what the 256x256 kernels need along N and K.
bool big_nk_full(const QmmArgs& p, int nsplit) {
    return p.N % big::BN == 0 && p.K % (big::BK * nsplit) == 0 && p.lda < (1 << 24) && p.sbk < (1 << 24) &&
           p.sbn < (1 << 24) && (uintptr_t)p.epi.out % 16 == 0 && p.epi.ldo % 8 == 0;
}

// The direct-to-LDS kernel (any M: a ragged last row tile reads zeros past M and stores only its rows): K
// ranges of whole 4-stage rings, 16-byte aligned rows, and every operand range of a tile addressable by a
// 32-bit buffer offset.
bool big_dma_ok(const QmmArgs& p, bool b_kn, int nsplit) {
    return plan_override().qmm_dma && big_nk_full(p, nsplit) && (p.K / nsplit) % (dm::BK * dm::NST) == 0 &&
           p.lda % 16 == 0 && (uintptr_t)p.a % 16 == 0 && (uintptr_t)p.b % 16 == 0 &&
           (b_kn ? (p.sbk % 16 == 0 && (uint64_t)p.K * (uint64_t)p.sbk < (1ull << 32)) : (p.sbn % 16 == 0));
}

// qmm_dma's round length for walking K backwards in every other round: one workgroup per CU (INT_MAX: never)
int dma_rev_from() {
    const int cus = plan_override().qmm_rev ? device_cus() : 0;
    return cus > 0 ? cus : INT_MAX;
}

template <int OUT>
hipError_t launch_big(const QmmArgs& p, bool b_kn, int tiles_m, int tiles_n, int nsplit, int32_t* partial,
                      hipStream_t stream) {
    const dim3 grid((uint32_t)(tiles_m * tiles_n * nsplit));
    const bool full = big_nk_full(p, nsplit) && p.M % big::BM == 0;  // the register-staged kernel's whole tiles
    const bool dma = big_dma_ok(p, b_kn, nsplit);
    if (nsplit > 1 && !full && !dma) return hipErrorInvalidValue;  // not planned (launch_quant_matmul unsplits)
    if (dma) {
        if (b_kn) qmm_dma<kLayKN, OUT><<<grid, dim3(dm::NT), 0, stream>>>(p, tiles_m, tiles_n, nsplit, partial, dma_rev_from());
        else qmm_dma<kLayNK, OUT><<<grid, dim3(dm::NT), 0, stream>>>(p, tiles_m, tiles_n, nsplit, partial, dma_rev_from());
    } else if (full) {
        if (b_kn) qmm_big<true, OUT, 8, true><<<grid, dim3(512), 0, stream>>>(p, tiles_m, tiles_n, nsplit, partial);
        else qmm_big<false, OUT, 8, true><<<grid, dim3(512), 0, stream>>>(p, tiles_m, tiles_n, nsplit, partial);
    } else {
        if (b_kn) qmm_big<true, OUT, 8, false><<<grid, dim3(512), 0, stream>>>(p, tiles_m, tiles_n, 1, partial);
        else qmm_big<false, OUT, 8, false><<<grid, dim3(512), 0, stream>>>(p, tiles_m, tiles_n, 1, partial);
    }
    return hipGetLastError();
}

// 256x256 tiles: enough of them (192 fill three quarters of the CUs) run as
// they are; fewer whole tiles get a power-of-two K split (K/nsplit a multiple
// of 128 and at least 512) until about 192 workgroups run, when the int32
// partials stay within 512 MB.  From sizes only, so the workspace query and
// the launch agree.
// bm = 128: the split runs on 128-row tiles of the direct-to-LDS kernel (qmm_dma<.., 128>, tiled partials and
// qmm_reduce_tiled), chosen where it needs fewer splits than 256-row tiles: half the partial bytes written and
// read again (cfg5's down projection, 512 x 4096 x 14336: 4 splits of 64 tiles instead of 8 of 32; measured
// 34.3 + ~8 us against 36.7 + 15.5 us).
struct BigPlan {
    bool ok = false;
    int tiles_m = 0, tiles_n = 0, nsplit = 1;
    int bm = 256;
};

// the power-of-two K split that brings `tiles` to about 192 workgroups (each split at least 512 deep)
int big_splits(int64_t tiles, int64_t K) {
    int ns = 1;
    while (tiles * ns < 192 && ns < 16 && K % ((int64_t)ns * 2 * big::BK) == 0 && K / (ns * 2) >= 512) ns *= 2;
    return ns;
}

BigPlan big_plan(int64_t M, int64_t N, int64_t K, bool allow128 = true) {
    BigPlan b;
    const int64_t tm = (M + big::BM - 1) / big::BM, tn = (N + big::BN - 1) / big::BN;
    if (K <= 0 || tm * tn >= (1 << 30)) return b;
    b.tiles_m = (int)tm;
    b.tiles_n = (int)tn;
    if (tm * tn >= 192) {
        b.ok = true;
        return b;
    }
    // a split needs whole tiles along N and K; a ragged M only runs split on the direct-to-LDS kernel
    if (N % big::BN != 0 || K % big::BK != 0) return b;
    const int ns = big_splits(tm * tn, K);
    if (ns == 1 || tm * tn * ns < 64 || (int64_t)ns * M * N * 4 > ((int64_t)512 << 20)) return b;
    b.nsplit = ns;
    b.ok = true;
    // 128-row tiles run only as K splits (their kernel writes int32 partials): where the 128-row tiles alone
    // already fill the CUs (ns2 == 1) the 256-row split stays
    const int64_t tm2 = (M + 127) / 128;
    const int ns2 = big_splits(tm2 * tn, K);
    if (allow128 && plan_override().qmm_bm128 && ns2 > 1 && ns2 < ns && tm2 * tn * ns2 >= 64 &&
        K % ((int64_t)ns2 * dm::BK * dm::NST) == 0) {
        b.bm = 128;
        b.tiles_m = (int)tm2;
        b.nsplit = ns2;
    }
    return b;
}

// [split-K counters][partials]: int32 [nsplit][M][N], or for 128-row tiles [nsplit][tiles][128 x 256]
size_t big_split_workspace(const BigPlan& b, int64_t M, int64_t N) {
    const size_t rows = b.bm == 128 ? (size_t)b.tiles_m * 128 : (size_t)M;
    return QK_SPLIT_COUNTER_BYTES + (size_t)b.nsplit * rows * (size_t)N * sizeof(int32_t);
}

template <int BL>
hipError_t launch_split128(const QmmArgs& p, const BigPlan& b, int32_t* partial, hipStream_t stream) {
    const dim3 sgrid((uint32_t)((int64_t)b.tiles_m * b.tiles_n * b.nsplit)), sblock(dm::NT);
    qmm_dma<BL, QK_I32, 128><<<sgrid, sblock, 0, stream>>>(p, b.tiles_m, b.tiles_n, b.nsplit, partial, dma_rev_from());
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    int64_t blocks = ((int64_t)b.tiles_m * b.tiles_n * 8 * 16 * 64 + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    const dim3 grid((uint32_t)blocks), block(kThreads);
    const i32x4* part = reinterpret_cast<const i32x4*>(partial);
    switch (b.nsplit) {  // big_plan's 128-row splits: 2, 4 or 8
    case 2: qmm_reduce_tiled<2><<<grid, block, 0, stream>>>(p, b.tiles_m, b.tiles_n, part); break;
    case 4: qmm_reduce_tiled<4><<<grid, block, 0, stream>>>(p, b.tiles_m, b.tiles_n, part); break;
    case 8: qmm_reduce_tiled<8><<<grid, block, 0, stream>>>(p, b.tiles_m, b.tiles_n, part); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

namespace {

struct SkinnyPlan {
    int mt = 0, nsplit = 1, tiles_n = 0, tiles_m = 0, pf = 1;
};

// Decode and small-M shapes (M <= 128, K a multiple of 128): row tiles of
// 16/32/64/128, and K splits so about 512 workgroups stream the weight.
// Shared by the workspace query and the launch.
SkinnyPlan skinny_plan(int64_t M, int64_t N, int64_t K) {
    SkinnyPlan s;
    if (M <= 0 || M > 128 || K <= 0 || K % sk::BK != 0 || N <= 0) return s;
    s.mt = M <= 16 ? 1 : (M <= 32 ? 2 : (M <= 64 ? 4 : 8));
    s.tiles_m = (int)((M + 16 * s.mt - 1) / (16 * s.mt));
    s.tiles_n = (int)((N + sk::BN - 1) / sk::BN);
    const int64_t base = (int64_t)s.tiles_m * s.tiles_n;
    // split while short of ~512 workgroups (~256, one per CU, for 16-row tiles: the decode stream
    // measured fastest there), keeping the int32 partials (nsplit*M*N*4 bytes) within the weight's K*N
    // bytes and every split at least 256 rows of K
    const int64_t target = s.mt == 1 ? 256 : 512;
    auto fits = [&](int64_t ns) {
        return K % (ns * sk::BK) == 0 && ns * M * 4 <= K && K / ns >= 256;
    };
    while (base * s.nsplit * 2 <= target && fits((int64_t)s.nsplit * 2)) s.nsplit *= 2;
    // debug override: a power of two within the same bounds as the planned count
    if (const int v = plan_override().skinny_splits) {
        if (v == 1 || fits(v)) s.nsplit = v;
    }
    // stages loaded ahead in registers: two for 16-row tiles (the decode stream: cfg2 M=1/16 42.6-45.1 ->
    // 41.4-43.6 us, N = 11008, K = 4096: 15.8-16.8 -> 15.0-15.9 us; three measured slower), one for taller
    // tiles (M = 32: 17.1 -> 20.7 us with two)
    s.pf = s.mt == 1 ? 2 : 1;
    if (const int v = plan_override().skinny_pf) s.pf = v;
    if (base * s.nsplit >= ((int64_t)1 << 31)) s.mt = 0;
    if (s.mt == 8 && s.nsplit == 1) s.mt = 0;  // 128-row tiles only as a split stream (their in-place epilogue is not unrolled)
    return s;
}

template <bool B_KN, int MT>
hipError_t launch_skinny_t(const QmmArgs& p, const SkinnyPlan& s, int32_t* partial, hipStream_t stream) {
    const dim3 grid((uint32_t)((int64_t)s.tiles_m * s.tiles_n * s.nsplit));
    if (s.nsplit == 1) {
        // 128-row tiles run only as a split stream (skinny_plan), so that instance is not built
        if constexpr (MT == 8) return hipErrorInvalidValue;
        else {
            const auto k = s.pf == 3 ? qmm_skinny<B_KN, MT, true, 3>
                           : s.pf == 2 ? qmm_skinny<B_KN, MT, true, 2> : qmm_skinny<B_KN, MT, true, 1>;
            k<<<grid, dim3(kThreads), 0, stream>>>(p, s.tiles_n, 1, nullptr);
            return hipGetLastError();
        }
    }
    const auto k = s.pf == 3 ? qmm_skinny<B_KN, MT, false, 3>
                   : s.pf == 2 ? qmm_skinny<B_KN, MT, false, 2> : qmm_skinny<B_KN, MT, false, 1>;
    k<<<grid, dim3(kThreads), 0, stream>>>(p, s.tiles_n, s.nsplit, partial);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // qmm_reduce takes 4 outputs per thread where N % 4 == 0 (grid-stride loops either way)
    int64_t blocks = ((p.N % 4 == 0 ? p.M * p.N / 4 : p.M * p.N) + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    qmm_reduce<<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(p, s.nsplit, partial);
    return hipGetLastError();
}

template <bool B_KN>
hipError_t launch_skinny(const QmmArgs& p, const SkinnyPlan& s, int32_t* partial, hipStream_t stream) {
    switch (s.mt) {
    case 1: return launch_skinny_t<B_KN, 1>(p, s, partial, stream);
    case 2: return launch_skinny_t<B_KN, 2>(p, s, partial, stream);
    case 4: return launch_skinny_t<B_KN, 4>(p, s, partial, stream);
    default: return launch_skinny_t<B_KN, 8>(p, s, partial, stream);
    }
}

}  // namespace

// Mid-M shapes (M <= 128, or M <= 256 with N <= 8192 -- beyond that the 256x256 tiles move fewer bytes
// per CU; N % 64 == 0, K % 256 == 0): qmm_mid, no workspace.  Column blocks of 128 for a [K,N]
// weight whose N allows it (whole-line k rows), else 64; the row block (64, 32 or 16; 32 at most with
// 128 columns) that moves the fewest operand bytes per CU.  A [K,N] weight with M <= 32 keeps the split
// stream (measured faster there), so for M <= 32 the workspace query still reports the split stream's
// workspace, which a [N,K] weight's qmm_mid launch leaves unused.  With 128 columns the plan may split K
// in two (each split finishing through device-coherent int32 partials and a tagged counter per tile, the
// last split applying the epilogue) when that moves fewer bytes per CU; the workspace query reports that
// [K,N] plan's workspace for every mid shape, and a launch given less runs unsplit.  Eligibility from
// sizes only, so the workspace query and the launch agree.
struct MidPlan {
    int bm = 0, bn = 0, tiles_m = 0, tiles = 0, nsplit = 1;
};


MidPlan mid_plan(int64_t M, int64_t N, int64_t K, bool b_kn) {
    MidPlan m;
    if (!plan_override().qmm_mid) return m;  // debug override: the split stream / tiled kernels instead
    if (M <= 0 || M > 256 || (M > 128 && N > 8192) || N <= 0 || N % 64 != 0 || K <= 0 || K % md::KS != 0)
        return m;
    const PlanOverride& ov = plan_override();  // debug override: a row block, column block and / or split
    const int bn = (b_kn && N % 128 == 0 && ov.mid_bn != 64) ? 128 : 64;
    const int64_t tn = N / bn;
    if (tn * ((M + 15) / 16) >= ((int64_t)1 << 30)) return m;
    // the row block (and, with 128 columns, K split) with the fewest bytes per CU: rounds of workgroups over
    // the 256 CUs times each workgroup's (BM + BN) * K / nsplit operand bytes, plus a split's partial tile
    // written and read (ties to the larger block, then to no split)
    int bm = 16, ns = 1;
    int64_t best = -1;
    for (int c : {64, 32, 16}) {
        if (bn == 128 && c == 64) continue;
        if (ov.mid_bm && c != ov.mid_bm) continue;
        const int64_t tiles = ((M + c - 1) / c) * tn;
        for (int sp : {1, 2}) {
            if (ov.mid_split && sp != ov.mid_split) continue;
            // a split only while it keeps one round of workgroups and at least three stages in flight
            // (measured: a second round, or a split K range behind a two-stage ring, costs more than the
            // halved bytes save)
            const int nst = (160 * 1024 - 1024) / ((c + bn) * md::KS);
            if (sp > 1 && (bn != 128 || tiles * sp > 256 || nst < 4 || K % ((int64_t)sp * md::KS) != 0 ||
                           tiles > (int64_t)(QK_SPLIT_COUNTER_BYTES / sizeof(uint64_t)) ||
                           tiles * sp * c * bn * 4 >= ((int64_t)1 << 31)))
                continue;
            const int64_t rounds = (tiles * sp + 255) / 256;
            const int64_t cost = rounds * (c + bn) * (K / sp) + (sp > 1 ? (int64_t)c * bn * 8 : 0);
            if (best < 0 || cost < best) {
                best = cost;
                bm = c;
                ns = sp;
            }
        }
    }
    if (best < 0) return m;  // the override asked for a block or split the shape does not allow
    m.bm = bm;
    m.bn = bn;
    m.nsplit = ns;
    m.tiles_m = (int)((M + bm - 1) / bm);
    m.tiles = (int)(m.tiles_m * tn);
    return m;
}

size_t mid_workspace(const MidPlan& m) {
    return m.nsplit > 1 ? QK_SPLIT_COUNTER_BYTES + (size_t)m.tiles * m.nsplit * m.bm * m.bn * sizeof(int32_t) : 0;
}

// [K,N] and int8 NZ weights with 32 < M <= 128: qmm_mid reads the weight once per row block and fills LDS at
// ~45 GB/s per CU, so on wide or deep weights the 128-row K splits of the direct-to-LDS kernel (one row tile:
// every weight byte read once; exact int32 partials, then qmm_reduce_tiled) finish sooner.  A cost model in
// microseconds from measured rates (a CU's LDS fill ~45 GB/s; one HBM stream ~5 TB/s, and for qmm_mid's weight
// reads ~3.1 TB/s on [K,N] rows, ~4.6 TB/s on NZ blocks; the reduce ~4 TB/s plus ~3 us):
//   qmm_mid: the larger of its plan's rounds x (BM + BN) x K / nsplit bytes per CU at the fill rate and its
//            weight at its HBM rate;
//   split:   the larger of its fill time (the M rows of A: rows past M read as zeros without a fetch) and its
//            HBM time (the weight and the partials written), plus the reduce of the partials.
// The split count with the lowest estimate is taken when it is below 0.9 of qmm_mid's.  The sums are exact, so
// the bits equal qmm_mid's.  Returns the split count, or 0 for qmm_mid.
constexpr double kMidHbmKn = 3.1e6, kMidHbmNz = 4.6e6;  // qmm_mid's weight read rate, bytes per us

int small_split(int64_t M, int64_t N, int64_t K, const MidPlan& mp, double mid_hbm = kMidHbmKn) {
    const PlanOverride& ov = plan_override();  // debug override: qmm_small=0 never, =<n> that split count
    if (ov.qmm_small == 0 || mp.bm == 0 || M <= 32 || M > 128 || N % 256 != 0 || K <= 0) return 0;
    auto rounds = [](int64_t wgs) { return (double)((wgs + 255) / 256); };
    constexpr double kFill = 45e3, kHbm = 5e6, kReduce = 4e6, kReduceFixed = 3.0;  // bytes per us; us
    const double w_bytes = (double)K * (double)N;
    const double t_mid_fill = rounds((int64_t)mp.tiles * mp.nsplit) * (mp.bm + mp.bn) * (double)(K / mp.nsplit) / kFill;
    const double t_mid = t_mid_fill > w_bytes / mid_hbm ? t_mid_fill : w_bytes / mid_hbm;
    int best = 0;
    double t_best = 0.9 * t_mid;
    for (int ns : {2, 4, 8}) {
        if (ov.qmm_small > 0 && ns != ov.qmm_small) continue;
        if (K % ((int64_t)ns * dm::BK * dm::NST) != 0) continue;
        const double part = (double)ns * 128.0 * (double)N * 4.0;
        const double t_fill = rounds(N / 256 * ns) * (double)(M + 256) * (double)(K / ns) / kFill;
        const double t_hbm = (w_bytes + part) / kHbm;
        const double t = (t_fill > t_hbm ? t_fill : t_hbm) + part / kReduce + kReduceFixed;
        if (ov.qmm_small > 0 || t < t_best) {
            best = ns;
            t_best = t;
        }
    }
    return best;
}

BigPlan small_split_plan(int64_t M, int64_t N, int ns) {
    BigPlan b;
    b.ok = true;
    b.bm = 128;
    b.tiles_m = (int)((M + 127) / 128);
    b.tiles_n = (int)(N / 256);
    b.nsplit = ns;
    return b;
}

template <int BL, int BM, int BN, int OUT>
hipError_t launch_mid_o(const QmmArgs& p, const MidPlan& mp, int32_t* partial, uint64_t* ctr, hipStream_t stream) {
    // 8 waves; a prefetch wave 12 stages ahead for a [K,N] weight (measured: it shortens the [K,N]
    // cfg1 shape by a sixth and lengthens the [N,K] one, whose 256-byte rows stream well without it)
    constexpr int NW = 8, PD = BL == kLayKN ? 12 : 0;
    const dim3 grid((uint32_t)(mp.tiles * mp.nsplit)), block(64 * NW + (PD > 0 ? 64 : 0));
    if (mp.nsplit > 1) {
        if constexpr (BN == 128)  // splits only with 128-column blocks
            qmm_mid<BL, BM, BN, NW, PD, OUT, true><<<grid, block, 0, stream>>>(p, mp.tiles_m, mp.nsplit, partial,
                                                                                ctr, next_split_tag());
        else
            return hipErrorInvalidValue;
    } else {
        qmm_mid<BL, BM, BN, NW, PD, OUT, false><<<grid, block, 0, stream>>>(p, mp.tiles_m, 1, nullptr, nullptr, 0);
    }
    return hipGetLastError();
}

template <int BL, int BM, int BN>
hipError_t launch_mid_t(const QmmArgs& p, const MidPlan& mp, int32_t* partial, uint64_t* ctr, hipStream_t stream) {
    switch (p.epi.out_dtype) {
    case QK_BF16: return launch_mid_o<BL, BM, BN, QK_BF16>(p, mp, partial, ctr, stream);
    case QK_F16: return launch_mid_o<BL, BM, BN, QK_F16>(p, mp, partial, ctr, stream);
    case QK_F32: return launch_mid_o<BL, BM, BN, QK_F32>(p, mp, partial, ctr, stream);
    case QK_I8: return launch_mid_o<BL, BM, BN, QK_I8>(p, mp, partial, ctr, stream);
    default: return launch_mid_o<BL, BM, BN, QK_I32>(p, mp, partial, ctr, stream);
    }
}

template <int BL>
hipError_t launch_mid(const QmmArgs& p, const MidPlan& mp, int32_t* partial, uint64_t* ctr, hipStream_t stream) {
    if constexpr (BL == kLayKN) {  // 128-column blocks only for a [K,N] weight
        if (mp.bn == 128) {
            if (mp.bm == 32) return launch_mid_t<BL, 32, 128>(p, mp, partial, ctr, stream);
            return launch_mid_t<BL, 16, 128>(p, mp, partial, ctr, stream);
        }
    }
    if (mp.bm == 64) return launch_mid_t<BL, 64, 64>(p, mp, partial, ctr, stream);
    if (mp.bm == 32) return launch_mid_t<BL, 32, 64>(p, mp, partial, ctr, stream);
    return launch_mid_t<BL, 16, 64>(p, mp, partial, ctr, stream);
}

// The kernels that need no workspace and no alignment beyond the tiled kernels' (or none at all).
hipError_t launch_qmm_fallback(const QmmArgs& p, bool a_ok, bool b_kn, bool b_nk, hipStream_t stream) {
    if (p.K > 0 && a_ok && b_kn) return launch_by_m<true>(p, stream);
    if (p.K > 0 && a_ok && b_nk) return launch_by_m<false>(p, stream);
    const int64_t total = p.M * p.N;
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    qmm_generic<<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(p);
    return hipGetLastError();
}

// A split workspace is [split-K counters][int32 partials [nsplit][M][N]].
size_t quant_matmul_workspace(int64_t M, int64_t N, int64_t K) {
    if (mid_plan(M, N, K, false).bm != 0 && M > 32) {  // eligibility does not depend on the layout; the
        const MidPlan mk = mid_plan(M, N, K, true);     // [K,N] plan's splits need a workspace
        size_t need = mid_workspace(mk);
        if (const int ns = small_split(M, N, K, mk)) {
            const size_t alt = big_split_workspace(small_split_plan(M, N, ns), M, N);
            if (alt > need) need = alt;
        }
        return need;
    }
    const SkinnyPlan s = skinny_plan(M, N, K);
    if (s.mt != 0)
        return s.nsplit == 1 ? 0 : QK_SPLIT_COUNTER_BYTES + (size_t)s.nsplit * (size_t)M * (size_t)N * sizeof(int32_t);
    const BigPlan b = big_plan(M, N, K);
    if (!b.ok || b.nsplit == 1) return 0;
    // a 128-row split plan falls back to the 256-row one where its kernel does not apply: room for either
    const size_t need = big_split_workspace(b, M, N);
    if (b.bm == 128) {
        const size_t alt = big_split_workspace(big_plan(M, N, K, false), M, N);
        return need > alt ? need : alt;
    }
    return need;
}

hipError_t launch_quant_matmul(const QmmArgs& p, void* workspace, size_t ws_bytes, hipStream_t stream) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    const bool a_ok = (p.K % 16 == 0) && (p.lda % 16 == 0) && ((uintptr_t)p.a % 16 == 0);
    const bool b_nk = (p.sbk == 1) && (p.sbn % 16 == 0) && ((uintptr_t)p.b % 16 == 0);
    const bool b_kn = (p.sbn == 1) && (p.sbk % 8 == 0) && (p.N % 8 == 0) && ((uintptr_t)p.b % 8 == 0);
    const bool b_kn16 = b_kn && p.N % 16 == 0 && p.sbk % 16 == 0 && (uintptr_t)p.b % 16 == 0;
    char* ws = static_cast<char*>(workspace);
    int32_t* partial = ws ? reinterpret_cast<int32_t*>(ws + QK_SPLIT_COUNTER_BYTES) : nullptr;
    MidPlan mp = mid_plan(p.M, p.N, p.K, b_kn16);
    if (mp.bm != 0 && (p.M > 32 || !b_kn16)) {
        if (b_kn16) {  // wide or deep [K,N] weights: 128-row K splits where the cost model favours them
            if (const int ns = small_split(p.M, p.N, p.K, mp)) {
                const BigPlan sb = small_split_plan(p.M, p.N, ns);
                if (big_dma_ok(p, true, ns) && partial && ws_bytes >= big_split_workspace(sb, p.M, p.N) &&
                    (uintptr_t)partial % 16 == 0)
                    return launch_split128<kLayKN>(p, sb, partial, stream);
            }
        }
        // a split plan needs its partials and counters; with less workspace the same blocks run unsplit
        const size_t need = mid_workspace(mp);
        if (need && (!ws || ws_bytes < need || (uintptr_t)ws % 16 != 0)) mp.nsplit = 1;
        // direct-to-LDS loads need 16-byte aligned rows and 32-bit buffer offsets; the 8-output epilogue
        // stores need 16-byte aligned output rows.  Otherwise the tiled kernels (no workspace) take it.
        const int osz = p.epi.out_dtype == QK_I8 ? 1 : ((p.epi.out_dtype == QK_BF16 || p.epi.out_dtype == QK_F16) ? 2 : 4);
        const bool ok = a_ok && (uint64_t)mp.bm * (uint64_t)p.lda < (1ull << 31) &&
                        (uintptr_t)p.epi.out % 16 == 0 && (p.epi.ldo * osz) % 16 == 0 &&
                        (b_kn16 ? (uint64_t)p.K * (uint64_t)p.sbk < (1ull << 32)
                                : (b_nk && (uint64_t)mp.bn * (uint64_t)p.sbn < (1ull << 32)));
        uint64_t* ctr = mp.nsplit > 1 ? reinterpret_cast<uint64_t*>(ws) : nullptr;
        if (ok) return b_kn16 ? launch_mid<kLayKN>(p, mp, partial, ctr, stream) : launch_mid<kLayNK>(p, mp, partial, ctr, stream);
        return launch_qmm_fallback(p, a_ok, b_kn, b_nk, stream);
    }
    const SkinnyPlan sp = skinny_plan(p.M, p.N, p.K);
    if (sp.mt != 0 && a_ok && (b_nk || b_kn16)) {
        const size_t need = sp.nsplit > 1 ? QK_SPLIT_COUNTER_BYTES + (size_t)sp.nsplit * p.M * p.N * sizeof(int32_t) : 0;
        if (need && (!workspace || ws_bytes < need)) return hipErrorInvalidValue;
        return b_kn16 ? launch_skinny<true>(p, sp, partial, stream) : launch_skinny<false>(p, sp, partial, stream);
    }
    BigPlan bp = big_plan(p.M, p.N, p.K);
    bool big_ok = bp.ok && a_ok && (b_nk || (b_kn && p.N % 16 == 0 && p.sbk % 16 == 0 && (uintptr_t)p.b % 16 == 0));
    if (big_ok && bp.bm == 128) {
        // the 128-row split needs the direct-to-LDS kernel and its workspace; otherwise the shape runs unsplit
        const size_t need = big_split_workspace(bp, p.M, p.N);
        if (big_dma_ok(p, b_kn, bp.nsplit) && partial && ws_bytes >= need && (uintptr_t)partial % 16 == 0)
            return b_kn ? launch_split128<kLayKN>(p, bp, partial, stream) : launch_split128<kLayNK>(p, bp, partial, stream);
        bp = big_plan(p.M, p.N, p.K, false);
    }
    // a split of a ragged M runs only on the direct-to-LDS kernel; otherwise the register-staged kernel runs
    // the shape unsplit (the planned workspace is then unused)
    if (big_ok && bp.nsplit > 1 && p.M % big::BM != 0 && !big_dma_ok(p, b_kn, bp.nsplit)) bp.nsplit = 1;
    if (big_ok && bp.nsplit > 1) {
        // splits need whole aligned tiles and the workspace; otherwise the tiled kernels take the shape
        const size_t need = QK_SPLIT_COUNTER_BYTES + (size_t)bp.nsplit * p.M * p.N * sizeof(int32_t);
        big_ok = p.lda < (1 << 24) && p.sbk < (1 << 24) && p.sbn < (1 << 24) && partial && ws_bytes >= need &&
                 (uintptr_t)partial % 16 == 0;
        if (big_ok) {
            const hipError_t e = b_kn ? launch_big<QK_I32>(p, true, bp.tiles_m, bp.tiles_n, bp.nsplit, partial, stream)
                                      : launch_big<QK_I32>(p, false, bp.tiles_m, bp.tiles_n, bp.nsplit, partial, stream);
            if (e != hipSuccess) return e;
            int64_t blocks = (p.M * p.N / 4 + kThreads - 1) / kThreads;
            if (blocks > 65536) blocks = 65536;
            qmm_reduce<<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(p, bp.nsplit, partial);
            return hipGetLastError();
        }
    } else if (big_ok) {
        const int tm = bp.tiles_m, tn = bp.tiles_n;
        switch (p.epi.out_dtype) {
        case QK_BF16: return launch_big<QK_BF16>(p, b_kn, tm, tn, 1, nullptr, stream);
        case QK_F16: return launch_big<QK_F16>(p, b_kn, tm, tn, 1, nullptr, stream);
        case QK_F32: return launch_big<QK_F32>(p, b_kn, tm, tn, 1, nullptr, stream);
        case QK_I8: return launch_big<QK_I8>(p, b_kn, tm, tn, 1, nullptr, stream);
        default: return launch_big<QK_I32>(p, b_kn, tm, tn, 1, nullptr, stream);
        }
    }
    return launch_qmm_fallback(p, a_ok, b_kn, b_nk, stream);
}

// ---------------------------------------------------------------------------
// W8A8 on an int8 NZ weight (p.b: [N/16][K/64][64][16]; p.sbk and p.sbn unused).  By shape: M <= 16 the
// decode stream qmm_nzd (no workspace); the mid-M plan qmm_mid on NZ blocks (64-column blocks, no split);
// 256-column tiles (any M) qmm_dma on NZ blocks (a K split as planned for the row-major weight); any other
// shape unpacks the weight to [K,N] in the workspace and runs the row-major kernels on it:
// [ND weight, 256-byte rounded][that call's workspace].  The C ABI guarantees 16-byte aligned x1 rows
// (row stride below 2^24), weight and output.
namespace {

struct NzdPlan {
    int nb = 0, nwg = 0;
};

// every CU one workgroup of ceil(N/16 / 256) n-blocks (at most NBMAX), then as few workgroups as give
// none more
NzdPlan nzd_plan(int64_t M, int64_t N, int64_t K) {
    NzdPlan z;
    if (M < 1 || M > 16 || N < 16 || N % 16 != 0 || K <= 0 || K % 64 != 0) return z;
    const int64_t nbt = N / 16;
    int64_t nb = (nbt + 255) / 256;
    if (nb > nzd::NBMAX) nb = nzd::NBMAX;
    const int64_t nwg = (nbt + nb - 1) / nb;
    if (nwg >= ((int64_t)1 << 30)) return z;
    z.nb = (int)nb;
    z.nwg = (int)nwg;
    return z;
}

hipError_t launch_nzd(const QmmArgs& p, const NzdPlan& z, hipStream_t stream) {
    const dim3 grid((uint32_t)z.nwg), block(nzd::NT);
    switch (z.nb) {
    case 1: qmm_nzd<1><<<grid, block, 0, stream>>>(p, z.nwg); break;
    case 2: qmm_nzd<2><<<grid, block, 0, stream>>>(p, z.nwg); break;
    case 3: qmm_nzd<3><<<grid, block, 0, stream>>>(p, z.nwg); break;
    case 4: qmm_nzd<4><<<grid, block, 0, stream>>>(p, z.nwg); break;
    case 5: qmm_nzd<5><<<grid, block, 0, stream>>>(p, z.nwg); break;
    case 6: qmm_nzd<6><<<grid, block, 0, stream>>>(p, z.nwg); break;
    case 7: qmm_nzd<7><<<grid, block, 0, stream>>>(p, z.nwg); break;
    default: qmm_nzd<8><<<grid, block, 0, stream>>>(p, z.nwg); break;
    }
    return hipGetLastError();
}

// qmm_dma on NZ blocks: whole 256-column tiles (any M) and K ranges of whole four-stage rings
bool nz_dma_ok(const BigPlan& b, int64_t M, int64_t N, int64_t K) {
    (void)M;
    return plan_override().qmm_dma && b.ok && N % dm::BN == 0 && K % ((int64_t)b.nsplit * dm::BK * dm::NST) == 0;
}

template <int OUT>
hipError_t launch_dma_nz(const QmmArgs& p, const BigPlan& b, int32_t* partial, hipStream_t stream) {
    if (b.bm != 256) return hipErrorInvalidValue;  // 256-row tiles: tiles_m counts them
    qmm_dma<kLayNZ, OUT><<<dim3((uint32_t)(b.tiles_m * b.tiles_n * b.nsplit)), dim3(dm::NT), 0, stream>>>(
        p, b.tiles_m, b.tiles_n, b.nsplit, partial, dma_rev_from());
    return hipGetLastError();
}

size_t round_up256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

size_t quant_matmul_nz_workspace(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    if (nzd_plan(M, N, K).nb) return 0;
    if (mid_plan(M, N, K, false).bm) {  // the mid-M shapes: qmm_mid on NZ blocks (no workspace) or split tiles
        const int ns = small_split(M, N, K, mid_plan(M, N, K, false), kMidHbmNz);
        return ns ? big_split_workspace(small_split_plan(M, N, ns), M, N) : 0;
    }
    const BigPlan b = big_plan(M, N, K);
    if (nz_dma_ok(b, M, N, K)) return b.nsplit > 1 ? big_split_workspace(b, M, N) : 0;
    return round_up256((size_t)K * (size_t)N) + quant_matmul_workspace(M, N, K);
}

hipError_t launch_quant_matmul_nz(const QmmArgs& p, void* workspace, size_t ws_bytes, hipStream_t stream) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    if (p.K == 0) return launch_qmm_fallback(p, false, false, false, stream);  // reads no weight
    const NzdPlan z = nzd_plan(p.M, p.N, p.K);
    if (z.nb) return launch_nzd(p, z, stream);
    char* ws = static_cast<char*>(workspace);
    const MidPlan mp = mid_plan(p.M, p.N, p.K, false);
    if (mp.bm) {
        // wide or deep weights: 128-row K-split tiles where the cost model favours them (a workspace smaller
        // than the query's runs qmm_mid, the same bits)
        if (const int ns = small_split(p.M, p.N, p.K, mp, kMidHbmNz)) {
            const BigPlan sb = small_split_plan(p.M, p.N, ns);
            if (plan_override().qmm_dma && ws && ws_bytes >= big_split_workspace(sb, p.M, p.N) &&
                (uintptr_t)ws % 16 == 0)
                return launch_split128<kLayNZ>(p, sb, reinterpret_cast<int32_t*>(ws + QK_SPLIT_COUNTER_BYTES),
                                               stream);
        }
        return launch_mid<kLayNZ>(p, mp, nullptr, nullptr, stream);
    }
    const BigPlan b = big_plan(p.M, p.N, p.K);
    if (nz_dma_ok(b, p.M, p.N, p.K)) {
        if (b.nsplit == 1) {
            switch (p.epi.out_dtype) {
            case QK_BF16: return launch_dma_nz<QK_BF16>(p, b, nullptr, stream);
            case QK_F16: return launch_dma_nz<QK_F16>(p, b, nullptr, stream);
            case QK_F32: return launch_dma_nz<QK_F32>(p, b, nullptr, stream);
            case QK_I8: return launch_dma_nz<QK_I8>(p, b, nullptr, stream);
            default: return launch_dma_nz<QK_I32>(p, b, nullptr, stream);
            }
        }
        const size_t need = big_split_workspace(b, p.M, p.N);
        if (!ws || ws_bytes < need || (uintptr_t)ws % 16 != 0) return hipErrorInvalidValue;
        int32_t* partial = reinterpret_cast<int32_t*>(ws + QK_SPLIT_COUNTER_BYTES);
        if (b.bm == 128) return launch_split128<kLayNZ>(p, b, partial, stream);
        const hipError_t e = launch_dma_nz<QK_I32>(p, b, partial, stream);
        if (e != hipSuccess) return e;
        int64_t blocks = (p.M * p.N / 4 + kThreads - 1) / kThreads;
        if (blocks > 65536) blocks = 65536;
        qmm_reduce<<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(p, b.nsplit, partial);
        return hipGetLastError();
    }
    const size_t nd = round_up256((size_t)p.K * (size_t)p.N);
    const size_t rest = quant_matmul_workspace(p.M, p.N, p.K);
    if (!ws || ws_bytes < nd + rest || (uintptr_t)ws % 256 != 0) return hipErrorInvalidValue;
    const hipError_t e = launch_w8_nz_cast(p.b, false, p.K, p.N, reinterpret_cast<int8_t*>(ws), stream);
    if (e != hipSuccess) return e;
    QmmArgs q = p;
    q.b = reinterpret_cast<const int8_t*>(ws);
    q.sbk = p.N;
    q.sbn = 1;
    return launch_quant_matmul(q, rest ? ws + nd : nullptr, rest, stream);
}

hipError_t launch_quant_matmul_swiglu(const QmmArgs& p, bool nz, float* amax_part, hipStream_t stream) {
    const int64_t I = p.N / 2;
    const QmmEpilogue& e = p.epi;
    const bool ok =
        p.M > 0 && I > 0 && p.N == 2 * I && I % 128 == 0 && p.K > 0 && p.K % (dm::BK * dm::NST) == 0 &&
        p.lda % 16 == 0 && p.lda < (1 << 24) && (uintptr_t)p.a % 16 == 0 && (uintptr_t)p.b % 16 == 0 &&
        (uintptr_t)e.out % 16 == 0 && e.ldo % 8 == 0 && e.bias_dtype == 0 && e.offset == nullptr && e.scale &&
        (e.out_dtype == QK_BF16 || e.out_dtype == QK_F16) &&
        (nz ? (uint64_t)p.N * (uint64_t)p.K < (1ull << 32)
            : (p.sbn == 1 && p.sbk % 16 == 0 && p.sbk >= p.N && p.sbk < (1 << 24) &&
               (uint64_t)(p.K - 1) * (uint64_t)p.sbk + (uint64_t)I + 128 < (1ull << 32)));
    const int64_t tiles_m = (p.M + dm::BM - 1) / dm::BM, tiles_n = I / 128;
    if (!ok || tiles_m * tiles_n >= ((int64_t)1 << 30)) return hipErrorInvalidValue;
    const dim3 grid((uint32_t)(tiles_m * tiles_n)), block(dm::NT);
    const int tm = (int)tiles_m, tn = (int)tiles_n;
    constexpr int S = kOutSwiGLU;
    int32_t* ap = reinterpret_cast<int32_t*>(amax_part);
    if (nz) {
        if (e.out_dtype == QK_BF16) qmm_dma<kLayNZ, S + QK_BF16><<<grid, block, 0, stream>>>(p, tm, tn, 1, ap, dma_rev_from());
        else qmm_dma<kLayNZ, S + QK_F16><<<grid, block, 0, stream>>>(p, tm, tn, 1, ap, dma_rev_from());
    } else {
        if (e.out_dtype == QK_BF16) qmm_dma<kLayKN, S + QK_BF16><<<grid, block, 0, stream>>>(p, tm, tn, 1, ap, dma_rev_from());
        else qmm_dma<kLayKN, S + QK_F16><<<grid, block, 0, stream>>>(p, tm, tn, 1, ap, dma_rev_from());
    }
    return hipGetLastError();
}

}  // namespace qk
