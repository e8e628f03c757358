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
// Decode kernel (w4_decode), an HBM weight stream for M <= 16 rows per
// workgroup: a workgroup owns a strip of 32 packed words (256 output columns,
// one 128-byte line per weight row) and a K range (a "split").  Its four waves
// are 2 (word halves) x 2 (K halves); a wave streams 128-row chunks with the
// next chunk's loads in flight.  MFMA lane (c, kg) holds word column c of the
// wave's half for rows 8kg..8kg+7 of a 32-row block, and nibble j of those 8
// words is the B operand of MFMA tile j, so each lane finally owns 8
// consecutive output columns.  Splits write fp32 partials to the workspace
// and w4_reduce sums them in split order (deterministic); with one split the
// decode kernel writes the output itself.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.h"

namespace qk {
namespace {

constexpr int kThreads = 256;
constexpr int CHUNK = 128;  // K rows per streamed chunk (4 MFMA K-blocks)
constexpr int STRIP = 32;   // packed words per workgroup

// B operand of MFMA tile j: nibble j of 8 offset-binary words (rows 0..7),
// packed as 16-bit magic values, two rows per dword.
template <uint32_t MAGIC, int J>
__device__ __forceinline__ u32x4 unpack_tile(const uint32_t w[8]) {
    constexpr uint32_t bj = (uint32_t)J >> 1;
    constexpr uint32_t sel = bj | ((4u + bj) << 16) | 0x0c000c00u;  // byte bj of each word -> bits 0..7 / 16..23
    const uint32_t mask = __builtin_amdgcn_readfirstlane(0x000f000fu);
    const uint32_t magic = __builtin_amdgcn_readfirstlane(MAGIC);
    u32x4 b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t pair = __builtin_amdgcn_perm(w[2 * q + 1], w[2 * q], sel);
        if constexpr (J & 1) pair >>= 4;
        b[q] = (pair & mask) | magic;
    }
    return b;
}

// v_perm_b32 selector: byte b of the low source to bits 0..7, byte b of the
// high source to bits 16..23, zeros elsewhere.
__host__ __device__ constexpr uint32_t byte_sel(uint32_t b) { return b | ((4u + b) << 16) | 0x0c000c00u; }

// Two's-complement nibble r straight to the magic operand: (r & 0xf) ^ 0x..08
// leaves MAGIC's high bits and puts u = r ^ 8 = w + 8 in the low bits, so the
// offset-binary flip costs nothing (gfx950 does and+xor in one v_bitop3_b32).
// `sel` (per lane) picks byte b of rows 2q and 2q+1; odd nibbles are shifted
// down first.
template <uint32_t MAGIC, bool ODD>
__device__ __forceinline__ u32x4 unpack_raw(const uint32_t w[8], uint32_t sel) {
    const uint32_t mask = __builtin_amdgcn_readfirstlane(0x000f000fu);
    const uint32_t magic = __builtin_amdgcn_readfirstlane(MAGIC | 0x00080008u);
    u32x4 b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t pair = __builtin_amdgcn_perm(w[2 * q + 1], w[2 * q], sel);
        if constexpr (ODD) pair >>= 4;
        b[q] = (pair & mask) ^ magic;
    }
    return b;
}

// int8 weights: byte t of rows 2q and 2q+1 as exact 16-bit values (every
// int8 is both a bf16 and an fp16 number), two rows per dword.
template <int DT>
__device__ __forceinline__ u32x4 unpack_i8(const uint32_t w[8], int t) {
    u32x4 b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float lo = (float)(int8_t)(w[2 * q] >> (8 * t));
        const float hi = (float)(int8_t)(w[2 * q + 1] >> (8 * t));
        if constexpr (DT == QK_BF16)  // exact values: the upper halves are the bf16 numbers
            b[q] = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
        else  // exact values: round-toward-zero packing is exact
            b[q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
    return b;
}

__device__ __forceinline__ void halves8(u32x4 v, int dt, float f[8]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[2 * e] = load_half_bits(v[e] & 0xffffu, dt);
        f[2 * e + 1] = load_half_bits(v[e] >> 16, dt);
    }
}

template <int OUTDT>
__device__ __forceinline__ void store8(void* out, int64_t off, const float v[8]) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t lo = OUTDT == QK_BF16 ? f32_to_bf16_bits(v[2 * e]) : f32_to_f16_bits(v[2 * e]);
        const uint32_t hi = OUTDT == QK_BF16 ? f32_to_bf16_bits(v[2 * e + 1]) : f32_to_f16_bits(v[2 * e + 1]);
        o[e] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + off) = o;
}

// PIECE_KB: 32-row K-blocks per scaling piece (min(group,128)/32).
// FINAL: one split, write bf16/fp16 output (+bias) directly.
// UPFRONT: each wave's K range is exactly 256 rows, loaded before any math.
template <int DT, int PIECE_KB, bool HAS_OFF, bool FINAL, bool UPFRONT>
__global__ __launch_bounds__(kThreads) void w4_decode(WqbmmArgs p, float* __restrict__ partial, int nsplit,
                                                      int nstrip) {
    typedef Mfma<DT> MM;
    constexpr int NP = 4 / PIECE_KB;  // pieces per chunk
    // LDS: the upfront path's per-wave transposed tiles, later reused by the
    // cross-wave reduction (red)
    constexpr int LDS_U32 = UPFRONT ? 4 * 16 * 260 : 2 * 16 * 132;
    __shared__ __attribute__((aligned(16))) uint32_t lds_u32[LDS_U32];
    float (*red)[16][132] = reinterpret_cast<float (*)[16][132]>(lds_u32);

    // wave index through readfirstlane so everything derived from it is scalar
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = wave & 1, kh = wave >> 1;
    const int c = lane & 15, kg = lane >> 4;
    const int blk = blockIdx.x;
    const int strip = blk % nstrip;
    const int split = (blk / nstrip) % nsplit;
    const int rb = blk / (nstrip * nsplit);

    const int NW = (int)(p.N >> 3);
    const int wc_raw = strip * STRIP + 16 * h + c;
    const bool col_ok = wc_raw < NW;
    const int wc = col_ok ? wc_raw : NW - 1;  // clamped: loads stay in bounds, results discarded
    const int M = (int)p.M, K = (int)p.K, N = (int)p.N, G = (int)p.group;
    const int m_raw = rb * 16 + c;
    const bool row_ok = m_raw < M;
    const int m = row_ok ? m_raw : M - 1;

    const int rows_split = K / nsplit;
    const int k_begin = split * rows_split + kh * (rows_split >> 1);
    const int nch = (rows_split >> 1) / CHUNK;

    const uint32_t rowbytes = (uint32_t)NW * 4u;
    const char* Wb = static_cast<const char*>(p.w);
    const uint32_t w_lane = (uint32_t)(8 * kg) * rowbytes + (uint32_t)wc * 4u;
    const char* Xb = static_cast<const char*>(p.x);
    const uint32_t x_lane = ((uint32_t)m * (uint32_t)K + 8u * (uint32_t)kg) * 2u;
    const char* Sb = static_cast<const char*>(p.scale);
    const char* Ob = static_cast<const char*>(p.offset);
    const uint32_t s_lane = (uint32_t)(8 * wc) * 2u;
    const u32x4 ones = {MM::ONES, MM::ONES, MM::ONES, MM::ONES};
    const u32x4 zero4 = {0u, 0u, 0u, 0u};

    f32x4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // The K range streams in 64-row halves (2 MFMA K-blocks) through two
    // alternating register buffers: the next half's loads are in flight while
    // the current half is unpacked and multiplied.  A chunk (128 rows) is an
    // even half followed by an odd half, so piece ends (every 32/64/128 rows)
    // fall at compile-time positions.
    constexpr int HKB = 2;
    constexpr int PPH = PIECE_KB <= HKB ? HKB / PIECE_KB : 1;  // scale points held per half
    struct Half {
        uint32_t w[HKB][8];
        u32x4 x[HKB];
        u32x4 s[PPH], o[PPH];
    };

    auto load = [&](int hidx, Half& d, bool odd) {
        const int k0 = k_begin + hidx * 64;
#pragma unroll
        for (int kb = 0; kb < HKB; ++kb) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const char* rowp = Wb + (size_t)(uint32_t)(k0 + kb * 32 + r) * rowbytes;
                d.w[kb][r] = *reinterpret_cast<const uint32_t*>(rowp + w_lane);
            }
            const u32x4 xv = *reinterpret_cast<const u32x4*>(Xb + (size_t)(k0 + kb * 32) * 2u + x_lane);
            d.x[kb] = row_ok ? xv : zero4;
        }
        if (PIECE_KB <= HKB || odd) {
#pragma unroll
            for (int pp = 0; pp < PPH; ++pp) {
                const uint32_t g = (uint32_t)(k0 + pp * PIECE_KB * 32) / (uint32_t)G;
                d.s[pp] = *reinterpret_cast<const u32x4*>(Sb + (size_t)g * (uint32_t)N * 2u + s_lane);
                if (HAS_OFF) d.o[pp] = *reinterpret_cast<const u32x4*>(Ob + (size_t)g * (uint32_t)N * 2u + s_lane);
            }
        }
    };

    f32x4 ag[8], xs;
    auto reset = [&]() {
        xs = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 8; ++t) ag[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };
    auto fold = [&](u32x4 sv, u32x4 ov) {  // acc += s*A + s*(offset - BASE)*xs, then start a new piece
        float sf[8], of[8];
        halves8(sv, p.s_dtype, sf);
        if (HAS_OFF) halves8(ov, p.s_dtype, of);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float sb = sf[t] * ((HAS_OFF ? of[t] : 0.0f) - MM::BASE);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(sf[t], ag[t][r], __builtin_fmaf(sb, xs[r], acc[t][r]));
        }
        reset();
    };
    auto compute = [&](const Half& d, bool odd) {
#pragma unroll
        for (int kb = 0; kb < HKB; ++kb) {
            uint32_t w8[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) w8[r] = d.w[kb][r] ^ 0x88888888u;
            ag[0] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 0>(w8), ag[0]);
            ag[1] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 1>(w8), ag[1]);
            ag[2] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 2>(w8), ag[2]);
            ag[3] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 3>(w8), ag[3]);
            ag[4] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 4>(w8), ag[4]);
            ag[5] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 5>(w8), ag[5]);
            ag[6] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 6>(w8), ag[6]);
            ag[7] = MM::mma(d.x[kb], unpack_tile<MM::MAGIC, 7>(w8), ag[7]);
            xs = MM::mma(d.x[kb], ones, xs);
            if (PIECE_KB == 1) fold(d.s[kb], d.o[kb]);
        }
        if (PIECE_KB == 2 || (PIECE_KB == 4 && odd)) fold(d.s[0], d.o[0]);
    };

    reset();
    Half b0, b1;
    const int nhalf = 2 * nch;
    if constexpr (UPFRONT) {
        // 256 rows per wave, every load issued before the first MFMA.  The
        // loads are 16 bytes per lane (4 lanes per 64-byte row piece, 16 rows
        // per instruction); each wave transposes its own 16x256 word tile
        // through LDS ([column][row], 260-dword columns: conflict-free 32-bit
        // writes and 128-bit reads) into the MFMA lane layout.  LDS traffic
        // of a wave stays inside that wave, so no barrier is needed.
        uint32_t* wt = lds_u32 + wave * (16 * 260);
        const int cw = lane & 3, rr = lane >> 2;
        const int wcol_raw = strip * STRIP + 16 * h + 4 * cw;
        const int wcol = wcol_raw < NW ? wcol_raw : NW - 4;  // NW % 4 == 0
        const char* src = Wb + (size_t)(uint32_t)(k_begin + rr) * rowbytes + (uint32_t)wcol * 4u;
        u32x4 raw[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) raw[i] = *reinterpret_cast<const u32x4*>(src + (size_t)(16 * i) * rowbytes);
        u32x4 xa[8];
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            const u32x4 xv = *reinterpret_cast<const u32x4*>(Xb + (size_t)(k_begin + kb * 32) * 2u + x_lane);
            xa[kb] = row_ok ? xv : zero4;
        }
        constexpr int NPW = 8 / PIECE_KB;  // pieces per wave
        u32x4 sv[NPW], ov[NPW];
#pragma unroll
        for (int pp = 0; pp < NPW; ++pp) {
            const uint32_t gi = (uint32_t)(k_begin + pp * PIECE_KB * 32) / (uint32_t)G;
            sv[pp] = *reinterpret_cast<const u32x4*>(Sb + (size_t)gi * (uint32_t)N * 2u + s_lane);
            if (HAS_OFF) ov[pp] = *reinterpret_cast<const u32x4*>(Ob + (size_t)gi * (uint32_t)N * 2u + s_lane);
        }
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
#pragma unroll
            for (int ii = 2 * kb; ii < 2 * kb + 2; ++ii)
#pragma unroll
                for (int w = 0; w < 4; ++w) wt[(4 * cw + w) * 260 + 16 * ii + rr] = raw[ii][w];
            const u32x4 lo = *reinterpret_cast<const u32x4*>(wt + c * 260 + 32 * kb + 8 * kg);
            const u32x4 hi = *reinterpret_cast<const u32x4*>(wt + c * 260 + 32 * kb + 8 * kg + 4);
            uint32_t w8[8] = {lo[0] ^ 0x88888888u, lo[1] ^ 0x88888888u, lo[2] ^ 0x88888888u, lo[3] ^ 0x88888888u,
                              hi[0] ^ 0x88888888u, hi[1] ^ 0x88888888u, hi[2] ^ 0x88888888u, hi[3] ^ 0x88888888u};
            ag[0] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 0>(w8), ag[0]);
            ag[1] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 1>(w8), ag[1]);
            ag[2] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 2>(w8), ag[2]);
            ag[3] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 3>(w8), ag[3]);
            ag[4] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 4>(w8), ag[4]);
            ag[5] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 5>(w8), ag[5]);
            ag[6] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 6>(w8), ag[6]);
            ag[7] = MM::mma(xa[kb], unpack_tile<MM::MAGIC, 7>(w8), ag[7]);
            xs = MM::mma(xa[kb], ones, xs);
            if ((kb + 1) % PIECE_KB == 0) fold(sv[kb / PIECE_KB], ov[kb / PIECE_KB]);
        }
        __syncthreads();  // the reduction below reuses the LDS tile area
    } else {
        if (nhalf > 0) load(0, b0, false);
        for (int hidx = 0; hidx < nhalf; hidx += 2) {
            load(hidx + 1, b1, true);
            compute(b0, false);
            if (hidx + 2 < nhalf) load(hidx + 2, b0, false);
            compute(b1, true);
        }
    }

    // K-half 1 hands its sums to K-half 0 (fixed order: half 0 + half 1)
    if (kh == 1) {
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[h][4 * kg + r][8 * c + t] = acc[t][r];
    }
    __syncthreads();
    if (kh == 1) return;
    const int64_t n0 = 8 * (int64_t)wc_raw;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t mm = (int64_t)rb * 16 + 4 * kg + r;
        float v[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = acc[t][r] + red[h][4 * kg + r][8 * c + t];
        if (!col_ok || mm >= M) continue;
        if (FINAL) {
            if (p.bias_dtype) {
#pragma unroll
                for (int t = 0; t < 8; ++t) v[t] += load_scalar(p.bias, n0 + t, p.bias_dtype);
            }
            if (p.out_dtype == QK_BF16) store8<QK_BF16>(p.out, mm * N + n0, v);
            else store8<QK_F16>(p.out, mm * N + n0, v);
        } else {
            f32x4* dst = reinterpret_cast<f32x4*>(partial + ((int64_t)split * M + mm) * N + n0);
            dst[0] = (f32x4){v[0], v[1], v[2], v[3]};
            dst[1] = (f32x4){v[4], v[5], v[6], v[7]};
        }
    }
}

// Decode weight stream for up to 16 rows of x per workgroup.
//
// A workgroup owns a strip of 32 packed words (256 output columns: one full
// 128-byte line of every weight row) and a K split.  Its waves are
// HALVES = 32/WPL column sub-strips x KW = NWAVE/HALVES K ranges of NKB
// 32-row K-blocks.  MFMA lane (c, kg) = (lane & 15, lane >> 4) reads, for each
// of its K-blocks, rows 8kg..8kg+7 of one word column straight from HBM (one
// dword per row; the 16 lanes of a k-group cover WPL consecutive words), so the
// B operands are built in registers without any LDS transpose:
//   WPL == 32: slot c owns words 2c and 2c+1 (one 8-byte load per row, so a
//              k-group's 16 lanes read the whole 128-byte line) and their 16
//              nibbles (16 MFMA tiles, columns 16c + t);
//   WPL == 16: slot c owns word c and all 8 of its nibbles (8 MFMA tiles);
//   WPL == 8:  slots c and c+8 share word c&7, slot c takes nibbles
//              4(c>>3)..4(c>>3)+3 (4 tiles).
// The sub-strip waves of one K range read the same rows, so every 128-byte
// line is consumed whole inside one workgroup (lines split between
// workgroups read at about 2/3 of the bandwidth).  Each wave issues its loads
// block by block before its first MFMA.  The K ranges are added through LDS
// in order (deterministic), each thread finishing 4 columns of one row.  With
// one split the sums are the output (+bias, cast); otherwise fp32 partials
// [split][M][N]: with a counter array (ctr) they are stored device-coherent
// and the strip's last split to arrive adds them in split order, adds bias
// and casts (one kernel); without one, w4_reduce finishes.
// W8 (int8 weights [K, N], W8A16): a strip is 64 dwords (256 columns, two
// lines per row) and WPL is 16, 32 or 64 (a quarter, half or whole row per
// wave): slot c owns LW = WPL/16 adjacent dwords of its sub-strip (one 4-,
// 8- or 16-byte load per row) and their 4*LW bytes (MFMA tiles, columns
// 4*LW*c + t), and the operands are the exact 16-bit values of the bytes (no
// magic offset: BASE = 0).
template <int DT, int WPL, int NWAVE, int NKB, int PF, int PIECE_KB, bool HAS_OFF, bool FINAL, bool W8>
__global__ __launch_bounds__(64 * NWAVE) void w4_stream(WqbmmArgs p, float* __restrict__ partial, int nstrip,
                                                        int nsplit, uint64_t* __restrict__ ctr, uint64_t tag) {
    typedef Mfma<DT> MM;
    static_assert(!W8 || WPL == 16 || WPL == 32 || WPL == 64, "int8 weights use 16-, 32- or 64-dword sub-strips");
    constexpr int CPW = W8 ? 4 : 8;         // output columns per weight dword
    constexpr int SW = 256 / CPW;           // dwords per strip row (256 columns)
    constexpr int LW = W8 ? WPL / 16 : (WPL == 32 ? 2 : 1);  // dwords per lane and row
    constexpr int TPL = W8 ? 4 * LW : (WPL == 32 ? 16 : WPL == 16 ? 8 : 4);  // MFMA tiles per lane
    constexpr int HALVES = SW / WPL;        // column sub-strips per workgroup
    constexpr int KW = NWAVE / HALVES;      // K ranges per workgroup
    constexpr int NCOL = CPW * WPL;         // output columns per wave
    constexpr float BASE = W8 ? 0.0f : MM::BASE;
    constexpr int RSTR = NCOL + 4;          // LDS row pitch in floats
    constexpr int NPIECE = NKB / PIECE_KB;
    static_assert(NKB % PIECE_KB == 0, "pieces must tile the wave's K range");
    static_assert(KW >= 1 && KW * HALVES == NWAVE, "waves must tile the strip");
    __shared__ __attribute__((aligned(16))) float red[NWAVE][16][RSTR];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, kg = lane >> 4;
    const int h = wave % HALVES, kw = wave / HALVES;
    // same-split strips share the x rows: keep neighbours on one XCD (one L2)
    const int blk = xcd_swizzle(blockIdx.x, gridDim.x);
    const int strip = blk % nstrip;
    const int split = (blk / nstrip) % nsplit;
    const int rb = blk / (nstrip * nsplit);

    const int M = (int)p.M, K = (int)p.K, N = (int)p.N, G = (int)p.group;
    const int NW = W8 ? (N >> 2) : (N >> 3);  // weight dwords per row
    const int slot = WPL >= 16 ? c : (c & 7);
    const int nh = WPL == 8 ? (c >> 3) : 0;  // nibble half (WPL == 8)
    const int wc_raw = strip * SW + h * WPL + LW * slot;
    // clamped: loads stay in bounds, those columns are not stored (LW == 2: the planner gives it an even NW,
    // so a pair is either whole in the row or wholly past it)
    const int wc = wc_raw <= NW - LW ? wc_raw : NW - LW;
    // rows past M read row M-1: every output row depends only on its own x row, and those rows are not stored
    const int m = rb * 16 + c < M ? rb * 16 + c : M - 1;
    const int k_wave = split * (KW * NKB * 32) + kw * (NKB * 32);

    // buffer resources over this wave's rows: lane offsets in VGPRs, row
    // offsets in SGPRs (no per-load address arithmetic)
    const uint32_t rowbytes = (uint32_t)NW * 4u;
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(static_cast<const char*>(p.w) + (size_t)(uint32_t)k_wave * rowbytes, NKB * 32 * rowbytes);
    const uint32_t w_lane = (uint32_t)(8 * kg) * rowbytes + (uint32_t)wc * 4u;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
    const uint32_t x_lane = ((uint32_t)m * (uint32_t)K + (uint32_t)k_wave + 8u * (uint32_t)kg) * 2u;
    const uint32_t s_lane = (uint32_t)(CPW * wc + 4 * nh) * 2u;

    // Scale/offset of every piece first (small, needed from the first fold
    // on), then the K-blocks as a software pipeline PF blocks deep: block
    // kb+PF is issued right before block kb is consumed, into one of PF+1
    // register slots.  Loads return in order, so consuming block kb waits only
    // for it; keeping few blocks in flight per wave makes each block arrive
    // early instead of every block finishing near the end of the stream.
    typedef typename std::conditional<TPL >= 8, u32x4, u32x2>::type SV;  // 8 (or 4) halves
    constexpr int SVN = TPL >= 8 ? TPL / 8 : 1;
    SV sv[NPIECE][SVN], ov[NPIECE][SVN];
#pragma unroll
    for (int pc = 0; pc < NPIECE; ++pc) {
        const uint32_t g = (uint32_t)(k_wave + pc * PIECE_KB * 32) / (uint32_t)G;
        const size_t goff = (size_t)g * (uint32_t)N * 2u;
#pragma unroll
        for (int v = 0; v < SVN; ++v) {
            const size_t o = goff + s_lane + (size_t)v * sizeof(SV);
            sv[pc][v] = *reinterpret_cast<const SV*>(static_cast<const char*>(p.scale) + o);
            if (HAS_OFF) ov[pc][v] = *reinterpret_cast<const SV*>(static_cast<const char*>(p.offset) + o);
        }
    }
    constexpr int SL = PF + 1;
    uint32_t wv[SL][LW][8];
    u32x4 xa[SL];
    auto issue = [&](int kb) {
        // the scheduler must not interleave blocks: a later block's load moved
        // ahead, or its use moved up, turns the in-order wait into a drain
        __builtin_amdgcn_sched_barrier(0);
        xa[kb % SL] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, x_lane, kb * 64, 0));
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const uint32_t ro = (uint32_t)(kb * 32 + r) * rowbytes;
            if constexpr (LW == 4) {
                const u32x4 d = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, w_lane, ro, 0));
#pragma unroll
                for (int e = 0; e < 4; ++e) wv[kb % SL][e][r] = d[e];
            } else if constexpr (LW == 2) {
                const u32x2 d = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, w_lane, ro, 0));
                wv[kb % SL][0][r] = d[0];
                wv[kb % SL][1][r] = d[1];
            } else {
                wv[kb % SL][0][r] = __builtin_amdgcn_raw_buffer_load_b32(wr, w_lane, ro, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int kb = 0; kb < (PF < NKB ? PF : NKB); ++kb) issue(kb);

    const u32x4 ones = {MM::ONES, MM::ONES, MM::ONES, MM::ONES};
    // per-lane byte selectors: tiles 2i, 2i+1 read byte (2nh + i) of each word
    const uint32_t sel0 = byte_sel(2u * nh), sel1 = byte_sel(2u * nh + 1u);

    f32x4 acc[TPL], ag[TPL], xs;
#pragma unroll
    for (int t = 0; t < TPL; ++t) acc[t] = ag[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    xs = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
        if (kb + PF < NKB) issue(kb + PF);
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 xk = xa[kb % SL];
        const uint32_t* wk = wv[kb % SL][0];
        if constexpr (W8) {  // tile 4d + t: byte t of dword d (column 4 * LW * c + 4d + t)
#pragma unroll
            for (int d = 0; d < LW; ++d)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    ag[4 * d + t] = MM::mma(xk, unpack_i8<DT>(wv[kb % SL][d], t), ag[4 * d + t]);
        } else if constexpr (WPL == 32) {  // tile 8d + 2b + o: nibble 2b + o of dword d (column 16c + 8d + 2b + o)
#pragma unroll
            for (int d = 0; d < 2; ++d)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    ag[8 * d + 2 * b] = MM::mma(xk, unpack_raw<MM::MAGIC, false>(wv[kb % SL][d], byte_sel(b)),
                                                ag[8 * d + 2 * b]);
                    ag[8 * d + 2 * b + 1] = MM::mma(xk, unpack_raw<MM::MAGIC, true>(wv[kb % SL][d], byte_sel(b)),
                                                    ag[8 * d + 2 * b + 1]);
                }
        } else if constexpr (WPL == 16) {
            ag[0] = MM::mma(xk, unpack_raw<MM::MAGIC, false>(wk, byte_sel(0)), ag[0]);
            ag[1] = MM::mma(xk, unpack_raw<MM::MAGIC, true>(wk, byte_sel(0)), ag[1]);
            ag[2] = MM::mma(xk, unpack_raw<MM::MAGIC, false>(wk, byte_sel(1)), ag[2]);
            ag[3] = MM::mma(xk, unpack_raw<MM::MAGIC, true>(wk, byte_sel(1)), ag[3]);
            ag[4] = MM::mma(xk, unpack_raw<MM::MAGIC, false>(wk, byte_sel(2)), ag[4]);
            ag[5] = MM::mma(xk, unpack_raw<MM::MAGIC, true>(wk, byte_sel(2)), ag[5]);
            ag[6] = MM::mma(xk, unpack_raw<MM::MAGIC, false>(wk, byte_sel(3)), ag[6]);
            ag[7] = MM::mma(xk, unpack_raw<MM::MAGIC, true>(wk, byte_sel(3)), ag[7]);
        } else {
            ag[0] = MM::mma(xk, unpack_raw<MM::MAGIC, false>(wk, sel0), ag[0]);
            ag[1] = MM::mma(xk, unpack_raw<MM::MAGIC, true>(wk, sel0), ag[1]);
            ag[2] = MM::mma(xk, unpack_raw<MM::MAGIC, false>(wk, sel1), ag[2]);
            ag[3] = MM::mma(xk, unpack_raw<MM::MAGIC, true>(wk, sel1), ag[3]);
        }
        xs = MM::mma(xk, ones, xs);
        if ((kb + 1) % PIECE_KB == 0) {
            // acc += s*A + s*(offset - BASE)*xs, then a new piece starts
            const int pc = kb / PIECE_KB;
#pragma unroll
            for (int t = 0; t < TPL; ++t) {
                const uint32_t sb = sv[pc][t >> 3][(t & 7) >> 1] >> (16 * (t & 1));
                const float sf = load_half_bits(sb & 0xffffu, p.s_dtype);
                float of = 0.0f;
                if (HAS_OFF) of = load_half_bits((ov[pc][t >> 3][(t & 7) >> 1] >> (16 * (t & 1))) & 0xffffu, p.s_dtype);
                const float sx = sf * (of - BASE);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[t][r] = __builtin_fmaf(sf, ag[t][r], __builtin_fmaf(sx, xs[r], acc[t][r]));
                ag[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
            }
            xs = (f32x4){0.f, 0.f, 0.f, 0.f};
        }
    }

    // lane (c, kg) holds rows 4kg..4kg+3 of columns  LW*CPW*slot + 4*nh + t
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float* dst = &red[wave][4 * kg + r][LW * CPW * slot + 4 * nh];
#pragma unroll
        for (int t = 0; t < TPL; t += 4)
            *reinterpret_cast<f32x4*>(dst + t) = (f32x4){acc[t][r], acc[t + 1][r], acc[t + 2][r], acc[t + 3][r]};
    }
    __syncthreads();

    // each thread finishes 4 consecutive columns of one row, summing the K ranges in order
    constexpr int QUADS = 16 * 256 / 4;
    constexpr int QPT = QUADS / (64 * NWAVE);  // quads per thread
    static_assert(QPT * 64 * NWAVE == QUADS, "every thread finishes the same number of quads");
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(partial, (uint32_t)((int64_t)nsplit * M * N * 4));
    const int n_strip0 = strip * 256;
    f32x4 own[QPT];  // this split's sums, reused if this workgroup finishes the strip
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const int q = threadIdx.x + i * 64 * NWAVE;
        const int row = q >> 6, col = 4 * (q & 63);
        const int hh = col / NCOL, local = col % NCOL;
        f32x4 v = *reinterpret_cast<const f32x4*>(&red[hh][row][local]);
#pragma unroll
        for (int w = 1; w < KW; ++w) v += *reinterpret_cast<const f32x4*>(&red[hh + HALVES * w][row][local]);
        own[i] = v;
        const int mm = rb * 16 + row, n = n_strip0 + col;
        if (mm >= M || n >= N) continue;
        if (FINAL) {
            if (p.bias_dtype) {
#pragma unroll
                for (int t = 0; t < 4; ++t) v[t] += load_scalar(p.bias, n + t, p.bias_dtype);
            }
            u32x2 packed;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const bool bf = p.out_dtype == QK_BF16;
                const uint32_t lo = bf ? f32_to_bf16_bits(v[2 * e]) : f32_to_f16_bits(v[2 * e]);
                const uint32_t hi = bf ? f32_to_bf16_bits(v[2 * e + 1]) : f32_to_f16_bits(v[2 * e + 1]);
                packed[e] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + (int64_t)mm * N + n) = packed;
        } else if (ctr) {  // finished in this kernel by the strip's last split: device-coherent stores
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                                   (uint32_t)(((int64_t)split * M + mm) * N + n) * 4u, 0, kCoherent);
        } else {
            *reinterpret_cast<f32x4*>(partial + ((int64_t)split * M + mm) * N + n) = v;
        }
    }
    // split-K: the last split of this strip to finish adds all splits in split order (deterministic)
    if constexpr (!FINAL) {
        if (ctr == nullptr || !splitk_last(ctr + (int64_t)rb * nstrip + strip, (uint32_t)nsplit, tag)) return;
        uint32_t qoff[QPT];
        bool qok[QPT];
#pragma unroll
        for (int i = 0; i < QPT; ++i) {
            const int q = threadIdx.x + i * 64 * NWAVE;
            const int mm = rb * 16 + (q >> 6), n = n_strip0 + 4 * (q & 63);
            qok[i] = mm < M && n < N;
            qoff[i] = (uint32_t)(qok[i] ? (int64_t)mm * N + n : 0) * 4u;
        }
        // four splits' loads in flight at a time (this split's own sums come from registers), added in
        // split order
        const uint32_t sstride = (uint32_t)((int64_t)M * N * 4);
        f32x4 v[QPT];
        for (int s0 = 0; s0 < nsplit; s0 += 4) {
            f32x4 part[4][QPT];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < QPT; ++i) {
                    if (s0 + j == split)
                        part[j][i] = own[i];
                    else if (s0 + j < nsplit)
                        part[j][i] = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, qoff[i], (uint32_t)(s0 + j) * sstride,
                                                                         kCoherent));
                }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < QPT; ++i)
                    if (s0 + j < nsplit) v[i] = (s0 + j == 0) ? part[j][i] : v[i] + part[j][i];
        }
#pragma unroll
        for (int i = 0; i < QPT; ++i) {
            if (!qok[i]) continue;
            const int q = threadIdx.x + i * 64 * NWAVE;
            const int mm = rb * 16 + (q >> 6), n = n_strip0 + 4 * (q & 63);
            f32x4 w = v[i];
            if (p.bias_dtype) {
#pragma unroll
                for (int t = 0; t < 4; ++t) w[t] += load_scalar(p.bias, n + t, p.bias_dtype);
            }
            u32x2 packed;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const bool bf = p.out_dtype == QK_BF16;
                const uint32_t lo = bf ? f32_to_bf16_bits(w[2 * e]) : f32_to_f16_bits(w[2 * e]);
                const uint32_t hi = bf ? f32_to_bf16_bits(w[2 * e + 1]) : f32_to_f16_bits(w[2 * e + 1]);
                packed[e] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + (int64_t)mm * N + n) = packed;
        }
    }
}

// Sum split partials in split order, add bias, cast; 4 outputs per thread,
// all split loads of a thread issued together (latency-bound at decode sizes).
template <int OUTDT>
__global__ __launch_bounds__(kThreads) void w4_reduce(const float* __restrict__ partial, int nsplit, int64_t M,
                                                      int64_t N, const void* bias, int bias_dtype, void* out) {
    const int64_t total4 = (M * N) >> 2;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total4;
         idx += (int64_t)gridDim.x * kThreads) {
        const f32x4* src = reinterpret_cast<const f32x4*>(partial) + idx;
        f32x4 part[16];
        const int ns = nsplit < 16 ? nsplit : 16;
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < ns) part[s] = src[(int64_t)s * total4];
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < ns) v += part[s];
        for (int s = 16; s < nsplit; ++s) v += src[(int64_t)s * total4];
        const int64_t o = idx * 4, n0 = o % N;
        if (bias_dtype) {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] += load_scalar(bias, n0 + t, bias_dtype);
        }
        u32x2 packed;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t lo = OUTDT == QK_BF16 ? f32_to_bf16_bits(v[2 * e]) : f32_to_f16_bits(v[2 * e]);
            const uint32_t hi = OUTDT == QK_BF16 ? f32_to_bf16_bits(v[2 * e + 1]) : f32_to_f16_bits(v[2 * e + 1]);
            packed[e] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + o) = packed;
    }
}

// ---------------------------------------------------------------------------
// Prefill (large M): a bf16 / fp16 MFMA GEMM on the raw int4 values, with the
// same group-wise algebra as the decode kernels, so the weights are never
// rounded:  for each group g,  A_g = x . (128 + u)  (MFMA on exact magic
// values),  xs_g = x . 1  (one MFMA per row tile against a vector of ones),
// then  acc += s * A_g + s * (offset - BASE) * xs_g.
//
// Tile 256 x 128, 8 waves as 4 (M) x 2 (N), each 64 x 64 (16 MFMA tiles:
// 64 accumulators + 64 group sums + 16 row sums per lane).  A stage holds
// 64 k: x rows and weight columns are both 128-byte LDS rows ([m][k], [n][k])
// with a 16-byte-chunk XOR swizzle; the weight columns also flip row parity in
// odd groups of 8 so the unpacking threads' 8-byte writes are conflict-free.
// A thread unpacks 4 rows x 1 packed word (8 columns): per column two
// v_perm_b32 + two v_bitop3_b32 give 4 k of magic values.  Stage s+1 is
// written to LDS between the two MFMA halves of stage s while stage s+2's
// global loads are in flight.
namespace pf {
constexpr int BM = 256, BN = 128, BK = 64, ROWB = 128;
__device__ __forceinline__ int off(int r, int c) { return r * ROWB + 16 * (c ^ ((r >> 1) & 7)); }
__device__ __forceinline__ int boff(int n, int c) { return (n ^ ((n >> 3) & 1)) * ROWB + 16 * (c ^ ((n >> 1) & 7)); }
}  // namespace pf

// The group sums are folded into the accumulators after G/32 MFMA steps
// (counted at run time) and zeroed for the next group.
// W8: int8 weights [K, N] (W8A16).  Every thread loads one dword (4
// columns) of 4 rows per stage and writes their exact 16-bit values (no
// magic offset, BASE = 0) to the same LDS layout.
template <int DT, bool HAS_OFF, bool FULL, bool W8>
__global__ __launch_bounds__(512) void w4_gemm(WqbmmArgs p, int tiles_m, int tiles_n) {
    typedef Mfma<DT> MM;
    constexpr int NT = 512, BN = pf::BN;
    constexpr int A_BYTES = pf::BM * pf::ROWB, B_BYTES = BN * pf::ROWB, STAGE = A_BYTES + B_BYTES;
    constexpr int TM = 4, TN = 4;           // MFMA tiles per wave (wave tile 64 x 64)
    constexpr int WQ = BN / 8;              // packed words per weight row of the tile (16)
    constexpr int WT = WQ * 16;             // unpacking threads (4 rows each, 64 rows)
    constexpr float BASE = W8 ? 0.0f : MM::BASE;
    constexpr int OROWB = 2 * BN + 16;      // padded output staging row (bytes)
    constexpr int SMEM = 2 * STAGE > pf::BM * OROWB ? 2 * STAGE : pf::BM * OROWB;
    __shared__ __attribute__((aligned(16))) char smem[SMEM];
    // group scale s and s*(offset - BASE) per column, a ring of 4 groups
    // (written with the stage the group starts in, read by its fold)
    __shared__ float sc_s[4][BN], sc_x[4][BN];

    const int bid = xcd_swizzle(blockIdx.x, tiles_m * tiles_n);
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const int grp = bid / per_group;
    const int first_m = grp * GM;
    const int gm = min(tiles_m - first_m, GM);
    const int tm = first_m + (bid % per_group) % gm;
    const int tn = (bid % per_group) / gm;
    const int M = (int)p.M, N = (int)p.N, K = (int)p.K, G = (int)p.group;
    const int m0 = tm * pf::BM, n0 = tn * BN;
    const int NWD = W8 ? (N >> 2) : (N >> 3);  // weight dwords per row

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, g4 = lane >> 4;

    // ---- A (x) loads: 4 x 16 bytes per thread per stage, rows tid/8 + 64i;
    // buffer loads: per-lane offsets in VGPRs, the stage's k offset in an SGPR
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
    uint32_t a_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int r = m0 + tid / 8 + 64 * i;
        if (!FULL) r = r < M ? r : M - 1;  // rows past M are computed and not stored
        a_off[i] = ((uint32_t)r * (uint32_t)K + 8u * (uint32_t)(tid % 8)) * 2u;
    }
    // ---- W loads: threads < WT take word column tid / 16, rows 4 (tid % 16) .. +3
    const bool wthr = W8 || tid < WT;
    const int wcol_l = W8 ? tid / 16 : (tid / 16) % WQ, rg = tid & 15;
    int wcol = n0 / (W8 ? 4 : 8) + wcol_l;
    if (!FULL) wcol = wcol < NWD ? wcol : NWD - 1;
    const uint32_t rowb = (uint32_t)NWD * 4u;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (uint32_t)K * rowb);
    const uint32_t w_off = (uint32_t)(4 * rg) * rowb + (uint32_t)wcol * 4u;
    // LDS byte address of column 8*wcol_l + j, k chunk rg/2, half rg&1 of the
    // weight tile is  wb_base + (KJ(j) ^ wb_x)  with  KJ(j) = 128 j | 16 (j/2)
    // (the pf::boff layout written out so each column costs one v_xad_u32)
    const uint32_t wb_base = 1024u * (uint32_t)wcol_l + 8u * (uint32_t)(rg & 1);
    const uint32_t wb_x = (16u * ((uint32_t)(rg >> 1) ^ (4u * (uint32_t)(wcol_l & 1)))) | (128u * (uint32_t)(wcol_l & 1));
    // scale / offset of the groups that start inside a stage: threads
    // WT .. WT+BN-1 each fetch one column (G = 32 starts two groups per stage)
    const bool sthr = tid >= WT && tid < WT + BN;
    const int scol_l = tid - WT;
    const int scol = n0 + scol_l < N ? n0 + scol_l : N - 1;

    u32x4 ra[4];
    uint32_t rw[4];
    uint32_t rsc0 = 0, rof0 = 0, rsc1 = 0, rof1 = 0;
    // next group start (k) and its index, advanced by gload (no division in the loop);
    // a stage starts at most two groups (G = 32)
    int ld_gk = 0, ld_g = 0;
    int st_g0 = 0, st_n = 0;
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ra[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, a_off[i], (uint32_t)k0 * 2u, 0));
        if (wthr) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                rw[i] = __builtin_amdgcn_raw_buffer_load_b32(wr, w_off, (uint32_t)(k0 + i) * rowb, 0);
        }
        const bool s0 = ld_gk < k0 + pf::BK;
        const bool s1 = s0 && ld_gk + G < k0 + pf::BK;
        if (sthr) {
            const uint16_t* S = static_cast<const uint16_t*>(p.scale);
            const uint16_t* O = static_cast<const uint16_t*>(p.offset);
            if (s0) {
                rsc0 = S[(size_t)ld_g * N + scol];
                if (HAS_OFF) rof0 = O[(size_t)ld_g * N + scol];
            }
            if (s1) {
                rsc1 = S[(size_t)(ld_g + 1) * N + scol];
                if (HAS_OFF) rof1 = O[(size_t)(ld_g + 1) * N + scol];
            }
        }
        st_g0 = ld_g;
        st_n = (int)s0 + (int)s1;
        ld_g += st_n;
        ld_gk += st_n * G;
    };
    auto lstore = [&](int st) {
        char* As = smem + st * STAGE;
        char* Bs = As + A_BYTES;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(As + pf::off(tid / 8 + 64 * i, tid % 8)) = ra[i];
        if (sthr && st_n > 0) {
            const float sf = load_half_bits(rsc0, p.s_dtype);
            const float of = HAS_OFF ? load_half_bits(rof0, p.s_dtype) : 0.0f;
            sc_s[st_g0 & 3][scol_l] = sf;
            sc_x[st_g0 & 3][scol_l] = sf * (of - BASE);
            if (st_n > 1) {
                const float sf1 = load_half_bits(rsc1, p.s_dtype);
                const float of1 = HAS_OFF ? load_half_bits(rof1, p.s_dtype) : 0.0f;
                sc_s[(st_g0 + 1) & 3][scol_l] = sf1;
                sc_x[(st_g0 + 1) & 3][scol_l] = sf1 * (of1 - BASE);
            }
        }
        if constexpr (W8) {
            // columns 4*wcol_l + j, rows 4rg..4rg+3: half (rg & 1) of k chunk rg / 2
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t q[4] = {rw[0], rw[1], rw[2], rw[3]};
                u32x2 v;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float lo = (float)(int8_t)(q[2 * e] >> (8 * j));
                    const float hi = (float)(int8_t)(q[2 * e + 1] >> (8 * j));
                    if constexpr (DT == QK_BF16)
                        v[e] = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
                    else
                        v[e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
                }
                *reinterpret_cast<u32x2*>(Bs + pf::boff(4 * wcol_l + j, rg >> 1) + 8 * (rg & 1)) = v;
            }
        } else if (wthr) {
            const uint32_t mask = __builtin_amdgcn_readfirstlane(0x000f000fu);
            const uint32_t magic = __builtin_amdgcn_readfirstlane(MM::MAGIC | 0x00080008u);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // rows (0,1) and (2,3): byte j/2 of each word, odd nibbles shifted down
                uint32_t p01 = __builtin_amdgcn_perm(rw[1], rw[0], byte_sel(j >> 1));
                uint32_t p23 = __builtin_amdgcn_perm(rw[3], rw[2], byte_sel(j >> 1));
                if (j & 1) {
                    p01 >>= 4;
                    p23 >>= 4;
                }
                const u32x2 v = {(p01 & mask) ^ magic, (p23 & mask) ^ magic};
                constexpr uint32_t kj[8] = {0u, 128u, 256u | 16u, 384u | 16u, 512u | 32u, 640u | 32u, 768u | 48u, 896u | 48u};
                *reinterpret_cast<u32x2*>(Bs + wb_base + (kj[j] ^ wb_x)) = v;
            }
        }
    };

    f32x4 acc[TM][TN], ag[TM][TN], xs[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        xs[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = ag[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    const u32x4 ones = {MM::ONES, MM::ONES, MM::ONES, MM::ONES};
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const int nk = K / pf::BK;
    // acc += s*A + s*(offset - BASE)*xs for group slot `slot`
    auto fold = [&](int slot) {
        float sf[TN], sx[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            sf[j] = sc_s[slot][wn * 64 + 16 * j + fr];
            sx[j] = sc_x[slot][wn * 64 + 16 * j + fr];
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[i][j][r] = __builtin_fmaf(sf[j], ag[i][j][r], __builtin_fmaf(sx[j], xs[i][r], acc[i][j][r]));
    };
    auto frags = [&](const char* As, const char* Bs, int kk, u32x4 (&af)[TM], u32x4 (&bfr)[TN]) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[i] = *reinterpret_cast<const u32x4*>(As + pf::off(wm * 64 + 16 * i + fr, 4 * kk + g4));
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bfr[j] = *reinterpret_cast<const u32x4*>(Bs + pf::boff(wn * 64 + 16 * j + fr, 4 * kk + g4));
    };
    auto mma = [&](const u32x4 (&af)[TM], const u32x4 (&bfr)[TN]) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) ag[i][j] = MM::mma(af[i], bfr[j], ag[i][j]);
            xs[i] = MM::mma(af[i], ones, xs[i]);
        }
    };
    gload(0);
    lstore(0);
    if (nk > 1) gload(pf::BK);
    {
        const int gsub = G / 32;  // 32-k MFMA steps per group
        int sub_left = gsub, fold_g = 0;
        for (int it = 0; it < nk; ++it) {
            __syncthreads();
            const int st = it & 1;
            const char* As = smem + st * STAGE;
            const char* Bs = As + A_BYTES;
            u32x4 af[TM], bfr[TN];
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                frags(As, Bs, kk, af, bfr);
                mma(af, bfr);
                if (kk == 0 && it + 1 < nk) {
                    lstore(st ^ 1);
                    if (it + 2 < nk) gload((it + 2) * pf::BK);
                }
                if (--sub_left == 0) {
                    fold(fold_g & 3);
                    ++fold_g;
                    sub_left = gsub;
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        xs[i] = zero4;
#pragma unroll
                        for (int j = 0; j < TN; ++j) ag[i][j] = zero4;
                    }
                }
            }
        }
    }

    // ---- epilogue: + bias, cast
    float bv[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * 64 + 16 * j + fr;
        bv[j] = (p.bias_dtype && n < N) ? load_scalar(p.bias, n, p.bias_dtype) : 0.0f;
    }
    if constexpr (FULL) {
        __syncthreads();
        uint16_t* ot = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = wm * 64 + 16 * i + 4 * g4 + r;
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const float v = acc[i][j][r] + bv[j];
                    ot[row * (OROWB / 2) + wn * 64 + 16 * j + fr] =
                        (uint16_t)(p.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
                }
            }
        __syncthreads();
        constexpr int CPRO = 2 * BN / 16;
        for (int q = tid; q < pf::BM * CPRO; q += NT) {
            const int row = q / CPRO, c = q % CPRO;
            const u32x4 v = *reinterpret_cast<const u32x4*>(smem + row * OROWB + 16 * c);
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.out) + (size_t)(m0 + row) * N +
                                                                n0 + 8 * c));  // written once
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * 64 + 16 * i + 4 * g4 + r;
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + wn * 64 + 16 * j + fr;
                if (n >= N) continue;
                const float v = acc[i][j][r] + bv[j];
                static_cast<uint16_t*>(p.out)[(size_t)m * N + n] =
                    (uint16_t)(p.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
            }
        }
}

// Group sums of the activations for the prefill kernel: xsum[g][m] =
// sum of x[m][k] over group g, in fp32, k ascending (one thread per (m, g),
// consecutive threads on consecutive rows so the stores are contiguous; the
// group is read 64 elements at a time, eight 16-byte loads in flight).
__global__ __launch_bounds__(kThreads) void w4_xsum(WqbmmArgs p, float* __restrict__ xsum) {
    const int64_t M = p.M, G = p.group, ng = p.K / G;
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= M * ng) return;
    const int64_t g = t / M, m = t - g * M;
    const uint16_t* row = static_cast<const uint16_t*>(p.x) + m * p.K + g * G;
    float s = 0.0f;
    for (int64_t k0 = 0; k0 < G; k0 += 64) {  // G is a multiple of 64 on this path
        u32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const u32x4*>(row + k0 + 8 * j);
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s += load_half_bits(v[j][e] & 0xffffu, p.x_dtype);
                s += load_half_bits(v[j][e] >> 16, p.x_dtype);
            }
    }
    xsum[t] = s;
}

// Prefill on whole tiles (M % 256 == 0, N % 128 == 0, G % 64 == 0): the tile
// and MFMA layout of w4_gemm and its group algebra, with a deeper pipeline
// and the group sums of x taken from w4_xsum instead of a ones-vector MFMA
// (a fifth of w4_gemm's MFMAs).  The activation stages go from HBM straight
// into a ring of three LDS slots by DMA, two stages ahead, with each stage's
// scale / offset rows and group sums; the packed weight words go into
// registers three stages ahead and are unpacked into the LDS weight tile one
// stage ahead.  Waves 4-7 issue the DMAs and count them with their own vmcnt
// waits (asm DMAs are invisible to the compiler's wait counts); waves 0-3
// issue only the register loads, so the compiler's waits before the unpack
// stay exact.
namespace pd {
constexpr int BM = 256, BN = 128, BK = 64, NT = 512, NSX = 3;
constexpr int X_SL = BM * 128;               // x stage [row][128 B] in the pf::off layout (32 KB)
constexpr int B_SL = BN * 128;               // unpacked weight stage in the pf::boff layout (16 KB)
constexpr int SC_SL = 3072;                  // scale row, offset row, group sums of the 256 rows (1 KB DMA each)
constexpr int B_BASE = NSX * X_SL;
constexpr int SC_BASE = B_BASE + 2 * B_SL;
constexpr int RING = SC_BASE + NSX * SC_SL;  // 137 KB
constexpr int OROWB = 2 * BN + 16;           // padded output staging row (bytes)
constexpr int OUT_BYTES = BM * OROWB;
constexpr int SMEM = RING > OUT_BYTES ? RING : OUT_BYTES;
constexpr int LGKM0 = 0xc07f;                // s_waitcnt lgkmcnt(0) alone
}  // namespace pd

template <int DT, bool HAS_OFF, bool W8>
__global__ __launch_bounds__(pd::NT) void w4_dma(WqbmmArgs p, int tiles_m, int tiles_n, const float* __restrict__ xsum) {
    typedef Mfma<DT> MM;
    using namespace pd;
    constexpr int TM = 4, TN = 4;           // MFMA tiles per wave (wave tile 64 x 64)
    constexpr float BASE = W8 ? 0.0f : MM::BASE;
    constexpr int NSC = HAS_OFF ? 3 : 2;    // scale (+ offset) + group-sum DMAs per stage, issued by wave 4
    constexpr int NWL = W8 ? 8 : 4;         // weight loads per thread per stage (waves 0-3)
    __shared__ __attribute__((aligned(1024))) char smem[SMEM];

    const int bid = xcd_swizzle(blockIdx.x, tiles_m * tiles_n);
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const int grp = bid / per_group;
    const int first_m = grp * GM;
    const int gm = min(tiles_m - first_m, GM);
    const int tm = first_m + (bid % per_group) % gm;
    const int tn = (bid % per_group) / gm;
    const int N = (int)p.N, K = (int)p.K, G = (int)p.group;
    const int m0 = tm * BM, n0 = tn * BN;
    const int NWD = W8 ? (N >> 2) : (N >> 3);  // weight dwords per row
    const int nk = K / BK, gst = G / BK;       // stages, stages per group

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, g4 = lane >> 4;
    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;

    // ---- waves 4-7: x rows m0..m0+255, one DMA = rows 8b..8b+7 x 128 B (64 k); lane l -> row 8b + (l>>3),
    // LDS chunk l&7, which holds k chunk (l&7) ^ ((row>>1)&7), and (row>>1)&7 = 4*(b&1) + (l>>4)
    const uint32_t ldx = (uint32_t)K * 2u;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const char*>(p.x) + (size_t)m0 * ldx, (uint32_t)BM * ldx);
    const uint32_t vx0 = (uint32_t)(lane >> 3) * ldx + 16u * (uint32_t)((lane & 7) ^ (lane >> 4));
    const uint32_t vx1 = (uint32_t)(lane >> 3) * ldx + 16u * (uint32_t)((lane & 7) ^ (4 + (lane >> 4)));
    const int xw = wave - 4;  // DMA wave xw issues blocks 8xw .. 8xw+7
    // scale / offset row of a stage's group: lanes 16..63 repeat lanes 0..15 (the first 256 B are used)
    const uint32_t nsb = (uint32_t)(K / G) * (uint32_t)N * 2u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scale, nsb);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(HAS_OFF ? p.offset : p.scale, nsb);
    const uint32_t vsc = (uint32_t)n0 * 2u + 16u * (uint32_t)(lane & 15);
    // group sums xsum[g][m0 .. m0+255]: 1 KB, one DMA
    const __amdgpu_buffer_rsrc_t rxs = make_rsrc(xsum, (uint32_t)(K / G) * (uint32_t)p.M * 4u);
    const uint32_t vxs = ((uint32_t)m0 + 4u * (uint32_t)lane) * 4u;
    int sc_g = 0, sc_left = gst;  // group of the next stage whose scale rows go out
    // stage s into slot s % 3 (past the end: the last stage again, into a slot no wave reads)
    auto issue_x = [&](int s) {
        const int sl = s < nk ? s : nk - 1;
        const uint32_t k2 = (uint32_t)sl * (uint32_t)(BK * 2);
        const uint32_t dst = sbase + (uint32_t)(s % NSX) * X_SL;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int b = 8 * xw + j;
            dma16(rx, dst + (uint32_t)b * 1024u, (j & 1) ? vx1 : vx0, (uint32_t)(8 * b) * ldx + k2);
        }
        if (wave == 4) {
            const uint32_t sdst = sbase + SC_BASE + (uint32_t)(s % NSX) * SC_SL;
            const uint32_t goff = (uint32_t)sc_g * (uint32_t)N * 2u;
            dma16(rs, sdst, vsc, goff);
            if (HAS_OFF) dma16(ro, sdst + 1024u, vsc, goff);
            dma16(rxs, sdst + 2048u, vxs, (uint32_t)sc_g * (uint32_t)p.M * 4u);
            if (s < nk - 1 && --sc_left == 0) {
                ++sc_g;
                sc_left = gst;
            }
        }
    };

    // ---- waves 0-3: packed words; thread t takes word column (t>>4)&15 (and +16 for int8 weights), rows
    // 4(t&15) .. +3 of the stage
    const int wcol_l = (tid >> 4) & 15, rg = tid & 15;
    const uint32_t rowb = (uint32_t)NWD * 4u;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (uint32_t)K * rowb);
    const uint32_t w_off = (uint32_t)(4 * rg) * rowb + (uint32_t)(n0 / (W8 ? 4 : 8) + wcol_l) * 4u;
    uint32_t rw[3][NWL];
    auto issue_w = [&](int s, uint32_t(&r)[NWL]) {
        const uint32_t k0 = (uint32_t)(s < nk ? s : nk - 1) * (uint32_t)BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = __builtin_amdgcn_raw_buffer_load_b32(wr, w_off, (k0 + i) * rowb, 0);
        if constexpr (W8) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                r[4 + i] = __builtin_amdgcn_raw_buffer_load_b32(wr, w_off + 64u, (k0 + i) * rowb, 0);
        }
    };
    // LDS byte address of column 8*wcol_l + j, k chunk rg/2, half rg&1 of the weight tile (int4) is
    // wb_base + (KJ(j) ^ wb_x) with KJ(j) = 128 j | 16 (j/2): the pf::boff layout written out
    const uint32_t wb_base = 1024u * (uint32_t)wcol_l + 8u * (uint32_t)(rg & 1);
    const uint32_t wb_x = (16u * ((uint32_t)(rg >> 1) ^ (4u * (uint32_t)(wcol_l & 1)))) | (128u * (uint32_t)(wcol_l & 1));
    auto unpack = [&](const uint32_t(&r)[NWL], char* Bs) {
        if constexpr (W8) {
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int wc = wcol_l + 16 * hf;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    u32x2 v;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float lo = (float)(int8_t)(r[4 * hf + 2 * e] >> (8 * j));
                        const float hi = (float)(int8_t)(r[4 * hf + 2 * e + 1] >> (8 * j));
                        if constexpr (DT == QK_BF16)
                            v[e] = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
                        else
                            v[e] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
                    }
                    *reinterpret_cast<u32x2*>(Bs + pf::boff(4 * wc + j, rg >> 1) + 8 * (rg & 1)) = v;
                }
            }
        } else {
            const uint32_t mask = __builtin_amdgcn_readfirstlane(0x000f000fu);
            const uint32_t magic = __builtin_amdgcn_readfirstlane(MM::MAGIC | 0x00080008u);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // rows (0,1) and (2,3): byte j/2 of each word, odd nibbles shifted down
                uint32_t p01 = __builtin_amdgcn_perm(r[1], r[0], byte_sel(j >> 1));
                uint32_t p23 = __builtin_amdgcn_perm(r[3], r[2], byte_sel(j >> 1));
                if (j & 1) {
                    p01 >>= 4;
                    p23 >>= 4;
                }
                const u32x2 v = {(p01 & mask) ^ magic, (p23 & mask) ^ magic};
                constexpr uint32_t kj[8] = {0u, 128u, 256u | 16u, 384u | 16u, 512u | 32u, 640u | 32u, 768u | 48u, 896u | 48u};
                *reinterpret_cast<u32x2*>(Bs + wb_base + (kj[j] ^ wb_x)) = v;
            }
        }
    };

    f32x4 acc[TM][TN], ag[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = ag[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    // acc += s*A + s*(offset - BASE)*xsum with the group's rows from scale slot `slot`
    auto fold = [&](int slot) {
        const char* sc = smem + SC_BASE + slot * SC_SL;
        f32x4 xs[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) xs[i] = *reinterpret_cast<const f32x4*>(sc + 2048 + 4 * (wm * 64 + 16 * i + 4 * g4));
        float sf[TN], sx[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = wn * 64 + 16 * j + fr;
            sf[j] = load_half_bits(*reinterpret_cast<const uint16_t*>(sc + 2 * col), p.s_dtype);
            const float of = HAS_OFF ? load_half_bits(*reinterpret_cast<const uint16_t*>(sc + 1024 + 2 * col), p.s_dtype)
                                     : 0.0f;
            sx[j] = sf[j] * (of - BASE);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[i][j][r] = __builtin_fmaf(sf[j], ag[i][j][r], __builtin_fmaf(sx[j], xs[i][r], acc[i][j][r]));
    };
    auto mma_step = [&](const char* As, const char* Bs, int kk) {
        u32x4 af[TM], bfr[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[i] = *reinterpret_cast<const u32x4*>(As + pf::off(wm * 64 + 16 * i + fr, 4 * kk + g4));
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bfr[j] = *reinterpret_cast<const u32x4*>(Bs + pf::boff(wn * 64 + 16 * j + fr, 4 * kk + g4));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) ag[i][j] = MM::mma(af[i], bfr[j], ag[i][j]);
    };

    // Stage i reads x slot i % 3, scale slot i % 3 and weight buffer i & 1.  Iteration i issues x stage i+2
    // (into the slot stage i-1 read) and weight words of stage i+3 (into the registers stage i's words
    // left), and unpacks stage i+1 (into the buffer stage i-1 read); one barrier per stage.  A DMA wave
    // waits, before that barrier, for all but the DMAs it issued in iteration i-1, which lands stage i.
    // The two kinds of wave run loops of their own (same barriers, same order): a branch inside one loop
    // would merge a path without the weight loads into the compiler's wait counts, and it would then wait
    // for every load before each unpack.
    int left = gst;
    auto stage_mma = [&](int i, int u) {
        const char* As = smem + u * X_SL;
        const char* Bs = smem + B_BASE + (i & 1) * B_SL;
        mma_step(As, Bs, 0);
        return Bs;
    };
    auto stage_end = [&](int i, int u) {
        const char* As = smem + u * X_SL;
        const char* Bs = smem + B_BASE + (i & 1) * B_SL;
        mma_step(As, Bs, 1);
        if (--left == 0) {
            fold(u);
            left = gst;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) ag[a][b] = zero4;
        }
    };
    auto bar = [&]() {
        __builtin_amdgcn_s_waitcnt(LGKM0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    };
    // whole triples of stages in the loop, the last one or two after it: an exit from inside the loop body
    // becomes (after the compiler restructures it) a path back to the loop head that skips loads, and the
    // compiler's waits then count too few loads in flight
    const int nk3 = nk - nk % 3;
    if (wave < 4) {
        auto w_stage = [&](int i, int u) {
            bar();
            issue_w(i + 3, rw[u]);
            __builtin_amdgcn_sched_barrier(0);
            stage_mma(i, u);
            // unconditional (past the last stage it fills a buffer no stage reads)
            unpack(rw[(u + 1) % 3], smem + B_BASE + ((i + 1) & 1) * B_SL);
            stage_end(i, u);
        };
        // in stage order (interleaved stages would make the loop's first waits count too few loads)
        issue_w(0, rw[0]);
        __builtin_amdgcn_sched_barrier(0);
        issue_w(1, rw[1]);
        __builtin_amdgcn_sched_barrier(0);
        issue_w(2, rw[2]);
        __builtin_amdgcn_sched_barrier(0);
        unpack(rw[0], smem + B_BASE);
        for (int i0 = 0; i0 < nk3; i0 += 3) {
#pragma unroll
            for (int u = 0; u < 3; ++u) w_stage(i0 + u, u);
        }
        if (nk3 < nk) w_stage(nk3, 0);
        if (nk3 + 1 < nk) w_stage(nk3 + 1, 1);
    } else {
        auto x_stage = [&](int i, int u) {
            if (wave == 4)
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(8 + NSC));
            else
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
            bar();
            issue_x(i + 2);
            stage_mma(i, u);
            stage_end(i, u);
        };
        issue_x(0);
        issue_x(1);
        for (int i0 = 0; i0 < nk3; i0 += 3) {
#pragma unroll
            for (int u = 0; u < 3; ++u) x_stage(i0 + u, u);
        }
        if (nk3 < nk) x_stage(nk3, 0);
        if (nk3 + 1 < nk) x_stage(nk3 + 1, 1);
    }
    // the trailing loads (past the last stage) land before the LDS is reused
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();

    // ---- epilogue: + bias, cast, staged through LDS for 16-byte row stores
    float bv[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * 64 + 16 * j + fr;
        bv[j] = p.bias_dtype ? load_scalar(p.bias, n, p.bias_dtype) : 0.0f;
    }
    uint16_t* ot = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = wm * 64 + 16 * i + 4 * g4 + r;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const float v = acc[i][j][r] + bv[j];
                ot[row * (OROWB / 2) + wn * 64 + 16 * j + fr] =
                    (uint16_t)(p.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
            }
        }
    __syncthreads();
    constexpr int CPRO = 2 * BN / 16;
    for (int q = tid; q < BM * CPRO; q += NT) {
        const int row = q / CPRO, c = q % CPRO;
        const u32x4 v = *reinterpret_cast<const u32x4*>(smem + row * OROWB + 16 * c);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.out) + (size_t)(m0 + row) * N +
                                                                n0 + 8 * c));  // written once
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

// ---------------------------------------------------------------- host-side planning

struct DecodePlan {
    bool ok;
    bool upfront;
    int nsplit, nstrip, nrb;
    int piece_kb;
};

// The decode kernel's preconditions and its split count; used by both the
// workspace query and the launch so the two always agree.
DecodePlan decode_plan(const WqbmmArgs& p) {
    DecodePlan d{false, false, 1, 0, 0, 4};
    const int64_t G = p.group == 0 ? p.K : p.group;
    if (p.w_dtype != QK_I32 || p.K <= 0 || p.N <= 0 || p.M <= 0) return d;
    if (p.K % (2 * CHUNK) != 0 || G <= 0 || p.K % G != 0) return d;
    if (!(G % CHUNK == 0 || G == 32 || G == 64)) return d;
    // 32-bit offsets inside the kernel
    if (p.K * (p.N / 2) >= ((int64_t)1 << 31) || p.M * p.K * 2 >= ((int64_t)1 << 31) ||
        (p.K / G) * p.N * 2 >= ((int64_t)1 << 31))
        return d;
    if (((uintptr_t)p.x | (uintptr_t)p.scale | (uintptr_t)p.out) % 16 != 0 || (uintptr_t)p.w % 4 != 0 ||
        (p.offset && (uintptr_t)p.offset % 16 != 0))
        return d;
    d.piece_kb = G >= CHUNK ? 4 : (int)(G / 32);
    d.nstrip = (int)((p.N / 8 + STRIP - 1) / STRIP);
    d.nrb = (int)((p.M + 15) / 16);
    const int64_t tiles = (int64_t)d.nstrip * d.nrb;
    int s = 1;
    if (tiles < 256) {
        // few output tiles (decode): split K so every wave owns 256 rows and
        // issues all its loads at once; otherwise keep doubling splits while
        // workgroups are short of ~2 per CU
        if (p.K % 512 == 0 && (p.K / 512) * tiles <= 4096 && (p.N / 8) % 4 == 0 && d.piece_kb != 1) {
            s = (int)(p.K / 512);
            d.upfront = true;
        } else {
            const int64_t want = 512 / tiles;
            while (s * 2 <= want && p.K % ((int64_t)(s * 2) * 2 * CHUNK) == 0) s *= 2;
        }
    }
    if (const int f = plan_override().w4_splits) {  // debug override
        if (p.K % ((int64_t)f * 2 * CHUNK) == 0) {
            s = f;
            d.upfront = p.K / f == 512 && (p.N / 8) % 4 == 0;
        }
    }
    // partial sums stay a small fraction of the weight stream
    if (s > 1 && (int64_t)s * p.M * p.N * 4 > ((int64_t)256 << 20)) {
        s = 1;
        d.upfront = false;
    }
    d.nsplit = s;
    d.ok = tiles * d.nsplit < ((int64_t)1 << 31);
    return d;
}

template <int DT, int PKB, bool HAS_OFF>
hipError_t launch_decode_t(const WqbmmArgs& p, const DecodePlan& d, float* partial, hipStream_t stream) {
    const dim3 grid((uint32_t)((int64_t)d.nstrip * d.nsplit * d.nrb));
    if (d.nsplit == 1)
        w4_decode<DT, PKB, HAS_OFF, true, false><<<grid, dim3(kThreads), 0, stream>>>(p, partial, 1, d.nstrip);
    else if (PKB != 1 && d.upfront)  // 32-row groups hold 8 scale pieces per wave up front: too many registers
        w4_decode<DT, PKB != 1 ? PKB : 2, HAS_OFF, false, true><<<grid, dim3(kThreads), 0, stream>>>(p, partial, d.nsplit,
                                                                                                      d.nstrip);
    else
        w4_decode<DT, PKB, HAS_OFF, false, false><<<grid, dim3(kThreads), 0, stream>>>(p, partial, d.nsplit, d.nstrip);
    return hipGetLastError();
}

template <int DT>
hipError_t launch_decode_dt(const WqbmmArgs& p, const DecodePlan& d, float* partial, hipStream_t stream) {
    const bool off = p.offset != nullptr;
    switch (d.piece_kb) {
    case 1: return off ? launch_decode_t<DT, 1, true>(p, d, partial, stream) : launch_decode_t<DT, 1, false>(p, d, partial, stream);
    case 2: return off ? launch_decode_t<DT, 2, true>(p, d, partial, stream) : launch_decode_t<DT, 2, false>(p, d, partial, stream);
    default: return off ? launch_decode_t<DT, 4, true>(p, d, partial, stream) : launch_decode_t<DT, 4, false>(p, d, partial, stream);
    }
}

// Stream kernel plan (M <= 16): a strip of 256 columns per workgroup of `nwave` waves, each wave `wpl` words
// wide, 128 rows of K per wave, K split into nsplit workgroup ranges.
struct StreamPlan {
    bool ok;
    int wpl, nwave, nkb, pf, nsplit, nstrip, piece_kb;
};

StreamPlan stream_plan(const WqbmmArgs& p) {
    StreamPlan s{false, 16, 8, 4, 2, 1, 0, 4};
    const int64_t G = p.group == 0 ? p.K : p.group;
    const bool w8 = p.w_dtype == QK_I8;
    if (!(p.w_dtype == QK_I32 || (w8 && p.N % 4 == 0)) || p.M <= 0 || p.M > 16 || p.N <= 0 || p.K <= 0) return s;
    if (G <= 0 || p.K % G != 0 || !(G % 128 == 0 || G == 32 || G == 64)) return s;
    if (p.K * (w8 ? p.N : p.N / 2) >= ((int64_t)1 << 31) || p.M * p.K * 2 >= ((int64_t)1 << 31) ||
        (p.K / G) * p.N * 2 >= ((int64_t)1 << 31))
        return s;
    if (((uintptr_t)p.x | (uintptr_t)p.scale) % 16 != 0 || (uintptr_t)p.out % 8 != 0 || (uintptr_t)p.w % 4 != 0 ||
        (p.offset && (uintptr_t)p.offset % 16 != 0))
        return s;
    s.piece_kb = G >= 128 ? 4 : (int)(G / 32);
    s.wpl = 16;
    s.nwave = 16;
    s.nkb = 4;
    s.pf = 2;
    const PlanOverride& ov = plan_override();  // debug override: a stream shape, or no stream kernel
    if (ov.w4_stream_off) return s;
    if (ov.w4_stream_nwave) {
        s.nwave = ov.w4_stream_nwave;
        s.nkb = ov.w4_stream_nkb;
        s.pf = ov.w4_stream_pf;
    }
    if (s.piece_kb != 4) {  // short groups: one instantiated shape, 8 waves (16 would spill their scales)
        s.nwave = 8;
        s.nkb = 4;
        s.pf = 2;
    }
    if (w8) {
        // int8 weights: 8-wave strips in which each lane loads 4 (whole 256-byte rows per wave) or 2 (half
        // rows) adjacent dwords, where groups are whole 128-row pieces; else 16-wave quarter-row strips.
        // cfg3's shape with int8 weights, M = 16 / 1: 19.9 / 17.4 us quarter rows, 18.5 / 16.2 half rows,
        // 14.8 / 13.5 whole rows; K = 8192, N = 28672, M = 16 / 1: 81 / 65.5, 66 / 51.5, 66 / 58.4 us.  Whole
        // rows (1024 K rows per workgroup, one workgroup per CU by its LDS) while at most 512 workgroups run.
        s.nwave = 16;
        s.nkb = 4;
        s.pf = 2;
        int wpl = ov.w4_stream_wpl;
        if (wpl == 0 && s.piece_kb == 4) {
            const int64_t strips = (p.N + 255) / 256;
            if (p.N % 16 == 0 && p.K % 1024 == 0 && strips * (p.K / 1024) <= 512) wpl = 64;
            else if (p.N % 8 == 0 && p.K % 512 == 0) wpl = 32;
        }
        if (s.piece_kb == 4 && (wpl == 32 || wpl == 64) && p.N % (wpl / 4) == 0) {
            s.wpl = wpl;
            s.nwave = 8;
        }
    } else if (s.piece_kb == 4 && p.N % 16 == 0 &&
               (ov.w4_stream_wpl == 32 || (ov.w4_stream_wpl == 0 && !ov.w4_stream_nwave && p.M > 4))) {
        // whole 128-byte rows per wave (8-wave strips): cfg3 M=16 12.3 -> 11.8 us, K=8192 N=28672 M=16
        // 49.2 -> 47.2 us; at M=1 10.3 -> 10.45 us, so few rows keep the 16-wave half-line strips.  An even
        // word count per row keeps every lane's 8-byte pair inside the row (a clamped pair is all columns
        // past N, which are not stored).
        s.wpl = 32;
        s.nwave = 8;
        s.nkb = 4;
        s.pf = ov.w4_stream_pf == 3 ? 3 : 2;
    }
    const int halves = (w8 ? 64 : 32) / s.wpl;
    int kw = s.nwave / halves;
    const int rows = s.nkb * 32;
    while (kw > 1 && p.K % (kw * rows) != 0) kw >>= 1;  // fewer K ranges when K is short
    if (p.K % (kw * rows) != 0) return s;
    s.nwave = kw * halves;
    if (s.nwave != 8 && s.nwave != 16) return s;  // the instantiated shapes
    if (w8 && s.nwave != (s.wpl == 16 ? 16 : 8)) return s;
    s.nsplit = (int)(p.K / (kw * rows));
    s.nstrip = (int)((p.N + 255) / 256);
    if (s.nsplit > 1 && (int64_t)s.nsplit * p.M * p.N * 4 > ((int64_t)256 << 20)) return s;
    s.ok = (int64_t)s.nstrip * s.nsplit < ((int64_t)1 << 31);
    return s;
}

template <int DT, int NWAVE, int NKB, int PF, int PKB, bool HAS_OFF, bool W8, int WPL = 16>
hipError_t launch_stream_t(const WqbmmArgs& p, const StreamPlan& s, float* partial, uint64_t* ctr,
                           hipStream_t stream) {
    const dim3 grid((uint32_t)((int64_t)s.nstrip * s.nsplit));
    if (s.nsplit == 1)
        w4_stream<DT, WPL, NWAVE, NKB, PF, PKB, HAS_OFF, true, W8><<<grid, dim3(64 * NWAVE), 0, stream>>>(
            p, partial, s.nstrip, 1, nullptr, 0);
    else
        w4_stream<DT, WPL, NWAVE, NKB, PF, PKB, HAS_OFF, false, W8><<<grid, dim3(64 * NWAVE), 0, stream>>>(
            p, partial, s.nstrip, s.nsplit, ctr, ctr ? next_split_tag() : 0);
    return hipGetLastError();
}

template <int DT, int NWAVE, bool HAS_OFF>
hipError_t launch_stream_w(const WqbmmArgs& p, const StreamPlan& s, float* partial, uint64_t* ctr,
                           hipStream_t stream) {
    if (p.w_dtype == QK_I8) {  // int8 weights: the default shape, or 8-wave strips of wider rows per wave
        if constexpr (NWAVE == 16) {
            switch (s.piece_kb) {
            case 1: return launch_stream_t<DT, 16, 4, 2, 1, HAS_OFF, true>(p, s, partial, ctr, stream);
            case 2: return launch_stream_t<DT, 16, 4, 2, 2, HAS_OFF, true>(p, s, partial, ctr, stream);
            default: return launch_stream_t<DT, 16, 4, 2, 4, HAS_OFF, true>(p, s, partial, ctr, stream);
            }
        } else {
            if (s.piece_kb == 4 && s.wpl == 64) return launch_stream_t<DT, 8, 4, 2, 4, HAS_OFF, true, 64>(p, s, partial, ctr, stream);
            if (s.piece_kb == 4 && s.wpl == 32) return launch_stream_t<DT, 8, 4, 2, 4, HAS_OFF, true, 32>(p, s, partial, ctr, stream);
        }
        return hipErrorInvalidValue;
    }
    if constexpr (NWAVE == 8) {  // short groups and 8-row-block waves run 8-wave strips only (16 would spill)
        if (s.wpl == 32 && s.piece_kb == 4 && s.nkb == 4)  // whole-line rows per wave
            return s.pf == 3 ? launch_stream_t<DT, 8, 4, 3, 4, HAS_OFF, false, 32>(p, s, partial, ctr, stream)
                             : launch_stream_t<DT, 8, 4, 2, 4, HAS_OFF, false, 32>(p, s, partial, ctr, stream);
        switch (s.piece_kb) {
        case 1: return launch_stream_t<DT, 8, 4, 2, 1, HAS_OFF, false>(p, s, partial, ctr, stream);
        case 2: return launch_stream_t<DT, 8, 4, 2, 2, HAS_OFF, false>(p, s, partial, ctr, stream);
        default: break;
        }
        if (s.nkb == 8)
            return s.pf == 3 ? launch_stream_t<DT, 8, 8, 3, 4, HAS_OFF, false>(p, s, partial, ctr, stream)
                             : launch_stream_t<DT, 8, 8, 2, 4, HAS_OFF, false>(p, s, partial, ctr, stream);
    } else if (s.piece_kb != 4 || s.nkb != 4) {
        return hipErrorInvalidValue;  // not planned (stream_plan gives these shapes 8 waves)
    }
    return s.pf == 4 ? launch_stream_t<DT, NWAVE, 4, 4, 4, HAS_OFF, false>(p, s, partial, ctr, stream)
                     : launch_stream_t<DT, NWAVE, 4, 2, 4, HAS_OFF, false>(p, s, partial, ctr, stream);
}

template <int DT>
hipError_t launch_stream_dt(const WqbmmArgs& p, const StreamPlan& s, float* partial, uint64_t* ctr,
                            hipStream_t stream) {
    const bool off = p.offset != nullptr;
    if (s.nwave == 8)
        return off ? launch_stream_w<DT, 8, true>(p, s, partial, ctr, stream)
                   : launch_stream_w<DT, 8, false>(p, s, partial, ctr, stream);
    return off ? launch_stream_w<DT, 16, true>(p, s, partial, ctr, stream)
               : launch_stream_w<DT, 16, false>(p, s, partial, ctr, stream);
}

// Prefill plan: large M, int4 weights, K a multiple of the 64-row stage and
// G a multiple of the 32-row MFMA step.
struct GemmPlan {
    bool ok, full, dma;
    int tiles_m, tiles_n;
};

GemmPlan gemm_plan(const WqbmmArgs& p, bool any_tiles = false) {
    GemmPlan g{false, false, false, 0, 0};
    const int64_t G = p.group == 0 ? p.K : p.group;
    const bool w8 = p.w_dtype == QK_I8;
    if (!(p.w_dtype == QK_I32 || (w8 && p.N % 4 == 0)) || p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % 64 != 0)
        return g;
    if (G <= 0 || p.K % G != 0 || G % 32 != 0) return g;
    if (p.M * p.K * 2 >= ((int64_t)1 << 31) || p.K * (w8 ? p.N : p.N / 2) >= ((int64_t)1 << 31) ||
        (p.K / G) * p.N >= ((int64_t)1 << 31) || p.M * p.N >= ((int64_t)1 << 31))
        return g;
    if (((uintptr_t)p.x | (uintptr_t)p.out) % 16 != 0 || (uintptr_t)p.w % 4 != 0) return g;
    g.tiles_m = (int)((p.M + 255) / 256);
    g.tiles_n = (int)((p.N + 127) / 128);
    // debug override: "force" (even with few tiles), "nodma" (register-staged kernel only) or "off"
    const int force = plan_override().w4_gemm;
    if (force == 3) return g;
    const bool forced = force == 1;
    // too few tiles: the decode kernels stream an int4 weight better (they take no int8 weight)
    if (!forced && !any_tiles && !w8 && (int64_t)g.tiles_m * g.tiles_n < 128) return g;
    g.full = p.M % 256 == 0 && p.N % 128 == 0;
    // the DMA pipeline: whole tiles, whole 64-row stages per group, 16-byte aligned scale / offset rows
    g.dma = g.full && G % 64 == 0 && ((uintptr_t)p.scale | (uintptr_t)(p.offset ? p.offset : p.scale)) % 16 == 0 &&
            force != 2;
    g.ok = true;
    return g;
}

template <int DT, bool OFF>
hipError_t launch_gemm_t(const WqbmmArgs& p, const GemmPlan& g, float* xsum, hipStream_t stream) {
    const dim3 grid((uint32_t)(g.tiles_m * g.tiles_n));
    if (g.dma) {
        const int64_t sums = p.M * (p.K / p.group);
        w4_xsum<<<dim3((uint32_t)((sums + kThreads - 1) / kThreads)), dim3(kThreads), 0, stream>>>(p, xsum);
        if (p.w_dtype == QK_I8) w4_dma<DT, OFF, true><<<grid, dim3(pd::NT), 0, stream>>>(p, g.tiles_m, g.tiles_n, xsum);
        else w4_dma<DT, OFF, false><<<grid, dim3(pd::NT), 0, stream>>>(p, g.tiles_m, g.tiles_n, xsum);
    } else if (p.w_dtype == QK_I8) {
        if (g.full) w4_gemm<DT, OFF, true, true><<<grid, dim3(512), 0, stream>>>(p, g.tiles_m, g.tiles_n);
        else w4_gemm<DT, OFF, false, true><<<grid, dim3(512), 0, stream>>>(p, g.tiles_m, g.tiles_n);
    } else if (g.full) {
        w4_gemm<DT, OFF, true, false><<<grid, dim3(512), 0, stream>>>(p, g.tiles_m, g.tiles_n);
    } else {
        w4_gemm<DT, OFF, false, false><<<grid, dim3(512), 0, stream>>>(p, g.tiles_m, g.tiles_n);
    }
    return hipGetLastError();
}

template <int DT>
hipError_t launch_gemm_dt(const WqbmmArgs& p, const GemmPlan& g, float* xsum, hipStream_t stream) {
    return p.offset != nullptr ? launch_gemm_t<DT, true>(p, g, xsum, stream) : launch_gemm_t<DT, false>(p, g, xsum, stream);
}

// workspace of the DMA prefill kernel: [split counters, unused][group sums fp32 [K/G][M]]
size_t gemm_dma_workspace(const WqbmmArgs& p) {
    return QK_SPLIT_COUNTER_BYTES + (size_t)(p.K / p.group) * (size_t)p.M * sizeof(float);
}

template <int OUTDT>
hipError_t launch_reduce(const WqbmmArgs& p, int nsplit, const float* partial, hipStream_t stream) {
    const int64_t total = p.M * p.N / 4;
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    w4_reduce<OUTDT><<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(partial, nsplit, p.M, p.N, p.bias,
                                                                           p.bias_dtype, p.out);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_w4_xsum(const WqbmmArgs& p, float* xsum, hipStream_t stream) {
    const int64_t sums = p.M * (p.K / p.group);
    w4_xsum<<<dim3((uint32_t)((sums + kThreads - 1) / kThreads)), dim3(kThreads), 0, stream>>>(p, xsum);
    return hipGetLastError();
}

// An int8 row-major weight with 16 < M <= 128 (where no cast plan runs): the decode stream on slices of 16 rows,
// one launch each (cfg3's shape: ~16 us per slice, against ~130 us for the register-staged prefill kernel on one
// 256-row tile).  The slice of row r0 is the call with x and out advanced by r0 rows.  Returns the workspace the
// slices need (the larger of the full and the last slice's plan), or -1 where the slices do not apply.
constexpr int64_t kW8SliceRows = 16, kW8SliceMaxM = 128;

WqbmmArgs w8_slice(const WqbmmArgs& p, int64_t r0) {
    WqbmmArgs q = p;
    const int xs = 2, os = 2;  // 16-bit activations and outputs
    q.x = static_cast<const char*>(p.x) + r0 * p.K * xs;
    q.out = static_cast<char*>(p.out) + r0 * p.N * os;
    q.M = p.M - r0 < kW8SliceRows ? p.M - r0 : kW8SliceRows;
    return q;
}

int64_t w8_slices_workspace(const WqbmmArgs& p) {
    if (p.w_dtype != QK_I8 || p.M <= kW8SliceRows || p.M > kW8SliceMaxM || plan_override().w4_gemm != 0) return -1;
    int64_t need = 0;
    for (int64_t r0 : {(int64_t)0, (p.M - 1) / kW8SliceRows * kW8SliceRows}) {
        const StreamPlan s = stream_plan(w8_slice(p, r0));
        if (!s.ok) return -1;
        const int64_t rows = w8_slice(p, r0).M;
        const int64_t w = s.nsplit == 1 ? 0 : QK_SPLIT_COUNTER_BYTES + (int64_t)s.nsplit * rows * p.N * (int64_t)sizeof(float);
        if (w > need) need = w;
    }
    return need;
}

size_t weight_quant_bmm_workspace(int64_t M, int64_t N, int64_t K, int w_dtype, int64_t group, int level) {
    WqbmmArgs p{};
    p.M = M;
    p.N = N;
    p.K = K;
    p.w_dtype = w_dtype;
    p.group = group;
    // alignment does not change the split count; use aligned dummies
    p.x = p.scale = p.offset = p.out = (void*)(uintptr_t)256;
    p.w = (void*)(uintptr_t)256;
    if (p.group == 0) p.group = p.K;
    if (w_dtype == QK_I4_NZ || w_dtype == QK_I8_NZ || w_dtype == QK_I8_NK) return w4_nz_workspace(p, level == kWsFull);
    if (level != kWsNoCast)
        if (const size_t c = w4_cast_nz_workspace(p, level == kWsFull)) return c;
    if (const int64_t sl = w8_slices_workspace(p); sl >= 0) return (size_t)sl;
    // [split-K counters][fp32 partials [nsplit][M][N]]
    const StreamPlan s = stream_plan(p);
    if (s.ok) return s.nsplit == 1 ? 0 : QK_SPLIT_COUNTER_BYTES + (size_t)s.nsplit * (size_t)M * (size_t)N * sizeof(float);
    const GemmPlan gp = gemm_plan(p);
    if (gp.ok) return gp.dma ? gemm_dma_workspace(p) : 0;
    const DecodePlan d = decode_plan(p);
    if (!d.ok || d.nsplit == 1) return 0;
    return QK_SPLIT_COUNTER_BYTES + (size_t)d.nsplit * (size_t)M * (size_t)N * sizeof(float);
}

hipError_t launch_weight_quant_bmm(const WqbmmArgs& a, void* workspace, size_t ws_bytes, hipStream_t stream) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    WqbmmArgs p = a;
    if (p.group == 0) p.group = p.K;  // per channel == one group spanning K
    if (p.w_dtype == QK_I4_NZ || p.w_dtype == QK_I8_NZ || p.w_dtype == QK_I8_NK)
        return launch_w4_nz_bmm(p, workspace, ws_bytes, stream);
    // a split workspace is [counters][partials]: the stream kernel finishes each strip in its last
    // split's workgroup (one counter per strip); the decode kernel uses the reduce kernel
    char* ws = static_cast<char*>(workspace);
    float* partial = ws ? reinterpret_cast<float*>(ws + QK_SPLIT_COUNTER_BYTES) : nullptr;
    const StreamPlan sp = stream_plan(p);
    if (sp.ok) {
        if (sp.nsplit > 1 && (!ws || ws_bytes < QK_SPLIT_COUNTER_BYTES + (size_t)sp.nsplit * p.M * p.N * sizeof(float) ||
                              (uintptr_t)ws % 256 != 0))
            return hipErrorInvalidValue;
        // one 64-bit tagged counter per strip (no initialisation needed); more strips than the
        // counter area holds, or more splits than the count field holds, take the reduce kernel
        uint64_t* ctr = (sp.nsplit > 1 && (size_t)sp.nstrip * 8 <= QK_SPLIT_COUNTER_BYTES &&
                         sp.nsplit < (1 << kSplitCountBits))
                            ? reinterpret_cast<uint64_t*>(ws) : nullptr;
        hipError_t e = p.x_dtype == QK_BF16 ? launch_stream_dt<QK_BF16>(p, sp, partial, ctr, stream)
                                            : launch_stream_dt<QK_F16>(p, sp, partial, ctr, stream);
        if (e != hipSuccess || sp.nsplit == 1 || ctr) return e;
        return p.out_dtype == QK_BF16 ? launch_reduce<QK_BF16>(p, sp.nsplit, partial, stream)
                                      : launch_reduce<QK_F16>(p, sp.nsplit, partial, stream);
    }
    if (!sp.ok) {
        hipError_t ce = hipSuccess;  // large M: cast to NZ in the workspace, NZ prefill GEMM
        if (launch_w4_cast_nz(p, workspace, ws_bytes, stream, &ce)) return ce;
        const int64_t sl = w8_slices_workspace(p);  // int8, 16 < M <= 128: the decode stream per 16 rows
        if (sl >= 0 && (sl == 0 || (ws && ws_bytes >= (size_t)sl && (uintptr_t)ws % 256 == 0))) {
            for (int64_t r0 = 0; r0 < p.M; r0 += kW8SliceRows) {
                const WqbmmArgs q = w8_slice(p, r0);
                const StreamPlan s = stream_plan(q);
                if (!s.ok) return hipErrorInvalidValue;  // checked for both slice sizes above
                uint64_t* ctr = (s.nsplit > 1 && (size_t)s.nstrip * 8 <= QK_SPLIT_COUNTER_BYTES &&
                                 s.nsplit < (1 << kSplitCountBits))
                                    ? reinterpret_cast<uint64_t*>(ws) : nullptr;
                hipError_t e = q.x_dtype == QK_BF16 ? launch_stream_dt<QK_BF16>(q, s, partial, ctr, stream)
                                                    : launch_stream_dt<QK_F16>(q, s, partial, ctr, stream);
                if (e == hipSuccess && s.nsplit > 1 && !ctr)
                    e = q.out_dtype == QK_BF16 ? launch_reduce<QK_BF16>(q, s.nsplit, partial, stream)
                                               : launch_reduce<QK_F16>(q, s.nsplit, partial, stream);
                if (e != hipSuccess) return e;
            }
            return hipSuccess;
        }
        GemmPlan gp = gemm_plan(p);
        if (gp.ok) {
            // without the workspace the size query asked for, the register-staged kernel runs
            float* xsum = nullptr;
            if (gp.dma && ws && ws_bytes >= gemm_dma_workspace(p) && (uintptr_t)ws % 256 == 0)
                xsum = reinterpret_cast<float*>(ws + QK_SPLIT_COUNTER_BYTES);
            else
                gp.dma = false;
            return p.x_dtype == QK_BF16 ? launch_gemm_dt<QK_BF16>(p, gp, xsum, stream)
                                        : launch_gemm_dt<QK_F16>(p, gp, xsum, stream);
        }
    }
    const DecodePlan d = decode_plan(p);
    if (d.ok) {
        if (d.nsplit > 1 && (!ws || ws_bytes < QK_SPLIT_COUNTER_BYTES + (size_t)d.nsplit * p.M * p.N * sizeof(float) ||
                             (uintptr_t)ws % 256 != 0))
            return hipErrorInvalidValue;
        hipError_t e = p.x_dtype == QK_BF16 ? launch_decode_dt<QK_BF16>(p, d, partial, stream)
                                            : launch_decode_dt<QK_F16>(p, d, partial, stream);
        if (e != hipSuccess || d.nsplit == 1) return e;
        const int64_t total = p.M * p.N / 4;
        int64_t blocks = (total + kThreads - 1) / kThreads;
        if (blocks > 65536) blocks = 65536;
        if (p.out_dtype == QK_BF16)
            w4_reduce<QK_BF16><<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(partial, d.nsplit, p.M, p.N, p.bias,
                                                                                     p.bias_dtype, p.out);
        else
            w4_reduce<QK_F16><<<dim3((uint32_t)blocks), dim3(kThreads), 0, stream>>>(partial, d.nsplit, p.M, p.N, p.bias,
                                                                                    p.bias_dtype, p.out);
        return hipGetLastError();
    }
    // shapes the decode kernels do not take (K not a multiple of 256, say): the register-staged prefill kernel
    // whatever its tile count (one round of tiles), which needs no workspace, before the generic kernel
    if (GemmPlan gf = gemm_plan(p, true); gf.ok) {
        gf.dma = false;
        return p.x_dtype == QK_BF16 ? launch_gemm_dt<QK_BF16>(p, gf, nullptr, stream)
                                    : launch_gemm_dt<QK_F16>(p, gf, nullptr, stream);
    }
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
