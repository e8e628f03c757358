// Device helpers shared by the gfx950 kernels: element conversions with
// explicit rounding, MFMA operand types, and launch-side declarations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/qk_abi.h"

namespace qk {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- 16-bit MFMA
// v_mfma_f32_16x16x32 in the activations' 16-bit type, with the magic-exponent
// constants of the int4 unpack: a nibble u in the low mantissa bits of MAGIC
// reads as 128 + u (bf16) / 1024 + u (fp16) exactly, so a two's-complement
// nibble w flipped to u = w + 8 is the operand w + BASE.
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

// ---------------------------------------------------------------- conversions
// fp16 -> fp32 is exact; bf16 -> fp32 is a shift.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}

// fp32 -> bf16 with round-to-nearest-even; a NaN keeps its upper bits and is
// quieted ((u >> 16) | 0x40).  This is the hardware conversion
// (v_cvt_pk_bf16_f32), which gives exactly that result for all 2^32 fp32
// patterns with fp32 denormals enabled, as this library is built (checked
// exhaustively on gfx950).  The empty asm pins f as a rounded fp32 value, so
// the compiler cannot fold an fmaf feeding it into a mixed-precision fma that
// rounds only once.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    asm volatile("" : "+v"(f));
    const __bf16 h = (__bf16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// fp32 -> fp16 with round-to-nearest-even (hardware conversion, default mode).
// The empty asm pins f as a rounded fp32 value: without it the compiler folds
// fmaf(a, b, c) followed by this cast into one v_fma_mixlo_f16, which rounds
// once from the exact product-sum instead of first to fp32, and so differs by
// an ulp from the fp32-then-fp16 rounding the ops specify.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    asm volatile("" : "+v"(f));
    _Float16 h = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// SwiGLU of one gate / up pair, a * sigmoid(a) * b, evaluated as (a * rcp(1 + exp2(-a * log2(e)))) * b on the
// hardware exp2 and reciprocal (exp(-a) is +inf below a = -88.7).  Shared by the SwiGLU kernels and the
// gate-up GEMM's fused epilogue, so both round the same fp32 value.
__device__ __forceinline__ float silu_mul(float a, float b) {
    const float e = __builtin_amdgcn_exp2f(-a * 1.44269504088896341f);
    return (a * __builtin_amdgcn_rcpf(1.0f + e)) * b;
}

// Largest value over each row of 16 lanes, at every lane of the row: DPP row rotations by 8, 4, 2 and 1 lanes
// (row_ror, dpp_ctrl 0x120 + n), one VALU max each, no LDS round trip.  Every lane of the row must be active.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false)));
    return v;
}
// Sum over each row of 16 lanes, at every lane of the row, by the same rotations: lane i adds the value of lane
// i +- 8, then of i +- 4, 2, 1, and as addition is commutative every lane of the row ends with the same bits.
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false));
    return v;
}
// Sum over the wave (all 64 lanes active), uniform: row16_sum, then (row 0 + row 1) + (row 2 + row 3).
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
}
// Largest value over the wave (all 64 lanes active), uniform: row16_max, then the four rows' lanes 0, 16, 32, 48.
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ float load_half_bits(uint32_t bits, int dtype) {
    return dtype == QK_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

__device__ __forceinline__ float load_scalar(const void* p, int64_t i, int dtype) {
    switch (dtype) {
    case QK_F16: return f16_bits_to_f32(((const uint16_t*)p)[i]);
    case QK_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    case QK_F32: return ((const float*)p)[i];
    default: return 0.0f;
    }
}

// ---------------------------------------------------------------- raw buffer loads
// A raw buffer resource over [base, base + bytes).  Loads through it take a
// 32-bit per-lane offset plus a wave-uniform offset that lives in an SGPR, so
// a run of rows costs no 64-bit VALU address arithmetic; an offset past
// `bytes` reads zero instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt immediate for vmcnt(n) alone (gfx9 encoding: vmcnt[3:0], [15:14]; others at their maximum)
constexpr int vmcnt_imm(int n) { return (n & 0xf) | (0x7 << 4) | (0xf << 8) | ((n >> 4) << 14); }

// 16 bytes per lane from a buffer into LDS bytes [lds + 16*lane, +16).  Written
// as asm so the compiler's wait-count pass, which cannot tell which LDS bytes
// a DMA writes, does not put a vmcnt(0) before every LDS read; the kernel
// waits on vmcnt itself.  m0 (the LDS base) is an operand, so the compiler
// sets it and knows it is in use.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds));
}

// ---------------------------------------------------------------- split-K completion
// Each of the nsplit workgroups that own one output tile stores its partial
// sums device-coherently (buffer stores with kCoherent: written through the
// XCD's L2) and then calls splitk_last, which returns true in exactly one of
// them -- the last to arrive.  That workgroup reads the other splits' partials
// device-coherently (buffer loads with kCoherent: not served from a possibly
// stale L2 line) and finishes the tile.  Whole 16-byte pieces of output rows
// per lane keep these write-through stores and loads as full lines; scattered
// 4-byte pieces make them an order of magnitude slower.  A split's stores have completed (s_waitcnt vmcnt(0)) before its
// arrival is counted, so the last arrival sees them all; no cache-wide
// writeback or invalidate is needed.  Call from every thread of the workgroup
// (it contains barriers).
//
// A counter is one 64-bit word.  Every call draws a tag T (48 bits, never 0
// and never all ones), and each arrival adds D = T * 2^16 + 1 with one
// fetch-and-add, so after j arrivals of this call on an empty word the word
// is j * D (mod 2^64), whose low 16 bits are j.  An arrival that reads such a
// value (j < nsplit, the word equal to j * D) is arrival j + 1: one atomic
// round trip, the same as a plain counter.  Zero is j = 0, and the last
// arrival sets the word back to zero (every other arrival has happened by
// then), so a workspace the library used before, or a zero fill, counts from
// zero; a captured graph that replays one tag likewise finds zero each time.
// Any other value is a stale word (a 0xFF fill, other data: a multiple of D
// below nsplit * D by chance only, odds about 2^-48 per word): that arrival's
// add is void and it registers with a compare-and-swap loop instead, which
// replaces a stale word by D (arrival 1) and adds D to a valid one.  Adds that
// land on a stale word are wiped by that replacement, and their arrivals
// register by compare-and-swap themselves; adds that land on a valid word
// count.  So each arrival is counted exactly once.
// Cache-policy operand of the raw buffer loads/stores for device-coherent
// access (the sc1 bit on gfx950).
constexpr int kCoherent = 16;
// Cache-policy operand for a load of data read once (the nt bit: the line is
// not kept in the L2 against the lines other workgroups read again).
constexpr int kNonTemporal = 2;
constexpr int kSplitCountBits = 16;
__device__ __forceinline__ bool splitk_last(uint64_t* ctr, uint32_t nsplit, uint64_t tag) {
    __shared__ uint32_t splitk_count;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint64_t d = (tag << kSplitCountBits) | 1u;
        constexpr uint64_t kCount = ((uint64_t)1 << kSplitCountBits) - 1;
        auto valid = [&](uint64_t w) { return (w & kCount) < nsplit && w == (w & kCount) * d; };
        uint64_t old = __hip_atomic_fetch_add(ctr, d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t n;
        if (valid(old)) {
            n = (uint32_t)(old & kCount) + 1u;
        } else {
            old += d;  // the word as this add left it; a failed compare-and-swap returns the actual value
            uint64_t nw;
            do {
                nw = valid(old) ? old + d : d;
            } while (!__hip_atomic_compare_exchange_weak(ctr, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT));
            n = (uint32_t)(nw & kCount);
        }
        if (n == nsplit) __hip_atomic_store(ctr, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        splitk_count = n;
    }
    __syncthreads();
    return splitk_count == nsplit;
}

// Host side: a fresh 48-bit tag per call for splitk_last (never 0, never all ones).
uint64_t next_split_tag();

// ---------------------------------------------------------------- per-row quantization
// Row reductions for 256-thread workgroups (4 wave64): DPP and lane reads inside
// a wave, LDS across the four waves.  Every thread gets the result.
__device__ __forceinline__ float block_absmax(float amax) {
    __shared__ float red_absmax[4];
    amax = wave_max(amax);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red_absmax[wave] = amax;
    __syncthreads();
    float r = red_absmax[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) r = fmaxf(r, red_absmax[w]);
    return r;
}

// Symmetric int8 of one value under the row scale s = absmax / 127 (the
// npu_dynamic_quant contract): clamp(rint(v / s)) with an IEEE division and
// ties to even; a zero row (s == 0) quantizes to 0.
__device__ __forceinline__ int32_t quant1(float v, float s) {
    if (s == 0.0f) return 0;
    float t = __builtin_rintf(v / s);
    t = fminf(fmaxf(t, -128.0f), 127.0f);
    return (int32_t)t;
}

// The same result as quant1 for every v of a row with |v| <= absmax, without
// a division for almost all elements.  With r = RN(1/s) and t = RN(v * r),
// t lies within 2^-16 of the exact v/s (two roundings, |v/s| <= 127.x < 128)
// and the IEEE quotient RN(v/s) within 2^-17 of it.  When t is more than
// 2^-14 from floor(t) + 0.5 (the half-integer nearest t), no rounding
// boundary lies between t and RN(v/s), so rint(t) = rint(RN(v/s)).  The other
// elements (a fraction of about 2^-13) and rows whose 1/s is not a safely
// normal number take the division.
struct RowQuant {
    float s, r;
    bool fast;
};
__device__ __forceinline__ RowQuant row_quant(float s) {
    RowQuant q;
    q.s = s;
    q.r = 1.0f / s;  // correctly rounded (the kernels are built with correctly rounded division)
    q.fast = s >= 0x1p-96f && s <= 0x1p96f;
    return q;
}
__device__ __forceinline__ int32_t quant_row(float v, const RowQuant& q) {
    if (q.fast) {
        const float t = v * q.r;
        const float h = __builtin_floorf(t) + 0.5f;
        if (fabsf(t - h) > 0x1p-14f) {
            const float n = fminf(fmaxf(__builtin_rintf(t), -128.0f), 127.0f);
            return (int32_t)n;
        }
    }
    return quant1(v, q.s);
}

// Eight values of one row -> eight int8 (element e in byte e % 4 of dword e / 4), each equal to
// quant1(v[e], s).  On a row whose 1/s is safely normal (q.fast), t = v * r is rounded to an integer by
// adding 1.5 * 2^23 (the fp32 add rounds to nearest even, as rint does), and the low byte of the sum's bits is
// the two's-complement int8: |t| <= 127 * (1 + 2^-22) here (s = RN(absmax / 127), r = RN(1 / s), |v| <=
// absmax), so it rounds into [-127, 127] and needs no clamp.  The fast and the exact rule agree unless t lies
// within 2^-14 of a half-integer (see quant_row) or is NaN; such a group of eight (about one in a thousand) is
// redone element by element with quant_row.  No branch per element on the common path.
__device__ __forceinline__ u32x2 quant8(const float (&v)[8], const RowQuant& q) {
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
    uint32_t m[8];
    bool exact = !q.fast;
    if (q.fast) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float t = v[e] * q.r;
            const float mf = t + kMagic;
            const float d = t - (mf - kMagic);  // t - rint(t), exact
            exact |= !(fabsf(d) < 0.5f - 0x1p-14f);
            m[e] = __float_as_uint(mf);
        }
    }
    if (exact) {
#pragma unroll
        for (int e = 0; e < 8; ++e) m[e] = (uint32_t)quant_row(v[e], q);
    }
    // byte 0 of each: two v_perm_b32 (bytes of m[2k+1] and m[2k] into the low half) and one shift-or per dword
    const uint32_t p01 = __builtin_amdgcn_perm(m[1], m[0], 0x0c0c0400u), p23 = __builtin_amdgcn_perm(m[3], m[2], 0x0c0c0400u);
    const uint32_t p45 = __builtin_amdgcn_perm(m[5], m[4], 0x0c0c0400u), p67 = __builtin_amdgcn_perm(m[7], m[6], 0x0c0c0400u);
    return (u32x2){p01 | (p23 << 16), p45 | (p67 << 16)};
}

// ---------------------------------------------------------------- XCD-aware ids
// The dispatcher hands consecutive workgroup ids to the 8 XCDs round-robin,
// and each XCD has its own L2.  Renumbering so that the ids one XCD receives
// are consecutive logical ids keeps neighbouring tiles (which share cache
// lines of A, B or a packed weight row) inside one L2.  Bijective on [0, nblk).
__device__ __forceinline__ int xcd_swizzle(int bid, int nblk) {
    const int full = nblk & ~7;
    if (bid >= full) return bid;
    return (bid & 7) * (full >> 3) + (bid >> 3);
}

// ---------------------------------------------------------------- W8A8 epilogue
// Applied to the exact int32 accumulator of one output element.  The float
// operations (and their order) are part of the op contract:
//   v = float(acc [+ int32 bias]); v *= pertoken[m] (if any);
//   v = fmaf(v, scale[n], float bias[n] or +0); cast with RNE.
// int8 output: clamp(rint(fmaf(float(acc), scale[n], offset[n]))).
struct QmmEpilogue {
    const float* scale;
    const float* offset;
    const float* pertoken;
    const void* bias;
    void* out;
    int64_t ldo;
    int scale_per_ch;
    int offset_per_ch;
    int bias_dtype;   // 0 = none
    int out_dtype;
};

__device__ __forceinline__ void qmm_store(const QmmEpilogue& e, int64_t m, int64_t n, int32_t acc) {
    float bf = 0.0f;
    if (e.bias_dtype == QK_I32) acc = (int32_t)((uint32_t)acc + (uint32_t)((const int32_t*)e.bias)[n]);
    else if (e.bias_dtype) bf = load_scalar(e.bias, n, e.bias_dtype);
    int64_t o = m * e.ldo + n;
    if (e.out_dtype == QK_I32) { ((int32_t*)e.out)[o] = acc; return; }
    float s = e.scale[e.scale_per_ch ? n : 0];
    float v = (float)acc;
    if (e.out_dtype == QK_I8) {
        float off = e.offset ? e.offset[e.offset_per_ch ? n : 0] : 0.0f;
        float t = __builtin_rintf(__builtin_fmaf(v, s, off));
        t = fminf(fmaxf(t, -128.0f), 127.0f);
        ((int8_t*)e.out)[o] = (int8_t)(int)t;
        return;
    }
    if (e.pertoken) v = v * e.pertoken[m];
    v = __builtin_fmaf(v, s, bf);
    if (e.out_dtype == QK_BF16) ((uint16_t*)e.out)[o] = (uint16_t)f32_to_bf16_bits(v);
    else if (e.out_dtype == QK_F16) ((uint16_t*)e.out)[o] = (uint16_t)f32_to_f16_bits(v);
    else ((float*)e.out)[o] = v;
}

// ---------------------------------------------------------------- planner override
// One debug override of the kernel planners, for tests and tuning only: parsed
// once from the QK_DEBUG_PLAN environment variable, or replaced through
// qk_debug_set_plan().  Planners read one snapshot per call (an atomic
// pointer, no environment lookups), so the workspace query and the launch of
// a call agree unless the override changes between them.  Spec: a
// comma-separated list of
//   w4_stream=off | w4_stream=<nwave>:<nkb>:<pf>   decode stream shape (16:4:2 16:4:4 8:4:2 8:4:4 8:8:2 8:8:3)
//   w4_stream_wpl=<16|32|64>                        decode stream: dwords of each weight row per wave (int4: 16
//                                                   half lines, 32 whole lines; int8: 16 quarter, 32 half, 64
//                                                   whole 256-byte rows)
//   w4_gemm=force | nodma | off                     prefill kernels on few tiles / register-staged only / never
//   w4_splits=<n>                                   K splits of the 32-row-block decode kernel
//   qmm_dma=0                                       W8A8 prefill: register-staged kernel instead of the DMA one
//   qmm_bm128=0                                     W8A8 K splits: 256-row tiles only (no 128-row split tiles)
//   qmm_rev=0                                       W8A8 DMA kernel: every round walks K forwards (by default
//                                                   every other round of one workgroup per CU walks it backwards)
//   qmm_mid=0                                       W8A8 M <= 256: split stream / tiled kernels instead of qmm_mid
//   qmm_small=<0|2|4|8>                             W8A8 [K,N], 32 < M <= 128: 0 always qmm_mid; n 128-row tiles
//                                                   with n K splits where the shape allows (default: cost model)
//   mid_bm=<16|32|64>, mid_split=<1|2>              qmm_mid: row block and K split (where the shape allows them)
//   mid_bn=<64|128>                                 qmm_mid: column block (128 only for a [K,N] weight)
//   skinny_splits=<n>                               W8A8 small-M stream: K splits (power of two, same bounds)
//   skinny_pf=<1..3>                                W8A8 small-M stream: stages loaded ahead in registers
//   w4nz=off                                        NZ int4 weights: unpack to ND and take the row-major kernels
//   nzg_sk=<0|1|tailfirst>                          NZ prefill GEMM: 0 whole tiles per workgroup (no stream-K);
//                                                   tailfirst: stream-K with each workgroup's tail segment run
//                                                   first, so it arrives before the head it would continue
//                                                   from and runs the whole tile itself (the fallback path)
//   nzg_sk_dp=<n>                                   NZ prefill stream-K: n whole-tile rounds first
//   w4nz_wg=<n>                                     NZ decode kernel: workgroups along N
//   w4nz_nit=<1..8>                                 NZ decode kernel: 128-row superblocks per wave (K/128 must
//                                                   split evenly into at most 16 waves of them)
struct PlanOverride {
    int w4_stream_nwave = 0, w4_stream_nkb = 0, w4_stream_pf = 0;  // 0: the planner's choice
    bool w4_stream_off = false;
    int w4_stream_wpl = 0;  // decode stream: weight-row dwords per wave (0: the planner's choice)
    int w4_gemm = 0;  // 0 planner, 1 force, 2 nodma, 3 off
    int w4_splits = 0;
    bool qmm_dma = true;
    bool qmm_bm128 = true;
    bool qmm_mid = true;
    int mid_bm = 0, mid_split = 0, mid_bn = 0;
    int skinny_splits = 0;
    int skinny_pf = 0;  // W8A8 small-M stream: stages loaded ahead in registers (0: the planner's choice)
    bool w4nz_off = false;
    int nzg_sk = 1;
    int nzg_sk_dp = -1;  // whole-tile rounds before the stream-K share (-1: the planner's choice)
    int qmm_rev = 1;
    int qmm_small = -1;
    int w4nz_wg = 0, w4nz_nit = 0;
};
const PlanOverride& plan_override();
// CUs of the current device (cached per device; 0 if it cannot be read)
int device_cus();
bool set_plan_override(const char* spec);  // false: spec not understood (override unchanged)

// ---------------------------------------------------------------- launchers
// Host-side entry points of each kernel file (validated arguments only).
hipError_t launch_dynamic_quant(const void* x, int x_dtype, int64_t rows, int64_t K,
                                const float* smooth, int8_t* y, float* scale, hipStream_t stream);
// npu_dynamic_quant of x [rows, K] (16-byte aligned rows, K % 8 == 0) whose row absmax is the largest of
// amax_part[row * parts + j], j < parts (partial absmax of column slices of the row, written by the kernel that
// produced x): the same y and scale as launch_dynamic_quant, in one elementwise pass with no row reduction.
hipError_t launch_dynamic_quant_premax(const void* x, int x_dtype, int64_t rows, int64_t K, const float* amax_part,
                                       int parts, int8_t* y, float* scale, hipStream_t stream);

struct QmmArgs {
    const int8_t* a;
    int64_t lda;
    const int8_t* b;
    int64_t sbk, sbn;     // x2 strides (one of them is 1)
    int64_t M, N, K;
    QmmEpilogue epi;
};
hipError_t launch_quant_matmul(const QmmArgs& args, void* workspace, size_t ws_bytes, hipStream_t stream);
size_t quant_matmul_workspace(int64_t M, int64_t N, int64_t K);
// the same op on an int8 NZ weight (args.b: [N/16][K/64][64][16]; args.sbk / args.sbn unused)
hipError_t launch_quant_matmul_nz(const QmmArgs& args, void* workspace, size_t ws_bytes, hipStream_t stream);
size_t quant_matmul_nz_workspace(int64_t M, int64_t N, int64_t K);
// The quantized MLP block's gate-up GEMM with SwiGLU fused: args.N = 2I weight columns (gate, then up), the
// output h [M, I] (bf16 / fp16, args.epi.ldo = I); the weight as NZ blocks (nz) or [K, 2I] rows.  amax_part (or
// null): fp32 [M][I / 128], each 128-column slice's largest |h| per row.
// hipErrorInvalidValue where the shape or operands do not fit the kernel.
hipError_t launch_quant_matmul_swiglu(const QmmArgs& args, bool nz, float* amax_part, hipStream_t stream);

struct WqbmmArgs {
    const void* x;
    int x_dtype;
    const void* w;
    int w_dtype;          // QK_I32 (int4 packed), QK_I8, QK_I4_NZ, QK_I8_NZ or QK_I8_NK
    const void* scale;
    const void* offset;
    int s_dtype;
    int64_t M, N, K, group;  // group == 0: per channel (one group of K)
    const void* bias;
    int bias_dtype;       // 0 = none
    void* out;
    int out_dtype;
};
hipError_t launch_weight_quant_bmm(const WqbmmArgs& args, void* workspace, size_t ws_bytes, hipStream_t stream);
// xsum[g][m] = fp32 sum of x[m][k] over group g (G a multiple of 64), for the prefill kernels' group algebra
hipError_t launch_w4_xsum(const WqbmmArgs& p, float* xsum, hipStream_t stream);
// Workspace sizes of one call, largest first.  kWsFull: the plan as planned.  kWsNoStreamK: without the NZ
// prefill kernel's stream-K partials (the same kernels and the same bits, tiles whole per workgroup).
// kWsNoCast: also without the plan that casts a row-major int4 / int8 weight to NZ in the workspace (the launch
// then runs the row-major kernels).  For callers whose scratch is bounded; a launch takes the largest plan
// its workspace holds.
constexpr int kWsFull = 0, kWsNoStreamK = 1, kWsNoCast = 2;
size_t weight_quant_bmm_workspace(int64_t M, int64_t N, int64_t K, int w_dtype, int64_t group, int level = kWsFull);

// NZ weights (nz_weights.hip): the ND <-> NZ casts (int4, int8) and the weight-quant matmul on NZ weights.
hipError_t launch_w4_nz_cast(const int32_t* src, bool to_nz, int64_t K, int64_t N, int32_t* dst, hipStream_t stream);
hipError_t launch_w8_nz_cast(const int8_t* src, bool to_nz, int64_t K, int64_t N, int8_t* dst, hipStream_t stream);
// int8 [N, K] -> [K, N]
hipError_t launch_w8_nk_transpose(const int8_t* src, int64_t K, int64_t N, int8_t* dst, hipStream_t stream);
size_t w4_nz_workspace(const WqbmmArgs& args, bool stream_k = true);
// A row-major int4 or int8 weight at large M: cast to NZ into the workspace, then the NZ prefill GEMM.  The size is 0
// when the plan does not apply; the launch returns false (running nothing) when it does not apply to these
// operands or the workspace cannot hold it, else true with the launch status in *err.
size_t w4_cast_nz_workspace(const WqbmmArgs& args, bool stream_k = true);
bool launch_w4_cast_nz(const WqbmmArgs& args, void* workspace, size_t ws_bytes, hipStream_t stream, hipError_t* err);
hipError_t launch_w4_nz_bmm(const WqbmmArgs& args, void* workspace, size_t ws_bytes, hipStream_t stream);

// Static quantization (static_quant.hip): x [outer][C][inner] (fp32/fp16/bf16) -> q (int8/uint8/int32);
// scales == nullptr: per tensor with scale0 / zp0.
hipError_t launch_quantize(const void* x, int x_dtype, int64_t outer, int64_t C, int64_t inner, const float* scales,
                           const int64_t* zps, float scale0, int64_t zp0, void* q, int q_dtype, hipStream_t stream);
hipError_t launch_dequantize(const void* q, int q_dtype, int64_t n, float* out, hipStream_t stream);

hipError_t launch_int4_pack(const void* w, int w_dtype, int64_t K, int64_t N, int32_t* packed,
                            hipStream_t stream);

// Quantized MLP block neighbours (x, gamma, h, y in the 16-bit dtype `dt`; launch_rms_norm also
// takes QK_F32 without q).
hipError_t launch_rms_norm(const void* x, int dt, const void* gamma, int64_t rows, int64_t D, float eps, void* y,
                           int8_t* q, float* scale, float* rstd, hipStream_t stream);
hipError_t launch_swiglu(const void* h, int dt, int64_t rows, int64_t I, void* y, int8_t* q, float* scale,
                         hipStream_t stream);

}  // namespace qk
