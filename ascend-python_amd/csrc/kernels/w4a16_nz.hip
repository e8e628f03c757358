// npu_weight_quant_batchmatmul on an int4 weight in the MFMA-tiled "NZ"
// layout, and the format casts that produce and undo that layout.
//
// Layout (this build's device-native counterpart of the FRACTAL_NZ weight
// casts the reference applies before matmuls,
// op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:303-316 and
// op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:103-107):
// int32 [N/16][K/128][64][4].  One 16-column block ("n-block") over 128 k
// ("superblock") is 1 KB: lane l = n%16 + 16*g holds four words j = 0..3, and
// word j carries the 8 consecutive k of chunk c = 4*j + g (k%128 = 8*c + i),
// even i in nibbles 0..3 and odd i in nibbles 4..7 (two's complement).  So one
// 16-byte load per lane brings a wave the whole superblock of an n-block, and
// word j is, after ((w >> 4q) & 0x000f000f) ^ magic for q = 0..3, exactly the
// B operand of one v_mfma_f32_16x16x32 (column n%16, k = 8c..8c+7, even k in
// the low halves) -- no LDS, no cross-lane shuffles, whole 128-byte lines.
// The matching A operand of lane (m, g) is x[m, 128s + 8*(4j+g) .. +8], 16
// contiguous bytes.
//
// Decode kernel (w4nz_decode), M <= 64: each workgroup owns a few n-blocks
// over all of K, so no partial sums leave the workgroup.  Its waves split K
// into equal runs of superblocks; every wave issues the loads of two
// superblocks ahead (for K = 4096 that is all of its loads, issued before the
// first MFMA), folds group scale and offset into its accumulators per
// superblock with the algebra of the row-major kernels,
//   acc += s * sum_k x*(w + BASE) + s*(offset - BASE) * sum_k x,
// and the waves' sums are added through LDS in K order (deterministic).
#include "common.h"

namespace qk {
namespace {

constexpr int kNzThreads = 256;
constexpr int kNzMaxWaves = 16;
constexpr int kNzTilePitch = 320; // floats per 16x16 tile in the reduction buffer

// word index and nibble of weight element (k, n) in the NZ layout
__host__ __device__ __forceinline__ int64_t nz4_index(int64_t k, int64_t n, int64_t S, int* nibble) {
    const int64_t c = (k & 127) >> 3, i = k & 7;
    const int64_t lane = (n & 15) + 16 * (c & 3), j = c >> 2;
    *nibble = (int)((i & 1) ? 4 + (i >> 1) : (i >> 1));
    return ((((n >> 4) * S + (k >> 7)) * 64 + lane) << 2) + j;
}

// ND [K, N/8] -> NZ: one thread per NZ word, gathering its 8 nibbles.
__global__ __launch_bounds__(kNzThreads) void w4_nz_pack_kernel(const int32_t* __restrict__ nd, int64_t K, int64_t N,
                                                                int32_t* __restrict__ nz) {
    const int64_t total = K * N / 8, NW = N / 8, S = K / 128;
    for (int64_t idx = (int64_t)blockIdx.x * kNzThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kNzThreads) {
        const int64_t j = idx & 3, lane = (idx >> 2) & 63, sb = idx >> 8;
        const int64_t s = sb % S, nb = sb / S;
        const int64_t n = nb * 16 + (lane & 15), c = 4 * j + (lane >> 4), k0 = s * 128 + 8 * c;
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = ((uint32_t)nd[(k0 + i) * NW + (n >> 3)] >> (4 * (n & 7))) & 0xfu;
            word |= v << (4 * ((i & 1) ? 4 + (i >> 1) : (i >> 1)));
        }
        nz[idx] = (int32_t)word;
    }
}

// NZ -> ND [K, N/8]: one thread per ND word.
__global__ __launch_bounds__(kNzThreads) void w4_nz_unpack_kernel(const int32_t* __restrict__ nz, int64_t K, int64_t N,
                                                                  int32_t* __restrict__ nd) {
    const int64_t total = K * N / 8, NW = N / 8, S = K / 128;
    for (int64_t idx = (int64_t)blockIdx.x * kNzThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kNzThreads) {
        const int64_t k = idx / NW, n0 = (idx % NW) * 8;
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int p;
            const int64_t w = nz4_index(k, n0 + i, S, &p);
            word |= (((uint32_t)nz[w] >> (4 * p)) & 0xfu) << (4 * i);
        }
        nd[idx] = (int32_t)word;
    }
}

// The B operand held in one NZ word: dword q takes nibbles q (k = 2q, low
// half) and 4 + q (k = 2q + 1, high half) as magic values 128 + (w + 8)
// (bf16) or 1024 + (w + 8) (fp16): one shift and one and-xor each.
template <uint32_t MAGIC>
__device__ __forceinline__ u32x4 nz_operand(uint32_t w) {
    const uint32_t mask = __builtin_amdgcn_readfirstlane(0x000f000fu);
    const uint32_t magic = __builtin_amdgcn_readfirstlane(MAGIC | 0x00080008u);
    u32x4 b;
    b[0] = (w & mask) ^ magic;
    b[1] = ((w >> 4) & mask) ^ magic;
    b[2] = ((w >> 8) & mask) ^ magic;
    b[3] = ((w >> 12) & mask) ^ magic;
    return b;
}

// NB: n-blocks per workgroup (the last workgroups may own one fewer: their
// extra block repeats a real one and is not stored).  NIT: superblocks per
// wave.  The grid is (workgroups along N) x (16-row blocks of M); a
// workgroup has K / (128 * NIT) waves.  A superblock's scale and offset rows
// (the workgroup's NB*16 columns of one group) come in with one 16-byte load
// per fetching lane and reach the other lanes through the wave's own LDS slot.
template <int DT, int NB, int NIT, bool HAS_OFF>
__global__ __launch_bounds__(64 * kNzMaxWaves) void w4nz_decode(WqbmmArgs p, int nwg, int nrb) {
    typedef Mfma<DT> MM;
    constexpr int PF = NIT < 2 ? NIT : 2;  // superblocks in flight per wave
    constexpr int SL = PF;                 // register slots
    constexpr int NT = HAS_OFF ? 2 : 1;    // scale rows per superblock (scale, offset)
    constexpr int RL = 2 * NB;             // 16-byte pieces of one row (NB*16 columns)
    static_assert(NT * RL <= 64, "one load instruction fetches a superblock's scale rows");
    __shared__ __attribute__((aligned(16))) float red[kNzMaxWaves][NB][kNzTilePitch];
    __shared__ __attribute__((aligned(16))) uint16_t srow[kNzMaxWaves][SL][NT][NB * 16];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwave = blockDim.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    // row blocks of one n range are consecutive logical ids, so they share an XCD (one L2)
    const int lid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int rb = lid % nrb, wg = lid / nrb;
    const int M = (int)p.M, K = (int)p.K, N = (int)p.N, G = (int)p.group;
    const int NBT = N >> 4, S = K >> 7;
    // block range of this workgroup (32-bit: (nwg + 1) * NBT < 2^31, checked by the planner)
    const int b0 = (int)((uint32_t)(wg * NBT) / (uint32_t)nwg), b1 = (int)((uint32_t)((wg + 1) * NBT) / (uint32_t)nwg);
    const int s0 = wave * NIT;
    // rows past M read row M-1 (each output row depends on its own x row only) and are not stored
    const int m = rb * 16 + c < M ? rb * 16 + c : M - 1;

    const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
    const uint32_t x_lane = ((uint32_t)m * (uint32_t)K + 8u * (uint32_t)g) * 2u;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (uint32_t)K * (uint32_t)N / 2u);
    const uint32_t w_lane = (uint32_t)lane * 16u;
    // lane l < NT*RL fetches 16 bytes of row l / RL (scale, offset) of a superblock's group: columns
    // 16*b0 + 8*(l % RL) .. +8, clamped into the row (the clamped columns belong to no block of this
    // workgroup and are never used); the other lanes repeat lane 0's address
    const int sl_t = lane < NT * RL ? lane / RL : 0;
    const int sl_col0 = 16 * b0 + 8 * (lane < NT * RL ? lane % RL : 0);
    const int sl_col = sl_col0 < N ? sl_col0 : N - 8;
    const uint16_t* sl_base = static_cast<const uint16_t*>(sl_t == 0 || !HAS_OFF ? p.scale : p.offset) + sl_col;

    int blk[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) blk[b] = b0 + b < b1 ? b0 + b : b1 - 1;

    u32x4 xa[SL][4], wv[SL][NB], sa[SL];
    auto issue = [&](int it) {
        __builtin_amdgcn_sched_barrier(0);
        const int s = s0 + it, sl = it % SL;
        const uint32_t grp = (uint32_t)(s * 128) / (uint32_t)G;
        sa[sl] = *reinterpret_cast<const u32x4*>(sl_base + (size_t)grp * (uint32_t)N);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xa[sl][j] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, x_lane, (uint32_t)(s * 256 + 64 * j), 0));
#pragma unroll
        for (int b = 0; b < NB; ++b)
            wv[sl][b] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           wr, w_lane, ((uint32_t)blk[b] * (uint32_t)S + (uint32_t)s) * 1024u, 0));
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int it = 0; it < PF; ++it) issue(it);

    const u32x4 ones = {MM::ONES, MM::ONES, MM::ONES, MM::ONES};
    constexpr float BASE = MM::BASE;
    f32x4 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int sl = it % SL;
        // this superblock's scale rows through the wave's LDS slot
        if (lane < NT * RL) *reinterpret_cast<u32x4*>(&srow[wave][sl][0][0] + 8 * lane) = sa[sl];
        u32x4 xk[4], wk[NB];
#pragma unroll
        for (int j = 0; j < 4; ++j) xk[j] = xa[sl][j];
#pragma unroll
        for (int b = 0; b < NB; ++b) wk[b] = wv[sl][b];
        f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) xs = MM::mma(xk[j], ones, xs);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            f32x4 ag = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) ag = MM::mma(xk[j], nz_operand<MM::MAGIC>(wk[b][j]), ag);
            const float sf = load_half_bits(srow[wave][sl][0][16 * b + c], p.s_dtype);
            const float of = HAS_OFF ? load_half_bits(srow[wave][sl][NT - 1][16 * b + c], p.s_dtype) : 0.0f;
            const float sx = sf * (of - BASE);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[b][r] = __builtin_fmaf(sf, ag[r], __builtin_fmaf(sx, xs[r], acc[b][r]));
        }
        if (it + PF < NIT) issue(it + PF);
    }

    // the K ranges of waves a short K leaves out add as zeros in the reduction below
    for (int w = nwave + wave; w < kNzMaxWaves; w += nwave)
#pragma unroll
        for (int b = 0; b < NB; ++b)
            for (int e = lane; e < kNzTilePitch; e += 64) red[w][b][e] = 0.0f;
    // lane (c, g) holds rows 4g..4g+3 of column c of each block; row r of a
    // tile sits at 16*(r + r/4) + column, so the 64 lanes of one store hit 64 banks
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][b][16 * (5 * g + r) + c] = acc[b][r];
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // the waves' K ranges are added in K order; all 16 reads are issued before the adds
    const int nb = b1 - b0;
    for (int t = threadIdx.x; t < NB * 256; t += blockDim.x) {
        const int b = t >> 8, row = (t >> 4) & 15, col = t & 15;
        const int at = 16 * (row + (row >> 2)) + col;
        float part[kNzMaxWaves];
#pragma unroll
        for (int w = 0; w < kNzMaxWaves; ++w) part[w] = red[w][b][at];
        float v = part[0];
#pragma unroll
        for (int w = 1; w < kNzMaxWaves; ++w) v += part[w];
        const int mm = rb * 16 + row, n = (b0 + b) * 16 + col;
        if (b >= nb || mm >= M) continue;
        if (p.bias_dtype) v += load_scalar(p.bias, n, p.bias_dtype);
        const uint32_t o = p.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        static_cast<uint16_t*>(p.out)[(int64_t)mm * N + n] = (uint16_t)o;
    }
}

// The most blocks per workgroup that a wave of `nit` superblocks holds in registers without
// spilling (two superblocks in flight, NB accumulators): 4 up to 3 superblocks, 3 for 4, 2 for 5,
// 1 beyond.  Only these (NB, NIT) pairs are built.
constexpr int nz_max_blocks(int nit) { return nit <= 3 ? 4 : nit == 4 ? 3 : nit == 5 ? 2 : 1; }

struct NzPlan {
    bool ok;
    int nb, nit, nwave, nwg, nrb;
};

NzPlan nz_plan(const WqbmmArgs& p) {
    NzPlan z{false, 0, 0, 0, 0, 0};
    const int64_t G = p.group == 0 ? p.K : p.group;
    if (p.w_dtype != QK_I4_NZ || p.M <= 0 || p.M > 64 || p.N <= 0 || p.K <= 0) return z;
    if (p.N % 16 != 0 || p.K % 128 != 0 || G <= 0 || G % 128 != 0 || p.K % G != 0) return z;
    // 32-bit buffer offsets
    if (p.K * p.N / 2 >= ((int64_t)1 << 31) || p.M * p.K * 2 >= ((int64_t)1 << 31) ||
        (p.K / G) * p.N * 2 >= ((int64_t)1 << 31))
        return z;
    if ((uintptr_t)p.x % 16 != 0 || (uintptr_t)p.w % 16 != 0 || (uintptr_t)p.scale % 16 != 0 ||
        (uintptr_t)p.out % 2 != 0 || (p.offset && (uintptr_t)p.offset % 16 != 0))
        return z;
    const int64_t S = p.K / 128, NBT = p.N / 16;
    // superblocks per wave: the fewest that give at most 16 waves and split K evenly
    int nit = 0;
    for (int t = 1; t <= 8; ++t)
        if (S % t == 0 && S / t <= kNzMaxWaves) {
            nit = t;
            break;
        }
    if (nit == 0) return z;
    z.nit = nit;
    z.nwave = (int)(S / nit);
    z.nrb = (int)((p.M + 15) / 16);
    // blocks per workgroup: what one workgroup per CU needs, within what fits the wave's registers
    // (nz_max_blocks); then as few workgroups as give no workgroup more blocks than that
    const int cap = nz_max_blocks(nit);
    int64_t nb = (NBT + 255) / 256;
    if (const int f = plan_override().w4nz_wg) nb = (NBT + f - 1) / f;  // debug override: a workgroup count
    if (nb > cap) nb = cap;
    z.nb = (int)nb;
    z.nwg = (int)((NBT + nb - 1) / nb);
    z.ok = (int64_t)z.nwg * z.nrb < ((int64_t)1 << 31) && ((int64_t)z.nwg + 1) * NBT < ((int64_t)1 << 31);
    return z;
}

template <int DT, int NB, int NIT, bool OFF>
hipError_t launch_nz_k(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    if constexpr (NB <= nz_max_blocks(NIT)) {
        const dim3 grid((uint32_t)(z.nwg * z.nrb)), block((uint32_t)(64 * z.nwave));
        w4nz_decode<DT, NB, NIT, OFF><<<grid, block, 0, stream>>>(p, z.nwg, z.nrb);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;  // not planned (nz_plan caps NB by nz_max_blocks)
}

template <int DT, int NB, bool OFF>
hipError_t launch_nz_nit(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    switch (z.nit) {
    case 1: return launch_nz_k<DT, NB, 1, OFF>(p, z, stream);
    case 2: return launch_nz_k<DT, NB, 2, OFF>(p, z, stream);
    case 3: return launch_nz_k<DT, NB, 3, OFF>(p, z, stream);
    case 4: return launch_nz_k<DT, NB, 4, OFF>(p, z, stream);
    case 5: return launch_nz_k<DT, NB, 5, OFF>(p, z, stream);
    case 6: return launch_nz_k<DT, NB, 6, OFF>(p, z, stream);
    case 7: return launch_nz_k<DT, NB, 7, OFF>(p, z, stream);
    default: return launch_nz_k<DT, NB, 8, OFF>(p, z, stream);
    }
}

template <int DT, bool OFF>
hipError_t launch_nz_nb(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    switch (z.nb) {
    case 1: return launch_nz_nit<DT, 1, OFF>(p, z, stream);
    case 2: return launch_nz_nit<DT, 2, OFF>(p, z, stream);
    case 3: return launch_nz_nit<DT, 3, OFF>(p, z, stream);
    default: return launch_nz_nit<DT, 4, OFF>(p, z, stream);
    }
}

template <int DT>
hipError_t launch_nz_dt(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    return p.offset ? launch_nz_nb<DT, true>(p, z, stream) : launch_nz_nb<DT, false>(p, z, stream);
}

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

int64_t grid_for(int64_t total) {
    int64_t blocks = (total + kNzThreads - 1) / kNzThreads;
    return blocks > 65536 ? 65536 : (blocks < 1 ? 1 : blocks);
}

}  // namespace

hipError_t launch_w4_nz_cast(const int32_t* src, bool to_nz, int64_t K, int64_t N, int32_t* dst, hipStream_t stream) {
    const int64_t total = K * N / 8;
    if (total == 0) return hipSuccess;
    if (to_nz)
        w4_nz_pack_kernel<<<dim3((uint32_t)grid_for(total)), dim3(kNzThreads), 0, stream>>>(src, K, N, dst);
    else
        w4_nz_unpack_kernel<<<dim3((uint32_t)grid_for(total)), dim3(kNzThreads), 0, stream>>>(src, K, N, dst);
    return hipGetLastError();
}

// NZ weights: the decode kernel where it applies (no workspace); otherwise the
// weight is unpacked into the workspace and the row-major kernels run on it:
// [QK_SPLIT_COUNTER_BYTES, unused][ND weight, K*N/2 B][row-major call's workspace].
size_t w4_nz_workspace(const WqbmmArgs& p) {
    if (!plan_override().w4nz_off && nz_plan(p).ok) return 0;
    return QK_SPLIT_COUNTER_BYTES + round256((size_t)(p.K * p.N / 2)) +
           weight_quant_bmm_workspace(p.M, p.N, p.K, QK_I32, p.group);
}

hipError_t launch_w4_nz_bmm(const WqbmmArgs& p, void* workspace, size_t ws_bytes, hipStream_t stream) {
    const NzPlan z = plan_override().w4nz_off ? NzPlan{false, 0, 0, 0, 0, 0} : nz_plan(p);
    if (z.ok)
        return p.x_dtype == QK_BF16 ? launch_nz_dt<QK_BF16>(p, z, stream) : launch_nz_dt<QK_F16>(p, z, stream);
    const size_t nd_bytes = round256((size_t)(p.K * p.N / 2));
    const size_t rest = weight_quant_bmm_workspace(p.M, p.N, p.K, QK_I32, p.group);
    if (!workspace || ws_bytes < QK_SPLIT_COUNTER_BYTES + nd_bytes + rest || (uintptr_t)workspace % 256 != 0)
        return hipErrorInvalidValue;
    char* ws = static_cast<char*>(workspace);
    int32_t* nd = reinterpret_cast<int32_t*>(ws + QK_SPLIT_COUNTER_BYTES);
    hipError_t e = launch_w4_nz_cast(static_cast<const int32_t*>(p.w), false, p.K, p.N, nd, stream);
    if (e != hipSuccess) return e;
    WqbmmArgs q = p;
    q.w = nd;
    q.w_dtype = QK_I32;
    return launch_weight_quant_bmm(q, rest ? ws + QK_SPLIT_COUNTER_BYTES + nd_bytes : nullptr, rest, stream);
}

}  // namespace qk
