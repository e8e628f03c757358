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
// The int8 NZ layout (W8A16 and W8A8 weights) is int8 [N/16][K/64][64][16]:
// lane l = n%16 + 16*g of a 16-column x 64-row block holds rows 16g..16g+15 of
// its column, the B operand of one v_mfma_i32_16x16x64_i8, or two 8-row
// operands of a 16-bit MFMA once the bytes are converted.
//
// Decode kernel (w4nz_decode), M <= 64: each workgroup owns a few n-blocks
// over all of K, so no partial sums leave the workgroup.  Its waves split K
// into equal runs of superblocks; every wave issues the loads of two
// superblocks ahead (for K = 4096 that is all of its loads, issued before the
// first MFMA; x by whole-line DMAs into the wave's LDS slots, the weights
// non-temporal), folds group scale and offset into its accumulators per
// superblock with the algebra of the row-major kernels,
//   acc += s * sum_k x*(w + BASE) + s*(offset - BASE) * sum_k x,
// and the waves' sums are added through LDS in K order (deterministic).
#include <atomic>

#include "common.h"

namespace qk {

// CUs of the current device (cached per device; 0 if it cannot be read)
int device_cus() {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cache[kMaxDev];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 0) n = 0;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

namespace {

constexpr int kNzThreads = 256;
constexpr int kNzMaxWaves = 16;
constexpr int kNzTilePitch = 320; // floats per 16x16 tile in the reduction buffer

// The casts move one tile per workgroup through LDS: 16 n-blocks (256 columns; fewer in the last group) by one
// K block row (128 rows for int4, 64 for int8).  The NZ side is read or written as its whole 1 KB blocks and
// the ND side as whole row pieces (32 words / 256 bytes per row, one dword per lane), so both are streamed in
// whole lines; the change of layout is a register transpose of nibbles or bytes between the two.
constexpr int kCastNB = 16;    // n-blocks per tile
constexpr int kCastPad = 4;    // dwords of padding per NZ block in LDS (spreads the blocks over the banks)

// nibble of row i (0..7) of an 8-row chunk inside an NZ word: even rows in nibbles 0..3, odd rows in 4..7
__host__ __device__ __forceinline__ int nz4_nibble(int i) { return (i & 1) ? 4 + (i >> 1) : (i >> 1); }

// NZ -> ND [K, N/8] (int4).  Tile = superblock sb (128 rows) x n-block group nbg.
__global__ __launch_bounds__(kNzThreads) void w4_nz_unpack_kernel(const int32_t* __restrict__ nz, int64_t K,
                                                                  int64_t N, int32_t* __restrict__ nd) {
    __shared__ uint32_t blk[kCastNB][64 * 4 + kCastPad];
    const int64_t S = K / 128, NBT = N / 16, NW = N / 8;
    const int64_t sb = blockIdx.x % S, nbg = blockIdx.x / S;
    const int nb = (int)(NBT - nbg * kCastNB < kCastNB ? NBT - nbg * kCastNB : kCastNB);
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < 4; ++u) {  // 1024 lane chunks of 16 bytes: chunk q = block q>>6, lane q&63
        const int q = t + kNzThreads * u, b = q >> 6, l = q & 63;
        if (b < nb)
            *reinterpret_cast<u32x4*>(&blk[b][4 * l]) =
                *reinterpret_cast<const u32x4*>(nz + (((nbg * kCastNB + b) * S + sb) * 64 + l) * 4);
    }
    __syncthreads();
    // thread -> word column wc of the tile (block wc>>1, columns 8*(wc&1)..+7 of it) and 8-row chunks c
    const int wc = t & 31, b = wc >> 1, h = wc & 1;
    if (b >= nb) return;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        const int c = (t >> 5) + 8 * pass;  // rows 8c..8c+7 of the superblock
        uint32_t d[8];                      // NZ word c>>2 of the 8 lanes holding columns 8h..8h+7
#pragma unroll
        for (int q = 0; q < 8; ++q) d[q] = blk[b][4 * (8 * h + 16 * (c & 3) + q) + (c >> 2)];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t w = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) w |= ((d[q] >> (4 * nz4_nibble(i))) & 0xfu) << (4 * q);
            nd[(sb * 128 + 8 * c + i) * NW + nbg * (2 * kCastNB) + wc] = (int32_t)w;
        }
    }
}

// ND [K, N/8] -> NZ (int4): the inverse tile.
__global__ __launch_bounds__(kNzThreads) void w4_nz_pack_kernel(const int32_t* __restrict__ nd, int64_t K, int64_t N,
                                                                int32_t* __restrict__ nz) {
    __shared__ uint32_t rows[128][2 * kCastNB + 1];
    const int64_t S = K / 128, NBT = N / 16, NW = N / 8;
    const int64_t sb = blockIdx.x % S, nbg = blockIdx.x / S;
    const int nb = (int)(NBT - nbg * kCastNB < kCastNB ? NBT - nbg * kCastNB : kCastNB);
    const int nw = 2 * nb, t = threadIdx.x;
    if (nb == kCastNB && NW % 4 == 0 && (uintptr_t)nd % 16 == 0) {
        // whole 128-byte row pieces on 16-byte aligned rows: one 16-byte load per lane (4 per thread)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = t + kNzThreads * u, r = e >> 3, v = e & 7;
            const u32x4 d = *reinterpret_cast<const u32x4*>(nd + (sb * 128 + r) * NW + nbg * (2 * kCastNB) + 4 * v);
#pragma unroll
            for (int i = 0; i < 4; ++i) rows[r][4 * v + i] = d[i];
        }
    } else {
        for (int e = t; e < 128 * 2 * kCastNB; e += kNzThreads) {  // one dword per lane: 128-byte row pieces
            const int r = e >> 5, w = e & 31;
            if (w < nw) rows[r][w] = (uint32_t)nd[(sb * 128 + r) * NW + nbg * (2 * kCastNB) + w];
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {  // lane chunk q = (block q>>6, lane q&63): 4 words j, chunk c = 4j + lane/16
        const int q = t + kNzThreads * u, b = q >> 6, l = q & 63;
        if (b >= nb) continue;
        const int n16 = l & 15, wc = 2 * b + (n16 >> 3), sh = 4 * (n16 & 7);
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = 4 * j + (l >> 4);
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) w |= ((rows[8 * c + i][wc] >> sh) & 0xfu) << (4 * nz4_nibble(i));
            o[j] = w;
        }
        *reinterpret_cast<u32x4*>(nz + (((nbg * kCastNB + b) * S + sb) * 64 + l) * 4) = o;
    }
}

// 4 x 4 byte transpose: o[j] byte i = r[i] byte j.
__device__ __forceinline__ void bytes4x4(const uint32_t r[4], uint32_t o[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(r[1], r[0], 0x05010400u);  // r0b0 r1b0 r0b1 r1b1
    const uint32_t t1 = __builtin_amdgcn_perm(r[1], r[0], 0x07030602u);  // r0b2 r1b2 r0b3 r1b3
    const uint32_t t2 = __builtin_amdgcn_perm(r[3], r[2], 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(r[3], r[2], 0x07030602u);
    o[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// int8 NZ -> ND [K, N].  Tile = K block kb (64 rows) x n-block group nbg (256 bytes per row).
__global__ __launch_bounds__(kNzThreads) void w8_nz_unpack_kernel(const int8_t* __restrict__ nz, int64_t K, int64_t N,
                                                                  int8_t* __restrict__ nd) {
    __shared__ uint32_t blk[kCastNB][64 * 4 + kCastPad];
    const int64_t KB = K / 64, NBT = N / 16;
    const int64_t kb = blockIdx.x % KB, nbg = blockIdx.x / KB;
    const int nb = (int)(NBT - nbg * kCastNB < kCastNB ? NBT - nbg * kCastNB : kCastNB);
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int q = t + kNzThreads * u, b = q >> 6, l = q & 63;
        if (b < nb)
            *reinterpret_cast<u32x4*>(&blk[b][4 * l]) =
                *reinterpret_cast<const u32x4*>(nz + (((nbg * kCastNB + b) * KB + kb) * 64 + l) * 16);
    }
    __syncthreads();
    // thread -> 4-column group w (columns 4w..4w+3 of the tile: block w>>2) and 4-row groups rq
    const int w = t & 63, b = w >> 2;
    if (b >= nb) return;
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int rq = (t >> 6) + 4 * pass;  // rows 4rq..4rq+3 of the K block
        uint32_t r[4], o[4];                 // r[e]: rows 4rq..+3 of column 4w+e (dword rq&3 of its lane)
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = blk[b][4 * ((4 * w + e) % 16 + 16 * (rq >> 2)) + (rq & 3)];
        bytes4x4(r, o);                      // o[kk]: columns 4w..4w+3 of row 4rq+kk
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            *reinterpret_cast<uint32_t*>(nd + (kb * 64 + 4 * rq + kk) * N + nbg * (16 * kCastNB) + 4 * w) = o[kk];
    }
}

// int8 ND [K, N] -> NZ: the inverse tile.
__global__ __launch_bounds__(kNzThreads) void w8_nz_pack_kernel(const int8_t* __restrict__ nd, int64_t K, int64_t N,
                                                                int8_t* __restrict__ nz) {
    __shared__ uint32_t rows[64][4 * kCastNB + 1];
    const int64_t KB = K / 64, NBT = N / 16;
    const int64_t kb = blockIdx.x % KB, nbg = blockIdx.x / KB;
    const int nb = (int)(NBT - nbg * kCastNB < kCastNB ? NBT - nbg * kCastNB : kCastNB);
    const int nw = 4 * nb, t = threadIdx.x;
    if ((uintptr_t)nd % 16 == 0) {
        // 16-byte loads (N % 16 == 0, so every row and every 16-column block starts on 16 bytes): 4 per thread
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = t + kNzThreads * u, r = e >> 4, v = e & 15;
            if (4 * v < nw) {
                const u32x4 d =
                    *reinterpret_cast<const u32x4*>(nd + (kb * 64 + r) * N + nbg * (16 * kCastNB) + 16 * v);
#pragma unroll
                for (int i = 0; i < 4; ++i) rows[r][4 * v + i] = d[i];
            }
        }
    } else {
        for (int e = t; e < 64 * 4 * kCastNB; e += kNzThreads) {  // one dword per lane: 256-byte row pieces
            const int r = e >> 6, w = e & 63;
            if (w < nw)
                rows[r][w] = *reinterpret_cast<const uint32_t*>(nd + (kb * 64 + r) * N + nbg * (16 * kCastNB) + 4 * w);
        }
    }
    __syncthreads();
    // thread -> (block b, 16-row group g, 4-column group cg): the whole 16-byte chunks of lanes 4cg + e + 16g,
    // e = 0..3 (64 contiguous bytes; the 4 threads of one (b, g) write 256)
    const int b = t >> 4, g = (t >> 2) & 3, cg = t & 3;
    if (b >= nb) return;
    uint32_t o[4][4];  // o[e][dw]: rows 16g + 4dw .. +3 of column 4cg + e
#pragma unroll
    for (int dw = 0; dw < 4; ++dw) {
        uint32_t r[4], c[4];  // r[kk]: columns 4cg..+3 of row 16g + 4dw + kk
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) r[kk] = rows[16 * g + 4 * dw + kk][4 * b + cg];
        bytes4x4(r, c);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e][dw] = c[e];
    }
    int8_t* dst = nz + (((nbg * kCastNB + b) * KB + kb) * 64 + 4 * cg + 16 * g) * 16;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        *reinterpret_cast<u32x4*>(dst + 16 * e) = (u32x4){o[e][0], o[e][1], o[e][2], o[e][3]};
}

// int8 [N, K] -> [K, N] (the row-major weight the prefill kernels read), for the shapes the decode kernel's
// in-place read of an [N, K] weight does not take.  A 64 x 64 tile per workgroup through LDS: each thread moves
// 16 bytes of a source row in (one 16-byte load where the row piece is whole and aligned) and 16 bytes of a
// destination row out; the ragged edges go byte by byte.
constexpr int kTrT = 64;
__global__ __launch_bounds__(kNzThreads) void w8_nk_transpose_kernel(const int8_t* __restrict__ src, int64_t K,
                                                                     int64_t N, int8_t* __restrict__ dst) {
    __shared__ int8_t tile[kTrT][kTrT + 4];
    const int64_t k0 = (int64_t)blockIdx.x * kTrT, n0 = (int64_t)blockIdx.y * kTrT;
    const int t = threadIdx.x, r = t >> 2, q = 16 * (t & 3);
    {   // source row n0 + r, bytes k0 + q .. +15
        const int64_t n = n0 + r, k = k0 + q;
        const int8_t* sp = src + n * K + k;
        if (n < N && k + 16 <= K && ((uintptr_t)sp & 15) == 0) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(sp);
#pragma unroll
            for (int e = 0; e < 16; ++e) tile[r][q + e] = (int8_t)(v[e >> 2] >> (8 * (e & 3)));
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) tile[r][q + e] = (n < N && k + e < K) ? sp[e] : (int8_t)0;
        }
    }
    __syncthreads();
    {   // destination row k0 + r, bytes n0 + q .. +15: column r of the tile, rows q .. q+15
        const int64_t k = k0 + r, n = n0 + q;
        int8_t* dp = dst + k * N + n;
        if (k >= K) return;
        if (n + 16 <= N && ((uintptr_t)dp & 15) == 0) {
            u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e >> 2] |= (uint32_t)(uint8_t)tile[q + e][r] << (8 * (e & 3));
            *reinterpret_cast<u32x4*>(dp) = v;
        } else {
            for (int e = 0; e < 16 && n + e < N; ++e) dp[e] = tile[q + e][r];
        }
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

// Eight int8 weights (two dwords, 8 consecutive rows of one column) as a
// 16-bit MFMA operand of offset-binary values u = w + 128 (BASE 128): each
// byte converts exactly to float (v_cvt_f32_ubyte) and from there to
// bf16 (the upper half: u <= 255 fits 8 significant bits) or fp16.
template <int DT>
__device__ __forceinline__ u32x4 nz8_operand(uint32_t lo, uint32_t hi) {
    const uint32_t flip = __builtin_amdgcn_readfirstlane(0x80808080u);
    const uint32_t w[2] = {lo ^ flip, hi ^ flip};
    u32x4 b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t src = w[q >> 1];
        const float f0 = (float)((src >> (16 * (q & 1))) & 0xffu);
        const float f1 = (float)((src >> (16 * (q & 1) + 8)) & 0xffu);
        if constexpr (DT == QK_BF16)
            b[q] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
        else
            b[q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f0, f1));
    }
    return b;
}

// NB: n-blocks per workgroup (the last workgroups may own one fewer: their
// extra block repeats a real one and is not stored).  NIT: superblocks per
// wave.  The grid is (workgroups along N) x (16-row blocks of M); a
// workgroup has K / (128 * NIT) waves.
// * The x rows of a superblock (16 rows x 256 bytes) come into the wave's own
//   LDS slot by four direct-to-LDS loads of four whole rows each (whole
//   128-byte lines; loads into VGPRs in the MFMA's lane order would touch 16
//   half lines per instruction), and the A operands are read back from there.
//   Superblock it's DMAs have landed once at most the vector-memory loads
//   issued after them are outstanding (the wave waits on vmcnt itself; the
//   compiler does not count these loads).
// * The packed weights are read once, with the non-temporal hint, so that
//   they stream past the L2 instead of evicting the x rows every workgroup of
//   the XCD reads again (measured: 8.5 -> 7.4 us on the cfg3 decode shape,
//   with either change alone about half of that).
// * A superblock's scale and offset rows (the workgroup's NB*16 columns of
//   one group) come in with one 16-byte load per fetching lane and reach the
//   other lanes through the wave's own LDS slot.
// * The waves' sums meet in LDS (each wave's in its own x slots, which it no
//   longer reads) and are added in K order.
// W8: int8 NZ weights (two 1 KB blocks per 128 rows; the operand of 16-bit MFMA
// step j is rows 16g + 8*(j&1) .. +8 of block j>>1, and its A operand is
// x[m, 128s + 64*(j>>1) + 16g + 8*(j&1) ..]).
constexpr int kNzXSlot = 4096;  // bytes of x per superblock and wave: 16 rows x 256 bytes

// s_waitcnt vmcnt(n) for a value known after unrolling; "memory" keeps the LDS reads after it
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
#define QK_WAIT_CASE(v) \
    case v: asm volatile("s_waitcnt vmcnt(" #v ")" ::: "memory"); break;
        QK_WAIT_CASE(0) QK_WAIT_CASE(1) QK_WAIT_CASE(2) QK_WAIT_CASE(3) QK_WAIT_CASE(4) QK_WAIT_CASE(5)
        QK_WAIT_CASE(6) QK_WAIT_CASE(7) QK_WAIT_CASE(8) QK_WAIT_CASE(9) QK_WAIT_CASE(10) QK_WAIT_CASE(11)
        QK_WAIT_CASE(12) QK_WAIT_CASE(13) QK_WAIT_CASE(14) QK_WAIT_CASE(15) QK_WAIT_CASE(16) QK_WAIT_CASE(17)
        QK_WAIT_CASE(18) QK_WAIT_CASE(19) QK_WAIT_CASE(20) QK_WAIT_CASE(21) QK_WAIT_CASE(22) QK_WAIT_CASE(23)
#undef QK_WAIT_CASE
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

// SDT: the dtype of the scale and offset rows (QK_F16 or QK_BF16), fixed at compile time.
// NK (int8 only): the weight is stored [N, K] (row n holds column n's K bytes, the nn.Linear layout) instead
// of in NZ blocks.  The 16 bytes lane (c, g) takes from an NZ block -- rows 16g..16g+15 of column c -- are
// contiguous in such a row, so the same loads read it in place: per lane c*K + 16g, per 64-row block
// 16*K*(n-block) + 64*(K block).  The two 64-row blocks of a superblock are the two halves of each
// column's 128-byte line, loaded back to back.
template <int DT, int NB, int NIT, bool HAS_OFF, bool W8, int SDT, bool NK = false>
__global__ __launch_bounds__(64 * kNzMaxWaves) void w4nz_decode(WqbmmArgs p, int nwg, int nrb) {
    typedef Mfma<DT> MM;
    constexpr int WL = W8 ? 2 : 1;         // weight loads per block and superblock
    constexpr int PF = NIT < 2 ? NIT : 2;  // superblocks in flight per wave
    constexpr int SL = PF;                 // x slots and scale rows per wave
    constexpr int NT = HAS_OFF ? 2 : 1;    // scale rows per superblock (scale, offset)
    constexpr int RL = 2 * NB;             // 16-byte pieces of one row (NB*16 columns)
    constexpr int GRP = 5 + NB * WL;       // vector-memory loads per superblock: 4 x DMAs, scale rows, weights
    static_assert(NT * RL <= 64, "one load instruction fetches a superblock's scale rows");
    // per wave: its x slots, later its partial sums (NB tiles of kNzTilePitch floats)
    constexpr int WSLOT = SL * kNzXSlot > NB * kNzTilePitch * 4 ? SL * kNzXSlot : NB * kNzTilePitch * 4;
    __shared__ __attribute__((aligned(16))) char xbuf[kNzMaxWaves * WSLOT];
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

    // x DMA q of a superblock: rows 4q .. 4q+3 of the row block, lane -> (row 4q + lane/16, 16-byte piece
    // lane%16); rows past M read row M-1 (each output row depends on its own x row only) and are not stored
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
    uint32_t x_dma[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int row = rb * 16 + 4 * q + (lane >> 4);
        x_dma[q] = (uint32_t)(row < M ? row : M - 1) * (uint32_t)K * 2u + 16u * (uint32_t)(lane & 15);
    }
    char* const xw = xbuf + wave * WSLOT;
    const uint32_t xw_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)xbuf + (uint32_t)(wave * WSLOT);
    static_assert(!NK || W8, "the [N, K] layout is an int8 weight's");
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (uint32_t)K * (uint32_t)N / (W8 ? 1u : 2u));
    const uint32_t w_lane = NK ? (uint32_t)c * (uint32_t)K + 16u * (uint32_t)g : (uint32_t)lane * 16u;
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

    u32x4 wv[SL][NB][WL], sa[SL];
    // one superblock's loads in a fixed order: 4 x DMAs, the scale rows, the weights (non-temporal)
    auto issue = [&](int it) {
        asm volatile("" ::: "memory");  // the LDS reads of the slot's previous superblock stay before its DMAs
        __builtin_amdgcn_sched_barrier(0);
        const int s = s0 + it, sl = it % SL;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            dma16(xr, xw_lds + (uint32_t)(sl * kNzXSlot + q * 1024), x_dma[q], (uint32_t)s * 256u);
        const uint32_t grp = (uint32_t)(s * 128) / (uint32_t)G;
        sa[sl] = *reinterpret_cast<const u32x4*>(sl_base + (size_t)grp * (uint32_t)N);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int h = 0; h < WL; ++h)
                wv[sl][b][h] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               wr, w_lane,
                               NK ? (uint32_t)blk[b] * 16u * (uint32_t)K + (uint32_t)(128 * s + 64 * h)
                                  : ((uint32_t)blk[b] * (uint32_t)(WL * S) + (uint32_t)(WL * s + h)) * 1024u,
                               kNonTemporal));
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int it = 0; it < PF; ++it) issue(it);

    const u32x4 ones = {MM::ONES, MM::ONES, MM::ONES, MM::ONES};
    constexpr float BASE = W8 ? 128.0f : MM::BASE;
    f32x4 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int sl = it % SL;
        // superblock it's x DMAs have landed: after them this wave issued its scale rows and weights and
        // the whole groups of the superblocks up to it + PF - 1
        const int later = (it + PF - 1 < NIT - 1 ? PF - 1 : NIT - 1 - it);
        wait_vmcnt(1 + NB * WL + later * GRP);
        // this superblock's scale rows through the wave's LDS slot
        if (lane < NT * RL) *reinterpret_cast<u32x4*>(&srow[wave][sl][0][0] + 8 * lane) = sa[sl];
        u32x4 xk[4], wk[NB][WL];
        const char* xrow = xw + sl * kNzXSlot + c * 256;  // x row c of the row block
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xk[j] = *reinterpret_cast<const u32x4*>(xrow + (W8 ? 128 * (j >> 1) + 32 * g + 16 * (j & 1) : 64 * j + 16 * g));
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int h = 0; h < WL; ++h) wk[b][h] = wv[sl][b][h];
        f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) xs = MM::mma(xk[j], ones, xs);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            f32x4 ag = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (W8)
                    ag = MM::mma(xk[j], nz8_operand<DT>(wk[b][j >> 1][2 * (j & 1)], wk[b][j >> 1][2 * (j & 1) + 1]),
                                 ag);
                else
                    ag = MM::mma(xk[j], nz_operand<MM::MAGIC>(wk[b][0][j]), ag);
            }
            const float sf = load_half_bits(srow[wave][sl][0][16 * b + c], SDT);
            const float of = HAS_OFF ? load_half_bits(srow[wave][sl][NT - 1][16 * b + c], SDT) : 0.0f;
            const float sx = sf * (of - BASE);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[b][r] = __builtin_fmaf(sf, ag[r], __builtin_fmaf(sx, xs[r], acc[b][r]));
        }
        // the x reads of slot sl were consumed by the MFMAs above, so its next DMA may land
        if (it + PF < NIT) issue(it + PF);
    }

    // partial sums of wave w: NB tiles at xbuf + w * WSLOT; lane (c, g) holds rows 4g..4g+3 of column c of
    // each block, row r of a tile sits at 16*(r + r/4) + column, so the 64 lanes of one store hit 64 banks.
    // The K ranges of waves a short K leaves out add as zeros.
    for (int w = nwave + wave; w < kNzMaxWaves; w += nwave)
        for (int e = lane; e < NB * kNzTilePitch; e += 64) reinterpret_cast<float*>(xbuf + w * WSLOT)[e] = 0.0f;
    float* const red = reinterpret_cast<float*>(xw);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[b * kNzTilePitch + 16 * (5 * g + r) + c] = acc[b][r];
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // the waves' K ranges are added in K order; all 16 reads are issued before the adds
    const int nb = b1 - b0;
    for (int t = threadIdx.x; t < NB * 256; t += blockDim.x) {
        const int b = t >> 8, row = (t >> 4) & 15, col = t & 15;
        const int at = b * kNzTilePitch + 16 * (row + (row >> 2)) + col;
        float part[kNzMaxWaves];
#pragma unroll
        for (int w = 0; w < kNzMaxWaves; ++w) part[w] = reinterpret_cast<const float*>(xbuf + w * WSLOT)[at];
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

// ---------------------------------------------------------------------------
// Prefill on an int4 NZ weight (M > 64): a 128 x 256 output tile per 512-thread
// workgroup, K in steps of 128 (one NZ block row).  Per step, DMAs
// (buffer_load_dwordx4 ... lds, counted with each wave's own vmcnt waits) bring
// the tile's 128 activation rows ([row][256 B], chunk c of row r at
// r*256 + 16*(c ^ (r & 15))), its 16 NZ weight blocks (1 KB each, copied as
// they are: a lane's 16 bytes of a block are its B operands for the step's
// four MFMA k-steps) and the step's group rows (scale and offset of the 256
// columns, x group sums of the 128 rows) into a ring of three LDS stages, two
// ahead.  Wave w owns all 128 rows and columns 32w..32w+31 (its two NZ blocks,
// unpacked once, in registers, by the magic-number conversion): 8 x 2 MFMA
// tiles accumulate the group's raw sums ag, and at each group's end
// acc += s * ag + s * (offset - BASE) * xsum (the decode kernel's algebra).
// The output tile is staged through LDS for 16-byte row stores.
namespace nzg {
constexpr int BM = 128, BN = 256, KS = 128, NT = 512, NSTG = 3;
constexpr int X_BYTES = BM * KS * 2;          // 32 KB
constexpr int W_BYTES = (BN / 16) * 1024;     // 16 KB
constexpr int SC_BYTES = 3072;                // scale row, offset row, x group sums
constexpr int STAGE = X_BYTES + W_BYTES + SC_BYTES;
constexpr int RING = NSTG * STAGE;            // 153 KB
constexpr int OROWB = 2 * BN + 16;            // padded output staging row (bytes)
constexpr int SMEM = RING > BM * OROWB ? RING : BM * OROWB;
static_assert(SMEM <= 160 * 1024, "LDS");
// int8 NZ weights (W8A16): 64-row steps, so a step's weight is again one 1 KB NZ block per 16 columns and its
// activation rows are 128 bytes
constexpr int KS8 = 64;
constexpr int X8_BYTES = BM * KS8 * 2;        // 16 KB
constexpr int STAGE8 = X8_BYTES + W_BYTES + SC_BYTES;
constexpr int RING8 = NSTG * STAGE8;          // 105 KB
constexpr int SMEM8 = RING8 > BM * OROWB ? RING8 : BM * OROWB;
}  // namespace nzg

// G1: the group is one step (G == the step's K), so every step starts a group: its first MFMAs take a zero
// accumulator and each row tile is folded right after its last MFMAs, between the later tiles' MFMAs.
// W8: an int8 NZ weight ([N/16][K/64][64][16]).  A step is 64 rows: one 1 KB block per 16 columns (the int4
// step's DMA pattern), 128-byte activation rows (chunk c of row r at r*128 + 16*(c ^ (r & 7))), two MFMA k-steps.
// The B operand of k-step t is rows 16g + 8t .. +8 of the lane's block column (lane c + 16g holds rows 16g ..
// 16g+15), converted to offset-binary 16-bit values w + 128 (exact); the A operand is the matching 16 bytes of x,
// k = 16g + 8t .. +8, so both operands run over the step's 64 k in the same permuted order.  The fold's base is
// 128 instead of the int4 magic base.
template <int DT, bool HAS_OFF, bool G1, bool W8 = false, bool SK = false>
__global__ __launch_bounds__(nzg::NT) void w4nz_gemm(WqbmmArgs p, int tiles_m, int tiles_n,
                                                     const float* __restrict__ xsum, uint64_t* __restrict__ ctr,
                                                     float* __restrict__ part, uint64_t tag, int tail_first,
                                                     int dp_rounds) {
    typedef Mfma<DT> MM;
    using namespace nzg;
    constexpr int TM = 8, TN = 2;
    constexpr int NSC = HAS_OFF ? 3 : 2;  // group-row DMAs per step: waves 0 .. NSC-1 issue one each
    constexpr int KSW = W8 ? KS8 : KS;           // K rows per step
    constexpr int XB = W8 ? X8_BYTES : X_BYTES;  // activation bytes per stage
    constexpr int STG = XB + W_BYTES + SC_BYTES;
    constexpr int NKT = KSW / 32;                // MFMA k-steps per step
    constexpr float BASE = W8 ? 128.0f : MM::BASE;
    __shared__ __attribute__((aligned(1024))) char smem[W8 ? SMEM8 : SMEM];

    const int M = (int)p.M, N = (int)p.N, K = (int)p.K, G = (int)p.group;
    const int kb_n = K / KSW;                 // NZ blocks along K per column block
    const int gsteps = G / KSW, nu = K / G;   // steps per group; groups per tile
    const int ntiles = tiles_m * tiles_n;
    // tile t -> (tm, tn): groups of 8 row tiles, row tile fastest, so neighbouring tiles share a column block
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    auto tile_mn = [&](int t, int& tm, int& tn) {
        const int first_m = (t / per_group) * GM;
        const int gm = min(tiles_m - first_m, GM);
        tm = first_m + (t % per_group) % gm;
        tn = (t % per_group) / gm;
    };

    // The workgroup's segments, in the order it runs them.  Whole tiles: one, the workgroup's own.  Stream-K
    // (P workgroups, one per CU, workgroup r = the XCD-swizzled block index): first dp_rounds whole tiles in
    // lockstep (tile seg * P + r), then range r of the other tiles' U = (ntiles - D) * nu groups, tile-major,
    // r * U / P .. (r+1) * U / P.  A range runs first the head of the tile it ends in (groups 0 .. ub of tile
    // tb, handed on to range r + 1 through partial slot r), then its whole tiles, then the tail of the tile it
    // starts in (groups ua .. nu of tile ta), which continues from range r - 1's head.  Each tile has at most
    // two segments (a range holds at least one tile's groups).
    int r = 0, ta = 0, ua = 0, tb = 0, ub = 0, nseg = 1;
    bool has_head = false, has_tail = false;
    const int P = (int)gridDim.x;
    if constexpr (SK) {
        r = xcd_swizzle(blockIdx.x, P);
        const int D = dp_rounds * P;  // tiles run whole first, one per workgroup per round (lockstep)
        const int64_t U = (int64_t)(ntiles - D) * nu;
        const int64_t a = (int64_t)r * U / P, b = (int64_t)(r + 1) * U / P;
        ta = D + (int)(a / nu);
        ua = (int)(a % nu);
        tb = D + (int)((b - 1) / nu);
        ub = (int)(b - (int64_t)(tb - D) * nu);
        has_head = ub < nu;
        has_tail = ua != 0;
        nseg = dp_rounds + (int)has_head + (tb - (int)has_head) - (ta + (int)has_tail) + 1 + (int)has_tail;
    } else {
        ta = xcd_swizzle(blockIdx.x, ntiles);
    }

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 15, g4 = lane >> 4;
    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;
    const uint32_t ldx = (uint32_t)K * 2u;
    // int4: an instruction covers rows 4q..4q+3: lane l -> row 4q + (l>>4), LDS chunk l&15, k chunk
    // (l&15) ^ (row&15); W8: rows 8q..8q+7: lane l -> row 8q + (l>>3), LDS chunk l&7, k chunk (l&7) ^ (row&7)
    auto vx = [&](int q) {
        if constexpr (W8) {
            const int row = 8 * q + (lane >> 3);
            return (uint32_t)row * ldx + 16u * (uint32_t)((lane & 7) ^ (row & 7));
        } else {
            const int row = 4 * q + (lane >> 4);
            return (uint32_t)row * ldx + 16u * (uint32_t)((lane & 15) ^ (row & 15));
        }
    };
    // group rows: 512 bytes each (lanes 32..63 repeat 0..31 into the unused upper half of the KB)
    const uint32_t nsb = (uint32_t)(K / G) * (uint32_t)N * 2u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scale, nsb);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(HAS_OFF ? p.offset : p.scale, nsb);
    const __amdgpu_buffer_rsrc_t rxs = make_rsrc(xsum, (uint32_t)(K / G) * (uint32_t)M * 4u);
    const uint32_t l32 = 16u * (uint32_t)(lane & 31);
    // stream-K partial slots: slot [wave][row tile][column tile][lane] x 16 B, whole KB per store instruction
    constexpr uint32_t SLOT = BM * BN * 4;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, SK ? (uint32_t)(gridDim.x - 1) * SLOT : 0u);
    auto part_off = [&](int slot, int i, int j) {
        return (uint32_t)slot * SLOT + (uint32_t)((wave * TM * TN + i * TN + j) * 1024 + 16 * lane);
    };

    for (int seg = 0; seg < nseg; ++seg) {
        int t = ta, u0 = 0, u1 = nu;
        bool head = false, tail = false;
        if constexpr (SK) {
            // first the lockstep rounds; then the stream-K share.  tail_first (a debug order): the tail
            // segment first, then the head, then the whole tiles
            const int sg = seg - dp_rounds;
            const int hs = tail_first ? (int)has_tail : 0;                 // the head's position
            const int ts = tail_first ? 0 : nseg - dp_rounds - 1;            // the tail's position
            const int fs = tail_first ? (int)has_tail + (int)has_head : (int)has_head;  // the first whole tile's
            if (sg < 0) {
                t = seg * P + r;
            } else if (has_head && sg == hs) {
                t = tb;
                u1 = ub;
                head = true;
            } else if (has_tail && sg == ts) {
                u0 = ua;
                tail = true;
            } else {
                t = ta + (int)has_tail + sg - fs;
            }
        }
        int tm, tn;
        tile_mn(t, tm, tn);
        const int m0 = tm * BM, n0 = tn * BN;
        const int rows = M - m0 < BM ? M - m0 : BM;
        // activations: rows past M read as zeros (range-checked offsets), K*2 bytes per row
        const __amdgpu_buffer_rsrc_t rx =
            make_rsrc(static_cast<const char*>(p.x) + (size_t)m0 * ldx, (uint32_t)(rows - 1) * ldx + ldx);
        // the 16 NZ blocks of the column block: block i of step s at ((n0/16 + i) * kb_n + s) KB
        const __amdgpu_buffer_rsrc_t rw =
            make_rsrc(static_cast<const char*>(p.w) + (size_t)(n0 / 16) * kb_n * 1024, (uint32_t)(16 * kb_n * 1024));

        auto issue = [&](int s) {
            const uint32_t base = sbase + (uint32_t)(s % NSTG) * STG;
#pragma unroll
            for (int u = 0; u < XB / 8192; ++u) {  // the stage's activation rows, 1 KB per DMA
                const int q = wave + 8 * u;
                dma16(rx, base + (uint32_t)q * 1024u, vx(q), (uint32_t)s * (uint32_t)(KSW * 2));
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int i = wave + 8 * u;
                dma16(rw, base + XB + (uint32_t)i * 1024u, (uint32_t)i * (uint32_t)kb_n * 1024u + 16u * lane,
                      (uint32_t)s * 1024u);
            }
            const uint32_t g = (uint32_t)(s * KSW / G);
            const uint32_t sdst = base + XB + W_BYTES;
            if (wave == 0) dma16(rs, sdst, (g * (uint32_t)N + (uint32_t)n0) * 2u + l32, 0);
            if (HAS_OFF && wave == 1) dma16(ro, sdst + 1024u, (g * (uint32_t)N + (uint32_t)n0) * 2u + l32, 0);
            if (wave == NSC - 1) dma16(rxs, sdst + 2048u, (g * (uint32_t)M + (uint32_t)m0) * 4u + l32, 0);
        };

        f32x4 acc[TM][TN], ag[TM][TN];
        const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = ag[i][j] = zero4;
        int s0 = u0 * gsteps;
        const int s1 = u1 * gsteps;
        if constexpr (SK) {
            if (tail) {
                // continue from range r - 1's head if it has arrived (the usual case: it ran first there);
                // otherwise run the whole tile here.  Either way the groups fold in order from zero.
                if (splitk_last(ctr + (r - 1), 2u, tag)) {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rp, part_off(r - 1, i, j), 0,
                                                                                  kCoherent);
                            acc[i][j] = __builtin_bit_cast(f32x4, v);
                        }
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
                } else {
                    s0 = 0;
                }
            }
        }

        const bool more = wave < NSC;  // this wave issues one more DMA per step
        for (int s = s0; s < s0 + 2 && s < s1; ++s) issue(s);
        for (int s = s0; s < s1; ++s) {
            // stage s has landed once at most stage s+1's DMAs are outstanding
            if (s + 1 < s1) {  // one step's DMAs: XB / 8 KB activation, 2 weight (+1 group row for waves < NSC)
                constexpr int PER = XB / 8192 + 2;
                if (more) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER + 1));
                else __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            }
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();  // stage s visible to every wave; every wave is done with stage s-1
            __builtin_amdgcn_sched_barrier(0);
            if (s + 2 < s1) issue(s + 2);  // into the buffer of stage s-1
            const char* As = smem + (s % NSTG) * STG;
            const char* Bs = As + XB;
            u32x4 bw[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bw[j] = *reinterpret_cast<const u32x4*>(Bs + (2 * wave + j) * 1024 + 16 * lane);
            const char* sc = As + XB + W_BYTES;
            // the group's per-column factors s and s * (offset - BASE) of this wave's columns
            auto col_factors = [&](float (&sf)[TN], float (&sx)[TN]) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int col = 32 * wave + 16 * j + fr;
                    sf[j] = load_half_bits(*reinterpret_cast<const uint16_t*>(sc + 2 * col), p.s_dtype);
                    const float of = HAS_OFF
                                         ? load_half_bits(*reinterpret_cast<const uint16_t*>(sc + 1024 + 2 * col),
                                                          p.s_dtype)
                                         : 0.0f;
                    sx[j] = sf[j] * (of - BASE);
                }
            };
            auto fold_row = [&](int i, const float (&sf)[TN], const float (&sx)[TN]) {
                const f32x4 xs = *reinterpret_cast<const f32x4*>(sc + 2048 + 4 * (16 * i + 4 * g4));
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[i][j][q] = __builtin_fmaf(sf[j], ag[i][j][q], __builtin_fmaf(sx[j], xs[q], acc[i][j][q]));
            };
            // k-step t's operands: the activation fragments of the wave's 8 row tiles, the weight of its 2 blocks
            auto a_frag = [&](int i, int kt) {
                const int rr = 16 * i + fr;
                if constexpr (W8)
                    return *reinterpret_cast<const u32x4*>(As + rr * 128 + 16 * ((2 * g4 + kt) ^ (rr & 7)));
                else
                    return *reinterpret_cast<const u32x4*>(As + rr * 256 + 16 * ((4 * kt + g4) ^ (rr & 15)));
            };
            auto b_op = [&](int j, int kt) {
                if constexpr (W8) return nz8_operand<DT>(bw[j][2 * kt], bw[j][2 * kt + 1]);
                else return nz_operand<MM::MAGIC>(bw[j][kt]);
            };
            if constexpr (G1) {
                float sf[TN], sx[TN];
                col_factors(sf, sx);
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    u32x4 af[TM], b[TN];
#pragma unroll
                    for (int i = 0; i < TM; ++i) af[i] = a_frag(i, kt);
#pragma unroll
                    for (int j = 0; j < TN; ++j) b[j] = b_op(j, kt);
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
#pragma unroll
                        for (int j = 0; j < TN; ++j) ag[i][j] = MM::mma(af[i], b[j], kt == 0 ? zero4 : ag[i][j]);
                        if (kt == NKT - 1 && i >= 2) fold_row(i - 2, sf, sx);  // two row tiles behind the MFMAs
                    }
                }
                fold_row(TM - 2, sf, sx);
                fold_row(TM - 1, sf, sx);
                continue;
            }
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                u32x4 af[TM], b[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) af[i] = a_frag(i, kt);
#pragma unroll
                for (int j = 0; j < TN; ++j) b[j] = b_op(j, kt);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) ag[i][j] = MM::mma(af[i], b[j], ag[i][j]);
            }
            if (((s + 1) * KSW) % G == 0) {  // the group ends with this step: fold it into acc
                float sf[TN], sx[TN];
                col_factors(sf, sx);
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    fold_row(i, sf, sx);
#pragma unroll
                    for (int j = 0; j < TN; ++j) ag[i][j] = zero4;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();  // every wave is past its last reads of the ring

        if constexpr (SK) {
            if (head) {  // hand the folded groups 0 .. ub to range r + 1 (stores through the L2), then arrive
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), rp,
                                                               part_off(r, i, j), 0, kCoherent);
                splitk_last(ctr + r, 2u, tag);
                continue;
            }
        }

        // ---- epilogue: + bias, cast, staged through LDS for 16-byte row stores
        float bv[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bv[j] = p.bias_dtype ? load_scalar(p.bias, n0 + 32 * wave + 16 * j + fr, p.bias_dtype) : 0.0f;
        uint16_t* ot = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = 16 * i + 4 * g4 + q;
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const float v = acc[i][j][q] + bv[j];
                    ot[row * (OROWB / 2) + 32 * wave + 16 * j + fr] =
                        (uint16_t)(p.out_dtype == QK_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
                }
            }
        __syncthreads();
        constexpr int CPRO = 2 * BN / 16;  // 16-byte chunks per output row
        for (int q = tid; q < BM * CPRO; q += NT) {
            const int row = q / CPRO, c = q % CPRO;
            if (row >= rows) break;
            const u32x4 v = *reinterpret_cast<const u32x4*>(smem + row * OROWB + 16 * c);
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.out) +
                                                                    (size_t)(m0 + row) * N + n0 + 8 * c));  // written once
        }
        if constexpr (SK) __syncthreads();  // the staging is read before the next segment's DMAs land
    }
}

// The most blocks per workgroup that a wave of `nit` superblocks holds in registers without
// spilling (two superblocks in flight, NB accumulators): int4, 4 up to 3 superblocks, 3 for 4, 2 for 5,
// 1 beyond; int8 (two loads per block), 3 up to 2 superblocks, 2 for 3, 1 beyond.  Only these
// (NB, NIT) pairs are built.
constexpr int nz_max_blocks(int nit, bool w8) {
    return w8 ? (nit <= 2 ? 3 : nit == 3 ? 2 : 1) : (nit <= 3 ? 4 : nit == 4 ? 3 : nit == 5 ? 2 : 1);
}

struct NzPlan {
    bool ok;
    int nb, nit, nwave, nwg, nrb;
};

NzPlan nz_plan(const WqbmmArgs& p) {
    NzPlan z{false, 0, 0, 0, 0, 0};
    const int64_t G = p.group == 0 ? p.K : p.group;
    const bool w8 = p.w_dtype == QK_I8_NZ || p.w_dtype == QK_I8_NK;
    if (!(p.w_dtype == QK_I4_NZ || w8) || p.M <= 0 || p.M > 64 || p.N <= 0 || p.K <= 0) return z;
    if (p.N % 16 != 0 || p.K % 128 != 0 || G <= 0 || G % 128 != 0 || p.K % G != 0) return z;
    // 32-bit buffer offsets
    if (p.K * p.N >= ((int64_t)1 << 31) || p.M * p.K * 2 >= ((int64_t)1 << 31) ||
        (p.K / G) * p.N * 2 >= ((int64_t)1 << 31))
        return z;
    if ((uintptr_t)p.x % 16 != 0 || (uintptr_t)p.w % 16 != 0 || (uintptr_t)p.scale % 16 != 0 ||
        (uintptr_t)p.out % 2 != 0 || (p.offset && (uintptr_t)p.offset % 16 != 0))
        return z;
    const int64_t S = p.K / 128, NBT = p.N / 16;
    // superblocks per wave: the fewest that give at most 16 waves and split K evenly
    int nit = 0;
    const int want = plan_override().w4nz_nit;  // debug override: superblocks per wave
    for (int t = 1; t <= 8; ++t)
        if (S % t == 0 && S / t <= kNzMaxWaves && (want == 0 || t == want)) {
            nit = t;
            break;
        }
    if (nit == 0) return z;
    z.nit = nit;
    z.nwave = (int)(S / nit);
    z.nrb = (int)((p.M + 15) / 16);
    // blocks per workgroup: what one workgroup per CU needs, within what fits the wave's registers
    // (nz_max_blocks); then as few workgroups as give no workgroup more blocks than that
    const int cap = nz_max_blocks(nit, w8);
    int64_t nb = (NBT + 255) / 256;
    if (const int f = plan_override().w4nz_wg) nb = (NBT + f - 1) / f;  // debug override: a workgroup count
    if (nb > cap) nb = cap;
    z.nb = (int)nb;
    z.nwg = (int)((NBT + nb - 1) / nb);
    z.ok = (int64_t)z.nwg * z.nrb < ((int64_t)1 << 31) && ((int64_t)z.nwg + 1) * NBT < ((int64_t)1 << 31);
    return z;
}

template <int DT, int NB, int NIT, bool OFF, bool W8, bool NK>
hipError_t launch_nz_k(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    if constexpr (NB <= nz_max_blocks(NIT, W8)) {
        const dim3 grid((uint32_t)(z.nwg * z.nrb)), block((uint32_t)(64 * z.nwave));
        if (p.s_dtype == QK_BF16)
            w4nz_decode<DT, NB, NIT, OFF, W8, QK_BF16, NK><<<grid, block, 0, stream>>>(p, z.nwg, z.nrb);
        else
            w4nz_decode<DT, NB, NIT, OFF, W8, QK_F16, NK><<<grid, block, 0, stream>>>(p, z.nwg, z.nrb);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;  // not planned (nz_plan caps NB by nz_max_blocks)
}

template <int DT, int NB, bool OFF, bool W8, bool NK>
hipError_t launch_nz_nit(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    switch (z.nit) {
    case 1: return launch_nz_k<DT, NB, 1, OFF, W8, NK>(p, z, stream);
    case 2: return launch_nz_k<DT, NB, 2, OFF, W8, NK>(p, z, stream);
    case 3: return launch_nz_k<DT, NB, 3, OFF, W8, NK>(p, z, stream);
    case 4: return launch_nz_k<DT, NB, 4, OFF, W8, NK>(p, z, stream);
    case 5: return launch_nz_k<DT, NB, 5, OFF, W8, NK>(p, z, stream);
    case 6: return launch_nz_k<DT, NB, 6, OFF, W8, NK>(p, z, stream);
    case 7: return launch_nz_k<DT, NB, 7, OFF, W8, NK>(p, z, stream);
    default: return launch_nz_k<DT, NB, 8, OFF, W8, NK>(p, z, stream);
    }
}

template <int DT, bool OFF, bool W8, bool NK = false>
hipError_t launch_nz_nb(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    switch (z.nb) {
    case 1: return launch_nz_nit<DT, 1, OFF, W8, NK>(p, z, stream);
    case 2: return launch_nz_nit<DT, 2, OFF, W8, NK>(p, z, stream);
    case 3: return launch_nz_nit<DT, 3, OFF, W8, NK>(p, z, stream);
    default: return launch_nz_nit<DT, 4, OFF, W8, NK>(p, z, stream);
    }
}

template <int DT>
hipError_t launch_nz_dt(const WqbmmArgs& p, const NzPlan& z, hipStream_t stream) {
    if (p.w_dtype == QK_I8_NK)
        return p.offset ? launch_nz_nb<DT, true, true, true>(p, z, stream)
                        : launch_nz_nb<DT, false, true, true>(p, z, stream);
    if (p.w_dtype == QK_I8_NZ)
        return p.offset ? launch_nz_nb<DT, true, true>(p, z, stream) : launch_nz_nb<DT, false, true>(p, z, stream);
    return p.offset ? launch_nz_nb<DT, true, false>(p, z, stream) : launch_nz_nb<DT, false, false>(p, z, stream);
}

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }


// bytes of the ND form of an NZ (or [N, K]) weight
size_t nd_weight_bytes(const WqbmmArgs& p) {
    return (size_t)(p.w_dtype == QK_I8_NZ || p.w_dtype == QK_I8_NK ? p.K * p.N : p.K * p.N / 2);
}

// Prefill plan on an int4 NZ weight: M > 64 with at least 96 tiles of 128 x 256, N % 256 == 0, groups of
// whole 128-row NZ blocks, 16-byte aligned operands and 32-bit buffer offsets.  The workspace holds the x
// group sums ([split counters, unused][fp32 [K/G][M]]).
struct NzGemmPlan {
    bool ok;
    int tiles_m, tiles_n;
};

NzGemmPlan nzg_plan(const WqbmmArgs& p) {
    NzGemmPlan g{false, 0, 0};
    const int64_t G = p.group == 0 ? p.K : p.group;
    const bool w8 = p.w_dtype == QK_I8_NZ;
    const int64_t ks = w8 ? nzg::KS8 : nzg::KS;  // K rows per step
    if (!(p.w_dtype == QK_I4_NZ || w8) || p.M <= 64 || p.N <= 0 || p.N % nzg::BN != 0 || p.K <= 0 || p.K % ks != 0)
        return g;
    if (G <= 0 || G % ks != 0 || p.K % G != 0) return g;
    if (p.M * p.K * 2 >= ((int64_t)1 << 31) || p.K * p.N / (w8 ? 1 : 2) >= ((int64_t)1 << 31) ||
        (p.K / G) * p.N * 2 >= ((int64_t)1 << 31) || (p.K / G) * p.M * 4 >= ((int64_t)1 << 31) ||
        p.M * p.N >= ((int64_t)1 << 31))
        return g;
    if (((uintptr_t)p.x | (uintptr_t)p.w | (uintptr_t)p.scale | (uintptr_t)p.out |
         (uintptr_t)(p.offset ? p.offset : p.scale)) % 16 != 0)
        return g;
    g.tiles_m = (int)((p.M + nzg::BM - 1) / nzg::BM);
    g.tiles_n = (int)(p.N / nzg::BN);
    // measured at N = 11008: from 86 tiles (M = 129-256) this kernel beats unpacking to ND and the row-major
    // kernels; with 43 (M = 65-128) the row-major split kernels are faster even after the unpack
    if ((int64_t)g.tiles_m * g.tiles_n < 64) return g;
    g.ok = true;
    return g;
}

// Stream-K schedule of the NZ prefill GEMM: one workgroup per CU takes an equal share of all tiles' groups,
// where whole tiles per workgroup would leave at least an eighth of the last round's CUs idle (cfg3, M = 2048:
// 688 tiles on 256 CUs, 2.69 rounds run as 3).  Needs at least one tile per CU (so a tile has at most two
// segments) and two groups per tile; at most 512 workgroups (one split-counter word per range boundary).
// The result bits do not depend on it: a split tile's second segment continues from the first one's folded
// fp32 accumulator (or runs the whole tile itself when the first has not arrived yet), so each output folds
// its groups in order from zero exactly as with whole tiles.
int nzg_stream_k_wgs(const WqbmmArgs& p, const NzGemmPlan& g) {
    if (plan_override().nzg_sk == 0) return 0;
    const int64_t G = p.group == 0 ? p.K : p.group;
    const int64_t nu = p.K / G, T = (int64_t)g.tiles_m * g.tiles_n;
    const int P = device_cus() < 512 ? device_cus() : 512;
    if (P < 2 || nu < 2 || T < P || T % P == 0) return 0;
    if ((((T + P - 1) / P) * P - T) * 8 < P) return 0;
    return P;
}

// Whole-tile rounds run before the stream-K share (all but the last one to two rounds' worth of tiles, the
// data-parallel + stream-K hybrid of Osama et al., "Stream-K: Work-centric Parallel Decomposition for Dense
// Matrix Multiplication on the GPU", 2023): in lockstep, the workgroups of an XCD read the same activation
// rows and weight blocks at about the same time (L2 hits), where stream-K ranges drift apart in K.  cfg3,
// M = 2048 (one box, three passes, 8 rotating int4 NZ weights): 195-197 us against 199-201 for stream-K
// throughout and 200-201 with whole tiles only.
int nzg_dp_rounds(const NzGemmPlan& g, int wgs) {
    const int most = (g.tiles_m * g.tiles_n) / wgs - 1;  // the stream-K share keeps a tile per workgroup
    const int want = plan_override().nzg_sk_dp;
    return want < 0 || want > most ? most : want;
}

// bytes of the stream-K partial slots: one folded 128 x 256 fp32 tile per range boundary
size_t nzg_stream_k_bytes(int wgs) { return wgs > 1 ? (size_t)(wgs - 1) * nzg::BM * nzg::BN * sizeof(float) : 0; }

size_t nzg_xsum_bytes(const WqbmmArgs& p) {
    const int64_t G = p.group == 0 ? p.K : p.group;
    return (size_t)(p.K / G) * (size_t)p.M * sizeof(float);
}

// [split counters][x group sums fp32 [K/G][M]][stream-K partial slots, when planned and stream_k]
size_t nzg_workspace(const WqbmmArgs& p, bool stream_k) {
    const size_t sk = stream_k ? nzg_stream_k_bytes(nzg_stream_k_wgs(p, nzg_plan(p))) : 0;
    return QK_SPLIT_COUNTER_BYTES + (sk ? round256(nzg_xsum_bytes(p)) + sk : nzg_xsum_bytes(p));
}

template <int DT, bool W8, bool SK>
void launch_nzg_k(const WqbmmArgs& p, const NzGemmPlan& g, const float* xsum, uint64_t* ctr, float* part, int wgs,
                  hipStream_t stream) {
    const dim3 grid((uint32_t)(SK ? wgs : g.tiles_m * g.tiles_n)), block(nzg::NT);
    const uint64_t tag = SK ? next_split_tag() : 0;
    const int tail_first = plan_override().nzg_sk == 2 ? 1 : 0;
    const auto k = p.group == (W8 ? nzg::KS8 : nzg::KS)
                       ? (p.offset ? w4nz_gemm<DT, true, true, W8, SK> : w4nz_gemm<DT, false, true, W8, SK>)
                       : (p.offset ? w4nz_gemm<DT, true, false, W8, SK> : w4nz_gemm<DT, false, false, W8, SK>);
    k<<<grid, block, 0, stream>>>(p, g.tiles_m, g.tiles_n, xsum, ctr, part, tag, tail_first,
                                  SK ? nzg_dp_rounds(g, wgs) : 0);
}

// The x group sums, then the GEMM.  ws: the call's workspace, whose counters open it; xsum inside it; the
// stream-K partial slots follow the group sums when ws_end leaves room for them.
template <int DT>
hipError_t launch_nzg_dt(const WqbmmArgs& p, const NzGemmPlan& g, char* ws, float* xsum, const char* ws_end,
                         hipStream_t stream) {
    hipError_t e = launch_w4_xsum(p, xsum, stream);
    if (e != hipSuccess) return e;
    int wgs = nzg_stream_k_wgs(p, g);
    char* part = reinterpret_cast<char*>(xsum) + round256(nzg_xsum_bytes(p));
    if (wgs && (part > ws_end || (size_t)(ws_end - part) < nzg_stream_k_bytes(wgs) ||
                (uintptr_t)part % 16 != 0))
        wgs = 0;
    uint64_t* ctr = reinterpret_cast<uint64_t*>(ws);
    float* pf = reinterpret_cast<float*>(part);
    if (p.w_dtype == QK_I8_NZ) {
        if (wgs) launch_nzg_k<DT, true, true>(p, g, xsum, ctr, pf, wgs, stream);
        else launch_nzg_k<DT, true, false>(p, g, xsum, ctr, pf, 0, stream);
    } else {
        if (wgs) launch_nzg_k<DT, false, true>(p, g, xsum, ctr, pf, wgs, stream);
        else launch_nzg_k<DT, false, false>(p, g, xsum, ctr, pf, 0, stream);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_w4_nz_cast(const int32_t* src, bool to_nz, int64_t K, int64_t N, int32_t* dst, hipStream_t stream) {
    if (K * N == 0) return hipSuccess;
    const int64_t tiles = (K / 128) * ((N / 16 + kCastNB - 1) / kCastNB);
    if (tiles >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    if (to_nz)
        w4_nz_pack_kernel<<<dim3((uint32_t)tiles), dim3(kNzThreads), 0, stream>>>(src, K, N, dst);
    else
        w4_nz_unpack_kernel<<<dim3((uint32_t)tiles), dim3(kNzThreads), 0, stream>>>(src, K, N, dst);
    return hipGetLastError();
}

hipError_t launch_w8_nk_transpose(const int8_t* src, int64_t K, int64_t N, int8_t* dst, hipStream_t stream) {
    if (K * N == 0) return hipSuccess;
    const int64_t gk = (K + kTrT - 1) / kTrT, gn = (N + kTrT - 1) / kTrT;
    if (gk >= ((int64_t)1 << 31) || gn > 65535) return hipErrorInvalidValue;
    w8_nk_transpose_kernel<<<dim3((uint32_t)gk, (uint32_t)gn), dim3(kNzThreads), 0, stream>>>(src, K, N, dst);
    return hipGetLastError();
}

hipError_t launch_w8_nz_cast(const int8_t* src, bool to_nz, int64_t K, int64_t N, int8_t* dst, hipStream_t stream) {
    if (K * N == 0) return hipSuccess;
    const int64_t tiles = (K / 64) * ((N / 16 + kCastNB - 1) / kCastNB);
    if (tiles >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    if (to_nz)
        w8_nz_pack_kernel<<<dim3((uint32_t)tiles), dim3(kNzThreads), 0, stream>>>(src, K, N, dst);
    else
        w8_nz_unpack_kernel<<<dim3((uint32_t)tiles), dim3(kNzThreads), 0, stream>>>(src, K, N, dst);
    return hipGetLastError();
}

// NZ weights (int4 QK_I4_NZ, int8 QK_I8_NZ): the decode kernel where it applies (no workspace);
// otherwise the weight is unpacked into the workspace and the row-major kernels run on it:
// [QK_SPLIT_COUNTER_BYTES, unused][ND weight][row-major call's workspace].
// An int8 [N, K] weight (QK_I8_NK) takes the same decode kernel (reading it in place) or is transposed into the
// workspace for the row-major kernels: [QK_SPLIT_COUNTER_BYTES, unused][[K, N] weight][row-major call's workspace].
// int8 NZ / [N,K] weights with 64 < M <= 192, or up to 256 where the NZ prefill kernel does not take the shape
// (it needs 64 tiles): the decode kernel on row chunks of at most 64, no workspace.  The alternative unpacks the
// weight and runs the row-major int8 kernels (N = 4096, K = 4096: M = 65 / 128 68 / 103 us, against ~2 x 21 us;
// M = 129-256 ~130 us against 3-4 x 21 us).  int4 keeps the unpack, which is faster there (28-35 us against
// ~2 x 19 us).
constexpr int64_t kNzChunkRows = 64;

bool nz_chunks_ok(const WqbmmArgs& p) {
    if (plan_override().w4nz_off || p.w_dtype == QK_I4_NZ || p.M <= kNzChunkRows || p.M > 4 * kNzChunkRows)
        return false;
    if (p.M > 3 * kNzChunkRows) {  // four chunks only where the NZ prefill kernel does not take the shape as NZ
        WqbmmArgs z = p;           // (an [N,K] weight gets there by its transpose and cast: N = 11008, M = 256
        z.w_dtype = QK_I8_NZ;      // 135 us against 169 us for four chunks; three chunks, M = 129 / 192, 97 / 124
        if (nzg_plan(z).ok) return false;  // us against 136 / 135 us)
    }
    WqbmmArgs c = p;
    c.M = kNzChunkRows;
    if (!nz_plan(c).ok) return false;
    const int64_t last = (p.M - 1) / kNzChunkRows * kNzChunkRows;  // the last chunk's first row
    c.x = static_cast<const char*>(p.x) + last * p.K * 2;  // 16-bit activations and outputs
    c.out = static_cast<char*>(p.out) + last * p.N * 2;
    c.M = p.M - last;
    return nz_plan(c).ok;
}

size_t w4_nz_workspace(const WqbmmArgs& p, bool stream_k) {
    if (!plan_override().w4nz_off && nz_plan(p).ok) return 0;
    if (nz_chunks_ok(p)) return 0;
    if (!plan_override().w4nz_off && nzg_plan(p).ok) return nzg_workspace(p, stream_k);
    const int nd_dtype = p.w_dtype == QK_I4_NZ ? QK_I32 : QK_I8;
    return QK_SPLIT_COUNTER_BYTES + round256(nd_weight_bytes(p)) +
           weight_quant_bmm_workspace(p.M, p.N, p.K, nd_dtype, p.group, true);
}

hipError_t launch_w4_nz_bmm(const WqbmmArgs& p, void* workspace, size_t ws_bytes, hipStream_t stream) {
    const NzPlan z = plan_override().w4nz_off ? NzPlan{false, 0, 0, 0, 0, 0} : nz_plan(p);
    if (z.ok)
        return p.x_dtype == QK_BF16 ? launch_nz_dt<QK_BF16>(p, z, stream) : launch_nz_dt<QK_F16>(p, z, stream);
    if (nz_chunks_ok(p)) {
        for (int64_t r0 = 0; r0 < p.M; r0 += kNzChunkRows) {
            WqbmmArgs c = p;
            c.x = static_cast<const char*>(p.x) + r0 * p.K * 2;
            c.out = static_cast<char*>(p.out) + r0 * p.N * 2;
            c.M = p.M - r0 < kNzChunkRows ? p.M - r0 : kNzChunkRows;
            const NzPlan zc = nz_plan(c);
            if (!zc.ok) return hipErrorInvalidValue;  // both chunk shapes checked above
            const hipError_t e = p.x_dtype == QK_BF16 ? launch_nz_dt<QK_BF16>(c, zc, stream)
                                                      : launch_nz_dt<QK_F16>(c, zc, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const NzGemmPlan g = plan_override().w4nz_off ? NzGemmPlan{false, 0, 0} : nzg_plan(p);
    if (g.ok) {
        if (!workspace || ws_bytes < nzg_workspace(p, false) || (uintptr_t)workspace % 16 != 0)
            return hipErrorInvalidValue;
        char* ws = static_cast<char*>(workspace);
        float* xs = reinterpret_cast<float*>(ws + QK_SPLIT_COUNTER_BYTES);
        return p.x_dtype == QK_BF16 ? launch_nzg_dt<QK_BF16>(p, g, ws, xs, ws + ws_bytes, stream)
                                    : launch_nzg_dt<QK_F16>(p, g, ws, xs, ws + ws_bytes, stream);
    }
    const bool w8 = p.w_dtype != QK_I4_NZ;
    const int nd_dtype = w8 ? QK_I8 : QK_I32;
    const size_t nd_bytes = round256(nd_weight_bytes(p));
    const size_t rest = weight_quant_bmm_workspace(p.M, p.N, p.K, nd_dtype, p.group, true);
    if (!workspace || ws_bytes < QK_SPLIT_COUNTER_BYTES + nd_bytes + rest || (uintptr_t)workspace % 256 != 0)
        return hipErrorInvalidValue;
    char* ws = static_cast<char*>(workspace);
    void* nd = ws + QK_SPLIT_COUNTER_BYTES;
    hipError_t e;
    if (p.w_dtype == QK_I8_NK)
        e = launch_w8_nk_transpose(static_cast<const int8_t*>(p.w), p.K, p.N, static_cast<int8_t*>(nd), stream);
    else if (w8)
        e = launch_w8_nz_cast(static_cast<const int8_t*>(p.w), false, p.K, p.N, static_cast<int8_t*>(nd), stream);
    else
        e = launch_w4_nz_cast(static_cast<const int32_t*>(p.w), false, p.K, p.N, static_cast<int32_t*>(nd), stream);
    if (e != hipSuccess) return e;
    WqbmmArgs q = p;
    q.w = nd;
    q.w_dtype = nd_dtype;
    return launch_weight_quant_bmm(q, rest ? ws + QK_SPLIT_COUNTER_BYTES + nd_bytes : nullptr, rest, stream);
}

// Row-major int4 [K, N/8] and int8 [K, N] weights past the decode rows: the call casts the weight into its
// workspace ([QK_SPLIT_COUNTER_BYTES, unused][NZ weight][x group sums fp32 [K/G][M]]) and runs the NZ prefill
// GEMM on it.  The cast reads and writes the weight once (cfg3's 4096 x 11008 weight: int4 ~10 us, int8
// ~25 us).  Measured per call at that shape (one box, 6 rotating weights), cast + NZ GEMM against the row-major
// kernels: int4 M = 257 / 384 / 512 / 640 / 896 86 / 79 / 80 / 84 / 111 us against 126 / 120 / 87 / 228 / 234 us
// (the row-major prefill kernel's register-staged form takes a ragged M), while at M = 200 / 256 the decode
// kernels are faster (67 / 72 against 77 us); int8 M = 200 / 256 / 384 / 640 116 / 117 / 116 / 120 us against
// 6450 / 7927 / 126 / 246 us.  So int4 casts from M = 257 and int8 from M = 129.  The debug overrides that
// force or disable a prefill kernel switch it off.
int64_t cast_nz_min_m(int w_dtype) { return w_dtype == QK_I8 ? 129 : 257; }

// An int8 row-major weight with 32 < M <= 128 (or up to 256 where the NZ prefill kernel does not take the shape)
// is cast too, for the NZ decode kernel (on row chunks past 64 rows): N = 4096, K = 4096, M = 65 / 128 41 / 53 us
// against 68 / 90 us for the row-major decode stream on 16-row slices; at N = 11008 60 / 80 against 68 / 107 us.
// The call's workspace then holds the NZ weight alone.
bool nz_decode_ok(const WqbmmArgs& q) { return q.M <= kNzChunkRows ? nz_plan(q).ok : nz_chunks_ok(q); }

bool cast_nz_decode(const WqbmmArgs& p) {
    if (p.w_dtype != QK_I8 || p.M <= 32 || p.M > 4 * kNzChunkRows) return false;
    WqbmmArgs q = p;
    q.w = reinterpret_cast<const void*>((uintptr_t)256);
    q.w_dtype = QK_I8_NZ;
    return nz_decode_ok(q);
}

size_t w4_cast_nz_workspace(const WqbmmArgs& p, bool stream_k) {
    const PlanOverride& ov = plan_override();
    if (!(p.w_dtype == QK_I32 || p.w_dtype == QK_I8) || ov.w4nz_off || ov.w4_gemm != 0) return 0;
    WqbmmArgs q = p;
    q.w = reinterpret_cast<const void*>((uintptr_t)256);  // the cast's destination: 256-byte aligned
    q.w_dtype = p.w_dtype == QK_I8 ? QK_I8_NZ : QK_I4_NZ;
    if (cast_nz_decode(p)) return round256(QK_SPLIT_COUNTER_BYTES + round256(nd_weight_bytes(q)));
    if (p.M < cast_nz_min_m(p.w_dtype) || !nzg_plan(q).ok) return 0;
    return round256(QK_SPLIT_COUNTER_BYTES + round256(nd_weight_bytes(q)) +
                    (nzg_workspace(q, stream_k) - QK_SPLIT_COUNTER_BYTES));
}

bool launch_w4_cast_nz(const WqbmmArgs& p, void* workspace, size_t ws_bytes, hipStream_t stream, hipError_t* err) {
    const size_t need = w4_cast_nz_workspace(p, false);
    if (need == 0 || !workspace || ws_bytes < need || (uintptr_t)workspace % 256 != 0) return false;
    char* ws = static_cast<char*>(workspace);
    void* nz = ws + QK_SPLIT_COUNTER_BYTES;
    const bool w8 = p.w_dtype == QK_I8;
    WqbmmArgs q = p;
    q.w = nz;
    q.w_dtype = w8 ? QK_I8_NZ : QK_I4_NZ;
    if (cast_nz_decode(p)) {
        if (!nz_decode_ok(q)) return false;  // with the call's own operands (their alignment)
        hipError_t e = launch_w8_nz_cast(static_cast<const int8_t*>(p.w), true, p.K, p.N, static_cast<int8_t*>(nz),
                                         stream);
        if (e == hipSuccess) e = launch_w4_nz_bmm(q, nullptr, 0, stream);
        *err = e;
        return true;
    }
    const NzGemmPlan g = nzg_plan(q);  // with the call's own operands (their alignment)
    if (!g.ok) return false;
    hipError_t e = w8 ? launch_w8_nz_cast(static_cast<const int8_t*>(p.w), true, p.K, p.N, static_cast<int8_t*>(nz),
                                          stream)
                      : launch_w4_nz_cast(static_cast<const int32_t*>(p.w), true, p.K, p.N, static_cast<int32_t*>(nz),
                                          stream);
    if (e == hipSuccess) {
        float* xs = reinterpret_cast<float*>(ws + QK_SPLIT_COUNTER_BYTES + round256(nd_weight_bytes(q)));
        e = p.x_dtype == QK_BF16 ? launch_nzg_dt<QK_BF16>(q, g, ws, xs, ws + ws_bytes, stream)
                                 : launch_nzg_dt<QK_F16>(q, g, ws, xs, ws + ws_bytes, stream);
    }
    *err = e;
    return true;
}

}  // namespace qk
