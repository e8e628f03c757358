// Roofline calibration kernels (measurement only; not part of the op path or
// of libqk_hip.so's C ABI).  bench.py --calibrate times them to give the
// ceilings the kernels of this library are judged against on the same box:
//
//  calib_mfma_i8     the int8 MFMA issue ceiling: every wave issues
//                    v_mfma_i32_16x16x64_i8 back to back on register
//                    operands (8 independent accumulators, no memory
//                    traffic), with constant or pseudo-random operand bits
//                    (the clock of this part is power-limited by the bits
//                    the MFMA unit toggles).
//  calib_stream_read the HBM read ceiling of one launch: every thread issues
//                    its 16-byte loads of a buffer up front and folds them
//                    into one word (so the loads are not removed).
//  calib_stream_wave the same read in the load form of the decode kernels:
//                    each wave instruction is one contiguous KB (64 lanes x
//                    16 bytes, buffer loads with the non-temporal hint or the
//                    default policy), U per lane issued up front, W waves per
//                    workgroup, as many workgroups as cover the buffer; a
//                    sweep over (W, U) gives the best one launch of that size
//                    reaches.
//  calib_dma_fill    the rate at which one CU fills its LDS by direct
//                    global->LDS loads (buffer_load_dwordx4 ... lds, as the
//                    GEMM kernels stage operands): NW waves each keep 16 such
//                    1 KB loads in flight, in row pieces of PIECE contiguous
//                    bytes from rows `rowstride` apart (rowstride == PIECE:
//                    one contiguous KB), from a span that stays in L2 or one
//                    read once from HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t mix(uint32_t x) {  // a 32-bit integer hash (xorshift-multiply)
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

__global__ __launch_bounds__(512) void calib_mfma_i8(int64_t iters, int random, int32_t* out) {
    const uint32_t seed = (blockIdx.x * blockDim.x + threadIdx.x) * 16u + 1u;
    i32x4 a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) a[i][e] = random ? (int32_t)mix(seed + 4 * i + e) : 0x01010101;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) b[i][e] = random ? (int32_t)mix(seed + 100 + 4 * i + e) : 0x01010101;
    i32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = (i32x4){0, 0, 0, 0};
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[j & 3], b[j >> 2], acc[j], 0, 0, 0);
    }
    int32_t s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) s ^= acc[j][0] ^ acc[j][1] ^ acc[j][2] ^ acc[j][3];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// PER: 16-byte loads per thread, all issued before the first use.
template <int PER>
__global__ __launch_bounds__(1024) void calib_stream_read(const u32x4* __restrict__ buf, int64_t n16,
                                                          uint32_t* out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    u32x4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int64_t idx = t + i * stride;
        v[i] = idx < n16 ? buf[idx] : (u32x4){0u, 0u, 0u, 0u};
    }
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) s ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    out[t] = s;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// An empty kernel: what a launch of a given grid costs inside its own duration (dispatch, wave launch, end of
// kernel), with no work at all.
__global__ __launch_bounds__(1024) void calib_empty(uint32_t* out) {
    if (threadIdx.x == 1023 && blockIdx.x == 0x7fffffff) out[0] = 1u;  // never true
}

// Wave w of workgroup b reads KB chunks (b*W + w)*U .. +U-1 of the buffer (loads past its end return zeros).
template <int W, int U, int POL>
__global__ __launch_bounds__(64 * W) void calib_stream_wave(const void* buf, uint32_t bytes, uint32_t* out) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(buf, bytes);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t c0 = (uint32_t)(blockIdx.x * W + wave) * U;
    u32x4 v[U];
#pragma unroll
    for (int i = 0; i < U; ++i)
        v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 16u * lane, (c0 + i) * 1024u, POL));
    u32x4 a = v[0];
#pragma unroll
    for (int i = 1; i < U; ++i) a ^= v[i];
    if (a[0] == 0x9e3779b9u && a[1] == 0x7f4a7c15u) out[blockIdx.x] = a[2];  // never true: keeps the loads
}

// 16 bytes per lane into LDS bytes [lds + 16*lane, +16); the kernel counts vmcnt itself
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds));
}

constexpr int vmcnt_imm(int n) { return (n & 0xf) | (0x7 << 4) | (0xf << 8) | ((n >> 4) << 14); }

// Workgroup b streams n_instr 1 KB loads per wave from offset (b * stride_wg + row block) % span into a
// 128 KB LDS ring (which nothing reads: only the fill rate is measured); the buffer must hold span bytes
// plus 64 rows of rowstride.
template <int NW, int PIECE>
__global__ __launch_bounds__(64 * NW) void calib_dma_fill(const int8_t* buf, uint32_t span, uint32_t rowstride,
                                                          int n_instr, uint32_t stride_wg, int32_t* out) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[128 * 1024];
    constexpr int DEPTH = 16;
    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)smem;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(buf, span + 64u * rowstride);
    constexpr int LPR = PIECE / 16;  // lanes per row piece
    constexpr int RPI = 64 / LPR;    // rows per load
    const uint32_t voff = (uint32_t)(lane / LPR) * rowstride + 16u * (uint32_t)(lane % LPR);
    const uint32_t base = (uint32_t)blockIdx.x * stride_wg;
    for (int i = 0; i < n_instr; ++i) {
        const uint32_t blk = (uint32_t)(i * NW + wave);
        const uint32_t soff = (base + blk * (uint32_t)RPI * rowstride) % span;
        dma16(rs, sbase + (blk % 128u) * 1024u, voff, soff);
        if (i >= DEPTH) __builtin_amdgcn_s_waitcnt(vmcnt_imm(DEPTH));
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = smem[blockIdx.x & 1023];
}

}  // namespace

extern "C" {

// grid x 512 threads, each wave issuing iters x 8 MFMAs; out holds grid*512 words.
int qk_calib_mfma_i8(int grid, int64_t iters, int random, int32_t* out, hipStream_t stream) {
    calib_mfma_i8<<<dim3((uint32_t)grid), dim3(512), 0, stream>>>(iters, random, out);
    return (int)hipGetLastError();
}

// bytes (a multiple of 16) read by `grid` workgroups of 1024 threads, 8 loads each in flight
// (the grid must cover the buffer: grid * 1024 * 8 * 16 >= bytes); out holds grid*1024 words.
int qk_calib_stream_read(const void* buf, int64_t bytes, int grid, uint32_t* out, hipStream_t stream) {
    const int64_t n16 = bytes / 16;
    if ((int64_t)grid * 1024 * 8 < n16) return -1;
    calib_stream_read<8><<<dim3((uint32_t)grid), dim3(1024), 0, stream>>>(static_cast<const u32x4*>(buf), n16, out);
    return (int)hipGetLastError();
}

// The read of calib_stream_wave: shape s of {W, U, policy} below (-1: past the last shape); grid from the size.
// out holds at least (bytes / 1024 + 1) words.
int qk_calib_stream_wave(int shape, const void* buf, int64_t bytes, uint32_t* out, hipStream_t stream) {
    struct Shape { int w, u, nt; };
    static const Shape shapes[] = {{16, 6, 1}, {16, 6, 0}, {16, 3, 1}, {16, 2, 1}, {8, 4, 1},
                                   {8, 2, 1}, {4, 8, 1}, {4, 4, 1}, {4, 2, 1}, {4, 1, 1}};
    if (shape < 0 || shape >= (int)(sizeof(shapes) / sizeof(shapes[0])) || bytes <= 0 || bytes >= (1ll << 31)) return -1;
    const Shape& sh = shapes[shape];
    const int64_t chunks = (bytes + 1023) / 1024;
    const uint32_t grid = (uint32_t)((chunks + sh.w * sh.u - 1) / (sh.w * sh.u));
    const uint32_t b = (uint32_t)bytes;
    switch (shape) {
    case 0: calib_stream_wave<16, 6, 2><<<grid, 1024, 0, stream>>>(buf, b, out); break;
    case 1: calib_stream_wave<16, 6, 0><<<grid, 1024, 0, stream>>>(buf, b, out); break;
    case 2: calib_stream_wave<16, 3, 2><<<grid, 1024, 0, stream>>>(buf, b, out); break;
    case 3: calib_stream_wave<16, 2, 2><<<grid, 1024, 0, stream>>>(buf, b, out); break;
    case 4: calib_stream_wave<8, 4, 2><<<grid, 512, 0, stream>>>(buf, b, out); break;
    case 5: calib_stream_wave<8, 2, 2><<<grid, 512, 0, stream>>>(buf, b, out); break;
    case 6: calib_stream_wave<4, 8, 2><<<grid, 256, 0, stream>>>(buf, b, out); break;
    case 7: calib_stream_wave<4, 4, 2><<<grid, 256, 0, stream>>>(buf, b, out); break;
    case 8: calib_stream_wave<4, 2, 2><<<grid, 256, 0, stream>>>(buf, b, out); break;
    default: calib_stream_wave<4, 1, 2><<<grid, 256, 0, stream>>>(buf, b, out); break;
    }
    return (int)hipGetLastError();
}

// grid x threads empty workgroups (threads <= 1024).
int qk_calib_empty(int grid, int threads, uint32_t* out, hipStream_t stream) {
    if (grid <= 0 || threads <= 0 || threads > 1024) return -1;
    calib_empty<<<dim3((uint32_t)grid), dim3((uint32_t)threads), 0, stream>>>(out);
    return (int)hipGetLastError();
}

// The (W, U, non-temporal) of shape s, for the report.
int qk_calib_stream_wave_shape(int shape, int* w, int* u, int* nt) {
    static const int t[][3] = {{16, 6, 1}, {16, 6, 0}, {16, 3, 1}, {16, 2, 1}, {8, 4, 1},
                               {8, 2, 1}, {4, 8, 1}, {4, 4, 1}, {4, 2, 1}, {4, 1, 1}};
    if (shape < 0 || shape >= 10) return -1;
    *w = t[shape][0];
    *u = t[shape][1];
    *nt = t[shape][2];
    return 0;
}

// variant: 0 = 4 waves, 1 = 8 waves, 2 = 16 waves (256-byte pieces).  buf holds span + 64 * rowstride
// bytes; out holds grid words.
int qk_calib_dma_fill(int variant, int grid, const void* buf, uint32_t span, uint32_t rowstride, int n_instr,
                      uint32_t stride_wg, int32_t* out, hipStream_t stream) {
    const int8_t* b = static_cast<const int8_t*>(buf);
    switch (variant) {
    case 0: calib_dma_fill<4, 256><<<grid, 256, 0, stream>>>(b, span, rowstride, n_instr, stride_wg, out); break;
    case 1: calib_dma_fill<8, 256><<<grid, 512, 0, stream>>>(b, span, rowstride, n_instr, stride_wg, out); break;
    case 2: calib_dma_fill<16, 256><<<grid, 1024, 0, stream>>>(b, span, rowstride, n_instr, stride_wg, out); break;
    default: return -1;
    }
    return (int)hipGetLastError();
}

}  // extern "C"
