/*
 * qk_abi.h -- C ABI of libqk_hip.so, the MI355X (gfx950) kernels of the
 * quantized-inference hot path: npu_dynamic_quant, npu_quant_matmul (W8A8)
 * and npu_weight_quant_batchmatmul (W4A16 / W8A16).
 *
 * This is the layer the reference reaches through EXEC_NPU_CMD
 * (op_plugin/utils/op_api_common.h:520-570): a two-phase C call,
 * "<op>GetWorkspaceSize" then "<op>(workspace, size, executor, stream)",
 * resolved by dlsym from libcust_opapi.so / libopapi.so
 * (op_plugin/utils/op_api_common.h:80-123).  Here the two phases are
 * qk_*_workspace_size() and the op call itself; operands are plain device
 * pointers, sizes and strides instead of aclTensor descriptors, so no torch
 * or vendor type appears in a signature.
 *
 * Contract, as in the reference boundary:
 *   - the caller allocates every output and the workspace
 *     (op_plugin/ops/base_ops/opapi/MmKernelNpuOpApi.cpp:27-30,
 *      op_plugin/utils/op_api_common.h:547-551); the library allocates nothing;
 *   - work is enqueued on `stream` and never synchronised
 *     (op_plugin/utils/op_api_common.h:530, 563-566);
 *   - a non-zero return is an error and qk_last_error() gives a thread-local
 *     message (the reference's aclGetRecentErrMsg(),
 *     op_plugin/utils/op_api_common.h:546, 555).
 * All functions are thread-safe; calls on one stream execute in order.
 *
 * Workspaces, as the reference's per-call scratch
 * (op_plugin/utils/op_api_common.h:547-551, unsafe_empty_workspace): the
 * caller passes at least *_workspace_size() bytes, 256-byte aligned, of any
 * contents -- uninitialised memory is fine.  A non-empty workspace begins with
 * QK_SPLIT_COUNTER_BYTES of split-K arrival counters, followed by the partial
 * sums (split-K shapes) or by the activations' per-group sums (weight-quant
 * matmul at large M; from M = 257 on a row-major int4 weight, and from M = 33
 * on a row-major int8 weight, the weight cast to NZ, K*N/2 (int4) or K*N
 * (int8) bytes rounded to 256, comes first, then the sums (none up to M = 128
 * on int8, where the NZ decode kernel runs); where the NZ
 * prefill kernel runs stream-K, (P - 1) x 128 KB of fp32 partial slots follow
 * the sums, P being the current device's CU count).  Each arrival adds D = tag * 2^16 + 1 to its
 * counter (a 48-bit tag drawn per call, never 0 or all ones), so a counter of
 * this call holds j * D after j arrivals; a zero word is empty (the last
 * arrival leaves zero behind), and any other word that is not such a multiple
 * -- what another user left there, a 0xFF fill -- is recognised as stale and
 * replaced.  The one exception is memory whose counter words happen to hold a
 * small multiple of this call's D (odds below 2^-48 per counter word for
 * random contents, zero for zero- or 0xFF-filled memory).  The workgroup that completes a tile's splits
 * adds them up itself, so no second kernel runs.  Calls that may be in flight
 * at the same time need distinct workspaces.
 */
#ifndef QK_ABI_H
#define QK_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t; NULL is the default (null) stream. */
typedef struct ihipStream_t* qk_stream_t;

/* Element types.  F16 = IEEE binary16, BF16 = bfloat16. */
typedef enum {
    QK_F16 = 1,
    QK_BF16 = 2,
    QK_F32 = 3,
    QK_I8 = 4,
    QK_I32 = 5,
    QK_U8 = 6,
    /* weight codes of qk_weight_quant_bmm for weights in the MFMA-tiled NZ
     * layouts that qk_weight_format_cast writes: int4, int32 [N/16][K/128][64][4];
     * int8, int8 [N/16][K/64][64][16] */
    QK_I4_NZ = 16,
    QK_I8_NZ = 17,
    /* weight code of qk_weight_quant_bmm for an int8 weight stored [N, K] (row n
     * holds column n's K values: the nn.Linear layout, which the op receives as
     * the transposed view [K, N] of that tensor); read in place, as the reference
     * flags a transposed mat2 instead of copying it
     * (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:40-53,
     * op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:39-40) */
    QK_I8_NK = 18
} qk_dtype;

/* Weight storage formats: the reference's aclFormat numbers for ND and
 * FRACTAL_NZ (op_plugin/third_party/acl/inc/graph/types.h:111, 138). */
#define QK_FORMAT_ND 2
#define QK_FORMAT_FRACTAL_NZ 29

/* Return codes. */
enum {
    QK_OK = 0,
    QK_ERR_ARG = -1,          /* invalid argument (shape, dtype, pointer, alignment) */
    QK_ERR_UNSUPPORTED = -2,  /* valid request this build does not implement */
    QK_ERR_WORKSPACE = -3,    /* workspace missing or smaller than *_workspace_size() */
    QK_ERR_LAUNCH = -4        /* the HIP runtime refused a launch */
};

/* Thread-local description of the last failure on this thread ("" if none). */
const char* qk_last_error(void);

/* ABI revision; bumped on any incompatible signature or contract change
 * (2: the split-K counters at the head of a workspace; 3: the counters are
 * tagged per call, so a workspace needs no initialisation; 4: NZ weights,
 * qk_weight_format_cast, static quantization; 5: the [N, K] int8 weight code
 * QK_I8_NK, int8 NZ weights with K % 64 == 0 in qk_weight_quant_bmm; 6: qk_quant_matmul_swiglu,
 * qk_quant_matmul_swiglu_quant). */
int qk_abi_version(void);

/* Debug and test hook, no counterpart in the reference: forces kernel choices
 * of the planners (spec grammar in csrc/kernels/common.h, "PlanOverride"; NULL
 * or "" restores the planners' own choices).  The library reads the
 * QK_DEBUG_PLAN environment variable once at first use; this call replaces
 * that for the rest of the process.  Not meant for production callers.
 * Returns QK_ERR_ARG (override unchanged) for a spec it does not understand. */
int qk_debug_set_plan(const char* spec);

/* Bytes of split-K counters at the start of every non-empty workspace. */
#define QK_SPLIT_COUNTER_BYTES 4096

/*
 * npu_dynamic_quant -- replaces aclnnDynamicQuant behind EXEC_NPU_CMD
 * (op_plugin/utils/op_api_common.h:520-570); the nearest reference op is the
 * static quantize_per_channel (op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:69-92).
 * x: [rows, K] fp16/bf16, row-major.  smooth_scales: [K] fp32 or NULL.
 * y: [rows, K] int8.  scale: [rows] fp32.
 * Per row: s = max|x*smooth| / 127 (fp32 division), y = clamp(rint(x*smooth / s)),
 * ties to even; an all-zero row gives s = 0, y = 0.  No workspace.
 */
int qk_dynamic_quant(const void* x, int x_dtype, int64_t rows, int64_t K,
                     const float* smooth_scales, int8_t* y, float* scale, qk_stream_t stream);

/*
 * npu_quant_matmul (W8A8), phase 1 -- replaces aclnnQuantMatmul*GetWorkspaceSize
 * (op_plugin/utils/op_api_common.h:543-546).  Writes the workspace bytes the
 * call with the same shape needs (0 when none) to *bytes.
 */
int qk_quant_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int out_dtype, size_t* bytes);

/*
 * npu_quant_matmul (W8A8), phase 2 -- replaces aclnnQuantMatmul* behind
 * EXEC_NPU_CMD (op_plugin/utils/op_api_common.h:552-566); shape/bias rules
 * follow mm / addmm (op_plugin/ops/base_ops/opapi/MmKernelNpuOpApi.cpp:24-32,
 * op_plugin/ops/base_ops/opapi/AddmmKernelNpuOpApi.cpp:24-55).
 * x1: int8 [M,K], row stride ldx1.  x2: int8 [K,N] addressed as
 * x2[k*x2_stride_k + n*x2_stride_n]; exactly one stride must be 1
 * ([K,N]-contiguous: (N',1); transposed view of [N,K]: (1,K')), as the
 * reference flags a transposed mat2 instead of copying it
 * (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:40-53).
 * acc = sum_k x1*x2 in int32, exact: K above 131071 is refused (QK_ERR_UNSUPPORTED).
 * scale: fp32 [scale_len], scale_len 1 or N.  offset (int8 output only): fp32 [1|N] or NULL.
 * pertoken_scale: fp32 [M] or NULL.  bias: [N] of bias_dtype
 * (QK_I32: added to acc; QK_BF16/QK_F16/QK_F32: added after scaling) or NULL.
 * out: [M,N] row-major of out_dtype:
 *   QK_BF16/QK_F16: cast(fmaf(float(acc) [* pertoken[m]], scale[n], bias[n]))
 *   QK_I8:          clamp(rint(fmaf(float(acc), scale[n], offset[n])))
 *   QK_I32:         acc (+ int32 bias)
 */
int qk_quant_matmul(const int8_t* x1, int64_t ldx1,
                    const int8_t* x2, int64_t x2_stride_k, int64_t x2_stride_n,
                    int64_t M, int64_t N, int64_t K,
                    const float* scale, int64_t scale_len,
                    const float* offset, int64_t offset_len,
                    const float* pertoken_scale,
                    const void* bias, int bias_dtype,
                    void* out, int out_dtype,
                    void* workspace, size_t workspace_bytes, qk_stream_t stream);

/*
 * npu_quant_matmul (W8A8) on an int8 weight in the NZ layout, phase 1: the
 * workspace bytes qk_quant_matmul_nz needs for this shape (0 when none).
 */
int qk_quant_matmul_nz_workspace_size(int64_t M, int64_t N, int64_t K, int out_dtype, size_t* bytes);

/*
 * npu_quant_matmul (W8A8) on an int8 weight in the NZ layout, phase 2 -- the
 * same op as qk_quant_matmul with x2 already cast to the device-native tiled
 * format, as the reference casts matmul weights to FRACTAL_NZ before its
 * matmuls (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:303-316,
 * op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:103-107) and hands
 * aclnnQuantMatmul* the NZ tensor behind EXEC_NPU_CMD
 * (op_plugin/utils/op_api_common.h:552-566).
 * x2_nz: int8 [N/16][K/64][64][16] as qk_weight_format_cast writes it from
 * an int8 [K,N] weight (K % 64 == 0, N % 16 == 0).  x1, x2_nz and out must be
 * 16-byte aligned, ldx1 a multiple of 16 below 2^24.  Every other argument,
 * the arithmetic and the result are those of qk_quant_matmul (bit-identical
 * outputs for the same weight in either layout).
 */
int qk_quant_matmul_nz(const int8_t* x1, int64_t ldx1, const int8_t* x2_nz,
                       int64_t M, int64_t N, int64_t K,
                       const float* scale, int64_t scale_len,
                       const float* offset, int64_t offset_len,
                       const float* pertoken_scale,
                       const void* bias, int bias_dtype,
                       void* out, int out_dtype,
                       void* workspace, size_t workspace_bytes, qk_stream_t stream);

/*
 * npu_weight_quant_batchmatmul, phase 1 (see qk_quant_matmul_workspace_size).
 */
int qk_weight_quant_bmm_workspace_size(int64_t M, int64_t N, int64_t K, int weight_dtype,
                                       int64_t group_size, size_t* bytes);

/*
 * npu_weight_quant_batchmatmul (W4A16 / W8A16), phase 2 -- replaces
 * aclnnWeightQuantBatchMatmul* behind EXEC_NPU_CMD; the nearest reference op
 * is bmm (op_plugin/ops/base_ops/opapi/BmmKernelNpuOpApi.cpp:24-52).
 * x: [M,K] fp16/bf16 row-major.  weight: QK_I32 -> int4 packed [K, N/8]
 * (nibble i of word j is column 8j+i, two's complement); QK_I8 -> int8 [K,N];
 * QK_I8_NK -> int8 stored [N,K] (element (k, n) at weight[n*K + k]); QK_I4_NZ /
 * QK_I8_NZ -> int4 / int8 in the NZ layouts of qk_weight_format_cast
 * (N % 16 == 0; K % 128 == 0 for int4, K % 64 == 0 for int8).
 * antiquant_scale / antiquant_offset: [K/group, N] (group_size > 0) or [N]
 * (group_size == 0, per channel), of scale_dtype (fp16/bf16); offset may be NULL.
 * bias: [N] or NULL.  out: [M,N] of out_dtype (fp16/bf16).
 * out = sum_k x[m,k] * (w[k,n] + offset[g,n]) * scale[g,n] + bias[n], g = k/group,
 * with fp32 accumulation; the dequantized weight is never rounded to 16 bits.
 */
int qk_weight_quant_bmm(const void* x, int x_dtype,
                        const void* weight, int weight_dtype,
                        const void* antiquant_scale, const void* antiquant_offset, int scale_dtype,
                        int64_t M, int64_t N, int64_t K, int64_t group_size,
                        const void* bias, int bias_dtype,
                        void* out, int out_dtype,
                        void* workspace, size_t workspace_bytes, qk_stream_t stream);

/* Bytes of the library-held scratch that qk_weight_quant_bmm_noalloc uses on each GPU. */
#define QK_NOALLOC_SCRATCH_BYTES (16 << 20)

/*
 * npu_weight_quant_batchmatmul without a workspace argument.  No counterpart
 * in the reference (whose calls always take caller-allocated scratch): this
 * entry point is for callers that cannot allocate device memory -- code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * Arguments and results are those of qk_weight_quant_bmm; the scratch the
 * call needs (split-K partials, group sums) lives in a library-owned device
 * array of QK_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, and
 * the call allocates nothing.  Where the workspace qk_weight_quant_bmm_workspace_size
 * reports fits in that array, the call runs exactly the kernels qk_weight_quant_bmm
 * runs (the same bits).  Where only the NZ prefill kernel's stream-K partial
 * slots do not fit, it runs that kernel with whole tiles per workgroup (the
 * same bits again).  Otherwise, for a row-major int4 weight at M >= 257 or int8
 * weight at M >= 33 whose cast to NZ is what does not fit, it runs the
 * row-major kernels without the cast (within the same 1e-2 bar; for int4 on
 * cfg3's shape, N = 11008, K = 4096, 128-row groups, at M = 1024 and 2048 the
 * same bits); a shape whose scratch exceeds
 * QK_NOALLOC_SCRATCH_BYTES even so is refused with QK_ERR_UNSUPPORTED.  The call uses the array of the current device, so
 * `stream` must belong to it.  All calls on one GPU share that array: calls
 * that may run at the same time on one GPU (several streams or threads) race
 * on it and give wrong results, so serialise them (e.g. one stream).
 */
int qk_weight_quant_bmm_noalloc(const void* x, int x_dtype,
                                const void* weight, int weight_dtype,
                                const void* antiquant_scale, const void* antiquant_offset, int scale_dtype,
                                int64_t M, int64_t N, int64_t K, int64_t group_size,
                                const void* bias, int bias_dtype,
                                void* out, int out_dtype, qk_stream_t stream);

/*
 * npu_format_cast for a matmul weight -- the MI355X counterpart of the
 * FRACTAL_NZ casts the reference applies to matmul operands
 * (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:303-316,
 * op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:103-107), done once when
 * weights are loaded.  src_format -> dst_format is QK_FORMAT_ND ->
 * QK_FORMAT_FRACTAL_NZ or back; N % 16 == 0; src and dst must not overlap and
 * must be 16-byte aligned.
 * weight_dtype QK_I32 (int4 packed, [K, N/8] in ND; K % 128 == 0): NZ is int32
 * [N/16][K/128][64][4]; element (k, n) is in word
 *   ((n/16 * (K/128) + k/128) * 64 + lane) * 4 + j,
 *   c = (k%128)/8, lane = n%16 + 16*(c%4), j = c/4,
 * at nibble i/2 for even i = k%8 and 4 + i/2 for odd i (two's complement).
 * weight_dtype QK_I8 ([K, N] in ND; K % 64 == 0): NZ is int8 [N/16][K/64][64][16];
 * element (k, n) is byte ((n/16 * (K/64) + k/64) * 64 + n%16 + 16*((k%64)/16)) * 16 + k%16.
 * Either way a 1 KB block (16 columns) is read by a wave as one 16-byte load
 * per lane, each lane's bytes being its MFMA B operands.  No workspace.
 */
int qk_weight_format_cast(const void* src, int src_format, void* dst, int dst_format, int weight_dtype,
                          int64_t K, int64_t N, qk_stream_t stream);

/*
 * npu_convert_weight_to_int4pack -- packs int4 values held one per element
 * (int8 or int32 [K,N], values in [-8,7]) into int32 [K, N/8] in the layout
 * qk_weight_quant_bmm reads.  No counterpart exists in the reference snapshot
 * (int4 is disabled there: op_plugin/third_party/acl/inc/graph/types.h:57).
 */
int qk_int4_pack(const void* w, int w_dtype, int64_t K, int64_t N, int32_t* packed,
                 qk_stream_t stream);

/*
 * quantize_per_tensor -- replaces the CANN Quantize call of
 * op_plugin/ops/base_ops/aclops/QuantizePerTensorKernelNpu.cpp:50-82 (schema
 * op_plugin/config/v2r2/op_plugin_functions.yaml:1233).  x: n elements,
 * fp32/fp16/bf16.  q: n elements of q_dtype QK_I8 (qint8), QK_U8 (quint8) or
 * QK_I32 (qint32), the plain integer tensor the reference returns (dtype map
 * :60-67).  Per element: q = clamp(RN(rint(x * RN(1/scale)) + float(zero_point)),
 * qmin, qmax), ties to even, the zero point added in float32 (torch's affine
 * quantizer); NaN gives qmin.  scale must be a positive finite float.
 */
int qk_quantize_per_tensor(const void* x, int x_dtype, int64_t n, float scale, int64_t zero_point, void* q,
                           int q_dtype, qk_stream_t stream);

/*
 * quantize_per_channel -- replaces the CANN Quantize call of
 * op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:69-92 (schema
 * op_plugin/config/v2r2/op_plugin_functions.yaml:1231).  x is viewed as
 * [outer][C][inner] with C the quantized axis; scales: fp32 [C] (device);
 * zero_points: int64 [C] (device).  Element rule as qk_quantize_per_tensor with
 * the channel's scale and zero point.
 */
int qk_quantize_per_channel(const void* x, int x_dtype, int64_t outer, int64_t C, int64_t inner, const float* scales,
                            const int64_t* zero_points, void* q, int q_dtype, qk_stream_t stream);

/*
 * dequantize -- the reference's op_plugin/ops/v1r11/opapi/DequantizeKernelNpuOpApi.cpp:22-24
 * (schema op_plugin/config/v1r11/op_plugin_functions.yaml:127): the integers of
 * q (QK_I8, QK_U8 or QK_I32, n elements) cast to float32 (round to nearest even
 * past 2^24).
 */
int qk_dequantize(const void* q, int q_dtype, int64_t n, float* out, qk_stream_t stream);

/*
 * npu_rms_norm -- replaces aclnnRmsNorm behind EXEC_NPU_CMD
 * (op_plugin/ops/base_ops/opapi/RmsNormKernelOpApi.cpp:24-35: y has the dtype
 * of x, :31; rstd is fp32, :32; schema op_plugin/config/v2r2/op_plugin_functions.yaml:2047).
 * x: [rows, D] fp16/bf16/fp32 (fp32 is the reference's golden case).  gamma:
 * [D], same dtype.  y: [rows, D], x's dtype.
 * rstd: [rows] fp32 or NULL.  rstd = 1/sqrt(mean(x^2) + eps); y = x * rstd * gamma
 * (golden test/test_custom_ops/test_npu_rms_norm.py:10-17), fp32 arithmetic.
 */
int qk_rms_norm(const void* x, int x_dtype, const void* gamma, int64_t rows, int64_t D, float eps,
                void* y, float* rstd, qk_stream_t stream);

/*
 * RMSNorm followed by npu_dynamic_quant of its 16-bit output, in one pass
 * (the first two steps of the quantized MLP block).  No single reference op:
 * the unfused chain is qk_rms_norm then qk_dynamic_quant, and q / scale are
 * bit-identical to it.  x: fp16/bf16 only (npu_dynamic_quant takes no fp32).
 * q: [rows, D] int8.  scale: [rows] fp32.  rstd as above.
 */
int qk_rms_norm_quant(const void* x, int x_dtype, const void* gamma, int64_t rows, int64_t D, float eps,
                      int8_t* q, float* scale, float* rstd, qk_stream_t stream);

/*
 * npu_swiglu (dim = -1) -- silu(a) * b with a, b = h.chunk(2, -1), the first
 * half the gate; the gated halving follows npu_geglu
 * (op_plugin/ops/v1r11/opapi/GeGluKernelNpuOpApi.cpp:23-40), silu follows
 * op_plugin/ops/base_ops/opapi/SiluKernelNpuOpApi.cpp:22-43.
 * h: [rows, 2*I] fp16/bf16.  y: [rows, I], same dtype.  fp32 arithmetic.
 */
int qk_swiglu(const void* h, int dtype, int64_t rows, int64_t I, void* y, qk_stream_t stream);

/*
 * SwiGLU followed by npu_dynamic_quant of its 16-bit output, in one pass (the
 * activation step of the quantized MLP block); bit-identical to qk_swiglu then
 * qk_dynamic_quant.  q: [rows, I] int8.  scale: [rows] fp32.
 */
int qk_swiglu_quant(const void* h, int dtype, int64_t rows, int64_t I, int8_t* q, float* scale,
                    qk_stream_t stream);

/*
 * The quantized MLP block's gate-up projection with the SwiGLU fused into the
 * GEMM's epilogue.  No single reference op: the unfused chain is
 * qk_quant_matmul (x1 [M,K] int8 x x2 [K,2I] int8, per-channel or per-tensor
 * scale of 2I or 1 elements, optional pertoken_scale [M], no bias, 16-bit
 * output) then qk_swiglu, and h [M, I] (out_dtype QK_BF16 or QK_F16, rows of
 * I elements) is bit-identical to it: the gate and up outputs are rounded to
 * out_dtype as the GEMM rounds them, and silu(gate) * up as qk_swiglu rounds
 * it.  Quantizing h with qk_dynamic_quant gives qk_swiglu_quant's q and scale.
 * x2: x2_format QK_FORMAT_FRACTAL_NZ (the NZ blocks npu_format_cast writes) or
 * QK_FORMAT_ND ([K, 2I] rows of x2_stride_k >= 2I bytes).  Runs where
 * I % 128 == 0, K % 256 == 0, ldx1 % 16 == 0 (< 2^24), x1 / x2 / out 16-byte
 * aligned and every offset fits 32 bits; other requests return
 * QK_ERR_UNSUPPORTED (the caller composes the two calls instead).  No
 * workspace.
 */
int qk_quant_matmul_swiglu(const int8_t* x1, int64_t ldx1, const int8_t* x2, int x2_format, int64_t x2_stride_k,
                           int64_t M, int64_t I, int64_t K, const float* scale, int64_t scale_len,
                           const float* pertoken_scale, void* out, int out_dtype, qk_stream_t stream);

/*
 * The same projection followed by qk_dynamic_quant of h, as the quantized MLP
 * block uses it: q [M, I] int8 (rows of I bytes, 8-byte aligned) and q_scale
 * [M] fp32 equal qk_dynamic_quant(h) bit for bit, h [M, I] being
 * qk_quant_matmul_swiglu's output rounded to h_dtype (QK_BF16 / QK_F16).  h
 * lives in the workspace, and the GEMM's epilogue also stores each row's
 * largest |h| per 128-column slice there, so the quantizer needs no row
 * reduction.  No single reference op: the chain npu_quant_matmul ->
 * npu_swiglu -> npu_dynamic_quant.  Workspace: the bytes
 * qk_quant_matmul_swiglu_quant_workspace_size gives (h plus M * I / 128
 * floats), 256-byte aligned, any contents.  The shapes
 * qk_quant_matmul_swiglu takes (I % 128 == 0, K % 256 == 0, ...); others
 * return QK_ERR_UNSUPPORTED (the caller composes the calls).
 */
int qk_quant_matmul_swiglu_quant_workspace_size(int64_t M, int64_t I, size_t* bytes);
int qk_quant_matmul_swiglu_quant(const int8_t* x1, int64_t ldx1, const int8_t* x2, int x2_format,
                                 int64_t x2_stride_k, int64_t M, int64_t I, int64_t K, const float* scale,
                                 int64_t scale_len, const float* pertoken_scale, int h_dtype, int8_t* q,
                                 float* q_scale, void* workspace, size_t workspace_bytes, qk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QK_ABI_H */
