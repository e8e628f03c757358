/*
 * qk_oracle.c -- CPU restatement of the quantized-inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels under ascend-python_amd/csrc.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it; the product path never links it.
 *
 * The three ops restated here (npu_dynamic_quant, npu_quant_matmul,
 * npu_weight_quant_batchmatmul) do not exist in the reference snapshot: a
 * search of /root/reference for dynamic_quant|quant_matmul|weight_quant finds
 * nothing, and int4 is not even an enabled dtype there
 * (op_plugin/third_party/acl/inc/graph/types.h:57 has "// DT_INT4 = 28").
 * The arithmetic follows the closed forms the op contract states, and each
 * function names the reference file whose convention it keeps:
 *   - int8 output dtype for a quantize op: QInt8 -> kChar
 *     (op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:81-88);
 *   - "accumulate wide, cast once" for low-precision GEMM outputs
 *     (test/test_custom_ops/test_mm_reduce_scatter_base.py:69-81,
 *      test/test_custom_ops/test_all_gather_base_mm.py:72-78);
 *   - transposed weight given as a strided view, not a copy
 *     (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:40-53);
 *   - RMSNorm closed form (test/test_custom_ops/test_npu_rms_norm.py:10-17).
 *
 * Pinning (what checks each function, in tests/test_oracle.py):
 *   qo_f16_to_f32 / qo_bf16_to_f32 / qo_f32_to_bf16 / qo_f32_to_f16:
 *       exhaustively against torch's own dtype conversions (all 65536 half
 *       patterns; random and tie-crafted float32 patterns for the casts).
 *   qo_dynamic_quant: closed-form invariants (max|y|==127 on a nonzero row,
 *       |y*s-x| <= s/2, sign agreement), exact hand-built ties that must go to
 *       the even integer, zero rows, single-nonzero rows, brute force against
 *       an independent float64 computation of the same quotient on tiny rows.
 *   qo_w8a8_acc: int64 numpy matmul (a library routine) on random shapes,
 *       all-ones known answer (== K), identity-weight known answer.
 *   qo_quant_matmul epilogue: float64 recomputation within one float32 ulp
 *       before the output cast; bf16 cast pinned as above.
 *   qo_int4_pack / unpack: hand-computed packed words, round trip over all
 *       16 nibble values at every position.
 *   qo_w4_nz_pack / unpack: round trip on random weights (a bijection of
 *       words), hand-computed word/nibble positions of single nonzero
 *       elements, and the MFMA operand property the kernels rely on (the 8
 *       nibbles of one word are 8 consecutive k of one column, even k low).
 *   qo_w8_nz_pack / unpack: round trip, hand-computed byte positions, and the
 *       int8-MFMA operand property (a lane's 16 bytes are 16 consecutive k).
 *   qo_weight_quant_bmm: scale=1/offset=0 reduces to torch.matmul in float64;
 *       a hand-computed 1x2x128 example; linearity in x.
 *   qo_rms_norm / qo_rms_norm_f32: the reference's numpy closed form, restated
 *       in float64; pinned against torch.nn.functional.rms_norm (a library
 *       routine) in float64 and a hand-computed row.
 *   qo_swiglu: torch.nn.functional.silu (a library routine) on float64.
 *   qo_quantize: torch.quantize_per_tensor / quantize_per_channel on the CPU
 *       (.int_repr(), library routines) for qint8 / quint8 / qint32 on random
 *       data, planted exact ties and values past the clamp bounds; hand-computed
 *       cases.  qo_dequantize: torch's integer -> float32 cast.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* Scalar format conversions (IEEE 754 binary16 / bfloat16).           */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float qo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

float qo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: value = man * 2^-24, exact in float32 */
        float v = (float)man * u2f(0x33800000u); /* 2^-24 */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* float32 -> bfloat16, round to nearest, ties to even; NaN stays NaN (quiet). */
uint16_t qo_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* float32 -> binary16, round to nearest, ties to even (subnormals, overflow to inf). */
uint16_t qo_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);       /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);      /* >= 65520: inf */
    if (a < 0x38800000u) {                                        /* < 2^-14: subnormal / zero */
        /* value / 2^-24, rounded to nearest even integer (exact arithmetic in double) */
        double q = (double)u2f(a) * 16777216.0;
        double r = nearbyint(q); /* default rounding mode: ties to even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    /* normal: drop 13 mantissa bits with RNE; carry may bump the exponent */
    uint32_t e = (a >> 23) - 112u;
    uint32_t m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

/* dtype codes shared with include/qk_abi.h */
enum { QO_F16 = 1, QO_BF16 = 2, QO_F32 = 3, QO_I8 = 4, QO_I32 = 5, QO_U8 = 6 };

static inline float load_half(const uint16_t* p, int64_t i, int dt) {
    return dt == QO_BF16 ? qo_bf16_to_f32(p[i]) : qo_f16_to_f32(p[i]);
}

static inline float load_any(const void* p, int64_t i, int dt) {
    switch (dt) {
    case QO_F16: return qo_f16_to_f32(((const uint16_t*)p)[i]);
    case QO_BF16: return qo_bf16_to_f32(((const uint16_t*)p)[i]);
    case QO_F32: return ((const float*)p)[i];
    default: return 0.0f;
    }
}

/*
 * Saturating conversion of an integral float to int8 with C99 fmaxf / fminf
 * (IEEE 754 maxNum / minNum): t is clamped to [-128, 127] before the integer
 * conversion, so the conversion is always defined, and a NaN t gives -128
 * (fmaxf(NaN, -128) = -128).  These are the clamp operations the kernels use
 * (fmaxf / fminf on gfx950, which return the non-NaN operand).
 */
static int8_t qo_sat_i8(float t) {
    t = fminf(fmaxf(t, -128.0f), 127.0f);
    return (int8_t)(int)t;
}

/* ------------------------------------------------------------------ */
/* npu_dynamic_quant: per-row symmetric int8, scale = absmax / 127.    */
/* ------------------------------------------------------------------ */
/*
 * For each row r of x viewed as [rows, K]:
 *   xf[k]  = float(x[r,k]) (* smooth[k] when given, one float32 multiply)
 *   a      = max_k |xf[k]|                     (fmaxf from 0: NaN elements do not enter)
 *   s      = a / 127.0f                        (IEEE float32 division)
 *   y[r,k] = qo_sat_i8(rint(xf[k] / s))        (rint: ties to even; clamp to [-128, 127])
 * A row of zeros gives s = 0 and y = 0.
 * Non-finite inputs follow the same formula: a row holding +-Inf gets
 * s = +Inf, its finite elements 0 (x / Inf = +-0) and its +-Inf elements
 * -128 (Inf / Inf = NaN); a NaN element of a row with s > 0 gives -128; a row
 * whose nonzero values are all NaN has a = 0, so s = 0 and y = 0.
 * Dtype map int8 output as QInt8 -> kChar
 * (op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:81-84).
 */
void qo_dynamic_quant(const uint16_t* x, int x_dtype, int64_t rows, int64_t K,
                      const float* smooth, int8_t* y, float* scale) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* xr = x + r * K;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float v = load_half(xr, k, x_dtype);
            if (smooth) v = v * smooth[k];
            amax = fmaxf(amax, fabsf(v));
        }
        float s = amax / 127.0f;
        scale[r] = s;
        for (int64_t k = 0; k < K; ++k) {
            int8_t q = 0;
            if (s != 0.0f) {
                float v = load_half(xr, k, x_dtype);
                if (smooth) v = v * smooth[k];
                q = qo_sat_i8(rintf(v / s));
            }
            y[r * K + k] = q;
        }
    }
}

/* ------------------------------------------------------------------ */
/* npu_quant_matmul (W8A8)                                             */
/* ------------------------------------------------------------------ */
/*
 * acc[m,n] = sum_k int32(a[m,k]) * int32(w[k,n]), exact in int32 for
 * K <= 131072.  The weight is addressed through (stride_k, stride_n) so a
 * [K,N]-contiguous tensor (stride_k=N, stride_n=1) and a transposed view of an
 * [N,K] tensor (stride_k=1, stride_n=K) are both read in place, as the
 * reference handles a transposed mat2 by a flag rather than a copy
 * (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:40-53).
 */
void qo_w8a8_acc(const int8_t* a, int64_t lda, const int8_t* w, int64_t w_sk, int64_t w_sn,
                 int64_t M, int64_t N, int64_t K, int32_t* acc) {
    for (int64_t m = 0; m < M; ++m) {
        int32_t* row = acc + m * N;
        for (int64_t n = 0; n < N; ++n) row[n] = 0;
        const int8_t* am = a + m * lda;
        if (w_sn == 1) {
            for (int64_t k = 0; k < K; ++k) {
                int32_t av = am[k];
                const int8_t* wk = w + k * w_sk;
                for (int64_t n = 0; n < N; ++n) row[n] += av * (int32_t)wk[n];
            }
        } else {
            for (int64_t n = 0; n < N; ++n) {
                const int8_t* wn = w + n * w_sn;
                int32_t s = 0;
                for (int64_t k = 0; k < K; ++k) s += (int32_t)am[k] * (int32_t)wn[k * w_sk];
                row[n] = s;
            }
        }
    }
}

/*
 * Epilogue of npu_quant_matmul, applied to the exact int32 accumulator.
 *   int32 bias (bias_dtype QO_I32) is added to the accumulator first (exact).
 *   v = float(acc) (round to nearest even)
 *   with pertoken_scale: v = fmaf(v * pertoken[m], scale[n], bias_f[n])
 *   without:             v = fmaf(v,               scale[n], bias_f[n])
 *   where bias_f is the float bias (bf16/f16/f32 -> float32) or +0.
 *   out_dtype QO_BF16 / QO_F16: RNE cast of v.
 *   out_dtype QO_I8: clamp(rint(fmaf(float(acc), scale[n], offset[n])), -128, 127)
 *   out_dtype QO_I32: acc itself.
 * scale_len / offset_len are 1 (per-tensor) or N (per-channel).
 * Output written row-major [M,N].  Bias semantics follow addmm
 * (op_plugin/ops/base_ops/opapi/AddmmKernelNpuOpApi.cpp:24-55): bias
 * broadcast over rows.
 */
void qo_quant_matmul_epilogue(const int32_t* acc, int64_t M, int64_t N,
                              const float* scale, int64_t scale_len,
                              const float* offset, int64_t offset_len,
                              const float* pertoken, const void* bias, int bias_dtype,
                              void* out, int out_dtype) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            int32_t a = acc[m * N + n];
            float bf = 0.0f;
            if (bias) {
                if (bias_dtype == QO_I32) a = (int32_t)((uint32_t)a + (uint32_t)((const int32_t*)bias)[n]);
                else bf = load_any(bias, n, bias_dtype);
            }
            int64_t o = m * N + n;
            if (out_dtype == QO_I32) { ((int32_t*)out)[o] = a; continue; }
            float s = scale[scale_len == 1 ? 0 : n];
            float v = (float)a;
            if (out_dtype == QO_I8) {
                float off = offset ? offset[offset_len == 1 ? 0 : n] : 0.0f;
                ((int8_t*)out)[o] = qo_sat_i8(rintf(fmaf(v, s, off)));
                continue;
            }
            if (pertoken) v = v * pertoken[m];
            v = fmaf(v, s, bf);
            if (out_dtype == QO_BF16) ((uint16_t*)out)[o] = qo_f32_to_bf16(v);
            else if (out_dtype == QO_F16) ((uint16_t*)out)[o] = qo_f32_to_f16(v);
            else ((float*)out)[o] = v;
        }
    }
}

/* ------------------------------------------------------------------ */
/* int4 packing: 8 signed nibbles per int32 along N.                   */
/* ------------------------------------------------------------------ */
/*
 * w is int8 [K,N] with values in [-8,7], N % 8 == 0.  packed[k, j] holds
 * w[k, 8j+i] in bits [4i, 4i+4) as a two's-complement nibble (i = 0 is the
 * lowest nibble).  int4 has no dtype in the reference
 * (op_plugin/third_party/acl/inc/graph/types.h:57), so this order is the
 * build's own convention.
 */
void qo_int4_pack(const int8_t* w, int64_t K, int64_t N, int32_t* packed) {
    int64_t NW = N / 8;
    for (int64_t k = 0; k < K; ++k)
        for (int64_t j = 0; j < NW; ++j) {
            uint32_t word = 0;
            for (int i = 0; i < 8; ++i) word |= ((uint32_t)(uint8_t)w[k * N + 8 * j + i] & 0xfu) << (4 * i);
            packed[k * NW + j] = (int32_t)word;
        }
}

void qo_int4_unpack(const int32_t* packed, int64_t K, int64_t N, int8_t* w) {
    int64_t NW = N / 8;
    for (int64_t k = 0; k < K; ++k)
        for (int64_t j = 0; j < NW; ++j) {
            uint32_t word = (uint32_t)packed[k * NW + j];
            for (int i = 0; i < 8; ++i) {
                int v = (int)((word >> (4 * i)) & 0xfu);
                w[k * N + 8 * j + i] = (int8_t)(v >= 8 ? v - 16 : v);
            }
        }
}

/* ------------------------------------------------------------------ */
/* MFMA-tiled ("NZ") int4 weight layout                                */
/* ------------------------------------------------------------------ */
/*
 * npu_format_cast(weight, FRACTAL_NZ) for an int4 weight: this build's
 * device-native counterpart of the FRACTAL_NZ weight casts the reference
 * applies before matmuls (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:303-316,
 * op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:103-107; format number 29,
 * op_plugin/third_party/acl/inc/graph/types.h:138).  The tiled tensor is
 * int32 [N/16][K/128][64][4].  Weight element (k, n) lives in word
 *   ((n/16 * (K/128) + k/128) * 64 + lane) * 4 + j,
 *   c = (k%128) / 8, lane = n%16 + 16*(c%4), j = c/4,
 * at nibble p = i/2 for even i = k%8 and p = 4 + i/2 for odd i (two's
 * complement, bits 4p..4p+3).  Both directions are plain gathers over (k, n).
 */
static inline int64_t nz4_word(int64_t k, int64_t n, int64_t K, int *nibble) {
    int64_t c = (k % 128) / 8, i = k % 8;
    int64_t lane = n % 16 + 16 * (c % 4), j = c / 4;
    *nibble = (int)((i % 2 == 0) ? i / 2 : 4 + i / 2);
    return (((n / 16) * (K / 128) + k / 128) * 64 + lane) * 4 + j;
}

/* nd: int32 [K, N/8] as qo_int4_pack writes it; nz: int32 [N/16][K/128][64][4]. */
void qo_w4_nz_pack(const int32_t* nd, int64_t K, int64_t N, int32_t* nz) {
    int64_t NW = N / 8;
    memset(nz, 0, (size_t)(K * N / 8) * sizeof(int32_t));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) {
            uint32_t v = ((uint32_t)nd[k * NW + n / 8] >> (4 * (n % 8))) & 0xfu;
            int p;
            int64_t w = nz4_word(k, n, K, &p);
            nz[w] = (int32_t)((uint32_t)nz[w] | (v << (4 * p)));
        }
}

void qo_w4_nz_unpack(const int32_t* nz, int64_t K, int64_t N, int32_t* nd) {
    int64_t NW = N / 8;
    memset(nd, 0, (size_t)(K * NW) * sizeof(int32_t));
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) {
            int p;
            int64_t w = nz4_word(k, n, K, &p);
            uint32_t v = ((uint32_t)nz[w] >> (4 * p)) & 0xfu;
            nd[k * NW + n / 8] = (int32_t)((uint32_t)nd[k * NW + n / 8] | (v << (4 * (n % 8))));
        }
}

/*
 * The int8 counterpart (W8A8 and W8A16 weights): int8 [N/16][K/64][64][16].
 * Weight element (k, n) is byte
 *   ((n/16 * (K/64) + k/64) * 64 + lane) * 16 + k%16,  lane = n%16 + 16*((k%64)/16),
 * so each lane's 16 bytes are 16 consecutive k of one column: the B operand of
 * one v_mfma_i32_16x16x64_i8, or two 8-row bf16 MFMA operands.
 */
static inline int64_t nz8_byte(int64_t k, int64_t n, int64_t K) {
    int64_t lane = n % 16 + 16 * ((k % 64) / 16);
    return (((n / 16) * (K / 64) + k / 64) * 64 + lane) * 16 + k % 16;
}

/* nd: int8 [K, N] row-major; nz: int8 [N/16][K/64][64][16]. */
void qo_w8_nz_pack(const int8_t* nd, int64_t K, int64_t N, int8_t* nz) {
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) nz[nz8_byte(k, n, K)] = nd[k * N + n];
}

void qo_w8_nz_unpack(const int8_t* nz, int64_t K, int64_t N, int8_t* nd) {
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) nd[k * N + n] = nz[nz8_byte(k, n, K)];
}

/* ------------------------------------------------------------------ */
/* npu_weight_quant_batchmatmul (W4A16 / W8A16)                        */
/* ------------------------------------------------------------------ */
/*
 * out[m,n] = cast_out( sum_k x[m,k] * (w[k,n] + off[g,n]) * scale[g,n] + bias[n] ),
 * g = k / group (group == 0: per-channel, g = 0).  The sum is carried in
 * float64 with the dequantized weight kept exact (no rounding of
 * (w+off)*scale to the activation dtype); the float64 total is rounded to
 * float32, then to the output dtype.  weight_dtype QO_I32: int4 packed as in
 * qo_int4_pack ([K, N/8]); QO_I8: int8 [K,N].  offset may be NULL.
 * "Upcast, accumulate, cast once" is the reference's golden convention for
 * low-precision matmuls (test/test_custom_ops/test_mm_reduce_scatter_base.py:74-79).
 */
void qo_weight_quant_bmm(const uint16_t* x, int x_dtype, const void* weight, int weight_dtype,
                         const uint16_t* scale, const uint16_t* offset, int scale_dtype,
                         int64_t M, int64_t N, int64_t K, int64_t group,
                         const void* bias, int bias_dtype, uint16_t* out, int out_dtype,
                         double* work /* (M + 1) * N doubles */) {
    int64_t NW = N / 8;
    double* wf = work + M * N;   /* dequantized weight row k, exact in float64 */
    for (int64_t i = 0; i < M * N; ++i) work[i] = 0.0;
    for (int64_t k = 0; k < K; ++k) {
        int64_t g = group > 0 ? k / group : 0;
        for (int64_t n = 0; n < N; ++n) {
            int wv;
            if (weight_dtype == QO_I32) {
                uint32_t word = (uint32_t)((const int32_t*)weight)[k * NW + n / 8];
                wv = (int)((word >> (4 * (n % 8))) & 0xfu);
                if (wv >= 8) wv -= 16;
            } else {
                wv = ((const int8_t*)weight)[k * N + n];
            }
            double off = offset ? (double)load_half(offset, g * N + n, scale_dtype) : 0.0;
            double s = (double)load_half(scale, g * N + n, scale_dtype);
            wf[n] = ((double)wv + off) * s;
        }
        for (int64_t m = 0; m < M; ++m) {
            double xv = (double)load_half(x, m * K + k, x_dtype);
            double* row = work + m * N;
            for (int64_t n = 0; n < N; ++n) row[n] += xv * wf[n];
        }
    }
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            double v = work[m * N + n];
            if (bias) v += (double)load_any(bias, n, bias_dtype);
            float f = (float)v;
            out[m * N + n] = out_dtype == QO_BF16 ? qo_f32_to_bf16(f) : qo_f32_to_f16(f);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Quantized MLP block neighbours: RMSNorm and SwiGLU.                 */
/* ------------------------------------------------------------------ */
/*
 * y = x * rstd * gamma, rstd = 1/sqrt(mean(x^2) + eps), following the numpy
 * golden in test/test_custom_ops/test_npu_rms_norm.py:10-17; carried in
 * float64 here, y rounded to the activation dtype, rstd to float32.
 */
/* float32 x, gamma, y (the reference's golden case, test_npu_rms_norm.py:24-33), float64 arithmetic. */
void qo_rms_norm_f32(const float* x, const float* gamma, int64_t rows, int64_t D, double eps, float* y,
                     float* rstd) {
    for (int64_t r = 0; r < rows; ++r) {
        double ss = 0.0;
        for (int64_t d = 0; d < D; ++d) ss += (double)x[r * D + d] * (double)x[r * D + d];
        double rs = 1.0 / sqrt(ss / (double)D + eps);
        rstd[r] = (float)rs;
        for (int64_t d = 0; d < D; ++d) y[r * D + d] = (float)((double)x[r * D + d] * rs * (double)gamma[d]);
    }
}

void qo_rms_norm(const uint16_t* x, int x_dtype, const uint16_t* gamma, int64_t rows, int64_t D,
                 double eps, uint16_t* y, float* rstd) {
    for (int64_t r = 0; r < rows; ++r) {
        double ss = 0.0;
        for (int64_t d = 0; d < D; ++d) {
            double v = load_half(x, r * D + d, x_dtype);
            ss += v * v;
        }
        double rs = 1.0 / sqrt(ss / (double)D + eps);
        rstd[r] = (float)rs;
        for (int64_t d = 0; d < D; ++d) {
            double v = (double)load_half(x, r * D + d, x_dtype) * rs * (double)load_half(gamma, d, x_dtype);
            float f = (float)v;
            y[r * D + d] = x_dtype == QO_BF16 ? qo_f32_to_bf16(f) : qo_f32_to_f16(f);
        }
    }
}

/*
 * h is [rows, 2*I]; out[r,i] = silu(h[r,i]) * h[r,I+i] (first half = gate),
 * silu(a) = a / (1 + exp(-a)), in float64, rounded to the activation dtype.
 * The gated split halves the last dim as npu_geglu does
 * (op_plugin/ops/v1r11/opapi/GeGluKernelNpuOpApi.cpp:29-38).
 */
void qo_swiglu(const uint16_t* h, int dt, int64_t rows, int64_t I, uint16_t* out) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < I; ++i) {
            double a = load_half(h, r * 2 * I + i, dt);
            double b = load_half(h, r * 2 * I + I + i, dt);
            double v = a / (1.0 + exp(-a)) * b;
            float f = (float)v;
            out[r * I + i] = dt == QO_BF16 ? qo_f32_to_bf16(f) : qo_f32_to_f16(f);
        }
}

/* Elementwise dtype conversion over an array (used to pin the scalar casts). */
/* ------------------------------------------------------------------ */
/* Static quantization: quantize_per_tensor / quantize_per_channel /   */
/* dequantize                                                          */
/* ------------------------------------------------------------------ */
/*
 * The reference's NPU quantize ops return plain integer tensors: QInt8 ->
 * int8, QUInt8 -> uint8, QInt32 -> int32
 * (op_plugin/ops/base_ops/aclops/QuantizePerTensorKernelNpu.cpp:60-67,
 * op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:81-88); the
 * element rule is in CANN's closed Quantize op, so this restates torch's own
 * affine quantizer for the same schema:
 *   q = clamp(RN(rint(x * RN(1 / float(scale))) + float(zero_point)), qmin, qmax),
 * one float32 multiply by the float32 reciprocal of the scale, ties to even,
 * then the zero point added to the rounded value in float32 (torch's
 * quantize_val adds its int64 zero point to a float, so past 2^24 the sum
 * rounds: 2e9 - 7 stays 2e9 for qint32).  x is viewed as
 * [outer][C][inner]; channel c uses scales[c], zero_points[c] (per tensor:
 * C == 1).  A NaN input gives qmin.  dequantize is the reference's
 * op_plugin/ops/v1r11/opapi/DequantizeKernelNpuOpApi.cpp:22-24: a plain cast of
 * the integers to float32.
 */
void qo_quantize(const void* x, int x_dtype, int64_t outer, int64_t C, int64_t inner, const float* scales,
                 const int64_t* zero_points, void* q, int q_dtype) {
    const double qmin = q_dtype == QO_I8 ? -128.0 : q_dtype == QO_U8 ? 0.0 : -2147483648.0;
    const double qmax = q_dtype == QO_I8 ? 127.0 : q_dtype == QO_U8 ? 255.0 : 2147483647.0;
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t c = 0; c < C; ++c) {
            const float r = 1.0f / scales[c];
            for (int64_t i = 0; i < inner; ++i) {
                const int64_t e = (o * C + c) * inner + i;
                const float v = load_any(x, e, x_dtype);
                const float t = v * r;
                const float z = rintf(t) + (float)zero_points[c];  /* float32 add, as torch's quantize_val */
                double d = isnan(z) ? qmin : (double)z;
                d = d < qmin ? qmin : (d > qmax ? qmax : d);
                if (q_dtype == QO_I8) ((int8_t*)q)[e] = (int8_t)d;
                else if (q_dtype == QO_U8) ((uint8_t*)q)[e] = (uint8_t)d;
                else ((int32_t*)q)[e] = (int32_t)d;
            }
        }
}

void qo_dequantize(const void* q, int q_dtype, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        if (q_dtype == QO_I8) out[i] = (float)((const int8_t*)q)[i];
        else if (q_dtype == QO_U8) out[i] = (float)((const uint8_t*)q)[i];
        else out[i] = (float)((const int32_t*)q)[i];
    }
}

void qo_cvt_array(const void* in, int in_dt, void* out, int out_dt, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float v = load_any(in, i, in_dt);
        if (out_dt == QO_F32) ((float*)out)[i] = v;
        else if (out_dt == QO_BF16) ((uint16_t*)out)[i] = qo_f32_to_bf16(v);
        else ((uint16_t*)out)[i] = qo_f32_to_f16(v);
    }
}
