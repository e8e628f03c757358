// extern "C" entry points of libqk_hip.so (declared in include/qk_abi.h).
//
// Each entry validates its plain-pointer arguments, turns a failure into a
// negative return code plus a thread-local message (the role
// aclGetRecentErrMsg() plays behind EXEC_NPU_CMD,
// op_plugin/utils/op_api_common.h:544-555), and enqueues the kernels on the
// caller's stream.  Nothing here allocates or synchronises.
#include <atomic>
#include <cmath>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include <unistd.h>

#include "kernels/common.h"

namespace qk {

// Split-K counter tags: a process-wide call counter seeded from the clock and
// the process id, scrambled by the splitmix64 output function (Steele, Lea and
// Flood, "Fast splittable pseudorandom number generators", 2014) so that tags
// look random against whatever data a fresh workspace holds, and cut to 48
// bits; 0 and all ones are skipped, so a zero- or 0xFF-filled counter word
// never carries a live tag.  A counter word left by an earlier call is zero
// (its last arrival cleared it), so tags of different calls need not differ.
uint64_t next_split_tag() {
    static std::atomic<uint64_t> seq{(uint64_t)std::chrono::steady_clock::now().time_since_epoch().count() ^
                                     ((uint64_t)getpid() << 32)};
    constexpr uint64_t kMask = ((uint64_t)1 << (64 - kSplitCountBits)) - 1;
    for (;;) {
        uint64_t z = seq.fetch_add(0x9e3779b97f4a7c15ull, std::memory_order_relaxed);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        const uint64_t tag = z & kMask;
        if (tag != 0 && tag != kMask) return tag;
    }
}

namespace {

bool parse_plan(const char* spec, PlanOverride& o) {
    PlanOverride r;
    std::string s(spec ? spec : "");
    size_t pos = 0;
    while (pos < s.size()) {
        size_t end = s.find(',', pos);
        if (end == std::string::npos) end = s.size();
        const std::string item = s.substr(pos, end - pos);
        pos = end + 1;
        if (item.empty()) continue;
        const size_t eq = item.find('=');
        if (eq == std::string::npos) return false;
        const std::string k = item.substr(0, eq), v = item.substr(eq + 1);
        int a = 0, b = 0, c = 0;
        if (k == "w4_stream") {
            if (v == "off") r.w4_stream_off = true;
            else if (std::sscanf(v.c_str(), "%d:%d:%d", &a, &b, &c) == 3 && (a == 8 || a == 16) &&
                     ((b == 4 && (c == 2 || c == 4)) || (a == 8 && b == 8 && (c == 2 || c == 3)))) {
                r.w4_stream_nwave = a;
                r.w4_stream_nkb = b;
                r.w4_stream_pf = c;
            } else return false;
        } else if (k == "w4_stream_wpl" && (v == "16" || v == "32" || v == "64")) {
            r.w4_stream_wpl = std::atoi(v.c_str());
        } else if (k == "w4_gemm") {
            if (v == "force") r.w4_gemm = 1;
            else if (v == "nodma") r.w4_gemm = 2;
            else if (v == "off") r.w4_gemm = 3;
            else return false;
        } else if (k == "w4_splits" && std::sscanf(v.c_str(), "%d", &a) == 1 && a >= 1 && a <= 4096) {
            r.w4_splits = a;
        } else if (k == "qmm_dma" && (v == "0" || v == "1")) {
            r.qmm_dma = v == "1";
        } else if (k == "qmm_bm128" && (v == "0" || v == "1")) {
            r.qmm_bm128 = v == "1";
        } else if (k == "qmm_mid" && (v == "0" || v == "1")) {
            r.qmm_mid = v == "1";
        } else if (k == "mid_bm" && (v == "16" || v == "32" || v == "64")) {
            r.mid_bm = std::atoi(v.c_str());
        } else if (k == "mid_split" && (v == "1" || v == "2")) {
            r.mid_split = std::atoi(v.c_str());
        } else if (k == "mid_bn" && (v == "64" || v == "128")) {
            r.mid_bn = std::atoi(v.c_str());
        } else if (k == "w4nz" && v == "off") {
            r.w4nz_off = true;
        } else if (k == "nzg_sk" && (v == "0" || v == "1" || v == "tailfirst")) {
            r.nzg_sk = v == "0" ? 0 : v == "1" ? 1 : 2;
        } else if (k == "nzg_sk_dp" && std::sscanf(v.c_str(), "%d", &a) == 1 && a >= 0 && a <= 64) {
            r.nzg_sk_dp = a;
        } else if (k == "qmm_rev" && (v == "0" || v == "1")) {
            r.qmm_rev = std::atoi(v.c_str());
        } else if (k == "qmm_small" && (v == "0" || v == "2" || v == "4" || v == "8")) {
            r.qmm_small = std::atoi(v.c_str());
        } else if (k == "w4nz_wg" && std::sscanf(v.c_str(), "%d", &a) == 1 && a >= 1 && a <= 65536) {
            r.w4nz_wg = a;
        } else if (k == "w4nz_nit" && std::sscanf(v.c_str(), "%d", &a) == 1 && a >= 1 && a <= 8) {
            r.w4nz_nit = a;
        } else if (k == "skinny_pf" && (v == "1" || v == "2" || v == "3")) {
            r.skinny_pf = std::atoi(v.c_str());
        } else if (k == "skinny_splits" && std::sscanf(v.c_str(), "%d", &a) == 1 && a >= 1 && a <= 64 &&
                   (a & (a - 1)) == 0) {
            r.skinny_splits = a;
        } else {
            return false;
        }
    }
    o = r;
    return true;
}

// Snapshots are never freed: a planner may still read the previous one.
std::atomic<const PlanOverride*>& plan_slot() {
    static std::atomic<const PlanOverride*> slot{[] {
        auto* o = new PlanOverride();
        if (const char* e = std::getenv("QK_DEBUG_PLAN")) {
            if (!parse_plan(e, *o)) std::fprintf(stderr, "libqk_hip: QK_DEBUG_PLAN=\"%s\" not understood, ignored\n", e);
        }
        return o;
    }()};
    return slot;
}

}  // namespace

const PlanOverride& plan_override() { return *plan_slot().load(std::memory_order_acquire); }

bool set_plan_override(const char* spec) {
    auto* o = new PlanOverride();
    if (!parse_plan(spec, *o)) {
        delete o;
        return false;
    }
    plan_slot().store(o, std::memory_order_release);
    return true;
}

}  // namespace qk

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int launched(hipError_t e, const char* op) {
    if (e != hipSuccess) return fail(QK_ERR_LAUNCH, "%s: kernel launch failed: %s", op, hipGetErrorString(e));
    return QK_OK;
}

bool is_half(int dt) { return dt == QK_F16 || dt == QK_BF16; }
bool is_float_out(int dt) { return dt == QK_F16 || dt == QK_BF16 || dt == QK_F32; }

constexpr int64_t kMaxGrid = (int64_t)1 << 31;  // gridDim.x limit
constexpr int64_t kMaxExactK = 131071;           // 131071 * 128 * 128 < 2^31

// The size, output-type and epilogue checks both W8A8 entry points share; fills p's sizes and epilogue.
int quant_matmul_args(const char* op, int64_t M, int64_t N, int64_t K, const float* scale, int64_t scale_len,
                      const float* offset, int64_t offset_len, const float* pertoken_scale, const void* bias,
                      int bias_dtype, void* out, int out_dtype, qk::QmmArgs& p) {
    if (M < 0 || N < 0 || K < 0) return fail(QK_ERR_ARG, "%s: negative size M=%lld N=%lld K=%lld", op, (long long)M, (long long)N, (long long)K);
    if (!(is_float_out(out_dtype) || out_dtype == QK_I8 || out_dtype == QK_I32))
        return fail(QK_ERR_ARG, "%s: unsupported output dtype %d", op, out_dtype);
    if (K > kMaxExactK) return fail(QK_ERR_UNSUPPORTED, "%s: K=%lld exceeds %lld, the int32-exact bound", op, (long long)K, (long long)kMaxExactK);
    if (M == 0 || N == 0) return QK_OK;
    if (!out) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (out_dtype != QK_I32) {
        if (!scale) return fail(QK_ERR_ARG, "%s: scale is required for output dtype %d", op, out_dtype);
        if (scale_len != 1 && scale_len != N)
            return fail(QK_ERR_ARG, "%s: scale must have 1 or N=%lld elements (got %lld)", op, (long long)N, (long long)scale_len);
    }
    if (offset) {
        if (out_dtype != QK_I8) return fail(QK_ERR_ARG, "%s: offset is only valid with an int8 output", op);
        if (offset_len != 1 && offset_len != N)
            return fail(QK_ERR_ARG, "%s: offset must have 1 or N elements (got %lld)", op, (long long)offset_len);
    }
    if (pertoken_scale && !is_float_out(out_dtype))
        return fail(QK_ERR_ARG, "%s: pertoken_scale needs a float16/bfloat16/float32 output", op);
    if (bias) {
        if (!(bias_dtype == QK_I32 || is_half(bias_dtype) || bias_dtype == QK_F32))
            return fail(QK_ERR_ARG, "%s: bias dtype %d unsupported", op, bias_dtype);
        if (bias_dtype != QK_I32 && !is_float_out(out_dtype))
            return fail(QK_ERR_ARG, "%s: a float bias needs a float output (int8/int32 outputs take an int32 bias)", op);
    }
    p.M = M;
    p.N = N;
    p.K = K;
    p.epi.scale = scale;
    p.epi.scale_per_ch = scale_len != 1;
    p.epi.offset = offset;
    p.epi.offset_per_ch = offset_len != 1;
    p.epi.pertoken = pertoken_scale;
    p.epi.bias = bias;
    p.epi.bias_dtype = bias ? bias_dtype : 0;
    p.epi.out = out;
    p.epi.ldo = N;
    p.epi.out_dtype = out_dtype;
    return QK_OK;
}

int check_workspace(const char* op, size_t need, const void* workspace, size_t workspace_bytes) {
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(QK_ERR_WORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, workspace_bytes);
    if (need > 0 && (uintptr_t)workspace % 256 != 0)
        return fail(QK_ERR_WORKSPACE, "%s: the workspace must be 256-byte aligned", op);
    return QK_OK;
}

}  // namespace

extern "C" {

const char* qk_last_error(void) { return g_last_error.c_str(); }

int qk_abi_version(void) { return 6; }

int qk_debug_set_plan(const char* spec) {
    g_last_error.clear();
    if (!qk::set_plan_override(spec)) return fail(QK_ERR_ARG, "qk_debug_set_plan: \"%s\" not understood", spec ? spec : "");
    return QK_OK;
}

int qk_dynamic_quant(const void* x, int x_dtype, int64_t rows, int64_t K, const float* smooth_scales, int8_t* y,
                     float* scale, qk_stream_t stream) {
    g_last_error.clear();
    if (!is_half(x_dtype)) return fail(QK_ERR_ARG, "npu_dynamic_quant: x must be float16 or bfloat16 (got dtype %d)", x_dtype);
    if (rows < 0 || K < 0) return fail(QK_ERR_ARG, "npu_dynamic_quant: negative size rows=%lld K=%lld", (long long)rows, (long long)K);
    if (rows == 0) return QK_OK;
    if (!scale || (K > 0 && (!x || !y))) return fail(QK_ERR_ARG, "npu_dynamic_quant: null pointer");
    if (rows >= kMaxGrid) return fail(QK_ERR_UNSUPPORTED, "npu_dynamic_quant: %lld rows exceed the launch limit", (long long)rows);
    return launched(qk::launch_dynamic_quant(x, x_dtype, rows, K, smooth_scales, y, scale, (hipStream_t)stream),
                    "npu_dynamic_quant");
}

int qk_quant_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int out_dtype, size_t* bytes) {
    g_last_error.clear();
    (void)out_dtype;
    if (!bytes) return fail(QK_ERR_ARG, "npu_quant_matmul: bytes is null");
    if (M < 0 || N < 0 || K < 0) return fail(QK_ERR_ARG, "npu_quant_matmul: negative size");
    *bytes = qk::quant_matmul_workspace(M, N, K);
    return QK_OK;
}

int qk_quant_matmul(const int8_t* x1, int64_t ldx1, const int8_t* x2, int64_t x2_stride_k, int64_t x2_stride_n,
                    int64_t M, int64_t N, int64_t K, const float* scale, int64_t scale_len, const float* offset,
                    int64_t offset_len, const float* pertoken_scale, const void* bias, int bias_dtype, void* out,
                    int out_dtype, void* workspace, size_t workspace_bytes, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_quant_matmul";
    qk::QmmArgs p;
    int rc = quant_matmul_args(op, M, N, K, scale, scale_len, offset, offset_len, pertoken_scale, bias, bias_dtype,
                               out, out_dtype, p);
    if (rc != QK_OK || M == 0 || N == 0) return rc;
    if (K > 0 && (!x1 || !x2)) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (ldx1 < K) return fail(QK_ERR_ARG, "%s: ldx1=%lld < K=%lld", op, (long long)ldx1, (long long)K);
    if (!(x2_stride_k == 1 || x2_stride_n == 1))
        return fail(QK_ERR_ARG, "%s: x2 must be [K,N]-contiguous or a transposed view of [N,K] (strides %lld,%lld)", op,
                    (long long)x2_stride_k, (long long)x2_stride_n);
    if ((rc = check_workspace(op, qk::quant_matmul_workspace(M, N, K), workspace, workspace_bytes)) != QK_OK) return rc;
    p.a = x1;
    p.lda = ldx1;
    p.b = x2;
    p.sbk = x2_stride_k;
    p.sbn = x2_stride_n;
    return launched(qk::launch_quant_matmul(p, workspace, workspace_bytes, (hipStream_t)stream), op);
}

int qk_quant_matmul_nz_workspace_size(int64_t M, int64_t N, int64_t K, int out_dtype, size_t* bytes) {
    g_last_error.clear();
    (void)out_dtype;
    if (!bytes) return fail(QK_ERR_ARG, "npu_quant_matmul: bytes is null");
    if (M < 0 || N < 0 || K < 0) return fail(QK_ERR_ARG, "npu_quant_matmul: negative size");
    *bytes = qk::quant_matmul_nz_workspace(M, N, K);
    return QK_OK;
}

int qk_quant_matmul_nz(const int8_t* x1, int64_t ldx1, const int8_t* x2_nz, int64_t M, int64_t N, int64_t K,
                       const float* scale, int64_t scale_len, const float* offset, int64_t offset_len,
                       const float* pertoken_scale, const void* bias, int bias_dtype, void* out, int out_dtype,
                       void* workspace, size_t workspace_bytes, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_quant_matmul";
    qk::QmmArgs p;
    int rc = quant_matmul_args(op, M, N, K, scale, scale_len, offset, offset_len, pertoken_scale, bias, bias_dtype,
                               out, out_dtype, p);
    if (rc != QK_OK || M == 0 || N == 0) return rc;
    if (K % 64 != 0 || N % 16 != 0)
        return fail(QK_ERR_ARG, "%s: an NZ weight needs K %% 64 == 0 and N %% 16 == 0 (K=%lld, N=%lld)", op,
                    (long long)K, (long long)N);
    if (K > 0 && (!x1 || !x2_nz)) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (ldx1 < K || ldx1 % 16 != 0 || ldx1 >= ((int64_t)1 << 24))
        return fail(QK_ERR_ARG, "%s: with an NZ weight ldx1 must be a multiple of 16 in [K, 2^24) (ldx1=%lld, K=%lld)",
                    op, (long long)ldx1, (long long)K);
    if ((uintptr_t)x1 % 16 != 0 || (uintptr_t)x2_nz % 16 != 0 || (uintptr_t)out % 16 != 0)
        return fail(QK_ERR_ARG, "%s: with an NZ weight x1, x2 and out must be 16-byte aligned", op);
    if ((rc = check_workspace(op, qk::quant_matmul_nz_workspace(M, N, K), workspace, workspace_bytes)) != QK_OK)
        return rc;
    p.a = x1;
    p.lda = ldx1;
    p.b = x2_nz;
    p.sbk = 0;
    p.sbn = 0;
    return launched(qk::launch_quant_matmul_nz(p, workspace, workspace_bytes, (hipStream_t)stream), op);
}

int qk_quant_matmul_swiglu(const int8_t* x1, int64_t ldx1, const int8_t* x2, int x2_format, int64_t x2_stride_k,
                           int64_t M, int64_t I, int64_t K, const float* scale, int64_t scale_len,
                           const float* pertoken_scale, void* out, int out_dtype, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_quant_matmul_swiglu";
    if (I < 0 || I > ((int64_t)1 << 40)) return fail(QK_ERR_ARG, "%s: bad I=%lld", op, (long long)I);
    if (!is_half(out_dtype)) return fail(QK_ERR_ARG, "%s: the output must be float16 or bfloat16 (got %d)", op, out_dtype);
    if (x2_format != QK_FORMAT_ND && x2_format != QK_FORMAT_FRACTAL_NZ)
        return fail(QK_ERR_ARG, "%s: x2_format must be QK_FORMAT_ND or QK_FORMAT_FRACTAL_NZ (got %d)", op, x2_format);
    qk::QmmArgs p;
    int rc = quant_matmul_args(op, M, 2 * I, K, scale, scale_len, nullptr, 0, pertoken_scale, nullptr, 0, out,
                               out_dtype, p);
    if (rc != QK_OK || M == 0 || I == 0) return rc;
    if (K > 0 && (!x1 || !x2)) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (ldx1 < K) return fail(QK_ERR_ARG, "%s: ldx1=%lld < K=%lld", op, (long long)ldx1, (long long)K);
    if (x2_format == QK_FORMAT_ND && x2_stride_k < 2 * I)
        return fail(QK_ERR_ARG, "%s: x2_stride_k=%lld < 2I=%lld", op, (long long)x2_stride_k, (long long)(2 * I));
    p.a = x1;
    p.lda = ldx1;
    p.b = x2;
    p.sbk = x2_format == QK_FORMAT_ND ? x2_stride_k : 0;
    p.sbn = x2_format == QK_FORMAT_ND ? 1 : 0;
    p.epi.ldo = I;
    const hipError_t e =
        qk::launch_quant_matmul_swiglu(p, x2_format == QK_FORMAT_FRACTAL_NZ, nullptr, (hipStream_t)stream);
    if (e == hipErrorInvalidValue)
        return fail(QK_ERR_UNSUPPORTED, "%s: the fused kernel does not take M=%lld I=%lld K=%lld with these operands "
                    "(I %% 128, K %% 256, 16-byte aligned rows and pointers)", op, (long long)M, (long long)I, (long long)K);
    return launched(e, op);
}

// h [M, I] (16-bit) at the head of the workspace, then the partial absmax fp32 [M][I / 128], 256-byte aligned
static size_t swiglu_quant_h_bytes(int64_t M, int64_t I) { return ((size_t)M * (size_t)I * 2 + 255) & ~(size_t)255; }

int qk_quant_matmul_swiglu_quant_workspace_size(int64_t M, int64_t I, size_t* bytes) {
    g_last_error.clear();
    if (!bytes) return fail(QK_ERR_ARG, "npu_quant_matmul_swiglu_quant: bytes is null");
    if (M < 0 || I < 0 || M > ((int64_t)1 << 40) || I > ((int64_t)1 << 40))
        return fail(QK_ERR_ARG, "npu_quant_matmul_swiglu_quant: bad M=%lld I=%lld", (long long)M, (long long)I);
    *bytes = swiglu_quant_h_bytes(M, I) + (size_t)M * (size_t)((I + 127) / 128) * 4;
    return QK_OK;
}

int qk_quant_matmul_swiglu_quant(const int8_t* x1, int64_t ldx1, const int8_t* x2, int x2_format,
                                 int64_t x2_stride_k, int64_t M, int64_t I, int64_t K, const float* scale,
                                 int64_t scale_len, const float* pertoken_scale, int h_dtype, int8_t* q,
                                 float* q_scale, void* workspace, size_t workspace_bytes, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_quant_matmul_swiglu_quant";
    size_t need = 0;
    int rc = qk_quant_matmul_swiglu_quant_workspace_size(M, I, &need);
    if (rc != QK_OK) return rc;
    if (M == 0 || I == 0) return QK_OK;
    if (!q || !q_scale) return fail(QK_ERR_ARG, "%s: null output", op);
    if ((rc = check_workspace(op, need, workspace, workspace_bytes)) != QK_OK) return rc;
    if (!is_half(h_dtype)) return fail(QK_ERR_ARG, "%s: h must be float16 or bfloat16 (got %d)", op, h_dtype);
    if (I % 128 != 0 || (uintptr_t)q % 8 != 0)
        return fail(QK_ERR_UNSUPPORTED, "%s: the fused kernels take I %% 128 == 0 and an 8-byte aligned q (I=%lld)", op,
                    (long long)I);
    void* h = workspace;
    float* amax = reinterpret_cast<float*>(static_cast<char*>(workspace) + swiglu_quant_h_bytes(M, I));
    if (x2_format != QK_FORMAT_ND && x2_format != QK_FORMAT_FRACTAL_NZ)
        return fail(QK_ERR_ARG, "%s: x2_format must be QK_FORMAT_ND or QK_FORMAT_FRACTAL_NZ (got %d)", op, x2_format);
    qk::QmmArgs p;
    if ((rc = quant_matmul_args(op, M, 2 * I, K, scale, scale_len, nullptr, 0, pertoken_scale, nullptr, 0, h, h_dtype,
                                p)) != QK_OK)
        return rc;
    if (K > 0 && (!x1 || !x2)) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (ldx1 < K) return fail(QK_ERR_ARG, "%s: ldx1=%lld < K=%lld", op, (long long)ldx1, (long long)K);
    if (x2_format == QK_FORMAT_ND && x2_stride_k < 2 * I)
        return fail(QK_ERR_ARG, "%s: x2_stride_k=%lld < 2I=%lld", op, (long long)x2_stride_k, (long long)(2 * I));
    p.a = x1;
    p.lda = ldx1;
    p.b = x2;
    p.sbk = x2_format == QK_FORMAT_ND ? x2_stride_k : 0;
    p.sbn = x2_format == QK_FORMAT_ND ? 1 : 0;
    p.epi.ldo = I;
    hipError_t e = qk::launch_quant_matmul_swiglu(p, x2_format == QK_FORMAT_FRACTAL_NZ, amax, (hipStream_t)stream);
    if (e == hipErrorInvalidValue)
        return fail(QK_ERR_UNSUPPORTED, "%s: the fused kernel does not take M=%lld I=%lld K=%lld with these operands "
                    "(I %% 128, K %% 256, 16-byte aligned rows and pointers)", op, (long long)M, (long long)I, (long long)K);
    if (e != hipSuccess) return launched(e, op);
    e = qk::launch_dynamic_quant_premax(h, h_dtype, M, I, amax, (int)(I / 128), q, q_scale, (hipStream_t)stream);
    return launched(e, op);
}

int qk_weight_quant_bmm_workspace_size(int64_t M, int64_t N, int64_t K, int weight_dtype, int64_t group_size,
                                       size_t* bytes) {
    g_last_error.clear();
    if (!bytes) return fail(QK_ERR_ARG, "npu_weight_quant_batchmatmul: bytes is null");
    if (M < 0 || N < 0 || K < 0 || group_size < 0) return fail(QK_ERR_ARG, "npu_weight_quant_batchmatmul: negative size");
    *bytes = qk::weight_quant_bmm_workspace(M, N, K, weight_dtype, group_size);
    return QK_OK;
}

}  // extern "C"

namespace {

// Checks shared by the two weight-quant entry points; `ws` of `ws_bytes` is the scratch the call may use.
int weight_quant_bmm_run(const char* op, const void* x, int x_dtype, const void* weight, int weight_dtype,
                         const void* antiquant_scale, const void* antiquant_offset, int scale_dtype, int64_t M,
                         int64_t N, int64_t K, int64_t group_size, const void* bias, int bias_dtype, void* out,
                         int out_dtype, void* (*scratch)(size_t need, size_t* bytes, int* rc), void* workspace,
                         size_t workspace_bytes, qk_stream_t stream) {
    if (!is_half(x_dtype)) return fail(QK_ERR_ARG, "%s: x must be float16 or bfloat16", op);
    if (weight_dtype != QK_I32 && weight_dtype != QK_I8 && weight_dtype != QK_I4_NZ && weight_dtype != QK_I8_NZ &&
        weight_dtype != QK_I8_NK)
        return fail(QK_ERR_ARG, "%s: weight must be int32 (packed int4), int8 ([K, N] or [N, K]), or NZ int4 / int8", op);
    if (!is_half(scale_dtype)) return fail(QK_ERR_ARG, "%s: antiquant_scale must be float16 or bfloat16", op);
    if (!is_half(out_dtype)) return fail(QK_ERR_ARG, "%s: output must be float16 or bfloat16", op);
    if (M < 0 || N < 0 || K < 0 || group_size < 0) return fail(QK_ERR_ARG, "%s: negative size", op);
    if (weight_dtype == QK_I32 && N % 8 != 0) return fail(QK_ERR_ARG, "%s: int4 packing needs N %% 8 == 0 (N=%lld)", op, (long long)N);
    if (weight_dtype == QK_I4_NZ && (N % 16 != 0 || K % 128 != 0))
        return fail(QK_ERR_ARG, "%s: an int4 NZ weight needs N %% 16 == 0 and K %% 128 == 0 (N=%lld K=%lld)", op,
                    (long long)N, (long long)K);
    if (weight_dtype == QK_I8_NZ && (N % 16 != 0 || K % 64 != 0))
        return fail(QK_ERR_ARG, "%s: an int8 NZ weight needs N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)", op,
                    (long long)N, (long long)K);
    if (group_size > 0 && K % group_size != 0)
        return fail(QK_ERR_ARG, "%s: K=%lld is not a multiple of antiquant_group_size=%lld", op, (long long)K, (long long)group_size);
    if (bias && !(is_half(bias_dtype) || bias_dtype == QK_F32)) return fail(QK_ERR_ARG, "%s: bias dtype %d unsupported", op, bias_dtype);
    if (M == 0 || N == 0) return QK_OK;
    if (!out || (K > 0 && (!x || !weight || !antiquant_scale))) return fail(QK_ERR_ARG, "%s: null pointer", op);
    // The no-allocation scratch runs the op's own plan (so the same kernels, the same bits) wherever that
    // plan's workspace fits in it; otherwise the same kernels with whole tiles per workgroup in place of the NZ
    // prefill kernel's stream-K partials (the same bits too); otherwise the plan without the cast to NZ of a
    // row-major int4 / int8 weight, whose cast weight is what does not fit.
    size_t need = qk::weight_quant_bmm_workspace(M, N, K, weight_dtype, group_size, qk::kWsFull);
    if (scratch && need > QK_NOALLOC_SCRATCH_BYTES)
        need = qk::weight_quant_bmm_workspace(M, N, K, weight_dtype, group_size, qk::kWsNoStreamK);
    if (scratch && need > QK_NOALLOC_SCRATCH_BYTES)
        need = qk::weight_quant_bmm_workspace(M, N, K, weight_dtype, group_size, qk::kWsNoCast);
    if (scratch && need > 0) {
        int rc = QK_OK;
        workspace = scratch(need, &workspace_bytes, &rc);
        if (rc != QK_OK) return rc;
    }
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(QK_ERR_WORKSPACE, "%s: workspace of %zu bytes required, %zu given", op, need, workspace_bytes);
    if (need > 0 && (uintptr_t)workspace % 256 != 0)
        return fail(QK_ERR_WORKSPACE, "%s: the workspace must be 256-byte aligned", op);
    qk::WqbmmArgs p;
    p.x = x;
    p.x_dtype = x_dtype;
    p.w = weight;
    p.w_dtype = weight_dtype;
    p.scale = antiquant_scale;
    p.offset = antiquant_offset;
    p.s_dtype = scale_dtype;
    p.M = M;
    p.N = N;
    p.K = K;
    p.group = group_size;
    p.bias = bias;
    p.bias_dtype = bias ? bias_dtype : 0;
    p.out = out;
    p.out_dtype = out_dtype;
    return launched(qk::launch_weight_quant_bmm(p, workspace, workspace_bytes, (hipStream_t)stream), op);
}

// Scratch of qk_weight_quant_bmm_noalloc: one array per GPU, held by the
// library until the process ends.  Its host-side name is only a handle: the
// device address of the current GPU's copy comes from hipGetSymbolAddress,
// looked up once per device (on that device's first call) and cached.  The
// kernels need no particular contents in it (split-K counters are tagged per
// call; partial and group sums are written before they are read), so nothing
// is cleared.
constexpr int kMaxDevices = 64;
__device__ __align__(256) static unsigned char scratch[QK_NOALLOC_SCRATCH_BYTES];
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

void* noalloc_scratch(size_t need, size_t* bytes, int* rc) {
    const char* op = "npu_weight_quant_batchmatmul (no allocation)";
    if (need > QK_NOALLOC_SCRATCH_BYTES) {
        *rc = fail(QK_ERR_UNSUPPORTED, "%s: this shape needs %zu bytes of scratch, more than the %d the library holds",
                   op, need, QK_NOALLOC_SCRATCH_BYTES);
        return nullptr;
    }
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *rc = fail(QK_ERR_LAUNCH, "%s: no usable current device (%s)", op, hipGetErrorString(e));
        return nullptr;
    }
    void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!ptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!ptr) {
            e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !ptr) {
                *rc = fail(QK_ERR_LAUNCH, "%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", op,
                           dev, hipGetErrorString(e));
                return nullptr;
            }
            g_scratch_ptr[dev].store(ptr, std::memory_order_release);
        }
    }
    *bytes = QK_NOALLOC_SCRATCH_BYTES;
    return ptr;
}

}  // namespace

extern "C" {

int qk_weight_quant_bmm(const void* x, int x_dtype, const void* weight, int weight_dtype, const void* antiquant_scale,
                        const void* antiquant_offset, int scale_dtype, int64_t M, int64_t N, int64_t K,
                        int64_t group_size, const void* bias, int bias_dtype, void* out, int out_dtype,
                        void* workspace, size_t workspace_bytes, qk_stream_t stream) {
    g_last_error.clear();
    return weight_quant_bmm_run("npu_weight_quant_batchmatmul", x, x_dtype, weight, weight_dtype, antiquant_scale,
                                antiquant_offset, scale_dtype, M, N, K, group_size, bias, bias_dtype, out, out_dtype,
                                nullptr, workspace, workspace_bytes, stream);
}

int qk_weight_quant_bmm_noalloc(const void* x, int x_dtype, const void* weight, int weight_dtype,
                                const void* antiquant_scale, const void* antiquant_offset, int scale_dtype, int64_t M,
                                int64_t N, int64_t K, int64_t group_size, const void* bias, int bias_dtype, void* out,
                                int out_dtype, qk_stream_t stream) {
    g_last_error.clear();
    return weight_quant_bmm_run("npu_weight_quant_batchmatmul (no allocation)", x, x_dtype, weight, weight_dtype,
                                antiquant_scale, antiquant_offset, scale_dtype, M, N, K, group_size, bias, bias_dtype,
                                out, out_dtype, noalloc_scratch, nullptr, 0, stream);
}

int qk_weight_format_cast(const void* src, int src_format, void* dst, int dst_format, int weight_dtype, int64_t K,
                          int64_t N, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_format_cast";
    if (weight_dtype != QK_I32 && weight_dtype != QK_I8)
        return fail(QK_ERR_UNSUPPORTED, "%s: only int4-packed (int32) and int8 weights have an NZ layout", op);
    const bool to_nz = src_format == QK_FORMAT_ND && dst_format == QK_FORMAT_FRACTAL_NZ;
    const bool to_nd = src_format == QK_FORMAT_FRACTAL_NZ && dst_format == QK_FORMAT_ND;
    if (!to_nz && !to_nd)
        return fail(QK_ERR_UNSUPPORTED, "%s: cast %d -> %d is not supported (ND = %d <-> FRACTAL_NZ = %d)", op,
                    src_format, dst_format, QK_FORMAT_ND, QK_FORMAT_FRACTAL_NZ);
    const int64_t kq = weight_dtype == QK_I32 ? 128 : 64;
    if (K < 0 || N < 0 || N % 16 != 0 || K % kq != 0)
        return fail(QK_ERR_ARG, "%s: NZ needs N %% 16 == 0 and K %% %lld == 0 (K=%lld N=%lld)", op, (long long)kq,
                    (long long)K, (long long)N);
    if (K * N == 0) return QK_OK;
    if (!src || !dst) return fail(QK_ERR_ARG, "%s: null pointer", op);
    const uintptr_t bytes = (uintptr_t)(weight_dtype == QK_I32 ? K * N / 2 : K * N);
    if ((uintptr_t)src < (uintptr_t)dst + bytes && (uintptr_t)dst < (uintptr_t)src + bytes)
        return fail(QK_ERR_ARG, "%s: src and dst overlap", op);
    if (((uintptr_t)src | (uintptr_t)dst) % 16 != 0)
        return fail(QK_ERR_ARG, "%s: src and dst must be 16-byte aligned", op);
    const hipError_t e =
        weight_dtype == QK_I32
            ? qk::launch_w4_nz_cast(static_cast<const int32_t*>(src), to_nz, K, N, static_cast<int32_t*>(dst),
                                    (hipStream_t)stream)
            : qk::launch_w8_nz_cast(static_cast<const int8_t*>(src), to_nz, K, N, static_cast<int8_t*>(dst),
                                    (hipStream_t)stream);
    return launched(e, op);
}

int qk_int4_pack(const void* w, int w_dtype, int64_t K, int64_t N, int32_t* packed, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_convert_weight_to_int4pack";
    if (w_dtype != QK_I8 && w_dtype != QK_I32) return fail(QK_ERR_ARG, "%s: weight must be int8 or int32", op);
    if (K < 0 || N < 0 || N % 8 != 0) return fail(QK_ERR_ARG, "%s: need K >= 0 and N %% 8 == 0 (N=%lld)", op, (long long)N);
    if (K * N == 0) return QK_OK;
    if (!w || !packed) return fail(QK_ERR_ARG, "%s: null pointer", op);
    return launched(qk::launch_int4_pack(w, w_dtype, K, N, packed, (hipStream_t)stream), op);
}

static int quant_common(const char* op, const void* x, int x_dtype, int64_t n, const void* q, int q_dtype) {
    if (!(x_dtype == QK_F32 || is_half(x_dtype)))
        return fail(QK_ERR_ARG, "%s: input must be float32, float16 or bfloat16 (got dtype %d)", op, x_dtype);
    if (!(q_dtype == QK_I8 || q_dtype == QK_U8 || q_dtype == QK_I32))
        return fail(QK_ERR_ARG, "%s: output must be int8 (qint8), uint8 (quint8) or int32 (qint32), got dtype %d", op,
                    q_dtype);
    if (n < 0) return fail(QK_ERR_ARG, "%s: negative size", op);
    if (n > 0 && (!x || !q)) return fail(QK_ERR_ARG, "%s: null pointer", op);
    return QK_OK;
}

int qk_quantize_per_tensor(const void* x, int x_dtype, int64_t n, float scale, int64_t zero_point, void* q,
                           int q_dtype, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "quantize_per_tensor";
    if (int rc = quant_common(op, x, x_dtype, n, q, q_dtype)) return rc;
    if (!(scale > 0.0f) || scale == INFINITY) return fail(QK_ERR_ARG, "%s: scale must be positive and finite", op);
    if (n == 0) return QK_OK;
    return launched(qk::launch_quantize(x, x_dtype, 1, 1, n, nullptr, nullptr, scale, zero_point, q, q_dtype,
                                        (hipStream_t)stream), op);
}

int qk_quantize_per_channel(const void* x, int x_dtype, int64_t outer, int64_t C, int64_t inner, const float* scales,
                            const int64_t* zero_points, void* q, int q_dtype, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "quantize_per_channel";
    if (outer < 0 || C < 0 || inner < 0) return fail(QK_ERR_ARG, "%s: negative size", op);
    const int64_t n = outer * C * inner;
    if (int rc = quant_common(op, x, x_dtype, n, q, q_dtype)) return rc;
    if (n == 0) return QK_OK;
    if (!scales || !zero_points) return fail(QK_ERR_ARG, "%s: null scales or zero_points", op);
    return launched(qk::launch_quantize(x, x_dtype, outer, C, inner, scales, zero_points, 1.0f, 0, q, q_dtype,
                                        (hipStream_t)stream), op);
}

int qk_dequantize(const void* q, int q_dtype, int64_t n, float* out, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "dequantize";
    if (!(q_dtype == QK_I8 || q_dtype == QK_U8 || q_dtype == QK_I32))
        return fail(QK_ERR_ARG, "%s: input must be int8, uint8 or int32, got dtype %d", op, q_dtype);
    if (n < 0) return fail(QK_ERR_ARG, "%s: negative size", op);
    if (n == 0) return QK_OK;
    if (!q || !out) return fail(QK_ERR_ARG, "%s: null pointer", op);
    return launched(qk::launch_dequantize(q, q_dtype, n, out, (hipStream_t)stream), op);
}

static int rms_common(const char* op, const void* x, int x_dtype, const void* gamma, int64_t rows, int64_t D,
                      float eps, const void* out, bool allow_f32) {
    if (!(is_half(x_dtype) || (allow_f32 && x_dtype == QK_F32)))
        return fail(QK_ERR_ARG, "%s: x must be float16 or bfloat16%s (got dtype %d)", op, allow_f32 ? " or float32" : "",
                    x_dtype);
    if (rows < 0 || D <= 0) return fail(QK_ERR_ARG, "%s: need rows >= 0 and D > 0 (rows=%lld D=%lld)", op, (long long)rows, (long long)D);
    if (!(eps >= 0.0f)) return fail(QK_ERR_ARG, "%s: epsilon must be >= 0", op);
    if (rows > 0 && (!x || !gamma || !out)) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (rows >= kMaxGrid) return fail(QK_ERR_UNSUPPORTED, "%s: %lld rows exceed the launch limit", op, (long long)rows);
    return QK_OK;
}

int qk_rms_norm(const void* x, int x_dtype, const void* gamma, int64_t rows, int64_t D, float eps, void* y,
                float* rstd, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_rms_norm";
    if (int rc = rms_common(op, x, x_dtype, gamma, rows, D, eps, y, true)) return rc;
    if (rows == 0) return QK_OK;
    return launched(qk::launch_rms_norm(x, x_dtype, gamma, rows, D, eps, y, nullptr, nullptr, rstd, (hipStream_t)stream), op);
}

int qk_rms_norm_quant(const void* x, int x_dtype, const void* gamma, int64_t rows, int64_t D, float eps, int8_t* q,
                      float* scale, float* rstd, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_rms_norm_dynamic_quant";
    if (int rc = rms_common(op, x, x_dtype, gamma, rows, D, eps, q, false)) return rc;
    if (rows == 0) return QK_OK;
    if (!scale) return fail(QK_ERR_ARG, "%s: null pointer", op);
    return launched(qk::launch_rms_norm(x, x_dtype, gamma, rows, D, eps, nullptr, q, scale, rstd, (hipStream_t)stream), op);
}

static int swiglu_common(const char* op, const void* h, int dtype, int64_t rows, int64_t I, const void* out) {
    if (!is_half(dtype)) return fail(QK_ERR_ARG, "%s: input must be float16 or bfloat16 (got dtype %d)", op, dtype);
    if (rows < 0 || I < 0) return fail(QK_ERR_ARG, "%s: negative size rows=%lld I=%lld", op, (long long)rows, (long long)I);
    if (rows > 0 && I > 0 && (!h || !out)) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (rows >= kMaxGrid) return fail(QK_ERR_UNSUPPORTED, "%s: %lld rows exceed the launch limit", op, (long long)rows);
    return QK_OK;
}

int qk_swiglu(const void* h, int dtype, int64_t rows, int64_t I, void* y, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_swiglu";
    if (int rc = swiglu_common(op, h, dtype, rows, I, y)) return rc;
    if (rows == 0 || I == 0) return QK_OK;
    return launched(qk::launch_swiglu(h, dtype, rows, I, y, nullptr, nullptr, (hipStream_t)stream), op);
}

int qk_swiglu_quant(const void* h, int dtype, int64_t rows, int64_t I, int8_t* q, float* scale, qk_stream_t stream) {
    g_last_error.clear();
    const char* op = "npu_swiglu_dynamic_quant";
    if (int rc = swiglu_common(op, h, dtype, rows, I, q)) return rc;
    if (rows == 0) return QK_OK;
    if (!scale) return fail(QK_ERR_ARG, "%s: null pointer", op);
    if (I == 0) return fail(QK_ERR_ARG, "%s: empty rows have no scale", op);
    return launched(qk::launch_swiglu(h, dtype, rows, I, nullptr, q, scale, (hipStream_t)stream), op);
}

}  // extern "C"
