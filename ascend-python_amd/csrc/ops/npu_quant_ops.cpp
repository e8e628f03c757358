// torch.ops.npu.* registration of the quantized-inference hot path.
//
// Mirrors the reference's op_api layer: a custom schema per op
// (op_plugin/config/v2r2/op_plugin_functions.yaml:1904 "custom:" section,
// impl_ns op_api), a host function that checks shapes and dtypes with
// TORCH_CHECK, allocates every output on the input's device
// (apply_tensor_without_format, op_plugin/ops/base_ops/opapi/MmKernelNpuOpApi.cpp:27-30),
// asks for the workspace size, takes the workspace from the caching
// allocator uninitialised (op_plugin/utils/op_api_common.h:547-551), and launches through
// the C ABI on the current stream (op_plugin/utils/op_api_common.h:530).
// A non-zero ABI return becomes a TORCH_CHECK failure carrying
// qk_last_error(), as EXEC_NPU_CMD does with aclGetRecentErrMsg()
// (op_plugin/utils/op_api_common.h:546, 555).
//
// Registered for the CUDA dispatch key (HIP tensors on PyTorch-ROCm) and for
// Meta (shape inference; runs the same checks without launching).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <ATen/ExpandUtils.h>

#include <cmath>
#include <map>
#include <mutex>
#include <optional>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "../../../include/qk_abi.h"

namespace {

int qk_dtype_of(at::ScalarType t) {
    switch (t) {
    case at::kHalf: return QK_F16;
    case at::kBFloat16: return QK_BF16;
    case at::kFloat: return QK_F32;
    case at::kChar: return QK_I8;
    case at::kInt: return QK_I32;
    default: return 0;
    }
}

qk_stream_t current_stream(const at::Tensor& t) {
    return reinterpret_cast<qk_stream_t>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_rc(int rc, const char* op) {
    TORCH_CHECK(rc == QK_OK, "call ", op, " failed, detail:", qk_last_error());
}

// Phase-2 scratch for one call, taken from the caching allocator on the
// call's stream and left uninitialised, as EXEC_NPU_CMD does
// (op_plugin/utils/op_api_common.h:547-551): the kernels need no particular
// contents (split-K counters are tagged per call), and the allocator's stream
// ordering keeps a later user of the block behind this call.
at::Tensor workspace_for(const at::Tensor& like, size_t bytes) {
    return at::empty({(int64_t)bytes}, like.options().dtype(at::kByte));
}

// Rows of an [..., K] operand: the product of the leading dims (also when K == 0).
int64_t leading_rows(const at::Tensor& t) {
    int64_t m = 1;
    for (int64_t i = 0; i + 1 < t.dim(); ++i) m *= t.size(i);
    return m;
}

// ---------------------------------------------------------------- npu_dynamic_quant

std::tuple<at::Tensor, at::Tensor> dynamic_quant_shapes(const at::Tensor& x, const std::optional<at::Tensor>& smooth) {
    TORCH_CHECK(x.scalar_type() == at::kHalf || x.scalar_type() == at::kBFloat16,
                "npu_dynamic_quant: input must be float16 or bfloat16, got ", x.scalar_type());
    TORCH_CHECK(x.dim() >= 1, "npu_dynamic_quant: input must have at least one dimension");
    const int64_t K = x.size(-1);
    if (smooth.has_value()) {
        TORCH_CHECK(smooth->scalar_type() == at::kFloat, "npu_dynamic_quant: smooth_scales must be float32");
        TORCH_CHECK(smooth->dim() == 1 && smooth->size(0) == K, "npu_dynamic_quant: smooth_scales must be [", K,
                    "], got ", smooth->sizes());
    }
    auto y = at::empty(x.sizes(), x.options().dtype(at::kChar));
    auto s = at::empty(x.sizes().slice(0, x.dim() - 1), x.options().dtype(at::kFloat));
    return {y, s};
}

std::tuple<at::Tensor, at::Tensor> npu_dynamic_quant(const at::Tensor& input,
                                                     const std::optional<at::Tensor>& smooth_scales) {
    auto [y, s] = dynamic_quant_shapes(input, smooth_scales);
    const c10::DeviceGuard guard(input.device());
    auto x = input.contiguous();
    const int64_t K = x.size(-1);
    const int64_t rows = K == 0 ? 0 : x.numel() / K;
    at::Tensor sm;
    if (smooth_scales.has_value()) sm = smooth_scales->contiguous();
    const int rc = qk_dynamic_quant(x.data_ptr(), qk_dtype_of(x.scalar_type()), K == 0 ? s.numel() : rows, K,
                                    sm.defined() ? sm.data_ptr<float>() : nullptr, y.data_ptr<int8_t>(),
                                    s.data_ptr<float>(), current_stream(x));
    check_rc(rc, "npu_dynamic_quant");
    return {y, s};
}

std::tuple<at::Tensor, at::Tensor> npu_dynamic_quant_meta(const at::Tensor& input,
                                                          const std::optional<at::Tensor>& smooth_scales) {
    return dynamic_quant_shapes(input, smooth_scales);
}

// ---------------------------------------------------------------- storage format

// The reference keeps a tensor's storage format (ND, FRACTAL_NZ, ...) in the
// NPU descriptor of its storage and reads it from there
// (npu_preparation::get_tensor_npu_format, op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:81;
// get_npu_desc, op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:57-66).  A
// PyTorch-ROCm storage has no such descriptor, so the format is kept here,
// keyed by the storage: npu_format_cast and npu_convert_weight_to_int4pack
// (inner_k_tiles=4) record the storage of every FRACTAL_NZ weight they return,
// with its sizes and dtype.  A tensor is FRACTAL_NZ when its storage is
// recorded and still alive and the tensor views all of it as recorded (offset
// 0, the recorded sizes and dtype, contiguous); every other tensor is ND,
// whatever its shape.  A weak reference per record tells the recorded storage
// from a new one allocated at the same address.  (As with a device-local
// descriptor, copies -- clone, .to(), a load from disk -- are ND until cast.)
struct NzRecord {
    c10::weak_intrusive_ptr<c10::StorageImpl> storage;
    std::vector<int64_t> sizes;
    at::ScalarType dtype;
};
std::mutex g_nz_mu;
std::unordered_map<const c10::StorageImpl*, NzRecord> g_nz;

void record_nz(const at::Tensor& t) {
    std::lock_guard<std::mutex> lock(g_nz_mu);
    for (auto it = g_nz.begin(); it != g_nz.end();) it = it->second.storage.expired() ? g_nz.erase(it) : std::next(it);
    g_nz.insert_or_assign(t.storage().unsafeGetStorageImpl(),
                          NzRecord{t.storage().getWeakStorageImpl(), t.sizes().vec(), t.scalar_type()});
}

bool recorded_nz(const at::Tensor& t) {
    if (!t.has_storage() || t.storage_offset() != 0 || !t.is_contiguous()) return false;
    const c10::StorageImpl* key = t.storage().unsafeGetStorageImpl();
    std::lock_guard<std::mutex> lock(g_nz_mu);
    auto it = g_nz.find(key);
    if (it == g_nz.end()) return false;
    const auto live = it->second.storage.lock();
    if (!live || live.get() != key) {  // a new storage at the address of a freed one
        g_nz.erase(it);
        return false;
    }
    return t.sizes().equals(it->second.sizes) && t.scalar_type() == it->second.dtype;
}

// An int4 weight in the NZ layout written by npu_format_cast(w, 29): int32 [N/16, K/128, 64, 4].
bool is_w4_nz(const at::Tensor& w) {
    return w.scalar_type() == at::kInt && w.dim() == 4 && w.size(2) == 64 && w.size(3) == 4 && recorded_nz(w);
}

// An int8 weight in the NZ layout: int8 [N/16, K/64, 64, 16].
bool is_w8_nz(const at::Tensor& w) {
    return w.scalar_type() == at::kChar && w.dim() == 4 && w.size(2) == 64 && w.size(3) == 16 && recorded_nz(w);
}

bool is_nz(const at::Tensor& w) { return is_w4_nz(w) || is_w8_nz(w); }

// torch_npu.get_npu_format for the formats of this path: FRACTAL_NZ (29) or ND (2).
int64_t get_npu_format(const at::Tensor& self) { return is_nz(self) ? QK_FORMAT_FRACTAL_NZ : QK_FORMAT_ND; }

// ---------------------------------------------------------------- batched weights

// A weight with batch dims (>= 3-D): the output batch is the broadcast of x's
// batch dims (those before [M, K]; a 2-D x has none) and the weight's (those
// before [K, N]), as the reference's matmul output rule
// (op_plugin/ops/base_ops/opapi/MatmulKernelNpuOpApi.cpp:45-73) and bmm
// (op_plugin/ops/base_ops/opapi/BmmKernelNpuOpApi.cpp:24-52).  Each element of
// the broadcast batch is one [M, K] x [K, N] call; `xb` / `wb` give the batch
// element of x / of the weight it reads (0 along a broadcast dim).
struct Batch {
    std::vector<int64_t> shape;  // broadcast batch dims
    std::vector<int64_t> xb, wb; // per element: linear batch index into x and into the weight
};

Batch batch_of(at::IntArrayRef x_batch, at::IntArrayRef w_batch, const char* op) {
    Batch b;
    try {
        b.shape = at::infer_size(x_batch, w_batch);
    } catch (const c10::Error&) {
        TORCH_CHECK(false, op, ": batch dims of x ", x_batch, " and of the weight ", w_batch, " do not broadcast");
    }
    int64_t n = 1;
    for (int64_t d : b.shape) n *= d;
    b.xb.resize(n);
    b.wb.resize(n);
    const int64_t nd = (int64_t)b.shape.size();
    for (int64_t e = 0; e < n; ++e) {
        int64_t rem = e, xi = 0, wi = 0, xs = 1, ws = 1;
        for (int64_t d = nd - 1; d >= 0; --d) {
            const int64_t idx = rem % b.shape[d];
            rem /= b.shape[d];
            const int64_t dx = d - (nd - (int64_t)x_batch.size()), dw = d - (nd - (int64_t)w_batch.size());
            if (dx >= 0) {
                xi += (x_batch[dx] == 1 ? 0 : idx) * xs;
                xs *= x_batch[dx];
            }
            if (dw >= 0) {
                wi += (w_batch[dw] == 1 ? 0 : idx) * ws;
                ws *= w_batch[dw];
            }
        }
        b.xb[e] = xi;
        b.wb[e] = wi;
    }
    return b;
}

// ---------------------------------------------------------------- npu_quant_matmul

struct QmmPlan {
    int64_t M, N, K;
    bool nz;  // x2 is an int8 NZ weight
    at::ScalarType out_type;
    std::vector<int64_t> out_shape;
    bool batched;  // x2 has batch dims: M is x1's second-to-last dim, one call per element of `batch`
    Batch batch;
};

// Element offset of batch element `lin` (row-major over the first nb dims) of t, by t's strides.
int64_t batch_offset(const at::Tensor& t, int64_t nb, int64_t lin) {
    int64_t off = 0;
    for (int64_t d = nb - 1; d >= 0; --d) {
        off += (lin % t.size(d)) * t.stride(d);
        lin /= t.size(d);
    }
    return off;
}

QmmPlan quant_matmul_plan(const at::Tensor& x1, const at::Tensor& x2, const at::Tensor& scale,
                          const std::optional<at::Tensor>& offset, const std::optional<at::Tensor>& pertoken_scale,
                          const std::optional<at::Tensor>& bias, std::optional<at::ScalarType> output_dtype) {
    const char* op = "npu_quant_matmul";
    TORCH_CHECK(x1.scalar_type() == at::kChar && x2.scalar_type() == at::kChar, op,
                ": x1 and x2 must be int8, got ", x1.scalar_type(), " and ", x2.scalar_type());
    TORCH_CHECK(x1.dim() >= 2 && x1.dim() <= 6, op, ": x1 must have 2 to 6 dimensions, got ", x1.dim());
    // x2 is [K, N] (or the transposed view of [N, K]), the int8 NZ weight npu_format_cast(x2, 29) writes, or
    // a batch of [K, N] weights [..., K, N] (2 to 6 dims in all)
    const bool nz = is_w8_nz(x2);
    TORCH_CHECK((x2.dim() >= 2 && x2.dim() <= 6) || nz, op,
                ": x2 must be [K, N], a batch [..., K, N] or an int8 NZ weight [N/16, K/64, 64, 16], got ", x2.sizes());
    const bool batched = !nz && x2.dim() >= 3;
    const int64_t K = x1.size(-1);
    const int64_t x2_k = nz ? x2.size(1) * 64 : x2.size(-2);
    TORCH_CHECK(x2_k == K, op, ": x1 last dim (", K, ") must equal the weight's K (", x2_k, ")");
    const int64_t N = nz ? x2.size(0) * 16 : x2.size(-1);
    const int64_t M = batched ? x1.size(-2) : leading_rows(x1);
    const at::ScalarType out_type = output_dtype.value_or(at::kChar);
    TORCH_CHECK(out_type == at::kBFloat16 || out_type == at::kHalf || out_type == at::kChar ||
                    out_type == at::kInt || out_type == at::kFloat,
                op, ": output_dtype must be bfloat16, float16, float32, int8 or int32, got ", out_type);
    TORCH_CHECK(scale.scalar_type() == at::kFloat || scale.scalar_type() == at::kBFloat16, op,
                ": scale must be float32 or bfloat16, got ", scale.scalar_type());
    TORCH_CHECK(scale.dim() == 1 && (scale.size(0) == 1 || scale.size(0) == N), op, ": scale must be [1] or [", N,
                "], got ", scale.sizes());
    if (offset.has_value()) {
        TORCH_CHECK(out_type == at::kChar, op, ": offset is only supported with an int8 output");
        TORCH_CHECK(offset->scalar_type() == at::kFloat, op, ": offset must be float32");
        TORCH_CHECK(offset->dim() == 1 && (offset->size(0) == 1 || offset->size(0) == N), op,
                    ": offset must be [1] or [", N, "]");
    }
    if (pertoken_scale.has_value()) {
        TORCH_CHECK(out_type == at::kBFloat16 || out_type == at::kHalf || out_type == at::kFloat, op,
                    ": pertoken_scale needs output_dtype bfloat16, float16 or float32");
        TORCH_CHECK(pertoken_scale->scalar_type() == at::kFloat, op, ": pertoken_scale must be float32");
        TORCH_CHECK(pertoken_scale->numel() == leading_rows(x1), op, ": pertoken_scale must have one element per row"
                    " of x1 (", leading_rows(x1), "), got ", pertoken_scale->numel());
    }
    if (bias.has_value()) {
        const auto bt = bias->scalar_type();
        TORCH_CHECK(bt == at::kInt || bt == at::kBFloat16 || bt == at::kHalf || bt == at::kFloat, op,
                    ": bias must be int32, bfloat16, float16 or float32, got ", bt);
        TORCH_CHECK(bias->numel() == N && (bias->dim() == 1 || (bias->dim() == 2 && bias->size(0) == 1)), op,
                    ": bias must be [", N, "], got ", bias->sizes());
        TORCH_CHECK(bt == at::kInt || !(out_type == at::kChar || out_type == at::kInt), op,
                    ": int8/int32 outputs take an int32 bias");
    }
    std::vector<int64_t> shape(x1.sizes().begin(), x1.sizes().end());
    shape.back() = N;
    Batch b;
    if (batched) {
        b = batch_of(x1.sizes().slice(0, x1.dim() - 2), x2.sizes().slice(0, x2.dim() - 2), op);
        shape = b.shape;
        shape.push_back(M);
        shape.push_back(N);
    }
    return {M, N, K, nz, out_type, shape, batched, b};
}

// The NZ weight (the layout the reference's matmuls read after npu_format_cast, op_plugin/ops/base_ops/aclops/
// MmKernelNpu.cpp:303-316): x1 rows and the output 16-byte aligned (a misaligned x1 view is copied).
at::Tensor quant_matmul_nz(const QmmPlan& pl, at::Tensor x1, const at::Tensor& x2_in, const at::Tensor& scale_in,
                           const std::optional<at::Tensor>& offset, const std::optional<at::Tensor>& pertoken_scale,
                           const std::optional<at::Tensor>& bias, at::Tensor out) {
    if (reinterpret_cast<uintptr_t>(x1.data_ptr()) % 16 != 0) x1 = x1.clone();
    auto x2 = x2_in.contiguous();
    if (reinterpret_cast<uintptr_t>(x2.data_ptr()) % 16 != 0) x2 = x2.clone();
    auto scale = scale_in.scalar_type() == at::kFloat ? scale_in.contiguous() : scale_in.to(at::kFloat);
    at::Tensor off, pt, b;
    if (offset.has_value()) off = offset->contiguous();
    if (pertoken_scale.has_value()) pt = pertoken_scale->contiguous();
    if (bias.has_value()) b = bias->contiguous();
    size_t ws_bytes = 0;
    check_rc(qk_quant_matmul_nz_workspace_size(pl.M, pl.N, pl.K, qk_dtype_of(pl.out_type), &ws_bytes),
             "npu_quant_matmul");
    at::Tensor ws = ws_bytes ? workspace_for(x1, ws_bytes) : at::Tensor();
    const int rc = qk_quant_matmul_nz(
        x1.data_ptr<int8_t>(), pl.K, x2.data_ptr<int8_t>(), pl.M, pl.N, pl.K, scale.data_ptr<float>(), scale.numel(),
        off.defined() ? off.data_ptr<float>() : nullptr, off.defined() ? off.numel() : 0,
        pt.defined() ? pt.data_ptr<float>() : nullptr, b.defined() ? b.data_ptr() : nullptr,
        b.defined() ? qk_dtype_of(b.scalar_type()) : 0, out.data_ptr(), qk_dtype_of(pl.out_type),
        ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(x1));
    check_rc(rc, "npu_quant_matmul");
    return out;
}

at::Tensor npu_quant_matmul(const at::Tensor& x1_in, const at::Tensor& x2_in, const at::Tensor& scale_in,
                            const std::optional<at::Tensor>& offset, const std::optional<at::Tensor>& pertoken_scale,
                            const std::optional<at::Tensor>& bias, std::optional<at::ScalarType> output_dtype) {
    QmmPlan pl = quant_matmul_plan(x1_in, x2_in, scale_in, offset, pertoken_scale, bias, output_dtype);
    const c10::DeviceGuard guard(x1_in.device());
    auto out = at::empty(pl.out_shape, x1_in.options().dtype(pl.out_type));
    if (out.numel() == 0) return out;
    auto x1 = x1_in.contiguous();
    if (pl.nz) return quant_matmul_nz(pl, x1, x2_in, scale_in, offset, pertoken_scale, bias, out);
    // Transposed view of an [N,K] weight is read in place, as the reference
    // flags mat2 instead of copying it (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:40-53).
    // For a batch of weights the same holds for the last two dims of every slice.
    at::Tensor x2 = x2_in;
    const int64_t d = x2.dim();
    const bool kn = x2.stride(d - 1) == 1 && x2.stride(d - 2) >= std::max<int64_t>(1, pl.N);
    const bool nk = x2.stride(d - 2) == 1 && x2.stride(d - 1) >= std::max<int64_t>(1, pl.K);
    if (!kn && !nk) x2 = x2.contiguous();
    const int64_t sbk = kn || (!nk) ? x2.stride(d - 2) : 1;
    const int64_t sbn = kn || (!nk) ? 1 : x2.stride(d - 1);
    auto scale = scale_in.scalar_type() == at::kFloat ? scale_in.contiguous() : scale_in.to(at::kFloat);
    at::Tensor off, pt, b;
    if (offset.has_value()) off = offset->contiguous();
    if (pertoken_scale.has_value()) pt = pertoken_scale->contiguous();
    if (bias.has_value()) b = bias->contiguous();
    size_t ws_bytes = 0;
    check_rc(qk_quant_matmul_workspace_size(pl.M, pl.N, pl.K, qk_dtype_of(pl.out_type), &ws_bytes),
             "npu_quant_matmul");
    at::Tensor ws = ws_bytes ? workspace_for(x1, ws_bytes) : at::Tensor();
    // one call per batch element (a single call with no batch); the calls share the workspace, in stream order
    const int64_t nb = pl.batched ? (int64_t)pl.batch.xb.size() : 1;
    const size_t osz = out.element_size();
    for (int64_t e = 0; e < nb; ++e) {
        const int64_t xb = pl.batched ? pl.batch.xb[e] : 0;
        const int64_t woff = pl.batched ? batch_offset(x2, d - 2, pl.batch.wb[e]) : 0;
        const int rc = qk_quant_matmul(
            x1.data_ptr<int8_t>() + xb * pl.M * pl.K, pl.K, x2.data_ptr<int8_t>() + woff, sbk, sbn, pl.M, pl.N, pl.K,
            scale.data_ptr<float>(), scale.numel(), off.defined() ? off.data_ptr<float>() : nullptr,
            off.defined() ? off.numel() : 0, pt.defined() ? pt.data_ptr<float>() + xb * pl.M : nullptr,
            b.defined() ? b.data_ptr() : nullptr, b.defined() ? qk_dtype_of(b.scalar_type()) : 0,
            static_cast<char*>(out.data_ptr()) + (size_t)(e * pl.M * pl.N) * osz, qk_dtype_of(pl.out_type),
            ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(x1));
        check_rc(rc, "npu_quant_matmul");
    }
    return out;
}

at::Tensor npu_quant_matmul_meta(const at::Tensor& x1, const at::Tensor& x2, const at::Tensor& scale,
                                 const std::optional<at::Tensor>& offset,
                                 const std::optional<at::Tensor>& pertoken_scale, const std::optional<at::Tensor>& bias,
                                 std::optional<at::ScalarType> output_dtype) {
    QmmPlan pl = quant_matmul_plan(x1, x2, scale, offset, pertoken_scale, bias, output_dtype);
    return at::empty(pl.out_shape, x1.options().dtype(pl.out_type));
}

// ---------------------------------------------------------------- npu_weight_quant_batchmatmul

struct WqPlan {
    int64_t M, N, K, group;
    bool int4, nz;
    std::vector<int64_t> out_shape;
    bool batched;      // the weight has batch dims: one call per element of `batch`
    Batch batch;
    bool scale_batched;  // antiquant_scale / antiquant_offset carry the weight's batch dims
};

WqPlan weight_quant_plan(const at::Tensor& x, const at::Tensor& weight, const at::Tensor& antiquant_scale,
                         const std::optional<at::Tensor>& antiquant_offset,
                         const std::optional<at::Tensor>& quant_scale, const std::optional<at::Tensor>& quant_offset,
                         const std::optional<at::Tensor>& bias, int64_t group) {
    const char* op = "npu_weight_quant_batchmatmul";
    TORCH_CHECK(x.scalar_type() == at::kHalf || x.scalar_type() == at::kBFloat16, op,
                ": x must be float16 or bfloat16, got ", x.scalar_type());
    TORCH_CHECK(x.dim() >= 2, op, ": x must be at least 2-D, got ", x.dim());
    const bool nz = is_nz(weight);
    TORCH_CHECK((weight.dim() >= 2 && weight.dim() <= 6) || nz, op,
                ": weight must be [K, N] (ND), a batch [..., K, N] or an NZ weight (int4 [N/16, K/128, 64, 4], int8 "
                "[N/16, K/64, 64, 16]), got ", weight.sizes());
    TORCH_CHECK(weight.scalar_type() == at::kInt || weight.scalar_type() == at::kChar, op,
                ": weight must be int32 (int4 packed 8 per element) or int8, got ", weight.scalar_type());
    TORCH_CHECK(!quant_scale.has_value() && !quant_offset.has_value(), op,
                ": quant_scale/quant_offset (int8 output) are not supported by this build");
    const bool int4 = weight.scalar_type() == at::kInt;
    const bool batched = !nz && weight.dim() >= 3;
    const int64_t K = x.size(-1);
    const int64_t wk = nz ? weight.size(1) * (int4 ? 128 : 64) : weight.size(-2);
    TORCH_CHECK(wk == K, op, ": x last dim (", K, ") must equal the weight's K (", wk, ")");
    const int64_t N = nz ? weight.size(0) * 16 : (int4 ? weight.size(-1) * 8 : weight.size(-1));
    TORCH_CHECK(group >= 0, op, ": antiquant_group_size must be >= 0");
    TORCH_CHECK(group == 0 || K % group == 0, op, ": K=", K, " must be a multiple of antiquant_group_size=", group);
    const auto st = antiquant_scale.scalar_type();
    TORCH_CHECK(st == at::kHalf || st == at::kBFloat16, op, ": antiquant_scale must be float16 or bfloat16");
    const int64_t ng = group > 0 ? K / group : 1;
    // with a batch of weights the scales may carry the weight's batch dims in front ([..., K/group, N] or [..., N])
    const at::IntArrayRef wbatch = batched ? weight.sizes().slice(0, weight.dim() - 2) : at::IntArrayRef();
    const int64_t snb = (int64_t)wbatch.size();
    const bool scale_batched = batched && antiquant_scale.dim() > (group > 0 ? 2 : 1) &&
                               antiquant_scale.dim() >= snb && antiquant_scale.sizes().slice(0, snb).equals(wbatch);
    const at::IntArrayRef ss = scale_batched ? antiquant_scale.sizes().slice(snb) : antiquant_scale.sizes();
    int64_t ss_numel = 1;
    for (int64_t v : ss) ss_numel *= v;
    const bool per_ch_ok = group == 0 && ss_numel == N && (ss.size() == 1 || (ss.size() == 2 && ss[0] == 1));
    const bool grouped_ok = group > 0 && ss.size() == 2 && ss[0] == ng && ss[1] == N;
    TORCH_CHECK(per_ch_ok || grouped_ok, op, ": antiquant_scale must be ", group > 0 ? "[K/group, N] = [" : "[N] = [",
                group > 0 ? ng : N, group > 0 ? ", " : "", group > 0 ? std::to_string(N) : std::string(""),
                "]", batched ? " (optionally after the weight's batch dims)" : "", ", got ", antiquant_scale.sizes());
    if (antiquant_offset.has_value()) {
        TORCH_CHECK(antiquant_offset->scalar_type() == st, op, ": antiquant_offset must match antiquant_scale's dtype");
        TORCH_CHECK(antiquant_offset->sizes() == antiquant_scale.sizes(), op,
                    ": antiquant_offset must have antiquant_scale's shape");
    }
    if (bias.has_value()) {
        const auto bt = bias->scalar_type();
        TORCH_CHECK(bt == at::kHalf || bt == at::kBFloat16 || bt == at::kFloat, op, ": bias must be a float type");
        TORCH_CHECK(bias->numel() == N, op, ": bias must have N=", N, " elements");
    }
    std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end());
    shape.back() = N;
    const int64_t M = batched ? x.size(-2) : leading_rows(x);
    Batch b;
    if (batched) {
        b = batch_of(x.sizes().slice(0, x.dim() - 2), wbatch, op);
        shape = b.shape;
        shape.push_back(M);
        shape.push_back(N);
    }
    return {M, N, K, group, int4, nz, shape, batched, b, scale_batched};
}

// An int8 ND weight passed as the transposed view of an [N, K] tensor (the nn.Linear layout): read in place
// as QK_I8_NK, as the reference flags a transposed mat2 instead of copying it
// (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:40-53, op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:39-40).
bool int8_nk_view(const at::Tensor& w, int64_t K, int64_t N) {
    const int64_t d = w.dim();
    return w.scalar_type() == at::kChar && K > 1 && N > 1 && w.stride(d - 2) == 1 && w.stride(d - 1) == K;
}

at::Tensor npu_weight_quant_batchmatmul(const at::Tensor& x_in, const at::Tensor& weight_in,
                                        const at::Tensor& antiquant_scale,
                                        const std::optional<at::Tensor>& antiquant_offset,
                                        const std::optional<at::Tensor>& quant_scale,
                                        const std::optional<at::Tensor>& quant_offset,
                                        const std::optional<at::Tensor>& bias, int64_t antiquant_group_size) {
    WqPlan pl = weight_quant_plan(x_in, weight_in, antiquant_scale, antiquant_offset, quant_scale, quant_offset, bias,
                                  antiquant_group_size);
    const c10::DeviceGuard guard(x_in.device());
    auto out = at::empty(pl.out_shape, x_in.options());
    if (out.numel() == 0) return out;
    auto x = x_in.contiguous();
    // the weight is read where it lies: NZ blocks, [K, N] rows, or an int8 [N, K] tensor seen transposed; any
    // other strides are made contiguous (per slice of a batch, the last two dims decide)
    const bool nk = !pl.nz && int8_nk_view(weight_in, pl.K, pl.N);
    const int64_t d = weight_in.dim();
    const bool rows = !pl.nz && weight_in.stride(d - 1) == 1 && weight_in.stride(d - 2) == weight_in.size(d - 1);
    auto w = (pl.nz || nk || rows) ? weight_in : weight_in.contiguous();
    auto sc = antiquant_scale.contiguous();
    at::Tensor off, b;
    if (antiquant_offset.has_value()) off = antiquant_offset->contiguous();
    if (bias.has_value()) b = bias->contiguous();
    const int wdt = pl.nz ? (pl.int4 ? QK_I4_NZ : QK_I8_NZ) : (pl.int4 ? QK_I32 : (nk ? QK_I8_NK : QK_I8));
    size_t ws_bytes = 0;
    check_rc(qk_weight_quant_bmm_workspace_size(pl.M, pl.N, pl.K, wdt, pl.group, &ws_bytes),
             "npu_weight_quant_batchmatmul");
    at::Tensor ws = ws_bytes ? workspace_for(x, ws_bytes) : at::Tensor();
    // one call per batch element (a single call with no batch); the calls share the workspace, in stream order
    const int64_t nb = pl.batched ? (int64_t)pl.batch.xb.size() : 1;
    const size_t xsz = x.element_size(), wsz = w.element_size(), ssz = sc.element_size(), osz = out.element_size();
    const int64_t s_slice = pl.group > 0 ? (pl.K / pl.group) * pl.N : pl.N;  // scale elements per weight
    for (int64_t e = 0; e < nb; ++e) {
        const int64_t xb = pl.batched ? pl.batch.xb[e] : 0, wb = pl.batched ? pl.batch.wb[e] : 0;
        const int64_t woff = pl.batched ? batch_offset(w, d - 2, wb) : 0;
        const int64_t soff = pl.scale_batched ? wb * s_slice : 0;
        const int rc = qk_weight_quant_bmm(
            static_cast<const char*>(x.data_ptr()) + (size_t)(xb * pl.M * pl.K) * xsz, qk_dtype_of(x.scalar_type()),
            static_cast<const char*>(w.data_ptr()) + (size_t)woff * wsz, wdt,
            static_cast<const char*>(sc.data_ptr()) + (size_t)soff * ssz,
            off.defined() ? static_cast<const char*>(off.data_ptr()) + (size_t)soff * ssz : nullptr,
            qk_dtype_of(sc.scalar_type()), pl.M, pl.N, pl.K, pl.group, b.defined() ? b.data_ptr() : nullptr,
            b.defined() ? qk_dtype_of(b.scalar_type()) : 0,
            static_cast<char*>(out.data_ptr()) + (size_t)(e * pl.M * pl.N) * osz, qk_dtype_of(out.scalar_type()),
            ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(x));
        check_rc(rc, "npu_weight_quant_batchmatmul");
    }
    return out;
}

at::Tensor npu_weight_quant_batchmatmul_meta(const at::Tensor& x, const at::Tensor& weight,
                                             const at::Tensor& antiquant_scale,
                                             const std::optional<at::Tensor>& antiquant_offset,
                                             const std::optional<at::Tensor>& quant_scale,
                                             const std::optional<at::Tensor>& quant_offset,
                                             const std::optional<at::Tensor>& bias, int64_t antiquant_group_size) {
    WqPlan pl = weight_quant_plan(x, weight, antiquant_scale, antiquant_offset, quant_scale, quant_offset, bias,
                                  antiquant_group_size);
    return at::empty(pl.out_shape, x.options());
}

// ---------------------------------------------------------------- npu_convert_weight_to_int4pack

std::vector<int64_t> int4pack_shape(const at::Tensor& w) {
    const char* op = "npu_convert_weight_to_int4pack";
    TORCH_CHECK(w.scalar_type() == at::kInt || w.scalar_type() == at::kChar, op, ": weight must be int32 or int8");
    TORCH_CHECK(w.dim() == 2, op, ": weight must be 2-D [K, N]");
    TORCH_CHECK(w.size(1) % 8 == 0, op, ": N=", w.size(1), " must be a multiple of 8");
    return {w.size(0), w.size(1) / 8};
}

// inner_k_tiles: 0 packs along N in the ND layout [K, N/8]; 4 writes the NZ
// layout [N/16, K/128, 64, 4] directly, whose lanes each hold 4 MFMA K-tiles
// of 32 (what npu_format_cast(npu_convert_weight_to_int4pack(w), 29) gives).
void int4pack_check_tiles(const at::Tensor& w, int64_t inner_k_tiles) {
    const char* op = "npu_convert_weight_to_int4pack";
    TORCH_CHECK(inner_k_tiles == 0 || inner_k_tiles == 4, op,
                ": inner_k_tiles must be 0 (ND) or 4 (the NZ layout's four 32-row K tiles per lane), got ",
                inner_k_tiles);
    if (inner_k_tiles == 4)
        TORCH_CHECK(w.size(0) % 128 == 0 && w.size(1) % 16 == 0, op,
                    ": the NZ layout needs K % 128 == 0 and N % 16 == 0, got ", w.sizes());
}

std::vector<int64_t> nz_shape(int64_t K, int64_t N) { return {N / 16, K / 128, 64, 4}; }

at::Tensor npu_convert_weight_to_int4pack(const at::Tensor& weight, int64_t inner_k_tiles) {
    auto shape = int4pack_shape(weight);
    int4pack_check_tiles(weight, inner_k_tiles);
    const c10::DeviceGuard guard(weight.device());
    auto w = weight.contiguous();
    auto out = at::empty(shape, w.options().dtype(at::kInt));
    check_rc(qk_int4_pack(w.data_ptr(), qk_dtype_of(w.scalar_type()), w.size(0), w.size(1), out.data_ptr<int32_t>(),
                          current_stream(w)),
             "npu_convert_weight_to_int4pack");
    if (inner_k_tiles == 0) return out;
    auto nz = at::empty(nz_shape(w.size(0), w.size(1)), w.options().dtype(at::kInt));
    check_rc(qk_weight_format_cast(out.data_ptr(), QK_FORMAT_ND, nz.data_ptr(), QK_FORMAT_FRACTAL_NZ, QK_I32,
                                   w.size(0), w.size(1), current_stream(w)),
             "npu_convert_weight_to_int4pack");
    record_nz(nz);
    return nz;
}

at::Tensor npu_convert_weight_to_int4pack_meta(const at::Tensor& weight, int64_t inner_k_tiles) {
    auto shape = int4pack_shape(weight);
    int4pack_check_tiles(weight, inner_k_tiles);
    if (inner_k_tiles == 0) return at::empty(shape, weight.options().dtype(at::kInt));
    auto nz = at::empty(nz_shape(weight.size(0), weight.size(1)), weight.options().dtype(at::kInt));
    record_nz(nz);
    return nz;
}

// ---------------------------------------------------------------- npu_format_cast

// npu_format_cast(self, acl_format) for matmul weights: ND (2) <-> FRACTAL_NZ (29)
// of an int4-packed int32 weight or an int8 weight, the casts the reference
// applies to matmul operands (op_plugin/ops/base_ops/aclops/MmKernelNpu.cpp:303-316,
// op_plugin/ops/base_ops/aclops/LinearKernelNpu.cpp:103-107).  A tensor
// already in the requested format is returned as is.
struct CastPlan {
    bool identity, to_nz, int4;
    int64_t K, N;
    std::vector<int64_t> shape;
};

CastPlan format_cast_plan(const at::Tensor& self, int64_t acl_format) {
    const char* op = "npu_format_cast";
    TORCH_CHECK(acl_format == QK_FORMAT_ND || acl_format == QK_FORMAT_FRACTAL_NZ, op,
                ": only ND (2) and FRACTAL_NZ (29) are supported, got ", acl_format);
    const bool int4 = self.scalar_type() == at::kInt;
    TORCH_CHECK(int4 || self.scalar_type() == at::kChar, op,
                ": only int4-packed int32 ([K, N/8]) and int8 ([K, N]) weights have an NZ layout, got ",
                self.scalar_type());
    const bool nz = is_nz(self);
    TORCH_CHECK(nz || self.dim() == 2, op, ": expected an ND weight (2-D) or an NZ weight (4-D), got ", self.sizes());
    CastPlan c{nz == (acl_format == QK_FORMAT_FRACTAL_NZ), !nz && acl_format == QK_FORMAT_FRACTAL_NZ, int4, 0, 0,
               self.sizes().vec()};
    const int64_t kq = int4 ? 128 : 64;
    if (nz) {
        c.N = self.size(0) * 16;
        c.K = self.size(1) * kq;
    } else {
        c.K = self.size(0);
        c.N = int4 ? self.size(1) * 8 : self.size(1);
    }
    if (c.identity) return c;
    if (c.to_nz) {
        TORCH_CHECK(c.K % kq == 0 && c.N % 16 == 0, op, ": FRACTAL_NZ needs K % ", kq, " == 0 and N % 16 == 0, got ",
                    int4 ? "[K, N/8] = " : "[K, N] = ", self.sizes());
        c.shape = int4 ? nz_shape(c.K, c.N) : std::vector<int64_t>{c.N / 16, c.K / 64, 64, 16};
    } else {
        c.shape = int4 ? std::vector<int64_t>{c.K, c.N / 8} : std::vector<int64_t>{c.K, c.N};
    }
    return c;
}

at::Tensor npu_format_cast(const at::Tensor& self, int64_t acl_format) {
    const CastPlan c = format_cast_plan(self, acl_format);
    if (c.identity) return self;
    const c10::DeviceGuard guard(self.device());
    auto src = self.contiguous();
    auto out = at::empty(c.shape, src.options());
    check_rc(qk_weight_format_cast(src.data_ptr(), c.to_nz ? QK_FORMAT_ND : QK_FORMAT_FRACTAL_NZ, out.data_ptr(),
                                   c.to_nz ? QK_FORMAT_FRACTAL_NZ : QK_FORMAT_ND, c.int4 ? QK_I32 : QK_I8, c.K, c.N,
                                   current_stream(src)),
             "npu_format_cast");
    if (c.to_nz) record_nz(out);
    return out;
}

at::Tensor npu_format_cast_meta(const at::Tensor& self, int64_t acl_format) {
    const CastPlan c = format_cast_plan(self, acl_format);
    if (c.identity) return self;
    auto out = at::empty(c.shape, self.options());
    if (c.to_nz) record_nz(out);
    return out;
}

// ---------------------------------------------------------------- quantize_per_tensor / _per_channel / dequantize

// The reference's NPU quantize ops return plain integer tensors, QInt8 -> kChar, QUInt8 -> kByte,
// QInt32 -> kInt (op_plugin/ops/base_ops/aclops/QuantizePerTensorKernelNpu.cpp:60-67,
// op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:81-88), not torch quantized tensors.
std::pair<at::ScalarType, int> quant_out_type(const char* op, at::ScalarType dtype) {
    switch (dtype) {
    case at::kQInt8: return {at::kChar, QK_I8};
    case at::kQUInt8: return {at::kByte, QK_U8};
    case at::kQInt32: return {at::kInt, QK_I32};
    default: TORCH_CHECK(false, op, ": dtype must be torch.qint8, torch.quint8 or torch.qint32, got ", dtype);
    }
}

void quant_input_check(const char* op, const at::Tensor& self) {
    const auto t = self.scalar_type();
    TORCH_CHECK(t == at::kFloat || t == at::kHalf || t == at::kBFloat16, op,
                ": self must be float32, float16 or bfloat16, got ", t);
}

at::Tensor quantize_per_tensor_meta(const at::Tensor& self, double scale, int64_t zero_point, at::ScalarType dtype) {
    const char* op = "quantize_per_tensor";
    quant_input_check(op, self);
    TORCH_CHECK(scale > 0.0 && std::isfinite((float)scale), op, ": scale must be positive and finite, got ", scale);
    (void)zero_point;
    return at::empty(self.sizes(), self.options().dtype(quant_out_type(op, dtype).first));
}

at::Tensor quantize_per_tensor(const at::Tensor& self, double scale, int64_t zero_point, at::ScalarType dtype) {
    const char* op = "quantize_per_tensor";
    auto out = quantize_per_tensor_meta(self, scale, zero_point, dtype);
    const c10::DeviceGuard guard(self.device());
    auto x = self.contiguous();
    out = at::empty(self.sizes(), self.options().dtype(out.scalar_type()));
    check_rc(qk_quantize_per_tensor(x.data_ptr(), qk_dtype_of(x.scalar_type()), x.numel(), (float)scale, zero_point,
                                    out.data_ptr(), quant_out_type(op, dtype).second, current_stream(x)),
             op);
    return out;
}

// axis wrapped as the reference does (make_warp_dim); the checks of
// op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:75-80
int64_t quantize_per_channel_check(const at::Tensor& self, const at::Tensor& scales, const at::Tensor& zero_points,
                                   int64_t axis) {
    const char* op = "quantize_per_channel";
    quant_input_check(op, self);
    TORCH_CHECK(self.dim() >= 1, op, ": self must have at least one dimension");
    if (axis < 0) axis += self.dim();
    TORCH_CHECK(axis >= 0 && axis < self.dim(), op, ": axis out of range for a ", self.dim(), "-d input");
    TORCH_CHECK(scales.dim() == 1, op, ": scales must be 1-D");
    TORCH_CHECK(zero_points.dim() == 1, op, ": zero_points must be 1-D");
    TORCH_CHECK(scales.size(0) == zero_points.size(0), op, ": scales and zero_points must have the same length");
    TORCH_CHECK(scales.size(0) == self.size(axis), op, ": scales must have as many elements as dimension ", axis,
                " of self (", self.size(axis), "), got ", scales.size(0));
    TORCH_CHECK(scales.is_floating_point(), op, ": scales must be a floating-point tensor");
    TORCH_CHECK(!zero_points.is_floating_point() && !zero_points.is_complex(), op,
                ": zero_points must be an integer tensor");
    return axis;
}

at::Tensor quantize_per_channel_meta(const at::Tensor& self, const at::Tensor& scales, const at::Tensor& zero_points,
                                     int64_t axis, at::ScalarType dtype) {
    quantize_per_channel_check(self, scales, zero_points, axis);
    return at::empty(self.sizes(), self.options().dtype(quant_out_type("quantize_per_channel", dtype).first));
}

at::Tensor quantize_per_channel(const at::Tensor& self, const at::Tensor& scales, const at::Tensor& zero_points,
                                int64_t axis, at::ScalarType dtype) {
    const char* op = "quantize_per_channel";
    axis = quantize_per_channel_check(self, scales, zero_points, axis);
    const auto qt = quant_out_type(op, dtype);
    const c10::DeviceGuard guard(self.device());
    auto x = self.contiguous();
    auto out = at::empty(self.sizes(), self.options().dtype(qt.first));
    // the scales are rounded to float32 (as torch's quantizer does with its double scales), the zero points widened
    auto sc = scales.to(self.device(), at::kFloat).contiguous();
    auto zp = zero_points.to(self.device(), at::kLong).contiguous();
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < axis; ++i) outer *= x.size(i);
    for (int64_t i = axis + 1; i < x.dim(); ++i) inner *= x.size(i);
    check_rc(qk_quantize_per_channel(x.data_ptr(), qk_dtype_of(x.scalar_type()), outer, x.size(axis), inner,
                                     sc.data_ptr<float>(), zp.data_ptr<int64_t>(), out.data_ptr(), qt.second,
                                     current_stream(x)),
             op);
    return out;
}

// dequantize.self: the integers as float32 (op_plugin/ops/v1r11/opapi/DequantizeKernelNpuOpApi.cpp:22-24)
int dequant_code(const at::Tensor& self) {
    switch (self.scalar_type()) {
    case at::kChar: return QK_I8;
    case at::kByte: return QK_U8;
    case at::kInt: return QK_I32;
    default: TORCH_CHECK(false, "dequantize: self must be int8, uint8 or int32 (a quantized NPU tensor), got ",
                         self.scalar_type());
    }
}

at::Tensor dequantize_meta(const at::Tensor& self) {
    dequant_code(self);
    return at::empty(self.sizes(), self.options().dtype(at::kFloat));
}

at::Tensor dequantize(const at::Tensor& self) {
    const int code = dequant_code(self);
    const c10::DeviceGuard guard(self.device());
    auto q = self.contiguous();
    auto out = at::empty(self.sizes(), self.options().dtype(at::kFloat));
    check_rc(qk_dequantize(q.data_ptr(), code, q.numel(), out.data_ptr<float>(), current_stream(q)), "dequantize");
    return out;
}

// ---------------------------------------------------------------- npu_rms_norm (+ dynamic quant)

// Normalized size D = gamma.numel() over the trailing gamma.dim() dims of self;
// rstd keeps the batch dims and has size 1 in the normalized ones
// (op_plugin/utils/KernelNpuOutputSize.cpp:1514-1530).
int64_t rms_norm_check(const char* op, const at::Tensor& self, const at::Tensor& gamma, bool quant) {
    const auto st = self.scalar_type();
    TORCH_CHECK(st == at::kHalf || st == at::kBFloat16 || (!quant && st == at::kFloat), op, ": self must be ",
                quant ? "float16 or bfloat16" : "float16, bfloat16 or float32", ", got ", st);
    TORCH_CHECK(gamma.scalar_type() == self.scalar_type(), op, ": gamma must have the dtype of self (",
                self.scalar_type(), "), got ", gamma.scalar_type());
    TORCH_CHECK(gamma.dim() >= 1 && gamma.dim() <= self.dim(), op, ": gamma must have 1..", self.dim(),
                " dims, got ", gamma.dim());
    TORCH_CHECK(!quant || gamma.dim() == 1, op, ": the fused quantization needs a 1-D gamma");
    for (int64_t i = 0; i < gamma.dim(); ++i)
        TORCH_CHECK(self.size(self.dim() - gamma.dim() + i) == gamma.size(i), op, ": gamma shape ", gamma.sizes(),
                    " does not match the trailing dims of self ", self.sizes());
    TORCH_CHECK(gamma.numel() > 0, op, ": the normalized dims must not be empty");
    return gamma.numel();
}

std::vector<int64_t> rstd_shape(const at::Tensor& self, const at::Tensor& gamma) {
    std::vector<int64_t> sh(self.sizes().begin(), self.sizes().end() - gamma.dim());
    for (int64_t i = 0; i < gamma.dim(); ++i) sh.push_back(1);
    return sh;
}

std::tuple<at::Tensor, at::Tensor> npu_rms_norm(const at::Tensor& self, const at::Tensor& gamma, double epsilon) {
    const int64_t D = rms_norm_check("npu_rms_norm", self, gamma, false);
    const c10::DeviceGuard guard(self.device());
    auto x = self.contiguous();
    auto g = gamma.contiguous();
    auto y = at::empty(x.sizes(), x.options());
    auto rstd = at::empty(rstd_shape(self, gamma), x.options().dtype(at::kFloat));
    const int rc = qk_rms_norm(x.data_ptr(), qk_dtype_of(x.scalar_type()), g.data_ptr(), x.numel() / D, D,
                               (float)epsilon, y.data_ptr(), rstd.data_ptr<float>(), current_stream(x));
    check_rc(rc, "npu_rms_norm");
    return {y, rstd};
}

std::tuple<at::Tensor, at::Tensor> npu_rms_norm_meta(const at::Tensor& self, const at::Tensor& gamma, double) {
    rms_norm_check("npu_rms_norm", self, gamma, false);
    return {at::empty(self.sizes(), self.options()), at::empty(rstd_shape(self, gamma), self.options().dtype(at::kFloat))};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> rms_norm_quant_outputs(const at::Tensor& self, const at::Tensor& gamma) {
    auto q = at::empty(self.sizes(), self.options().dtype(at::kChar));
    auto s = at::empty(self.sizes().slice(0, self.dim() - 1), self.options().dtype(at::kFloat));
    auto rstd = at::empty(rstd_shape(self, gamma), self.options().dtype(at::kFloat));
    return {q, s, rstd};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> npu_rms_norm_dynamic_quant(const at::Tensor& self,
                                                                          const at::Tensor& gamma, double epsilon) {
    const char* op = "npu_rms_norm_dynamic_quant";
    const int64_t D = rms_norm_check(op, self, gamma, true);
    const c10::DeviceGuard guard(self.device());
    auto x = self.contiguous();
    auto g = gamma.contiguous();
    auto [q, s, rstd] = rms_norm_quant_outputs(x, gamma);
    const int rc = qk_rms_norm_quant(x.data_ptr(), qk_dtype_of(x.scalar_type()), g.data_ptr(), x.numel() / D, D,
                                     (float)epsilon, q.data_ptr<int8_t>(), s.data_ptr<float>(), rstd.data_ptr<float>(),
                                     current_stream(x));
    check_rc(rc, op);
    return {q, s, rstd};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> npu_rms_norm_dynamic_quant_meta(const at::Tensor& self,
                                                                               const at::Tensor& gamma, double) {
    rms_norm_check("npu_rms_norm_dynamic_quant", self, gamma, true);
    return rms_norm_quant_outputs(self, gamma);
}

// ---------------------------------------------------------------- npu_swiglu (+ dynamic quant)

int64_t swiglu_check(const char* op, const at::Tensor& self, int64_t dim) {
    TORCH_CHECK(self.scalar_type() == at::kHalf || self.scalar_type() == at::kBFloat16, op,
                ": self must be float16 or bfloat16, got ", self.scalar_type());
    TORCH_CHECK(self.dim() >= 1, op, ": self must have at least one dimension");
    TORCH_CHECK(dim == -1 || dim == self.dim() - 1, op, ": only the last dimension can be split (dim=", dim, ")");
    TORCH_CHECK(self.size(-1) % 2 == 0, op, ": the split dimension must be even, got ", self.size(-1));
    return self.size(-1) / 2;
}

std::vector<int64_t> half_last(const at::Tensor& self) {
    std::vector<int64_t> sh(self.sizes().begin(), self.sizes().end());
    sh.back() /= 2;
    return sh;
}

at::Tensor npu_swiglu(const at::Tensor& self, int64_t dim) {
    const int64_t I = swiglu_check("npu_swiglu", self, dim);
    const c10::DeviceGuard guard(self.device());
    auto h = self.contiguous();
    auto y = at::empty(half_last(h), h.options());
    const int64_t rows = I == 0 ? 0 : h.numel() / (2 * I);
    const int rc = qk_swiglu(h.data_ptr(), qk_dtype_of(h.scalar_type()), rows, I, y.data_ptr(), current_stream(h));
    check_rc(rc, "npu_swiglu");
    return y;
}

at::Tensor npu_swiglu_meta(const at::Tensor& self, int64_t dim) {
    swiglu_check("npu_swiglu", self, dim);
    return at::empty(half_last(self), self.options());
}

std::tuple<at::Tensor, at::Tensor> npu_swiglu_dynamic_quant(const at::Tensor& self, int64_t dim) {
    const char* op = "npu_swiglu_dynamic_quant";
    const int64_t I = swiglu_check(op, self, dim);
    TORCH_CHECK(I > 0, op, ": the split dimension must not be empty");
    const c10::DeviceGuard guard(self.device());
    auto h = self.contiguous();
    auto q = at::empty(half_last(h), h.options().dtype(at::kChar));
    auto s = at::empty(h.sizes().slice(0, h.dim() - 1), h.options().dtype(at::kFloat));
    const int rc = qk_swiglu_quant(h.data_ptr(), qk_dtype_of(h.scalar_type()), h.numel() / (2 * I), I,
                                   q.data_ptr<int8_t>(), s.data_ptr<float>(), current_stream(h));
    check_rc(rc, op);
    return {q, s};
}

std::tuple<at::Tensor, at::Tensor> npu_swiglu_dynamic_quant_meta(const at::Tensor& self, int64_t dim) {
    const int64_t I = swiglu_check("npu_swiglu_dynamic_quant", self, dim);
    TORCH_CHECK(I > 0, "npu_swiglu_dynamic_quant: the split dimension must not be empty");
    return {at::empty(half_last(self), self.options().dtype(at::kChar)),
            at::empty(self.sizes().slice(0, self.dim() - 1), self.options().dtype(at::kFloat))};
}

// ---------------------------------------------------------------- fused gate-up + SwiGLU (quantized MLP block)
// h = npu_swiglu(npu_quant_matmul(x1, x2, scale, pertoken_scale=..., output_dtype=...)) with x2 [K, 2I] (row-major
// or the int8 NZ weight) in one GEMM whose epilogue applies the SwiGLU: bit-identical to that chain, which it
// runs instead where the fused kernel does not take the shape (qk_quant_matmul_swiglu: QK_ERR_UNSUPPORTED).
std::vector<int64_t> swiglu_matmul_check(const at::Tensor& x1, const at::Tensor& x2, const at::Tensor& scale,
                                         const std::optional<at::Tensor>& pertoken_scale, at::ScalarType out_type,
                                         int64_t& K, int64_t& I) {
    const char* op = "npu_quant_matmul_swiglu";
    TORCH_CHECK(x1.scalar_type() == at::kChar && x2.scalar_type() == at::kChar, op, ": x1 and x2 must be int8");
    TORCH_CHECK(x1.dim() >= 2, op, ": x1 must have at least 2 dimensions");
    const bool nz = is_w8_nz(x2);
    TORCH_CHECK(nz || x2.dim() == 2, op, ": x2 must be [K, 2I] or an int8 NZ weight, got ", x2.sizes());
    K = x1.size(-1);
    const int64_t x2_k = nz ? x2.size(1) * 64 : x2.size(0);
    TORCH_CHECK(x2_k == K, op, ": x1 last dim (", K, ") must equal the weight's K (", x2_k, ")");
    const int64_t N = nz ? x2.size(0) * 16 : x2.size(1);
    TORCH_CHECK(N % 2 == 0, op, ": the weight's column count (", N, ") must be even (gate and up halves)");
    I = N / 2;
    TORCH_CHECK(out_type == at::kBFloat16 || out_type == at::kHalf, op, ": output_dtype must be bfloat16 or float16");
    TORCH_CHECK(scale.dim() == 1 && (scale.size(0) == 1 || scale.size(0) == N), op, ": scale must be [1] or [", N, "]");
    TORCH_CHECK(scale.scalar_type() == at::kFloat || scale.scalar_type() == at::kBFloat16, op,
                ": scale must be float32 or bfloat16");
    if (pertoken_scale.has_value())
        TORCH_CHECK(pertoken_scale->scalar_type() == at::kFloat && pertoken_scale->numel() == leading_rows(x1), op,
                    ": pertoken_scale must be float32 with one element per row of x1");
    std::vector<int64_t> shape(x1.sizes().begin(), x1.sizes().end());
    shape.back() = I;
    return shape;
}

at::Tensor npu_quant_matmul_swiglu(const at::Tensor& x1_in, const at::Tensor& x2_in, const at::Tensor& scale_in,
                                   const std::optional<at::Tensor>& pertoken_scale,
                                   std::optional<at::ScalarType> output_dtype) {
    const at::ScalarType out_type = output_dtype.value_or(at::kBFloat16);
    int64_t K = 0, I = 0;
    const auto shape = swiglu_matmul_check(x1_in, x2_in, scale_in, pertoken_scale, out_type, K, I);
    const c10::DeviceGuard guard(x1_in.device());
    auto out = at::empty(shape, x1_in.options().dtype(out_type));
    if (out.numel() == 0) return out;
    const bool nz = is_w8_nz(x2_in);
    auto x1 = x1_in.contiguous();
    const bool kn = !nz && x2_in.stride(1) == 1 && x2_in.stride(0) >= 2 * I;
    if (nz || kn) {
        auto scale = scale_in.scalar_type() == at::kFloat ? scale_in.contiguous() : scale_in.to(at::kFloat);
        at::Tensor pt;
        if (pertoken_scale.has_value()) pt = pertoken_scale->contiguous();
        const int rc = qk_quant_matmul_swiglu(
            x1.data_ptr<int8_t>(), K, x2_in.data_ptr<int8_t>(), nz ? QK_FORMAT_FRACTAL_NZ : QK_FORMAT_ND,
            nz ? 0 : x2_in.stride(0), leading_rows(x1), I, K, scale.data_ptr<float>(), scale.numel(),
            pt.defined() ? pt.data_ptr<float>() : nullptr, out.data_ptr(), qk_dtype_of(out_type), current_stream(x1));
        if (rc != QK_ERR_UNSUPPORTED) {
            check_rc(rc, "npu_quant_matmul_swiglu");
            return out;
        }
    }
    // the shapes and layouts the fused kernel does not take: the unfused chain
    auto h2 = npu_quant_matmul(x1_in, x2_in, scale_in, std::nullopt, pertoken_scale, std::nullopt, out_type);
    return npu_swiglu(h2, -1);
}

// (q, q_scale) = npu_dynamic_quant(npu_quant_matmul_swiglu(...)) bit for bit: h and the GEMM's per-row partial
// absmax in a workspace, then one elementwise quantizing pass (qk_quant_matmul_swiglu_quant); the chain where
// the fused kernels do not take the shape.
std::tuple<at::Tensor, at::Tensor> npu_quant_matmul_swiglu_quant(const at::Tensor& x1_in, const at::Tensor& x2_in,
                                                                 const at::Tensor& scale_in,
                                                                 const std::optional<at::Tensor>& pertoken_scale,
                                                                 std::optional<at::ScalarType> output_dtype) {
    const at::ScalarType h_type = output_dtype.value_or(at::kBFloat16);
    int64_t K = 0, I = 0;
    const auto shape = swiglu_matmul_check(x1_in, x2_in, scale_in, pertoken_scale, h_type, K, I);
    const c10::DeviceGuard guard(x1_in.device());
    auto q = at::empty(shape, x1_in.options().dtype(at::kChar));
    auto qs = at::empty(at::IntArrayRef(shape).slice(0, shape.size() - 1), x1_in.options().dtype(at::kFloat));
    if (q.numel() == 0) return {q, qs};
    const bool nz = is_w8_nz(x2_in);
    auto x1 = x1_in.contiguous();
    const bool kn = !nz && x2_in.stride(1) == 1 && x2_in.stride(0) >= 2 * I;
    if (nz || kn) {
        auto scale = scale_in.scalar_type() == at::kFloat ? scale_in.contiguous() : scale_in.to(at::kFloat);
        at::Tensor pt;
        if (pertoken_scale.has_value()) pt = pertoken_scale->contiguous();
        const int64_t M = leading_rows(x1);
        size_t ws_bytes = 0;
        check_rc(qk_quant_matmul_swiglu_quant_workspace_size(M, I, &ws_bytes), "npu_quant_matmul_swiglu_quant");
        at::Tensor ws = workspace_for(x1, ws_bytes);
        const int rc = qk_quant_matmul_swiglu_quant(
            x1.data_ptr<int8_t>(), K, x2_in.data_ptr<int8_t>(), nz ? QK_FORMAT_FRACTAL_NZ : QK_FORMAT_ND,
            nz ? 0 : x2_in.stride(0), M, I, K, scale.data_ptr<float>(), scale.numel(),
            pt.defined() ? pt.data_ptr<float>() : nullptr, qk_dtype_of(h_type), q.data_ptr<int8_t>(),
            qs.data_ptr<float>(), ws.data_ptr(), ws_bytes, current_stream(x1));
        if (rc != QK_ERR_UNSUPPORTED) {
            check_rc(rc, "npu_quant_matmul_swiglu_quant");
            return {q, qs};
        }
    }
    return npu_dynamic_quant(npu_quant_matmul_swiglu(x1_in, x2_in, scale_in, pertoken_scale, h_type), std::nullopt);
}

std::tuple<at::Tensor, at::Tensor> npu_quant_matmul_swiglu_quant_meta(const at::Tensor& x1, const at::Tensor& x2,
                                                                      const at::Tensor& scale,
                                                                      const std::optional<at::Tensor>& pertoken_scale,
                                                                      std::optional<at::ScalarType> output_dtype) {
    const at::ScalarType h_type = output_dtype.value_or(at::kBFloat16);
    int64_t K = 0, I = 0;
    const auto shape = swiglu_matmul_check(x1, x2, scale, pertoken_scale, h_type, K, I);
    return {at::empty(shape, x1.options().dtype(at::kChar)),
            at::empty(at::IntArrayRef(shape).slice(0, shape.size() - 1), x1.options().dtype(at::kFloat))};
}

at::Tensor npu_quant_matmul_swiglu_meta(const at::Tensor& x1, const at::Tensor& x2, const at::Tensor& scale,
                                        const std::optional<at::Tensor>& pertoken_scale,
                                        std::optional<at::ScalarType> output_dtype) {
    const at::ScalarType out_type = output_dtype.value_or(at::kBFloat16);
    int64_t K = 0, I = 0;
    return at::empty(swiglu_matmul_check(x1, x2, scale, pertoken_scale, out_type, K, I), x1.options().dtype(out_type));
}

}  // namespace

TORCH_LIBRARY(npu, m) {
    m.def("npu_dynamic_quant(Tensor input, *, Tensor? smooth_scales=None) -> (Tensor, Tensor)");
    m.def(
        "npu_quant_matmul(Tensor x1, Tensor x2, Tensor scale, *, Tensor? offset=None, Tensor? pertoken_scale=None, "
        "Tensor? bias=None, ScalarType? output_dtype=None) -> Tensor");
    m.def(
        "npu_weight_quant_batchmatmul(Tensor x, Tensor weight, Tensor antiquant_scale, Tensor? antiquant_offset=None, "
        "Tensor? quant_scale=None, Tensor? quant_offset=None, Tensor? bias=None, int antiquant_group_size=0) -> Tensor");
    m.def("npu_convert_weight_to_int4pack(Tensor weight, int inner_k_tiles=0) -> Tensor");
    m.def("npu_format_cast(Tensor self, int acl_format) -> Tensor");
    // torch_npu.get_npu_format: the storage format the storage of self is recorded in (ND 2, FRACTAL_NZ 29)
    m.def("get_npu_format(Tensor self) -> int");
    // static quantization: op_plugin/config/v2r2/op_plugin_functions.yaml:1231, 1233 and
    // op_plugin/config/v1r11/op_plugin_functions.yaml:127
    m.def("quantize_per_channel(Tensor self, Tensor scales, Tensor zero_points, int axis, ScalarType dtype) -> Tensor");
    m.def("quantize_per_tensor(Tensor self, float scale, int zero_point, ScalarType dtype) -> Tensor");
    m.def("dequantize.self(Tensor self) -> Tensor");
    // schema as op_plugin/config/v2r2/op_plugin_functions.yaml:2047
    m.def("npu_rms_norm(Tensor self, Tensor gamma, float epsilon=1e-06) -> (Tensor, Tensor)");
    m.def("npu_swiglu(Tensor self, int dim=-1) -> Tensor");
    // fusions of this build for the quantized MLP block (no reference op): (q, scale, rstd) and (q, scale)
    m.def("npu_rms_norm_dynamic_quant(Tensor self, Tensor gamma, float epsilon=1e-06) -> (Tensor, Tensor, Tensor)");
    m.def("npu_swiglu_dynamic_quant(Tensor self, int dim=-1) -> (Tensor, Tensor)");
    m.def("npu_quant_matmul_swiglu(Tensor x1, Tensor x2, Tensor scale, *, Tensor? pertoken_scale=None, "
          "ScalarType? output_dtype=None) -> Tensor");
    m.def("npu_quant_matmul_swiglu_quant(Tensor x1, Tensor x2, Tensor scale, *, Tensor? pertoken_scale=None, "
          "ScalarType? output_dtype=None) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(npu, CUDA, m) {
    m.impl("npu_dynamic_quant", &npu_dynamic_quant);
    m.impl("npu_quant_matmul", &npu_quant_matmul);
    m.impl("npu_weight_quant_batchmatmul", &npu_weight_quant_batchmatmul);
    m.impl("npu_convert_weight_to_int4pack", &npu_convert_weight_to_int4pack);
    m.impl("npu_format_cast", &npu_format_cast);
    m.impl("quantize_per_channel", &quantize_per_channel);
    m.impl("quantize_per_tensor", &quantize_per_tensor);
    m.impl("dequantize.self", &dequantize);
    m.impl("npu_rms_norm", &npu_rms_norm);
    m.impl("npu_swiglu", &npu_swiglu);
    m.impl("npu_rms_norm_dynamic_quant", &npu_rms_norm_dynamic_quant);
    m.impl("npu_swiglu_dynamic_quant", &npu_swiglu_dynamic_quant);
    m.impl("npu_quant_matmul_swiglu", &npu_quant_matmul_swiglu);
    m.impl("npu_quant_matmul_swiglu_quant", &npu_quant_matmul_swiglu_quant);
}

TORCH_LIBRARY_IMPL(npu, CompositeExplicitAutograd, m) { m.impl("get_npu_format", &get_npu_format); }

TORCH_LIBRARY_IMPL(npu, Meta, m) {
    m.impl("npu_dynamic_quant", &npu_dynamic_quant_meta);
    m.impl("npu_quant_matmul", &npu_quant_matmul_meta);
    m.impl("npu_weight_quant_batchmatmul", &npu_weight_quant_batchmatmul_meta);
    m.impl("npu_convert_weight_to_int4pack", &npu_convert_weight_to_int4pack_meta);
    m.impl("npu_format_cast", &npu_format_cast_meta);
    m.impl("quantize_per_channel", &quantize_per_channel_meta);
    m.impl("quantize_per_tensor", &quantize_per_tensor_meta);
    m.impl("dequantize.self", &dequantize_meta);
    m.impl("npu_rms_norm", &npu_rms_norm_meta);
    m.impl("npu_swiglu", &npu_swiglu_meta);
    m.impl("npu_rms_norm_dynamic_quant", &npu_rms_norm_dynamic_quant_meta);
    m.impl("npu_swiglu_dynamic_quant", &npu_swiglu_dynamic_quant_meta);
    m.impl("npu_quant_matmul_swiglu", &npu_quant_matmul_swiglu_meta);
    m.impl("npu_quant_matmul_swiglu_quant", &npu_quant_matmul_swiglu_quant_meta);
}
