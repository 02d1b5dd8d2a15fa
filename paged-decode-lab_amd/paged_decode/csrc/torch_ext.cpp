// Thin PyTorch-ROCm extension over the C ABI in include/paged_decode.h.
//
// Exposes `decode(q, k, v, table, lengths, numerator, stats, out, split_tokens,
// merge_mode[, k_scale, v_scale])` with the argument list of reference
// src/paged_decode/csrc/bindings.cpp:3-9, and repeats the tensor checks of
// reference decode.cu:201-237 (as TORCH_CHECK -> RuntimeError), including
// the reference's workspace layout: numerator [B, Hq, 4 * splits, D] and
// stats [B, Hq, 4 * splits, 2], four states per partition. Launches go to the current
// torch stream of q's device, so calls follow torch stream semantics and can be
// captured by torch.cuda.CUDAGraph (hipGraph). Nothing is allocated here.

#include <torch/extension.h>

// PyTorch-ROCm tags HIP devices with torch's "cuda" device type. c10::hip's
// guard and stream accessors for such tensors are the *MasqueradingAsCUDA
// variants (the plain HIP ones expect DeviceType::HIP and reject them); both
// give a HIP device guard and the current hipStream_t, nothing CUDA-specific.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <algorithm>
#include <cstdint>
#include <string>

#include "paged_decode.h"

#ifndef PD_BUILD_DIGEST
#define PD_BUILD_DIGEST "unknown"
#endif

namespace {

void check_status(int status) {
    TORCH_CHECK(status == PD_OK, "paged_decode: ", pd_status_string(status), " (status ", status, ")");
}

hipStream_t current_stream(const torch::Tensor& like) {
    return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(like.get_device()).stream();
}

// Storage format code of a dtype or tensor (-1 for anything the library does
// not store).
int dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return PD_DTYPE_F32;
        case at::kHalf: return PD_DTYPE_F16;
        case at::kBFloat16: return PD_DTYPE_BF16;
        case at::kFloat8_e4m3fn: return PD_DTYPE_FP8_E4M3;
        case at::kFloat8_e5m2: return PD_DTYPE_FP8_E5M2;
        default: return -1;
    }
}

int dtype_code(const torch::Tensor& t) { return dtype_code(t.scalar_type()); }

bool is_fp8(const torch::Tensor& t) {
    return t.scalar_type() == at::kFloat8_e4m3fn || t.scalar_type() == at::kFloat8_e5m2;
}

struct Shape {
    int64_t batch, heads, dim, kv_heads, page_size, pages, width, splits;
};

Shape check_inputs(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                   const torch::Tensor& table, const torch::Tensor& lengths,
                   const torch::Tensor& numerator, const torch::Tensor& stats, int64_t split_tokens) {
    for (const auto& t : {q, k, v, table, lengths, numerator, stats}) {
        TORCH_CHECK(t.is_cuda() && t.is_contiguous(), "all tensors must be contiguous GPU tensors");
        TORCH_CHECK(t.device() == q.device(), "device mismatch");
    }
    TORCH_CHECK(q.dim() == 3 && k.dim() == 4 && v.sizes() == k.sizes(), "expected q[B,H,D], k/v[P,T,KV,D]");
    Shape s{q.size(0), q.size(1), q.size(2), 0, 0, 0, 0, 0};
    TORCH_CHECK(s.batch > 0 && s.batch <= 65535 && s.heads > 0 && s.heads <= 65535,
                "batch and head count must be in [1,65535]");
    TORCH_CHECK(s.dim == 64 || s.dim == 128, "supported head dimensions: 64,128");
    TORCH_CHECK(k.size(0) > 0 && k.size(1) > 0 && k.size(2) > 0 && k.size(3) == s.dim &&
                    s.heads % k.size(2) == 0 && k.size(0) <= INT32_MAX && (k.size(1) == 16 || k.size(1) == 32),
                "invalid cache shape");
    s.pages = k.size(0);
    s.page_size = k.size(1);
    s.kv_heads = k.size(2);
    TORCH_CHECK(v.scalar_type() == k.scalar_type() &&
                    (k.scalar_type() == q.scalar_type() || (is_fp8(k) && q.scalar_type() != at::kFloat)),
                "q/k/v dtype mismatch");
    TORCH_CHECK(q.scalar_type() == at::kHalf || q.scalar_type() == at::kFloat || q.scalar_type() == at::kBFloat16,
                "supported input dtypes: float16,float32,bfloat16 (k/v may also be float8_e4m3fn/float8_e5m2)");
    TORCH_CHECK(table.dim() == 2 && table.size(0) == s.batch && table.size(1) > 0 && table.size(1) <= 65536 &&
                    lengths.dim() == 1 && lengths.size(0) == s.batch,
                "metadata shape mismatch");
    TORCH_CHECK(table.scalar_type() == at::kInt && lengths.scalar_type() == at::kInt, "metadata must be int32");
    s.width = table.size(1);
    TORCH_CHECK(numerator.dim() == 4 && numerator.size(0) == s.batch && numerator.size(1) == s.heads &&
                    numerator.size(2) > 0 && numerator.size(2) % 4 == 0 && numerator.size(3) == s.dim,
                "invalid numerator workspace");
    s.splits = numerator.size(2) / 4;
    TORCH_CHECK(s.splits <= 65535 && split_tokens > 0 && split_tokens <= 1048576, "invalid split configuration");
    TORCH_CHECK(stats.dim() == 4 && stats.size(0) == s.batch && stats.size(1) == s.heads &&
                    stats.size(2) == numerator.size(2) && stats.size(3) == 2,
                "invalid stats workspace");
    TORCH_CHECK(numerator.scalar_type() == at::kFloat && stats.scalar_type() == at::kFloat,
                "workspaces must be float32");
    return s;
}

void check_output(const torch::Tensor& q, const torch::Tensor& out, int64_t merge_mode, int64_t splits) {
    TORCH_CHECK(out.is_cuda() && out.is_contiguous() && out.device() == q.device(),
                "output must be a contiguous tensor on the input device");
    TORCH_CHECK(out.sizes() == q.sizes(), "invalid output shape");
    TORCH_CHECK(out.scalar_type() == at::kFloat, "output must be float32");
    TORCH_CHECK(merge_mode == PD_MERGE_SERIAL ||
                    (merge_mode == PD_MERGE_SHARED && 4 * splits <= PD_SHARED_MERGE_MAX_PARTS),
                "shared merge requires at most 4096 partial states");
}

// PD_HINT_UNSHARED_PAGES when the caller knows no physical page is shared
// between sequences (the plan derives it from its metadata).
int hints(bool unshared_pages, bool ragged_lengths) {
    return (unshared_pages ? PD_HINT_UNSHARED_PAGES : 0) | (ragged_lengths ? PD_HINT_RAGGED_LENGTHS : 0);
}

// Host pointer of the optional per-sequence length bounds (a CPU int32
// tensor [batch]), or null.
const int32_t* bounds_pointer(const c10::optional<torch::Tensor>& bounds, int64_t batch) {
    if (!bounds.has_value()) return nullptr;
    const auto& t = *bounds;
    TORCH_CHECK(t.device().is_cpu() && t.scalar_type() == at::kInt && t.is_contiguous() && t.dim() == 1 &&
                    t.size(0) == batch,
                "length_bounds must be a contiguous CPU int32 tensor [batch]");
    return t.data_ptr<int32_t>();
}

// Host pointer of the optional shared-prefix runs (a CPU int32 tensor
// [2 * batch], see pd_prefix_runs), or null.
const int32_t* runs_pointer(const c10::optional<torch::Tensor>& runs, int64_t batch) {
    if (!runs.has_value()) return nullptr;
    const auto& t = *runs;
    TORCH_CHECK(t.device().is_cpu() && t.scalar_type() == at::kInt && t.is_contiguous() && t.dim() == 1 &&
                    t.size(0) == 2 * batch,
                "prefix_runs must be a contiguous CPU int32 tensor [2 * batch]");
    return t.data_ptr<int32_t>();
}

}  // namespace

void decode(torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor table, torch::Tensor lengths,
            torch::Tensor numerator, torch::Tensor stats, torch::Tensor out, int64_t split_tokens,
            int64_t merge_mode, double k_scale, double v_scale, bool unshared_pages, bool ragged_lengths,
            c10::optional<torch::Tensor> length_bounds, c10::optional<torch::Tensor> prefix_runs) {
    const Shape s = check_inputs(q, k, v, table, lengths, numerator, stats, split_tokens);
    check_output(q, out, merge_mode, s.splits);
    const int32_t* bounds = bounds_pointer(length_bounds, s.batch);
    const int32_t* runs = runs_pointer(prefix_runs, s.batch);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    check_status(pd_decode_prefix(q.data_ptr(), dtype_code(q), k.data_ptr(), v.data_ptr(), dtype_code(k),
                              static_cast<float>(k_scale), static_cast<float>(v_scale), table.data_ptr<int32_t>(),
                              lengths.data_ptr<int32_t>(), numerator.data_ptr<float>(), stats.data_ptr<float>(),
                              out.data_ptr<float>(), static_cast<int>(s.batch), static_cast<int>(s.heads),
                              static_cast<int>(s.kv_heads), static_cast<int>(s.dim), static_cast<int>(s.page_size),
                              static_cast<int>(s.width), static_cast<int>(s.pages), static_cast<int>(s.splits),
                              static_cast<int>(split_tokens), static_cast<int>(merge_mode),
                              hints(unshared_pages, ragged_lengths), bounds, runs, current_stream(q)));
}

// Partition stage alone (first launch of decode); used to time that kernel.
void partial(torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor table, torch::Tensor lengths,
             torch::Tensor numerator, torch::Tensor stats, int64_t split_tokens, double k_scale, double v_scale,
             bool unshared_pages, bool ragged_lengths, c10::optional<torch::Tensor> length_bounds,
             c10::optional<torch::Tensor> prefix_runs) {
    const Shape s = check_inputs(q, k, v, table, lengths, numerator, stats, split_tokens);
    const int32_t* bounds = bounds_pointer(length_bounds, s.batch);
    const int32_t* runs = runs_pointer(prefix_runs, s.batch);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    check_status(pd_decode_partial_prefix(
        q.data_ptr(), dtype_code(q), k.data_ptr(), v.data_ptr(), dtype_code(k), static_cast<float>(k_scale),
        static_cast<float>(v_scale), table.data_ptr<int32_t>(), lengths.data_ptr<int32_t>(),
        numerator.data_ptr<float>(), stats.data_ptr<float>(), static_cast<int>(s.batch), static_cast<int>(s.heads),
        static_cast<int>(s.kv_heads), static_cast<int>(s.dim), static_cast<int>(s.page_size),
        static_cast<int>(s.width), static_cast<int>(s.pages), static_cast<int>(s.splits),
        static_cast<int>(split_tokens), hints(unshared_pages, ragged_lengths), bounds, runs, current_stream(q)));
}

// Shared-prefix runs of a host page table [batch, width] (pd_prefix_runs):
// a CPU int32 tensor [2 * batch] of (leader, leading entries in common).
torch::Tensor prefix_runs(torch::Tensor table) {
    TORCH_CHECK(table.device().is_cpu() && table.scalar_type() == at::kInt && table.is_contiguous() &&
                    table.dim() == 2 && table.size(0) > 0 && table.size(1) > 0,
                "table must be a contiguous CPU int32 tensor [batch, width]");
    torch::Tensor runs = torch::empty({2 * table.size(0)}, torch::dtype(torch::kInt32));
    check_status(pd_prefix_runs(table.data_ptr<int32_t>(), static_cast<int>(table.size(0)),
                                static_cast<int>(table.size(1)), runs.data_ptr<int32_t>()));
    return runs;
}

// Merge stage alone (second launch of decode); lengths, page_size,
// table_width and split_tokens are those of the partition stage.
void merge(torch::Tensor numerator, torch::Tensor stats, torch::Tensor out, torch::Tensor lengths, int64_t page_size,
           int64_t table_width, int64_t split_tokens, int64_t merge_mode) {
    for (const auto& t : {numerator, stats, out, lengths}) {
        TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.device() == out.device(),
                    "all tensors must be contiguous GPU tensors on one device");
    }
    for (const auto& t : {numerator, stats, out}) TORCH_CHECK(t.scalar_type() == at::kFloat, "workspaces/output must be float32");
    TORCH_CHECK(lengths.scalar_type() == at::kInt && lengths.dim() == 1 && lengths.size(0) == out.size(0),
                "lengths must be int32 [batch]");
    TORCH_CHECK(numerator.dim() == 4 && stats.dim() == 4 && out.dim() == 3, "invalid workspace shapes");
    TORCH_CHECK(stats.size(0) == numerator.size(0) && stats.size(1) == numerator.size(1) &&
                    stats.size(2) == numerator.size(2) && numerator.size(2) % 4 == 0 && stats.size(3) == 2 &&
                    out.size(0) == numerator.size(0) && out.size(1) == numerator.size(1) &&
                    out.size(2) == numerator.size(3),
                "workspace/output shape mismatch");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
    check_status(pd_decode_merge(numerator.data_ptr<float>(), stats.data_ptr<float>(), out.data_ptr<float>(),
                                 lengths.data_ptr<int32_t>(), static_cast<int>(numerator.size(0)),
                                 static_cast<int>(numerator.size(1)), static_cast<int>(numerator.size(3)),
                                 static_cast<int>(page_size), static_cast<int>(table_width),
                                 static_cast<int>(numerator.size(2) / 4), static_cast<int>(split_tokens),
                                 static_cast<int>(merge_mode), current_stream(out)));
}

// KV-cache append: k_new/v_new [B, tokens, Hkv, D] into k_cache/v_cache
// [P, T, Hkv, D] at positions[b] + j (advance = false) or at lengths[b] + j with
// lengths advanced on the device (advance = true, all or nothing per sequence,
// positions below max_context only; max_context < 0 means the table's capacity).
void append_kv(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor table, torch::Tensor positions,
               torch::Tensor k_cache, torch::Tensor v_cache, bool advance, int64_t max_context) {
    for (const auto& t : {k_new, v_new, table, positions, k_cache, v_cache}) {
        TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.device() == k_cache.device(),
                    "all tensors must be contiguous GPU tensors on one device");
    }
    TORCH_CHECK(k_cache.dim() == 4 && v_cache.sizes() == k_cache.sizes(), "expected k/v cache [P,T,KV,D]");
    TORCH_CHECK(k_new.dim() == 4 && v_new.sizes() == k_new.sizes() && k_new.size(2) == k_cache.size(2) &&
                    k_new.size(3) == k_cache.size(3),
                "expected k_new/v_new [B,tokens,KV,D] matching the cache");
    TORCH_CHECK(k_new.scalar_type() == k_cache.scalar_type() && v_new.scalar_type() == k_cache.scalar_type() &&
                    v_cache.scalar_type() == k_cache.scalar_type(),
                "new tokens and cache must share one dtype");
    TORCH_CHECK(dtype_code(k_cache) >= 0,
                "supported cache dtypes: float32,float16,bfloat16,float8_e4m3fn,float8_e5m2");
    TORCH_CHECK(table.dim() == 2 && table.size(0) == k_new.size(0) && positions.dim() == 1 &&
                    positions.size(0) == k_new.size(0),
                "metadata shape mismatch");
    TORCH_CHECK(table.scalar_type() == at::kInt && positions.scalar_type() == at::kInt, "metadata must be int32");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(k_cache.device());
    const int dtype = dtype_code(k_cache);
    const int b = static_cast<int>(k_new.size(0)), tokens = static_cast<int>(k_new.size(1));
    const int kv = static_cast<int>(k_cache.size(2)), d = static_cast<int>(k_cache.size(3));
    const int page = static_cast<int>(k_cache.size(1)), width = static_cast<int>(table.size(1));
    const int pages = static_cast<int>(k_cache.size(0));
    hipStream_t stream = current_stream(k_cache);
    if (advance) {
        const int64_t capacity = static_cast<int64_t>(width) * page;
        const int64_t limit = max_context < 0 ? std::min<int64_t>(capacity, 1 << 20) : max_context;
        TORCH_CHECK(limit <= (1 << 20), "max_context must not exceed 1048576");
        check_status(pd_append_kv_advance(k_new.data_ptr(), v_new.data_ptr(), dtype, table.data_ptr<int32_t>(),
                                          positions.data_ptr<int32_t>(), k_cache.data_ptr(), v_cache.data_ptr(), b,
                                          tokens, kv, d, page, width, pages, static_cast<int>(limit), stream));
    } else {
        check_status(pd_append_kv(k_new.data_ptr(), v_new.data_ptr(), dtype, table.data_ptr<int32_t>(),
                                  positions.data_ptr<int32_t>(), k_cache.data_ptr(), v_cache.data_ptr(), b, tokens,
                                  kv, d, page, width, pages, stream));
    }
}

// CSR page lists (device tensors) -> the plan's page table and lengths.
void table_from_csr(torch::Tensor indptr, torch::Tensor indices, torch::Tensor last_page_len, torch::Tensor table,
                    torch::Tensor lengths, c10::optional<torch::Tensor> overflow, int64_t page_size,
                    int64_t max_context) {
    for (const auto& t : {indptr, indices, last_page_len, table, lengths}) {
        TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.device() == table.device() && t.scalar_type() == at::kInt,
                    "CSR metadata, table and lengths must be contiguous int32 tensors on one GPU");
    }
    TORCH_CHECK(table.dim() == 2 && lengths.dim() == 1 && lengths.size(0) == table.size(0) && indptr.dim() == 1 &&
                    indptr.size(0) == table.size(0) + 1 && last_page_len.dim() == 1 &&
                    last_page_len.size(0) == table.size(0) && indices.dim() == 1,
                "expected indptr [B+1], indices [nnz], last_page_len [B], table [B,W], lengths [B]");
    int32_t* flag = nullptr;
    if (overflow.has_value()) {
        const auto& o = *overflow;
        TORCH_CHECK(o.is_cuda() && o.device() == table.device() && o.scalar_type() == at::kInt && o.numel() >= 1,
                    "overflow must be an int32 GPU tensor");
        flag = o.data_ptr<int32_t>();
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(table.device());
    check_status(pd_table_from_csr(indptr.data_ptr<int32_t>(), indices.data_ptr<int32_t>(), indices.numel(),
                                   last_page_len.data_ptr<int32_t>(), table.data_ptr<int32_t>(),
                                   lengths.data_ptr<int32_t>(), flag, static_cast<int>(table.size(0)),
                                   static_cast<int>(table.size(1)), static_cast<int>(page_size),
                                   static_cast<int>(max_context), current_stream(table)));
}

// Kernel launches decode makes for these formats and shapes (1: whole rows,
// 2: partition and merge).
int64_t launch_count(at::ScalarType q_dtype, at::ScalarType kv_dtype, int64_t batch, int64_t query_heads,
                     int64_t kv_heads, int64_t head_dim, int64_t page_size, int64_t table_width,
                     int64_t physical_pages, int64_t splits, int64_t split_tokens, bool unshared_pages,
                     bool ragged_lengths) {
    int launches = 0;
    check_status(pd_decode_launch_count(dtype_code(q_dtype), dtype_code(kv_dtype), static_cast<int>(batch),
                                        static_cast<int>(query_heads), static_cast<int>(kv_heads),
                                        static_cast<int>(head_dim), static_cast<int>(page_size),
                                        static_cast<int>(table_width), static_cast<int>(physical_pages),
                                        static_cast<int>(splits), static_cast<int>(split_tokens),
                                        hints(unshared_pages, ragged_lengths), &launches));
    return launches;
}

// Partitions (count, tokens per partition) decode's two launches run over for
// these formats, shapes and optional host length bounds: the caller's split
// or a coarser one (see pd_decode_kernel_split).
std::tuple<int64_t, int64_t> kernel_split(at::ScalarType q_dtype, at::ScalarType kv_dtype, int64_t batch,
                                          int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                                          int64_t page_size, int64_t table_width, int64_t physical_pages,
                                          int64_t splits, int64_t split_tokens,
                                          c10::optional<torch::Tensor> length_bounds, int64_t compute_units) {
    const int32_t* bounds = bounds_pointer(length_bounds, batch);
    int kernel_splits = 0, kernel_split_tokens = 0;
    check_status(pd_decode_kernel_split(dtype_code(q_dtype), dtype_code(kv_dtype), static_cast<int>(batch),
                                        static_cast<int>(query_heads), static_cast<int>(kv_heads),
                                        static_cast<int>(head_dim), static_cast<int>(page_size),
                                        static_cast<int>(table_width), static_cast<int>(physical_pages),
                                        static_cast<int>(splits), static_cast<int>(split_tokens), bounds,
                                        static_cast<int>(compute_units), &kernel_splits, &kernel_split_tokens));
    return {kernel_splits, kernel_split_tokens};
}

// The launches decode makes for these formats, shapes, merge mode, hints and
// optional host length bounds (pd_decode_launch_plan), as a dict.
py::dict launch_plan(at::ScalarType q_dtype, at::ScalarType kv_dtype, int64_t batch, int64_t query_heads,
                     int64_t kv_heads, int64_t head_dim, int64_t page_size, int64_t table_width,
                     int64_t physical_pages, int64_t splits, int64_t split_tokens, int64_t merge_mode,
                     bool unshared_pages, bool ragged_lengths, c10::optional<torch::Tensor> length_bounds,
                     int64_t compute_units, c10::optional<torch::Tensor> prefix_runs) {
    const int32_t* bounds = bounds_pointer(length_bounds, batch);
    const int32_t* runs = runs_pointer(prefix_runs, batch);
    pd_launch_plan p{};
    check_status(pd_decode_launch_plan(dtype_code(q_dtype), dtype_code(kv_dtype), static_cast<int>(batch),
                                       static_cast<int>(query_heads), static_cast<int>(kv_heads),
                                       static_cast<int>(head_dim), static_cast<int>(page_size),
                                       static_cast<int>(table_width), static_cast<int>(physical_pages),
                                       static_cast<int>(splits), static_cast<int>(split_tokens),
                                       static_cast<int>(merge_mode), hints(unshared_pages, ragged_lengths), bounds,
                                       runs, static_cast<int>(compute_units), &p));
    static const char* kinds[] = {"rectangular", "rectangular+tails", "work list", "whole rows"};
    py::dict d;
    d["launches"] = p.launches;
    d["kernel_split"] = py::make_tuple(p.kernel_splits, p.kernel_split_tokens);
    d["grid"] = py::make_tuple(p.grid_x, p.grid_y, p.grid_z);
    d["waves_per_workgroup"] = p.waves_per_workgroup;
    d["kv_heads_per_workgroup"] = p.kv_heads_per_workgroup;
    d["quarters_per_workgroup"] = p.quarters_per_workgroup;
    d["head_tile"] = p.head_tile;
    d["grid_kind"] = kinds[std::min(std::max(p.grid_kind, 0), 3)];
    d["xcd_grouped"] = p.xcd_grouped != 0;
    d["combined"] = p.combined != 0;
    d["stream_mode"] = p.stream_mode;
    d["shared_prefix_items"] = p.shared_prefix_items;
    if (p.merge_kernel >= 0) {
        d["merge"] = py::make_tuple(p.merge_kernel == 0 ? "rows" : "cols", p.merge_loads, p.merge_chunk_floats,
                                    p.merge_xcd_grouped != 0, p.merge_state_stride);
    } else {
        d["merge"] = py::none();
    }
    return d;
}

// One streaming read of the leading a_bytes of a and b_bytes of b (the
// bandwidth ceiling of a decode launch over as many K/V bytes).
void stream_read(torch::Tensor a, torch::Tensor b, int64_t a_bytes, int64_t b_bytes, torch::Tensor sink) {
    for (const auto& t : {a, b, sink}) {
        TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.device() == a.device(),
                    "stream_read: contiguous tensors on one GPU");
    }
    TORCH_CHECK(a_bytes >= 0 && b_bytes >= 0 && a_bytes <= a.numel() * a.element_size() &&
                    b_bytes <= b.numel() * b.element_size(),
                "stream_read: byte counts must fit the tensors");
    TORCH_CHECK(sink.numel() * sink.element_size() >= 8, "stream_read: sink needs 8 bytes");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
    check_status(pd_stream_read(a.data_ptr(), static_cast<size_t>(a_bytes), b.data_ptr(), static_cast<size_t>(b_bytes),
                                static_cast<uint32_t*>(sink.data_ptr()), current_stream(a)));
}

PYBIND11_MODULE(_C, m) {
    m.doc() = "Split-K paged GQA decode for gfx950 (calls libpaged_decode_hip.so)";
    m.def("decode", &decode, "Paged split-K GQA decode (partition + merge)", py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("table"), py::arg("lengths"), py::arg("numerator"), py::arg("stats"), py::arg("out"),
          py::arg("split_tokens"), py::arg("merge_mode"), py::arg("k_scale") = 1.0, py::arg("v_scale") = 1.0,
          py::arg("unshared_pages") = false, py::arg("ragged_lengths") = false,
          py::arg("length_bounds") = py::none(), py::arg("prefix_runs") = py::none());
    m.def("partial", &partial, "Partition stage only", py::arg("q"), py::arg("k"), py::arg("v"), py::arg("table"),
          py::arg("lengths"), py::arg("numerator"), py::arg("stats"), py::arg("split_tokens"),
          py::arg("k_scale") = 1.0, py::arg("v_scale") = 1.0, py::arg("unshared_pages") = false,
          py::arg("ragged_lengths") = false, py::arg("length_bounds") = py::none(),
          py::arg("prefix_runs") = py::none());
    m.def("prefix_runs", &prefix_runs, "Shared-prefix runs of a host page table (pd_prefix_runs)", py::arg("table"));
    m.def("merge", &merge, "Merge stage only");
    m.def("append_kv", &append_kv, "Paged KV-cache append", py::arg("k_new"), py::arg("v_new"), py::arg("table"),
          py::arg("positions"), py::arg("k_cache"), py::arg("v_cache"), py::arg("advance"),
          py::arg("max_context") = -1);
    m.def("table_from_csr", &table_from_csr, "CSR page lists to page table and lengths on the device",
          py::arg("indptr"), py::arg("indices"), py::arg("last_page_len"), py::arg("table"), py::arg("lengths"),
          py::arg("overflow") = py::none(), py::arg("page_size"), py::arg("max_context"));
    m.def("workspace_bytes", [](int64_t b, int64_t h, int64_t d, int64_t s) {
        return static_cast<int64_t>(pd_workspace_bytes(static_cast<int>(b), static_cast<int>(h),
                                                       static_cast<int>(d), static_cast<int>(s)));
    });
    m.def("launch_count", &launch_count, "Kernel launches of a decode call (1: whole rows, 2: partition + merge)");
    m.def("kernel_split", &kernel_split, "Partitions (count, tokens) a decode call's launches run over",
          py::arg("q_dtype"), py::arg("kv_dtype"), py::arg("batch"), py::arg("query_heads"), py::arg("kv_heads"),
          py::arg("head_dim"), py::arg("page_size"), py::arg("table_width"), py::arg("physical_pages"),
          py::arg("splits"), py::arg("split_tokens"), py::arg("length_bounds") = py::none(),
          py::arg("compute_units") = 0);
    m.def("launch_plan", &launch_plan, "The launches a decode call makes (pd_decode_launch_plan)", py::arg("q_dtype"),
          py::arg("kv_dtype"), py::arg("batch"), py::arg("query_heads"), py::arg("kv_heads"), py::arg("head_dim"),
          py::arg("page_size"), py::arg("table_width"), py::arg("physical_pages"), py::arg("splits"),
          py::arg("split_tokens"), py::arg("merge_mode"), py::arg("unshared_pages") = false,
          py::arg("ragged_lengths") = false, py::arg("length_bounds") = py::none(), py::arg("compute_units") = 0,
          py::arg("prefix_runs") = py::none());
    m.def("stream_read", &stream_read, "One streaming read of the leading bytes of two tensors", py::arg("a"),
          py::arg("b"), py::arg("a_bytes"), py::arg("b_bytes"), py::arg("sink"));
    m.def("abi_version", &pd_abi_version, "ABI version the loaded HIP library reports");
    m.def("header_abi_version", [] { return PD_ABI_VERSION; }, "ABI version of the header this module was built with");
    m.def("build_digest", [] { return std::string(PD_BUILD_DIGEST); }, "Digest of the sources this module was built from");
}
