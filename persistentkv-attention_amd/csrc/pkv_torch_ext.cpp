// pkv_torch_ext.cpp — PyTorch op surface of the PersistentKV engine, over the C ABI.
//
// Same op names, positional arguments, validation messages and in-place `None` return
// as tests/persistentkv_torch_extension.cu (:9-31 checks, :35-317 ops, :319-336
// bindings), so tests/benchmark_serving_trace.py can call it unchanged.  Differences:
//   * q / pages / output may be fp16 or bf16 (all four the same dtype);
//   * G = Hq / Hkv may be any integer in [1, 32] (the reference accepts {1, 2, 4, 8});
//   * launch failures raise RuntimeError instead of terminating the process.
// Beyond the reference's four ops: the two work-queue stages, fp8 (float8_e4m3fn) K/V
// variants of the indexed and work-queue ops, the contiguous-layout decode and
// query-head baseline of its C++ API (cuh:1077-1108, :1263-1282), and the KV-cache append
// (fp16 / bf16 / fp8 pools) that a serving loop runs before each decode step, alone or
// fused into the indexed and work-queue ops (*_append).
// Work is enqueued on the current HIP stream of the tensors' device without a host sync,
// so the ops can be captured in HIP graphs.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "pkv.h"

namespace {

void check_tensor(const torch::Tensor& tensor, const char* name, at::ScalarType dtype, int64_t dims) {
  TORCH_CHECK(tensor.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(tensor.scalar_type() == dtype, name, " has wrong dtype");
  TORCH_CHECK(tensor.dim() == dims, name, " has wrong rank");
  TORCH_CHECK(tensor.is_contiguous(), name, " must be contiguous");
}

// The activation dtype is taken from q and must be fp16 or bf16.
at::ScalarType activation_dtype(const torch::Tensor& q, const char* name) {
  TORCH_CHECK(q.scalar_type() == at::kHalf || q.scalar_type() == at::kBFloat16, name,
              " has wrong dtype");
  return q.scalar_type();
}

int32_t pkv_dtype_of(at::ScalarType t) { return t == at::kBFloat16 ? PKV_DTYPE_BF16 : PKV_DTYPE_F16; }

void check_supported_gqa(int Hq, int Hkv) {
  TORCH_CHECK(Hkv > 0, "Hkv must be positive");
  TORCH_CHECK(Hq % Hkv == 0, "Hq must be divisible by Hkv");
  const int G = Hq / Hkv;
  TORCH_CHECK(G >= 1 && G <= PKV_MAX_GROUP, "PersistentKV supports G=Hq/Hkv in [1,32]; got G=", G,
              " from Hq=", Hq, " Hkv=", Hkv);
}

void check_workspace(const torch::Tensor& workspace) {
  TORCH_CHECK(workspace.is_cuda(), "workspace must be a CUDA tensor");
  TORCH_CHECK(workspace.is_contiguous(), "workspace must be contiguous");
}

void check_pages(const torch::Tensor& k_pages, const torch::Tensor& v_pages, int64_t page_size, int d) {
  const int64_t physical_pages = k_pages.size(0);
  const int64_t Hkv = k_pages.size(1);
  TORCH_CHECK(v_pages.size(0) == physical_pages && v_pages.size(1) == Hkv &&
                  v_pages.size(2) == page_size && v_pages.size(3) == d,
              "v_pages shape mismatch");
  TORCH_CHECK(k_pages.size(2) == page_size && k_pages.size(3) == d, "k_pages shape mismatch");
}

void* ws_ptr(const torch::Tensor& w) { return w.numel() > 0 ? w.data_ptr() : nullptr; }
size_t ws_bytes(const torch::Tensor& w) { return w.numel() > 0 ? (size_t)w.nbytes() : 0; }
void* stream_of(const torch::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}
int32_t i32(int64_t v, const char* name) {
  TORCH_CHECK(v >= INT32_MIN && v <= INT32_MAX, name, " does not fit in int32");
  return (int32_t)v;
}
void raise_on(int status) { TORCH_CHECK(status == PKV_OK, pkv_last_error()); }

}  // namespace

// tests/persistentkv_torch_extension.cu:35-93
void persistentkv_paged_attention(torch::Tensor q, torch::Tensor k_pages, torch::Tensor v_pages,
                                  torch::Tensor block_table, torch::Tensor output,
                                  torch::Tensor workspace, int64_t context, int64_t page_size,
                                  int64_t num_splits) {
  const auto dt = activation_dtype(q, "q");
  check_tensor(q, "q", dt, 3);
  check_tensor(k_pages, "k_pages", dt, 4);
  check_tensor(v_pages, "v_pages", dt, 4);
  check_tensor(block_table, "block_table", at::kInt, 2);
  check_tensor(output, "output", dt, 3);
  check_workspace(workspace);
  const int B = (int)q.size(0), Hq = (int)q.size(1), d = (int)q.size(2);
  const int Hkv = (int)k_pages.size(1);
  TORCH_CHECK(d == PKV_HEAD_DIM, "PersistentKV extension currently requires d=128");
  TORCH_CHECK(output.size(0) == B && output.size(1) == Hq && output.size(2) == d,
              "output shape must match q");
  check_pages(k_pages, v_pages, page_size, d);
  TORCH_CHECK(block_table.size(0) == B, "block_table batch mismatch");
  check_supported_gqa(Hq, Hkv);
  TORCH_CHECK(context > 0, "context must be positive");
  TORCH_CHECK(page_size > 0, "page_size must be positive");
  TORCH_CHECK(num_splits > 0, "num_splits must be positive");
  const c10::DeviceGuard guard(q.device());
  raise_on(pkv_paged_attention(
      q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
      output.data_ptr(), ws_ptr(workspace), ws_bytes(workspace), B, Hq, Hkv, d,
      i32(k_pages.size(0), "k_pages.size(0)"), i32(page_size, "page_size"),
      i32(block_table.size(1), "block_table.size(1)"), i32(context, "context"),
      i32(num_splits, "num_splits"), pkv_dtype_of(dt), stream_of(q)));
}

namespace {
void masked_op(torch::Tensor q, torch::Tensor k_pages, torch::Tensor v_pages,
               torch::Tensor block_table, torch::Tensor seq_lens, torch::Tensor output,
               torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
               int64_t num_splits, const torch::Tensor* k_new, const torch::Tensor* v_new);
}  // namespace

// tests/persistentkv_torch_extension.cu:95-157
void persistentkv_paged_attention_masked(torch::Tensor q, torch::Tensor k_pages,
                                         torch::Tensor v_pages, torch::Tensor block_table,
                                         torch::Tensor seq_lens, torch::Tensor output,
                                         torch::Tensor workspace, int64_t bucket_context,
                                         int64_t page_size, int64_t num_splits) {
  masked_op(q, k_pages, v_pages, block_table, seq_lens, output, workspace, bucket_context,
            page_size, num_splits, nullptr, nullptr);
}

// The masked op with the KV append fused in (as paged_attention_indexed_append).
void persistentkv_paged_attention_masked_append(
    torch::Tensor q, torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor block_table,
    torch::Tensor seq_lens, torch::Tensor output, torch::Tensor workspace,
    int64_t bucket_context, int64_t page_size, int64_t num_splits, torch::Tensor k_new,
    torch::Tensor v_new) {
  masked_op(q, k_pages, v_pages, block_table, seq_lens, output, workspace, bucket_context,
            page_size, num_splits, &k_new, &v_new);
}

namespace {
void check_new_token(const torch::Tensor& k_new, const torch::Tensor& v_new, at::ScalarType dt,
                     int64_t B, int64_t Hkv);

void masked_op(torch::Tensor q, torch::Tensor k_pages, torch::Tensor v_pages,
               torch::Tensor block_table, torch::Tensor seq_lens, torch::Tensor output,
               torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
               int64_t num_splits, const torch::Tensor* k_new, const torch::Tensor* v_new) {
  const auto dt = activation_dtype(q, "q");
  check_tensor(q, "q", dt, 3);
  check_tensor(k_pages, "k_pages", dt, 4);
  check_tensor(v_pages, "v_pages", dt, 4);
  check_tensor(block_table, "block_table", at::kInt, 2);
  check_tensor(seq_lens, "seq_lens", at::kInt, 1);
  check_tensor(output, "output", dt, 3);
  check_workspace(workspace);
  const int B = (int)q.size(0), Hq = (int)q.size(1), d = (int)q.size(2);
  const int Hkv = (int)k_pages.size(1);
  TORCH_CHECK(d == PKV_HEAD_DIM, "PersistentKV extension currently requires d=128");
  TORCH_CHECK(output.size(0) == B && output.size(1) == Hq && output.size(2) == d,
              "output shape must match q");
  TORCH_CHECK(seq_lens.size(0) == B, "seq_lens batch mismatch");
  check_pages(k_pages, v_pages, page_size, d);
  TORCH_CHECK(block_table.size(0) == B, "block_table batch mismatch");
  check_supported_gqa(Hq, Hkv);
  TORCH_CHECK(bucket_context > 0, "bucket_context must be positive");
  TORCH_CHECK(page_size > 0, "page_size must be positive");
  TORCH_CHECK(num_splits > 0, "num_splits must be positive");
  const c10::DeviceGuard guard(q.device());
  if (k_new) {
    check_new_token(*k_new, *v_new, dt, B, Hkv);
    raise_on(pkv_paged_attention_masked_append(
        q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), output.data_ptr(), ws_ptr(workspace), ws_bytes(workspace), B,
        Hq, Hkv, d, i32(k_pages.size(0), "k_pages.size(0)"), i32(page_size, "page_size"),
        i32(block_table.size(1), "block_table.size(1)"), i32(bucket_context, "bucket_context"),
        i32(num_splits, "num_splits"), k_new->data_ptr(), v_new->data_ptr(), pkv_dtype_of(dt),
        stream_of(q)));
    return;
  }
  raise_on(pkv_paged_attention_masked(
      q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
      seq_lens.data_ptr<int>(), output.data_ptr(), ws_ptr(workspace), ws_bytes(workspace), B, Hq,
      Hkv, d, i32(k_pages.size(0), "k_pages.size(0)"), i32(page_size, "page_size"),
      i32(block_table.size(1), "block_table.size(1)"), i32(bucket_context, "bucket_context"),
      i32(num_splits, "num_splits"), pkv_dtype_of(dt), stream_of(q)));
}
}  // namespace

namespace {

// Shared body of the indexed op and its fp8-K/V variant (kv_fp8: K/V are float8_e4m3fn
// pages dequantised by k_scale / v_scale).
// k_new / v_new of the *_append ops: each row's newest token, [B, Hkv, 128] in the
// activation dtype.
void check_new_token(const torch::Tensor& k_new, const torch::Tensor& v_new, at::ScalarType dt,
                     int64_t B, int64_t Hkv) {
  check_tensor(k_new, "k_new", dt, 3);
  check_tensor(v_new, "v_new", dt, 3);
  TORCH_CHECK(k_new.size(0) == B && k_new.size(1) == Hkv && k_new.size(2) == PKV_HEAD_DIM,
              "k_new must have shape [B, Hkv, 128]");
  TORCH_CHECK(v_new.sizes() == k_new.sizes(), "v_new shape mismatch");
}

void indexed_op(torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages,
                torch::Tensor block_table, torch::Tensor seq_lens, torch::Tensor q_indices,
                torch::Tensor out_indices, torch::Tensor output, torch::Tensor workspace,
                int64_t bucket_context, int64_t page_size, int64_t num_splits, bool kv_fp8,
                double k_scale, double v_scale, const torch::Tensor* k_new = nullptr,
                const torch::Tensor* v_new = nullptr) {
  const auto dt = activation_dtype(q_source, "q_source");
  const auto kv_dt = kv_fp8 ? at::kFloat8_e4m3fn : dt;
  check_tensor(q_source, "q_source", dt, 3);
  check_tensor(k_pages, "k_pages", kv_dt, 4);
  check_tensor(v_pages, "v_pages", kv_dt, 4);
  check_tensor(block_table, "block_table", at::kInt, 2);
  check_tensor(seq_lens, "seq_lens", at::kInt, 1);
  check_tensor(q_indices, "q_indices", at::kInt, 1);
  check_tensor(out_indices, "out_indices", at::kInt, 1);
  check_tensor(output, "output", dt, 3);
  check_workspace(workspace);
  const int B = (int)block_table.size(0), Hq = (int)q_source.size(1), d = (int)q_source.size(2);
  const int Hkv = (int)k_pages.size(1);
  TORCH_CHECK(d == PKV_HEAD_DIM, "PersistentKV extension currently requires d=128");
  TORCH_CHECK(output.size(1) == Hq && output.size(2) == d,
              "output shape must match q head dimensions");
  TORCH_CHECK(seq_lens.size(0) == B, "seq_lens batch mismatch");
  TORCH_CHECK(q_indices.size(0) == B, "q_indices batch mismatch");
  TORCH_CHECK(out_indices.size(0) == B, "out_indices batch mismatch");
  check_pages(k_pages, v_pages, page_size, d);
  check_supported_gqa(Hq, Hkv);
  TORCH_CHECK(bucket_context > 0, "bucket_context must be positive");
  TORCH_CHECK(page_size > 0, "page_size must be positive");
  TORCH_CHECK(num_splits > 0, "num_splits must be positive");
  const c10::DeviceGuard guard(q_source.device());
  const int32_t nq = i32(q_source.size(0), "q_source.size(0)");
  const int32_t no = i32(output.size(0), "output.size(0)");
  const int32_t np = i32(k_pages.size(0), "k_pages.size(0)");
  const int32_t mp = i32(block_table.size(1), "block_table.size(1)");
  if (k_new && kv_fp8) {
    check_new_token(*k_new, *v_new, dt, B, Hkv);
    raise_on(pkv_paged_attention_indexed_fp8_append(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), q_indices.data_ptr<int>(), out_indices.data_ptr<int>(),
        output.data_ptr(), no, ws_ptr(workspace), ws_bytes(workspace), B, Hq, Hkv, d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(num_splits, "num_splits"), (float)k_scale, (float)v_scale, k_new->data_ptr(),
        v_new->data_ptr(), pkv_dtype_of(dt), stream_of(q_source)));
  } else if (k_new) {
    check_new_token(*k_new, *v_new, dt, B, Hkv);
    raise_on(pkv_paged_attention_indexed_append(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), q_indices.data_ptr<int>(), out_indices.data_ptr<int>(),
        output.data_ptr(), no, ws_ptr(workspace), ws_bytes(workspace), B, Hq, Hkv, d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(num_splits, "num_splits"), k_new->data_ptr(), v_new->data_ptr(), pkv_dtype_of(dt),
        stream_of(q_source)));
  } else if (kv_fp8)
    raise_on(pkv_paged_attention_indexed_fp8(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), q_indices.data_ptr<int>(), out_indices.data_ptr<int>(),
        output.data_ptr(), no, ws_ptr(workspace), ws_bytes(workspace), B, Hq, Hkv, d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(num_splits, "num_splits"), (float)k_scale, (float)v_scale, pkv_dtype_of(dt),
        stream_of(q_source)));
  else
    raise_on(pkv_paged_attention_indexed(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), q_indices.data_ptr<int>(), out_indices.data_ptr<int>(),
        output.data_ptr(), no, ws_ptr(workspace), ws_bytes(workspace), B, Hq, Hkv, d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(num_splits, "num_splits"), pkv_dtype_of(dt), stream_of(q_source)));
}

}  // namespace

// tests/persistentkv_torch_extension.cu:159-228
void persistentkv_paged_attention_indexed(torch::Tensor q_source, torch::Tensor k_pages,
                                          torch::Tensor v_pages, torch::Tensor block_table,
                                          torch::Tensor seq_lens, torch::Tensor q_indices,
                                          torch::Tensor out_indices, torch::Tensor output,
                                          torch::Tensor workspace, int64_t bucket_context,
                                          int64_t page_size, int64_t num_splits) {
  indexed_op(q_source, k_pages, v_pages, block_table, seq_lens, q_indices, out_indices, output,
             workspace, bucket_context, page_size, num_splits, false, 1.0, 1.0);
}

// The indexed op over fp8 (float8_e4m3fn) K/V pages: K = k_scale * k8, V = v_scale * v8.
void persistentkv_paged_attention_indexed_fp8(torch::Tensor q_source, torch::Tensor k_pages,
                                              torch::Tensor v_pages, torch::Tensor block_table,
                                              torch::Tensor seq_lens, torch::Tensor q_indices,
                                              torch::Tensor out_indices, torch::Tensor output,
                                              torch::Tensor workspace, int64_t bucket_context,
                                              int64_t page_size, int64_t num_splits,
                                              double k_scale, double v_scale) {
  indexed_op(q_source, k_pages, v_pages, block_table, seq_lens, q_indices, out_indices, output,
             workspace, bucket_context, page_size, num_splits, true, k_scale, v_scale);
}

// The indexed op with the KV append fused in: equals append_kv(k_new, v_new, k_pages,
// v_pages, block_table, seq_lens) followed by paged_attention_indexed (2-byte pools).
void persistentkv_paged_attention_indexed_append(
    torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor block_table,
    torch::Tensor seq_lens, torch::Tensor q_indices, torch::Tensor out_indices,
    torch::Tensor output, torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
    int64_t num_splits, torch::Tensor k_new, torch::Tensor v_new) {
  indexed_op(q_source, k_pages, v_pages, block_table, seq_lens, q_indices, out_indices, output,
             workspace, bucket_context, page_size, num_splits, false, 1.0, 1.0, &k_new, &v_new);
}

namespace {

struct QueueTensors {
  int B, Hq, Hkv, d;
  at::ScalarType dt;
};

QueueTensors check_queue_tensors(const torch::Tensor& q_source, const torch::Tensor& k_pages,
                                 const torch::Tensor& v_pages, const torch::Tensor& block_table,
                                 const torch::Tensor& seq_lens, const torch::Tensor& work_items,
                                 const torch::Tensor& split_offsets, const torch::Tensor& q_indices,
                                 const torch::Tensor& workspace, int64_t bucket_context,
                                 int64_t page_size, int64_t total_partial_slots,
                                 bool kv_fp8 = false) {
  QueueTensors t;
  t.dt = activation_dtype(q_source, "q_source");
  const auto kv_dt = kv_fp8 ? at::kFloat8_e4m3fn : t.dt;
  check_tensor(q_source, "q_source", t.dt, 3);
  check_tensor(k_pages, "k_pages", kv_dt, 4);
  check_tensor(v_pages, "v_pages", kv_dt, 4);
  check_tensor(block_table, "block_table", at::kInt, 2);
  check_tensor(seq_lens, "seq_lens", at::kInt, 1);
  check_tensor(work_items, "work_items", at::kInt, 2);
  check_tensor(split_offsets, "split_offsets", at::kInt, 1);
  check_tensor(q_indices, "q_indices", at::kInt, 1);
  check_workspace(workspace);
  t.B = (int)block_table.size(0);
  t.Hq = (int)q_source.size(1);
  t.d = (int)q_source.size(2);
  t.Hkv = (int)k_pages.size(1);
  TORCH_CHECK(t.d == PKV_HEAD_DIM, "PersistentKV extension currently requires d=128");
  TORCH_CHECK(work_items.size(1) == 5, "work_items must have shape [T, 5]");
  TORCH_CHECK(split_offsets.size(0) == t.B + 1, "split_offsets batch mismatch");
  TORCH_CHECK(seq_lens.size(0) == t.B, "seq_lens batch mismatch");
  TORCH_CHECK(q_indices.size(0) == t.B, "q_indices batch mismatch");
  check_pages(k_pages, v_pages, page_size, t.d);
  check_supported_gqa(t.Hq, t.Hkv);
  TORCH_CHECK(bucket_context > 0, "bucket_context must be positive");
  TORCH_CHECK(page_size > 0, "page_size must be positive");
  TORCH_CHECK(work_items.size(0) > 0, "work_items must not be empty");
  TORCH_CHECK(total_partial_slots > 0, "total_partial_slots must be positive");
  return t;
}

}  // namespace

namespace {

// Shared body of the work-queue op and its fp8-K/V variant.
void workqueue_op(torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages,
                  torch::Tensor block_table, torch::Tensor seq_lens, torch::Tensor work_items,
                  torch::Tensor split_offsets, torch::Tensor merge_counters,
                  torch::Tensor q_indices, torch::Tensor out_indices, torch::Tensor output,
                  torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
                  int64_t total_partial_slots, bool fused_merge, bool kv_fp8, double k_scale,
                  double v_scale, const torch::Tensor* k_new = nullptr,
                  const torch::Tensor* v_new = nullptr) {
  const QueueTensors t = check_queue_tensors(q_source, k_pages, v_pages, block_table, seq_lens,
                                             work_items, split_offsets, q_indices, workspace,
                                             bucket_context, page_size, total_partial_slots,
                                             kv_fp8);
  check_tensor(merge_counters, "merge_counters", at::kInt, 2);
  check_tensor(out_indices, "out_indices", at::kInt, 1);
  check_tensor(output, "output", t.dt, 3);
  TORCH_CHECK(merge_counters.size(0) == t.B && merge_counters.size(1) == t.Hkv,
              "merge_counters shape mismatch");
  TORCH_CHECK(output.size(1) == t.Hq && output.size(2) == t.d,
              "output shape must match q head dimensions");
  TORCH_CHECK(out_indices.size(0) == t.B, "out_indices batch mismatch");
  const c10::DeviceGuard guard(q_source.device());
  const int32_t nq = i32(q_source.size(0), "q_source.size(0)");
  const int32_t nt = i32(work_items.size(0), "work_items.size(0)");
  const int32_t no = i32(output.size(0), "output.size(0)");
  const int32_t np = i32(k_pages.size(0), "k_pages.size(0)");
  const int32_t mp = i32(block_table.size(1), "block_table.size(1)");
  int32_t* counters = fused_merge ? merge_counters.data_ptr<int>() : nullptr;
  if (k_new && kv_fp8) {
    check_new_token(*k_new, *v_new, t.dt, t.B, t.Hkv);
    raise_on(pkv_paged_attention_workqueue_fp8_append(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), work_items.data_ptr<int>(), nt, split_offsets.data_ptr<int>(),
        counters, q_indices.data_ptr<int>(), out_indices.data_ptr<int>(), output.data_ptr(), no,
        ws_ptr(workspace), ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(total_partial_slots, "total_partial_slots"), fused_merge ? 1 : 0, (float)k_scale,
        (float)v_scale, k_new->data_ptr(), v_new->data_ptr(), pkv_dtype_of(t.dt),
        stream_of(q_source)));
  } else if (k_new) {
    check_new_token(*k_new, *v_new, t.dt, t.B, t.Hkv);
    raise_on(pkv_paged_attention_workqueue_append(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), work_items.data_ptr<int>(), nt, split_offsets.data_ptr<int>(),
        counters, q_indices.data_ptr<int>(), out_indices.data_ptr<int>(), output.data_ptr(), no,
        ws_ptr(workspace), ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(total_partial_slots, "total_partial_slots"), fused_merge ? 1 : 0, k_new->data_ptr(),
        v_new->data_ptr(), pkv_dtype_of(t.dt), stream_of(q_source)));
  } else if (kv_fp8)
    raise_on(pkv_paged_attention_workqueue_fp8(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), work_items.data_ptr<int>(), nt, split_offsets.data_ptr<int>(),
        counters, q_indices.data_ptr<int>(), out_indices.data_ptr<int>(), output.data_ptr(), no,
        ws_ptr(workspace), ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(total_partial_slots, "total_partial_slots"), fused_merge ? 1 : 0, (float)k_scale,
        (float)v_scale, pkv_dtype_of(t.dt), stream_of(q_source)));
  else
    raise_on(pkv_paged_attention_workqueue(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), work_items.data_ptr<int>(), nt, split_offsets.data_ptr<int>(),
        counters, q_indices.data_ptr<int>(), out_indices.data_ptr<int>(), output.data_ptr(), no,
        ws_ptr(workspace), ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.d, np,
        i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(total_partial_slots, "total_partial_slots"), fused_merge ? 1 : 0, pkv_dtype_of(t.dt),
        stream_of(q_source)));
}

}  // namespace

// tests/persistentkv_torch_extension.cu:230-317
void persistentkv_paged_attention_workqueue(
    torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor block_table,
    torch::Tensor seq_lens, torch::Tensor work_items, torch::Tensor split_offsets,
    torch::Tensor merge_counters, torch::Tensor q_indices, torch::Tensor out_indices,
    torch::Tensor output, torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
    int64_t total_partial_slots, bool fused_merge) {
  workqueue_op(q_source, k_pages, v_pages, block_table, seq_lens, work_items, split_offsets,
               merge_counters, q_indices, out_indices, output, workspace, bucket_context,
               page_size, total_partial_slots, fused_merge, false, 1.0, 1.0);
}

// The work-queue op over fp8 (float8_e4m3fn) K/V pages: K = k_scale * k8, V = v_scale * v8.
void persistentkv_paged_attention_workqueue_fp8(
    torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor block_table,
    torch::Tensor seq_lens, torch::Tensor work_items, torch::Tensor split_offsets,
    torch::Tensor merge_counters, torch::Tensor q_indices, torch::Tensor out_indices,
    torch::Tensor output, torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
    int64_t total_partial_slots, bool fused_merge, double k_scale, double v_scale) {
  workqueue_op(q_source, k_pages, v_pages, block_table, seq_lens, work_items, split_offsets,
               merge_counters, q_indices, out_indices, output, workspace, bucket_context,
               page_size, total_partial_slots, fused_merge, true, k_scale, v_scale);
}

// The fp8-K/V indexed op with the append fused in: equals append_kv_fp8(k_new, v_new, ...,
// k_scale, v_scale) followed by paged_attention_indexed_fp8.
void persistentkv_paged_attention_indexed_fp8_append(
    torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor block_table,
    torch::Tensor seq_lens, torch::Tensor q_indices, torch::Tensor out_indices,
    torch::Tensor output, torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
    int64_t num_splits, double k_scale, double v_scale, torch::Tensor k_new, torch::Tensor v_new) {
  indexed_op(q_source, k_pages, v_pages, block_table, seq_lens, q_indices, out_indices, output,
             workspace, bucket_context, page_size, num_splits, true, k_scale, v_scale, &k_new,
             &v_new);
}

// The work-queue op with the KV append fused in (as paged_attention_indexed_append).
void persistentkv_paged_attention_workqueue_append(
    torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor block_table,
    torch::Tensor seq_lens, torch::Tensor work_items, torch::Tensor split_offsets,
    torch::Tensor merge_counters, torch::Tensor q_indices, torch::Tensor out_indices,
    torch::Tensor output, torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
    int64_t total_partial_slots, bool fused_merge, torch::Tensor k_new, torch::Tensor v_new) {
  workqueue_op(q_source, k_pages, v_pages, block_table, seq_lens, work_items, split_offsets,
               merge_counters, q_indices, out_indices, output, workspace, bucket_context,
               page_size, total_partial_slots, fused_merge, false, 1.0, 1.0, &k_new, &v_new);
}

// The fp8-K/V work-queue op with the KV append fused in.
void persistentkv_paged_attention_workqueue_fp8_append(
    torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor block_table,
    torch::Tensor seq_lens, torch::Tensor work_items, torch::Tensor split_offsets,
    torch::Tensor merge_counters, torch::Tensor q_indices, torch::Tensor out_indices,
    torch::Tensor output, torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
    int64_t total_partial_slots, bool fused_merge, double k_scale, double v_scale,
    torch::Tensor k_new, torch::Tensor v_new) {
  workqueue_op(q_source, k_pages, v_pages, block_table, seq_lens, work_items, split_offsets,
               merge_counters, q_indices, out_indices, output, workspace, bucket_context,
               page_size, total_partial_slots, fused_merge, true, k_scale, v_scale, &k_new, &v_new);
}

namespace {

void queue_decode_op(torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages,
                     torch::Tensor block_table, torch::Tensor seq_lens, torch::Tensor work_items,
                     torch::Tensor split_offsets, torch::Tensor q_indices, torch::Tensor workspace,
                     int64_t bucket_context, int64_t page_size, int64_t total_partial_slots,
                     bool kv_fp8, double k_scale, double v_scale) {
  const QueueTensors t = check_queue_tensors(q_source, k_pages, v_pages, block_table, seq_lens,
                                             work_items, split_offsets, q_indices, workspace,
                                             bucket_context, page_size, total_partial_slots,
                                             kv_fp8);
  const c10::DeviceGuard guard(q_source.device());
  const int32_t nq = i32(q_source.size(0), "q_source.size(0)");
  const int32_t nt = i32(work_items.size(0), "work_items.size(0)");
  const int32_t np = i32(k_pages.size(0), "k_pages.size(0)");
  const int32_t mp = i32(block_table.size(1), "block_table.size(1)");
  if (kv_fp8)
    raise_on(pkv_workqueue_decode_fp8(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), work_items.data_ptr<int>(), nt, split_offsets.data_ptr<int>(),
        q_indices.data_ptr<int>(), ws_ptr(workspace), ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.d,
        np, i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(total_partial_slots, "total_partial_slots"), (float)k_scale, (float)v_scale,
        pkv_dtype_of(t.dt), stream_of(q_source)));
  else
    raise_on(pkv_workqueue_decode(
        q_source.data_ptr(), nq, k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(),
        seq_lens.data_ptr<int>(), work_items.data_ptr<int>(), nt, split_offsets.data_ptr<int>(),
        q_indices.data_ptr<int>(), ws_ptr(workspace), ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.d,
        np, i32(page_size, "page_size"), mp, i32(bucket_context, "bucket_context"),
        i32(total_partial_slots, "total_partial_slots"), pkv_dtype_of(t.dt), stream_of(q_source)));
}

}  // namespace

// Stage 1 of the work-queue op: the decode kernel alone, writing partial states.
void persistentkv_workqueue_decode(torch::Tensor q_source, torch::Tensor k_pages,
                                   torch::Tensor v_pages, torch::Tensor block_table,
                                   torch::Tensor seq_lens, torch::Tensor work_items,
                                   torch::Tensor split_offsets, torch::Tensor q_indices,
                                   torch::Tensor workspace, int64_t bucket_context,
                                   int64_t page_size, int64_t total_partial_slots) {
  queue_decode_op(q_source, k_pages, v_pages, block_table, seq_lens, work_items, split_offsets,
                  q_indices, workspace, bucket_context, page_size, total_partial_slots, false,
                  1.0, 1.0);
}

// Stage 1 over fp8 K/V.
void persistentkv_workqueue_decode_fp8(torch::Tensor q_source, torch::Tensor k_pages,
                                       torch::Tensor v_pages, torch::Tensor block_table,
                                       torch::Tensor seq_lens, torch::Tensor work_items,
                                       torch::Tensor split_offsets, torch::Tensor q_indices,
                                       torch::Tensor workspace, int64_t bucket_context,
                                       int64_t page_size, int64_t total_partial_slots,
                                       double k_scale, double v_scale) {
  queue_decode_op(q_source, k_pages, v_pages, block_table, seq_lens, work_items, split_offsets,
                  q_indices, workspace, bucket_context, page_size, total_partial_slots, true,
                  k_scale, v_scale);
}

// Stage 2 of the work-queue op: the segmented LSE merge alone.
void persistentkv_workqueue_merge(torch::Tensor seq_lens, torch::Tensor split_offsets,
                                  torch::Tensor out_indices, torch::Tensor output,
                                  torch::Tensor workspace, int64_t total_partial_slots,
                                  int64_t num_tasks, int64_t num_kv_heads) {
  const auto dt = activation_dtype(output, "output");
  check_tensor(seq_lens, "seq_lens", at::kInt, 1);
  check_tensor(split_offsets, "split_offsets", at::kInt, 1);
  check_tensor(out_indices, "out_indices", at::kInt, 1);
  check_tensor(output, "output", dt, 3);
  check_workspace(workspace);
  const int B = (int)seq_lens.size(0);
  TORCH_CHECK(split_offsets.size(0) == B + 1, "split_offsets batch mismatch");
  TORCH_CHECK(out_indices.size(0) == B, "out_indices batch mismatch");
  TORCH_CHECK(output.size(2) == PKV_HEAD_DIM, "PersistentKV extension currently requires d=128");
  const c10::DeviceGuard guard(output.device());
  raise_on(pkv_workqueue_merge(
      seq_lens.data_ptr<int>(), split_offsets.data_ptr<int>(), out_indices.data_ptr<int>(),
      output.data_ptr(), i32(output.size(0), "output.size(0)"), ws_ptr(workspace),
      ws_bytes(workspace), B, i32(output.size(1), "output.size(1)"),
      i32(total_partial_slots, "total_partial_slots"), i32(num_tasks, "num_tasks"),
      i32(num_kv_heads, "num_kv_heads"), pkv_dtype_of(dt), stream_of(output)));
}

namespace {

struct ContiguousShape {
  at::ScalarType dt;
  int32_t B, Hq, Hkv, N;
};

ContiguousShape check_contiguous(const torch::Tensor& q, const torch::Tensor& k,
                                 const torch::Tensor& v, const torch::Tensor& output) {
  const auto dt = activation_dtype(q, "q");
  check_tensor(q, "q", dt, 3);
  check_tensor(k, "k", dt, 4);
  check_tensor(v, "v", dt, 4);
  check_tensor(output, "output", dt, 3);
  TORCH_CHECK(q.size(2) == PKV_HEAD_DIM && k.size(3) == PKV_HEAD_DIM,
              "PersistentKV extension currently requires d=128");
  TORCH_CHECK(k.size(0) == q.size(0), "k batch mismatch");
  TORCH_CHECK(v.sizes() == k.sizes(), "v shape mismatch");
  TORCH_CHECK(output.sizes() == q.sizes(), "output shape must match q");
  const int32_t Hq = i32(q.size(1), "q.size(1)"), Hkv = i32(k.size(1), "k.size(1)");
  check_supported_gqa(Hq, Hkv);
  return {dt, i32(q.size(0), "q.size(0)"), Hq, Hkv, i32(k.size(2), "k.size(2)")};
}

}  // namespace

// Contiguous-layout decode: q [B, Hq, 128], k / v [B, Hkv, N, 128] (the reference's C++
// entry points persistentkv_dispatch and persistentkv_split_dispatch, cuh:1077-1108).
void persistentkv_attention_contiguous(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                       torch::Tensor output, torch::Tensor workspace,
                                       int64_t num_splits) {
  const ContiguousShape t = check_contiguous(q, k, v, output);
  check_workspace(workspace);
  const c10::DeviceGuard guard(q.device());
  raise_on(pkv_attention_contiguous(q.data_ptr(), k.data_ptr(), v.data_ptr(), output.data_ptr(),
                                    ws_ptr(workspace), ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.N,
                                    PKV_HEAD_DIM, i32(num_splits, "num_splits"), pkv_dtype_of(t.dt),
                                    stream_of(q)));
}

// Query-head baseline over contiguous K/V (persistentkv_baseline_dispatch, cuh:1263-1282).
void persistentkv_attention_query_head_baseline(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                                torch::Tensor output) {
  const ContiguousShape t = check_contiguous(q, k, v, output);
  const c10::DeviceGuard guard(q.device());
  raise_on(pkv_attention_query_head_baseline(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             output.data_ptr(), t.B, t.Hq, t.Hkv, t.N, PKV_HEAD_DIM,
                                             pkv_dtype_of(t.dt), stream_of(q)));
}

namespace {

// KV-cache append (no counterpart in the reference): row b's k_new[b], v_new[b]
// ([Hkv, 128]) go to token position seq_lens[b] - 1 of its block-table row.
void append_op(const torch::Tensor& k_new, const torch::Tensor& v_new, torch::Tensor& k_pages,
               torch::Tensor& v_pages, const torch::Tensor& block_table,
               const torch::Tensor& seq_lens, bool kv_fp8, double k_scale, double v_scale) {
  const auto dt = activation_dtype(k_new, "k_new");
  check_tensor(k_new, "k_new", dt, 3);
  check_tensor(v_new, "v_new", dt, 3);
  const auto kv_dt = kv_fp8 ? at::kFloat8_e4m3fn : dt;
  check_tensor(k_pages, "k_pages", kv_dt, 4);
  check_tensor(v_pages, "v_pages", kv_dt, 4);
  check_tensor(block_table, "block_table", at::kInt, 2);
  check_tensor(seq_lens, "seq_lens", at::kInt, 1);
  const int64_t B = k_new.size(0), Hkv = k_new.size(1);
  TORCH_CHECK(k_new.size(2) == PKV_HEAD_DIM, "PersistentKV extension currently requires d=128");
  TORCH_CHECK(v_new.sizes() == k_new.sizes(), "v_new shape mismatch");
  TORCH_CHECK(k_pages.size(1) == Hkv, "k_pages Hkv mismatch");
  check_pages(k_pages, v_pages, k_pages.size(2), PKV_HEAD_DIM);
  TORCH_CHECK(block_table.size(0) == B && seq_lens.size(0) == B, "batch size mismatch");
  const c10::DeviceGuard guard(k_pages.device());
  const int32_t batch = i32(B, "k_new.size(0)"), hkv = i32(Hkv, "Hkv");
  const int32_t pages = i32(k_pages.size(0), "k_pages.size(0)");
  const int32_t ps = i32(k_pages.size(2), "page_size"), cols = i32(block_table.size(1), "max_pages");
  if (kv_fp8)
    raise_on(pkv_append_kv_fp8(k_new.data_ptr(), v_new.data_ptr(), k_pages.data_ptr(),
                               v_pages.data_ptr(), block_table.data_ptr<int>(),
                               seq_lens.data_ptr<int>(), batch, hkv, PKV_HEAD_DIM, pages, ps, cols,
                               (float)k_scale, (float)v_scale, pkv_dtype_of(dt), stream_of(k_pages)));
  else
    raise_on(pkv_append_kv(k_new.data_ptr(), v_new.data_ptr(), k_pages.data_ptr(),
                           v_pages.data_ptr(), block_table.data_ptr<int>(), seq_lens.data_ptr<int>(),
                           batch, hkv, PKV_HEAD_DIM, pages, ps, cols, pkv_dtype_of(dt),
                           stream_of(k_pages)));
}

}  // namespace

void persistentkv_append_kv(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor k_pages,
                            torch::Tensor v_pages, torch::Tensor block_table,
                            torch::Tensor seq_lens) {
  append_op(k_new, v_new, k_pages, v_pages, block_table, seq_lens, false, 1.0, 1.0);
}

void persistentkv_append_kv_fp8(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor k_pages,
                                torch::Tensor v_pages, torch::Tensor block_table,
                                torch::Tensor seq_lens, double k_scale, double v_scale) {
  append_op(k_new, v_new, k_pages, v_pages, block_table, seq_lens, true, k_scale, v_scale);
}

// One stage of the work-queue op (1 = decode, 2 = merge) in the schedule the combined op
// takes for these tensors; kv_fp8 selects float8_e4m3fn pages with k_scale / v_scale.
void persistentkv_paged_attention_workqueue_stage(
    int64_t stage, torch::Tensor q_source, torch::Tensor k_pages, torch::Tensor v_pages,
    torch::Tensor block_table, torch::Tensor seq_lens, torch::Tensor work_items,
    torch::Tensor split_offsets, torch::Tensor q_indices, torch::Tensor out_indices,
    torch::Tensor output, torch::Tensor workspace, int64_t bucket_context, int64_t page_size,
    int64_t total_partial_slots, bool kv_fp8, double k_scale, double v_scale) {
  const QueueTensors t = check_queue_tensors(q_source, k_pages, v_pages, block_table, seq_lens,
                                             work_items, split_offsets, q_indices, workspace,
                                             bucket_context, page_size, total_partial_slots,
                                             kv_fp8);
  check_tensor(out_indices, "out_indices", at::kInt, 1);
  check_tensor(output, "output", t.dt, 3);
  TORCH_CHECK(output.size(1) == t.Hq && output.size(2) == t.d,
              "output shape must match q head dimensions");
  TORCH_CHECK(out_indices.size(0) == t.B, "out_indices batch mismatch");
  const c10::DeviceGuard guard(q_source.device());
  raise_on(pkv_paged_attention_workqueue_stage(
      i32(stage, "stage"), q_source.data_ptr(), i32(q_source.size(0), "q_source.size(0)"),
      k_pages.data_ptr(), v_pages.data_ptr(), block_table.data_ptr<int>(), seq_lens.data_ptr<int>(),
      work_items.data_ptr<int>(), i32(work_items.size(0), "work_items.size(0)"),
      split_offsets.data_ptr<int>(), q_indices.data_ptr<int>(), out_indices.data_ptr<int>(),
      output.data_ptr(), i32(output.size(0), "output.size(0)"), ws_ptr(workspace),
      ws_bytes(workspace), t.B, t.Hq, t.Hkv, t.d, i32(k_pages.size(0), "k_pages.size(0)"),
      i32(page_size, "page_size"), i32(block_table.size(1), "block_table.size(1)"),
      i32(bucket_context, "bucket_context"), i32(total_partial_slots, "total_partial_slots"),
      kv_fp8 ? 1 : 0, (float)k_scale, (float)v_scale, pkv_dtype_of(t.dt), stream_of(q_source)));
}

int64_t persistentkv_workqueue_schedule(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                        int64_t page_size, int64_t workspace_floats,
                                        bool fused_merge) {
  TORCH_CHECK(workspace_floats >= 0, "workspace_floats must be non-negative");
  return pkv_workqueue_schedule(i32(batch, "batch"), i32(num_q_heads, "Hq"),
                                i32(num_kv_heads, "Hkv"), i32(page_size, "page_size"),
                                (size_t)workspace_floats * sizeof(float), fused_merge ? 1 : 0);
}

int64_t persistentkv_direct_workspace_floats(int64_t batch, int64_t num_q_heads,
                                             int64_t num_kv_heads, int64_t context) {
  return (int64_t)(pkv_direct_workspace_bytes(i32(batch, "batch"), i32(num_q_heads, "Hq"),
                                              i32(num_kv_heads, "Hkv"), i32(context, "context")) /
                   sizeof(float));
}

int64_t persistentkv_split_workspace_floats(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                            int64_t context, int64_t num_splits) {
  return (int64_t)(pkv_split_workspace_bytes(i32(batch, "batch"), i32(num_q_heads, "Hq"),
                                             i32(num_kv_heads, "Hkv"), i32(context, "context"),
                                             i32(num_splits, "num_splits")) /
                   sizeof(float));
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("paged_attention_workqueue_stage", &persistentkv_paged_attention_workqueue_stage,
        "one stage (1 decode, 2 merge) of paged_attention_workqueue in the schedule it takes");
  m.def("workqueue_schedule", &persistentkv_workqueue_schedule,
        "1 when paged_attention_workqueue takes the balanced schedule for these sizes, else 0");
  m.def("direct_workspace_floats", &persistentkv_direct_workspace_floats,
        "fp32 workspace elements with which a num_splits == 1 launch runs its full internal split");
  m.def("split_workspace_floats", &persistentkv_split_workspace_floats,
        "fp32 workspace elements with which a num_splits > 1 launch of few units runs its full "
        "internal sub-split");
  m.def("paged_attention", &persistentkv_paged_attention, "PersistentKV native paged attention");
  m.def("paged_attention_masked", &persistentkv_paged_attention_masked,
        "PersistentKV native paged attention with per-request sequence lengths");
  m.def("paged_attention_indexed", &persistentkv_paged_attention_indexed,
        "PersistentKV native paged attention with indexed Q/O rows");
  m.def("paged_attention_workqueue", &persistentkv_paged_attention_workqueue,
        "PersistentKV native paged attention with compact work queue");
  m.def("workqueue_decode", &persistentkv_workqueue_decode,
        "Work-queue decode stage only (partial states into the workspace)");
  m.def("workqueue_merge", &persistentkv_workqueue_merge,
        "Work-queue segmented LSE merge stage only (num_tasks = work_items.size(0), or -1 "
        "for a builder queue of unknown size)",
        py::arg("seq_lens"), py::arg("split_offsets"), py::arg("out_indices"), py::arg("output"),
        py::arg("workspace"), py::arg("total_partial_slots"), py::arg("num_tasks") = -1,
        py::arg("num_kv_heads") = 0);
  m.def("paged_attention_indexed_fp8", &persistentkv_paged_attention_indexed_fp8,
        "paged_attention_indexed over fp8 (e4m3) K/V pages with per-tensor scales");
  m.def("paged_attention_workqueue_fp8", &persistentkv_paged_attention_workqueue_fp8,
        "paged_attention_workqueue over fp8 (e4m3) K/V pages with per-tensor scales");
  m.def("workqueue_decode_fp8", &persistentkv_workqueue_decode_fp8,
        "Work-queue decode stage over fp8 (e4m3) K/V pages");
  m.def("attention_contiguous", &persistentkv_attention_contiguous,
        "GQA decode over contiguous K/V [B, Hkv, N, 128]");
  m.def("paged_attention_masked_append", &persistentkv_paged_attention_masked_append,
        "paged_attention_masked with the KV append fused in (k_new, v_new)");
  m.def("paged_attention_indexed_append", &persistentkv_paged_attention_indexed_append,
        "paged_attention_indexed with the KV append fused in (k_new, v_new)");
  m.def("paged_attention_workqueue_append", &persistentkv_paged_attention_workqueue_append,
        "paged_attention_workqueue with the KV append fused in (k_new, v_new)");
  m.def("paged_attention_indexed_fp8_append", &persistentkv_paged_attention_indexed_fp8_append,
        "paged_attention_indexed_fp8 with the KV append fused in (k_new, v_new)");
  m.def("paged_attention_workqueue_fp8_append", &persistentkv_paged_attention_workqueue_fp8_append,
        "paged_attention_workqueue_fp8 with the KV append fused in (k_new, v_new)");
  m.def("append_kv", &persistentkv_append_kv,
        "write each row's newest token's K/V into its tail page (position seq_lens - 1)");
  m.def("append_kv_fp8", &persistentkv_append_kv_fp8,
        "append_kv into float8_e4m3fn pools, quantising x / scale with round-to-nearest-even");
  m.def("attention_query_head_baseline", &persistentkv_attention_query_head_baseline,
        "Query-head baseline over contiguous K/V (each query head streams its KV head)");
}
