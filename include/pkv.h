/*
 * pkv.h — C ABI of the MI355X (gfx950) PersistentKV paged decode-attention engine.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream passed as
 * `void*` (a hipStream_t; NULL selects the null stream).  Outputs, the split workspace
 * and the merge counters are owned by the caller, exactly as in the reference op surface,
 * and the library allocates no device memory.  A direct launch (num_splits == 1) of fewer
 * than 128 (row, kv head) pairs splits itself internally when the caller's workspace can
 * hold the partial states (pkv_direct_workspace_bytes gives the size for the full split;
 * a smaller or empty workspace gives a smaller split or the single launch, with the same
 * result to fp32 rounding; PKV_DIRECT_SPLIT=0 in the environment turns this off).  Calls
 * enqueue work asynchronously and never synchronise the host.
 * Errors are reported as a pkv_status code; a one-line message describing the last
 * failure on the calling thread is available from pkv_last_error().
 *
 * Layouts (all row-major, contiguous):
 *   q / q_source   [rows, num_q_heads, 128]                   fp16 or bf16
 *   k_pages/v_pages[num_pages, num_kv_heads, page_size, 128]  same dtype as q (fp8 e4m3
 *                                                             for the *_fp8 entries)
 *   block_table    [batch, max_pages]                         int32 physical page ids
 *   seq_lens       [batch]                                    int32 tokens per row
 *   output         [out_rows, num_q_heads, 128]               same dtype as q
 *   work_items     [num_tasks, 5] int32 = {row, kv_head, split, tile_begin, tile_end}
 *                  (tiles are 32-token units, independent of page_size)
 *   split_offsets  [batch + 1]                                int32 prefix sum of row splits
 *   merge_counters [batch, num_kv_heads]                      int32, zero on entry and exit
 *   workspace      fp32 [m: n][l: n][acc: n x 128] with n = batch*num_q_heads*num_splits
 *                  (grid split) or total_partial_slots*num_q_heads (work queue),
 *                  16-byte aligned (as any torch allocation is; others are rejected).
 *
 * Query head h reads KV head h / G with G = num_q_heads / num_kv_heads.  The softmax
 * scale is fixed at 1/sqrt(128).  G may be any integer in [1, 32]; the reference accepts
 * only {1, 2, 4, 8}.  Reference citations are into ahmed123hds/persistentkv-attention.
 */
#ifndef PKV_H_
#define PKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_HEAD_DIM 128     /* kernels/persistentkv_attention.cuh:26 (PKV_D) */
#define PKV_TILE_TOKENS 32   /* kernels/persistentkv_attention.cuh:28 (PKV_TILE) */
#define PKV_MAX_GROUP 32     /* largest supported Hq / Hkv */

typedef enum pkv_status {
  PKV_OK = 0,
  PKV_ERR_INVALID_ARGUMENT = 1,  /* a shape, pointer or size is inconsistent */
  PKV_ERR_UNSUPPORTED = 2,       /* a valid request this build does not implement */
  PKV_ERR_WORKSPACE_TOO_SMALL = 3,
  PKV_ERR_LAUNCH = 4,            /* the HIP runtime rejected a kernel launch */
  PKV_ERR_CAPACITY = 5           /* a host builder output buffer is too small */
} pkv_status;

typedef enum pkv_dtype { PKV_DTYPE_F16 = 0, PKV_DTYPE_BF16 = 1 } pkv_dtype;

/* Text of the most recent error on this thread ("" when none). */
const char* pkv_last_error(void);
/* Static name of a status code. */
const char* pkv_status_string(int status);
/* Library version as major*10000 + minor*100 + patch. */
int pkv_version(void);

/* ---------------------------------------------------------------------------------
 * Workspace sizing.
 * ------------------------------------------------------------------------------- */

/* Bytes of split workspace for the grid-split ops; 0 when num_splits <= 1.
 * Replaces persistentkv_workspace_bytes, kernels/persistentkv_attention.cuh:891-898. */
size_t pkv_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_splits);

/* Bytes of workspace for the work-queue op (total_partial_slots partial states per head).
 * Replaces persistentkv_partition_workqueue_workspace sizing, cuh:915-927. */
size_t pkv_workqueue_workspace_bytes(int32_t total_partial_slots, int32_t num_q_heads);

/* Bytes of workspace with which a direct launch (num_splits == 1) of the grid ops and of
 * pkv_attention_contiguous runs its full internal split: about 256 units of work for a
 * batch of few (row, kv head) pairs, whose partial states are merged by a second launch.
 * 0 when that launch is not split.  The reference's direct path takes no workspace
 * (cuh:929-946); this entry has no counterpart there. */
size_t pkv_direct_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                  int32_t context);

/* Bytes of workspace with which a split launch (num_splits > 1) of the grid ops and of
 * pkv_attention_contiguous runs its full internal sub-split: a launch of fewer
 * batch * num_kv_heads * num_splits units than about 3/4 of the CUs cuts each split into
 * sub-splits, to about one unit per CU (at least 2 tiles of 32 tokens each), merged
 * together.  pkv_workspace_bytes(batch, num_q_heads, num_splits) when the launch is not
 * sub-split; with that size (the reference's) the partial states keep the reference's
 * layout; sizes in between give fewer sub-splits, with the same result to fp32 rounding
 * (PKV_SPLIT_SUBDIVIDE=0 in the environment turns this off).  No counterpart in the
 * reference, whose split launches use exactly the caller's split (cuh:947-974). */
size_t pkv_split_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                 int32_t context, int32_t num_splits);

/* ---------------------------------------------------------------------------------
 * The four ops.  Argument order follows the torch op surface of
 * tests/persistentkv_torch_extension.cu, with the tensor shapes spelled out.
 * ------------------------------------------------------------------------------- */

/* Every row attends to exactly `context` tokens.
 * Replaces persistentkv_paged_attention (tests/persistentkv_torch_extension.cu:35-93)
 * and persistentkv_paged_dispatch (kernels/persistentkv_attention.cuh:1114-1136). */
int pkv_paged_attention(
    const void* q, const void* k_pages, const void* v_pages,
    const int32_t* block_table, void* output,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t context, int32_t num_splits, int32_t dtype, void* stream);

/* Row b attends to seq_lens[b] tokens; bucket_context bounds num_splits.
 * Replaces persistentkv_paged_attention_masked (extension.cu:95-157) and
 * persistentkv_paged_masked_dispatch (cuh:1138-1161). */
int pkv_paged_attention_masked(
    const void* q, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, void* output,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, int32_t dtype, void* stream);

/* Row b reads query row q_indices[b] of q_source and writes output row out_indices[b].
 * Replaces persistentkv_paged_attention_indexed (extension.cu:159-228) and
 * persistentkv_paged_masked_indexed_dispatch (cuh:1163-1189). */
int pkv_paged_attention_indexed(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, int32_t dtype, void* stream);

/* Compact work queue: one partial state per work item, then a segmented LSE merge
 * (or, with fused_merge != 0, the last work item of each (row, kv head) merges).
 * Replaces persistentkv_paged_attention_workqueue (extension.cu:230-317) and
 * persistentkv_paged_workqueue_indexed_dispatch (cuh:1191-1261).
 * Work-queue contract (the reference's, cuh:294-363, :648-716, :753-784):
 * - item (row, kvh, split, tile_begin, tile_end) writes the state of its own 32-token
 *   tile range into slot split_offsets[row] + split; a negative bound stands for the
 *   row-local split bound (cuh:330-337); a range without tiles writes the neutral state;
 *   items with row, kvh, split or slot out of range are ignored;
 * - row b's output folds the slots [split_offsets[b], split_offsets[b + 1]): every slot
 *   when num_tasks >= num_kv_heads x (split_offsets[batch] - split_offsets[0]) (a queue
 *   that writes each slot once, the queues on which the reference reads no unwritten
 *   memory); otherwise the slots of splits whose row-local range is empty are skipped
 *   (the builder's queues emit no item for them, and the reference then merges
 *   uninitialised memory);
 * - the fused merge waits for one arrival per slot in the first case (the reference's
 *   row_splits arrivals, cuh:659) and one per non-empty split in the second, and also
 *   merges rows of one slot (which the reference leaves unwritten). */
int pkv_paged_attention_workqueue(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t fused_merge,
    int32_t dtype, void* stream);

/* pkv_paged_attention_workqueue without the workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation).  It has no counterpart in the reference.  The partial states
 * go to a 16 MiB static scratch array in the library's code object (one per GPU, held
 * until the process ends); the call allocates nothing.  It returns
 * PKV_ERR_WORKSPACE_TOO_SMALL when pkv_workqueue_workspace_bytes(total_partial_slots,
 * num_q_heads) exceeds 16 MiB.  Every call on one GPU shares that GPU's scratch: calls
 * that overlap on one GPU (on other streams, or graph replays running at the same time)
 * race and give wrong results.  The scratch's address is taken on the calling thread's
 * current HIP device, which must be the device of `stream`.  Same results, bit for bit, as
 * pkv_paged_attention_workqueue with a workspace of exactly
 * pkv_workqueue_workspace_bytes(total_partial_slots, num_q_heads) bytes (the same
 * schedule, see pkv_workqueue_schedule). */
int pkv_paged_attention_workqueue_noalloc(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t fused_merge,
    int32_t dtype, void* stream);

/* Which schedule pkv_paged_attention_workqueue (and its fp8 and append variants) runs
 * for these sizes on the current device: 1 = the balanced schedule, 0 = one workgroup per
 * work item.  The balanced schedule streams every (row, kv head) pair's tiles [0, T) with
 * an equal share per wave (2 waves per CU, 4 with fp8 K/V) and merges the pieces; it
 * applies when fused_merge == 0, G = num_q_heads / num_kv_heads <= 16, page_size is a
 * multiple of 16, batch <= 256 and the workspace holds
 * pkv_workqueue_balanced_workspace_bytes (one threshold for every K/V dtype).
 * Streaming [0, T) is the reference's result for the queue pkv_build_workqueue (the
 * reference's compile_persistentkv_metadata) builds.  The decode checks on the device that
 * the caller's queue is exactly that one; for any other queue the merge stage computes
 * each (row, kv head) pair from the items' own tile ranges instead (slower), so both
 * schedules give the reference's result, to fp32 rounding, on every queue that writes
 * each slot once, and the builder's result on the builder's queues.  No counterpart in
 * the reference. */
int pkv_workqueue_schedule(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t page_size, size_t workspace_bytes, int32_t fused_merge);

/* Workspace bytes the balanced schedule needs on the current device, sized for its
 * largest wave count (4 per CU): the partial states,
 * (batch * num_kv_heads + 4 * CUs) * (num_q_heads / num_kv_heads) rounded up to even,
 * times 130 * 4 bytes, then a 16-byte plan entry per (row, kv head) pair (the waves that
 * hold the pair's tiles, written by the decode stage for the merge stage), then 4 bytes
 * per CU (each decode workgroup's part of the queue check); 0 for sizes it never takes
 * (G > 16 or batch > 256).  A complete queue's reference-sized workspace
 * (pkv_workqueue_workspace_bytes) often holds it already (C4: 2.66 MB against 2.26 MB).
 * No counterpart in the reference. */
size_t pkv_workqueue_balanced_workspace_bytes(int32_t batch, int32_t num_q_heads,
                                              int32_t num_kv_heads);

/* One stage of pkv_paged_attention_workqueue (fused_merge == 0), in whichever schedule
 * pkv_workqueue_schedule names: stage 1 = the decode kernel, 2 = the merge.  Stage 1 then
 * stage 2 on one stream equal the combined call bit for bit; they exist for per-kernel
 * timing and for callers that overlap the merge with other work.  Both stages take the
 * same arguments, the same workspace and workspace_bytes in particular (they choose the
 * schedule and where its partial states and plan lie): stage 2 folds what the last stage
 * 1 wrote into that workspace, so another step's stage 1 in between changes its result.
 * kv_fp8 != 0 selects the fp8 K/V pages of pkv_paged_attention_workqueue_fp8 with
 * k_scale / v_scale.  The reference launches both from one host function
 * (cuh:1005-1017); it has no separate entry points. */
int pkv_paged_attention_workqueue_stage(
    int32_t stage, const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t kv_fp8, float k_scale,
    float v_scale, int32_t dtype, void* stream);

/* The two stages of the per-item schedule of pkv_paged_attention_workqueue with
 * fused_merge == 0 (one workgroup per work item, partial states in the reference's slot
 * format (split_offsets[b] + s) * Hq + qh), callable on their own.  Running decode then
 * merge on one stream equals the combined call when it takes the per-item schedule
 * (pkv_workqueue_schedule == 0).  The reference launches both from one host function
 * (cuh:1005-1017); it has no separate entry points. */
int pkv_workqueue_decode(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, const int32_t* q_indices,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t dtype, void* stream);

/* num_tasks and num_kv_heads are the queue's item count and Hkv.  When num_tasks >=
 * num_kv_heads x (split_offsets[batch] - split_offsets[0]) (a queue that writes every
 * slot) the merge folds every slot of a row, as the reference's does (cuh:766-780);
 * otherwise (the builder's queues, whose splits without tiles emit no item) it skips the
 * slots whose row-local bounds are empty.  num_tasks < 0 selects the second rule. */
int pkv_workqueue_merge(
    const int32_t* seq_lens, const int32_t* split_offsets, const int32_t* out_indices,
    void* output, int32_t out_rows,
    const void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t total_partial_slots,
    int32_t num_tasks, int32_t num_kv_heads, int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------------
 * fp8 K/V: the same ops over K and V pages of OCP fp8 e4m3 (1 byte per element, same
 * [num_pages, num_kv_heads, page_size, 128] layout) dequantised with per-tensor scales,
 * K = k_scale * k8 and V = v_scale * v8.  q / output keep `dtype` (fp16 or bf16).
 * page_size must be a multiple of 16; k_scale must be positive and finite.  The
 * reference names fp8 / dequantising paged decode as future work
 * (paper/persistentkv_mlsys_workshop.tex:688-690); these entries have no counterpart
 * in its code and follow the signatures of the 2-byte ops they extend.
 * ------------------------------------------------------------------------------- */

/* pkv_paged_attention_indexed with fp8 K/V. */
int pkv_paged_attention_indexed_fp8(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, float k_scale, float v_scale,
    int32_t dtype, void* stream);

/* pkv_paged_attention_workqueue with fp8 K/V. */
int pkv_paged_attention_workqueue_fp8(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t fused_merge,
    float k_scale, float v_scale, int32_t dtype, void* stream);

/* pkv_workqueue_decode with fp8 K/V (stage 1 only; pkv_workqueue_merge is unchanged). */
int pkv_workqueue_decode_fp8(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, const int32_t* q_indices,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, float k_scale, float v_scale,
    int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------------
 * Contiguous-layout decode: K and V are [batch, num_kv_heads, context, 128] (every row
 * holds `context` tokens) and q / output are [batch, num_q_heads, 128].
 * ------------------------------------------------------------------------------- */

/* GQA decode over contiguous K/V, unsplit (num_splits == 1, no workspace) or split
 * (workspace of pkv_workspace_bytes(batch, num_q_heads, num_splits) bytes).
 * Replaces persistentkv_dispatch (cuh:1077-1090) and persistentkv_split_dispatch
 * (cuh:1092-1108) over PkvContiguousAccessor (cuh:128-178). */
int pkv_attention_contiguous(
    const void* q, const void* k, const void* v, void* output,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t context,
    int32_t head_dim, int32_t num_splits, int32_t dtype, void* stream);

/* Query-head baseline: each query head streams its KV head on its own, so every K/V
 * byte is read G times (the redundant GQA traffic the grouped path removes).  Same
 * output as pkv_attention_contiguous.  Replaces persistentkv_baseline_dispatch
 * (cuh:1263-1282) and pkv_query_head_baseline_kernel (cuh:786-889). */
int pkv_attention_query_head_baseline(
    const void* q, const void* k, const void* v, void* output,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t context,
    int32_t head_dim, int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------------
 * Host scheduling: split policy, cost model and compact work-queue builder.
 * Pure host code (no GPU needed).  "Reference" mode reproduces
 * tests/benchmark_serving_trace.py bit for bit; "mi355x" mode is re-tuned for 256 CUs.
 * ------------------------------------------------------------------------------- */

typedef enum pkv_policy { PKV_POLICY_REFERENCE = 0, PKV_POLICY_MI355X = 1 } pkv_policy;

typedef enum pkv_route {
  PKV_ROUTE_FLASHINFER = 0,   /* the reference's fallback route (reference policy only;
                                 this engine has no such route) */
  PKV_ROUTE_BUCKET = 1,       /* length-bucket split grid (paged_attention_indexed); with
                                 1 split, the direct launch */
  PKV_ROUTE_WORKQUEUE = 2     /* compact work queue (paged_attention_workqueue) */
} pkv_route;

/* Constants of the roofline cost model (benchmark_serving_trace.py:33-43). */
typedef struct pkv_cost_model {
  int32_t num_q_heads;        /* HQ */
  int32_t num_kv_heads;       /* HKV */
  int32_t head_dim;           /* DIM */
  int32_t compute_units;      /* SM_COUNT */
  double read_gbps;           /* ROOFLINE_READ_GBPS */
  double launch_overhead_us;  /* LAUNCH_OVERHEAD_US */
  double min_ctas_per_cu;     /* MIN_CTAS_PER_SM */
  int32_t supported_group;    /* SUPPORTED_PERSISTENTKV_GQA; 0 accepts every G */
  int32_t min_long_context;   /* 16384 in the reference's adaptive gate (:457) */
  int32_t policy;             /* pkv_policy used for the split choices */
  /* MI355X policy only (no counterpart in the reference's model): fixed costs of this
   * engine's launches, fitted to measured step times (profiles/cost_model_calibration.json,
   * persistentkv-attention_amd/pkv_calibrate.py). */
  double unit_round_us;       /* per round of two workgroups per CU of a split grid */
  double grid_merge_us;       /* a split grid's merge kernel */
  double queue_merge_us;      /* the work queue's merge kernel (balanced schedule) */
} pkv_cost_model;

/* Fills *model with the reference constants (RTX 3060) or the MI355X constants. */
void pkv_cost_model_preset(int32_t policy, pkv_cost_model* model);

/* choose_workqueue_row_splits, benchmark_serving_trace.py:370-393. */
int32_t pkv_choose_workqueue_row_splits(
    int32_t length, int32_t active_count, int32_t requested_splits,
    int32_t auto_splits, int32_t num_kv_heads, int32_t policy);

/* choose_splits, benchmark_serving_trace.py:328-367. */
int32_t pkv_choose_splits(
    const int32_t* lengths, int32_t count, int32_t requested_splits,
    int32_t auto_splits, int32_t single_bucket, int32_t num_kv_heads, int32_t policy);

/* model_bucket_splits / model_workqueue_splits, benchmark_serving_trace.py:396-415. */
int32_t pkv_model_bucket_splits(
    const int32_t* lengths, int32_t count, int32_t num_kv_heads, int32_t policy);
int32_t pkv_model_workqueue_splits(
    const int32_t* lengths, int32_t count, int32_t num_kv_heads, int32_t policy);

/* estimate_route_ms, benchmark_serving_trace.py:418-442.  `lengths` are the active
 * rows' current lengths. */
double pkv_estimate_route_ms(
    const int32_t* lengths, int32_t count, int32_t route, int32_t splits,
    const pkv_cost_model* model);

/* choose_adaptive_route_cost_model, benchmark_serving_trace.py:445-488.  Returns the
 * chosen pkv_route and writes its split count and estimate.  With model->policy ==
 * PKV_POLICY_MI355X it never returns PKV_ROUTE_FLASHINFER: every step, for any G, length
 * and active count, goes to the cheaper of PKV_ROUTE_BUCKET (splits from
 * pkv_model_bucket_splits, priced as one ragged grid launch plus its merge) and
 * PKV_ROUTE_WORKQUEUE (splits from pkv_model_workqueue_splits). */
int32_t pkv_choose_adaptive_route(
    const int32_t* lengths, int32_t count, const pkv_cost_model* model,
    int32_t* out_splits, double* out_estimated_ms);

/* Sizes the compact work queue for one decode step without building it.  num_q_heads
 * only matters for PKV_POLICY_MI355X, whose item size depends on the kernel that
 * G = num_q_heads / num_kv_heads selects; the reference policy ignores it. */
int pkv_workqueue_size(
    const int32_t* lengths, int32_t count, int32_t requested_splits,
    int32_t auto_splits, int32_t num_q_heads, int32_t num_kv_heads, int32_t policy,
    int32_t* out_num_tasks, int32_t* out_total_partial_slots);

/* Builds one decode step's work-queue metadata, bit-exact with the work-queue branch of
 * compile_persistentkv_metadata (benchmark_serving_trace.py:668-729).
 *   lengths[count], request_ids[count]: the active rows in step order.
 *   page_indptr[count+1], page_ids[]: each active row's reserved physical pages (CSR).
 * Outputs (host buffers):
 *   block_table[count * table_cols]: row r = its first ceil(max_len/page_size) pages,
 *     padded with its last reserved page; *out_table_cols receives the width.
 *   seq_lens[count], q_indices[count] (= request_ids), out_indices[count] (= r),
 *   work_items[5 * work_capacity], split_offsets[count + 1].
 * Returns PKV_ERR_CAPACITY (with the needed sizes written) when a buffer is too small. */
int pkv_build_workqueue(
    const int32_t* lengths, const int32_t* request_ids, int32_t count,
    const int32_t* page_indptr, const int32_t* page_ids,
    int32_t page_size, int32_t requested_splits, int32_t auto_splits,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t policy,
    int32_t* block_table, int32_t table_capacity, int32_t* out_table_cols,
    int32_t* seq_lens, int32_t* q_indices, int32_t* out_indices,
    int32_t* work_items, int32_t work_capacity, int32_t* out_num_tasks,
    int32_t* split_offsets, int32_t* out_total_partial_slots);

/* round_bucket_length, benchmark_serving_trace.py:316-321: `length` rounded up to a
 * multiple of bucket_tokens, then to a multiple of page_size (at least one page), capped
 * at the row's allocated_pages * page_size; `length` itself when bucket_tokens <= 0. */
int32_t pkv_round_bucket_length(int32_t length, int32_t bucket_tokens, int32_t allocated_pages,
                                int32_t page_size);

/* use_single_bucket_for_state, benchmark_serving_trace.py:491-504: 1 when the step's rows
 * go through one ragged bucket (requested, or adaptive with at least max(3, count - 1)
 * distinct lengths among count > 1 rows). */
int32_t pkv_use_single_bucket(const int32_t* lengths, int32_t count,
                              int32_t requested_single_bucket, int32_t adaptive_route);

/* Builds one decode step's length-bucket metadata, bit-exact with the bucket branch of
 * compile_persistentkv_metadata (benchmark_serving_trace.py:731-780): rows grouped by
 * pkv_round_bucket_length of their length (one bucket of max(lengths) when
 * pkv_use_single_bucket), buckets in order of first appearance, rows of a bucket in step
 * order.  Bucket j (j < *out_bucket_count <= count) holds bucket_rows[j] rows, which are
 * entries [sum of earlier bucket_rows, + bucket_rows[j]) of seq_lens (the row's length),
 * q_indices (its request id) and out_indices (its position in the step), and one
 * [bucket_rows[j], bucket_table_cols[j] = ceil(bucket_lengths[j] / page_size)] block
 * table, stored after the earlier buckets' tables in `tables`, each row its first
 * reserved pages padded with its last one.  bucket_splits[j] is choose_splits over the
 * bucket's lengths (pkv_choose_splits with `policy`).  Every bucket is one
 * pkv_paged_attention_indexed launch with bucket_context = bucket_lengths[j] (:986-1000).
 * Returns PKV_ERR_CAPACITY with *out_table_elems set when `tables` is too small. */
int pkv_build_buckets(const int32_t* lengths, const int32_t* request_ids, int32_t count,
                      const int32_t* page_indptr, const int32_t* page_ids, int32_t page_size,
                      int32_t requested_splits, int32_t auto_splits, int32_t bucket_tokens,
                      int32_t single_bucket, int32_t adaptive_route, int32_t num_kv_heads,
                      int32_t policy, int32_t* out_bucket_count, int32_t* bucket_lengths,
                      int32_t* bucket_rows, int32_t* bucket_splits, int32_t* bucket_table_cols,
                      int32_t* seq_lens, int32_t* q_indices, int32_t* out_indices,
                      int32_t* tables, int64_t table_capacity, int64_t* out_table_elems);

/* ---------------------------------------------------------------------------------
 * KV-cache append: the write of each row's newest token before its decode step.
 * No counterpart in the reference, whose harness grows the lengths without writing K/V
 * (tests/benchmark_serving_trace.py:285-298); fused KV-cache writes are future work in
 * paper/persistentkv_mlsys_workshop.tex:689.
 * ------------------------------------------------------------------------------- */

/* Writes k_new[b] and v_new[b] ([num_kv_heads, 128] each, dtype f16 or bf16, batch rows)
 * into the pools ([num_pages, num_kv_heads, page_size, 128], same dtype) at token position
 * seq_lens[b] - 1: page block_table[b * max_pages + pos / page_size], slot
 * pos % page_size.  Rows with seq_lens[b] <= 0, a position past the table, or a page id
 * outside [0, num_pages) are skipped.  Asynchronous on `stream`. */
int pkv_append_kv(const void* k_new, const void* v_new, void* k_pages, void* v_pages,
                  const int32_t* block_table, const int32_t* seq_lens, int32_t batch,
                  int32_t num_kv_heads, int32_t head_dim, int32_t num_pages, int32_t page_size,
                  int32_t max_pages, int32_t dtype, void* stream);

/* pkv_append_kv into fp8 (OCP e4m3) pools: each element is stored as
 * e4m3(clamp(x / scale, -448, 448)), rounded to nearest even (torch's float8_e4m3fn cast),
 * with k_scale for K and v_scale for V.  `dtype` is that of k_new and v_new. */
int pkv_append_kv_fp8(const void* k_new, const void* v_new, void* k_pages, void* v_pages,
                      const int32_t* block_table, const int32_t* seq_lens, int32_t batch,
                      int32_t num_kv_heads, int32_t head_dim, int32_t num_pages,
                      int32_t page_size, int32_t max_pages, float k_scale, float v_scale,
                      int32_t dtype, void* stream);

/* Decode with the append fused in: the result and the pools afterwards equal
 * pkv_append_kv(k_new, v_new, ...) followed by the op without the suffix, in one decode
 * launch.  The newest token of each row (position seq_lens[b] - 1) is read from k_new /
 * v_new ([batch, num_kv_heads, 128], `dtype`) by the one wave whose tiles hold it, which
 * also writes it into the pools.  Page sizes that are not multiples of 16 run
 * pkv_append_kv first on the same stream.  (fp8 pools: the *_fp8_append entries below.)  A row's tail slot must not be read
 * through another (row, position) of the same step (no two rows share a tail page, as
 * in any copy-on-write cache).  No counterpart in the reference (see pkv_append_kv). */
int pkv_paged_attention_masked_append(
    const void* q, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, void* output,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, const void* k_new, const void* v_new,
    int32_t dtype, void* stream);

int pkv_paged_attention_indexed_append(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, const void* k_new, const void* v_new,
    int32_t dtype, void* stream);

/* pkv_paged_attention_workqueue with the append fused in (as above). */
int pkv_paged_attention_workqueue_append(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t fused_merge,
    const void* k_new, const void* v_new, int32_t dtype, void* stream);

/* The fp8-K/V ops with the append: k_new / v_new are in `dtype` and stored as
 * pkv_append_kv_fp8 stores them, e4m3(clamp(x / k_scale)) and e4m3(clamp(x / v_scale)).
 * Same result as pkv_append_kv_fp8 followed by the fp8 op, which is what they run (two
 * launches; an in-decode fp8 append measured slower).  v_scale must be positive. */
int pkv_paged_attention_indexed_fp8_append(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, float k_scale, float v_scale,
    const void* k_new, const void* v_new, int32_t dtype, void* stream);

int pkv_paged_attention_workqueue_fp8_append(
    const void* q_source, int32_t q_rows,
    const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens,
    const int32_t* work_items, int32_t num_tasks,
    const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices,
    void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t fused_merge,
    float k_scale, float v_scale, const void* k_new, const void* v_new,
    int32_t dtype, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* PKV_H_ */
