// pkv_schedule.cpp — host scheduling for the PersistentKV decode engine: split policy,
// roofline cost-model router and the compact work-queue builder.
//
// PKV_POLICY_REFERENCE reproduces tests/benchmark_serving_trace.py bit for bit (integer
// results exactly; floating-point estimates with the same operation order in IEEE
// double, which is what CPython's float is).  PKV_POLICY_MI355X re-targets the split
// choice at 256 compute units: it sizes work items from the whole step's tile count so
// that every CU holds several workgroups, instead of the reference's fixed CTA target
// calibrated for a 28-SM RTX 3060.
//
// Pure host code: no HIP calls.

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <set>
#include <vector>

#include "pkv.h"

namespace {

constexpr int kTileTokens = 32;

// Python floor division for the non-negative operands used here; negative lengths are
// mapped through Python's floor semantics explicitly where the reference can see them.
inline int64_t floordiv(int64_t a, int64_t b) {
  int64_t q = a / b, r = a % b;
  return (r != 0 && ((r < 0) != (b < 0))) ? q - 1 : q;
}

inline int64_t ceil_div_pos(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int32_t round_up4(int64_t v) { return (int32_t)(floordiv(v + 3, 4) * 4); }  // :324-325

inline int64_t tiles_of(int64_t length) { return floordiv(length + 31, 32); }

// MI355X targets: 256 CUs with one decode workgroup each, about 1.5 work items per CU
// for G <= 16, and at least this many 32-token tiles per work item so the per-item Q
// load, LDS combine and partial write stay small next to the K/V stream.  Measured on
// equal-sized items over the C4 and C5 traces: 384 items was the fastest or tied for
// G <= 16 (C5 G=8: 242 us per step against 250-293 us at 372-496 items; C4 within 1 %),
// since every item pays a fixed chain of dependent loads and one decode workgroup (8
// waves, one tile in flight each) streams at most ~35 GB/s.  G > 16 plans at most one item per CU instead (plan_row_splits).
constexpr int kMiComputeUnits = 256;
constexpr int kMiTargetItems = kMiComputeUnits * 3 / 2;
constexpr int kMiMinTilesPerItem = 8;
constexpr int kMiWideGroup = 16;  // G above this runs the two-head-block kernel
constexpr int kMiMaxSplits = 128;
// Fixed costs of the MI355X route model (mi355x_route_us), fitted by non-negative least
// squares to the step times of both routes on up to 6 sampled steps of each of 14 workloads
// (this engine's configurations and the reference's review traces; pkv_serving.py
// --calibrate, fitted by pkv_calibrate.py): the per-CU read rate that prices a tile
// (kMiReadGbps), a cost per round of two workgroups per CU of a split grid, and the work
// queue's fixed cost (its merge, the launch gap and the balanced decode's ramp).  The
// grid's fixed cost fits to 0: its rounds carry it.  With these the router takes the
// faster route on every sampled step where the two differ by more than 3 %.
constexpr double kMiReadGbps = 6372.0;
constexpr double kMiUnitRoundUs = 5.88;
constexpr double kMiGridMergeUs = 0.0;
constexpr double kMiQueueMergeUs = 11.47;


}  // namespace

extern "C" {

void pkv_cost_model_preset(int32_t policy, pkv_cost_model* m) {
  if (!m) return;
  m->num_q_heads = 32;       // HQ, benchmark_serving_trace.py:33
  m->num_kv_heads = 8;       // HKV, :34
  m->head_dim = 128;         // DIM, :35
  m->min_long_context = 16384;  // adaptive gate, :457
  m->policy = policy;
  if (policy == PKV_POLICY_MI355X) {
    m->compute_units = kMiComputeUnits;
    m->read_gbps = kMiReadGbps;     // fitted (see kMiReadGbps)
    m->launch_overhead_us = 1.5;    // gap between dependent launches on one stream
    m->min_ctas_per_cu = 2.0;
    m->supported_group = 0;         // every G runs natively
    m->unit_round_us = kMiUnitRoundUs;
    m->grid_merge_us = kMiGridMergeUs;
    m->queue_merge_us = kMiQueueMergeUs;
  } else {
    m->compute_units = 28;          // SM_COUNT, :39
    m->read_gbps = 302.0;           // ROOFLINE_READ_GBPS, :40
    m->launch_overhead_us = 8.0;    // LAUNCH_OVERHEAD_US, :41
    m->min_ctas_per_cu = 4.0;       // MIN_CTAS_PER_SM, :42
    m->supported_group = 4;         // SUPPORTED_PERSISTENTKV_GQA, :43
    m->unit_round_us = m->grid_merge_us = m->queue_merge_us = 0.0;  // not in its model
  }
}

// choose_workqueue_row_splits, benchmark_serving_trace.py:370-393.
int32_t pkv_choose_workqueue_row_splits(int32_t length, int32_t active_count,
                                        int32_t requested_splits, int32_t auto_splits,
                                        int32_t num_kv_heads, int32_t policy) {
  if (!auto_splits) return requested_splits;
  const int64_t tiles = std::max<int64_t>(1, tiles_of(length));
  const int64_t hkv = num_kv_heads > 0 ? num_kv_heads : 1;
  const int64_t active = std::max<int32_t>(1, active_count);
  if (policy == PKV_POLICY_MI355X) {
    // Per-row view of the joint planner: assume the other rows are as long as this one.
    const int64_t target = kMiTargetItems;
    const int64_t per_item = std::max<int64_t>(kMiMinTilesPerItem,
                                               ceil_div_pos(tiles * active * hkv, target));
    const int64_t s = ceil_div_pos(tiles, per_item);
    return (int32_t)std::max<int64_t>(1, std::min<int64_t>(s, kMiMaxSplits));
  }
  const int32_t occupancy_floor = round_up4(ceil_div_pos(256, hkv * active));
  const int32_t length_target = round_up4(ceil_div_pos(tiles, 64));
  int32_t splits = std::max(occupancy_floor, length_target);
  if (active_count >= 8) splits = std::min(splits, 24);
  else if (active_count >= 4) splits = std::min(splits, 32);
  else if (active_count == 2) splits = std::min(splits, 40);
  else splits = std::min(splits, 48);
  return (int32_t)std::max<int64_t>(4, std::min<int64_t>(std::min(splits, 48), tiles));
}

// choose_splits, benchmark_serving_trace.py:328-367.
int32_t pkv_choose_splits(const int32_t* lengths, int32_t count, int32_t requested_splits,
                          int32_t auto_splits, int32_t single_bucket, int32_t num_kv_heads,
                          int32_t policy) {
  if (!auto_splits) return requested_splits;
  if (!lengths || count <= 0) return requested_splits;
  int64_t t_max = INT64_MIN, t_min = INT64_MAX;
  for (int i = 0; i < count; ++i) {
    const int64_t t = tiles_of(lengths[i]);
    t_max = std::max(t_max, t);
    t_min = std::min(t_min, t);
  }
  const int64_t batch = count;
  const int64_t hkv = num_kv_heads > 0 ? num_kv_heads : 1;
  auto clamp4 = [&](int64_t cap) { return (int32_t)std::max<int64_t>(4, std::min(cap, t_min)); };
  if (policy == PKV_POLICY_MI355X) {
    // One split count for the whole launch (a bucket, or a ragged grid with row-local
    // split bounds).  Rows of one length: one unit per CU, every unit in the first round
    // (C3 at 32k, B1 Hkv 8: 27.6 us per step with 32 splits against 32.2 us with 64 and
    // 40 us with 48 in the serving harness).  Rows of mixed lengths: also enough splits
    // that the longest row's unit is at most a quarter of a CU's share of the tiles, so
    // that it does not end the launch alone (C2, B8 MHA with lengths in [1024, 8192]:
    // 112 us per step with 8 splits against 130 us with 2).  At least 2 tiles per unit
    // of the longest row; shorter rows may hold empty splits.
    int64_t total = 0;
    for (int i = 0; i < count; ++i) total += std::max<int64_t>(1, tiles_of(lengths[i]));
    int64_t s = ceil_div_pos(kMiComputeUnits, hkv * batch);
    if (t_max * 10 > t_min * 11)
      s = std::max<int64_t>(s, ceil_div_pos(4 * t_max * kMiComputeUnits, hkv * total));
    s = std::min<int64_t>(s, std::max<int64_t>(1, t_max / 2));
    return (int32_t)std::max<int64_t>(1, std::min<int64_t>(s, kMiMaxSplits));
  }
  if (single_bucket) {
    if (batch >= 8) return clamp4(40);
    if (batch == 4) return clamp4(16);
    if (batch == 2) return clamp4(24);
    if (t_max >= 1024) return clamp4(36);
    return clamp4(24);
  }
  if (batch >= 8) return clamp4(24);
  if (batch == 4) return clamp4(28);
  if (batch == 2 && t_max >= 1024) return clamp4(32);
  const int64_t occupancy = ceil_div_pos(320, hkv * batch);
  const int64_t length_based = (int64_t)std::ceil((double)t_max / 32.0);
  int64_t splits = round_up4(std::max(occupancy, length_based));
  if (t_max <= 384) splits = std::min<int64_t>(splits, 24);
  if (batch >= 8) splits = std::min<int64_t>(splits, 40);
  if (batch <= 2 && t_max >= 1024) splits = std::max<int64_t>(splits, 32);
  return (int32_t)std::max<int64_t>(4, std::min(std::min<int64_t>(splits, 48), t_min));
}

// model_bucket_splits, benchmark_serving_trace.py:396-402.
int32_t pkv_model_bucket_splits(const int32_t* lengths, int32_t count, int32_t num_kv_heads,
                                int32_t policy) {
  if (!lengths || count <= 0) return 4;
  int64_t t_max = INT64_MIN, t_min = INT64_MAX;
  for (int i = 0; i < count; ++i) {
    const int64_t t = tiles_of(lengths[i]);
    t_max = std::max(t_max, t);
    t_min = std::min(t_min, t);
  }
  const int64_t hkv = num_kv_heads > 0 ? num_kv_heads : 1;
  if (policy == PKV_POLICY_MI355X) return pkv_choose_splits(lengths, count, 1, 1, 0, num_kv_heads, policy);
  const int64_t occupancy = ceil_div_pos(256, hkv * std::max<int64_t>(1, count));
  const int64_t length_based = (int64_t)std::ceil((double)t_max / 96.0);
  const int64_t r = round_up4(std::max(occupancy, length_based));
  return (int32_t)std::max<int64_t>(4, std::min(std::min<int64_t>(r, 48), t_min));
}

// model_workqueue_splits, benchmark_serving_trace.py:405-415.
int32_t pkv_model_workqueue_splits(const int32_t* lengths, int32_t count, int32_t num_kv_heads,
                                   int32_t policy) {
  int32_t best = INT32_MIN;
  for (int i = 0; i < count; ++i)
    best = std::max(best, pkv_choose_workqueue_row_splits(lengths[i], count, 1, 1, num_kv_heads, policy));
  return best;
}

// MI355X route cost: the makespan of the launch on this engine's kernels, in place of
// the reference's occupancy-penalty model (which charges a launch with fewer than
// min_ctas_per_cu workgroups per CU, while one equal unit per CU is this engine's fastest
// grid).  Each CU streams one 32-token tile of one kv head (16 KB at D = 128, 2-byte K/V)
// in tile_us at read_gbps / compute_units.
//   split grid (S splits per row, row-local bounds): max(share, longest unit) tiles,
//     plus a fixed cost per round of two 8-wave workgroups per CU, plus the merge;
//   work queue (balanced schedule: equal tile shares per wave): share tiles plus its merge.
double mi355x_route_us(const int32_t* lengths, int32_t count, int32_t route, int32_t splits,
                       const pkv_cost_model* m) {
  const int64_t hkv = m->num_kv_heads > 0 ? m->num_kv_heads : 1;
  const int64_t cus = m->compute_units > 0 ? m->compute_units : kMiComputeUnits;
  const double tile_bytes = (double)kTileTokens * m->head_dim * 2 * 2;
  const double tile_us = tile_bytes / (m->read_gbps * 1e3 / (double)cus);  // GB/s = 1e3 B/us
  int64_t total = 0, longest = 0;
  for (int i = 0; i < count; ++i) {
    const int64_t t = tiles_of(std::max<int32_t>(lengths[i], 0));
    total += t * hkv;
    longest = std::max(longest, t);
  }
  const double share = (double)total / (double)cus;
  const double launches_us = 2.0 * m->launch_overhead_us;
  if (route == PKV_ROUTE_WORKQUEUE) return share * tile_us + m->queue_merge_us + launches_us;
  const int64_t s = std::max<int32_t>(1, splits);
  const double unit = (double)ceil_div_pos(std::max<int64_t>(longest, 1), s);
  const double units = (double)count * hkv * s;
  const double rounds = std::ceil(units / (2.0 * cus));
  return std::max(share, unit) * tile_us + rounds * m->unit_round_us +
         (s > 1 ? m->grid_merge_us + launches_us : 0.5 * launches_us);
}

// estimate_route_ms, benchmark_serving_trace.py:418-442 (and useful_kv_mb_for_state :511-513).
// The MI355X policy prices PKV_ROUTE_BUCKET (the split grid) and PKV_ROUTE_WORKQUEUE with
// mi355x_route_us.
double pkv_estimate_route_ms(const int32_t* lengths, int32_t count, int32_t route, int32_t splits,
                             const pkv_cost_model* m) {
  if (!m || (!lengths && count > 0)) return NAN;
  if (m->policy == PKV_POLICY_MI355X) {
    if (route != PKV_ROUTE_BUCKET && route != PKV_ROUTE_WORKQUEUE) return NAN;
    return mi355x_route_us(lengths, count, route, splits, m) / 1000.0;
  }
  int64_t sum_len = 0;
  std::set<int32_t> unique;
  for (int i = 0; i < count; ++i) {
    sum_len += lengths[i];
    unique.insert(lengths[i]);
  }
  const int64_t bytes_read = sum_len * m->num_kv_heads * m->head_dim * 2 * 2;
  const double kv_mb = (double)bytes_read / (1024.0 * 1024.0);
  const double kv_ms = kv_mb / m->read_gbps;
  const int64_t active = count;
  double ctas_per_cu;
  int64_t launch_count;
  double merge_mb;
  const int64_t merge_bytes = active * m->num_q_heads * (int64_t)splits * (2 + m->head_dim) * 4;
  if (route == PKV_ROUTE_FLASHINFER) {
    ctas_per_cu = (double)(active * m->num_kv_heads) / (double)m->compute_units;
    launch_count = 1;
    merge_mb = 0.0;
  } else if (route == PKV_ROUTE_BUCKET) {
    ctas_per_cu = (double)(active * m->num_kv_heads * splits) / (double)m->compute_units;
    // The reference launches decode + merge per exact-length bucket.
    launch_count = 2 * (int64_t)unique.size();
    merge_mb = (double)merge_bytes / (1024.0 * 1024.0);
  } else if (route == PKV_ROUTE_WORKQUEUE) {
    ctas_per_cu = (double)(active * m->num_kv_heads * splits) / (double)m->compute_units;
    launch_count = 2;
    merge_mb = (double)merge_bytes / (1024.0 * 1024.0);
  } else {
    return NAN;
  }
  const double occupancy_penalty = std::max(1.0, m->min_ctas_per_cu / std::max(ctas_per_cu, 1e-6));
  const double launch_ms = (double)launch_count * m->launch_overhead_us / 1000.0;
  const double merge_ms = merge_mb / m->read_gbps;
  return kv_ms * occupancy_penalty + merge_ms + launch_ms;
}

// choose_adaptive_route_cost_model, benchmark_serving_trace.py:445-488.  The reference
// falls back to FlashInfer for unsupported G and short contexts.  The MI355X policy has
// no such route: every step goes to one of this engine's own routes, the split grid
// (PKV_ROUTE_BUCKET, with splits == 1 meaning the direct launch) or the compact work
// queue, whichever the cost model prices lower, for every G, length and active count.
int32_t pkv_choose_adaptive_route(const int32_t* lengths, int32_t count, const pkv_cost_model* m,
                                  int32_t* out_splits, double* out_ms) {
  if (!m || !lengths || count <= 0) return -1;
  if (m->policy == PKV_POLICY_MI355X) {
    const int32_t bs = pkv_model_bucket_splits(lengths, count, m->num_kv_heads, m->policy);
    const int32_t ws = pkv_model_workqueue_splits(lengths, count, m->num_kv_heads, m->policy);
    const double be = pkv_estimate_route_ms(lengths, count, PKV_ROUTE_BUCKET, bs, m);
    const double we = pkv_estimate_route_ms(lengths, count, PKV_ROUTE_WORKQUEUE, ws, m);
    const bool queue = we < be;  // ties keep the grid: one fewer metadata tensor per step
    if (out_splits) *out_splits = queue ? ws : bs;
    if (out_ms) *out_ms = queue ? we : be;
    return queue ? PKV_ROUTE_WORKQUEUE : PKV_ROUTE_BUCKET;
  }
  const int32_t g = m->num_kv_heads > 0 ? m->num_q_heads / m->num_kv_heads : 0;
  int32_t route = PKV_ROUTE_FLASHINFER, splits = 1;
  double best = pkv_estimate_route_ms(lengths, count, PKV_ROUTE_FLASHINFER, 1, m);
  const int32_t max_len = *std::max_element(lengths, lengths + count);
  const bool gate = (m->supported_group != 0 && g != m->supported_group) || max_len < m->min_long_context;
  if (!gate) {
    if (count <= 1) {
      const int32_t s = pkv_model_bucket_splits(lengths, count, m->num_kv_heads, m->policy);
      const double e = pkv_estimate_route_ms(lengths, count, PKV_ROUTE_BUCKET, s, m);
      if (e < best) { best = e; route = PKV_ROUTE_BUCKET; splits = s; }
    }
    if (count >= 8) {
      const int32_t s = pkv_model_workqueue_splits(lengths, count, m->num_kv_heads, m->policy);
      const double e = pkv_estimate_route_ms(lengths, count, PKV_ROUTE_WORKQUEUE, s, m);
      if (e < best) { best = e; route = PKV_ROUTE_WORKQUEUE; splits = s; }
    }
  }
  if (out_splits) *out_splits = splits;
  if (out_ms) *out_ms = best;
  return route;
}

static void plan_row_splits(const int32_t* lengths, int32_t count, int32_t requested_splits,
                            int32_t auto_splits, int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t policy, std::vector<int32_t>& out) {
  out.resize(count);
  if (auto_splits && policy == PKV_POLICY_MI355X) {
    // Joint plan: size items from the step's total tile count.
    int64_t total = 0, longest = 1;
    for (int i = 0; i < count; ++i) {
      const int64_t t = std::max<int64_t>(1, tiles_of(lengths[i]));
      total += t;
      longest = std::max(longest, t);
    }
    const int64_t hkv = num_kv_heads > 0 ? num_kv_heads : 1;
    const int64_t group = num_q_heads > 0 ? num_q_heads / hkv : 1;
    auto splits_of = [&](int64_t tiles, int64_t per_item) {
      return std::max<int64_t>(1, std::min<int64_t>(ceil_div_pos(tiles, per_item), kMiMaxSplits));
    };
    int64_t per_item;
    if (group > kMiWideGroup) {
      // The G > 16 kernel runs one workgroup per CU, one wave per SIMD, with a long
      // epilogue: every item should start in the first round.  Measured on C5 G=32
      // (bf16, B=64 Zipf): 232 items take 76.1 us per step, 259-291 items 90-100 us and
      // 415 items 86.0 us.  The launch lasts as long as its largest item, so take the
      // smallest item size at which there are at most kMiComputeUnits items (the item
      // count only falls as the size grows: a binary search).
      auto items_at = [&](int64_t size) {
        int64_t items = 0;
        for (int i = 0; i < count; ++i)
          items += splits_of(std::max<int64_t>(1, tiles_of(lengths[i])), size) * hkv;
        return items;
      };
      int64_t lo = std::max<int64_t>(kMiMinTilesPerItem, ceil_div_pos(total * hkv, kMiComputeUnits));
      int64_t hi = std::max(lo, longest);
      if (items_at(lo) > kMiComputeUnits) {
        while (hi - lo > 1) {  // items_at(lo) > CUs; items_at(hi) <= CUs or hi == longest
          const int64_t mid = lo + (hi - lo) / 2;
          if (items_at(mid) <= kMiComputeUnits) hi = mid;
          else lo = mid;
        }
        per_item = hi;
      } else {
        per_item = lo;
      }
    } else {
      per_item = std::max<int64_t>(kMiMinTilesPerItem, ceil_div_pos(total * hkv, kMiTargetItems));
    }
    for (int i = 0; i < count; ++i)
      out[i] = (int32_t)splits_of(std::max<int64_t>(1, tiles_of(lengths[i])), per_item);
    return;
  }
  for (int i = 0; i < count; ++i)
    out[i] = pkv_choose_workqueue_row_splits(lengths[i], count, requested_splits, auto_splits,
                                             num_kv_heads, policy);
}

int pkv_workqueue_size(const int32_t* lengths, int32_t count, int32_t requested_splits,
                       int32_t auto_splits, int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t policy, int32_t* out_num_tasks, int32_t* out_total_partial_slots) {
  if ((!lengths && count > 0) || count < 0 || num_kv_heads <= 0) return PKV_ERR_INVALID_ARGUMENT;
  std::vector<int32_t> splits;
  plan_row_splits(lengths, count, requested_splits, auto_splits, num_q_heads, num_kv_heads, policy,
                  splits);
  int64_t tasks = 0, slots = 0;
  for (int r = 0; r < count; ++r) {
    const int64_t total_tiles = tiles_of(lengths[r]);
    const int64_t s = splits[r];
    for (int64_t sp = 0; sp < s; ++sp)
      if (floordiv(total_tiles * sp, s) < floordiv(total_tiles * (sp + 1), s)) tasks += num_kv_heads;
    slots += s;
  }
  if (tasks > INT32_MAX || slots > INT32_MAX) return PKV_ERR_CAPACITY;
  if (out_num_tasks) *out_num_tasks = (int32_t)tasks;
  if (out_total_partial_slots) *out_total_partial_slots = (int32_t)slots;
  return PKV_OK;
}

// Work-queue branch of compile_persistentkv_metadata, benchmark_serving_trace.py:668-729.
int pkv_build_workqueue(const int32_t* lengths, const int32_t* request_ids, int32_t count,
                        const int32_t* page_indptr, const int32_t* page_ids, int32_t page_size,
                        int32_t requested_splits, int32_t auto_splits, int32_t num_q_heads,
                        int32_t num_kv_heads, int32_t policy, int32_t* block_table,
                        int32_t table_capacity,
                        int32_t* out_table_cols, int32_t* seq_lens, int32_t* q_indices,
                        int32_t* out_indices, int32_t* work_items, int32_t work_capacity,
                        int32_t* out_num_tasks, int32_t* split_offsets,
                        int32_t* out_total_partial_slots) {
  if (count <= 0 || !lengths || !request_ids || !page_indptr || !page_ids || page_size <= 0 ||
      num_kv_heads <= 0)
    return PKV_ERR_INVALID_ARGUMENT;
  const int32_t bucket_length = *std::max_element(lengths, lengths + count);  // :669
  const int64_t page_count = bucket_length > 0 ? ceil_div_pos(bucket_length, page_size) : 0;  // :670
  int32_t tasks = 0, slots = 0;
  int st = pkv_workqueue_size(lengths, count, requested_splits, auto_splits, num_q_heads,
                              num_kv_heads, policy, &tasks, &slots);
  if (st != PKV_OK) return st;
  if (out_table_cols) *out_table_cols = (int32_t)page_count;
  if (out_num_tasks) *out_num_tasks = tasks;
  if (out_total_partial_slots) *out_total_partial_slots = slots;
  if ((int64_t)count * page_count > table_capacity || tasks > work_capacity) return PKV_ERR_CAPACITY;
  if (!block_table || !seq_lens || !q_indices || !out_indices || !split_offsets ||
      (tasks > 0 && !work_items))
    return PKV_ERR_INVALID_ARGUMENT;
  std::vector<int32_t> splits;
  plan_row_splits(lengths, count, requested_splits, auto_splits, num_q_heads, num_kv_heads, policy,
                  splits);
  int32_t n = 0;
  split_offsets[0] = 0;
  for (int32_t r = 0; r < count; ++r) {
    const int32_t p0 = page_indptr[r], p1 = page_indptr[r + 1];
    if (p1 < p0) return PKV_ERR_INVALID_ARGUMENT;
    if (p1 == p0 && page_count > 0) return PKV_ERR_INVALID_ARGUMENT;  // reference indexes [-1]
    int32_t* row = block_table + (int64_t)r * page_count;
    for (int64_t c = 0; c < page_count; ++c)  // :679-683 pad with the last reserved page
      row[c] = (c < p1 - p0) ? page_ids[p0 + c] : page_ids[p1 - 1];
    seq_lens[r] = lengths[r];
    q_indices[r] = request_ids[r];
    out_indices[r] = r;
    const int64_t s = splits[r];
    const int64_t total_tiles = tiles_of(lengths[r]);  // :695
    for (int64_t sp = 0; sp < s; ++sp) {
      const int64_t tb = floordiv(total_tiles * sp, s), te = floordiv(total_tiles * (sp + 1), s);
      if (tb >= te) continue;  // :699-700
      for (int32_t kvh = 0; kvh < num_kv_heads; ++kvh) {
        int32_t* w = work_items + (int64_t)n * 5;
        w[0] = r;
        w[1] = kvh;
        w[2] = (int32_t)sp;
        w[3] = (int32_t)tb;
        w[4] = (int32_t)te;
        ++n;
      }
    }
    split_offsets[r + 1] = split_offsets[r] + (int32_t)s;  // :703 counts empty splits too
  }
  return PKV_OK;
}

// round_bucket_length, benchmark_serving_trace.py:316-321 (rounded_length :159-160 with
// the harness's PAGE_SIZE).
int32_t pkv_round_bucket_length(int32_t length, int32_t bucket_tokens, int32_t allocated_pages,
                                int32_t page_size) {
  if (bucket_tokens <= 0) return length;
  int64_t bucket = floordiv((int64_t)length + bucket_tokens - 1, bucket_tokens) * bucket_tokens;
  bucket = std::max<int64_t>(page_size, floordiv(bucket + page_size - 1, page_size) * page_size);
  return (int32_t)std::min<int64_t>(bucket, (int64_t)allocated_pages * page_size);
}

// use_single_bucket_for_state, benchmark_serving_trace.py:491-504.
int32_t pkv_use_single_bucket(const int32_t* lengths, int32_t count,
                              int32_t requested_single_bucket, int32_t adaptive_route) {
  if (requested_single_bucket) return 1;
  if (!adaptive_route) return 0;
  if (count <= 1 || !lengths) return 0;
  const int64_t unique = (int64_t)std::set<int32_t>(lengths, lengths + count).size();
  return unique >= std::max<int64_t>(3, (int64_t)count - 1) ? 1 : 0;
}

// Length-bucket route of compile_persistentkv_metadata (benchmark_serving_trace.py:731-780):
// active rows grouped by rounded length, buckets in order of first appearance (Python
// dict order), rows of a bucket in step order, one block table per bucket of
// ceil(bucket_length / page_size) columns padded with the row's last reserved page, and
// the bucket's split count from choose_splits over its rows' lengths.
int pkv_build_buckets(const int32_t* lengths, const int32_t* request_ids, int32_t count,
                      const int32_t* page_indptr, const int32_t* page_ids, int32_t page_size,
                      int32_t requested_splits, int32_t auto_splits, int32_t bucket_tokens,
                      int32_t single_bucket, int32_t adaptive_route, int32_t num_kv_heads,
                      int32_t policy, int32_t* out_bucket_count, int32_t* bucket_lengths,
                      int32_t* bucket_rows, int32_t* bucket_splits, int32_t* bucket_table_cols,
                      int32_t* seq_lens, int32_t* q_indices, int32_t* out_indices,
                      int32_t* tables, int64_t table_capacity, int64_t* out_table_elems) {
  if (count <= 0 || !lengths || !request_ids || !page_indptr || !page_ids || page_size <= 0 ||
      num_kv_heads <= 0)
    return PKV_ERR_INVALID_ARGUMENT;
  for (int32_t r = 0; r < count; ++r)
    if (page_indptr[r + 1] <= page_indptr[r]) return PKV_ERR_INVALID_ARGUMENT;  // :756 reads [-1]
  const int32_t single = pkv_use_single_bucket(lengths, count, single_bucket, adaptive_route);
  // Group rows (:734-745).
  std::vector<int32_t> keys;                 // bucket lengths, first-appearance order
  std::vector<std::vector<int32_t>> rows;    // offsets per bucket
  if (single) {
    keys.push_back(*std::max_element(lengths, lengths + count));
    rows.emplace_back();
    for (int32_t r = 0; r < count; ++r) rows[0].push_back(r);
  } else {
    for (int32_t r = 0; r < count; ++r) {
      const int32_t allocated = page_indptr[r + 1] - page_indptr[r];
      const int32_t key = pkv_round_bucket_length(lengths[r], bucket_tokens, allocated, page_size);
      size_t j = 0;
      while (j < keys.size() && keys[j] != key) ++j;
      if (j == keys.size()) {
        keys.push_back(key);
        rows.emplace_back();
      }
      rows[j].push_back(r);
    }
  }
  int64_t elems = 0;
  for (size_t j = 0; j < keys.size(); ++j)
    elems += (int64_t)rows[j].size() * (keys[j] > 0 ? ceil_div_pos(keys[j], page_size) : 0);
  if (out_bucket_count) *out_bucket_count = (int32_t)keys.size();
  if (out_table_elems) *out_table_elems = elems;
  if (elems > table_capacity) return PKV_ERR_CAPACITY;
  if (!bucket_lengths || !bucket_rows || !bucket_splits || !bucket_table_cols || !seq_lens ||
      !q_indices || !out_indices || (elems > 0 && !tables))
    return PKV_ERR_INVALID_ARGUMENT;
  int64_t t = 0;
  int32_t n = 0;
  std::vector<int32_t> lens;
  for (size_t j = 0; j < keys.size(); ++j) {
    const int64_t cols = keys[j] > 0 ? ceil_div_pos(keys[j], page_size) : 0;  // :748
    lens.clear();
    for (const int32_t r : rows[j]) {
      const int32_t p0 = page_indptr[r], p1 = page_indptr[r + 1];
      for (int64_t c = 0; c < cols; ++c)  // :752-757
        tables[t++] = c < p1 - p0 ? page_ids[p0 + c] : page_ids[p1 - 1];
      seq_lens[n] = lengths[r];
      q_indices[n] = request_ids[r];
      out_indices[n] = r;
      lens.push_back(lengths[r]);
      ++n;
    }
    bucket_lengths[j] = keys[j];
    bucket_rows[j] = (int32_t)rows[j].size();
    bucket_table_cols[j] = (int32_t)cols;
    bucket_splits[j] = pkv_choose_splits(lens.data(), (int32_t)lens.size(), requested_splits,
                                         auto_splits, single, num_kv_heads, policy);  // :759-761
  }
  return PKV_OK;
}

}  // extern "C"
