"""Pure-Python restatement of the reference's host scheduling (test infrastructure only).

Restates tests/benchmark_serving_trace.py of ahmed123hds/persistentkv-attention:
  round_up4                    :324-325
  choose_splits                :328-367
  choose_workqueue_row_splits  :370-393
  model_bucket_splits          :396-402
  model_workqueue_splits       :405-415
  estimate_route_ms            :418-442 (useful_kv_mb_for_state :511-513)
  choose_adaptive_route        :445-488
  round_bucket_length          :316-321 (rounded_length :159-160)
  use_single_bucket            :491-504 (use_single_bucket_for_state)
  build_workqueue              :668-729 (work-queue branch of compile_persistentkv_metadata)
  build_buckets                :731-780 (length-bucket branch of compile_persistentkv_metadata)

The reference reads HQ/HKV/DIM and the cost constants from module globals (:33-43);
here they are keyword arguments with the reference's values as defaults.  Integer
results must match the C++ builder bit for bit; float estimates use the same operation
order (CPython floats are IEEE doubles).
"""
from __future__ import annotations

import math

REFERENCE_COST = dict(hq=32, hkv=8, dim=128, sm_count=28, roofline_read_gbps=302.0,
                      launch_overhead_us=8.0, min_ctas_per_sm=4.0, supported_gqa=4,
                      min_long_context=16384)


def round_up4(value):
    return ((value + 3) // 4) * 4


def choose_splits(lengths, requested_splits, auto_splits, single_bucket, hkv=8):
    if not auto_splits:
        return requested_splits
    batch = len(lengths)
    tile_counts = [(length + 31) // 32 for length in lengths]
    t_max = max(tile_counts)
    t_min = min(tile_counts)
    if single_bucket:
        if batch >= 8:
            return max(4, min(40, t_min))
        if batch == 4:
            return max(4, min(16, t_min))
        if batch == 2:
            return max(4, min(24, t_min))
        if t_max >= 1024:
            return max(4, min(36, t_min))
        return max(4, min(24, t_min))
    if batch >= 8:
        return max(4, min(24, t_min))
    if batch == 4:
        return max(4, min(28, t_min))
    if batch == 2 and t_max >= 1024:
        return max(4, min(32, t_min))
    occupancy = math.ceil(320 / (hkv * batch))
    length_based = math.ceil(t_max / 32)
    splits = round_up4(max(occupancy, length_based))
    if t_max <= 384:
        splits = min(splits, 24)
    if batch >= 8:
        splits = min(splits, 40)
    if batch <= 2 and t_max >= 1024:
        splits = max(splits, 32)
    return max(4, min(splits, 48, t_min))


def choose_workqueue_row_splits(length, active_count, requested_splits, auto_splits, hkv=8):
    if not auto_splits:
        return requested_splits
    tiles = max(1, (length + 31) // 32)
    occupancy_floor = round_up4(math.ceil(256 / (hkv * max(1, active_count))))
    length_target = round_up4(math.ceil(tiles / 64))
    splits = max(occupancy_floor, length_target)
    if active_count >= 8:
        splits = min(splits, 24)
    elif active_count >= 4:
        splits = min(splits, 32)
    elif active_count == 2:
        splits = min(splits, 40)
    else:
        splits = min(splits, 48)
    return max(4, min(splits, 48, tiles))


def model_bucket_splits(lengths, hkv=8):
    active = len(lengths)
    max_tiles = max((length + 31) // 32 for length in lengths)
    min_tiles = min((length + 31) // 32 for length in lengths)
    occupancy = math.ceil(256 / (hkv * max(1, active)))
    length_based = math.ceil(max_tiles / 96)
    return max(4, min(round_up4(max(occupancy, length_based)), 48, min_tiles))


def model_workqueue_splits(lengths, hkv=8):
    return max(choose_workqueue_row_splits(length, len(lengths), 1, True, hkv) for length in lengths)


def useful_kv_mb(lengths, hkv=8, dim=128):
    return sum(lengths) * hkv * dim * 2 * 2 / (1024.0 * 1024.0)


def estimate_route_ms(lengths, route, splits, cost=REFERENCE_COST):
    hq, hkv, dim = cost["hq"], cost["hkv"], cost["dim"]
    kv_mb = useful_kv_mb(lengths, hkv, dim)
    kv_ms = kv_mb / cost["roofline_read_gbps"]
    active = len(lengths)
    unique_lengths = len(set(lengths))
    if route == "flashinfer":
        ctas_per_sm = active * hkv / cost["sm_count"]
        launch_count = 1
        merge_mb = 0.0
    elif route == "persistentkv_bucket":
        ctas_per_sm = active * hkv * splits / cost["sm_count"]
        launch_count = 2 * unique_lengths
        merge_mb = active * hq * splits * (2 + dim) * 4 / (1024.0 * 1024.0)
    elif route == "persistentkv_workqueue":
        ctas_per_sm = active * hkv * splits / cost["sm_count"]
        launch_count = 2
        merge_mb = active * hq * splits * (2 + dim) * 4 / (1024.0 * 1024.0)
    else:
        raise ValueError(f"unknown route: {route}")
    occupancy_penalty = max(1.0, cost["min_ctas_per_sm"] / max(ctas_per_sm, 1e-6))
    launch_ms = launch_count * cost["launch_overhead_us"] / 1000.0
    merge_ms = merge_mb / cost["roofline_read_gbps"]
    return kv_ms * occupancy_penalty + merge_ms + launch_ms


def choose_adaptive_route(lengths, cost=REFERENCE_COST):
    """Returns ``(route, splits, estimated_ms)`` (benchmark_serving_trace.py:445-488)."""
    hkv = cost["hkv"]
    gqa_ratio = cost["hq"] // hkv
    flash = ("flashinfer", 1, estimate_route_ms(lengths, "flashinfer", 1, cost))
    if cost["supported_gqa"] and gqa_ratio != cost["supported_gqa"]:
        return flash
    if max(lengths) < cost["min_long_context"]:
        return flash
    candidates = [flash]
    active = len(lengths)
    if active <= 1:
        s = model_bucket_splits(lengths, hkv)
        candidates.append(("persistentkv_bucket", s, estimate_route_ms(lengths, "persistentkv_bucket", s, cost)))
    if active >= 8:
        s = model_workqueue_splits(lengths, hkv)
        candidates.append(("persistentkv_workqueue", s,
                           estimate_route_ms(lengths, "persistentkv_workqueue", s, cost)))
    return min(candidates, key=lambda item: item[2])


def build_workqueue(lengths, request_ids, page_lists, page_size, requested_splits, auto_splits,
                    hkv=8):
    """One decode step's compact work queue (benchmark_serving_trace.py:668-729).

    ``page_lists[r]`` is the reserved physical page list of active row ``r``.
    """
    bucket_length = max(lengths)
    page_count = math.ceil(bucket_length / page_size)
    rows, seq_lens, q_indices, out_indices = [], [], [], []
    work_items = []
    split_offsets = [0]
    row_splits_all = []
    for offset, length in enumerate(lengths):
        pages = list(page_lists[offset][:page_count])
        if len(pages) < page_count:
            pages = pages + [page_lists[offset][-1]] * (page_count - len(pages))
        rows.append(pages)
        seq_lens.append(length)
        q_indices.append(request_ids[offset])
        out_indices.append(offset)
        row_splits = choose_workqueue_row_splits(length, len(lengths), requested_splits,
                                                 auto_splits, hkv)
        row_splits_all.append(row_splits)
        total_tiles = (length + 31) // 32
        for split in range(row_splits):
            tile_begin = (total_tiles * split) // row_splits
            tile_end = (total_tiles * (split + 1)) // row_splits
            if tile_begin >= tile_end:
                continue
            for kvh in range(hkv):
                work_items.append([offset, kvh, split, tile_begin, tile_end])
        split_offsets.append(split_offsets[-1] + row_splits)
    return dict(bucket_length=int(bucket_length), block_table=rows, seq_lens=seq_lens,
                q_indices=q_indices, out_indices=out_indices, work_items=work_items,
                split_offsets=split_offsets, total_partial_slots=split_offsets[-1],
                splits=max(1, max(row_splits_all)))


def round_bucket_length(length, bucket_tokens, allocated_pages, page_size=16):
    """benchmark_serving_trace.py:316-321 with rounded_length (:159-160) at ``page_size``."""
    if bucket_tokens <= 0:
        return length
    bucket = ((length + bucket_tokens - 1) // bucket_tokens) * bucket_tokens
    bucket = max(page_size, ((bucket + page_size - 1) // page_size) * page_size)
    return min(bucket, allocated_pages * page_size)


def use_single_bucket(lengths, requested_single_bucket, adaptive_route):
    """use_single_bucket_for_state, benchmark_serving_trace.py:491-504."""
    if requested_single_bucket:
        return True
    if not adaptive_route:
        return False
    active = len(lengths)
    if active <= 1:
        return False
    return len(set(lengths)) >= max(3, active - 1)


def build_buckets(lengths, request_ids, page_lists, page_size, requested_splits, auto_splits,
                  bucket_tokens=0, single_bucket=False, adaptive_route=False, hkv=8):
    """One decode step's length buckets (benchmark_serving_trace.py:731-780): a list of
    dicts with bucket_length, block_table (rows), seq_lens, q_indices, out_indices, splits,
    in the dict order the reference builds them."""
    state_single = use_single_bucket(lengths, single_bucket, adaptive_route)
    buckets = {}
    if state_single:
        buckets[max(lengths)] = list(range(len(lengths)))
    else:
        for offset, length in enumerate(lengths):
            key = round_bucket_length(length, bucket_tokens, len(page_lists[offset]), page_size)
            buckets.setdefault(key, []).append(offset)
    result = []
    for bucket_length, offsets in buckets.items():
        page_count = math.ceil(bucket_length / page_size)
        rows, seq_lens = [], []
        for offset in offsets:
            pages = list(page_lists[offset][:page_count])
            if len(pages) < page_count:
                pages = pages + [page_lists[offset][-1]] * (page_count - len(pages))
            rows.append(pages)
            seq_lens.append(lengths[offset])
        result.append(dict(bucket_length=int(bucket_length), block_table=rows, seq_lens=seq_lens,
                           q_indices=[request_ids[o] for o in offsets], out_indices=list(offsets),
                           splits=choose_splits(seq_lens, requested_splits, auto_splits,
                                                state_single, hkv)))
    return result
