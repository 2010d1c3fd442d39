"""Caller-built work queues for the work-queue op's contract tests.

The reference's work-queue kernels honour each item's explicit tile range (cuh:298-337),
write the neutral state for an item with no tiles (cuh:340-363) and merge every slot of
a row (cuh:753-784).  Any queue that writes every slot of every row once is therefore
well defined there, not only the one compile_persistentkv_metadata builds
(benchmark_serving_trace.py:668-729).  The builders below make such queues: each returns
(work_items, split_offsets, tiles_covered) with tiles_covered[b] the tile prefix that
row b's items cover (the whole row unless stated otherwise).
"""
from __future__ import annotations

import random

TILE = 32


def tiles_of(length):
    return (length + TILE - 1) // TILE


def _offsets(splits):
    offsets = [0]
    for s in splits:
        offsets.append(offsets[-1] + s)
    return offsets


def front_loaded(lengths, hkv, splits):
    """Split s < S - 1 takes tile s alone and the last non-empty split the rest; splits
    past the row's tiles get explicit empty items.  With fewer tiles than splits the
    tiles sit in the first splits (the builder's row-local bounds put them elsewhere)."""
    items = []
    for row, length in enumerate(lengths):
        t = tiles_of(length)
        for split in range(splits):
            if split < splits - 1:
                tb, te = (split, split + 1) if split < t else (t, t)
            else:
                tb, te = (min(split, t), t)
            for kvh in range(hkv):
                items.append([row, kvh, split, tb, te])
    return items, _offsets([splits] * len(lengths)), [tiles_of(n) for n in lengths]


def random_partition(lengths, hkv, splits, seed, prefix=None):
    """Each row's tiles [0, P) cut at random points into `splits` contiguous ranges (some
    empty), assigned to the splits in a random order; every kv head gets its own cut and
    order, and the items are shuffled.  P is the whole row, or `prefix(tiles)` tiles."""
    rng = random.Random(seed)
    items, covered = [], []
    for row, length in enumerate(lengths):
        t = tiles_of(length)
        p = t if prefix is None else max(0, min(t, prefix(t)))
        covered.append(p)
        for kvh in range(hkv):
            cuts = sorted(rng.randint(0, p) for _ in range(splits - 1))
            bounds = [0] + cuts + [p]
            order = list(range(splits))
            rng.shuffle(order)
            for i, split in enumerate(order):
                items.append([row, kvh, split, bounds[i], bounds[i + 1]])
    rng.shuffle(items)
    return items, _offsets([splits] * len(lengths)), covered


def per_row_splits(lengths, hkv, row_splits, seed):
    """random_partition with a different split count per row (rows of 1 split included)."""
    rng = random.Random(seed)
    items = []
    for row, length in enumerate(lengths):
        t = tiles_of(length)
        s = row_splits[row]
        for kvh in range(hkv):
            cuts = sorted(rng.randint(0, t) for _ in range(s - 1))
            bounds = [0] + cuts + [t]
            for split in range(s):
                items.append([row, kvh, split, bounds[split], bounds[split + 1]])
    return items, _offsets(row_splits), [tiles_of(n) for n in lengths]


def formula_markers(items):
    """The same queue with every range given as -1 (the row-local split bounds,
    cuh:330-337)."""
    return [[r, k, s, -1, -1] for r, k, s, _, _ in items]
