"""Layout of the balanced work-queue schedule, checked on the CPU.

The decode kernel (balanced_decode_kernel) lays out each (row, kv head) pair with tiles as
H start-up positions (no work; they charge each piece its fixed cost) followed by its
tiles, pairs end to end, and gives wave v of V the positions [floor(vT/V), floor((v+1)T/V));
the piece of pair p in wave v (when it holds tiles) is written to state group p + v.  The
merge (balanced_merge_kernel) folds, for pair p, the groups p + va .. p + vb with va, vb the
waves of the pair's first and last tile (position x lies in wave ceil((x+1)V/T) - 1),
skipping waves with no position by the empty-split rule floor(vT/V) == floor((v+1)T/V).
This simulation walks the decode's pieces position by position and checks what the merge
needs: every tile is covered once, no two pieces share a group, the groups stay below
B*Hkv + V - 1, and the merge's live groups for each pair are exactly the groups its pieces
were written to.  H is read from the kernel source (kBalPieceCost); 0 and 3 are checked too.
"""
import os
import random
import re

import pytest

_SRC = os.path.join(os.path.dirname(__file__), "..", "persistentkv-attention_amd", "csrc",
                    "pkv_decode.hip")
KERNEL_H = int(re.search(r"constexpr int kBalPieceCost = (\d+);", open(_SRC).read()).group(1))


def decode_pieces(tiles_per_row, hkv, waves, h):
    """(pair, wave, first tile, end tile) of every piece, walked position by position."""
    pairs = [(r, k) for r in range(len(tiles_per_row)) for k in range(hkv)]
    starts, x = [], 0  # first position of each pair (its start-up positions come first)
    for r, k in pairs:
        starts.append(x)
        x += tiles_per_row[r] + h if tiles_per_row[r] > 0 else 0
    total = x
    pieces = []
    for v in range(waves):
        lo, hi = v * total // waves, (v + 1) * total // waves
        pos = lo
        while pos < hi:
            p = max(i for i, s0 in enumerate(starts) if s0 <= pos and tiles_per_row[pairs[i][0]] > 0)
            t = tiles_per_row[pairs[p][0]]
            e = pos - starts[p]
            assert 0 <= e < t + h
            if e < h:  # a start-up position: no work
                pos += 1
                continue
            t0 = e - h
            t1 = min(t, t0 + (hi - pos))
            pieces.append((p, v, t0, t1))
            pos += t1 - t0
    return pairs, starts, total, pieces


def merge_groups(p, starts, tiles, total, waves, h):
    if tiles == 0:
        return []
    x0 = starts[p] + h
    va = ((x0 + 1) * waves + total - 1) // total - 1
    vb = ((x0 + tiles) * waves + total - 1) // total - 1
    live = [v for v in range(va, vb + 1)
            if total * v // waves != total * (v + 1) // waves]
    return [p + v for v in live]


def check(tiles_per_row, hkv, waves, h):
    pairs, starts, total, pieces = decode_pieces(tiles_per_row, hkv, waves, h)
    covered = {}
    for p, v, t0, t1 in pieces:
        assert t0 < t1
        for t in range(t0, t1):
            covered[(p, t)] = covered.get((p, t), 0) + 1
    assert sorted(covered.values()) == [1] * sum(tiles_per_row[r] for r, _ in pairs)
    groups = [p + v for p, v, _, _ in pieces]
    assert len(groups) == len(set(groups))
    assert all(g <= len(pairs) + waves - 2 for g in groups)
    for p in range(len(pairs)):
        written = sorted(pp + v for pp, v, _, _ in pieces if pp == p)
        assert merge_groups(p, starts, tiles_per_row[pairs[p][0]], total, waves, h) == written


@pytest.mark.parametrize("h", sorted({0, KERNEL_H, 3}))
def test_layout_hand_cases(h):
    check([125, 19, 254], 2, 1024, h)      # fewer positions than waves (the G = 16 case)
    check([3, 0, 5], 8, 16, h)             # a row with no tokens
    check([1024, 1024, 20, 10], 8, 64, h)  # C4-like, more tiles than waves
    check([1], 1, 7, h)                    # one tile, many waves
    check([7, 7, 7], 3, 7, h)              # equal shares
    check([1, 1, 1, 1, 1], 4, 64, h)       # one-tile pairs, waves that hold only start-up


@pytest.mark.parametrize("h", sorted({0, KERNEL_H, 3}))
def test_layout_random(h):
    rng = random.Random(5 + h)
    for _ in range(300):
        rows = rng.randint(1, 9)
        tiles = [rng.choice([0, 1, 2, 3, rng.randint(1, 60)]) for _ in range(rows)]
        if sum(tiles) == 0:
            tiles[0] = 1
        check(tiles, rng.choice([1, 2, 4, 8]), rng.choice([1, 3, 4, 16, 37, 64, 200]), h)


def test_start_up_positions_shift_tiles_away_from_short_rows():
    """With H > 0 a wave that starts many short pairs holds fewer tiles than one inside a
    long pair (the point of the start-up positions); with H = 0 the shares are equal."""
    def tiles_of_waves(h):
        _, _, _, pieces = decode_pieces([400] + [2] * 40, 1, 16, h)
        per_wave = [0] * 16
        for _, v, t0, t1 in pieces:
            per_wave[v] += t1 - t0
        return per_wave[0], per_wave[15]  # inside the 400-tile row; among the 2-tile rows
    inside, among_short = tiles_of_waves(0)
    assert abs(inside - among_short) <= 1
    inside, among_short = tiles_of_waves(max(KERNEL_H, 1))
    assert among_short < inside


def test_a_merge_that_does_not_skip_empty_waves_fails_when_waves_outnumber_positions():
    """Planted mistake: folding every group p + va .. p + vb (no empty-wave skip) reads
    groups no piece wrote as soon as some wave holds no position (T < V), and only then."""
    def unskipped(p, starts, tiles, total, waves, h):
        if tiles == 0:
            return []
        x0 = starts[p] + h
        va = ((x0 + 1) * waves + total - 1) // total - 1
        vb = ((x0 + tiles) * waves + total - 1) // total - 1
        return [p + v for v in range(va, vb + 1)]
    for tiles, hkv, waves, fewer in (([125, 19, 254], 2, 1024, True), ([1024, 1024, 20], 8, 64, False)):
        pairs, starts, total, pieces = decode_pieces(tiles, hkv, waves, KERNEL_H)
        assert (total < waves) == fewer
        mismatch = any(
            unskipped(p, starts, tiles[pairs[p][0]], total, waves, KERNEL_H)
            != sorted(pp + v for pp, v, _, _ in pieces if pp == p) for p in range(len(pairs)))
        assert mismatch == fewer
