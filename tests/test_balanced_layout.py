"""Layout of the balanced work-queue schedule, checked on the CPU.

The decode kernel (balanced_decode_kernel) lays the (row, kv head) pairs' tiles end to end
and gives wave v of V the positions [floor(vT/V), floor((v+1)T/V)); the piece of pair p in
wave v is written to state group p + v.  The merge (balanced_merge_kernel) folds, for pair
p, the groups p + va .. p + vb with va, vb the waves of the pair's first and last tile
(position x lies in wave ceil((x+1)V/T) - 1), skipping waves with no position by the
empty-split rule floor(vT/V) == floor((v+1)T/V).  This simulation walks the decode's pieces
tile by tile and checks what the merge needs: every tile is covered once, no two pieces
share a group, the groups stay below B*Hkv + V - 1, and the merge's live groups for each
pair are exactly the groups its pieces were written to.
"""
import random


def decode_pieces(tiles_per_row, hkv, waves):
    """(pair, wave, first tile, end tile) of every piece, walked position by position."""
    pairs = [(r, k) for r in range(len(tiles_per_row)) for k in range(hkv)]
    starts, x = [], 0
    for r, k in pairs:
        starts.append(x)
        x += tiles_per_row[r]
    total = x
    pieces = []
    for v in range(waves):
        lo, hi = v * total // waves, (v + 1) * total // waves
        pos = lo
        while pos < hi:
            p = max(i for i, s0 in enumerate(starts) if s0 <= pos and tiles_per_row[pairs[i][0]] > 0)
            t = tiles_per_row[pairs[p][0]]
            t0 = pos - starts[p]
            t1 = min(t, t0 + (hi - pos))
            pieces.append((p, v, t0, t1))
            pos += t1 - t0
    return pairs, starts, total, pieces


def merge_groups(p, starts, tiles, total, waves):
    if tiles == 0:
        return []
    x0 = starts[p]
    va = ((x0 + 1) * waves + total - 1) // total - 1
    vb = ((x0 + tiles) * waves + total - 1) // total - 1
    live = [v for v in range(va, vb + 1)
            if total * v // waves != total * (v + 1) // waves]
    return [p + v for v in live]


def check(tiles_per_row, hkv, waves):
    pairs, starts, total, pieces = decode_pieces(tiles_per_row, hkv, waves)
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
        assert merge_groups(p, starts, tiles_per_row[pairs[p][0]], total, waves) == written


def test_layout_hand_cases():
    check([125, 19, 254], 2, 1024)      # fewer tiles than waves (the G = 16 case)
    check([3, 0, 5], 8, 16)             # a row with no tokens
    check([1024, 1024, 20, 10], 8, 64)  # C4-like, more tiles than waves
    check([1], 1, 7)                    # one tile, many waves
    check([7, 7, 7], 3, 7)              # equal shares


def test_layout_random():
    rng = random.Random(5)
    for _ in range(300):
        rows = rng.randint(1, 9)
        tiles = [rng.choice([0, 1, 2, 3, rng.randint(1, 60)]) for _ in range(rows)]
        if sum(tiles) == 0:
            tiles[0] = 1
        check(tiles, rng.choice([1, 2, 4, 8]), rng.choice([1, 3, 4, 16, 37, 64, 200]))
