"""Fits the MI355X cost model of the adaptive router to measured step times.

The router (pkv_choose_adaptive_route, policy MI355X) prices a step's two routes with the
makespan model of pkv_schedule.cpp (mi355x_route_us):

  split grid, S > 1:  max(share, unit) * tile_us + rounds * unit_round_us + grid_merge_us + 2 L
  work queue:         share * tile_us + queue_merge_us + 2 L

with share = (sum over rows of ceil(len / 32)) * Hkv / CUs tiles per CU, unit = ceil(longest
row's tiles / S), rounds = ceil(rows * Hkv * S / (2 CUs)), tile_us the time one CU takes
for one 16 KB tile at read_gbps / CUs, and L the launch gap (launch_overhead_us, kept as
measured).  The model is linear in (tile_us, unit_round_us, grid_merge_us,
queue_merge_us); this fits them by non-negative least squares to the samples of
``pkv_serving.py --calibrate FILE`` (both routes timed on sampled steps of every
configuration and review trace), leaving out the work queue's samples at G > 16, where
the op runs one workgroup per item rather than the balanced schedule the model prices.

  python pkv_calibrate.py profiles/cost_model_calibration.json
"""
from __future__ import annotations

import argparse
import json
import math

import numpy as np
from scipy.optimize import nnls

TILE_TOKENS = 32
TILE_BYTES = TILE_TOKENS * 128 * 2 * 2  # one tile of K and V at D = 128, 2-byte elements
LAUNCH_US = 1.5


def features(lengths, hkv, splits, cus):
    tiles = [(max(n, 0) + TILE_TOKENS - 1) // TILE_TOKENS for n in lengths]
    share = sum(tiles) * hkv / cus
    s = max(1, splits)
    unit = -(-max(max(tiles), 1) // s)
    rounds = math.ceil(len(lengths) * hkv * s / (2.0 * cus))
    return share, unit, rounds


def fit(samples, cus):
    """(tile_us, unit_round_us, grid_merge_us, queue_merge_us) and the rows used."""
    rows, target = [], []
    for smp in samples:
        share, unit, rounds = features(smp["lengths"], smp["hkv"], smp["grid_splits"], cus)
        if smp["grid_splits"] > 1:
            rows.append([max(share, unit), rounds, 1.0, 0.0])
            target.append(smp["grid_us"] - 2 * LAUNCH_US)
        if smp["hq"] // smp["hkv"] <= 16:
            rows.append([share, 0.0, 0.0, 1.0])
            target.append(smp["queue_us"] - 2 * LAUNCH_US)
    a, b = np.array(rows), np.array(target)
    x, _ = nnls(a, b)
    return x, a, b


def constants(x, cus):
    tile_us, round_us, grid_merge, queue_merge = (float(v) for v in x)
    return {"read_gbps": TILE_BYTES * cus / (tile_us * 1e3), "unit_round_us": round_us,
            "grid_merge_us": grid_merge, "queue_merge_us": queue_merge,
            "launch_overhead_us": LAUNCH_US}


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("calibration", help="the JSON file pkv_serving.py --calibrate writes")
    a = p.parse_args(argv)
    with open(a.calibration) as fh:
        data = json.load(fh)
    cus = data.get("compute_units", 256)
    x, rows, target = fit(data["samples"], cus)
    pred = rows @ x
    err = np.abs(pred - target) / np.maximum(target, 1e-9)
    print(json.dumps({k: round(v, 3) for k, v in constants(x, cus).items()}))
    print(f"{len(target)} route samples: relative error median {np.median(err):.3f}, "
          f"p90 {np.quantile(err, 0.9):.3f}")


if __name__ == "__main__":
    main()
