"""The MI355X cost model of the adaptive router against measured step times
(profiles/cost_model_calibration.json: both routes, the split grid with the router's split
count and the work queue with the MI355X planner, timed on up to 6 sampled steps of each of
this engine's configurations and the reference's review traces by
``pkv_serving.py --calibrate``).

* The preset's constants are the non-negative least-squares fit of the model to those
  times (pkv_calibrate.py), so they follow the measurements, not a hand setting.
* With the preset, the router takes the measured-faster route on every sampled step whose
  two routes differ by more than 3 %, and its choices cost less than 1 % over always
  taking the faster route.
* A planted mistake (the queue's fixed cost swapped with the grid's) fails the second.
"""
import json
import os

import pytest

import pkv_calibrate as cal
import pkv_native as nat

CALIBRATION = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                           "profiles", "cost_model_calibration.json")


@pytest.fixture(scope="module")
def data():
    with open(CALIBRATION) as fh:
        return json.load(fh)


def test_preset_is_the_fit_of_the_measurements(data):
    x, _, _ = cal.fit(data["samples"], data["compute_units"])
    fitted = cal.constants(x, data["compute_units"])
    m = nat.cost_model(nat.POLICY_MI355X)
    assert m.read_gbps == pytest.approx(fitted["read_gbps"], rel=0.01)
    assert m.unit_round_us == pytest.approx(fitted["unit_round_us"], abs=0.05)
    assert m.grid_merge_us == pytest.approx(fitted["grid_merge_us"], abs=0.05)
    assert m.queue_merge_us == pytest.approx(fitted["queue_merge_us"], abs=0.05)
    assert m.launch_overhead_us == fitted["launch_overhead_us"]


def _route_costs(data, **overrides):
    """(steps where a clearly faster route was missed, total chosen us, total best us)."""
    missed, chosen, best = [], 0.0, 0.0
    for s in data["samples"]:
        m = nat.cost_model(nat.POLICY_MI355X, num_q_heads=s["hq"], num_kv_heads=s["hkv"],
                           **overrides)
        route, _, _ = nat.choose_adaptive_route(s["lengths"], m)
        got = s["grid_us"] if route == "persistentkv_bucket" else s["queue_us"]
        low, high = sorted((s["grid_us"], s["queue_us"]))
        chosen += got
        best += low
        if got > low and high > 1.03 * low:
            missed.append((s["workload"], s["step"], got, low))
    return missed, chosen, best


def test_router_takes_the_measured_faster_route(data):
    missed, chosen, best = _route_costs(data)
    assert not missed, missed
    assert chosen <= 1.01 * best


def test_planted_cost_swap_fails(data):
    m = nat.cost_model(nat.POLICY_MI355X)
    missed, chosen, best = _route_costs(data, grid_merge_us=m.queue_merge_us,
                                        queue_merge_us=m.grid_merge_us)
    assert missed and chosen > 1.01 * best
