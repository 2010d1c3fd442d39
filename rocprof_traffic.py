"""HBM traffic per decode launch from rocprofv3 --pmc counter CSVs.

FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are each scaled by what the same counter
reads for ``pkv_probe_copy`` of a known byte count (``hbm_probe.py copy``), then averaged
over the last ``--launches`` dispatches of the decode kernel (bench.py's decode-only pass
with ``--steps`` equal to ``--launches``, which replays the same trace sample):

  python rocprof_traffic.py --fetch F.csv --write W.csv --copy-fetch CF.csv \
      --copy-write CW.csv --copy-mib 1024 --launches 96 --workload c4 -o traffic.json

The output's ``hbm_bytes_per_launch`` is what bench.py reports as ``roofline.traffic``;
``algorithmic_bytes_per_launch`` is the same launches' KV bytes (sum of active lengths x
Hkv x 128 x 2 x element bytes) for comparison.
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(_HERE, "persistentkv-attention_amd"), _HERE):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def counter_values(path, counter, kernel_substring):
    """Per-dispatch values of ``counter`` for kernels whose name contains the substring,
    in dispatch order."""
    rows = []
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] == counter and kernel_substring in r["Kernel_Name"]:
                rows.append((int(r["Dispatch_Id"]), float(r["Counter_Value"])))
    rows.sort()
    return [v for _, v in rows]


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--fetch", required=True)
    p.add_argument("--write", required=True)
    p.add_argument("--copy-fetch", required=True)
    p.add_argument("--copy-write", required=True)
    p.add_argument("--copy-mib", type=int, required=True)
    p.add_argument("--launches", type=int, default=96)
    p.add_argument("--kernel", default="pkv::decode_kernel")
    p.add_argument("--workload", default="c4")
    p.add_argument("--kv-fp8", action="store_true", help="1-byte K/V elements (bench.py --kv-fp8)")
    p.add_argument("--seed", type=int, default=20260623)
    p.add_argument("-o", "--output", required=True)
    a = p.parse_args(argv)

    copy_bytes = a.copy_mib << 20
    cf = counter_values(a.copy_fetch, "FETCH_SIZE", "probe_copy_kernel")
    cw = counter_values(a.copy_write, "WRITE_SIZE", "probe_copy_kernel")
    fetch_scale = copy_bytes / (sum(cf) / len(cf) * 1024)
    write_scale = copy_bytes / (sum(cw) / len(cw) * 1024)
    f = counter_values(a.fetch, "FETCH_SIZE", a.kernel)[-a.launches:]
    w = counter_values(a.write, "WRITE_SIZE", a.kernel)[-a.launches:]
    fetch_bytes = sum(f) / len(f) * 1024 * fetch_scale
    write_bytes = sum(w) / len(w) * 1024 * write_scale

    import pkv_workloads as wl

    work = wl.CONFIGS[a.workload](seed=a.seed)
    elem = 1 if a.kv_fp8 else 2
    step_bytes = [sum(s.lengths) * work.hkv * 128 * 2 * elem for s in work.steps]
    from bench import trace_sample  # the trace steps bench.py's decode-only pass replays

    alg = sum(step_bytes[i] for i in trace_sample(a.launches, len(step_bytes))) / a.launches
    out = {
        "kernel": a.kernel, "workload": a.workload + ("_fp8kv" if a.kv_fp8 else ""),
        "launches": len(f),
        "fetch_kib_per_launch": round(sum(f) / len(f), 3),
        "write_kib_per_launch": round(sum(w) / len(w), 3),
        "fetch_scale": round(fetch_scale, 4), "write_scale": round(write_scale, 4),
        "hbm_bytes_per_launch": int(round(fetch_bytes + write_bytes)),
        "hbm_read_bytes_per_launch": int(round(fetch_bytes)),
        "hbm_write_bytes_per_launch": int(round(write_bytes)),
        "algorithmic_bytes_per_launch": int(round(alg)),
        "read_over_algorithmic": round(fetch_bytes / alg, 4),
    }
    with open(a.output, "w") as fh:
        json.dump(out, fh, indent=1)
        fh.write("\n")
    print(json.dumps(out))


if __name__ == "__main__":
    main()
