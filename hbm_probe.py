"""Achievable-HBM-bandwidth probes and rocprof byte-counter calibration.

The MI355X counterpart of the reference's micro_benchmarks/01_hbm_bandwidth.cu:20-51
(hbm_read / hbm_copy), driving ``pkv_probe_read`` / ``pkv_probe_copy`` of
``persistentkv-attention_amd/libpkv_probe.so`` (include/pkv_probe.h; built by
``make -C persistentkv-attention_amd/csrc``), a measurement library kept apart from the
engine's libpkv.so:

  python hbm_probe.py read            # read bandwidth for the decode kernel's access patterns
  python hbm_probe.py copy --mib 1024 # one known-size copy per launch, for rocprofv3 --pmc
  python hbm_probe.py cus             # read bandwidth of 8 .. 256 CUs, one workgroup each
  python hbm_probe.py inflight        # bandwidth and loaded latency vs bytes in flight per wave

``read`` reports GB/s per pattern (contiguous, K-operand 16 rows x 64 B, V-operand 4 rows
x 256 B) and size; sizes above the 256 MB Infinity Cache measure HBM.  ``copy`` launches
``pkv_probe_copy`` ``--iters`` times over ``--mib`` MiB: the FETCH_SIZE and WRITE_SIZE that
rocprofv3 reports per dispatch divided by the known byte count is the counter scale factor.
"""
from __future__ import annotations

import argparse
import os
import sys

import ctypes

_HERE = os.path.dirname(os.path.abspath(__file__))
PROBE_LIBRARY = os.path.join(_HERE, "persistentkv-attention_amd", "libpkv_probe.so")

PATTERNS = {0: "contiguous", 1: "K operand (16 rows x 64 B)", 2: "V operand (4 rows x 256 B)",
            3: "K whole lines via LDS (4 rows x 256 B)"}
_lib = None


def _probe_lib():
    """libpkv_probe.so with argument types declared (torch is imported first, so the
    library binds to torch's HIP runtime)."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401
        if not os.path.exists(PROBE_LIBRARY):
            raise ImportError(f"{PROBE_LIBRARY} is not built; run `make -C persistentkv-attention_amd/csrc`")
        so = ctypes.CDLL(PROBE_LIBRARY)
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32
        so.pkv_probe_read.argtypes = [vp, sz, i32, vp, vp]
        so.pkv_probe_copy.argtypes = [vp, vp, sz, vp]
        so.pkv_probe_read_cus.argtypes = [vp, sz, i32, i32, vp, vp]
        so.pkv_probe_read_inflight.argtypes = [vp, sz, i32, i32, i32, i32, vp, vp]
        for f in (so.pkv_probe_read, so.pkv_probe_copy, so.pkv_probe_read_cus,
                  so.pkv_probe_read_inflight):
            f.restype = ctypes.c_int
        _lib = so
    return _lib


def _time_ms(torch, fn, iters):
    fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / iters


def _check(lib, status):
    if status != 0:
        raise RuntimeError(f"probe launch failed with status {status}")


def run_read(sizes_mib, iters):
    import torch

    lib = _probe_lib()
    dev = torch.device("cuda:0")
    buf = torch.empty(max(sizes_mib) << 20, dtype=torch.uint8, device=dev).random_(0, 256)
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    rows = []
    for pattern, name in PATTERNS.items():
        for mib in sizes_mib:
            nbytes = mib << 20
            ms = _time_ms(torch, lambda: _check(lib, lib.pkv_probe_read(
                buf.data_ptr(), nbytes, pattern, sink.data_ptr(), stream)), iters)
            rows.append((name, mib, nbytes / ms / 1e6, ms * 1e3))
            print(f"read {name:28s} {mib:6d} MiB: {nbytes / ms / 1e6:8.0f} GB/s "
                  f"({ms * 1e3:8.1f} us)", flush=True)
    return rows


def run_cus(counts, mib, iters):
    """Read bandwidth of 1 GiB-class streams with `n` workgroups of 8 waves, at most one
    per CU: the per-CU ceiling when n is below the CU count."""
    import torch

    lib = _probe_lib()
    dev = torch.device("cuda:0")
    nbytes = mib << 20
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(0, 256)
    sink = torch.zeros(65536, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    for n in counts:
        ms = _time_ms(torch, lambda: _check(lib, lib.pkv_probe_read_cus(
            buf.data_ptr(), nbytes, 1, n, sink.data_ptr(), stream)), iters)
        gbps = nbytes / ms / 1e6
        print(f"cus {n:4d} workgroups x 8 waves (K operand): {gbps:8.0f} GB/s, {gbps / n:6.1f} GB/s "
              f"per workgroup ({ms * 1e3:8.1f} us)", flush=True)


def run_inflight(counts, mib, iters, patterns):
    """Read bandwidth of `n` workgroups (at most one per CU) for 8 and 16 waves per
    workgroup and 1, 2 or 4 chunks of 4 KB in flight per wave.  Latency is Little's law:
    bytes in flight per CU / bandwidth per CU."""
    import torch

    lib = _probe_lib()
    dev = torch.device("cuda:0")
    nbytes = mib << 20
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(0, 256)
    sink = torch.zeros(65536, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    print("| pattern | waves | KB in flight per wave | workgroups | GB/s | GB/s per CU | latency us |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for pattern in patterns:
        for waves in (8, 16):
            for u in (1, 2, 4):
                for n in counts:
                    ms = _time_ms(torch, lambda: _check(lib, lib.pkv_probe_read_inflight(
                        buf.data_ptr(), nbytes, pattern, waves, u, n, sink.data_ptr(), stream)), iters)
                    gbps = nbytes / ms / 1e6
                    per_cu = gbps / n
                    kb = waves * u * 4
                    print(f"| {PATTERNS[pattern]} | {waves} | {4 * u} | {n} | {gbps:.0f} | "
                          f"{per_cu:.1f} | {kb * 1024 / (per_cu * 1e3):.2f} |", flush=True)


def run_copy(mib, iters):
    import torch

    lib = _probe_lib()
    dev = torch.device("cuda:0")
    nbytes = mib << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(0, 256)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream().cuda_stream
    ms = _time_ms(torch, lambda: _check(lib, lib.pkv_probe_copy(
        src.data_ptr(), dst.data_ptr(), nbytes, stream)), iters)
    if not torch.equal(src, dst):
        raise RuntimeError("probe copy produced wrong bytes")
    print(f"copy {mib} MiB per launch x {iters + 1} launches: read {nbytes} B + write {nbytes} B "
          f"per launch, {2 * nbytes / ms / 1e6:.0f} GB/s read+write ({ms * 1e3:.1f} us)", flush=True)


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = p.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("read")
    r.add_argument("--mib", type=int, nargs="+", default=[4096, 256, 64])
    r.add_argument("--iters", type=int, default=10)
    u = sub.add_parser("cus")
    u.add_argument("--workgroups", type=int, nargs="+", default=[8, 32, 64, 128, 160, 192, 256])
    u.add_argument("--mib", type=int, default=1024)
    u.add_argument("--iters", type=int, default=3)
    f = sub.add_parser("inflight")
    f.add_argument("--workgroups", type=int, nargs="+", default=[8, 128, 256])
    f.add_argument("--mib", type=int, default=4096)
    f.add_argument("--iters", type=int, default=2)
    f.add_argument("--patterns", type=int, nargs="+", default=[1, 2, 3])
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=1024)
    c.add_argument("--iters", type=int, default=4)
    a = p.parse_args(argv)
    if a.cmd == "read":
        run_read(a.mib, a.iters)
    elif a.cmd == "cus":
        run_cus(a.workgroups, a.mib, a.iters)
    elif a.cmd == "inflight":
        run_inflight(a.workgroups, a.mib, a.iters, a.patterns)
    else:
        run_copy(a.mib, a.iters)


if __name__ == "__main__":
    main()
