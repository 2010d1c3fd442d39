"""The host scheduler (pkv_schedule.cpp) under AddressSanitizer and UBSan, on the CPU.

tests/native/sched_sanitize.cpp drives pkv_workqueue_size, pkv_build_workqueue,
pkv_build_buckets and the split and route choices over random decode steps (0-300 rows,
lengths 0-300k with some negative, page sizes 1-256, short page lists, both policies),
with every output buffer sized exactly to what the call reports it needs.  Any write
past a buffer, any undefined behaviour, a built queue whose size differs from
pkv_workqueue_size's, or a crash on invalid input fails the test.
"""
import os
import shutil
import subprocess

import pytest

NATIVE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native")


def test_scheduler_is_clean_under_asan_and_ubsan():
    if shutil.which("g++") is None:
        pytest.skip("no g++")
    build = subprocess.run(["make", "-s", "-C", NATIVE, "_build/sched_sanitize"],
                           capture_output=True, text=True)
    if build.returncode != 0 and "asan" in (build.stderr + build.stdout).lower():
        pytest.skip("the sanitizer runtime is not installed: " + build.stderr[-300:])
    assert build.returncode == 0, build.stderr[-2000:]
    # verify_asan_link_order=0: the environment may preload other libraries before the
    # ASan runtime; they are left as they are.
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([os.path.join(NATIVE, "_build", "sched_sanitize"), "1500"],
                         capture_output=True, text=True, env=env, timeout=600)
    assert run.returncode == 0, (run.stdout[-1000:], run.stderr[-3000:])
    assert "ERROR: AddressSanitizer" not in run.stderr and "runtime error" not in run.stderr
    ok = int(run.stdout.split("ok ")[1].split(",")[0])
    assert ok > 1000, run.stdout
