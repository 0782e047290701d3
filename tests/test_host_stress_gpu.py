"""GPU tier: the host-pointer API from compiled C++ threads under residency
churn.  tests/stress/zq_host_stress.cpp runs 4 threads of random gemv /
gemv_batch / gemm / gemm_batch / stats / release / release_all calls on Q8_0
weights with the residency budget lowered to 4 MB, so uploads keep evicting
the resident set, and host buffers are freed and reallocated at reused
addresses after a release (the contract of the reference's
include/zen/hip_backend.h:52-58).  Every OK result must match an fp64 dot
product within 1e-4 of the absolute sum; declines are allowed, errors are
not.  build() compiles the program; the binary travels with the tree."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "stress", "_bin", "zq_host_stress")


def test_host_api_threads_under_residency_churn():
    assert os.path.exists(BIN), "tests/stress/_bin/zq_host_stress is not built: run __graft_entry__.build()"
    env = dict(os.environ, ZQ_HIP_RESIDENT_BUDGET="4000000")
    for k in ("ZEN_HIP_MIN_ELEMENTS",):
        env.pop(k, None)
    r = subprocess.run([BIN, "4", "200"], env=env, capture_output=True, text=True, timeout=150)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "stress ok" in r.stdout
    fields = dict(kv.split("=") for kv in r.stdout.split()[2:])
    assert int(fields["ok"]) > 300 and int(fields["evictions"]) > 10, r.stdout
