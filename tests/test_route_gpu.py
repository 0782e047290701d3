"""GPU tier: the drop-in exercised from compiled C++ in the reference's own
route order (src/quant.cpp:1007-1012 gemv, :1656-1659 gemm, :1521-1554
gemm_batch): try zq_hip_*, fall through to the reference's CPU quant::gemv /
quant::gemm (oracle/_ref) on any non-OK status.  The program and its checks are
tests/route/zq_route.cpp; build() compiles it where the reference tree is
present, and the binary travels with the tree."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "route", "_bin", "zq_route")


def test_cpp_route_order():
    if not os.path.exists(BIN):
        pytest.skip("tests/route/_bin/zq_route not built (needs the reference tree at build time)")
    env = {k: v for k, v in os.environ.items() if k not in ("ZEN_HIP", "ZEN_BACKEND", "ZEN_HIP_MIN_ELEMENTS")}
    r = subprocess.run([BIN], env=env, capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "route ok" in r.stdout
