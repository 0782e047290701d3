"""GPU tier: zq_hip_gemm_dev_noalloc, the GEMM entry point that allocates
nothing (its workspace is the library's fixed device scratch), against
zq_hip_gemm_dev with a caller workspace on the same inputs: bit-identical,
on consecutive calls whose second input is smaller (the scratch keeps the
previous call's contents), for int8 and fp32 activations, the split-K and the
unsplit kernels; and a request beyond the scratch is refused."""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
DEV = "cuda:0"


def _run_pair(zq, orc, fmt, act, m, n, k, seed):
    w = torch.zeros(zq.weight_bytes(fmt, n, k), dtype=torch.uint8, device=DEV)
    zq.synth_weights_dev(fmt, seed, w, n, k)
    X = torch.from_numpy(orc.gen_normal(seed + 1, m * k)).to(DEV)
    Y0 = torch.full((m * n,), float("nan"), device=DEV)
    Y1 = torch.full((m * n,), float("nan"), device=DEV)
    wsb = zq.gemm_workspace_bytes(fmt, m, n, k, act)
    assert wsb <= zq.noalloc_scratch_bytes()
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    zq.gemm_dev(fmt, w, X, Y0, m, n, k, act, ws, wsb)
    zq.gemm_dev_noalloc(fmt, w, X, Y1, m, n, k, act)
    torch.cuda.synchronize()
    assert torch.equal(Y0, Y1), f"noalloc differs: fmt={fmt} act={act} {m}x{n}x{k}"
    return Y1


@pytest.mark.parametrize("fmt,act,big,small", [
    (O.Q8_0, 1, (512, 4096, 4096), (37, 1000, 2048)),     # 128-token tile, then the split 32-token tile
    (O.Q8_0, 1, (32, 4096, 14336), (3, 301, 14336)),      # split-K both times, odd output count second
    (O.Q4_0, 1, (2048, 1024, 4096), (70, 300, 320)),      # large M, then the staged kernel
    (O.Q8_0, 2, (64, 2048, 4096), (5, 300, 4096)),        # fp32 activations (split-K partials in scratch)
    (O.Q6_K, 2, (129, 512, 2048), (1, 70, 768)),
    (O.Q4_K, 2, (129, 512, 2048), (1, 70, 768)),      # split activations in scratch
    (O.Q5_K, 2, (300, 256, 4096), (17, 40, 512)),
])
def test_noalloc_matches_workspace_entry_point(zq, orc, fmt, act, big, small):
    _run_pair(zq, orc, fmt, act, *big, seed=900)
    Y = _run_pair(zq, orc, fmt, act, *small, seed=910)
    assert torch.isfinite(Y).all()


def test_noalloc_refuses_beyond_scratch(zq):
    m, n, k = 8192, 4096, 14336  # 117 MB of int8 activations + scales
    assert zq.gemm_workspace_bytes(O.Q8_0, m, n, k, zq.ACT_INT8) > zq.noalloc_scratch_bytes()
    # real operands of the full sizes (zeros), so a regression of the size
    # check would run a valid GEMM rather than touch unmapped memory
    w = torch.zeros(zq.weight_bytes(O.Q8_0, n, k), dtype=torch.uint8, device=DEV)
    X = torch.zeros(m * k, device=DEV)
    Y = torch.full((m * n,), float("nan"), device=DEV)
    st = zq.lib().zq_hip_gemm_dev_noalloc(O.Q8_0, w.data_ptr(), X.data_ptr(), Y.data_ptr(), m, n, k, zq.ACT_INT8, None)
    torch.cuda.synchronize()
    assert st == zq.ERR_TOO_LARGE
    assert "scratch" in zq.status_string(st)
    assert torch.isnan(Y).all(), "a refused call wrote its output"
