"""The parity bar for fp32 outputs: |gpu - cpu| <= 1e-4 + 1e-5*|cpu| element-wise
(1e-5 relative / 1e-4 absolute of the reference CPU kernel)."""
import numpy as np

RTOL = 1e-5
ATOL = 1e-4


def assert_close(got, want, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want)
    bound = ATOL + RTOL * np.abs(want)
    bad = np.nonzero(err > bound)[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {got.size} outside tolerance; first at {i}: "
                             f"got {got[i]!r} want {want[i]!r} err {err[i]:.3e} bound {bound[i]:.3e}")
    return float((err / np.maximum(np.abs(want).max(), 1e-30)).max())
