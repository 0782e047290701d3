"""GPU tier: the rest of the reference's GPU slot at the C ABI --
gemm_batch (include/zen/quant.h:77-84), rms_norm (include/zen/hip_backend.h:77)
and ffn_residual_fused (include/zen/quant.h:97-106) -- against the C oracle and
numpy statements of the reference CPU arithmetic, plus the Stats counters the
reference keeps (include/zen/hip_backend.h:25-41)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.tolerance import assert_close

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
DEV = "cuda:0"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def dev_weights(zq, fmt, w_np, rows, cols):
    buf = torch.zeros(zq.weight_bytes(fmt, rows, cols), dtype=torch.uint8, device=DEV)
    buf[: w_np.size] = to_dev(w_np)
    return buf


@pytest.fixture(autouse=True)
def _small_shapes_allowed(zq):
    prev = zq.set_min_elements(0)
    yield
    zq.set_min_elements(prev)


def rmsnorm_ref(x, w, eps):
    """dense_transformer_runtime.cpp:117-124: sum of squares in double,
    inv = 1/sqrtf(float(ss/n) + eps), y = x*inv*w in float."""
    x = np.asarray(x, np.float32)
    ss = np.sum(x.astype(np.float64) ** 2)
    inv = np.float32(1.0) / np.sqrt(np.float32(ss / x.size) + np.float32(eps))
    return (x * inv * np.asarray(w, np.float32)).astype(np.float32)


# --------------------------------------------------------------- gemm_batch ---
@pytest.mark.parametrize("fmt,act,m,k", [(O.Q8_0, 1, 37, 4096), (O.Q4_0, 1, 70, 2048), (O.Q8_0, 2, 9, 1024),
                                         (O.Q6_K, 2, 17, 2048), (O.Q8_0, 1, 130, 320)])
def test_gemm_batch_matches_single_gemms(zq, orc, fmt, act, m, k):
    rows = [512, 128, 128]  # Q|K|V-like
    ws = [orc.gen_weights(fmt, 700 + i, r, k) for i, r in enumerate(rows)]
    X = orc.gen_normal(710 + m, m * k)
    before = zq.stats()["batches"]
    Ys = zq.gemm_batch(fmt, ws, X, m, rows, k, act)
    assert zq.stats()["batches"] == before + 1
    ref = orc.gemm_i8 if act == zq.ACT_INT8 else orc.gemm_f32
    for w, Y, r in zip(ws, Ys, rows):
        assert_close(Y, ref(fmt, w, X, m, r, k), f"gemm_batch fmt={fmt} act={act}")
        # the batch runs the single GEMM's kernels on the same activations
        assert np.array_equal(Y, zq.gemm(fmt, w, X, m, r, k, act))
        zq.release(w)


def test_gemm_batch_dev_matches_gemm_dev(zq, orc):
    fmt, m, k = O.Q8_0, 96, 4096
    rows = [1024, 1024, 256]
    ws = [dev_weights(zq, fmt, orc.gen_weights(fmt, 720 + i, r, k), r, k) for i, r in enumerate(rows)]
    X = to_dev(orc.gen_normal(721, m * k))
    Ys = [torch.empty(m * r, device=DEV) for r in rows]
    wsb = zq.gemm_batch_workspace_bytes(fmt, rows, m, k, zq.ACT_INT8)
    assert wsb >= zq.gemm_workspace_bytes(fmt, m, max(rows), k, zq.ACT_INT8) - 1
    wsp = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    zq.gemm_batch_dev(fmt, X, list(zip(ws, Ys, rows)), m, k, zq.ACT_INT8, wsp, wsb)
    for w, Y, r in zip(ws, Ys, rows):
        one = torch.empty(m * r, device=DEV)
        b1 = zq.gemm_workspace_bytes(fmt, m, r, k, zq.ACT_INT8)
        w1 = torch.empty(b1, dtype=torch.uint8, device=DEV)
        zq.gemm_dev(fmt, w, X, one, m, r, k, zq.ACT_INT8, w1, b1)
        torch.cuda.synchronize()
        assert torch.equal(Y, one)
    with pytest.raises(zq.ZQError) as e:  # a short workspace is refused, not overrun
        zq.gemm_batch_dev(fmt, X, list(zip(ws, Ys, rows)), m, k, zq.ACT_INT8, wsp, wsb - 256)
    assert e.value.status == zq.ERR_ARG


# ----------------------------------------------------------------- rms_norm ---
@pytest.mark.parametrize("rows,cols", [(1, 4096), (5, 1000), (3, 14336)])
def test_rms_norm(zq, orc, rows, cols):
    x = orc.gen_normal(730 + cols, rows * cols) * np.float32(3.0)
    w = orc.gen_normal(731, cols)
    y = zq.rms_norm(x, w, rows, cols, 1e-5)
    want = np.concatenate([rmsnorm_ref(x[r * cols:(r + 1) * cols], w, 1e-5) for r in range(rows)])
    assert_close(y, want, "rms_norm")
    yd = torch.empty(rows * cols, device=DEV)
    zq.rms_norm_dev(to_dev(x), to_dev(w), yd, rows, cols, 1e-5)
    assert np.array_equal(yd.cpu().numpy(), y)


# ------------------------------------------------------- ffn_residual_fused ---
def ffn_residual_ref(orc, fmt, wo, wg, wu, wd, nw, x, a, hidden, aw, ffn, eps):
    t0 = orc.gemv_f32(fmt, wo, a, hidden, aw)
    h1 = (t0 + x).astype(np.float32)
    h2 = rmsnorm_ref(h1, nw, eps)
    g = orc.gemv_f32(fmt, wg, h2, ffn, hidden)
    u = orc.gemv_f32(fmt, wu, h2, ffn, hidden)
    f = (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float32)
    d = orc.gemv_f32(fmt, wd, f, hidden, ffn)
    return (h1 + d).astype(np.float32), f


@pytest.mark.parametrize("fmt,hidden,aw,ffn", [(O.Q8_0, 1024, 1024, 2816), (O.Q4_0, 2048, 1024, 5632),
                                                (O.Q6_K, 1024, 2048, 2816), (O.Q8_0, 4096, 4096, 14336),
                                                (O.Q4_K, 1024, 1024, 2816), (O.Q5_K, 2304, 1024, 2816),
                                                (O.Q6_K, 2048, 2048, 2816)])
def test_ffn_residual_fused(zq, orc, fmt, hidden, aw, ffn):
    wo = orc.gen_weights(fmt, 740, hidden, aw)
    wg = orc.gen_weights(fmt, 741, ffn, hidden)
    wu = orc.gen_weights(fmt, 742, ffn, hidden)
    wd = orc.gen_weights(fmt, 743, hidden, ffn)
    nw = orc.gen_normal(744, hidden)
    x = orc.gen_normal(745, hidden)
    a = orc.gen_normal(746, aw)
    got = zq.ffn_residual_fused(fmt, wo, wg, wu, wd, nw, x, a, hidden, aw, ffn, 1e-5)
    want, f = ffn_residual_ref(orc, fmt, wo, wg, wu, wd, nw, x, a, hidden, aw, ffn, 1e-5)
    # a chain of four projections, a norm and expf: the GEMV bar relative to
    # the magnitude summed by the last projection plus the residual
    dd = orc.dequantize(fmt, wd, hidden * ffn).reshape(hidden, ffn).astype(np.float64)
    mag = np.abs(dd) @ np.abs(f.astype(np.float64)) + np.abs(want)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(np.isfinite(got))
    assert np.all(err <= 1e-4 + 1e-5 * mag), float(np.max(err / (1e-4 + 1e-5 * mag)))
    # the device variant, writing over x in place (out may alias x)
    xd = to_dev(x)
    wsb = zq.ffn_residual_workspace_bytes(hidden, ffn)
    wsp = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    zq.ffn_residual_fused_dev(fmt, dev_weights(zq, fmt, wo, hidden, aw), dev_weights(zq, fmt, wg, ffn, hidden),
                              dev_weights(zq, fmt, wu, ffn, hidden), dev_weights(zq, fmt, wd, hidden, ffn),
                              to_dev(nw), xd, to_dev(a), xd, hidden, aw, ffn, 1e-5, wsp, wsb)
    torch.cuda.synchronize()
    assert np.array_equal(xd.cpu().numpy(), got)
    for w in (wo, wg, wu, wd):
        zq.release(w)


# -------------------------------------------------------------------- stats ---
def test_stats_fallbacks_and_timers(zq, orc):
    zq.reset_stats()
    w = orc.gen_weights(O.Q8_0, 750, 256, 1024)
    x = orc.gen_normal(751, 1024)
    zq.gemv(O.Q8_0, w, x, 256, 1024)
    s = zq.stats()
    assert s["submits"] == 1 and s["dispatches"] == 1 and s["fallbacks"] == 0
    assert s["alloc_us"] > 0 or s["uploads"] == 0
    # a declined call after init is a fallback for the caller (hip_backend.hip:946-949)
    w6 = orc.gen_weights(O.Q6_K, 752, 8, 256)
    with pytest.raises(zq.ZQError):
        zq.gemm(O.Q6_K, w6, orc.gen_normal(753, 2 * 256), 2, 8, 256, zq.ACT_INT8)
    assert zq.stats()["fallbacks"] == 1
    zq.release_all()


# ------------------------------------------------------- measurement probe ---
def test_read_probe(zq):
    """The streaming-read yardstick runs on a device buffer, stores nothing
    for real data, and refuses sizes its 16-byte loads cannot cover."""
    buf = torch.ones(1 << 22, dtype=torch.uint8, device=DEV)
    sink = torch.zeros(zq.read_probe_sink_bytes(), dtype=torch.uint8, device=DEV)
    zq.read_probe_dev(buf, buf.numel(), sink)
    torch.cuda.synchronize()
    assert int(sink.sum()) == 0
    with pytest.raises(zq.ZQError) as e:
        zq.read_probe_dev(buf, 1000, sink)  # not a multiple of 16
    assert e.value.status == zq.ERR_ARG


# ------------------------------------------------------ concurrent streams ---
def test_device_calls_on_concurrent_streams(zq, orc):
    """The device-pointer entry points keep no device state between calls:
    GEMVs and GEMMs (int8 with split-K partials, fp32, a super-block format)
    enqueued alternately on two streams, each call with its own output and
    workspace, give bit-identical results to the same calls run one at a
    time on one stream."""
    cases = [(O.Q8_0, zq.ACT_INT8, 32, 14336, 4096), (O.Q8_0, zq.ACT_INT8, 200, 1024, 4096),
             (O.Q4_0, zq.ACT_INT8, 7, 3000, 2048), (O.Q8_0, zq.ACT_F32, 5, 777, 1024),
             (O.Q6_K, zq.ACT_F32, 40, 512, 2048), (O.Q4_K, zq.ACT_F32, 1, 4096, 4096)]
    ops = []
    for i, (fmt, act, m, n, k) in enumerate(cases):
        w = dev_weights(zq, fmt, orc.gen_weights(fmt, 500 + i, n, k), n, k)
        X = to_dev(orc.gen_normal(600 + i, m * k))
        x = to_dev(orc.gen_normal(700 + i, k))
        wsb = zq.gemm_workspace_bytes(fmt, m, n, k, act)
        ops.append((fmt, act, m, n, k, w, X, x, wsb))

    def run(streams):
        # outputs and workspaces first (filled on the current stream), then
        # every stream waits for that before its launches
        outs = [(torch.full((m * n,), float("nan"), device=DEV), torch.full((n,), float("nan"), device=DEV),
                 torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)) for fmt, act, m, n, k, w, X, x, wsb in ops]
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for j, ((fmt, act, m, n, k, w, X, x, wsb), (Y, y, ws)) in enumerate(zip(ops, outs)):
            s = streams[j % len(streams)]
            zq.gemm_dev(fmt, w, X, Y, m, n, k, act, ws, wsb, stream=s)
            zq.gemv_dev(fmt, w, x, y, n, k, stream=s)
        torch.cuda.synchronize()
        return [(Y.cpu(), y.cpu()) for Y, y, _ in outs]

    serial = run([torch.cuda.current_stream()])
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for rep in range(3):
        par = run([s1, s2])
        for (Ya, ya), (Yb, yb), c in zip(serial, par, cases):
            assert torch.equal(Ya, Yb) and torch.equal(ya, yb), f"concurrent streams differ: {c} rep {rep}"
    for (Y, y), (fmt, act, m, n, k, *_), in zip(serial, ops):
        assert torch.isfinite(Y).all() and torch.isfinite(y).all()


# ------------------------------------------------------------ graph capture ---
def test_device_calls_under_graph_capture(zq, orc):
    """Callers may capture the device-pointer calls in a HIP graph: an int8
    GEMM with split-K partials, a GEMM batch, a GEMV, a GEMV batch, RMSNorm,
    the fused FFN half-layer and the allocation-free GEMM are captured once
    and replayed four times, with new inputs written eagerly between the
    replays; every replay must equal eager calls on the same inputs bit for
    bit."""
    F, m, k, n, h, ffn = O.Q8_0, 32, 4096, 4096, 1024, 2048
    W = dev_weights(zq, F, orc.gen_weights(F, 801, n, k), n, k)
    Wb = [dev_weights(zq, F, orc.gen_weights(F, 802 + i, r, k), r, k) for i, r in enumerate((512, 256))]
    wo, wg, wu, wd = (dev_weights(zq, F, orc.gen_weights(F, 810 + i, r, c), r, c)
                      for i, (r, c) in enumerate(((h, h), (ffn, h), (ffn, h), (h, ffn))))
    X = torch.empty(m * k, device=DEV)
    x = torch.empty(k, device=DEV)
    hx, ha, nw = (torch.empty(h, device=DEV) for _ in range(3))
    wsb = zq.gemm_workspace_bytes(F, m, n, k, zq.ACT_INT8)
    wsbb = zq.gemm_batch_workspace_bytes(F, [512, 256], m, k, zq.ACT_INT8)
    wsf = zq.ffn_residual_workspace_bytes(h, ffn)

    def outputs():
        return {"gemm": torch.empty(m * n, device=DEV), "b0": torch.empty(m * 512, device=DEV),
                "b1": torch.empty(m * 256, device=DEV), "gemv": torch.empty(n, device=DEV),
                "v0": torch.empty(512, device=DEV), "v1": torch.empty(256, device=DEV),
                "norm": torch.empty(m * k, device=DEV), "ffn": torch.empty(h, device=DEV),
                "noalloc": torch.empty(m * n, device=DEV),
                "ws": torch.empty(wsb, dtype=torch.uint8, device=DEV),
                "wsb": torch.empty(wsbb, dtype=torch.uint8, device=DEV),
                "wsf": torch.empty(wsf, dtype=torch.uint8, device=DEV)}

    def calls(o, s):
        zq.gemm_dev(F, W, X, o["gemm"], m, n, k, zq.ACT_INT8, o["ws"], wsb, stream=s)
        zq.gemm_batch_dev(F, X, [(Wb[0], o["b0"], 512), (Wb[1], o["b1"], 256)], m, k, zq.ACT_INT8, o["wsb"], wsbb,
                          stream=s)
        zq.gemv_dev(F, W, x, o["gemv"], n, k, stream=s)
        zq.gemv_batch_dev(F, x, [(Wb[0], o["v0"], 512), (Wb[1], o["v1"], 256)], k, stream=s)
        zq.rms_norm_dev(X, x, o["norm"], m, k, 1e-5, stream=s)
        zq.ffn_residual_fused_dev(F, wo, wg, wu, wd, nw, hx, ha, o["ffn"], h, h, ffn, 1e-5, o["wsf"], wsf, stream=s)
        zq.gemm_dev_noalloc(F, W, X, o["noalloc"], m, n, k, zq.ACT_INT8, stream=s)

    def fill(rep):
        X.copy_(to_dev(orc.gen_normal(900 + rep, m * k)))
        x.copy_(to_dev(orc.gen_normal(910 + rep, k)))
        for i, t in enumerate((hx, ha, nw)):
            t.copy_(to_dev(orc.gen_normal(920 + 3 * rep + i, h)))

    fill(0)
    cap = outputs()
    calls(cap, torch.cuda.current_stream())  # eager once first (occupancy and other caches)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            calls(cap, s)
    torch.cuda.synchronize()
    for rep in range(4):
        fill(rep + 1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = outputs()
        calls(ref, torch.cuda.current_stream())
        torch.cuda.synchronize()
        for key in ("gemm", "b0", "b1", "gemv", "v0", "v1", "norm", "ffn", "noalloc"):
            assert torch.isfinite(ref[key]).all(), key
            assert torch.equal(cap[key], ref[key]), f"graph replay {rep} differs from eager: {key}"
    assert torch.equal(cap["noalloc"], cap["gemm"])
