"""GPU tier: the chained decode GEMV (zq_hip_chain_*, one persistent launch
for a sequence of projections whose inputs are produced inside the launch).

- Plain stages equal zq_hip_gemv_batch_dev on the same input bit for bit
  (same kernel arithmetic and work split), including a stage whose x is the
  output of the previous stage in the same launch.
- Add + RMSNorm stages are within the GEMV bar of the unchained GEMV applied
  to the host-computed input, and the residual they write is the exact float
  sum; the gate/up SiLU epilogue is within the bar of silu(gate) * up of the
  unchained GEMVs.
- Consecutive launches (the kernel resets its own counters) and HIP-graph
  replays with eager work in between give identical outputs.
- A bounded wait forced to give up from the host (a spin bound of 0 polls)
  is reported, the grid still drains, and after a reset the chain is correct.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.tolerance import assert_close

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
DEV = "cuda:0"


def rmsnorm_ref(v, w, eps):
    v = np.asarray(v, np.float32)
    ss = np.sum(v.astype(np.float64) ** 2)
    inv = np.float32(1.0) / np.sqrt(np.float32(ss / v.size) + np.float32(eps))
    return (v * inv * np.asarray(w, np.float32)).astype(np.float32)


def silu_mul_ref(g, u):
    g = np.asarray(g, np.float32)
    return (g / (np.float32(1.0) + np.exp(-g)) * np.asarray(u, np.float32)).astype(np.float32)


class Layer:
    def __init__(self, zq, fmt, E, KV, F, seed):
        def W(rows, cols, s):
            t = torch.zeros(zq.weight_bytes(fmt, rows, cols), dtype=torch.uint8, device=DEV)
            zq.synth_weights_dev(fmt, s, t, rows, cols)
            return t
        self.E, self.KV, self.F = E, KV, F
        self.q, self.k, self.v = W(E, E, seed), W(KV, E, seed + 1), W(KV, E, seed + 2)
        self.o, self.g, self.u, self.d = W(E, E, seed + 3), W(F, E, seed + 4), W(F, E, seed + 5), W(E, F, seed + 6)


def vec(n, seed, zq, scale=1.0):
    t = torch.empty(n, device=DEV)
    zq.synth_normal_dev(seed, t, n)
    return t * scale


def make_program(zq, L, x0, resid0, n1, n2, eps=1e-5):
    E, KV, F = L.E, L.KV, L.F
    out = {k: torch.full((n,), float("nan"), device=DEV) for k, n in
           (("q", E), ("k", KV), ("v", KV), ("o", E), ("g", F), ("d", E), ("r1", E),
            ("q2", E), ("k2", KV), ("v2", KV), ("r2", E))}
    stages = [
        dict(tasks=[(L.q, out["q"], E), (L.k, out["k"], KV), (L.v, out["v"], KV)], cols=E, a=x0),
        dict(tasks=[(L.o, out["o"], E)], cols=E, a=out["q"], wait=0),
        dict(tasks=[(L.g, out["g"], F), (L.u, None, F)], cols=E, kind=2, a=out["o"], b=resid0, w=n1,
             r_out=out["r1"], eps=eps, wait=1, epilogue=1),
        dict(tasks=[(L.d, out["d"], E)], cols=F, a=out["g"], wait=2),
        dict(tasks=[(L.q, out["q2"], E), (L.k, out["k2"], KV), (L.v, out["v2"], KV)], cols=E, kind=2,
             a=out["d"], b=out["r1"], w=n2, r_out=out["r2"], eps=eps, wait=3),
    ]
    return stages, out


def unchained(zq, fmt, L, x0, resid0, n1, n2, out, eps=1e-5):
    """The same projections, one launch each, with the prologues computed on
    the host from the chain's own intermediate outputs."""
    E, KV, F = L.E, L.KV, L.F
    res = {}
    y = [torch.empty(n, device=DEV) for n in (E, KV, KV)]
    zq.gemv_batch_dev(fmt, x0, [(L.q, y[0], E), (L.k, y[1], KV), (L.v, y[2], KV)], E)
    res["q"], res["k"], res["v"] = y
    yo = torch.empty(E, device=DEV)
    zq.gemv_dev(fmt, L.o, out["q"], yo, E, E)
    res["o"] = yo
    h = (out["o"].cpu().numpy() + resid0.cpu().numpy()).astype(np.float32)
    res["r1"] = h
    x2 = torch.from_numpy(rmsnorm_ref(h, n1.cpu().numpy(), eps)).to(DEV)
    yg, yu = torch.empty(F, device=DEV), torch.empty(F, device=DEV)
    zq.gemv_batch_dev(fmt, x2, [(L.g, yg, F), (L.u, yu, F)], E)
    res["g"] = torch.from_numpy(silu_mul_ref(yg.cpu().numpy(), yu.cpu().numpy()))  # f = silu(gate) * up
    yd = torch.empty(E, device=DEV)
    zq.gemv_dev(fmt, L.d, out["g"], yd, E, F)  # down of the chain's own f: a plain stage
    res["d"] = yd
    h2 = (out["d"].cpu().numpy() + out["r1"].cpu().numpy()).astype(np.float32)
    res["r2"] = h2
    x4 = torch.from_numpy(rmsnorm_ref(h2, n2.cpu().numpy(), eps)).to(DEV)
    y2 = [torch.empty(n, device=DEV) for n in (E, KV, KV)]
    zq.gemv_batch_dev(fmt, x4, [(L.q, y2[0], E), (L.k, y2[1], KV), (L.v, y2[2], KV)], E)
    res["q2"], res["k2"], res["v2"] = y2
    torch.cuda.synchronize()
    return res


def check_against_unchained(zq, fmt, L, x0, resid0, n1, n2, out):
    ref = unchained(zq, fmt, L, x0, resid0, n1, n2, out)
    host = {k: v.cpu().numpy() for k, v in out.items()}
    for k in ("q", "k", "v", "o", "d"):  # plain stages: the unchained kernel's bits
        assert np.array_equal(host[k], ref[k].cpu().numpy()), f"stage output {k} differs"
    for k in ("r1", "r2"):  # residual = the exact float sum
        assert np.array_equal(host[k], ref[k]), f"residual {k} differs"
    for k in ("g", "q2", "k2", "v2"):  # norm prologue / SiLU epilogue stages: the GEMV bar
        assert_close(host[k], ref[k].cpu().numpy(), f"chain {k}")


@pytest.mark.parametrize("fmt,E,KV,F", [(O.Q8_0, 4096, 1024, 14336), (O.Q4_0, 2048, 512, 5632),
                                        (O.Q8_0, 1024, 256, 2816)])
def test_chain_layer_matches_unchained(zq, fmt, E, KV, F):
    L = Layer(zq, fmt, E, KV, F, 1000 + E)
    x0, resid0 = vec(E, 1, zq), vec(E, 2, zq, 3.0)
    n1, n2 = vec(E, 3, zq), vec(E, 4, zq)
    stages, out = make_program(zq, L, x0, resid0, n1, n2)
    ch = zq.Chain(fmt, stages)
    ch.launch()
    assert not ch.timed_out()
    first = {k: v.clone() for k, v in out.items()}
    check_against_unchained(zq, fmt, L, x0, resid0, n1, n2, out)
    # a second launch: the counters were reset by the kernel itself
    for v in out.values():
        v.fill_(float("nan"))
    ch.launch()
    assert not ch.timed_out()
    for k in out:
        assert torch.equal(out[k], first[k]), k
    ch.close()


def test_chain_graph_replay(zq):
    fmt, E, KV, F = O.Q8_0, 4096, 1024, 14336
    L = Layer(zq, fmt, E, KV, F, 77)
    x0, resid0 = vec(E, 11, zq), vec(E, 12, zq)
    n1, n2 = vec(E, 13, zq), vec(E, 14, zq)
    stages, out = make_program(zq, L, x0, resid0, n1, n2)
    ch = zq.Chain(fmt, stages)
    ch.launch()
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in out.items()}
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            ch.launch(s)
    torch.cuda.synchronize()
    for rep in range(3):
        for v in out.values():
            v.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for k in out:
            assert torch.equal(out[k], eager[k]), (rep, k)
        # eager work between replays, on the same buffers
        ch.launch()
        torch.cuda.synchronize()
    assert not ch.timed_out()
    ch.close()


def test_chain_bounded_wait_gives_up_and_recovers(zq):
    fmt, E, KV, F = O.Q8_0, 2048, 512, 5632
    L = Layer(zq, fmt, E, KV, F, 88)
    x0, resid0 = vec(E, 21, zq), vec(E, 22, zq)
    n1, n2 = vec(E, 23, zq), vec(E, 24, zq)
    stages, out = make_program(zq, L, x0, resid0, n1, n2)
    ch = zq.Chain(fmt, stages)
    ch.set_spin_limit(0)  # every wait that is not already satisfied gives up at once
    ch.launch()
    assert ch.timed_out()
    ch.reset()
    ch.set_spin_limit(1 << 22)
    ch.launch()
    assert not ch.timed_out()
    check_against_unchained(zq, fmt, L, x0, resid0, n1, n2, out)
    ch.close()


def test_chain_declines_uncovered_stages(zq):
    E = 4096
    w = torch.zeros(zq.weight_bytes(O.Q6_K, 256, E), dtype=torch.uint8, device=DEV)
    y, x = torch.empty(256, device=DEV), torch.empty(E, device=DEV)
    with pytest.raises(zq.ZQError) as e:  # format without a chained kernel
        zq.Chain(O.Q6_K, [dict(tasks=[(w, y, 256)], cols=E, a=x)])
    assert e.value.status == zq.DECLINED
    w8 = torch.zeros(zq.weight_bytes(O.Q8_0, 256, E), dtype=torch.uint8, device=DEV)
    with pytest.raises(zq.ZQError) as e:  # a wait that does not point backwards
        zq.Chain(O.Q8_0, [dict(tasks=[(w8, y, 256)], cols=E, a=x, wait=0)])
    assert e.value.status == zq.ERR_ARG
    with pytest.raises(zq.ZQError) as e:  # the SiLU*up prologue: declined (an epilogue of the gate/up stage instead)
        zq.Chain(O.Q8_0, [dict(tasks=[(w8, y, 256)], cols=E, kind=1, a=x, b=x)])
    assert e.value.status == zq.DECLINED
