"""GPU tier: BASELINE config 4 at its real shape (Llama-3-8B: 32 layers,
hidden 4096, FFN 14336, 32/8 heads of 128, vocab 128256) on the
device-resident decoder, through size-independent properties -- the
reference runtime cannot hold an 8.5 GB model in this test, so the full shape
is pinned by what must hold whatever the weights are:

- the resident weights are the seeded generator's bytes (sampled rows of
  several tensors against the C oracle's generator of the same seed);
- prefill and decode logits are finite;
- HIP-graph decode is bit-identical to eager decode, step after step;
- the last prompt token's prefill logits equal feeding the prompt one decode
  step at a time (prefill GEMM + prefill attention vs decode GEMV + decode
  attention over the same cache), within a bar stated below.

and, for the benchmarked config-4 workload itself (int8-activation prefill of
512 tokens, then greedy decode to position 640):

- graph and eager runs agree bit for bit, prefill and all 128 decode steps;
- every logit is finite;
- layer 0's int8 GEMM outputs (q|k|v, o, gate, up, down), recorded through
  the model's tap hook on the activations the model itself produced, match
  the oracle's int8 GEMM on sampled tokens and rows to the fp32 bar;
- the int8 prefill's last-token logits stay within the activation
  quantisation error of the fp32 path (bar stated in the test).
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

SHAPE = dict(embedding=4096, layers=32, heads=32, kv_heads=8, ffn=14336, vocab=128256, context=8192,
             max_positions=1024, rope_base=500000.0, rms_epsilon=1e-5, eos_token=0xFFFFFFFF)
PROMPT_LEN, DECODE_TO = 512, 640  # 512-token prompt, 128 greedy tokens
SEED = 0x5EED0004


def _hip():
    lib = ctypes.CDLL("libamdhip64.so")
    lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    lib.hipMemcpy.restype = ctypes.c_int
    return lib


def read_rows(hip, addr, row_bytes, rows):
    out = np.empty(len(rows) * row_bytes, np.uint8)
    for i, r in enumerate(rows):
        st = hip.hipMemcpy(out[i * row_bytes:].ctypes.data, addr + int(r) * row_bytes, row_bytes, 2)
        assert st == 0, f"hipMemcpy {st}"
    return out


def make(graph):
    from zeninfer_amd.model import Model, PREFILL_F32
    os.environ["ZQ_MODEL_GRAPH"] = "1" if graph else "0"
    try:
        m = Model.synthetic(seed=SEED, **SHAPE)
    finally:
        os.environ.pop("ZQ_MODEL_GRAPH", None)
    return m


@pytest.fixture(scope="module")
def models(zq):
    g, e = make(True), make(False)
    yield g, e
    g.close()
    e.close()


def test_config4_weights_are_the_seeded_generator(models, zq, orc):
    from zeninfer_amd import model as M
    m = models[0]
    hip = _hip()
    for layer, which, seed in ((M.GLOBAL, M.W_EMBED, SEED), (M.GLOBAL, M.W_OUTPUT, SEED + 1),
                               (0, M.W_Q, SEED + 2), (31, M.W_DOWN, SEED + 2 + 7 * 31 + 6),
                               (17, M.W_K, SEED + 2 + 7 * 17 + 1)):
        addr, rows, cols, fmt = m.weight(layer, which)
        assert fmt == O.Q8_0
        rb = zq.row_bytes(fmt, cols)
        pick = np.unique(np.concatenate([np.random.default_rng(seed).choice(rows, 16, replace=False), [rows - 1]]))
        got = read_rows(hip, addr, rb, pick)
        full = orc.gen_weights(fmt, seed, rows, cols)
        want = np.concatenate([full[r * rb:(r + 1) * rb] for r in pick])
        # scales go through double log/cos on two math libraries: a rare
        # last-ulp scale difference is allowed, never a quant byte
        diff = np.nonzero(got != want)[0]
        assert diff.size <= 2, (layer, which, diff[:10])
        assert np.all(diff % 34 < 2), "a quant byte differs"


def test_config4_graph_decode_equals_eager_and_prefill_matches_decode(models, zq):
    from zeninfer_amd.model import PREFILL_F32
    g, e = models
    g.set_prefill_mode(PREFILL_F32)
    e.set_prefill_mode(PREFILL_F32)
    prompt = np.random.default_rng(SEED).integers(0, SHAPE["vocab"], size=12).tolist()
    ng, lg = g.prefill(prompt)
    ne, le = e.prefill(prompt)
    assert np.all(np.isfinite(lg))
    assert np.array_equal(lg, le) and ng == ne
    tok = ng
    for _ in range(4):
        ng, lg = g.decode(tok)
        ne, le = e.decode(tok)
        assert np.all(np.isfinite(lg))
        assert np.array_equal(lg, le), "graph replay differs from eager decode"
        assert ng == ne == int(np.argmax(lg))
        tok = ng
    # prefill of the whole prompt vs the prompt fed one decode step at a time
    _, lp = g.prefill(prompt)
    g.prefill(prompt[:1], logits=False)
    for t in prompt[1:-1]:
        g.decode(t, logits=False)
    _, ld = g.decode(prompt[-1])
    scale = float(np.abs(lp).max())
    err = float(np.abs(ld - lp).max())
    # 32 layers of fp32 arithmetic in two summation orders (MFMA GEMM vs GEMV,
    # chunked vs tiled attention): within 1e-4 of the largest logit
    assert err <= 1e-4 * scale, (err, scale)
    assert int(np.argmax(ld)) == int(np.argmax(lp))


def _prompt():
    return np.random.default_rng(SEED + 4).integers(0, SHAPE["vocab"], size=PROMPT_LEN).tolist()


def test_config4_int8_workload_graph_equals_eager(models, zq):
    """The bench's config-4 run: int8 prefill of 512 tokens, then greedy
    decode to position 640, graph replay against eager launches."""
    from zeninfer_amd.model import PREFILL_INT8
    g, e = models
    g.set_prefill_mode(PREFILL_INT8)
    e.set_prefill_mode(PREFILL_INT8)
    prompt = _prompt()
    ng, lg = g.prefill(prompt)
    ne, le = e.prefill(prompt)
    assert np.all(np.isfinite(lg))
    assert np.array_equal(lg, le) and ng == ne == int(np.argmax(lg))
    tok = ng
    for pos in range(PROMPT_LEN, DECODE_TO):
        ng, lg = g.decode(tok)
        ne, le = e.decode(tok)
        assert np.all(np.isfinite(lg)), pos
        assert np.array_equal(lg, le), f"graph replay differs from eager decode at position {pos}"
        assert ng == ne == int(np.argmax(lg))
        tok = ng


def test_config4_int8_prefill_layer0_gemms_match_oracle(models, zq, orc):
    """Layer 0 of the 512-token int8 prefill: each GEMM's output (its split-K
    planes summed in plane order, as the layer's readers do) against the
    oracle's int8 GEMM on the very int8 activations and scales the model fed
    it, for 8 sampled tokens x 32 sampled rows (with the first and last of
    each), to the fp32 bar widened by the rounding of the two fp32 sums
    (stated at the assertion)."""
    _check_layer_taps(models[0], zq, orc, 0)


def _check_layer_taps(g, zq, orc, layer):
    import torch
    from zeninfer_amd.model import PREFILL_INT8
    from zeninfer_amd import model as M
    g.set_prefill_mode(PREFILL_INT8)
    cap = 512 << 20
    buf = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    g.set_tap(layer, buf.data_ptr(), cap)
    try:
        g.prefill(_prompt(), logits=False)
        recs = g.tap_records()
    finally:
        g.set_tap(0, 0, 0)
    E, F = SHAPE["embedding"], SHAPE["ffn"]
    QKV = (SHAPE["heads"] + 2 * SHAPE["kv_heads"]) * 128
    want_shapes = {M.TAP_QKV: (QKV, E), M.TAP_O: (E, E), M.TAP_GATE: (F, E), M.TAP_UP: (F, E), M.TAP_DOWN: (E, F)}
    assert sorted(r.proj for r in recs) == sorted(want_shapes), [r.proj for r in recs]
    hip = _hip()
    host = buf.cpu().numpy()
    for r in recs:
        assert (r.n, r.k) == want_shapes[r.proj] and r.m == PROMPT_LEN and r.fmt == O.Q8_0
        m, n, k, nb = r.m, r.n, r.k, r.k // 32
        xq = host[r.xq_off:r.xq_off + m * k].view(np.int8).reshape(m, k)
        xs = host[r.xs_off:r.xs_off + m * nb * 4].view(np.float32).reshape(m, nb)
        planes = host[r.y_off:r.y_off + r.splits * m * n * 4].view(np.float32).reshape(r.splits, m, n)
        y = planes[0].copy()
        for p in planes[1:]:
            y += p
        assert np.all(np.isfinite(y))
        if r.proj == M.TAP_QKV:
            # attention scores of head 0 (RoPE rotates pairs, so it keeps the
            # norms these are made of): their spread says how saturated the
            # softmax of this random-init model is
            qh, kh = y[:, :128].astype(np.float64), y[:, SHAPE["heads"] * 128:SHAPE["heads"] * 128 + 128]
            score_std = float((qh @ kh.T.astype(np.float64) / np.sqrt(128.0)).std())
            print(f"layer {layer}: head-0 attention score std {score_std:.1f}")
        rng = np.random.default_rng(100 + 8 * layer + r.proj)
        toks = np.unique(np.concatenate([rng.choice(m, 6, replace=False), [0, m - 1]]))
        rows = np.unique(np.concatenate([rng.choice(n, 30, replace=False), [0, n - 1]]))
        rb = zq.row_bytes(r.fmt, k)
        sub = read_rows(hip, r.w, rb, rows)
        xq_t, xs_t = xq[toks].reshape(-1), xs[toks].reshape(-1)
        want = orc.gemm_i8_prequant(r.fmt, sub, xq_t, xs_t, len(toks), len(rows), k)
        # the exact value and the size of its terms, from the oracle's integer dots
        dots = orc.block_dots(r.fmt, sub, xq_t, len(toks), len(rows), k).reshape(len(toks), len(rows), nb)
        dw = sub.reshape(len(rows), nb, 34)[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float64)
        terms = dots * (xs[toks].astype(np.float64)[:, None, :] * dw[None, :, :])
        exact, mag = terms.sum(-1).reshape(-1), np.abs(terms).sum(-1).reshape(-1)
        got = y[np.ix_(toks, rows)].reshape(-1).astype(np.float64)
        # Bar: the fp32 bar (1e-4 + 1e-5*|y|) widened by the rounding of two
        # fp32 sums of the same nb terms in different orders.  Each rounding is
        # at most 2^-24 of a partial sum no larger than sum|terms|; modelled as
        # independent and uniform, the two sums' difference has a standard
        # deviation below sqrt(2*nb/12) * 2^-24 * sum|terms| ~ 5e-7 * sum|terms|
        # at nb = 448, and the bar allows 3e-6 (six sigma).  It matters for the
        # down projection, whose inputs (silu(gate) * up of random-init
        # weights) make outputs that are small differences of terms in the
        # thousands.
        bar = 1e-4 + 1e-5 * np.abs(want) + 3e-6 * mag
        err = np.abs(got - want)
        worst = int(np.argmax(err / bar))
        print(f"layer {layer} proj {r.proj}: splits {r.splits}, max|y| {np.abs(got).max():.1f}, max err vs oracle {err.max():.2e}, "
              f"worst err/bar {err[worst] / bar[worst]:.2f}; |gpu-exact| {np.abs(got - exact).max():.2e}, "
              f"|oracle-exact| {np.abs(want - exact).max():.2e}")
        assert np.all(err <= bar), (layer, r.proj, worst, got[worst], want[worst], exact[worst], mag[worst])


def test_config4_int8_prefill_all_depths_gemms_match_oracle(models, zq, orc):
    """The same check at the middle and last decoder layers, whose inputs have
    been through 16 and 31 layers of the int8 prefill."""
    for layer in (16, 31):
        _check_layer_taps(models[0], zq, orc, layer)


@pytest.fixture(scope="module")
def shallow(zq):
    from zeninfer_amd.model import Model
    m = Model.synthetic(seed=SEED + 9, **dict(SHAPE, layers=2))
    yield m
    m.close()


def test_config4_width_int8_prefill_within_quantisation_error(shallow, zq):
    """512 tokens through two decoder layers of config-4 width (hidden 4096,
    FFN 14336, 32/8 heads, vocab 128256): the last-token logits of the int8
    and fp32 prefills against the same prompt fed one decode step at a time
    (fp32 GEMVs and decode attention over the cache).

    fp32 prefill: within 1e-4 of max|logit| (two fp32 summation orders).

    int8 prefill: per-32 int8 blocks carry a relative rounding error of about
    (amax/127)/sqrt(12)/rms ~ 0.5% per GEMM input (amax ~ 2.1 rms for a
    Gaussian block).  On a well-conditioned model that keeps logits within 5%
    (the small model's bar against the reference runtime).  This random-init
    model is not well conditioned: its attention scores have a standard
    deviation of ~88 (printed by the tap tests above), so the softmax is nearly one-hot
    and a 0.5% change of q or k moves scores by ~0.3-0.5, enough to change
    which key wins for rows whose top two scores are that close.  Such rows
    change their attention output outright, and the logits move by far more
    than 0.5%.  The bar therefore checks what survives that: the two
    prefills' logits stay strongly correlated (above 0.95) and within 25% of
    max|logit|, and the fp32 prefill, which flips no scores, meets the fp32
    bar.  At 32 layers the divergence saturates (correlation ~0.93 measured),
    so the full-depth run is checked layer by layer through the GEMM taps."""
    from zeninfer_amd.model import PREFILL_F32, PREFILL_INT8
    g = shallow
    prompt = _prompt()
    g.set_prefill_mode(PREFILL_INT8)
    _, li = g.prefill(prompt)
    g.set_prefill_mode(PREFILL_F32)
    _, lf = g.prefill(prompt)
    g.prefill(prompt[:1], logits=False)
    for t in prompt[1:-1]:
        g.decode(t, logits=False)
    _, ld = g.decode(prompt[-1])
    assert np.all(np.isfinite(li)) and np.all(np.isfinite(ld))
    scale = float(np.abs(ld).max())
    ef = float(np.abs(lf - ld).max())
    ei = float(np.abs(li - ld).max())
    corr = float(np.corrcoef(li, ld)[0, 1])
    print(f"512 tokens, 2 layers vs decode chain: fp32 prefill max err {ef:.3e}, int8 prefill max err {ei:.3e} "
          f"of max|logit| {scale:.3f}, int8 correlation {corr:.6f}")
    assert ef <= 1e-4 * scale, (ef, scale)
    assert ei <= 0.25 * scale, (ei, scale)
    assert corr > 0.95, corr


@pytest.mark.parametrize("fmt", [O.Q4_0, O.Q6_K, O.Q4_K, O.Q5_K])
def test_config4_shape_other_formats(zq, fmt):
    """The config-4 shape with the projections in the other formats (the
    embedding table and output stay Q8_0, as in many real GGUFs): fp32
    prefill and decode logits finite, HIP-graph decode bit-identical to
    eager, and the prompt's last-token logits from prefill (the super-block
    GEMM on the f16 MFMA, or the Q4_0 one) against the prompt fed one decode
    step at a time (the streaming GEMVs) within the same bar as Q8_0."""
    from zeninfer_amd.model import Model, PREFILL_F32
    models = []
    for graph in (True, False):
        os.environ["ZQ_MODEL_GRAPH"] = "1" if graph else "0"
        try:
            models.append(Model.synthetic(seed=SEED + fmt, weight_format=fmt, **SHAPE))
        finally:
            os.environ.pop("ZQ_MODEL_GRAPH", None)
    g, e = models
    try:
        for m in models:
            m.set_prefill_mode(PREFILL_F32)
        prompt = np.random.default_rng(SEED + fmt).integers(0, SHAPE["vocab"], size=12).tolist()
        ng, lg = g.prefill(prompt)
        ne, le = e.prefill(prompt)
        assert np.all(np.isfinite(lg)) and np.array_equal(lg, le) and ng == ne
        tok = ng
        for _ in range(3):
            ng, lg = g.decode(tok)
            ne, le = e.decode(tok)
            assert np.all(np.isfinite(lg))
            assert np.array_equal(lg, le), "graph replay differs from eager decode"
            assert ng == ne == int(np.argmax(lg))
            tok = ng
        _, lp = g.prefill(prompt)
        g.prefill(prompt[:1], logits=False)
        for t in prompt[1:-1]:
            g.decode(t, logits=False)
        _, ld = g.decode(prompt[-1])
        scale = float(np.abs(lp).max())
        err = float(np.abs(ld - lp).max())
        assert err <= 1e-4 * scale, (fmt, err, scale)
    finally:
        g.close()
        e.close()
