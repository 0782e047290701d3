"""GPU tier: the device-resident decoder (include/zq_model.h) against the
reference's own DenseTransformerRuntime (compiled into oracle/_ref), on a
small llama GGUF written by zeninfer_amd.gguf.

Bars (stated per test):
- fp32-activation prefill (the reference CPU arithmetic): prefill and every
  decode step's logits within |g - c| <= 1e-4 + 1e-4 * max|c| of the
  reference's forward_batch / forward, and greedy generation token-identical
  to the reference's generate();
- int8-activation prefill (the reference GPU route's arithmetic; the
  reference CPU runtime has no int8-activation GEMM to compare with, and the
  int8 GEMM itself is pinned per block against the oracle): logits within
  5% of max|c| (activation quantisation error, ~2.5% measured), correlation
  above 0.999 and our greedy token among the reference's top three;
- HIP-graph decode bit-identical to eager decode;
- a prompt longer than one prefill pass (1024 tokens) equals the same tokens
  fed one decode step at a time, to the fp32 bar.
"""
import os

import numpy as np
import pytest

from zeninfer_amd import gguf as G

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libzenref.so")
SHAPE = G.LlamaShape(embedding=256, layers=2, heads=4, kv_heads=2, ffn=512, vocab=512, context=2048)
PROMPT = [5, 17, 99, 3, 250, 7, 8, 400, 31, 77, 123, 500, 2 + 1, 64, 65, 66]


@pytest.fixture(scope="module")
def tiny_path(tmp_path_factory):
    p = tmp_path_factory.mktemp("model") / "tiny_llama.gguf"
    G.synthetic_llama(p, SHAPE, seed=7)
    return p


@pytest.fixture(scope="module")
def reference(tiny_path):
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built")
    from oracle.oracle import ReferenceModel
    r = ReferenceModel(tiny_path)
    yield r
    r.close()


def load(tiny_path, mode, graph=True, max_positions=128):
    from zeninfer_amd.model import Model
    os.environ["ZQ_MODEL_GRAPH"] = "1" if graph else "0"
    try:
        m = Model.from_gguf(G.GGUFFile(tiny_path), max_positions=max_positions)
    finally:
        os.environ.pop("ZQ_MODEL_GRAPH", None)
    m.set_prefill_mode(mode)
    return m


def close_to(g, c, rel):
    scale = float(np.abs(c).max())
    err = float(np.abs(g - c).max())
    return err <= 1e-4 + rel * scale, err, scale


def test_config_matches_reference(tiny_path, reference, zq):
    m = load(tiny_path, 1)
    c, r = m.config, reference.config
    for k in ("embedding", "layers", "heads", "kv_heads", "head_dim", "ffn", "vocab", "context"):
        assert c[k] == r[k], k
    assert c["eos_token"] == r["eos"] and c["weight_format"] == 8
    mem = m.memory()
    assert mem["weights"] >= os.path.getsize(tiny_path) - 20000
    m.close()


def test_f32_prefill_and_decode_logits(tiny_path, reference, zq):
    from zeninfer_amd.model import PREFILL_F32
    m = load(tiny_path, PREFILL_F32)
    nxt, lg = m.prefill(PROMPT)
    lr = reference.prefill(PROMPT, capacity=128)
    ok, err, scale = close_to(lg, lr, 1e-4)
    print(f"prefill: max err {err:.3e} of max|logit| {scale:.3f}")
    assert ok and nxt == int(np.argmax(lr))
    tok = nxt
    for step in range(8):
        pos = len(PROMPT) + step
        nxt, lg = m.decode(tok)
        lr = reference.step(tok, pos)
        ok, err, scale = close_to(lg, lr, 1e-4)
        print(f"decode pos {pos}: max err {err:.3e} of {scale:.3f}")
        assert ok and nxt == int(np.argmax(lr)), (pos, err)
        tok = nxt
    m.close()


def test_f32_generate_matches_reference(tiny_path, reference, zq):
    from zeninfer_amd.model import PREFILL_F32
    m = load(tiny_path, PREFILL_F32)
    ours, _, _ = m.generate(PROMPT, 24)
    ref, _, _ = reference.generate(PROMPT, 24)
    assert ours == ref, (ours, ref)
    m.close()


@pytest.mark.parametrize("plen", [16, 120])
def test_int8_prefill_close_to_reference(tiny_path, reference, zq, plen):
    """16 tokens run the skinny int8 GEMM; 120 the 128-token tile, with q|k|v
    as one projection."""
    from zeninfer_amd.model import PREFILL_INT8
    prompt = PROMPT if plen == 16 else [int(t) for t in np.random.default_rng(9).integers(0, SHAPE.vocab, plen)]
    m = load(tiny_path, PREFILL_INT8)
    nxt, lg = m.prefill(prompt)
    lr = reference.prefill(prompt, capacity=128)
    ok, err, scale = close_to(lg, lr, 5e-2)
    corr = float(np.corrcoef(lg, lr)[0, 1])
    print(f"int8 prefill: max err {err:.3e} of {scale:.3f}, correlation {corr:.6f}")
    assert ok and corr > 0.999 and nxt in np.argsort(lr)[-3:]
    m.close()


def test_graph_decode_equals_eager(tiny_path, zq):
    from zeninfer_amd.model import PREFILL_F32
    runs = []
    for graph in (True, False):
        m = load(tiny_path, PREFILL_F32, graph=graph)
        nxt, _ = m.prefill(PROMPT[:9])
        seq = []
        for _ in range(6):
            nxt, lg = m.decode(nxt)
            seq.append(lg.copy())
        runs.append(seq)
        m.close()
    for a, b in zip(*runs):
        assert np.array_equal(a, b)


def test_chunked_prefill_and_capacity(tiny_path, zq):
    """A prompt longer than one prefill pass (two chunks) must equal a
    decode-by-decode run of the same tokens to the fp32 bar; a step past the
    capacity is refused."""
    from zeninfer_amd.model import PREFILL_F32
    from zeninfer_amd import zq as Z
    m = load(tiny_path, PREFILL_F32, max_positions=1100)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, 512, size=1100).tolist()
    _, full = m.prefill(prompt)
    _, lg = m.prefill(prompt[:1])
    for t in prompt[1:]:
        _, lg = m.decode(t)
    ok, err, scale = close_to(lg, full, 1e-4)
    assert ok, err
    with pytest.raises(Z.ZQError):
        m.decode(1)  # position 1100 == capacity
    m.close()


def test_synthetic_model_runs(zq):
    from zeninfer_amd.model import Model
    m = Model.synthetic(embedding=512, layers=2, heads=8, kv_heads=2, ffn=1024, vocab=1000, context=64,
                        max_positions=64, rope_base=500000.0, rms_epsilon=1e-5, eos_token=2)
    toks, pm, dm = m.generate([1, 2, 3, 4], 8)
    assert 1 <= len(toks) <= 8 and all(0 <= t < 1000 for t in toks)
    _, lg = m.prefill([1, 2, 3, 4])
    assert np.isfinite(lg).all()
    m.close()


@pytest.mark.parametrize("ptype", [G.GGML_Q4_K, G.GGML_Q5_K, G.GGML_Q6_K])
def test_kquant_model_matches_reference(tmp_path, zq, ptype):
    """A Q4_K / Q5_K llama (projections and output K-quants, Q8_0 embedding):
    prefill and decode logits of the device model within the fp32 bar of the
    reference runtime, and greedy generation token-identical.  K-quant
    projections always take fp32 activations (their only reference routes),
    whatever the prefill mode."""
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built")
    from oracle.oracle import ReferenceModel
    from zeninfer_amd.model import PREFILL_INT8
    path = tmp_path / f"tiny_{ptype}.gguf"
    G.synthetic_llama(path, SHAPE, seed=11, proj_type=ptype)
    ref = ReferenceModel(path)
    m = load(path, PREFILL_INT8)
    assert m.config["weight_format"] == ptype
    nxt, lg = m.prefill(PROMPT)
    lr = ref.prefill(PROMPT, capacity=128)
    ok, err, scale = close_to(lg, lr, 1e-4)
    print(f"fmt {ptype} prefill: max err {err:.3e} of {scale:.3f}")
    assert ok and nxt == int(np.argmax(lr))
    tok = nxt
    for step in range(4):
        nxt, lg = m.decode(tok)
        lr = ref.step(tok, len(PROMPT) + step)
        ok, err, scale = close_to(lg, lr, 1e-4)
        assert ok and nxt == int(np.argmax(lr)), (step, err)
        tok = nxt
    m.close()
    m = load(path, PREFILL_INT8)
    ours, _, _ = m.generate(PROMPT, 16)
    theirs, _, _ = ref.generate(PROMPT, 16)
    assert ours == theirs
    m.close()
    ref.close()


def test_fused_decode_equals_unfused(tiny_path, zq):
    """The decode step with the norms and SiLU folded into the GEMVs against
    the separate-kernel step (ZQ_MODEL_FUSED=0): the same arithmetic except
    the order of the double-precision sum of squares, so logits agree to a
    few fp32 ulps and the greedy tokens are identical."""
    from zeninfer_amd.model import PREFILL_F32
    runs = []
    for fused in ("1", "0"):
        os.environ["ZQ_MODEL_FUSED"] = fused
        try:
            m = load(tiny_path, PREFILL_F32)
        finally:
            os.environ.pop("ZQ_MODEL_FUSED", None)
        nxt, _ = m.prefill(PROMPT)
        seq = []
        for _ in range(8):
            nxt, lg = m.decode(nxt)
            seq.append((nxt, lg.copy()))
        runs.append(seq)
        m.close()
    for (ta, la), (tb, lb) in zip(*runs):
        assert ta == tb
        assert np.abs(la - lb).max() <= 1e-5 * np.abs(lb).max() + 1e-6


@pytest.mark.parametrize("ptype,embedding,heads,kv_heads", [
    (G.GGML_Q4_K, 256, 4, 2), (G.GGML_Q4_K, 2304, 18, 6), (G.GGML_Q5_K, 256, 4, 2), (G.GGML_Q5_K, 2304, 18, 6),
    (G.GGML_Q6_K, 2048, 16, 4), (G.GGML_Q6_K, 4096, 32, 8)])
def test_kquant_silu_pair_decode_equals_unfused(tmp_path, zq, ptype, embedding, heads, kv_heads):
    """Decode on Q4_K / Q5_K / Q6_K against ZQ_MODEL_FUSED=0 (gate|up GEMV,
    SiLU*up kernel, add+RMSNorm kernels).  Q6_K: gate|up as one paired GEMV
    that stores silu(gate)*up (one gate row and one up row per team); each
    row's sum is the unpaired kernel's and the activation is the same
    expression, so the logits are bit-identical.  Q4_K / Q5_K also carry the
    residual adds and RMSNorms in the GEMVs (the o / down GEMVs add into the
    residual and accumulate its sum of squares in double through atomics; QKV
    and gate|up normalise x as they load it): the same arithmetic except the
    order of the double sum of squares, so the logits agree to a few fp32 ulps
    and the greedy tokens are identical.  Embedding 256 (Q6_K: 2048) takes the
    one-slice form (S = 1), 2304 (Q6_K: 4096) the slice-sum form (S = 2)."""
    from zeninfer_amd.model import PREFILL_F32
    shape = G.LlamaShape(embedding=embedding, layers=2, heads=heads, kv_heads=kv_heads, ffn=768, vocab=512,
                         context=2048)
    path = tmp_path / f"sp_{ptype}_{embedding}.gguf"
    G.synthetic_llama(path, shape, seed=21, proj_type=ptype)
    runs = []
    for fused in ("1", "0"):
        os.environ["ZQ_MODEL_FUSED"] = fused
        try:
            m = load(path, PREFILL_F32)
        finally:
            os.environ.pop("ZQ_MODEL_FUSED", None)
        nxt, _ = m.prefill(PROMPT)
        seq = []
        for _ in range(6):
            nxt, lg = m.decode(nxt)
            seq.append((nxt, lg.copy()))
        runs.append(seq)
        m.close()
    for (ta, la), (tb, lb) in zip(*runs):
        assert ta == tb
        if ptype == G.GGML_Q6_K:
            np.testing.assert_array_equal(la, lb)
        else:
            assert np.abs(la - lb).max() <= 1e-5 * np.abs(lb).max() + 1e-6


@pytest.mark.parametrize("ptype,rope_dim", [(G.GGML_Q8_0, 0), (G.GGML_Q4_0, 0), (G.GGML_Q8_0, 62)])
def test_fused_prefill_quantiser_equals_unfused(tmp_path, zq, ptype, rope_dim):
    """Int8 prefill with the activations quantised inside the RMSNorm and
    SiLU*up kernels, and the GEMMs' split-K partial sums left to their readers
    (the RoPE + KV-append kernel and the add+RMSNorms sum the planes), against
    ZQ_MODEL_FUSED=0: separate quantiser launches and the GEMMs' own split-K
    reduction.  The same per-block arithmetic on the same fp32 values, and the
    planes summed in the same order, so the prefill logits are bit-identical,
    for a 16-token and a 150-token prompt.  rope_dim 62 (31 rotary pairs, odd)
    takes the scalar RoPE kernel, which reduces the q|k|v planes itself before
    rotating; the tap records show that the split-K paths were taken."""
    from zeninfer_amd.model import PREFILL_INT8
    import torch
    shape = SHAPE if not rope_dim else G.LlamaShape(embedding=512, layers=2, heads=4, kv_heads=2, ffn=512, vocab=512,
                                                    context=2048, rope_dim=rope_dim)
    path = tmp_path / f"fq_{ptype}_{rope_dim}.gguf"
    G.synthetic_llama(path, shape, seed=23, proj_type=ptype)
    long_prompt = [int(t) for t in np.random.default_rng(5).integers(0, shape.vocab, 150)]
    outs = []
    for fused in ("1", "0"):
        os.environ["ZQ_MODEL_FUSED"] = fused
        try:
            m = load(path, PREFILL_INT8, max_positions=256)
        finally:
            os.environ.pop("ZQ_MODEL_FUSED", None)
        buf = torch.empty(64 << 20, dtype=torch.uint8, device="cuda:0")
        m.set_tap(0, buf.data_ptr(), buf.numel())
        res = []
        for prompt in (PROMPT, long_prompt):
            nxt, lg = m.prefill(prompt)
            splits = {r.proj: r.splits for r in m.tap_records()}
            res.append((nxt, lg.copy(), splits))
        m.set_tap(0, 0, 0)
        outs.append(res)
        m.close()
    for (ta, la, sa), (tb, lb, sb) in zip(*outs):
        assert ta == tb
        assert np.array_equal(la, lb)
        assert all(v == 1 for v in sb.values()), sb  # unfused: the GEMMs reduced their planes
    assert any(v > 1 for v in outs[0][1][2].values()), outs[0][1][2]  # fused: some reader summed planes


@pytest.mark.parametrize("rope_dim", [64, 32])
def test_partial_rope_matches_reference(tmp_path, zq, rope_dim):
    """rope.dimension_count below the head dim (128): only the first rope_dim
    dimensions of q and k rotate, the rest pass through (the reference's
    rope()).  150-token fp32 prefill and 4 decode steps within the fp32 bar,
    through the float4 RoPE kernel (rope_dim / 2 even) and the decode kernel's
    fused RoPE."""
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built")
    from oracle.oracle import ReferenceModel
    from zeninfer_amd.model import PREFILL_F32
    shape = G.LlamaShape(embedding=512, layers=1, heads=4, kv_heads=2, ffn=512, vocab=512, context=2048,
                         rope_dim=rope_dim)
    path = tmp_path / f"rope_{rope_dim}.gguf"
    G.synthetic_llama(path, shape, seed=31)
    prompt = [int(t) for t in np.random.default_rng(rope_dim).integers(0, shape.vocab, 150)]
    ref = ReferenceModel(path)
    m = load(path, PREFILL_F32, max_positions=256)
    nxt, lg = m.prefill(prompt)
    lr = ref.prefill(prompt, capacity=256)
    ok, err, scale = close_to(lg, lr, 1e-4)
    assert ok and nxt == int(np.argmax(lr)), err
    tok = nxt
    for step in range(4):
        nxt, lg = m.decode(tok)
        lr = ref.step(tok, len(prompt) + step)
        ok, err, scale = close_to(lg, lr, 1e-4)
        assert ok and nxt == int(np.argmax(lr)), (step, err)
        tok = nxt
    m.close()
    ref.close()


@pytest.mark.parametrize("embedding,heads,kv_heads", [(512, 4, 2), (1024, 8, 1), (768, 3, 1), (896, 14, 2)])
def test_prefill_attention_shapes_match_reference(tmp_path, zq, embedding, heads, kv_heads):
    """head_dim 128 with 2 and 8 query heads per kv head, a 150-token prompt
    (three 64-key tiles, a partial last query tile): fp32 prefill logits and
    the following decode step within the fp32 bar of the reference.  Also
    head_dim 256 with 3 query heads per kv head and head_dim 64 with 7: the
    prefill falls back to the one-workgroup-per-row kernel (the MFMA kernel
    takes head_dim 64/128 with G dividing 64) and the decode kernel runs
    its G = 3 and G = 7 instances."""
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built")
    from oracle.oracle import ReferenceModel
    from zeninfer_amd.model import PREFILL_F32
    shape = G.LlamaShape(embedding=embedding, layers=1, heads=heads, kv_heads=kv_heads, ffn=512, vocab=512,
                         context=2048)
    path = tmp_path / f"attn_{embedding}_{heads}_{kv_heads}.gguf"
    G.synthetic_llama(path, shape, seed=5)
    prompt = np.random.default_rng(9).integers(0, 512, size=150).tolist()
    ref = ReferenceModel(path)
    m = load(path, PREFILL_F32, max_positions=256)
    nxt, lg = m.prefill(prompt)
    lr = ref.prefill(prompt, capacity=256)
    ok, err, scale = close_to(lg, lr, 1e-4)
    print(f"E={embedding} H={heads} KV={kv_heads}: prefill max err {err:.3e} of {scale:.3f}")
    assert ok and nxt == int(np.argmax(lr))
    nxt2, lg2 = m.decode(nxt)
    lr2 = ref.step(nxt, len(prompt))
    ok, err, scale = close_to(lg2, lr2, 1e-4)
    assert ok, err
    m.close()
    ref.close()


@pytest.mark.parametrize("ptype,down,out", [(G.GGML_Q4_0, None, None), (G.GGML_Q4_K, G.GGML_Q6_K, G.GGML_Q6_K)])
def test_other_formats_match_reference(tmp_path, zq, ptype, down, out):
    """A Q4_0 model (fp32 prefill GEMM, the fused decode step's Q4_0
    prologue kernels) and a mixed Q4_K / Q6_K model (ffn_down and output in
    Q6_K, as llama.cpp's Q4_K_M files; the unfused decode): fp32-prefill and
    decode logits within the fp32 bar of the reference, greedy generation
    token-identical."""
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built")
    from oracle.oracle import ReferenceModel
    from zeninfer_amd.model import PREFILL_F32
    path = tmp_path / f"m_{ptype}_{down}.gguf"
    G.synthetic_llama(path, SHAPE, seed=13, proj_type=ptype, down_type=down, out_type=out)
    ref = ReferenceModel(path)
    m = load(path, PREFILL_F32)
    nxt, lg = m.prefill(PROMPT)
    lr = ref.prefill(PROMPT, capacity=128)
    ok, err, scale = close_to(lg, lr, 1e-4)
    print(f"fmt {ptype}/{down}: prefill max err {err:.3e} of {scale:.3f}")
    assert ok and nxt == int(np.argmax(lr))
    tok = nxt
    for step in range(4):
        nxt, lg = m.decode(tok)
        lr = ref.step(tok, len(PROMPT) + step)
        ok, err, scale = close_to(lg, lr, 1e-4)
        assert ok and nxt == int(np.argmax(lr)), (step, err)
        tok = nxt
    m.close()
    m = load(path, PREFILL_F32)
    ours, _, _ = m.generate(PROMPT, 16)
    theirs, _, _ = ref.generate(PROMPT, 16)
    assert ours == theirs
    m.close()
    ref.close()


def test_random_decoder_shapes_match_reference(tmp_path, zq):
    """Twelve seeded random llama configurations (head dim 64 / 128 / 256,
    1-8 query heads over 1-8 kv heads, partial RoPE, FFN and vocabulary sizes
    off the usual multiples, every projection format including Q6_K
    ffn_down / output beside Q4_K / Q5_K, prompts of 1-70 tokens): fp32
    prefill and three decode steps within the fp32 bar of the reference."""
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built")
    from oracle.oracle import ReferenceModel
    from zeninfer_amd.model import Model, PREFILL_F32
    rng = np.random.default_rng(2024)
    done = 0
    while done < 12:
        hd = int(rng.choice([64, 128, 256]))
        heads = int(rng.choice([1, 2, 4, 6, 8]))
        kv = int(rng.choice([d for d in (1, 2, 3, 4, 8) if heads % d == 0]))
        emb = hd * heads
        if emb % 256 or emb > 2048:
            continue
        pt = int(rng.choice([G.GGML_Q8_0, G.GGML_Q4_0, G.GGML_Q4_K, G.GGML_Q5_K, G.GGML_Q6_K]))
        down = G.GGML_Q6_K if pt in (G.GGML_Q4_K, G.GGML_Q5_K) and rng.random() < 0.5 else None
        shape = G.LlamaShape(embedding=emb, layers=int(rng.choice([1, 2])), heads=heads, kv_heads=kv,
                             ffn=int(rng.choice([256, 768, 1536, 2816])), vocab=int(rng.choice([300, 1000, 2051])),
                             context=512, rope_dim=int(rng.choice([0, hd // 2])))
        prompt = [int(t) for t in rng.integers(3, shape.vocab, size=int(rng.choice([1, 7, 33, 70])))]
        path = tmp_path / f"r{done}.gguf"
        G.synthetic_llama(path, shape, seed=int(rng.integers(1 << 30)), proj_type=pt, down_type=down, out_type=down)
        what = f"{shape} type {pt}/{down} prompt {len(prompt)}"
        ref = ReferenceModel(path)
        m = Model.from_gguf(G.GGUFFile(path), max_positions=128)
        m.set_prefill_mode(PREFILL_F32)
        tok, lg = m.prefill(prompt)
        ok, err, scale = close_to(lg, ref.prefill(prompt, capacity=128), 1e-4)
        assert ok, (what, "prefill", err, scale)
        for step in range(3):
            nxt, lg = m.decode(tok)
            ok, err, scale = close_to(lg, ref.step(tok, len(prompt) + step), 1e-4)
            assert ok, (what, "decode", step, err, scale)
            tok = nxt
        m.close()
        ref.close()
        done += 1
