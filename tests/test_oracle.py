"""CPU tier: pins the C oracle (oracle/zq_oracle.c) before anything is
checked against it.  Each check is chosen so that a plausible mistake in the
restatement (a dropped term, a wrong shift, a transposed index, a different
rounding) fails: known answers from the reference's own tests, the
reference's independent fp16 corpus, exhaustive / brute-force checks, the
compiled reference itself (oracle/_ref), and the committed golden vectors
the compiled reference produced (tests/golden/ref_vectors.npz).
"""
import json
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O
from tests.tolerance import assert_close

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- fp16 ----
def test_fp16_exhaustive_round_trip(orc):
    # tests/core_tests.cpp:252-262: every non-NaN binary16 survives 16->32->16.
    h = np.arange(65536, dtype=np.uint16)
    f = orc.decode_fp16(h)
    # decode against numpy's IEEE binary16 conversion (independent implementation)
    assert np.array_equal(f.view(np.uint32)[~np.isnan(f)], h.view(np.float16).astype(np.float32).view(np.uint32)[~np.isnan(f)])
    back = orc.encode_fp16(f)
    nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    assert np.array_equal(back[~nan], h[~nan])
    assert np.all((back[nan] & 0x7C00) == 0x7C00) and np.all((back[nan] & 0x3FF) != 0)


def test_fp16_known_answers(orc):
    # tests/core_tests.cpp:248-251 and 263-270 (ties-to-even, subnormal edge, overflow)
    assert list(orc.decode_fp16(np.array([0x3C00, 0xC000, 0x3800], np.uint16))) == [1.0, -2.0, 0.5]
    assert np.isinf(orc.decode_fp16(np.array([0x7C00], np.uint16))[0])
    inputs = np.array([1.0, 1.00048828125, 1.00146484375, 5.960464477539063e-8, 2.9802322387695312e-8,
                       65520.0, -0.0, np.inf], np.float32)
    expect = [0x3C00, 0x3C00, 0x3C02, 0x0001, 0x0000, 0x7C00, 0x8000, 0x7C00]
    assert list(orc.encode_fp16(inputs)) == expect


def test_fp16_reference_corpus(orc):
    # the reference's independent corpus (tests/data/fp16_reference_corpus.h), as data
    pairs = np.array(json.load(open(os.path.join(GOLDEN, "fp16_corpus.json")))["pairs"], np.uint64)
    f = pairs[:, 0].astype(np.uint32).view(np.float32)
    assert np.array_equal(orc.encode_fp16(f), pairs[:, 1].astype(np.uint16))


def test_fp16_encode_matches_numpy_rne(orc):
    # random finite binary32 values in the binary16 normal range: numpy's RNE cast is independent
    rng = np.random.default_rng(3)
    f = (rng.standard_normal(200000) * np.exp2(rng.integers(-13, 15, 200000))).astype(np.float32)
    assert np.array_equal(orc.encode_fp16(f), f.astype(np.float16).view(np.uint16))


# ------------------------------------------------------------ dequantise ---
def test_q8_0_kat(orc):
    # tests/core_tests.cpp:272-277: scale 1.0, 32 unit weights, ones -> 32
    blk = np.zeros(34, np.uint8); blk[1] = 0x3C; blk[2:] = 1
    assert orc.gemv_f32(O.Q8_0, blk, np.ones(32, np.float32), 1, 32)[0] == 32.0
    assert np.all(orc.dequantize(O.Q8_0, blk, 32) == 1.0)


def test_q6_k_kat(orc):
    # tests/core_tests.cpp:305-310
    b = np.zeros(210, np.uint8); b[209] = 0x3C; b[192:208] = 1; b[0] = 1
    out = orc.dequantize(O.Q6_K, b, 256)
    assert out[0] == -31.0 and out[32] == -32.0 and out[64] == -32.0 and out[96] == -32.0
    mask = np.ones(256, bool); mask[[0, 32, 64, 96]] = False
    assert np.all(out[mask] == -32.0)


def _build_q6k(rng, rows, cols):
    """Constructive Q6_K builder after tests/q6k_gemm_tests.cpp:17-45: the
    expected weights come from the chosen quants and scales, not a decoder."""
    nb = cols // 256
    packed = np.zeros((rows, nb, 210), np.uint8)
    expected = np.zeros((rows, cols), np.float32)
    halves = [0x3400, 0xB800, 0x0001, 0x3C00]
    factors = [0.25, -0.5, 2.0 ** -24, 1.0]
    for r in range(rows):
        for b in range(nb):
            di = (r + b) % 4
            p = packed[r, b]
            p[208], p[209] = halves[di] & 0xFF, halves[di] >> 8
            scales = rng.integers(-15, 16, 16)
            p[192:208] = scales.astype(np.int8).view(np.uint8)
            q = rng.integers(0, 64, (2, 4, 32))
            for half in range(2):
                for g in range(4):
                    col = b * 256 + half * 128 + g * 32 + np.arange(32)
                    expected[r, col] = np.float32(factors[di]) * np.float32(scales[half * 8 + g * 2 + np.arange(32) // 16]) * (q[half, g] - 32)
                p[half * 64: half * 64 + 32] = (q[half, 0] & 15) | ((q[half, 2] & 15) << 4)
                p[half * 64 + 32: half * 64 + 64] = (q[half, 1] & 15) | ((q[half, 3] & 15) << 4)
                p[128 + half * 32: 128 + half * 32 + 32] = (q[half, 0] >> 4) | ((q[half, 1] >> 4) << 2) | ((q[half, 2] >> 4) << 4) | ((q[half, 3] >> 4) << 6)
    return packed.reshape(-1), expected


def test_q6_k_constructive(orc):
    rng = np.random.default_rng(11)
    packed, expected = _build_q6k(rng, 5, 768)
    got = orc.dequantize(O.Q6_K, packed, 5 * 768).reshape(5, 768)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


def _np_dequant(fmt, w, rows, cols):
    """Closed-form numpy decoders (src/quant.cpp:391-416), independent of the C oracle."""
    if fmt == O.Q8_0:
        b = w.reshape(rows, cols // 32, 34)
        d = b[:, :, :2].copy().view(np.float16).astype(np.float32)
        return (b[:, :, 2:].view(np.int8).astype(np.float32) * d).reshape(rows, cols)
    if fmt == O.Q4_0:
        b = w.reshape(rows, cols // 32, 18)
        d = b[:, :, :2].copy().view(np.float16).astype(np.float32)
        q = b[:, :, 2:]
        vals = np.concatenate([(q & 15).astype(np.int32) - 8, (q >> 4).astype(np.int32) - 8], axis=2)
        return (vals.astype(np.float32) * d).reshape(rows, cols)
    raise ValueError


@pytest.mark.parametrize("fmt", [O.Q8_0, O.Q4_0])
def test_dequant_closed_form(orc, fmt):
    w = orc.gen_weights(fmt, 5, 9, 512)
    got = orc.dequantize(fmt, w, 9 * 512).reshape(9, 512)
    assert np.array_equal(got.view(np.uint32), _np_dequant(fmt, w, 9, 512).view(np.uint32))


# ------------------------------------------------------ Q4_K / Q5_K ----
def test_kquant_kat(orc):
    """tests/core_tests.cpp:134-159: d=1, dmin=0, scales 1, nibbles 1/2; the
    Q5_K variant sets qh[0] bit 0, which lifts element 0 by 16."""
    q4 = np.zeros(144, np.uint8)
    q4[0:4] = [0x00, 0x3C, 0x00, 0x00]
    q4[4:8] = 1
    q4[12:16] = 1
    q4[16:] = 0x21
    out = orc.dequantize(O.Q4_K, q4, 256)
    assert np.array_equal(out, np.where((np.arange(256) // 32) % 2 == 0, 1.0, 2.0).astype(np.float32))
    q5 = np.zeros(176, np.uint8)
    q5[0:4] = [0x00, 0x3C, 0x00, 0x00]
    q5[4:8] = 1
    q5[12:16] = 1
    q5[16] = 1
    q5[48:] = 0x21
    want = np.where((np.arange(256) // 32) % 2 == 0, 1.0, 2.0).astype(np.float32)
    want[0] += 16
    assert np.array_equal(orc.dequantize(O.Q5_K, q5, 256), want)


def _build_q5k(rng, rows, cols):
    """Constructive Q5_K after tests/q5k_gemm_tests.cpp:12-30: d=0.25,
    dmin=0.5, every scale and min 1, so element = 0.25*q - 0.5 for the
    independently drawn q in 0..31, packed nibble by nibble and bit by bit."""
    nb = cols // 256
    w = np.zeros((rows, nb, 176), np.uint8)
    q = rng.integers(0, 32, size=(rows, nb, 8, 32))  # [row, sb, group, lane]
    w[:, :, 0:4] = [0x00, 0x34, 0x00, 0x38]
    w[:, :, 4:12] = 1
    w[:, :, 12:16] = 0x11
    for g in range(8):
        nib = (q[:, :, g, :] & 15).astype(np.uint8)
        sl = slice(48 + (g // 2) * 32, 48 + (g // 2) * 32 + 32)
        w[:, :, sl] |= nib << 4 if g % 2 else nib
        w[:, :, 16:48] |= ((q[:, :, g, :] >> 4) << g).astype(np.uint8)
    known = (0.25 * q - 0.5).astype(np.float32).reshape(rows, cols)
    return w.reshape(-1), known


def test_q5_k_constructive(orc):
    rng = np.random.default_rng(12)
    for rows, cols in ((1, 256), (5, 768), (67, 768)):
        w, known = _build_q5k(rng, rows, cols)
        got = orc.dequantize(O.Q5_K, w, rows * cols).reshape(rows, cols)
        assert np.array_equal(got, known)
        for tokens in (1, 2, 3, 8):
            x = (rng.integers(0, 256, size=tokens * cols) - 128).astype(np.float32) / 128
            ref = known.astype(np.float64) @ x.reshape(tokens, cols).T.astype(np.float64)
            mag = np.abs(known.astype(np.float64)) @ np.abs(x.reshape(tokens, cols).T.astype(np.float64))
            y = orc.gemm_f32(O.Q5_K, w, x, tokens, rows, cols).reshape(tokens, rows)
            assert (np.abs(y - ref.T) <= 2e-5 * np.maximum(1.0, mag.T)).all()


def _np_kquant_dequant(w, rows, cols, q5):
    """Textbook decoder of the GGML K-quant layout, independent of the C
    oracle: 6-bit scale/min pairs (j<4: q[j]&63, q[j+4]&63; j>=4: low/high
    nibble of q[j+4] with the top two bits of q[j-4] / q[j]), value
    (d*sc)*q - dmin*m."""
    bb = 176 if q5 else 144
    b = w.reshape(rows, cols // 256, bb)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    dm = b[:, :, 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
    s = b[:, :, 4:16].astype(np.uint32)
    sc = np.empty(b.shape[:2] + (8,), np.uint32)
    mn = np.empty_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j], mn[..., j] = s[..., j] & 63, s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    qs = b[:, :, (48 if q5 else 16):].reshape(rows, cols // 256, 4, 32).astype(np.uint32)
    q = np.empty(b.shape[:2] + (8, 32), np.uint32)
    for j in range(8):
        q[:, :, j] = (qs[:, :, j // 2] >> (4 * (j % 2))) & 15
        if q5:
            q[:, :, j] |= ((b[:, :, 16:48].astype(np.uint32) >> j) & 1) << 4
    ds = (d[..., None] * sc.astype(np.float32)).astype(np.float32)
    ms = (dm[..., None] * mn.astype(np.float32)).astype(np.float32)
    v = (ds[..., None] * q.astype(np.float32)).astype(np.float32) - ms[..., None]
    return v.astype(np.float32).reshape(rows, cols)


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q5_K])
def test_kquant_closed_form_random_blocks(orc, fmt):
    """Random bytes with finite scales incl. fp16 subnormals and negative d,
    as in tests/core_tests.cpp:202-216."""
    rows, cols = 67, 768
    bb = 176 if fmt == O.Q5_K else 144
    rng = np.random.default_rng(13)
    w = rng.integers(0, 256, size=(rows, cols // 256, bb), dtype=np.uint8)
    for r in range(rows):
        for b in range(cols // 256):
            ds = 0x0001 if b % 3 == 0 else (0xA800 if r % 2 else 0x2800)
            dm = 0x2000 if b % 2 else 0x1800
            w[r, b, 0:4] = [ds & 255, ds >> 8, dm & 255, dm >> 8]
    w = w.reshape(-1)
    got = orc.dequantize(fmt, w, rows * cols).reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), _np_kquant_dequant(w, rows, cols, fmt == O.Q5_K).view(np.uint32))
    x = np.array([float(int((c * 17) % 101) - 50) * 0.013 for c in range(cols)], np.float32)
    y = orc.gemv_f32(fmt, w, x, rows, cols)
    ref = got.astype(np.float64) @ x.astype(np.float64)
    mag = np.abs(got.astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert (np.abs(y - ref) <= 2e-5 * np.maximum(1.0, mag)).all()


# ------------------------------------------------- activation quantiser ----
def _np_quantize(x, m, k):
    """kernels/avx2.cpp:502-524 in numpy float32 arithmetic."""
    xb = x.reshape(m, k // 32, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=2)
    d = np.where(amax > 0, amax / np.float32(127.0), np.float32(0)).astype(np.float32)
    inv = np.where(d > 0, np.float32(1.0) / np.where(d > 0, d, 1), np.float32(0)).astype(np.float32)
    v = np.clip(xb * inv[:, :, None], -127, 127).astype(np.float32)
    q = np.where(v >= 0, np.floor(v + np.float64(0.5)), np.ceil(v - np.float64(0.5)))  # lround, in double: exact
    return q.astype(np.int8).reshape(-1), d.reshape(-1)


def test_quantize_acts_ties_and_edges(orc):
    # amax = 127 -> d = 1, inv = 1: exact .5 ties round away from zero
    b0 = np.array([127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [0.0] * 24, np.float32)
    b1 = np.zeros(32, np.float32)                       # amax == 0 -> d = 0, q = 0
    b2 = np.full(32, -3.0, np.float32)                  # all equal, negative
    b3 = np.array([1e-30] + [0.0] * 31, np.float32)     # tiny amax
    x = np.concatenate([b0, b1, b2, b3])
    q, d = orc.quantize_acts(x, 1, 128)
    assert list(q[:8]) == [127, 3, -3, 1, -1, 2, -2, 127]
    assert d[1] == 0 and np.all(q[32:64] == 0)
    assert np.all(q[64:96] == -127)
    q2, d2 = _np_quantize(x, 1, 128)
    assert np.array_equal(q, q2) and np.array_equal(d.view(np.uint32), d2.view(np.uint32))


def test_quantize_acts_random(orc):
    x = orc.gen_normal(77, 64 * 4096)
    q, d = orc.quantize_acts(x, 64, 4096)
    q2, d2 = _np_quantize(x, 64, 4096)
    assert np.array_equal(q, q2) and np.array_equal(d.view(np.uint32), d2.view(np.uint32))


# --------------------------------------------------------- block dots ------
@pytest.mark.parametrize("fmt,cols", [(O.Q8_0, 256), (O.Q4_0, 256), (O.Q6_K, 512)])
def test_block_dots_brute_force(orc, fmt, cols):
    rows, m = 7, 3
    w = orc.gen_weights(fmt, 9, rows, cols)
    xq, _ = orc.quantize_acts(orc.gen_normal(10, m * cols), m, cols)
    got = orc.block_dots(fmt, w, xq, m, rows, cols).reshape(m, rows, cols // 32)
    if fmt == O.Q6_K:
        # integer weights: dequantised value / d, exactly (q-32)*sc
        deq = orc.dequantize(fmt, w, rows * cols).reshape(rows, cols // 256, 256)
        d = w.reshape(rows, cols // 256, 210)[:, :, 208:210].copy().view(np.float16).astype(np.float64)
        wi = np.rint(deq / d).astype(np.int64).reshape(rows, cols)
    else:
        deq = orc.dequantize(fmt, w, rows * cols).reshape(rows, cols // 32, 32)
        bs = 34 if fmt == O.Q8_0 else 18
        d = w.reshape(rows, cols // 32, bs)[:, :, :2].copy().view(np.float16).astype(np.float64)
        wi = np.rint(deq / d).astype(np.int64).reshape(rows, cols)
    want = (xq.reshape(m, 1, cols // 32, 32).astype(np.int64) * wi.reshape(1, rows, cols // 32, 32)).sum(-1)
    assert np.array_equal(got, want)


# ------------------------------------------ oracle vs compiled reference ----
def _golden():
    return dict(np.load(os.path.join(GOLDEN, "ref_vectors.npz")))


FMT_OF = {"q8": O.Q8_0, "q4": O.Q4_0, "q6": O.Q6_K, "k4": O.Q4_K, "k5": O.Q5_K}


def _cases():
    g = _golden()
    return sorted(k[:-6] for k in g if k.endswith("_shape"))


@pytest.mark.parametrize("case", _cases())
def test_oracle_matches_reference_golden(orc, case):
    g = _golden()
    fmt = FMT_OF[case[:2]]
    rows, cols, tokens = (int(v) for v in g[case + "_shape"])
    w, X = g[case + "_w"], g[case + "_x"]
    # the seeded generators still reproduce the stored inputs
    assert np.array_equal(orc.gen_weights(fmt, 0xA11CE + _cases_index(case), rows, cols), w)
    assert np.array_equal(orc.dequantize(fmt, w, rows * cols).view(np.uint32), g[case + "_ref_dequant"].view(np.uint32))
    # bit equality with the reference's AVX2 kernels (same fp32 operation order)
    assert np.array_equal(orc.gemv_f32(fmt, w, X[:cols], rows, cols), g[case + "_ref_gemv"])
    assert np.array_equal(orc.gemm_f32(fmt, w, X, tokens, rows, cols), g[case + "_ref_gemm"])
    assert np.array_equal(orc.gemm_f32(fmt, w, X[:cols], 1, rows, cols), g[case + "_ref_gemm1"])
    if case + "_ref_gemm_i8" in g:
        assert np.array_equal(orc.gemm_i8(fmt, w, X, tokens, rows, cols), g[case + "_ref_gemm_i8"])


def _cases_index(case):
    from tests.golden.make_golden import CASES, NAME
    keys = [f"{NAME[f]}_{r}x{c}" for f, r, c, _ in CASES]
    return keys.index(case)


@pytest.mark.parametrize("fmt,rows,cols", [(O.Q8_0, 67, 1024), (O.Q4_0, 35, 768), (O.Q6_K, 35, 1280),
                                           (O.Q8_0, 130, 4096), (O.Q4_K, 67, 768), (O.Q4_K, 9, 4096),
                                           (O.Q5_K, 67, 768), (O.Q5_K, 10, 4096)])
def test_oracle_matches_compiled_reference(orc, ref, fmt, rows, cols):
    w = orc.gen_weights(fmt, 21, rows, cols)
    x = orc.gen_normal(22, 9 * cols)
    assert np.array_equal(orc.dequantize(fmt, w, rows * cols), ref.dequantize(fmt, w, rows * cols))
    assert np.array_equal(orc.gemv_f32(fmt, w, x[:cols], rows, cols), ref.gemv(fmt, w, x[:cols], rows, cols))
    for m in (1, 2, 5, 9):
        assert np.array_equal(orc.gemm_f32(fmt, w, x[:m * cols], m, rows, cols), ref.gemm(fmt, w, x[:m * cols], m, rows, cols))


def test_fp16_codec_matches_compiled_reference(orc, ref):
    h = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(orc.decode_fp16(h).view(np.uint32), ref.decode_fp16(h).view(np.uint32))
    rng = np.random.default_rng(5)
    f = rng.integers(0, 2 ** 32, 500000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert np.array_equal(orc.encode_fp16(f), ref.encode_fp16(f))


# --------------------------------------------------- double references -----
@pytest.mark.parametrize("fmt,cols", [(O.Q8_0, 4096), (O.Q4_0, 4096), (O.Q6_K, 4096), (O.Q8_0, 14336),
                                      (O.Q4_K, 4096), (O.Q5_K, 14336)])
def test_fp32_paths_within_tolerance_of_double(orc, fmt, cols):
    rows, m = 16, 3
    w = orc.gen_weights(fmt, 31, rows, cols)
    X = orc.gen_normal(32, m * cols)
    y64, _ = orc.gemm_f64(fmt, w, X, m, rows, cols)
    assert_close(orc.gemm_f32(fmt, w, X, m, rows, cols), y64, "gemm_f32 vs double")
    assert_close(orc.gemv_f32(fmt, w, X[:cols], rows, cols), y64[:rows], "gemv_f32 vs double")


def test_int8_gemm_against_double_of_quantised(orc):
    # the int8 route's value is sum_b dx*dw*dot_b; its double evaluation bounds the fp32 one
    fmt, rows, cols, m = O.Q8_0, 12, 4096, 3
    w = orc.gen_weights(fmt, 41, rows, cols)
    X = orc.gen_normal(42, m * cols)
    xq, xs = orc.quantize_acts(X, m, cols)
    dots = orc.block_dots(fmt, w, xq, m, rows, cols).reshape(m, rows, cols // 32).astype(np.float64)
    dw = w.reshape(rows, cols // 32, 34)[:, :, :2].copy().view(np.float16).astype(np.float32)
    s = (dw[None, :, :, 0] * xs.reshape(m, 1, cols // 32)).astype(np.float64)
    want = (dots * s).sum(-1).reshape(-1)
    assert_close(orc.gemm_i8(fmt, w, X, m, rows, cols), want, "gemm_i8 vs double")


@pytest.mark.parametrize("fmt", [O.Q8_0, O.Q4_0, O.Q6_K])
def test_int8_gemm_prequant_is_the_int8_gemm_after_quantisation(orc, fmt):
    # gemm_i8 = quantize_acts then gemm_i8_prequant; the Q8_0 gemm_i8 is pinned
    # bit-exact to the reference's int8 route by the golden vectors above
    rows, cols, m = 9, 2048, 4
    w = orc.gen_weights(fmt, 43, rows, cols)
    X = orc.gen_normal(44, m * cols)
    xq, xs = orc.quantize_acts(X, m, cols)
    assert np.array_equal(orc.gemm_i8_prequant(fmt, w, xq, xs, m, rows, cols), orc.gemm_i8(fmt, w, X, m, rows, cols))


def test_generators_are_counter_based(orc):
    # draw i of a stream is the (i+1)-th output of sequential SplitMix64
    state, seq = 12345, []
    M = (1 << 64) - 1
    for _ in range(5):
        state = (state + 0x9E3779B97F4A7C15) & M
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        seq.append(z ^ (z >> 31))
    assert [orc.L.zqo_splitmix64_at(12345, i) for i in range(5)] == seq
    x = orc.gen_normal(1, 200000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1) < 0.01
