"""Writes tests/golden/ref_vectors.npz and fp16_corpus.json.

Run in the build container, where the reference sources exist and
oracle/_ref/libzenref.so (the reference's own CPU quant path, compiled from
its sources by oracle/Makefile) can be built:

    python tests/golden/make_golden.py

Inputs are generated with the oracle's seeded generators and stored next to
the reference's outputs, so the fixture is self-contained data.  The int8
activation route of the reference (ZEN_CPU_Q8_ACT=1, src/quant.cpp:1087-1122)
is read from a child process because the reference caches that switch.
fp16_corpus.json is the pair list of the reference's independent binary16
corpus (tests/data/fp16_reference_corpus.h), transcribed as data.
"""
import json
import os
import re
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

CASES = [  # (fmt, rows, cols, tokens)
    (O.Q8_0, 33, 256, 5), (O.Q8_0, 8, 4096, 3), (O.Q8_0, 5, 96, 2),
    (O.Q4_0, 33, 256, 5), (O.Q4_0, 7, 1024, 4),
    (O.Q6_K, 33, 256, 5), (O.Q6_K, 6, 1280, 3),
    (O.Q4_K, 33, 256, 5), (O.Q4_K, 6, 1280, 3), (O.Q5_K, 33, 256, 5), (O.Q5_K, 7, 768, 4),
]
NAME = {O.Q8_0: "q8", O.Q4_0: "q4", O.Q6_K: "q6", O.Q4_K: "k4", O.Q5_K: "k5"}


def int8_route(path_npz):
    """Child process: the reference's int8 GEMV per token for every Q8_0 case."""
    env = dict(os.environ, ZEN_CPU_Q8_ACT="1")
    code = f"""
import sys, numpy as np
sys.path.insert(0, {ROOT!r})
from oracle import oracle as O
r = O.Reference()
d = dict(np.load({path_npz!r}))
out = {{}}
for key in [k for k in d if k.endswith('_w') and k.startswith('q8')]:
    p = key[:-2]
    rows, cols, tokens = (int(v) for v in d[p + '_shape'])
    X = d[p + '_x']
    out[p + '_ref_gemm_i8'] = np.concatenate([r.gemv(O.Q8_0, d[key], X[t*cols:(t+1)*cols], rows, cols, 1) for t in range(tokens)])
np.savez({path_npz + '.i8.npz'!r}, **out)
"""
    subprocess.check_call([sys.executable, "-c", code], env=env)
    res = dict(np.load(path_npz + ".i8.npz"))
    os.remove(path_npz + ".i8.npz")
    return res


def main():
    O.build()
    o, r = O.Oracle(), O.Reference()
    name = NAME
    data = {}
    for i, (fmt, rows, cols, tokens) in enumerate(CASES):
        p = f"{name[fmt]}_{rows}x{cols}"
        w = o.gen_weights(fmt, 0xA11CE + i, rows, cols)
        X = o.gen_normal(0xB0B + i, tokens * cols)
        data[p + "_shape"] = np.array([rows, cols, tokens], np.int64)
        data[p + "_w"] = w
        data[p + "_x"] = X
        data[p + "_ref_dequant"] = r.dequantize(fmt, w, rows * cols)
        data[p + "_ref_gemv"] = r.gemv(fmt, w, X[:cols], rows, cols, 1)
        data[p + "_ref_gemm"] = r.gemm(fmt, w, X, tokens, rows, cols, 1)
        data[p + "_ref_gemm1"] = r.gemm(fmt, w, X[:cols], 1, rows, cols, 1)
    tmp = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(tmp, **data)
    data.update(int8_route(tmp))
    np.savez_compressed(tmp, **data)

    hdr = "/root/reference/tests/data/fp16_reference_corpus.h"
    pairs = re.findall(r"\{0x([0-9a-fA-F]+)u,0x([0-9a-fA-F]+)u\}", open(hdr).read())
    with open(os.path.join(HERE, "fp16_corpus.json"), "w") as f:
        json.dump({"source": "tests/data/fp16_reference_corpus.h (reference tree)",
                   "pairs": [[int(a, 16), int(b, 16)] for a, b in pairs]}, f)
    print(f"{len(data)} arrays, {len(pairs)} fp16 pairs")


if __name__ == "__main__":
    main()
