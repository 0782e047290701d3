"""ctypes bindings for the C oracle (liboracle.so) and the compiled reference
(_ref/libzenref.so).  TEST INFRASTRUCTURE ONLY -- the checker, never the
product; see zq_oracle.c for what each function restates and how it is pinned.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libzenref.so")

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

_P = ctypes.c_void_p
_S = ctypes.c_size_t
_U64 = ctypes.c_uint64


def build(reference_root="/root/reference"):
    """Compile liboracle.so, and _ref/libzenref.so when the reference tree exists."""
    targets = ["oracle"]
    if os.path.isdir(reference_root):
        targets.append("ref")
    subprocess.check_call(["make", "-s", "-C", HERE, f"REF={reference_root}", "-j8", *targets])


def _ptr(a):
    return a.ctypes.data_as(_P)


class Oracle:
    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run oracle.build())")
        L = ctypes.CDLL(path)
        L.zqo_half_to_float.restype = ctypes.c_float
        L.zqo_half_to_float.argtypes = [ctypes.c_uint16]
        L.zqo_float_to_half.restype = ctypes.c_uint16
        L.zqo_float_to_half.argtypes = [ctypes.c_float]
        L.zqo_row_bytes.restype = _S
        L.zqo_row_bytes.argtypes = [ctypes.c_int, _S]
        L.zqo_splitmix64_at.restype = _U64
        L.zqo_splitmix64_at.argtypes = [_U64, _U64]
        L.zqo_normal_at.restype = ctypes.c_double
        L.zqo_normal_at.argtypes = [_U64, _U64]
        for name in ("zqo_gen_q8_0", "zqo_gen_q4_0", "zqo_gen_q6_k", "zqo_gen_q4_k", "zqo_gen_q5_k"):
            getattr(L, name).argtypes = [_U64, _S, _S, _P]
        L.zqo_gen_normal_f32.argtypes = [_U64, _S, _P]
        L.zqo_decode_fp16.argtypes = [_P, _P, _S]
        L.zqo_encode_fp16.argtypes = [_P, _P, _S]
        L.zqo_dequantize.restype = ctypes.c_int
        L.zqo_dequantize.argtypes = [ctypes.c_int, _P, _S, _P]
        L.zqo_quantize_acts.argtypes = [_P, _S, _S, _P, _P]
        L.zqo_block_dots.restype = ctypes.c_int
        L.zqo_block_dots.argtypes = [ctypes.c_int, _P, _P, _S, _S, _S, _P]
        L.zqo_gemv_f32.restype = ctypes.c_int
        L.zqo_gemv_f32.argtypes = [ctypes.c_int, _P, _P, _P, _S, _S]
        L.zqo_gemm_f32.restype = ctypes.c_int
        L.zqo_gemm_f32.argtypes = [ctypes.c_int, _P, _P, _P, _S, _S, _S]
        L.zqo_gemm_i8.restype = ctypes.c_int
        L.zqo_gemm_i8.argtypes = [ctypes.c_int, _P, _P, _P, _S, _S, _S]
        L.zqo_gemm_i8_prequant.restype = ctypes.c_int
        L.zqo_gemm_i8_prequant.argtypes = [ctypes.c_int, _P, _P, _P, _P, _S, _S, _S]
        L.zqo_gemm_f64.restype = ctypes.c_int
        L.zqo_gemm_f64.argtypes = [ctypes.c_int, _P, _P, _P, _P, _S, _S, _S]
        self.L = L

    # --- codec -------------------------------------------------------------
    def decode_fp16(self, h):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.L.zqo_decode_fp16(_ptr(h), _ptr(out), h.size)
        return out

    def encode_fp16(self, f):
        f = np.ascontiguousarray(f, dtype=np.float32)
        out = np.empty(f.shape, np.uint16)
        self.L.zqo_encode_fp16(_ptr(f), _ptr(out), f.size)
        return out

    def row_bytes(self, fmt, cols):
        return self.L.zqo_row_bytes(fmt, cols)

    # --- synthetic inputs ---------------------------------------------------
    def gen_weights(self, fmt, seed, rows, cols):
        rb = self.row_bytes(fmt, cols)
        if not rb:
            raise ValueError("cols not a multiple of the block size")
        out = np.empty(rows * rb, np.uint8)
        fn = {Q8_0: self.L.zqo_gen_q8_0, Q4_0: self.L.zqo_gen_q4_0, Q6_K: self.L.zqo_gen_q6_k,
              Q4_K: self.L.zqo_gen_q4_k, Q5_K: self.L.zqo_gen_q5_k}[fmt]
        fn(seed, rows, cols, _ptr(out))
        return out

    def gen_normal(self, seed, n):
        out = np.empty(n, np.float32)
        self.L.zqo_gen_normal_f32(seed, n, _ptr(out))
        return out

    # --- arithmetic -----------------------------------------------------------
    def dequantize(self, fmt, src, n):
        src = np.ascontiguousarray(src, dtype=np.uint8)
        out = np.empty(n, np.float32)
        if not self.L.zqo_dequantize(fmt, _ptr(src), n, _ptr(out)):
            raise ValueError("dequantize declined")
        return out

    def quantize_acts(self, x, m, k):
        x = np.ascontiguousarray(x, dtype=np.float32)
        xq = np.empty(m * k, np.int8)
        xs = np.empty(m * (k // 32), np.float32)
        self.L.zqo_quantize_acts(_ptr(x), m, k, _ptr(xq), _ptr(xs))
        return xq, xs

    def block_dots(self, fmt, w, xq, m, n, k):
        out = np.empty(m * n * (k // 32), np.int32)
        xq = np.ascontiguousarray(xq, dtype=np.int8)
        if not self.L.zqo_block_dots(fmt, _ptr(w), _ptr(xq), m, n, k, _ptr(out)):
            raise ValueError("block_dots declined")
        return out

    def gemv_f32(self, fmt, w, x, rows, cols):
        y = np.empty(rows, np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        if not self.L.zqo_gemv_f32(fmt, _ptr(w), _ptr(x), _ptr(y), rows, cols):
            raise ValueError("gemv declined")
        return y

    def gemm_f32(self, fmt, w, X, m, n, k):
        Y = np.empty(m * n, np.float32)
        X = np.ascontiguousarray(X, dtype=np.float32)
        if not self.L.zqo_gemm_f32(fmt, _ptr(w), _ptr(X), _ptr(Y), m, n, k):
            raise ValueError("gemm declined")
        return Y

    def gemm_i8(self, fmt, w, X, m, n, k):
        Y = np.empty(m * n, np.float32)
        X = np.ascontiguousarray(X, dtype=np.float32)
        if not self.L.zqo_gemm_i8(fmt, _ptr(w), _ptr(X), _ptr(Y), m, n, k):
            raise ValueError("gemm_i8 declined")
        return Y

    def gemm_i8_prequant(self, fmt, w, xq, xs, m, n, k):
        """gemm_i8 on activations already quantised (int8 [m][k], scales [m][k/32])."""
        Y = np.empty(m * n, np.float32)
        xq = np.ascontiguousarray(xq, dtype=np.int8)
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        assert xq.size == m * k and xs.size == m * (k // 32)
        if not self.L.zqo_gemm_i8_prequant(fmt, _ptr(w), _ptr(xq), _ptr(xs), _ptr(Y), m, n, k):
            raise ValueError("gemm_i8_prequant declined")
        return Y

    def gemm_f64(self, fmt, w, X, m, n, k):
        Y = np.empty(m * n, np.float64)
        mag = np.empty(m * n, np.float64)
        X = np.ascontiguousarray(X, dtype=np.float32)
        if not self.L.zqo_gemm_f64(fmt, _ptr(w), _ptr(X), _ptr(Y), _ptr(mag), m, n, k):
            raise ValueError("gemm_f64 declined")
        return Y, mag


class Reference:
    """The reference's own CPU quant surface, compiled from its sources."""

    def __init__(self, path=REF_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"reference library missing: {path}")
        L = ctypes.CDLL(path)
        L.zr_gemv.restype = ctypes.c_int
        L.zr_gemv.argtypes = [ctypes.c_int, _P, _P, _P, _S, _S, ctypes.c_uint]
        L.zr_gemm.restype = ctypes.c_int
        L.zr_gemm.argtypes = [ctypes.c_int, _P, _P, _P, _S, _S, _S, ctypes.c_uint]
        L.zr_dequantize.restype = ctypes.c_int
        L.zr_dequantize.argtypes = [ctypes.c_int, _P, _S, _P]
        L.zr_decode_fp16.argtypes = [_P, _P, _S]
        L.zr_encode_fp16.argtypes = [_P, _P, _S]
        L.zr_row_bytes.restype = _S
        L.zr_row_bytes.argtypes = [ctypes.c_int, _S]
        L.zr_pool_workers.restype = ctypes.c_uint
        L.zr_has_avx2.restype = ctypes.c_int
        self.L = L

    def has_avx2(self):
        return bool(self.L.zr_has_avx2())

    def pool_workers(self):
        return int(self.L.zr_pool_workers())

    def row_bytes(self, fmt, cols):
        return self.L.zr_row_bytes(fmt, cols)

    def decode_fp16(self, h):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.L.zr_decode_fp16(_ptr(h), _ptr(out), h.size)
        return out

    def encode_fp16(self, f):
        f = np.ascontiguousarray(f, dtype=np.float32)
        out = np.empty(f.shape, np.uint16)
        self.L.zr_encode_fp16(_ptr(f), _ptr(out), f.size)
        return out

    def dequantize(self, fmt, src, n):
        out = np.empty(n, np.float32)
        if not self.L.zr_dequantize(fmt, _ptr(np.ascontiguousarray(src, np.uint8)), n, _ptr(out)):
            raise ValueError("reference dequantize declined")
        return out

    def gemv(self, fmt, w, x, rows, cols, workers=1):
        y = np.empty(rows, np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        if not self.L.zr_gemv(fmt, _ptr(w), _ptr(x), _ptr(y), rows, cols, workers):
            raise ValueError("reference gemv declined")
        return y

    def gemm(self, fmt, w, X, m, n, k, workers=1):
        Y = np.empty(m * n, np.float32)
        X = np.ascontiguousarray(X, dtype=np.float32)
        if not self.L.zr_gemm(fmt, _ptr(w), _ptr(X), _ptr(Y), m, n, k, workers):
            raise ValueError("reference gemm declined")
        return Y


def reference_available():
    return os.path.exists(REF_PATH)


class ReferenceModel:
    """The reference's own DenseTransformerRuntime (load / forward_batch /
    forward / generate), compiled from its sources into oracle/_ref.  Test
    infrastructure: the end-to-end checker of the device-resident model."""

    def __init__(self, path, lib_path=REF_PATH):
        if not os.path.exists(lib_path):
            raise RuntimeError(f"reference library missing: {lib_path}")
        L = ctypes.CDLL(lib_path)
        L.zr_model_load.restype = _P
        L.zr_model_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _S]
        L.zr_model_free.argtypes = [_P]
        L.zr_model_config.argtypes = [_P, _P]
        L.zr_model_prefill.restype = ctypes.c_int
        L.zr_model_prefill.argtypes = [_P, _P, _S, _S, _P]
        L.zr_model_step.restype = ctypes.c_int
        L.zr_model_step.argtypes = [_P, ctypes.c_uint32, ctypes.c_uint32, _P]
        L.zr_model_generate.restype = ctypes.c_int
        L.zr_model_generate.argtypes = [_P, _P, _S, ctypes.c_uint32, _P, _P, _P, _P]
        self.L = L
        err = ctypes.create_string_buffer(512)
        self.h = L.zr_model_load(str(path).encode(), err, 512)
        if not self.h:
            raise RuntimeError(f"reference load failed: {err.value.decode()}")
        c = (ctypes.c_uint32 * 9)()
        L.zr_model_config(self.h, c)
        self.config = dict(zip(("embedding", "layers", "heads", "kv_heads", "head_dim", "ffn", "vocab", "context",
                                "eos"), list(c)))

    def close(self):
        if self.h:
            self.L.zr_model_free(self.h)
            self.h = None

    def prefill(self, tokens, capacity):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.config["vocab"], np.float32)
        if not self.L.zr_model_prefill(self.h, _ptr(t), t.size, capacity, _ptr(out)):
            raise RuntimeError("reference forward_batch failed")
        return out

    def step(self, token, pos):
        out = np.empty(self.config["vocab"], np.float32)
        if not self.L.zr_model_step(self.h, int(token), int(pos), _ptr(out)):
            raise RuntimeError("reference forward failed")
        return out

    def generate(self, prompt, max_new):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = ctypes.c_size_t()
        pm, dm = ctypes.c_double(), ctypes.c_double()
        if not self.L.zr_model_generate(self.h, _ptr(p), p.size, max_new, _ptr(out), ctypes.byref(n),
                                        ctypes.byref(pm), ctypes.byref(dm)):
            raise RuntimeError("reference generate failed")
        return out[:n.value].tolist(), pm.value, dm.value
