"""Python handle of the device-resident decoder (include/zq_model.h).

``Model.from_gguf(GGUFFile(...))`` uploads a llama-architecture GGUF once;
``Model.synthetic(config)`` builds a random-init model directly in HBM.  Every
call goes through the HIP library; there is no CPU fallback.  The interface
mirrors the reference runtime's (DenseTransformerRuntime::forward_batch /
forward / generate, include/zen/dense_transformer_runtime.h:20-78).
"""
import ctypes

import numpy as np

from . import zq

PREFILL_INT8, PREFILL_F32 = 0, 1
GLOBAL = 0xFFFFFFFF
W_EMBED, W_OUTPUT, W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN = range(9)
TAP_QKV, TAP_Q, TAP_K, TAP_V, TAP_O, TAP_GATE, TAP_UP, TAP_DOWN = range(8)


class ModelError(RuntimeError):
    pass


class Model:
    def __init__(self, handle, cfg):
        self._L = zq.lib()
        self._h = handle
        self.config = {n: getattr(cfg, n) for n, _ in cfg._fields_}

    @classmethod
    def from_gguf(cls, gguf, max_positions=0):
        L = zq.lib()
        cfg = zq.ModelConfig()
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        st = L.zq_model_load_gguf(gguf._h, max_positions, ctypes.byref(cfg), ctypes.byref(h), err, 512)
        if st != 0:
            raise ModelError(f"model load failed ({st}): {err.value.decode()}")
        return cls(h, cfg)

    @classmethod
    def synthetic(cls, seed=0x5EED0004, **shape):
        L = zq.lib()
        cfg = zq.ModelConfig()
        for k, v in shape.items():
            setattr(cfg, k, v)
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        st = L.zq_model_create_synthetic(ctypes.byref(cfg), seed, ctypes.byref(h), err, 512)
        if st != 0:
            raise ModelError(f"synthetic model failed ({st}): {err.value.decode()}")
        return cls(h, cfg)

    def close(self):
        if self._h:
            self._L.zq_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_prefill_mode(self, mode):
        zq.check(self._L.zq_model_set_prefill_mode(self._h, mode), "set_prefill_mode")

    def prefill(self, tokens, logits=True):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.config["vocab"], np.float32) if logits else None
        nxt = ctypes.c_uint32()
        zq.check(self._L.zq_model_prefill(self._h, t.ctypes.data_as(ctypes.c_void_p), t.size,
                                          out.ctypes.data_as(ctypes.c_void_p) if logits else None, ctypes.byref(nxt)),
                 "prefill")
        return nxt.value, out

    def decode(self, token, logits=True):
        out = np.empty(self.config["vocab"], np.float32) if logits else None
        nxt = ctypes.c_uint32()
        zq.check(self._L.zq_model_decode(self._h, int(token), out.ctypes.data_as(ctypes.c_void_p) if logits else None,
                                         ctypes.byref(nxt)), "decode")
        return nxt.value, out

    def generate(self, prompt, max_new):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = ctypes.c_size_t()
        pm, dm = ctypes.c_double(), ctypes.c_double()
        zq.check(self._L.zq_model_generate(self._h, p.ctypes.data_as(ctypes.c_void_p), p.size, max_new,
                                           out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n), ctypes.byref(pm),
                                           ctypes.byref(dm)), "generate")
        return out[:n.value].tolist(), pm.value, dm.value

    def weight(self, layer, which):
        """(device address, rows, cols, GGML type) of one resident weight."""
        p, r, c, f = ctypes.c_void_p(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_int()
        zq.check(self._L.zq_model_weight(self._h, layer, which, ctypes.byref(p), ctypes.byref(r), ctypes.byref(c),
                                         ctypes.byref(f)), "weight")
        return p.value, r.value, c.value, f.value

    def set_tap(self, layer, dev_ptr, cap):
        """Record one layer's int8 prefill projections into a device buffer
        (zq_model_set_tap); dev_ptr 0 turns it off."""
        zq.check(self._L.zq_model_set_tap(self._h, layer, dev_ptr or None, cap), "set_tap")

    def tap_records(self):
        """The last prefill's tap records (zq_model_tap_records); raises
        ZQError(TOO_LARGE) when the buffer could not hold every projection."""
        recs = (zq.TapRecord * 16)()
        n = ctypes.c_size_t()
        zq.check(self._L.zq_model_tap_records(self._h, recs, 16, ctypes.byref(n)), "tap_records")
        return [recs[i] for i in range(n.value)]

    def memory(self):
        w, c, a = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        zq.check(self._L.zq_model_memory(self._h, ctypes.byref(w), ctypes.byref(c), ctypes.byref(a)), "memory")
        return {"weights": w.value, "kv_cache": c.value, "activations": a.value}
