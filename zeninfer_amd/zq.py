"""Python binding of the C ABI in include/zq_hip.h (ctypes).

The library must be built (``zeninfer_amd.build``); loading fails loudly when
it is missing -- there is no CPU fallback on this path.  Host-pointer calls
take numpy arrays; the *_dev calls take torch tensors (device memory and
streams only) or raw integer device pointers.
"""
import ctypes
import os

import numpy as np

from .build import LIB

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
FORMATS = {"Q4_0": Q4_0, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
ACT_DEFAULT, ACT_INT8, ACT_F32 = 0, 1, 2
OK, DECLINED = 0, 1
ERR_ARG, ERR_NO_DEVICE, ERR_OOM, ERR_HIP, ERR_TOO_LARGE = -1, -2, -3, -4, -5
WEIGHT_TAIL_PAD = 64
MAX_BATCH = 8

_P = ctypes.c_void_p
_S = ctypes.c_size_t


class ZQError(RuntimeError):
    def __init__(self, status, what):
        self.status = status
        super().__init__(f"{what}: status {status} ({status_string(status)})")


class Info(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("arch", ctypes.c_char * 64), ("vram_bytes", ctypes.c_uint64),
                ("compute_units", ctypes.c_int), ("wave_size", ctypes.c_int), ("lds_per_block", ctypes.c_int),
                ("clock_khz", ctypes.c_int), ("mem_clock_khz", ctypes.c_int), ("mem_bus_width", ctypes.c_int)]


class Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "dispatches", "submits", "batches", "uploads", "upload_bytes", "resident_bytes", "resident_tensors",
        "evictions", "declined", "errors", "upload_us", "transfer_us", "wait_us", "fallbacks", "alloc_us",
        "launch_us", "readback_us", "gpu_us")]


class GemvTask(ctypes.Structure):
    _fields_ = [("weights", _P), ("y", _P), ("rows", _S)]


class GemmTask(ctypes.Structure):
    _fields_ = [("weights", _P), ("Y", _P), ("rows", _S)]




# Every symbol include/zq_hip.h declares, with (restype, argtypes).
SIGNATURES = {
    "zq_hip_opted_in": (ctypes.c_int, []),
    "zq_hip_init": (ctypes.c_int, []),
    "zq_hip_enabled": (ctypes.c_int, []),
    "zq_hip_shutdown": (None, []),
    "zq_hip_get_info": (ctypes.c_int, [ctypes.POINTER(Info)]),
    "zq_hip_get_stats": (ctypes.c_int, [ctypes.POINTER(Stats)]),
    "zq_hip_reset_stats": (None, []),
    "zq_hip_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "zq_row_bytes": (_S, [ctypes.c_int, _S]),
    "zq_weight_bytes": (_S, [ctypes.c_int, _S, _S]),
    "zq_hip_set_min_elements": (_S, [_S]),
    "zq_hip_gemv": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _S, _S]),
    "zq_hip_gemv_batch": (ctypes.c_int, [ctypes.c_int, _P, ctypes.POINTER(GemvTask), _S, _S]),
    "zq_hip_gemm": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _S, _S, _S, ctypes.c_int]),
    "zq_hip_ffn_gemv": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _S, _S, _S]),
    "zq_hip_gemm_batch": (ctypes.c_int, [ctypes.c_int, _P, ctypes.POINTER(GemmTask), _S, _S, _S, ctypes.c_int]),
    "zq_hip_rms_norm": (ctypes.c_int, [_P, _P, _P, _S, _S, ctypes.c_float]),
    "zq_hip_ffn_residual_fused": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _P, _S, _S, _S,
                                                 ctypes.c_float]),
    "zq_hip_gemm_batch_workspace_bytes": (_S, [ctypes.c_int, ctypes.POINTER(GemmTask), _S, _S, _S, ctypes.c_int]),
    "zq_hip_gemm_batch_dev": (ctypes.c_int, [ctypes.c_int, _P, ctypes.POINTER(GemmTask), _S, _S, _S, ctypes.c_int,
                                             _P, _S, _P]),
    "zq_hip_rms_norm_dev": (ctypes.c_int, [_P, _P, _P, _S, _S, ctypes.c_float, _P]),
    "zq_hip_ffn_residual_workspace_bytes": (_S, [_S, _S]),
    "zq_hip_ffn_residual_fused_dev": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _P, _S, _S, _S,
                                                     ctypes.c_float, _P, _S, _P]),
    "zq_hip_release": (ctypes.c_int, [_P]),
    "zq_hip_release_all": (ctypes.c_int, []),
    "zq_hip_gemv_dev": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _S, _S, _P]),
    "zq_hip_gemv_batch_dev": (ctypes.c_int, [ctypes.c_int, _P, ctypes.POINTER(GemvTask), _S, _S, _P]),
    "zq_hip_gemm_workspace_bytes": (_S, [ctypes.c_int, _S, _S, _S, ctypes.c_int]),
    "zq_hip_gemm_dev": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _S, _S, _S, ctypes.c_int, _P, _S, _P]),
    "zq_hip_noalloc_scratch_bytes": (_S, []),
    "zq_hip_gemm_dev_noalloc": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _S, _S, _S, ctypes.c_int, _P]),
    "zq_hip_quantize_acts_dev": (ctypes.c_int, [_P, _P, _P, _S, _S, _P]),
    "zq_hip_block_dots_dev": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _S, _S, _S, _P]),
    "zq_hip_dequantize_dev": (ctypes.c_int, [ctypes.c_int, _P, _P, _S, _S, _P]),
    "zq_hip_mfma_peak": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double)] * 3),
    "zq_hip_read_probe_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]),
    "zq_hip_read_probe_sink_bytes": (ctypes.c_size_t, []),
    "zq_hip_synth_weights_dev": (ctypes.c_int, [ctypes.c_int, ctypes.c_uint64, _P, _S, _S, _P]),
    "zq_hip_synth_normal_dev": (ctypes.c_int, [ctypes.c_uint64, _P, _S, _P]),
}

class GGUFTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 4),
                ("ggml_type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("byte_size", ctypes.c_uint64),
                ("data", _P)]


class GGUFConfig(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("data_offset", ctypes.c_uint64), ("file_size", ctypes.c_uint64)] + [
        (n, ctypes.c_uint32) for n in ("embedding_length", "block_count", "head_count", "head_count_kv",
                                       "feed_forward_length", "context_length", "vocabulary_size", "bos_token_id",
                                       "eos_token_id")] + [("architecture", ctypes.c_char * 64), ("name", ctypes.c_char * 128)]


# Every symbol include/zq_gguf.h declares.
GGUF_SIGNATURES = {
    "zq_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_P), ctypes.c_char_p, _S]),
    "zq_gguf_open_bytes": (ctypes.c_int, [_P, _S, ctypes.c_int, ctypes.POINTER(_P), ctypes.c_char_p, _S]),
    "zq_gguf_close": (None, [_P]),
    "zq_gguf_get_config": (ctypes.c_int, [_P, ctypes.POINTER(GGUFConfig)]),
    "zq_gguf_tensor_count": (_S, [_P]),
    "zq_gguf_get_tensor": (ctypes.c_int, [_P, _S, ctypes.POINTER(GGUFTensor)]),
    "zq_gguf_find_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(GGUFTensor)]),
    "zq_gguf_meta_count": (_S, [_P]),
    "zq_gguf_meta_key": (ctypes.c_char_p, [_P, _S]),
    "zq_gguf_meta_value": (ctypes.c_char_p, [_P, ctypes.c_char_p]),
}

class ModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("embedding", "layers", "heads", "kv_heads", "head_dim", "ffn", "vocab",
                                               "context", "max_positions", "rope_dim")] + [
        ("rope_base", ctypes.c_float), ("rms_epsilon", ctypes.c_float), ("eos_token", ctypes.c_uint32),
        ("weight_format", ctypes.c_int)]


class TapRecord(ctypes.Structure):
    """zq_model_tap_record (include/zq_model.h)."""
    _fields_ = [("proj", ctypes.c_int), ("fmt", ctypes.c_int), ("w", ctypes.c_void_p), ("m", ctypes.c_uint32),
                ("n", ctypes.c_uint32), ("k", ctypes.c_uint32), ("splits", ctypes.c_uint32),
                ("xq_off", ctypes.c_uint64), ("xs_off", ctypes.c_uint64), ("y_off", ctypes.c_uint64)]


# Every symbol include/zq_model.h declares.
MODEL_SIGNATURES = {
    "zq_model_load_gguf": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.POINTER(ModelConfig), ctypes.POINTER(_P),
                                          ctypes.c_char_p, _S]),
    "zq_model_create_synthetic": (ctypes.c_int, [ctypes.POINTER(ModelConfig), ctypes.c_uint64, ctypes.POINTER(_P),
                                                 ctypes.c_char_p, _S]),
    "zq_model_free": (None, [_P]),
    "zq_model_weight": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.c_int, ctypes.POINTER(_P),
                                       ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                                       ctypes.POINTER(ctypes.c_int)]),
    "zq_model_set_prefill_mode": (ctypes.c_int, [_P, ctypes.c_int]),
    "zq_model_prefill": (ctypes.c_int, [_P, _P, _S, _P, ctypes.POINTER(ctypes.c_uint32)]),
    "zq_model_decode": (ctypes.c_int, [_P, ctypes.c_uint32, _P, ctypes.POINTER(ctypes.c_uint32)]),
    "zq_model_generate": (ctypes.c_int, [_P, _P, _S, ctypes.c_uint32, _P, ctypes.POINTER(_S),
                                         ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "zq_model_memory": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                                       ctypes.POINTER(ctypes.c_uint64)]),
    "zq_model_set_tap": (ctypes.c_int, [_P, ctypes.c_uint32, _P, _S]),
    "zq_model_tap_records": (ctypes.c_int, [_P, ctypes.POINTER(TapRecord), _S, ctypes.POINTER(_S)]),
}

_lib = None


def lib():
    """The loaded libzq_hip.so; raises when it has not been built."""
    global _lib
    if _lib is None:
        path = os.environ.get("ZQ_HIP_LIB", LIB)  # alternate build of the same library (A/B runs)
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `python -m zeninfer_amd.build` "
                               "(there is no CPU fallback for this path)")
        L = ctypes.CDLL(path)
        for name, (res, args) in {**SIGNATURES, **GGUF_SIGNATURES, **MODEL_SIGNATURES}.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def status_string(status):
    try:
        return lib().zq_hip_status_string(status).decode()
    except Exception:  # pragma: no cover - only while the library is missing
        return "?"


def check(status, what):
    if status != OK:
        raise ZQError(status, what)
    return status


def _np_ptr(a):
    return a.ctypes.data_as(_P)


def _dptr(t):
    """Device pointer of a torch tensor or a raw integer address."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _device_index():
    """Device the library runs on: ZEN_HIP_DEVICE, default 0 (as zq_hip_init)."""
    try:
        return int(os.environ.get("ZEN_HIP_DEVICE", "0"))
    except ValueError:
        return 0


def _check_device(t, what):
    if not getattr(t, "is_cuda", False):
        raise ValueError(f"{what}: tensor must be on the GPU, got device {getattr(t, 'device', '?')}")
    if t.device.index is not None and t.device.index != _device_index():
        raise ValueError(f"{what}: tensor is on {t.device}, the library runs on cuda:{_device_index()}")


def _need(t, nbytes, what):
    """A torch tensor passed as a device buffer must live on the library's GPU,
    be contiguous and hold at least nbytes: the kernels index it from the sizes
    alone, so a short buffer would be read or written past its end, and the
    address of a host tensor handed to a kernel faults the GPU.  Raw addresses
    are the caller's responsibility."""
    if t is None or isinstance(t, int):
        return
    _check_device(t, what)
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    have = t.numel() * t.element_size()
    if have < nbytes:
        raise ValueError(f"{what}: buffer holds {have} bytes, the call needs {nbytes}")


def _stream(stream):
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


# ---- lifecycle -------------------------------------------------------------
def init():
    return lib().zq_hip_init()


def info():
    i = Info()
    check(lib().zq_hip_get_info(ctypes.byref(i)), "zq_hip_get_info")
    return {f: (getattr(i, f).decode() if isinstance(getattr(i, f), bytes) else getattr(i, f)) for f, _ in Info._fields_}


def stats():
    s = Stats()
    check(lib().zq_hip_get_stats(ctypes.byref(s)), "zq_hip_get_stats")
    return {f: getattr(s, f) for f, _ in Stats._fields_}


def reset_stats():
    lib().zq_hip_reset_stats()


def shutdown():
    lib().zq_hip_shutdown()


def row_bytes(fmt, cols):
    return lib().zq_row_bytes(fmt, cols)


def weight_bytes(fmt, rows, cols):
    return lib().zq_weight_bytes(fmt, rows, cols)


def set_min_elements(n):
    return lib().zq_hip_set_min_elements(n)


# ---- host-pointer API (numpy) ---------------------------------------------
def _host(a, nbytes, what):
    """A host array handed to the library by address must be a C-contiguous
    numpy array of at least nbytes: the library reads nbytes from its first
    byte, so a strided view would give it other bytes and a short array bytes
    past its end.  Weights are not copied to make them so: residency is keyed
    by their address."""
    if not isinstance(a, np.ndarray) or not a.flags["C_CONTIGUOUS"]:
        raise ValueError(f"{what}: must be a C-contiguous numpy array")
    if a.nbytes < nbytes:
        raise ValueError(f"{what}: array holds {a.nbytes} bytes, the call needs {nbytes}")
    return a


def _host_w(fmt, w, rows, cols, what):
    return _host(w, rows * row_bytes(fmt, cols), what)


def _host_f32(a, n, what):
    return _host(np.ascontiguousarray(a, dtype=np.float32), 4 * n, what)


def _same_len(ws, rows, what):
    if len(ws) != len(rows):
        raise ValueError(f"{what}: {len(ws)} weight arrays but {len(rows)} row counts")


def gemv(fmt, w, x, rows, cols):
    _host_w(fmt, w, rows, cols, "gemv weights")
    x = _host_f32(x, cols, "gemv x")
    y = np.empty(rows, np.float32)
    check(lib().zq_hip_gemv(fmt, _np_ptr(w), _np_ptr(x), _np_ptr(y), rows, cols), "zq_hip_gemv")
    return y


def gemv_batch(fmt, ws, x, rows, cols):
    _same_len(ws, rows, "gemv_batch")
    for w, r in zip(ws, rows):
        _host_w(fmt, w, r, cols, "gemv_batch weights")
    x = _host_f32(x, cols, "gemv_batch x")
    ys = [np.empty(r, np.float32) for r in rows]
    tasks = (GemvTask * len(ws))(*[GemvTask(w.ctypes.data, y.ctypes.data, r) for w, y, r in zip(ws, ys, rows)])
    check(lib().zq_hip_gemv_batch(fmt, _np_ptr(x), tasks, len(ws), cols), "zq_hip_gemv_batch")
    return ys


def gemm(fmt, w, X, tokens, rows, cols, act=ACT_DEFAULT):
    _host_w(fmt, w, rows, cols, "gemm weights")
    X = _host_f32(X, tokens * cols, "gemm X")
    Y = np.empty(tokens * rows, np.float32)
    check(lib().zq_hip_gemm(fmt, _np_ptr(w), _np_ptr(X), _np_ptr(Y), tokens, rows, cols, act), "zq_hip_gemm")
    return Y


def ffn_gemv(fmt, gate, up, down, x, ffn_rows, cols, out_rows):
    _host_w(fmt, gate, ffn_rows, cols, "ffn_gemv gate")
    _host_w(fmt, up, ffn_rows, cols, "ffn_gemv up")
    _host_w(fmt, down, out_rows, ffn_rows, "ffn_gemv down")
    x = _host_f32(x, cols, "ffn_gemv x")
    y = np.empty(out_rows, np.float32)
    check(lib().zq_hip_ffn_gemv(fmt, _np_ptr(gate), _np_ptr(up), _np_ptr(down), _np_ptr(x), _np_ptr(y),
                                ffn_rows, cols, out_rows), "zq_hip_ffn_gemv")
    return y


def gemm_batch(fmt, ws, X, tokens, rows, cols, act=ACT_DEFAULT):
    """Y_i = X . W_i^T for every weight of ws (shared X), one submission."""
    _same_len(ws, rows, "gemm_batch")
    for w, r in zip(ws, rows):
        _host_w(fmt, w, r, cols, "gemm_batch weights")
    X = _host_f32(X, tokens * cols, "gemm_batch X")
    Ys = [np.empty(tokens * r, np.float32) for r in rows]
    tasks = (GemmTask * len(ws))(*[GemmTask(w.ctypes.data, Y.ctypes.data, r) for w, Y, r in zip(ws, Ys, rows)])
    check(lib().zq_hip_gemm_batch(fmt, _np_ptr(X), tasks, len(ws), tokens, cols, act), "zq_hip_gemm_batch")
    return Ys


def rms_norm(x, w, rows, cols, eps):
    x = _host_f32(x, rows * cols, "rms_norm x")
    w = _host_f32(w, cols, "rms_norm weight")
    y = np.empty(rows * cols, np.float32)
    check(lib().zq_hip_rms_norm(_np_ptr(x), _np_ptr(w), _np_ptr(y), rows, cols, eps), "zq_hip_rms_norm")
    return y


def ffn_residual_fused(fmt, wo, wg, wu, wd, norm_w, x, attn_out, hidden, attn_width, ffn_rows, eps):
    _host_w(fmt, wo, hidden, attn_width, "ffn_residual_fused attn_output")
    _host_w(fmt, wg, ffn_rows, hidden, "ffn_residual_fused gate")
    _host_w(fmt, wu, ffn_rows, hidden, "ffn_residual_fused up")
    _host_w(fmt, wd, hidden, ffn_rows, "ffn_residual_fused down")
    x = _host_f32(x, hidden, "ffn_residual_fused x")
    a = _host_f32(attn_out, attn_width, "ffn_residual_fused attn_out")
    nw = _host_f32(norm_w, hidden, "ffn_residual_fused norm_weight")
    out = np.empty(hidden, np.float32)
    check(lib().zq_hip_ffn_residual_fused(fmt, _np_ptr(wo), _np_ptr(wg), _np_ptr(wu), _np_ptr(wd), _np_ptr(nw),
                                          _np_ptr(x), _np_ptr(a), _np_ptr(out), hidden, attn_width, ffn_rows, eps),
          "zq_hip_ffn_residual_fused")
    return out


def release(w):
    return lib().zq_hip_release(_np_ptr(w))


def release_all():
    return lib().zq_hip_release_all()


# ---- device-pointer API (torch tensors or raw addresses) ------------------
def gemv_dev(fmt, w, x, y, rows, cols, stream=None):
    _need(w, weight_bytes(fmt, rows, cols), "gemv_dev weights")
    _need(x, 4 * cols, "gemv_dev x")
    _need(y, 4 * rows, "gemv_dev y")
    return check(lib().zq_hip_gemv_dev(fmt, _dptr(w), _dptr(x), _dptr(y), rows, cols, _stream(stream)),
                 "zq_hip_gemv_dev")


def gemv_batch_dev(fmt, x, tasks, cols, stream=None):
    """tasks: list of (weights, y, rows)."""
    _need(x, 4 * cols, "gemv_batch_dev x")
    for w, y, r in tasks:
        _need(w, weight_bytes(fmt, r, cols), "gemv_batch_dev weights")
        _need(y, 4 * r, "gemv_batch_dev y")
    arr = (GemvTask * len(tasks))(*[GemvTask(_dptr(w), _dptr(y), r) for w, y, r in tasks])
    return check(lib().zq_hip_gemv_batch_dev(fmt, _dptr(x), arr, len(tasks), cols, _stream(stream)),
                 "zq_hip_gemv_batch_dev")


def gemm_workspace_bytes(fmt, tokens, rows, cols, act=ACT_DEFAULT):
    return lib().zq_hip_gemm_workspace_bytes(fmt, tokens, rows, cols, act)


def gemm_dev(fmt, w, X, Y, tokens, rows, cols, act=ACT_DEFAULT, workspace=None, workspace_bytes=0, stream=None):
    _need(w, weight_bytes(fmt, rows, cols), "gemm_dev weights")
    _need(X, 4 * tokens * cols, "gemm_dev X")
    _need(Y, 4 * tokens * rows, "gemm_dev Y")
    _need(workspace, workspace_bytes, "gemm_dev workspace")
    return check(lib().zq_hip_gemm_dev(fmt, _dptr(w), _dptr(X), _dptr(Y), tokens, rows, cols, act,
                                       _dptr(workspace), workspace_bytes, _stream(stream)), "zq_hip_gemm_dev")


def _gemm_tasks(tasks):
    return (GemmTask * len(tasks))(*[GemmTask(_dptr(w), _dptr(Y), r) for w, Y, r in tasks])


def gemm_batch_workspace_bytes(fmt, rows, tokens, cols, act=ACT_DEFAULT):
    arr = (GemmTask * len(rows))(*[GemmTask(None, None, r) for r in rows])
    return lib().zq_hip_gemm_batch_workspace_bytes(fmt, arr, len(rows), tokens, cols, act)


def gemm_batch_dev(fmt, X, tasks, tokens, cols, act=ACT_DEFAULT, workspace=None, workspace_bytes=0, stream=None):
    """tasks: list of (weights, Y, rows)."""
    _need(X, 4 * tokens * cols, "gemm_batch_dev X")
    for w, Y, r in tasks:
        _need(w, weight_bytes(fmt, r, cols), "gemm_batch_dev weights")
        _need(Y, 4 * tokens * r, "gemm_batch_dev Y")
    _need(workspace, workspace_bytes, "gemm_batch_dev workspace")
    return check(lib().zq_hip_gemm_batch_dev(fmt, _dptr(X), _gemm_tasks(tasks), len(tasks), tokens, cols, act,
                                             _dptr(workspace), workspace_bytes, _stream(stream)),
                 "zq_hip_gemm_batch_dev")


def rms_norm_dev(x, w, y, rows, cols, eps, stream=None):
    _need(x, 4 * rows * cols, "rms_norm_dev x")
    _need(w, 4 * cols, "rms_norm_dev weight")
    _need(y, 4 * rows * cols, "rms_norm_dev y")
    return check(lib().zq_hip_rms_norm_dev(_dptr(x), _dptr(w), _dptr(y), rows, cols, eps, _stream(stream)),
                 "zq_hip_rms_norm_dev")


def ffn_residual_workspace_bytes(hidden, ffn_rows):
    return lib().zq_hip_ffn_residual_workspace_bytes(hidden, ffn_rows)


def ffn_residual_fused_dev(fmt, wo, wg, wu, wd, norm_w, x, attn_out, out, hidden, attn_width, ffn_rows, eps,
                           workspace, workspace_bytes, stream=None):
    _need(wo, weight_bytes(fmt, hidden, attn_width), "ffn_residual_fused_dev attn_output")
    for w, what in ((wg, "gate"), (wu, "up")):
        _need(w, weight_bytes(fmt, ffn_rows, hidden), f"ffn_residual_fused_dev {what}")
    _need(wd, weight_bytes(fmt, hidden, ffn_rows), "ffn_residual_fused_dev down")
    _need(norm_w, 4 * hidden, "ffn_residual_fused_dev norm_weight")
    _need(x, 4 * hidden, "ffn_residual_fused_dev x")
    _need(attn_out, 4 * attn_width, "ffn_residual_fused_dev attn_out")
    _need(out, 4 * hidden, "ffn_residual_fused_dev out")
    _need(workspace, workspace_bytes, "ffn_residual_fused_dev workspace")
    return check(lib().zq_hip_ffn_residual_fused_dev(fmt, _dptr(wo), _dptr(wg), _dptr(wu), _dptr(wd), _dptr(norm_w),
                                                     _dptr(x), _dptr(attn_out), _dptr(out), hidden, attn_width,
                                                     ffn_rows, eps, _dptr(workspace), workspace_bytes,
                                                     _stream(stream)), "zq_hip_ffn_residual_fused_dev")


def noalloc_scratch_bytes():
    return lib().zq_hip_noalloc_scratch_bytes()


def gemm_dev_noalloc(fmt, w, X, Y, tokens, rows, cols, act=ACT_DEFAULT, stream=None):
    """zq_hip_gemm_dev with the library's fixed device scratch: no workspace,
    no allocation (ERR_TOO_LARGE beyond noalloc_scratch_bytes())."""
    _need(w, weight_bytes(fmt, rows, cols), "gemm_dev_noalloc weights")
    _need(X, 4 * tokens * cols, "gemm_dev_noalloc X")
    _need(Y, 4 * tokens * rows, "gemm_dev_noalloc Y")
    return check(lib().zq_hip_gemm_dev_noalloc(fmt, _dptr(w), _dptr(X), _dptr(Y), tokens, rows, cols, act,
                                               _stream(stream)), "zq_hip_gemm_dev_noalloc")


def quantize_acts_dev(X, xq, xs, tokens, cols, stream=None):
    _need(X, 4 * tokens * cols, "quantize_acts_dev X")
    _need(xq, tokens * cols, "quantize_acts_dev xq")
    _need(xs, 4 * tokens * (cols // 32), "quantize_acts_dev xs")
    return check(lib().zq_hip_quantize_acts_dev(_dptr(X), _dptr(xq), _dptr(xs), tokens, cols, _stream(stream)),
                 "zq_hip_quantize_acts_dev")


def block_dots_dev(fmt, w, xq, out, tokens, rows, cols, stream=None):
    _need(w, weight_bytes(fmt, rows, cols), "block_dots_dev weights")
    _need(xq, tokens * cols, "block_dots_dev xq")
    _need(out, 4 * tokens * rows * (cols // 32), "block_dots_dev out")
    return check(lib().zq_hip_block_dots_dev(fmt, _dptr(w), _dptr(xq), _dptr(out), tokens, rows, cols,
                                             _stream(stream)), "zq_hip_block_dots_dev")


def dequantize_dev(fmt, w, out, rows, cols, stream=None):
    _need(w, weight_bytes(fmt, rows, cols), "dequantize_dev weights")
    _need(out, 4 * rows * cols, "dequantize_dev out")
    return check(lib().zq_hip_dequantize_dev(fmt, _dptr(w), _dptr(out), rows, cols, _stream(stream)),
                 "zq_hip_dequantize_dev")


def mfma_peak():
    """(sclk MHz, cycles per int8 MFMA, int8 TOPS peak) measured on the device."""
    a, b, c = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    check(lib().zq_hip_mfma_peak(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)), "zq_hip_mfma_peak")
    return a.value, b.value, c.value


def read_probe_sink_bytes():
    return lib().zq_hip_read_probe_sink_bytes()


def read_probe_dev(buf, nbytes, sink, stream=None):
    """Enqueue one streaming read of nbytes of device memory (the GEMV roofline's yardstick)."""
    _need(buf, nbytes, "read_probe_dev buffer")
    _need(sink, read_probe_sink_bytes(), "read_probe_dev sink")
    return check(lib().zq_hip_read_probe_dev(_dptr(buf), nbytes, _dptr(sink), _stream(stream)), "zq_hip_read_probe_dev")


def synth_weights_dev(fmt, seed, w, rows, cols, stream=None):
    _need(w, weight_bytes(fmt, rows, cols), "synth_weights_dev weights")
    return check(lib().zq_hip_synth_weights_dev(fmt, seed, _dptr(w), rows, cols, _stream(stream)),
                 "zq_hip_synth_weights_dev")


def synth_normal_dev(seed, out, n, stream=None):
    _need(out, 4 * n, "synth_normal_dev out")
    return check(lib().zq_hip_synth_normal_dev(seed, _dptr(out), n, _stream(stream)), "zq_hip_synth_normal_dev")
