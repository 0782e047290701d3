"""CPU tier: the C-ABI library loads and exports every symbol include/zq_hip.h
declares (no compute calls without a GPU), and host-side argument checks
answer without touching a device."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zq_hip.h")
GGUF_HEADER = os.path.join(ROOT, "include", "zq_gguf.h")
MODEL_HEADER = os.path.join(ROOT, "include", "zq_model.h")


def declared_symbols(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    for s in ("zq_hip_gemv", "zq_hip_gemm", "zq_hip_gemv_batch", "zq_hip_init", "zq_hip_release",
              "zq_hip_gemv_dev", "zq_hip_gemm_dev", "zq_hip_block_dots_dev", "zq_hip_dequantize_dev"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from zeninfer_amd import zq
    lib = zq.lib()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(declared_symbols()) == set(zq.SIGNATURES), "Python binding out of sync with the header"
    gguf = declared_symbols(GGUF_HEADER)
    missing = [s for s in gguf if not hasattr(lib, s)]
    assert not missing, missing
    assert set(gguf) == set(zq.GGUF_SIGNATURES), "Python binding out of sync with include/zq_gguf.h"
    model = declared_symbols(MODEL_HEADER)
    missing = [s for s in model if not hasattr(lib, s)]
    assert not missing, missing
    assert set(model) == set(zq.MODEL_SIGNATURES), "Python binding out of sync with include/zq_model.h"


def test_layout_helpers_without_device():
    from zeninfer_amd import zq
    assert zq.row_bytes(zq.Q8_0, 4096) == 4352
    assert zq.row_bytes(zq.Q8_0, 14336) == 15232
    assert zq.row_bytes(zq.Q4_0, 4096) == 2304
    assert zq.row_bytes(zq.Q6_K, 4096) == 3360
    assert zq.row_bytes(zq.Q6_K, 4000) == 0 and zq.row_bytes(zq.Q8_0, 100) == 0 and zq.row_bytes(99, 4096) == 0
    assert zq.weight_bytes(zq.Q8_0, 2, 64) == 2 * 68 + zq.WEIGHT_TAIL_PAD


def test_argument_errors_without_device():
    from zeninfer_amd import zq
    L = zq.lib()
    # null pointers / bad shapes are rejected before any device work
    assert L.zq_hip_gemv(zq.Q8_0, None, None, None, 4, 64) == -1
    assert L.zq_hip_gemm(zq.Q8_0, None, None, None, 1, 4, 64, 0) == -1
    assert L.zq_hip_gemv_dev(zq.Q8_0, 0, 0, 0, 4, 100, None) == -1
    assert zq.status_string(1) == "declined"
    # int8 activations + scales (256-byte aligned sections) + split-K partials for small grids
    ws = L.zq_hip_gemm_workspace_bytes(zq.Q8_0, 4, 4096, 4096, zq.ACT_INT8)
    assert ws >= 4 * 4096 + 4 * 128 * 4 and ws % 4 == 0
    assert L.zq_hip_gemm_workspace_bytes(zq.Q8_0, 2048, 14336, 4096, zq.ACT_INT8) == 2048 * 4096 + 2048 * 128 * 4
    # fp32 activations: split-K partial sums (whole fp32 [M][N] planes) for small grids only
    ws = L.zq_hip_gemm_workspace_bytes(zq.Q8_0, 4, 4096, 4096, zq.ACT_F32)
    assert ws > 0 and ws % (4 * 4096 * 4) == 0
    assert L.zq_hip_gemm_workspace_bytes(zq.Q8_0, 2048, 14336, 4096, zq.ACT_F32) == 0
    # the default activation mode is fp32 for Q8_0 / Q4_0 too (int8 is opt-in)
    for fmt in (zq.Q8_0, zq.Q4_0):
        for m in (4, 2048):
            assert (L.zq_hip_gemm_workspace_bytes(fmt, m, 4096, 4096, zq.ACT_DEFAULT)
                    == L.zq_hip_gemm_workspace_bytes(fmt, m, 4096, 4096, zq.ACT_F32))
    # Q6_K also holds its split activations: f16 hi + lo [M][K] and the row
    # scales, 256-byte aligned, ahead of the partial sums
    split = lambda m, k: (m * k * 4 + m * 4 + 255) // 256 * 256
    ws = L.zq_hip_gemm_workspace_bytes(zq.Q6_K, 4, 4096, 4096, zq.ACT_DEFAULT)
    assert ws > split(4, 4096) and (ws - split(4, 4096)) % (4 * 4096 * 4) == 0
    assert L.zq_hip_gemm_workspace_bytes(zq.Q6_K, 2048, 14336, 4096, zq.ACT_DEFAULT) == split(2048, 4096)
    for fmt in (zq.Q4_K, zq.Q5_K):  # the same split activations as Q6_K
        ws = L.zq_hip_gemm_workspace_bytes(fmt, 4, 4096, 4096, zq.ACT_DEFAULT)
        assert ws > split(4, 4096) and (ws - split(4, 4096)) % (4 * 4096 * 4) == 0
        assert L.zq_hip_gemm_workspace_bytes(fmt, 2048, 14336, 4096, zq.ACT_DEFAULT) == split(2048, 4096)


def test_opt_in_semantics(monkeypatch):
    # ZEN_BACKEND=hip|rocm|amd or ZEN_HIP=1 (src/backends/hip/hip_backend.hip:266-282)
    from zeninfer_amd import zq
    L = zq.lib()
    for k in ("ZEN_BACKEND", "ZEN_HIP"):
        monkeypatch.delenv(k, raising=False)
    assert L.zq_hip_opted_in() == 0
    for v in ("hip", "rocm", "amd"):
        monkeypatch.setenv("ZEN_BACKEND", v)
        assert L.zq_hip_opted_in() == 1
    monkeypatch.setenv("ZEN_BACKEND", "cpu")
    assert L.zq_hip_opted_in() == 0
    monkeypatch.setenv("ZEN_HIP", "1")
    assert L.zq_hip_opted_in() == 1


def test_device_wrappers_reject_host_tensors():
    """A host tensor handed to a device entry point is refused before any
    library call: its address would reach a kernel and fault the GPU."""
    import torch
    from zeninfer_amd import zq
    wb = zq.weight_bytes(zq.Q8_0, 64, 256)
    with pytest.raises(ValueError, match="gemv_dev weights: tensor must be on the GPU"):
        zq.gemv_dev(zq.Q8_0, torch.empty(wb, dtype=torch.uint8), torch.empty(256), torch.empty(64), 64, 256)
    with pytest.raises(ValueError, match="synth_normal_dev out: tensor must be on the GPU"):
        zq.synth_normal_dev(1, torch.empty(64), 64)
    with pytest.raises(ValueError, match="gemm_dev workspace: tensor must be on the GPU"):
        zq.gemm_dev(zq.Q8_0, 1 << 20, 2 << 20, 3 << 20, 3, 64, 256, zq.ACT_INT8, torch.empty(16), 64)


def test_device_wrappers_reject_short_buffers(monkeypatch):
    """The Python device-pointer wrappers refuse a tensor shorter than the
    call's sizes (the kernels would run past its end) before any library call.
    Host tensors stand in for device ones here (the device check is bypassed:
    no GPU on the CPU runner)."""
    import torch
    from zeninfer_amd import zq
    monkeypatch.setattr(zq, "_check_device", lambda t, what: None)
    wb = zq.weight_bytes(zq.Q8_0, 64, 256)
    w = torch.empty(wb, dtype=torch.uint8)
    with pytest.raises(ValueError, match="gemm_dev X"):
        zq.gemm_dev(zq.Q8_0, w, torch.empty(3 * 256 - 1), torch.empty(3 * 64), 3, 64, 256)
    with pytest.raises(ValueError, match="gemm_dev weights"):
        zq.gemm_dev(zq.Q8_0, w[:-1], torch.empty(3 * 256), torch.empty(3 * 64), 3, 64, 256)
    with pytest.raises(ValueError, match="gemv_dev y"):
        zq.gemv_dev(zq.Q8_0, w, torch.empty(256), torch.empty(63), 64, 256)
    with pytest.raises(ValueError, match="gemv_batch_dev weights"):
        zq.gemv_batch_dev(zq.Q8_0, torch.empty(256), [(w, torch.empty(64), 64), (w, torch.empty(65), 65)], 256)
    with pytest.raises(ValueError, match="quantize_acts_dev xs"):
        zq.quantize_acts_dev(torch.empty(2 * 256), torch.empty(512, dtype=torch.int8), torch.empty(15), 2, 256)
    with pytest.raises(ValueError, match="contiguous"):
        zq.synth_normal_dev(1, torch.empty(8, 8).t(), 64)


def test_host_wrappers_reject_strided_or_short_arrays():
    """The host-pointer wrappers refuse, before any library call, a weight
    array that is a strided view or shorter than rows x row_bytes, a short
    activation array, and mismatched batch lists: the library reads the
    bytes from the array's address."""
    from zeninfer_amd import zq
    rows, cols = 64, 256
    wb = rows * zq.row_bytes(zq.Q8_0, cols)
    w = np.zeros(wb, np.uint8)
    x = np.zeros(cols, np.float32)
    with pytest.raises(ValueError, match="gemv weights: must be a C-contiguous"):
        zq.gemv(zq.Q8_0, np.zeros(2 * wb, np.uint8)[::2], x, rows, cols)
    with pytest.raises(ValueError, match="gemv weights: array holds"):
        zq.gemv(zq.Q8_0, w[:-1], x, rows, cols)
    with pytest.raises(ValueError, match="gemv x"):
        zq.gemv(zq.Q8_0, w, x[:-1], rows, cols)
    with pytest.raises(ValueError, match="gemm X"):
        zq.gemm(zq.Q8_0, w, np.zeros(3 * cols - 1, np.float32), 3, rows, cols)
    with pytest.raises(ValueError, match="gemv_batch: 2 weight arrays but 1 row counts"):
        zq.gemv_batch(zq.Q8_0, [w, w], x, [rows], cols)
    with pytest.raises(ValueError, match="ffn_gemv down"):
        zq.ffn_gemv(zq.Q8_0, w, w, w[: 10], x, rows, cols, cols)
    with pytest.raises(ValueError, match="rms_norm weight"):
        zq.rms_norm(np.zeros(2 * cols, np.float32), np.zeros(cols - 1, np.float32), 2, cols, 1e-5)
