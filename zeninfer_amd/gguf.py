"""GGUF v3 writer and synthetic Llama-layout model builder.

The file layout follows the GGUF v2/v3 format the reference parses
(src/gguf.cpp:113-236 of the reference): magic, version u32, tensor count u64,
metadata count u64, metadata key/type/value records, tensor directory records
(name, ndim u32, dims u64[ndim] with dims[0] the contiguous axis, ggml type
u32, payload offset u64), then the payload section aligned to
``general.alignment`` (default 32), every tensor payload aligned too.

``synthetic_llama`` writes the Llama tensor set the reference's dense runtime
loads (token_embd, per-layer attn_norm / attn_q / attn_k / attn_v /
attn_output / ffn_norm / ffn_gate / ffn_up / ffn_down, output_norm, output),
as the reference's own synthetic writers do (tests/make_qwen2_synthetic.py:13-70),
with Q8_0 projections quantised from seeded uniform weights and F32 norms.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

# metadata value types (src/gguf.cpp:21 of the reference)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
# ggml tensor types used here
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 0, 1, 2, 8, 12, 13, 14

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}


def _string(s: str | bytes) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _string(v)
    if t == ARRAY:
        sub, items = v
        return struct.pack("<IQ", sub, len(items)) + b"".join(_value(sub, x) for x in items)
    return struct.pack(_SCALAR[t], v)


@dataclass
class GGUFWriter:
    """Collects metadata and tensors, then writes one GGUF v3 file."""

    alignment: int = 32
    metadata: list = field(default_factory=list)
    tensors: list = field(default_factory=list)

    def add_meta(self, key: str, t: int, value) -> None:
        self.metadata.append((key, t, value))

    def add_tensor(self, name: str, dims, ggml_type: int, payload: bytes) -> None:
        self.tensors.append((name, [int(d) for d in dims], int(ggml_type), bytes(payload)))

    def to_bytes(self) -> bytes:
        a = self.alignment
        meta = list(self.metadata)
        if a != 32 and not any(k == "general.alignment" for k, _, _ in meta):
            meta.append(("general.alignment", U32, a))
        out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(meta)))
        for key, t, v in meta:
            out += _string(key) + struct.pack("<I", t) + _value(t, v)
        offsets, off = [], 0
        for _, _, _, data in self.tensors:
            off = (off + a - 1) // a * a
            offsets.append(off)
            off += len(data)
        for (name, dims, t, _), o in zip(self.tensors, offsets):
            out += _string(name) + struct.pack("<I", len(dims)) + struct.pack("<" + "Q" * len(dims), *dims)
            out += struct.pack("<IQ", t, o)
        out += bytes((-len(out)) % a)
        start = len(out)
        for (_, _, _, data), o in zip(self.tensors, offsets):
            out += bytes(start + o - len(out))
            out += data
        return bytes(out)

    def write(self, path) -> int:
        data = self.to_bytes()
        with open(path, "wb") as f:
            f.write(data)
        return len(data)


def quantize_q8_0(w: np.ndarray) -> bytes:
    """GGML Q8_0 blocks of a row-major fp32 matrix (rows x cols, cols % 32 == 0):
    d = amax/127 stored as fp16, q = round(x/d) (ggml quantize_row_q8_0_ref)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.shape[-1] % 32:
        raise ValueError("Q8_0 rows must be a multiple of 32 elements")
    b = w.reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    d = amax / 127.0
    inv = np.divide(1.0, d, out=np.zeros_like(d), where=d != 0)
    q = np.clip(np.rint(b * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((b.shape[0], 34), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.tobytes()


def quantize_q4_0(w: np.ndarray) -> bytes:
    """Row-major fp32 [rows, cols] (cols % 32 == 0) to GGML Q4_0 blocks: fp16
    d = max|v| / 8 with the sign of the extreme value (so it maps to -8),
    nibble = clamp(round(v/d) + 8, 0, 15); byte j holds elements j (low
    nibble) and j+16 (high nibble) (src/quant.cpp:391-397)."""
    b = w.reshape(-1, 32).astype(np.float32)
    idx = np.abs(b).argmax(axis=1)
    ext = b[np.arange(b.shape[0]), idx]
    d = (ext / -8.0).astype(np.float16)
    d32 = d.astype(np.float32)
    inv = np.where(d32 != 0, 1.0 / np.where(d32 != 0, d32, 1), 0.0)
    n = np.clip(np.rint(b * inv[:, None]) + 8, 0, 15).astype(np.uint8)
    out = np.empty((b.shape[0], 18), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = n[:, :16] | (n[:, 16:] << 4)
    return out.tobytes()


def quantize_q6_k(w: np.ndarray) -> bytes:
    """Row-major fp32 [rows, cols] (cols % 256 == 0) to GGML Q6_K super-blocks:
    per 16 elements an int8 scale, per super-block fp16 d, element =
    d*sc*(q-32) with q in 0..63 (src/quant.cpp:500-517 read in reverse)."""
    g = w.reshape(-1, 16, 16).astype(np.float32)             # [sb, sub-block, 16]
    amax = np.abs(g).max(axis=2)
    sub = amax / 31.0                                        # per sub-block step
    d = (sub.max(axis=1) / 127.0).astype(np.float16)
    d32 = d.astype(np.float32)
    sc = np.clip(np.rint(sub / np.where(d32 > 0, d32, 1)[:, None]), 1, 127).astype(np.int32)
    step = d32[:, None] * sc.astype(np.float32)
    q = np.clip(np.rint(g / np.where(step > 0, step, 1)[:, :, None]) + 32, 0, 63).astype(np.uint32).reshape(-1, 256)
    nsb = q.shape[0]
    out = np.zeros((nsb, 210), np.uint8)
    for half in range(2):
        for l in range(32):
            e = half * 128 + l
            q0, q1, q2, q3 = q[:, e], q[:, e + 32], q[:, e + 64], q[:, e + 96]
            out[:, half * 64 + l] = (q0 & 15) | ((q2 & 15) << 4)
            out[:, half * 64 + 32 + l] = (q1 & 15) | ((q3 & 15) << 4)
            out[:, 128 + half * 32 + l] = (q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return out.tobytes()


def quantize_kquant(w: np.ndarray, q5: bool = False) -> bytes:
    """Row-major fp32 [rows, cols] (cols % 256 == 0) to GGML Q4_K / Q5_K
    super-blocks: per 32-element group a 6-bit scale and min, per super-block
    fp16 d and dmin, element = d*sc*q - dmin*m with q in 0..15 (0..31).  A
    plain min/max quantiser (no search); the packing is the inverse of the
    reference's k_scale_min (src/quant.cpp:133-141)."""
    qmax = 31 if q5 else 15
    g = w.reshape(-1, 8, 32).astype(np.float32)              # [super-blocks, groups, 32]
    lo = np.minimum(g.min(axis=2), 0.0)                      # the offset is subtracted: min <= 0
    hi = g.max(axis=2)
    scale = np.maximum(hi - lo, 1e-12) / qmax                # per group
    minv = -lo                                               # >= 0
    d = scale.max(axis=1) / 63.0
    dm = minv.max(axis=1) / 63.0
    d16 = d.astype(np.float16)
    dm16 = dm.astype(np.float16)
    d32, dm32 = d16.astype(np.float32), dm16.astype(np.float32)
    sc = np.clip(np.rint(scale / np.where(d32 > 0, d32, 1)[:, None]), 0, 63).astype(np.uint32)
    mn = np.clip(np.rint(minv / np.where(dm32 > 0, dm32, 1)[:, None]), 0, 63).astype(np.uint32)
    eff_s = d32[:, None] * sc.astype(np.float32)
    eff_m = dm32[:, None] * mn.astype(np.float32)
    q = np.rint((g + eff_m[:, :, None]) / np.where(eff_s > 0, eff_s, 1)[:, :, None])
    q = np.clip(q, 0, qmax).astype(np.uint32)                # [sb, group, 32]
    nsb = g.shape[0]
    scales = np.zeros((nsb, 12), np.uint32)
    for j in range(4):
        scales[:, j] = sc[:, j] | ((sc[:, j + 4] >> 4) << 6)
        scales[:, j + 4] = mn[:, j] | ((mn[:, j + 4] >> 4) << 6)
        scales[:, j + 8] = (sc[:, j + 4] & 15) | ((mn[:, j + 4] & 15) << 4)
    qs = np.zeros((nsb, 4, 32), np.uint32)
    for j in range(8):
        qs[:, j // 2] |= (q[:, j] & 15) << (4 * (j % 2))
    out = np.zeros((nsb, 176 if q5 else 144), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dm16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = scales.astype(np.uint8)
    if q5:
        qh = np.zeros((nsb, 32), np.uint32)
        for j in range(8):
            qh |= ((q[:, j] >> 4) & 1) << j
        out[:, 16:48] = qh.astype(np.uint8)
        out[:, 48:] = qs.reshape(nsb, 128).astype(np.uint8)
    else:
        out[:, 16:] = qs.reshape(nsb, 128).astype(np.uint8)
    return out.tobytes()


@dataclass
class LlamaShape:
    embedding: int = 4096
    layers: int = 32
    heads: int = 32
    kv_heads: int = 8
    ffn: int = 14336
    vocab: int = 128256
    context: int = 8192
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    rope_dim: int = 0  # rotated dimensions per head (0: the whole head)


def synthetic_llama(path, shape: LlamaShape, seed: int = 0x5EED0004, weight_scale: float = 0.12,
                    name: str = "synthetic-llama-q8_0", proj_type: int = GGML_Q8_0, down_type: int = None,
                    out_type: int = None) -> int:
    """Write a random-init Llama-layout GGUF: projections of proj_type (Q8_0,
    Q4_0, Q4_K, Q5_K or Q6_K; ffn_down and output may differ, as in
    llama.cpp's mixed files), a Q8_0 token embedding and F32 norms.  Returns
    the file size in bytes."""
    s = shape
    rng = np.random.default_rng(seed)
    hd = s.embedding // s.heads
    w = GGUFWriter()
    tokens = ["<unk>", "<s>", "</s>"] + [f"<t{i}>" for i in range(3, s.vocab)]
    for key, t, v in [
        ("general.architecture", STRING, "llama"), ("general.name", STRING, name),
        ("llama.embedding_length", U32, s.embedding), ("llama.block_count", U32, s.layers),
        ("llama.attention.head_count", U32, s.heads), ("llama.attention.head_count_kv", U32, s.kv_heads),
        ("llama.feed_forward_length", U32, s.ffn), ("llama.context_length", U32, s.context),
        ("llama.rope.dimension_count", U32, s.rope_dim or hd), ("llama.rope.freq_base", F32, s.rope_theta),
        ("llama.attention.layer_norm_rms_epsilon", F32, s.rms_eps),
        ("tokenizer.ggml.model", STRING, "llama"), ("tokenizer.ggml.tokens", ARRAY, (STRING, tokens)),
        ("tokenizer.ggml.bos_token_id", U32, 1), ("tokenizer.ggml.eos_token_id", U32, 2),
    ]:
        w.add_meta(key, t, v)

    def proj(name, rows, cols, ty=proj_type):
        m = rng.uniform(-weight_scale, weight_scale, size=(rows, cols)).astype(np.float32)
        enc = {GGML_Q8_0: quantize_q8_0, GGML_Q4_0: quantize_q4_0, GGML_Q6_K: quantize_q6_k,
               GGML_Q4_K: lambda a: quantize_kquant(a, False), GGML_Q5_K: lambda a: quantize_kquant(a, True)}[ty]
        w.add_tensor(name, [cols, rows], ty, enc(m))

    def norm(name, n):
        w.add_tensor(name, [n], GGML_F32, rng.uniform(0.85, 1.15, size=n).astype(np.float32).tobytes())

    proj("token_embd.weight", s.vocab, s.embedding, GGML_Q8_0)
    for l in range(s.layers):
        p = f"blk.{l}."
        norm(p + "attn_norm.weight", s.embedding)
        proj(p + "attn_q.weight", s.heads * hd, s.embedding)
        proj(p + "attn_k.weight", s.kv_heads * hd, s.embedding)
        proj(p + "attn_v.weight", s.kv_heads * hd, s.embedding)
        proj(p + "attn_output.weight", s.embedding, s.heads * hd)
        norm(p + "ffn_norm.weight", s.embedding)
        proj(p + "ffn_gate.weight", s.ffn, s.embedding)
        proj(p + "ffn_up.weight", s.ffn, s.embedding)
        proj(p + "ffn_down.weight", s.embedding, s.ffn, down_type or proj_type)
    norm("output_norm.weight", s.embedding)
    proj("output.weight", s.vocab, s.embedding, out_type or proj_type)
    return w.write(path)


class GGUFFile:
    """A parsed GGUF (file mapped, or an in-memory image) through include/zq_gguf.h.

    ``GGUFFile(path)`` / ``GGUFFile(data=bytes)``; raises ``GGUFError`` with the
    parser's message on a malformed input (the reference's gguf::inspect /
    inspect_bytes contract, include/zen/gguf.h:19-26)."""

    def __init__(self, path=None, data=None, q8_1_layout=0):
        import ctypes
        from . import zq
        self._zq = zq
        self._L = zq.lib()
        self._h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        if path is not None:
            st = self._L.zq_gguf_open(str(path).encode(), q8_1_layout, ctypes.byref(self._h), err, 512)
        else:
            self._image = bytes(data) if data is not None else b""
            buf = ctypes.create_string_buffer(self._image, len(self._image)) if self._image else None
            self._buf = buf
            st = self._L.zq_gguf_open_bytes(ctypes.cast(buf, ctypes.c_void_p) if buf else None, len(self._image),
                                            q8_1_layout, ctypes.byref(self._h), err, 512)
        if st != 0:
            self._h = None
            raise GGUFError(err.value.decode(errors="replace"))

    def close(self):
        if self._h:
            self._L.zq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def config(self) -> dict:
        c = self._zq.GGUFConfig()
        self._L.zq_gguf_get_config(self._h, c)
        out = {n: getattr(c, n) for n, _ in c._fields_}
        out["architecture"] = c.architecture.decode(errors="replace")
        out["name"] = c.name.decode(errors="replace")
        return out

    def tensors(self) -> list:
        out = []
        for i in range(self._L.zq_gguf_tensor_count(self._h)):
            t = self._zq.GGUFTensor()
            self._L.zq_gguf_get_tensor(self._h, i, t)
            out.append(self._tinfo(t))
        return out

    def tensor(self, name):
        t = self._zq.GGUFTensor()
        if self._L.zq_gguf_find_tensor(self._h, name.encode(), t) != 0:
            raise KeyError(name)
        return self._tinfo(t)

    def tensor_bytes(self, name) -> bytes:
        import ctypes
        info = self.tensor(name)
        return ctypes.string_at(info["data"], info["byte_size"])

    @staticmethod
    def _tinfo(t):
        return {"name": t.name.decode(errors="replace"), "dims": list(t.dims[:t.n_dims]), "ggml_type": t.ggml_type,
                "offset": t.offset, "byte_size": t.byte_size, "data": t.data}

    def metadata(self) -> dict:
        n = self._L.zq_gguf_meta_count(self._h)
        keys = [self._L.zq_gguf_meta_key(self._h, i) for i in range(n)]
        out = {}
        for k in keys:
            v = self._L.zq_gguf_meta_value(self._h, k)
            out[k.decode(errors="replace")] = v.decode(errors="replace") if v is not None else ""
        return out

    def describe(self) -> str:
        """The same text layout as the reference-side checker's description."""
        c = self.config()
        lines = ["ok=1", "error=", f"version={c['version']}", f"data_offset={c['data_offset']}",
                 f"architecture={c['architecture']}", f"name={c['name']}"]
        for k in ("embedding_length", "block_count"):
            lines.append(f"{k}={c[k]}")
        lines += [f"head_count={c['head_count']}", f"head_count_kv={c['head_count_kv']}",
                  f"feed_forward_length={c['feed_forward_length']}", f"context_length={c['context_length']}",
                  f"vocabulary_size={c['vocabulary_size']}", f"bos={c['bos_token_id']}", f"eos={c['eos_token_id']}"]
        for k, v in self.metadata().items():
            lines.append(f"M {k}={v}")
        for t in self.tensors():
            lines.append(f"T {t['name']} {t['ggml_type']} {t['offset']} {t['byte_size']} " + ",".join(map(str, t["dims"])))
        return "\n".join(lines) + "\n"


class GGUFError(ValueError):
    pass
