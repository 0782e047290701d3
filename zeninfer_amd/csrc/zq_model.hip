// zq_model.hip -- the device-resident Llama-layout decoder behind
// include/zq_model.h.
//
// Everything a forward pass touches lives in HBM: the weights in their native
// GGML blocks (one arena, uploaded once from the mapped GGUF), the fp32 KV
// cache, the RoPE cos/sin table, the activations and the GEMM workspace.  The
// host only sends token ids and positions (4-byte copies) and reads back ids
// and, on request, logits.  A decode step is captured once as a HIP graph and
// replayed: token id and position are read by the kernels from device memory,
// so the graph never changes.
//
// Forward semantics follow the reference runtime's llama path
// (src/adapters/dense_transformer_runtime.cpp of the reference):
//   load (:673-925): llama metadata keys, head_dim = embedding / heads,
//     rope.dimension_count (default head_dim), rope.freq_base (default 1e4),
//     attention.layer_norm_rms_epsilon (default 1e-5), output.weight falling
//     back to token_embd.weight, adjacent RoPE pairs for llama;
//   forward (:3670-4606) / forward_batch (:2296-): embed -> per layer
//     { x += W_o . attn(rope(W_q h), rope(W_k h), W_v h), h = rms(x) ;
//       x += W_down . (silu(W_gate h) * W_up h), h = rms(x) } -> rms -> W_out;
//   generate (:4652-4808): prefill, then greedy tokens until EOS or max_new.
#include "../../include/zq_hip.h"
#include "../../include/zq_model.h"
#include "zq_device.hpp"
#include "zq_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

constexpr uint32_t kPrefillChunk = 1024;  // tokens per prefill pass (activations sized for this)
constexpr size_t kAlign = 256;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Weight {
    const uint8_t* p = nullptr;
    int fmt = 0;
    uint32_t rows = 0, cols = 0;
};

struct Layer {
    Weight q, k, v, o, gate, up, down;
    const float* attn_norm = nullptr;
    const float* ffn_norm = nullptr;
    float* kc = nullptr;
    float* vc = nullptr;
};

}  // namespace

struct zq_model {
    zq_model_config cfg{};
    int prefill_mode = ZQ_PREFILL_INT8;
    hipStream_t stream = nullptr;
    std::vector<void*> allocs;
    uint64_t weight_bytes = 0, cache_bytes = 0, act_bytes = 0;

    std::vector<Layer> layers;
    Weight embd, out;
    const float* out_norm = nullptr;
    float* cos_tab = nullptr;
    float* sin_tab = nullptr;
    uint32_t pairs = 0;
    float attn_scale = 1.0f;

    // device scalars and host mirrors (pinned)
    uint32_t* tokens_dev = nullptr;  // kPrefillChunk ids
    uint32_t* pos_dev = nullptr;
    uint32_t* next_dev = nullptr;
    uint32_t* host_small = nullptr;  // [0] pos, [1] next, [2..] token staging

    // activations (rows = kPrefillChunk)
    float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *tmp = nullptr;
    float *gate = nullptr, *up = nullptr, *act = nullptr, *logits = nullptr;
    int8_t* xq = nullptr;
    float* xs = nullptr;
    float* partial = nullptr;
    size_t partial_bytes = 0;  // its size (GEMM split-K partials, split Q6_K activations)
    float* attn_part = nullptr;  // decode attention chunk partials
    float* qkv = nullptr;        // prefill output of the fused Q|K|V projection, [T][QW + 2 KW]
    void* argmax_part = nullptr;
    double* ss = nullptr;  // 2 x zq::kRnSlots sum-of-squares slots of the residual-norm decode

    uint32_t cur_pos = 0;  // positions held in the cache
    bool use_graph = true;
    bool fused = false;    // decode step with norms and SiLU folded into the GEMVs
    bool fuse_quant = true;  // prefill norms / SiLU*up also write the int8 activations; K-quant gate|up pair
    bool resid_norm = false;  // Q4_K / Q5_K decode with the norms carried by the GEMVs (zq::ResidNorm)
    hipGraphExec_t decode_exec = nullptr;
    hipGraph_t decode_graph = nullptr;

    // zq_model_set_tap: one layer's int8 prefill projections copied to tap_dev
    uint32_t tap_layer = 0;
    uint8_t* tap_dev = nullptr;
    size_t tap_cap = 0, tap_used = 0;
    bool tap_overflow = false;
    std::vector<zq_model_tap_record> tap_recs;

    ~zq_model() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (decode_exec) (void)hipGraphExecDestroy(decode_exec);
        if (decode_graph) (void)hipGraphDestroy(decode_graph);
        for (void* p : allocs) (void)hipFree(p);
        if (host_small) (void)hipHostFree(host_small);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

void set_err(char* err, size_t cap, const std::string& m) {
    if (err && cap) std::snprintf(err, cap, "%s", m.c_str());
}

// The reference's rope_table for the unscaled / linear cases (:260-284): angle
// = position * base^(-2i/rotary_dim) in float, cos/sin in float.
void build_rope_table(uint32_t positions, uint32_t rotary_dim, float base, float linear_factor, std::vector<float>& cs,
                      std::vector<float>& sn) {
    rotary_dim -= rotary_dim % 2;
    const uint32_t half = rotary_dim / 2;
    cs.resize(size_t(positions) * half);
    sn.resize(size_t(positions) * half);
    std::vector<float> freq(half);
    for (uint32_t i = 0; i < half; ++i) freq[i] = std::pow(base, -2.0f * float(i) / float(rotary_dim));
    for (uint32_t p = 0; p < positions; ++p)
        for (uint32_t i = 0; i < half; ++i) {
            float position = float(p);
            if (linear_factor > 0.0f) position /= std::max(1.0f, linear_factor);
            const float angle = position * freq[i];
            cs[size_t(p) * half + i] = std::cos(angle);
            sn[size_t(p) * half + i] = std::sin(angle);
        }
}

bool dev_alloc(zq_model& m, void** p, size_t bytes) {
    if (hipMalloc(p, std::max<size_t>(bytes, 1)) != hipSuccess) return false;
    m.allocs.push_back(*p);
    return true;
}

// Activation buffers, GEMM workspace, device scalars, KV cache, RoPE table.
bool alloc_runtime(zq_model& m, std::string& e) {
    const auto& c = m.cfg;
    const size_t T = kPrefillChunk, E = c.embedding, QW = size_t(c.heads) * c.head_dim,
                 KW = size_t(c.kv_heads) * c.head_dim, F = c.ffn;
    const size_t widest = std::max({E, QW, F});
    struct B { float** p; size_t n; };
    const B bufs[] = {{&m.x, T * E}, {&m.h, T * E}, {&m.q, T * QW}, {&m.k, T * KW}, {&m.v, T * KW}, {&m.att, T * QW},
                      {&m.tmp, T * E}, {&m.gate, T * F}, {&m.up, T * F}, {&m.act, T * F}, {&m.logits, c.vocab},
                      {&m.qkv, T * (QW + 2 * KW)}};
    size_t total = 0;
    for (const B& b : bufs) total += align_up(b.n * 4, kAlign);
    // int8 activations + scales + split-K partials for the widest projection
    size_t partial = 0;
    for (uint32_t M = 1; M <= kPrefillChunk; ++M)
        for (auto nk : {std::pair<size_t, size_t>{QW, E}, {KW, E}, {QW + 2 * KW, E}, {E, QW}, {F, E}, {E, F}})
            partial = std::max({partial, zq::gemm_i8_partial_bytes(M, nk.first, nk.second),
                                zq::gemm_f32_workspace_bytes(zq::kQ4_K, M, nk.first, nk.second)});
    const size_t xq_bytes = align_up(T * widest, kAlign), xs_bytes = align_up(T * widest / 32 * 4, kAlign);
    const size_t attn_bytes = align_up(zq::attention_decode_partial_floats(c.heads, c.head_dim, c.max_positions) * 4, kAlign);
    const size_t arg_bytes = align_up(zq::argmax_partial_bytes(), kAlign);
    const size_t ss_bytes = align_up(2 * zq::kRnSlots * sizeof(double), kAlign);
    total += xq_bytes + xs_bytes + align_up(partial, kAlign) + 3 * kAlign + align_up(T * 4, kAlign) + attn_bytes + arg_bytes +
             ss_bytes;
    void* arena;
    if (!dev_alloc(m, &arena, total)) { e = "device allocation failed (activations)"; return false; }
    m.act_bytes = total;
    uint8_t* p = static_cast<uint8_t*>(arena);
    for (const B& b : bufs) { *b.p = reinterpret_cast<float*>(p); p += align_up(b.n * 4, kAlign); }
    m.xq = reinterpret_cast<int8_t*>(p); p += xq_bytes;
    m.xs = reinterpret_cast<float*>(p); p += xs_bytes;
    m.partial = partial ? reinterpret_cast<float*>(p) : nullptr; p += align_up(partial, kAlign);
    m.partial_bytes = partial;
    m.attn_part = reinterpret_cast<float*>(p); p += attn_bytes;
    if (hipMemset(m.attn_part, 0, attn_bytes) != hipSuccess) { e = "device memset failed (attention counters)"; return false; }
    m.argmax_part = p; p += arg_bytes;
    m.ss = reinterpret_cast<double*>(p); p += ss_bytes;
    // the residual-norm decode's first o GEMV adds into slots that start at 0;
    // every decode step leaves them at 0 again
    if (hipMemset(m.ss, 0, ss_bytes) != hipSuccess) { e = "device memset failed (norm slots)"; return false; }
    m.pos_dev = reinterpret_cast<uint32_t*>(p); p += kAlign;
    m.next_dev = reinterpret_cast<uint32_t*>(p); p += kAlign;
    p += kAlign;
    m.tokens_dev = reinterpret_cast<uint32_t*>(p);

    // KV cache: [layer][position][kv_heads * head_dim] for K and V
    const size_t per = size_t(c.max_positions) * KW * 4;
    void* kv;
    if (!dev_alloc(m, &kv, 2 * per * c.layers)) { e = "device allocation failed (KV cache)"; return false; }
    m.cache_bytes = 2 * per * c.layers;
    for (uint32_t l = 0; l < c.layers; ++l) {
        m.layers[l].kc = reinterpret_cast<float*>(static_cast<uint8_t*>(kv) + 2 * l * per);
        m.layers[l].vc = reinterpret_cast<float*>(static_cast<uint8_t*>(kv) + (2 * l + 1) * per);
    }
    // RoPE table
    std::vector<float> cs, sn;
    build_rope_table(c.max_positions, c.rope_dim, c.rope_base, 0.0f, cs, sn);
    m.pairs = c.rope_dim / 2;
    void* rt;
    if (!dev_alloc(m, &rt, 2 * cs.size() * 4)) { e = "device allocation failed (RoPE table)"; return false; }
    m.cos_tab = static_cast<float*>(rt);
    m.sin_tab = m.cos_tab + cs.size();
    if (hipMemcpy(m.cos_tab, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m.sin_tab, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        e = "RoPE table upload failed";
        return false;
    }
    if (hipHostMalloc(reinterpret_cast<void**>(&m.host_small), (8 + kPrefillChunk) * 4) != hipSuccess) {
        e = "pinned allocation failed";
        return false;
    }
    m.attn_scale = 1.0f / std::sqrt(float(c.head_dim));
    return true;
}

bool init_common(zq_model& m, std::string& e) {
    const auto& c = m.cfg;
    if (!c.embedding || !c.layers || !c.heads || !c.kv_heads || !c.head_dim || !c.ffn || !c.vocab || !c.max_positions) {
        e = "invalid model dimensions";
        return false;
    }
    if (c.heads % c.kv_heads) { e = "heads must be a multiple of kv_heads"; return false; }
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) { e = "head_dim must be 64, 128 or 256"; return false; }
    if (c.rope_dim == 0 || c.rope_dim > c.head_dim || c.rope_dim % 2) { e = "Invalid rotary dimension"; return false; }
    if (size_t(c.max_positions) * 4 > 96 * 1024) { e = "max_positions above 24576"; return false; }
    if (c.embedding % 32 || c.ffn % 32 || (size_t(c.heads) * c.head_dim) % 32) { e = "dimensions must divide into 32-blocks"; return false; }
    if (zq_hip_init() != ZQ_OK) { e = "no usable gfx950 device"; return false; }
    if (hipStreamCreateWithFlags(&m.stream, hipStreamNonBlocking) != hipSuccess) { e = "stream creation failed"; return false; }
    const char* g = std::getenv("ZQ_MODEL_GRAPH");
    m.use_graph = !(g && g[0] == '0');
    m.layers.resize(c.layers);
    return true;
}

// y[M][N] = X[M][K] . W^T through the GEMM (prefill) -- X already quantised
// into xq/xs when `quantized` (int8 mode).
// splits (optional, int8 activations only): the split-K reduction is left to
// the reader of Y, which sums the *splits planes at m.partial (Y is not
// written when *splits > 1).
hipError_t project(zq_model& m, const Weight& w, const float* X, float* Y, uint32_t M, bool quantized,
                   uint32_t* splits = nullptr) {
    if (splits) *splits = 1;
    if (!m.fuse_quant) splits = nullptr;  // ZQ_MODEL_FUSED=0: the GEMM reduces its own split-K planes
    if (quantized)
        return zq::launch_gemm_i8(w.fmt, w.p, m.xq, m.xs, Y, m.partial, M, w.rows, w.cols, m.stream, splits);
    return zq::launch_gemm_f32(w.fmt, w.p, X, Y, m.partial, m.partial_bytes, M, w.rows, w.cols, m.stream);
}

bool int8_ok(int fmt) { return fmt == zq::kQ8_0 || fmt == zq::kQ4_0; }

// q, k and v of one type stored back to back: one [QW + 2 KW] x E weight.
bool qkv_packed(const Layer& L, Weight& qkv) {
    const size_t rb = zq::row_bytes(L.q.fmt, L.q.cols);
    if (L.k.fmt != L.q.fmt || L.v.fmt != L.q.fmt || L.k.cols != L.q.cols || L.v.cols != L.q.cols ||
        L.k.p != L.q.p + size_t(L.q.rows) * rb || L.v.p != L.k.p + size_t(L.k.rows) * rb)
        return false;
    qkv = Weight{L.q.p, L.q.fmt, L.q.rows + L.k.rows + L.v.rows, L.q.cols};
    return true;
}

// Whether the projections ws read their input as int8 activations (prefill
// in ZQ_PREFILL_INT8 mode, formats with an int8 GEMM).
bool int8_inputs(const zq_model& m, std::initializer_list<const Weight*> ws) {
    bool q = m.prefill_mode == ZQ_PREFILL_INT8;
    for (const Weight* w : ws) q = q && int8_ok(w->fmt);
    return q;
}

// Quantise X[M][K] once for every projection that reads it in int8 mode.
hipError_t quantize_for(zq_model& m, std::initializer_list<const Weight*> ws, const float* X, uint32_t M, uint32_t K,
                        bool& quantized) {
    quantized = int8_inputs(m, ws);
    if (!quantized) return hipSuccess;
    return zq::launch_quantize_acts(X, m.xq, m.xs, M, K, m.stream);
}

#define HIPCHK(x)                              \
    do {                                       \
        const hipError_t e_ = (x);             \
        if (e_ != hipSuccess) return e_;       \
    } while (0)

// zq_model_set_tap: after an int8 projection of the tapped layer, copy its
// activations, scales and output planes (m.partial when split) to the tap
// buffer, in stream order.
hipError_t tap(zq_model& m, uint32_t layer, int proj, const Weight& w, uint32_t M, bool quantized, const float* Y,
               uint32_t splits) {
    if (!m.tap_dev || layer != m.tap_layer || !quantized) return hipSuccess;
    const size_t xq = size_t(M) * w.cols, xs = size_t(M) * (w.cols / 32) * 4;
    const size_t y = size_t(splits) * M * w.rows * 4;
    const size_t o0 = align_up(m.tap_used, kAlign), o1 = align_up(o0 + xq, kAlign), o2 = align_up(o1 + xs, kAlign);
    if (o2 + y > m.tap_cap) {
        m.tap_overflow = true;
        return hipSuccess;
    }
    HIPCHK(hipMemcpyAsync(m.tap_dev + o0, m.xq, xq, hipMemcpyDeviceToDevice, m.stream));
    HIPCHK(hipMemcpyAsync(m.tap_dev + o1, m.xs, xs, hipMemcpyDeviceToDevice, m.stream));
    HIPCHK(hipMemcpyAsync(m.tap_dev + o2, splits > 1 ? m.partial : Y, y, hipMemcpyDeviceToDevice, m.stream));
    m.tap_used = o2 + y;
    m.tap_recs.push_back(zq_model_tap_record{proj, w.fmt, w.p, M, w.rows, w.cols, splits, o0, o1, o2});
    return hipSuccess;
}

// Decoder layers over T tokens at positions pos0 .. pos0+T-1 (pos0 in device
// memory).  On entry x holds the embeddings; on exit x is the residual stream
// and h = rmsnorm(x) * output_norm, every residual add fused into the norm
// that follows it.
hipError_t enqueue_layers(zq_model& m, uint32_t T) {
    const auto& c = m.cfg;
    const uint32_t E = c.embedding, QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim, F = c.ffn;
    // In prefill the RMSNorm and SiLU*up kernels write the int8 activations
    // of their output when the projections that read it take them (the
    // quantiser's own arithmetic, one launch fewer per GEMM group), and then
    // skip the fp32 output, which nothing reads.
    auto qin = [&](std::initializer_list<const Weight*> ws) { return T > 1 && m.fuse_quant && int8_inputs(m, ws); };
    {
        const Layer& L0 = m.layers[0];
        const bool q0 = qin({&L0.q, &L0.k, &L0.v});
        HIPCHK(zq::launch_rmsnorm(m.x, L0.attn_norm, q0 ? nullptr : m.h, T, E, c.rms_epsilon, m.stream,
                                  q0 ? m.xq : nullptr, q0 ? m.xs : nullptr));
    }
    for (uint32_t l = 0; l < c.layers; ++l) {
        Layer& L = m.layers[l];
        // split-K planes of the qkv / o / down GEMM outputs left to their readers
        // (the RoPE + KV-append kernel, the norms)
        uint32_t qkv_splits = 1, o_splits = 1, d_splits = 1;
        if (T == 1) {
            // decode: the three projections share x -> one batched GEMV per format
            zq::GemvTask t[3] = {{L.q.p, m.q, QW}, {L.k.p, m.k, KW}, {L.v.p, m.v, KW}};
            if (L.q.fmt == L.k.fmt && L.k.fmt == L.v.fmt) {
                HIPCHK(zq::launch_gemv(L.q.fmt, t, 3, m.h, E, m.stream));
            } else {
                HIPCHK(zq::launch_gemv(L.q.fmt, &t[0], 1, m.h, E, m.stream));
                HIPCHK(zq::launch_gemv(L.k.fmt, &t[1], 1, m.h, E, m.stream));
                HIPCHK(zq::launch_gemv(L.v.fmt, &t[2], 1, m.h, E, m.stream));
            }
        } else {
            bool qz = qin({&L.q, &L.k, &L.v});  // h's int8 activations came with its norm
            if (!qz) HIPCHK(quantize_for(m, {&L.q, &L.k, &L.v}, m.h, T, E, qz));
            Weight qkv;
            if (qkv_packed(L, qkv)) {
                HIPCHK(project(m, qkv, m.h, m.qkv, T, qz, &qkv_splits));
                HIPCHK(tap(m, l, ZQ_TAP_QKV, qkv, T, qz, m.qkv, qkv_splits));
            } else {
                HIPCHK(project(m, L.q, m.h, m.q, T, qz));
                HIPCHK(tap(m, l, ZQ_TAP_Q, L.q, T, qz, m.q, 1));
                HIPCHK(project(m, L.k, m.h, m.k, T, qz));
                HIPCHK(tap(m, l, ZQ_TAP_K, L.k, T, qz, m.k, 1));
                HIPCHK(project(m, L.v, m.h, m.v, T, qz));
                HIPCHK(tap(m, l, ZQ_TAP_V, L.v, T, qz, m.v, 1));
            }
        }
        if (T == 1) {
            HIPCHK(zq::launch_attention_decode(m.q, m.k, m.v, L.kc, L.vc, m.cos_tab, m.sin_tab, m.attn_part, m.att,
                                               m.pos_dev, c.heads, c.kv_heads, c.head_dim, m.pairs, c.max_positions,
                                               m.attn_scale, m.stream));
            zq::GemvTask t = {L.o.p, m.tmp, E};
            HIPCHK(zq::launch_gemv(L.o.fmt, &t, 1, m.att, QW, m.stream));
        } else {
            Weight qkv;
            if (qkv_packed(L, qkv)) {
                const float* base = qkv_splits > 1 ? m.partial : m.qkv;
                HIPCHK(zq::launch_rope_kv(m.q, base + QW, base + QW + KW, L.kc, L.vc, m.cos_tab, m.sin_tab, m.pos_dev, T,
                                          c.heads, c.kv_heads, c.head_dim, m.pairs, true, m.stream, QW + 2 * KW, base,
                                          qkv_splits, m.qkv));
            }
            else
                HIPCHK(zq::launch_rope_kv(m.q, m.k, m.v, L.kc, L.vc, m.cos_tab, m.sin_tab, m.pos_dev, T, c.heads,
                                          c.kv_heads, c.head_dim, m.pairs, true, m.stream));
            // with int8 o inputs the attention kernel writes them itself when it can
            const bool qo = qin({&L.o});
            bool qz = false;
            HIPCHK(zq::launch_attention(m.q, L.kc, L.vc, m.att, m.pos_dev, T, c.heads, c.kv_heads, c.head_dim,
                                        c.max_positions, m.attn_scale, m.stream, qo ? m.xq : nullptr,
                                        qo ? m.xs : nullptr, &qz));
            if (!qz) HIPCHK(quantize_for(m, {&L.o}, m.att, T, QW, qz));
            HIPCHK(project(m, L.o, m.att, m.tmp, T, qz, &o_splits));
            HIPCHK(tap(m, l, ZQ_TAP_O, L.o, T, qz, m.tmp, o_splits));
        }
        // the o projection's split-K partials, if any, are summed by the norm
        const bool qgu = qin({&L.gate, &L.up});
        HIPCHK(zq::launch_add_rmsnorm(m.x, o_splits > 1 ? m.partial : m.tmp, L.ffn_norm, qgu ? nullptr : m.h, T, E,
                                      c.rms_epsilon, m.stream, qgu ? m.xq : nullptr, qgu ? m.xs : nullptr, o_splits));
        // decode on Q4_K / Q5_K / Q6_K: gate|up storing silu(gate)*up itself (the
        // per-row sums and the activation of the separate launches)
        bool act_done = false;
        if (T == 1 && m.fuse_quant && L.gate.fmt == L.up.fmt) {
            const hipError_t e = zq::launch_gemv_silu_pair(L.gate.fmt, {L.gate.p, m.act, F}, {L.up.p, m.up, F}, m.h, E,
                                                           m.stream);
            if (e != hipSuccess && e != hipErrorInvalidConfiguration) return e;
            act_done = e == hipSuccess;
        }
        if (T == 1 && !act_done) {
            zq::GemvTask t[2] = {{L.gate.p, m.gate, F}, {L.up.p, m.up, F}};
            if (L.gate.fmt == L.up.fmt) {
                HIPCHK(zq::launch_gemv(L.gate.fmt, t, 2, m.h, E, m.stream));
            } else {
                HIPCHK(zq::launch_gemv(L.gate.fmt, &t[0], 1, m.h, E, m.stream));
                HIPCHK(zq::launch_gemv(L.up.fmt, &t[1], 1, m.h, E, m.stream));
            }
        } else if (T > 1) {
            bool qz = qgu;
            if (!qz) HIPCHK(quantize_for(m, {&L.gate, &L.up}, m.h, T, E, qz));
            HIPCHK(project(m, L.gate, m.h, m.gate, T, qz));
            HIPCHK(tap(m, l, ZQ_TAP_GATE, L.gate, T, qz, m.gate, 1));
            HIPCHK(project(m, L.up, m.h, m.up, T, qz));
            HIPCHK(tap(m, l, ZQ_TAP_UP, L.up, T, qz, m.up, 1));
        }
        const bool qd = qin({&L.down});
        if (!act_done)
            HIPCHK(zq::launch_silu_mul(m.gate, m.up, qd ? nullptr : m.act, size_t(T) * F, m.stream,
                                       qd ? m.xq : nullptr, qd ? m.xs : nullptr));
        if (T == 1) {
            zq::GemvTask t = {L.down.p, m.tmp, E};
            HIPCHK(zq::launch_gemv(L.down.fmt, &t, 1, m.act, F, m.stream));
        } else {
            bool qz = qd;
            if (!qz) HIPCHK(quantize_for(m, {&L.down}, m.act, T, F, qz));
            HIPCHK(project(m, L.down, m.act, m.tmp, T, qz, &d_splits));
            HIPCHK(tap(m, l, ZQ_TAP_DOWN, L.down, T, qz, m.tmp, d_splits));
        }
        const float* next_norm = l + 1 < c.layers ? m.layers[l + 1].attn_norm : m.out_norm;
        const bool qn = l + 1 < c.layers && qin({&m.layers[l + 1].q, &m.layers[l + 1].k, &m.layers[l + 1].v});
        HIPCHK(zq::launch_add_rmsnorm(m.x, d_splits > 1 ? m.partial : m.tmp, next_norm, qn ? nullptr : m.h, T, E,
                                      c.rms_epsilon, m.stream, qn ? m.xq : nullptr, qn ? m.xs : nullptr, d_splits));
    }
    return hipSuccess;
}

// The output projection of row `row` of h (already output-normed) and the
// greedy id.
hipError_t enqueue_head(zq_model& m, uint32_t row) {
    const auto& c = m.cfg;
    zq::GemvTask t = {m.out.p, m.logits, c.vocab};
    HIPCHK(zq::launch_gemv(m.out.fmt, &t, 1, m.h + size_t(row) * c.embedding, c.embedding, m.stream));
    return zq::launch_argmax(m.logits, c.vocab, m.next_dev, m.argmax_part, m.stream);
}

// Decode step with every residual add + RMSNorm and the SiLU*up folded into
// the GEMV that consumes it (zq::XPrologue): per layer QKV, attention, o,
// gate|up, down.  The residual stream alternates between x and h (h is not
// otherwise used on this path), so no workgroup's residual write races the
// reads of another.
hipError_t enqueue_decode_fused(zq_model& m) {
    const auto& c = m.cfg;
    const uint32_t E = c.embedding, QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim, F = c.ffn;
    float* r = m.x;
    float* ralt = m.h;
    const float* delta = nullptr;  // the pending residual add (down output)
    for (uint32_t l = 0; l < c.layers; ++l) {
        Layer& L = m.layers[l];
        zq::GemvTask tq[3] = {{L.q.p, m.q, QW}, {L.k.p, m.k, KW}, {L.v.p, m.v, KW}};
        const zq::XPrologue pq{zq::kAddNorm, r, delta, L.attn_norm, delta ? ralt : nullptr, c.rms_epsilon};
        HIPCHK(zq::launch_gemv_prologue(L.q.fmt, tq, 3, pq, E, m.stream));
        if (delta) std::swap(r, ralt);
        HIPCHK(zq::launch_attention_decode(m.q, m.k, m.v, L.kc, L.vc, m.cos_tab, m.sin_tab, m.attn_part, m.att,
                                           m.pos_dev, c.heads, c.kv_heads, c.head_dim, m.pairs, c.max_positions,
                                           m.attn_scale, m.stream));
        zq::GemvTask to = {L.o.p, m.tmp, E};
        HIPCHK(zq::launch_gemv(L.o.fmt, &to, 1, m.att, QW, m.stream));
        zq::GemvTask tg[2] = {{L.gate.p, m.gate, F}, {L.up.p, m.up, F}};
        const zq::XPrologue pg{zq::kAddNorm, r, m.tmp, L.ffn_norm, ralt, c.rms_epsilon};
        zq::GemvTask td = {L.down.p, m.tmp, E};
        // gate|up storing silu(gate)*up itself, then a plain down GEMV; where
        // that form does not apply, gate|up and a down GEMV with the SiLU*up
        // prologue
        const hipError_t ep = L.gate.fmt == L.up.fmt
                                  ? zq::launch_gemv_prologue_silu_pair(L.gate.fmt, tg[0], tg[1], pg, E, m.stream)
                                  : hipErrorInvalidConfiguration;
        if (ep == hipSuccess) {
            std::swap(r, ralt);
            HIPCHK(zq::launch_gemv(L.down.fmt, &td, 1, m.gate, F, m.stream));
        } else {
            if (ep != hipErrorInvalidConfiguration) return ep;
            HIPCHK(zq::launch_gemv_prologue(L.gate.fmt, tg, 2, pg, E, m.stream));
            std::swap(r, ralt);
            const zq::XPrologue pd{zq::kSiluMul, m.gate, m.up, nullptr, nullptr, 0.0f};
            HIPCHK(zq::launch_gemv_prologue(L.down.fmt, &td, 1, pd, F, m.stream));
        }
        delta = m.tmp;
    }
    zq::GemvTask th = {m.out.p, m.logits, c.vocab};
    const zq::XPrologue ph{zq::kAddNorm, r, delta, m.out_norm, nullptr, c.rms_epsilon};
    HIPCHK(zq::launch_gemv_prologue(m.out.fmt, &th, 1, ph, E, m.stream));
    return zq::launch_argmax(m.logits, c.vocab, m.next_dev, m.argmax_part, m.stream);
}

// Decode step on Q4_K / Q5_K projections with the residual adds and RMSNorms
// carried by the GEMVs (zq::ResidNorm): the o and down GEMVs add their rows
// into the residual x and their squares into slot set A (o) or B (down), and
// clear the other set; QKV (from B) and the gate|up pair (from A) normalise x
// as they load it.  Layer 0's input and the output norm keep their RMSNorm
// launches.  Per layer: QKV, attention, o, gate|up, down.
hipError_t enqueue_decode_resid(zq_model& m) {
    const auto& c = m.cfg;
    const uint32_t E = c.embedding, QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim, F = c.ffn;
    double* A = m.ss;
    double* B = m.ss + zq::kRnSlots;
    HIPCHK(zq::launch_rmsnorm(m.x, m.layers[0].attn_norm, m.h, 1, E, c.rms_epsilon, m.stream));
    for (uint32_t l = 0; l < c.layers; ++l) {
        Layer& L = m.layers[l];
        zq::GemvTask tq[3] = {{L.q.p, m.q, QW}, {L.k.p, m.k, KW}, {L.v.p, m.v, KW}};
        if (l == 0) {
            HIPCHK(zq::launch_gemv(L.q.fmt, tq, 3, m.h, E, m.stream));
        } else {
            const zq::ResidNorm rq{B, L.attn_norm, nullptr, nullptr, c.rms_epsilon};
            HIPCHK(zq::launch_gemv_resid(L.q.fmt, zq::kRnNormIn, tq, 3, m.x, E, rq, m.stream));
        }
        HIPCHK(zq::launch_attention_decode(m.q, m.k, m.v, L.kc, L.vc, m.cos_tab, m.sin_tab, m.attn_part, m.att,
                                           m.pos_dev, c.heads, c.kv_heads, c.head_dim, m.pairs, c.max_positions,
                                           m.attn_scale, m.stream));
        const zq::GemvTask to{L.o.p, m.x, E};
        const zq::ResidNorm ro{nullptr, nullptr, A, B, 0.0f};
        HIPCHK(zq::launch_gemv_resid(L.o.fmt, zq::kRnAddOut, &to, 1, m.att, QW, ro, m.stream));
        const zq::ResidNorm rg{A, L.ffn_norm, nullptr, nullptr, c.rms_epsilon};
        HIPCHK(zq::launch_gemv_silu_pair(L.gate.fmt, {L.gate.p, m.act, F}, {L.up.p, m.up, F}, m.x, E, m.stream, &rg));
        const zq::GemvTask td{L.down.p, m.x, E};
        const zq::ResidNorm rd{nullptr, nullptr, B, A, 0.0f};
        HIPCHK(zq::launch_gemv_resid(L.down.fmt, zq::kRnAddOut, &td, 1, m.act, F, rd, m.stream));
    }
    HIPCHK(zq::launch_rmsnorm(m.x, m.out_norm, m.h, 1, E, c.rms_epsilon, m.stream));
    return enqueue_head(m, 0);
}

hipError_t enqueue_decode(zq_model& m) {
    HIPCHK(zq::launch_embed(m.embd.fmt, m.embd.p, m.tokens_dev, m.cfg.vocab, m.x, m.cfg.embedding, 1, m.stream));
    if (m.fused) return enqueue_decode_fused(m);
    if (m.resid_norm) return enqueue_decode_resid(m);
    HIPCHK(enqueue_layers(m, 1));
    return enqueue_head(m, 0);
}

// The fused decode covers Q8_0 / Q4_0 projections on the streaming GEMV's
// shapes; anything else keeps the separate norm / activation kernels.
// ZQ_MODEL_FUSED=0 disables it, the super-block formats' paired gate|up
// GEMV and, in prefill, the quantisers folded into the norm / SiLU kernels
// and the split-K sums left to the GEMMs' readers (A/B runs and the
// equivalence tests).
void choose_fused(zq_model& m) {
    const char* e = std::getenv("ZQ_MODEL_FUSED");
    const auto& c = m.cfg;
    auto ok = [](int f) { return f == zq::kQ8_0 || f == zq::kQ4_0; };
    bool f = !(e && e[0] == '0') && c.embedding % 256 == 0 && c.ffn % 256 == 0 && c.embedding <= 16384 &&
             c.ffn <= 16384 && ok(m.out.fmt);
    for (const Layer& L : m.layers)
        f = f && ok(L.q.fmt) && L.k.fmt == L.q.fmt && L.v.fmt == L.q.fmt && ok(L.gate.fmt) && L.up.fmt == L.gate.fmt &&
            ok(L.down.fmt) && ok(L.o.fmt);
    m.fused = f;
    m.fuse_quant = !(e && e[0] == '0');
    // Q4_K / Q5_K: every projection of every layer on the residual-norm GEMVs
    const uint32_t QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
    auto rs = [&](const Weight& w, uint32_t cols) { return zq::gemv_resid_supported(w.fmt, cols); };
    bool r = m.fuse_quant && !f && QW % 256 == 0 && KW > 0;
    for (const Layer& L : m.layers)
        r = r && rs(L.q, c.embedding) && L.k.fmt == L.q.fmt && L.v.fmt == L.q.fmt && rs(L.o, QW) &&
            rs(L.gate, c.embedding) && L.up.fmt == L.gate.fmt && rs(L.down, c.ffn);
    m.resid_norm = r;
}

int finish_outputs(zq_model& m, float* logits, uint32_t* next) {
    if (hipMemcpyAsync(&m.host_small[1], m.next_dev, 4, hipMemcpyDeviceToHost, m.stream) != hipSuccess) return ZQ_ERR_HIP;
    if (logits && hipMemcpyAsync(logits, m.logits, size_t(m.cfg.vocab) * 4, hipMemcpyDeviceToHost, m.stream) != hipSuccess)
        return ZQ_ERR_HIP;
    if (hipStreamSynchronize(m.stream) != hipSuccess) return ZQ_ERR_HIP;
    if (next) *next = m.host_small[1];
    return ZQ_OK;
}

int prefill(zq_model& m, const uint32_t* tokens, size_t n, float* logits, uint32_t* next) {
    if (!tokens || !n || n > m.cfg.max_positions) return ZQ_ERR_ARG;
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= m.cfg.vocab) return ZQ_ERR_ARG;
    m.cur_pos = 0;
    m.tap_used = 0;
    m.tap_overflow = false;
    m.tap_recs.clear();
    for (size_t s = 0; s < n; s += kPrefillChunk) {
        const uint32_t T = uint32_t(std::min<size_t>(kPrefillChunk, n - s));
        m.host_small[0] = uint32_t(s);
        std::memcpy(&m.host_small[8], tokens + s, size_t(T) * 4);
        if (hipMemcpyAsync(m.pos_dev, &m.host_small[0], 4, hipMemcpyHostToDevice, m.stream) != hipSuccess ||
            hipMemcpyAsync(m.tokens_dev, &m.host_small[8], size_t(T) * 4, hipMemcpyHostToDevice, m.stream) != hipSuccess)
            return ZQ_ERR_HIP;
        if (zq::launch_embed(m.embd.fmt, m.embd.p, m.tokens_dev, m.cfg.vocab, m.x, m.cfg.embedding, T, m.stream) != hipSuccess ||
            enqueue_layers(m, T) != hipSuccess)
            return ZQ_ERR_HIP;
        if (s + T == n && enqueue_head(m, T - 1) != hipSuccess) return ZQ_ERR_HIP;
        // the staging words are reused by the next chunk: wait for the copies
        if (s + T < n && hipStreamSynchronize(m.stream) != hipSuccess) return ZQ_ERR_HIP;
    }
    m.cur_pos = uint32_t(n);
    return finish_outputs(m, logits, next);
}

int decode(zq_model& m, uint32_t token, float* logits, uint32_t* next) {
    if (token >= m.cfg.vocab || m.cur_pos >= m.cfg.max_positions) return ZQ_ERR_ARG;
    m.host_small[0] = m.cur_pos;
    m.host_small[8] = token;
    if (hipMemcpyAsync(m.pos_dev, &m.host_small[0], 4, hipMemcpyHostToDevice, m.stream) != hipSuccess ||
        hipMemcpyAsync(m.tokens_dev, &m.host_small[8], 4, hipMemcpyHostToDevice, m.stream) != hipSuccess)
        return ZQ_ERR_HIP;
    if (m.use_graph) {
        if (!m.decode_exec) {
            if (hipStreamBeginCapture(m.stream, hipStreamCaptureModeThreadLocal) != hipSuccess) return ZQ_ERR_HIP;
            const hipError_t e = enqueue_decode(m);
            hipGraph_t g = nullptr;
            const hipError_t e2 = hipStreamEndCapture(m.stream, &g);
            if (e != hipSuccess || e2 != hipSuccess || !g) {
                if (g) (void)hipGraphDestroy(g);
                return ZQ_ERR_HIP;
            }
            m.decode_graph = g;
            if (hipGraphInstantiate(&m.decode_exec, g, nullptr, nullptr, 0) != hipSuccess) {
                m.decode_exec = nullptr;
                return ZQ_ERR_HIP;
            }
        }
        if (hipGraphLaunch(m.decode_exec, m.stream) != hipSuccess) return ZQ_ERR_HIP;
    } else if (enqueue_decode(m) != hipSuccess) {
        return ZQ_ERR_HIP;
    }
    const int st = finish_outputs(m, logits, next);
    if (st == ZQ_OK) ++m.cur_pos;
    return st;
}

}  // namespace

extern "C" {

int zq_model_load_gguf(const zq_gguf* g, uint32_t max_positions, zq_model_config* cfg_out, zq_model** model,
                       char* err, size_t err_cap) {
    if (!g || !model) return ZQ_ERR_ARG;
    *model = nullptr;
    zq_gguf_config gc;
    zq_gguf_get_config(g, &gc);
    auto fail = [&](const std::string& m, int st = ZQ_ERR_ARG) { set_err(err, err_cap, m); return st; };
    if (std::strcmp(gc.architecture, "llama") != 0) return fail("only the llama architecture is supported", ZQ_DECLINED);
    auto meta_f = [&](const char* k, float fb) {
        const char* v = zq_gguf_meta_value(g, k);
        if (!v) return fb;
        char* end = nullptr;
        const float f = std::strtof(v, &end);
        return end != v ? f : fb;
    };
    auto meta_u = [&](const char* k, uint32_t fb) {
        const char* v = zq_gguf_meta_value(g, k);
        if (!v) return fb;
        char* end = nullptr;
        const unsigned long u = std::strtoul(v, &end, 10);
        return end != v ? uint32_t(u) : fb;
    };
    auto* m = new zq_model;
    zq_model_config& c = m->cfg;
    c.embedding = gc.embedding_length;
    c.layers = gc.block_count;
    c.heads = gc.head_count;
    c.kv_heads = gc.head_count_kv ? gc.head_count_kv : gc.head_count;
    c.ffn = gc.feed_forward_length;
    c.context = gc.context_length;
    c.head_dim = c.heads ? meta_u("llama.attention.key_length", 0) : 0;
    if (!c.head_dim && c.heads) c.head_dim = c.embedding / c.heads;
    c.rope_dim = meta_u("llama.rope.dimension_count", c.head_dim);
    c.rope_base = meta_f("llama.rope.freq_base", 10000.0f);
    c.rms_epsilon = meta_f("llama.attention.layer_norm_rms_epsilon", 1.0e-5f);
    c.eos_token = gc.eos_token_id;
    c.max_positions = max_positions ? max_positions : std::min<uint32_t>(c.context ? c.context : 4096, 4096);
    if (c.context && c.max_positions > c.context) c.max_positions = c.context;
    if (zq_gguf_meta_value(g, "llama.rope.scaling.type")) {
        const std::string st = zq_gguf_meta_value(g, "llama.rope.scaling.type");
        if (!st.empty() && st != "none") { delete m; return fail("RoPE scaling type not supported: " + st); }
    }
    // vocab from the embedding table
    zq_gguf_tensor te, to, tn;
    if (zq_gguf_find_tensor(g, "token_embd.weight", &te) != ZQ_OK) { delete m; return fail("missing token_embd.weight"); }
    c.vocab = te.n_dims == 2 ? uint32_t(te.dims[1]) : 0;
    const bool tied = zq_gguf_find_tensor(g, "output.weight", &to) != ZQ_OK;
    if (tied) to = te;
    if (zq_gguf_find_tensor(g, "output_norm.weight", &tn) != ZQ_OK) { delete m; return fail("missing output_norm.weight"); }
    std::string e;
    if (!init_common(*m, e)) { delete m; return fail(e, ZQ_ERR_NO_DEVICE); }
    const uint32_t E = c.embedding, QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim, F = c.ffn;

    // collect every tensor with its expected shape
    struct Need { std::string name; uint32_t rows, cols; Weight* w; const float** f32; bool qkv_head = false; };
    std::vector<Need> needs;
    needs.push_back({"token_embd.weight", c.vocab, E, &m->embd, nullptr});
    needs.push_back({tied ? "token_embd.weight" : "output.weight", c.vocab, E, &m->out, nullptr});
    needs.push_back({"output_norm.weight", 1, E, nullptr, &m->out_norm});
    for (uint32_t l = 0; l < c.layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        Layer& L = m->layers[l];
        needs.push_back({p + "attn_norm.weight", 1, E, nullptr, &L.attn_norm});
        needs.push_back({p + "ffn_norm.weight", 1, E, nullptr, &L.ffn_norm});
        needs.push_back({p + "attn_q.weight", QW, E, &L.q, nullptr, true});
        needs.push_back({p + "attn_k.weight", KW, E, &L.k, nullptr});
        needs.push_back({p + "attn_v.weight", KW, E, &L.v, nullptr});
        needs.push_back({p + "attn_output.weight", E, QW, &L.o, nullptr});
        needs.push_back({p + "ffn_gate.weight", F, E, &L.gate, nullptr});
        needs.push_back({p + "ffn_up.weight", F, E, &L.up, nullptr});
        needs.push_back({p + "ffn_down.weight", E, F, &L.down, nullptr});
    }
    std::vector<zq_gguf_tensor> ts(needs.size());
    std::vector<size_t> advance(needs.size());
    size_t arena = 0;
    for (size_t i = 0; i < needs.size(); ++i) {
        const Need& n = needs[i];
        if (zq_gguf_find_tensor(g, n.name.c_str(), &ts[i]) != ZQ_OK) { delete m; return fail("missing tensor " + n.name); }
        const zq_gguf_tensor& t = ts[i];
        const uint64_t rows = t.n_dims >= 2 ? t.dims[1] : 1;
        if (t.dims[0] != n.cols || rows != n.rows || t.n_dims > 2) { delete m; return fail("unexpected shape of " + n.name); }
        if (n.f32 && t.ggml_type != 0) { delete m; return fail("norm tensors must be F32: " + n.name); }
        if (n.w) {
            const bool embd = n.w == &m->embd;
            const int ty = int(t.ggml_type);
            const bool proj_ok = ty == zq::kQ8_0 || ty == zq::kQ4_0 || ty == zq::kQ4_K || ty == zq::kQ5_K ||
                                 ty == zq::kQ6_K;
            if (embd ? !(ty == zq::kQ8_0 || ty == 0) : !proj_ok) {
                delete m;
                return fail("unsupported tensor type " + std::to_string(ty) + " for " + n.name, ZQ_DECLINED);
            }
            if (n.w == &m->out && !proj_ok) {
                delete m;
                return fail("output projection must be Q8_0, Q4_0, Q4_K, Q5_K or Q6_K", ZQ_DECLINED);
            }
        }
        advance[i] = align_up(size_t(t.byte_size) + ZQ_WEIGHT_TAIL_PAD, kAlign);
    }
    // A layer's q, k and v of one type sit back to back (no padding between
    // them), so prefill runs them as one [QW + 2 KW] x E projection.
    for (size_t i = 0; i + 2 < needs.size(); ++i)
        if (needs[i].qkv_head && ts[i + 1].ggml_type == ts[i].ggml_type && ts[i + 2].ggml_type == ts[i].ggml_type &&
            ts[i].byte_size % 16 == 0 && ts[i + 1].byte_size % 16 == 0) {
            advance[i] = size_t(ts[i].byte_size);
            advance[i + 1] = size_t(ts[i + 1].byte_size);
        }
    for (size_t a : advance) arena += a;
    void* base;
    if (!dev_alloc(*m, &base, arena)) { delete m; return fail("device allocation failed (weights)", ZQ_ERR_OOM); }
    m->weight_bytes = arena;
    uint8_t* p = static_cast<uint8_t*>(base);
    for (size_t i = 0; i < needs.size(); ++i) {
        const zq_gguf_tensor& t = ts[i];
        if (hipMemcpy(p, t.data, size_t(t.byte_size), hipMemcpyHostToDevice) != hipSuccess) {
            delete m;
            return fail("weight upload failed", ZQ_ERR_HIP);
        }
        const Need& n = needs[i];
        if (n.w) *n.w = Weight{p, int(t.ggml_type), n.rows, n.cols};
        if (n.f32) *n.f32 = reinterpret_cast<const float*>(p);
        p += advance[i];
    }
    c.weight_format = m->layers.empty() ? m->out.fmt : m->layers[0].q.fmt;
    if (!alloc_runtime(*m, e)) { delete m; return fail(e, ZQ_ERR_OOM); }
    choose_fused(*m);
    if (cfg_out) *cfg_out = c;
    *model = m;
    set_err(err, err_cap, "");
    return ZQ_OK;
}

int zq_model_create_synthetic(const zq_model_config* cfg, uint64_t seed, zq_model** model, char* err, size_t err_cap) {
    if (!cfg || !model) return ZQ_ERR_ARG;
    *model = nullptr;
    auto* m = new zq_model;
    m->cfg = *cfg;
    zq_model_config& c = m->cfg;
    if (!c.head_dim && c.heads) c.head_dim = c.embedding / c.heads;
    if (!c.rope_dim) c.rope_dim = c.head_dim;
    if (!c.rope_base) c.rope_base = 10000.0f;
    if (!c.rms_epsilon) c.rms_epsilon = 1e-5f;
    // the projections in the requested format (default Q8_0); the embedding
    // table and the output projection stay Q8_0
    const int pf = c.weight_format ? c.weight_format : zq::kQ8_0;
    if (pf != zq::kQ8_0 && pf != zq::kQ4_0 && pf != zq::kQ6_K && pf != zq::kQ4_K && pf != zq::kQ5_K) {
        delete m;
        set_err(err, err_cap, "weight_format must be Q8_0, Q4_0, Q6_K, Q4_K or Q5_K");
        return ZQ_ERR_ARG;
    }
    c.weight_format = pf;
    std::string e;
    if (!init_common(*m, e)) { delete m; set_err(err, err_cap, e); return ZQ_ERR_NO_DEVICE; }
    const uint32_t E = c.embedding, QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim, F = c.ffn;
    if (pf != zq::kQ8_0 && pf != zq::kQ4_0 && (E % 256 || QW % 256 || F % 256)) {
        delete m;
        set_err(err, err_cap, "super-block formats need hidden, attention and FFN widths that are multiples of 256");
        return ZQ_ERR_ARG;
    }
    // q and k are followed by k and v without padding (one Q|K|V weight)
    struct W { Weight* w; uint32_t rows, cols; int fmt; bool packed = false; };
    std::vector<W> ws = {{&m->embd, c.vocab, E, zq::kQ8_0}, {&m->out, c.vocab, E, zq::kQ8_0}};
    for (auto& L : m->layers)
        for (auto x : {W{&L.q, QW, E, pf, true}, W{&L.k, KW, E, pf, true}, W{&L.v, KW, E, pf}, W{&L.o, E, QW, pf},
                       W{&L.gate, F, E, pf}, W{&L.up, F, E, pf}, W{&L.down, E, F, pf}})
            ws.push_back(x);
    auto advance = [](const W& w) {
        return w.packed && (size_t(w.rows) * zq::row_bytes(w.fmt, w.cols)) % 16 == 0
                   ? size_t(w.rows) * zq::row_bytes(w.fmt, w.cols)
                   : align_up(zq_weight_bytes(w.fmt, w.rows, w.cols), kAlign);
    };
    size_t arena = align_up(size_t(E) * 4, kAlign);  // one shared unit norm vector
    for (const W& w : ws) arena += advance(w);
    void* base;
    if (!dev_alloc(*m, &base, arena)) { delete m; set_err(err, err_cap, "device allocation failed (weights)"); return ZQ_ERR_OOM; }
    m->weight_bytes = arena;
    uint8_t* p = static_cast<uint8_t*>(base);
    std::vector<float> ones(E, 1.0f);
    if (hipMemcpy(p, ones.data(), size_t(E) * 4, hipMemcpyHostToDevice) != hipSuccess) { delete m; return ZQ_ERR_HIP; }
    const float* unit = reinterpret_cast<const float*>(p);
    p += align_up(size_t(E) * 4, kAlign);
    m->out_norm = unit;
    for (auto& L : m->layers) L.attn_norm = L.ffn_norm = unit;
    uint64_t s = seed;
    for (const W& w : ws) {
        *w.w = Weight{p, w.fmt, w.rows, w.cols};
        if (zq::launch_synth_weights(w.fmt, s++, p, w.rows, w.cols, m->stream) != hipSuccess) { delete m; return ZQ_ERR_HIP; }
        p += advance(w);
    }
    if (hipStreamSynchronize(m->stream) != hipSuccess) { delete m; return ZQ_ERR_HIP; }
    if (!alloc_runtime(*m, e)) { delete m; set_err(err, err_cap, e); return ZQ_ERR_OOM; }
    choose_fused(*m);
    *model = m;
    set_err(err, err_cap, "");
    return ZQ_OK;
}

void zq_model_free(zq_model* m) { delete m; }

int zq_model_weight(const zq_model* m, uint32_t layer, int which, const void** dev, uint32_t* rows, uint32_t* cols,
                    int* fmt) {
    if (!m || !dev) return ZQ_ERR_ARG;
    const Weight* w = nullptr;
    if (layer == ZQ_MODEL_GLOBAL) {
        if (which == ZQ_W_EMBED) w = &m->embd;
        else if (which == ZQ_W_OUTPUT) w = &m->out;
    } else if (layer < m->layers.size() && which >= ZQ_W_Q && which <= ZQ_W_DOWN) {
        const Layer& L = m->layers[layer];
        const Weight* t[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
        w = t[which - ZQ_W_Q];
    }
    if (!w || !w->p) return ZQ_ERR_ARG;
    *dev = w->p;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (fmt) *fmt = w->fmt;
    return ZQ_OK;
}

int zq_model_set_prefill_mode(zq_model* m, int mode) {
    if (!m || (mode != ZQ_PREFILL_INT8 && mode != ZQ_PREFILL_F32)) return ZQ_ERR_ARG;
    m->prefill_mode = mode;
    return ZQ_OK;
}

int zq_model_prefill(zq_model* m, const uint32_t* tokens, size_t n, float* logits, uint32_t* next) {
    if (!m) return ZQ_ERR_ARG;
    return prefill(*m, tokens, n, logits, next);
}

int zq_model_decode(zq_model* m, uint32_t token, float* logits, uint32_t* next) {
    if (!m) return ZQ_ERR_ARG;
    return decode(*m, token, logits, next);
}

int zq_model_generate(zq_model* m, const uint32_t* prompt, size_t n, uint32_t max_new, uint32_t* out, size_t* n_out,
                      double* prefill_ms, double* decode_ms) {
    if (!m || !prompt || !n || (max_new && !out) || !n_out) return ZQ_ERR_ARG;
    if (n + max_new > m->cfg.max_positions) return ZQ_ERR_ARG;
    using clk = std::chrono::steady_clock;
    const auto t0 = clk::now();
    uint32_t next = 0;
    int st = prefill(*m, prompt, n, nullptr, &next);
    if (st != ZQ_OK) return st;
    const auto t1 = clk::now();
    size_t count = 0;
    for (uint32_t i = 0; i < max_new; ++i) {
        out[count++] = next;
        if (next == m->cfg.eos_token || i + 1 == max_new) break;
        st = decode(*m, next, nullptr, &next);
        if (st != ZQ_OK) return st;
    }
    const auto t2 = clk::now();
    *n_out = count;
    if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (decode_ms) *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    return ZQ_OK;
}

int zq_model_set_tap(zq_model* m, uint32_t layer, void* dev, size_t cap) {
    if (!m || (dev && layer >= m->layers.size())) return ZQ_ERR_ARG;
    m->tap_layer = layer;
    m->tap_dev = static_cast<uint8_t*>(dev);
    m->tap_cap = dev ? cap : 0;
    m->tap_used = 0;
    m->tap_overflow = false;
    m->tap_recs.clear();
    return ZQ_OK;
}

int zq_model_tap_records(const zq_model* m, zq_model_tap_record* out, size_t cap, size_t* n) {
    if (!m || !n || (cap && !out)) return ZQ_ERR_ARG;
    const size_t c = std::min(cap, m->tap_recs.size());
    std::copy(m->tap_recs.begin(), m->tap_recs.begin() + c, out);
    *n = c;
    return m->tap_overflow ? ZQ_ERR_TOO_LARGE : ZQ_OK;
}

int zq_model_memory(zq_model* m, uint64_t* weight_bytes, uint64_t* cache_bytes, uint64_t* activation_bytes) {
    if (!m) return ZQ_ERR_ARG;
    if (weight_bytes) *weight_bytes = m->weight_bytes;
    if (cache_bytes) *cache_bytes = m->cache_bytes;
    if (activation_bytes) *activation_bytes = m->act_bytes;
    return ZQ_OK;
}

}  // extern "C"
