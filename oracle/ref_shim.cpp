// ref_shim.cpp -- TEST INFRASTRUCTURE ONLY.
// A C-callable shim over the reference's own CPU code, compiled together with
// the reference's sources by oracle/Makefile into oracle/_ref/libzenref.so:
//   - the quant surface (include/zen/quant.h:20-33, 106);
//   - the GGUF parse core (include/zen/gguf.h:22-29, src/gguf.cpp:113-350);
//   - the dense transformer runtime (include/zen/dense_transformer_runtime.h:20-78,
//     src/adapters/dense_transformer_runtime.cpp:673, 2296, 3670, 4652).
// It pins the C oracle (zq_oracle.c), is the end-to-end checker of the GGUF
// loader and the device-resident model, and is the CPU baseline in bench.py;
// the HIP product never loads it.
#include "zen/quant.h"
#include "zen/compute_pool.h"
#include "zen/kernels.h"
#include "zen/gguf.h"
#include "zen/dense_transformer_runtime.h"
#include <algorithm>
#include <cstdint>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

namespace {
const zen::quant::Format* fmt_of(int ggml_type) {
    switch (ggml_type) {  // ggml type ids, src/gguf.cpp:370-393
    case 2: return zen::quant::find("Q4_0");
    case 8: return zen::quant::find("Q8_0");
    case 12: return zen::quant::find("Q4_K");
    case 13: return zen::quant::find("Q5_K");
    case 14: return zen::quant::find("Q6_K");
    default: return nullptr;
    }
}
}

extern "C" {
int zr_gemv(int fmt, const std::uint8_t* w, const float* x, float* y, std::size_t rows, std::size_t cols, unsigned workers) {
    const auto* f = fmt_of(fmt); if (!f) return 0;
    return zen::quant::gemv(*f, w, x, y, rows, cols, 1.0f, workers) ? 1 : 0;
}
int zr_gemm(int fmt, const std::uint8_t* w, const float* X, float* Y, std::size_t tokens, std::size_t rows, std::size_t cols, unsigned workers) {
    const auto* f = fmt_of(fmt); if (!f) return 0;
    return zen::quant::gemm(*f, w, X, Y, tokens, rows, cols, 1.0f, workers) ? 1 : 0;
}
int zr_dequantize(int fmt, const std::uint8_t* src, std::size_t n, float* dst) {
    const auto* f = fmt_of(fmt); if (!f) return 0;
    return zen::quant::dequantize(*f, src, n, dst) ? 1 : 0;
}
int zr_decode_fp16(const std::uint16_t* src, float* dst, std::size_t n) { return zen::quant::decode_fp16(src, dst, n) ? 1 : 0; }
int zr_encode_fp16(const float* src, std::uint16_t* dst, std::size_t n) { return zen::quant::encode_fp16(src, dst, n) ? 1 : 0; }
std::size_t zr_row_bytes(int fmt, std::size_t cols) { const auto* f = fmt_of(fmt); return f ? zen::quant::row_bytes(*f, cols) : 0; }
unsigned zr_pool_workers(void) { return zen::ComputePool::instance().worker_count(); }
int zr_has_avx2(void) { return zen::cpu_has_avx2_fma() ? 1 : 0; }

// ---- GGUF parse core ---------------------------------------------------------
// Text description of a parse: "ok=<0|1>\nerror=<msg>\n" then, when ok,
// version, data offset, the llama config fields, every metadata key=value line
// ("M key=value", keys sorted) and one line per tensor
// ("T name type offset bytes d0,d1,...").  Returns the full length; writes at
// most cap bytes (NUL-terminated).
std::size_t zr_gguf_describe(const std::uint8_t* data, std::size_t size, int q8_1_layout, char* out, std::size_t cap) {
    zen::gguf::InspectOptions opt;
    opt.q8_1_layout = q8_1_layout == 1 ? zen::gguf::Q8_1Layout::fp16_36
                    : q8_1_layout == 2 ? zen::gguf::Q8_1Layout::fp32_40 : zen::gguf::Q8_1Layout::unspecified;
    const auto r = zen::gguf::inspect_bytes(data, size, opt);
    std::ostringstream o;
    o << "ok=" << (r.ok ? 1 : 0) << "\nerror=" << r.error << "\n";
    if (r.ok) {
        const auto& c = r.config;
        o << "version=" << r.version << "\ndata_offset=" << r.tensor_data_offset << "\n";
        o << "architecture=" << c.architecture_name << "\nname=" << c.model_name << "\n";
        o << "embedding_length=" << c.embedding_length << "\nblock_count=" << c.block_count
          << "\nhead_count=" << c.attention_head_count << "\nhead_count_kv=" << c.kv_head_count
          << "\nfeed_forward_length=" << c.feed_forward_length << "\ncontext_length=" << c.context_length
          << "\nvocabulary_size=" << c.vocabulary_size << "\nbos=" << c.bos_token_id << "\neos=" << c.eos_token_id << "\n";
        std::vector<std::string> keys;
        for (const auto& kv : c.metadata) keys.push_back(kv.first);
        std::sort(keys.begin(), keys.end());
        for (const auto& k : keys) o << "M " << k << "=" << c.metadata.at(k) << "\n";
        for (const auto& t : r.tensors) {
            o << "T " << t.name << " " << t.ggml_type << " " << t.offset << " " << t.byte_size << " ";
            for (std::size_t i = 0; i < t.dimensions.size(); ++i) o << (i ? "," : "") << t.dimensions[i];
            o << "\n";
        }
    }
    const std::string s = o.str();
    if (out && cap) {
        const std::size_t n = std::min(cap - 1, s.size());
        std::memcpy(out, s.data(), n);
        out[n] = 0;
    }
    return s.size();
}

// ---- dense transformer runtime -------------------------------------------------
struct ZrModel {
    zen::runtime::DenseTransformerRuntime rt;
    std::vector<std::vector<float>> kc, vc;
};
void* zr_model_load(const char* path, char* err, std::size_t cap) {
    auto m = std::make_unique<ZrModel>();
    std::string e;
    if (!m->rt.load(path, &e)) {
        if (err && cap) std::snprintf(err, cap, "%s", e.c_str());
        return nullptr;
    }
    return m.release();
}
void zr_model_free(void* h) { delete static_cast<ZrModel*>(h); }
// embedding, layers, heads, kv_heads, head_dim, ffn, vocab, context, eos
int zr_model_config(void* h, std::uint32_t* out9) {
    const auto& c = static_cast<ZrModel*>(h)->rt.config();
    const std::uint32_t v[9] = {c.embedding, c.layers, c.heads, c.kv_heads, c.head_dim, c.ffn, c.vocab, c.context, c.eos_token};
    std::memcpy(out9, v, sizeof(v));
    return 1;
}
// Prefill `n` tokens from position 0 (forward_batch) into fresh KV caches sized
// for `capacity` positions; logits of the last token into `logits` (vocab floats).
int zr_model_prefill(void* h, const std::uint32_t* tokens, std::size_t n, std::size_t capacity, float* logits) {
    auto* m = static_cast<ZrModel*>(h);
    const auto& c = m->rt.config();
    const std::size_t kv = std::size_t(c.kv_heads) * c.head_dim * capacity;
    m->kc.assign(c.layers, std::vector<float>(kv));
    m->vc.assign(c.layers, std::vector<float>(kv));
    std::vector<std::uint32_t> t(tokens, tokens + n);
    std::vector<float> l;
    if (!m->rt.forward_batch(t, m->kc, m->vc, l)) return 0;
    std::memcpy(logits, l.data(), l.size() * sizeof(float));
    return 1;
}
// One decode step (forward) at `pos` with the caches of the last prefill.
int zr_model_step(void* h, std::uint32_t token, std::uint32_t pos, float* logits) {
    auto* m = static_cast<ZrModel*>(h);
    std::vector<float> l;
    if (!m->rt.forward(token, pos, m->kc, m->vc, l)) return 0;
    std::memcpy(logits, l.data(), l.size() * sizeof(float));
    return 1;
}
// Greedy generate (temperature 0): token ids into out (max_new), count into *n_out.
int zr_model_generate(void* h, const std::uint32_t* prompt, std::size_t n, std::uint32_t max_new,
                      std::uint32_t* out, std::size_t* n_out, double* prefill_ms, double* decode_ms) {
    auto* m = static_cast<ZrModel*>(h);
    zen::runtime::Generation g;
    zen::runtime::GenerationOptions o;
    o.temperature = 0.0f;
    o.seed = 1;
    std::string e;
    if (!m->rt.generate(std::vector<std::uint32_t>(prompt, prompt + n), max_new, g, &e, {}, o)) return 0;
    std::memcpy(out, g.token_ids.data(), g.token_ids.size() * sizeof(std::uint32_t));
    *n_out = g.token_ids.size();
    if (prefill_ms) *prefill_ms = g.prefill_ms;
    if (decode_ms) *decode_ms = g.decode_ms;
    return 1;
}
}
