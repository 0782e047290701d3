// zq_gguf.cpp -- memory-mapped GGUF v2/v3 parser behind include/zq_gguf.h.
//
// Behaviour restated from the reference's parse core (src/gguf.cpp:13-350):
// the same header / metadata / tensor-directory walk, the same safety limits
// (directory counts <= 1e6, strings <= 2^24 bytes, arrays <= 2^32 elements,
// metadata nesting <= 64, 1..4 dimensions, overflow-checked element counts,
// GGML blocks row-local on dims[0], payloads inside the file), the same rule
// that config fields only take values that fit 32 bits, the same textual
// metadata map and the same error strings, so a caller sees the reference's
// decisions.  The file is mapped read-only (MAP_PRIVATE) instead of streamed:
// tensor payloads are then addressable in place and go to HBM in one copy.
#include "../../include/zq_gguf.h"
#include "../../include/zq_hip.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <new>
#include <string>
#include <vector>

namespace {

// Metadata value types (GGUF spec; src/gguf.cpp:21).
enum : uint32_t { M_U8 = 0, M_I8, M_U16, M_I16, M_U32, M_I32, M_F32, M_BOOL, M_STRING, M_ARRAY, M_U64, M_I64, M_F64 };
constexpr unsigned kMaxDepth = 64;

// Bounded little-endian cursor over the image.
struct Cursor {
    const uint8_t* p;
    uint64_t size, off = 0;
    template <class T>
    bool get(T& v) {
        if (size - off < sizeof(T)) return false;
        std::memcpy(&v, p + off, sizeof(T));
        off += sizeof(T);
        return true;
    }
    bool skip(uint64_t n) {
        if (size - off < n) return false;
        off += n;
        return true;
    }
    bool str(std::string& s) {
        uint64_t n;
        if (!get(n) || n > (uint64_t(1) << 24) || size - off < n) return false;
        s.assign(reinterpret_cast<const char*>(p + off), size_t(n));
        off += n;
        return true;
    }
};

// Storage size of `elements` of GGML type `type`; 0 when the type is unknown
// or the count does not divide into its blocks.  The (id, block elements,
// block bytes) table is the canonical GGML one (ggml type ids and block
// sizes, as listed in src/gguf.cpp:64-73).
uint64_t type_bytes(uint32_t type, uint64_t elements, int q81) {
    if (type == 9 && q81 == ZQ_GGUF_Q8_1_FP32_40) {
        if (elements % 32 || elements / 32 > std::numeric_limits<uint64_t>::max() / 40) return 0;
        return elements / 32 * 40;
    }
    struct T { uint32_t id, block, bytes; };
    static const T table[] = {
        {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
        {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
        {20, 32, 18},   {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
        {26, 1, 4},     {27, 1, 8},     {28, 1, 8},     {29, 256, 56},  {30, 1, 2},     {34, 256, 54},
        {35, 256, 66},  {39, 32, 17},   {40, 64, 36},   {41, 128, 18},  {42, 64, 18},   {43, 1, 1},
        {100, 32, 18},  {101, 32, 17},  {142, 128, 34}, {143, 128, 28}};
    for (const T& t : table)
        if (t.id == type) {
            if (elements % t.block) return 0;
            const uint64_t blocks = elements / t.block;
            if (blocks > std::numeric_limits<uint64_t>::max() / t.bytes) return 0;
            return blocks * t.bytes;
        }
    return 0;
}

// Reads (or skips) one value of type t; `number` receives the raw unsigned
// value (bit pattern for floats, element count for arrays).
bool read_value(Cursor& c, uint32_t t, std::string* s, uint64_t* number, unsigned depth) {
    if (depth > kMaxDepth) return false;
    switch (t) {
    case M_U8: case M_I8: { uint8_t v; if (!c.get(v)) return false; if (number) *number = v; return true; }
    case M_U16: case M_I16: { uint16_t v; if (!c.get(v)) return false; if (number) *number = v; return true; }
    case M_U32: case M_I32: case M_F32: { uint32_t v; if (!c.get(v)) return false; if (number) *number = v; return true; }
    case M_U64: case M_I64: case M_F64: { uint64_t v; if (!c.get(v)) return false; if (number) *number = v; return true; }
    case M_BOOL: { uint8_t v; if (!c.get(v) || v > 1) return false; if (number) *number = v; return true; }
    case M_STRING: { std::string v; if (!c.str(v)) return false; if (s) *s = std::move(v); return true; }
    case M_ARRAY: {
        uint32_t sub; uint64_t n;
        if (!c.get(sub) || !c.get(n) || n > (uint64_t(1) << 32)) return false;
        if (number) *number = n;
        for (uint64_t i = 0; i < n; ++i)
            if (!read_value(c, sub, nullptr, nullptr, depth + 1)) return false;
        return true;
    }
    default: return false;
    }
}

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

// Architectures whose "<arch>.<field>" keys shape the config (src/gguf.cpp:205-236).
const char* const kArchPrefixes[] = {
    "llama", "qwen2", "qwen3", "qwen2moe", "qwen3moe", "bitnet", "qwen35", "lfm2moe", "laguna", "nemotron_h",
    "nemotron_h_moe", "dflash", "olmoe", "qwen35moe", "gemma4", "phi3", "deepseek2", "starcoder2", "k2-horizon",
    "gpt-oss", "spark2_5", "mistral3", "llada-moe", "mellum", "muse-glimmer", "qwen3vl", "flint"};

}  // namespace

struct zq_gguf {
    void* map = nullptr;
    size_t map_len = 0;
    const uint8_t* image = nullptr;
    uint64_t size = 0;
    zq_gguf_config cfg{};
    std::map<std::string, std::string> meta;
    std::vector<std::string> meta_keys;
    struct T {
        std::string name;
        std::vector<uint64_t> dims;
        uint32_t type;
        uint64_t offset, bytes;
    };
    std::vector<T> tensors;
    ~zq_gguf() {
        if (map) munmap(map, map_len);
    }
};

namespace {

// The parse core.  Returns an empty string on success, else the error text.
std::string parse(zq_gguf& g, int q81) {
    if (q81 == ZQ_GGUF_Q8_1_UNSPECIFIED) {
        if (const char* e = std::getenv("ZEN_GGUF_Q8_1_LAYOUT")) {
            if (std::strcmp(e, "fp16") == 0) q81 = ZQ_GGUF_Q8_1_FP16_36;
            else if (std::strcmp(e, "fp32") == 0) q81 = ZQ_GGUF_Q8_1_FP32_40;
        }
    }
    Cursor c{g.image, g.size};
    zq_gguf_config& cfg = g.cfg;
    cfg.bos_token_id = 1;
    cfg.eos_token_id = 2;
    cfg.file_size = g.size;
    char magic[4];
    if (g.size < 4 || (std::memcpy(magic, g.image, 4), std::memcmp(magic, "GGUF", 4) != 0)) return "Invalid GGUF magic";
    c.off = 4;
    uint64_t n_tensors = 0, n_meta = 0;
    if (!c.get(cfg.version) || cfg.version < 2 || cfg.version > 3 || !c.get(n_tensors) || !c.get(n_meta))
        return "Unsupported or truncated GGUF header (supports v2/v3)";
    if (n_tensors > 1000000 || n_meta > 1000000) return "GGUF directory count exceeds safety limit";

    std::vector<std::string> hadamard_names, hadamard_inverse;
    uint32_t hadamard_version = 0;
    std::string hadamard_transform, hadamard_axis, hadamard_sign_mode;
    std::string arch, name;

    for (uint64_t i = 0; i < n_meta; ++i) {
        std::string key, value;
        uint32_t type;
        if (!c.str(key) || !c.get(type)) return "Truncated metadata key";
        uint64_t number = 0;
        const bool is_array = type == M_ARRAY;
        auto array_head = [&](uint32_t& sub, uint64_t& count) { return c.get(sub) && c.get(count); };
        if (is_array && (key == "prism.hadamard.weight_names" || key == "prism.hadamard.inverse_weight_names")) {
            uint32_t sub; uint64_t count;
            if (!array_head(sub, count) || count > 100000) return "Invalid hadamard metadata array: " + key;
            if (sub != M_STRING) return "Hadamard name array is not a string array";
            auto& dst = key == "prism.hadamard.weight_names" ? hadamard_names : hadamard_inverse;
            for (uint64_t j = 0; j < count; ++j) {
                std::string t;
                if (!c.str(t)) return "Truncated hadamard name array";
                dst.push_back(std::move(t));
            }
            continue;
        }
        if (is_array && (key == "prism.hadamard.sign_widths" || key == "prism.hadamard.sign_values")) {
            uint32_t sub; uint64_t count;
            if (!array_head(sub, count) || count > 10000000) return "Invalid hadamard metadata array: " + key;
            if (sub != M_I32 && sub != M_U32) return "Hadamard numeric array is not 32-bit integer";
            for (uint64_t j = 0; j < count; ++j) {
                uint32_t v;
                if (!c.get(v)) return "Truncated hadamard numeric array";
            }
            continue;
        }
        if (is_array && key.size() > 23 && ends_with(key, "rope.dimension_sections")) {
            uint32_t sub; uint64_t count;
            if (!array_head(sub, count) || count > 4) return "Invalid rope dimension_sections array";
            for (uint64_t j = 0; j < count; ++j) {
                uint32_t v;
                if (!c.get(v)) return "Truncated rope dimension_sections";
            }
            continue;
        }
        if (is_array && (ends_with(key, ".attention.sliding_window_pattern") || ends_with(key, ".attention.rope_pattern"))) {
            const bool swa = ends_with(key, ".attention.sliding_window_pattern");
            uint32_t sub; uint64_t count;
            if (!array_head(sub, count) || count > 100000)
                return (swa ? "Invalid sliding-window pattern array: " : "Invalid rope pattern array: ") + key;
            if (sub != M_BOOL && sub != M_U32 && sub != M_I32)
                return (swa ? "Sliding-window pattern array is not BOOL: " : "Rope pattern array is not BOOL: ") + key;
            for (uint64_t j = 0; j < count; ++j) {
                bool okv;
                if (sub == M_BOOL) { uint8_t b; okv = c.get(b); } else { uint32_t v; okv = c.get(v); }
                if (!okv) return swa ? "Truncated sliding-window pattern array" : "Truncated rope pattern array";
            }
            continue;
        }
        if (is_array && (ends_with(key, ".feed_forward_length") || ends_with(key, ".attention.head_count_kv") ||
                         ends_with(key, ".attention.head_count"))) {
            uint32_t sub; uint64_t count;
            if (!array_head(sub, count) || count > 100000) return "Invalid per-layer metadata array: " + key;
            if (sub != M_U32 && sub != M_I32) return "Per-layer metadata array is not U32/I32: " + key;
            for (uint64_t j = 0; j < count; ++j) {
                uint32_t v;
                if (!c.get(v)) return "Truncated per-layer metadata array";
            }
            continue;
        }
        if (is_array && (key == "tokenizer.ggml.tokens" || key == "tokenizer.ggml.scores" || key == "tokenizer.ggml.token_type")) {
            uint32_t sub; uint64_t count;
            if (!array_head(sub, count) || count > 1000000) return "Invalid tokenizer metadata array: " + key;
            number = count;
            if (key == "tokenizer.ggml.tokens") {
                if (sub != M_STRING) return "Tokenizer tokens array is not a string array";
                for (uint64_t j = 0; j < count; ++j) {
                    std::string t;
                    if (!c.str(t)) return "Truncated tokenizer token array";
                }
                cfg.vocabulary_size = uint32_t(count);
            } else if (key == "tokenizer.ggml.scores") {
                if (sub != M_F32 && sub != M_I32 && sub != M_U32) return "Tokenizer scores array is not a 32-bit numeric array";
                for (uint64_t j = 0; j < count; ++j) {
                    uint32_t v;
                    if (!c.get(v)) return "Truncated tokenizer scores array";
                }
            } else {
                if (sub != M_I32 && sub != M_U32) return "Tokenizer token_type array is not 32-bit integer";
                for (uint64_t j = 0; j < count; ++j) {
                    uint32_t v;
                    if (!c.get(v)) return "Truncated tokenizer token_type array";
                }
            }
        } else if (!read_value(c, type, &value, &number, 0)) {
            return "Unsupported or truncated metadata value: " + key;
        }
        // textual metadata map (src/gguf.cpp:201-204)
        char buf[512];
        if (type == M_STRING) g.meta[key] = value;
        else if (type == M_F32) {
            float f; const uint32_t bits = uint32_t(number); std::memcpy(&f, &bits, 4);
            std::snprintf(buf, sizeof(buf), "%f", f); g.meta[key] = buf;
        } else if (type == M_F64) {
            double d; std::memcpy(&d, &number, 8);
            std::snprintf(buf, sizeof(buf), "%f", d); g.meta[key] = buf;
        } else if (type != M_ARRAY) {
            std::snprintf(buf, sizeof(buf), "%llu", (unsigned long long)number); g.meta[key] = buf;
        }
        // config fields: only values that fit 32 bits are applied
        auto set = [&](const std::string& k, uint32_t& dst) {
            if (key == k && number <= std::numeric_limits<uint32_t>::max()) dst = uint32_t(number);
        };
        const size_t dot = key.find('.');
        if (dot != std::string::npos) {
            const std::string prefix = key.substr(0, dot);
            for (const char* p : kArchPrefixes)
                if (prefix == p) {
                    const std::string pr = prefix + ".";
                    set(pr + "embedding_length", cfg.embedding_length);
                    set(pr + "block_count", cfg.block_count);
                    set(pr + "attention.head_count", cfg.head_count);
                    set(pr + "attention.head_count_kv", cfg.head_count_kv);
                    set(pr + "feed_forward_length", cfg.feed_forward_length);
                    set(pr + "context_length", cfg.context_length);
                    break;
                }
        }
        if (key == "prism.hadamard.version" && type != M_ARRAY) hadamard_version = uint32_t(number);
        if (type == M_STRING) {
            if (key == "prism.hadamard.transform") hadamard_transform = value;
            if (key == "prism.hadamard.axis") hadamard_axis = value;
            if (key == "prism.hadamard.sign_mode") hadamard_sign_mode = value;
            if (key == "general.architecture") arch = value;
            if (key == "general.name") name = value;
        }
        set("tokenizer.ggml.bos_token_id", cfg.bos_token_id);
        set("tokenizer.ggml.eos_token_id", cfg.eos_token_id);
    }

    g.tensors.reserve(size_t(n_tensors));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        zq_gguf::T t;
        uint32_t nd;
        if (!c.str(t.name) || !c.get(nd) || nd == 0 || nd > 4) return "Invalid tensor descriptor";
        t.dims.resize(nd);
        uint64_t elements = 1;
        for (auto& d : t.dims) {
            if (!c.get(d) || d == 0 || elements > std::numeric_limits<uint64_t>::max() / d) return "Invalid tensor dimensions";
            elements *= d;
        }
        if (!c.get(t.type) || !c.get(t.offset)) return "Truncated tensor descriptor";
        if (t.type == 9 && q81 != ZQ_GGUF_Q8_1_FP16_36 && q81 != ZQ_GGUF_Q8_1_FP32_40)
            return "Q8_1 layout is ambiguous (36-byte fp16 or 40-byte fp32): explicitly set ZEN_GGUF_Q8_1_LAYOUT=fp16 or "
                   "fp32 after verifying the file, or use InspectOptions";
        // blocks are row-local: dims[0] alone must divide into blocks
        t.bytes = type_bytes(t.type, t.dims[0], q81) ? type_bytes(t.type, elements, q81) : 0;
        g.tensors.push_back(std::move(t));
    }
    uint32_t alignment = 32;
    auto it = g.meta.find("general.alignment");
    if (it != g.meta.end()) {
        // std::stoul semantics: strtoul, a conversion must happen and fit unsigned long
        const char* s = it->second.c_str();
        char* end = nullptr;
        errno = 0;
        const unsigned long v = std::strtoul(s, &end, 10);
        if (end != s && errno != ERANGE) alignment = uint32_t(v);
    }
    if (alignment == 0 || (alignment & (alignment - 1)) != 0) return "Invalid GGUF tensor alignment";
    cfg.data_offset = (c.off + alignment - 1) & ~uint64_t(alignment - 1);
    if (cfg.data_offset > g.size) return "GGUF tensor-data offset exceeds file size";
    for (const auto& t : g.tensors) {
        if (t.bytes == 0) return "Tensor uses unsupported or invalid GGML type " + std::to_string(t.type) + ": " + t.name;
        if (t.offset > g.size - cfg.data_offset || t.bytes > g.size - cfg.data_offset - t.offset)
            return "Tensor payload exceeds GGUF file bounds: " + t.name;
    }
    if (!hadamard_names.empty() || !hadamard_inverse.empty()) {
        if (hadamard_version != 0 && hadamard_version != 1 && hadamard_version != 2)
            return "Unsupported prism.hadamard.version " + std::to_string(hadamard_version);
        if (!hadamard_transform.empty() && hadamard_transform != "normalized-sylvester-walsh-hadamard")
            return "Unsupported prism.hadamard.transform: " + hadamard_transform;
        if (!hadamard_axis.empty() && hadamard_axis != "input-last-dimension")
            return "Unsupported prism.hadamard.axis: " + hadamard_axis;
        if (!hadamard_sign_mode.empty() && hadamard_sign_mode != "explicit" && hadamard_sign_mode != "identity")
            return "Unsupported prism.hadamard.sign_mode: " + hadamard_sign_mode;
    } else {
        for (const auto& t : g.tensors)
            if (t.type == 143 || t.type == 142)
                return "Tensor " + t.name + " uses Prism ternary type " + std::to_string(t.type) +
                       " but the file carries no prism.hadamard.* contract; its weights would be read in the wrong basis";
    }
    std::snprintf(cfg.architecture, sizeof(cfg.architecture), "%s", arch.c_str());
    std::snprintf(cfg.name, sizeof(cfg.name), "%s", name.c_str());
    g.meta_keys.reserve(g.meta.size());
    for (const auto& kv : g.meta) g.meta_keys.push_back(kv.first);
    return {};
}

int finish(zq_gguf* g, int q81, zq_gguf** out, char* err, size_t cap) {
    const std::string e = parse(*g, q81);
    if (!e.empty()) {
        if (err && cap) std::snprintf(err, cap, "%s", e.c_str());
        delete g;
        return ZQ_ERR_ARG;
    }
    if (err && cap) err[0] = 0;
    *out = g;
    return ZQ_OK;
}

void put_err(char* err, size_t cap, const char* msg) {
    if (err && cap) std::snprintf(err, cap, "%s", msg);
}

}  // namespace

extern "C" {

int zq_gguf_open(const char* path, int q8_1_layout, zq_gguf** out, char* err, size_t err_cap) {
    if (!path || !out) return ZQ_ERR_ARG;
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) { put_err(err, err_cap, "Cannot open GGUF file"); return ZQ_ERR_ARG; }
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); put_err(err, err_cap, "Cannot determine GGUF file size"); return ZQ_ERR_ARG; }
    zq_gguf* g = new (std::nothrow) zq_gguf;
    if (!g) { ::close(fd); return ZQ_ERR_OOM; }
    static const uint8_t empty = 0;
    g->size = uint64_t(st.st_size);
    g->image = &empty;
    if (st.st_size > 0) {
        void* m = mmap(nullptr, size_t(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) { ::close(fd); delete g; put_err(err, err_cap, "Cannot open GGUF file"); return ZQ_ERR_ARG; }
        g->map = m;
        g->map_len = size_t(st.st_size);
        g->image = static_cast<const uint8_t*>(m);
    }
    ::close(fd);
    return finish(g, q8_1_layout, out, err, err_cap);
}

int zq_gguf_open_bytes(const uint8_t* data, size_t size, int q8_1_layout, zq_gguf** out, char* err, size_t err_cap) {
    if (!out) return ZQ_ERR_ARG;
    *out = nullptr;
    zq_gguf* g = new (std::nothrow) zq_gguf;
    if (!g) return ZQ_ERR_OOM;
    static const uint8_t empty = 0;
    g->image = data ? data : &empty;
    g->size = data ? size : 0;
    return finish(g, q8_1_layout, out, err, err_cap);
}

void zq_gguf_close(zq_gguf* g) { delete g; }

int zq_gguf_get_config(const zq_gguf* g, zq_gguf_config* out) {
    if (!g || !out) return ZQ_ERR_ARG;
    *out = g->cfg;
    return ZQ_OK;
}

size_t zq_gguf_tensor_count(const zq_gguf* g) { return g ? g->tensors.size() : 0; }

static void fill(const zq_gguf* g, const zq_gguf::T& t, zq_gguf_tensor* out) {
    out->name = t.name.c_str();
    out->n_dims = uint32_t(t.dims.size());
    for (int i = 0; i < 4; ++i) out->dims[i] = i < int(t.dims.size()) ? t.dims[i] : 1;
    out->ggml_type = t.type;
    out->offset = t.offset;
    out->byte_size = t.bytes;
    out->data = g->image + g->cfg.data_offset + t.offset;
}

int zq_gguf_get_tensor(const zq_gguf* g, size_t index, zq_gguf_tensor* out) {
    if (!g || !out || index >= g->tensors.size()) return ZQ_ERR_ARG;
    fill(g, g->tensors[index], out);
    return ZQ_OK;
}

int zq_gguf_find_tensor(const zq_gguf* g, const char* name, zq_gguf_tensor* out) {
    if (!g || !name || !out) return ZQ_ERR_ARG;
    for (const auto& t : g->tensors)
        if (t.name == name) {
            fill(g, t, out);
            return ZQ_OK;
        }
    return ZQ_DECLINED;
}

size_t zq_gguf_meta_count(const zq_gguf* g) { return g ? g->meta_keys.size() : 0; }

const char* zq_gguf_meta_key(const zq_gguf* g, size_t index) {
    return g && index < g->meta_keys.size() ? g->meta_keys[index].c_str() : nullptr;
}

const char* zq_gguf_meta_value(const zq_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : it->second.c_str();
}

}  // extern "C"
