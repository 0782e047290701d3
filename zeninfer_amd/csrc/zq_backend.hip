// zq_backend.hip -- the C-ABI runtime: device init, weight residency in HBM,
// activation staging, stream handling and statistics.  Kernels live in
// zq_gemv.hip, zq_gemm.hip and zq_misc.hip.
//
// Residency: a weight tensor is uploaded once, byte-for-byte in its GGML
// block layout (no repack), into one hipMalloc allocation of
// rows*row_bytes + ZQ_WEIGHT_TAIL_PAD bytes, and stays there until released,
// evicted or shutdown.  The key is the host pointer; the entry also records
// (format, rows, cols) and a different shape at the same address re-uploads
// (reference contract, include/zen/hip_backend.h:52-58).  When the budget
// (80% of device memory, as hip_backend.hip:459-475) would be exceeded,
// every resident tensor is evicted first; a call that reads several weights
// is declined when they cannot be resident together.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_map>
#include <vector>

#include "../../include/zq_hip.h"
#include "zq_internal.hpp"

// Fixed device scratch of zq_hip_gemm_dev_noalloc: the int8 activations,
// their scales and the split-K partial sums of one GEMM, for callers that
// cannot allocate.  Every GPU the library runs on holds its own copy until
// the process ends.  Host code never uses the array's name as an address:
// its device address is looked up per device (scratch_ptr) and passed on.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

using Clock = std::chrono::steady_clock;
uint64_t us_since(Clock::time_point t0) {
    return static_cast<uint64_t>(std::chrono::duration_cast<std::chrono::microseconds>(Clock::now() - t0).count());
}

struct Resident {
    int fmt;
    size_t rows, cols, bytes;
    uint8_t* dev;
};

struct Backend {
    std::mutex mu;
    bool initialised = false;
    bool failed = false;
    int device = 0;
    zq_hip_info info{};
    zq_hip_stats stats{};
    hipStream_t stream = nullptr;
    size_t budget = 0;
    uint64_t frees = 0;  // bumped whenever a resident copy is freed
    size_t min_elements = 262144;
    std::unordered_map<const uint8_t*, Resident> resident;
    // staging
    void* dev_scratch = nullptr;  // activations in, outputs out, int8 workspace
    size_t dev_scratch_bytes = 0;
    void* host_pinned = nullptr;
    size_t host_pinned_bytes = 0;
    // ZEN_HIP_TRACE=1: events around each host call's kernels feed gpu_us
    // (hip_backend.hip:549-565, 889-891)
    bool trace = false;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
};

Backend& B() {
    static Backend b;
    return b;
}

// Device address of `scratch` on the current device, looked up once per
// device with that device current (each GPU holds its own copy).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

void* scratch_ptr() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

// Status of a launcher's result: hipErrorInvalidValue is its refusal of the
// arguments (a misaligned operand, a shape its kernels cannot take), any
// other error a HIP failure.
int launch_status(hipError_t e) {
    return e == hipSuccess ? ZQ_OK : e == hipErrorInvalidValue ? ZQ_ERR_ARG : ZQ_ERR_HIP;
}

int fail_hip(Backend& b) {
    ++b.stats.errors;
    return ZQ_ERR_HIP;
}

bool env_opted_in() {
    const char* be = std::getenv("ZEN_BACKEND");
    if (be && (!std::strcmp(be, "hip") || !std::strcmp(be, "rocm") || !std::strcmp(be, "amd"))) return true;
    const char* h = std::getenv("ZEN_HIP");
    return h && h[0] == '1';
}

int init_locked(Backend& b) {
    if (b.initialised) return ZQ_OK;
    if (b.failed) return ZQ_ERR_NO_DEVICE;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
        b.failed = true;
        return ZQ_ERR_NO_DEVICE;
    }
    const char* dv = std::getenv("ZEN_HIP_DEVICE");
    b.device = dv ? std::atoi(dv) : 0;
    if (b.device < 0 || b.device >= count || hipSetDevice(b.device) != hipSuccess) {
        b.failed = true;
        return ZQ_ERR_NO_DEVICE;
    }
    hipDeviceProp_t p{};
    if (hipGetDeviceProperties(&p, b.device) != hipSuccess) {
        b.failed = true;
        return ZQ_ERR_NO_DEVICE;
    }
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) {  // code objects are built for gfx950 only
        b.failed = true;
        return ZQ_ERR_NO_DEVICE;
    }
    std::snprintf(b.info.name, sizeof(b.info.name), "%s", p.name);
    std::snprintf(b.info.arch, sizeof(b.info.arch), "%s", p.gcnArchName);
    b.info.vram_bytes = p.totalGlobalMem;
    b.info.compute_units = p.multiProcessorCount;
    b.info.wave_size = p.warpSize;
    b.info.lds_per_block = static_cast<int>(p.sharedMemPerBlock);
    b.info.clock_khz = p.clockRate;
    b.info.mem_clock_khz = p.memoryClockRate;
    b.info.mem_bus_width = p.memoryBusWidth;
    if (hipStreamCreateWithFlags(&b.stream, hipStreamNonBlocking) != hipSuccess) {
        b.failed = true;
        return ZQ_ERR_NO_DEVICE;
    }
    const char* tr = std::getenv("ZEN_HIP_TRACE");
    b.trace = tr && tr[0] == '1';
    if (b.trace && (hipEventCreate(&b.ev0) != hipSuccess || hipEventCreate(&b.ev1) != hipSuccess)) b.trace = false;
    if (!scratch_ptr()) {  // the no-allocation GEMM's scratch on this device
        b.failed = true;
        return ZQ_ERR_NO_DEVICE;
    }
    b.budget = static_cast<size_t>(static_cast<double>(p.totalGlobalMem) * 0.8);
    if (const char* rb = std::getenv("ZQ_HIP_RESIDENT_BUDGET")) {  // bytes; lower only, to rehearse eviction
        const size_t v = std::strtoull(rb, nullptr, 10);
        if (v > 0 && v < b.budget) b.budget = v;
    }
    if (const char* me = std::getenv("ZEN_HIP_MIN_ELEMENTS")) b.min_elements = std::strtoull(me, nullptr, 10);
    b.initialised = true;
    return ZQ_OK;
}

void free_resident(Backend& b) {
    if (!b.resident.empty()) ++b.frees;
    for (auto& kv : b.resident) (void)hipFree(kv.second.dev);
    b.stats.evictions += b.resident.size();
    b.resident.clear();
    b.stats.resident_bytes = 0;
    b.stats.resident_tensors = 0;
}

// Device copy of a host weight tensor, uploading on first use.
int ensure_resident(Backend& b, int fmt, const uint8_t* w, size_t rows, size_t cols, const uint8_t** out) {
    auto it = b.resident.find(w);
    if (it != b.resident.end()) {
        if (it->second.fmt == fmt && it->second.rows == rows && it->second.cols == cols) {
            *out = it->second.dev;
            return ZQ_OK;
        }
        (void)hipFree(it->second.dev);
        ++b.frees;
        b.stats.resident_bytes -= it->second.bytes;
        --b.stats.resident_tensors;
        b.resident.erase(it);
    }
    const size_t payload = rows * zq::row_bytes(fmt, cols);
    const size_t bytes = payload + ZQ_WEIGHT_TAIL_PAD;
    if (bytes > b.budget) return ZQ_DECLINED;
    if (b.stats.resident_bytes + bytes > b.budget) free_resident(b);
    auto t0 = Clock::now();
    uint8_t* dev = nullptr;
    if (hipMalloc(&dev, bytes) != hipSuccess) {
        free_resident(b);
        if (hipMalloc(&dev, bytes) != hipSuccess) return ZQ_ERR_OOM;
    }
    b.stats.alloc_us += us_since(t0);
    t0 = Clock::now();
    if (hipMemcpy(dev, w, payload, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(dev + payload, 0, ZQ_WEIGHT_TAIL_PAD) != hipSuccess) {
        (void)hipFree(dev);
        return fail_hip(b);
    }
    b.resident.emplace(w, Resident{fmt, rows, cols, bytes, dev});
    b.stats.uploads++;
    b.stats.upload_bytes += payload;
    b.stats.resident_bytes += bytes;
    b.stats.resident_tensors++;
    b.stats.upload_us += us_since(t0);
    *out = dev;
    return ZQ_OK;
}

// Device copies of every weight one call reads, resolved before any launch.
// An upload that would overflow the budget evicts every resident tensor,
// including ones this call resolved a moment earlier, so a pass that freed
// anything is repeated, and the second pass must free nothing.  A set whose
// distinct tensors do not fit the budget together, or one whose second pass
// still frees (an allocation retried after an eviction, one address given
// with two shapes), is declined: launching it would read freed memory.
struct Want {
    const uint8_t* w;
    size_t rows, cols;
};
int resolve_set(Backend& b, int fmt, const Want* want, size_t n, const uint8_t** out) {
    size_t need = 0;
    for (size_t i = 0; i < n; ++i) {
        bool seen = false;
        for (size_t j = 0; j < i; ++j) seen = seen || want[j].w == want[i].w;
        if (!seen) need += want[i].rows * zq::row_bytes(fmt, want[i].cols) + ZQ_WEIGHT_TAIL_PAD;
    }
    if (need > b.budget) {
        ++b.stats.declined;
        return ZQ_DECLINED;
    }
    for (int pass = 0; pass < 2; ++pass) {
        const uint64_t frees = b.frees;
        for (size_t i = 0; i < n; ++i) {
            const int st = ensure_resident(b, fmt, want[i].w, want[i].rows, want[i].cols, &out[i]);
            if (st == ZQ_DECLINED) ++b.stats.declined;
            if (st != ZQ_OK) return st;
        }
        if (b.frees == frees) return ZQ_OK;
    }
    ++b.stats.declined;
    return ZQ_DECLINED;
}

int ensure_scratch(Backend& b, size_t dev_bytes, size_t host_bytes) {
    const auto t0 = Clock::now();
    struct Tally {
        Backend& b;
        Clock::time_point t0;
        ~Tally() { b.stats.alloc_us += us_since(t0); }
    } tally{b, t0};
    if (dev_bytes > b.dev_scratch_bytes) {
        if (b.dev_scratch) (void)hipFree(b.dev_scratch);
        b.dev_scratch = nullptr;
        b.dev_scratch_bytes = 0;
        if (hipMalloc(&b.dev_scratch, dev_bytes) != hipSuccess) return ZQ_ERR_OOM;
        b.dev_scratch_bytes = dev_bytes;
    }
    if (host_bytes > b.host_pinned_bytes) {
        if (b.host_pinned) (void)hipHostFree(b.host_pinned);
        b.host_pinned = nullptr;
        b.host_pinned_bytes = 0;
        if (hipHostMalloc(&b.host_pinned, host_bytes, hipHostMallocDefault) != hipSuccess) return ZQ_ERR_OOM;
        b.host_pinned_bytes = host_bytes;
    }
    return ZQ_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

bool valid_fmt(int fmt) {
    return fmt == ZQ_FMT_Q4_0 || fmt == ZQ_FMT_Q8_0 || fmt == ZQ_FMT_Q4_K || fmt == ZQ_FMT_Q5_K || fmt == ZQ_FMT_Q6_K;
}
// Formats with an int8-activation GEMM (per-32 blocks).  The K-quants keep
// fp32 activations, as every reference route for them does (the CPU
// gemm_q4k/q5k_kblk_avx2 and the D3D12 shaders/q8_0_gemm_q4k.hlsl).
bool int8_fmt(int fmt) { return fmt == ZQ_FMT_Q4_0 || fmt == ZQ_FMT_Q8_0; }

// ZQ_ACT_DEFAULT is fp32 activations for every format, as in the routes the
// drop-in replaces; int8 activations are the caller's explicit choice.
int resolve_act(int fmt, int act_mode) {
    (void)fmt;
    return act_mode == ZQ_ACT_DEFAULT ? ZQ_ACT_F32 : act_mode;
}

// GEMM support check shared by the host and device entry points.
int gemm_supported(int fmt, size_t cols, int act) {
    if (act != ZQ_ACT_INT8 && act != ZQ_ACT_F32) return ZQ_ERR_ARG;
    if (act == ZQ_ACT_INT8 && (!int8_fmt(fmt) || cols % 64)) return ZQ_DECLINED;
    return ZQ_OK;
}

// Enqueue a GEMM whose operands are all on the device.
int enqueue_gemm(int fmt, const uint8_t* w, const float* X, float* Y, size_t tokens, size_t rows, size_t cols, int act,
                 void* ws, size_t ws_bytes, hipStream_t s, uint64_t* dispatches) {
    if (act == ZQ_ACT_INT8) {
        const size_t qbytes = align_up(tokens * cols, 256);
        const size_t sbytes = align_up(tokens * (cols / 32) * sizeof(float), 256);
        const size_t pbytes = zq::gemm_i8_partial_bytes(tokens, rows, cols);
        if (!ws || ws_bytes < qbytes + sbytes + pbytes) return ZQ_ERR_ARG;
        int8_t* xq = static_cast<int8_t*>(ws);
        float* xs = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + qbytes);
        float* part = pbytes ? reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + qbytes + sbytes) : nullptr;
        if (const int ls = launch_status(zq::launch_quantize_acts(X, xq, xs, tokens, cols, s)); ls != ZQ_OK) return ls;
        if (const int ls = launch_status(zq::launch_gemm_i8(fmt, w, xq, xs, Y, part, tokens, rows, cols, s));
            ls != ZQ_OK)
            return ls;
        *dispatches += pbytes ? 3 : 2;
        return ZQ_OK;
    }
    // fp32 activations: the workspace, when large enough, holds the split
    // activations (Q6_K, Q4_K, Q5_K) and split-K partial sums; with less the
    // GEMM runs with what fits
    uint32_t n = 0;
    if (const int ls =
            launch_status(zq::launch_gemm_f32(fmt, w, X, Y, ws, ws ? ws_bytes : 0, tokens, rows, cols, s, &n));
        ls != ZQ_OK)
        return ls;
    *dispatches += n;
    return ZQ_OK;
}

// Workspace of a batched GEMM: the shared int8 activations and scales (int8
// mode), then room for the largest task's split-K partial sums (reused task
// after task on the one stream).
size_t batch_workspace_bytes(int fmt, const size_t* rows, size_t count, size_t tokens, size_t cols, int act) {
    size_t part = 0;
    for (size_t i = 0; i < count; ++i)
        part = std::max(part, act == ZQ_ACT_INT8 ? zq::gemm_i8_partial_bytes(tokens, rows[i], cols)
                                                 : zq::gemm_f32_workspace_bytes(fmt, tokens, rows[i], cols));
    if (act != ZQ_ACT_INT8) return part;
    return align_up(tokens * cols, 256) + align_up(tokens * (cols / 32) * sizeof(float), 256) + part;
}

// Enqueue the GEMMs of tasks sharing X: with int8 activations X is quantised
// once (the reference batches exactly this sharing, src/quant.cpp:1521-1554).
int enqueue_gemm_batch(int fmt, const uint8_t* const* w, float* const* Y, const size_t* rows, size_t count,
                       const float* X, size_t tokens, size_t cols, int act, void* ws, size_t ws_bytes, hipStream_t s,
                       uint64_t* dispatches) {
    if (ws_bytes < batch_workspace_bytes(fmt, rows, count, tokens, cols, act)) return ZQ_ERR_ARG;
    if (act == ZQ_ACT_INT8) {
        if (!ws) return ZQ_ERR_ARG;
        const size_t qbytes = align_up(tokens * cols, 256);
        const size_t sbytes = align_up(tokens * (cols / 32) * sizeof(float), 256);
        int8_t* xq = static_cast<int8_t*>(ws);
        float* xs = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + qbytes);
        float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + qbytes + sbytes);
        if (const int ls = launch_status(zq::launch_quantize_acts(X, xq, xs, tokens, cols, s)); ls != ZQ_OK) return ls;
        ++*dispatches;
        for (size_t i = 0; i < count; ++i) {
            const size_t pb = zq::gemm_i8_partial_bytes(tokens, rows[i], cols);
            if (const int ls = launch_status(
                    zq::launch_gemm_i8(fmt, w[i], xq, xs, Y[i], pb ? part : nullptr, tokens, rows[i], cols, s));
                ls != ZQ_OK)
                return ls;
            *dispatches += pb ? 2 : 1;
        }
        return ZQ_OK;
    }
    for (size_t i = 0; i < count; ++i) {
        uint32_t n = 0;
        if (const int ls = launch_status(
                zq::launch_gemm_f32(fmt, w[i], X, Y[i], ws, ws ? ws_bytes : 0, tokens, rows[i], cols, s, &n));
            ls != ZQ_OK)
            return ls;
        *dispatches += n;
    }
    return ZQ_OK;
}

bool ffn_residual_args_ok(int fmt, const void* wo, const void* wg, const void* wu, const void* wd, const float* norm_w,
                          const float* x, const float* attn_out, const float* out, size_t hidden, size_t attn_width,
                          size_t ffn_rows) {
    return wo && wg && wu && wd && norm_w && x && attn_out && out && hidden && attn_width && ffn_rows &&
           valid_fmt(fmt) && zq::row_bytes(fmt, attn_width) && zq::row_bytes(fmt, hidden) &&
           zq::row_bytes(fmt, ffn_rows) && hidden <= (1u << 24) && attn_width <= (1u << 24) && ffn_rows <= (1u << 24);
}

// The FFN half of a decoder layer, every intermediate on the device
// (d3d12_backend.h:352-364):
//   t0 = Wo . attn_out;  h1 = t0 + x;  h2 = rmsnorm(h1) * norm_w;
//   g = Wg . h2;  u = Wu . h2;  f = silu(g) * u;  d = Wd . f;  out = h1 + d.
// Q8_0 / Q4_0 on the streaming shapes fold the add + norm into the gate|up
// GEMV and silu * up into the down GEMV; Q4_K / Q5_K / Q6_K form silu * up
// in a paired gate|up GEMV; otherwise they run as kernels of their own.  x
// is read before out is written, so out may alias x.
int enqueue_ffn_residual(int fmt, const uint8_t* wo, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                         const float* norm_w, const float* x, const float* attn_out, float* out, size_t hidden,
                         size_t attn_width, size_t ffn_rows, float eps, void* ws, size_t ws_bytes, hipStream_t s,
                         uint64_t* dispatches);

}  // namespace

extern "C" size_t zq_hip_ffn_residual_workspace_bytes(size_t hidden, size_t ffn_rows) {
    if (!hidden || !ffn_rows) return 0;
    return 3 * align_up(hidden * sizeof(float), 256) + 2 * align_up(ffn_rows * sizeof(float), 256);
}

namespace {
int enqueue_ffn_residual(int fmt, const uint8_t* wo, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                         const float* norm_w, const float* x, const float* attn_out, float* out, size_t hidden,
                         size_t attn_width, size_t ffn_rows, float eps, void* ws, size_t ws_bytes, hipStream_t s,
                         uint64_t* dispatches) {
    if (!ws || ws_bytes < zq_hip_ffn_residual_workspace_bytes(hidden, ffn_rows)) return ZQ_ERR_ARG;
    const size_t hb = align_up(hidden * sizeof(float), 256), fb = align_up(ffn_rows * sizeof(float), 256);
    uint8_t* base = static_cast<uint8_t*>(ws);
    float* t0 = reinterpret_cast<float*>(base);
    float* h1 = reinterpret_cast<float*>(base + hb);
    float* d = reinterpret_cast<float*>(base + 2 * hb);
    float* g = reinterpret_cast<float*>(base + 3 * hb);
    float* u = reinterpret_cast<float*>(base + 3 * hb + fb);
    const uint32_t H = uint32_t(hidden), F = uint32_t(ffn_rows);
    zq::GemvTask to{wo, t0, H};
    if (const int ls = launch_status(zq::launch_gemv(fmt, &to, 1, attn_out, attn_width, s)); ls != ZQ_OK) return ls;
    zq::GemvTask gu[2] = {{wg, g, F}, {wu, u, F}};
    const zq::XPrologue norm{zq::kAddNorm, t0, x, norm_w, h1, eps};
    hipError_t e = zq::launch_gemv_prologue(fmt, gu, 2, norm, hidden, s);
    zq::GemvTask dn{wd, d, H};
    bool paired = false;  // g already holds silu(gate) * up
    if (e == hipErrorInvalidConfiguration) {
        // unfused: h1 = t0 + x, h2 = rmsnorm(h1) * w (into d), then gate|up
        // of h2 -- as one paired GEMV storing silu(gate) * up into g where the
        // format takes it (Q4_K / Q5_K / Q6_K), else as a 2-task GEMV
        if (zq::launch_add_to(t0, x, h1, hidden, s) != hipSuccess ||
            zq::launch_rmsnorm(h1, norm_w, d, 1, H, eps, s) != hipSuccess)
            return ZQ_ERR_HIP;
        *dispatches += 2;
        const hipError_t pe = zq::launch_gemv_silu_pair(fmt, gu[0], gu[1], d, hidden, s);
        if (pe != hipSuccess && pe != hipErrorInvalidConfiguration) return ZQ_ERR_HIP;
        paired = pe == hipSuccess;
        if (!paired && zq::launch_gemv(fmt, gu, 2, d, hidden, s) != hipSuccess) return ZQ_ERR_HIP;
        ++*dispatches;
    } else if (e != hipSuccess) {
        return ZQ_ERR_HIP;
    } else {
        ++*dispatches;
    }
    const zq::XPrologue act{zq::kSiluMul, g, u, nullptr, nullptr, 0.0f};
    e = paired ? hipErrorInvalidConfiguration : zq::launch_gemv_prologue(fmt, &dn, 1, act, ffn_rows, s);
    if (paired) {
        if (zq::launch_gemv(fmt, &dn, 1, g, ffn_rows, s) != hipSuccess) return ZQ_ERR_HIP;
        ++*dispatches;
    } else if (e == hipErrorInvalidConfiguration) {
        if (zq::launch_silu_mul(g, u, g, ffn_rows, s) != hipSuccess || zq::launch_gemv(fmt, &dn, 1, g, ffn_rows, s) != hipSuccess)
            return ZQ_ERR_HIP;
        *dispatches += 2;
    } else if (e != hipSuccess) {
        return ZQ_ERR_HIP;
    } else {
        ++*dispatches;
    }
    if (const int ls = launch_status(zq::launch_add_to(h1, d, out, hidden, s)); ls != ZQ_OK) return ls;
    *dispatches += 2;
    return ZQ_OK;
}

// Accounting of one synchronous host-pointer call, as zen::hip keeps it
// (hip_backend.hip:549-565, 597-607): inputs staged through pinned memory
// (transfer_us), kernel enqueue (launch_us), the stream wait (wait_us; the
// kernels' event time in gpu_us when tracing), then the read-back
// (readback_us, also counted in transfer_us).
struct HostCall {
    Backend& b;
    Clock::time_point t_launch{};
    explicit HostCall(Backend& bb) : b(bb) {}
    int put(void* dev, const void* src, size_t bytes) {
        const auto t0 = Clock::now();
        std::memcpy(b.host_pinned, src, bytes);
        const hipError_t e = hipMemcpyAsync(dev, b.host_pinned, bytes, hipMemcpyHostToDevice, b.stream);
        // the staging buffer is reused by the next put: wait for this copy
        const hipError_t w = e == hipSuccess ? hipStreamSynchronize(b.stream) : e;
        b.stats.transfer_us += us_since(t0);
        return w == hipSuccess ? ZQ_OK : fail_hip(b);
    }
    void begin() {
        t_launch = Clock::now();
        if (b.trace) (void)hipEventRecord(b.ev0, b.stream);
    }
    void launched(uint64_t n) {
        b.stats.dispatches += n;
        b.stats.launch_us += us_since(t_launch);
    }
    int end() {
        if (b.trace) (void)hipEventRecord(b.ev1, b.stream);
        const auto t0 = Clock::now();
        if (hipStreamSynchronize(b.stream) != hipSuccess) return fail_hip(b);
        b.stats.wait_us += us_since(t0);
        if (b.trace) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, b.ev0, b.ev1) == hipSuccess && ms > 0.0f)
                b.stats.gpu_us += static_cast<uint64_t>(ms * 1000.0f);
        }
        ++b.stats.submits;
        return ZQ_OK;
    }
    int get(void* dst, const void* dev, size_t bytes) {
        const auto t0 = Clock::now();
        if (hipMemcpyAsync(b.host_pinned, dev, bytes, hipMemcpyDeviceToHost, b.stream) != hipSuccess ||
            hipStreamSynchronize(b.stream) != hipSuccess)
            return fail_hip(b);
        std::memcpy(dst, b.host_pinned, bytes);
        const uint64_t us = us_since(t0);
        b.stats.readback_us += us;
        b.stats.transfer_us += us;
        return ZQ_OK;
    }
};

}  // namespace

extern "C" {

int zq_hip_opted_in(void) { return env_opted_in() ? 1 : 0; }

int zq_hip_init(void) {
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    return init_locked(b);
}

int zq_hip_enabled(void) {
    if (!env_opted_in()) return 0;
    return zq_hip_init() == ZQ_OK ? 1 : 0;
}

void zq_hip_shutdown(void) {
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    if (b.initialised) {
        (void)hipStreamSynchronize(b.stream);
        free_resident(b);
        if (b.dev_scratch) (void)hipFree(b.dev_scratch);
        if (b.host_pinned) (void)hipHostFree(b.host_pinned);
        if (b.ev0) (void)hipEventDestroy(b.ev0);
        if (b.ev1) (void)hipEventDestroy(b.ev1);
        (void)hipStreamDestroy(b.stream);
    }
    b.ev0 = b.ev1 = nullptr;
    b.trace = false;
    b.dev_scratch = nullptr;
    b.dev_scratch_bytes = 0;
    b.host_pinned = nullptr;
    b.host_pinned_bytes = 0;
    b.stream = nullptr;
    b.initialised = false;
    b.failed = false;
}

int zq_hip_get_info(zq_hip_info* out) {
    if (!out) return ZQ_ERR_ARG;
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    const int st = init_locked(b);
    if (st != ZQ_OK) return st;
    *out = b.info;
    return ZQ_OK;
}

int zq_hip_get_stats(zq_hip_stats* out) {
    if (!out) return ZQ_ERR_ARG;
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    *out = b.stats;
    return ZQ_OK;
}

void zq_hip_reset_stats(void) {
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    const uint64_t rb = b.stats.resident_bytes, rt = b.stats.resident_tensors;
    b.stats = zq_hip_stats{};
    b.stats.resident_bytes = rb;
    b.stats.resident_tensors = rt;
}

const char* zq_hip_status_string(int status) {
    switch (status) {
    case ZQ_OK: return "ok";
    case ZQ_DECLINED: return "declined";
    case ZQ_ERR_ARG: return "invalid argument";
    case ZQ_ERR_NO_DEVICE: return "no usable gfx950 device";
    case ZQ_ERR_OOM: return "out of memory";
    case ZQ_ERR_HIP: return "HIP runtime error";
    case ZQ_ERR_TOO_LARGE: return "request exceeds the fixed no-allocation scratch (zq_hip_noalloc_scratch_bytes)";
    default: return "unknown status";
    }
}

size_t zq_row_bytes(int fmt, size_t cols) { return zq::row_bytes(fmt, cols); }

size_t zq_weight_bytes(int fmt, size_t rows, size_t cols) {
    const size_t rb = zq::row_bytes(fmt, cols);
    return rb && rows ? rows * rb + ZQ_WEIGHT_TAIL_PAD : 0;
}

size_t zq_hip_set_min_elements(size_t elements) {
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    const size_t prev = b.min_elements;
    b.min_elements = elements;
    return prev;
}

}  // extern "C"

// Host-pointer calls.  Each public entry point takes the mutex, runs its
// *_locked body and counts a non-OK result after a successful init as a
// fallback (the caller runs its CPU route), as zen::hip does
// (hip_backend.hip:940-1015).
namespace {

int counted(Backend& b, int st) {
    if (st != ZQ_OK && b.initialised) ++b.stats.fallbacks;
    return st;
}

int gemv_batch_locked(Backend& b, int fmt, const float* x, const zq_gemv_task* tasks, size_t count, size_t cols,
                      size_t total_rows) {
    int st = init_locked(b);
    if (st != ZQ_OK) return st;
    if (total_rows * cols < b.min_elements) {
        ++b.stats.declined;
        return ZQ_DECLINED;
    }
    zq::GemvTask dt[zq::kMaxTasks];
    Want want[zq::kMaxTasks];
    const uint8_t* dw[zq::kMaxTasks];
    for (size_t i = 0; i < count; ++i) want[i] = Want{tasks[i].weights, tasks[i].rows, cols};
    if ((st = resolve_set(b, fmt, want, count, dw)) != ZQ_OK) return st;
    for (size_t i = 0; i < count; ++i) dt[i] = zq::GemvTask{dw[i], nullptr, static_cast<uint32_t>(tasks[i].rows)};
    const size_t xbytes = align_up(cols * sizeof(float), 256);
    const size_t ybytes = total_rows * sizeof(float);
    st = ensure_scratch(b, xbytes + ybytes, std::max(xbytes, ybytes));
    if (st != ZQ_OK) return st;
    float* dx = static_cast<float*>(b.dev_scratch);
    float* dy = reinterpret_cast<float*>(static_cast<uint8_t*>(b.dev_scratch) + xbytes);
    size_t off = 0;
    for (size_t i = 0; i < count; ++i) {
        dt[i].y = dy + off;
        off += tasks[i].rows;
    }
    HostCall c(b);
    if ((st = c.put(dx, x, cols * sizeof(float))) != ZQ_OK) return st;
    c.begin();
    if (zq::launch_gemv(fmt, dt, static_cast<int>(count), dx, cols, b.stream) != hipSuccess) return fail_hip(b);
    c.launched(1);
    if ((st = c.end()) != ZQ_OK) return st;
    off = 0;
    for (size_t i = 0; i < count; ++i) {
        if ((st = c.get(tasks[i].y, dy + off, tasks[i].rows * sizeof(float))) != ZQ_OK) return st;
        off += tasks[i].rows;
    }
    if (count > 1) ++b.stats.batches;
    return ZQ_OK;
}

int gemm_batch_locked(Backend& b, int fmt, const float* X, const zq_gemm_task* tasks, size_t count, size_t tokens,
                      size_t cols, int act, size_t total_rows) {
    int st = init_locked(b);
    if (st != ZQ_OK) return st;
    st = gemm_supported(fmt, cols, act);
    if (st == ZQ_DECLINED) ++b.stats.declined;
    if (st != ZQ_OK) return st;
    if (tokens * total_rows * cols < b.min_elements) {
        ++b.stats.declined;
        return ZQ_DECLINED;
    }
    const uint8_t* dw[ZQ_MAX_BATCH];
    size_t rows[ZQ_MAX_BATCH];
    Want want[ZQ_MAX_BATCH];
    for (size_t i = 0; i < count; ++i) {
        want[i] = Want{tasks[i].weights, tasks[i].rows, cols};
        rows[i] = tasks[i].rows;
    }
    if ((st = resolve_set(b, fmt, want, count, dw)) != ZQ_OK) return st;
    const size_t xbytes = align_up(tokens * cols * sizeof(float), 256);
    size_t ybytes = 0, ymax = 0;
    for (size_t i = 0; i < count; ++i) {
        ybytes += align_up(tokens * rows[i] * sizeof(float), 256);
        ymax = std::max(ymax, tokens * rows[i] * sizeof(float));
    }
    const size_t wsbytes = batch_workspace_bytes(fmt, rows, count, tokens, cols, act);
    st = ensure_scratch(b, xbytes + ybytes + wsbytes, std::max(xbytes, ymax));
    if (st != ZQ_OK) return st;
    uint8_t* base = static_cast<uint8_t*>(b.dev_scratch);
    float* dx = reinterpret_cast<float*>(base);
    float* dy[ZQ_MAX_BATCH];
    size_t off = xbytes;
    for (size_t i = 0; i < count; ++i) {
        dy[i] = reinterpret_cast<float*>(base + off);
        off += align_up(tokens * rows[i] * sizeof(float), 256);
    }
    void* ws = wsbytes ? base + off : nullptr;
    HostCall c(b);
    if ((st = c.put(dx, X, tokens * cols * sizeof(float))) != ZQ_OK) return st;
    c.begin();
    uint64_t n = 0;
    st = enqueue_gemm_batch(fmt, dw, dy, rows, count, dx, tokens, cols, act, ws, wsbytes, b.stream, &n);
    if (st != ZQ_OK) {
        ++b.stats.errors;
        return st;
    }
    c.launched(n);
    if ((st = c.end()) != ZQ_OK) return st;
    for (size_t i = 0; i < count; ++i)
        if ((st = c.get(tasks[i].Y, dy[i], tokens * rows[i] * sizeof(float))) != ZQ_OK) return st;
    if (count > 1) ++b.stats.batches;
    return ZQ_OK;
}

int ffn_gemv_locked(Backend& b, int fmt, const uint8_t* gate, const uint8_t* up, const uint8_t* down, const float* x,
                    float* y, size_t ffn_rows, size_t cols, size_t out_rows) {
    int st = init_locked(b);
    if (st != ZQ_OK) return st;
    if ((2 * ffn_rows * cols + out_rows * ffn_rows) < b.min_elements) {
        ++b.stats.declined;
        return ZQ_DECLINED;
    }
    const Want want[3] = {{gate, ffn_rows, cols}, {up, ffn_rows, cols}, {down, out_rows, ffn_rows}};
    const uint8_t* dev[3];
    if ((st = resolve_set(b, fmt, want, 3, dev)) != ZQ_OK) return st;
    const uint8_t *dg = dev[0], *du = dev[1], *dd = dev[2];
    const size_t xbytes = align_up(cols * sizeof(float), 256);
    const size_t hbytes = align_up(ffn_rows * sizeof(float), 256);
    const size_t ybytes = align_up(out_rows * sizeof(float), 256);
    st = ensure_scratch(b, xbytes + 3 * hbytes + ybytes, std::max(xbytes, ybytes));
    if (st != ZQ_OK) return st;
    uint8_t* base = static_cast<uint8_t*>(b.dev_scratch);
    float* dx = reinterpret_cast<float*>(base);
    float* dgate = reinterpret_cast<float*>(base + xbytes);
    float* dup = reinterpret_cast<float*>(base + xbytes + hbytes);
    float* dact = reinterpret_cast<float*>(base + xbytes + 2 * hbytes);
    float* dy = reinterpret_cast<float*>(base + xbytes + 3 * hbytes);
    HostCall c(b);
    if ((st = c.put(dx, x, cols * sizeof(float))) != ZQ_OK) return st;
    c.begin();
    zq::GemvTask gu[2] = {{dg, dgate, static_cast<uint32_t>(ffn_rows)}, {du, dup, static_cast<uint32_t>(ffn_rows)}};
    // Q4_K / Q5_K / Q6_K: gate|up as one paired GEMV storing silu(gate) * up
    // (the same per-row sums and activation as the two launches below)
    const hipError_t pe = zq::launch_gemv_silu_pair(fmt, {dg, dact, gu[0].rows}, gu[1], dx, cols, b.stream);
    if (pe != hipSuccess && pe != hipErrorInvalidConfiguration) return fail_hip(b);
    if (pe != hipSuccess) {
        if (zq::launch_gemv(fmt, gu, 2, dx, cols, b.stream) != hipSuccess) return fail_hip(b);
        if (zq::launch_silu_mul(dgate, dup, dact, ffn_rows, b.stream) != hipSuccess) return fail_hip(b);
    }
    zq::GemvTask dn{dd, dy, static_cast<uint32_t>(out_rows)};
    if (zq::launch_gemv(fmt, &dn, 1, dact, ffn_rows, b.stream) != hipSuccess) return fail_hip(b);
    c.launched(pe == hipSuccess ? 2 : 3);
    if ((st = c.end()) != ZQ_OK) return st;
    return c.get(y, dy, out_rows * sizeof(float));
}

int rms_norm_locked(Backend& b, const float* x, const float* w, float* y, size_t rows, size_t cols, float eps) {
    int st = init_locked(b);
    if (st != ZQ_OK) return st;
    const size_t xbytes = align_up(rows * cols * sizeof(float), 256);
    const size_t wbytes = align_up(cols * sizeof(float), 256);
    st = ensure_scratch(b, 2 * xbytes + wbytes, xbytes);
    if (st != ZQ_OK) return st;
    uint8_t* base = static_cast<uint8_t*>(b.dev_scratch);
    float* dx = reinterpret_cast<float*>(base);
    float* dw = reinterpret_cast<float*>(base + xbytes);
    float* dy = reinterpret_cast<float*>(base + xbytes + wbytes);
    HostCall c(b);
    if ((st = c.put(dx, x, rows * cols * sizeof(float))) != ZQ_OK) return st;
    if ((st = c.put(dw, w, cols * sizeof(float))) != ZQ_OK) return st;
    c.begin();
    if (zq::launch_rmsnorm(dx, dw, dy, uint32_t(rows), uint32_t(cols), eps, b.stream) != hipSuccess) return fail_hip(b);
    c.launched(1);
    if ((st = c.end()) != ZQ_OK) return st;
    return c.get(y, dy, rows * cols * sizeof(float));
}

int ffn_residual_locked(Backend& b, int fmt, const uint8_t* wo, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                        const float* norm_w, const float* x, const float* attn_out, float* out, size_t hidden,
                        size_t attn_width, size_t ffn_rows, float eps) {
    int st = init_locked(b);
    if (st != ZQ_OK) return st;
    if ((hidden * attn_width + 3 * ffn_rows * hidden) < b.min_elements) {
        ++b.stats.declined;
        return ZQ_DECLINED;
    }
    const Want want[4] = {{wo, hidden, attn_width}, {wg, ffn_rows, hidden}, {wu, ffn_rows, hidden}, {wd, hidden, ffn_rows}};
    const uint8_t* dev[4];
    if ((st = resolve_set(b, fmt, want, 4, dev)) != ZQ_OK) return st;
    const uint8_t *dwo = dev[0], *dwg = dev[1], *dwu = dev[2], *dwd = dev[3];
    const size_t hb = align_up(hidden * sizeof(float), 256), ab = align_up(attn_width * sizeof(float), 256);
    const size_t wsb = zq_hip_ffn_residual_workspace_bytes(hidden, ffn_rows);
    st = ensure_scratch(b, 3 * hb + ab + wsb, std::max(hb, ab));
    if (st != ZQ_OK) return st;
    uint8_t* base = static_cast<uint8_t*>(b.dev_scratch);
    float* dx = reinterpret_cast<float*>(base);
    float* dn = reinterpret_cast<float*>(base + hb);
    float* dout = reinterpret_cast<float*>(base + 2 * hb);
    float* da = reinterpret_cast<float*>(base + 3 * hb);
    void* ws = base + 3 * hb + ab;
    HostCall c(b);
    if ((st = c.put(dx, x, hidden * sizeof(float))) != ZQ_OK || (st = c.put(dn, norm_w, hidden * sizeof(float))) != ZQ_OK ||
        (st = c.put(da, attn_out, attn_width * sizeof(float))) != ZQ_OK)
        return st;
    c.begin();
    uint64_t n = 0;
    st = enqueue_ffn_residual(fmt, dwo, dwg, dwu, dwd, dn, dx, da, dout, hidden, attn_width, ffn_rows, eps, ws, wsb,
                              b.stream, &n);
    if (st != ZQ_OK) {
        ++b.stats.errors;
        return st;
    }
    c.launched(n);
    if ((st = c.end()) != ZQ_OK) return st;
    return c.get(out, dout, hidden * sizeof(float));
}

}  // namespace

extern "C" {

int zq_hip_gemv_batch(int fmt, const float* x, const zq_gemv_task* tasks, size_t count, size_t cols) {
    if (!x || !tasks || count < 1 || count > ZQ_MAX_BATCH || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols))
        return ZQ_ERR_ARG;
    size_t total_rows = 0;
    for (size_t i = 0; i < count; ++i) {
        if (!tasks[i].weights || !tasks[i].y || !tasks[i].rows || tasks[i].rows > (1u << 30)) return ZQ_ERR_ARG;
        total_rows += tasks[i].rows;
    }
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    try {
        return counted(b, gemv_batch_locked(b, fmt, x, tasks, count, cols, total_rows));
    } catch (const std::bad_alloc&) {
        return counted(b, ZQ_ERR_OOM);
    } catch (...) {
        return counted(b, ZQ_ERR_HIP);
    }
}

int zq_hip_gemv(int fmt, const uint8_t* weights, const float* x, float* y, size_t rows, size_t cols) {
    if (!weights || !y) return ZQ_ERR_ARG;
    const zq_gemv_task t{weights, y, rows};
    return zq_hip_gemv_batch(fmt, x, &t, 1, cols);
}

int zq_hip_gemm_batch(int fmt, const float* X, const zq_gemm_task* tasks, size_t count, size_t tokens, size_t cols,
                      int act_mode) {
    if (!X || !tasks || count < 1 || count > ZQ_MAX_BATCH || !tokens || !valid_fmt(fmt) ||
        !zq::row_bytes(fmt, cols) || tokens > (1u << 24))
        return ZQ_ERR_ARG;
    size_t total_rows = 0;
    for (size_t i = 0; i < count; ++i) {
        if (!tasks[i].weights || !tasks[i].Y || !tasks[i].rows || tasks[i].rows > (1u << 24)) return ZQ_ERR_ARG;
        total_rows += tasks[i].rows;
    }
    const int act = resolve_act(fmt, act_mode);
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    try {
        return counted(b, gemm_batch_locked(b, fmt, X, tasks, count, tokens, cols, act, total_rows));
    } catch (const std::bad_alloc&) {
        return counted(b, ZQ_ERR_OOM);
    } catch (...) {
        return counted(b, ZQ_ERR_HIP);
    }
}

int zq_hip_gemm(int fmt, const uint8_t* weights, const float* X, float* Y, size_t tokens, size_t rows, size_t cols,
                int act_mode) {
    if (!weights || !Y || !rows) return ZQ_ERR_ARG;
    const zq_gemm_task t{weights, Y, rows};
    return zq_hip_gemm_batch(fmt, X, &t, 1, tokens, cols, act_mode);
}

int zq_hip_ffn_gemv(int fmt, const uint8_t* gate, const uint8_t* up, const uint8_t* down, const float* x, float* y,
                    size_t ffn_rows, size_t cols, size_t out_rows) {
    if (!gate || !up || !down || !x || !y || !ffn_rows || !out_rows || !valid_fmt(fmt) ||
        !zq::row_bytes(fmt, cols) || !zq::row_bytes(fmt, ffn_rows) || ffn_rows > (1u << 24) ||
        out_rows > (1u << 24))
        return ZQ_ERR_ARG;
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    try {
        return counted(b, ffn_gemv_locked(b, fmt, gate, up, down, x, y, ffn_rows, cols, out_rows));
    } catch (const std::bad_alloc&) {
        return counted(b, ZQ_ERR_OOM);
    } catch (...) {
        return counted(b, ZQ_ERR_HIP);
    }
}

int zq_hip_rms_norm(const float* x, const float* weight, float* y, size_t rows, size_t cols, float eps) {
    if (!x || !weight || !y || !rows || !cols || rows > (1u << 24) || cols > (1u << 24)) return ZQ_ERR_ARG;
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    try {
        return counted(b, rms_norm_locked(b, x, weight, y, rows, cols, eps));
    } catch (const std::bad_alloc&) {
        return counted(b, ZQ_ERR_OOM);
    } catch (...) {
        return counted(b, ZQ_ERR_HIP);
    }
}

int zq_hip_ffn_residual_fused(int fmt, const uint8_t* attn_output, const uint8_t* gate, const uint8_t* up,
                              const uint8_t* down, const float* norm_weight, const float* x, const float* attn_out,
                              float* out, size_t hidden, size_t attn_width, size_t ffn_rows, float eps) {
    if (!ffn_residual_args_ok(fmt, attn_output, gate, up, down, norm_weight, x, attn_out, out, hidden, attn_width,
                              ffn_rows))
        return ZQ_ERR_ARG;
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    try {
        return counted(b, ffn_residual_locked(b, fmt, attn_output, gate, up, down, norm_weight, x, attn_out, out,
                                              hidden, attn_width, ffn_rows, eps));
    } catch (const std::bad_alloc&) {
        return counted(b, ZQ_ERR_OOM);
    } catch (...) {
        return counted(b, ZQ_ERR_HIP);
    }
}

int zq_hip_release(const uint8_t* weights) {
    if (!weights) return ZQ_ERR_ARG;
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    auto it = b.resident.find(weights);
    if (it == b.resident.end()) return ZQ_DECLINED;
    if (b.stream) (void)hipStreamSynchronize(b.stream);
    (void)hipFree(it->second.dev);
    b.stats.resident_bytes -= it->second.bytes;
    --b.stats.resident_tensors;
    b.resident.erase(it);
    return ZQ_OK;
}

int zq_hip_release_all(void) {
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    if (b.stream) (void)hipStreamSynchronize(b.stream);
    free_resident(b);
    return ZQ_OK;
}

// ---------------------------------------------------------------- device --
int zq_hip_gemv_batch_dev(int fmt, const float* x, const zq_gemv_task* tasks, size_t count, size_t cols,
                          void* stream) {
    if (!x || !tasks || count < 1 || count > ZQ_MAX_BATCH || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols))
        return ZQ_ERR_ARG;
    zq::GemvTask dt[zq::kMaxTasks];
    for (size_t i = 0; i < count; ++i) {
        if (!tasks[i].weights || !tasks[i].y || !tasks[i].rows || tasks[i].rows > (1u << 30)) return ZQ_ERR_ARG;
        dt[i] = zq::GemvTask{tasks[i].weights, tasks[i].y, static_cast<uint32_t>(tasks[i].rows)};
    }
    if (const int ls = launch_status(
            zq::launch_gemv(fmt, dt, static_cast<int>(count), x, cols, static_cast<hipStream_t>(stream)));
        ls != ZQ_OK)
        return ls;
    return ZQ_OK;
}

int zq_hip_gemv_dev(int fmt, const void* weights, const float* x, float* y, size_t rows, size_t cols, void* stream) {
    const zq_gemv_task t{static_cast<const uint8_t*>(weights), y, rows};
    return zq_hip_gemv_batch_dev(fmt, x, &t, 1, cols, stream);
}

size_t zq_hip_gemm_workspace_bytes(int fmt, size_t tokens, size_t rows, size_t cols, int act_mode) {
    if (!valid_fmt(fmt) || !zq::row_bytes(fmt, cols) || !tokens || !rows) return 0;
    if (resolve_act(fmt, act_mode) != ZQ_ACT_INT8) return zq::gemm_f32_workspace_bytes(fmt, tokens, rows, cols);
    return align_up(tokens * cols, 256) + align_up(tokens * (cols / 32) * sizeof(float), 256) +
           zq::gemm_i8_partial_bytes(tokens, rows, cols);
}

int zq_hip_gemm_dev(int fmt, const void* weights, const float* X, float* Y, size_t tokens, size_t rows, size_t cols,
                    int act_mode, void* workspace, size_t workspace_bytes, void* stream) {
    if (!weights || !X || !Y || !tokens || !rows || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols) ||
        tokens > (1u << 24) || rows > (1u << 24))
        return ZQ_ERR_ARG;
    const int act = resolve_act(fmt, act_mode);
    const int st = gemm_supported(fmt, cols, act);
    if (st != ZQ_OK) return st;
    uint64_t d = 0;
    return enqueue_gemm(fmt, static_cast<const uint8_t*>(weights), X, Y, tokens, rows, cols, act, workspace,
                        workspace_bytes, static_cast<hipStream_t>(stream), &d);
}

size_t zq_hip_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int zq_hip_gemm_dev_noalloc(int fmt, const void* weights, const float* X, float* Y, size_t tokens, size_t rows,
                            size_t cols, int act_mode, void* stream) {
    if (!weights || !X || !Y || !tokens || !rows || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols) ||
        tokens > (1u << 24) || rows > (1u << 24))
        return ZQ_ERR_ARG;
    const int act = resolve_act(fmt, act_mode);
    int st = gemm_supported(fmt, cols, act);
    if (st != ZQ_OK) return st;
    const size_t need = zq_hip_gemm_workspace_bytes(fmt, tokens, rows, cols, act);
    if (need > kNoAllocScratchBytes) return ZQ_ERR_TOO_LARGE;  // before any launch or copy
    void* ws = scratch_ptr();
    if (!ws) return ZQ_ERR_HIP;
    uint64_t d = 0;
    return enqueue_gemm(fmt, static_cast<const uint8_t*>(weights), X, Y, tokens, rows, cols, act, ws,
                        kNoAllocScratchBytes, static_cast<hipStream_t>(stream), &d);
}

size_t zq_hip_gemm_batch_workspace_bytes(int fmt, const zq_gemm_task* tasks, size_t count, size_t tokens, size_t cols,
                                         int act_mode) {
    if (!tasks || count < 1 || count > ZQ_MAX_BATCH || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols) || !tokens) return 0;
    size_t rows[ZQ_MAX_BATCH];
    for (size_t i = 0; i < count; ++i) {
        if (!tasks[i].rows) return 0;
        rows[i] = tasks[i].rows;
    }
    return batch_workspace_bytes(fmt, rows, count, tokens, cols, resolve_act(fmt, act_mode));
}

int zq_hip_gemm_batch_dev(int fmt, const float* X, const zq_gemm_task* tasks, size_t count, size_t tokens, size_t cols,
                          int act_mode, void* workspace, size_t workspace_bytes, void* stream) {
    if (!X || !tasks || count < 1 || count > ZQ_MAX_BATCH || !tokens || !valid_fmt(fmt) ||
        !zq::row_bytes(fmt, cols) || tokens > (1u << 24))
        return ZQ_ERR_ARG;
    const uint8_t* w[ZQ_MAX_BATCH];
    float* Y[ZQ_MAX_BATCH];
    size_t rows[ZQ_MAX_BATCH];
    for (size_t i = 0; i < count; ++i) {
        if (!tasks[i].weights || !tasks[i].Y || !tasks[i].rows || tasks[i].rows > (1u << 24)) return ZQ_ERR_ARG;
        w[i] = tasks[i].weights;
        Y[i] = tasks[i].Y;
        rows[i] = tasks[i].rows;
    }
    const int act = resolve_act(fmt, act_mode);
    const int st = gemm_supported(fmt, cols, act);
    if (st != ZQ_OK) return st;
    uint64_t d = 0;
    return enqueue_gemm_batch(fmt, w, Y, rows, count, X, tokens, cols, act, workspace, workspace_bytes,
                              static_cast<hipStream_t>(stream), &d);
}

int zq_hip_rms_norm_dev(const float* x, const float* weight, float* y, size_t rows, size_t cols, float eps,
                        void* stream) {
    if (!x || !weight || !y || !rows || !cols || rows > (1u << 24) || cols > (1u << 24)) return ZQ_ERR_ARG;
    return launch_status(zq::launch_rmsnorm(x, weight, y, uint32_t(rows), uint32_t(cols), eps,
                         static_cast<hipStream_t>(stream)));
}

int zq_hip_ffn_residual_fused_dev(int fmt, const void* attn_output, const void* gate, const void* up, const void* down,
                                  const float* norm_weight, const float* x, const float* attn_out, float* out,
                                  size_t hidden, size_t attn_width, size_t ffn_rows, float eps, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    if (!ffn_residual_args_ok(fmt, attn_output, gate, up, down, norm_weight, x, attn_out, out, hidden, attn_width,
                              ffn_rows))
        return ZQ_ERR_ARG;
    uint64_t d = 0;
    return enqueue_ffn_residual(fmt, static_cast<const uint8_t*>(attn_output), static_cast<const uint8_t*>(gate),
                                static_cast<const uint8_t*>(up), static_cast<const uint8_t*>(down), norm_weight, x,
                                attn_out, out, hidden, attn_width, ffn_rows, eps, workspace, workspace_bytes,
                                static_cast<hipStream_t>(stream), &d);
}

int zq_hip_quantize_acts_dev(const float* X, int8_t* xq, float* xs, size_t tokens, size_t cols, void* stream) {
    if (!X || !xq || !xs || !tokens || !cols || cols % 32) return ZQ_ERR_ARG;
    return launch_status(zq::launch_quantize_acts(X, xq, xs, tokens, cols, static_cast<hipStream_t>(stream)));
}

int zq_hip_block_dots_dev(int fmt, const void* weights, const int8_t* xq, int32_t* out, size_t tokens, size_t rows,
                          size_t cols, void* stream) {
    if (!weights || !xq || !out || !tokens || !rows || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols)) return ZQ_ERR_ARG;
    if (!int8_fmt(fmt) || cols % 64) return ZQ_DECLINED;
    return launch_status(zq::launch_block_dots(fmt, static_cast<const uint8_t*>(weights), xq, out, tokens, rows, cols,
                                 static_cast<hipStream_t>(stream)));
}

int zq_hip_dequantize_dev(int fmt, const void* weights, float* out, size_t rows, size_t cols, void* stream) {
    if (!weights || !out || !rows || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols)) return ZQ_ERR_ARG;
    return launch_status(zq::launch_dequantize(fmt, static_cast<const uint8_t*>(weights), out, rows, cols,
                                 static_cast<hipStream_t>(stream)));
}

int zq_hip_read_probe_dev(const void* buf, size_t bytes, void* sink, void* stream) {
    if (!buf || !sink || !bytes || bytes % 16 || (reinterpret_cast<uintptr_t>(buf) & 15u)) return ZQ_ERR_ARG;
    return launch_status(zq::launch_read_probe(buf, bytes, static_cast<uint32_t*>(sink),
                         static_cast<hipStream_t>(stream)));
}
size_t zq_hip_read_probe_sink_bytes(void) { return zq::read_probe_sink_bytes(); }

int zq_hip_mfma_peak(double* sclk_mhz, double* cycles_per_mfma, double* int8_tops) {
    if (!sclk_mhz || !cycles_per_mfma || !int8_tops) return ZQ_ERR_ARG;
    Backend& b = B();
    std::lock_guard<std::mutex> lock(b.mu);
    int st = init_locked(b);
    if (st != ZQ_OK) return st;
    const uint32_t wgs = uint32_t(b.info.compute_units), iters = 20000;
    uint64_t* d = nullptr;
    if (hipMalloc(&d, size_t(wgs) * 4 * sizeof(uint64_t)) != hipSuccess) return ZQ_ERR_OOM;
    std::vector<uint64_t> h(size_t(wgs) * 4);
    const bool ok = zq::launch_mfma_probe(d, wgs, iters / 10, b.stream) == hipSuccess &&  // warm-up (clock ramp)
                    zq::launch_mfma_probe(d, wgs, iters, b.stream) == hipSuccess &&
                    hipStreamSynchronize(b.stream) == hipSuccess &&
                    hipMemcpy(h.data(), d, h.size() * sizeof(uint64_t), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(d);
    if (!ok) return fail_hip(b);
    double cyc = 0.0, ticks = 0.0;
    for (uint32_t i = 0; i < wgs; ++i) {
        cyc += double(h[4 * i]);
        ticks += double(h[4 * i + 1]);
    }
    cyc /= wgs;
    ticks /= wgs;
    if (ticks <= 0.0 || cyc <= 0.0) return ZQ_ERR_HIP;
    *sclk_mhz = cyc / ticks * 100.0;  // s_memrealtime counts at 100 MHz
    *cycles_per_mfma = cyc / (4.0 * iters);
    // 32x32x32 MACs = 65536 ops per MFMA, one MFMA pipe per SIMD, 4 SIMDs per CU
    *int8_tops = double(wgs) * 4.0 * 65536.0 / *cycles_per_mfma * (*sclk_mhz * 1e6) / 1e12;
    return ZQ_OK;
}

int zq_hip_synth_weights_dev(int fmt, uint64_t seed, void* weights, size_t rows, size_t cols, void* stream) {
    if (!weights || !rows || !valid_fmt(fmt) || !zq::row_bytes(fmt, cols)) return ZQ_ERR_ARG;
    return launch_status(zq::launch_synth_weights(fmt, seed, static_cast<uint8_t*>(weights), rows, cols,
                                    static_cast<hipStream_t>(stream)));
}

int zq_hip_synth_normal_dev(uint64_t seed, float* out, size_t n, void* stream) {
    if (!out || !n) return ZQ_ERR_ARG;
    return launch_status(zq::launch_synth_normal(seed, out, n, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
