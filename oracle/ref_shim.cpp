// ref_shim.cpp -- TEST INFRASTRUCTURE ONLY.
// A C-callable shim over the reference's own CPU quant surface
// (include/zen/quant.h:20-33, 106), compiled together with the reference's
// sources by oracle/Makefile into oracle/_ref/libzenref.so.  It is used to pin
// the C oracle (zq_oracle.c) and as the CPU baseline in bench.py; the HIP
// product never loads it.
#include "zen/quant.h"
#include "zen/compute_pool.h"
#include "zen/kernels.h"
#include <cstdint>
#include <cstddef>

namespace {
const zen::quant::Format* fmt_of(int ggml_type) {
    switch (ggml_type) {  // ggml type ids, src/gguf.cpp:370-393
    case 2: return zen::quant::find("Q4_0");
    case 8: return zen::quant::find("Q8_0");
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
}
