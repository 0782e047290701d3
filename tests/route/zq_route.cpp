// zq_route.cpp -- TEST: a compiled C++ caller of the drop-in boundary.
//
// It plays the reference's own dispatch order for a projection, the way
// src/quant.cpp does once the HIP backend is compiled in:
//   quant::gemv  (src/quant.cpp:963-968, 1007-1012): reject null/zero/non-finite
//                scale and indivisible cols; then, for scale == 1 and an
//                enabled backend, try the GPU; on any non-OK status fall
//                through to the CPU kernels.
//   quant::gemm  (src/quant.cpp:1613-1617, 1656-1659): the same.
//   quant::gemm_batch (src/quant.cpp:1521-1554): the GPU batch, else one
//                quant::gemm per task.
// The GPU side is libzq_hip.so through include/zq_hip.h; the CPU side is the
// reference's own quant::gemv / quant::gemm (AVX2 + ComputePool), compiled
// from the reference sources into oracle/_ref/libzenref.so and reached
// through its C shim (zr_gemv / zr_gemm).  Exit status 0 when every check
// holds; each failed check prints one line.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "zq_hip.h"

extern "C" {
int zr_gemv(int fmt, const uint8_t* w, const float* x, float* y, size_t rows, size_t cols, unsigned workers);
int zr_gemm(int fmt, const uint8_t* w, const float* X, float* Y, size_t tokens, size_t rows, size_t cols,
            unsigned workers);
size_t zr_row_bytes(int fmt, size_t cols);
}

namespace {

int g_failures = 0;
unsigned g_gpu = 0, g_cpu = 0;

void check(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL %s\n", what);
        ++g_failures;
    }
}

bool route_gemv(int fmt, const uint8_t* w, const float* x, float* y, size_t rows, size_t cols, float scale) {
    if (!w || !x || !y || !rows || !cols || !std::isfinite(scale)) return false;
    if (!zr_row_bytes(fmt, cols)) return false;
    if (scale == 1.0f && zq_hip_enabled() && zq_hip_gemv(fmt, w, x, y, rows, cols) == ZQ_OK) {
        ++g_gpu;
        return true;
    }
    ++g_cpu;
    if (!zr_gemv(fmt, w, x, y, rows, cols, 0)) return false;
    if (scale != 1.0f)
        for (size_t i = 0; i < rows; ++i) y[i] *= scale;
    return true;
}

bool route_gemm(int fmt, const uint8_t* w, const float* X, float* Y, size_t tokens, size_t rows, size_t cols,
                int act) {
    if (!w || !X || !Y || !tokens || !rows || !cols) return false;
    if (!zr_row_bytes(fmt, cols)) return false;
    if (zq_hip_enabled() && zq_hip_gemm(fmt, w, X, Y, tokens, rows, cols, act) == ZQ_OK) {
        ++g_gpu;
        return true;
    }
    ++g_cpu;
    return zr_gemm(fmt, w, X, Y, tokens, rows, cols, 0) != 0;
}

bool route_gemm_batch(int fmt, const uint8_t* const* w, const float* X, float* const* Y, const size_t* rows,
                      size_t tokens, size_t cols, size_t count, int act) {
    if (!w || !X || !Y || !rows || !count || !tokens || !cols) return false;
    if (count <= ZQ_MAX_BATCH && zq_hip_enabled()) {
        zq_gemm_task t[ZQ_MAX_BATCH];
        for (size_t i = 0; i < count; ++i) t[i] = zq_gemm_task{w[i], Y[i], rows[i]};
        if (zq_hip_gemm_batch(fmt, X, t, count, tokens, cols, act) == ZQ_OK) {
            ++g_gpu;
            return true;
        }
    }
    for (size_t i = 0; i < count; ++i)
        if (!route_gemm(fmt, w[i], X, Y[i], tokens, rows[i], cols, act)) return false;
    return true;
}

// Q8_0 rows: fp16 scale |N(0,1)|*0.002 (rounded through the reference's own
// binary16 encoder is not needed: any finite half works) + uniform int8.
std::vector<uint8_t> q8_weights(size_t rows, size_t cols, uint32_t seed) {
    std::mt19937 rng(seed);
    std::vector<uint8_t> w(rows * (cols / 32) * 34 + 64, 0);
    for (size_t b = 0; b < rows * (cols / 32); ++b) {
        const uint16_t h = uint16_t(0x1000 + (rng() % 0x0C00));  // 2^-12 .. ~2^-10, normal halves
        std::memcpy(&w[b * 34], &h, 2);
        for (int j = 0; j < 32; ++j) w[b * 34 + 2 + j] = uint8_t(int8_t(int(rng() % 255) - 127));
    }
    return w;
}

std::vector<float> normal(size_t n, uint32_t seed) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> d(0.0f, 1.0f);
    std::vector<float> v(n);
    for (auto& f : v) f = d(rng);
    return v;
}

bool close(const float* got, const float* want, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!(std::fabs(double(got[i]) - want[i]) <= 1e-4 + 1e-5 * std::fabs(double(want[i])))) return false;
    return true;
}

}  // namespace

int main() {
    setenv("ZEN_HIP", "1", 1);
    if (zq_hip_init() != ZQ_OK || !zq_hip_enabled()) {
        std::printf("FAIL no gfx950 device\n");
        return 2;
    }
    const int Q8 = ZQ_FMT_Q8_0;

    // 1. accepted GEMV: the GPU takes it; within the bar of the reference CPU
    {
        const size_t rows = 1024, cols = 4096;
        auto w = q8_weights(rows, cols, 1);
        auto x = normal(cols, 2);
        std::vector<float> y(rows), ref(rows);
        const unsigned g0 = g_gpu;
        check(route_gemv(Q8, w.data(), x.data(), y.data(), rows, cols, 1.0f), "gemv accepted: route");
        check(g_gpu == g0 + 1, "gemv accepted: taken by the GPU");
        check(zr_gemv(Q8, w.data(), x.data(), ref.data(), rows, cols, 0) == 1, "gemv accepted: reference");
        check(close(y.data(), ref.data(), rows), "gemv accepted: within 1e-4 + 1e-5|ref|");
        zq_hip_release(w.data());
    }
    // 2. declined GEMV (rows*cols below the backend's minimum): the CPU route
    //    runs and its output is the reference's, bit for bit
    {
        const size_t rows = 16, cols = 256;
        auto w = q8_weights(rows, cols, 3);
        auto x = normal(cols, 4);
        std::vector<float> y(rows), ref(rows);
        const unsigned c0 = g_cpu;
        check(zq_hip_gemv(Q8, w.data(), x.data(), y.data(), rows, cols) == ZQ_DECLINED, "gemv small: declined");
        check(route_gemv(Q8, w.data(), x.data(), y.data(), rows, cols, 1.0f), "gemv small: route");
        check(g_cpu == c0 + 1, "gemv small: CPU route");
        zr_gemv(Q8, w.data(), x.data(), ref.data(), rows, cols, 0);
        check(std::memcmp(y.data(), ref.data(), rows * 4) == 0, "gemv small: bit-equal to the reference CPU");
    }
    // 3. scale != 1 never reaches the GPU (quant.cpp:1010)
    {
        const size_t rows = 1024, cols = 1024;
        auto w = q8_weights(rows, cols, 5);
        auto x = normal(cols, 6);
        std::vector<float> y(rows);
        const unsigned g0 = g_gpu;
        check(route_gemv(Q8, w.data(), x.data(), y.data(), rows, cols, 0.5f), "gemv scaled: route");
        check(g_gpu == g0, "gemv scaled: stays on the CPU");
    }
    // 4. indivisible cols: rejected before either route, as quant::gemv does
    {
        auto w = q8_weights(64, 64, 7);
        auto x = normal(80, 8);
        std::vector<float> y(64);
        check(!route_gemv(Q8, w.data(), x.data(), y.data(), 64, 80, 1.0f), "gemv cols%32: rejected");
        check(zq_hip_gemv(Q8, w.data(), x.data(), y.data(), 64, 80) == ZQ_ERR_ARG, "gemv cols%32: ZQ_ERR_ARG");
    }
    // 5. accepted GEMM with fp32 activations (the reference CPU arithmetic)
    {
        const size_t t = 37, rows = 512, cols = 4096;
        auto w = q8_weights(rows, cols, 9);
        auto X = normal(t * cols, 10);
        std::vector<float> Y(t * rows), ref(t * rows);
        const unsigned g0 = g_gpu;
        check(route_gemm(Q8, w.data(), X.data(), Y.data(), t, rows, cols, ZQ_ACT_F32), "gemm f32: route");
        check(g_gpu == g0 + 1, "gemm f32: taken by the GPU");
        zr_gemm(Q8, w.data(), X.data(), ref.data(), t, rows, cols, 0);
        check(close(Y.data(), ref.data(), t * rows), "gemm f32: within 1e-4 + 1e-5|ref|");
        zq_hip_release(w.data());
    }
    // 6. declined GEMM (int8 activations asked of Q6_K): the CPU route
    {
        const size_t t = 4, rows = 256, cols = 1024;
        std::vector<uint8_t> w(rows * (cols / 256) * 210 + 64, 0);
        std::mt19937 rng(11);
        for (size_t sb = 0; sb < rows * (cols / 256); ++sb) {
            uint8_t* p = &w[sb * 210];
            for (int i = 0; i < 192; ++i) p[i] = uint8_t(rng());
            for (int i = 0; i < 16; ++i) p[192 + i] = uint8_t(int8_t(int(rng() % 64) - 32));
            const uint16_t d = 0x1400;
            std::memcpy(p + 208, &d, 2);
        }
        auto X = normal(t * cols, 12);
        std::vector<float> Y(t * rows), ref(t * rows);
        const unsigned c0 = g_cpu;
        check(route_gemm(ZQ_FMT_Q6_K, w.data(), X.data(), Y.data(), t, rows, cols, ZQ_ACT_INT8), "gemm q6k: route");
        check(g_cpu == c0 + 1, "gemm q6k int8: CPU route");
        zr_gemm(ZQ_FMT_Q6_K, w.data(), X.data(), ref.data(), t, rows, cols, 0);
        check(std::memcmp(Y.data(), ref.data(), Y.size() * 4) == 0, "gemm q6k: bit-equal to the reference CPU");
    }
    // 7. gemm_batch: the GPU batch, within the bar of per-task reference GEMMs
    {
        const size_t t = 20, cols = 2048, count = 3;
        const size_t rows[3] = {512, 128, 128};
        std::vector<uint8_t> w[3];
        std::vector<float> Y[3], ref(t * 512);
        const uint8_t* wp[3];
        float* yp[3];
        for (size_t i = 0; i < count; ++i) {
            w[i] = q8_weights(rows[i], cols, 20 + uint32_t(i));
            Y[i].resize(t * rows[i]);
            wp[i] = w[i].data();
            yp[i] = Y[i].data();
        }
        auto X = normal(t * cols, 30);
        check(route_gemm_batch(Q8, wp, X.data(), yp, rows, t, cols, count, ZQ_ACT_F32), "gemm_batch: route");
        for (size_t i = 0; i < count; ++i) {
            zr_gemm(Q8, wp[i], X.data(), ref.data(), t, rows[i], cols, 0);
            check(close(Y[i].data(), ref.data(), t * rows[i]), "gemm_batch: within 1e-4 + 1e-5|ref|");
            zq_hip_release(wp[i]);
        }
    }
    // 8. backend not opted in: zq_hip_enabled() is 0 and every call stays on the CPU
    {
        unsetenv("ZEN_HIP");
        unsetenv("ZEN_BACKEND");
        const size_t rows = 1024, cols = 4096;
        auto w = q8_weights(rows, cols, 40);
        auto x = normal(cols, 41);
        std::vector<float> y(rows), ref(rows);
        const unsigned g0 = g_gpu;
        check(zq_hip_enabled() == 0, "not opted in: disabled");
        check(route_gemv(Q8, w.data(), x.data(), y.data(), rows, cols, 1.0f), "not opted in: route");
        check(g_gpu == g0, "not opted in: CPU route");
        zr_gemv(Q8, w.data(), x.data(), ref.data(), rows, cols, 0);
        check(std::memcmp(y.data(), ref.data(), rows * 4) == 0, "not opted in: bit-equal to the reference CPU");
    }
    zq_hip_stats s{};
    zq_hip_get_stats(&s);
    std::printf("route %s: %u GPU, %u CPU, submits %llu, fallbacks %llu, declined %llu\n",
                g_failures ? "FAILED" : "ok", g_gpu, g_cpu, (unsigned long long)s.submits,
                (unsigned long long)s.fallbacks, (unsigned long long)s.declined);
    zq_hip_shutdown();
    return g_failures ? 1 : 0;
}
