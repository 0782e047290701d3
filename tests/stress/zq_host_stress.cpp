// Host-pointer API under concurrency and residency churn (test infrastructure).
//
// Several threads call the host-pointer entry points (gemv, gemv_batch, gemm,
// gemm_batch, stats, release, release_all) on their own Q8_0 weight buffers,
// with the residency budget lowered (ZQ_HIP_RESIDENT_BUDGET, set by the
// caller) so that uploads keep evicting the whole resident set.  Weight
// buffers are released, freed and reallocated, often at the same address
// with another shape, which the residency contract requires a release for
// (the reference's hip_backend.h:52-58).  Every OK result is checked against
// an fp64 dot product of the same blocks; a declined call is allowed (a batch
// whose weights cannot be resident together is declined); any error status or
// mismatch fails the run.  Prints "stress ok ..." and exits 0 on success.
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#include "zq_hip.h"

namespace {

std::atomic<long> n_ok{0}, n_declined{0}, n_bad{0}, n_err{0};

// fp16 <-> fp32 for normal values (the scales here are all normal)
float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h >> 15) << 31, exp = (h >> 10) & 31, man = h & 1023;
    const uint32_t bits = exp == 0 ? sign : sign | ((exp + 112) << 23) | (man << 13);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}
uint16_t float_to_half(float f) {  // round to nearest, normal range only
    uint32_t b;
    std::memcpy(&b, &f, 4);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int exp = int((b >> 23) & 255) - 112;
    uint32_t man = b & 0x7FFFFFu;
    uint32_t h = sign | (uint32_t(exp) << 10) | (man >> 13);
    if ((man & 0x1FFFu) > 0x1000u || ((man & 0x1FFFu) == 0x1000u && (h & 1u))) ++h;
    return uint16_t(h);
}

struct Weights {
    uint8_t* p = nullptr;
    size_t rows = 0, cols = 0;
};

void fill(Weights& w, std::mt19937& g) {
    const size_t rb = zq_row_bytes(ZQ_FMT_Q8_0, w.cols);
    w.p = static_cast<uint8_t*>(std::malloc(w.rows * rb));
    std::uniform_int_distribution<int> q(-127, 127);
    std::uniform_real_distribution<float> d(0.001f, 0.02f);
    for (size_t r = 0; r < w.rows; ++r)
        for (size_t b = 0; b < w.cols / 32; ++b) {
            uint8_t* blk = w.p + r * rb + b * 34;
            const uint16_t h = float_to_half(d(g));
            std::memcpy(blk, &h, 2);
            for (int i = 0; i < 32; ++i) blk[2 + i] = uint8_t(int8_t(q(g)));
        }
}

// fp64 dot of every row with x; mag = sum of |terms| (the error scale)
void reference(const Weights& w, const float* x, std::vector<double>& y, std::vector<double>& mag) {
    const size_t rb = zq_row_bytes(ZQ_FMT_Q8_0, w.cols);
    y.assign(w.rows, 0.0);
    mag.assign(w.rows, 0.0);
    for (size_t r = 0; r < w.rows; ++r)
        for (size_t b = 0; b < w.cols / 32; ++b) {
            const uint8_t* blk = w.p + r * rb + b * 34;
            uint16_t h;
            std::memcpy(&h, blk, 2);
            const double d = half_to_float(h);
            for (int i = 0; i < 32; ++i) {
                const double t = d * int8_t(blk[2 + i]) * x[b * 32 + i];
                y[r] += t;
                mag[r] += std::fabs(t);
            }
        }
}

bool matches(const float* got, const Weights& w, const float* x) {
    std::vector<double> y, mag;
    reference(w, x, y, mag);
    for (size_t r = 0; r < w.rows; ++r)
        if (!(std::fabs(got[r] - y[r]) <= 1e-4 * mag[r] + 1e-5)) return false;
    return true;
}

void tally(int st, bool good) {
    if (st == ZQ_OK)
        (good ? n_ok : n_bad)++;
    else if (st == ZQ_DECLINED)
        n_declined++;
    else {
        n_err++;
        std::fprintf(stderr, "status %d (%s)\n", st, zq_hip_status_string(st));
    }
}

void worker(int t, int iters) {
    std::mt19937 g(1000u + unsigned(t));
    const size_t cols = 1024 * size_t(1 + t % 4);
    const size_t row_choice[] = {64, 128, 256, 512};
    std::vector<Weights> pool(6);
    for (auto& w : pool) {
        w.cols = cols;
        w.rows = row_choice[g() % 4];
        fill(w, g);
    }
    std::vector<float> x(cols);
    std::normal_distribution<float> nd;
    for (int it = 0; it < iters; ++it) {
        for (auto& v : x) v = nd(g);
        const int op = int(g() % 7);
        if (op == 0) {
            Weights& w = pool[g() % pool.size()];
            std::vector<float> y(w.rows);
            const int st = zq_hip_gemv(ZQ_FMT_Q8_0, w.p, x.data(), y.data(), w.rows, cols);
            tally(st, st != ZQ_OK || matches(y.data(), w, x.data()));
        } else if (op == 1) {  // 2..4 tasks, a slot may repeat
            const int n = 2 + int(g() % 3);
            zq_gemv_task tk[4];
            std::vector<std::vector<float>> ys(n);
            int idx[4];
            for (int i = 0; i < n; ++i) {
                idx[i] = int(g() % pool.size());
                ys[i].resize(pool[idx[i]].rows);
                tk[i] = zq_gemv_task{pool[idx[i]].p, ys[i].data(), pool[idx[i]].rows};
            }
            const int st = zq_hip_gemv_batch(ZQ_FMT_Q8_0, x.data(), tk, size_t(n), cols);
            bool good = true;
            if (st == ZQ_OK)
                for (int i = 0; i < n; ++i) good = good && matches(ys[i].data(), pool[idx[i]], x.data());
            tally(st, good);
        } else if (op == 2) {  // fp32-activation GEMM
            Weights& w = pool[g() % pool.size()];
            const size_t tok = 1 + g() % 6;
            std::vector<float> X(tok * cols), Y(tok * w.rows);
            for (auto& v : X) v = nd(g);
            const int st = zq_hip_gemm(ZQ_FMT_Q8_0, w.p, X.data(), Y.data(), tok, w.rows, cols, ZQ_ACT_F32);
            bool good = true;
            if (st == ZQ_OK)
                for (size_t k = 0; k < tok; ++k) good = good && matches(Y.data() + k * w.rows, w, X.data() + k * cols);
            tally(st, good);
        } else if (op == 3) {  // release, free, reallocate (often the same address, another shape)
            Weights& w = pool[g() % pool.size()];
            zq_hip_release(w.p);
            std::free(w.p);
            w.rows = row_choice[g() % 4];
            fill(w, g);
        } else if (op == 4) {
            zq_hip_stats s;
            zq_hip_get_stats(&s);
            if (g() % 50 == 0) zq_hip_reset_stats();
        } else if (op == 5) {  // GEMM batch
            const int n = 2 + int(g() % 2);
            const size_t tok = 2 + g() % 4;
            std::vector<float> X(tok * cols);
            for (auto& v : X) v = nd(g);
            zq_gemm_task tk[3];
            std::vector<std::vector<float>> Ys(n);
            int idx[3];
            for (int i = 0; i < n; ++i) {
                idx[i] = int(g() % pool.size());
                Ys[i].resize(tok * pool[idx[i]].rows);
                tk[i] = zq_gemm_task{pool[idx[i]].p, Ys[i].data(), pool[idx[i]].rows};
            }
            const int st = zq_hip_gemm_batch(ZQ_FMT_Q8_0, X.data(), tk, size_t(n), tok, cols, ZQ_ACT_F32);
            bool good = true;
            if (st == ZQ_OK)
                for (int i = 0; i < n; ++i)
                    for (size_t k = 0; k < tok; ++k)
                        good = good && matches(Ys[i].data() + k * pool[idx[i]].rows, pool[idx[i]], X.data() + k * cols);
            tally(st, good);
        } else if (t == 0 && g() % 20 == 0) {
            zq_hip_release_all();
        }
    }
    for (auto& w : pool) {
        zq_hip_release(w.p);
        std::free(w.p);
    }
}

}  // namespace

int main(int argc, char** argv) {
    const int threads = argc > 1 ? std::atoi(argv[1]) : 4;
    const int iters = argc > 2 ? std::atoi(argv[2]) : 200;
    if (zq_hip_init() != ZQ_OK) {
        std::printf("zq_hip_init failed\n");
        return 2;
    }
    zq_hip_set_min_elements(0);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) pool.emplace_back(worker, t, iters);
    for (auto& th : pool) th.join();
    zq_hip_stats s;
    zq_hip_get_stats(&s);
    std::printf("%s ok=%ld declined=%ld bad=%ld err=%ld evictions=%llu uploads=%llu\n",
                n_bad || n_err ? "stress FAILED" : "stress ok", n_ok.load(), n_declined.load(), n_bad.load(),
                n_err.load(), static_cast<unsigned long long>(s.evictions), static_cast<unsigned long long>(s.uploads));
    std::fflush(stdout);  // the verdict line survives whatever the runtime's teardown does
    zq_hip_shutdown();
    return n_bad || n_err ? 1 : 0;
}
