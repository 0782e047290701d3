// stream_ceiling.hip -- the per-launch floor and the streaming-read ceiling of
// the GPU it runs on, the yardsticks for the decode GEMVs:
//   - back-to-back launches of an empty kernel (the launch/drain floor of a
//     stream, what every dependent kernel of a decode step pays);
//   - a plain non-temporal read of S bytes (no compute), launched back to back
//     over distinct buffers whose total (1 GiB) exceeds the 256 MB MALL, so
//     every launch reads HBM: per-launch time and GB/s for S = 4 .. 558 MB.
// Times are HIP events around n back-to-back launches, as bench.py measures.
// Build and run:
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         -o /tmp/stream_ceiling zeninfer_amd/probes/stream_ceiling.hip && /tmp/stream_ceiling
#include <hip/hip_runtime.h>
#include <cstdio>

#define CK(x)                                                                       \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);   \
            return 1;                                                               \
        }                                                                           \
    } while (0)

typedef unsigned u4 __attribute__((ext_vector_type(4)));

__global__ void empty_kernel(float* y) {
    if (threadIdx.x == 0 && blockIdx.x == 0 && y[0] == 12345.f) y[1] = 1.0f;
}

// each workgroup owns a contiguous share; each thread issues 4 independent
// 16-byte non-temporal loads per step
__global__ __launch_bounds__(256) void read_kernel(const u4* __restrict__ w, size_t n16, float* y) {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t b = blockIdx.x * per, e = b + per < n16 ? b + per : n16;
    unsigned acc = 0;
    for (size_t i = b + threadIdx.x; i < e; i += 4 * 256) {
        u4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const size_t j = i + size_t(k) * 256;
            v[k] = j < e ? __builtin_nontemporal_load(&w[j]) : u4{0, 0, 0, 0};
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    if (acc == 0x12345u) y[blockIdx.x] = float(acc);
}

int main() {
    const size_t pool = size_t(1) << 30;  // 1 GiB of distinct buffers
    float* y;
    u4* w;
    CK(hipMalloc(&y, 1 << 20));
    CK(hipMalloc(&w, pool + (size_t(600) << 20)));
    CK(hipMemset(w, 1, pool + (size_t(600) << 20)));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    auto timed = [&](auto launch, int n) {
        for (int i = 0; i < 3; ++i) launch(i);
        (void)hipEventRecord(a);
        for (int i = 0; i < n; ++i) launch(i);
        (void)hipEventRecord(b);
        (void)hipEventSynchronize(b);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, a, b);
        return ms * 1e3f / n;
    };
    printf("empty kernel 256 x 1024 threads: %.2f us per launch\n",
           timed([&](int) { hipLaunchKernelGGL(empty_kernel, dim3(256), dim3(1024), 0, 0, y); }, 200));
    printf("empty kernel 1 x 64 threads:     %.2f us per launch\n",
           timed([&](int) { hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, 0, y); }, 200));
    for (size_t mb : {4, 16, 32, 64, 128, 558}) {
        const size_t bytes = mb << 20, n16 = bytes / 16;
        const size_t slots = pool / bytes > 1 ? pool / bytes : 1;
        const float us = timed(
            [&](int i) {
                const u4* p = w + (size_t(i) % slots) * n16;
                hipLaunchKernelGGL(read_kernel, dim3(1024), dim3(256), 0, 0, p, n16, y);
            },
            int(slots * 4 > 40 ? slots * 4 : 40));
        printf("read %4zu MB over %2zu distinct buffers: %8.2f us per launch  %7.1f GB/s\n", mb, slots, us,
               double(bytes) / us / 1e3);
    }
    return 0;
}
