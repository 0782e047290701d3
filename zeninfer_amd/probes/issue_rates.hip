// issue_rates.hip -- measures, on the GPU it runs on, the per-SIMD cost of the
// instruction mixes the int8 GEMM epilogue is built from: int8 and fp32
// MFMAs, plain fp32 VALU FMAs, cvt+fma pairs, and MFMAs interleaved with
// independent VALU work (to see whether the two co-execute).
//
// One workgroup per CU (96 KiB of dynamic LDS is reserved to force it), 1, 2
// or 4 waves per SIMD; every wave runs the same loop and the workgroup's time
// is taken from before its first to after its last wave (s_memtime, shader
// clock).  Build and run:
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         -o /tmp/issue_rates zeninfer_amd/probes/issue_rates.hip && /tmp/issue_rates
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
constexpr int ITERS = 2000;
constexpr int LDS_RESERVE = 98304;

#define CHECK(x)                                                                    \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));          \
            exit(1);                                                                \
        }                                                                           \
    } while (0)

template <int KIND>
__global__ void mix(float* out, unsigned long long* cyc, int seed) {
    extern __shared__ float reserve[];
    if (seed == 12345) reserve[threadIdx.x] = 1.0f;  // never true; keeps the reservation live
    float* lds_pool = reserve;  // 64 KiB of the reservation, filled below for KIND 10
    if constexpr (KIND == 10) {
        for (int i = threadIdx.x; i < 16384; i += blockDim.x) lds_pool[i] = float(i & 127);
    }
    v4i a = {seed, seed + 1, seed + 2, int(threadIdx.x)};
    v16i ci[4] = {};
    v16f cf[4] = {};
    v32f c2 = {};
    const float x0 = threadIdx.x, x1 = x0 + 1, x3 = x0 + 3, y = seed * 0.5f;
    float acc[16], acc2[16];
    for (int i = 0; i < 16; ++i) acc[i] = i * x0, acc2[i] = i * x1;
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < ITERS; ++it) {
        if constexpr (KIND == 0) {  // 4 independent v_mfma_i32_32x32x32_i8
#pragma unroll
            for (int j = 0; j < 4; ++j) ci[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, ci[j], 0, 0, 0);
        } else if constexpr (KIND == 1) {  // v_mfma_f32_32x32x1_2b_f32
#pragma unroll
            for (int j = 0; j < 4; ++j) c2 = __builtin_amdgcn_mfma_f32_32x32x1f32(x0 + j, x1, c2, 0, 0, 0);
        } else if constexpr (KIND == 2) {  // v_mfma_f32_32x32x16_bf16
            v8bf b;
            for (int q = 0; q < 8; ++q) b[q] = (__bf16)(x0 + q);
#pragma unroll
            for (int j = 0; j < 4; ++j) cf[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, b, cf[j], 0, 0, 0);
        } else if constexpr (KIND == 3) {  // fp32 fma, 16 independent chains
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[j] = fmaf(acc[j], y, x3);
        } else if constexpr (KIND == 4) {  // cvt + fma pairs (the GEMM epilogue)
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[j] = fmaf(float(ci[0][j] + r), y, acc[j]);
        } else if constexpr (KIND == 5 || KIND == 6) {  // int8 MFMA + 16 / 48 independent fma
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ci[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, ci[j], 0, 0, 0);
#pragma unroll
                for (int r = 0; r < (KIND == 5 ? 1 : 3); ++r)
#pragma unroll
                    for (int q = 0; q < 16; ++q) acc[q] = fmaf(acc[q], y, x3);
            }
        } else if constexpr (KIND == 10) {
            // the unit of KIND 8 with its operands read from LDS as the GEMM
            // does per block: two ds_read_b128 (A of both tiles), five dwords
            // of raw weights (B, with four v_alignbyte), a u16 weight scale and
            // an activation scale
            const v16i zero = {};
            const v32f szero = {};
            const int base = (int(threadIdx.x) * 5 + it * 64) & 0x3FFF;
            const v4i a0 = *reinterpret_cast<const v4i*>(&lds_pool[(base & ~3) + 0]);
            const v4i a1 = *reinterpret_cast<const v4i*>(&lds_pool[(base & ~3) + 4096]);
            unsigned t5[5];
            for (int i = 0; i < 5; ++i) t5[i] = reinterpret_cast<const unsigned*>(lds_pool)[(base + 8192 + i) & 0x3FFF];
            const unsigned dwh = reinterpret_cast<const unsigned short*>(lds_pool)[base & 0x7FFF];
            const float dx = lds_pool[(base + 12288) & 0x3FFF];
            v4i w;
            for (int i = 0; i < 4; ++i) w[i] = int(__builtin_amdgcn_alignbyte(t5[i + 1], t5[i], 2));
            v16i n0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, w, zero, 0, 0, 0);
            v16i n1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, w, zero, 0, 0, 0);
            v32f ns = __builtin_amdgcn_mfma_f32_32x32x1f32(dx, float(dwh), szero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                acc[v] = fmaf(float(n0[v]), ns[v], acc[v]);
                acc2[v] = fmaf(float(n1[v]), ns[16 + v], acc2[v]);
            }
        } else if constexpr (KIND == 8 || KIND == 9) {
            // the int8 GEMM's per-block unit for a wave's two 32x32 tiles: two
            // int8 MFMAs, one 2-block dx*dw MFMA, then cvt + fma on all 32
            // results.  8: the epilogue consumes this block's results; 9: it
            // consumes the previous block's (one-block software pipeline).
            const v16i zero = {};
            const v32f szero = {};
            v16i n0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, zero, 0, 0, 0);
            v16i n1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a + it, a, zero, 0, 0, 0);
            v32f ns = __builtin_amdgcn_mfma_f32_32x32x1f32(x0 + it, x1, szero, 0, 0, 0);
            if constexpr (KIND == 8) {
                ci[0] = n0;
                ci[1] = n1;
                c2 = ns;
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                acc[v] = fmaf(float(ci[0][v]), c2[v], acc[v]);
                acc2[v] = fmaf(float(ci[1][v]), c2[16 + v], acc2[v]);
            }
            if constexpr (KIND == 9) {
                ci[0] = n0;
                ci[1] = n1;
                c2 = ns;
            }
        } else if constexpr (KIND == 7) {  // fp32 2-block MFMA + 16 independent fma
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c2 = __builtin_amdgcn_mfma_f32_32x32x1f32(x0 + j, x1, c2, 0, 0, 0);
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[q] = fmaf(acc[q], y, x3);
            }
        }
    }
    float s = 0;
    for (int j = 0; j < 4; ++j)
        for (int v = 0; v < 16; ++v) s += float(ci[j][v]) + cf[j][v];
    for (int v = 0; v < 32; ++v) s += c2[v];
    for (int i = 0; i < 16; ++i) s += acc[i] + acc2[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
    __syncthreads();
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

template <int KIND>
void run(const char* name, int waves_per_simd, int insts_per_iter, int cus) {
    float* out;
    unsigned long long* cyc;
    const int threads = 256 * waves_per_simd;
    CHECK(hipMalloc(&out, size_t(cus) * threads * 4));
    CHECK(hipMalloc(&cyc, size_t(cus) * 8));
    CHECK(hipFuncSetAttribute((const void*)mix<KIND>, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_RESERVE));
    hipLaunchKernelGGL(mix<KIND>, dim3(cus), dim3(threads), LDS_RESERVE, 0, out, cyc, 3);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    unsigned long long* h = new unsigned long long[cus];
    CHECK(hipMemcpy(h, cyc, size_t(cus) * 8, hipMemcpyDeviceToHost));
    double m = 0;
    for (int i = 0; i < cus; ++i) m += double(h[i]);
    m /= cus;
    printf("| %-34s | %d | %7.1f |\n", name, waves_per_simd, m / (double(ITERS) * insts_per_iter * waves_per_simd));
    delete[] h;
    CHECK(hipFree(out));
    CHECK(hipFree(cyc));
}

int main() {
    hipDeviceProp_t p;
    CHECK(hipGetDeviceProperties(&p, 0));
    printf("%s (%s), %d CUs; cycles per instruction per SIMD (s_memtime)\n\n", p.name, p.gcnArchName,
           p.multiProcessorCount);
    printf("| mix (per unit) | waves/SIMD | cycles |\n|---|---|---|\n");
    const int cus = p.multiProcessorCount;
    for (int w = 1; w <= 4; w *= 2) {
        run<0>("mfma_i32_32x32x32_i8", w, 4, cus);
        run<1>("mfma_f32_32x32x1_2b_f32", w, 4, cus);
        run<2>("mfma_f32_32x32x16_bf16", w, 4, cus);
        run<3>("fp32 fma", w, 64, cus);
        run<4>("cvt_f32_i32 + fma (per instruction)", w, 32, cus);
        run<5>("i8 MFMA + 16 fma (per MFMA)", w, 4, cus);
        run<6>("i8 MFMA + 48 fma (per MFMA)", w, 4, cus);
        run<7>("f32 2b MFMA + 16 fma (per MFMA)", w, 4, cus);
        run<8>("GEMM block unit, dependent (per unit)", w, 1, cus);
        run<9>("GEMM block unit, pipelined (per unit)", w, 1, cus);
        run<10>("GEMM block unit + its LDS reads", w, 1, cus);
    }
    return 0;
}
