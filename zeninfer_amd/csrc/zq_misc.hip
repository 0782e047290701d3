// zq_misc.hip -- dequantisation (bit-exact tier) and synthetic-input
// generation on the device.
#include "zq_device.hpp"
#include "zq_internal.hpp"

namespace zq {
namespace {

constexpr int kThreads = 256;

// One thread per 32-element run; out is row-major fp32 [rows][cols].
template <int FMT>
__global__ __launch_bounds__(kThreads) void dequantize_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                              size_t rows, size_t cols) {
    const size_t runs_per_row = cols / 32;
    const size_t id = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (id >= rows * runs_per_row) return;
    const size_t r = id / runs_per_row, run = id % runs_per_row;
    float o[32];
    dequant32<FMT>(w + r * row_bytes_dev(FMT, cols), uint32_t(run * 32), o);
    float4* dst = reinterpret_cast<float4*>(out + r * cols + run * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

// ------------------------------------------------------ synthetic data ---
// Counter-based SplitMix64: draw i of stream `seed` equals the (i+1)-th
// output of the sequential generator seeded with `seed`.
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// Box-Muller in double from draws 2i and 2i+1.
__device__ __forceinline__ double normal_at(uint64_t seed, uint64_t i) {
    const uint64_t a = splitmix64_at(seed, 2 * i), b = splitmix64_at(seed, 2 * i + 1);
    const double u1 = (double(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = double(b >> 11) * (1.0 / 9007199254740992.0);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) { return __half_as_ushort(__float2half_rn(v)); }

__device__ __forceinline__ uint64_t seed_quant(uint64_t s) { return s ^ 0x51ull; }
__device__ __forceinline__ uint64_t seed_scale(uint64_t s) { return s ^ 0x5CA1Eull; }
__device__ __forceinline__ uint64_t seed_sub(uint64_t s) { return s ^ 0x5B5Cull; }

// One thread per block / super-block.  Recipes:
//   Q8_0: q ~ U{-127..127}, d = fp16(|N(0,1)| * 0.002)
//   Q4_0: nibble ~ U{0..15}, d = fp16(|N(0,1)| * 0.02)
//   Q6_K: q ~ U{0..63}, sc ~ U{-32..31}, d = fp16(|N(0,1)| * 0.001)
//   Q4_K / Q5_K: d, dmin = fp16(|N(0,1)| * 0.001) (draws 2g, 2g+1), the 12
//     packed scale bytes, the Q5_K fifth-bit bytes and the 128 nibble bytes
//     each a uniform byte
template <int FMT>
__global__ __launch_bounds__(kThreads) void synth_kernel(uint64_t seed, uint8_t* __restrict__ w, size_t nblocks) {
    const size_t g = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= nblocks) return;
    if constexpr (FMT == kQ8_0) {
        uint8_t* p = w + g * 34;
        const uint16_t h = f32_to_f16_bits(float(fabs(normal_at(seed_scale(seed), g)) * 0.002));
        p[0] = uint8_t(h); p[1] = uint8_t(h >> 8);
        for (int j = 0; j < 32; ++j) {
            const uint64_t u = splitmix64_at(seed_quant(seed), g * 32 + j);
            p[2 + j] = uint8_t(int8_t(int((u >> 32) % 255u) - 127));
        }
    } else if constexpr (FMT == kQ4_0) {
        uint8_t* p = w + g * 18;
        const uint16_t h = f32_to_f16_bits(float(fabs(normal_at(seed_scale(seed), g)) * 0.02));
        p[0] = uint8_t(h); p[1] = uint8_t(h >> 8);
        for (int j = 0; j < 16; ++j) p[2 + j] = uint8_t(splitmix64_at(seed_quant(seed), g * 16 + j) >> 56);
    } else if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
        constexpr int BB = FMT == kQ5_K ? 176 : 144, QS = FMT == kQ5_K ? 48 : 16;
        uint8_t* p = w + g * BB;
        const uint16_t d = f32_to_f16_bits(float(fabs(normal_at(seed_scale(seed), 2 * g)) * 0.001));
        const uint16_t m = f32_to_f16_bits(float(fabs(normal_at(seed_scale(seed), 2 * g + 1)) * 0.001));
        p[0] = uint8_t(d); p[1] = uint8_t(d >> 8); p[2] = uint8_t(m); p[3] = uint8_t(m >> 8);
        for (int i = 0; i < 12; ++i) p[4 + i] = uint8_t(splitmix64_at(seed_sub(seed), g * 12 + i) >> 56);
        for (int i = 16; i < QS; ++i) p[i] = uint8_t(splitmix64_at(seed_quant(seed) ^ 0xB17ull, g * 32 + (i - 16)) >> 56);
        for (int i = 0; i < 128; ++i) p[QS + i] = uint8_t(splitmix64_at(seed_quant(seed), g * 128 + i) >> 56);
    } else {
        uint8_t* p = w + g * 210;
        for (int i = 0; i < 16; ++i) {
            const uint64_t u = splitmix64_at(seed_sub(seed), g * 16 + i);
            p[192 + i] = uint8_t(int8_t(int((u >> 32) % 64u) - 32));
        }
        const uint16_t h = f32_to_f16_bits(float(fabs(normal_at(seed_scale(seed), g)) * 0.001));
        p[208] = uint8_t(h); p[209] = uint8_t(h >> 8);
        for (int half = 0; half < 2; ++half)
            for (int l = 0; l < 32; ++l) {
                unsigned q[4];
                for (int grp = 0; grp < 4; ++grp) {
                    const size_t e = size_t(half) * 128 + size_t(grp) * 32 + size_t(l);
                    q[grp] = unsigned(splitmix64_at(seed_quant(seed), g * 256 + e) >> 58);
                }
                p[half * 64 + l] = uint8_t((q[0] & 15u) | ((q[2] & 15u) << 4));
                p[half * 64 + 32 + l] = uint8_t((q[1] & 15u) | ((q[3] & 15u) << 4));
                p[128 + half * 32 + l] = uint8_t((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6));
            }
    }
}

__global__ __launch_bounds__(kThreads) void synth_normal_kernel(uint64_t seed, float* __restrict__ out, size_t n) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) out[i] = float(normal_at(seed, i));
}

// SiLU(gate) * up, the FFN activation between gate|up and down
// (g / (1 + e^-g)) * u.
// With xq: also the int8 activations of o for the GEMM that reads it
// (n % 32 == 0, so each 32-lane half-wave is one whole block, live or not).
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                            float* __restrict__ o, size_t n, int8_t* __restrict__ xq,
                                                            float* __restrict__ xs) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (xq) {
        if (i >= n) return;
        const float gv = g[i];
        const float v = gv / (1.0f + expf(-gv)) * u[i];
        if (o) o[i] = v;  // null with xq: only the int8 form is wanted
        quantize_lane_block32(v, xq + i, xs + i / 32);
        return;
    }
    if (i < n) {
        const float gv = g[i];
        o[i] = gv / (1.0f + expf(-gv)) * u[i];
    }
}

// The same for n % 4 == 0 and 16-byte aligned operands, four elements per
// lane (float4 loads and stores; 8 lanes per quantiser block).
__global__ __launch_bounds__(kThreads) void silu_mul4_kernel(const float4* __restrict__ g, const float4* __restrict__ u,
                                                             float4* __restrict__ o, size_t n4, int8_t* __restrict__ xq,
                                                             float* __restrict__ xs) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n4) return;  // n % 32 == 0 with xq: whole 8-lane blocks leave together
    const float4 a = g[i], b = u[i];
    auto f = [](float gv, float uv) { return gv / (1.0f + expf(-gv)) * uv; };
    const float4 v = make_float4(f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w));
    if (o) o[i] = v;  // null with xq: only the int8 form is wanted
    if (xq) quantize_lane4_block32(v, xq + 4 * i, xs + i / 8);
}

}  // namespace

namespace {
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));
// Int8 MFMA rate probe: every wave of every CU issues `iters` x 4
// independent v_mfma_i32_32x32x32_i8; wave 0 of each workgroup records the
// shader-clock counter (s_memtime) and the 100 MHz constant clock
// (s_memrealtime) around the loop.  out[4*wg] = shader cycles, [4*wg+1] =
// 100 MHz ticks, [4*wg+2] = a sink of the results (so the loop is kept).
__global__ __launch_bounds__(256) void mfma_probe_kernel(uint64_t* out, uint32_t iters, int seed) {
    v4i_t a = {seed, seed + 1, seed + 2, int(threadIdx.x)};
    v16i_t c[4] = {};
    __syncthreads();
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c[j], 0, 0, 0);
    }
    int sink = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) sink ^= c[j][v];
    __syncthreads();
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[4 * blockIdx.x] = t1 - t0;
        out[4 * blockIdx.x + 1] = r1 - r0;
    }
    if (sink == 0x7FFFFFFF) out[4 * blockIdx.x + 2] = uint64_t(sink);
}
}  // namespace

// Plain streaming read, the yardstick of the GEMV rooflines: `bytes` (a
// multiple of 16) read once with non-temporal 16-byte loads, each workgroup
// a contiguous share, two loads per thread in flight per step; the xor of
// everything is stored only if it equals a value no input produces here,
// so the loads cannot be dropped.
constexpr uint32_t kReadProbeWgs = 4096;
typedef uint32_t u32x4_probe_t __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(kThreads) void read_probe_kernel(const u32x4_probe_t* __restrict__ w, size_t n16,
                                                              uint32_t* sink) {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t b = size_t(blockIdx.x) * per, e = min(b + per, n16);
    uint32_t acc = 0;
    for (size_t i = b + threadIdx.x; i < e; i += 2 * kThreads) {
        const size_t j = i + kThreads;
        const u32x4_probe_t v0 = __builtin_nontemporal_load(&w[i]);
        const u32x4_probe_t v1 = j < e ? __builtin_nontemporal_load(&w[j]) : u32x4_probe_t{0, 0, 0, 0};
        acc ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

hipError_t launch_read_probe(const void* buf, size_t bytes, uint32_t* sink, hipStream_t stream) {
    if (!buf || !sink || !bytes || bytes % 16 || (reinterpret_cast<uintptr_t>(buf) & 15u)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(read_probe_kernel, dim3(kReadProbeWgs), dim3(kThreads), 0, stream, static_cast<const u32x4_probe_t*>(buf),
                       bytes / 16, sink);
    return hipGetLastError();
}
size_t read_probe_sink_bytes() { return size_t(kReadProbeWgs) * sizeof(uint32_t); }

hipError_t launch_mfma_probe(uint64_t* out, uint32_t wgs, uint32_t iters, hipStream_t stream) {
    if (!out || !wgs || !iters) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(wgs), dim3(256), 0, stream, out, iters, 3);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* gate, const float* up, float* out, size_t n, hipStream_t stream, int8_t* xq,
                           float* xs) {
    if (!gate || !up || (!out && !xq) || !n || (xq && (!xs || n % 32))) return hipErrorInvalidValue;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (n % 4 == 0 && a16(gate) && a16(up) && a16(out) && (reinterpret_cast<uintptr_t>(xq) & 3u) == 0) {
        const size_t n4 = n / 4;
        hipLaunchKernelGGL(silu_mul4_kernel, dim3(static_cast<uint32_t>((n4 + kThreads - 1) / kThreads)), dim3(kThreads),
                           0, stream, reinterpret_cast<const float4*>(gate), reinterpret_cast<const float4*>(up),
                           reinterpret_cast<float4*>(out), n4, xq, xs);
        return hipGetLastError();
    }
    const dim3 grid(static_cast<uint32_t>((n + kThreads - 1) / kThreads));
    hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(kThreads), 0, stream, gate, up, out, n, xq, xs);
    return hipGetLastError();
}

hipError_t launch_dequantize(int fmt, const uint8_t* w, float* out, size_t rows, size_t cols, hipStream_t stream) {
    if (!w || !out || !rows || !row_bytes(fmt, cols) || (reinterpret_cast<uintptr_t>(w) & 1u) ||
        (reinterpret_cast<uintptr_t>(out) & 15u))
        return hipErrorInvalidValue;
    if ((fmt == kQ4_K || fmt == kQ5_K) && (reinterpret_cast<uintptr_t>(w) & 3u)) return hipErrorInvalidValue;
    const size_t n = rows * (cols / 32);
    const dim3 grid(static_cast<uint32_t>((n + kThreads - 1) / kThreads));
    switch (fmt) {
    case kQ8_0: hipLaunchKernelGGL(dequantize_kernel<kQ8_0>, grid, dim3(kThreads), 0, stream, w, out, rows, cols); break;
    case kQ4_0: hipLaunchKernelGGL(dequantize_kernel<kQ4_0>, grid, dim3(kThreads), 0, stream, w, out, rows, cols); break;
    case kQ6_K: hipLaunchKernelGGL(dequantize_kernel<kQ6_K>, grid, dim3(kThreads), 0, stream, w, out, rows, cols); break;
    case kQ4_K: hipLaunchKernelGGL(dequantize_kernel<kQ4_K>, grid, dim3(kThreads), 0, stream, w, out, rows, cols); break;
    case kQ5_K: hipLaunchKernelGGL(dequantize_kernel<kQ5_K>, grid, dim3(kThreads), 0, stream, w, out, rows, cols); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_synth_weights(int fmt, uint64_t seed, uint8_t* w, size_t rows, size_t cols, hipStream_t stream) {
    if (!w || !rows || !row_bytes(fmt, cols)) return hipErrorInvalidValue;
    const size_t nblocks = rows * cols / (fmt == kQ4_0 || fmt == kQ8_0 ? 32 : 256);
    const dim3 grid(static_cast<uint32_t>((nblocks + kThreads - 1) / kThreads));
    switch (fmt) {
    case kQ8_0: hipLaunchKernelGGL(synth_kernel<kQ8_0>, grid, dim3(kThreads), 0, stream, seed, w, nblocks); break;
    case kQ4_0: hipLaunchKernelGGL(synth_kernel<kQ4_0>, grid, dim3(kThreads), 0, stream, seed, w, nblocks); break;
    case kQ6_K: hipLaunchKernelGGL(synth_kernel<kQ6_K>, grid, dim3(kThreads), 0, stream, seed, w, nblocks); break;
    case kQ4_K: hipLaunchKernelGGL(synth_kernel<kQ4_K>, grid, dim3(kThreads), 0, stream, seed, w, nblocks); break;
    case kQ5_K: hipLaunchKernelGGL(synth_kernel<kQ5_K>, grid, dim3(kThreads), 0, stream, seed, w, nblocks); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_synth_normal(uint64_t seed, float* out, size_t n, hipStream_t stream) {
    if (!out || !n) return hipErrorInvalidValue;
    const dim3 grid(static_cast<uint32_t>((n + kThreads - 1) / kThreads));
    hipLaunchKernelGGL(synth_normal_kernel, grid, dim3(kThreads), 0, stream, seed, out, n);
    return hipGetLastError();
}

}  // namespace zq
