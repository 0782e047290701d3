// zq_gemm.hip -- quantised prefill GEMM for gfx950.
//
// Y[t][n] = sum_k X[t][k] * W[n][k]   (token-major output, include/zen/quant.h:28-30
// of the reference).  Two arithmetic modes:
//
//  * int8 activations (Q8_0 and Q4_0).  X is first quantised per 32-element
//    block exactly as the reference CPU quantiser does (kernels/avx2.cpp:502-524:
//    d = amax/127, inv = 1/d, round half away from zero).  Each 32-block dot is
//    one v_mfma_i32_32x32x32_i8 (K = 32 = one GGML block, so the int32 result
//    is exactly the per-block integer dot), and the epilogue adds
//    float(dot) * (d_x * d_w) into an fp32 accumulator per output element, the
//    arithmetic of gemv_q8_0_avx2_int8_prequant (kernels/avx2.cpp:562-585) and
//    of the D3D12 int8 GEMM (shaders/q8_0_gemm_i8.hlsl:249-257).
//
//  * fp32 activations (all formats; the reference CPU arithmetic).  Weights
//    are dequantised exactly into LDS (the reference's dequantize values) and
//    multiplied with v_mfma_f32_32x32x2_f32 in fp32.
//
// Tiling: a 256-thread workgroup computes a 128 (tokens) x 128 (weight rows)
// tile with 4 waves in 2x2, each wave 2x2 MFMA tiles of 32x32.  Weight rows
// are read in their native GGML layout and converted while being staged into
// LDS (one conversion per weight element per workgroup, amortised over 128
// tokens).  Workgroup ids are remapped so that the workgroups a given XCD
// receives (ids congruent mod 8) walk the token tiles of one weight panel
// before moving on, keeping that panel in the XCD's L2.
#include "zq_device.hpp"
#include "zq_internal.hpp"

namespace zq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BM = 128;             // tokens per tile
constexpr int BN = 128;             // weight rows per tile
constexpr int KB = 4;               // 32-element blocks per K stage
constexpr int ROWB = KB * 32 + 16;  // LDS bytes per tile row (16 B pad)

// ------------------------------------------------- activation quantiser ---
// One thread per 32-element block.  Bit-exact with kernels/avx2.cpp:502-524.
__device__ __forceinline__ int round_half_away(float v) {
    const float t = truncf(v);
    const float f = v - t;  // exact for |v| < 2^23
    return static_cast<int>(t) + (f >= 0.5f ? 1 : (f <= -0.5f ? -1 : 0));
}

__global__ __launch_bounds__(kThreads) void quantize_acts_kernel(const float* __restrict__ X, int8_t* __restrict__ xq,
                                                                 float* __restrict__ xs, size_t nblocks) {
    const size_t b = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (b >= nblocks) return;
    const float4* src = reinterpret_cast<const float4*>(X + b * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = src[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    xs[b] = d;
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float t = v[4 * i + k] * inv;
            t = t > 127.0f ? 127.0f : (t < -127.0f ? -127.0f : t);
            w |= (uint32_t(round_half_away(t)) & 0xffu) << (8 * k);
        }
        packed[i] = w;
    }
    uint4* dst = reinterpret_cast<uint4*>(xq + b * 32);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

// ------------------------------------------------------- tile mapping ---
__device__ __forceinline__ void tile_of(uint32_t tiles_m, uint32_t tiles_n, uint32_t& tm, uint32_t& tn) {
    const uint32_t total = tiles_m * tiles_n;
    uint32_t slot = blockIdx.x;
    if (total % 8u == 0) {
        const uint32_t per_xcd = total / 8u;
        slot = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    }
    tn = slot / tiles_m;
    tm = slot % tiles_m;
}

// ------------------------------------------------------- int8 GEMM -------
// Weight staging for one (row, block pair) into LDS as int8 + fp32 scales.
// Q8_0 pair (68 B): block a quants are bytes 2..33 (alignbyte by 2), block b
// quants are dwords 9..16.  Q4_0 pair (36 B): nibble bytes per block become
// 32 int8 values n-8 (elements 0..15 = low nibbles, 16..31 = high nibbles).
template <int FMT>
__device__ __forceinline__ void stage_weight_pair(const uint8_t* src, bool valid, int8_t* lds_row, float& d0,
                                                  float& d1) {
    uint32_t out[16];
    if (FMT == kQ8_0) {
        uint32_t q[17];
        const uint32_t* s = reinterpret_cast<const uint32_t*>(src);
#pragma unroll
        for (int i = 0; i < 17; ++i) q[i] = valid ? s[i] : 0u;
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) out[8 + i] = q[9 + i];
        d0 = half_bits_to_float(q[0]);
        d1 = half_bits_to_float(q[8] >> 16);
    } else {
        uint32_t q[9];
        const uint32_t* s = reinterpret_cast<const uint32_t*>(src);
#pragma unroll
        for (int i = 0; i < 9; ++i) q[i] = valid ? s[i] : 0x88888888u;
        uint32_t a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], 2);
            b[i] = q[5 + i];
        }
        // byte-wise n - 8 for n in [0,15]: ((n | 0x80) - 8) ^ 0x80, no borrow across bytes
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[i] = (((a[i] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
            out[4 + i] = ((((a[i] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
            out[8 + i] = (((b[i] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
            out[12 + i] = ((((b[i] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        }
        d0 = half_bits_to_float(q[0]);
        d1 = half_bits_to_float(q[4] >> 16);
    }
    if (!valid) { d0 = 0.0f; d1 = 0.0f; }
    uint4* dst = reinterpret_cast<uint4*>(lds_row);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
}

// DOTS = true is the bit-exact test mode: instead of accumulating, the
// kernel stores every per-block int32 MFMA result to dots[(m*N + n)*nb + b].
template <int FMT, bool DOTS>
__global__ __launch_bounds__(kThreads) void gemm_i8_kernel(const uint8_t* __restrict__ W, const int8_t* __restrict__ XQ,
                                                           const float* __restrict__ XS, float* __restrict__ Y,
                                                           int32_t* __restrict__ dots, uint32_t M, uint32_t N,
                                                           uint32_t K, uint32_t tiles_m, uint32_t tiles_n) {
    constexpr uint32_t PB = FMT == kQ8_0 ? 68 : 36;  // bytes per block pair
    __shared__ __align__(16) int8_t As[BM * ROWB];
    __shared__ __align__(16) int8_t Bs[BN * ROWB];
    __shared__ __align__(16) float Sx[KB][BM];
    __shared__ __align__(16) float Sw[KB][BN];

    uint32_t tm, tn;
    tile_of(tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t nb = K >> 5;
    const uint32_t rb = (nb >> 1) * PB;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lh = lane >> 5;

    // loader coordinates
    const int ld_row = tid >> 1, ld_half = tid & 1;
    const uint32_t a_row = min(m0 + ld_row, M - 1);
    const uint32_t b_row = min(n0 + ld_row, N - 1);
    const int8_t* a_src = XQ + size_t(a_row) * K;
    const uint8_t* b_src = W + size_t(b_row) * rb;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    for (uint32_t kb = 0; kb < nb; kb += KB) {
        __syncthreads();
        // activations: 64 bytes (2 blocks) per thread
        {
            const uint32_t blk = kb + 2 * ld_half;
            const bool valid = blk < nb;
            const uint4* s = reinterpret_cast<const uint4*>(a_src + size_t(blk) * 32);
            uint4* d = reinterpret_cast<uint4*>(As + ld_row * ROWB + ld_half * 64);
#pragma unroll
            for (int i = 0; i < 4; ++i) d[i] = valid ? s[i] : make_uint4(0, 0, 0, 0);
        }
        // activation scales: KB*BM = 512 floats, 2 per thread
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int idx = tid + r * kThreads;
            const int kk = idx / BM, row = idx % BM;
            const uint32_t blk = kb + kk;
            Sx[kk][row] = blk < nb ? XS[size_t(min(m0 + row, M - 1)) * nb + blk] : 0.0f;
        }
        // weights: one block pair per thread
        {
            const uint32_t blk = kb + 2 * ld_half;
            const bool valid = blk < nb;
            float d0, d1;
            stage_weight_pair<FMT>(b_src + size_t(blk >> 1) * PB, valid, Bs + ld_row * ROWB + ld_half * 64, d0, d1);
            Sw[2 * ld_half][ld_row] = d0;
            Sw[2 * ld_half + 1][ld_row] = d1;
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            v4i a[2], w[2];
            float sw[2];
            float sx[2][16];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                a[i] = *reinterpret_cast<const v4i*>(As + (wm * 64 + i * 32 + l32) * ROWB + b * 32 + lh * 16);
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 s4 = *reinterpret_cast<const float4*>(&Sx[b][wm * 64 + i * 32 + 8 * g + 4 * lh]);
                    sx[i][4 * g] = s4.x; sx[i][4 * g + 1] = s4.y; sx[i][4 * g + 2] = s4.z; sx[i][4 * g + 3] = s4.w;
                }
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                w[j] = *reinterpret_cast<const v4i*>(Bs + (wn * 64 + j * 32 + l32) * ROWB + b * 32 + lh * 16);
                sw[j] = Sw[b][wn * 64 + j * 32 + l32];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], w[j], zero, 0, 0, 0);
                    if constexpr (DOTS) {
                        const uint32_t n = n0 + wn * 64 + j * 32 + l32;
                        const uint32_t blk = kb + b;
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                            if (m < M && n < N && blk < nb) dots[(size_t(m) * N + n) * nb + blk] = c[v];
                        }
                    } else {
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(float(c[v]), sx[i][v] * sw[j], acc[i][j][v]);
                    }
                }
        }
    }
    if constexpr (DOTS) return;
    // store: lane holds column n = l32 and token rows 8g + 4*lh + r
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64 + j * 32 + l32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (m < M && n < N) Y[size_t(m) * N + n] = acc[i][j][v];
            }
        }
}

// ------------------------------------------------------- fp32 GEMM -------
constexpr int FK = 32;          // K elements per fp32 stage
constexpr int FROW = FK + 4;    // LDS floats per row (pad)

template <int FMT>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                            float* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
                                                            uint32_t tiles_m, uint32_t tiles_n) {
    __shared__ __align__(16) float As[BM * FROW];
    __shared__ __align__(16) float Bs[BN * FROW];
    uint32_t tm, tn;
    tile_of(tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const size_t rb = row_bytes_dev(FMT, K);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lh = lane >> 5;
    const int ld_row = tid >> 1, ld_half = tid & 1;
    const float* a_src = X + size_t(min(m0 + ld_row, M - 1)) * K;
    const uint8_t* b_src = W + size_t(min(n0 + ld_row, N - 1)) * rb;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    for (uint32_t k0 = 0; k0 < K; k0 += FK) {
        __syncthreads();
        {
            const float4* s = reinterpret_cast<const float4*>(a_src + k0 + ld_half * 16);
            float4* d = reinterpret_cast<float4*>(As + ld_row * FROW + ld_half * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) d[i] = s[i];
        }
        if (ld_half == 0) {
            float w[32];
            dequant32<FMT>(b_src, k0, w);
            float4* d = reinterpret_cast<float4*>(Bs + ld_row * FROW);
#pragma unroll
            for (int i = 0; i < 8; ++i) d[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < FK; kk += 2) {
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = As[(wm * 64 + i * 32 + l32) * FROW + kk + lh];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = Bs[(wn * 64 + j * 32 + l32) * FROW + kk + lh];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64 + j * 32 + l32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (m < M && n < N) Y[size_t(m) * N + n] = acc[i][j][v];
            }
        }
}

}  // namespace

hipError_t launch_quantize_acts(const float* X, int8_t* xq, float* xs, size_t M, size_t K, hipStream_t stream) {
    if (!X || !xq || !xs || !M || !K || K % 32) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(X) & 15u) || (reinterpret_cast<uintptr_t>(xq) & 15u)) return hipErrorInvalidValue;
    const size_t nblocks = M * (K / 32);
    const size_t grid = (nblocks + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(quantize_acts_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream, X, xq, xs,
                       nblocks);
    return hipGetLastError();
}

static hipError_t launch_i8_common(int fmt, const uint8_t* w, const int8_t* xq, const float* xs, float* Y,
                                   int32_t* dots, size_t M, size_t N, size_t K, hipStream_t stream) {
    if (!w || !xq || !M || !N || !K || K % 64 || M > (1u << 24) || N > (1u << 24) || K > (1u << 24))
        return hipErrorInvalidValue;
    if (fmt != kQ8_0 && fmt != kQ4_0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(w) & 3u) || (reinterpret_cast<uintptr_t>(xq) & 15u)) return hipErrorInvalidValue;
    const uint32_t tiles_m = static_cast<uint32_t>((M + BM - 1) / BM);
    const uint32_t tiles_n = static_cast<uint32_t>((N + BN - 1) / BN);
    const dim3 grid(tiles_m * tiles_n);
    const uint32_t m = uint32_t(M), n = uint32_t(N), k = uint32_t(K);
    if (dots) {
        if (fmt == kQ8_0)
            hipLaunchKernelGGL((gemm_i8_kernel<kQ8_0, true>), grid, dim3(kThreads), 0, stream, w, xq, xs, Y, dots, m, n,
                               k, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((gemm_i8_kernel<kQ4_0, true>), grid, dim3(kThreads), 0, stream, w, xq, xs, Y, dots, m, n,
                               k, tiles_m, tiles_n);
    } else {
        if (!xs || !Y) return hipErrorInvalidValue;
        if (fmt == kQ8_0)
            hipLaunchKernelGGL((gemm_i8_kernel<kQ8_0, false>), grid, dim3(kThreads), 0, stream, w, xq, xs, Y, dots, m,
                               n, k, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL((gemm_i8_kernel<kQ4_0, false>), grid, dim3(kThreads), 0, stream, w, xq, xs, Y, dots, m,
                               n, k, tiles_m, tiles_n);
    }
    return hipGetLastError();
}

hipError_t launch_gemm_i8(int fmt, const uint8_t* w, const int8_t* xq, const float* xs, float* Y, size_t M, size_t N,
                          size_t K, hipStream_t stream) {
    return launch_i8_common(fmt, w, xq, xs, Y, nullptr, M, N, K, stream);
}

hipError_t launch_block_dots(int fmt, const uint8_t* w, const int8_t* xq, int32_t* out, size_t M, size_t N, size_t K,
                             hipStream_t stream) {
    if (!out) return hipErrorInvalidValue;
    return launch_i8_common(fmt, w, xq, nullptr, nullptr, out, M, N, K, stream);
}

hipError_t launch_gemm_f32(int fmt, const uint8_t* w, const float* X, float* Y, size_t M, size_t N, size_t K,
                           hipStream_t stream) {
    if (!w || !X || !Y || !M || !N || !row_bytes(fmt, K) || M > (1u << 24) || N > (1u << 24) || K > (1u << 24))
        return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(w) & 1u) || (reinterpret_cast<uintptr_t>(X) & 15u)) return hipErrorInvalidValue;
    const uint32_t tiles_m = static_cast<uint32_t>((M + BM - 1) / BM);
    const uint32_t tiles_n = static_cast<uint32_t>((N + BN - 1) / BN);
    const dim3 grid(tiles_m * tiles_n);
    switch (fmt) {
    case kQ8_0:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ8_0>, grid, dim3(kThreads), 0, stream, w, X, Y, uint32_t(M), uint32_t(N),
                           uint32_t(K), tiles_m, tiles_n);
        break;
    case kQ4_0:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ4_0>, grid, dim3(kThreads), 0, stream, w, X, Y, uint32_t(M), uint32_t(N),
                           uint32_t(K), tiles_m, tiles_n);
        break;
    case kQ6_K:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ6_K>, grid, dim3(kThreads), 0, stream, w, X, Y, uint32_t(M), uint32_t(N),
                           uint32_t(K), tiles_m, tiles_n);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace zq
