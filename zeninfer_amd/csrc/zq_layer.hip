// zq_layer.hip -- the non-projection kernels of a Llama-layout decoder layer,
// kept on the device between the quantised GEMV / GEMM projections:
// embedding lookup, RMSNorm, RoPE + KV-cache append, causal GQA attention,
// residual add and greedy argmax.
//
// Arithmetic follows the reference's CPU forward
// (src/adapters/dense_transformer_runtime.cpp of the reference):
//   - embedding rows are dequantised exactly (int8(q) * d for Q8_0);
//   - RMSNorm (:117-124): ss summed in double, inv = 1/sqrtf(float(ss/n)+eps),
//     y = x * inv * w;
//   - RoPE (:317-328) on adjacent pairs (llama) or half-split pairs, from a
//     cos/sin table the host builds once per position (the reference's
//     rope_table, :260-284) -- the device never computes angles;
//   - attention (:4284-4330): scores = dot(q, k) * 1/sqrt(D), max-subtracted
//     expf, denominator summed in double, out = sum_t (score_t * inv) * v_t;
//   - greedy selection (:391-403): the lowest index among the finite maxima.
// Reduction orders differ from the CPU's (parallel vs sequential); the
// double-precision sums keep the difference at the last bit of fp32.
#include "zq_device.hpp"
#include "zq_internal.hpp"

#include <math.h>

namespace zq {
namespace {

constexpr int kT = 256;

__device__ __forceinline__ double block_sum_d(double v, double* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

__device__ __forceinline__ float block_max_f(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < nw; ++i) m = fmaxf(m, red[i]);
    return m;
}

// x[t][e] = dequantised row tokens[t] of a Q8_0 table (rows of E elements).
__global__ __launch_bounds__(kT) void embed_q8_0_kernel(const uint8_t* __restrict__ table, size_t row_bytes,
                                                        const uint32_t* __restrict__ tokens, uint32_t vocab,
                                                        float* __restrict__ x, uint32_t E) {
    const uint32_t t = blockIdx.y;
    const uint32_t e = blockIdx.x * kT + threadIdx.x;
    if (e >= E) return;
    const uint32_t tok = tokens[t];
    float v = 0.0f;
    if (tok < vocab) {
        const uint8_t* blk = table + size_t(tok) * row_bytes + (e >> 5) * 34;
        v = float(int8_t(blk[2 + (e & 31)])) * half_bits_to_float(uint16_t(blk[0] | (blk[1] << 8)));
    }
    x[size_t(t) * E + e] = v;
}

// fp32 table rows
__global__ __launch_bounds__(kT) void embed_f32_kernel(const float* __restrict__ table, const uint32_t* __restrict__ tokens,
                                                       uint32_t vocab, float* __restrict__ x, uint32_t E) {
    const uint32_t t = blockIdx.y;
    const uint32_t e = blockIdx.x * kT + threadIdx.x;
    if (e >= E) return;
    const uint32_t tok = tokens[t];
    x[size_t(t) * E + e] = tok < vocab ? table[size_t(tok) * E + e] : 0.0f;
}

// One workgroup per row.
__global__ __launch_bounds__(kT) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                     float* __restrict__ y, uint32_t n, float eps) {
    __shared__ double red[kT / 64];
    const float* xr = x + size_t(blockIdx.x) * n;
    float* yr = y + size_t(blockIdx.x) * n;
    double ss = 0.0;
    for (uint32_t i = threadIdx.x; i < n; i += kT) ss += double(xr[i]) * double(xr[i]);
    ss = block_sum_d(ss, red);
    const float inv = 1.0f / sqrtf(float(ss / double(n)) + eps);
    for (uint32_t i = threadIdx.x; i < n; i += kT) yr[i] = xr[i] * inv * w[i];
}

// RoPE on q (in place) and k, then k and v appended to the caches at
// position pos0 + t.  One workgroup per token.  `pairs` rotated pairs per head:
// adjacent (x[2i], x[2i+1]) or half-split (x[i], x[i+pairs]); dimensions past
// 2*pairs are left as they are (rope(), :317-328 of the reference runtime).
__global__ __launch_bounds__(kT) void rope_kv_kernel(float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, float* __restrict__ kc,
                                                     float* __restrict__ vc, const float* __restrict__ cos_tab,
                                                     const float* __restrict__ sin_tab, const uint32_t* __restrict__ pos0,
                                                     uint32_t H, uint32_t KH, uint32_t D, uint32_t pairs, int adjacent) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = *pos0 + t;
    const float* cs = cos_tab + size_t(pos) * pairs;
    const float* sn = sin_tab + size_t(pos) * pairs;
    float* qt = q + size_t(t) * H * D;
    const float* kt = k + size_t(t) * KH * D;
    const float* vt = v + size_t(t) * KH * D;
    float* kd = kc + size_t(pos) * KH * D;
    float* vd = vc + size_t(pos) * KH * D;
    // q in place: one thread per rotated pair
    for (uint32_t j = threadIdx.x; j < H * pairs; j += kT) {
        const uint32_t h = j / pairs, i = j - h * pairs;
        float* vh = qt + size_t(h) * D;
        const uint32_t ia = adjacent ? 2 * i : i, ib = adjacent ? 2 * i + 1 : i + pairs;
        const float a = vh[ia], b = vh[ib], c = cs[i], s = sn[i];
        vh[ia] = a * c - b * s;
        vh[ib] = a * s + b * c;
    }
    // k into the cache: one thread per element, from the unrotated input
    for (uint32_t j = threadIdx.x; j < KH * D; j += kT) {
        const uint32_t h = j / D, d = j - h * D;
        const float* src = kt + size_t(h) * D;
        float r = src[d];
        if (d < 2 * pairs) {
            uint32_t i, ia, ib;
            bool first;
            if (adjacent) { i = d >> 1; ia = 2 * i; ib = ia + 1; first = (d & 1) == 0; }
            else { first = d < pairs; i = first ? d : d - pairs; ia = i; ib = i + pairs; }
            const float a = src[ia], b = src[ib], c = cs[i], s = sn[i];
            r = first ? a * c - b * s : a * s + b * c;
        }
        kd[j] = r;
        vd[j] = vt[j];
    }
}

// Causal GQA attention for query token t (position pos0 + t) of head h:
// grid (H, T), 256 threads, scores for positions [0, pos] in dynamic LDS.
// D must be a multiple of 64 and at most 256.
__global__ __launch_bounds__(kT) void attention_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                       const float* __restrict__ vc, float* __restrict__ out,
                                                       const uint32_t* __restrict__ pos0, uint32_t H, uint32_t KH,
                                                       uint32_t D, float scale) {
    extern __shared__ float scores[];
    __shared__ double red_d[kT / 64];
    __shared__ float red_f[kT / 64];
    __shared__ float part[kT];
    const uint32_t h = blockIdx.x, t = blockIdx.y;
    const uint32_t pos = *pos0 + t;
    const uint32_t kh = h / (H / KH);
    const uint32_t KW = KH * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* qh = q + (size_t(t) * H + h) * D;
    // q slice of this lane: D/64 values
    float qv[4];
    const uint32_t per = D / 64;
    for (uint32_t i = 0; i < per; ++i) qv[i] = qh[lane * per + i];
    for (uint32_t p = wave; p <= pos; p += kT / 64) {
        const float* kr = kc + size_t(p) * KW + size_t(kh) * D + lane * per;
        float s = 0.0f;
        for (uint32_t i = 0; i < per; ++i) s = fmaf(qv[i], kr[i], s);
        s = wave_sum(s);
        if (lane == 0) scores[p] = s * scale;
    }
    __syncthreads();
    float m = -INFINITY;
    for (uint32_t p = threadIdx.x; p <= pos; p += kT) m = fmaxf(m, scores[p]);
    m = block_max_f(m, red_f);
    double den = 0.0;
    for (uint32_t p = threadIdx.x; p <= pos; p += kT) {
        const float e = expf(scores[p] - m);
        scores[p] = e;
        den += double(e);
    }
    den = block_sum_d(den, red_d);  // ends with a barrier: every score is written
    const float inv = 1.0f / float(den);
    // out[d] = sum_p (score_p * inv) * v[p][d]; threads split (d, position group)
    const uint32_t groups = kT / D;  // 1, 2 or 4
    const uint32_t d = threadIdx.x % D, g = threadIdx.x / D;
    float acc = 0.0f;
    if (g < groups)
        for (uint32_t p = g; p <= pos; p += groups)
            acc = fmaf(scores[p] * inv, vc[size_t(p) * KW + size_t(kh) * D + d], acc);
    part[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < D) {
        float s = part[threadIdx.x];
        for (uint32_t i = 1; i < groups; ++i) s += part[threadIdx.x + i * D];
        out[(size_t(t) * H + h) * D + threadIdx.x] = s;
    }
}

__global__ __launch_bounds__(kT) void add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    const size_t i = size_t(blockIdx.x) * kT + threadIdx.x;
    if (i < n) x[i] += y[i];
}

// One workgroup of 1024 threads: lowest index among the finite maxima.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, uint32_t n, uint32_t* __restrict__ out) {
    __shared__ float bv[16];
    __shared__ uint32_t bi[16];
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
        const float v = x[i];
        if (isfinite(v) && (v > best || idx == 0xffffffffu)) {
            if (v > best || idx == 0xffffffffu) { best = v; idx = i; }
        }
    }
    // wave reduce: larger value wins, ties -> lower index
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const uint32_t oi = __shfl_xor(idx, o);
        if (oi != 0xffffffffu && (idx == 0xffffffffu || ov > best || (ov == best && oi < idx))) { best = ov; idx = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < 16; ++i)
            if (bi[i] != 0xffffffffu && (idx == 0xffffffffu || bv[i] > best || (bv[i] == best && bi[i] < idx))) {
                best = bv[i];
                idx = bi[i];
            }
        *out = idx == 0xffffffffu ? 0u : idx;
    }
}

}  // namespace

hipError_t launch_embed(int fmt, const void* table, const uint32_t* tokens, uint32_t vocab, float* x, uint32_t E,
                        uint32_t T, hipStream_t stream) {
    if (!table || !tokens || !x || !E || !T) return hipErrorInvalidValue;
    const dim3 grid((E + kT - 1) / kT, T);
    if (fmt == kQ8_0) {
        if (E % 32) return hipErrorInvalidValue;
        hipLaunchKernelGGL(embed_q8_0_kernel, grid, dim3(kT), 0, stream, static_cast<const uint8_t*>(table),
                           row_bytes(kQ8_0, E), tokens, vocab, x, E);
    } else if (fmt == 0) {
        hipLaunchKernelGGL(embed_f32_kernel, grid, dim3(kT), 0, stream, static_cast<const float*>(table), tokens, vocab,
                           x, E);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, uint32_t rows, uint32_t n, float eps,
                          hipStream_t stream) {
    if (!x || !w || !y || !rows || !n) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kT), 0, stream, x, w, y, n, eps);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float* q, const float* k, const float* v, float* kc, float* vc, const float* cos_tab,
                          const float* sin_tab, const uint32_t* pos0, uint32_t T, uint32_t H, uint32_t KH, uint32_t D,
                          uint32_t pairs, bool adjacent, hipStream_t stream) {
    if (!q || !k || !v || !kc || !vc || !cos_tab || !sin_tab || !pos0 || !T || !H || !KH || !D || !pairs ||
        pairs > D / 2 || H % KH)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_kv_kernel, dim3(T), dim3(kT), 0, stream, q, k, v, kc, vc, cos_tab, sin_tab, pos0, H, KH, D,
                       pairs, adjacent ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, const uint32_t* pos0,
                            uint32_t T, uint32_t H, uint32_t KH, uint32_t D, uint32_t max_pos, float scale,
                            hipStream_t stream) {
    if (!q || !kc || !vc || !out || !pos0 || !T || !H || !KH || H % KH || D % 64 || D > 256 || !max_pos)
        return hipErrorInvalidValue;
    const size_t lds = size_t(max_pos) * sizeof(float);
    if (lds > 96 * 1024) return hipErrorInvalidValue;  // positions are bounded by the cache capacity
    hipLaunchKernelGGL(attention_kernel, dim3(H, T), dim3(kT), lds, stream, q, kc, vc, out, pos0, H, KH, D, scale);
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t stream) {
    if (!x || !y || !n) return hipErrorInvalidValue;
    hipLaunchKernelGGL(add_kernel, dim3(uint32_t((n + kT - 1) / kT)), dim3(kT), 0, stream, x, y, n);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* x, uint32_t n, uint32_t* out, hipStream_t stream) {
    if (!x || !n || !out) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, stream, x, n, out);
    return hipGetLastError();
}

}  // namespace zq
