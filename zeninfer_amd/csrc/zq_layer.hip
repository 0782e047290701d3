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
#include <stdlib.h>

namespace zq {
namespace {

constexpr int kT = 256;

__device__ __forceinline__ double block_sum_d(double v, double* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

__device__ __forceinline__ float block_max_f(float v, float* red) {
    v = wave_max(v);
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

// One workgroup of 1024 threads per row.  With ADD the residual update
// x += r comes first (x is written back) and the norm is of the updated row.
constexpr int kNormT = 1024;
template <bool ADD>
__global__ __launch_bounds__(kNormT) void rmsnorm_kernel(float* __restrict__ x, const float* __restrict__ r,
                                                         const float* __restrict__ w, float* __restrict__ y, uint32_t n,
                                                         float eps, int8_t* __restrict__ xq, float* __restrict__ xs,
                                                         uint32_t rsplit) {
    __shared__ double red[kNormT / 64];
    float* xr = x + size_t(blockIdx.x) * n;
    float* yr = y ? y + size_t(blockIdx.x) * n : nullptr;  // null with xq: only the int8 form is wanted
    const float* rr = ADD ? r + size_t(blockIdx.x) * n : nullptr;
    double ss = 0.0;
    for (uint32_t i = threadIdx.x; i < n; i += kNormT) {
        float v = xr[i];
        if constexpr (ADD) {
            float t = rr[i];  // r's planes summed in split order (splitk_reduce_kernel's)
            for (uint32_t s = 1; s < rsplit; ++s) t += rr[size_t(s) * gridDim.x * n + i];
            v += t;
            xr[i] = v;
        }
        ss += double(v) * double(v);
    }
    ss = block_sum_d(ss, red);
    const float inv = 1.0f / sqrtf(float(ss / double(n)) + eps);
    if (xq) {  // also the int8 activations of y for the GEMMs that read it (n % 32 == 0: whole blocks per half-wave)
        int8_t* qr = xq + size_t(blockIdx.x) * n;
        float* sr = xs + size_t(blockIdx.x) * (n / 32);
        for (uint32_t i = threadIdx.x; i < n; i += kNormT) {
            const float v = xr[i] * inv * w[i];
            if (yr) yr[i] = v;
            quantize_lane_block32(v, qr + i, sr + i / 32);
        }
        return;
    }
    for (uint32_t i = threadIdx.x; i < n; i += kNormT) yr[i] = xr[i] * inv * w[i];
}

// rmsnorm_kernel for n % 4 == 0, n <= 4 * kNormV * kNormT, 16-byte aligned
// rows: every load of a row (x, r, w) is issued up front as float4, the row
// stays in registers across the reduction, so the row costs one memory
// round trip.  Same arithmetic per element (the double sum of squares in
// another order).
constexpr int kNormV = 4;
template <bool ADD>
__global__ __launch_bounds__(kNormT) void rmsnorm4_kernel(float* __restrict__ x, const float* __restrict__ r,
                                                          const float* __restrict__ w, float* __restrict__ y, uint32_t n,
                                                          float eps, int8_t* __restrict__ xq, float* __restrict__ xs,
                                                          uint32_t rsplit) {
    __shared__ double red[kNormT / 64];
    const uint32_t n4 = n / 4;
    float4* xr = reinterpret_cast<float4*>(x + size_t(blockIdx.x) * n);
    float4* yr = y ? reinterpret_cast<float4*>(y + size_t(blockIdx.x) * n) : nullptr;  // null with xq
    const float4* rr = ADD ? reinterpret_cast<const float4*>(r + size_t(blockIdx.x) * n) : nullptr;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 v[kNormV], b[ADD ? kNormV : 1], wv[kNormV];
#pragma unroll
    for (int j = 0; j < kNormV; ++j) {
        const uint32_t i = threadIdx.x + j * kNormT;
        const bool live = i < n4;
        v[j] = live ? xr[i] : make_float4(0, 0, 0, 0);
        if constexpr (ADD) b[j] = live ? rr[i] : make_float4(0, 0, 0, 0);
        if constexpr (ADD)  // r's further planes, summed in split order (splitk_reduce_kernel's)
            for (uint32_t s = 1; s < rsplit; ++s) {
                const float4 t = live ? rr[size_t(s) * gridDim.x * n4 + i] : make_float4(0, 0, 0, 0);
                b[j] = make_float4(b[j].x + t.x, b[j].y + t.y, b[j].z + t.z, b[j].w + t.w);
            }
        wv[j] = live ? w4[i] : make_float4(0, 0, 0, 0);
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < kNormV; ++j) {
        const uint32_t i = threadIdx.x + j * kNormT;
        if constexpr (ADD) {
            v[j] = make_float4(v[j].x + b[j].x, v[j].y + b[j].y, v[j].z + b[j].z, v[j].w + b[j].w);
            if (i < n4) xr[i] = v[j];
        }
        ss += double(v[j].x) * double(v[j].x);
        ss += double(v[j].y) * double(v[j].y);
        ss += double(v[j].z) * double(v[j].z);
        ss += double(v[j].w) * double(v[j].w);
    }
    ss = block_sum_d(ss, red);
    const float inv = 1.0f / sqrtf(float(ss / double(n)) + eps);
    int8_t* qr = xq ? xq + size_t(blockIdx.x) * n : nullptr;
    float* sr = xq ? xs + size_t(blockIdx.x) * (n / 32) : nullptr;
#pragma unroll
    for (int j = 0; j < kNormV; ++j) {
        const uint32_t i = threadIdx.x + j * kNormT;
        if (j * kNormT >= n4) break;  // uniform: no element of this round is live
        const float4 o = make_float4(v[j].x * inv * wv[j].x, v[j].y * inv * wv[j].y, v[j].z * inv * wv[j].z,
                                     v[j].w * inv * wv[j].w);
        if (yr && i < n4) yr[i] = o;
        // n % 32 == 0 with xq: a round's live lanes are whole 8-lane blocks
        if (qr && i < n4) quantize_lane4_block32(o, qr + 4 * i, sr + i / 8);
    }
}

// RoPE on q (in place) and k, then k and v appended to the caches at
// position pos0 + t.  One workgroup per token.  `pairs` rotated pairs per head:
// adjacent (x[2i], x[2i+1]) or half-split (x[i], x[i+pairs]); dimensions past
// 2*pairs are left as they are (rope(), :317-328 of the reference runtime).
__global__ __launch_bounds__(kT) void rope_kv_kernel(const float* q, float* q_out, const float* __restrict__ k,
                                                     const float* __restrict__ v, float* __restrict__ kc,
                                                     float* __restrict__ vc, const float* __restrict__ cos_tab,
                                                     const float* __restrict__ sin_tab, const uint32_t* __restrict__ pos0,
                                                     uint32_t H, uint32_t KH, uint32_t D, uint32_t pairs, int adjacent,
                                                     uint32_t ldq, uint32_t ldkv) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = *pos0 + t;
    const float* cs = cos_tab + size_t(pos) * pairs;
    const float* sn = sin_tab + size_t(pos) * pairs;
    const float* qt = q + size_t(t) * ldq;
    float* qo = q_out + size_t(t) * H * D;
    const float* kt = k + size_t(t) * ldkv;
    const float* vt = v + size_t(t) * ldkv;
    float* kd = kc + size_t(pos) * KH * D;
    float* vd = vc + size_t(pos) * KH * D;
    // q (in place, or into q_out): one thread per rotated pair; elements past
    // the rotated ones are copied when q_out is another buffer
    for (uint32_t j = threadIdx.x; j < H * pairs; j += kT) {
        const uint32_t h = j / pairs, i = j - h * pairs;
        const float* vh = qt + size_t(h) * D;
        float* oh = qo + size_t(h) * D;
        const uint32_t ia = adjacent ? 2 * i : i, ib = adjacent ? 2 * i + 1 : i + pairs;
        const float a = vh[ia], b = vh[ib], c = cs[i], s = sn[i];
        oh[ia] = a * c - b * s;
        oh[ib] = a * s + b * c;
    }
    if (q_out != q && 2 * pairs < D)
        for (uint32_t j = threadIdx.x; j < H * (D - 2 * pairs); j += kT) {
            const uint32_t h = j / (D - 2 * pairs), d = 2 * pairs + (j - h * (D - 2 * pairs));
            qo[size_t(h) * D + d] = qt[size_t(h) * D + d];
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


// Causal GQA prefill attention, tiled: workgroup (kh, i) takes a tile of 64
// rows = (query head g of kv head kh, token t) pairs, t in [i*TQ, i*TQ + TQ)
// with TQ = 64 / G, so the G heads that share a K/V row read it once.  Key
// tiles of 64 positions stream through LDS, with an online softmax (running
// max m, sum l, rescale of O by exp(m_old - m_new)).  The result equals the
// reference's softmax(q.k * scale) . v to fp32-level accuracy.
typedef float v16f_t __attribute__((ext_vector_type(16)));
constexpr int kFRows = 64, kFKeys = 64;

// The products run on the f16 MFMA
// (v_mfma_f32_32x32x16_f16, 16x the fp32 MFMA rate) at fp32-level accuracy,
// computed transposed so the softmax stays in registers:
//  * every operand x is scaled by a power of two 2^e (exact) so max |x| lies
//    in [2^14, 2^15) -- per query row, per K tile, per V tile, and P (in
//    [0, 1]) by 2^14 -- then split into h = f16(x) and l = f16(x - h) (x - h
//    is exact in fp32); a product is h_a h_b + h_a l_b + l_a h_b (the dropped
//    l_a l_b is below 2^-22 of the operands' maxima), accumulated in fp32, and
//    the scales come off exactly;
//  * S^T = K Q^T: a lane holds 16 scores of its query, so the row max and
//    sum need one cross-half exchange, and P^T is the B operand of
//    O^T = V^T P^T straight from the lane's registers (the MFMA's k slots
//    take the keys in the order the S^T accumulator holds them; V^T is read
//    in that order, two 4-key runs per operand);
//  * wave w takes query rows 32 (w & 1) .. + 31 of the tile and keys
//    32 (w >> 1) .. + 31 of every 64-key tile, with its own running max, sum
//    and O; the two waves of a row set merge at the end.
// K is staged row-major and V transposed ([column][key], 8 keys of one
// column per lane load group), both as f16 pairs; two barriers per key tile.
constexpr int kFHP(int D) { return D + 8; }  // halves per padded K (and Q staging) row
constexpr int kFKP = kFKeys + 8;             // halves per padded V^T row
constexpr size_t attention_prefill_t_lds(int D) {
    return size_t(2) * kFKeys * kFHP(D) * 2 + size_t(2) * D * kFKP * 2;
}

template <int D>
__global__ __launch_bounds__(kT) void attention_prefill_t_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                                 const float* __restrict__ vc, float* __restrict__ out,
                                                                 const uint32_t* __restrict__ pos0_ptr, uint32_t T,
                                                                 uint32_t H, uint32_t KH, float scale,
                                                                 int8_t* __restrict__ xq, float* __restrict__ xs) {
    constexpr int HP = kFHP(D), KP = kFKP;
    constexpr int NT = D / 32;  // 32-row O^T tiles (head-dim blocks)
    constexpr int KS = D / 16;  // k-steps of S^T
    constexpr int RL = D / 4;   // lanes per row in the float4 row layout (16 or 32)
    extern __shared__ __align__(16) uint8_t fsm_raw[];
    _Float16* khi = reinterpret_cast<_Float16*>(fsm_raw);  // [64][HP]
    _Float16* klo = khi + kFKeys * HP;
    _Float16* vth = klo + kFKeys * HP;                      // [D][KP]
    _Float16* vtl = vth + D * KP;
    float* mrg = reinterpret_cast<float*>(fsm_raw);         // end-of-kernel merge, over K and V
    static_assert(size_t(2) * 64 * (NT * 16 + 2) * 4 <= attention_prefill_t_lds(D), "merge area fits");
    __shared__ float inv_q[kFRows], kred[kT / 64], vred[kT / 64];
    const uint32_t G = H / KH, TQ = kFRows / G;
    const uint32_t kh = blockIdx.x, t0 = blockIdx.y * TQ;
    const uint32_t pos0 = *pos0_ptr;
    const uint32_t KW = KH * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, lh = lane >> 5;
    const int qh = wave & 1, kh2 = wave >> 1;
    const uint32_t qrow = 32 * qh + l32;  // this lane's query row of the tile
    const uint32_t qt = qrow % TQ;        // its token offset

    // ---- Q: per-row scale, split, staged over the K area, operands into registers ----
    {
        _Float16* qhi = khi;
        _Float16* qlo = klo;
        constexpr int QL = kFRows * D / 4 / kT;
        float4 qv[QL];
#pragma unroll
        for (int j = 0; j < QL; ++j) {
            const uint32_t i = tid + j * kT, r = (4 * i) / D, d = (4 * i) % D;
            const uint32_t g = r / TQ, t = r % TQ;
            qv[j] = t0 + t < T ? *reinterpret_cast<const float4*>(q + (size_t(t0 + t) * H + kh * G + g) * D + d)
                               : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < QL; ++j) {
            const uint32_t i = tid + j * kT, r = (4 * i) / D, d = (4 * i) % D;
            float m = fmaxf(fmaxf(fabsf(qv[j].x), fabsf(qv[j].y)), fmaxf(fabsf(qv[j].z), fabsf(qv[j].w)));
#pragma unroll
            for (int o = RL / 2; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
            const int e = split_exp(m);
            const float f = pow2f(e);
            if (d == 0) inv_q[r] = pow2f(-e);
            h4_t h, l;
            split_h(qv[j].x * f, h, l, 0);
            split_h(qv[j].y * f, h, l, 1);
            split_h(qv[j].z * f, h, l, 2);
            split_h(qv[j].w * f, h, l, 3);
            *reinterpret_cast<h4_t*>(qhi + r * HP + d) = h;
            *reinterpret_cast<h4_t*>(qlo + r * HP + d) = l;
        }
    }
    __syncthreads();
    h8_t bqh[KS], bql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        bqh[ks] = *reinterpret_cast<const h8_t*>(khi + qrow * HP + ks * 16 + 8 * lh);
        bql[ks] = *reinterpret_cast<const h8_t*>(klo + qrow * HP + ks * 16 + 8 * lh);
    }
    const float iq2 = inv_q[qrow];

    v16f_t o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[n][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f, fv_prev = 1.0f;

    const uint32_t nkeys = pos0 + min(t0 + TQ, T);  // keys any row of the tile sees
    constexpr int KVL = kFKeys * D / 4 / kT;
    constexpr int VG = kFKeys * D / kT / 8;  // 8-key groups per thread
    constexpr int VGS = kT / D;              // threads per column
    constexpr int KRJ = kT * 4 / D;          // K rows per float4 round
    const uint32_t vcol = tid % D, vgi = tid / D;
    const uint32_t koff = ((tid * 4 / D) * KW + (tid * 4) % D) * 4;  // byte offsets within a tile
    const uint32_t voff = (vgi * 8 * KW + vcol) * 4;
    float4 kr4[KVL];
    float vr[VG][8];
    // Buffer loads bounded to the tile's live rows: rows past the last key
    // read 0 (no request), so no address clamps and no zeroing.
    auto load_tile = [&](uint32_t k0) {
        const uint32_t rows = min(nkeys - k0, uint32_t(kFKeys));
        const int bytes = int(((rows - 1) * KW + D) * 4);
        const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(kc + size_t(k0) * KW + size_t(kh) * D), 0, bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vc + size_t(k0) * KW + size_t(kh) * D), 0, bytes, 0x00020000);
#pragma unroll
        for (int j = 0; j < KVL; ++j) {
            const u32x4_attn_t t = __builtin_amdgcn_raw_buffer_load_b128(krs, koff + uint32_t(j * KRJ) * KW * 4, 0, 0);
            kr4[j] = make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w));
        }
#pragma unroll
        for (int g = 0; g < VG; ++g)
#pragma unroll
            for (int c = 0; c < 8; ++c)
                vr[g][c] = __uint_as_float(
                    __builtin_amdgcn_raw_buffer_load_b32(vrs, voff + uint32_t(g * VGS * 8 + c) * KW * 4, 0, 0));
    };
    load_tile(0);
    for (uint32_t k0 = 0; k0 < nkeys; k0 += kFKeys) {
        // the K and V tiles' maxima, for their scales
        float vm = 0.0f, km = 0.0f;
#pragma unroll
        for (int g = 0; g < VG; ++g)
#pragma unroll
            for (int c = 0; c < 8; ++c) vm = fmaxf(vm, fabsf(vr[g][c]));
#pragma unroll
        for (int j = 0; j < KVL; ++j)
            km = fmaxf(km, fmaxf(fmaxf(fabsf(kr4[j].x), fabsf(kr4[j].y)), fmaxf(fabsf(kr4[j].z), fabsf(kr4[j].w))));
        vm = wave_max(vm);
        km = wave_max(km);
        if (lane == 0) {
            vred[wave] = vm;
            kred[wave] = km;
        }
        __syncthreads();  // the previous tile's readers are done (and the Q operands read); maxima complete
        float vmax = vred[0], kmax = kred[0];
#pragma unroll
        for (int w = 1; w < kT / 64; ++w) {
            vmax = fmaxf(vmax, vred[w]);
            kmax = fmaxf(kmax, kred[w]);
        }
        const int ev = split_exp(vmax), ek = split_exp(kmax);
        const float fv = pow2f(ev), f = pow2f(ek), ik = pow2f(-ek);
#pragma unroll
        for (int j = 0; j < KVL; ++j) {
            const uint32_t i = tid + j * kT, kr = (4 * i) / D, d = (4 * i) % D;
            const float4 kv = kr4[j];
            h4_t h, l;
            split_h(kv.x * f, h, l, 0);
            split_h(kv.y * f, h, l, 1);
            split_h(kv.z * f, h, l, 2);
            split_h(kv.w * f, h, l, 3);
            *reinterpret_cast<h4_t*>(khi + kr * HP + d) = h;
            *reinterpret_cast<h4_t*>(klo + kr * HP + d) = l;
        }
#pragma unroll
        for (int g = 0; g < VG; ++g) {
            h8_t h, l;
#pragma unroll
            for (int c = 0; c < 8; ++c) split_h(vr[g][c] * fv, h, l, c);
            const uint32_t kb = (g * VGS + vgi) * 8;
            *reinterpret_cast<h8_t*>(vth + vcol * KP + kb) = h;
            *reinterpret_cast<h8_t*>(vtl + vcol * KP + kb) = l;
        }
        if (k0 + kFKeys < nkeys) load_tile(k0 + kFKeys);
        __syncthreads();
        // ---- S^T for keys 32*kh2 .. + 31 and this wave's 32 queries ----
        v16f_t sacc;
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[v] = 0.0f;
        {
            const int krow = 32 * kh2 + l32;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const h8_t ah = *reinterpret_cast<const h8_t*>(khi + krow * HP + ks * 16 + 8 * lh);
                const h8_t al = *reinterpret_cast<const h8_t*>(klo + krow * HP + ks * 16 + 8 * lh);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bqh[ks], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bql[ks], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bqh[ks], sacc, 0, 0, 0);
            }
        }
        // ---- online softmax of this lane's query over the wave's 32 keys ----
        float sv[16];
        float mx = -INFINITY;
        const uint32_t lim = pos0 + t0 + qt;  // last key this query sees
        const bool qok = t0 + qt < T;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t kk = 32 * kh2 + 8 * (v >> 2) + 4 * lh + (v & 3);
            const bool ok = qok && k0 + kk <= lim;
            sv[v] = ok ? sacc[v] * (ik * iq2) * scale : -INFINITY;
            mx = fmaxf(mx, sv[v]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        float sum = 0.0f;
        h8_t ph[2], pl[2];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float pv = m_new == -INFINITY ? 0.0f : expf(sv[v] - m_new);
            sum += pv;
            split_h(pv * 16384.0f, ph[v >> 3], pl[v >> 3], v & 7);
        }
        sum += __shfl_xor(sum, 32);
        const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
        l_run = l_run * alpha + sum;
        m_run = m_new;
        // O^T is kept in units of this tile's V scale: rescale by alpha and the scale change
        const float ro = alpha * (fv / fv_prev);
        fv_prev = fv;
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[n][v] *= ro;
        // ---- O^T += V^T P^T: k slot j of step st is key 32*kh2 + kk(8 st + j) ----
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int kb = 32 * kh2 + 16 * st + 4 * lh;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const int vrow = 32 * n + l32;
                h8_t ah, al;
                const h4_t a0 = *reinterpret_cast<const h4_t*>(vth + vrow * KP + kb);
                const h4_t a1 = *reinterpret_cast<const h4_t*>(vth + vrow * KP + kb + 8);
                const h4_t b0 = *reinterpret_cast<const h4_t*>(vtl + vrow * KP + kb);
                const h4_t b1 = *reinterpret_cast<const h4_t*>(vtl + vrow * KP + kb + 8);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ah[j] = a0[j]; ah[j + 4] = a1[j];
                    al[j] = b0[j]; al[j + 4] = b1[j];
                }
                o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ph[st], o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, pl[st], o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, ph[st], o[n], 0, 0, 0);
            }
        }
    }
    // ---- merge the two key halves of each query row set; O / (2^14 fv) / l ----
    __syncthreads();  // every wave is done with K and V
    float* mp = mrg + size_t(qh) * 64 * (NT * 16 + 2);
    if (kh2 == 1) {
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int v = 0; v < 16; ++v) mp[(n * 16 + v) * 64 + lane] = o[n][v];
        mp[(NT * 16) * 64 + lane] = m_run;
        mp[(NT * 16 + 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (kh2 == 1 || t0 + qt >= T) return;
    {
        const float m1 = mp[(NT * 16) * 64 + lane], l1 = mp[(NT * 16 + 1) * 64 + lane];
        const float M = fmaxf(m_run, m1);
        const float a0 = m_run == -INFINITY ? 0.0f : expf(m_run - M);
        const float a1 = m1 == -INFINITY ? 0.0f : expf(m1 - M);
        const float L = l_run * a0 + l1 * a1;
        const float inv = pow2f(-14) / fv_prev / L;
        const uint32_t g = qrow / TQ;
        const size_t row_off = (size_t(t0 + qt) * H + kh * G + g) * D;
        float* orow = out + row_off;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            float4 r[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                r[j].x = (o[n][4 * j] * a0 + mp[(n * 16 + 4 * j) * 64 + lane] * a1) * inv;
                r[j].y = (o[n][4 * j + 1] * a0 + mp[(n * 16 + 4 * j + 1) * 64 + lane] * a1) * inv;
                r[j].z = (o[n][4 * j + 2] * a0 + mp[(n * 16 + 4 * j + 2) * 64 + lane] * a1) * inv;
                r[j].w = (o[n][4 * j + 3] * a0 + mp[(n * 16 + 4 * j + 3) * 64 + lane] * a1) * inv;
            }
            if (!xq) {
#pragma unroll
                for (int j = 0; j < 4; ++j) *reinterpret_cast<float4*>(orow + 32 * n + 8 * j + 4 * lh) = r[j];
                continue;
            }
            // only the int8 form for the o GEMM: the 32-element block 32n..32n+31
            // of this row is split over this lane (4 * lh + 8j + 0..3) and its
            // partner lane ^ 32; the quantiser's arithmetic (quantize_acts_kernel)
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(r[j].x), fabsf(r[j].y)), fmaxf(fabsf(r[j].z), fabsf(r[j].w))));
            amax = fmaxf(amax, __shfl_xor(amax, 32));
            const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            if (lh == 0) xs[(row_off >> 5) + n] = d;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float e[4] = {r[j].x, r[j].y, r[j].z, r[j].w};
                uint32_t w = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float qv = e[k] * id;
                    qv = qv > 127.0f ? 127.0f : (qv < -127.0f ? -127.0f : qv);
                    w |= (uint32_t(round_half_away(qv)) & 0xffu) << (8 * k);
                }
                *reinterpret_cast<uint32_t*>(xq + row_off + 32 * n + 8 * j + 4 * lh) = w;
            }
        }
    }
}

// Decode attention (one query token at position pos) with RoPE and the KV
// append fused in, split over positions: workgroup (kh, s) covers positions
// [s*C, s*C + C) of kv head kh for the G query heads that share it, reading
// each K and V row once.  Every workgroup rotates the G query rows in LDS;
// the workgroup whose chunk holds `pos` also rotates the new key, appends key
// and value to the caches and uses them from LDS.  All global loads of a
// workgroup are issued up front, so its cost is about one memory latency.
// Per query head it writes the chunk's max score m, l = sum exp(score - m)
// and acc[d] = sum exp(score - m) * v[d].  The last chunk workgroup of a kv
// head to finish (an agent-scope arrival counter per kv head) merges the
// chunks of its G heads, out = sum_s exp(m_s - M) acc_s / sum_s exp(m_s - M)
// l_s, equal to the single-pass softmax of the reference up to rounding.
// Partials are written with agent-scope stores and read back with
// agent-scope loads (coherent across XCDs without cache write-back or
// invalidation); a chunk workgroup waits for its own partial stores
// (s_waitcnt) before it arrives.  The merging workgroup resets the counter,
// so the kernel needs no clearing between steps (HIP-graph replays).
constexpr int kAttnChunk = 32;
constexpr int kAttnMaxG = 8;
constexpr int kAttnMaxSplits = 1024;  // positions <= 32768


// out[g][d] of the G query heads of one kv head from their ns chunk partials
// (part: [g][splits][D + 2]), by one workgroup, in batches of NB chunks.  All
// loads of a batch (every thread's acc values and the batch's (m, l) pairs)
// are issued together, so a batch costs one memory round trip.  Per head a
// group of NB lanes takes the batch's max, the weights w_s = exp(m_s - M)
// against the running max M and L = sum l_s w_s (in double); the running
// acc and L are rescaled by exp(M_old - M) when the max grows.  With ns <= NB
// (positions < 32 * NB) that is out = (sum_s acc_s[d] w_s, in chunk order) / L.
template <int D, int G>
__device__ void merge_chunks(const float* part, float* out, uint32_t ns, uint32_t splits) {
    constexpr int E = (G * D + kT - 1) / kT;     // output elements per thread
    constexpr int NB = E <= 2 ? 32 : (E <= 4 ? 16 : 8);  // chunks per batch: E * NB <= 64 loads per thread
    static_assert(G * NB <= kT && (64 % NB) == 0, "one lane per (head, chunk) of a batch, groups inside a wave");
    __shared__ float wgt[G][NB];
    __shared__ float rs[G];
    __shared__ float Ms[G];
    __shared__ double Ls[G];
    const uint32_t n = G * splits * (D + 2);
    const int tid = threadIdx.x;
    const bool wt = tid < G * NB;
    const uint32_t wg = tid / NB, wj = tid % NB;
    if (tid < G) {
        Ms[tid] = -INFINITY;
        Ls[tid] = 0.0;
    }
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.0f;
    for (uint32_t b0 = 0; b0 < ns; b0 += NB) {
        const uint32_t nb = min(ns - b0, uint32_t(NB));
        float a[E][NB];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t el = tid + e * kT, g = el / D, d = el % D;
#pragma unroll
            for (int j = 0; j < NB; ++j)
                a[e][j] = el < G * D && uint32_t(j) < nb ? coherent_load_f(part, n, (g * splits + b0 + j) * (D + 2) + d)
                                                         : 0.0f;
        }
        float mj = -INFINITY, lj = 0.0f;
        if (wt && wj < nb) {
            const uint32_t o = (wg * splits + b0 + wj) * (D + 2) + D;
            mj = coherent_load_f(part, n, o);
            lj = coherent_load_f(part, n, o + 1);
        }
        __syncthreads();  // Ms / Ls of the previous batch written; its wgt reads done
        if (wt) {
            float mb = mj;
#pragma unroll
            for (int o = NB / 2; o > 0; o >>= 1) mb = fmaxf(mb, __shfl_xor(mb, o));
            const float mo = Ms[wg], mn = fmaxf(mo, mb);
            const float w = wj < nb ? expf(mj - mn) : 0.0f;
            double ls = double(lj) * double(w);
#pragma unroll
            for (int o = NB / 2; o > 0; o >>= 1) ls += __shfl_xor(ls, o);
            wgt[wg][wj] = w;
            if (wj == 0) {  // the group's lanes have read Ms[wg] (one wave, in order)
                const float r = expf(mo - mn);  // 0 for the first batch (mo = -inf)
                rs[wg] = r;
                Ms[wg] = mn;
                Ls[wg] = Ls[wg] * double(r) + ls;
            }
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t el = tid + e * kT, g = min(el / D, uint32_t(G - 1));
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < NB; ++j) t = fmaf(a[e][j], wgt[g][j], t);
            acc[e] = acc[e] * rs[g] + t;
        }
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const uint32_t el = tid + e * kT;
        if (el < G * D) out[el] = acc[e] * (1.0f / float(Ls[el / D]));
    }
}

template <int D, int G>
__global__ __launch_bounds__(kT) void attention_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ knew, const float* __restrict__ vnew, float* __restrict__ kc,
    float* __restrict__ vc, const float* __restrict__ cos_tab, const float* __restrict__ sin_tab,
    float* __restrict__ part, float* __restrict__ out, const uint32_t* __restrict__ pos_ptr, uint32_t H, uint32_t KH,
    uint32_t pairs, float scale, uint32_t splits) {
    constexpr int C = kAttnChunk;
    constexpr int LPP = kT / C;       // lanes per position in the score phase (8)
    constexpr int DPL = D / LPP;      // key elements per lane (16 for D = 128)
    constexpr int HALVES = kT / D;    // position groups in the value phase
    constexpr int VPT = C / HALVES;   // value rows per thread
    constexpr int QPT = (G * D + kT - 1) / kT;
    __shared__ float qs[G][D];
    __shared__ float kn[D], vn[D];
    __shared__ __align__(16) float sc[C][G];  // position-major: the G weights of a position are adjacent
    __shared__ float red[G][kT];
    const uint32_t kh = blockIdx.x, s = blockIdx.y;
    const uint32_t pos = *pos_ptr;
    const uint32_t p0 = s * C;
    if (p0 > pos) return;  // chunk past the current position: nothing to contribute
    const uint32_t n = min(uint32_t(C), pos + 1 - p0);
    const bool owns_new = pos < p0 + C;
    const uint32_t KW = KH * D;
    const int tid = threadIdx.x;

    // ---- issue every global load ----
    const uint32_t sp = tid / LPP, sj = tid % LPP;  // score phase: position, slice
    float kv[DPL];
    {
        const uint32_t pp = sp < n ? p0 + sp : p0;
        const float4* kr = reinterpret_cast<const float4*>(kc + size_t(pp) * KW + size_t(kh) * D + sj * DPL);
#pragma unroll
        for (int i = 0; i < DPL / 4; ++i) {
            const float4 f = kr[i];
            kv[4 * i] = f.x; kv[4 * i + 1] = f.y; kv[4 * i + 2] = f.z; kv[4 * i + 3] = f.w;
        }
    }
    const uint32_t vd = tid % D, vh = tid / D;      // value phase: element, position group
    float vv[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t p = vh + i * HALVES;
        vv[i] = vc[size_t(p0 + (p < n ? p : 0)) * KW + size_t(kh) * D + vd];
    }
    float qr[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const uint32_t e = tid + i * kT;
        qr[i] = e < G * D ? q[size_t(kh * G) * D + e] : 0.0f;
    }
    float knr = 0.0f, vnr = 0.0f;
    if (owns_new && tid < D) {
        knr = knew[size_t(kh) * D + tid];
        vnr = vnew[size_t(kh) * D + tid];
    }
    const float* cs = cos_tab + size_t(pos) * pairs;
    const float* sn = sin_tab + size_t(pos) * pairs;
    // the rotation factors come in with the other loads, not after them
    constexpr int QP = (G * D / 2 + kT - 1) / kT;  // q pairs per thread
    float cq[QP], sq[QP];
#pragma unroll
    for (int k = 0; k < QP; ++k) {
        const uint32_t j = tid + k * kT, i = j % (pairs ? pairs : 1u);
        cq[k] = j < G * pairs ? cs[i] : 0.0f;
        sq[k] = j < G * pairs ? sn[i] : 0.0f;
    }
    const float ck = owns_new && uint32_t(tid) < pairs ? cs[tid] : 0.0f;
    const float sk = owns_new && uint32_t(tid) < pairs ? sn[tid] : 0.0f;

    // ---- RoPE (adjacent pairs) on q and the new key, in LDS ----
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
        const uint32_t e = tid + i * kT;
        if (e < G * D) qs[e / D][e % D] = qr[i];
    }
    if (owns_new && tid < D) { kn[tid] = knr; vn[tid] = vnr; }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < QP; ++k) {
        const uint32_t j = tid + k * kT;
        if (j < G * pairs) {
            const uint32_t g = j / pairs, i = j - g * pairs;
            const float a = qs[g][2 * i], b = qs[g][2 * i + 1], c = cq[k], sv = sq[k];
            qs[g][2 * i] = a * c - b * sv;
            qs[g][2 * i + 1] = a * sv + b * c;
        }
    }
    if (owns_new && uint32_t(tid) < pairs) {
        const float a = kn[2 * tid], b = kn[2 * tid + 1], c = ck, sv = sk;
        kn[2 * tid] = a * c - b * sv;
        kn[2 * tid + 1] = a * sv + b * c;
    }
    __syncthreads();
    if (owns_new && tid < D) {  // append to the caches for later steps
        kc[size_t(pos) * KW + size_t(kh) * D + tid] = kn[tid];
        vc[size_t(pos) * KW + size_t(kh) * D + tid] = vn[tid];
    }
    // ---- scores ----
    if (sp < n && p0 + sp == pos) {
#pragma unroll
        for (int i = 0; i < DPL; ++i) kv[i] = kn[sj * DPL + i];
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) d = fmaf(qs[g][sj * DPL + i], kv[i], d);
        d = group_sum<LPP>(d);
        if (sj == 0 && sp < n) sc[sp][g] = d * scale;
    }
    __syncthreads();
    // ---- chunk softmax: one wave per head, one lane per position ----
    float* outp = part + size_t(kh * G) * splits * (D + 2);
    {
        const int wv = tid >> 6, ln = tid & 63;
        for (int g = wv; g < G; g += kT / 64) {
            const float sv = uint32_t(ln) < n ? sc[ln][g] : -INFINITY;
            const float m = wave_max(sv);
            const float e = uint32_t(ln) < n ? expf(sv - m) : 0.0f;
            if (ln < C) sc[ln][g] = e;  // zero past the chunk's last position
            const float l = wave_sum(e);
            if (ln == 0) {
                float* o = outp + (size_t(g) * splits + s) * (D + 2);
                coherent_store_f(o + D, m);
                coherent_store_f(o + D + 1, l);
            }
        }
    }
    __syncthreads();
    // ---- acc[g][d] = sum_p e[g][p] * v[p][d]; past the last position e = 0
    // and v is selected to 0 (the row read there may be an unwritten one) ----
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t p = vh + i * HALVES;
        const float v = p0 + p == pos ? vn[vd] : (p < n ? vv[i] : 0.0f);
        float e[G];
        if constexpr (G % 4 == 0) {
#pragma unroll
            for (int g4 = 0; g4 < G; g4 += 4) {
                const float4 w = *reinterpret_cast<const float4*>(&sc[p][g4]);
                e[g4] = w.x; e[g4 + 1] = w.y; e[g4 + 2] = w.z; e[g4 + 3] = w.w;
            }
        } else {
#pragma unroll
            for (int g = 0; g < G; ++g) e[g] = sc[p][g];
        }
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g] = fmaf(e[g], v, acc[g]);
    }
    if (HALVES > 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) red[g][tid] = acc[g];
        __syncthreads();
        if (vh == 0)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float t = 0.0f;
                for (int k = 0; k < HALVES; ++k) t += red[g][vd + k * D];
                coherent_store_f(outp + (size_t(g) * splits + s) * (D + 2) + vd, t);
            }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) coherent_store_f(outp + (size_t(g) * splits + s) * (D + 2) + vd, acc[g]);
    }
    // ---- arrival; the last chunk of this kv head merges ----
    __shared__ uint32_t last;
    // Every wave waits for its own agent-scope partial stores to be
    // acknowledged (written through to the device-coherent level) before the
    // barrier, so the arrival below follows all of them.  A workgroup-scope
    // release fence would not do: it emits no wait for global stores.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const uint32_t ns = pos / C + 1;
    uint32_t* cnt = reinterpret_cast<uint32_t*>(part + size_t(H) * splits * (D + 2)) + kh;
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old + 1 == ns ? 1u : 0u;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // all ns have arrived
    }
    __syncthreads();
    if (!last) return;
    merge_chunks<D, G>(outp, out + size_t(kh * G) * D, ns, splits);
}

// out = x + y (out may be x)
__global__ __launch_bounds__(kT) void add_kernel(const float* x, const float* __restrict__ y, float* out, size_t n) {
    const size_t i = size_t(blockIdx.x) * kT + threadIdx.x;
    if (i < n) out[i] = x[i] + y[i];
}

// Greedy id: the lowest index among the finite maxima.  Stage 1: kArgBlocks
// workgroups each reduce a strided share into (value, index); stage 2 reduces
// the partials.  "Better" = larger value, or equal value and lower index.
constexpr int kArgBlocks = 128;
__device__ __forceinline__ void better(float& bv, uint32_t& bi, float ov, uint32_t oi) {
    if (oi != 0xffffffffu && (bi == 0xffffffffu || ov > bv || (ov == bv && oi < bi))) {
        bv = ov;
        bi = oi;
    }
}
__device__ __forceinline__ void block_best(float& best, uint32_t& idx, float* sv, uint32_t* si) {
    for (int o = 32; o > 0; o >>= 1) better(best, idx, __shfl_xor(best, o), __shfl_xor(idx, o));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = best; si[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int i = 1; i < kT / 64; ++i) better(best, idx, sv[i], si[i]);
}
__global__ __launch_bounds__(kT) void argmax_partial_kernel(const float* __restrict__ x, uint32_t n,
                                                            float* __restrict__ pv, uint32_t* __restrict__ pi) {
    __shared__ float sv[kT / 64];
    __shared__ uint32_t si[kT / 64];
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    for (uint32_t i = blockIdx.x * kT + threadIdx.x; i < n; i += kArgBlocks * kT) {
        const float v = x[i];
        if (isfinite(v)) better(best, idx, v, i);
    }
    block_best(best, idx, sv, si);
    if (threadIdx.x == 0) { pv[blockIdx.x] = best; pi[blockIdx.x] = idx; }
}
__global__ __launch_bounds__(kT) void argmax_final_kernel(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                          uint32_t* __restrict__ out) {
    __shared__ float sv[kT / 64];
    __shared__ uint32_t si[kT / 64];
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    if (threadIdx.x < kArgBlocks) better(best, idx, pv[threadIdx.x], pi[threadIdx.x]);
    block_best(best, idx, sv, si);
    if (threadIdx.x == 0) *out = idx == 0xffffffffu ? 0u : idx;
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

static bool norm4_ok(const void* x, const void* r, const void* w, const void* y, const void* xq, uint32_t n) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return n % 4 == 0 && n <= uint32_t(4 * kNormV * kNormT) && a16(x) && a16(r) && a16(w) && a16(y) &&
           (reinterpret_cast<uintptr_t>(xq) & 3u) == 0;
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, uint32_t rows, uint32_t n, float eps,
                          hipStream_t stream, int8_t* xq, float* xs) {
    if (!x || !w || (!y && !xq) || !rows || !n || (xq && (!xs || n % 32))) return hipErrorInvalidValue;
    if (norm4_ok(x, nullptr, w, y, xq, n))
        hipLaunchKernelGGL(rmsnorm4_kernel<false>, dim3(rows), dim3(kNormT), 0, stream, const_cast<float*>(x), nullptr, w,
                           y, n, eps, xq, xs, 1u);
    else
        hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(rows), dim3(kNormT), 0, stream, const_cast<float*>(x), nullptr, w,
                           y, n, eps, xq, xs, 1u);
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm(float* x, const float* r, const float* w, float* y, uint32_t rows, uint32_t n, float eps,
                              hipStream_t stream, int8_t* xq, float* xs, uint32_t rsplit) {
    if (rsplit < 1) return hipErrorInvalidValue;
    if (!x || !r || !w || (!y && !xq) || !rows || !n || (xq && (!xs || n % 32))) return hipErrorInvalidValue;
    if (norm4_ok(x, r, w, y, xq, n))
        hipLaunchKernelGGL(rmsnorm4_kernel<true>, dim3(rows), dim3(kNormT), 0, stream, x, r, w, y, n, eps, xq, xs, rsplit);
    else
        hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(rows), dim3(kNormT), 0, stream, x, r, w, y, n, eps, xq, xs, rsplit);
    return hipGetLastError();
}

// rope_kv_kernel with adjacent pairs, float4 accesses (a float4 is two whole
// pairs: 2 * pairs % 4 == 0) and every load of a token issued up front: q
// (H * D <= 4 * kRopeQV * kT) and k, v (KH * D <= 4 * kRopeKV * kT).  The
// same expressions per element.
constexpr int kRopeQV = 8, kRopeKV = 2;
__global__ __launch_bounds__(kT) void rope_kv4_kernel(const float* q, float* q_out, const float* __restrict__ k,
                                                      const float* __restrict__ v, float* __restrict__ kc,
                                                      float* __restrict__ vc, const float* __restrict__ cos_tab,
                                                      const float* __restrict__ sin_tab,
                                                      const uint32_t* __restrict__ pos0, uint32_t H, uint32_t KH,
                                                      uint32_t D, uint32_t pairs, uint32_t ldq, uint32_t ldkv,
                                                      uint32_t splits, size_t plane4) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = *pos0 + t;
    const float* cs = cos_tab + size_t(pos) * pairs;
    const float* sn = sin_tab + size_t(pos) * pairs;
    const float4* qt = reinterpret_cast<const float4*>(q + size_t(t) * ldq);
    float4* qo = reinterpret_cast<float4*>(q_out + size_t(t) * H * D);
    const float4* kt = reinterpret_cast<const float4*>(k + size_t(t) * ldkv);
    const float4* vt = reinterpret_cast<const float4*>(v + size_t(t) * ldkv);
    float4* kd = reinterpret_cast<float4*>(kc + size_t(pos) * KH * D);
    float4* vd = reinterpret_cast<float4*>(vc + size_t(pos) * KH * D);
    const uint32_t nq = H * D / 4, nk = KH * D / 4, D4 = D / 4, rot4 = pairs / 2;  // float4s rotated per head
    float4 qv[kRopeQV], kv[kRopeKV], vv[kRopeKV];
    float4 qc[kRopeQV], kcs[kRopeKV];  // (cos i, cos i+1, sin i, sin i+1)
    auto factors = [&](uint32_t d4) {
        const float2 c = *reinterpret_cast<const float2*>(cs + 2 * d4);
        const float2 s = *reinterpret_cast<const float2*>(sn + 2 * d4);
        return make_float4(c.x, c.y, s.x, s.y);
    };
    auto add4 = [](float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); };
#pragma unroll
    for (int j = 0; j < kRopeQV; ++j) {
        const uint32_t i = threadIdx.x + j * kT, d4 = i % D4;
        qv[j] = i < nq ? qt[i] : make_float4(0, 0, 0, 0);
        qc[j] = i < nq && d4 < rot4 ? factors(d4) : make_float4(1, 1, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kRopeKV; ++j) {
        const uint32_t i = threadIdx.x + j * kT, d4 = i % D4;
        kv[j] = i < nk ? kt[i] : make_float4(0, 0, 0, 0);
        vv[j] = i < nk ? vt[i] : make_float4(0, 0, 0, 0);
        kcs[j] = i < nk && d4 < rot4 ? factors(d4) : make_float4(1, 1, 0, 0);
    }
    // splits > 1: q, k, v are a GEMM's split-K partial planes (plane4 float4s
    // apart), summed here in split order (splitk_reduce_kernel's)
    for (uint32_t s = 1; s < splits; ++s) {
#pragma unroll
        for (int j = 0; j < kRopeQV; ++j) {
            const uint32_t i = threadIdx.x + j * kT;
            if (i < nq) qv[j] = add4(qv[j], qt[s * plane4 + i]);
        }
#pragma unroll
        for (int j = 0; j < kRopeKV; ++j) {
            const uint32_t i = threadIdx.x + j * kT;
            if (i < nk) {
                kv[j] = add4(kv[j], kt[s * plane4 + i]);
                vv[j] = add4(vv[j], vt[s * plane4 + i]);
            }
        }
    }
    auto rot = [](float4 x, float4 f) {  // pairs (x, y) and (z, w)
        return make_float4(x.x * f.x - x.y * f.z, x.x * f.z + x.y * f.x, x.z * f.y - x.w * f.w, x.z * f.w + x.w * f.y);
    };
#pragma unroll
    for (int j = 0; j < kRopeQV; ++j) {
        const uint32_t i = threadIdx.x + j * kT;
        if (i < nq) qo[i] = i % D4 < rot4 ? rot(qv[j], qc[j]) : qv[j];
    }
#pragma unroll
    for (int j = 0; j < kRopeKV; ++j) {
        const uint32_t i = threadIdx.x + j * kT;
        if (i < nk) {
            kd[i] = i % D4 < rot4 ? rot(kv[j], kcs[j]) : kv[j];
            vd[i] = vv[j];
        }
    }
}

hipError_t launch_rope_kv(float* q, const float* k, const float* v, float* kc, float* vc, const float* cos_tab,
                          const float* sin_tab, const uint32_t* pos0, uint32_t T, uint32_t H, uint32_t KH, uint32_t D,
                          uint32_t pairs, bool adjacent, hipStream_t stream, uint32_t ld, const float* q_in,
                          uint32_t splits, float* reduce_to) {
    if (!q || !k || !v || !kc || !vc || !cos_tab || !sin_tab || !pos0 || !T || !H || !KH || !D || !pairs ||
        pairs > D / 2 || H % KH || (ld && ld < (H + 2 * KH) * D) || (q_in && !ld) || !splits ||
        (splits > 1 && (!q_in || !reduce_to)))
        return hipErrorInvalidValue;
    const float* qi = q_in ? q_in : q;
    const uint32_t ldq = ld ? ld : H * D, ldkv = ld ? ld : KH * D;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (adjacent && pairs % 2 == 0 && D % 4 == 0 && ldq % 4 == 0 && ldkv % 4 == 0 && H * D <= 4u * kRopeQV * kT &&
        KH * D <= 4u * kRopeKV * kT && a16(qi) && a16(q) && a16(k) && a16(v) && a16(kc) && a16(vc) && a16(cos_tab) &&
        a16(sin_tab)) {
        hipLaunchKernelGGL(rope_kv4_kernel, dim3(T), dim3(kT), 0, stream, qi, q, k, v, kc, vc, cos_tab, sin_tab, pos0, H,
                           KH, D, pairs, ldq, ldkv, splits, size_t(T) * ld / 4);
        return hipGetLastError();
    }
    if (splits > 1) {  // the partial planes reduced into reduce_to first (q_in's layout), then as one plane
        const hipError_t e = launch_splitk_reduce(q_in, reduce_to, T, ld, splits, stream);
        if (e != hipSuccess) return e;
        k = reduce_to + (k - q_in);
        v = reduce_to + (v - q_in);
        qi = reduce_to;
    }
    hipLaunchKernelGGL(rope_kv_kernel, dim3(T), dim3(kT), 0, stream, qi, q, k, v, kc, vc, cos_tab, sin_tab, pos0, H, KH,
                       D, pairs, adjacent ? 1 : 0, ld ? ld : H * D, ld ? ld : KH * D);
    return hipGetLastError();
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, const uint32_t* pos0,
                            uint32_t T, uint32_t H, uint32_t KH, uint32_t D, uint32_t max_pos, float scale,
                            hipStream_t stream, int8_t* xq, float* xs, bool* quantized) {
    if (quantized) *quantized = false;
    if (!q || !kc || !vc || !out || !pos0 || !T || !H || !KH || H % KH || D % 64 || D > 256 || !max_pos ||
        (xq && (!xs || !quantized)))
        return hipErrorInvalidValue;
    const uint32_t G = H / KH;
    if (kFRows % G == 0 && (D == 64 || D == 128)) {
        const uint32_t TQ = kFRows / G;
        const dim3 grid(KH, (T + TQ - 1) / TQ);
        if (D == 64)
            hipLaunchKernelGGL(attention_prefill_t_kernel<64>, grid, dim3(kT), attention_prefill_t_lds(64), stream, q, kc,
                               vc, out, pos0, T, H, KH, scale, xq, xs);
        else
            hipLaunchKernelGGL(attention_prefill_t_kernel<128>, grid, dim3(kT), attention_prefill_t_lds(128), stream, q,
                               kc, vc, out, pos0, T, H, KH, scale, xq, xs);
        if (quantized) *quantized = xq != nullptr;
        return hipGetLastError();
    }
    const size_t lds = size_t(max_pos) * sizeof(float);
    if (lds > 96 * 1024) return hipErrorInvalidValue;  // positions are bounded by the cache capacity
    hipLaunchKernelGGL(attention_kernel, dim3(H, T), dim3(kT), lds, stream, q, kc, vc, out, pos0, H, KH, D, scale);
    return hipGetLastError();
}

size_t attention_decode_partial_floats(uint32_t H, uint32_t D, uint32_t max_pos) {
    const uint32_t splits = (max_pos + kAttnChunk - 1) / kAttnChunk;
    return size_t(H) * splits * (D + 2) + H;  // + one arrival counter per kv head (<= H), zero at rest
}

hipError_t launch_attention_decode(const float* q, const float* knew, const float* vnew, float* kc, float* vc,
                                   const float* cos_tab, const float* sin_tab, float* part, float* out,
                                   const uint32_t* pos, uint32_t H, uint32_t KH, uint32_t D, uint32_t pairs,
                                   uint32_t max_pos, float scale, hipStream_t stream) {
    if (!q || !knew || !vnew || !kc || !vc || !cos_tab || !sin_tab || !part || !out || !pos || !H || !KH || H % KH ||
        H / KH > uint32_t(kAttnMaxG) || !max_pos || !pairs || pairs > D / 2)
        return hipErrorInvalidValue;
    const uint32_t splits = (max_pos + kAttnChunk - 1) / kAttnChunk;
    if (splits > uint32_t(kAttnMaxSplits)) return hipErrorInvalidValue;
    const dim3 grid(KH, splits);
    const uint32_t G = H / KH;
#define ZQ_ATTN(DD, GG)                                                                                                \
    hipLaunchKernelGGL((attention_decode_kernel<DD, GG>), grid, dim3(kT), 0, stream, q, knew, vnew, kc, vc, cos_tab,  \
                       sin_tab, part, out, pos, H, KH, pairs, scale, splits)
#define ZQ_ATTN_G(DD)                      \
    switch (G) {                           \
    case 1: ZQ_ATTN(DD, 1); break;         \
    case 2: ZQ_ATTN(DD, 2); break;         \
    case 3: ZQ_ATTN(DD, 3); break;         \
    case 4: ZQ_ATTN(DD, 4); break;         \
    case 5: ZQ_ATTN(DD, 5); break;         \
    case 6: ZQ_ATTN(DD, 6); break;         \
    case 7: ZQ_ATTN(DD, 7); break;         \
    case 8: ZQ_ATTN(DD, 8); break;         \
    default: return hipErrorInvalidValue;  \
    }
    switch (D) {
    case 64: ZQ_ATTN_G(64); break;
    case 128: ZQ_ATTN_G(128); break;
    case 256: ZQ_ATTN_G(256); break;
    default: return hipErrorInvalidValue;
    }
#undef ZQ_ATTN_G
#undef ZQ_ATTN
    return hipGetLastError();
}

hipError_t launch_add_to(const float* x, const float* y, float* out, size_t n, hipStream_t stream) {
    if (!x || !y || !out || !n) return hipErrorInvalidValue;
    hipLaunchKernelGGL(add_kernel, dim3(uint32_t((n + kT - 1) / kT)), dim3(kT), 0, stream, x, y, out, n);
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t stream) { return launch_add_to(x, y, x, n, stream); }

size_t argmax_partial_bytes() { return size_t(kArgBlocks) * 8; }

hipError_t launch_argmax(const float* x, uint32_t n, uint32_t* out, void* partial, hipStream_t stream) {
    if (!x || !n || !out || !partial) return hipErrorInvalidValue;
    float* pv = static_cast<float*>(partial);
    uint32_t* pi = reinterpret_cast<uint32_t*>(pv + kArgBlocks);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks), dim3(kT), 0, stream, x, n, pv, pi);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kT), 0, stream, pv, pi, out);
    return hipGetLastError();
}

}  // namespace zq
