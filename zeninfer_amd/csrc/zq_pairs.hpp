// zq_pairs.hpp -- device helpers of the Q8_0 / Q4_0 block-pair GEMV kernels
// (zq_gemv.hip): range-limited 16-byte buffer loads and the per-lane dot of one block pair with 64
// activation values.
#pragma once
#include "zq_device.hpp"

namespace zq {
namespace {

constexpr int kPadStride = 68;  // floats per 64-float x chunk in LDS

#ifndef ZQ_GEMV_NT
#define ZQ_GEMV_NT 0
#endif
__device__ __forceinline__ constexpr bool use_nt() { return ZQ_GEMV_NT != 0; }
// The streaming kernels load every 16 B unit exactly once with lane-contiguous
// dwordx4 loads, whole cache lines per instruction: there the non-temporal
// hint pays (measured: a plain float4 read stream reaches ~5.4 TB/s on MI355X,
// the same stream with the hint ~7 TB/s).
#ifndef ZQ_GEMV_STREAM_NT
#define ZQ_GEMV_STREAM_NT 1
#endif
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));


// 16 B load through a raw buffer resource covering `bytes` from a
// wave-uniform base: lanes past the end read 0 and generate no memory
// request (the non-temporal bit is aux bit 1 on gfx950).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const uint8_t* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 span_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, ZQ_GEMV_STREAM_NT != 0 ? 2 : 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------- Q8_0 ---
// Dot of one 68-byte Q8_0 block pair with 64 x values.
//   dword 0      : d0 (bytes 0-1) | q0 q1
//   dwords 1..7  : q2 .. q29
//   dword 8      : q30 q31 | d1 (bytes 2-3)
//   dwords 9..16 : second block's 32 quants
__device__ __forceinline__ float q8_pair_dot(const uint32_t (&q)[17], const float (&xv)[64]) {
    float s0 = 0.0f, s1 = 0.0f;
    s0 = fmaf(sbyte(q[0], 2), xv[0], s0);
    s0 = fmaf(sbyte(q[0], 3), xv[1], s0);
#pragma unroll
    for (int i = 1; i < 8; ++i) {
#pragma unroll
        for (int k = 0; k < 4; ++k) s0 = fmaf(sbyte(q[i], k), xv[4 * i - 2 + k], s0);
    }
    s0 = fmaf(sbyte(q[8], 0), xv[30], s0);
    s0 = fmaf(sbyte(q[8], 1), xv[31], s0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int k = 0; k < 4; ++k) s1 = fmaf(sbyte(q[9 + i], k), xv[32 + 4 * i + k], s1);
    }
    const float d0 = half_bits_to_float(q[0]);
    const float d1 = half_bits_to_float(q[8] >> 16);
    return fmaf(d1, s1, d0 * s0);
}

// Dot of one 36-byte Q4_0 block pair with 64 x values.
//   dword 0     : d0 | n0 n1      dwords 1..3 : n2 .. n13
//   dword 4     : n14 n15 | d1    dwords 5..8 : second block's 16 bytes
// Byte j holds element j (low nibble) and j+16 (high nibble); value (n-8)*d.
// ((n ^ 8) << 4) read as a signed byte is 16*(n-8): exact, scaled out by d/16.
__device__ __forceinline__ float q4_block_dot(const uint32_t (&u)[4], const float* xv) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = ((u[i] << 4) & 0xF0F0F0F0u) ^ 0x80808080u;
        const uint32_t hi = (u[i] & 0xF0F0F0F0u) ^ 0x80808080u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            s = fmaf(sbyte(lo, k), xv[4 * i + k], s);
            s = fmaf(sbyte(hi, k), xv[16 + 4 * i + k], s);
        }
    }
    return s;
}
__device__ __forceinline__ float q4_pair_dot(const uint32_t (&q)[9], const float (&xv)[64]) {
    uint32_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], 2);
        b[i] = q[5 + i];
    }
    const float s0 = q4_block_dot(a, xv);
    const float s1 = q4_block_dot(b, xv + 32);
    const float d0 = half_bits_to_float(q[0]) * 0.0625f;
    const float d1 = half_bits_to_float(q[4] >> 16) * 0.0625f;
    return fmaf(d1, s1, d0 * s0);
}

// Q4_0 pair dot on the mixed-precision FMA.  A nibble n (0..15) placed in a
// 16-bit half is the binary16 denormal n * 2^-24, exactly; v_fma_mix_f32 takes
// it straight from either half of a register, so two elements cost one mask
// (0x000F000F over a shifted word) and two FMAs, and the products n*2^-24*x
// and their sums are the cvt+fma ones scaled by 2^-24, exactly.  The offset
// is applied once per block: sum (n-8)*x = 2^24 * sum n*x*2^-24 - 8 * sum x,
// with sum x of the lane's two blocks precomputed (x is fixed per lane).
__device__ __forceinline__ float mix_lo(uint32_t pair, float x, float acc) {
    return fmaf(float(__builtin_bit_cast(_Float16, uint16_t(pair))), x, acc);
}
__device__ __forceinline__ float mix_hi(uint32_t pair, float x, float acc) {
    return fmaf(float(__builtin_bit_cast(_Float16, uint16_t(pair >> 16))), x, acc);
}
__device__ __forceinline__ float q4_block_nx(const uint32_t (&u)[4], const float* xv) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a02 = u[i] & 0x000F000Fu, a13 = (u[i] >> 8) & 0x000F000Fu;
        const uint32_t b02 = (u[i] >> 4) & 0x000F000Fu, b13 = (u[i] >> 12) & 0x000F000Fu;
        s = mix_lo(a02, xv[4 * i], s);
        s = mix_lo(a13, xv[4 * i + 1], s);
        s = mix_hi(a02, xv[4 * i + 2], s);
        s = mix_hi(a13, xv[4 * i + 3], s);
        s = mix_lo(b02, xv[16 + 4 * i], s);
        s = mix_lo(b13, xv[16 + 4 * i + 1], s);
        s = mix_hi(b02, xv[16 + 4 * i + 2], s);
        s = mix_hi(b13, xv[16 + 4 * i + 3], s);
    }
    return s;
}
__device__ __forceinline__ float q4_pair_dot_mix(const uint32_t (&q)[9], const float (&xv)[64], float sx0, float sx1) {
    uint32_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], 2);
        b[i] = q[5 + i];
    }
    const float s0 = fmaf(q4_block_nx(a, xv), 16777216.0f, -8.0f * sx0);
    const float s1 = fmaf(q4_block_nx(b, xv + 32), 16777216.0f, -8.0f * sx1);
    const float d0 = half_bits_to_float(q[0]);
    const float d1 = half_bits_to_float(q[4] >> 16);
    return fmaf(d1, s1, d0 * s0);
}


// The same two pair dots with the 64 x values read from LDS (xp: the pair's
// 64 floats, 16-byte aligned) a block at a time, so at most 32 x values are
// live in VGPRs; the FMA order is that of q8_pair_dot / q4_pair_dot_mix.
__device__ __forceinline__ float q8_pair_dot_lds(const uint32_t (&q)[17], const float* xp) {
    float s[2] = {0.0f, 0.0f};
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        float x[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = reinterpret_cast<const float4*>(xp + 32 * blk)[i];
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            // element e = 32*blk + j: block 0 starts at byte 2 of dword 0, block 1 at dword 9
            const int word = blk == 0 ? (j + 2) / 4 : 9 + j / 4;
            const int byte = blk == 0 ? (j + 2) % 4 : j % 4;
            s[blk] = fmaf(sbyte(q[word], byte), x[j], s[blk]);
        }
    }
    const float d0 = half_bits_to_float(q[0]);
    const float d1 = half_bits_to_float(q[8] >> 16);
    return fmaf(d1, s[1], d0 * s[0]);
}
__device__ __forceinline__ float q4_pair_dot_mix_lds(const uint32_t (&q)[9], const float* xp, float sx0, float sx1) {
    uint32_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], 2);
        b[i] = q[5 + i];
    }
    float s[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        float x[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = reinterpret_cast<const float4*>(xp + 32 * blk)[i];
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
        s[blk] = fmaf(q4_block_nx(blk == 0 ? a : b, x), 16777216.0f, -8.0f * (blk == 0 ? sx0 : sx1));
    }
    const float d0 = half_bits_to_float(q[0]);
    const float d1 = half_bits_to_float(q[4] >> 16);
    return fmaf(d1, s[1], d0 * s[0]);
}

}  // namespace
}  // namespace zq
