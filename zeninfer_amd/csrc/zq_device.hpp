// zq_device.hpp -- device-side helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

namespace zq {

// GGML type ids (src/gguf.cpp:370-393 of the reference: 2=Q4_0, 8=Q8_0,
// 12=Q4_K, 13=Q5_K, 14=Q6_K).
constexpr int kQ4_0 = 2;
constexpr int kQ8_0 = 8;
constexpr int kQ4_K = 12;
constexpr int kQ5_K = 13;
constexpr int kQ6_K = 14;

constexpr int kWave = 64;

// binary16 -> binary32.  v_cvt_f32_f16 is exact for every binary16 input,
// subnormals included (fp16 denormals are enabled in the HIP default mode).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits16 & 0xffffu)));
}

// Sign-extended byte k of a dword as float (one v_cvt_f32_i32 with SDWA sext).
__device__ __forceinline__ float sbyte(uint32_t v, int k) {
    return static_cast<float>(static_cast<int8_t>(v >> (8 * k)));
}

// 32 bits starting at an arbitrary byte address, from two naturally aligned
// dword loads and one v_alignbyte.  Used where GGML block boundaries put
// fields at addresses that are 2 mod 4.
__device__ __forceinline__ uint32_t load_u32_any(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
    const uint32_t lo = base[0];
    const uint32_t sh = static_cast<uint32_t>(a & 3u);
    if (sh == 0) return lo;
    const uint32_t hi = base[1];
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}

// 32 bits from a 2-byte-aligned address as two 16-bit loads; never reads
// past p+3, so it is safe on the last bytes of a buffer.
__device__ __forceinline__ uint32_t load_u32_a2(const uint8_t* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return uint32_t(h[0]) | (uint32_t(h[1]) << 16);
}

__host__ __device__ inline size_t row_bytes_dev(int fmt, size_t cols) {
    return fmt == kQ8_0   ? cols / 32 * 34
           : fmt == kQ4_0 ? cols / 32 * 18
           : fmt == kQ4_K ? cols / 256 * 144
           : fmt == kQ5_K ? cols / 256 * 176
                          : cols / 256 * 210;
}

// Q4_K / Q5_K packed 6-bit scale and min of group j (0..7) from the 12 bytes
// at s (src/quant.cpp:133-141 of the reference).
__device__ __forceinline__ void kquant_scale_min(const uint8_t* s, uint32_t j, uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = s[j] & 63u;
        mn = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 15u) | (uint32_t(s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | (uint32_t(s[j] >> 6) << 4);
    }
}

// Exact dequantisation of the 32 consecutive elements [k0, k0+32) of one
// weight row (k0 % 32 == 0), to the values of the reference's dequantize:
// Q8_0 int8(q)*d (src/quant.cpp:410-416), Q4_0 (n-8)*d (:391-397), Q6_K
// (d*sc)*(q-32) (:500-517), Q4_K / Q5_K (d*sc)*q - dmin*m (:439-476; d*sc,
// dmin*m and (d*sc)*q are exact, the subtraction is the one rounding).
// Reads stay inside the blocks they decode.
template <int FMT>
__device__ __forceinline__ void dequant32(const uint8_t* row, uint32_t k0, float (&o)[32]) {
    if constexpr (FMT == kQ8_0) {
        const uint8_t* p = row + size_t(k0 >> 5) * 34;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(p));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = load_u32_a2(p + 2 + 4 * i);
#pragma unroll
            for (int k = 0; k < 4; ++k) o[4 * i + k] = sbyte(u, k) * d;
        }
    } else if constexpr (FMT == kQ4_0) {
        const uint8_t* p = row + size_t(k0 >> 5) * 18;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(p));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = load_u32_a2(p + 2 + 4 * i);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t byte = (u >> (8 * k)) & 0xffu;
                o[4 * i + k] = float(int(byte & 15u) - 8) * d;
                o[16 + 4 * i + k] = float(int(byte >> 4) - 8) * d;
            }
        }
    } else if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
        constexpr uint32_t BB = FMT == kQ5_K ? 176 : 144;
        const uint8_t* p = row + size_t(k0 >> 8) * BB;
        const uint32_t j = (k0 & 255u) >> 5;  // group
        uint32_t sc, mn;
        kquant_scale_min(p + 4, j, sc, mn);
        const float ds = half_bits_to_float(*reinterpret_cast<const uint16_t*>(p)) * float(sc);
        const float ms = half_bits_to_float(*reinterpret_cast<const uint16_t*>(p + 2)) * float(mn);
        const uint8_t* qs = p + (FMT == kQ5_K ? 48 : 16) + (j >> 1) * 32;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = *reinterpret_cast<const uint32_t*>(qs + 4 * i);
            uint32_t hb = 0;
            if constexpr (FMT == kQ5_K) hb = *reinterpret_cast<const uint32_t*>(p + 16 + 4 * i);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t q = (u >> (8 * k + 4 * (j & 1u))) & 15u;
                if constexpr (FMT == kQ5_K) q |= ((hb >> (8 * k + j)) & 1u) << 4;
                o[4 * i + k] = __fsub_rn(__fmul_rn(ds, float(q)), ms);
            }
        }
    } else {
        const uint8_t* p = row + size_t(k0 >> 8) * 210;
        const uint32_t in_sb = k0 & 255u;
        const uint32_t h = in_sb >> 7, grp = (in_sb >> 5) & 3u;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(p + 208));
        const int8_t* sc = reinterpret_cast<const int8_t*>(p + 192);
        const float ds0 = d * float(sc[h * 8 + grp * 2]);
        const float ds1 = d * float(sc[h * 8 + grp * 2 + 1]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = load_u32_a2(p + h * 64 + (grp & 1u) * 32 + 4 * i);
            const uint32_t hi = load_u32_a2(p + 128 + h * 32 + 4 * i);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t l = (lo >> (8 * k)) & 0xffu;
                if (grp >= 2) l >>= 4;
                const uint32_t hb = ((hi >> (8 * k)) >> (2 * grp)) & 3u;
                const int q = int((l & 15u) | (hb << 4)) - 32;
                o[4 * i + k] = (i < 4 ? ds0 : ds1) * float(q);
            }
        }
    }
}

// Split-f16 operands for the f16 MFMA at fp32-level accuracy (prefill
// attention, the Q6_K fp32-activation GEMM): a value x, scaled by a power of
// two so its block's maximum lies in [2^14, 2^15), is carried as
// h = f16(x) and l = f16(x - h) (x - h is exact in fp32).
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_attn_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float pow2f(int e) { return __int_as_float((e + 127) << 23); }
// exponent e with max |x| * 2^e in [2^14, 2^15); 0 for max 0.  Clamped to
// [-40, 40]: a change of scale between tiles multiplies a running accumulator
// by at most 2^80, which stays finite.  Operands whose maximum lies below 2^-26
// lose precision (f16 subnormals); above 2^56 they would overflow f16.
__device__ __forceinline__ int split_exp(float amax) {
    if (!(amax > 0.0f)) return 0;
    return min(max(15 - __builtin_amdgcn_frexp_expf(amax), -40), 40);
}
// element i of h and l: h = f16(x), l = f16(x - h)
template <class V>
__device__ __forceinline__ void split_h(float x, V& h, V& l, int i) {
    const _Float16 a = _Float16(x);
    h[i] = a;
    l[i] = _Float16(x - float(a));
}
// Cross-lane reductions on DPP (quad_perm, row_half_mirror, row_mirror move
// data between lanes of a 16-lane row inside the VALU, a few cycles each)
// plus v_readlane for the four rows; ds_bpermute (what __shfl_xor lowers
// to) costs an LDS round trip per step.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(b)), CTRL, 0xF, 0xF, false));
    const uint32_t hi = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(b >> 32)), CTRL, 0xF, 0xF, false));
    return __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i in each 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i in each 16

// Sum over aligned groups of G lanes (G = 2, 4, 8, 16): every lane of a
// group ends with the group's sum.  After the two quad steps every lane holds
// its quad's sum, and the mirrors pair each lane with one of the other quad
// (half-row) of its group.
template <int G, typename T>
__device__ __forceinline__ T group_sum(T v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group of 1..16 lanes");
    auto step = [](T a, auto ctrl) {
        if constexpr (sizeof(T) == 8) return a + dpp_d<decltype(ctrl)::value>(a);
        else return a + dpp_f<decltype(ctrl)::value>(a);
    };
    if constexpr (G >= 2) v = step(v, std::integral_constant<int, kDppXor1>{});
    if constexpr (G >= 4) v = step(v, std::integral_constant<int, kDppXor2>{});
    if constexpr (G >= 8) v = step(v, std::integral_constant<int, kDppHalfMirror>{});
    if constexpr (G >= 16) v = step(v, std::integral_constant<int, kDppMirror>{});
    return v;
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), l));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), l));
    return __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
}
// Wave64 sum: every lane ends with the total (rows summed in lane order).
__device__ __forceinline__ float wave_sum(float v) {
    v = group_sum<16>(v);
    return ((readlane_f(v, 0) + readlane_f(v, 16)) + readlane_f(v, 32)) + readlane_f(v, 48);
}
__device__ __forceinline__ double wave_sum(double v) {
    v = group_sum<16>(v);
    return ((readlane_d(v, 0) + readlane_d(v, 16)) + readlane_d(v, 32)) + readlane_d(v, 48);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Round half away from zero (the reference quantiser's lround), exact for
// |v| < 2^23.
__device__ __forceinline__ int round_half_away(float v) {
    const float t = truncf(v);
    const float f = v - t;  // exact for |v| < 2^23
    return static_cast<int>(t) + (f >= 0.5f ? 1 : (f <= -0.5f ? -1 : 0));
}
// The per-32 activation quantiser (kernels/avx2.cpp:502-524) with one element
// per lane: the 32 consecutive lanes of a half-wave hold one block.  The
// block's amax is the max over its lanes (exact in any order), then d =
// amax/127, inv = 1/d, q = round_half_away(clamp(v * inv, +-127)) -- the
// arithmetic of quantize_acts_kernel, so the bytes and scales are equal.
// Every lane of the wave must call it (the max crosses lanes).
__device__ __forceinline__ void quantize_lane_block32(float v, int8_t* q_out, float* d_out) {
    float amax = fabsf(v);
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    if ((threadIdx.x & 31u) == 0) *d_out = d;
    float q = v * inv;
    q = q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q);
    *q_out = int8_t(round_half_away(q));
}

// The same quantiser with four consecutive elements per lane: the 8
// consecutive lanes of an aligned group hold one block, q_out receives the
// lane's 4 bytes (4-byte aligned).  Every lane of the wave must call it.
__device__ __forceinline__ void quantize_lane4_block32(float4 v, int8_t* q_out, float* d_out) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    if ((threadIdx.x & 7u) == 0) *d_out = d;
    const float e[4] = {v.x, v.y, v.z, v.w};
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float q = e[k] * inv;
        q = q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q);
        w |= (uint32_t(round_half_away(q)) & 0xffu) << (8 * k);
    }
    *reinterpret_cast<uint32_t*>(q_out) = w;
}

// Cross-workgroup hand-off inside one launch (workgroups run on 8 XCDs with
// private L2s): the producer writes with agent-scope stores (through to the
// device-coherent level) and waits for them (s_waitcnt) before it signals;
// the consumer reads with the device-scope cache policy (SC1), from the
// device-coherent level and not from a stale line of its own L2.  No L2
// write-back or invalidate is needed.
__device__ __forceinline__ void coherent_store_f(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Element i of the n floats at `base`, written by another workgroup of this
// launch.  Not an atomic, so the compiler may issue many before waiting.
__device__ __forceinline__ float coherent_load_f(const float* base, uint32_t n, uint32_t i) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, int(n * 4), 0x00020000);
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, i * 4, 0, 0x10));
}

}  // namespace zq
