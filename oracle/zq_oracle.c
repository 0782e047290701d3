/*
 * zq_oracle.c -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * A plain-C restatement of ZenInfer's CPU algorithms for the block-quantised
 * projection path (Q8_0 / Q4_0 / Q6_K / Q4_K / Q5_K GEMV and GEMM).  Only tests/, the
 * smoke check in __graft_entry__.py and the cpu_baseline leg of bench.py may
 * load this library.  The HIP product path never links or calls it.
 *
 * Each function cites the reference file:line it follows (paths relative to
 * the ZenInfer source tree).  Floating-point operations are written out one
 * by one, in the reference's order, with fmaf() exactly where the reference
 * uses an FMA instruction; the file is compiled with -ffp-contract=off so the
 * compiler adds no contractions of its own.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   fp16 codec            exhaustive 65536 round trip, the reference's KATs
 *                         (tests/core_tests.cpp:248-270) and its independent
 *                         corpus (tests/data/fp16_reference_corpus.h, copied
 *                         as data into tests/golden/fp16_corpus.json), and
 *                         bit equality with the compiled reference.
 *   dequantize            closed form + KATs (core_tests.cpp:272-310), the
 *                         constructive Q6_K builder (q6k_gemm_tests.cpp:17-45)
 *                         and bit equality with the compiled reference.
 *   quantize_acts         brute force over ties / amax==0 / clamp cases and
 *                         bit equality with the reference's int8 GEMV route.
 *   block_dots            int64 brute force.
 *   gemv_f32 / gemm_f32   bit equality with the compiled reference's AVX2
 *                         kernels where the reference order is fixed, plus a
 *                         double-precision reference within tolerance.
 *   gemm_i8 (Q8_0)        bit equality with the reference's int8 route
 *                         (ZEN_CPU_Q8_ACT=1) token by token.
 *   gemm_i8 (Q4_0, Q6_K)  the reference has no int8-activation route for
 *                         these formats; the integer part is pinned by
 *                         block_dots brute force and the float combination by
 *                         a double reference (tolerance only).
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <stdlib.h>

#define ZQO_Q4_0 2
#define ZQO_Q8_0 8
#define ZQO_Q4_K 12
#define ZQO_Q5_K 13
#define ZQO_Q6_K 14

/* ---------------------------------------------------------------- fp16 --- */
/* half_to_float: src/quant.cpp:80-89 (same algorithm as kernels/avx2.cpp:86-95). */
float zqo_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 31u, mant = h & 1023u, out;
    if (exp == 0) {
        if (mant == 0) out = sign;
        else {
            int e = -14;
            while ((mant & 1024u) == 0) { mant <<= 1; --e; }
            mant &= 1023u;
            out = sign | ((uint32_t)(e + 127) << 23) | (mant << 13);
        }
    } else if (exp == 31) out = sign | 0x7f800000u | (mant << 13);
    else out = sign | ((exp + 112u) << 23) | (mant << 13);
    float f; memcpy(&f, &out, 4); return f;
}

static uint32_t rounded_shift(uint32_t x, unsigned shift) {
    if (shift == 0) return x;
    if (shift >= 32) return 0;
    uint32_t q = x >> shift, mask = (1u << shift) - 1u;
    uint32_t rem = x & mask, halfway = 1u << (shift - 1);
    return q + ((rem > halfway || (rem == halfway && (q & 1u))) ? 1u : 0u);
}

/* float_to_half (round to nearest even, binary32 subnormals flush to signed
 * zero, NaN payload kept non-zero): src/quant.cpp:90-122. */
uint16_t zqo_float_to_half(float value) {
    uint32_t bits; memcpy(&bits, &value, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    uint32_t exp = (bits >> 23) & 0xffu, mant = bits & 0x7fffffu;
    if (exp == 0xffu) {
        if (mant == 0) return (uint16_t)(sign | 0x7c00u);
        uint16_t payload = (uint16_t)(mant >> 13);
        if (payload == 0) payload = 1;
        return (uint16_t)(sign | 0x7c00u | payload);
    }
    if (exp == 0) return sign;
    int e = (int)exp - 127;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    uint32_t significand = 0x800000u | mant;
    if (e >= -14) {
        uint32_t hm = rounded_shift(mant, 13);
        int he = e + 15;
        if (hm == 0x400u) { hm = 0; ++he; }
        if (he >= 31) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | ((uint16_t)he << 10) | (uint16_t)hm);
    }
    unsigned shift = (unsigned)(-e - 1);
    uint32_t sub = rounded_shift(significand, shift);
    return (uint16_t)(sign | (uint16_t)sub);
}

void zqo_decode_fp16(const uint16_t* src, float* dst, size_t n) { for (size_t i = 0; i < n; ++i) dst[i] = zqo_half_to_float(src[i]); }
void zqo_encode_fp16(const float* src, uint16_t* dst, size_t n) { for (size_t i = 0; i < n; ++i) dst[i] = zqo_float_to_half(src[i]); }

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* -------------------------------------------------------------- layout --- */
/* row_bytes: src/quant.cpp:894-943 (Q4_0 :917, Q8_0 :921, Q4_K :919,
 * Q5_K :920, Q6_K :940). */
size_t zqo_row_bytes(int fmt, size_t cols) {
    size_t blk, bytes;
    switch (fmt) {
    case ZQO_Q4_0: blk = 32; bytes = 18; break;
    case ZQO_Q8_0: blk = 32; bytes = 34; break;
    case ZQO_Q4_K: blk = 256; bytes = 144; break;
    case ZQO_Q5_K: blk = 256; bytes = 176; break;
    case ZQO_Q6_K: blk = 256; bytes = 210; break;
    default: return 0;
    }
    if (cols == 0 || cols % blk) return 0;
    return cols / blk * bytes;
}

/* ---------------------------------------------------- synthetic inputs --- */
/* SplitMix64, counter form: draw i of stream `seed` is the (i+1)-th output of
 * the sequential generator started at state `seed`. */
uint64_t zqo_splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
/* Box-Muller in double: uses draws 2i and 2i+1 of the stream. */
double zqo_normal_at(uint64_t seed, uint64_t i) {
    uint64_t a = zqo_splitmix64_at(seed, 2 * i), b = zqo_splitmix64_at(seed, 2 * i + 1);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);          /* [0,1) */
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}
/* Sub-stream seeds, so quants, scales and sub-scales never share draws. */
#define SEED_QUANT(s) ((s) ^ 0x51ull)
#define SEED_SCALE(s) ((s) ^ 0x5CA1Eull)
#define SEED_SUB(s)   ((s) ^ 0x5B5Cull)

void zqo_gen_normal_f32(uint64_t seed, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)zqo_normal_at(seed, i);
}
/* Config 0/1/2 weights: int8 quants U{-127..127}, fp16 scale |N(0,1)|*0.002. */
void zqo_gen_q8_0(uint64_t seed, size_t rows, size_t cols, uint8_t* out) {
    size_t nb = cols / 32;
    for (size_t g = 0; g < rows * nb; ++g) {
        uint8_t* p = out + g * 34;
        uint16_t h = zqo_float_to_half((float)(fabs(zqo_normal_at(SEED_SCALE(seed), g)) * 0.002));
        p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; ++j) {
            uint64_t u = zqo_splitmix64_at(SEED_QUANT(seed), g * 32 + j);
            p[2 + j] = (uint8_t)(int8_t)((int)((u >> 32) % 255u) - 127);
        }
    }
}
/* Config 3 Q4_0: nibbles U{0..15}, fp16 scale |N(0,1)|*0.02. */
void zqo_gen_q4_0(uint64_t seed, size_t rows, size_t cols, uint8_t* out) {
    size_t nb = cols / 32;
    for (size_t g = 0; g < rows * nb; ++g) {
        uint8_t* p = out + g * 18;
        uint16_t h = zqo_float_to_half((float)(fabs(zqo_normal_at(SEED_SCALE(seed), g)) * 0.02));
        p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 16; ++j) {
            uint64_t u = zqo_splitmix64_at(SEED_QUANT(seed), g * 16 + j);
            p[2 + j] = (uint8_t)(u >> 56);
        }
    }
}
/* Config 3 Q6_K: 6-bit q U{0..63} (element order of the decoder,
 * src/quant.cpp:500-517), 16 int8 sub-scales U{-32..31}, fp16 d = |N|*0.001.
 * Packing follows the constructive builder of tests/q6k_gemm_tests.cpp:36-42. */
void zqo_gen_q6_k(uint64_t seed, size_t rows, size_t cols, uint8_t* out) {
    size_t nb = cols / 256;
    for (size_t g = 0; g < rows * nb; ++g) {
        uint8_t* p = out + g * 210;
        memset(p, 0, 210);
        for (int i = 0; i < 16; ++i) {
            uint64_t u = zqo_splitmix64_at(SEED_SUB(seed), g * 16 + i);
            p[192 + i] = (uint8_t)(int8_t)((int)((u >> 32) % 64u) - 32);
        }
        uint16_t h = zqo_float_to_half((float)(fabs(zqo_normal_at(SEED_SCALE(seed), g)) * 0.001));
        p[208] = (uint8_t)h; p[209] = (uint8_t)(h >> 8);
        for (int half = 0; half < 2; ++half)
            for (int l = 0; l < 32; ++l) {
                unsigned q[4];
                for (int grp = 0; grp < 4; ++grp) {
                    size_t e = (size_t)half * 128 + (size_t)grp * 32 + (size_t)l;
                    q[grp] = (unsigned)(zqo_splitmix64_at(SEED_QUANT(seed), g * 256 + e) >> 58);
                }
                p[half * 64 + l] = (uint8_t)((q[0] & 15u) | ((q[2] & 15u) << 4));
                p[half * 64 + 32 + l] = (uint8_t)((q[1] & 15u) | ((q[3] & 15u) << 4));
                p[128 + half * 32 + l] = (uint8_t)((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6));
            }
    }
}

/* Q4_K / Q5_K (config-3 style; the reference names no generator for them):
 * fp16 d = |N|*0.001 and dmin = |N|*0.001, twelve bytes of uniformly random
 * packed 6-bit scales/mins, quants U{0..15} (Q4_K) or U{0..31} (Q5_K, the
 * fifth bit in the qh plane).  Every byte of the packed fields is a uniform
 * draw, so all scale/min bit positions are exercised. */
static void gen_kquant(uint64_t seed, size_t rows, size_t cols, uint8_t* out, int q5) {
    size_t nb = cols / 256, bb = q5 ? 176 : 144, qs = q5 ? 48 : 16;
    for (size_t g = 0; g < rows * nb; ++g) {
        uint8_t* p = out + g * bb;
        uint16_t d = zqo_float_to_half((float)(fabs(zqo_normal_at(SEED_SCALE(seed), 2 * g)) * 0.001));
        uint16_t m = zqo_float_to_half((float)(fabs(zqo_normal_at(SEED_SCALE(seed), 2 * g + 1)) * 0.001));
        p[0] = (uint8_t)d; p[1] = (uint8_t)(d >> 8); p[2] = (uint8_t)m; p[3] = (uint8_t)(m >> 8);
        for (int i = 0; i < 12; ++i) p[4 + i] = (uint8_t)(zqo_splitmix64_at(SEED_SUB(seed), g * 12 + i) >> 56);
        for (size_t i = 16; i < qs; ++i) p[i] = (uint8_t)(zqo_splitmix64_at(SEED_QUANT(seed) ^ 0xB17ull, g * 32 + (i - 16)) >> 56);
        for (int i = 0; i < 128; ++i) p[qs + i] = (uint8_t)(zqo_splitmix64_at(SEED_QUANT(seed), g * 128 + i) >> 56);
    }
}
void zqo_gen_q4_k(uint64_t seed, size_t rows, size_t cols, uint8_t* out) { gen_kquant(seed, rows, cols, out, 0); }
void zqo_gen_q5_k(uint64_t seed, size_t rows, size_t cols, uint8_t* out) { gen_kquant(seed, rows, cols, out, 1); }

/* k_scale_min: src/quant.cpp:133-141 (the 12-byte packed 6-bit scale/min
 * pairs of Q4_K / Q5_K). */
static void k_scale_min(unsigned j, const uint8_t* q, unsigned* sc, unsigned* mn) {
    if (j < 4) { *sc = q[j] & 63u; *mn = q[j + 4] & 63u; }
    else {
        *sc = (q[j + 4] & 15u) | ((unsigned)(q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((unsigned)(q[j] >> 6) << 4);
    }
}
/* Element e (0..255) of a Q4_K / Q5_K super-block as its integer quant and
 * group index: group j = e/32 reads the low (j even) or high (j odd) nibble
 * of qs[(j/2)*32 + e%32]; Q5_K adds bit j of qh[e%32] as bit 4
 * (src/quant.cpp:439-476). */
static unsigned kquant_q(const uint8_t* p, unsigned e, int q5) {
    unsigned j = e / 32, l = e % 32;
    const uint8_t* qs = p + (q5 ? 48 : 16);
    unsigned q = (qs[(j / 2) * 32 + l] >> ((j & 1u) * 4)) & 15u;
    if (q5) q |= ((p[16 + l] >> j) & 1u) << 4;
    return q;
}

/* ----------------------------------------------------------- dequantize -- */
/* Q4_0: src/quant.cpp:391-397.  Q8_0: :410-416.  Q6_K: :500-517.
 * Q4_K: :439-457, Q5_K: :458-476: value = (d*sc)*q - dmin*m.  d*sc and
 * dmin*m are exact (11-bit by 6-bit significands) and so is (d*sc)*q (a
 * further 5 bits), so the one rounding is the subtraction, whether or not a
 * compiler fuses the multiply into it. */
int zqo_dequantize(int fmt, const uint8_t* src, size_t n, float* dst) {
    switch (fmt) {
    case ZQO_Q4_0:
        if (n % 32) return 0;
        for (size_t b = 0; b < n / 32; ++b) {
            const uint8_t* p = src + b * 18; float d = zqo_half_to_float(rd16(p));
            for (int j = 0; j < 16; ++j) {
                uint8_t q = p[2 + j];
                dst[b * 32 + j] = (float)((int)(q & 15) - 8) * d;
                dst[b * 32 + j + 16] = (float)((int)(q >> 4) - 8) * d;
            }
        }
        return 1;
    case ZQO_Q8_0:
        if (n % 32) return 0;
        for (size_t b = 0; b < n / 32; ++b) {
            const uint8_t* p = src + b * 34; float d = zqo_half_to_float(rd16(p));
            for (int j = 0; j < 32; ++j) dst[b * 32 + j] = (float)(int8_t)p[2 + j] * d;
        }
        return 1;
    case ZQO_Q4_K:
    case ZQO_Q5_K: {
        int q5 = fmt == ZQO_Q5_K;
        size_t bb = q5 ? 176 : 144;
        if (n % 256) return 0;
        for (size_t b = 0; b < n / 256; ++b) {
            const uint8_t* p = src + b * bb;
            float d = zqo_half_to_float(rd16(p)), dmin = zqo_half_to_float(rd16(p + 2));
            for (unsigned e = 0; e < 256; ++e) {
                unsigned sc, mn;
                k_scale_min(e / 32, p + 4, &sc, &mn);
                float ds = d * (float)sc, ms = dmin * (float)mn;
                float t = ds * (float)kquant_q(p, e, q5);
                dst[b * 256 + e] = t - ms;
            }
        }
        return 1;
    }
    case ZQO_Q6_K:
        if (n % 256) return 0;
        for (size_t b = 0; b < n / 256; ++b) {
            const uint8_t* p = src + b * 210;
            const uint8_t* ql = p; const uint8_t* qh = p + 128;
            const int8_t* sc = (const int8_t*)(p + 192);
            float d = zqo_half_to_float(rd16(p + 208));
            for (unsigned n128 = 0; n128 < 256; n128 += 128) {
                for (unsigned l = 0; l < 32; ++l) {
                    unsigned is = l / 16;
                    int q1 = (int)((ql[l] & 15u) | (((qh[l] >> 0) & 3u) << 4)) - 32;
                    int q2 = (int)((ql[l + 32] & 15u) | (((qh[l] >> 2) & 3u) << 4)) - 32;
                    int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3u) << 4)) - 32;
                    int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3u) << 4)) - 32;
                    size_t base = b * 256 + n128 + l;
                    /* d*sc[is]*q evaluates left to right: (d*sc)*q. */
                    dst[base + 0] = d * (float)sc[is + 0] * (float)q1;
                    dst[base + 32] = d * (float)sc[is + 2] * (float)q2;
                    dst[base + 64] = d * (float)sc[is + 4] * (float)q3;
                    dst[base + 96] = d * (float)sc[is + 6] * (float)q4;
                }
                ql += 64; qh += 32; sc += 8;
            }
        }
        return 1;
    }
    return 0;
}

/* ------------------------------------------------ activation quantiser --- */
/* quantise_acts_q8_0: kernels/avx2.cpp:502-524 (identical copy inside the
 * quant::gemv int8 route, src/quant.cpp:1093-1113).  d = amax/127 (binary32
 * divide), inv = 1/d, v = x*inv clamped to +-127, lround (half away from 0). */
void zqo_quantize_acts(const float* x, size_t m, size_t k, int8_t* xq, float* xs) {
    size_t nb = k / 32;
    for (size_t t = 0; t < m; ++t)
        for (size_t b = 0; b < nb; ++b) {
            const float* xb = x + t * k + b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) { float a = fabsf(xb[i]); amax = a > amax ? a : amax; }
            float d = amax > 0.0f ? amax / 127.0f : 0.0f;
            float inv = d > 0.0f ? 1.0f / d : 0.0f;
            xs[t * nb + b] = d;
            for (int i = 0; i < 32; ++i) {
                float v = xb[i] * inv;
                v = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v);
                xq[t * k + b * 32 + i] = (int8_t)lroundf(v);
            }
        }
}

/* ---------------------------------------------------- integer block dots --- */
/* Per 32-element activation block b, the exact integer dot of one weight row
 * with the int8 activations:
 *   Q8_0: sum q*xq                         (avx2.cpp:574-581 maddubs/madd)
 *   Q4_0: sum (nib-8)*xq                   (build-defined; quant.cpp:391-397 values)
 *   Q6_K: sum over the two 16-element sub-blocks of sc*sum (q-32)*xq
 *         (build-defined; quant.cpp:500-517 values, d applied outside).
 * out is [m][n][k/32] int32, computed in int64 and checked to fit. */
int zqo_block_dots(int fmt, const uint8_t* w, const int8_t* xq, size_t m, size_t n, size_t k, int32_t* out) {
    size_t rb = zqo_row_bytes(fmt, k); if (!rb || k % 32 || fmt == ZQO_Q4_K || fmt == ZQO_Q5_K) return 0;
    size_t nb = k / 32;
    float* row = NULL; (void)row;
    int* qi = (int*)malloc(sizeof(int) * k);
    int* si = (int*)malloc(sizeof(int) * (k / 16));
    if (!qi || !si) { free(qi); free(si); return 0; }
    for (size_t r = 0; r < n; ++r) {
        const uint8_t* wr = w + r * rb;
        /* integer weight values and the per-16 integer multiplier */
        for (size_t i = 0; i < k / 16; ++i) si[i] = 1;
        if (fmt == ZQO_Q8_0) {
            for (size_t b = 0; b < nb; ++b) for (int j = 0; j < 32; ++j) qi[b * 32 + j] = (int8_t)wr[b * 34 + 2 + j];
        } else if (fmt == ZQO_Q4_0) {
            for (size_t b = 0; b < nb; ++b) for (int j = 0; j < 16; ++j) {
                uint8_t q = wr[b * 18 + 2 + j];
                qi[b * 32 + j] = (int)(q & 15) - 8; qi[b * 32 + j + 16] = (int)(q >> 4) - 8;
            }
        } else {
            for (size_t sb = 0; sb < k / 256; ++sb) {
                const uint8_t* p = wr + sb * 210;
                for (int half = 0; half < 2; ++half) for (int l = 0; l < 32; ++l) {
                    const uint8_t* ql = p + half * 64; const uint8_t* qh = p + 128 + half * 32;
                    size_t base = sb * 256 + (size_t)half * 128 + (size_t)l;
                    qi[base + 0] = (int)((ql[l] & 15u) | (((qh[l] >> 0) & 3u) << 4)) - 32;
                    qi[base + 32] = (int)((ql[l + 32] & 15u) | (((qh[l] >> 2) & 3u) << 4)) - 32;
                    qi[base + 64] = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3u) << 4)) - 32;
                    qi[base + 96] = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3u) << 4)) - 32;
                }
                for (int i = 0; i < 16; ++i) si[sb * 16 + i] = (int8_t)p[192 + i];
            }
        }
        for (size_t t = 0; t < m; ++t)
            for (size_t b = 0; b < nb; ++b) {
                int64_t acc = 0;
                for (int h = 0; h < 2; ++h) {
                    int64_t part = 0;
                    for (int j = 0; j < 16; ++j) {
                        size_t c = b * 32 + (size_t)h * 16 + (size_t)j;
                        part += (int64_t)qi[c] * (int64_t)xq[t * k + c];
                    }
                    acc += part * si[b * 2 + h];
                }
                if (acc > INT32_MAX || acc < INT32_MIN) { free(qi); free(si); return 0; }
                out[(t * n + r) * nb + b] = (int32_t)acc;
            }
    }
    free(qi); free(si);
    return 1;
}

/* ------------------------------------------------ 8-lane helpers (AVX2) --- */
/* hsum_ps256: kernels/avx2.cpp:97-104: lo+hi, then two horizontal adds. */
static float hsum8(const float v[8]) {
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s1) + (s2 + s3);
}

/* ------------------------------------------------------ fp32 GEMV rows --- */
/* Q8_0: gemv_q8_0_avx2, kernels/avx2.cpp:587-641 (default fp32 path). */
static float gemv_row_q8_0(const uint8_t* row, const float* x, size_t cols) {
    float acc[8] = {0};
    for (size_t b = 0; b < cols / 32; ++b) {
        const uint8_t* p = row + b * 34;
        float d = zqo_half_to_float(rd16(p));
        float a[4][8];
        for (int c = 0; c < 4; ++c)
            for (int i = 0; i < 8; ++i)
                a[c][i] = fmaf((float)(int8_t)p[2 + c * 8 + i], x[b * 32 + c * 8 + i], 0.0f);
        for (int i = 0; i < 8; ++i) {
            float s = (a[0][i] + a[1][i]) + (a[2][i] + a[3][i]);
            acc[i] = fmaf(d, s, acc[i]);
        }
    }
    return hsum8(acc);
}
/* Q6_K: gemv_q6k_avx2 + q6k_decode8, kernels/avx2.cpp:383-422. */
static float gemv_row_q6_k(const uint8_t* row, const float* x, size_t cols) {
    float sums[4][8] = {{0}};
    for (size_t b = 0; b < cols / 256; ++b) {
        const uint8_t* p = row + b * 210;
        float d = zqo_half_to_float(rd16(p + 208));
        const int8_t* scales = (const int8_t*)(p + 192);
        for (unsigned half = 0; half < 2; ++half)
            for (unsigned group = 0; group < 4; ++group)
                for (unsigned lane = 0; lane < 32; lane += 8) {
                    float ds = d * (float)scales[half * 8 + group * 2 + lane / 16];
                    for (unsigned i = 0; i < 8; ++i) {
                        unsigned lo = p[half * 64 + (group % 2) * 32 + lane + i];
                        unsigned hi = p[128 + half * 32 + lane + i];
                        if (group >= 2) lo >>= 4;
                        hi >>= group * 2;
                        int q = (int)((lo & 15u) | ((hi & 3u) << 4)) - 32;
                        float wv = ds * (float)q;
                        sums[lane / 8][i] = fmaf(wv, x[b * 256 + half * 128 + group * 32 + lane + i], sums[lane / 8][i]);
                    }
                }
    }
    float v[8];
    for (int i = 0; i < 8; ++i) v[i] = (sums[0][i] + sums[1][i]) + (sums[2][i] + sums[3][i]);
    return hsum8(v);
}
/* Q4_K / Q5_K: gemv_q4k_q5k_avx2, kernels/avx2.cpp:329-378.  Four 8-lane
 * accumulators: element group*32 + chunk*8 + i of every super-block goes to
 * acc[chunk][i] as fma(w, x, acc) with w = (d*sc)*q - dmin*m (exact product,
 * one rounding); the end is hsum_ps256((acc0 + acc1) + (acc2 + acc3)). */
static float gemv_row_kquant(const uint8_t* row, const float* x, size_t cols, int q5) {
    float acc[4][8] = {{0}};
    size_t bb = q5 ? 176 : 144;
    for (size_t b = 0; b < cols / 256; ++b) {
        const uint8_t* p = row + b * bb;
        float d = zqo_half_to_float(rd16(p)), dm = zqo_half_to_float(rd16(p + 2));
        for (unsigned group = 0; group < 8; ++group) {
            unsigned sc, mn;
            k_scale_min(group, p + 4, &sc, &mn);
            float ds = d * (float)sc, ms = dm * (float)mn;
            for (unsigned chunk = 0; chunk < 4; ++chunk)
                for (unsigned i = 0; i < 8; ++i) {
                    unsigned e = group * 32 + chunk * 8 + i;
                    float t = ds * (float)kquant_q(p, e, q5);
                    float w = t - ms;
                    acc[chunk][i] = fmaf(w, x[b * 256 + e], acc[chunk][i]);
                }
        }
    }
    float v[8];
    for (int i = 0; i < 8; ++i) v[i] = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
    return hsum8(v);
}
/* gemv_avx2 on one fp32 row: kernels/avx2.cpp:16-39 (four 8-lane
 * accumulators over 32-column strides, sequential lane sum). */
static float dot_gemv_avx2(const float* row, const float* x, size_t k) {
    float s[4][8] = {{0}};
    size_t p = 0;
    for (; p + 31 < k; p += 32)
        for (int c = 0; c < 4; ++c)
            for (int i = 0; i < 8; ++i) s[c][i] = fmaf(row[p + c * 8 + i], x[p + c * 8 + i], s[c][i]);
    float sum[8];
    for (int i = 0; i < 8; ++i) sum[i] = (s[0][i] + s[1][i]) + (s[2][i] + s[3][i]);
    for (; p + 7 < k; p += 8) for (int i = 0; i < 8; ++i) sum[i] = fmaf(row[p + i], x[p + i], sum[i]);
    float total = sum[0] + sum[1] + sum[2] + sum[3] + sum[4] + sum[5] + sum[6] + sum[7];
    for (; p < k; ++p) total += row[p] * x[p];
    return total;
}

/* quant::gemv with fp32 activations (the reference default):
 * Q8_0 -> gemv_q8_0_avx2 (src/quant.cpp:1080-1133), Q6_K -> gemv_q6k_avx2
 * (:1039-1054), Q4_K / Q5_K -> gemv_q4k_q5k_avx2 (:1016-1032), Q4_0 ->
 * dequantise row + gemv_avx2 (:1135-1162). */
int zqo_gemv_f32(int fmt, const uint8_t* w, const float* x, float* y, size_t rows, size_t cols) {
    size_t rb = zqo_row_bytes(fmt, cols); if (!rb) return 0;
    float* tmp = NULL;
    if (fmt == ZQO_Q4_0) { tmp = (float*)malloc(sizeof(float) * cols); if (!tmp) return 0; }
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t* row = w + r * rb;
        if (fmt == ZQO_Q8_0) y[r] = gemv_row_q8_0(row, x, cols);
        else if (fmt == ZQO_Q6_K) y[r] = gemv_row_q6_k(row, x, cols);
        else if (fmt == ZQO_Q4_K || fmt == ZQO_Q5_K) y[r] = gemv_row_kquant(row, x, cols, fmt == ZQO_Q5_K);
        else { zqo_dequantize(fmt, row, cols, tmp); y[r] = dot_gemv_avx2(tmp, x, cols); }
    }
    free(tmp);
    return 1;
}

/* Double-precision reference over the dequantised weights, in the style of
 * tools/hip_parity.cpp:106-124.  mag receives sum |w*x| when non-NULL. */
int zqo_gemm_f64(int fmt, const uint8_t* w, const float* X, double* Y, double* mag, size_t m, size_t n, size_t k) {
    size_t rb = zqo_row_bytes(fmt, k); if (!rb) return 0;
    float* row = (float*)malloc(sizeof(float) * k); if (!row) return 0;
    for (size_t r = 0; r < n; ++r) {
        zqo_dequantize(fmt, w + r * rb, k, row);
        for (size_t t = 0; t < m; ++t) {
            double acc = 0, a = 0;
            for (size_t c = 0; c < k; ++c) { double term = (double)row[c] * (double)X[t * k + c]; acc += term; a += fabs(term); }
            Y[t * n + r] = acc; if (mag) mag[t * n + r] = a;
        }
    }
    free(row);
    return 1;
}

/* dot_f32_avx2: kernels/avx2.cpp:696-710 (two 8-lane accumulators over
 * 16-column strides, one 8-wide tail, sequential lane sum, scalar tail). */
static float dot_f32_avx2(const float* a, const float* b, size_t n) {
    float s0[8] = {0}, s1[8] = {0}, s[8];
    size_t i = 0;
    for (; i + 15 < n; i += 16)
        for (int j = 0; j < 8; ++j) { s0[j] = fmaf(a[i + j], b[i + j], s0[j]); s1[j] = fmaf(a[i + 8 + j], b[i + 8 + j], s1[j]); }
    for (int j = 0; j < 8; ++j) s[j] = s0[j] + s1[j];
    for (; i + 7 < n; i += 8) for (int j = 0; j < 8; ++j) s[j] = fmaf(a[i + j], b[i + j], s[j]);
    float t = s[0] + s[1] + s[2] + s[3] + s[4] + s[5] + s[6] + s[7];
    for (; i < n; ++i) t += a[i] * b[i];
    return t;
}
/* Main-block order shared by gemm_q8_0_avx2 (kernels/avx2.cpp:797-820),
 * gemm_q8_0_kblk_avx2 (:878-1061) and gemm_kblk_impl (:1470-1534): one 8-lane
 * FMA accumulator over c = 0,8,16,..., then lane0+...+lane7, then a scalar
 * tail for columns past the last multiple of 8. */
static float dot_main_order(const float* row, const float* x, size_t k) {
    float a[8] = {0};
    size_t c = 0;
    for (; c + 8 <= k; c += 8) for (int i = 0; i < 8; ++i) a[i] = fmaf(row[c + i], x[c + i], a[i]);
    float total = a[0] + a[1] + a[2] + a[3] + a[4] + a[5] + a[6] + a[7];
    for (; c < k; ++c) total += row[c] * x[c];
    return total;
}

/* quant::gemm with fp32 activations (reference CPU semantics on one worker;
 * output token-major Y[t*n + r], include/zen/quant.h:28-30).
 *  Q8_0, tokens >= 2 (src/quant.cpp:1661-1684, 1366-1388):
 *    tokens*cols >= 131072 (q8_use_kblk, :1188-1192) -> gemm_q8_0_kblk_avx2:
 *      rows in groups of 4 use the main order, trailing rows dot_f32_avx2;
 *    otherwise gemm_q8_0_avx2 (kernels/avx2.cpp:772-840): row pairs x token
 *      quads use the main order, leftover tokens and an odd last row use
 *      dot_f32_avx2.
 *  Q6_K -> gemm_q6k_kblk_avx2 = gemm_kblk_impl (:1729-1770, :1470-1545),
 *  Q4_K -> gemm_q4k_kblk_avx2 (:1613-1628), Q5_K -> gemm_q5k_kblk_avx2
 *    (:1605-1611), both gemm_kblk_impl over panels that dequantise to the
 *    dequantize() values (:1351-1435): rows in groups of 4 main order,
 *    trailing rows dot_f32_avx2.
 *  Q4_0 -> generic route (src/quant.cpp:1747-1776): dequantise row, then
 *    gemv_avx2 per token.
 *  tokens == 1: every fast route needs tokens >= 2 (:1661, :1701, :1715), so
 *    a single token takes the generic route too. */
int zqo_gemm_f32(int fmt, const uint8_t* w, const float* X, float* Y, size_t m, size_t n, size_t k) {
    size_t rb = zqo_row_bytes(fmt, k); if (!rb) return 0;
    float* row = (float*)malloc(sizeof(float) * k); if (!row) return 0;
    int kblk = fmt == ZQO_Q6_K || fmt == ZQO_Q4_K || fmt == ZQO_Q5_K || (fmt == ZQO_Q8_0 && m * k >= 131072);
    size_t rows_main = kblk ? n / 4 * 4 : n / 2 * 2;
    for (size_t r = 0; r < n; ++r) {
        zqo_dequantize(fmt, w + r * rb, k, row);
        for (size_t t = 0; t < m; ++t) {
            const float* x = X + t * k;
            float v;
            if (fmt == ZQO_Q4_0 || m == 1) v = dot_gemv_avx2(row, x, k);
            else if (r >= rows_main) v = dot_f32_avx2(row, x, k);
            else if (kblk) v = dot_main_order(row, x, k);
            else v = t < m / 4 * 4 ? dot_main_order(row, x, k) : dot_f32_avx2(row, x, k);
            Y[t * n + r] = v;
        }
    }
    free(row);
    return 1;
}

/* GEMM with int8 activations (the reference's int8 arithmetic).
 * Q8_0 follows gemv_q8_0_avx2_int8_prequant (kernels/avx2.cpp:562-585) per
 * token: per block, eight int32 lane partials (each the sum of four
 * neighbouring products), d = d_w*d_x, acc[lane] = fma(d, float(p), acc),
 * then hsum_ps256.  Q4_0 / Q6_K have no int8 route in the reference; here
 * acc = fma(d_w*d_x, float(block_dot), acc) per block, with block_dot from
 * zqo_block_dots (Q6_K: d_w is the super-block d; the int8 sub-scales are
 * inside the integer dot).  xq / xs are already-quantised activations
 * (zqo_quantize_acts's layout: int8 [m][k], fp32 [m][k/32]). */
int zqo_gemm_i8_prequant(int fmt, const uint8_t* w, const int8_t* xq, const float* xs, float* Y, size_t m, size_t n,
                         size_t k) {
    size_t rb = zqo_row_bytes(fmt, k); if (!rb || k % 32 || fmt == ZQO_Q4_K || fmt == ZQO_Q5_K) return 0;
    size_t nb = k / 32;
    int32_t* dots = NULL;
    if (fmt != ZQO_Q8_0) {
        dots = (int32_t*)malloc(sizeof(int32_t) * m * n * nb);
        if (!dots || !zqo_block_dots(fmt, w, xq, m, n, k, dots)) { free(dots); return 0; }
    }
    for (size_t t = 0; t < m; ++t)
        for (size_t r = 0; r < n; ++r) {
            const uint8_t* row = w + r * rb;
            if (fmt == ZQO_Q8_0) {
                float acc[8] = {0};
                for (size_t b = 0; b < nb; ++b) {
                    const uint8_t* p = row + b * 34;
                    float d = zqo_half_to_float(rd16(p)) * xs[t * nb + b];
                    const int8_t* qa = xq + t * k + b * 32;
                    for (int i = 0; i < 8; ++i) {
                        int32_t p32 = 0;
                        for (int j = 0; j < 4; ++j) p32 += (int32_t)(int8_t)p[2 + 4 * i + j] * (int32_t)qa[4 * i + j];
                        acc[i] = fmaf(d, (float)p32, acc[i]);
                    }
                }
                Y[t * n + r] = hsum8(acc);
            } else {
                float acc = 0.0f;
                for (size_t b = 0; b < nb; ++b) {
                    float dw = fmt == ZQO_Q4_0 ? zqo_half_to_float(rd16(row + b * 18))
                                               : zqo_half_to_float(rd16(row + (b / 8) * 210 + 208));
                    float d = dw * xs[t * nb + b];
                    acc = fmaf(d, (float)dots[(t * n + r) * nb + b], acc);
                }
                Y[t * n + r] = acc;
            }
        }
    free(dots);
    return 1;
}

/* The same from fp32 activations: zqo_quantize_acts, then the above. */
int zqo_gemm_i8(int fmt, const uint8_t* w, const float* X, float* Y, size_t m, size_t n, size_t k) {
    size_t rb = zqo_row_bytes(fmt, k); if (!rb || k % 32 || fmt == ZQO_Q4_K || fmt == ZQO_Q5_K) return 0;
    int8_t* xq = (int8_t*)malloc(m * k); float* xs = (float*)malloc(sizeof(float) * m * (k / 32));
    if (!xq || !xs) { free(xq); free(xs); return 0; }
    zqo_quantize_acts(X, m, k, xq, xs);
    int ok = zqo_gemm_i8_prequant(fmt, w, xq, xs, Y, m, n, k);
    free(xq); free(xs);
    return ok;
}
