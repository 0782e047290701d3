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
// Kernels (int8 mode):
//  * gemm_i8_direct4_kernel (K % 256 == 0, M > 64):
//    128 (tokens) x 128 (weight rows) tiles, 8 waves of 64x32; activations,
//    raw weight blocks and scales stream straight from HBM into LDS
//    (buffer_load ... lds), double-buffered by 4 K blocks; the B
//    operand is assembled per lane from the raw Q8_0 / Q4_0 blocks;
//  * gemm_i8_small_kernel (K % 256 == 0, M <= 64): the same body with
//    32-token tiles, 4 waves;
//  * gemm_i8_kernel (any K % 64 == 0): 4 waves of 2x2 MFMA tiles, weights
//    converted while staged through registers into LDS.
// Small grids split K; the partial sums are reduced in a fixed order.
// Workgroup ids are remapped so that the workgroups a given XCD receives
// (ids congruent mod 8) walk the token tiles of one weight panel before
// moving on, keeping that panel in the XCD's L2.
#include "zq_device.hpp"
#include "zq_internal.hpp"

#include <algorithm>
#include <type_traits>
#include <cmath>
#include <cstdlib>

namespace zq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int kThreads = 256;
constexpr int BM = 128;             // tokens per tile
constexpr int BN = 128;             // weight rows per tile
constexpr int KB = 8;               // 32-element blocks per K stage
constexpr int ROWB = KB * 32 + 16;  // LDS bytes per tile row (16 B pad)

// ------------------------------------------------- activation quantiser ---
// Bit-exact with kernels/avx2.cpp:502-524.

// Eight lanes per block, four elements each (a coalesced float4 load and a
// 4-byte store per lane); the block's amax is the max over its eight lanes
// (DPP, exact), so d, 1/d and every quant equal the one-thread-per-block form.
__global__ __launch_bounds__(kThreads) void quantize_acts_kernel(const float* __restrict__ X, int8_t* __restrict__ xq,
                                                                 float* __restrict__ xs, size_t nblocks) {
    const size_t g = size_t(blockIdx.x) * kThreads + threadIdx.x;  // lane's 4-element group
    const size_t b = g >> 3;
    const bool live = b < nblocks;
    const float4 t = live ? reinterpret_cast<const float4*>(X)[g] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float v[4] = {t.x, t.y, t.z, t.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    amax = fmaxf(amax, dpp_f<kDppXor1>(amax));  // |x| >= 0, so fmaxf is the same max
    amax = fmaxf(amax, dpp_f<kDppXor2>(amax));
    amax = fmaxf(amax, dpp_f<kDppHalfMirror>(amax));
    if (!live) return;
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    if ((g & 7) == 0) xs[b] = d;
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float q = v[k] * inv;
        q = q > 127.0f ? 127.0f : (q < -127.0f ? -127.0f : q);
        w |= (uint32_t(round_half_away(q)) & 0xffu) << (8 * k);
    }
    reinterpret_cast<uint32_t*>(xq)[g] = w;
}

// ------------------------------------------------------- tile mapping ---
#ifndef ZQ_GEMM_XCD_BLOCKS
#define ZQ_GEMM_XCD_BLOCKS 1
#endif
__device__ __forceinline__ void tile_of(uint32_t tiles_m, uint32_t tiles_n, uint32_t id, uint32_t& tm, uint32_t& tn) {
    const uint32_t total = tiles_m * tiles_n;
    uint32_t slot = id;
    if (ZQ_GEMM_XCD_BLOCKS && tiles_m % 4 == 0 && tiles_n % 2 == 0) {
        // XCD x (ids congruent to x mod 8) owns a quarter of the token tiles
        // and half of the weight panels, walking its token tiles per panel:
        // its activation rows stay in its L2, and each weight panel is read
        // by two XCDs.
        const uint32_t x = id % 8u, local = id / 8u, qm = tiles_m / 4;
        tm = (x & 3u) * qm + local % qm;
        tn = (x >> 2) * (tiles_n / 2) + local / qm;
        return;
    }
    if (total % 8u == 0) {
        const uint32_t per_xcd = total / 8u;
        slot = (id % 8u) * per_xcd + id / 8u;
    }
    tn = slot / tiles_m;
    tm = slot % tiles_m;
}

// ------------------------------------------------------- int8 GEMM -------
// DOTS = true is the bit-exact test mode: instead of accumulating, the
// kernel stores every per-block int32 MFMA result to dots[(m*N + n)*nb + b].
//
// Pipeline per K stage (KB = 4 blocks): the stage's activations, weights and
// scales were fetched into registers during the previous stage's compute;
// they are written to LDS (weights converted from native blocks), then the
// next stage's global loads are issued, then the 4 blocks are computed.
// Epilogue per (32x32 tile, block): the scale products dx[m]*dw[n] come from
// one fp32 outer-product MFMA (v_mfma_f32_32x32x2f32 with the second K slot
// zero), which lands them in exactly the accumulator layout, so the VALU
// work is one v_cvt_f32_i32 and one v_fma per output element and block.
//
// Split-K: with ksplit > 1 the grid is ksplit x tiles; workgroup group `split`
// covers stages [split*spw, (split+1)*spw) and stores its partial tile to
// Y + split*M*N (a workspace), summed afterwards in fixed order by
// splitk_reduce_kernel, so results do not depend on scheduling.
template <int FMT, bool DOTS>
__global__ __launch_bounds__(kThreads, 2) void gemm_i8_kernel(const uint8_t* __restrict__ W, const int8_t* __restrict__ XQ,
                                                           const float* __restrict__ XS, float* __restrict__ Y,
                                                           int32_t* __restrict__ dots, uint32_t M, uint32_t N,
                                                           uint32_t K, uint32_t tiles_m, uint32_t tiles_n,
                                                           uint32_t ksplit, uint32_t stages_per_split) {
    constexpr uint32_t PB = FMT == kQ8_0 ? 68 : 36;  // bytes per block pair
    constexpr int PW = FMT == kQ8_0 ? 17 : 9;         // dwords per block pair
    __shared__ __align__(16) int8_t As[BM * ROWB];
    __shared__ __align__(16) int8_t Bs[BN * ROWB];
    __shared__ __align__(16) float Sx[KB][BM];
    __shared__ __align__(16) float Sw[KB][BN];

    const uint32_t total_tiles = tiles_m * tiles_n;
    const uint32_t split = blockIdx.x / total_tiles;
    uint32_t tm, tn;
    tile_of(tiles_m, tiles_n, blockIdx.x % total_tiles, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t nb = K >> 5;
    const uint32_t rb = (nb >> 1) * PB;
    const uint32_t kb_begin = split * stages_per_split * KB;
    const uint32_t kb_end = min(nb, kb_begin + stages_per_split * KB);
    float* Yout = Y + (ksplit > 1 ? size_t(split) * M * N : 0);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lh = lane >> 5;

    // loader coordinates: 2 threads per tile row; thread (row, half) moves the
    // half's 4 blocks (2 pairs) of activations and weights, and 4 scales
    constexpr int SPT = KB * BM / kThreads;  // activation scales per thread
    const int ld_row = tid >> 1, ld_half = tid & 1;
    const int8_t* a_src = XQ + size_t(min(m0 + ld_row, M - 1)) * K;
    const uint8_t* b_src = W + size_t(min(n0 + ld_row, N - 1)) * rb;
    const float* s_src[SPT];
#pragma unroll
    for (int r = 0; r < SPT; ++r) s_src[r] = DOTS ? nullptr : XS + size_t(min(m0 + ((tid + r * kThreads) % BM), M - 1)) * nb;

    uint4 ra[2][4];
    uint32_t rw[2][PW];
    float rs[SPT] = {};
    // Loads are unconditional (block index clamped into the row, nb is even),
    // so the compiler emits no branch / vmcnt(0) around them; blocks past the
    // end of K are neutralised through zero scales in commit().
    auto fetch = [&](uint32_t kb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t blk = min(kb + 4 * ld_half + 2 * h, nb - 2);
            const uint4* sa = reinterpret_cast<const uint4*>(a_src + size_t(blk) * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) ra[h][i] = sa[i];
            const uint32_t* sw = reinterpret_cast<const uint32_t*>(b_src + size_t(blk >> 1) * PB);
#pragma unroll
            for (int i = 0; i < PW; ++i) rw[h][i] = sw[i];
        }
        if constexpr (!DOTS) {  // the DOTS launch has no scale buffer (XS is null)
#pragma unroll
            for (int r = 0; r < SPT; ++r) {
                const uint32_t kk = (tid + r * kThreads) / BM;
                rs[r] = s_src[r][min(kb + kk, nb - 1)];
            }
        }
    };
    auto commit_pair = [&](uint32_t kb, int h) {
        const uint32_t* rwp = rw[h];
        uint4* da = reinterpret_cast<uint4*>(As + ld_row * ROWB + ld_half * 128 + h * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) da[i] = ra[h][i];
        uint32_t out[16];
        float d0, d1;
        if constexpr (FMT == kQ8_0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) out[i] = __builtin_amdgcn_alignbyte(rwp[i + 1], rwp[i], 2);
#pragma unroll
            for (int i = 0; i < 8; ++i) out[8 + i] = rwp[9 + i];
            d0 = half_bits_to_float(rwp[0]);
            d1 = half_bits_to_float(rwp[8] >> 16);
        } else {
            uint32_t qa[4], qb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qa[i] = __builtin_amdgcn_alignbyte(rwp[i + 1], rwp[i], 2);
                qb[i] = rwp[5 + i];
            }
            // byte-wise n - 8 for n in [0,15]: ((n | 0x80) - 8) ^ 0x80, no borrow across bytes
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                out[i] = (((qa[i] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
                out[4 + i] = ((((qa[i] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
                out[8 + i] = (((qb[i] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
                out[12 + i] = ((((qb[i] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
            }
            d0 = half_bits_to_float(rwp[0]);
            d1 = half_bits_to_float(rwp[4] >> 16);
        }
        const int bl = 4 * ld_half + 2 * h;  // block index within the stage
        if (kb + bl >= nb) { d0 = 0.0f; d1 = 0.0f; }
        uint4* db = reinterpret_cast<uint4*>(Bs + ld_row * ROWB + bl * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) db[i] = make_uint4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
        Sw[bl][ld_row] = d0;
        Sw[bl + 1][ld_row] = d1;
    };
    auto commit = [&](uint32_t kb) {
        // Opaque register fence: the conversion below must not be hoisted up to
        // the prefetch loads (that would make the compiler wait for them right
        // after issuing them, before the compute loop).
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < PW; ++i) asm volatile("" : "+v"(rw[h][i]));
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(ra[h][i].x), "+v"(ra[h][i].y), "+v"(ra[h][i].z), "+v"(ra[h][i].w));
        }
#pragma unroll
        for (int r = 0; r < SPT; ++r) asm volatile("" : "+v"(rs[r]));
        commit_pair(kb, 0);
        commit_pair(kb, 1);
        if constexpr (!DOTS) {
#pragma unroll
            for (int r = 0; r < SPT; ++r) {
                const int idx = tid + r * kThreads;
                Sx[idx / BM][idx % BM] = kb + idx / BM < nb ? rs[r] : 0.0f;
            }
        }
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const v16f fzero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    if (kb_begin < kb_end) fetch(kb_begin);
    else return;
    for (uint32_t kb = kb_begin; kb < kb_end; kb += KB) {
        __syncthreads();
        commit(kb);
        __syncthreads();
        fetch(min(kb + KB, kb_end - 1));  // unconditional: the last one re-reads in-range data, unused
        // Operands of block b+1 are read from LDS while block b computes, and
        // tile t+1's two MFMAs are issued before tile t's VALU epilogue, so
        // the matrix pipe, LDS and VALU overlap inside one wave.
        struct Ops {
            v4i a[2], w[2];
            float dx[2], dw[2];
        };
        auto read_ops = [&](int b, Ops& o) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                o.a[i] = *reinterpret_cast<const v4i*>(As + (wm * 64 + i * 32 + l32) * ROWB + b * 32 + lh * 16);
                o.dx[i] = lh ? 0.0f : Sx[b][wm * 64 + i * 32 + l32];
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                o.w[j] = *reinterpret_cast<const v4i*>(Bs + (wn * 64 + j * 32 + l32) * ROWB + b * 32 + lh * 16);
                o.dw[j] = lh ? 0.0f : Sw[b][wn * 64 + j * 32 + l32];
            }
        };
        Ops cur;
        read_ops(0, cur);
#pragma unroll 1
        for (int b = 0; b < KB; ++b) {
            Ops nxt;
            read_ops(b + 1 < KB ? b + 1 : b, nxt);
            if constexpr (DOTS) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int i = t >> 1, j = t & 1;
                    const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[i], cur.w[j], zero, 0, 0, 0);
                    const uint32_t n = n0 + wn * 64 + j * 32 + l32;
                    const uint32_t blk = kb + b;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                        if (m < M && n < N && blk < nb) dots[(size_t(m) * N + n) * nb + blk] = c[v];
                    }
                }
            } else {
                v16i c[2];
                v16f sc[2];
                c[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[0], cur.w[0], zero, 0, 0, 0);
                sc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.dx[0], cur.dw[0], fzero, 0, 0, 0);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int i = t >> 1, j = t & 1;
                    if (t < 3) {
                        const int i2 = (t + 1) >> 1, j2 = (t + 1) & 1;
                        c[(t + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[i2], cur.w[j2], zero, 0, 0, 0);
                        sc[(t + 1) & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.dx[i2], cur.dw[j2], fzero, 0, 0, 0);
                    }
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(float(c[t & 1][v]), sc[t & 1][v], acc[i][j][v]);
                }
            }
            cur = nxt;
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
                if (m < M && n < N) Yout[size_t(m) * N + n] = acc[i][j][v];
            }
        }
}

// Y = sum of the ksplit partial planes in split order; four outputs a thread
// (float4) when n % 4 == 0 and both buffers are 16-byte aligned, else one.
template <bool VEC4>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(const float* __restrict__ part, float* __restrict__ Y,
                                                                 size_t n, uint32_t ksplit) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if constexpr (VEC4) {
        const size_t n4 = n / 4;
        if (i >= n4) return;
        const float4* p = reinterpret_cast<const float4*>(part);
        float4 acc = p[i];
        for (uint32_t s = 1; s < ksplit; ++s) {
            const float4 t = p[size_t(s) * n4 + i];
            acc.x += t.x; acc.y += t.y; acc.z += t.z; acc.w += t.w;
        }
        reinterpret_cast<float4*>(Y)[i] = acc;
    } else {
        if (i >= n) return;
        float acc = part[i];
        for (uint32_t s = 1; s < ksplit; ++s) acc += part[size_t(s) * n + i];
        Y[i] = acc;
    }
}

// Q8_0 int8 GEMM with direct-to-LDS staging (K % 256 == 0, 16 B aligned
// weight rows).  512 threads = 8 waves in 2 (tokens) x 4 (rows), each wave a
// 64 x 32 output tile (two 32x32 MFMA tiles).  A K stage is 8 blocks.
//
// Staging: global_load_lds_dwordx4 moves 16 B per lane from HBM straight into
// LDS (64 lanes -> 1 KiB contiguous), so stages cost no VGPRs and no LDS
// store instructions.  LDS holds two stages; stage s+1 streams into one
// buffer while stage s is computed from the other, with one barrier a stage.
//  * activations: 128 rows x 256 B, the 16 B columns of row r XOR-swizzled
//    by (r & 15) so the MFMA A reads (32 consecutive rows, one column) hit
//    distinct banks without row padding;
//  * weights: 128 rows x 272 B, the raw native blocks (8 x 34 B contiguous in
//    the row), units of 16 B in row-major order; the B operand of block b,
//    half h is assembled at read time: odd blocks start dword-aligned
//    (4 dword reads), even blocks at 2 mod 4 (5 reads + 4 v_alignbyte);
//  * activation scales: [8][128] floats, one 4 B lane load each.
// Epilogue: per block one 2-block outer-product MFMA gives dx*dw for both
// tiles in the accumulator layout, then one cvt + one fma per element.
constexpr int QTH = 512;
// Stage geometry for QKB blocks per K stage (8: 144 KB of LDS, one workgroup
// per CU; 4: 72 KB, two).  Weight row r starts at LDS dword r * W_STRIDE, the
// row's stage bytes rounded up to whole 16 B units, so each weight load moves
// 16 B per lane.  (An odd stride, 69 / 35 dwords, made the B reads conflict-free
// but needed 4 B loads, 4x the load instructions; the 16 B form measured 4-7%
// faster at M = 512 and 2048 despite 2-way B-read conflicts.)
template <int QKB, int BMT = BM, int NW = QTH / 64, int BB = 34>
struct QStage {
    static constexpr int A_BYTES = BMT * QKB * 32;          // activation tile
    static constexpr int UPR = QKB * 2;                     // 16 B units per activation row
    // XOR swizzle of a row's 16 B units, so the 16 rows that a half-wave's
    // ds_read_b128 touches fall on distinct 16 B bank groups: with 256 B rows
    // (8-block stages) row % 16; with 128 B rows two rows share a 256 B bank
    // line, so the swizzle takes (row / 2) % 8.
    __device__ static int swz(int row) { return UPR == 16 ? row % 16 : (row >> 1) & 7; }
    static_assert(UPR == 8 || UPR == 16, "4- or 8-block stages");
    static constexpr int WD = QKB * BB / 4;                 // raw dwords of a weight row per stage (BB = block bytes)
    static constexpr int W_STRIDE = (WD + 4) & ~3;          // 36 / 20: whole 16 B units per row
    static constexpr int W_UNITS = BN * W_STRIDE / 4;
    static constexpr int W_LOADS = (W_UNITS + 63) / 64;     // 64-lane 16 B loads per stage
    static constexpr int W_PER_WAVE = (W_LOADS + NW - 1) / NW;
    static constexpr int W_BYTES = W_LOADS * 64 * 16;
    static constexpr int S_BYTES = QKB * BMT * 4;
    static constexpr int S_UNITS = S_BYTES / 256;           // 64-lane dword loads of scales per stage
    static constexpr int S_PER_WAVE = (S_UNITS + NW - 1) / NW;
    static constexpr int BUF = A_BYTES + W_BYTES + S_BYTES;  // bytes per stage buffer
    static_assert(2 * BUF <= 160 * 1024, "two stage buffers must fit the 160 KiB LDS");
    static_assert(A_BYTES % (1024 * NW) == 0, "activation units split evenly over the waves");
    static_assert(S_BYTES % 256 == 0 && A_BYTES % 16 == 0 && W_BYTES % 16 == 0, "LDS regions stay 16 B aligned");
};

typedef __attribute__((address_space(3))) void lds_void;

// Word 3 of a raw buffer resource on gfx9-family parts (32-bit data format,
// no swizzle, stride 0): offsets are plain byte offsets from the base.
constexpr int kBufferWord3 = 0x00020000;

// The kernel body, one instantiation per stage depth QKB and per tile height:
// WM = 2 is the 128-token tile above (8 waves in 2 x 4, two 32x32 MFMA tiles
// each); WM = 1 is a 32-token tile for small M (4 waves side by side, one
// MFMA tile each), where the scale products of a pair of K blocks come from
// one 2-block outer-product MFMA (block i = lane half i = K block 2j + i).
// The __global__ wrappers below carry the launch bounds (second argument:
// minimum waves per SIMD).
template <int FMT, bool DOTS, int QKB, int WM = 2>
__device__ __forceinline__ void gemm_i8_direct_body(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ XQ, const float* __restrict__ XS,
    float* __restrict__ Y, int32_t* __restrict__ dots, uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m,
    uint32_t tiles_n, uint32_t ksplit, uint32_t stages_per_split) {
    constexpr int BMT = WM == 2 ? BM : 32;  // tokens per tile
    constexpr int NW = WM == 2 ? 8 : 4;     // waves per workgroup
    constexpr int BB = FMT == kQ8_0 ? 34 : 18;  // block bytes: fp16 d + 32 int8 / 16 nibble bytes
    static_assert(FMT == kQ8_0 || FMT == kQ4_0, "int8-activation formats only");
    using G = QStage<QKB, BMT, NW, BB>;
    extern __shared__ __align__(16) uint8_t lds[];  // 2 * G::BUF bytes, sized at launch

    const uint32_t total_tiles = tiles_m * tiles_n;
    const uint32_t split = blockIdx.x / total_tiles;
    uint32_t tm, tn;
    tile_of(tiles_m, tiles_n, blockIdx.x % total_tiles, tm, tn);
    const uint32_t m0 = tm * BMT, n0 = tn * BN;
    const uint32_t nb = K >> 5;
    const uint32_t rb = nb * BB;
    const uint32_t kb_begin = split * stages_per_split * QKB;
    const uint32_t kb_end = min(nb, kb_begin + stages_per_split * QKB);
    float* Yout = Y + (ksplit > 1 ? size_t(split) * M * N : 0);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = WM == 2 ? wave >> 2 : 0, wn = wave & 3;
    const int l32 = lane & 31, lh = lane >> 5;

    // Direct loads go through buffer resources based at this tile's first
    // activation row, weight row and scale row: per-lane 32-bit offsets
    // (computed once) plus the stage's scalar offset.  Rows past M or N are
    // clamped to the last one.
    constexpr int A_LOADS = G::A_BYTES / 1024 / NW;
    const __amdgpu_buffer_rsrc_t a_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(XQ + size_t(m0) * K), 0, -1, kBufferWord3);
    const __amdgpu_buffer_rsrc_t w_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(W + size_t(n0) * rb), 0, -1, kBufferWord3);
    const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(DOTS ? XQ : reinterpret_cast<const int8_t*>(XS + size_t(m0) * nb)), 0, -1, kBufferWord3);
    uint32_t a_off[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        const int unit = (wave * A_LOADS + i) * 64 + lane;  // physical 16 B slot
        const int row = unit / G::UPR, col = (unit % G::UPR) ^ G::swz(row);
        a_off[i] = (min(m0 + row, M - 1) - m0) * K + col * 16;
    }
    // Weight loads in 16 B units: LDS dword p of the region holds raw dword d
    // of row r (p = r*G::W_STRIDE + d); a row's last unit runs 2 dwords past its
    // stage bytes into the row's next bytes (the matrix's tail pad after the
    // last row), unused.
    // Rows 16-31 of every 32-row group are fetched 8 bytes early, so their
    // stage bytes sit 2 dwords further into their LDS row: with the stride a
    // multiple of 4 dwords the two halves of a B read then fall on disjoint
    // banks (dword index = 0 or 2 mod 4), where they would pair up 2-way.
    // Only a row clamped onto the tile's first row (past N) could reach
    // before the tile; it reads offset 0 instead, and is never used.
    uint32_t w_off[G::W_PER_WAVE];
#pragma unroll
    for (int i = 0; i < G::W_PER_WAVE; ++i) {
        const uint32_t u = uint32_t((wave + NW * i) * 64 + lane);
        const uint32_t r = min(4 * u / G::W_STRIDE, uint32_t(BN - 1));
        const uint32_t d = 4 * u - r * G::W_STRIDE;
        const uint32_t off = (min(n0 + r, N - 1) - n0) * rb + d * 4;
        const uint32_t sh = (r & 16u) ? 8u : 0u;
        w_off[i] = off >= sh ? off - sh : 0u;
    }
    uint32_t s_off[G::S_PER_WAVE];
#pragma unroll
    for (int i = 0; i < G::S_PER_WAVE; ++i) {
        const int idx = (wave * G::S_PER_WAVE + i) * 64 + lane;  // = b * BMT + m
        s_off[i] = ((min(m0 + uint32_t(idx % BMT), M - 1) - m0) * nb + uint32_t(idx / BMT)) * 4;
    }
    auto stage_in = [&](uint32_t kb, int buf) {
        uint8_t* base = lds + buf * G::BUF;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_void*)(base + (wave * A_LOADS + i) * 1024), 16,
                                                     a_off[i], kb * 32, 0, 0);
#pragma unroll
        for (int i = 0; i < G::W_PER_WAVE; ++i)
            if (wave + NW * i < G::W_LOADS)  // wave-uniform
                __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_void*)(base + G::A_BYTES + (wave + NW * i) * 1024), 16,
                                                         w_off[i], kb * BB, 0, 0);
        if constexpr (!DOTS) {
#pragma unroll
            for (int i = 0; i < G::S_PER_WAVE; ++i)
                if (wave * G::S_PER_WAVE + i < G::S_UNITS)  // wave-uniform
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        s_rsrc, (lds_void*)(base + G::A_BYTES + G::W_BYTES + (wave * G::S_PER_WAVE + i) * 256), 4,
                        s_off[i], kb * 4, 0, 0);
        }
    };

    v16f acc[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    v32f szero;
#pragma unroll
    for (int v = 0; v < 32; ++v) szero[v] = 0.0f;
    const uint32_t nrow = wn * 32 + l32;  // this lane's weight row within the tile
    const uint32_t wrow = nrow * G::W_STRIDE + ((l32 & 16) ? 2u : 0u);  // its first LDS dword (rows 16-31 shifted)

    // LDS operands of one block, read one step ahead of their MFMAs.
    struct Ops {
        v4i a[WM];
        uint32_t t[5];  // raw weight dwords (4 used for odd blocks)
        uint32_t dwh;   // fp16 weight scale bits
        float dx;
    };
    auto read_ops = [&](const uint8_t* base, int b, int odd, Ops& o) {
        const uint32_t* Bw = reinterpret_cast<const uint32_t*>(base + G::A_BYTES) + wrow;
        // Q8_0: lane half lh takes quant bytes lh*16..+15; Q4_0: both halves
        // read the 16 nibble bytes (low nibbles = elements 0-15, high 16-31)
        const int off = (b * BB + 2 + (FMT == kQ8_0 ? lh * 16 : 0)) >> 2;
#pragma unroll
        for (int i = 0; i < 4 + (odd ? 0 : 1); ++i) o.t[i] = Bw[off + i];
        // WM = 2: scales of block b (lane half = tile); WM = 1: of block
        // b - 1 + lh for the odd block of a pair (the even block needs none)
        const int sb = WM == 2 ? b : b - 1 + lh;
        o.dwh = WM == 2 || odd ? reinterpret_cast<const uint16_t*>(Bw)[sb * (BB / 2)] : 0u;
        o.dx = DOTS || (WM == 1 && !odd)
                   ? 0.0f
                   : reinterpret_cast<const float*>(base + G::A_BYTES + G::W_BYTES)[WM == 2 ? b * BMT + wm * 64 + lh * 32 + l32
                                                                                         : sb * BMT + l32];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int row = wm * 64 + i * 32 + l32, col = (b * 2 + lh) ^ G::swz(row);
            o.a[i] = *reinterpret_cast<const v4i*>(base + row * (QKB * 32) + col * 16);
        }
    };
    // In-flight results of one block: the tiles' int32 dots and, from one
    // 2-block outer-product MFMA, the dx*dw products in the same layout.  WM =
    // 2: block i of the product = tile i of this K block.  WM = 1: issued with
    // the odd block of a pair, block i = K block 2j + i of the single tile.
    struct Blk {
        v16i c[WM];
        v32f s;
    };
    auto issue = [&](const Ops& o, int odd, Blk& r) {
        if constexpr (!DOTS && WM == 1)  // first, so the even block's retire finds it done
            if (odd) r.s = __builtin_amdgcn_mfma_f32_32x32x1f32(o.dx, half_bits_to_float(uint16_t(o.dwh)), szero, 0, 0, 0);
        v4i w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = odd ? int(o.t[i]) : int(__builtin_amdgcn_alignbyte(o.t[i + 1], o.t[i], 2));
        if constexpr (FMT == kQ4_0) {
            // nibble u of this lane half -> int8 u - 8, per byte without carries:
            // u + 0x78 stays below 0x100, and flipping bit 7 subtracts 0x80
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[i] = int(((uint32_t(w[i]) >> (4 * lh)) & 0x0F0F0F0Fu) + 0x78787878u) ^ int(0x80808080u);
        }
#pragma unroll
        for (int i = 0; i < WM; ++i) r.c[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[i], w, zero, 0, 0, 0);
        if constexpr (!DOTS && WM == 2)
            r.s = __builtin_amdgcn_mfma_f32_32x32x1f32(o.dx, half_bits_to_float(uint16_t(o.dwh)), szero, 0, 0, 0);
    };
    // Accumulates block r; sc/half name its dx*dw products (WM = 1: the pair's
    // odd block and this block's half of it; WM = 2: r itself).
    auto retire = [&](const Blk& r, const Blk& sc, int half) {
        if constexpr (WM == 2) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][v] = fmaf(float(r.c[i][v]), r.s[16 * i + v], acc[i][v]);
        } else {
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[0][v] = fmaf(float(r.c[0][v]), sc.s[16 * half + v], acc[0][v]);
        }
    };

    if (kb_begin >= kb_end) return;
    stage_in(kb_begin, 0);
    int buf = 0;
    for (uint32_t kb = kb_begin; kb < kb_end; kb += QKB, buf ^= 1) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct loads of stage kb landed
        __syncthreads();                     // ... and everyone's; the other buffer is free again
        if (kb + QKB < kb_end) stage_in(kb + QKB, buf ^ 1);
        const uint8_t* base = lds + buf * G::BUF;
        // Waves sharing a SIMD start the stage at different block pairs, so
        // one wave's MFMAs overlap the other's VALU epilogue instead of both
        // running the same phase in lockstep after the barrier.
        const int rot = (wave & 1) * (QKB / 2);
        if constexpr (DOTS) {
#pragma unroll 1
            for (int it = 0; it < QKB; it += 2) {
#pragma unroll
                for (int bp = 0; bp < 2; ++bp) {
                    const int b = ((it + rot) & (QKB - 1)) + bp;
                    Ops o;
                    Blk r;
                    read_ops(base, b, bp, o);
                    issue(o, bp, r);
                    const uint32_t n = n0 + nrow;
#pragma unroll
                    for (int i = 0; i < WM; ++i)
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                            if (m < M && n < N) dots[(size_t(m) * N + n) * nb + kb + b] = r.c[i][v];
                        }
                }
            }
        } else {
            // Three-step software pipeline over the stage's blocks: LDS reads
            // of block b+2, MFMAs of block b+1 and the cvt/fma epilogue of
            // block b are in flight together.
            Ops oe, oo;
            Blk p, q;
            read_ops(base, rot, 0, oe);
            read_ops(base, rot + 1, 1, oo);
            issue(oe, 0, p);
#pragma unroll 1
            for (int it = 0; it < QKB - 2; it += 2) {
                read_ops(base, (it + 2 + rot) & (QKB - 1), 0, oe);
                issue(oo, 1, q);
                retire(p, q, 0);
                read_ops(base, (it + 3 + rot) & (QKB - 1), 1, oo);
                issue(oe, 0, p);
                retire(q, q, 1);
            }
            issue(oo, 1, q);
            retire(p, q, 0);
            retire(q, q, 1);
        }
    }
    if constexpr (DOTS) return;
    const uint32_t n = n0 + nrow;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
            if (m < M && n < N) Yout[size_t(m) * N + n] = acc[i][v];
        }
}

template <int FMT, bool DOTS>
__global__ __launch_bounds__(QTH, 4) void gemm_i8_direct4_kernel(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ XQ, const float* __restrict__ XS,
    float* __restrict__ Y, int32_t* __restrict__ dots, uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m,
    uint32_t tiles_n, uint32_t ksplit, uint32_t stages_per_split) {
    gemm_i8_direct_body<FMT, DOTS, 4>(W, XQ, XS, Y, dots, M, N, K, tiles_m, tiles_n, ksplit, stages_per_split);
}
// 32-token tiles, 4 waves; 4-block stages (45 KB of LDS for both buffers) so
// three workgroups share a CU.
template <int FMT, bool DOTS>
__global__ __launch_bounds__(256, 3) void gemm_i8_small_kernel(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ XQ, const float* __restrict__ XS,
    float* __restrict__ Y, int32_t* __restrict__ dots, uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m,
    uint32_t tiles_n, uint32_t ksplit, uint32_t stages_per_split) {
    gemm_i8_direct_body<FMT, DOTS, 4, 1>(W, XQ, XS, Y, dots, M, N, K, tiles_m, tiles_n, ksplit, stages_per_split);
}

// Skinny int8 GEMM for M <= 64 (Q8_0 / Q4_0, K % 512 == 0): a 32-token x
// 32-row tile per workgroup, K stages of 16 blocks, and the workgroup's 4
// waves sharing the tile, each taking 4 of a stage's 16 blocks (the same
// 32x32x32 int8 MFMA and 2-block scale MFMA per block pair as the 32-token
// kernel above); the 4 partial tiles are summed through LDS in wave order at
// the end.  Why: at small M the weights are the traffic, and a stage now
// reads 32 rows x 16 blocks (544 B contiguous per Q8_0 row) instead of 128
// rows x 4 blocks (136 B): measured, the longer row segments alone bring a
// 32-token GEMM from 27.5 to 23.5 us at 14336x4096 (HBM serves short
// scattered segments at a lower rate).  With N / 32 tiles a 14336-row matrix
// needs no K split.
constexpr int SKB = 16;                        // blocks per K stage
constexpr int SK_ROWS = 32;                    // weight rows per tile
template <int BB>
struct SkinnyStage {
    static constexpr int A_BYTES = 32 * SKB * 32;                // 32 tokens x 16 blocks x 32 int8
    static constexpr int UPR = SKB * 2;                          // 16 B units per activation row
    static constexpr int WD = SKB * BB / 4;                      // raw dwords of a weight row per stage
    static constexpr int W_STRIDE = WD | 1;                      // odd: conflict-free B reads
    static constexpr int W_DWORDS = (SK_ROWS - 1) * W_STRIDE + WD + 1;  // +1: the 5th dword read
    static constexpr int W_LOADS = (W_DWORDS + 63) / 64;
    static constexpr int W_PER_WAVE = (W_LOADS + 3) / 4;
    static constexpr int W_BYTES = (W_LOADS * 256 + 15) / 16 * 16;
    static constexpr int S_BYTES = SKB * 32 * 4;
    static constexpr int S_UNITS = S_BYTES / 256;
    static constexpr int S_PER_WAVE = (S_UNITS + 3) / 4;
    static constexpr int BUF = A_BYTES + W_BYTES + S_BYTES;
    static_assert(2 * BUF <= 80 * 1024, "two workgroups per CU");
    static_assert(A_BYTES % 4096 == 0 && S_UNITS % 4 == 0, "loads split evenly over the 4 waves");
    // row r's 16 B units XOR-swizzled by r % 16: the 16 rows a quarter-wave's
    // ds_read_b128 touches fall on distinct 16 B bank groups
    __device__ static int swz(int row) { return row & 15; }
};

// (a __device__ body under a __global__ wrapper: a __global__ template with
// dynamic LDS declared inside left its host launch stub undefined)
// DOTS = true: the bit-exact test mode of the other int8 kernels -- every
// per-block int32 MFMA result goes to dots[(m*N + n)*nb + b] instead.
template <int FMT, bool DOTS>
__device__ __forceinline__ void gemm_i8_skinny_body(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ XQ, const float* __restrict__ XS,
    float* __restrict__ Y, int32_t* __restrict__ dots, uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m,
    uint32_t tiles_n, uint32_t ksplit, uint32_t stages_per_split) {
    constexpr int BB = FMT == kQ8_0 ? 34 : 18;
    static_assert(FMT == kQ8_0 || FMT == kQ4_0, "int8-activation formats only");
    using G = SkinnyStage<BB>;
    extern __shared__ __align__(16) uint8_t lds[];  // 2 * G::BUF bytes
    const uint32_t total_tiles = tiles_m * tiles_n;
    const uint32_t split = blockIdx.x / total_tiles;
    uint32_t tm, tn;
    tile_of(tiles_m, tiles_n, blockIdx.x % total_tiles, tm, tn);
    const uint32_t m0 = tm * 32, n0 = tn * SK_ROWS;
    const uint32_t nb = K >> 5, rb = nb * BB;
    const uint32_t kb_begin = split * stages_per_split * SKB;
    const uint32_t kb_end = min(nb, kb_begin + stages_per_split * SKB);
    float* Yout = Y + (ksplit > 1 ? size_t(split) * M * N : 0);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, lh = lane >> 5;

    constexpr int A_LOADS = G::A_BYTES / 1024 / 4;
    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)(XQ + size_t(m0) * K), 0, -1, kBufferWord3);
    const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)(W + size_t(n0) * rb), 0, -1, kBufferWord3);
    const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(DOTS ? reinterpret_cast<const float*>(XQ) : XS + size_t(m0) * nb), 0, -1, kBufferWord3);
    uint32_t a_off[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        const int unit = (wave * A_LOADS + i) * 64 + lane;
        const int row = unit / G::UPR, col = (unit % G::UPR) ^ G::swz(row);
        a_off[i] = (min(m0 + row, M - 1) - m0) * K + col * 16;
    }
    uint32_t w_off[G::W_PER_WAVE];
#pragma unroll
    for (int i = 0; i < G::W_PER_WAVE; ++i) {
        const uint32_t p = uint32_t((wave + 4 * i) * 64 + lane);
        const uint32_t r = min(p / G::W_STRIDE, uint32_t(SK_ROWS - 1));
        uint32_t d = p - r * G::W_STRIDE;
        if (d >= uint32_t(G::WD)) d = 0;
        w_off[i] = (min(n0 + r, N - 1) - n0) * rb + d * 4;
    }
    uint32_t s_off[G::S_PER_WAVE];
#pragma unroll
    for (int i = 0; i < G::S_PER_WAVE; ++i) {
        const int idx = (wave * G::S_PER_WAVE + i) * 64 + lane;  // = b * 32 + m
        s_off[i] = ((min(m0 + uint32_t(idx % 32), M - 1) - m0) * nb + uint32_t(idx / 32)) * 4;
    }
    auto stage_in = [&](uint32_t kb, int buf) {
        uint8_t* base = lds + buf * G::BUF;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_void*)(base + (wave * A_LOADS + i) * 1024), 16,
                                                     a_off[i], kb * 32, 0, 0);
#pragma unroll
        for (int i = 0; i < G::W_PER_WAVE; ++i)
            if (wave + 4 * i < G::W_LOADS)  // wave-uniform
                __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_void*)(base + G::A_BYTES + (wave + 4 * i) * 256), 4,
                                                         w_off[i], kb * BB, 0, 0);
        if constexpr (!DOTS) {
#pragma unroll
            for (int i = 0; i < G::S_PER_WAVE; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    s_rsrc, (lds_void*)(base + G::A_BYTES + G::W_BYTES + (wave * G::S_PER_WAVE + i) * 256), 4, s_off[i],
                    kb * 4, 0, 0);
        }
    };

    v16f acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    v32f szero;
#pragma unroll
    for (int v = 0; v < 32; ++v) szero[v] = 0.0f;
    const uint32_t wrow = uint32_t(l32) * G::W_STRIDE;  // this lane's weight row (n0 + l32), first LDS dword

    // one block pair (2j, 2j+1) of this wave's quarter: operands, the two
    // int8 MFMAs and one 2-block scale MFMA (block i of it = lane half i =
    // K block 2j + i), then cvt + fma per output element and block
    auto pair = [&](const uint8_t* base, int b0, uint32_t kb) {
        const uint32_t* Bw = reinterpret_cast<const uint32_t*>(base + G::A_BYTES) + wrow;
        v4i a[2], w[2];
        uint32_t t[2][5];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int b = b0 + h;
            const int off = (b * BB + 2 + (FMT == kQ8_0 ? lh * 16 : 0)) >> 2;
#pragma unroll
            for (int i = 0; i < 4 + (h ? 0 : 1); ++i) t[h][i] = Bw[off + i];
            const int col = (b * 2 + lh) ^ G::swz(l32);
            a[h] = *reinterpret_cast<const v4i*>(base + l32 * (SKB * 32) + col * 16);
        }
        const int sb = b0 + lh;  // scales of this lane half's block
        v32f sc = szero;
        if constexpr (!DOTS) {
            const uint32_t dwh = reinterpret_cast<const uint16_t*>(Bw)[sb * (BB / 2)];
            const float dx = reinterpret_cast<const float*>(base + G::A_BYTES + G::W_BYTES)[sb * 32 + l32];
            sc = __builtin_amdgcn_mfma_f32_32x32x1f32(dx, half_bits_to_float(uint16_t(dwh)), szero, 0, 0, 0);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[h][i] = h ? int(t[h][i]) : int(__builtin_amdgcn_alignbyte(t[h][i + 1], t[h][i], 2));
            if constexpr (FMT == kQ4_0) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    w[h][i] = int(((uint32_t(w[h][i]) >> (4 * lh)) & 0x0F0F0F0Fu) + 0x78787878u) ^ int(0x80808080u);
            }
        }
        const v16i c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], w[0], zero, 0, 0, 0);
        const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[1], w[1], zero, 0, 0, 0);
        if constexpr (DOTS) {
            const uint32_t n = n0 + l32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t m = m0 + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (m < M && n < N) {
                    dots[(size_t(m) * N + n) * nb + kb + b0] = c0[v];
                    dots[(size_t(m) * N + n) * nb + kb + b0 + 1] = c1[v];
                }
            }
            return;
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = fmaf(float(c0[v]), sc[v], acc[v]);
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = fmaf(float(c1[v]), sc[16 + v], acc[v]);
    };

    if (kb_begin < kb_end) {
        stage_in(kb_begin, 0);
        int buf = 0;
        for (uint32_t kb = kb_begin; kb < kb_end; kb += SKB, buf ^= 1) {
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct loads of stage kb landed
            __syncthreads();                     // ... and everyone's; the other buffer is free again
            if (kb + SKB < kb_end) stage_in(kb + SKB, buf ^ 1);
            const uint8_t* base = lds + buf * G::BUF;
            pair(base, 4 * wave, kb);
            pair(base, 4 * wave + 2, kb);
        }
    }
    if constexpr (DOTS) return;
    // the four waves' partial tiles, summed in wave order
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds);  // [wave][16][64]
#pragma unroll
    for (int v = 0; v < 16; ++v) red[(wave * 16 + v) * 64 + lane] = acc[v];
    __syncthreads();
    if (wave == 0) {
        const uint32_t n = n0 + l32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            float t = red[v * 64 + lane];
#pragma unroll
            for (int w = 1; w < 4; ++w) t += red[(w * 16 + v) * 64 + lane];
            const uint32_t m = m0 + 8 * (v >> 2) + 4 * lh + (v & 3);
            if (m < M && n < N) Yout[size_t(m) * N + n] = t;
        }
    }
}
template <int FMT, bool DOTS>
__global__ __launch_bounds__(256, 2) void gemm_i8_skinny_kernel(
    const uint8_t* __restrict__ W, const int8_t* __restrict__ XQ, const float* __restrict__ XS,
    float* __restrict__ Y, int32_t* __restrict__ dots, uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m,
    uint32_t tiles_n, uint32_t ksplit, uint32_t stages_per_split) {
    gemm_i8_skinny_body<FMT, DOTS>(W, XQ, XS, Y, dots, M, N, K, tiles_m, tiles_n, ksplit, stages_per_split);
}

// ------------------------------------------------------- fp32 GEMM -------
constexpr int FK = 32;          // K elements per fp32 stage
constexpr int FROW = FK + 4;    // LDS floats per row (pad)

// Split K (ksplit > 1): workgroup blockIdx.x / tiles covers stages
// [split * stages_per_split, ...) of FK elements and writes its partial sums
// to Y + split * M * N; splitk_reduce_kernel adds them in split order.
template <int FMT>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                            float* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
                                                            uint32_t tiles_m, uint32_t tiles_n, uint32_t ksplit,
                                                            uint32_t stages_per_split) {
    __shared__ __align__(16) float As[BM * FROW];
    __shared__ __align__(16) float Bs[BN * FROW];
    const uint32_t total_tiles = tiles_m * tiles_n;
    const uint32_t split = blockIdx.x / total_tiles;
    uint32_t tm, tn;
    tile_of(tiles_m, tiles_n, blockIdx.x % total_tiles, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t k_begin = split * stages_per_split * FK;
    const uint32_t k_end = min(K, k_begin + stages_per_split * FK);
    float* Yout = Y + (ksplit > 1 ? size_t(split) * M * N : 0);
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

    for (uint32_t k0 = k_begin; k0 < k_end; k0 += FK) {
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
                if (m < M && n < N) Yout[size_t(m) * N + n] = acc[i][j][v];
            }
        }
}

// ------------------------------------------- K-quants on the f16 MFMA ---
// The fp32-activation GEMM of the super-block formats (Q6_K, Q4_K, Q5_K)
// with its products on v_mfma_f32_32x32x16_f16 (16x the fp32 MFMA rate) at
// fp32-level accuracy:
//  * each activation row is scaled by a power of two (split_rows_kernel) and
//    carried as f16 hi + lo;
//  * each weight is dequantised as the reference does (Q6_K d*sc*(q-32),
//    Q4_K / Q5_K d*sc*q - dmin*m, one fp32 rounding), scaled by a power of
//    two per weight row (so the row's largest possible value lies below
//    2^15) and carried as h = f16(w) and l = f16(w - h);
//  * a product is Xh*Wh + Xl*Wh + Xh*Wl, accumulated in fp32 per super-block
//    and the super-blocks summed; the row scales come off at the end.
// Against the reference's dequantise-then-fp32 arithmetic the difference is
// rounding order, the 22-bit operand splits and the dropped lo*lo products
// (all below 2^-21 of each operand).
// A workgroup barrier that orders LDS only: unlike __syncthreads it does not
// wait for the wave's outstanding global loads (a prefetch stays in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
#ifndef ZQ_KQ_HKS
#define ZQ_KQ_HKS 32
#endif

// One workgroup per row.
__global__ __launch_bounds__(kThreads) void split_rows_kernel(const float* __restrict__ X, _Float16* __restrict__ xh,
                                                              _Float16* __restrict__ xl, float* __restrict__ inv,
                                                              uint32_t K) {
    __shared__ float red[kThreads / 64];
    const float4* r = reinterpret_cast<const float4*>(X + size_t(blockIdx.x) * K);
    const uint32_t K4 = K / 4;
    float m = 0.0f;
    for (uint32_t i = threadIdx.x; i < K4; i += kThreads) {
        const float4 v = r[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w]);
    const int e = split_exp(m);
    const float f = pow2f(e);
    if (threadIdx.x == 0) inv[blockIdx.x] = pow2f(-e);
    h4_t* oh = reinterpret_cast<h4_t*>(xh + size_t(blockIdx.x) * K);
    h4_t* ol = reinterpret_cast<h4_t*>(xl + size_t(blockIdx.x) * K);
    for (uint32_t i = threadIdx.x; i < K4; i += kThreads) {
        const float4 v = r[i];
        h4_t h, l;
        split_h(v.x * f, h, l, 0);
        split_h(v.y * f, h, l, 1);
        split_h(v.z * f, h, l, 2);
        split_h(v.w * f, h, l, 3);
        oh[i] = h;
        ol[i] = l;
    }
}

// Split K as in gemm_f32_kernel; stages_per_split is a multiple of the
// stages of a super-block.  HKS: K elements per stage (32 or 64).
template <int FMT, int HKS>
__global__ __launch_bounds__(kThreads, 2) void gemm_kq_h_kernel(const uint8_t* __restrict__ W,
                                                                 const _Float16* __restrict__ XH,
                                                                 const _Float16* __restrict__ XL,
                                                                 const float* __restrict__ xinv, float* __restrict__ Y,
                                                                 uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m,
                                                                 uint32_t tiles_n, uint32_t ksplit,
                                                                 uint32_t stages_per_split) {
    static_assert(FMT == kQ6_K || FMT == kQ4_K || FMT == kQ5_K, "super-block formats");
    static_assert(HKS == 32 || HKS == 64, "stage depth");
    constexpr bool Q6 = FMT == kQ6_K;
    constexpr uint32_t BB = FMT == kQ6_K ? 210 : (FMT == kQ5_K ? 176 : 144);
    constexpr int HR = HKS + 8;      // halves per LDS row (pad: 16 B)
    constexpr int EPT = HKS / 2;     // elements per loader thread per stage
    constexpr int XU = EPT / 8;      // 16-byte units of activations per thread, each of hi and lo
    constexpr int QWN = EPT / 4;     // words of codes per thread (one byte per element)
    __shared__ __align__(16) _Float16 Ah[BM * HR];
    __shared__ __align__(16) _Float16 Al[BM * HR];
    __shared__ __align__(16) _Float16 Bh[BN * HR];
    __shared__ __align__(16) _Float16 Bl[BN * HR];
    __shared__ float binv[BN];
    const uint32_t total_tiles = tiles_m * tiles_n;
    const uint32_t split = blockIdx.x / total_tiles;
    uint32_t tm, tn;
    tile_of(tiles_m, tiles_n, blockIdx.x % total_tiles, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t k_begin = split * stages_per_split * HKS;
    const uint32_t k_end = min(K, k_begin + stages_per_split * HKS);
    float* Yout = Y + (ksplit > 1 ? size_t(split) * M * N : 0);
    const size_t rb = row_bytes_dev(FMT, K);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lh = lane >> 5;
    const uint32_t ld_row = tid >> 1, ld_half = tid & 1;  // loader: row, half of the stage
    const _Float16* ah_src = XH + size_t(min(m0 + ld_row, M - 1)) * K + ld_half * EPT;
    const _Float16* al_src = XL + size_t(min(m0 + ld_row, M - 1)) * K + ld_half * EPT;
    const uint8_t* b_src = W + size_t(min(n0 + ld_row, N - 1)) * rb;

    // The loader row's scale 2^e: its dequantised weights over this split's
    // super-blocks, times 2^e, lie below 2^15 in magnitude (a bound from d,
    // dmin and the largest code and scale), so each is h + l in f16 with
    // normal h.  The two threads of a row scan alternate super-blocks.
    float wscale;
    {
        float bound = 0.0f;
        for (uint32_t sb = k_begin / 256 + ld_half; sb < (k_end + 255) / 256; sb += 2) {
            const uint8_t* p = b_src + size_t(sb) * BB;
            if constexpr (Q6) {
                bound = fmaxf(bound, fabsf(half_bits_to_float(*reinterpret_cast<const uint16_t*>(p + 208))) * 4096.0f);
            } else {
                const uint32_t dd = *reinterpret_cast<const uint32_t*>(p);
                const float dmax = FMT == kQ5_K ? 1953.0f : 945.0f;  // 63 x 31, 63 x 15
                bound = fmaxf(bound, fmaf(fabsf(half_bits_to_float(dd & 0xffffu)), dmax,
                                          fabsf(half_bits_to_float(dd >> 16)) * 63.0f));
            }
        }
        bound = fmaxf(bound, __shfl_xor(bound, 1));
        const int e = split_exp(bound);
        wscale = pow2f(e);
        if (ld_half == 0) binv[ld_row] = pow2f(-e);
    }

    // part: the current super-block's products; acc: the sum of the
    // super-blocks' (a two-level sum, so rounding grows with the number of
    // super-blocks rather than of MFMA steps)
    v16f acc[2][2], part[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = part[i][j][v] = 0.0f;

    // Raw stage data of this thread: EPT activations (hi, lo), the words of
    // its EPT weight codes, their group scales and the super-block's d (and
    // dmin).  The next stage's are loaded while the current one is converted
    // and multiplied.  The thread's codes are one 32-element line of the
    // super-block (a Q6_K quarter of a half, a Q4_K / Q5_K group): for HKS =
    // 32 its half, for HKS = 64 line ld_half of the stage's two.
    struct Raw {
        u32x4_attn_t xa[XU], xb[XU];
        uint32_t qw[QWN], hw[Q6 || FMT == kQ5_K ? QWN : 1];
        uint32_t sc;   // Q6_K: the int8 scales of the thread's 16-element groups; else the 12 scale bytes' words
        uint32_t sc1, sc2;
        uint32_t dd;   // d (| dmin << 16)
    };
    auto line_of = [&](uint32_t k0, uint32_t& line, uint32_t& ls) {
        const uint32_t in_sb = k0 & 255u;
        line = (in_sb >> 5) + (HKS == 64 ? ld_half : 0u);
        ls = HKS == 64 ? 0u : ld_half * 16u;
    };
    auto load_raw = [&](uint32_t k0, Raw& r) {
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            r.xa[u] = *reinterpret_cast<const u32x4_attn_t*>(ah_src + k0 + 8 * u);
            r.xb[u] = *reinterpret_cast<const u32x4_attn_t*>(al_src + k0 + 8 * u);
        }
        const uint8_t* p = b_src + size_t(k0 >> 8) * BB;
        uint32_t line, ls;
        line_of(k0, line, ls);
        if constexpr (Q6) {
            const uint32_t h = line >> 2, q4 = line & 3u;
            const uint8_t* lo = p + h * 64 + (q4 & 1u) * 32 + ls;
            const uint8_t* hi = p + 128 + h * 32 + ls;
#pragma unroll
            for (int i = 0; i < QWN; ++i) {
                r.qw[i] = load_u32_a2(lo + 4 * i);
                r.hw[i] = load_u32_a2(hi + 4 * i);
            }
            const uint8_t* s = p + 192 + h * 8 + q4 * 2 + (ls >> 4);
            r.sc = HKS == 64 ? uint32_t(*reinterpret_cast<const uint16_t*>(s)) : uint32_t(*s);
            r.dd = *reinterpret_cast<const uint16_t*>(p + 208);
            r.sc1 = r.sc2 = 0;
        } else {
            const uint32_t* qs =
                reinterpret_cast<const uint32_t*>(p + (FMT == kQ5_K ? 48 : 16) + (line >> 1) * 32 + ls);
#pragma unroll
            for (int i = 0; i < QWN; ++i) r.qw[i] = qs[i];
            if constexpr (FMT == kQ5_K) {
                const uint32_t* qh = reinterpret_cast<const uint32_t*>(p + 16 + ls);
#pragma unroll
                for (int i = 0; i < QWN; ++i) r.hw[i] = qh[i];
            }
            const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
            r.dd = w[0];
            r.sc = w[1];
            r.sc1 = w[2];
            r.sc2 = w[3];
        }
    };
    // one stage from `cur`, prefetching the next into `nxt` (two named
    // records used alternately: no copy between them)
    auto stage = [&](uint32_t k0, Raw& cur, Raw& nxt) {
        // unconditional (the last stage reloads itself), so the wait for the
        // current stage's data counts the prefetch statically
        load_raw(min(k0 + HKS, k_end - HKS), nxt);
        u32x4_attn_t xa[XU], xb[XU];
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            xa[u] = cur.xa[u];
            xb[u] = cur.xb[u];
        }
        h8_t wh[EPT / 8], wl[EPT / 8];
        {
            uint32_t line, ls;
            line_of(k0, line, ls);
            // per 16-element group: value = a * code - b (exact in fp32), times 2^e
            float a[EPT / 16], b[EPT / 16];
            if constexpr (Q6) {
                const float ds = half_bits_to_float(cur.dd & 0xffffu) * wscale;
#pragma unroll
                for (int g = 0; g < EPT / 16; ++g) {
                    a[g] = ds * float(int(int8_t(uint8_t(cur.sc >> (8 * g)))));
                    b[g] = 32.0f * a[g];
                }
            } else {
                // scale / min of group `line` (src/quant.cpp:133-141) from the
                // words of scale bytes 0-3, 4-7, 8-11
                const uint32_t sh = 8 * (line & 3u);
                const uint32_t sa = cur.sc >> sh, sbb = cur.sc1 >> sh, scc = cur.sc2 >> sh;
                const uint32_t sc = line < 4 ? sa & 63u : (scc & 15u) | ((sa >> 2) & 0x30u);
                const uint32_t mn = line < 4 ? sbb & 63u : ((scc >> 4) & 15u) | ((sbb >> 2) & 0x30u);
                const float d = half_bits_to_float(cur.dd & 0xffffu) * wscale;
                const float dm = half_bits_to_float(cur.dd >> 16) * wscale;
#pragma unroll
                for (int g = 0; g < EPT / 16; ++g) {
                    a[g] = d * float(sc);
                    b[g] = dm * float(mn);
                }
            }
#pragma unroll
            for (int i = 0; i < QWN; ++i) {
                const uint32_t qw = cur.qw[i];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    uint32_t q;
                    if constexpr (Q6) {
                        const uint32_t q4 = line & 3u;
                        uint32_t l = (qw >> (8 * k)) & 0xffu;
                        if (q4 >= 2) l >>= 4;
                        const uint32_t hb = ((cur.hw[i] >> (8 * k)) >> (2 * q4)) & 3u;
                        q = (l & 15u) | (hb << 4);
                    } else {
                        q = (qw >> (8 * k + 4 * (line & 1u))) & 15u;
                        if constexpr (FMT == kQ5_K) q |= ((cur.hw[i] >> (8 * k + line)) & 1u) << 4;
                    }
                    const int e = 4 * i + k;
                    const float v = fmaf(a[e / 16], float(q), -b[e / 16]);
                    split_h(v, wh[e / 8], wl[e / 8], e % 8);
                }
            }
        }
        lds_barrier();  // the previous stage's readers are done (the prefetch stays in flight)
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            *reinterpret_cast<u32x4_attn_t*>(Ah + ld_row * HR + ld_half * EPT + 8 * u) = xa[u];
            *reinterpret_cast<u32x4_attn_t*>(Al + ld_row * HR + ld_half * EPT + 8 * u) = xb[u];
            *reinterpret_cast<h8_t*>(Bh + ld_row * HR + ld_half * EPT + 8 * u) = wh[u];
            *reinterpret_cast<h8_t*>(Bl + ld_row * HR + ld_half * EPT + 8 * u) = wl[u];
        }
        lds_barrier();
#pragma unroll
        for (int ks = 0; ks < HKS / 16; ++ks) {
            h8_t ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = (wm * 64 + i * 32 + l32) * HR + ks * 16 + 8 * lh;
                ah[i] = *reinterpret_cast<const h8_t*>(Ah + r);
                al[i] = *reinterpret_cast<const h8_t*>(Al + r);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r = (wn * 64 + j * 32 + l32) * HR + ks * 16 + 8 * lh;
                bh[j] = *reinterpret_cast<const h8_t*>(Bh + r);
                bl[j] = *reinterpret_cast<const h8_t*>(Bl + r);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], part[i][j], 0, 0, 0);
                    part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], part[i][j], 0, 0, 0);
                    part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], part[i][j], 0, 0, 0);
                }
        }
        if (((k0 + HKS) & 255u) == 0) {  // end of a super-block
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        acc[i][j][v] += part[i][j][v];
                        part[i][j][v] = 0.0f;
                    }
        }
    };
    Raw r0, r1;
    if (k_begin < k_end) load_raw(k_begin, r0);
    // a split holds whole super-blocks: an even number of stages
    for (uint32_t k0 = k_begin; k0 < k_end; k0 += 2 * HKS) {
        stage(k0, r0, r1);
        stage(k0 + HKS, r1, r0);
    }
    lds_barrier();  // binv
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t nl = wn * 64 + j * 32 + l32;
            const uint32_t n = n0 + nl;
            const float bs = binv[nl];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (m < M && n < N) Yout[size_t(m) * N + n] = acc[i][j][v] * xinv[m] * bs;
            }
        }
}

}  // namespace

hipError_t launch_quantize_acts(const float* X, int8_t* xq, float* xs, size_t M, size_t K, hipStream_t stream) {
    if (!X || !xq || !xs || !M || !K || K % 32) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(X) & 15u) || (reinterpret_cast<uintptr_t>(xq) & 15u)) return hipErrorInvalidValue;
    const size_t nblocks = M * (K / 32);
    const size_t grid = (nblocks * 8 + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(quantize_acts_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream, X, xq, xs,
                       nblocks);
    return hipGetLastError();
}

// Split factor of the staged-conversion kernel: the grid reaches about two
// workgroups per CU (the LDS budget allows two), keeping at least two K
// stages per split.
static uint32_t choose_ksplit(uint32_t tiles, uint32_t nb) {
    const uint32_t stages = (nb + KB - 1) / KB;
    const uint32_t ks = (512 + tiles - 1) / tiles;
    return std::max(1u, std::min(ks, std::max(1u, stages / 2)));
}

// Split factor of the 4-block direct-load kernels, from a cost model fitted
// to their measured times over M = 32..2048 at 14336x4096 and 4096x14336:
// one K stage of a tile takes `alone` us for a workgroup alone on its CU and
// `shared` us x L when L workgroups share a CU (or queue for it) -- 2.5 and
// 2.0 for the 128-token tile; a split factor ks > 1 adds the partial sums'
// write and read (8 B per output per split at about 6 TB/s) and the reduce
// launch (about 3 us).  Among equal costs the smaller split wins.
struct StageCost {
    double alone, shared;
};
constexpr StageCost kTileCost{2.5, 2.0};
constexpr StageCost kSmallTileCost{1.0, 0.6};
static uint32_t choose_ksplit_model(uint32_t tiles, uint32_t stages, size_t M, size_t N, StageCost c = kTileCost) {
    const double cus = double(device_cu_count());
    uint32_t best = 1;
    double best_t = 1e300;
    for (uint32_t ks = 1; ks <= std::min(stages, 32u); ++ks) {
        const uint32_t spw = (stages + ks - 1) / ks;
        if ((stages + spw - 1) / spw != ks) continue;  // would leave empty splits
        const double L = std::ceil(double(tiles) * ks / cus);
        double t = spw * (L <= 1.0 ? c.alone : c.shared * L);
        if (ks > 1) t += double(ks) * double(M) * double(N) * 8.0 / 6.0e6 + 3.0;
        if (t < best_t) best_t = t, best = ks;
    }
    return best;
}

// Split factor of the skinny kernel: as many splits as keep the whole grid
// resident at once (two workgroups per CU, its LDS budget), at least 2 K
// stages per split.  A grid past one round measured slower than fewer splits.
static uint32_t choose_ksplit_skinny(uint32_t tiles, uint32_t stages) {
    const uint32_t fit = std::max(1u, 2u * uint32_t(device_cu_count()) / tiles);
    return std::max(1u, std::min(fit, std::max(1u, stages / 2)));
}

size_t gemm_i8_partial_bytes(size_t M, size_t N, size_t K) {
    const uint32_t tiles = uint32_t(((M + BM - 1) / BM) * ((N + BN - 1) / BN));
    const uint32_t nb = uint32_t(K / 32);
    // sized for every kernel choice: the direct-load kernels (128- and
    // 32-token tiles) and the staged-conversion kernel
    const uint32_t small_tiles = uint32_t(((M + 31) / 32) * ((N + BN - 1) / BN));
    const uint32_t skinny_tiles = uint32_t(((M + 31) / 32) * ((N + SK_ROWS - 1) / SK_ROWS));
    const uint32_t ks = std::max({choose_ksplit(tiles, nb),
                                  choose_ksplit_model(tiles, (nb + 3) / 4, M, N),
                                  choose_ksplit_model(small_tiles, (nb + 3) / 4, M, N, kSmallTileCost),
                                  choose_ksplit_skinny(skinny_tiles, (nb + SKB - 1) / SKB)});
    return ks > 1 ? size_t(ks) * M * N * sizeof(float) : 0;
}

// Largest M that takes the 32-token tile.  Measured crossover at 14336x4096
// and 4096x14336: the 32-token tile is faster at M = 48 and 64 (36-39 vs
// 41-43 us), slower from M = 96 (46-49 vs 45-46 us), where its token tiles
// re-read each weight panel.
constexpr size_t kSmallMLimit = 64;

// Reduces the K splits of `partial` into Y (fixed order) when ks > 1.
// deferred (optional): receives the split count instead of the reduction
// being enqueued; with more than one split the partial planes are left for
// the caller to sum (in split order, as splitk_reduce_kernel does).
static hipError_t finish_splits(hipError_t e, const float* partial, float* Y, size_t M, size_t N, uint32_t ks,
                                hipStream_t stream, uint32_t* deferred = nullptr) {
    if (deferred) *deferred = ks;
    if (e != hipSuccess || ks <= 1 || deferred) return e;
    const size_t total = M * N;
    const bool vec4 = total % 4 == 0 && !(reinterpret_cast<uintptr_t>(partial) & 15u) &&
                      !(reinterpret_cast<uintptr_t>(Y) & 15u);
    if (vec4)
        hipLaunchKernelGGL(splitk_reduce_kernel<true>, dim3(static_cast<uint32_t>((total / 4 + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, stream, partial, Y, total, ks);
    else
        hipLaunchKernelGGL(splitk_reduce_kernel<false>, dim3(static_cast<uint32_t>((total + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, stream, partial, Y, total, ks);
    return hipGetLastError();
}

// The direct-to-LDS kernels (K % 256 == 0): the 32-token tile for small M,
// else the 128-token tile with 4-block (default) or 8-block stages.
template <int FMT>
static hipError_t launch_direct(const uint8_t* w, const int8_t* xq, const float* xs, float* Y, int32_t* dots,
                                float* partial, size_t M, size_t N, size_t K, hipStream_t stream,
                                uint32_t* deferred = nullptr) {
    constexpr int BB = FMT == kQ8_0 ? 34 : 18;
    constexpr size_t kSmallLds = 2 * QStage<4, 32, 4, BB>::BUF;
    constexpr size_t kLds4 = 2 * QStage<4, BM, QTH / 64, BB>::BUF;
    const uint32_t m = uint32_t(M), n = uint32_t(N), k = uint32_t(K), nb = uint32_t(K / 32);
    const uint32_t tiles_n = static_cast<uint32_t>((N + BN - 1) / BN);
    if (M <= kSmallMLimit && K % (SKB * 32) == 0) {
        const uint32_t stm = uint32_t((M + 31) / 32), stn = uint32_t((N + SK_ROWS - 1) / SK_ROWS), sst = nb / SKB;
        constexpr size_t lds = 2 * SkinnyStage<BB>::BUF;
        if (dots) {
            hipLaunchKernelGGL((gemm_i8_skinny_kernel<FMT, true>), dim3(stm * stn), dim3(256), lds, stream, w, xq, xs, Y,
                               dots, m, n, k, stm, stn, 1u, sst);
            return hipGetLastError();
        }
        uint32_t ks = partial ? choose_ksplit_skinny(stm * stn, sst) : 1u;
        const uint32_t spw = (sst + ks - 1) / ks;
        ks = (sst + spw - 1) / spw;  // no empty splits
        hipLaunchKernelGGL((gemm_i8_skinny_kernel<FMT, false>), dim3(stm * stn * ks), dim3(256), lds, stream, w, xq, xs,
                           ks > 1 ? partial : Y, dots, m, n, k, stm, stn, ks, spw);
        return finish_splits(hipGetLastError(), partial, Y, M, N, ks, stream, deferred);
    }
    if (M <= kSmallMLimit) {
        const uint32_t stm = uint32_t((M + 31) / 32), sst = (nb + 3) / 4;
        if (dots) {
            hipLaunchKernelGGL((gemm_i8_small_kernel<FMT, true>), dim3(stm * tiles_n), dim3(256), kSmallLds, stream, w, xq,
                               xs, Y, dots, m, n, k, stm, tiles_n, 1u, sst);
            return hipGetLastError();
        }
        uint32_t ks = partial ? choose_ksplit_model(stm * tiles_n, sst, M, N, kSmallTileCost) : 1u;
        const uint32_t spw = (sst + ks - 1) / ks;
        ks = (sst + spw - 1) / spw;  // no empty splits
        hipLaunchKernelGGL((gemm_i8_small_kernel<FMT, false>), dim3(stm * tiles_n * ks), dim3(256), kSmallLds, stream, w,
                           xq, xs, ks > 1 ? partial : Y, dots, m, n, k, stm, tiles_n, ks, spw);
        return finish_splits(hipGetLastError(), partial, Y, M, N, ks, stream, deferred);
    }
    const uint32_t tiles_m = static_cast<uint32_t>((M + BM - 1) / BM);
    const uint32_t st = (nb + 3) / 4;
    if (dots) {
        hipLaunchKernelGGL((gemm_i8_direct4_kernel<FMT, true>), dim3(tiles_m * tiles_n), dim3(QTH), kLds4, stream, w, xq,
                           xs, Y, dots, m, n, k, tiles_m, tiles_n, 1u, st);
        return hipGetLastError();
    }
    uint32_t ks = partial ? choose_ksplit_model(tiles_m * tiles_n, st, M, N) : 1u;
    const uint32_t spw = (st + ks - 1) / ks;
    ks = (st + spw - 1) / spw;  // no empty splits
    float* out = ks > 1 ? partial : Y;
    hipLaunchKernelGGL((gemm_i8_direct4_kernel<FMT, false>), dim3(tiles_m * tiles_n * ks), dim3(QTH), kLds4, stream, w,
                       xq, xs, out, dots, m, n, k, tiles_m, tiles_n, ks, spw);
    return finish_splits(hipGetLastError(), partial, Y, M, N, ks, stream, deferred);
}

static hipError_t launch_i8_common(int fmt, const uint8_t* w, const int8_t* xq, const float* xs, float* Y,
                                   int32_t* dots, float* partial, size_t M, size_t N, size_t K, hipStream_t stream,
                                   uint32_t* deferred = nullptr) {
    if (!w || !xq || !M || !N || !K || K % 64 || M > (1u << 24) || N > (1u << 24) || K > (1u << 24))
        return hipErrorInvalidValue;
    if (fmt != kQ8_0 && fmt != kQ4_0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(w) & 3u) || (reinterpret_cast<uintptr_t>(xq) & 15u)) return hipErrorInvalidValue;
    if (!dots && (!xs || !Y)) return hipErrorInvalidValue;
    // The direct-load kernels address a tile with 32-bit offsets from its
    // first row: 129 activation rows and 129 weight rows must stay below 2 GiB.
    const size_t rb = row_bytes(fmt, K);
    const bool offsets_fit = size_t(BM + 1) * K < (size_t(1) << 31) && size_t(BN + 1) * rb < (size_t(1) << 31);
    if (K % 256 == 0 && offsets_fit)
        return fmt == kQ8_0 ? launch_direct<kQ8_0>(w, xq, xs, Y, dots, partial, M, N, K, stream, deferred)
                            : launch_direct<kQ4_0>(w, xq, xs, Y, dots, partial, M, N, K, stream, deferred);

    // Staged-conversion kernel (any K % 64 == 0).
    const uint32_t tiles_m = static_cast<uint32_t>((M + BM - 1) / BM);
    const uint32_t tiles_n = static_cast<uint32_t>((N + BN - 1) / BN);
    const uint32_t nb = uint32_t(K / 32);
    const uint32_t stages = (nb + KB - 1) / KB;
    const uint32_t m = uint32_t(M), n = uint32_t(N), k = uint32_t(K);
    if (dots) {
        const dim3 grid(tiles_m * tiles_n);
        if (fmt == kQ8_0)
            hipLaunchKernelGGL((gemm_i8_kernel<kQ8_0, true>), grid, dim3(kThreads), 0, stream, w, xq, xs, Y, dots, m, n,
                               k, tiles_m, tiles_n, 1u, stages);
        else
            hipLaunchKernelGGL((gemm_i8_kernel<kQ4_0, true>), grid, dim3(kThreads), 0, stream, w, xq, xs, Y, dots, m, n,
                               k, tiles_m, tiles_n, 1u, stages);
        return hipGetLastError();
    }
    uint32_t ks = partial ? choose_ksplit(tiles_m * tiles_n, nb) : 1u;
    const uint32_t spw = (stages + ks - 1) / ks;
    ks = (stages + spw - 1) / spw;  // no empty splits
    float* out = ks > 1 ? partial : Y;
    const dim3 grid(tiles_m * tiles_n * ks);
    if (fmt == kQ8_0)
        hipLaunchKernelGGL((gemm_i8_kernel<kQ8_0, false>), grid, dim3(kThreads), 0, stream, w, xq, xs, out, dots, m, n,
                           k, tiles_m, tiles_n, ks, spw);
    else
        hipLaunchKernelGGL((gemm_i8_kernel<kQ4_0, false>), grid, dim3(kThreads), 0, stream, w, xq, xs, out, dots, m, n,
                           k, tiles_m, tiles_n, ks, spw);
    return finish_splits(hipGetLastError(), partial, Y, M, N, ks, stream, deferred);
}

hipError_t launch_splitk_reduce(const float* partial, float* Y, size_t M, size_t N, uint32_t splits, hipStream_t stream) {
    if (!partial || !Y || !splits) return hipErrorInvalidValue;
    return finish_splits(hipSuccess, partial, Y, M, N, splits, stream);
}

hipError_t launch_gemm_i8(int fmt, const uint8_t* w, const int8_t* xq, const float* xs, float* Y, float* partial,
                          size_t M, size_t N, size_t K, hipStream_t stream, uint32_t* splits) {
    return launch_i8_common(fmt, w, xq, xs, Y, nullptr, partial, M, N, K, stream, splits);
}

hipError_t launch_block_dots(int fmt, const uint8_t* w, const int8_t* xq, int32_t* out, size_t M, size_t N, size_t K,
                             hipStream_t stream) {
    if (!out) return hipErrorInvalidValue;
    return launch_i8_common(fmt, w, xq, nullptr, nullptr, out, nullptr, M, N, K, stream);
}

// Split factor of the fp32-activation GEMM: enough workgroups for two per CU,
// at least 16 K stages per split.
static uint32_t choose_ksplit_f32(uint32_t tiles, uint32_t stages) {
    const uint32_t want = (2u * uint32_t(device_cu_count()) + tiles - 1) / tiles;
    return std::max(1u, std::min(want, std::max(1u, stages / 16)));
}

size_t gemm_f32_partial_bytes(size_t M, size_t N, size_t K) {
    const uint32_t tiles = uint32_t(((M + BM - 1) / BM) * ((N + BN - 1) / BN));
    const uint32_t ks = choose_ksplit_f32(tiles, uint32_t((K + FK - 1) / FK));
    return ks > 1 ? size_t(ks) * M * N * sizeof(float) : 0;
}

// The super-block formats on the f16 MFMA: the split activations (hi and lo
// halves, [M][K] each) and the row scales come first in the workspace, the
// section rounded up to 256 bytes.
static bool kq_f16(int fmt, size_t K) { return (fmt == kQ6_K || fmt == kQ4_K || fmt == kQ5_K) && K % 256 == 0; }
static size_t a256(size_t v) { return (v + 255) / 256 * 256; }
static size_t kq_split_bytes(int, size_t M, size_t K) { return a256(M * K * 2 * sizeof(_Float16) + M * sizeof(float)); }

size_t gemm_f32_workspace_bytes(int fmt, size_t M, size_t N, size_t K) {
    return (kq_f16(fmt, K) ? kq_split_bytes(fmt, M, K) : 0) + gemm_f32_partial_bytes(M, N, K);
}

hipError_t launch_gemm_f32(int fmt, const uint8_t* w, const float* X, float* Y, void* ws, size_t ws_bytes, size_t M,
                           size_t N, size_t K, hipStream_t stream, uint32_t* launches) {
    if (!w || !X || !Y || !M || !N || !row_bytes(fmt, K) || M > (1u << 24) || N > (1u << 24) || K > (1u << 24))
        return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(w) & 1u) || (reinterpret_cast<uintptr_t>(X) & 15u)) return hipErrorInvalidValue;
    if ((fmt == kQ4_K || fmt == kQ5_K) && (reinterpret_cast<uintptr_t>(w) & 3u)) return hipErrorInvalidValue;
    const uint32_t tiles_m = static_cast<uint32_t>((M + BM - 1) / BM);
    const uint32_t tiles_n = static_cast<uint32_t>((N + BN - 1) / BN);
    const uint32_t stages = uint32_t((K + FK - 1) / FK);
    const uint32_t m = uint32_t(M), n = uint32_t(N), k = uint32_t(K);
    const size_t pbytes = gemm_f32_partial_bytes(M, N, K);
    if (kq_f16(fmt, K) && ws && ws_bytes >= kq_split_bytes(fmt, M, K) && !(reinterpret_cast<uintptr_t>(ws) & 255u)) {
        uint8_t* b = static_cast<uint8_t*>(ws);
        _Float16* xh = reinterpret_cast<_Float16*>(b);
        _Float16* xl = xh + M * K;
        float* inv = reinterpret_cast<float*>(xl + M * K);
        const size_t sb = kq_split_bytes(fmt, M, K);
        float* partial = ws_bytes >= sb + pbytes && pbytes ? reinterpret_cast<float*>(b + sb) : nullptr;
        uint32_t ks = partial ? choose_ksplit_f32(tiles_m * tiles_n, stages) : 1u;
        constexpr uint32_t HKS = ZQ_KQ_HKS, SPB = 256 / HKS;  // stages per super-block
        const uint32_t hstages = k / HKS;
        const uint32_t spw = ((hstages + ks - 1) / ks + SPB - 1) / SPB * SPB;  // whole super-blocks per split
        ks = (hstages + spw - 1) / spw;
        float* out = ks > 1 ? partial : Y;
        const dim3 grid(tiles_m * tiles_n * ks);
        hipLaunchKernelGGL(split_rows_kernel, dim3(m), dim3(kThreads), 0, stream, X, xh, xl, inv, k);
        if (fmt == kQ6_K)
            hipLaunchKernelGGL((gemm_kq_h_kernel<kQ6_K, HKS>), grid, dim3(kThreads), 0, stream, w, xh, xl, inv, out, m, n,
                               k, tiles_m, tiles_n, ks, spw);
        else if (fmt == kQ4_K)
            hipLaunchKernelGGL((gemm_kq_h_kernel<kQ4_K, HKS>), grid, dim3(kThreads), 0, stream, w, xh, xl, inv, out, m, n,
                               k, tiles_m, tiles_n, ks, spw);
        else
            hipLaunchKernelGGL((gemm_kq_h_kernel<kQ5_K, HKS>), grid, dim3(kThreads), 0, stream, w, xh, xl, inv, out, m, n,
                               k, tiles_m, tiles_n, ks, spw);
        if (launches) *launches = ks > 1 ? 3 : 2;
        return finish_splits(hipGetLastError(), partial, Y, M, N, ks, stream);
    }
    float* partial = ws && pbytes && ws_bytes >= pbytes ? static_cast<float*>(ws) : nullptr;
    uint32_t ks = partial ? choose_ksplit_f32(tiles_m * tiles_n, stages) : 1u;
    const uint32_t spw = (stages + ks - 1) / ks;
    ks = (stages + spw - 1) / spw;  // no empty splits
    float* out = ks > 1 ? partial : Y;
    const dim3 grid(tiles_m * tiles_n * ks);
    switch (fmt) {
    case kQ8_0:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ8_0>, grid, dim3(kThreads), 0, stream, w, X, out, m, n, k, tiles_m, tiles_n, ks, spw);
        break;
    case kQ4_0:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ4_0>, grid, dim3(kThreads), 0, stream, w, X, out, m, n, k, tiles_m, tiles_n, ks, spw);
        break;
    case kQ6_K:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ6_K>, grid, dim3(kThreads), 0, stream, w, X, out, m, n, k, tiles_m, tiles_n, ks, spw);
        break;
    case kQ4_K:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ4_K>, grid, dim3(kThreads), 0, stream, w, X, out, m, n, k, tiles_m, tiles_n, ks, spw);
        break;
    case kQ5_K:
        hipLaunchKernelGGL(gemm_f32_kernel<kQ5_K>, grid, dim3(kThreads), 0, stream, w, X, out, m, n, k, tiles_m, tiles_n, ks, spw);
        break;
    default: return hipErrorInvalidValue;
    }
    if (launches) *launches = ks > 1 ? 2 : 1;
    return finish_splits(hipGetLastError(), partial, Y, M, N, ks, stream);
}

}  // namespace zq
