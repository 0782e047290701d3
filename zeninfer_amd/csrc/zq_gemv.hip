// zq_gemv.hip -- decode GEMV (batch 1, fp32 activations) over native GGML
// blocks for gfx950.
//
// Weights stay in their GGUF block layout in HBM: Q8_0 = 34-byte blocks
// (fp16 d, 32 x int8), Q4_0 = 18-byte blocks (fp16 d, 16 bytes of nibbles),
// Q6_K = 210-byte super-blocks (ql[128] | qh[64] | int8 sc[16] | fp16 d).
//
// Q8_0 / Q4_0 (cols % 64 == 0): one lane owns a PAIR of consecutive blocks.
// A pair is 68 B (Q8_0) / 36 B (Q4_0), a multiple of 4 bytes, so every pair
// starts dword-aligned even though single blocks alternate between 0 and 2
// mod 4.  Inside a pair every field sits at a fixed byte position, so the
// lane decodes with static byte selects (v_cvt_f32_i32 with SDWA sext) and
// one v_alignbyte per misaligned dword; no repack on upload.  The 64 lanes of
// a wave cover 64 consecutive pairs = 4352 contiguous bytes of a Q8_0 row
// (exactly one row at K=4096), so a wave's loads touch whole cache lines.
//
// The activation vector is staged once per workgroup in LDS with a 4-float
// pad after every 64 floats: lane L reads its pair's 64 floats with
// ds_read_b128 at a 68-dword stride, which spreads 8 consecutive lanes over
// all 32 banks.  Each wave processes R rows at a time so the x values read
// from LDS are reused R times from registers, and R rows x 68 B per lane are
// in flight per iteration.  The per-lane partial sums are reduced across the
// wave with a butterfly (ds_swizzle/DPP), then one lane stores R outputs.
//
// Q4_K / Q5_K (144 / 176-byte super-blocks: fp16 d, fp16 dmin, 12 bytes of
// packed 6-bit scales/mins, [Q5_K: 32 bytes of fifth bits], 128 bytes of
// nibbles): one lane owns a 16-byte unit of nibbles, i.e. 16 elements of an
// even group and the 16 matching elements of the next odd group.  Its 32 x
// values and their two sums stay in VGPRs, so per row the lane needs only
// sum(q*x) per group: w*x summed = (d*sc)*sum(q*x) - (dmin*m)*sum(x).
//
// Q6_K, fallback kernel: one lane owns a 16-element unit (half h, l-quad l0)
// of a super-block: 3 data dwords (ql low/high streams and qh), 4 int8
// sub-scales and d.  The four 4-element groups are decoded byte-parallel:
// q = lo4 | hi2 << 4, then ((q ^ 0x20) << 2) is 4*(q-32) as a signed byte.
// The streaming Q6_K kernel (cols % 2048 == 0) instead gives each lane 16
// consecutive elements of one quarter (one sub-block scale), builds the
// 6-bit codes four per dword and converts each with one v_cvt_f32_ubyteN,
// the code offset applied once per unit through a precomputed sum of x; see
// gemv_q6k_stream_kernel.
#include "zq_device.hpp"
#include "zq_internal.hpp"
#include "zq_pairs.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>

namespace zq {

size_t row_bytes(int fmt, size_t cols) {
    switch (fmt) {
    case kQ4_0: return (cols && cols % 32 == 0) ? cols / 32 * 18 : 0;
    case kQ8_0: return (cols && cols % 32 == 0) ? cols / 32 * 34 : 0;
    case kQ4_K: return (cols && cols % 256 == 0) ? cols / 256 * 144 : 0;
    case kQ5_K: return (cols && cols % 256 == 0) ? cols / 256 * 176 : 0;
    case kQ6_K: return (cols && cols % 256 == 0) ? cols / 256 * 210 : 0;
    default: return 0;
    }
}

namespace {

struct TaskTable {
    GemvTask t[kMaxTasks];
    uint32_t group_start[kMaxTasks + 1];  // prefix sums of per-task row groups
    int count;
};

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

// Locate the task owning row-group g (count <= 8, linear scan).
__device__ __forceinline__ int find_task(const TaskTable& tt, uint32_t g) {
    int i = 0;
#pragma unroll
    for (int k = 1; k < kMaxTasks; ++k)
        if (k < tt.count && g >= tt.group_start[k]) i = k;
    return i;
}

// Stage x (cols floats) into LDS.  Padded layout when PAD: chunk c of 64
// floats at c*68.
template <bool PAD>
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, uint32_t cols) {
    for (uint32_t i = threadIdx.x; i < cols; i += kThreads) {
        const uint32_t dst = PAD ? (i >> 6) * kPadStride + (i & 63u) : i;
        xs[dst] = x[i];
    }
    __syncthreads();
}

// Pair-lane kernel for Q8_0 (DW=17) and Q4_0 (DW=9).
template <int FMT, int R>
__global__ __launch_bounds__(kThreads) void gemv_pairs_kernel(TaskTable tt, const float* __restrict__ x,
                                                              uint32_t cols, uint32_t total_groups) {
    constexpr int DW = FMT == kQ8_0 ? 17 : 9;
    extern __shared__ float xs[];
    stage_x<true>(xs, x, cols);
    const uint32_t pairs = cols >> 6;
    const uint32_t rb = pairs * DW * 4;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    for (uint32_t g = blockIdx.x * kWavesPerBlock + wave; g < total_groups; g += gridDim.x * kWavesPerBlock) {
        const int ti = find_task(tt, g);
        const GemvTask task = tt.t[ti];
        const uint32_t r0 = (g - tt.group_start[ti]) * R;
        float acc[R];
        const uint8_t* rowp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
            const uint32_t row = min(r0 + r, task.rows - 1);
            rowp[r] = task.w + (size_t)row * rb;
        }
        for (uint32_t p = lane; p < pairs; p += kWave) {
            uint32_t q[R][DW];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t* src = reinterpret_cast<const uint32_t*>(rowp[r] + (size_t)p * DW * 4);
#pragma unroll
                for (int i = 0; i < DW; ++i) q[r][i] = use_nt() ? __builtin_nontemporal_load(src + i) : src[i];
            }
            float xv[64];
            const float4* xp = reinterpret_cast<const float4*>(xs + p * kPadStride);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float4 v = xp[i];
                xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if constexpr (FMT == kQ8_0) acc[r] += q8_pair_dot(q[r], xv);
                else acc[r] += q4_pair_dot(q[r], xv);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[r]);
            if (lane == r && r0 + r < task.rows) task.y[r0 + r] = v;
        }
    }
}

// x-in-registers pair kernel (cols % 64 == 0, up to 256 pairs = 16384 cols).
// A row is split into S column slices of W = ceil(pairs/S) <= 64 pairs; a
// "team" of S waves covers one row, wave s owning slice s, and lane L of it
// owning pair s*W + L for every row the kernel visits.  So each lane loads
// its 64 x values ONCE (from LDS when S == 1, where the workgroup's four
// waves share one staged copy; straight from global memory otherwise) and
// keeps them in VGPRs, and the loop body only streams weights: R rows x DW
// dwords per lane per iteration, software-pipelined one iteration ahead.
// The workgroup walks row blocks of RB = (4/S)*R rows with a grid-stride
// loop whose trip count is uniform across the workgroup, so the S > 1
// cross-wave reduction can use __syncthreads (double-buffered by parity).
template <int FMT, int R, int S>
__global__ __launch_bounds__(kThreads) void gemv_xreg_kernel(TaskTable tt, const float* __restrict__ x,
                                                             uint32_t cols, uint32_t total_blocks) {
    constexpr int DW = FMT == kQ8_0 ? 17 : 9;
    constexpr int TEAMS = kWavesPerBlock / S;
    extern __shared__ float xs[];
    __shared__ float red[2][kWavesPerBlock][R];
    const uint32_t pairs = cols >> 6;
    const uint32_t W = (pairs + S - 1) / S;
    const uint32_t rb = pairs * DW * 4;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int team = wave / S, slice = wave % S;
    const uint32_t p = slice * W + lane;
    const bool active = uint32_t(lane) < W && p < pairs;

    // row block -> (task, first row of this team)
    auto locate = [&](uint32_t blk, const uint8_t*(&rowp)[R], uint32_t& row0, int& ti) {
        ti = find_task(tt, blk);
        const GemvTask& t = tt.t[ti];
        row0 = (blk - tt.group_start[ti]) * (TEAMS * R) + team * R;
#pragma unroll
        for (int r = 0; r < R; ++r) rowp[r] = t.w + (size_t)min(row0 + r, t.rows - 1) * rb + (size_t)p * DW * 4;
    };
    auto load = [&](const uint8_t*(&rowp)[R], uint32_t (&q)[R][DW]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(rowp[r]);
#pragma unroll
            for (int i = 0; i < DW; ++i) q[r][i] = active ? (use_nt() ? __builtin_nontemporal_load(src + i) : src[i]) : 0u;
        }
    };

    uint32_t blk = blockIdx.x;
    uint32_t q[R][DW];
    const uint8_t* rowp[R];
    uint32_t row0 = 0;
    int ti = 0;
    if (blk < total_blocks) {
        locate(blk, rowp, row0, ti);
        load(rowp, q);  // weight loads go out before x is fetched
    }
    float xv[64];
    if constexpr (S == 1) {
        for (uint32_t i = threadIdx.x; i < (cols >> 2); i += kThreads) {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            *reinterpret_cast<float4*>(xs + (i >> 4) * kPadStride + ((i & 15u) << 2)) = v;
        }
        __syncthreads();
        const float4* xp = reinterpret_cast<const float4*>(xs + (active ? p : 0) * kPadStride);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = xp[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
    } else {
        const float4* xp = reinterpret_cast<const float4*>(x + (size_t)(active ? p : 0) * 64);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = xp[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
    }
    int parity = 0;
    while (blk < total_blocks) {
        const uint32_t nblk = blk + gridDim.x;
        uint32_t qn[R][DW];
        const uint8_t* rowpn[R];
        uint32_t row0n = 0;
        int tin = 0;
        if (nblk < total_blocks) {
            locate(nblk, rowpn, row0n, tin);
            load(rowpn, qn);
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (FMT == kQ8_0) acc[r] = q8_pair_dot(q[r], xv);
            else acc[r] = q4_pair_dot(q[r], xv);
            acc[r] = wave_sum(acc[r]);
        }
        const GemvTask& t = tt.t[ti];
        if constexpr (S == 1) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (lane == r && row0 + r < t.rows) t.y[row0 + r] = acc[r];
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) red[parity][wave][r] = acc[r];
            }
            __syncthreads();
            if (slice == 0 && lane < R) {
                float v = 0.0f;
#pragma unroll
                for (int s2 = 0; s2 < S; ++s2) v += red[parity][team * S + s2][lane];
                if (row0 + lane < t.rows) t.y[row0 + lane] = v;
            }
            parity ^= 1;
        }
        blk = nblk;
        if (blk < total_blocks) {
            row0 = row0n;
            ti = tin;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int i = 0; i < DW; ++i) q[r][i] = qn[r][i];
        }
    }
}

// Coalesced streaming pair kernel: the x-in-registers organisation of
// gemv_xreg_kernel, but weights are fetched with lane-contiguous dwordx4
// loads (each load instruction covers 1 KiB of consecutive bytes) into a
// per-wave LDS buffer, and every lane then reads its own pair back with DW
// ds_read_b32 at a DW-dword stride (17 or 9: odd, so the 64 lanes hit 64
// distinct banks).  Requires the slice-row byte ranges to be 16 B aligned:
// cols % 256 == 0 and a 16 B aligned weight base.  The next row block's
// loads are issued before the current block is decoded.
// EP = 1 (S = 1, R = 1, NW = 16, two tasks of equal rows: gate, up): a row
// block is 8 rows of both tasks, teams 0-7 the gate rows and 8-15 the same
// up rows, and the block stores f = silu(gate.x) * (up.x) into the first
// task's y (the expression of silu_mul_kernel), so the down projection reads
// f as a plain vector.
template <int FMT, int R, int S, int NW, int D, int XK, int EP = 0>
__global__ __launch_bounds__(NW * 64) void gemv_stream_kernel(TaskTable tt, const float* __restrict__ x,
                                                               uint32_t cols, uint32_t total_blocks, XPrologue pro) {
    static_assert(EP == 0 || (S == 1 && R == 1 && NW == 16), "the SiLU pair epilogue takes one row per wave");
    constexpr int DW = FMT == kQ8_0 ? 17 : 9;
    constexpr int NT = NW * 64;
    constexpr int TEAMS = NW / S;
    constexpr int UMAX = 64 * DW / 4;        // 16 B units of a full 64-pair slice-row
    constexpr int NU = (UMAX + 63) / 64;     // dwordx4 loads per lane per row
    constexpr int WBUF = 64 * DW;            // dwords per slice-row buffer
    constexpr bool XLDS = S == 1 || NW > S;  // teams share the x slices: stage x once per workgroup
    constexpr int XPT = XLDS ? (S * 1024 + NT - 1) / NT : 16;  // float4 of x per thread (cols <= S * 4096)
    extern __shared__ uint32_t lds[];        // [waves][R][WBUF]; the padded x is staged over it first
    __shared__ float red[2][NW][R];
    const uint32_t pairs = cols >> 6;
    const uint32_t W = min(64u, (((pairs + S - 1) / S) + 3u) & ~3u);
    const uint32_t rb = pairs * DW * 4;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = wave / S, slice = wave % S;
    const uint32_t p0 = slice * W;
    const uint32_t np = p0 < pairs ? min(W, pairs - p0) : 0u;   // pairs in this wave's slice (multiple of 4)
    const uint32_t nunits = np * DW / 4;
    const bool active = uint32_t(lane) < np;
    const uint32_t p = p0 + lane;
    uint32_t* buf = lds + wave * (R * WBUF);
    float* xs = reinterpret_cast<float*>(lds);

    auto locate = [&](uint32_t blk, const uint8_t*(&rowp)[R], uint32_t& row0, int& ti) {
        if constexpr (EP == 1) {
            ti = team >> 3;
            row0 = blk * 8 + (team & 7);
        } else {
            ti = find_task(tt, blk);
            row0 = (blk - tt.group_start[ti]) * (TEAMS * R) + team * R;
        }
        const GemvTask& t = tt.t[ti];
#pragma unroll
        for (int r = 0; r < R; ++r)
            rowp[r] = t.w + (size_t)min(row0 + r, t.rows - 1) * rb + (size_t)(np ? p0 : 0) * DW * 4;
    };
    // units past the slice read 0 without a memory request
    auto load = [&](const uint8_t*(&rowp)[R], uint4 (&u)[R][NU]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const __amdgpu_buffer_rsrc_t rs = span_rsrc(rowp[r], nunits * 16);
#pragma unroll
            for (int i = 0; i < NU; ++i) u[r][i] = span_load16(rs, uint32_t(lane + 64 * i) * 16);
        }
    };
    auto stash = [&](const uint4 (&u)[R][NU]) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < NU; ++i) {
                const uint32_t unit = lane + 64 * i;
                if (unit < uint32_t(UMAX)) reinterpret_cast<uint4*>(buf + r * WBUF)[unit] = u[r][i];
            }
    };

    // x (or its producer's operands) is loaded first: loads retire in issue
    // order, so x must not queue behind the weight blocks.
    static_assert(XK == kXPlain || XLDS, "x prologues run on the LDS-staged path");
    const uint32_t nx4 = cols >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(XK == kXPlain ? x : pro.a);
    float4 xr[XPT], xb[XK == kXPlain ? 1 : XPT], xw[XK == kAddNorm ? XPT : 1];
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
        if constexpr (XLDS) {
            const uint32_t idx = min(threadIdx.x + uint32_t(k) * NT, nx4 - 1);
            xr[k] = x4[idx];
            if constexpr (XK == kSiluMul) xb[k] = reinterpret_cast<const float4*>(pro.b)[idx];
            if constexpr (XK == kAddNorm) {
                xb[k] = pro.b ? reinterpret_cast<const float4*>(pro.b)[idx] : make_float4(0, 0, 0, 0);
                xw[k] = reinterpret_cast<const float4*>(pro.w)[idx];
            }
        } else {
            xr[k] = x4[(active ? p : 0u) * 16 + k];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the x loads ahead of the weight loads
    // D row blocks in flight
    uint32_t blk = blockIdx.x;
    uint4 u[D][R][NU];
    uint32_t row0s[D];
    int tis[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {  // branch-free, so the x loads stay first: a slot past the end re-reads the last block
        const uint32_t b = min(blk + uint32_t(d) * gridDim.x, total_blocks - 1);
        const uint8_t* rowp[R];
        locate(b, rowp, row0s[d], tis[d]);
        load(rowp, u[d]);
    }
    float xv[64];
    if constexpr (XK == kSiluMul) {
        // g / (1 + e^-g) * u, the expression of silu_mul_kernel
        auto f = [](float g, float u) { return g / (1.0f + expf(-g)) * u; };
#pragma unroll
        for (int k = 0; k < XPT; ++k)
            xr[k] = make_float4(f(xr[k].x, xb[k].x), f(xr[k].y, xb[k].y), f(xr[k].z, xb[k].z), f(xr[k].w, xb[k].w));
    }
    if constexpr (XK == kAddNorm) {
        // v = a + b; sum of squares in double; inv = 1/sqrtf(float(ss/n) + eps);
        // x = v * inv * w -- the arithmetic of rmsnorm_kernel
        __shared__ double xred[NW];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            xr[k] = make_float4(xr[k].x + xb[k].x, xr[k].y + xb[k].y, xr[k].z + xb[k].z, xr[k].w + xb[k].w);
            if (threadIdx.x + uint32_t(k) * NT < nx4) {
                ss += double(xr[k].x) * double(xr[k].x);
                ss += double(xr[k].y) * double(xr[k].y);
                ss += double(xr[k].z) * double(xr[k].z);
                ss += double(xr[k].w) * double(xr[k].w);
                if (pro.r_out && blockIdx.x == 0)
                    reinterpret_cast<float4*>(pro.r_out)[threadIdx.x + uint32_t(k) * NT] = xr[k];
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) xred[wave] = ss;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int i = 0; i < NW; ++i) tot += xred[i];
        const float inv = 1.0f / sqrtf(float(tot / double(cols)) + pro.eps);
#pragma unroll
        for (int k = 0; k < XPT; ++k)
            xr[k] = make_float4(xr[k].x * inv * xw[k].x, xr[k].y * inv * xw[k].y, xr[k].z * inv * xw[k].z,
                                xr[k].w * inv * xw[k].w);
    }
    if constexpr (XLDS) {
#pragma unroll
        for (int k = 0; k < XPT; ++k) {  // out-of-range threads rewrite the last float4 with the same value
            const uint32_t i = min(threadIdx.x + uint32_t(k) * NT, nx4 - 1);
            *reinterpret_cast<float4*>(xs + (i >> 4) * kPadStride + ((i & 15u) << 2)) = xr[k];
        }
        __syncthreads();
        const float4* xp = reinterpret_cast<const float4*>(xs + (active ? p : 0) * kPadStride);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 v = xp[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
        __syncthreads();  // the x staging area is the weight buffers
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            xv[4 * i] = xr[i].x; xv[4 * i + 1] = xr[i].y; xv[4 * i + 2] = xr[i].z; xv[4 * i + 3] = xr[i].w;
        }
    }
    float sx0 = 0.0f, sx1 = 0.0f;  // Q4_0: sum of x over the lane's two blocks
    if constexpr (FMT == kQ4_0) {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            sx0 += xv[i];
            sx1 += xv[32 + i];
        }
    }
    int parity = 0;
    // one row block from ring slot d (a compile-time index, so the slot's
    // registers are never addressed dynamically)
    auto step = [&](auto dc) {
        constexpr int d = decltype(dc)::value;
        {
            {
                stash(u[d]);
                const uint32_t row0 = row0s[d];
                const int ti = tis[d];
                const uint32_t nblk = blk + uint32_t(D) * gridDim.x;
                if (nblk < total_blocks) {
                    const uint8_t* rowp[R];
                    locate(nblk, rowp, row0s[d], tis[d]);
                    load(rowp, u[d]);
                }
                float acc[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    uint32_t q[DW];
#pragma unroll
                    for (int j = 0; j < DW; ++j) q[j] = active ? buf[r * WBUF + DW * lane + j] : 0u;
                    if constexpr (FMT == kQ8_0) acc[r] = q8_pair_dot(q, xv);
                    else acc[r] = q4_pair_dot_mix(q, xv, sx0, sx1);
                    acc[r] = wave_sum(acc[r]);
                }
                const GemvTask& t = tt.t[ti];
                if constexpr (EP == 1) {
                    // gate (teams 0-7) and up (teams 8-15) of the same 8 rows
                    if (lane == 0) red[parity][wave][0] = acc[0];
                    __syncthreads();
                    if (wave < 8 && lane == 0 && row0 < t.rows) {
                        const float g = red[parity][wave][0], u = red[parity][wave + 8][0];
                        t.y[row0] = g / (1.0f + expf(-g)) * u;
                    }
                    parity ^= 1;
                } else if constexpr (S == 1) {
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (lane == r && row0 + r < t.rows) t.y[row0 + r] = acc[r];
                } else {
                    if (lane == 0) {
#pragma unroll
                        for (int r = 0; r < R; ++r) red[parity][wave][r] = acc[r];
                    }
                    __syncthreads();
                    if (slice == 0 && lane < R) {
                        float v = 0.0f;
#pragma unroll
                        for (int s2 = 0; s2 < S; ++s2) v += red[parity][team * S + s2][lane];
                        if (row0 + lane < t.rows) t.y[row0 + lane] = v;
                    }
                    parity ^= 1;
                }
                blk += gridDim.x;
            }
        }
    };
    while (blk < total_blocks) {
        step(std::integral_constant<int, 0>{});
        if constexpr (D > 1) if (blk < total_blocks) step(std::integral_constant<int, 1>{});
        if constexpr (D > 2) if (blk < total_blocks) step(std::integral_constant<int, 2>{});
    }
}

// ---------------------------------------------------------------- Q6_K ---
// One lane = one 16-element unit (super-block sb, half h, l-quad l0).
// XG: x is read from global memory (rows too long to stage x in LDS).
template <int R, bool XG = false>
__global__ __launch_bounds__(kThreads) void gemv_q6k_kernel(TaskTable tt, const float* __restrict__ x,
                                                            uint32_t cols, uint32_t total_groups) {
    extern __shared__ float xs_lds[];
    if constexpr (!XG) stage_x<false>(xs_lds, x, cols);
    const float* xs = XG ? x : xs_lds;
    const uint32_t nsb = cols >> 8;
    const uint32_t units = nsb * 16;
    const uint32_t rb = nsb * 210;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    for (uint32_t g = blockIdx.x * kWavesPerBlock + wave; g < total_groups; g += gridDim.x * kWavesPerBlock) {
        const int ti = find_task(tt, g);
        const GemvTask task = tt.t[ti];
        const uint32_t r0 = (g - tt.group_start[ti]) * R;
        float acc[R];
        const uint8_t* rowp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
            rowp[r] = task.w + (size_t)min(r0 + r, task.rows - 1) * rb;
        }
        for (uint32_t u = lane; u < units; u += kWave) {
            const uint32_t sb = u >> 4, h = (u >> 3) & 1u, l0 = (u & 7u) * 4u;
            const uint32_t xbase = sb * 256 + h * 128 + l0;
            float xv[4][4];
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const float4 v = *reinterpret_cast<const float4*>(xs + xbase + gi * 32);
                xv[gi][0] = v.x; xv[gi][1] = v.y; xv[gi][2] = v.z; xv[gi][3] = v.w;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t* sbp = rowp[r] + (size_t)sb * 210;
                const uint32_t qlA = load_u32_any(sbp + h * 64 + l0);
                const uint32_t qlB = load_u32_any(sbp + h * 64 + 32 + l0);
                const uint32_t qh = load_u32_any(sbp + 128 + h * 32 + l0);
                const uint32_t sc0 = load_u32_any(sbp + 192 + h * 8);
                const uint32_t sc1 = load_u32_any(sbp + 196 + h * 8);
                const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(sbp + 208)) * 0.25f;
                const uint32_t shsel = l0 >> 4;  // which of the two 16-element sub-blocks
                float part = 0.0f;
#pragma unroll
                for (int gi = 0; gi < 4; ++gi) {
                    uint32_t lo = (gi & 1) ? qlB : qlA;
                    if (gi >= 2) lo >>= 4;
                    lo &= 0x0F0F0F0Fu;
                    const uint32_t hi = ((qh >> (2 * gi)) & 0x03030303u) << 4;
                    const uint32_t v = ((lo | hi) ^ 0x20202020u) << 2;  // 4*(q-32) per byte
                    float s = 0.0f;
#pragma unroll
                    for (int k = 0; k < 4; ++k) s = fmaf(sbyte(v, k), xv[gi][k], s);
                    const uint32_t scw = gi < 2 ? sc0 : sc1;
                    const float sc = sbyte(scw, (2 * gi + shsel) & 3);
                    part = fmaf(d * sc, s, part);
                }
                acc[r] += part;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[r]);
            if (lane == r && r0 + r < task.rows) task.y[r0 + r] = v;
        }
    }
}

// Q6_K streaming kernel (cols % 2048 == 0, 16 B aligned rows).  A row is cut
// into chunks of 8 super-blocks (1680 B, a multiple of 16 B); a team of S =
// chunks-per-row waves covers a row, wave s owning chunk s, so each lane's x
// values (two 16-element units: 32 floats) stay in VGPRs for the whole
// kernel.  Each chunk is fetched with lane-contiguous dwordx4 loads into a
// per-wave LDS buffer; lane L then decodes its two 16-element units (one
// quarter of one half of super-block 2*(L/16) + k, a single sub-block scale)
// from LDS.  Fields of odd super-blocks sit at 2 mod 4 and are assembled
// with v_alignbyte.  PAIR as in the K-quant streaming kernel below: gate
// row i and up row i per team, silu(gate_i) * up_i stored into gate's y.
template <int R, int S, int NW, bool PAIR = false>
__global__ __launch_bounds__(NW * 64) void gemv_q6k_stream_kernel(TaskTable tt, const float* __restrict__ x,
                                                                 uint32_t cols, uint32_t total_blocks) {
    constexpr int TEAMS = NW / S;
    static_assert(!PAIR || R == 2, "a pair step holds one gate row and one up row");
    constexpr uint32_t CHUNK = 8 * 210;                  // bytes
    constexpr uint32_t CUNITS = CHUNK / 16;              // 105 dwordx4 units
    constexpr uint32_t BUFW = CHUNK / 4 + 4;             // dwords per row buffer (+pad for alignbyte reads)
    extern __shared__ uint32_t lds[];                    // [waves][R][BUFW]
    __shared__ float red[2][NW][R];
    const uint32_t rb = (cols >> 8) * 210;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = wave / S, slice = wave % S;
    uint32_t* wbuf = lds + wave * (R * BUFW);

    // A lane's unit k (two per lane) is 16 consecutive elements of one
    // quarter, so one sub-block scale covers it: super-block 2*(lane/16) + k
    // of the chunk, half h, quarter q, l0 = 0 or 16 from lane % 16.  One LDS
    // read instruction thus touches super-blocks {0,2,4,6} (k = 0, all 4-byte
    // aligned) or {1,3,5,7} (k = 1, all at 2 mod 4), whose dword starts fall
    // in four distinct residues mod 4: no bank conflicts.  x of both units
    // is kept in registers, loaded before any weights.
    float xv[2][16];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t sb = slice * 8 + ((uint32_t(lane) >> 4) << 1) + k, h = (lane >> 3) & 1u, q = (lane >> 1) & 3u,
                       l0 = (lane & 1u) * 16u;
        const float4* xp = reinterpret_cast<const float4*>(x + sb * 256 + h * 128 + q * 32 + l0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = xp[i];
            xv[k][4 * i] = v.x; xv[k][4 * i + 1] = v.y; xv[k][4 * i + 2] = v.z; xv[k][4 * i + 3] = v.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    auto locate = [&](uint32_t blk, const uint8_t*(&rowp)[R], uint32_t& row0, int& ti) {
        if constexpr (PAIR) {
            ti = 0;
            row0 = blk * TEAMS + team;
            const size_t off = (size_t)min(row0, tt.t[0].rows - 1) * rb + (size_t)slice * CHUNK;
            rowp[0] = tt.t[0].w + off;
            rowp[1] = tt.t[1].w + off;
            return;
        }
        ti = find_task(tt, blk);
        const GemvTask& t = tt.t[ti];
        row0 = (blk - tt.group_start[ti]) * (TEAMS * R) + team * R;
#pragma unroll
        for (int r = 0; r < R; ++r) rowp[r] = t.w + (size_t)min(row0 + r, t.rows - 1) * rb + (size_t)slice * CHUNK;
    };
    // the second unit of lanes past the chunk reads 0 without a memory request
    auto load = [&](const uint8_t*(&rowp)[R], uint4 (&u)[R][2]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const __amdgpu_buffer_rsrc_t rs = span_rsrc(rowp[r], CUNITS * 16);
            u[r][0] = span_load16(rs, uint32_t(lane) * 16);
            u[r][1] = span_load16(rs, uint32_t(lane + 64) * 16);
        }
    };

    uint32_t blk = blockIdx.x;
    uint4 u[R][2];
    uint32_t row0 = 0;
    int ti = 0;
    {
        const uint8_t* rowp[R];
        locate(min(blk, total_blocks - 1), rowp, row0, ti);
        load(rowp, u);
    }
    float nsx[2];  // -32 * sum of x over each of the lane's two units
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) a0 += xv[kk][i], a1 += xv[kk][i + 1];
        nsx[kk] = -32.0f * (a0 + a1);
    }
    int parity = 0;
    while (blk < total_blocks) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            reinterpret_cast<uint4*>(wbuf + r * BUFW)[lane] = u[r][0];
            if (lane + 64 < int(CUNITS)) reinterpret_cast<uint4*>(wbuf + r * BUFW)[lane + 64] = u[r][1];
        }
        const uint32_t nblk = blk + gridDim.x;
        const uint32_t row0c = row0;
        const int tic = ti;
        if (nblk < total_blocks) {
            const uint8_t* rowp[R];
            locate(nblk, rowp, row0, ti);
            load(rowp, u);
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t* buf = wbuf + r * BUFW;
            const uint8_t* bbytes = reinterpret_cast<const uint8_t*>(buf);
            // 16 bytes at a chunk offset that is 4-byte aligned (even
            // super-blocks) or at 2 mod 4 (odd: five dword reads, four
            // v_alignbyte)
            auto lds16 = [&](uint32_t off, bool odd, uint32_t (&o)[4]) {
                const uint32_t* w = buf + (off >> 2);
                if (!odd) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = w[i];
                } else {
                    uint32_t t5[5];
#pragma unroll
                    for (int i = 0; i < 5; ++i) t5[i] = w[i];
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = __builtin_amdgcn_alignbyte(t5[i + 1], t5[i], 2);
                }
            };
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t sbl = ((uint32_t(lane) >> 4) << 1) + k, h = (lane >> 3) & 1u, q = (lane >> 1) & 3u,
                               l0 = (lane & 1u) * 16u;
                const uint32_t base = sbl * 210;
                uint32_t ql[4], qh[4];
                lds16(base + h * 64 + (q & 1u) * 32 + l0, k == 1, ql);  // low nibbles (q < 2) or high (q >= 2)
                lds16(base + 128 + h * 32 + l0, k == 1, qh);            // 2-bit fields, quarter q at bit 2q
                const float sc = float(int8_t(bbytes[base + 192 + h * 8 + q * 2 + (l0 >> 4)]));
                const float d = half_bits_to_float(reinterpret_cast<const uint16_t*>(bbytes)[(base + 208) >> 1]);
                // rotations that bring quarter q's nibble to bits 0-3 and its
                // 2-bit field to bits 4-5 of every byte (bits rotated in from
                // neighbouring bytes land outside the masks)
                const uint32_t nrot = (q >> 1) * 4, hrot = (2 * q + 28) & 31u;
                float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // the four 6-bit codes u = q + 32 of elements 4j..4j+3, one per
                    // byte; sum (u-32)*x = sum u*x - 32 * sum x
                    const uint32_t lo4 = __builtin_amdgcn_alignbit(ql[j], ql[j], nrot);
                    const uint32_t hi2 = __builtin_amdgcn_alignbit(qh[j], qh[j], hrot) & 0x30303030u;
                    uint32_t codes = (lo4 & 0x0F0F0F0Fu) | hi2;
                    // opaque to the combiner, so each byte converts with one
                    // v_cvt_f32_ubyteN (one instruction per code, like Q8_0's SDWA
                    // conversion; v_fma_mix_f32 on the codes as binary16
                    // denormals issued more slowly)
                    asm volatile("" : "+v"(codes));
                    t0 = fmaf(float(codes & 0xffu), xv[k][4 * j], t0);
                    t1 = fmaf(float((codes >> 8) & 0xffu), xv[k][4 * j + 1], t1);
                    t0 = fmaf(float((codes >> 16) & 0xffu), xv[k][4 * j + 2], t0);
                    t1 = fmaf(float(codes >> 24), xv[k][4 * j + 3], t1);
                }
                a = fmaf(d * sc, (t0 + t1) + nsx[k], a);
            }
            acc[r] = wave_sum(a);
        }
        const GemvTask& t = tt.t[tic];
        if constexpr (PAIR && S == 1) {
            if (lane == 0 && row0c < t.rows) t.y[row0c] = acc[0] / (1.0f + expf(-acc[0])) * acc[1];
        } else if constexpr (S == 1) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (lane == r && row0c + r < t.rows) t.y[row0c + r] = acc[r];
        } else if constexpr (PAIR) {
            if (lane == 0) {
                red[parity][wave][0] = acc[0];
                red[parity][wave][1] = acc[1];
            }
            __syncthreads();
            if (slice == 0 && lane == 0 && row0c < t.rows) {
                float g = 0.0f, up = 0.0f;
#pragma unroll
                for (int s2 = 0; s2 < S; ++s2) {
                    g += red[parity][team * S + s2][0];
                    up += red[parity][team * S + s2][1];
                }
                t.y[row0c] = g / (1.0f + expf(-g)) * up;
            }
            parity ^= 1;
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) red[parity][wave][r] = acc[r];
            }
            __syncthreads();
            if (slice == 0 && lane < R) {
                float v = 0.0f;
#pragma unroll
                for (int s2 = 0; s2 < S; ++s2) v += red[parity][team * S + s2][lane];
                if (row0c + lane < t.rows) t.y[row0c + lane] = v;
            }
            parity ^= 1;
        }
        blk = nblk;
    }
}

// ------------------------------------------------------------ Q4_K / Q5_K ---
// A lane's fixed unit: super-block sb, nibble unit c (0..7) -> group pair
// j2 = c/2 (groups 2*j2 low nibbles, 2*j2+1 high nibbles), byte offset
// l0 = 16*(c%2) inside the 32-byte group pair.
struct KUnit {
    uint32_t hoff, qoff, boff, j2;
};
template <int FMT>
__device__ __forceinline__ KUnit kquant_unit(uint32_t u) {
    constexpr uint32_t BB = FMT == kQ5_K ? 176 : 144;
    constexpr uint32_t QOFF = FMT == kQ5_K ? 48 : 16;
    const uint32_t sb = u >> 3, c = u & 7u, j2 = c >> 1, l0 = (c & 1u) * 16u;
    return KUnit{sb * BB, sb * BB + QOFF + j2 * 32 + l0, sb * BB + 16 + l0, j2};
}
// The unit's 32 x values (16 of group 2*j2, 16 of group 2*j2+1) and their sums.
__device__ __forceinline__ void kquant_x(const float* __restrict__ x, uint32_t u, bool active, float (&xl)[16],
                                         float (&xh)[16], float& sxl, float& sxh) {
    const uint32_t sb = u >> 3, c = u & 7u;
    const float* p = x + sb * 256 + (c >> 1) * 64 + (c & 1u) * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 a = active ? reinterpret_cast<const float4*>(p)[i] : make_float4(0, 0, 0, 0);
        const float4 b = active ? reinterpret_cast<const float4*>(p + 32)[i] : make_float4(0, 0, 0, 0);
        xl[4 * i] = a.x; xl[4 * i + 1] = a.y; xl[4 * i + 2] = a.z; xl[4 * i + 3] = a.w;
        xh[4 * i] = b.x; xh[4 * i + 1] = b.y; xh[4 * i + 2] = b.z; xh[4 * i + 3] = b.w;
    }
    sxl = 0.0f;
    sxh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        sxl += xl[i];
        sxh += xh[i];
    }
}
// Dot of one unit of one row.  h = the super-block's first 16 bytes (d, dmin,
// scales), q = the unit's 16 nibble bytes, b = the 16 fifth-bit bytes (Q5_K).
// Scale/min of group j (src/quant.cpp:133-141): j < 4 from scales[j] and
// scales[j+4]; j >= 4 from the nibbles of scales[j+4] with the top two bits
// of scales[j-4] / scales[j].  In the 16-byte header scales[i] is byte i+4,
// so with jj = j & 3: a = byte jj of h.y, b = byte jj of h.z, c = byte jj of h.w.
template <int FMT>
__device__ __forceinline__ float kquant_dot(const uint4& h, const uint4& q, const uint4& b, const float (&xl)[16],
                                            const float (&xh)[16], float sxl, float sxh, uint32_t j2) {
    // lane constants: groups 2*j2 and 2*j2+1 sit at byte (j & 3) of the
    // scale words; the upper four groups take the split encoding
    const uint32_t upper = j2 >= 2 ? ~0u : 0u;
    const uint32_t sh0 = 16u * (j2 & 1u), sh1 = sh0 + 8u;
    auto scale_min = [&](uint32_t sh, float& sc, float& mn) {
        const uint32_t a = h.y >> sh, bb = h.z >> sh, c = h.w >> sh;
        const uint32_t s_lo = a & 63u, m_lo = bb & 63u;
        const uint32_t s_hi = (c & 15u) | ((a >> 2) & 0x30u), m_hi = ((c >> 4) & 15u) | ((bb >> 2) & 0x30u);
        sc = float((s_lo & ~upper) | (s_hi & upper));
        mn = float((m_lo & ~upper) | (m_hi & upper));
    };
    float sc0, mn0, sc1, mn1;
    scale_min(sh0, sc0, mn0);
    scale_min(sh1, sc1, mn1);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
    float slo = 0.0f, shi = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo = qw[i] & 0x0F0F0F0Fu;
        uint32_t hi = (qw[i] >> 4) & 0x0F0F0F0Fu;
        if constexpr (FMT == kQ5_K) {
            lo |= ((bw[i] >> (2 * j2)) & 0x01010101u) << 4;
            hi |= ((bw[i] >> (2 * j2 + 1)) & 0x01010101u) << 4;
        }
        // opaque to the combiner, so each byte converts with one v_cvt_f32_ubyteN
        asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            slo = fmaf(float((lo >> (8 * k)) & 0xffu), xl[4 * i + k], slo);
            shi = fmaf(float((hi >> (8 * k)) & 0xffu), xh[4 * i + k], shi);
        }
    }
    const float d = half_bits_to_float(h.x), dm = half_bits_to_float(h.x >> 16);
    const float mins = fmaf(dm * mn0, sxl, dm * mn1 * sxh);
    return fmaf(d * sc0, slo, fmaf(d * sc1, shi, -mins));
}

// Streaming K-quant GEMV (16-byte aligned rows and x).  A row is cut into
// slices of 8 super-blocks (64 nibble units); a team of S waves covers a row,
// wave s owning slice s, so a lane's unit (and its x) is fixed for the whole
// kernel.  Each slice-row (1152 / 1408 B) is fetched with lane-contiguous
// dwordx4 loads (every byte once, two loads per lane), stashed in a per-wave
// LDS buffer, and each lane reads its header, nibble unit and fifth-bit unit
// back with ds_read_b128.  R rows per team per block; the next block's loads
// are issued before the current one is decoded; slices are summed in LDS.
// PAIR (R = 2, tasks gate and up of equal rows): a team's two rows are gate
// row i and up row i, and it stores silu(gate_i) * up_i into gate's y -- the
// two sums are the ones the unpaired kernel computes for those rows.
template <int FMT, int R, int S, int NW, bool PAIR = false, int RN = kRnNone>
__global__ __launch_bounds__(NW * 64) void gemv_kquant_stream_kernel(TaskTable tt, const float* __restrict__ x,
                                                                     uint32_t cols, uint32_t total_blocks,
                                                                     ResidNorm rn) {
    constexpr uint32_t BB = FMT == kQ5_K ? 176 : 144;
    constexpr uint32_t QOFF = FMT == kQ5_K ? 48 : 16;
    constexpr uint32_t CUNITS = 8 * BB / 16;  // 16 B units of a full slice-row (72 / 88)
    constexpr int TEAMS = NW / S;
    static_assert(!PAIR || R == 2, "a pair step holds one gate row and one up row");
    static_assert(!(PAIR && RN == kRnAddOut), "a pair's output is not a residual");
    extern __shared__ uint4 klds[];           // [waves][R][CUNITS]
    __shared__ float red[2][NW][R];
    const uint32_t nsb = cols >> 8;
    const uint32_t rb = nsb * BB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = wave / S, slice = wave % S;
    const uint32_t sb0 = slice * 8;
    const uint32_t nsb_s = sb0 < nsb ? min(8u, nsb - sb0) : 0u;  // super-blocks in this slice
    const uint32_t nunits = nsb_s * (BB / 16);
    const uint32_t u = slice * 64 + lane;
    const bool active = uint32_t(lane >> 3) < nsb_s;
    uint4* buf = klds + wave * (R * CUNITS);

    // x first (loads retire in issue order); norm-in: the norm weight and the
    // sum-of-squares slots too, applied once the first weight block is issued
    float xl[16], xh[16], sxl, sxh;
    float wl[RN == kRnNormIn ? 16 : 1], wh[RN == kRnNormIn ? 16 : 1];
    double slot = 0.0;
    {
        const uint32_t uu = active ? u : 0u;
        const uint32_t sb = uu >> 3, c = uu & 7u;
        const float4* p = reinterpret_cast<const float4*>(x + sb * 256 + (c >> 1) * 64 + (c & 1u) * 16);
        float4 a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = p[i];
            b[i] = p[8 + i];
        }
        float4 wa[RN == kRnNormIn ? 4 : 1], wb[RN == kRnNormIn ? 4 : 1];
        if constexpr (RN == kRnNormIn) {
            const float4* pw = reinterpret_cast<const float4*>(rn.w + (reinterpret_cast<const float*>(p) - x));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wa[i] = pw[i];
                wb[i] = pw[8 + i];
            }
            slot = lane < kRnSlots ? rn.ss_in[lane] : 0.0;
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (RN == kRnNormIn) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wl[4 * i] = wa[i].x; wl[4 * i + 1] = wa[i].y; wl[4 * i + 2] = wa[i].z; wl[4 * i + 3] = wa[i].w;
                wh[4 * i] = wb[i].x; wh[4 * i + 1] = wb[i].y; wh[4 * i + 2] = wb[i].z; wh[4 * i + 3] = wb[i].w;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xl[4 * i] = a[i].x; xl[4 * i + 1] = a[i].y; xl[4 * i + 2] = a[i].z; xl[4 * i + 3] = a[i].w;
            xh[4 * i] = b[i].x; xh[4 * i + 1] = b[i].y; xh[4 * i + 2] = b[i].z; xh[4 * i + 3] = b[i].w;
        }
    }
    auto locate = [&](uint32_t blk, const uint8_t*(&rowp)[R], uint32_t& row0, int& ti) {
        if constexpr (PAIR) {
            ti = 0;
            row0 = blk * TEAMS + team;
            const size_t off = (size_t)min(row0, tt.t[0].rows - 1) * rb + (size_t)sb0 * BB * (nsb_s != 0);
            rowp[0] = tt.t[0].w + off;
            rowp[1] = tt.t[1].w + off;
            return;
        }
        ti = find_task(tt, blk);
        const GemvTask& t = tt.t[ti];
        row0 = (blk - tt.group_start[ti]) * (TEAMS * R) + team * R;
#pragma unroll
        for (int r = 0; r < R; ++r) rowp[r] = t.w + (size_t)min(row0 + r, t.rows - 1) * rb + (size_t)sb0 * BB * (nsb_s != 0);
    };
    // units past the slice read 0 without a memory request
    auto load = [&](const uint8_t*(&rowp)[R], uint4 (&v)[R][2]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const __amdgpu_buffer_rsrc_t rs = span_rsrc(rowp[r], nunits * 16);
            v[r][0] = span_load16(rs, uint32_t(lane) * 16);
            v[r][1] = span_load16(rs, uint32_t(lane + 64) * 16);
        }
    };
    auto stash = [&](const uint4 (&v)[R][2]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            buf[r * CUNITS + lane] = v[r][0];
            if (lane + 64 < int(CUNITS)) buf[r * CUNITS + lane + 64] = v[r][1];
        }
    };
    // add-out: lane r's residual value of row row0 + r, fetched with the
    // block's weights
    auto resid = [&](uint32_t row0, int ti) {
        const GemvTask& t = tt.t[ti];
        return lane < R ? t.y[min(row0 + uint32_t(lane), t.rows - 1)] : 0.0f;
    };
    uint32_t blk = blockIdx.x;
    uint4 v[R][2];
    uint32_t row0 = 0;
    int ti = 0;
    float res = 0.0f;
    double ssacc = 0.0;
    {
        const uint8_t* rowp[R];
        locate(min(blk, total_blocks - 1), rowp, row0, ti);
        load(rowp, v);
        if constexpr (RN == kRnAddOut) res = resid(row0, ti);
    }
    if constexpr (RN == kRnNormIn) {
        // x is the residual: v * inv * w, the RMSNorm kernel's arithmetic;
        // after the first weight block is issued
        __builtin_amdgcn_sched_barrier(0);
        const double ss = wave_sum(slot);
        const float inv = 1.0f / sqrtf(float(ss / double(cols)) + rn.eps);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            xl[i] = xl[i] * inv * wl[i];
            xh[i] = xh[i] * inv * wh[i];
        }
    }
    sxl = 0.0f;
    sxh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        sxl += xl[i];
        sxh += xh[i];
    }
    const uint32_t sbl = uint32_t(lane >> 3), c = uint32_t(lane & 7), j2 = c >> 1, l0 = (c & 1u) * 16;
    const uint32_t hidx = sbl * (BB / 16), qidx = (sbl * BB + QOFF + j2 * 32 + l0) / 16,
                   bidx = (sbl * BB + 16 + l0) / 16;
    int parity = 0;
    while (blk < total_blocks) {
        stash(v);
        const uint32_t nblk = blk + gridDim.x;
        const uint32_t row0c = row0;
        const int tic = ti;
        const float resc = res;
        if (nblk < total_blocks) {
            const uint8_t* rowp[R];
            locate(nblk, rowp, row0, ti);
            load(rowp, v);
            if constexpr (RN == kRnAddOut) res = resid(row0, ti);
        }
        // the row value lane r stores: the sum, or the residual plus the sum
        auto out = [&](float sum) {
            if constexpr (RN == kRnAddOut) {
                const float nv = resc + sum;
                ssacc += double(nv) * double(nv);
                return nv;
            } else {
                return sum;
            }
        };
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint4* rb4 = buf + r * CUNITS;
            const uint4 h = rb4[hidx], q = rb4[qidx];
            const uint4 bq = FMT == kQ5_K ? rb4[bidx] : make_uint4(0, 0, 0, 0);
            acc[r] = active ? kquant_dot<FMT>(h, q, bq, xl, xh, sxl, sxh, j2) : 0.0f;
            acc[r] = wave_sum(acc[r]);
        }
        const GemvTask& t = tt.t[tic];
        if constexpr (PAIR && S == 1) {
            if (lane == 0 && row0c < t.rows) t.y[row0c] = acc[0] / (1.0f + expf(-acc[0])) * acc[1];
        } else if constexpr (S == 1) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (lane == r && row0c + r < t.rows) t.y[row0c + r] = out(acc[r]);
        } else if constexpr (PAIR) {
            if (lane == 0) {
                red[parity][wave][0] = acc[0];
                red[parity][wave][1] = acc[1];
            }
            __syncthreads();
            if (slice == 0 && lane == 0 && row0c < t.rows) {
                float g = 0.0f, up = 0.0f;
#pragma unroll
                for (int s2 = 0; s2 < S; ++s2) {
                    g += red[parity][team * S + s2][0];
                    up += red[parity][team * S + s2][1];
                }
                t.y[row0c] = g / (1.0f + expf(-g)) * up;
            }
            parity ^= 1;
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) red[parity][wave][r] = acc[r];
            }
            __syncthreads();
            if (slice == 0 && lane < R) {
                float sum = 0.0f;
#pragma unroll
                for (int s2 = 0; s2 < S; ++s2) sum += red[parity][team * S + s2][lane];
                if (row0c + lane < t.rows) t.y[row0c + lane] = out(sum);
            }
            parity ^= 1;
        }
        blk = nblk;
    }
    if constexpr (RN == kRnAddOut) {
        // every wave leaves the loop together: one atomic per workgroup
        __shared__ double ssw[NW];
        const double sw = wave_sum(ssacc);
        if (lane == 0) ssw[wave] = sw;
        __syncthreads();
        if (threadIdx.x == 0) {
            double tot = 0.0;
#pragma unroll
            for (int i = 0; i < NW; ++i) tot += ssw[i];
            atomicAdd(rn.ss_out + blockIdx.x % kRnSlots, tot);
        }
        if (blockIdx.x == 0 && threadIdx.x < kRnSlots && rn.ss_zero) rn.ss_zero[threadIdx.x] = 0.0;
    }
}

// Generic K-quant GEMV: any cols % 256 == 0 with dword-aligned rows; one wave
// per row, lanes stride over the row's units, x read from global memory.
template <int FMT>
__global__ __launch_bounds__(kThreads) void gemv_kquant_generic_kernel(TaskTable tt, const float* __restrict__ x,
                                                                       uint32_t cols, uint32_t total_groups) {
    constexpr uint32_t BB = FMT == kQ5_K ? 176 : 144;
    const uint32_t units = cols >> 5;
    const uint32_t rb = (cols >> 8) * BB;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    auto ld4 = [](const uint8_t* p) {
        const uint32_t* d = reinterpret_cast<const uint32_t*>(p);
        return make_uint4(d[0], d[1], d[2], d[3]);
    };
    for (uint32_t g = blockIdx.x * kWavesPerBlock + wave; g < total_groups; g += gridDim.x * kWavesPerBlock) {
        const int ti = find_task(tt, g);
        const GemvTask task = tt.t[ti];
        const uint32_t row = g - tt.group_start[ti];
        const uint8_t* rp = task.w + (size_t)row * rb;
        float acc = 0.0f;
        for (uint32_t u = lane; u < units; u += kWave) {
            const KUnit ku = kquant_unit<FMT>(u);
            float xl[16], xh[16], sxl, sxh;
            kquant_x(x, u, true, xl, xh, sxl, sxh);
            const uint4 h = ld4(rp + ku.hoff), q = ld4(rp + ku.qoff);
            const uint4 b = FMT == kQ5_K ? ld4(rp + ku.boff) : make_uint4(0, 0, 0, 0);
            acc += kquant_dot<FMT>(h, q, b, xl, xh, sxl, sxh, ku.j2);
        }
        acc = wave_sum(acc);
        if (lane == 0) task.y[row] = acc;
    }
}

// ------------------------------------------------------------- generic ---
// Lane-per-block fallback for Q8_0 / Q4_0 rows whose block count is odd or
// whose base is not dword-aligned.  x is read from global memory.
template <int FMT>
__global__ __launch_bounds__(kThreads) void gemv_block_kernel(TaskTable tt, const float* __restrict__ x,
                                                              uint32_t cols, uint32_t total_groups) {
    constexpr uint32_t BB = FMT == kQ8_0 ? 34 : 18;
    const uint32_t nb = cols >> 5;
    const uint32_t rb = nb * BB;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    for (uint32_t g = blockIdx.x * kWavesPerBlock + wave; g < total_groups; g += gridDim.x * kWavesPerBlock) {
        const int ti = find_task(tt, g);
        const GemvTask task = tt.t[ti];
        const uint32_t row = g - tt.group_start[ti];
        const uint8_t* rp = task.w + (size_t)row * rb;
        float acc = 0.0f;
        for (uint32_t b = lane; b < nb; b += kWave) {
            const uint8_t* p = rp + (size_t)b * BB;
            const float d = half_bits_to_float(uint32_t(p[0]) | (uint32_t(p[1]) << 8));
            const float* xb = x + b * 32;
            float s = 0.0f;
            if constexpr (FMT == kQ8_0) {
                for (int j = 0; j < 32; ++j) s = fmaf(float(int8_t(p[2 + j])), xb[j], s);
            } else {
                for (int j = 0; j < 16; ++j) {
                    s = fmaf(float(int(p[2 + j] & 15) - 8), xb[j], s);
                    s = fmaf(float(int(p[2 + j] >> 4) - 8), xb[j + 16], s);
                }
            }
            acc = fmaf(d, s, acc);
        }
        const float v = wave_sum(acc);
        if (lane == 0) task.y[row] = v;
    }
}

// ------------------------------------------------- MFMA streaming GEMV ---
// Q8_0 / Q4_0 decode GEMV with the per-block integer dots on the matrix
// cores.  x (fp32) is split exactly into four int8 "digit" vectors per 64-
// element pair: X = trunc(x * 2^s) with one exponent s per pair such that
// |X| < 2^30, and X = sum_j d_j 256^j with balanced digits d_j in [-128, 127]
// (the bytes of (X + 0x80808080) ^ 0x80808080).  Each 32-element block dot
// with one digit vector is then an exact int32 (|sum| < 2^20), computed by
// v_mfma_i32_4x4x4_16b_i8: 16 independent 4x4x4 products per instruction,
// product b = (4 weight rows of pair b) x (4 digit vectors of pair b), 8
// instructions per block (K = 4 each), accumulating in C.  The lane of
// product b and digit j then holds, for each of the 4 rows, the block's dot
// with digit j; it adds float(dot) * d_w (v_fma_mix_f32 reads the fp16 scale
// in place) for both blocks of the pair and scales the sum by 2^(8j - s),
// exactly.  The only rounding is that of the fp32 sums (and of x below 2^-30
// of its pair's largest element, which X drops), so the result is within the
// fp32 reference's own rounding level.  Against the fp32-FMA kernel this
// replaces ~2 VALU instructions per weight element by ~24 per 4096 elements,
// so the decode tail after the last weight block shrinks.  Non-finite x makes
// every output NaN.
//
// Work split: a wave owns a slice of 16 pairs (1024 columns) for the whole
// kernel -- its digits stay in 16 VGPRs -- and each row block it streams
// ROWS = 4 (Q8_0) or 8 (Q4_0) rows x 16 pairs (coalesced 16 B loads, stashed
// through LDS at a row stride that makes the lane reads conflict-free), so
// S = ceil(pairs / 16) waves cover a row and TEAMS = 16 / S teams of S waves
// share a workgroup (ROWS x TEAMS rows per row block).  The S partial sums
// of a row are added through LDS in slice order.
typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int kMfmaPairs = 16;  // pairs per slice
template <int FMT>
struct MfmaGeo {
    static constexpr int DW = FMT == kQ8_0 ? 17 : 9;       // dwords per pair
    static constexpr int UPR = kMfmaPairs * DW / 4;         // 16 B units per row segment (68 / 36)
    static constexpr int WROW = FMT == kQ8_0 ? 280 : 152;  // LDS dwords per stashed row (bank-conflict-free reads)
    // 4-row groups per wave step: Q4_0's 4 rows are half of Q8_0's bytes, and
    // a step's cost is mostly its latency chain (stash, MFMAs, sums,
    // barrier), so Q4_0 takes two groups per step
    static constexpr int RG = FMT == kQ8_0 ? 1 : 2;
    static constexpr int ROWS = 4 * RG;                     // rows per wave step
    static constexpr int WBUF = ROWS * WROW;                // dwords per wave stash
    static constexpr int NU = (ROWS * UPR + 63) / 64;       // 16 B loads per lane per row block
};

template <int FMT, int XPT, int D, int XK>
__global__ __launch_bounds__(1024) void gemv_mfma_kernel(TaskTable tt, const float* __restrict__ x, uint32_t cols,
                                                          uint32_t total_blocks, uint32_t S, uint32_t TEAMS,
                                                          XPrologue pro) {
    using G = MfmaGeo<FMT>;
    constexpr int DW = G::DW;
    extern __shared__ uint32_t lds[];
    // LDS map: [0, NW*WBUF) weight stashes; then the digits (S*16 pairs x 68
    // dwords: 16 float4 x 4 digits, 4 dwords of padding); then the pair
    // exponents; then the partial sums [2][NW][ROWS][4 lane groups].
    const uint32_t NW = S * TEAMS, NT = NW * 64;
    const uint32_t pairs = cols >> 6;
    const uint32_t spairs = S * kMfmaPairs;                 // pairs incl. the last slice's padding
    uint32_t* gdig = lds + NW * G::WBUF;
    int* sexp = reinterpret_cast<int*>(gdig + spairs * 68);
    float* red = reinterpret_cast<float*>(sexp + spairs);
    const uint32_t rb = pairs * DW * 4;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t team = wave / S, slice = wave % S;
    const uint32_t p0 = slice * kMfmaPairs;
    const uint32_t np = p0 < pairs ? min(uint32_t(kMfmaPairs), pairs - p0) : 0u;
    const uint32_t seg = np * DW * 4;                      // valid bytes of a row segment
    const int qb = lane >> 2, qi = lane & 3;               // product (pair) and row / digit of this lane
    uint32_t* buf = lds + wave * G::WBUF;

    // ---- x (or its producer's operands) first: loads retire in order
    const uint32_t nx4 = cols >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(XK == kXPlain ? x : pro.a);
    float4 xr[XPT], xb[XK == kXPlain ? 1 : XPT], xw[XK == kAddNorm ? XPT : 1];
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
        const uint32_t idx = min(threadIdx.x + uint32_t(k) * NT, nx4 - 1);
        xr[k] = x4[idx];
        if constexpr (XK == kSiluMul) xb[k] = reinterpret_cast<const float4*>(pro.b)[idx];
        if constexpr (XK == kAddNorm) {
            xb[k] = pro.b ? reinterpret_cast<const float4*>(pro.b)[idx] : make_float4(0, 0, 0, 0);
            xw[k] = reinterpret_cast<const float4*>(pro.w)[idx];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- weight ring: D row blocks in flight
    auto locate = [&](uint32_t blk, uint32_t& row0, int& ti) {
        // wave-uniform, so the task table is read with scalar loads
        ti = __builtin_amdgcn_readfirstlane(find_task(tt, blk));
        row0 = __builtin_amdgcn_readfirstlane((blk - tt.group_start[ti]) * (TEAMS * G::ROWS) + team * G::ROWS);
    };
    auto load = [&](uint32_t row0, int ti, uint4 (&u)[G::NU]) {
        const GemvTask& t = tt.t[ti];
        const __amdgpu_buffer_rsrc_t rs = span_rsrc(t.w, t.rows * rb);
#pragma unroll
        for (int m = 0; m < G::NU; ++m) {
            const uint32_t unit = uint32_t(lane + 64 * m);
            const uint32_t i = unit / G::UPR, o = unit - i * G::UPR;
            const uint32_t row = min(row0 + i, t.rows - 1);
            const uint32_t off = (i < G::ROWS && 16 * o < seg) ? row * rb + p0 * DW * 4 + 16 * o : 0xFFFFFFF0u;
            u[m] = span_load16(rs, off);
        }
    };
    auto stash = [&](const uint4 (&u)[G::NU]) {
#pragma unroll
        for (int m = 0; m < G::NU; ++m) {
            const uint32_t unit = uint32_t(lane + 64 * m);
            const uint32_t i = unit / G::UPR, o = unit - i * G::UPR;
            if (i < G::ROWS) reinterpret_cast<uint4*>(buf + i * G::WROW)[o] = u[m];
        }
    };
    uint32_t blk = blockIdx.x;
    uint4 u[D][G::NU];
    uint32_t row0s[D];
    int tis[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {  // branch-free: a slot past the end re-reads the last block
        const uint32_t b = min(blk + uint32_t(d) * gridDim.x, total_blocks - 1);
        locate(b, row0s[d], tis[d]);
        load(row0s[d], tis[d], u[d]);
    }

    // ---- x prologue, then x (fp32) into LDS
    if constexpr (XK == kSiluMul) {
        auto f = [](float g, float u) { return g / (1.0f + expf(-g)) * u; };
#pragma unroll
        for (int k = 0; k < XPT; ++k)
            xr[k] = make_float4(f(xr[k].x, xb[k].x), f(xr[k].y, xb[k].y), f(xr[k].z, xb[k].z), f(xr[k].w, xb[k].w));
    }
    if constexpr (XK == kAddNorm) {
        // v = a + b; sum of squares in double; inv = 1/sqrtf(float(ss/n) + eps);
        // x = v * inv * w -- the arithmetic of rmsnorm_kernel
        __shared__ double xred[16];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            xr[k] = make_float4(xr[k].x + xb[k].x, xr[k].y + xb[k].y, xr[k].z + xb[k].z, xr[k].w + xb[k].w);
            if (threadIdx.x + uint32_t(k) * NT < nx4) {
                ss += double(xr[k].x) * double(xr[k].x);
                ss += double(xr[k].y) * double(xr[k].y);
                ss += double(xr[k].z) * double(xr[k].z);
                ss += double(xr[k].w) * double(xr[k].w);
                if (pro.r_out && blockIdx.x == 0)
                    reinterpret_cast<float4*>(pro.r_out)[threadIdx.x + uint32_t(k) * NT] = xr[k];
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) xred[wave] = ss;
        __syncthreads();
        double tot = 0.0;
        for (uint32_t i = 0; i < NW; ++i) tot += xred[i];
        const float inv = 1.0f / sqrtf(float(tot / double(cols)) + pro.eps);
#pragma unroll
        for (int k = 0; k < XPT; ++k)
            xr[k] = make_float4(xr[k].x * inv * xw[k].x, xr[k].y * inv * xw[k].y, xr[k].z * inv * xw[k].z,
                                xr[k].w * inv * xw[k].w);
    }
    // ---- digits, straight from the registers: thread t holds float4 t + k*NT,
    // so the 16 float4 of a pair sit in 16 consecutive lanes (NT % 64 == 0);
    // their max comes from a 16-lane DPP reduction.  Digit j of the pair's
    // float4 e lands at dword p*68 + 4e + j (one 16 B write per float4; the
    // 68-dword pair stride makes the B reads below conflict-free).
    int bad = 0;
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
        const uint32_t idx = threadIdx.x + uint32_t(k) * NT;
        const float4 t = idx < nx4 ? xr[k] : make_float4(0, 0, 0, 0);
        float am = fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w)));
        am = fmaxf(am, dpp_f<kDppXor1>(am));
        am = fmaxf(am, dpp_f<kDppXor2>(am));
        am = fmaxf(am, dpp_f<kDppHalfMirror>(am));
        am = fmaxf(am, dpp_f<kDppMirror>(am));
        bad |= !(am <= 3.402823466e38f);  // inf or NaN
        const int s = 30 - (am > 0.0f && am <= 3.402823466e38f ? __builtin_amdgcn_frexp_expf(am) : 0);
        const uint32_t y0 = uint32_t(int(ldexpf(t.x, s))) + 0x80808080u;
        const uint32_t y1 = uint32_t(int(ldexpf(t.y, s))) + 0x80808080u;
        const uint32_t y2 = uint32_t(int(ldexpf(t.z, s))) + 0x80808080u;
        const uint32_t y3 = uint32_t(int(ldexpf(t.w, s))) + 0x80808080u;
        const uint32_t t01a = __builtin_amdgcn_perm(y1, y0, 0x05010400u);
        const uint32_t t01b = __builtin_amdgcn_perm(y1, y0, 0x07030602u);
        const uint32_t t23a = __builtin_amdgcn_perm(y3, y2, 0x05010400u);
        const uint32_t t23b = __builtin_amdgcn_perm(y3, y2, 0x07030602u);
        if (idx < spairs * 16) {
            const uint32_t p = idx >> 4, e = idx & 15;
            *reinterpret_cast<uint4*>(gdig + p * 68 + 4 * e) =
                make_uint4(__builtin_amdgcn_perm(t23a, t01a, 0x05040100u) ^ 0x80808080u,
                           __builtin_amdgcn_perm(t23a, t01a, 0x07060302u) ^ 0x80808080u,
                           __builtin_amdgcn_perm(t23b, t01b, 0x05040100u) ^ 0x80808080u,
                           __builtin_amdgcn_perm(t23b, t01b, 0x07060302u) ^ 0x80808080u);
            if (e == 0) sexp[p] = s;
        }
    }
    const bool nan_out = __syncthreads_or(bad) != 0;
    // this lane's B operand: digit qi of pair p0 + qb (16 dwords, K order)
    int dig[16];
    {
        const uint32_t* src = gdig + (p0 + qb) * 68 + qi;
#pragma unroll
        for (int e = 0; e < 16; ++e) dig[e] = int(src[4 * e]);
    }
    const int fexp = 8 * qi - sexp[p0 + qb];
    // Q4_0: the codes enter the MFMA as n (0..15); the -8 offset is added to
    // each block's dot as -8 * (sum of the block's digits), one per lane
    // (the lane's digit column is the same for its 4 rows)
    int o0 = 0, o1 = 0;
    if constexpr (FMT == kQ4_0) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            o0 = __builtin_amdgcn_sdot4(dig[t], 0x01010101, o0, false);
            o1 = __builtin_amdgcn_sdot4(dig[8 + t], 0x01010101, o1, false);
        }
        o0 *= -8;
        o1 *= -8;
    }

    int parity = 0;
    // One row block from ring slot d.  The stash is this wave's own LDS
    // buffer (a wave's LDS accesses complete in order, so no barrier guards
    // it); the partial sums alternate between two buffers, and the one
    // barrier per row block separates a buffer's reads from its next writes.
    auto step = [&](auto dc) {
        constexpr int d = decltype(dc)::value;
        stash(u[d]);
        const uint32_t row0 = row0s[d];
        const int ti = tis[d];
        const uint32_t nblk = blk + uint32_t(D) * gridDim.x;
        if (nblk < total_blocks) {
            locate(nblk, row0s[d], tis[d]);
            load(row0s[d], tis[d], u[d]);
        }
        float* rp = red + parity * (16 * 16 * G::RG);
#pragma unroll
        for (int g = 0; g < G::RG; ++g) {
            const uint32_t* gb = buf + 4 * g * G::WROW;
            const uint32_t* pr = gb + qi * G::WROW + qb * DW;  // A: row 4g + qi, pair qb
            uint32_t q[DW];
#pragma unroll
            for (int k = 0; k < DW; ++k) q[k] = pr[k];
            // scales of rows 0..3 of pair qb, read with the operands: d0 in the
            // low half of dword 0, d1 in the high half of dword 8 (Q8_0) / 4 (Q4_0)
            uint32_t sw0[4], sw1[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t* pi = gb + i * G::WROW + qb * DW;
                sw0[i] = pi[0];
                sw1[i] = pi[FMT == kQ8_0 ? 8 : 4];
            }
            // two accumulation chains per block (K slices 0-3 and 4-7), so
            // dependent MFMAs are four deep instead of eight
            v4i e0 = {0, 0, 0, 0}, e1 = {0, 0, 0, 0}, f0 = {0, 0, 0, 0}, f1 = {0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                int a0, a1;
                if constexpr (FMT == kQ8_0) {
                    a0 = int(__builtin_amdgcn_alignbyte(q[t + 1], q[t], 2));
                    a1 = int(q[9 + t]);
                } else {
                    const uint32_t w0 = __builtin_amdgcn_alignbyte(q[(t & 3) + 1], q[t & 3], 2);
                    a0 = int((t < 4 ? w0 : w0 >> 4) & 0x0F0F0F0Fu);
                    a1 = int((t < 4 ? q[5 + t] : q[1 + t] >> 4) & 0x0F0F0F0Fu);
                }
                if (t < 4) {
                    e0 = __builtin_amdgcn_mfma_i32_4x4x4i8(a0, dig[t], e0, 0, 0, 0);
                    e1 = __builtin_amdgcn_mfma_i32_4x4x4i8(a1, dig[8 + t], e1, 0, 0, 0);
                } else {
                    f0 = __builtin_amdgcn_mfma_i32_4x4x4i8(a0, dig[t], f0, 0, 0, 0);
                    f1 = __builtin_amdgcn_mfma_i32_4x4x4i8(a1, dig[8 + t], f1, 0, 0, 0);
                }
            }
            float acc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float a = float(e0[i] + f0[i] + o0) * float(__builtin_bit_cast(_Float16, uint16_t(sw0[i])));
                a = fmaf(float(e1[i] + f1[i] + o1), float(__builtin_bit_cast(_Float16, uint16_t(sw1[i] >> 16))), a);
                acc[i] = ldexpf(a, fexp);
            }
            // sum over the 4 digits (quad), then each lane keeps row (lane & 3)
            // and sums its 16-lane row's 4 quads; lanes 16g' + i then hold row
            // i's sum over the pairs 4g' .. 4g'+3
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[i] += dpp_f<kDppXor1>(acc[i]);
                acc[i] += dpp_f<kDppXor2>(acc[i]);
            }
            float v = qi == 0 ? acc[0] : qi == 1 ? acc[1] : qi == 2 ? acc[2] : acc[3];
            v += dpp_f<0x124>(v);  // row_ror:4
            v += dpp_f<0x128>(v);  // row_ror:8
            if ((lane & 15) < 4) rp[(wave * G::RG + g) * 16 + qi * 4 + (lane >> 4)] = v;
        }
        __syncthreads();
        if (slice == 0 && lane < G::ROWS) {
            // slice order; every load issued before the adds
            const uint32_t g = lane >> 2, r = lane & 3;
            float4 w[16];
#pragma unroll
            for (uint32_t s2 = 0; s2 < 16; ++s2)
                if (s2 < S) w[s2] = *reinterpret_cast<const float4*>(rp + ((team * S + s2) * G::RG + g) * 16 + r * 4);
            float s = 0.0f;
#pragma unroll
            for (uint32_t s2 = 0; s2 < 16; ++s2)
                if (s2 < S) s += ((w[s2].x + w[s2].y) + w[s2].z) + w[s2].w;
            const GemvTask& t = tt.t[ti];
            if (row0 + lane < t.rows) t.y[row0 + lane] = nan_out ? __builtin_nanf("") : s;
        }
        parity ^= 1;
        blk += gridDim.x;
    };
    while (blk < total_blocks) {
        step(std::integral_constant<int, 0>{});
        if constexpr (D > 1) if (blk < total_blocks) step(std::integral_constant<int, 1>{});
    }
}

int rows_per_wave(uint32_t total_rows) {
    static const int forced = [] {
        const char* e = getenv("ZQ_GEMV_ROWS_PER_WAVE");
        const int v = e ? atoi(e) : 0;
        return (v == 1 || v == 2 || v == 4) ? v : 0;
    }();
    if (forced) return forced;
    if (total_rows >= 8192) return 4;
    if (total_rows >= 2048) return 2;
    return 1;
}

int xreg_rows(uint32_t total_rows) {
    static const int forced = [] {
        const char* e = getenv("ZQ_GEMV_ROWS_PER_WAVE");
        const int v = e ? atoi(e) : 0;
        return (v == 1 || v == 2 || v == 4) ? v : 0;
    }();
    if (forced) return forced;
    (void)total_rows;
    return 1;
}

template <int FMT, int R>
hipError_t launch_pairs(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    uint32_t groups = 0;
    for (int i = 0; i < tt.count; ++i) {
        tt.group_start[i] = groups;
        groups += (tt.t[i].rows + R - 1) / R;
    }
    tt.group_start[tt.count] = groups;
    const uint32_t blocks = std::min<uint32_t>((groups + kWavesPerBlock - 1) / kWavesPerBlock, 4096u);
    const size_t lds = size_t(cols >> 6) * kPadStride * sizeof(float);
    hipLaunchKernelGGL((gemv_pairs_kernel<FMT, R>), dim3(blocks), dim3(kThreads), lds, stream, tt, x, cols, groups);
    return hipGetLastError();
}
// LDS budget of one workgroup for the staged activation vector.
size_t lds_limit() {
    static const size_t limit = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess) return size_t(65536);
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            return size_t(65536);
        return size_t(v);
    }();
    return limit;
}

int cu_count() {
    static const int n = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            return 256;
        return v;
    }();
    return n;
}
// Workgroups per CU of the x-in-registers kernel.
constexpr int kXregWgPerCu = 4;

template <int FMT, int R, int S, int NW, int D, int XK = kXPlain, int EP = 0>
hipError_t launch_stream(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream,
                         const XPrologue& pro = XPrologue{}) {
    constexpr uint32_t RB = (NW / S) * R;
    constexpr int DW = FMT == kQ8_0 ? 17 : 9;
    uint32_t blocks = 0;
    for (int i = 0; i < tt.count; ++i) {
        tt.group_start[i] = blocks;
        blocks += (tt.t[i].rows + RB - 1) / RB;
    }
    if (EP == 1) blocks = (tt.t[0].rows + 7) / 8;  // 8 rows of each task per block
    tt.group_start[tt.count] = blocks;
    size_t lds = size_t(NW) * R * 64 * DW * 4;
    if (S == 1 || NW > S) lds = std::max(lds, size_t(cols >> 6) * kPadStride * sizeof(float));
    if (lds > lds_limit()) return hipErrorInvalidConfiguration;
    // workgroups per CU: one at 16 waves, else the occupancy at this LDS size
    // (it depends on cols), cached per size
    int resident = 1;
    if constexpr (NW != 16) {
        static std::mutex mu;
        static size_t keys[8];
        static int vals[8], nkeys = 0;
        std::lock_guard<std::mutex> lock(mu);
        int i = 0;
        while (i < nkeys && keys[i] != lds) ++i;
        if (i < nkeys) {
            resident = vals[i];
        } else {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, gemv_stream_kernel<FMT, R, S, NW, D, XK, EP>,
                                                             NW * 64, lds) != hipSuccess || resident < 1)
                resident = 1;
            if (nkeys < 8) keys[nkeys] = lds, vals[nkeys++] = resident;
        }
    }
    const uint32_t grid = std::min<uint32_t>(blocks, uint32_t(cu_count() * resident));
    hipLaunchKernelGGL((gemv_stream_kernel<FMT, R, S, NW, D, XK, EP>), dim3(grid), dim3(NW * 64), lds, stream, tt, x,
                       cols, blocks, pro);
    return hipGetLastError();
}
// One workgroup of 16 waves per CU, one row block prefetched (D = 1): the
// steady state already streams at ~6.9 TB/s on MI355X; deeper register rings
// (8 waves x 2-3 blocks, 16 waves x 2 blocks) measured slower.  Outputs of at
// most 2048 rows with one slice per row take 8-wave workgroups, two per CU
// (Q8_0 1024x4096: 4.9 -> 4.5 us; 4096x4096 was slower: 5.9 -> 6.5 us).
template <int FMT, int S>
hipError_t launch_stream_r(int R, TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    (void)R;
    uint32_t rows = 0;
    for (int i = 0; i < tt.count; ++i) rows += tt.t[i].rows;
    if (S == 1 && rows <= 2048) return launch_stream<FMT, 1, S, 8, 1>(tt, x, cols, stream);
    return launch_stream<FMT, 1, S, 16, 1>(tt, x, cols, stream);
}
template <int FMT>
hipError_t launch_stream_any(int R, TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    const uint32_t pairs = cols >> 6;
    if (pairs <= 64) return launch_stream_r<FMT, 1>(R, tt, x, cols, stream);
    if (pairs <= 128) return launch_stream_r<FMT, 2>(R, tt, x, cols, stream);
    return launch_stream_r<FMT, 4>(R, tt, x, cols, stream);
}

// The MFMA streaming GEMV (gemv_mfma_kernel): S slices of 16 pairs per row,
// TEAMS = 16 / S teams, one workgroup per CU.
template <int FMT, int XK = kXPlain>
hipError_t launch_mfma(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream,
                       const XPrologue& pro = XPrologue{}) {
    using G = MfmaGeo<FMT>;
    const uint32_t pairs = cols >> 6;
    const uint32_t S = (pairs + kMfmaPairs - 1) / kMfmaPairs;
    if (!S || S > 16) return hipErrorInvalidConfiguration;
    const uint32_t TEAMS = 16 / S, NW = S * TEAMS, RB = G::ROWS * TEAMS;
    const size_t rb = size_t(pairs) * G::DW * 4;
    uint32_t blocks = 0;
    for (int i = 0; i < tt.count; ++i) {
        if (size_t(tt.t[i].rows) * rb >= (size_t(1) << 32) - 16) return hipErrorInvalidConfiguration;
        tt.group_start[i] = blocks;
        blocks += (tt.t[i].rows + RB - 1) / RB;
    }
    tt.group_start[tt.count] = blocks;
    const size_t lds = (size_t(NW) * G::WBUF + size_t(S) * kMfmaPairs * 69 + 512 * G::RG) * 4;
    if (lds > lds_limit()) return hipErrorInvalidConfiguration;
    const uint32_t grid = std::min<uint32_t>(blocks, uint32_t(cu_count()));
    const uint32_t xpt = (S * kMfmaPairs * 16 + NW * 64 - 1) / (NW * 64);  // float4 per thread, padded pairs included
#define ZQ_MFMA_LAUNCH(XPT)                                                                                        \
    hipLaunchKernelGGL((gemv_mfma_kernel<FMT, XPT, 1, XK>), dim3(grid), dim3(NW * 64), lds, stream, tt, x, cols, \
                       blocks, S, TEAMS, pro)
    if (xpt <= 1) ZQ_MFMA_LAUNCH(1);
    else if (xpt <= 2) ZQ_MFMA_LAUNCH(2);
    else if (xpt <= 4) ZQ_MFMA_LAUNCH(4);
    else return hipErrorInvalidConfiguration;
#undef ZQ_MFMA_LAUNCH
    return hipGetLastError();
}
// Which streaming kernel a shape takes.  Measured on MI355X (per launch,
// Q8_0): the MFMA kernel wins where a CU streams many row blocks or long rows
// (down 4096x14336: 15.0 -> 13.6 us; lm_head 128256x4096: 88.5 -> 80.6 us)
// and loses a little on short launches of 4096-column rows (q/o 6.1 -> 7.1
// us, gate|up 13.8 -> 14.1 us), whose fixed costs (the digit split, one more
// barrier) are not amortised.  Q4_0, with two 4-row groups per wave step,
// wins from 8192 rows on (14336x4096 10.7 -> 10.4 us, 4096x14336 11.7 ->
// 10.5 us, 128256x4096 64.4 -> 54.0 us) and loses on one-block launches
// (4096x4096 4.7 -> 6.8 us).  ZQ_GEMV_MFMA=0 / 1 forces the fp32-FMA / MFMA
// kernel everywhere (A/B runs).
// With an x prologue the SiLU*up form measured slower on the MFMA kernel
// (the down projection of the decoder: 15.3 -> 15.9 us), the add+RMSNorm
// form faster at vocabulary size (lm_head 87.7 -> 83.5 us).
int mfma_gemv_forced() {
    static const int forced = [] {
        const char* e = getenv("ZQ_GEMV_MFMA");
        return e && (e[0] == '0' || e[0] == '1') ? e[0] - '0' : -1;
    }();
    return forced;
}
bool mfma_gemv_for(int fmt, uint32_t cols, uint32_t total_rows, int xk = kXPlain) {
    if (mfma_gemv_forced() >= 0) return mfma_gemv_forced() == 1;
    const bool vocab = fmt == kQ8_0 && total_rows >= 32768;
    const bool tall = fmt == kQ4_0 && total_rows >= 8192;
    return xk == kXPlain ? cols > 4096 || vocab || tall : xk == kAddNorm && vocab;
}

template <int FMT, int R, int S>
hipError_t launch_xreg(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    constexpr uint32_t RB = (kWavesPerBlock / S) * R;
    uint32_t blocks = 0;
    for (int i = 0; i < tt.count; ++i) {
        tt.group_start[i] = blocks;
        blocks += (tt.t[i].rows + RB - 1) / RB;
    }
    tt.group_start[tt.count] = blocks;
    const uint32_t grid = std::min<uint32_t>(blocks, uint32_t(cu_count() * kXregWgPerCu));
    const size_t lds = S == 1 ? size_t(cols >> 6) * kPadStride * sizeof(float) : 0;
    hipLaunchKernelGGL((gemv_xreg_kernel<FMT, R, S>), dim3(grid), dim3(kThreads), lds, stream, tt, x, cols, blocks);
    return hipGetLastError();
}
template <int FMT, int S>
hipError_t launch_xreg_r(int R, TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    if (R == 4) return launch_xreg<FMT, 4, S>(tt, x, cols, stream);
    if (R == 2) return launch_xreg<FMT, 2, S>(tt, x, cols, stream);
    return launch_xreg<FMT, 1, S>(tt, x, cols, stream);
}
template <int FMT>
hipError_t launch_xreg_any(int R, TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    const uint32_t pairs = cols >> 6;
    if (pairs <= 64) return launch_xreg_r<FMT, 1>(R, tt, x, cols, stream);
    if (pairs <= 128) return launch_xreg_r<FMT, 2>(R, tt, x, cols, stream);
    return launch_xreg_r<FMT, 4>(R, tt, x, cols, stream);
}

template <int R>
hipError_t launch_q6k(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    uint32_t groups = 0;
    for (int i = 0; i < tt.count; ++i) {
        tt.group_start[i] = groups;
        groups += (tt.t[i].rows + R - 1) / R;
    }
    tt.group_start[tt.count] = groups;
    const uint32_t blocks = std::min<uint32_t>((groups + kWavesPerBlock - 1) / kWavesPerBlock, 4096u);
    if (size_t(cols) * sizeof(float) > lds_limit())
        hipLaunchKernelGGL((gemv_q6k_kernel<R, true>), dim3(blocks), dim3(kThreads), 0, stream, tt, x, cols, groups);
    else
        hipLaunchKernelGGL((gemv_q6k_kernel<R>), dim3(blocks), dim3(kThreads), size_t(cols) * sizeof(float), stream, tt,
                           x, cols, groups);
    return hipGetLastError();
}
template <int R, int S, int NW, bool PAIR = false>
hipError_t launch_q6k_stream(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream, uint32_t wg_per_cu = 1) {
    constexpr uint32_t TEAMS = NW / S;
    uint32_t blocks = 0;
    if (PAIR) {
        blocks = (tt.t[0].rows + TEAMS - 1) / TEAMS;  // one gate row and one up row per team
    } else {
        for (int i = 0; i < tt.count; ++i) {
            tt.group_start[i] = blocks;
            blocks += (tt.t[i].rows + TEAMS * R - 1) / (TEAMS * R);
        }
        tt.group_start[tt.count] = blocks;
    }
    const uint32_t grid = std::min<uint32_t>(blocks, uint32_t(cu_count()) * wg_per_cu);
    const size_t lds = size_t(NW) * R * (8 * 210 / 4 + 4) * 4;
    hipLaunchKernelGGL((gemv_q6k_stream_kernel<R, S, NW, PAIR>), dim3(grid), dim3(NW * 64), lds, stream, tt, x, cols,
                       blocks);
    return hipGetLastError();
}
// chunks per row -> (S, waves per workgroup); two workgroups per CU.  Two
// 8-wave workgroups measured faster than one 16-wave one (the per-step
// slice reduction then synchronises 8 waves, not 16), and 2 rows per step
// faster than 1 or 4: 14336x4096 19.6 -> 17.0 us, lm_head 96.6 -> 89.5 us.
template <int R, bool PAIR = false>
hipError_t launch_q6k_stream_s(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    switch ((cols >> 8) / 8) {
    case 1: return launch_q6k_stream<R, 1, 8, PAIR>(tt, x, cols, stream, 2);
    case 2: return launch_q6k_stream<R, 2, 8, PAIR>(tt, x, cols, stream, 2);
    case 3: return launch_q6k_stream<R, 3, 6, PAIR>(tt, x, cols, stream, 2);
    case 4: return launch_q6k_stream<R, 4, 8, PAIR>(tt, x, cols, stream, 2);
    case 5: return launch_q6k_stream<R, 5, 5, PAIR>(tt, x, cols, stream, 2);
    case 6: return launch_q6k_stream<R, 6, 6, PAIR>(tt, x, cols, stream, 2);
    case 7: return launch_q6k_stream<R, 7, 7, PAIR>(tt, x, cols, stream, 2);
    case 8: return launch_q6k_stream<R, 8, 8, PAIR>(tt, x, cols, stream, 2);
    default: return hipErrorInvalidConfiguration;
    }
}
hipError_t launch_q6k_stream_any(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream, uint32_t total_rows) {
    return total_rows >= 4096 ? launch_q6k_stream_s<2>(tt, x, cols, stream) : launch_q6k_stream_s<1>(tt, x, cols, stream);
}

template <int FMT, int R, int S, int NW, bool PAIR = false, int RN = kRnNone>
hipError_t launch_kquant_stream(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream, uint32_t wg_per_cu = 1,
                                const ResidNorm& rn = ResidNorm{}) {
    constexpr uint32_t RB = (NW / S) * R;
    constexpr uint32_t CUNITS = 8 * (FMT == kQ5_K ? 176 : 144) / 16;
    uint32_t blocks = 0;
    if (PAIR) {
        blocks = (tt.t[0].rows + NW / S - 1) / (NW / S);  // one gate row and one up row per team
    } else {
        for (int i = 0; i < tt.count; ++i) {
            tt.group_start[i] = blocks;
            blocks += (tt.t[i].rows + RB - 1) / RB;
        }
        tt.group_start[tt.count] = blocks;
    }
    const uint32_t grid = std::min<uint32_t>(blocks, uint32_t(cu_count()) * wg_per_cu);
    const size_t lds = size_t(NW) * R * CUNITS * 16;
    hipLaunchKernelGGL((gemv_kquant_stream_kernel<FMT, R, S, NW, PAIR, RN>), dim3(grid), dim3(NW * 64), lds, stream, tt,
                       x, cols, blocks, rn);
    return hipGetLastError();
}
// 64-unit slices per row -> (S, waves per workgroup); two workgroups per CU
// (measured faster than one 16-wave workgroup with the same rows per step:
// Q4_K 14336x4096 15.2 -> 13.9 us, Q5_K 17.0 -> 15.4 us at 2 rows per step).
template <int FMT, int R, bool PAIR = false, int RN = kRnNone>
hipError_t launch_kquant_stream_s(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream,
                                  const ResidNorm& rn = ResidNorm{}) {
    switch ((cols + 2047) / 2048) {
    case 1: return launch_kquant_stream<FMT, R, 1, 8, PAIR, RN>(tt, x, cols, stream, 2, rn);
    case 2: return launch_kquant_stream<FMT, R, 2, 8, PAIR, RN>(tt, x, cols, stream, 2, rn);
    case 3: return launch_kquant_stream<FMT, R, 3, 6, PAIR, RN>(tt, x, cols, stream, 2, rn);
    case 4: return launch_kquant_stream<FMT, R, 4, 8, PAIR, RN>(tt, x, cols, stream, 2, rn);
    case 5: return launch_kquant_stream<FMT, R, 5, 5, PAIR, RN>(tt, x, cols, stream, 2, rn);
    case 6: return launch_kquant_stream<FMT, R, 6, 6, PAIR, RN>(tt, x, cols, stream, 2, rn);
    case 7: return launch_kquant_stream<FMT, R, 7, 7, PAIR, RN>(tt, x, cols, stream, 2, rn);
    case 8: return launch_kquant_stream<FMT, R, 8, 8, PAIR, RN>(tt, x, cols, stream, 2, rn);
    default: return hipErrorInvalidConfiguration;
    }
}
template <int FMT>
hipError_t launch_kquant(int R, bool stream_ok, TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    if (stream_ok) {
        const hipError_t e = R >= 4   ? launch_kquant_stream_s<FMT, 4>(tt, x, cols, stream)
                             : R == 2 ? launch_kquant_stream_s<FMT, 2>(tt, x, cols, stream)
                                      : launch_kquant_stream_s<FMT, 1>(tt, x, cols, stream);
        if (e != hipErrorInvalidConfiguration) return e;
    }
    uint32_t groups = 0;
    for (int i = 0; i < tt.count; ++i) {
        tt.group_start[i] = groups;
        groups += tt.t[i].rows;
    }
    tt.group_start[tt.count] = groups;
    const uint32_t blocks = std::min<uint32_t>((groups + kWavesPerBlock - 1) / kWavesPerBlock, 4096u);
    hipLaunchKernelGGL((gemv_kquant_generic_kernel<FMT>), dim3(blocks), dim3(kThreads), 0, stream, tt, x, cols, groups);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_blocks(TaskTable& tt, const float* x, uint32_t cols, hipStream_t stream) {
    uint32_t groups = 0;
    for (int i = 0; i < tt.count; ++i) {
        tt.group_start[i] = groups;
        groups += tt.t[i].rows;
    }
    tt.group_start[tt.count] = groups;
    const uint32_t blocks = std::min<uint32_t>((groups + kWavesPerBlock - 1) / kWavesPerBlock, 4096u);
    hipLaunchKernelGGL((gemv_block_kernel<FMT>), dim3(blocks), dim3(kThreads), 0, stream, tt, x, cols, groups);
    return hipGetLastError();
}

}  // namespace

int device_cu_count() { return cu_count(); }

hipError_t launch_gemv(int fmt, const GemvTask* tasks, int count, const float* x, size_t cols,
                       hipStream_t stream) {
    if (count < 1 || count > kMaxTasks || !x || !row_bytes(fmt, cols) || cols > (1u << 24))
        return hipErrorInvalidValue;
    TaskTable tt{};
    tt.count = count;
    uint32_t total_rows = 0;
    bool aligned = true;
    for (int i = 0; i < count; ++i) {
        if (!tasks[i].w || !tasks[i].y || !tasks[i].rows) return hipErrorInvalidValue;
        tt.t[i] = tasks[i];
        total_rows += tasks[i].rows;
        aligned = aligned && (reinterpret_cast<uintptr_t>(tasks[i].w) & 3u) == 0;
    }
    const uint32_t c = static_cast<uint32_t>(cols);
    const int R = rows_per_wave(total_rows);
    if (fmt == kQ4_K || fmt == kQ5_K) {
        if (reinterpret_cast<uintptr_t>(x) & 15u) return hipErrorInvalidValue;
        bool w16 = true;
        for (int i = 0; i < count; ++i) {
            if (reinterpret_cast<uintptr_t>(tasks[i].w) & 3u) return hipErrorInvalidValue;
            w16 = w16 && (reinterpret_cast<uintptr_t>(tasks[i].w) & 15u) == 0;
        }
        static const int forced = [] {
            const char* e = getenv("ZQ_GEMV_ROWS_PER_WAVE");
            const int v = e ? atoi(e) : 0;
            return (v == 1 || v == 2 || v == 4) ? v : 0;
        }();
        // rows per step: 4 for vocabulary-sized outputs, 2 for projection-sized
        const int Rk = forced ? forced : (total_rows >= 32768 ? 4 : total_rows >= 4096 ? 2 : 1);
        return fmt == kQ4_K ? launch_kquant<kQ4_K>(Rk, w16, tt, x, c, stream)
                            : launch_kquant<kQ5_K>(Rk, w16, tt, x, c, stream);
    }
    if (fmt == kQ6_K) {
        if (reinterpret_cast<uintptr_t>(x) & 15u) return hipErrorInvalidValue;
        bool w16 = true;
        for (int i = 0; i < count; ++i) w16 = w16 && (reinterpret_cast<uintptr_t>(tasks[i].w) & 15u) == 0;
        if (w16 && c % 2048 == 0 && c / 2048 <= 8) {
            const hipError_t e = launch_q6k_stream_any(tt, x, c, stream, total_rows);
            if (e != hipErrorInvalidConfiguration) return e;
        }
        for (int i = 0; i < count; ++i)
            if (reinterpret_cast<uintptr_t>(tasks[i].w) & 1u) return hipErrorInvalidValue;
        if (R == 4) return launch_q6k<4>(tt, x, c, stream);
        if (R == 2) return launch_q6k<2>(tt, x, c, stream);
        return launch_q6k<1>(tt, x, c, stream);
    }
    const bool x16 = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    bool w16 = true;
    for (int i = 0; i < count; ++i) w16 = w16 && (reinterpret_cast<uintptr_t>(tasks[i].w) & 15u) == 0;
    if (w16 && x16 && c % 256 == 0 && c / 64 <= 256) {
        if (mfma_gemv_for(fmt, c, total_rows)) {
            const hipError_t e = fmt == kQ8_0 ? launch_mfma<kQ8_0>(tt, x, c, stream) : launch_mfma<kQ4_0>(tt, x, c, stream);
            if (e != hipErrorInvalidConfiguration) return e;
        }
        const int Rx = xreg_rows(total_rows);
        return fmt == kQ8_0 ? launch_stream_any<kQ8_0>(Rx, tt, x, c, stream) : launch_stream_any<kQ4_0>(Rx, tt, x, c, stream);
    }
    if (aligned && x16 && c % 64 == 0 && c / 64 <= 256) {
        const int Rx = xreg_rows(total_rows);
        return fmt == kQ8_0 ? launch_xreg_any<kQ8_0>(Rx, tt, x, c, stream) : launch_xreg_any<kQ4_0>(Rx, tt, x, c, stream);
    }
    const bool pairs_ok = aligned && (c % 64 == 0) && size_t(c / 64) * kPadStride * 4 <= lds_limit();
    if (!pairs_ok) return fmt == kQ8_0 ? launch_blocks<kQ8_0>(tt, x, c, stream) : launch_blocks<kQ4_0>(tt, x, c, stream);
    if (fmt == kQ8_0) {
        if (R == 4) return launch_pairs<kQ8_0, 4>(tt, x, c, stream);
        if (R == 2) return launch_pairs<kQ8_0, 2>(tt, x, c, stream);
        return launch_pairs<kQ8_0, 1>(tt, x, c, stream);
    }
    if (R == 4) return launch_pairs<kQ4_0, 4>(tt, x, c, stream);
    if (R == 2) return launch_pairs<kQ4_0, 2>(tt, x, c, stream);
    return launch_pairs<kQ4_0, 1>(tt, x, c, stream);
}


namespace {
template <int FMT, int XK>
hipError_t launch_prologue_s(TaskTable& tt, uint32_t cols, const XPrologue& pro, hipStream_t stream) {
    const uint32_t pairs = cols >> 6;
    if (pairs <= 64) return launch_stream<FMT, 1, 1, 16, 1, XK>(tt, nullptr, cols, stream, pro);
    if (pairs <= 128) return launch_stream<FMT, 1, 2, 16, 1, XK>(tt, nullptr, cols, stream, pro);
    return launch_stream<FMT, 1, 4, 16, 1, XK>(tt, nullptr, cols, stream, pro);
}
}  // namespace

hipError_t launch_gemv_prologue(int fmt, const GemvTask* tasks, int count, const XPrologue& pro, size_t cols,
                                hipStream_t stream) {
    if (count < 1 || count > kMaxTasks || !row_bytes(fmt, cols) || !pro.a) return hipErrorInvalidValue;
    if ((fmt != kQ8_0 && fmt != kQ4_0) || cols % 256 || cols / 64 > 256) return hipErrorInvalidConfiguration;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!a16(pro.a) || !a16(pro.b) || !a16(pro.w) || !a16(pro.r_out)) return hipErrorInvalidConfiguration;
    if ((pro.kind == kSiluMul && !pro.b) || (pro.kind == kAddNorm && !pro.w) ||
        (pro.kind != kSiluMul && pro.kind != kAddNorm))
        return hipErrorInvalidValue;
    TaskTable tt{};
    tt.count = count;
    for (int i = 0; i < count; ++i) {
        if (!tasks[i].w || !tasks[i].y || !tasks[i].rows) return hipErrorInvalidValue;
        if (!a16(tasks[i].w)) return hipErrorInvalidConfiguration;
        tt.t[i] = tasks[i];
    }
    const uint32_t c = static_cast<uint32_t>(cols);
    uint32_t total_rows = 0;
    for (int i = 0; i < count; ++i) total_rows += tasks[i].rows;
    if (mfma_gemv_for(fmt, c, total_rows, pro.kind)) {
        hipError_t e;
        if (pro.kind == kSiluMul)
            e = fmt == kQ8_0 ? launch_mfma<kQ8_0, kSiluMul>(tt, nullptr, c, stream, pro)
                             : launch_mfma<kQ4_0, kSiluMul>(tt, nullptr, c, stream, pro);
        else
            e = fmt == kQ8_0 ? launch_mfma<kQ8_0, kAddNorm>(tt, nullptr, c, stream, pro)
                             : launch_mfma<kQ4_0, kAddNorm>(tt, nullptr, c, stream, pro);
        if (e != hipErrorInvalidConfiguration) return e;
    }
    if (pro.kind == kSiluMul)
        return fmt == kQ8_0 ? launch_prologue_s<kQ8_0, kSiluMul>(tt, c, pro, stream)
                            : launch_prologue_s<kQ4_0, kSiluMul>(tt, c, pro, stream);
    return fmt == kQ8_0 ? launch_prologue_s<kQ8_0, kAddNorm>(tt, c, pro, stream)
                        : launch_prologue_s<kQ4_0, kAddNorm>(tt, c, pro, stream);
}

hipError_t launch_gemv_prologue_silu_pair(int fmt, const GemvTask& gate, const GemvTask& up, const XPrologue& pro,
                                          size_t cols, hipStream_t stream) {
    if (!row_bytes(fmt, cols) || !pro.a || !gate.w || !gate.y || !up.w || !gate.rows) return hipErrorInvalidValue;
    if ((fmt != kQ8_0 && fmt != kQ4_0) || cols % 256 || cols / 64 > 64 || up.rows != gate.rows)
        return hipErrorInvalidConfiguration;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!a16(pro.a) || !a16(pro.b) || !a16(pro.w) || !a16(pro.r_out) || !a16(gate.w) || !a16(up.w))
        return hipErrorInvalidConfiguration;
    if (pro.kind != kAddNorm || !pro.w) return hipErrorInvalidValue;
    TaskTable tt{};
    tt.count = 2;
    tt.t[0] = gate;
    tt.t[1] = GemvTask{up.w, gate.y, up.rows};
    const uint32_t c = static_cast<uint32_t>(cols);
    return fmt == kQ8_0 ? launch_stream<kQ8_0, 1, 1, 16, 1, kAddNorm, 1>(tt, nullptr, c, stream, pro)
                        : launch_stream<kQ4_0, 1, 1, 16, 1, kAddNorm, 1>(tt, nullptr, c, stream, pro);
}

hipError_t launch_gemv_silu_pair(int fmt, const GemvTask& gate, const GemvTask& up, const float* x, size_t cols,
                                 hipStream_t stream, const ResidNorm* rn) {
    if (!x || !row_bytes(fmt, cols) || cols > (1u << 24) || !gate.w || !gate.y || !up.w || !gate.rows)
        return hipErrorInvalidValue;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const bool q6k = fmt == kQ6_K && cols % 2048 == 0;  // whole 8-super-block chunks
    if ((fmt != kQ4_K && fmt != kQ5_K && !q6k) || cols > 16384 || up.rows != gate.rows || !a16(x) || !a16(gate.w) ||
        !a16(up.w))
        return hipErrorInvalidConfiguration;
    TaskTable tt{};
    tt.count = 2;
    tt.t[0] = gate;
    tt.t[1] = GemvTask{up.w, gate.y, up.rows};
    const uint32_t c = static_cast<uint32_t>(cols);
    if (rn) {
        if (q6k || !rn->ss_in || !a16(rn->w)) return hipErrorInvalidConfiguration;
        return fmt == kQ4_K ? launch_kquant_stream_s<kQ4_K, 2, true, kRnNormIn>(tt, x, c, stream, *rn)
                            : launch_kquant_stream_s<kQ5_K, 2, true, kRnNormIn>(tt, x, c, stream, *rn);
    }
    if (q6k) return launch_q6k_stream_s<2, true>(tt, x, c, stream);
    return fmt == kQ4_K ? launch_kquant_stream_s<kQ4_K, 2, true>(tt, x, c, stream)
                        : launch_kquant_stream_s<kQ5_K, 2, true>(tt, x, c, stream);
}

bool gemv_resid_supported(int fmt, size_t cols) {
    return (fmt == kQ4_K || fmt == kQ5_K) && cols && cols % 256 == 0 && cols <= 16384;
}

hipError_t launch_gemv_resid(int fmt, int mode, const GemvTask* tasks, int count, const float* x, size_t cols,
                             const ResidNorm& rn, hipStream_t stream) {
    if (count < 1 || count > kMaxTasks || !x || !row_bytes(fmt, cols)) return hipErrorInvalidValue;
    if ((mode == kRnNormIn && (!rn.ss_in || !rn.w)) || (mode == kRnAddOut && !rn.ss_out) ||
        (mode != kRnNormIn && mode != kRnAddOut))
        return hipErrorInvalidValue;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!gemv_resid_supported(fmt, cols) || !a16(x) || (mode == kRnNormIn && !a16(rn.w)))
        return hipErrorInvalidConfiguration;
    TaskTable tt{};
    tt.count = count;
    for (int i = 0; i < count; ++i) {
        if (!tasks[i].w || !tasks[i].y || !tasks[i].rows) return hipErrorInvalidValue;
        if (!a16(tasks[i].w)) return hipErrorInvalidConfiguration;
        tt.t[i] = tasks[i];
    }
    const uint32_t c = static_cast<uint32_t>(cols);
    // 2 rows per step: the projection-sized outputs' measured best
    if (mode == kRnNormIn)
        return fmt == kQ4_K ? launch_kquant_stream_s<kQ4_K, 2, false, kRnNormIn>(tt, x, c, stream, rn)
                            : launch_kquant_stream_s<kQ5_K, 2, false, kRnNormIn>(tt, x, c, stream, rn);
    return fmt == kQ4_K ? launch_kquant_stream_s<kQ4_K, 2, false, kRnAddOut>(tt, x, c, stream, rn)
                        : launch_kquant_stream_s<kQ5_K, 2, false, kRnAddOut>(tt, x, c, stream, rn);
}

}  // namespace zq
