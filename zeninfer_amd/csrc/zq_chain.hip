// zq_chain.hip -- chained decode GEMV: a whole sequence of Q8_0 / Q4_0
// projections (the stages of a decode step) in ONE persistent launch.
//
// Why: a single GEMV launch of a decode-sized projection loses several us to
// fixed costs -- the launch/drain floor of a stream, the first weight bytes'
// latency and the tail of its last row block -- against ~9 us of streaming
// for a 62 MB matrix.  Weight loads do not depend on the activation vector,
// so in one persistent kernel every workgroup keeps the loads of its next row
// blocks -- of this stage or the next ones -- in flight while it waits for
// the next stage's input to exist; the HBM stream does not drain between
// projections.
//
// Program: an array of ChainStage in device memory.  A stage is one
// gemv_batch (up to 8 projections sharing x and cols) whose x is a plain
// vector or the add+RMSNorm of two vectors (the prologue of
// gemv_stream_kernel), and which either stores each projection's rows or,
// for a gate/up pair, stores silu(gate.x) * (up.x).  A stage may wait for an
// earlier stage to complete before it reads x.
//
// Workgroup = 8 compute waves + 1 control wave, one per CU.
//   compute waves: stream weight row blocks through a ring of kDepth blocks
//     in registers (coalesced 16 B loads issued kDepth blocks ahead, across
//     stage boundaries, and waited for explicitly), transpose each block
//     through a per-wave LDS stash to one 68-byte block pair per lane, read
//     that pair's 64 x values from LDS, and leave one partial sum per (row
//     block, wave) in LDS.  They never store to global memory and never wait
//     for a global input, so their load queues only ever hold weights.
//   control wave: for each stage, waits for its dependency and lands x (and
//     the norm operands) in LDS by direct-to-LDS loads; all waves then lay x
//     out in the padded layout (applying the prologue); once the compute
//     waves' partial sums are in, it sums the column slices of each row and
//     stores the outputs.  Its stores are the workgroup's only global stores,
//     so waiting for them (s_waitcnt) does not wait for any weight load.
// Work split and arithmetic per row are those of gemv_stream_kernel with
// R = 1: S column slices of <= 64 block pairs per row, the same per-lane pair
// dot and the same cross-slice sum order, so a plain stage's output equals
// the unchained kernel's bit for bit.
//
// Cross-workgroup protocol (workgroups run on 8 XCDs with private L2s):
//   - outputs (y, the residual r_out) are written with agent-scope relaxed
//     atomic stores (written through to the device-coherent level), and
//     stage inputs are read with the device-scope cache policy (SC1) from
//     the device-coherent level, so no L2 write-back or invalidate is needed;
//   - after its last output of stage s the control wave waits for its
//     stores to complete (workgroup-scope release: s_waitcnt) and adds 1 to
//     counters[s] (agent-scope atomic);
//   - a stage that waits spins (s_sleep between polls) until
//     counters[wait] == gridDim.x.  The spin is bounded: past `spin_limit`
//     polls it sets status[0] = 1 and proceeds, and every spinning
//     workgroup gives up as soon as status[0] != 0, so the grid always
//     drains (results are then invalid and the caller resets);
//   - the last workgroup to finish the last stage zeroes every counter for
//     the next launch (all others have passed all their waits by then).
// All workgroups must be resident at once: the launcher sizes the grid from
// the occupancy API (one workgroup per CU).
#include "zq_device.hpp"
#include "zq_internal.hpp"
#include "zq_pairs.hpp"

#include <algorithm>

namespace zq {
namespace {

constexpr int kCpolSC1 = 0x10;       // cache-policy bit SC1 (device scope) of gfx940+ memory instructions
constexpr int kCW = 8;               // compute waves per workgroup
constexpr int kNT = (kCW + 1) * 64;  // + one control wave
constexpr int kDepth = 5;            // row blocks in flight per compute wave
constexpr int kNU = 5;               // 16 B loads per lane per row block (a 64-pair Q8_0 slice-row is 272 units)
constexpr uint32_t kMaxCols = 14336;
constexpr uint32_t kMaxPairs = kMaxCols / 64;
constexpr uint32_t kMaxNormCols = 4608;  // a, b and w of the add+RMSNorm share the landing area
constexpr uint32_t kMaxLocal = 64;       // row blocks of one stage per workgroup (partial-sum slots)
typedef __attribute__((address_space(3))) void lds_void;

// LDS map (bytes): X = x of the stage in the padded layout (68 floats per
// 64: lane L reads pair L's floats at a 68-dword stride, conflict-free);
// L = landing area of the operands; SX = per-pair sums of x (Q4_0);
// S = per-compute-wave weight stash; P = partial sums; R = reductions.
constexpr uint32_t kXBytes = kMaxPairs * kPadStride * 4;
constexpr uint32_t kLBytes = kMaxCols * 4;
constexpr uint32_t kSXBytes = kMaxPairs * 2 * 4;
constexpr uint32_t kStashBytes = kNU * 1024;
constexpr uint32_t kOffL = kXBytes, kOffSX = kOffL + kLBytes, kOffS = kOffSX + kSXBytes;
constexpr uint32_t kOffP = kOffS + kCW * kStashBytes, kOffR = kOffP + kMaxLocal * kCW * 4;
constexpr uint32_t kLdsBytes = kOffR + (kCW + 1) * 8;

__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A pointer read from the program, made provably wave-uniform (SGPRs).
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v)), hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return reinterpret_cast<T*>((uint64_t(hi) << 32) | lo);
}
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// The program is read through the constant address space: every field is
// wave-uniform, so it comes in with scalar loads into SGPRs.
typedef const __attribute__((address_space(4))) ChainStage CStage;

// Task owning row block `blk` of a stage (count <= 8, linear scan).
__device__ __forceinline__ int find_stage_task(CStage& st, uint32_t blk) {
    int i = 0;
#pragma unroll
    for (int k = 1; k < kMaxTasks; ++k)
        if (k < st.count && blk >= st.group_start[k]) i = k;
    return i;
}

struct Geo {  // one stage's geometry for one compute wave
    uint32_t pairs, S, W, p0, np, nunits, rb, teams;
    int team, slice;
};
__device__ __forceinline__ Geo geometry(CStage& st, int wave, int DW) {
    Geo g;
    g.pairs = uniform(st.cols) >> 6;
    g.S = uniform(st.S);           // 1, 2 or 4
    const uint32_t ls = g.S >> 1;  // log2(S)
    g.teams = uint32_t(kCW) >> ls;
    g.team = wave >> ls;
    g.slice = wave & int(g.S - 1);
    g.W = min(64u, (((g.pairs + g.S - 1) >> ls) + 3u) & ~3u);
    g.p0 = g.slice * g.W;
    g.np = g.p0 < g.pairs ? min(g.W, g.pairs - g.p0) : 0u;
    g.nunits = g.np * DW / 4;
    g.rb = g.pairs * DW * 4;
    return g;
}

// `n` floats from global `src` into LDS at `dst`, 1 KiB per instruction
// straight from memory (no VGPRs).  Vectors produced inside the launch are
// read with the device-scope policy (cpol = kCpolSC1); vectors that exist
// before it (cpol = 0) may come from this XCD's L2.
template <int CPOL>
__device__ __forceinline__ void dma_floats(uint8_t* lds_base, uint32_t dst_off, const float* src, uint32_t n, int lane) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), 0, int(n * 4), 0x00020000);
    const uint32_t chunks = (n * 4 + 1023) / 1024;
    for (uint32_t c = 0; c < chunks; ++c)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(lds_base + dst_off + c * 1024), 16, uint32_t(lane) * 16,
                                                 c * 1024, 0, CPOL);
}

template <int FMT>
__global__ __launch_bounds__(kNT) void gemv_chain_kernel(const ChainStage* __restrict__ prog, uint32_t nstages,
                                                          uint32_t* counters, uint32_t* status, uint32_t spin_limit) {
    constexpr int DW = FMT == kQ8_0 ? 17 : 9;
    extern __shared__ __align__(16) uint8_t lds[];
    float* X = reinterpret_cast<float*>(lds);
    float* Lf = reinterpret_cast<float*>(lds + kOffL);
    float* SX = reinterpret_cast<float*>(lds + kOffSX);
    float* P = reinterpret_cast<float*>(lds + kOffP);
    double* RD = reinterpret_cast<double*>(lds + kOffR);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t grid = gridDim.x;
    CStage* cprog = (CStage*)prog;
    auto has_blocks = [&](uint32_t cs) { return blockIdx.x < uniform(cprog[cs].total_blocks); };

    // x of stage cs into X, by every wave of the workgroup once the control
    // wave has landed the operands in L: a plain copy, or v = a + b,
    // x = v * inv * w with inv = 1/sqrtf(float(ss/n) + eps) and the sum of
    // squares in double (rmsnorm_kernel's arithmetic); then, for Q4_0, the
    // per-pair sums of x.
    auto lay_out_x = [&](CStage& st) {
        const int kind = uniform(st.kind);
        const uint32_t cols = uniform(st.cols), n4 = cols >> 2;
        if (kind == kAddNorm) {
            const bool has_b = uniform_ptr(st.b) != nullptr;
            double ss = 0.0;
            for (uint32_t i = threadIdx.x; i < n4; i += kNT) {
                float4 v = reinterpret_cast<const float4*>(Lf)[i];
                if (has_b) {
                    const float4 b4 = reinterpret_cast<const float4*>(Lf + cols)[i];
                    v = make_float4(v.x + b4.x, v.y + b4.y, v.z + b4.z, v.w + b4.w);
                    reinterpret_cast<float4*>(Lf)[i] = v;  // v, for the second pass and r_out
                }
                ss += double(v.x) * double(v.x);
                ss += double(v.y) * double(v.y);
                ss += double(v.z) * double(v.z);
                ss += double(v.w) * double(v.w);
            }
            ss = wave_sum(ss);
            if (lane == 0) RD[wave] = ss;
            __syncthreads();
            double tot = 0.0;
#pragma unroll
            for (int i = 0; i <= kCW; ++i) tot += RD[i];
            const float eps = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, st.eps)));
            const float inv = 1.0f / sqrtf(float(tot / double(cols)) + eps);
            const float4* w4 = reinterpret_cast<const float4*>(Lf + 2 * cols);
            for (uint32_t i = threadIdx.x; i < n4; i += kNT) {
                const float4 v = reinterpret_cast<const float4*>(Lf)[i], w = w4[i];
                *reinterpret_cast<float4*>(X + (i >> 4) * kPadStride + ((i & 15u) << 2)) =
                    make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
            }
            // the residual v: workgroup 0's control wave (the only wave that
            // stores to global memory) writes all of it
            float* r_out = uniform_ptr(st.r_out);
            if (r_out && blockIdx.x == 0 && wave == kCW)
                for (uint32_t i = lane; i < cols; i += 64) coherent_store(r_out + i, Lf[i]);
        } else {
            for (uint32_t i = threadIdx.x; i < n4; i += kNT)
                *reinterpret_cast<float4*>(X + (i >> 4) * kPadStride + ((i & 15u) << 2)) =
                    reinterpret_cast<const float4*>(Lf)[i];
        }
        if constexpr (FMT == kQ4_0) {
            __syncthreads();
            for (uint32_t p = threadIdx.x; p < (cols >> 6); p += kNT) {
                const float* xp = X + p * kPadStride;
                float s0 = 0.0f, s1 = 0.0f;
                for (int i = 0; i < 32; ++i) {
                    s0 += xp[i];
                    s1 += xp[32 + i];
                }
                SX[2 * p] = s0;
                SX[2 * p + 1] = s1;
            }
        }
    };

    if (wave == kCW) {
        // ---------------------------------------------------- control wave
        for (uint32_t cs = 0; cs < nstages; ++cs) {
            CStage& st = cprog[cs];
            if (has_blocks(cs)) {
                const int dep = int(uniform(uint32_t(st.wait)));
                const uint32_t cols = uniform(st.cols);
                const bool norm = uniform(st.kind) == kAddNorm;
                if (norm)  // the norm weight exists before the launch: land it while waiting
                    dma_floats<0>(lds, kOffL + 2 * cols * 4, uniform_ptr(st.w), cols, lane);
                if (dep >= 0) {
                    uint32_t polls = 0;
                    while (__hip_atomic_load(&counters[dep], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < grid) {
                        if (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
                        if (++polls > spin_limit) {
                            __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
                if (dep >= 0) dma_floats<kCpolSC1>(lds, kOffL, uniform_ptr(st.a), cols, lane);
                else dma_floats<0>(lds, kOffL, uniform_ptr(st.a), cols, lane);
                if (norm && uniform_ptr(st.b)) {  // b is produced in the launch (a residual) when the stage waits
                    if (dep >= 0) dma_floats<kCpolSC1>(lds, kOffL + cols * 4, uniform_ptr(st.b), cols, lane);
                    else dma_floats<0>(lds, kOffL + cols * 4, uniform_ptr(st.b), cols, lane);
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the landed bytes are in LDS
                __syncthreads();                     // A1: operands landed
                lay_out_x(st);
                __syncthreads();  // A2: x of stage cs is in X
                __syncthreads();  // B: the compute waves' partial sums of stage cs are in P
                // outputs: sum the column slices of each row in slice order, store
                const uint32_t S = uniform(st.S), teams = kCW / S;
                const uint32_t tb = uniform(st.total_blocks);
                const uint32_t nlocal = (tb - blockIdx.x + grid - 1) / grid;
                auto row_sum = [&](uint32_t lb, uint32_t team) {
                    const float* pp = P + lb * kCW + team * S;
                    if (S == 1) return pp[0];
                    float v = 0.0f;
                    for (uint32_t s2 = 0; s2 < S; ++s2) v += pp[s2];
                    return v;
                };
                if (uniform(st.epi) == kEpiSiluPair) {
                    // a block is h = teams/2 rows of gate (teams 0..h-1) and the same rows of up
                    const uint32_t h = teams / 2, rows = uniform(st.t[0].rows);
                    float* f = uniform_ptr(st.t[0].y);
                    for (uint32_t k = lane; k < nlocal * h; k += 64) {
                        const uint32_t lb = k / h, t = k % h;
                        const uint32_t row = (blockIdx.x + lb * grid) * h + t;
                        if (row < rows) {
                            const float gv = row_sum(lb, t), uv = row_sum(lb, h + t);
                            coherent_store(f + row, gv / (1.0f + expf(-gv)) * uv);  // silu_mul_kernel's expression
                        }
                    }
                } else {
                    for (uint32_t k = lane; k < nlocal * teams; k += 64) {
                        const uint32_t lb = k / teams, team = k % teams;
                        const uint32_t blk = blockIdx.x + lb * grid;
                        const int ti = find_stage_task(st, blk);
                        const uint32_t row = (blk - st.group_start[ti]) * teams + team;
                        if (row < st.t[ti].rows) coherent_store(st.t[ti].y + row, row_sum(lb, team));
                    }
                }
            }
            // arrive: this wave's output stores (the only global stores of
            // the workgroup) completed, then one agent-scope add
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) {
                if (cs + 1 < nstages) {  // fire and forget: nothing here needs the old value
                    __hip_atomic_fetch_add(&counters[cs], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    const uint32_t old = __hip_atomic_fetch_add(&counters[cs], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old + 1 == grid)  // last arrival of the last stage: reset for the next launch
                        for (uint32_t i = 0; i < nstages; ++i)
                            __hip_atomic_store(&counters[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        return;
    }

    // -------------------------------------------------------- compute waves
    uint32_t* stash = reinterpret_cast<uint32_t*>(lds + kOffS + wave * kStashBytes);
    // the item after (s, blk) for this workgroup: next row block of s, else
    // the first block of the next stage that has one
    auto advance = [&](uint32_t& s, uint32_t& blk) {
        blk += grid;
        while (s < nstages && blk >= cprog[s].total_blocks) {
            ++s;
            blk = blockIdx.x;
        }
    };
    // loads of item (s, blk); past the last item the same instructions run on
    // an empty range (no memory request, zeros).  Issued as inline asm: the
    // compiler does not track these loads and the ring waits for them
    // explicitly (ring_wait), so kDepth blocks stay in flight together.
    auto load_item = [&](uint32_t s, uint32_t blk, uint4 (&u)[kNU]) {
        const uint8_t* rowp = reinterpret_cast<const uint8_t*>(prog);
        uint32_t bytes = 0;
        if (s < nstages) {
            CStage& st = cprog[s];
            const Geo g = geometry(st, wave, DW);
            const uint8_t* tw;
            uint32_t trows, row;
            if (uniform(st.epi) == kEpiSiluPair) {
                const uint32_t h = g.teams / 2;
                const uint32_t half = uint32_t(g.team) >= h ? 1u : 0u;
                tw = uniform_ptr(st.t[half].w);
                trows = uniform(st.t[half].rows);
                row = blk * h + uint32_t(g.team) - half * h;
            } else {
                const int ti = find_stage_task(st, blk);
                tw = uniform_ptr(st.t[ti].w);
                trows = uniform(st.t[ti].rows);
                row = (blk - st.group_start[ti]) * g.teams + g.team;
            }
            rowp = tw + (size_t)min(row, trows - 1) * g.rb + (size_t)(g.np ? g.p0 : 0) * DW * 4;
            bytes = g.nunits * 16;
        }
        const __amdgpu_buffer_rsrc_t rs = span_rsrc(rowp, bytes);
        const uint32_t off = uint32_t(lane) * 16;
#pragma unroll
        for (int i = 0; i < kNU; ++i)
            asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen nt"  // (the 12-bit immediate offset cannot hold 4096)
                         : "=&v"(u[i])
                         : "v"(off), "s"(rs), "s"(uint32_t(i * 1024))
                         : "memory");
    };
    // the oldest slot's loads are complete; the kDepth - 1 later slots may
    // stay outstanding (loads return in issue order)
    auto ring_wait = [&]() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kDepth - 1) * kNU) : "memory"); };

    uint4 u[kDepth][kNU];
    uint32_t ss[kDepth];
    uint32_t ns = 0, nb = blockIdx.x;
    while (ns < nstages && nb >= cprog[ns].total_blocks) {
        ++ns;
        nb = blockIdx.x;
    }
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        ss[d] = ns;
        load_item(ns, nb, u[d]);
        if (ns < nstages) advance(ns, nb);
    }
    uint32_t cur = nstages, lb = 0;
    Geo g{};
    bool active = false;
    auto enter = [&](uint32_t cs) {
        if (cur < nstages) __syncthreads();  // B of the previous stage
        cur = cs;
        lb = 0;
        __syncthreads();  // A1: operands landed
        lay_out_x(cprog[cs]);
        __syncthreads();  // A2: x of stage cs is in X
        g = geometry(cprog[cs], wave, DW);
        active = uint32_t(lane) < g.np;
    };
    // one row block from ring slot d (a compile-time index)
    auto step = [&](auto dc) -> bool {
        constexpr int d = decltype(dc)::value;
        const uint32_t s = ss[d];
        if (s >= nstages) return false;
        if (s != cur) enter(s);
        ring_wait();
#pragma unroll
        for (int i = 0; i < kNU; ++i)  // lanes past the slice-row write zeros into the stash's padding
            reinterpret_cast<uint4*>(stash)[lane + 64 * i] = u[d][i];
        ss[d] = ns;
        load_item(ns, nb, u[d]);  // the item kDepth ahead, possibly of a later stage
        if (ns < nstages) advance(ns, nb);
        uint32_t q[DW];
#pragma unroll
        for (int j = 0; j < DW; ++j) q[j] = active ? stash[DW * lane + j] : 0u;
        const uint32_t pr = active ? g.p0 + lane : 0u;
        const float* xp = X + pr * kPadStride;
        float acc;
        if constexpr (FMT == kQ8_0) acc = q8_pair_dot_lds(q, xp);
        else acc = q4_pair_dot_mix_lds(q, xp, SX[2 * pr], SX[2 * pr + 1]);
        acc = wave_sum(acc);
        if (lane == 0) P[lb * kCW + wave] = acc;
        ++lb;
        return true;
    };
    static_assert(kDepth == 5, "the ring below is unrolled for kDepth slots");
    while (true) {
        if (!step(std::integral_constant<int, 0>{})) break;
        if (!step(std::integral_constant<int, 1>{})) break;
        if (!step(std::integral_constant<int, 2>{})) break;
        if (!step(std::integral_constant<int, 3>{})) break;
        if (!step(std::integral_constant<int, 4>{})) break;
    }
    if (cur < nstages) __syncthreads();  // B of the last stage this workgroup computed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring's trailing (empty) loads
}

}  // namespace

// One workgroup per CU, all resident together (checked with the occupancy
// API: a workgroup must fit each CU at least once); 0 when it cannot.
uint32_t chain_grid(int fmt) {
    int per_cu = 0;
    const hipError_t e =
        fmt == kQ8_0 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_chain_kernel<kQ8_0>, kNT, kLdsBytes)
                     : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_chain_kernel<kQ4_0>, kNT, kLdsBytes);
    if (e != hipSuccess || per_cu < 1) return 0;
    return uint32_t(device_cu_count());
}

size_t chain_lds_bytes(int) { return kLdsBytes; }

hipError_t launch_gemv_chain(int fmt, const ChainStage* prog, uint32_t nstages, uint32_t* counters, uint32_t* status,
                             uint32_t spin_limit, hipStream_t stream) {
    if (!prog || !nstages || !counters || !status || (fmt != kQ8_0 && fmt != kQ4_0)) return hipErrorInvalidValue;
    const uint32_t grid = chain_grid(fmt);
    if (!grid) return hipErrorInvalidConfiguration;
    if (fmt == kQ8_0)
        hipLaunchKernelGGL(gemv_chain_kernel<kQ8_0>, dim3(grid), dim3(kNT), kLdsBytes, stream, prog, nstages, counters,
                           status, spin_limit);
    else
        hipLaunchKernelGGL(gemv_chain_kernel<kQ4_0>, dim3(grid), dim3(kNT), kLdsBytes, stream, prog, nstages, counters,
                           status, spin_limit);
    return hipGetLastError();
}

namespace {
__global__ void chain_reset_kernel(uint32_t* counters, uint32_t n, uint32_t* status) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) counters[i] = 0u;
    if (threadIdx.x == 0) status[0] = 0u;
}
}  // namespace

hipError_t launch_chain_reset(uint32_t* counters, uint32_t nstages, uint32_t* status, hipStream_t stream) {
    if (!counters || !status) return hipErrorInvalidValue;
    hipLaunchKernelGGL(chain_reset_kernel, dim3(1), dim3(256), 0, stream, counters, nstages, status);
    return hipGetLastError();
}

hipError_t chain_stage_prepare(int fmt, ChainStage& st, uint32_t index) {
    if (fmt != kQ8_0 && fmt != kQ4_0) return hipErrorInvalidConfiguration;
    if (st.count < 1 || st.count > kMaxTasks || !st.a || !row_bytes(fmt, st.cols)) return hipErrorInvalidValue;
    if (st.cols % 256 || st.cols > kMaxCols) return hipErrorInvalidConfiguration;
    if (st.kind == kSiluMul) return hipErrorInvalidConfiguration;  // as a gate/up epilogue instead (kEpiSiluPair)
    if (st.kind != kXPlain && st.kind != kAddNorm) return hipErrorInvalidValue;
    if (st.kind == kAddNorm && !st.w) return hipErrorInvalidValue;
    if (st.kind == kAddNorm && st.cols > kMaxNormCols) return hipErrorInvalidConfiguration;
    if (st.epi != kEpiStore && st.epi != kEpiSiluPair) return hipErrorInvalidValue;
    if (st.wait >= int32_t(index) || st.wait < -1) return hipErrorInvalidValue;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!a16(st.a) || !a16(st.b) || !a16(st.w) || !a16(st.r_out)) return hipErrorInvalidConfiguration;
    const uint32_t pairs = st.cols >> 6;
    st.S = pairs <= 64 ? 1u : pairs <= 128 ? 2u : 4u;
    const uint32_t teams = uint32_t(kCW) / st.S;
    for (int i = 0; i < st.count; ++i) {
        if (!st.t[i].w || !st.t[i].rows) return hipErrorInvalidValue;
        if (!st.t[i].y && !(st.epi == kEpiSiluPair && i == 1)) return hipErrorInvalidValue;
        if (!a16(st.t[i].w)) return hipErrorInvalidConfiguration;
    }
    uint32_t blocks = 0;
    if (st.epi == kEpiSiluPair) {
        if (st.count != 2 || st.t[0].rows != st.t[1].rows) return hipErrorInvalidValue;
        const uint32_t h = teams / 2;
        blocks = (st.t[0].rows + h - 1) / h;
        for (int i = 0; i <= kMaxTasks; ++i) st.group_start[i] = 0;
    } else {
        for (int i = 0; i < st.count; ++i) {
            st.group_start[i] = blocks;
            blocks += (st.t[i].rows + teams - 1) / teams;
        }
        for (int i = st.count; i <= kMaxTasks; ++i) st.group_start[i] = blocks;
    }
    st.total_blocks = blocks;
    const uint32_t grid = chain_grid(fmt);
    if (!grid || (blocks + grid - 1) / grid > kMaxLocal) return hipErrorInvalidConfiguration;
    return hipSuccess;
}

}  // namespace zq
