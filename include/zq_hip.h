/*
 * zq_hip.h -- C ABI of the MI355X (gfx950) block-quantised projection
 * backend: Q8_0 / Q4_0 / Q6_K decode GEMV and quantised prefill GEMM over
 * GGML blocks kept resident in HBM in their native layout.
 *
 * This header contains no HIP or C++ types: plain pointers, sizes and int
 * status codes, so the reference's compiler-agnostic dispatch layer
 * (src/quant.cpp) can call it from any translation unit, the same way it
 * reaches the backend declared in include/zen/hip_backend.h:6-14.
 *
 * Citations are to the ZenInfer reference tree (file:line) whose interface
 * each entry point replaces.  Conventions carried over from that slot:
 *   - nothing throws across this boundary; every call returns a status;
 *   - ZQ_DECLINED means "not taken, run your CPU route", exactly where the
 *     reference's zen::hip::* returned false and quant.cpp fell through
 *     (src/quant.cpp:1007-1012, 1656-1659);
 *   - host-pointer entry points are synchronous and key device residency by
 *     the weight pointer plus (format, rows, cols) (hip_backend.h:52-58): a
 *     tensor must keep its host address and bytes for as long as it is used;
 *     a reused address with a different shape is re-uploaded, with the same
 *     shape it is NOT re-read (call zq_hip_release first);
 *   - one process-wide mutex serialises the host-pointer entry points
 *     (src/backends/hip/hip_backend.hip:232-233); initialisation is lazy,
 *     cached and failure-latched until zq_hip_shutdown (:392-436).
 * The *_dev entry points take device pointers and a hipStream_t (as void*,
 * NULL = the null stream), only enqueue work and never synchronise.
 */
#ifndef ZQ_HIP_H
#define ZQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define ZQ_OK 0
#define ZQ_DECLINED 1          /* valid call the backend does not take: use the CPU route */
#define ZQ_ERR_ARG (-1)        /* invalid arguments: null pointer, bad shape/format, misaligned device operand */
#define ZQ_ERR_NO_DEVICE (-2)  /* no usable gfx950 device / init failed                    */
#define ZQ_ERR_OOM (-3)        /* device or host allocation failed                         */
#define ZQ_ERR_HIP (-4)        /* a HIP runtime call or kernel launch failed               */
#define ZQ_ERR_TOO_LARGE (-5)  /* the call needs more than the fixed no-allocation scratch */

/* ---- weight formats: GGML type ids (src/gguf.cpp:370-393) ---------------- */
#define ZQ_FMT_Q4_0 2   /* 32 el / 18 B: fp16 d + 16 B nibbles   (src/quant.cpp:253)  */
#define ZQ_FMT_Q8_0 8   /* 32 el / 34 B: fp16 d + 32 int8        (src/quant.cpp:257)  */
#define ZQ_FMT_Q4_K 12  /* 256 el / 144 B super-block            (src/quant.cpp:273)  */
#define ZQ_FMT_Q5_K 13  /* 256 el / 176 B super-block            (src/quant.cpp:274)  */
#define ZQ_FMT_Q6_K 14  /* 256 el / 210 B super-block            (src/quant.cpp:259)  */

/* ---- GEMM activation handling -------------------------------------------- */
#define ZQ_ACT_DEFAULT 0 /* fp32 for every format: the arithmetic of the functions this
                            slot replaces (quant::gemm, src/quant.cpp:1613-1777, and
                            zen::hip::gemm_q8_0, hip_backend.hip:127-177); the reference
                            keeps int8 activations opt-in (quant.cpp:1083-1091) */
#define ZQ_ACT_INT8 1    /* per-32 int8 activations, kernels/avx2.cpp:502-524 quantiser: the
                            D3D12 prefill route's arithmetic (d3d12_backend.cpp:845-854);
                            Q8_0 / Q4_0 only */
#define ZQ_ACT_F32 2     /* fp32 activations, the reference CPU GEMM arithmetic          */

/* Bytes of slack every device weight buffer must carry past its last block
 * (the library's own uploads always do; see zq_weight_bytes). */
#define ZQ_WEIGHT_TAIL_PAD 64

/* Adapter description.  Replaces zen::hip::AdapterInfo (include/zen/hip_backend.h:17-24). */
typedef struct zq_hip_info {
    char name[128];
    char arch[64];           /* gcnArchName, e.g. gfx950:sramecc+:xnack- */
    uint64_t vram_bytes;
    int compute_units;
    int wave_size;
    int lds_per_block;
    int clock_khz;
    int mem_clock_khz;
    int mem_bus_width;
} zq_hip_info;

/* Counters.  Replaces zen::hip::Stats (include/zen/hip_backend.h:25-41). */
typedef struct zq_hip_stats {
    uint64_t dispatches;      /* kernels launched                        */
    uint64_t submits;         /* host-pointer calls that ran on the GPU  */
    uint64_t batches;         /* batched GEMV submissions                */
    uint64_t uploads;         /* weight tensors uploaded                 */
    uint64_t upload_bytes;
    uint64_t resident_bytes;  /* currently resident weight bytes         */
    uint64_t resident_tensors;
    uint64_t evictions;
    uint64_t declined;        /* calls answered ZQ_DECLINED              */
    uint64_t errors;
    uint64_t upload_us;       /* weight copies to the device             */
    uint64_t transfer_us;     /* activation H2D + output D2H, host clock */
    uint64_t wait_us;         /* stream synchronisation                  */
    uint64_t fallbacks;       /* host calls after init that returned non-OK (the caller
                                 ran its CPU route), Stats::fallbacks         */
    uint64_t alloc_us;        /* device/pinned allocation, Stats::alloc_us    */
    uint64_t launch_us;       /* kernel enqueue, Stats::launch_us             */
    uint64_t readback_us;     /* output D2H + copy out, Stats::readback_us    */
    uint64_t gpu_us;          /* event-timed kernels of host calls; only with
                                 ZEN_HIP_TRACE=1 (hip_backend.hip:889-891)    */
} zq_hip_stats;

/* One projection of a batched GEMV.  Replaces zen::hip::GemvTask
 * (include/zen/hip_backend.h:62-71) without its `columns` field: every task
 * of a batch shares x, so cols is one argument of the batch call (the
 * reference's quant::gemv_batch also takes a single `columns`,
 * include/zen/quant.h:71-74). */
typedef struct zq_gemv_task {
    const uint8_t* weights;  /* host pointer (zq_hip_gemv_batch) or device pointer (_dev) */
    float* y;
    size_t rows;
} zq_gemv_task;
#define ZQ_MAX_BATCH 8       /* zen::hip::kMaxBatch (include/zen/hip_backend.h:72) */

/* One projection of a batched GEMM: all tasks share X, tokens and cols.
 * Replaces one (weights[i], outputs[i], rows[i]) triple of quant::gemm_batch
 * (include/zen/quant.h:77-84). */
typedef struct zq_gemm_task {
    const uint8_t* weights;  /* host pointer (zq_hip_gemm_batch) or device pointer (_dev) */
    float* Y;                /* [tokens x rows], token-major */
    size_t rows;
} zq_gemm_task;

/* ---- lifecycle (include/zen/hip_backend.h:46-50) -------------------------- */
/* 1 when ZEN_BACKEND is hip|rocm|amd or ZEN_HIP=1 (hip_backend.hip:266-282). */
int zq_hip_opted_in(void);
/* Lazy, cached, failure-latched init of device 0 (zen::hip::init). */
int zq_hip_init(void);
/* 1 when opted in and a usable device initialised (zen::hip::enabled). */
int zq_hip_enabled(void);
/* Frees residency and staging, clears the failure latch (zen::hip::shutdown). */
void zq_hip_shutdown(void);
int zq_hip_get_info(zq_hip_info* out);          /* zen::hip::info  */
int zq_hip_get_stats(zq_hip_stats* out);        /* zen::hip::stats */
void zq_hip_reset_stats(void);
const char* zq_hip_status_string(int status);

/* ---- layout helpers (src/quant.cpp:894-943) ------------------------------- */
size_t zq_row_bytes(int fmt, size_t cols);                 /* 0 if cols is not block-aligned */
size_t zq_weight_bytes(int fmt, size_t rows, size_t cols); /* rows*row_bytes + ZQ_WEIGHT_TAIL_PAD */
/* Host-pointer calls with rows*cols below this many elements are declined so
 * the CPU keeps tiny projections (hip_backend.hip:49, 939); default 262144,
 * env ZEN_HIP_MIN_ELEMENTS.  Returns the previous value. */
size_t zq_hip_set_min_elements(size_t elements);

/* ---- host-pointer projections (synchronous) ------------------------------ */
/* y[rows] = W[rows x cols] . x[cols], fp32 activations.
 * Replaces zen::hip::gemv_q8_0 (include/zen/hip_backend.h:59-60), called from
 * quant::gemv (src/quant.cpp:1007-1012), for Q8_0, Q4_0 and Q6_K. */
int zq_hip_gemv(int fmt, const uint8_t* weights, const float* x, float* y, size_t rows, size_t cols);
/* Several projections sharing x, one submission.  Replaces
 * zen::hip::gemv_q8_0_batch (include/zen/hip_backend.h:74), called from
 * quant::gemv_batch (src/quant.cpp:1457-1467). */
int zq_hip_gemv_batch(int fmt, const float* x, const zq_gemv_task* tasks, size_t count, size_t cols);
/* Y[tokens x rows] = X[tokens x cols] . W^T, token-major.  Replaces
 * zen::hip::gemm_q8_0 (include/zen/hip_backend.h:61-62), called from
 * quant::gemm (src/quant.cpp:1656-1659). */
int zq_hip_gemm(int fmt, const uint8_t* weights, const float* X, float* Y, size_t tokens, size_t rows,
                size_t cols, int act_mode);
/* Several GEMMs sharing X (prefill Q|K|V, gate|up), one submission; with
 * int8 activations X is quantised once for all tasks.  Replaces
 * quant::gemm_batch (include/zen/quant.h:77-84, src/quant.cpp:1521-1554),
 * whose GPU route is the D3D12 gemm_q8_0_batch. */
int zq_hip_gemm_batch(int fmt, const float* X, const zq_gemm_task* tasks, size_t count, size_t tokens, size_t cols,
                      int act_mode);
/* gate|up -> SiLU(gate)*up -> down with the FFN activation kept on the
 * device.  Replaces zen::hip::gemv_q8_0_ffn (include/zen/hip_backend.h:80-82),
 * called from quant::ffn_gemv (src/quant.cpp:1566-1571). */
int zq_hip_ffn_gemv(int fmt, const uint8_t* gate, const uint8_t* up, const uint8_t* down, const float* x,
                    float* y, size_t ffn_rows, size_t cols, size_t out_rows);
/* y[r] = rmsnorm(x[r]) * weight for rows of cols floats: sum of squares in
 * double, inv = 1/sqrtf(float(ss/cols) + eps), y = x*inv*w -- the reference
 * CPU rms_norm (src/adapters/dense_transformer_runtime.cpp:117-124).
 * Replaces zen::hip::rms_norm (include/zen/hip_backend.h:77-78,
 * src/backends/hip/hip_backend.hip:990-1001). */
int zq_hip_rms_norm(const float* x, const float* weight, float* y, size_t rows, size_t cols, float eps);
/* The FFN half of a decoder layer in one submission, every intermediate on
 * the device:  t0 = Wo.attn_out; h1 = t0 + x; h2 = rmsnorm(h1)*norm_weight;
 * f = silu(Wg.h2) * (Wu.h2); out = h1 + Wd.f.  Wo is [hidden x attn_width],
 * Wg/Wu [ffn_rows x hidden], Wd [hidden x ffn_rows], all of format fmt
 * (other mixes are declined to the caller's separate operations).  out may
 * alias x.  Replaces quant::ffn_residual_fused (include/zen/quant.h:97-106,
 * src/quant.cpp:1580-1612), whose GPU route is the D3D12 one
 * (include/zen/d3d12_backend.h:352-364). */
int zq_hip_ffn_residual_fused(int fmt, const uint8_t* attn_output, const uint8_t* gate, const uint8_t* up,
                              const uint8_t* down, const float* norm_weight, const float* x, const float* attn_out,
                              float* out, size_t hidden, size_t attn_width, size_t ffn_rows, float eps);
/* Drops the device copy of one weight tensor (the D3D12 slot's
 * release_q8_0_weights, include/zen/d3d12_backend.h:87-91). */
int zq_hip_release(const uint8_t* weights);
int zq_hip_release_all(void);

/* ---- device-pointer projections (asynchronous on `stream`) --------------- */
/* Weight buffers must be readable ZQ_WEIGHT_TAIL_PAD bytes past the last block. */
int zq_hip_gemv_dev(int fmt, const void* weights, const float* x, float* y, size_t rows, size_t cols,
                    void* stream);
int zq_hip_gemv_batch_dev(int fmt, const float* x, const zq_gemv_task* tasks, size_t count, size_t cols,
                          void* stream);
/* Workspace (device bytes) a zq_hip_gemm_dev call needs: int8 activations,
 * their scales and, for small grids, split-K partial sums (ZQ_ACT_INT8);
 * with fp32 activations, the super-block formats' split activations (Q6_K,
 * Q4_K, Q5_K: f16 hi + lo and row scales; they let the GEMM run on the f16
 * MFMA) and split-K partial sums for small grids,
 * else 0 (a smaller or null workspace runs with what fits: the fp32 MFMA,
 * unsplit). */
size_t zq_hip_gemm_workspace_bytes(int fmt, size_t tokens, size_t rows, size_t cols, int act_mode);
int zq_hip_gemm_dev(int fmt, const void* weights, const float* X, float* Y, size_t tokens, size_t rows,
                    size_t cols, int act_mode, void* workspace, size_t workspace_bytes, void* stream);

/* Batched GEMM on the device; workspace as zq_hip_gemm_batch_workspace_bytes
 * (the shared int8 activations and the largest task's split-K partials). */
size_t zq_hip_gemm_batch_workspace_bytes(int fmt, const zq_gemm_task* tasks, size_t count, size_t tokens, size_t cols,
                                         int act_mode);
int zq_hip_gemm_batch_dev(int fmt, const float* X, const zq_gemm_task* tasks, size_t count, size_t tokens, size_t cols,
                          int act_mode, void* workspace, size_t workspace_bytes, void* stream);
int zq_hip_rms_norm_dev(const float* x, const float* weight, float* y, size_t rows, size_t cols, float eps,
                        void* stream);
/* zq_hip_ffn_residual_fused on device pointers; workspace holds
 * zq_hip_ffn_residual_workspace_bytes(hidden, ffn_rows) bytes. */
size_t zq_hip_ffn_residual_workspace_bytes(size_t hidden, size_t ffn_rows);
int zq_hip_ffn_residual_fused_dev(int fmt, const void* attn_output, const void* gate, const void* up, const void* down,
                                  const float* norm_weight, const float* x, const float* attn_out, float* out,
                                  size_t hidden, size_t attn_width, size_t ffn_rows, float eps, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* zq_hip_gemm_dev without a workspace and without any allocation: the
 * quantised activations, scales and split-K partials live in a fixed
 * file-scope device array (zq_hip_noalloc_scratch_bytes(), 64 MiB) that each
 * GPU holds for the life of the process.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Calls whose
 * workspace (zq_hip_gemm_workspace_bytes) exceeds the scratch return
 * ZQ_ERR_TOO_LARGE before any launch or memory operation.  Every call on a GPU shares
 * that GPU's scratch: calls that overlap on one GPU (two streams, two
 * threads) race; calls in one stream are ordered and safe.  Nothing in the
 * scratch needs to start at zero (each call writes what it reads). */
size_t zq_hip_noalloc_scratch_bytes(void);
int zq_hip_gemm_dev_noalloc(int fmt, const void* weights, const float* X, float* Y, size_t tokens, size_t rows,
                            size_t cols, int act_mode, void* stream);

/* ---- bit-exact tier hooks (device pointers, asynchronous) ---------------- */
/* Per-32 activation quantiser, kernels/avx2.cpp:502-524: xq[tokens*cols],
 * xs[tokens*cols/32]. */
int zq_hip_quantize_acts_dev(const float* X, int8_t* xq, float* xs, size_t tokens, size_t cols, void* stream);
/* Per-block int32 dots of the int8 GEMM, taken from its MFMA results:
 * out[(t*rows + r)*(cols/32) + b].  Q8_0 and Q4_0. */
int zq_hip_block_dots_dev(int fmt, const void* weights, const int8_t* xq, int32_t* out, size_t tokens,
                          size_t rows, size_t cols, void* stream);
/* Dequantised weights, row-major fp32 (src/quant.cpp:391-416, 500-517). */
int zq_hip_dequantize_dev(int fmt, const void* weights, float* out, size_t rows, size_t cols, void* stream);

/* ---- measurement helper --------------------------------------------------- */
/* The int8 MFMA peak of this device from measurement: every CU runs
 * v_mfma_i32_32x32x32_i8 back to back on all four SIMDs; sclk is the shader
 * clock measured against the 100 MHz constant clock during that run, and
 * int8_tops = CUs x 4 SIMDs x 65536 ops / cycles_per_mfma x sclk.  No
 * counterpart in the reference (roofline reporting). */
int zq_hip_mfma_peak(double* sclk_mhz, double* cycles_per_mfma, double* int8_tops);
/* The streaming-read yardstick of the GEMV rooflines: enqueues one kernel
 * that reads `bytes` of device memory at `buf` (16 B aligned, a multiple of
 * 16) once, with the GEMVs' non-temporal 16-byte loads and nothing else, on
 * `stream`.  `sink` is device memory of zq_hip_read_probe_sink_bytes()
 * bytes.  Timed by the caller (events around back-to-back launches), it is
 * the practical ceiling of one launch that must read those bytes.  No
 * counterpart in the reference (roofline reporting). */
int zq_hip_read_probe_dev(const void* buf, size_t bytes, void* sink, void* stream);
size_t zq_hip_read_probe_sink_bytes(void);

/* ---- synthetic inputs on the device (bench workloads) -------------------- */
int zq_hip_synth_weights_dev(int fmt, uint64_t seed, void* weights, size_t rows, size_t cols, void* stream);
int zq_hip_synth_normal_dev(uint64_t seed, float* out, size_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ZQ_HIP_H */
