// zq_internal.hpp -- launch interface between the C-ABI runtime (zq_backend.hip)
// and the kernel translation units.  Host-only declarations; no HIP types
// beyond hipStream_t / hipError_t cross this header.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace zq {

// One projection of a batched decode GEMV: all tasks share the input vector
// and the column count (the Q|K|V and gate|up pattern).
struct GemvTask {
    const uint8_t* w;  // device pointer, native GGML blocks, row-major
    float* y;          // device pointer, rows floats
    uint32_t rows;
};
constexpr int kMaxTasks = 8;

// Row bytes of one GGML row (0 when cols does not divide into blocks).
size_t row_bytes(int fmt, size_t cols);

// Decode GEMV with fp32 activations: y_i = W_i . x for every task.
hipError_t launch_gemv(int fmt, const GemvTask* tasks, int count, const float* x,
                       size_t cols, hipStream_t stream);

// The producer of a decode GEMV's input folded into the GEMV itself (every
// workgroup recomputes it while staging x):
//   kSiluMul   x = silu(a) * b, elementwise as launch_silu_mul
//   kAddNorm   v = a + b (b may be null), x = rmsnorm(v) * w as
//              launch_add_rmsnorm; r_out (may be null) receives v, written by
//              workgroup 0 only, so it must not alias a or b.
struct XPrologue {
    int kind;
    const float* a;
    const float* b;
    const float* w;
    float* r_out;
    float eps;
};
constexpr int kXPlain = 0, kSiluMul = 1, kAddNorm = 2;
// Q8_0 / Q4_0 only, on the streaming kernel's shapes (cols % 256 == 0,
// cols <= 16384, 16-byte aligned operands); hipErrorInvalidConfiguration
// when the shape or format is not covered, so the caller runs the unfused
// kernels instead.
hipError_t launch_gemv_prologue(int fmt, const GemvTask* tasks, int count, const XPrologue& pro, size_t cols,
                                hipStream_t stream);
// gate|up with the add+RMSNorm prologue that stores f = silu(gate.x) *
// (up.x) into gate.y (up.y unused): Q8_0 / Q4_0, cols % 256 == 0 and
// cols <= 4096, equal rows; hipErrorInvalidConfiguration otherwise.
hipError_t launch_gemv_prologue_silu_pair(int fmt, const GemvTask& gate, const GemvTask& up, const XPrologue& pro,
                                          size_t cols, hipStream_t stream);
// The decode residual stream carried between K-quant GEMVs without RMSNorm
// launches.  An add-out GEMV adds each output row into the residual (y is
// the residual: y_i += W_i . x), adds the new values' squares (in double)
// into kRnSlots accumulator slots (ss_out, workgroup g into slot g %
// kRnSlots) and clears the slots of ss_zero.  A norm-in GEMV takes x = the
// residual and uses x * inv * w with inv = 1/sqrtf(float(ss/cols) + eps), ss
// the slots of ss_in summed in slot order -- the RMSNorm kernel's formula.
struct ResidNorm {
    const double* ss_in;
    const float* w;
    double* ss_out;
    double* ss_zero;
    float eps;
};
constexpr int kRnNone = 0, kRnNormIn = 1, kRnAddOut = 2;
constexpr int kRnSlots = 64;  // one per lane of the reading wave
// Q4_K / Q5_K, cols % 256 == 0, cols <= 16384, 16-byte aligned x, weights and
// norm weight; hipErrorInvalidConfiguration otherwise.
hipError_t launch_gemv_resid(int fmt, int mode, const GemvTask* tasks, int count, const float* x, size_t cols,
                             const ResidNorm& rn, hipStream_t stream);
bool gemv_resid_supported(int fmt, size_t cols);

// gate|up over a plain x that stores f = silu(gate.x) * (up.x) into gate.y
// (up.y unused): Q4_K / Q5_K, and Q6_K with cols % 2048 == 0; cols <= 16384,
// equal rows, 16-byte aligned x and weights; hipErrorInvalidConfiguration
// otherwise.
// With rn (Q4_K / Q5_K only), x is the residual and is normalised as a
// norm-in GEMV's.
hipError_t launch_gemv_silu_pair(int fmt, const GemvTask& gate, const GemvTask& up, const float* x, size_t cols,
                                 hipStream_t stream, const ResidNorm* rn = nullptr);

// Per-32-element activation quantiser (int8 + fp32 scale per block).
hipError_t launch_quantize_acts(const float* X, int8_t* xq, float* xs, size_t M, size_t K,
                                hipStream_t stream);

// Prefill GEMM on int8 activations already quantised by launch_quantize_acts.
// Y is token-major [M][N].  `partial` (gemm_i8_partial_bytes, may be 0) is
// the split-K workspace; with partial == nullptr the GEMM runs unsplit.
size_t gemm_i8_partial_bytes(size_t M, size_t N, size_t K);
// Compute units of the current device (256 on MI355X; 256 if the query fails).
int device_cu_count();
// splits (optional): the split-K reduction is left to the caller, which gets
// the split count; with more than one, Y is untouched and the partial planes
// (partial + s * M * N, s < splits) are to be summed in split order.
hipError_t launch_gemm_i8(int fmt, const uint8_t* w, const int8_t* xq, const float* xs,
                          float* Y, float* partial, size_t M, size_t N, size_t K, hipStream_t stream,
                          uint32_t* splits = nullptr);
// Y[M][N] = the sum of `splits` partial planes in split order (the reduction
// launch_gemm_i8 leaves to its caller when asked to).
hipError_t launch_splitk_reduce(const float* partial, float* Y, size_t M, size_t N, uint32_t splits, hipStream_t stream);

// Prefill GEMM on fp32 activations (the reference CPU arithmetic).  `ws`
// (ws_bytes, may be null) is the workspace: gemm_f32_workspace_bytes() lets
// Q6_K run on the f16 MFMA (split activations) and any format split K; with
// less the GEMM runs with what fits (fp32 MFMA, unsplit).  `launches`
// (optional) receives the number of kernels enqueued.
size_t gemm_f32_partial_bytes(size_t M, size_t N, size_t K);
size_t gemm_f32_workspace_bytes(int fmt, size_t M, size_t N, size_t K);
hipError_t launch_gemm_f32(int fmt, const uint8_t* w, const float* X, float* Y, void* ws, size_t ws_bytes, size_t M,
                           size_t N, size_t K, hipStream_t stream, uint32_t* launches = nullptr);

// Bit-exact tier helpers.
hipError_t launch_dequantize(int fmt, const uint8_t* w, float* out, size_t rows, size_t cols,
                             hipStream_t stream);
hipError_t launch_block_dots(int fmt, const uint8_t* w, const int8_t* xq, int32_t* out,
                             size_t M, size_t N, size_t K, hipStream_t stream);

// Int8 MFMA rate probe (one 4-wave workgroup per CU): out[4*wg] shader
// cycles and out[4*wg+1] 100 MHz ticks of iters x 4 MFMAs per wave.
hipError_t launch_mfma_probe(uint64_t* out, uint32_t wgs, uint32_t iters, hipStream_t stream);
// Streaming read of `bytes` (16 B aligned, multiple of 16); `sink` holds
// read_probe_sink_bytes().
hipError_t launch_read_probe(const void* buf, size_t bytes, uint32_t* sink, hipStream_t stream);
size_t read_probe_sink_bytes();

// Synthetic inputs generated on the device (bench workloads).
hipError_t launch_synth_weights(int fmt, uint64_t seed, uint8_t* w, size_t rows, size_t cols,
                                hipStream_t stream);
hipError_t launch_synth_normal(uint64_t seed, float* out, size_t n, hipStream_t stream);

}  // namespace zq

namespace zq {
// Decoder-layer kernels (zq_layer.hip).  Token ids and the first position are
// read from device memory, so a captured decode step replays unchanged.
hipError_t launch_embed(int fmt, const void* table, const uint32_t* tokens, uint32_t vocab, float* x, uint32_t E,
                        uint32_t T, hipStream_t stream);
// xq/xs (optional, n % 32 == 0): y's int8 activations and scales as
// launch_quantize_acts would write them, for the int8 GEMMs that read y.
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, uint32_t rows, uint32_t n, float eps,
                          hipStream_t stream, int8_t* xq = nullptr, float* xs = nullptr);
// q is rotated in place ([T][H*D]), and k, v ([T][KH*D]) go to the caches.
// With ld != 0 the inputs are rows of one [T][ld] buffer (the fused Q|K|V
// projection's output): q_in, k and v point at its q, k and v columns, and
// the rotated q is written to q ([T][H*D]).
hipError_t launch_rope_kv(float* q, const float* k, const float* v, float* kc, float* vc, const float* cos_tab,
                          const float* sin_tab, const uint32_t* pos0, uint32_t T, uint32_t H, uint32_t KH, uint32_t D,
                          uint32_t pairs, bool adjacent, hipStream_t stream, uint32_t ld = 0,
                          const float* q_in = nullptr, uint32_t splits = 1, float* reduce_to = nullptr);
// xq / xs (optional, with `quantized`): the output's int8 activations and
// block scales instead of out, when the kernel taken supports it (*quantized
// then true; else out is written as usual).
hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, const uint32_t* pos0,
                            uint32_t T, uint32_t H, uint32_t KH, uint32_t D, uint32_t max_pos, float scale,
                            hipStream_t stream, int8_t* xq = nullptr, float* xs = nullptr, bool* quantized = nullptr);
// Decode attention split over 32-position chunks, the last chunk of each kv
// head merging; `part` holds attention_decode_partial_floats(H, D, max_pos)
// floats and must be zero when first used (its tail holds arrival counters
// that the kernel leaves at zero).
size_t attention_decode_partial_floats(uint32_t H, uint32_t D, uint32_t max_pos);
// RoPE (adjacent pairs) of q and the new key, the KV append at *pos and the
// attention of the one query token, fused.
hipError_t launch_attention_decode(const float* q, const float* knew, const float* vnew, float* kc, float* vc,
                                   const float* cos_tab, const float* sin_tab, float* part, float* out,
                                   const uint32_t* pos, uint32_t H, uint32_t KH, uint32_t D, uint32_t pairs,
                                   uint32_t max_pos, float scale, hipStream_t stream);
hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t stream);
// out = x + y elementwise (out may alias x)
hipError_t launch_add_to(const float* x, const float* y, float* out, size_t n, hipStream_t stream);
// x += r, then y = rmsnorm(x) * w (rows of n).  rsplit > 1: r is that many
// [rows][n] planes (a GEMM's split-K partials), summed in split order first.
hipError_t launch_add_rmsnorm(float* x, const float* r, const float* w, float* y, uint32_t rows, uint32_t n, float eps,
                              hipStream_t stream, int8_t* xq = nullptr, float* xs = nullptr, uint32_t rsplit = 1);
// Greedy id over n values; `partial` holds argmax_partial_bytes().
size_t argmax_partial_bytes();
hipError_t launch_argmax(const float* x, uint32_t n, uint32_t* out, void* partial, hipStream_t stream);
hipError_t launch_silu_mul(const float* gate, const float* up, float* out, size_t n, hipStream_t stream,
                           int8_t* xq = nullptr, float* xs = nullptr);
}  // namespace zq
