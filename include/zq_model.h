/*
 * zq_model.h -- C ABI of the device-resident Llama-layout decoder: weights
 * uploaded once into HBM in their native GGML block layout, KV cache and
 * activations kept on the device, projections through the zq_hip kernels
 * (quantised GEMV for decode, int8 or fp32 GEMM for prefill), decode steps
 * replayed as one HIP graph.
 *
 * It replaces the reference's dense runtime for the llama architecture
 * (include/zen/dense_transformer_runtime.h:20-78;
 * src/adapters/dense_transformer_runtime.cpp:673 load, :2296 forward_batch,
 * :3670 forward, :4652 generate) on the path its D3D12 backend accelerates
 * (include/zen/d3d12_backend.h:174-360).
 *
 * Status codes are those of zq_hip.h.  One zq_model is used by one thread at
 * a time; calls are synchronous (they return once results are on the host).
 */
#ifndef ZQ_MODEL_H
#define ZQ_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include "zq_gguf.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct zq_model zq_model;

/* Prefill projection arithmetic. */
#define ZQ_PREFILL_INT8 0 /* per-32 int8 activations: the reference GPU route
                             (shaders/q8_0_gemm_i8.hlsl, d3d12_backend.cpp:845-854) */
#define ZQ_PREFILL_F32 1  /* fp32 activations: the reference CPU forward_batch */

/* RuntimeConfig fields of a llama model (include/zen/runtime_types.h:8-40). */
typedef struct zq_model_config {
    uint32_t embedding;
    uint32_t layers;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t ffn;
    uint32_t vocab;
    uint32_t context;       /* model context length (metadata) */
    uint32_t max_positions; /* KV-cache capacity allocated on the device */
    uint32_t rope_dim;
    float rope_base;
    float rms_epsilon;
    uint32_t eos_token;
    int weight_format;      /* GGML type of the projections (8 = Q8_0) */
} zq_model_config;

/* Load a llama-architecture GGUF: validate shapes, upload every tensor once.
 * max_positions bounds prompt + generation (the KV-cache capacity); 0 means
 * min(context, 4096).  On failure returns < 0 and a message in err. */
int zq_model_load_gguf(const zq_gguf* gguf, uint32_t max_positions, zq_model_config* cfg_out, zq_model** model,
                       char* err, size_t err_cap);
/* A random-init model of the given shape generated directly on the device
 * (weights with the bench generator, unit norms): the config-4 shape without
 * an 8.5 GB file.  cfg->weight_format picks the projections' format (0 or 8 =
 * Q8_0; 2 = Q4_0; 14 = Q6_K; 12 = Q4_K; 13 = Q5_K); the embedding table and
 * the output projection are Q8_0.  cfg->max_positions is the KV capacity. */
int zq_model_create_synthetic(const zq_model_config* cfg, uint64_t seed, zq_model** model, char* err, size_t err_cap);
void zq_model_free(zq_model* model);
int zq_model_set_prefill_mode(zq_model* model, int mode);
/* Prefill `n` tokens from position 0 (the cache is reset).  Logits of the
 * last token to `logits` (vocab floats, may be NULL); greedy id to *next. */
int zq_model_prefill(zq_model* model, const uint32_t* tokens, size_t n, float* logits, uint32_t* next);
/* One decode step at the next position. */
int zq_model_decode(zq_model* model, uint32_t token, float* logits, uint32_t* next);
/* Greedy generate (generate(), :4652-4808): prefill, then up to max_new
 * tokens, stopping after EOS.  Wall times of the two phases in ms. */
int zq_model_generate(zq_model* model, const uint32_t* prompt, size_t n, uint32_t max_new, uint32_t* out,
                      size_t* n_out, double* prefill_ms, double* decode_ms);
/* Device address, shape and GGML type of one resident weight, so a caller can
 * run its own projections on it (zq_hip_*_dev) or check it: which is one of
 * ZQ_W_Q..ZQ_W_DOWN with layer < layers, or ZQ_W_EMBED / ZQ_W_OUTPUT with
 * layer == ZQ_MODEL_GLOBAL.  The tensor names of dense_transformer_runtime.cpp
 * (blk.N.attn_q.weight ... token_embd.weight, output.weight).
 * A synthetic model's weights are zq_hip_synth_weights_dev of seeds seed+0
 * (token_embd), seed+1 (output), then seed+2+7*layer+i for q, k, v, o, gate,
 * up, down. */
#define ZQ_MODEL_GLOBAL 0xFFFFFFFFu
#define ZQ_W_EMBED 0
#define ZQ_W_OUTPUT 1
#define ZQ_W_Q 2
#define ZQ_W_K 3
#define ZQ_W_V 4
#define ZQ_W_O 5
#define ZQ_W_GATE 6
#define ZQ_W_UP 7
#define ZQ_W_DOWN 8
int zq_model_weight(const zq_model* model, uint32_t layer, int which, const void** dev, uint32_t* rows,
                    uint32_t* cols, int* fmt);
/* Test hook (no counterpart in the reference, whose runtime keeps no device
 * intermediates): record the inputs and outputs of one decoder layer's
 * int8-activation prefill projections, so a checker can recompute them.
 * While set (dev != NULL), each prefill clears the records, and every int8
 * GEMM of decoder layer `layer` copies into dev, after its launch, the
 * int8 activations [m][k], their fp32 block scales [m][k/32] and its
 * output planes [splits][m][n] (split-K partial sums; the layer's readers
 * add them in plane order).  A projection whose copies would pass cap is
 * not recorded and zq_model_tap_records returns ZQ_ERR_TOO_LARGE.
 * dev == NULL turns the hook off.  Prefill only; decode is never recorded. */
#define ZQ_TAP_QKV 0  /* the packed q|k|v weight (n = q + k + v rows) */
#define ZQ_TAP_Q 1
#define ZQ_TAP_K 2
#define ZQ_TAP_V 3
#define ZQ_TAP_O 4
#define ZQ_TAP_GATE 5
#define ZQ_TAP_UP 6
#define ZQ_TAP_DOWN 7
typedef struct zq_model_tap_record {
    int proj;           /* ZQ_TAP_* */
    int fmt;            /* GGML type of the weight */
    const void* w;      /* device address of its rows */
    uint32_t m, n, k;   /* tokens, weight rows, columns */
    uint32_t splits;    /* output planes */
    uint64_t xq_off, xs_off, y_off; /* byte offsets into dev */
} zq_model_tap_record;
int zq_model_set_tap(zq_model* model, uint32_t layer, void* dev, size_t cap);
/* The records of the last prefill (at most cap of them; *n = how many). */
int zq_model_tap_records(const zq_model* model, zq_model_tap_record* out, size_t cap, size_t* n);

/* Device bytes held: weights, KV cache, activations. */
int zq_model_memory(zq_model* model, uint64_t* weight_bytes, uint64_t* cache_bytes, uint64_t* activation_bytes);

#ifdef __cplusplus
}
#endif
#endif /* ZQ_MODEL_H */
