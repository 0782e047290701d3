/*
 * zq_gguf.h -- C ABI of the GGUF loader: a memory-mapped GGUF v2/v3 parser
 * whose tensor payloads are handed, in their native block layout, to the
 * device-resident model (zq_model.h) for one upload into HBM.
 *
 * It replaces the reference's zen::gguf surface (include/zen/gguf.h:5-30,
 * src/gguf.cpp:113-398): the same parse core checks, limits and error
 * strings, with the file mapped instead of streamed so tensor payloads are
 * addressable in place (the reference's runtime maps the file itself,
 * src/adapters/dense_transformer_runtime.cpp:673-700).
 *
 * Status codes are those of zq_hip.h (ZQ_OK / ZQ_ERR_ARG ...).  No call
 * throws.  A zq_gguf handle is immutable after open and may be read from
 * several threads.
 */
#ifndef ZQ_GGUF_H
#define ZQ_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type 9 (Q8_1) has two historical layouts; it must be chosen
 * explicitly (include/zen/gguf.h:6-9).  UNSPECIFIED defers to the env
 * ZEN_GGUF_Q8_1_LAYOUT=fp16|fp32, else a type-9 tensor fails the parse. */
#define ZQ_GGUF_Q8_1_UNSPECIFIED 0
#define ZQ_GGUF_Q8_1_FP16_36 1
#define ZQ_GGUF_Q8_1_FP32_40 2

typedef struct zq_gguf zq_gguf;

/* One tensor directory entry (model::TensorDesc, include/zen/model_ir.h:16-23). */
typedef struct zq_gguf_tensor {
    const char* name;        /* valid while the handle is open */
    uint32_t n_dims;
    uint64_t dims[4];        /* dims[0] is the contiguous (column) axis */
    uint32_t ggml_type;
    uint64_t offset;         /* relative to the tensor-data section */
    uint64_t byte_size;
    const uint8_t* data;     /* the payload inside the mapping / image */
} zq_gguf_tensor;

/* Header and the model fields of gguf::LoadReport / model::ModelConfig
 * (include/zen/gguf.h:10-18, include/zen/model_ir.h:24-56). */
typedef struct zq_gguf_config {
    uint32_t version;
    uint64_t data_offset;
    uint64_t file_size;
    uint32_t embedding_length;
    uint32_t block_count;
    uint32_t head_count;
    uint32_t head_count_kv;
    uint32_t feed_forward_length;
    uint32_t context_length;
    uint32_t vocabulary_size;
    uint32_t bos_token_id;
    uint32_t eos_token_id;
    char architecture[64];
    char name[128];
} zq_gguf_config;

/* gguf::inspect (include/zen/gguf.h:22): map and parse a file.  On failure
 * returns ZQ_ERR_ARG and writes the reference's error text into err. */
int zq_gguf_open(const char* path, int q8_1_layout, zq_gguf** out, char* err, size_t err_cap);
/* gguf::inspect_bytes (include/zen/gguf.h:26): parse an in-memory image.
 * The image is borrowed and must outlive the handle. */
int zq_gguf_open_bytes(const uint8_t* data, size_t size, int q8_1_layout, zq_gguf** out, char* err,
                       size_t err_cap);
void zq_gguf_close(zq_gguf* g);
int zq_gguf_get_config(const zq_gguf* g, zq_gguf_config* out);
size_t zq_gguf_tensor_count(const zq_gguf* g);
int zq_gguf_get_tensor(const zq_gguf* g, size_t index, zq_gguf_tensor* out);
/* ZQ_DECLINED when no tensor has that name. */
int zq_gguf_find_tensor(const zq_gguf* g, const char* name, zq_gguf_tensor* out);
/* Scalar / string metadata as text, the way the reference stores it in
 * ModelConfig::metadata (src/gguf.cpp:201-204): sorted keys; NULL when absent. */
size_t zq_gguf_meta_count(const zq_gguf* g);
const char* zq_gguf_meta_key(const zq_gguf* g, size_t index);
const char* zq_gguf_meta_value(const zq_gguf* g, const char* key);

#ifdef __cplusplus
}
#endif
#endif /* ZQ_GGUF_H */
