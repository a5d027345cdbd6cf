/*
 * slm_gguf -- GGUF model files for static-lm on MI355X.
 *
 * Reads the format static-lm's loader reads (src/memory/loader.rs): a GGUF v2
 * or v3 file, memory-mapped read-only, its metadata (all thirteen value
 * types, arrays kept as byte ranges) and tensor directory, the tensor data
 * at `general.alignment` (default 32) after the directory.  Tensor views are
 * checked like GgufFile::raw_tensor_bytes (loader.rs:464-507): type, bounds,
 * and alignment of the view's element type.  slm_model_load_gguf uploads a
 * whole model's tensors (GgufFile::model_weights, loader.rs:508-552) to the
 * device for the slm_model_*_dev entry points of slm_layer.h.
 *
 * Errors mirror GgufError (loader.rs:161-178) one code each; the message of
 * slm_attn_last_error(NULL) names the variant and its operand.
 */
#ifndef SLM_GGUF_H
#define SLM_GGUF_H

#include <stdint.h>

#include "slm_layer.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SLM_ERR_IO (-12)          /* GgufError::Io (open / map failed) */
#define SLM_ERR_EOF (-13)         /* GgufError::UnexpectedEof */
#define SLM_ERR_MAGIC (-14)       /* GgufError::InvalidMagic */
#define SLM_ERR_VERSION (-15)     /* GgufError::UnsupportedVersion */
#define SLM_ERR_UTF8 (-16)        /* GgufError::InvalidUtf8 */
#define SLM_ERR_VALUE_TYPE (-17)  /* GgufError::InvalidValueType */
#define SLM_ERR_DIMS (-18)        /* GgufError::InvalidDimensions */
#define SLM_ERR_NOT_FOUND (-19)   /* GgufError::TensorNotFound (or a missing metadata key) */
#define SLM_ERR_TYPE (-20)        /* GgufError::TypeMismatch */
#define SLM_ERR_BOUNDS (-21)      /* GgufError::OutOfBounds */
#define SLM_ERR_UNALIGNED (-22)   /* GgufError::UnalignedTensor */

/* GGML tensor types the reference knows (GgmlType, loader.rs:14-65). */
#define SLM_GGML_F32 0
#define SLM_GGML_F16 1
#define SLM_GGML_Q4_0 2
#define SLM_GGML_Q8_0 8

/* GGUF metadata value types (read_value, loader.rs:284-317). */
enum {
    SLM_GGUF_U8 = 0, SLM_GGUF_I8 = 1, SLM_GGUF_U16 = 2, SLM_GGUF_I16 = 3,
    SLM_GGUF_U32 = 4, SLM_GGUF_I32 = 5, SLM_GGUF_F32 = 6, SLM_GGUF_BOOL = 7,
    SLM_GGUF_STR = 8, SLM_GGUF_ARRAY = 9, SLM_GGUF_U64 = 10, SLM_GGUF_I64 = 11,
    SLM_GGUF_F64 = 12
};

typedef struct slm_gguf slm_gguf;

/* GgufFile::open (loader.rs:330-400): magic, version 2 or 3, metadata,
 * tensor directory, alignment and data offset. */
int slm_gguf_open(const char* path, slm_gguf** out);
void slm_gguf_close(slm_gguf* g);
int32_t slm_gguf_version(const slm_gguf* g);
int64_t slm_gguf_alignment(const slm_gguf* g);
int64_t slm_gguf_data_offset(const slm_gguf* g);
int64_t slm_gguf_tensor_count(const slm_gguf* g);
int64_t slm_gguf_kv_count(const slm_gguf* g);

/* A metadata value: its type and raw scalar.  Integers and bool come in i64
 * (u64 in u64), floats in f64, a string as a pointer into the mapping and its
 * length (not NUL-terminated), an array as its element type, length and
 * byte range in the file. */
typedef struct slm_gguf_value {
    int32_t type;
    int64_t i64;
    uint64_t u64;
    double f64;
    const char* str;
    uint64_t str_len;
    int32_t elem_type;
    uint64_t len;
    uint64_t byte_offset;
    uint64_t byte_len;
} slm_gguf_value;
int slm_gguf_get(const slm_gguf* g, const char* key, slm_gguf_value* out);

/* The typed getters of GgufFile (loader.rs:405-425), with GgufValue's
 * conversions (as_u32, as_usize, as_f32, as_str: loader.rs:91-125);
 * SLM_ERR_NOT_FOUND when the key is absent or does not convert. */
int slm_gguf_get_u32(const slm_gguf* g, const char* key, uint32_t* out);
int slm_gguf_get_usize(const slm_gguf* g, const char* key, uint64_t* out);
int slm_gguf_get_f32(const slm_gguf* g, const char* key, float* out);
/* *len bytes at *str, inside the mapping (valid until slm_gguf_close). */
int slm_gguf_get_str(const slm_gguf* g, const char* key, const char** str, uint64_t* len);

/* A tensor directory entry (TensorInfo, loader.rs:127-158). */
typedef struct slm_gguf_tensor {
    int32_t ggml_type;
    int32_t n_dims;
    uint64_t dims[4];    /* dims[0] is the innermost (row length) */
    uint64_t offset;     /* relative to the data section */
    uint64_t n_elements;
} slm_gguf_tensor;
int slm_gguf_tensor_info(const slm_gguf* g, const char* name, slm_gguf_tensor* out);
/* A checked view of a tensor's bytes in the mapping: raw_tensor_bytes with the
 * expected type, then the element alignment tensor_f32 / tensor_q4_0 need
 * (bytemuck::try_cast_slice: 4 bytes for F32, 2 for Q4_0). */
int slm_gguf_tensor_data(const slm_gguf* g, const char* name, int32_t expected_type,
                         const void** data, uint64_t* bytes);

/* The model config main.rs builds from the metadata (main.rs:282-305):
 * {arch}.block_count (default 2), .attention.head_count (8),
 * .embedding_length (256), .feed_forward_length (768),
 * .attention.head_count_kv (head_count), .context_length (64),
 * .attention.layer_norm_rms_epsilon (1e-5), with arch =
 * general.architecture (default "llama"); and {arch}.rope.freq_base
 * (default 10000, the reference's fixed value), which the reference does not
 * read.  max_seq_len is the file's context length, without the CLI's cap. */
typedef struct slm_model_config {
    int32_t dim;
    int32_t hidden_dim;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t max_seq_len;
    int32_t num_layers;
    float rms_eps;
    float rope_theta;
} slm_model_config;
int slm_gguf_model_config(const slm_gguf* g, slm_model_config* out);

/* A whole model's weights on one device. */
typedef struct slm_model slm_model;
/* GgufFile::model_weights (loader.rs:523-552) for num_layers layers, uploaded
 * to `device`: token_embd.weight (Q4_0, vocab = dims[1]), blk.{l}.attn_norm /
 * attn_q / attn_k / attn_v / attn_output / ffn_norm / ffn_gate / ffn_up /
 * ffn_down, output_norm.weight, output.weight (token_embd when absent).
 * Every tensor is checked before anything is uploaded: a missing one or one
 * of the wrong type gives its GgufError code, and a norm vector whose length
 * is not the model dimension (token_embd's dims[0]) gives SLM_ERR_SHAPE (the
 * reference's RMSNorm asserts weights.len() == dst.len, engine.rs:199). */
int slm_model_load_gguf(const slm_gguf* g, int32_t device, int32_t num_layers,
                        slm_model** out);
void slm_model_destroy(slm_model* m);
/* The weights view the slm_model_*_dev calls take; valid until destroy. */
const slm_model_weights* slm_model_weights_view(const slm_model* m);
int32_t slm_model_vocab_size(const slm_model* m);

#ifdef __cplusplus
}
#endif

#endif /* SLM_GGUF_H */
