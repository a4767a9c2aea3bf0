/**
 * vitna_model.h - The model types the forward-step interface passes across
 * the boundary, declared so that a struct built by the engine's loader is the
 * struct this library reads, field for field.
 *
 * The engine's loader (engine/src/model.c) fills a vitna_llama_t and hands a
 * pointer to vitna_cuda_create (vitna_hip.h). This library never includes the
 * engine's headers, so the layouts below restate them: the same members, in
 * the same order, with the same C types, as
 *   engine/include/safetensors.h:23-45  (vitna_dtype_t, enum order)
 *   engine/include/model.h:46-63        (vitna_llama_config_t)
 *   engine/include/model.h:65-70        (vitna_matrix_t)
 *   engine/include/model.h:72-80        (VITNA_EXPERTS_USED_MAX, vitna_expert_t)
 *   engine/include/model.h:82-92        (vitna_llama_layer_t)
 *   engine/include/model.h:97-185       (vitna_llama_t)
 * A test compiles the engine's model.h beside this file and compares every
 * offset and size. Members this library never reads keep their place and type
 * only, with pointers to the engine's own structs made opaque.
 *
 * GGUF block formats (bytes per block of weights), unchanged on the host side:
 *   Q8_0  34 B / 32 w : d f16 | q int8 x32                      w = q * d
 *   Q4_K 144 B / 256 w: d f16 | dmin f16 | 12 B 6-bit scales/mins | 128 B q4
 *                       w = (d * sc_g) * q - (dmin * mn_g), group g of 32
 *   Q6_K 210 B / 256 w: ql 128 B | qh 64 B | 16 int8 scales | d f16
 *                       w = (d * sc_{i/16}) * (q - 32)
 */

#ifndef VITNA_MODEL_TYPES_H
#define VITNA_MODEL_TYPES_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element and block types; the numeric values are the engine's enum order. */
typedef enum {
    VITNA_DTYPE_UNKNOWN = 0,
    VITNA_DTYPE_F32,
    VITNA_DTYPE_F16,
    VITNA_DTYPE_BF16,
    VITNA_DTYPE_I32,
    VITNA_DTYPE_I16,
    VITNA_DTYPE_I8,
    VITNA_DTYPE_U8,
    VITNA_DTYPE_BOOL,
    VITNA_DTYPE_F64,
    VITNA_DTYPE_I64,
    VITNA_DTYPE_U16,
    VITNA_DTYPE_U32,
    VITNA_DTYPE_U64,
    VITNA_DTYPE_Q8_0,
    VITNA_DTYPE_Q2_K,
    VITNA_DTYPE_Q3_K,
    VITNA_DTYPE_Q4_K,
    VITNA_DTYPE_Q5_K,
    VITNA_DTYPE_Q6_K
} vitna_dtype_t;

typedef struct {
    size_t n_layers;
    size_t hidden;
    size_t intermediate;
    size_t n_heads;
    size_t n_kv_heads;
    size_t head_dim;
    size_t vocab;
    size_t max_positions;
    float rms_eps;
    float rope_theta;
    bool tied_embeddings;
    bool qk_norm;
    bool qk_norm_per_head;
    size_t n_experts;
    size_t n_experts_used;
    bool renormalize;
    bool qwen3;
} vitna_llama_config_t;

/* A weight matrix in its stored dtype: rows of cols weights, a block format's
   row whole blocks, rows back to back. */
typedef struct {
    const void* data;
    vitna_dtype_t dtype;
    size_t rows;
    size_t cols;
} vitna_matrix_t;

#define VITNA_EXPERTS_USED_MAX 64

typedef struct {
    vitna_matrix_t gate, up, down;
} vitna_expert_t;

typedef struct {
    float* attn_norm;
    float* mlp_norm;
    vitna_matrix_t q, k, v, o, gate, up, down;
    float* q_norm;
    float* k_norm;
    vitna_matrix_t router;
    vitna_expert_t* experts;
} vitna_llama_layer_t;

struct vitna_cuda_model;
struct vitna_safetensors;
struct vitna_expert_stream;

typedef struct {
    vitna_llama_config_t cfg;
    struct vitna_safetensors* shards;
    char** shard_paths;
    size_t n_shards;
    vitna_matrix_t embed;
    vitna_matrix_t lm_head;
    float* final_norm;
    vitna_llama_layer_t* layers;
    float* inv_freq;

    size_t ctx;
    size_t seqs;
    size_t* past;
    float* k_cache;
    float* v_cache;

    float *x, *xn, *q, *k, *v, *att, *proj, *gate, *up, *scores, *cos_t, *sin_t;
    float *router_logits, *expert_out;

    struct vitna_expert_stream* stream;
    float *pred_xn, *pred_logits;
    int32_t predicted[VITNA_EXPERTS_USED_MAX];
    int64_t predicted_layer;
    uint64_t predicted_right, predicted_total;

    float* trace_logits;
    int32_t* trace_chosen;
    size_t trace_positions;
    const int32_t* pin;
    size_t pin_positions;

    struct vitna_cuda_model* cuda;

    size_t rows_max;
    float *rows_logits, *rows_next, *rows_weights;
    int32_t *rows_order, *rows_pred;
    void* rows_chunk;
    float** rows_outs;
    bool no_rows;

    int gpu_kv_layers;
    bool gpu_fast;

    bool device_lost;
    char device_error[160];

    bool fail_armed;
    bool fail_loses;
    size_t fail_at;
} vitna_llama_t;

/* Weights in one block of a dtype (1 for an element type, 0 if unknown), and
   its bytes. */
static inline size_t vitna_block_elems(vitna_dtype_t t) {
    switch (t) {
        case VITNA_DTYPE_Q8_0: return 32;
        case VITNA_DTYPE_Q2_K: case VITNA_DTYPE_Q3_K: case VITNA_DTYPE_Q4_K:
        case VITNA_DTYPE_Q5_K: case VITNA_DTYPE_Q6_K: return 256;
        case VITNA_DTYPE_F32: case VITNA_DTYPE_F16: case VITNA_DTYPE_BF16: return 1;
        default: return 0;
    }
}

static inline size_t vitna_block_bytes(vitna_dtype_t t) {
    switch (t) {
        case VITNA_DTYPE_Q8_0: return 34;
        case VITNA_DTYPE_Q2_K: return 84;
        case VITNA_DTYPE_Q3_K: return 110;
        case VITNA_DTYPE_Q4_K: return 144;
        case VITNA_DTYPE_Q5_K: return 176;
        case VITNA_DTYPE_Q6_K: return 210;
        case VITNA_DTYPE_F32: return 4;
        case VITNA_DTYPE_F16: case VITNA_DTYPE_BF16: return 2;
        default: return 0;
    }
}

/* Bytes in a row of cols weights; 0 if cols is not whole blocks. */
static inline size_t vitna_matrix_row_bytes(vitna_dtype_t t, size_t cols) {
    const size_t be = vitna_block_elems(t);
    if (!be || cols % be) return 0;
    return cols / be * vitna_block_bytes(t);
}

#ifdef __cplusplus
}
#endif

#endif /* VITNA_MODEL_TYPES_H */
