/**
 * vitna_gguf.h - A GGUF checkpoint (versions 2 and 3) read into the engine's
 * vitna_llama_t, for vitna_cuda_create (vitna_hip.h).
 *
 * The reference reads a GGUF file in two steps: engine/src/gguf.c:229
 * (vitna_gguf_open) maps it and lists its tensors under the Hugging Face
 * names (gguf.c:160-214: llama.cpp's "blk.L.ffn_gate_exps" stacks split into
 * one tensor per expert, each a view of its contiguous slice), and
 * engine/src/model.c:302-410 (vitna_llama_load_ex) binds those names to the
 * layers and allocates the caches. This reader does both for the
 * mixture-of-experts models this library serves (OLMoE's and Qwen3-MoE's
 * GGUF files), with the same checks and refusals, so the vitna_llama_t it
 * returns is the one the reference's loader returns for the same file and
 * config: every matrix points at the same byte of the file, in the same
 * dtype and shape; the norm weights are the same floats.
 *
 * The file stays mapped, read-only, for the handle's life; nothing is copied
 * on the host. vitna_cuda_create then copies each tensor to the device once.
 */

#ifndef VITNA_GGUF_H
#define VITNA_GGUF_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>
#include "vitna_model.h"

#ifdef __cplusplus
extern "C" {
#endif

/* What the file's metadata says: engine/include/gguf.h:37-57 (vitna_gguf_info_t), the same fields in the same
   order. A field the file leaves out stays 0. */
typedef struct {
    char arch[64];
    uint32_t version;
    uint64_t alignment;
    uint64_t block_count;
    uint64_t embedding_length;
    uint64_t feed_forward_length;
    uint64_t expert_feed_forward_length;
    uint64_t head_count;
    uint64_t head_count_kv;
    uint64_t key_length;
    uint64_t context_length;
    uint64_t expert_count;
    uint64_t expert_used_count;
    double rms_eps;
    double rope_freq_base;
    size_t file_tensors;
    uint16_t split_no;
    uint16_t split_count;
    uint64_t split_tensors_count;
} vitna_hip_gguf_info_t;

/* One tensor of the directory, under its Hugging Face name: engine/include/safetensors.h:40-48
   (vitna_tensor_desc_t) without the unused shape slots. Offsets count from the start of the data section. */
typedef struct {
    char name[256];
    vitna_dtype_t dtype;
    size_t ndim;
    size_t shape[2]; /* rows, cols (ndim 2) or n (ndim 1) */
    uint64_t offset_begin;
    uint64_t offset_end;
    const void* data;
} vitna_hip_gguf_tensor_t;

typedef struct vitna_hip_gguf vitna_hip_gguf_t;

/** Map path and read its header, metadata and tensor directory (replaces
    engine/src/gguf.c:229 vitna_gguf_open for one unsplit file). Refuses, with
    the reason in err, what the reference refuses: another magic or version,
    a tensor name it does not know, a dtype it does not compute with, rows that
    are not whole blocks, data off its alignment or past the file's end, a
    llama-architecture file (permuted q/k rows). NULL on failure. */
vitna_hip_gguf_t* vitna_hip_gguf_open(const char* path, vitna_hip_gguf_info_t* info, char* err, size_t err_len);

/** Tensors in the directory (each expert of a stack its own). */
size_t vitna_hip_gguf_count(const vitna_hip_gguf_t* g);

/** Tensor i of the directory, in the file's order (a stack's experts in
    expert order). False when i is out of range. */
bool vitna_hip_gguf_tensor(const vitna_hip_gguf_t* g, size_t i, vitna_hip_gguf_tensor_t* out);

/** The offset of the data section from the start of the file. */
uint64_t vitna_hip_gguf_data_offset(const vitna_hip_gguf_t* g);

/** Bind the directory into *m for the model cfg describes (the reference reads
    cfg from config.json, engine/src/model.c:54-137), as
    engine/src/model.c:302-410 binds it, after checking the file's metadata
    against cfg as model.c:160-175 does: matrices point into the mapping; the
    norm weights are widened to float32 copies; the key-value cache (seqs
    sequences of ctx positions, ctx 0 meaning min(max_positions, 4096)), the
    rotary frequencies and the step's scratch are allocated as the reference
    allocates them. Free with vitna_hip_gguf_llama_free before closing g. */
bool vitna_hip_gguf_llama(vitna_hip_gguf_t* g, const vitna_llama_config_t* cfg, size_t ctx, size_t seqs, vitna_llama_t* m, char* err,
                          size_t err_len);

/** Free what vitna_hip_gguf_llama allocated in *m (the mapping stays with g). */
void vitna_hip_gguf_llama_free(vitna_llama_t* m);

/** Unmap the file and free the directory. */
void vitna_hip_gguf_close(vitna_hip_gguf_t* g);

#ifdef __cplusplus
}
#endif

#endif /* VITNA_GGUF_H */
