/**
 * vitna_synth.h - Seeded synthetic models and inputs for the benchmark
 * configurations: the weights and activations both the HIP library and its
 * CPU checker run on. Workload generation only; no arithmetic of the path.
 *
 * Randomness: every row of every tensor has its own stream, keyed by
 * (seed, tensor tag, row) through splitmix64 into xoshiro256**, so a tensor is
 * the same bytes however its rows are split across threads. Normals are
 * Box-Muller in double precision. Block formats take their integer fields
 * from uniform random bits (every 4- and 6-bit field of Q4_K and Q6_K is then
 * uniform), Q8_0's integers uniform in [-127, 127], Q6_K's scales uniform in
 * [-32, 31], and every float16 scale is round-to-nearest-even of
 * |N(0,1)| * scale_mul.
 */

#ifndef VITNA_SYNTH_H
#define VITNA_SYNTH_H

#include <stddef.h>
#include <stdint.h>
#ifndef VITNA_MODEL_H /* the engine's model.h declares the same types, laid out alike */
#include "../../include/vitna_model.h"
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    size_t n_layers, hidden, intermediate;
    size_t n_heads, n_kv_heads, head_dim, vocab;
    size_t n_experts, n_experts_used;
    int renormalize;
    int attention;         /* 0: the layers hold a mixture of experts only (no attention, embedding or head) */
    float rms_eps, rope_theta;
    int dt_gate_up, dt_down, dt_q, dt_k, dt_v, dt_o, dt_head, dt_embed;
    float router_std;      /* router entries N(0, router_std), F32 */
    float q8_scale;        /* Q8_0: d = f16(|N| * q8_scale) */
    float k_scale;         /* Q4_K / Q6_K: d, dmin = f16(|N| * k_scale) */
    float norm_std;        /* norm weights 1 + N(0, norm_std); 0 for all ones */
    size_t ctx, seqs;      /* key-value cache the model carries (host) */
    int kv_host;           /* allocate the host key-value cache and step scratch (for the CPU checker) */
} vitna_synth_shape_t;

/* A model of the given shape, every weight drawn from seed. The returned
   struct is laid out as the engine's vitna_llama_t; free with
   vitna_synth_free. threads <= 0 uses 8. NULL on failure, with err. */
vitna_llama_t* vitna_synth_model(const vitna_synth_shape_t* s, uint64_t seed, int threads, char* err, size_t err_len);
void vitna_synth_free(vitna_llama_t* m);

/* n normals N(0,1) as float32 from stream (seed, tag). */
void vitna_synth_normal(uint64_t seed, uint64_t tag, float* out, size_t n);

/* A rows x cols matrix of a dtype (F32: N(0, scale); Q8_0, Q4_K, Q6_K as
   above with scale_mul) into out, row_bytes each row. Returns 0, or -1 for an
   unsupported dtype or shape. */
int vitna_synth_matrix(int dtype, uint64_t seed, uint64_t tag, size_t rows, size_t cols, float scale, void* out, int threads);

/* The model written into directory dir as model.gguf (GGUF version 3, llama.cpp's tensor names, expert stacks,
   data aligned to alignment, norm weights stored as norm_dtype: F32, F16 or BF16) and config.json (the keys the
   engine's loader reads). The model must hold attention and a mixture of experts. Returns 0, or -1 with err. */
int vitna_synth_write_gguf(const vitna_llama_t* m, const char* dir, int norm_dtype, uint32_t alignment, char* err, size_t err_len);

/* Round-to-nearest-even float32 to float16 bits. */
uint16_t vitna_synth_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif

#endif
