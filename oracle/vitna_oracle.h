/**
 * vitna_oracle.h - TEST INFRASTRUCTURE ONLY. A CPU restatement of the
 * reference engine's float32 arithmetic for the quantized mixture-of-experts
 * decode path, used as the parity checker for the HIP library.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only to check or time against it: the HIP product path
 * never calls it and has no CPU fallback.
 *
 * Every function names the reference file:line whose arithmetic it restates.
 * "AVX2 order" means the order of engine/src/ops.c:212-229 (matvec_blocks_avx2)
 * and engine/src/kernels.c:115-160 (vitna_rmsnorm_avx2): sixteen fused
 * multiply-add chains, chain j taking elements 16m + j in order of m, then
 * v[j] = a[j] + a[j + 8] and the horizontal tree
 * ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)).
 */

#ifndef VITNA_ORACLE_H
#define VITNA_ORACLE_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>
#include "../include/vitna_model.h"

#ifdef __cplusplus
extern "C" {
#endif

float orc_f16_to_f32(uint16_t h);
void orc_dequant_q8_0(const uint8_t* block, float out[32]);
void orc_dequant_q4_k(const uint8_t* block, float out[256]);
void orc_dequant_q6_k(const uint8_t* block, float out[256]);
/* n weights of a dtype (F32, F16, BF16, Q8_0, Q4_K, Q6_K), n whole blocks. */
int orc_widen(const void* src, int dtype, float* dst, size_t n);

/* y = W x in the AVX2 order; threads > 1 splits rows across threads, which
   changes no bit (each row is one thread's). */
int orc_matvec(const void* w, int dtype, const float* x, float* y, size_t rows, size_t cols);
int orc_matvec_mt(const void* w, int dtype, const float* x, float* y, size_t rows, size_t cols, int threads);

void orc_rmsnorm(const float* x, const float* w, float* y, size_t n, float eps);
void orc_silu_mul(const float* gate, const float* up, float* out, size_t n);
void orc_rope_half(float* v, size_t head_dim, const float* cos_t, const float* sin_t);

void orc_top_k(const float* logits, size_t n, size_t k, int32_t* out);
void orc_route(const float* logits, size_t E, size_t K, bool renormalize, int32_t* chosen, int32_t* order, float* weights);

/* One layer's mixture of experts on xn (already normalized): router logits
   into logits (E), route, and the ordered weighted sum into proj (H). */
int orc_moe(const vitna_llama_t* m, size_t layer, const float* xn, float* logits, int32_t* chosen, int32_t* order,
            float* weights, float* proj, int threads);

/* One decode step of the whole model as the reference's CPU step runs it
   (token at position pos of sequence seq, keys and values written to
   m->k_cache/v_cache at pos), logits into logits (vocab) unless NULL. When
   trace_logits / trace_chosen are not NULL they receive each layer's router
   logits (n_layers x E) and top-k (n_layers x K). When resid is not NULL it
   receives the residual after each layer (n_layers x H). */
int orc_step(vitna_llama_t* m, size_t seq, int32_t token, size_t pos, float* logits, float* trace_logits, int32_t* trace_chosen,
             float* resid, int threads);

#ifdef __cplusplus
}
#endif

#endif
