/**
 * vitna_hip.h - The engine's GPU forward-step interface, served on an AMD
 * Instinct MI355X (gfx950) by libvitna_hip.so.
 *
 * The first part restates engine/include/model_cuda.h (the `vitna_cuda_*`
 * C ABI that engine/src/model.c calls under VITNA_CUDA) with the same names,
 * argument meanings and error convention, so model.c links against this
 * library unchanged: every call returns false (or 0) and writes a sentence
 * into err[err_len] when it cannot do what was asked; the caller then asks
 * vitna_cuda_lost whether the device can still be used. Each declaration
 * cites the line of model_cuda.h it replaces.
 *
 * Differences of behaviour, each deliberate:
 *  - every expert of every layer is resident in device memory (288 GB of HBM
 *    holds the largest configuration several times over), so
 *    expert_cache_bytes and the guess arguments are accepted and unused, and
 *    vitna_cuda_cpu_experts (a PCIe workaround) is refused;
 *  - the dense-model entry points (vitna_cuda_step, _steps, _rows) refuse, as
 *    the reference's refuse a mixture of experts; this library serves the
 *    mixture-of-experts path only.
 *
 * The second part (vitna_hip_*) has no counterpart in the reference: a
 * device-resident decode step that routes on the GPU (no host round trip per
 * layer), single-layer entry points for benchmarking one MoE FFN, the grouped
 * prefill of one MoE layer, and key-value cache access for tests.
 */

#ifndef VITNA_HIP_H
#define VITNA_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>
#include "vitna_model.h"

#ifdef __cplusplus
extern "C" {
#endif

/* model_cuda.h:21-25 */
typedef struct {
    int32_t token;
    int32_t pos;
    int32_t seq;
} vitna_cuda_row_t;

/* model_cuda.h:31-36 */
typedef struct {
    char name[128];
    size_t total_bytes;
    size_t free_bytes;
    int major, minor;
} vitna_cuda_device_t;

/* model_cuda.h:28 */
bool vitna_cuda_probe(char* err, size_t err_len);
/* model_cuda.h:39 */
int vitna_cuda_devices(vitna_cuda_device_t* out, int max);
/* model_cuda.h:56-57 */
struct vitna_cuda_model* vitna_cuda_create(const vitna_llama_t* m, const float* cos_tab, const float* sin_tab, size_t expert_cache_bytes,
                                           char* err, size_t err_len);
/* model_cuda.h:77-78 */
bool vitna_cuda_moe_route(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, size_t layer, float* logits, float* next,
                          char* err, size_t err_len);
/* model_cuda.h:90-91 */
bool vitna_cuda_moe_experts(struct vitna_cuda_model* g, size_t layer, const int32_t* ids, const float* weights, size_t k,
                            const int32_t* guess, char* err, size_t err_len);
/* model_cuda.h:94 */
bool vitna_cuda_moe_head(struct vitna_cuda_model* g, float* logits, char* err, size_t err_len);
/* model_cuda.h:97 */
const char* vitna_cuda_moe_report(const struct vitna_cuda_model* g, char* buf, size_t len);
/* model_cuda.h:100 */
int vitna_cuda_kv_layers(const struct vitna_cuda_model* g);
/* model_cuda.h:103 */
void vitna_cuda_test_long_from(struct vitna_cuda_model* g, size_t n);
/* model_cuda.h:106 */
void vitna_cuda_test_fast_rows(struct vitna_cuda_model* g, size_t n);
/* model_cuda.h:121 */
bool vitna_cuda_cpu_experts(struct vitna_cuda_model* g, size_t threads, char* err, size_t err_len);
/* model_cuda.h:136 */
size_t vitna_cuda_moe_rows_max(const struct vitna_cuda_model* g);
/* model_cuda.h:145-146 */
bool vitna_cuda_moe_rows_route(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t n, size_t layer, float* logits, float* next,
                               char* err, size_t err_len);
/* model_cuda.h:157-158. With an expert cache the experts go in waves through the slots, and guess (n x k) starts
   the next layer's copies, as model_cuda.cu:5134-5386 does. */
bool vitna_cuda_moe_rows_experts(struct vitna_cuda_model* g, size_t layer, size_t n, const int32_t* ids, const float* weights, size_t k,
                                 const int32_t* guess, char* err, size_t err_len);
/* model_cuda.h:161 */
bool vitna_cuda_moe_rows_head(struct vitna_cuda_model* g, size_t n, float* const* logits, char* err, size_t err_len);
/* model_cuda.h:169 */
bool vitna_cuda_step(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, float* logits, char* err, size_t err_len);
/* model_cuda.h:175 */
size_t vitna_cuda_prompt_min(const struct vitna_cuda_model* g);
/* model_cuda.h:183 */
size_t vitna_cuda_prompt_piece_min(const struct vitna_cuda_model* g);
/* model_cuda.h:190 */
size_t vitna_cuda_exact_max(const struct vitna_cuda_model* g);
/* model_cuda.h:201-202 */
bool vitna_cuda_rows(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t count, float* const* logits, char* err,
                     size_t err_len);
/* model_cuda.h:213-214 */
bool vitna_cuda_steps(struct vitna_cuda_model* g, size_t seq, const int32_t* tokens, size_t count, size_t pos, float* logits, size_t rows,
                      char* err, size_t err_len);
/* model_cuda.h:217 */
const char* vitna_cuda_device_name(const struct vitna_cuda_model* g);
/* model_cuda.h:220 */
void vitna_cuda_wait(struct vitna_cuda_model* g);
/* model_cuda.h:231 */
bool vitna_cuda_lost(struct vitna_cuda_model* g, char* err, size_t err_len);
/* model_cuda.h:233 */
void vitna_cuda_free(struct vitna_cuda_model* g);
/* model_cuda.h:244 */
bool vitna_cuda_widen(const vitna_matrix_t* m, float* out, char* err, size_t err_len);
/* model_cuda.h:254-255 */
bool vitna_cuda_expert_check(const vitna_matrix_t* gate, const vitna_matrix_t* up, const vitna_matrix_t* down, const float* norm_w,
                             const float* x, float eps, float* xs, float* act, float* y, char* err, size_t err_len);

/* ---------------------------------------------------------------------------
 * Extensions (no counterpart in the reference's interface).
 * ------------------------------------------------------------------------- */

/** One whole decode step of the token at position pos of sequence seq on the
    device, routing included (the reference's router, top-k and weights,
    engine/src/model.c:626-703, computed on the GPU, bit-exact in the expert
    choice): embedding, every layer, the head. Vocab logits to logits unless
    NULL. The steps are captured once into a HIP graph and replayed. */
bool vitna_hip_moe_step(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, float* logits, char* err, size_t err_len);

/** Device-resident step as vitna_hip_moe_step, enqueued without waiting and
    with the logits left on the device (vitna_hip_logits_device). For
    throughput measurement. */
bool vitna_hip_moe_step_async(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, char* err, size_t err_len);

/** A whole decode step of n rows (tokens of any sequences at their own
    positions, as vitna_cuda_moe_rows_route takes them) on the device:
    attention over each row's cache, the router and top-k of every row on the
    device, the rows grouped by expert so each selected expert's weights are
    read once for all the rows routed to it, the head. logits[i] receives row
    i's vocab logits where logits and it are not NULL; with logits NULL the
    step is only enqueued. Captured into a HIP graph per row count. */
bool vitna_hip_moe_rows_step(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t n, float* const* logits, char* err,
                             size_t err_len);

/** Passes of the reference's rows ABI (vitna_cuda_moe_rows_route / _experts / _head) of at most n rows run each
    row with a single token's kernels, so that every row's logits are the bits a step of that row alone gives
    (model.c:1052-1190 relies on it for drafted tokens and batched steps); longer passes take the multi-row
    kernels (within 1e-3 of the CPU, other bits). n is 64 (model.c's PASS_MAX) from vitna_cuda_create; 0 sends
    every pass to the multi-row kernels (for their tests). At most 64. On a model with an expert cache, such a
    pass whose experts outnumber one wave of the cache's rule (its slots less k) is taken in groups of consecutive
    rows that each fit one wave, each group a pass of the cache: the bits stay those of every expert resident, and
    the cache's counts are those of the groups' passes. */
bool vitna_hip_set_exact_rows(struct vitna_cuda_model* g, size_t n, char* err, size_t err_len);

/** The mixture-of-experts half of layer (RMSNorm, router, top-k on the
    device, experts, weighted sum) on residual row 0, in place, enqueued. */
bool vitna_hip_moe_ffn(struct vitna_cuda_model* g, size_t layer, char* err, size_t err_len);

/** Residual row row (hidden floats) from or to the host, synchronously. */
bool vitna_hip_residual(struct vitna_cuda_model* g, size_t row, float* host, bool to_device, char* err, size_t err_len);

/** The latest routing of row row: router logits (n_experts), the choice
    largest first (K), the experts in order of id (K) and their weights (K).
    Any pointer may be NULL. Synchronous. */
bool vitna_hip_routing(struct vitna_cuda_model* g, size_t row, float* logits, int32_t* chosen, int32_t* ids, float* weights, char* err,
                       size_t err_len);

/** Which kernels a decode step runs: on = 0 (the default) the per-layer
    kernels replayed as one HIP graph; on = 1 the persistent step kernel, one
    cooperative launch that runs every layer with device-scope flags between
    its phases, where the model's shape takes it (*taken, if not NULL, says
    whether it does). Both give the same bits. An engine choice with no
    reference counterpart. */
bool vitna_hip_set_step_kernel(struct vitna_cuda_model* g, int on, int* taken, char* err, size_t err_len);

/** One decode step (or, for a model without attention, one pass over its
    layers on residual row 0) on the persistent step kernel with block
    block's control wave stamping each phase: for every layer,
    VITNA_HIP_TRACE_PER_LAYER 64-bit s_memrealtime readings (100 MHz) into out
    (n >= layers * that), in order: for each of the six phases (q/k/v,
    attention, o-projection, router, experts in, experts down) the start of
    its wait, its inputs ready, its results published; 0 where the block has
    no part. A measurement hook: no reference counterpart. */
#define VITNA_HIP_TRACE_PER_LAYER 32
bool vitna_hip_step_trace(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, int block, uint64_t* out, size_t n, char* err,
                          size_t err_len);

/** Row row's query projection (before its QK-norm and RoPE) and attention
    output (heads x head_dim each) as the last step or rows pass left them at
    its last layer. Either pointer may be NULL. Synchronous. A checker's hook
    for the split-position attention and its merge; no reference counterpart. */
bool vitna_hip_attention_io(struct vitna_cuda_model* g, size_t row, float* q, float* att, char* err, size_t err_len);

/** The routing the last device-routed step (vitna_hip_moe_step) chose at
    layer layer: the choice largest first (K), the experts in order of id (K)
    and their weights (K). Any pointer may be NULL. Synchronous. A checker's
    hook: the reference traces its routing on the host (main.c --experts-out). */
bool vitna_hip_step_routing(struct vitna_cuda_model* g, size_t layer, int32_t* chosen, int32_t* ids, float* weights, char* err,
                            size_t err_len);

/* The routing of row `row` at `layer` in the last device-routed rows step (vitna_hip_moe_rows_step): each row's
   chosen experts (largest logit first), ids (ascending) and weights. No counterpart in the reference: a checker. */
bool vitna_hip_rows_routing(struct vitna_cuda_model* g, size_t layer, size_t row, int32_t* chosen, int32_t* ids, float* weights,
                            char* err, size_t err_len);

/** One projection of a pass of n rows (1 <= n <= the rows maximum) as the
    rows step runs it: y[t] = W x[t] for W = layer's q, k, v, o (which = 0..3)
    or the LM head (which = 4, layer ignored); x is n x W's columns, y n x W's
    rows, both on the host. Synchronous. A test hook: the reference has no
    counterpart (its multi-row kernels are only reachable through a step). */
bool vitna_hip_rows_project(struct vitna_cuda_model* g, size_t layer, int which, const float* x, size_t n, float* y, char* err,
                            size_t err_len);

/** Keys and values of positions pos0 .. pos0 + n - 1 of one layer of one
    sequence, n x (n_kv_heads * head_dim) each, to (write) or from the device. */
bool vitna_hip_kv(struct vitna_cuda_model* g, size_t seq, size_t layer, size_t pos0, size_t n, float* k, float* v, bool write, char* err,
                  size_t err_len);

/** Fill every sequence's cache, every layer, positions 0 .. n_pos[seq] - 1,
    with seeded N(0, 1) values generated on the device. */
bool vitna_hip_kv_fill(struct vitna_cuda_model* g, uint64_t seed, const size_t* n_pos, char* err, size_t err_len);

/** Wait for the model's stream; false, with the reason, on a device error. */
bool vitna_hip_sync(struct vitna_cuda_model* g, char* err, size_t err_len);

/** The HIP stream every kernel of the model runs on (a hipStream_t). */
void* vitna_hip_stream(struct vitna_cuda_model* g);

/** Device pointer of the vocab logits of row 0 of the last head. */
const float* vitna_hip_logits_device(struct vitna_cuda_model* g);

/** Prefill of n tokens through the mixture-of-experts half of layer: x is
    n x hidden on the host; each row is normalized, routed (bit-exact expert
    choice), run through its experts as a grouped bf16 MFMA GEMM with fp32
    accumulation, and its weighted sum added to it in place. chosen (n x K,
    or NULL) receives each row's experts, largest first. The reference's
    prefill grouping: model_cuda.cu:5151-5176, :2288-2343. Q8_0 experts. */
bool vitna_hip_moe_prefill(struct vitna_cuda_model* g, size_t layer, float* x, size_t n, int32_t* chosen, char* err, size_t err_len);

/** vitna_hip_moe_prefill without allocating: no reference counterpart; for
    callers that cannot allocate device memory (code under HIP graph capture,
    tight serving loops, harnesses that forbid hipMalloc). x (n x hidden fp32)
    and chosen (n x K int32, or NULL) are DEVICE pointers; x is updated in
    place. The working buffers come from a static 128 MiB device region
    that each GPU the library runs on holds until the process ends; a call
    whose rows need more fails with the most rows of this model it holds.
    Asynchronous on the model's stream (vitna_hip_stream): the caller
    synchronizes. Calls that overlap on one GPU share the region and race;
    nothing in it has to start at zero. Same kernels, same results as
    vitna_hip_moe_prefill. */
bool vitna_hip_moe_prefill_noalloc(struct vitna_cuda_model* g, size_t layer, float* x, size_t n, int32_t* chosen, char* err,
                                   size_t err_len);

/** A prefill of n rows drawn N(0,1) on the device (seed), timed with HIP
    events over reps runs after a warm-up: us_total, and us_phase[5] = norm +
    router, routing + grouping, gate/up GEMM, down GEMM, ordered sum. The
    rows stay on the device for vitna_hip_prefill_rows. */
bool vitna_hip_time_prefill(struct vitna_cuda_model* g, size_t layer, size_t n, uint64_t seed, int reps, double* us_total,
                            double* us_phase, char* err, size_t err_len);

/** The rows step (vitna_hip_moe_rows_step, logits left on the device) for
    the same rows replayed steps times after one warm-up, timed with HIP
    events on the model's stream: milliseconds a step. */
bool vitna_hip_time_rows(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t n, int steps, double* ms_per_step, char* err,
                         size_t err_len);

/** The input rows, output rows and experts chosen (any may be NULL) of the
    first n rows of the last prefill on the device. */
bool vitna_hip_prefill_rows(struct vitna_cuda_model* g, size_t n, float* x_in, float* x_out, int32_t* chosen, char* err,
                            size_t err_len);

/** Average duration in microseconds of one launch of a kernel of the decode
    path, timed with HIP events on the model's stream over reps launches
    after warmup launches: which = 0 experts gate/up, 1 experts down, 2 router,
    3 attention projections q/k/v, 4 attention, 5 o-projection, 6 LM head.
    The layer advances with each launch (layer i % n_layers), so a working
    set larger than the last-level cache is streamed. Also reports the
    algorithmic bytes one launch reads and writes. */
bool vitna_hip_time_kernel(struct vitna_cuda_model* g, int which, int reps, int warmup, double* avg_us, double* bytes, char* err,
                           size_t err_len);

/** Timing: every layer's mixture-of-experts half (norm, router, top-k, experts, weighted sum) on residual row 0,
    one after another in one graph, reps times after two warm-up passes; *us_per_layer the mean per layer. A
    model of distinct layers larger than the MALL measures streaming from HBM (configs 0 and 1 of the
    benchmark). No counterpart in the reference. */
bool vitna_hip_time_ffn(struct vitna_cuda_model* g, int reps, double* us_per_layer, char* err, size_t err_len);

/** steps device-resident decode steps (as vitna_hip_moe_step_async, the
    same token and position each time) timed with HIP events on the model's
    stream: the average milliseconds a step. */
bool vitna_hip_time_steps(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, int steps, double* ms_per_step, char* err,
                          size_t err_len);

/** For checking: the device's routing rule (the one every expert kernel
    applies to a token's router logits) on n_experts given logits: the choice
    largest first, the chosen in order of id and their weights, as
    engine/src/model.c:626-703 routes. */
bool vitna_hip_route_check(const float* logits, int n_experts, int k, bool renormalize, int32_t* chosen, int32_t* ids, float* weights,
                           char* err, size_t err_len);

/** The reference's host routing (engine/src/model.c:626-703, top_k and
    route) on the host, for callers of the layer-at-a-time ABI that have
    none of their own: chosen largest first, order the chosen sorted by id,
    weights aligned with order. Runs no device code. */
bool vitna_hip_host_route(const float* logits, int n_experts, int k, bool renormalize, int32_t* chosen, int32_t* order, float* weights,
                          char* err, size_t err_len);

/** A plain device copy of bytes (a multiple of 16), reps times, on a buffer
    of its own: the average microseconds a copy. Its hardware counters of
    bytes fetched and written are the yardstick for the other kernels'. */
bool vitna_hip_copy_probe(size_t bytes, int reps, double* avg_us, char* err, size_t err_len);

/** blocks workgroups of one wave a SIMD doing nothing but back-to-back bf16
    MFMAs (32x32x16, eight independent accumulators), iters each, reps
    launches: the dense bf16 TFLOP/s the matrix cores sustain on this device,
    the yardstick for the prefill GEMMs beside the published peak. */
bool vitna_hip_mfma_probe(int blocks, int iters, int reps, double* tflops, char* err, size_t err_len);

/** For checking the expert cache (vitna_cuda_create with an expert_cache_bytes
    that holds fewer slots than the model has experts; the reference's
    expert_cache_t, engine/src/model_cuda.cu:249-290): where[layer * E + e]
    is the slot holding that expert or -1 (n_places entries, when where is not
    NULL), and counters[0..9] = slots, slot bytes, acquired, hits, still being
    copied, misses, copied for a guess, guesses used, copies, bytes copied.
    False (with a reason) for a model whose experts are all resident. */
bool vitna_hip_expert_cache_state(const struct vitna_cuda_model* g, int32_t* where, size_t n_places, uint64_t* counters, char* err,
                                  size_t err_len);

#ifdef __cplusplus
}
#endif

#endif
