/**
 * expert_cache.h - The experts of a model too large for the device: a cache of
 * slots in device memory, each holding one expert (gate, up and down of one
 * layer), filled from a page-locked host copy of every expert as the layers ask
 * for them.
 *
 * Reference counterpart: expert_cache_t (engine/src/model_cuda.cu:249-290),
 * create_experts (:3633), free_slot (:4334), fill (:4355), and the cache's part
 * of vitna_cuda_moe_experts (:4757-4913), vitna_cuda_moe_rows_experts (:5134-5386)
 * and vitna_cuda_moe_report (:4929).
 *
 * The rule the reference keeps:
 *   - a place is (layer, expert); each request of a place counts one use, and
 *     every 65,536 requests all counts are halved;
 *   - a slot for a place the device lacks is an empty slot, else the least used
 *     of the slots no request of the current call holds, the least recently
 *     used between equals;
 *   - after the layer's kernels are queued, the first ceil(k / 2) places of the
 *     guess (the next layer's experts by the router's rank) that the device
 *     lacks are copied in behind them, while slots are free to take;
 *   - the cache must hold at least twice the experts a token goes through.
 *
 * On this device the host copy is laid out as the slots are (the planes of
 * vitna_hip_internal.h, so a fill is one contiguous copy), and copies run on a
 * stream of their own, ordered after every kernel queued before the request
 * (a slot given to another expert is never read by a kernel still queued).
 * The reference's disk-backed expert stream and its CPU split are not kept:
 * the host copy holds every expert.
 */

#ifndef VITNA_EXPERT_CACHE_H
#define VITNA_EXPERT_CACHE_H

#include "vitna_kernels.h"
#include <vector>

struct ec_slot {
    int64_t place = -1;   /* layer * E + expert, or -1 for empty */
    bool held = false;    /* named by the request being served */
    bool guessed = false; /* filled for a guess, not yet asked for */
    bool filling = false; /* its copy may still be running */
    uint64_t last_use = 0;
    hipEvent_t filled = nullptr;
};

struct expert_cache {
    bool on = false;
    int n_layers = 0, E = 0, K = 0;
    int n_slots = 0;
    size_t slot_bytes = 0;
    std::vector<size_t> part_off;   /* [layer][3]: where gate, up and down start in a slot */
    std::vector<size_t> used_bytes; /* [layer]: a slot's bytes that layer fills */
    std::vector<int> part_dtype;    /* [layer][3] */
    std::vector<int> part_rows, part_cols;
    uint8_t* mem = nullptr;         /* device: n_slots x slot_bytes */
    uint8_t* host = nullptr;        /* page-locked: n_places x slot_bytes, every expert as a slot holds it */
    size_t n_places = 0;
    std::vector<ec_slot> slots;
    std::vector<int32_t> where;     /* [n_places]: the slot holding each, or -1 */
    std::vector<uint32_t> uses;     /* [n_places] */
    uint64_t clock = 0, acquired = 0;
    uint64_t hits = 0, in_flight = 0, misses = 0, prefetched = 0, prefetch_used = 0, copies = 0, bytes_copied = 0;
    hipStream_t copy = nullptr;
    hipEvent_t queued = nullptr;    /* the compute stream's work before a request */
};

/* The cache for model m when expert_cache_bytes leaves fewer slots than places; *on false (nothing allocated)
   when it holds every expert, or is 0. */
bool ec_create(expert_cache& c, const vitna_llama_t* m, size_t expert_cache_bytes, char* err, size_t err_len);
void ec_destroy(expert_cache& c);

/* Layer l's gate, up and down over the slots: expert index = slot. */
qmat ec_view(const expert_cache& c, int layer, int part);

/* The slots holding layer's experts ids[0..k), copies queued for those it lacks, all held until ec_finish. */
bool ec_acquire(expert_cache& c, int layer, const int32_t* ids, int k, hipStream_t compute, int32_t* slot_of, char* err,
                size_t err_len);
/* The compute stream made to wait for the copies into slot_of[0..k) that may still run. */
bool ec_wait(expert_cache& c, const int32_t* slot_of, int k, hipStream_t compute, char* err, size_t err_len);
/* After the layer's kernels are queued on compute: the guess's copies, then every hold released. */
bool ec_finish(expert_cache& c, int layer, const int32_t* guess, int k, char* err, size_t err_len);

/* A pass of rows (model_cuda.cu:5134-5386). ec_rows_count: every row's request of layer's expert x counts a use,
   cnt[x] of them; the halving of every count when the requests cross a multiple of 65,536. */
void ec_rows_count(expert_cache& c, int layer, const int32_t* cnt);
/* One wave of the pass: the experts xs[0..nx) (in order of expert, nx at most n_slots - k), each wanted by cnt[x]
   rows. The holds of the previous wave are released (first: none), copies are ordered after every kernel queued
   on compute so far, the experts present are held, those lacking copied in k at a time; slot_of[x] set. */
bool ec_rows_wave(expert_cache& c, int layer, const int32_t* xs, int nx, const int32_t* cnt, hipStream_t compute,
                  int32_t* slot_of, char* err, size_t err_len);
/* After the pass's kernels: of each row's guess (n x k, the next layer's experts by rank) the upper half the
   device lacks, each expert once, copied while slots are free; then every hold released. */
bool ec_rows_finish(expert_cache& c, int layer, const int32_t* guess, int n, int k, char* err, size_t err_len);

/* The reference's summary line (model_cuda.cu:4946-4953). */
void ec_report(const expert_cache& c, char* buf, size_t len);

#endif
