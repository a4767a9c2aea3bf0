/**
 * expert_cache.h - The experts of a model too large for the device: a table of
 * slots in device memory, each holding one expert (gate, up and down of one
 * layer), filled from a page-locked host image of every expert as the layers
 * ask for them.
 *
 * Reference counterpart (the behaviour kept, not the code): expert_cache_t
 * (engine/src/model_cuda.cu:249-290), create_experts (:3633), the slot choice
 * and the copy (:4334-4391), the cache's part of vitna_cuda_moe_experts
 * (:4757-4913), of vitna_cuda_moe_rows_experts (:5134-5386) and
 * vitna_cuda_moe_report (:4929).
 *
 * The choices the reference makes, which this table makes too:
 *   - a place is (layer, expert); each request of a place counts one use, and
 *     every 65,536 requests all counts are halved;
 *   - a slot for a place the device lacks is the lowest-numbered empty slot,
 *     else, of the slots the current request does not pin, the one whose place
 *     has the fewest uses, the least recently stamped between equals;
 *   - after the layer's kernels are queued, the first ceil(k / 2) places of the
 *     guess (the next layer's experts by the router's rank) that the device
 *     lacks are copied in behind them, while a slot can be taken;
 *   - the table holds at least twice the experts a token goes through.
 *
 * Design. A request (one token's layer, or one wave of a pass of rows) has a
 * number; a slot is pinned while its `pin` equals the open request's number,
 * so closing a request unpins every slot at once. Empty slots sit in an
 * ordered set, so the lowest is taken without a scan; the eviction scan runs
 * only when the set is empty, over the unpinned slots, by the key (uses,
 * stamp). A copy is one contiguous host-to-device transfer (the host image is
 * laid out as a slot: the planes of vitna_hip_internal.h) on a stream of its
 * own, ordered after every kernel queued before the request, so a slot handed
 * to another place is never read by a kernel still queued. The reference's
 * disk-backed expert stream and its CPU split are not built: the host image
 * holds every expert.
 */

#ifndef VITNA_EXPERT_CACHE_H
#define VITNA_EXPERT_CACHE_H

#include "vitna_kernels.h"
#include <set>
#include <vector>

struct ec_slot {
    int64_t place = -1;       /* layer * E + expert, or -1 while empty */
    uint64_t pin = 0;         /* the request that pins it; pinned while equal to the open request's number */
    uint64_t stamp = 0;       /* logical time of the last request or copy that named it */
    bool from_guess = false;  /* copied for a guess and not yet asked for */
    bool copying = false;     /* its copy may still be running: `landed` tells */
    hipEvent_t landed = nullptr;
};

/* What a cache has done, in the reference's terms (its report line). */
struct ec_counts {
    uint64_t acquired = 0;    /* requests of a place */
    uint64_t hits = 0;        /* already on the device */
    uint64_t in_flight = 0;   /* on its way (a guess's copy still running) */
    uint64_t misses = 0;      /* copied when asked for */
    uint64_t prefetched = 0;  /* copied for a guess */
    uint64_t prefetch_used = 0;
    uint64_t copies = 0, bytes_copied = 0;
};

struct expert_cache {
    bool on = false;
    int n_layers = 0, E = 0, K = 0;
    int n_slots = 0;
    size_t slot_bytes = 0, n_places = 0;
    /* a slot's layout for each layer: where gate, up and down start, their dtypes and shapes, and the bytes a copy
       of that layer's expert moves */
    std::vector<size_t> part_off, fill_bytes;
    std::vector<int> part_dtype, part_rows, part_cols;
    uint8_t* mem = nullptr;   /* device: n_slots x slot_bytes */
    uint8_t* host = nullptr;  /* page-locked: n_places x slot_bytes */
    std::vector<ec_slot> slots;
    std::set<int> empty;          /* empty slots, lowest first */
    std::vector<int32_t> where;   /* [n_places]: the slot holding each place, or -1 */
    std::vector<uint32_t> uses;   /* [n_places] */
    uint64_t request = 1;         /* the open request's number */
    uint64_t clock = 0;
    ec_counts n;
    hipStream_t copy = nullptr;
    hipEvent_t queued = nullptr;  /* the compute stream's work before a request */
};

/* The cache for model m when expert_cache_bytes leaves fewer slots than places; *on false (nothing allocated)
   when it holds every expert, or is 0. Refuses, with the sizes, when the host cannot pin the image. */
bool ec_create(expert_cache& c, const vitna_llama_t* m, size_t expert_cache_bytes, char* err, size_t err_len);
void ec_destroy(expert_cache& c);

/* Layer l's gate, up or down (part 0, 1, 2) over the slots: expert index = slot. */
qmat ec_view(const expert_cache& c, int layer, int part);

/* One token's experts of a layer (ids[0..k), distinct): uses counted, the places present pinned, those lacking
   copied in (in the order of ids) after every kernel queued on compute; slot_of[i] the slot of ids[i]. The slots
   stay pinned until ec_finish. */
bool ec_acquire(expert_cache& c, int layer, const int32_t* ids, int k, hipStream_t compute, int32_t* slot_of, char* err,
                size_t err_len);
/* compute made to wait for the copies into slot_of[0..k) that may still run. */
bool ec_wait(expert_cache& c, const int32_t* slot_of, int k, hipStream_t compute, char* err, size_t err_len);
/* After the layer's kernels are queued: the guess's copies for layer + 1 (its first ceil(k / 2) places), then the
   request closed. */
bool ec_finish(expert_cache& c, int layer, const int32_t* guess, int k, char* err, size_t err_len);

/* A pass of rows. ec_rows_count: layer's expert x asked for by cnt[x] rows, each a use; the halving whenever the
   requests cross a multiple of 65,536. */
void ec_rows_count(expert_cache& c, int layer, const int32_t* cnt);
/* One wave of the pass: experts xs[0..nx) in order of expert (nx at most n_slots - k), x wanted by cnt[x] rows.
   Opens a request (the previous wave's pins drop), orders the copies after compute's queued kernels, pins the
   experts present and copies in those lacking, k at a time as they are met; slot_of[x] set. */
bool ec_rows_wave(expert_cache& c, int layer, const int32_t* xs, int nx, const int32_t* cnt, hipStream_t compute,
                  int32_t* slot_of, char* err, size_t err_len);
/* After the pass's kernels: of each row's guess (n x k, by rank) the first ceil(k / 2) experts, each once, copied
   in while a slot can be taken; then the request closed. */
bool ec_rows_finish(expert_cache& c, int layer, const int32_t* guess, int n, int k, char* err, size_t err_len);

/* The reference's summary line (model_cuda.cu:4946-4953). */
void ec_report(const expert_cache& c, char* buf, size_t len);

#endif
