/**
 * expert_cache.hip - The device's expert cache (expert_cache.h): layout, the
 * host copy, the slot rule and the copies. Host code only.
 */

#include "expert_cache.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <algorithm>

static bool ec_fail(char* err, size_t len, const char* fmt, ...) {
    if (err && len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, len, fmt, ap);
        va_end(ap);
    }
    return false;
}

#define EC_TRY(call, what)                                                                                          \
    do {                                                                                                            \
        const hipError_t e_ = (call);                                                                               \
        if (e_ != hipSuccess) return ec_fail(err, err_len, "%s: %s (%s)", what, hipGetErrorString(e_), hipGetErrorName(e_)); \
    } while (0)

/* The planes of one matrix at base (vitna_hip_internal.h), planes 256-byte aligned one after another. */
static qmat planes_at(uint8_t* base, int dtype, size_t rows, size_t cols) {
    qmat q;
    memset(&q, 0, sizeof(q));
    size_t off = 0;
    for (int i = 0; i < 4; i++) {
        const size_t pb = plane_bytes(dtype, i, rows, cols);
        q.p[i] = pb ? base + off : nullptr;
        off += align256(pb);
    }
    q.rows = (int)rows;
    q.cols = (int)cols;
    q.nb = (int)(cols / (dtype == VITNA_DTYPE_Q8_0 ? 32 : 256));
    q.dtype = dtype;
    return q;
}

static size_t planes_bytes(int dtype, size_t rows, size_t cols) {
    size_t t = 0;
    for (int i = 0; i < 4; i++) t += align256(plane_bytes(dtype, i, rows, cols));
    return t;
}

/* GGUF blocks into planes on the host: the same regrouping repack_kernel makes on the device. */
static void repack_host(const uint8_t* src, const qmat& q) {
    uint8_t* P[4] = {const_cast<uint8_t*>(q.p[0]), const_cast<uint8_t*>(q.p[1]), const_cast<uint8_t*>(q.p[2]), const_cast<uint8_t*>(q.p[3])};
    const size_t n = (size_t)q.rows * q.nb;
    for (size_t i = 0; i < n; i++) {
        if (q.dtype == VITNA_DTYPE_Q8_0) {
            const uint8_t* b = src + i * 34;
            memcpy(P[1] + i * 2, b, 2);
            memcpy(P[0] + i * 32, b + 2, 32);
        } else if (q.dtype == VITNA_DTYPE_Q4_K) {
            const uint8_t* b = src + i * 144;
            memcpy(P[1] + i * 16, b, 16);
            memcpy(P[0] + i * 128, b + 16, 128);
        } else {
            const uint8_t* b = src + i * 210;
            memcpy(P[0] + i * 128, b, 128);
            memcpy(P[1] + i * 64, b + 128, 64);
            memcpy(P[2] + i * 16, b + 192, 16);
            memcpy(P[3] + i * 2, b + 208, 2);
        }
    }
}

void ec_destroy(expert_cache& c) {
    if (c.copy) (void)hipStreamSynchronize(c.copy);
    for (ec_slot& s : c.slots)
        if (s.filled) (void)hipEventDestroy(s.filled);
    if (c.queued) (void)hipEventDestroy(c.queued);
    if (c.copy) (void)hipStreamDestroy(c.copy);
    if (c.mem) (void)hipFree(c.mem);
    if (c.host) (void)hipHostFree(c.host);
    c = expert_cache();
}

bool ec_create(expert_cache& c, const vitna_llama_t* m, size_t expert_cache_bytes, char* err, size_t err_len) {
    const vitna_llama_config_t* cfg = &m->cfg;
    c = expert_cache();
    c.n_layers = (int)cfg->n_layers;
    c.E = (int)cfg->n_experts;
    c.K = (int)cfg->n_experts_used;
    c.n_places = cfg->n_layers * cfg->n_experts;
    c.part_off.assign(3 * cfg->n_layers, 0);
    c.used_bytes.assign(cfg->n_layers, 0);
    c.part_dtype.assign(3 * cfg->n_layers, 0);
    c.part_rows.assign(3 * cfg->n_layers, 0);
    c.part_cols.assign(3 * cfg->n_layers, 0);
    /* a slot: the layer's gate, up and down planes one after another; the widest layer sets its size */
    for (int l = 0; l < c.n_layers; l++) {
        const vitna_expert_t* x0 = &m->layers[l].experts[0];
        const vitna_matrix_t* parts[3] = {&x0->gate, &x0->up, &x0->down};
        size_t off = 0;
        for (int p = 0; p < 3; p++) {
            c.part_off[3 * l + p] = off;
            c.part_dtype[3 * l + p] = parts[p]->dtype;
            c.part_rows[3 * l + p] = (int)parts[p]->rows;
            c.part_cols[3 * l + p] = (int)parts[p]->cols;
            off += planes_bytes(parts[p]->dtype, parts[p]->rows, parts[p]->cols);
        }
        c.used_bytes[l] = off;
        c.slot_bytes = std::max(c.slot_bytes, off);
    }
    if (expert_cache_bytes == 0) return true;
    size_t slots = expert_cache_bytes / c.slot_bytes;
    if (slots >= c.n_places) return true; /* a slot for every expert: they are all resident */
    const size_t need = 2 * (size_t)c.K;  /* a layer's experts and its guess at the next layer's */
    if (slots < need)
        return ec_fail(err, err_len, "the GPU's expert cache must hold twice the experts a token goes through: %zu MiB or more",
                       (need * c.slot_bytes + ((size_t)1 << 20) - 1) >> 20);
    c.n_slots = (int)slots;
    EC_TRY(hipMalloc(&c.mem, slots * c.slot_bytes), "device memory for the expert cache");
    EC_TRY(hipHostMalloc((void**)&c.host, c.n_places * c.slot_bytes, 0), "page-locked host memory for the experts");
    for (int l = 0; l < c.n_layers; l++)
        for (int x = 0; x < c.E; x++) {
            const vitna_expert_t* ex = &m->layers[l].experts[x];
            const vitna_matrix_t* parts[3] = {&ex->gate, &ex->up, &ex->down};
            uint8_t* base = c.host + ((size_t)l * c.E + x) * c.slot_bytes;
            for (int p = 0; p < 3; p++)
                repack_host((const uint8_t*)parts[p]->data,
                            planes_at(base + c.part_off[3 * l + p], parts[p]->dtype, parts[p]->rows, parts[p]->cols));
        }
    c.slots.resize(slots);
    for (ec_slot& s : c.slots) EC_TRY(hipEventCreateWithFlags(&s.filled, hipEventDisableTiming), "an event of the expert cache");
    EC_TRY(hipEventCreateWithFlags(&c.queued, hipEventDisableTiming), "an event of the expert cache");
    EC_TRY(hipStreamCreateWithFlags(&c.copy, hipStreamNonBlocking), "the expert cache's copy stream");
    c.where.assign(c.n_places, -1);
    c.uses.assign(c.n_places, 0);
    c.on = true;
    return true;
}

qmat ec_view(const expert_cache& c, int layer, int part) {
    const int i = 3 * layer + part;
    qmat q = planes_at(c.mem + c.part_off[i], c.part_dtype[i], c.part_rows[i], c.part_cols[i]);
    for (int p = 0; p < 4; p++) q.estride[p] = q.p[p] ? c.slot_bytes : 0;
    return q;
}

/* An empty slot, else the least used of those not held, the least recently used between equals; -1 if every slot
   is held (model_cuda.cu:4334-4352). */
static int free_slot(const expert_cache& c) {
    int best = -1;
    for (int i = 0; i < c.n_slots; i++) {
        const ec_slot& x = c.slots[i];
        if (x.held) continue;
        if (x.place < 0) return i;
        if (best < 0) {
            best = i;
            continue;
        }
        const ec_slot& b = c.slots[best];
        const uint32_t ux = c.uses[x.place], ub = c.uses[b.place];
        if (ux < ub || (ux == ub && x.last_use < b.last_use)) best = i;
    }
    return best;
}

/* Slot s given to place, held, its copy queued on the copy stream (model_cuda.cu:4355-4391). */
static bool fill(expert_cache& c, int s, size_t place, bool guessed, char* err, size_t err_len) {
    ec_slot& x = c.slots[s];
    if (x.place >= 0) c.where[x.place] = -1;
    x.place = (int64_t)place;
    c.where[place] = s;
    x.held = true;
    x.guessed = guessed;
    x.last_use = ++c.clock;
    x.filling = true;
    const size_t layer = place / c.E, bytes = c.used_bytes[layer];
    hipError_t e = hipMemcpyAsync(c.mem + (size_t)s * c.slot_bytes, c.host + place * c.slot_bytes, bytes, hipMemcpyHostToDevice, c.copy);
    if (e == hipSuccess) e = hipEventRecord(x.filled, c.copy);
    c.copies++;
    c.bytes_copied += bytes;
    if (e != hipSuccess) {
        /* the slot cannot be trusted: empty */
        c.where[place] = -1;
        x.place = -1;
        return ec_fail(err, err_len, "copying an expert to the device: %s (%s)", hipGetErrorString(e), hipGetErrorName(e));
    }
    return true;
}

static void count_use(expert_cache& c, size_t place) {
    c.uses[place]++;
    if (++c.acquired % 65536 == 0)
        for (uint32_t& u : c.uses) u /= 2;
}

bool ec_acquire(expert_cache& c, int layer, const int32_t* ids, int k, hipStream_t compute, int32_t* slot_of, char* err, size_t err_len) {
    /* copies into slots start after every kernel queued so far */
    EC_TRY(hipEventRecord(c.queued, compute), "ordering the expert copies");
    EC_TRY(hipStreamWaitEvent(c.copy, c.queued, 0), "ordering the expert copies");
    int miss_at[ROUTE_K_MAX], n_miss = 0;
    for (int i = 0; i < k; i++) {
        const size_t place = (size_t)layer * c.E + ids[i];
        count_use(c, place);
        const int s = c.where[place];
        slot_of[i] = s;
        if (s < 0) {
            miss_at[n_miss++] = i;
            c.misses++;
            continue;
        }
        ec_slot& x = c.slots[s];
        x.held = true;
        x.last_use = ++c.clock;
        if (x.filling) {
            const hipError_t q = hipEventQuery(x.filled);
            if (q == hipSuccess) x.filling = false;
            else if (q != hipErrorNotReady) return ec_fail(err, err_len, "an expert copy failed: %s", hipGetErrorString(q));
        }
        if (x.filling) c.in_flight++;
        else c.hits++;
        if (x.guessed) {
            c.prefetch_used++;
            x.guessed = false;
        }
    }
    for (int j = 0; j < n_miss; j++) {
        const int i = miss_at[j];
        const int s = free_slot(c); /* at most k slots are held and there are at least 2k */
        if (s < 0) return ec_fail(err, err_len, "internal: no expert slot free");
        if (!fill(c, s, (size_t)layer * c.E + ids[i], false, err, err_len)) return false;
        slot_of[i] = s;
    }
    return true;
}

bool ec_wait(expert_cache& c, const int32_t* slot_of, int k, hipStream_t compute, char* err, size_t err_len) {
    for (int i = 0; i < k; i++) {
        const ec_slot& x = c.slots[slot_of[i]];
        if (x.filling) EC_TRY(hipStreamWaitEvent(compute, x.filled, 0), "waiting for an expert's copy");
    }
    return true;
}

bool ec_finish(expert_cache& c, int layer, const int32_t* guess, int k, char* err, size_t err_len) {
    bool ok = true;
    if (guess && layer + 1 < c.n_layers) {
        /* the upper half of the guess, by the next router's rank (model_cuda.cu:4886-4910) */
        for (int j = 0; ok && j < (k + 1) / 2; j++) {
            const size_t place = (size_t)(layer + 1) * c.E + guess[j];
            if (c.where[place] >= 0) continue;
            const int s = free_slot(c);
            if (s < 0) break;
            ok = fill(c, s, place, true, err, err_len);
            c.prefetched++;
        }
    }
    for (ec_slot& x : c.slots) x.held = false;
    return ok;
}

void ec_rows_count(expert_cache& c, int layer, const int32_t* cnt) {
    for (int x = 0; x < c.E; x++) {
        if (!cnt[x]) continue;
        c.uses[(size_t)layer * c.E + x] += (uint32_t)cnt[x];
        const uint64_t before = c.acquired;
        c.acquired += (uint64_t)cnt[x];
        if (before / 65536 != c.acquired / 65536)
            for (uint32_t& u : c.uses) u /= 2;
    }
}

bool ec_rows_wave(expert_cache& c, int layer, const int32_t* xs, int nx, const int32_t* cnt, hipStream_t compute,
                  int32_t* slot_of, char* err, size_t err_len) {
    if (nx < 1 || nx > c.n_slots - c.K) return ec_fail(err, err_len, "internal: a wave of %d experts", nx);
    /* the previous wave's slots are free to give up: its kernels are queued before the copies that may replace them */
    for (ec_slot& x : c.slots) x.held = false;
    EC_TRY(hipEventRecord(c.queued, compute), "ordering the expert copies");
    EC_TRY(hipStreamWaitEvent(c.copy, c.queued, 0), "ordering the expert copies");
    int batch[ROUTE_K_MAX], nb = 0;
    for (int i = 0; i <= nx; i++) {
        if (i < nx) {
            const int x = xs[i];
            const size_t place = (size_t)layer * c.E + x;
            const int s = c.where[place];
            if (s >= 0) {
                ec_slot& sl = c.slots[s];
                sl.held = true;
                sl.last_use = ++c.clock;
                if (sl.filling) {
                    const hipError_t q = hipEventQuery(sl.filled);
                    if (q == hipSuccess) sl.filling = false;
                    else if (q != hipErrorNotReady) return ec_fail(err, err_len, "an expert copy failed: %s", hipGetErrorString(q));
                }
                if (sl.filling) c.in_flight += (uint64_t)cnt[x];
                else c.hits += (uint64_t)cnt[x];
                if (sl.guessed) {
                    c.prefetch_used++;
                    sl.guessed = false;
                }
                slot_of[x] = s;
                continue;
            }
            /* copied once for all its rows: the first row's request a miss, the others' hits */
            c.misses++;
            c.hits += (uint64_t)cnt[x] - 1;
            batch[nb++] = x;
            if (nb < c.K) continue;
        }
        for (int j = 0; j < nb; j++) {
            const int s = free_slot(c); /* at most n_slots - k are held */
            if (s < 0) return ec_fail(err, err_len, "internal: no expert slot free");
            if (!fill(c, s, (size_t)layer * c.E + batch[j], false, err, err_len)) return false;
            slot_of[batch[j]] = s;
        }
        nb = 0;
    }
    return true;
}

bool ec_rows_finish(expert_cache& c, int layer, const int32_t* guess, int n, int k, char* err, size_t err_len) {
    bool ok = true;
    if (guess && layer + 1 < c.n_layers) {
        std::vector<uint8_t> mark(c.E, 0);
        bool room = true;
        for (int t = 0; ok && room && t < n; t++) {
            for (int j = 0; ok && j < (k + 1) / 2; j++) {
                const int x = guess[(size_t)t * k + j];
                if (mark[x]) continue;
                mark[x] = 1;
                const size_t place = (size_t)(layer + 1) * c.E + x;
                if (c.where[place] >= 0) continue;
                const int s = free_slot(c);
                if (s < 0) {
                    room = false;
                    break;
                }
                ok = fill(c, s, place, true, err, err_len);
                c.prefetched++;
            }
        }
    }
    for (ec_slot& x : c.slots) x.held = false;
    return ok;
}

void ec_report(const expert_cache& c, char* buf, size_t len) {
    snprintf(buf, len,
             "experts on the GPU: %d slots, %.0f MiB, copied from %s, %s. %llu acquired: %llu already on the GPU, %llu still being copied "
             "for a guess, %llu copied when asked for. %llu copied for a guess, %llu of those used. %.1f MiB copied in %llu copies",
             c.n_slots, (double)c.n_slots * (double)c.slot_bytes / 1048576.0, "a page-locked copy of every expert in host memory",
             "page-locked", (unsigned long long)c.acquired, (unsigned long long)c.hits, (unsigned long long)c.in_flight,
             (unsigned long long)c.misses, (unsigned long long)c.prefetched, (unsigned long long)c.prefetch_used,
             (double)c.bytes_copied / 1048576.0, (unsigned long long)c.copies);
}
