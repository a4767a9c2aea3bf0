/**
 * expert_cache.hip - The device's expert cache (expert_cache.h): the slot
 * layout, the host image, the slot table and its copies. Host code only.
 */

#include "expert_cache.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <algorithm>

namespace {

bool say_no(char* err, size_t len, const char* fmt, ...) {
    if (err && len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, len, fmt, ap);
        va_end(ap);
    }
    return false;
}

bool hip_ok(hipError_t e, const char* what, char* err, size_t len) {
    return e == hipSuccess || say_no(err, len, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

/* The planes of one matrix at base (vitna_hip_internal.h), each 256-byte aligned, one after another. */
qmat planes_at(uint8_t* base, int dtype, size_t rows, size_t cols) {
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

size_t planes_bytes(int dtype, size_t rows, size_t cols) {
    size_t t = 0;
    for (int i = 0; i < 4; i++) t += align256(plane_bytes(dtype, i, rows, cols));
    return t;
}

/* Field f of every GGUF block of a matrix into its plane: (offset in the block, bytes, plane). */
struct field {
    int at, len, plane;
};

/* GGUF blocks into planes on the host: the regrouping repack_kernel makes on the device. */
void split_blocks(const uint8_t* src, const qmat& q) {
    static const field q8[] = {{0, 2, 1}, {2, 32, 0}};
    static const field q4[] = {{0, 16, 1}, {16, 128, 0}};
    static const field q6[] = {{0, 128, 0}, {128, 64, 1}, {192, 16, 2}, {208, 2, 3}};
    const field* fs = q.dtype == VITNA_DTYPE_Q8_0 ? q8 : q.dtype == VITNA_DTYPE_Q4_K ? q4 : q6;
    const int nf = q.dtype == VITNA_DTYPE_Q6_K ? 4 : 2;
    const int bb = q.dtype == VITNA_DTYPE_Q8_0 ? 34 : q.dtype == VITNA_DTYPE_Q4_K ? 144 : 210;
    const size_t blocks = (size_t)q.rows * q.nb;
    for (int f = 0; f < nf; f++) {
        uint8_t* dst = const_cast<uint8_t*>(q.p[fs[f].plane]);
        for (size_t b = 0; b < blocks; b++) memcpy(dst + b * fs[f].len, src + b * bb + fs[f].at, fs[f].len);
    }
}

/* MemAvailable of /proc/meminfo in bytes, or 0 when it cannot be read. */
size_t host_available() {
    FILE* f = fopen("/proc/meminfo", "r");
    if (!f) return 0;
    char line[256];
    size_t kib = 0;
    while (fgets(line, sizeof(line), f))
        if (sscanf(line, "MemAvailable: %zu kB", &kib) == 1) break;
    fclose(f);
    return kib * 1024;
}

bool pinned(const expert_cache& c, int s) { return c.slots[s].pin == c.request; }

/* Whether slot s's copy has landed; false with err when the copy failed. */
bool settle(expert_cache& c, int s, char* err, size_t len) {
    ec_slot& x = c.slots[s];
    if (!x.copying) return true;
    const hipError_t q = hipEventQuery(x.landed);
    if (q == hipSuccess) x.copying = false;
    else if (q != hipErrorNotReady) return say_no(err, len, "an expert copy failed: %s", hipGetErrorString(q));
    return true;
}

/* The slot a new place takes: the lowest empty one, else the unpinned slot of least (uses, stamp); -1 when every
   slot is pinned. Stamps are distinct, so the key orders the candidates strictly. */
int victim(const expert_cache& c) {
    if (!c.empty.empty()) return *c.empty.begin();
    int best = -1;
    uint32_t bu = 0;
    uint64_t bs = 0;
    for (int s = 0; s < c.n_slots; s++) {
        if (pinned(c, s)) continue;
        const uint32_t u = c.uses[c.slots[s].place];
        const uint64_t st = c.slots[s].stamp;
        if (best < 0 || u < bu || (u == bu && st < bs)) {
            best = s;
            bu = u;
            bs = st;
        }
    }
    return best;
}

/* The place's copy into slot s, queued on the copy stream; s pinned and stamped. */
bool load(expert_cache& c, int s, size_t place, bool guess, char* err, size_t len) {
    ec_slot& x = c.slots[s];
    if (x.place >= 0) c.where[x.place] = -1;
    c.empty.erase(s);
    x.place = (int64_t)place;
    x.pin = c.request;
    x.stamp = ++c.clock;
    x.from_guess = guess;
    x.copying = true;
    c.where[place] = s;
    const size_t bytes = c.fill_bytes[place / c.E];
    c.n.copies++;
    c.n.bytes_copied += bytes;
    hipError_t e = hipMemcpyAsync(c.mem + (size_t)s * c.slot_bytes, c.host + place * c.slot_bytes, bytes, hipMemcpyHostToDevice, c.copy);
    if (e == hipSuccess) e = hipEventRecord(x.landed, c.copy);
    if (e != hipSuccess) {
        /* what the slot holds is unknown: it goes back to empty */
        c.where[place] = -1;
        x.place = -1;
        x.copying = false;
        c.empty.insert(s);
        return hip_ok(e, "copying an expert to the device", err, len);
    }
    return true;
}

/* A present place's slot pinned and stamped for a request asking rows times; its copy's state counted. */
bool touch(expert_cache& c, int s, uint64_t rows, char* err, size_t len) {
    ec_slot& x = c.slots[s];
    x.pin = c.request;
    x.stamp = ++c.clock;
    if (!settle(c, s, err, len)) return false;
    (x.copying ? c.n.in_flight : c.n.hits) += rows;
    if (x.from_guess) {
        c.n.prefetch_used++;
        x.from_guess = false;
    }
    return true;
}

/* n more requests of place; every count halved when the total crosses a multiple of 65,536. */
void count(expert_cache& c, size_t place, uint64_t n) {
    c.uses[place] += (uint32_t)n;
    const uint64_t was = c.n.acquired;
    c.n.acquired += n;
    if (was >> 16 != c.n.acquired >> 16)
        for (uint32_t& u : c.uses) u >>= 1;
}

/* A new request: every slot unpinned, the copies ordered after the kernels compute holds so far. */
bool open_request(expert_cache& c, hipStream_t compute, char* err, size_t len) {
    c.request++;
    return hip_ok(hipEventRecord(c.queued, compute), "ordering the expert copies", err, len) &&
           hip_ok(hipStreamWaitEvent(c.copy, c.queued, 0), "ordering the expert copies", err, len);
}

/* The guess's places copied in while a slot can be taken: those present or already taken are passed over. */
bool guess_in(expert_cache& c, const std::vector<size_t>& places, char* err, size_t len) {
    for (size_t place : places) {
        if (c.where[place] >= 0) continue;
        const int s = victim(c);
        if (s < 0) break;
        if (!load(c, s, place, true, err, len)) return false;
        c.n.prefetched++;
    }
    return true;
}

}  // namespace

void ec_destroy(expert_cache& c) {
    if (c.copy) (void)hipStreamSynchronize(c.copy);
    for (ec_slot& s : c.slots)
        if (s.landed) (void)hipEventDestroy(s.landed);
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
    c.part_off.resize(3 * cfg->n_layers);
    c.part_dtype.resize(3 * cfg->n_layers);
    c.part_rows.resize(3 * cfg->n_layers);
    c.part_cols.resize(3 * cfg->n_layers);
    c.fill_bytes.resize(cfg->n_layers);
    /* a slot: the layer's gate, up and down planes one after another; the widest layer sets the slot */
    for (int l = 0; l < c.n_layers; l++) {
        const vitna_expert_t& x0 = m->layers[l].experts[0];
        const vitna_matrix_t* parts[3] = {&x0.gate, &x0.up, &x0.down};
        size_t at = 0;
        for (int p = 0; p < 3; p++) {
            const int i = 3 * l + p;
            c.part_off[i] = at;
            c.part_dtype[i] = parts[p]->dtype;
            c.part_rows[i] = (int)parts[p]->rows;
            c.part_cols[i] = (int)parts[p]->cols;
            at += planes_bytes(parts[p]->dtype, parts[p]->rows, parts[p]->cols);
        }
        c.fill_bytes[l] = at;
        c.slot_bytes = std::max(c.slot_bytes, at);
    }
    if (expert_cache_bytes == 0) return true;
    const size_t slots = expert_cache_bytes / c.slot_bytes;
    if (slots >= c.n_places) return true; /* a slot for every expert: all resident */
    const size_t need = 2 * (size_t)c.K;  /* a layer's experts and its guess at the next layer's */
    if (slots < need)
        return say_no(err, err_len, "the GPU's expert cache must hold twice the experts a token goes through: %zu MiB or more",
                      (need * c.slot_bytes + ((size_t)1 << 20) - 1) >> 20);
    /* the host image pins a slot's bytes for every expert of every layer */
    const size_t image = c.n_places * c.slot_bytes, avail = host_available();
    if (avail && image > avail)
        return say_no(err, err_len,
                      "the expert cache keeps a page-locked image of every expert in host memory: %.1f GiB, and the host has %.1f GiB "
                      "available",
                      image / 1073741824.0, avail / 1073741824.0);
    c.n_slots = (int)slots;
    if (!hip_ok(hipMalloc(&c.mem, slots * c.slot_bytes), "device memory for the expert cache", err, err_len)) return false;
    if (!hip_ok(hipHostMalloc((void**)&c.host, image, 0), "page-locked host memory for the experts' image", err, err_len)) return false;
    for (size_t place = 0; place < c.n_places; place++) {
        const int l = (int)(place / c.E);
        const vitna_expert_t& ex = m->layers[l].experts[place % c.E];
        const vitna_matrix_t* parts[3] = {&ex.gate, &ex.up, &ex.down};
        uint8_t* base = c.host + place * c.slot_bytes;
        for (int p = 0; p < 3; p++)
            split_blocks(static_cast<const uint8_t*>(parts[p]->data),
                         planes_at(base + c.part_off[3 * l + p], parts[p]->dtype, parts[p]->rows, parts[p]->cols));
    }
    c.slots.resize(slots);
    for (int s = 0; s < c.n_slots; s++) {
        if (!hip_ok(hipEventCreateWithFlags(&c.slots[s].landed, hipEventDisableTiming), "an event of the expert cache", err, err_len))
            return false;
        c.empty.insert(s);
    }
    if (!hip_ok(hipEventCreateWithFlags(&c.queued, hipEventDisableTiming), "an event of the expert cache", err, err_len) ||
        !hip_ok(hipStreamCreateWithFlags(&c.copy, hipStreamNonBlocking), "the expert cache's copy stream", err, err_len))
        return false;
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

bool ec_acquire(expert_cache& c, int layer, const int32_t* ids, int k, hipStream_t compute, int32_t* slot_of, char* err, size_t err_len) {
    if (!open_request(c, compute, err, err_len)) return false;
    const size_t base = (size_t)layer * c.E;
    /* every place present is pinned before any copy chooses its slot, so a copy never takes one of them */
    for (int i = 0; i < k; i++) {
        const size_t place = base + ids[i];
        count(c, place, 1);
        slot_of[i] = c.where[place];
        if (slot_of[i] >= 0 && !touch(c, slot_of[i], 1, err, err_len)) return false;
    }
    for (int i = 0; i < k; i++) {
        if (slot_of[i] >= 0) continue;
        c.n.misses++;
        const int s = victim(c); /* k are pinned at most, of 2k or more */
        if (s < 0) return say_no(err, err_len, "internal: every expert slot is pinned");
        if (!load(c, s, base + ids[i], false, err, err_len)) return false;
        slot_of[i] = s;
    }
    return true;
}

bool ec_wait(expert_cache& c, const int32_t* slot_of, int k, hipStream_t compute, char* err, size_t err_len) {
    for (int i = 0; i < k; i++)
        if (c.slots[slot_of[i]].copying &&
            !hip_ok(hipStreamWaitEvent(compute, c.slots[slot_of[i]].landed, 0), "waiting for an expert's copy", err, err_len))
            return false;
    return true;
}

bool ec_finish(expert_cache& c, int layer, const int32_t* guess, int k, char* err, size_t err_len) {
    std::vector<size_t> places;
    if (guess && layer + 1 < c.n_layers)
        for (int j = 0; j < (k + 1) / 2; j++) places.push_back((size_t)(layer + 1) * c.E + guess[j]);
    const bool ok = guess_in(c, places, err, err_len);
    c.request++;
    return ok;
}

void ec_rows_count(expert_cache& c, int layer, const int32_t* cnt) {
    for (int x = 0; x < c.E; x++)
        if (cnt[x]) count(c, (size_t)layer * c.E + x, (uint64_t)cnt[x]);
}

bool ec_rows_wave(expert_cache& c, int layer, const int32_t* xs, int nx, const int32_t* cnt, hipStream_t compute,
                  int32_t* slot_of, char* err, size_t err_len) {
    if (nx < 1 || nx > c.n_slots - c.K) return say_no(err, err_len, "internal: a wave of %d experts", nx);
    if (!open_request(c, compute, err, err_len)) return false;
    const size_t base = (size_t)layer * c.E;
    /* the experts lacking are copied k at a time, each group as soon as it is complete: a copy may therefore take
       the slot of an expert later in the wave that is not pinned yet, which is then copied in again in turn */
    std::vector<int32_t> lacking;
    auto copy_lacking = [&]() {
        for (int32_t x : lacking) {
            const int s = victim(c); /* at most n_slots - k are pinned */
            if (s < 0) return say_no(err, err_len, "internal: every expert slot is pinned");
            if (!load(c, s, base + x, false, err, err_len)) return false;
            slot_of[x] = s;
        }
        lacking.clear();
        return true;
    };
    for (int i = 0; i < nx; i++) {
        const int32_t x = xs[i];
        const int s = c.where[base + x];
        if (s >= 0) {
            if (!touch(c, s, (uint64_t)cnt[x], err, err_len)) return false;
            slot_of[x] = s;
            continue;
        }
        /* one copy serves all its rows: the first row's request is the miss, the others find it */
        c.n.misses++;
        c.n.hits += (uint64_t)cnt[x] - 1;
        lacking.push_back(x);
        if ((int)lacking.size() == c.K && !copy_lacking()) return false;
    }
    return copy_lacking();
}

bool ec_rows_finish(expert_cache& c, int layer, const int32_t* guess, int n, int k, char* err, size_t err_len) {
    std::vector<size_t> places;
    if (guess && layer + 1 < c.n_layers) {
        std::vector<uint8_t> seen(c.E, 0);
        for (int t = 0; t < n; t++)
            for (int j = 0; j < (k + 1) / 2; j++) {
                const int32_t x = guess[(size_t)t * k + j];
                if (!seen[x]) {
                    seen[x] = 1;
                    places.push_back((size_t)(layer + 1) * c.E + x);
                }
            }
    }
    const bool ok = guess_in(c, places, err, err_len);
    c.request++;
    return ok;
}

void ec_report(const expert_cache& c, char* buf, size_t len) {
    snprintf(buf, len,
             "experts on the GPU: %d slots, %.0f MiB, copied from %s, %s. %llu acquired: %llu already on the GPU, %llu still being copied "
             "for a guess, %llu copied when asked for. %llu copied for a guess, %llu of those used. %.1f MiB copied in %llu copies",
             c.n_slots, (double)c.n_slots * (double)c.slot_bytes / 1048576.0, "a page-locked copy of every expert in host memory",
             "page-locked", (unsigned long long)c.n.acquired, (unsigned long long)c.n.hits, (unsigned long long)c.n.in_flight,
             (unsigned long long)c.n.misses, (unsigned long long)c.n.prefetched, (unsigned long long)c.n.prefetch_used,
             (double)c.n.bytes_copied / 1048576.0, (unsigned long long)c.n.copies);
}
