/**
 * vitna_synth.c - seeded synthetic models (vitna_synth.h).
 */

#include "vitna_synth.h"
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t splitmix(uint64_t* s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

typedef struct { uint64_t s[4]; } rng_t;

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static inline uint64_t rng_next(rng_t* r) {
    const uint64_t out = rotl(r->s[1] * 5, 7) * 9, t = r->s[1] << 17;
    r->s[2] ^= r->s[0];
    r->s[3] ^= r->s[1];
    r->s[1] ^= r->s[2];
    r->s[0] ^= r->s[3];
    r->s[2] ^= t;
    r->s[3] = rotl(r->s[3], 45);
    return out;
}

static rng_t rng_for(uint64_t seed, uint64_t tag, uint64_t row) {
    uint64_t k = seed ^ 0x5851f42d4c957f2dull;
    k = splitmix(&k) ^ tag;
    k = splitmix(&k) ^ row;
    rng_t r;
    for (int i = 0; i < 4; i++) r.s[i] = splitmix(&k);
    return r;
}

/* Uniform in (0, 1], 53 bits. */
static inline double unit(rng_t* r) { return (double)((rng_next(r) >> 11) + 1) * (1.0 / 9007199254740992.0); }

static inline double normal(rng_t* r) {
    const double u1 = unit(r), u2 = unit(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

uint16_t vitna_synth_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to infinity */
    if (ax < 0x38800000u) {
        /* subnormal half (or zero): value / 2^-24, rounded to nearest even */
        if (ax < 0x33000000u) return (uint16_t)sign;
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)e; /* 14 .. 24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

static void put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

static void fill_bytes(rng_t* r, uint8_t* p, size_t n) {
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        const uint64_t v = rng_next(r);
        memcpy(p + i, &v, 8);
    }
    if (i < n) {
        const uint64_t v = rng_next(r);
        memcpy(p + i, &v, n - i);
    }
}

static uint16_t scale16(rng_t* r, float mul) { return vitna_synth_f32_to_f16((float)(fabs(normal(r)) * (double)mul)); }

/* One row of a matrix. */
static void gen_row(int dtype, rng_t* r, size_t cols, float scale, uint8_t* out) {
    switch (dtype) {
        case VITNA_DTYPE_F32: {
            float* f = (float*)out;
            for (size_t c = 0; c < cols; c++) f[c] = (float)(normal(r) * (double)scale);
            break;
        }
        case VITNA_DTYPE_Q8_0:
            for (size_t b = 0; b < cols / 32; b++, out += 34) {
                put16(out, scale16(r, scale));
                for (int i = 0; i < 32; i += 4) {
                    const uint64_t v = rng_next(r);
                    for (int j = 0; j < 4; j++) {
                        const uint32_t u = (uint32_t)(v >> (16 * j)) & 0xffffu;
                        out[2 + i + j] = (uint8_t)(int8_t)((int)((u * 255u) >> 16) - 127);
                    }
                }
            }
            break;
        case VITNA_DTYPE_Q4_K:
            for (size_t b = 0; b < cols / 256; b++, out += 144) {
                put16(out, scale16(r, scale));
                put16(out + 2, scale16(r, scale));
                fill_bytes(r, out + 4, 140);
            }
            break;
        case VITNA_DTYPE_Q6_K:
            for (size_t b = 0; b < cols / 256; b++, out += 210) {
                fill_bytes(r, out, 192);
                const uint64_t v0 = rng_next(r), v1 = rng_next(r);
                for (int i = 0; i < 16; i++) {
                    const uint64_t v = i < 8 ? v0 : v1;
                    out[192 + i] = (uint8_t)(int8_t)((int)((v >> (8 * (i & 7))) & 63u) - 32);
                }
                put16(out + 208, scale16(r, scale));
            }
            break;
        default: break;
    }
}

typedef struct {
    int dtype;
    uint64_t seed, tag;
    size_t r0, r1, cols;
    float scale;
    uint8_t* out; /* row 0 of the matrix */
} gen_job_t;

typedef struct {
    gen_job_t* jobs;
    size_t n;
    size_t next;
    pthread_mutex_t lock;
} gen_queue_t;

static void run_job(const gen_job_t* j) {
    const size_t rb = vitna_matrix_row_bytes((vitna_dtype_t)j->dtype, j->cols);
    for (size_t row = j->r0; row < j->r1; row++) {
        rng_t r = rng_for(j->seed, j->tag, row);
        gen_row(j->dtype, &r, j->cols, j->scale, j->out + row * rb);
    }
}

static void* gen_worker(void* p) {
    gen_queue_t* q = (gen_queue_t*)p;
    for (;;) {
        pthread_mutex_lock(&q->lock);
        const size_t i = q->next++;
        pthread_mutex_unlock(&q->lock);
        if (i >= q->n) return NULL;
        run_job(&q->jobs[i]);
    }
}

static void run_jobs(gen_job_t* jobs, size_t n, int threads) {
    if (threads <= 0) threads = 8;
    if (threads > 64) threads = 64;
    gen_queue_t q = {jobs, n, 0, PTHREAD_MUTEX_INITIALIZER};
    pthread_t th[64];
    int started = 0;
    for (int t = 1; t < threads && (size_t)t < n; t++) {
        if (pthread_create(&th[started], NULL, gen_worker, &q) == 0) started++;
    }
    gen_worker(&q);
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
}

/* A growable list of jobs, big matrices cut into row ranges. */
typedef struct {
    gen_job_t* v;
    size_t n, cap;
    int failed;
} job_list_t;

static void add_matrix(job_list_t* L, int dtype, uint64_t seed, uint64_t tag, size_t rows, size_t cols, float scale, void* out) {
    const size_t rb = vitna_matrix_row_bytes((vitna_dtype_t)dtype, cols);
    if (!rb) { L->failed = 1; return; }
    size_t per = (1u << 20) / rb + 1; /* about a MiB a job */
    for (size_t r0 = 0; r0 < rows; r0 += per) {
        if (L->n == L->cap) {
            L->cap = L->cap ? 2 * L->cap : 1024;
            gen_job_t* nv = (gen_job_t*)realloc(L->v, L->cap * sizeof(gen_job_t));
            if (!nv) { L->failed = 1; return; }
            L->v = nv;
        }
        L->v[L->n++] = (gen_job_t){dtype, seed, tag, r0, r0 + per < rows ? r0 + per : rows, cols, scale, (uint8_t*)out};
    }
}

void vitna_synth_normal(uint64_t seed, uint64_t tag, float* out, size_t n) {
    /* rows of 4096 values, so long vectors can be regenerated piecewise */
    for (size_t r0 = 0; r0 < n; r0 += 4096) {
        rng_t r = rng_for(seed, tag, r0 / 4096);
        const size_t e = r0 + 4096 < n ? r0 + 4096 : n;
        for (size_t i = r0; i < e; i++) out[i] = (float)normal(&r);
    }
}

int vitna_synth_matrix(int dtype, uint64_t seed, uint64_t tag, size_t rows, size_t cols, float scale, void* out, int threads) {
    if (dtype != VITNA_DTYPE_F32 && dtype != VITNA_DTYPE_Q8_0 && dtype != VITNA_DTYPE_Q4_K && dtype != VITNA_DTYPE_Q6_K) return -1;
    job_list_t L = {0};
    add_matrix(&L, dtype, seed, tag, rows, cols, scale, out);
    if (!L.failed) run_jobs(L.v, L.n, threads);
    free(L.v);
    return L.failed ? -1 : 0;
}

/* Tags: the part in the low byte, the expert above it, the layer above that. */
enum { P_Q = 1, P_K, P_V, P_O, P_ROUTER, P_GATE, P_UP, P_DOWN, P_ATTN_NORM, P_MLP_NORM, P_QN, P_KN, P_EMBED, P_HEAD, P_FINAL };
static uint64_t tag_of(size_t layer, size_t expert, int part) { return ((uint64_t)(layer + 1) << 40) | ((uint64_t)expert << 8) | (uint64_t)part; }

static float scale_for(const vitna_synth_shape_t* s, int dtype) {
    if (dtype == VITNA_DTYPE_Q8_0) return s->q8_scale;
    return s->k_scale;
}

static float* norm_vec(const vitna_synth_shape_t* s, uint64_t seed, uint64_t tag, size_t n) {
    float* v = (float*)malloc(n * sizeof(float));
    if (!v) return NULL;
    if (s->norm_std == 0.0f) {
        for (size_t i = 0; i < n; i++) v[i] = 1.0f;
    } else {
        vitna_synth_normal(seed, tag, v, n);
        for (size_t i = 0; i < n; i++) v[i] = (float)(1.0 + (double)v[i] * (double)s->norm_std);
    }
    return v;
}

/* Memory the model owns besides the struct, released by vitna_synth_free:
   kept in a block after the struct. */
typedef struct {
    vitna_llama_t m;
    void* blobs[256];
    int n_blobs;
} synth_model_t;

static void* own(synth_model_t* sm, size_t bytes) {
    if (sm->n_blobs >= 256) return NULL;
    void* p = calloc(1, bytes ? bytes : 1);
    if (p) sm->blobs[sm->n_blobs++] = p;
    return p;
}

void vitna_synth_free(vitna_llama_t* m) {
    if (!m) return;
    synth_model_t* sm = (synth_model_t*)m;
    if (m->layers) {
        for (size_t l = 0; l < m->cfg.n_layers; l++) {
            free(m->layers[l].attn_norm);
            free(m->layers[l].mlp_norm);
            free(m->layers[l].q_norm);
            free(m->layers[l].k_norm);
            free(m->layers[l].experts);
            free((void*)m->layers[l].router.data);
            free((void*)m->layers[l].q.data);
            free((void*)m->layers[l].k.data);
            free((void*)m->layers[l].v.data);
            free((void*)m->layers[l].o.data);
        }
    }
    for (int i = 0; i < sm->n_blobs; i++) free(sm->blobs[i]);
    free(sm);
}

static int fail(char* err, size_t len, const char* msg) {
    if (err && len) snprintf(err, len, "%s", msg);
    return 0;
}

vitna_llama_t* vitna_synth_model(const vitna_synth_shape_t* s, uint64_t seed, int threads, char* err, size_t err_len) {
    const size_t H = s->hidden, I = s->intermediate, E = s->n_experts, K = s->n_experts_used, NL = s->n_layers;
    const size_t hd = s->head_dim, q_dim = s->n_heads * hd, kv_dim = s->n_kv_heads * hd;
    if (!H || !I || !E || !K || K > VITNA_EXPERTS_USED_MAX || K > E || !NL) {
        fail(err, err_len, "synthetic shape: hidden, intermediate, experts, experts used and layers must be set, experts used at most 64 and at most experts");
        return NULL;
    }
    synth_model_t* sm = (synth_model_t*)calloc(1, sizeof(synth_model_t));
    if (!sm) { fail(err, err_len, "out of memory"); return NULL; }
    vitna_llama_t* m = &sm->m;
    vitna_llama_config_t* c = &m->cfg;
    c->n_layers = NL;
    c->hidden = H;
    c->intermediate = I;
    c->n_heads = s->attention ? s->n_heads : 0;
    c->n_kv_heads = s->attention ? s->n_kv_heads : 0;
    c->head_dim = s->attention ? hd : 0;
    c->vocab = s->attention ? s->vocab : 0;
    c->max_positions = s->ctx;
    c->rms_eps = s->rms_eps;
    c->rope_theta = s->rope_theta;
    c->qk_norm = s->attention != 0;
    c->qk_norm_per_head = s->attention != 0;
    c->n_experts = E;
    c->n_experts_used = K;
    c->renormalize = s->renormalize != 0;
    c->qwen3 = s->renormalize != 0;
    m->ctx = s->ctx;
    m->seqs = s->seqs ? s->seqs : 1;
    m->predicted_layer = -1;

    job_list_t J = {0};
    m->layers = (vitna_llama_layer_t*)own(sm, NL * sizeof(vitna_llama_layer_t));
    const size_t gu_rb = vitna_matrix_row_bytes((vitna_dtype_t)s->dt_gate_up, H);
    const size_t dn_rb = vitna_matrix_row_bytes((vitna_dtype_t)s->dt_down, I);
    if (!m->layers || !gu_rb || !dn_rb) {
        vitna_synth_free(m);
        fail(err, err_len, "synthetic shape: the experts' widths are not whole blocks of their dtypes");
        return NULL;
    }
    const size_t ex_bytes = 2 * I * gu_rb + H * dn_rb;
    for (size_t l = 0; l < NL; l++) {
        vitna_llama_layer_t* L = &m->layers[l];
        L->mlp_norm = norm_vec(s, seed, tag_of(l, 0, P_MLP_NORM), H);
        L->router = (vitna_matrix_t){malloc(E * H * sizeof(float)), VITNA_DTYPE_F32, E, H};
        add_matrix(&J, VITNA_DTYPE_F32, seed, tag_of(l, 0, P_ROUTER), E, H, s->router_std, (void*)L->router.data);
        L->experts = (vitna_expert_t*)calloc(E, sizeof(vitna_expert_t));
        uint8_t* blob = (uint8_t*)own(sm, E * ex_bytes);
        if (!L->mlp_norm || !L->router.data || !L->experts || !blob) {
            free(J.v);
            vitna_synth_free(m);
            fail(err, err_len, "out of memory for the synthetic weights");
            return NULL;
        }
        for (size_t e = 0; e < E; e++) {
            uint8_t* p = blob + e * ex_bytes;
            vitna_expert_t* x = &L->experts[e];
            x->gate = (vitna_matrix_t){p, (vitna_dtype_t)s->dt_gate_up, I, H};
            x->up = (vitna_matrix_t){p + I * gu_rb, (vitna_dtype_t)s->dt_gate_up, I, H};
            x->down = (vitna_matrix_t){p + 2 * I * gu_rb, (vitna_dtype_t)s->dt_down, H, I};
            add_matrix(&J, s->dt_gate_up, seed, tag_of(l, e, P_GATE), I, H, scale_for(s, s->dt_gate_up), (void*)x->gate.data);
            add_matrix(&J, s->dt_gate_up, seed, tag_of(l, e, P_UP), I, H, scale_for(s, s->dt_gate_up), (void*)x->up.data);
            add_matrix(&J, s->dt_down, seed, tag_of(l, e, P_DOWN), H, I, scale_for(s, s->dt_down), (void*)x->down.data);
        }
        if (s->attention) {
            const int dts[4] = {s->dt_q, s->dt_k, s->dt_v, s->dt_o};
            const size_t rows[4] = {q_dim, kv_dim, kv_dim, H}, cols[4] = {H, H, H, q_dim};
            vitna_matrix_t* mats[4] = {&L->q, &L->k, &L->v, &L->o};
            for (int i = 0; i < 4; i++) {
                const size_t rb = vitna_matrix_row_bytes((vitna_dtype_t)dts[i], cols[i]);
                void* d = rb ? malloc(rows[i] * rb) : NULL;
                *mats[i] = (vitna_matrix_t){d, (vitna_dtype_t)dts[i], rows[i], cols[i]};
                if (!d) J.failed = 1;
                else add_matrix(&J, dts[i], seed, tag_of(l, 0, P_Q + i), rows[i], cols[i], scale_for(s, dts[i]), d);
            }
            L->attn_norm = norm_vec(s, seed, tag_of(l, 0, P_ATTN_NORM), H);
            L->q_norm = norm_vec(s, seed, tag_of(l, 0, P_QN), hd);
            L->k_norm = norm_vec(s, seed, tag_of(l, 0, P_KN), hd);
            if (!L->attn_norm || !L->q_norm || !L->k_norm) J.failed = 1;
        }
    }
    if (s->attention) {
        const size_t V = s->vocab;
        const size_t erb = vitna_matrix_row_bytes((vitna_dtype_t)s->dt_embed, H), hrb = vitna_matrix_row_bytes((vitna_dtype_t)s->dt_head, H);
        void* emb = erb ? own(sm, V * erb) : NULL;
        void* head = hrb ? own(sm, V * hrb) : NULL;
        m->embed = (vitna_matrix_t){emb, (vitna_dtype_t)s->dt_embed, V, H};
        m->lm_head = (vitna_matrix_t){head, (vitna_dtype_t)s->dt_head, V, H};
        m->final_norm = (float*)own(sm, H * sizeof(float));
        if (!emb || !head || !m->final_norm) J.failed = 1;
        else {
            add_matrix(&J, s->dt_embed, seed, tag_of(0, 0, P_EMBED) | (1ull << 60), V, H, scale_for(s, s->dt_embed), emb);
            add_matrix(&J, s->dt_head, seed, tag_of(0, 0, P_HEAD) | (1ull << 60), V, H, scale_for(s, s->dt_head), head);
            float* fnorm = norm_vec(s, seed, tag_of(0, 0, P_FINAL) | (1ull << 60), H);
            if (fnorm) { memcpy(m->final_norm, fnorm, H * sizeof(float)); free(fnorm); }
            else J.failed = 1;
        }
        const size_t half = hd / 2;
        m->inv_freq = (float*)own(sm, half * sizeof(float));
        if (m->inv_freq) {
            /* engine/src/model.c:388-393: 1 / theta^(2j / head_dim), float32 */
            for (size_t j = 0; j < half; j++) {
                const float e = (float)(2 * j) / (float)hd;
                m->inv_freq[j] = 1.0f / powf(s->rope_theta, e);
            }
        } else J.failed = 1;
    }
    if (s->kv_host) {
        /* what the engine's loader allocates for a step (engine/src/model.c:374-394) */
        const size_t cache = m->seqs * NL * m->ctx * kv_dim;
        m->past = (size_t*)own(sm, m->seqs * sizeof(size_t));
        m->k_cache = (float*)own(sm, (cache ? cache : 1) * sizeof(float));
        m->v_cache = (float*)own(sm, (cache ? cache : 1) * sizeof(float));
        m->x = (float*)own(sm, H * 4);
        m->xn = (float*)own(sm, H * 4);
        m->q = (float*)own(sm, (q_dim + 1) * 4);
        m->k = (float*)own(sm, (kv_dim + 1) * 4);
        m->v = (float*)own(sm, (kv_dim + 1) * 4);
        m->att = (float*)own(sm, (q_dim + 1) * 4);
        m->proj = (float*)own(sm, H * 4);
        m->gate = (float*)own(sm, I * 4);
        m->up = (float*)own(sm, I * 4);
        m->scores = (float*)own(sm, (m->ctx + 1) * 4);
        m->cos_t = (float*)own(sm, (hd / 2 + 1) * 4);
        m->sin_t = (float*)own(sm, (hd / 2 + 1) * 4);
        m->router_logits = (float*)own(sm, E * 4);
        m->expert_out = (float*)own(sm, H * 4);
        if (!m->past || !m->k_cache || !m->v_cache || !m->x || !m->expert_out) J.failed = 1;
    }
    if (!J.failed) run_jobs(J.v, J.n, threads);
    free(J.v);
    if (J.failed) {
        vitna_synth_free(m);
        fail(err, err_len, "out of memory, or a width that is not whole blocks, for the synthetic model");
        return NULL;
    }
    return m;
}
