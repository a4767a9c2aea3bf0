/**
 * engine.hip - libvitna_hip's host side: the vitna_cuda_* C ABI of
 * engine/include/model_cuda.h (the reference's boundary, model_cuda.cu
 * :3537-5536) over HIP on one MI355X, and the vitna_hip_* extensions.
 *
 * Upload (vitna_cuda_create, reference model_cuda.cu:3761): shapes are
 * checked first (check_shapes, reference :3558), then every weight goes to the
 * device once: GGUF blocks are copied to a staging buffer and split into
 * planes (vitna_hip_internal.h) by repack_kernel; every expert of every layer
 * is resident, one allocation a layer. The key-value cache is
 * [seq][layer][ctx][n_kv * head_dim] float32, as the reference's.
 *
 * Every kernel runs on one stream. A device-routed decode step
 * (vitna_hip_moe_step) is captured once into a HIP graph; its token, position
 * and sequence live in device memory (rows_dev[0]) and are copied in before
 * each replay, so one graph serves every position.
 */

#include "vitna_kernels.h"
#include "step_kernel.h"
#include "expert_cache.h"
#include "../../include/vitna_hip.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>
#include <algorithm>
#include <type_traits>
#include <mutex>

/* The most rows a pass takes (the reference's MOE_ROWS, model_cuda.cu:197): model.c runs a prompt in chunks of
   this many. Scratch for this many rows is allocated with the model. */
#define ROWS_MAX 1024
/* passes of this many rows or more, of a model whose experts are resident, take the grouped kernels on tiles of
   32 pairs (launch_gsx) instead of four (launch_gmma_in / _down). At top-8 of 128 experts (a 4096-token prompt
   in chunks, same box): 96-row chunks 961 -> 781 ms, 128 903 -> 707, 256 635 -> 433, 1024 415 -> 250; the
   32 rows of a ragged step (two pairs an expert) 12.55 -> 17.74 ms, so they keep the four-pair tiles */
#define GSX_ROWS 64
/* With the model's gpu_fast, a pass of at least this many rows runs its experts as the bf16 matrix-core grouped GEMM
   of the prefill (the reference's FAST_ROWS, model_cuda.cu:204); smaller passes keep the exact kernels. */
#define FAST_ROWS 64
/* Passes of the rows ABI of at most exact_rows rows (model.c's PASS_MAX, 64: the passes that check drafted tokens
   and the batched steps of a server, model.c:1052-1190) run each row through the kernels of a single token's step,
   several rows a launch: a row's logits are then the bits its step alone gives, as model.c expects of them ("every
   row is the one a step would give", main.c:1003-1007). Longer passes (a prompt's chunks) take the multi-row
   kernels, within 1e-3 of the checker but not those bits. */
#define EXACT_ROWS 64
/* passes of at least this many rows take the prefill's norm and router kernels for their routers */
#define ROUTE_WIDE_ROWS 128
/* rows step graphs kept at once: a prompt's passes take up to three attention grids, and a ragged step a fourth */
#define ROWS_GRAPHS 4

struct dlayer {
    qmat q, k, v, o;
    float *attn_norm, *mlp_norm, *q_norm, *k_norm;
    float* router;
    qmat gate, up, down;
    /* the experts' copies tiled for the crowded passes' grouped kernels (launch_gsx), or null */
    const uint8_t *sx_gate, *sx_up, *sx_down;
};

/* A prefill's working buffers for n rows (everything but the rows themselves), carved from one region by
   prefill_layout. Nothing in them has to start at zero: every kernel of the prefill writes what it later reads. */
struct pf_bufs {
    float *xn, *logits;
    uint16_t *xb, *act, *ypart;
    route_out* rt;
    int *count, *pairs, *off, *tiles, *ntiles;
};

struct vitna_cuda_model {
    int device;
    char name[320];
    hipStream_t stream;
    const vitna_llama_t* m;
    int H, I, E, K, NL, nh, nkv, hd, V, ctx, seqs, renorm, attention;
    float eps;
    std::vector<void*> allocs;
    std::vector<dlayer> L;
    qmat embed, head;
    float* final_norm;
    float *cos_tab, *sin_tab, *k_cache, *v_cache;
    size_t layer_kv;  /* floats of one (sequence, layer) cache */
    int splits_max;
    /* scratch, ROWS_MAX rows */
    float *x, *xn, *q, *k, *v, *qp, *att, *act, *ypart, *rlogits, *vocab, *partial;
    /* one row's o-projection in per-head-group parts (launch_attention_oproj), [OPROJ_PARTS_MAX][H]; parts_n > 0
       while they are still to be added to x (by the router's prologue and the experts' down kernel) */
    float* parts;
    int parts_n;
    route_out* rt;
    route_out* rt_layers; /* the device-routed step's routing of every layer (the last layer's is also in rt) */
    route_out* rows_rt;   /* the device-routed rows step's routing: [layer][ROWS_MAX] */
    row_rec* rows_dev;
    row_rec* rows_host; /* pinned */
    hipEvent_t rows_copied;
    bool row_set;       /* rows_dev[0] holds row_last (set_row); another pass of rows clears it */
    row_rec row_last;
    route_out* rt_host; /* pinned, ROWS_MAX: the routing a caller gives, on its way to rt */
    hipEvent_t rt_copied;
    float* h_logits;    /* pinned, 2 * ROWS_MAX * E */
    hipGraph_t step_graph_src; /* kept until free: graph tools may refer to its nodes */
    int *grp_count, *grp_pairs; /* expert grouping of a pass of rows: [E], [E][ROWS_MAX] */
    uint16_t *sk_xh, *sk_xl;    /* a pass's activations split into bf16 hi and lo, [ROWS_MAX][widest row] */
    uint32_t* sk_img[4];        /* or their operand images (orders A and B) and 32- and 16-column sums */
    float* sk_part;             /* split sums of the multi-row projections wider than 2048 columns */
    int* sk_cnt;                /* their per-tile counters, zero between calls */
    size_t sk_part_cap, sk_cnt_cap;
    uint16_t *gm_xs, *gm_as;    /* the grouped experts' split activations: [ROWS_MAX][2H], [ROWS_MAX * K][2I] */
    float *gm_xsum, *gm_asum;   /* and their sums over runs of 16 or more columns */
    /* the crowded passes' grouped experts (launch_gsx), made with the tiled copies: tile offsets and experts,
       operand images and sums of the pairs' rows and of the SwiGLU output, that output */
    int *gsx_toff, *gsx_te;
    uint32_t *gsx_img_in, *gsx_img_act;
    uint16_t *gsx_s32, *gsx_s16;
    float* gsx_act;
    bool rows_shared_seq;       /* the pass's rows include two of one sequence (attention prepares first) */
    bool rows_one_seq;          /* every row of the pass is of one sequence (a prompt's chunk: tiles of rows) */
    /* the rows step's captured graphs, a few kept (least recently used replaced): one a pass shape */
    struct rows_graph_t {
        hipGraph_t src;
        hipGraphExec_t exec;
        int n;                  /* rows, or 0 for an empty entry */
        bool shared, fast;      /* rows of one sequence; the experts as the grouped GEMM */
        int splits;             /* the attention's grid */
        int head;               /* the head's rows: HEAD_ALL, HEAD_NONE or the one row */
        uint64_t used;
    } rg[ROWS_GRAPHS];
    uint64_t rg_clock;
    int rg_cur;                 /* the entry the last ensure_rows_graph chose */
    hipGraphExec_t step_graph;
    bool graph_ready;
    /* the persistent decode step (kernels_step.hip): set up on first use when the model's shape takes it */
    int step_state;             /* 0: not looked at, 1: ready, -1: this model runs the per-layer kernels */
    const char* step_reason;    /* why not, for -1 */
    bool step_want;             /* the caller asked for the persistent step (vitna_hip_set_step_kernel) */
    step_layer* step_L;         /* device: the layer table */
    float* step_buf;            /* device: every layer's activation buffers */
    uint32_t* step_flags;       /* device: [NL][phases][256] epochs, then the abort word */
    uint32_t step_epoch;
    int step_nb;
    step_args step_base;        /* the arguments every launch shares */
    bool last_step_mega;        /* the last decode step ran the persistent kernel */
    int last_mega_n;            /* and over this many layers */
    uint64_t* step_trace;       /* device: a traced step's phase timeline */
    bool tiled_ready;           /* the multi-row paths' tiled copies made (ensure_tiled) */
    bool lost;
    bool fast;          /* m->gpu_fast: passes of fast_rows rows or more take the grouped GEMM for their experts */
    size_t fast_rows, long_from;
    int rows_n;         /* rows of the pass in flight (vitna_cuda_moe_rows_*) */
    int exact_rows;     /* passes of the rows ABI up to this many rows run the single-token kernels (EXACT_ROWS) */
    /* the attention's grid for the row(s) set last: the power of two of chunks at or above the most any row needs
       (at most splits_max), so that a short position in a long cache launches few blocks past its last chunk;
       the graphs are captured for one such size (graph_splits, rows_graph_t::splits) */
    int splits_grid, graph_splits;
    bool pass_exact;    /* and the pass in flight is one */
    /* prefill through one MoE layer: buffers for pf_cap rows, allocated on first use */
    size_t pf_cap;
    std::vector<void*> pf_allocs;
    float *pf_x, *pf_x0;
    pf_bufs pf;
    /* the experts through a cache of slots, when expert_cache_bytes leaves fewer slots than experts */
    expert_cache ec;
    /* a cached model's passes of rows: the grouped experts' tiled copy of each slot (gate, up, down areas, made on
       the first pass), the place each slot's copy was made from (-1: none), and the tile strides it was made with */
    uint8_t* st_area[3];
    size_t st_stride[3];
    std::vector<int64_t> st_place;
};

static bool fail(char* err, size_t len, const char* fmt, ...) {
    if (err && len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, len, fmt, ap);
        va_end(ap);
    }
    return false;
}

static bool fail_hip(char* err, size_t len, const char* what, hipError_t e) {
    return fail(err, len, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

/* Two timing events, destroyed on every path out. */
struct event_pair {
    hipEvent_t t0 = nullptr, t1 = nullptr;
    hipError_t make() {
        hipError_t e = hipEventCreate(&t0);
        return e == hipSuccess ? hipEventCreate(&t1) : e;
    }
    ~event_pair() {
        if (t0) (void)hipEventDestroy(t0);
        if (t1) (void)hipEventDestroy(t1);
    }
};

#define HIP_TRY(call, what)                                          \
    do {                                                             \
        hipError_t e_ = (call);                                      \
        if (e_ != hipSuccess) return fail_hip(err, err_len, what, e_); \
    } while (0)

static const char* dtype_name(int t) {
    switch (t) {
        case VITNA_DTYPE_F32: return "F32";
        case VITNA_DTYPE_F16: return "F16";
        case VITNA_DTYPE_BF16: return "BF16";
        case VITNA_DTYPE_Q8_0: return "Q8_0";
        case VITNA_DTYPE_Q2_K: return "Q2_K";
        case VITNA_DTYPE_Q3_K: return "Q3_K";
        case VITNA_DTYPE_Q4_K: return "Q4_K";
        case VITNA_DTYPE_Q5_K: return "Q5_K";
        case VITNA_DTYPE_Q6_K: return "Q6_K";
        default: return "an unsupported dtype";
    }
}

static bool quant_ok(int t) { return t == VITNA_DTYPE_Q8_0 || t == VITNA_DTYPE_Q4_K || t == VITNA_DTYPE_Q6_K; }

/* widths the GEMV kernels are built for: 32 * {4, 8, ..., 256} */
static bool width_ok(size_t cols) {
    const size_t s = cols / 32;
    return cols % 32 == 0 && (s == 4 || s == 8 || s == 16 || s == 32 || s == 64 || s == 128 || s == 256);
}

static bool matrix_ok(const vitna_matrix_t* w, size_t rows, size_t cols, const char* what, char* err, size_t err_len,
                      bool row_gemv = true) {
    if (!w->data) return fail(err, err_len, "%s has no data", what);
    if (w->rows != rows || w->cols != cols)
        return fail(err, err_len, "%s is %zu x %zu where %zu x %zu is needed", what, w->rows, w->cols, rows, cols);
    if (!quant_ok(w->dtype))
        return fail(err, err_len, "%s is %s; this device path reads Q8_0, Q4_K and Q6_K", what, dtype_name(w->dtype));
    if (!vitna_matrix_row_bytes(w->dtype, cols)) return fail(err, err_len, "%s: %zu columns are not whole %s blocks", what, cols, dtype_name(w->dtype));
    if (row_gemv && !width_ok(cols))
        return fail(err, err_len, "%s: width %zu is not one the kernels take (32 x 4 .. 256, powers of two)", what, cols);
    return true;
}

/* The reference's check_shapes (model_cuda.cu:3558), for what these kernels assume. */
static bool check_shapes(const vitna_llama_t* m, char* err, size_t err_len) {
    const vitna_llama_config_t* c = &m->cfg;
    if (!c->n_experts) return fail(err, err_len, "this device path serves a mixture of experts, and the model is dense");
    if (c->n_experts > ROUTE_E_MAX || c->n_experts % 4)
        return fail(err, err_len, "%zu experts; a multiple of 4, at most %d, are routed on the device", c->n_experts, ROUTE_E_MAX);
    if (c->n_experts_used < 1 || c->n_experts_used > ROUTE_K_MAX || c->n_experts_used > c->n_experts)
        return fail(err, err_len, "%zu experts a token; 1 to %d, and no more than the experts, are supported", c->n_experts_used, ROUTE_K_MAX);
    if (c->hidden % 256 || c->hidden > 8192) return fail(err, err_len, "hidden width %zu: a multiple of 256, at most 8192, is needed", c->hidden);
    const size_t S = c->intermediate / 32;
    if (c->intermediate % 256 || (c->n_experts_used * S + 63) / 64 > 8 || (c->n_experts_used * S + 63) / 64 == 7)
        return fail(err, err_len, "expert width %zu with %zu experts a token is not a shape the down kernel takes", c->intermediate,
                    c->n_experts_used);
    if (!m->ctx || !m->seqs) return fail(err, err_len, "the model has no key-value cache shape (ctx %zu, seqs %zu)", m->ctx, m->seqs);
    if (c->n_heads && m->ctx > (size_t)ATTN_SPLITS_MAX * ATTN_CHUNK)
        return fail(err, err_len, "a context of %zu positions: the device attention merges at most %d chunks of %d (%d positions)", m->ctx,
                    ATTN_SPLITS_MAX, ATTN_CHUNK, ATTN_SPLITS_MAX * ATTN_CHUNK);
    char what[96];
    for (size_t l = 0; l < c->n_layers; l++) {
        const vitna_llama_layer_t* L = &m->layers[l];
        if (!L->mlp_norm) return fail(err, err_len, "layer %zu has no MLP norm", l);
        if (!L->router.data || L->router.dtype != VITNA_DTYPE_F32 || L->router.rows != c->n_experts || L->router.cols != c->hidden)
            return fail(err, err_len, "layer %zu: the router must be F32, %zu x %zu", l, c->n_experts, c->hidden);
        if (!L->experts) return fail(err, err_len, "layer %zu has no experts", l);
        const int gdt = L->experts[0].gate.dtype, ddt = L->experts[0].down.dtype;
        for (size_t e = 0; e < c->n_experts; e++) {
            const vitna_expert_t* x = &L->experts[e];
            snprintf(what, sizeof(what), "layer %zu expert %zu gate", l, e);
            if (!matrix_ok(&x->gate, c->intermediate, c->hidden, what, err, err_len)) return false;
            snprintf(what, sizeof(what), "layer %zu expert %zu up", l, e);
            if (!matrix_ok(&x->up, c->intermediate, c->hidden, what, err, err_len)) return false;
            snprintf(what, sizeof(what), "layer %zu expert %zu down", l, e);
            if (!matrix_ok(&x->down, c->hidden, c->intermediate, what, err, err_len, false)) return false;
            if (x->gate.dtype != gdt || x->up.dtype != gdt || x->down.dtype != ddt)
                return fail(err, err_len, "layer %zu: every expert's gate and up, and every expert's down, must share a dtype", l);
        }
        if (c->n_heads) {
            const size_t qd = c->n_heads * c->head_dim, kd = c->n_kv_heads * c->head_dim;
            snprintf(what, sizeof(what), "layer %zu q", l);
            if (!matrix_ok(&L->q, qd, c->hidden, what, err, err_len)) return false;
            snprintf(what, sizeof(what), "layer %zu k", l);
            if (!matrix_ok(&L->k, kd, c->hidden, what, err, err_len)) return false;
            snprintf(what, sizeof(what), "layer %zu v", l);
            if (!matrix_ok(&L->v, kd, c->hidden, what, err, err_len)) return false;
            snprintf(what, sizeof(what), "layer %zu o", l);
            if (!matrix_ok(&L->o, c->hidden, qd, what, err, err_len)) return false;
            if (!L->attn_norm) return fail(err, err_len, "layer %zu has no attention norm", l);
            if (c->qk_norm && (!c->qk_norm_per_head || !L->q_norm || !L->k_norm))
                return fail(err, err_len, "layer %zu: only the per-head QK-norm (Qwen3) is served on the device", l);
        }
    }
    if (c->n_heads) {
        if (c->head_dim != 64 && c->head_dim != 128) return fail(err, err_len, "head width %zu: 64 or 128 is needed", c->head_dim);
        if (c->n_heads % c->n_kv_heads || c->n_heads / c->n_kv_heads > 8)
            return fail(err, err_len, "%zu query heads over %zu key-value heads: at most 8 a group", c->n_heads, c->n_kv_heads);
        if (!matrix_ok(&m->embed, c->vocab, c->hidden, "the embedding", err, err_len)) return false;
        if (!matrix_ok(&m->lm_head, c->vocab, c->hidden, "the output projection", err, err_len)) return false;
        if (!m->final_norm) return fail(err, err_len, "the model has no final norm");
    }
    return true;
}

template <typename T>
static bool dalloc(vitna_cuda_model* g, T** p, size_t bytes, const char* what, char* err, size_t err_len) {
    void* q = nullptr;
    const hipError_t e = hipMalloc(&q, bytes ? bytes : 256);
    if (e != hipSuccess) return fail(err, err_len, "device memory for %s (%zu bytes): %s", what, bytes, hipGetErrorString(e));
    g->allocs.push_back(q);
    *p = (T*)q;
    return true;
}

/* Planes of n matrices (experts) of one shape, back to back: qmat over the
   first, estride from one to the next. */
static size_t set_bytes(int dtype, size_t rows, size_t cols, size_t n) {
    size_t t = 0;
    for (int i = 0; i < 4; i++) t += align256(n * plane_bytes(dtype, i, rows, cols));
    return t;
}

static qmat place(uint8_t* base, int dtype, size_t rows, size_t cols, size_t n) {
    qmat q;
    memset(&q, 0, sizeof(q));
    size_t off = 0;
    for (int i = 0; i < 4; i++) {
        const size_t pb = plane_bytes(dtype, i, rows, cols);
        q.p[i] = pb ? base + off : nullptr;
        q.estride[i] = pb;
        off += align256(n * pb);
    }
    q.rows = (int)rows;
    q.cols = (int)cols;
    q.nb = (int)(cols / (dtype == VITNA_DTYPE_Q8_0 ? 32 : 256));
    q.dtype = dtype;
    return q;
}

/* n host matrices of one shape into planes at q (experts e0..): each copied to
   staging, then one repack over all of them. */
static bool upload_set(vitna_cuda_model* g, const vitna_matrix_t* const* mats, size_t n, const qmat& q, uint8_t* staging,
                       size_t staging_bytes, char* err, size_t err_len) {
    const size_t rb = vitna_matrix_row_bytes(mats[0]->dtype, mats[0]->cols), mb = rb * mats[0]->rows;
    const size_t per = staging_bytes / mb;
    if (per == 0) return fail(err, err_len, "internal: staging buffer too small");
    for (size_t e0 = 0; e0 < n; e0 += per) {
        const size_t cnt = std::min(per, n - e0);
        for (size_t e = 0; e < cnt; e++)
            HIP_TRY(hipMemcpyAsync(staging + e * mb, mats[e0 + e]->data, mb, hipMemcpyHostToDevice, g->stream), "copying weights to the device");
        qmat part = q;
        for (int i = 0; i < 4; i++)
            if (part.p[i]) part.p[i] += e0 * q.estride[i];
        part.rows = (int)(cnt * mats[0]->rows);
        HIP_TRY(launch_repack(staging, part, g->stream), "splitting blocks into planes");
        HIP_TRY(hipStreamSynchronize(g->stream), "uploading weights");
    }
    return true;
}

static bool upload_f32(vitna_cuda_model* g, float** out, const float* host, size_t n, const char* what, char* err, size_t err_len) {
    if (!dalloc(g, out, n * 4, what, err, err_len)) return false;
    HIP_TRY(hipMemcpy(*out, host, n * 4, hipMemcpyHostToDevice), what);
    return true;
}

static bool upload_matrix(vitna_cuda_model* g, qmat* out, const vitna_matrix_t* w, uint8_t* staging, size_t staging_bytes, const char* what,
                          char* err, size_t err_len) {
    uint8_t* mem;
    if (!dalloc(g, &mem, set_bytes(w->dtype, w->rows, w->cols, 1), what, err, err_len)) return false;
    *out = place(mem, w->dtype, w->rows, w->cols, 1);
    const vitna_matrix_t* one[1] = {w};
    return upload_set(g, one, 1, *out, staging, staging_bytes, err, err_len);
}

/* The tiled copy the multi-row kernels read (dense matrices whose width is a multiple of 256). */
static bool make_tiled(vitna_cuda_model* g, qmat* m, const char* what, char* err, size_t err_len) {
    const size_t tb = tile_bytes(m->dtype);
    if (!tb || m->cols % 256) return true;
    uint8_t* mem;
    if (!dalloc(g, &mem, tb * ((m->rows + 31) / 32) * (m->cols / 256), what, err, err_len)) return false;
    HIP_TRY(launch_tile(*m, mem, g->stream), "tiling a matrix");
    HIP_TRY(hipStreamSynchronize(g->stream), "tiling a matrix");
    m->tiled = mem;
    return true;
}

/* The tiled copies only the multi-row paths read (the dense matrices' for the projections, the experts' for the
   grouped experts), made on the first multi-row call, before any graph is captured: a model that only decodes
   never holds them. */
static bool ensure_tiled(vitna_cuda_model* g, char* err, size_t err_len) {
    if (g->tiled_ready) return true;
    for (int l = 0; l < g->NL; l++) {
        dlayer& d = g->L[l];
        if (g->attention && !(make_tiled(g, &d.q, "q", err, err_len) && make_tiled(g, &d.k, "k", err, err_len) &&
                              make_tiled(g, &d.v, "v", err, err_len) && make_tiled(g, &d.o, "o", err, err_len)))
            return false;
        /* (the experts' copy only where they are resident: a cached model's views hold slots, not experts) */
        if (!g->ec.on && gmma_fits(d.gate, d.up, d.down)) {
            qmat* sets[3] = {&d.gate, &d.up, &d.down};
            for (int i = 0; i < 3; i++) {
                uint8_t* t;
                if (!dalloc(g, &t, gmma_tiled_bytes(*sets[i], g->E), "the experts' tiled copy", err, err_len)) return false;
                HIP_TRY(launch_gmma_tile(*sets[i], g->E, t, g->stream), "tiling the experts");
                HIP_TRY(hipStreamSynchronize(g->stream), "tiling the experts");
                sets[i]->tiled = t;
            }
        }
    }
    if (g->attention && !make_tiled(g, &g->head, "the output projection", err, err_len)) return false;
    /* the crowded passes' copy of the experts and its buffers, when the device has room for them all (1 GB to
       spare): without it those passes keep the four-pair kernels */
    if (!g->ec.on && g->E <= ROUTE_E_MAX && gsx_fits(g->L[0].gate, g->L[0].up, g->L[0].down)) {
        const size_t T = (size_t)gsx_max_tiles(ROWS_MAX, g->K, g->E), H = g->H, I = g->L[0].gate.rows, W = std::max(H, I);
        size_t need = (g->E + 1 + T) * sizeof(int) + 32 * T * (H + 2 * I) * 4 + T * (W / 256) * 1536 * 3;
        for (int l = 0; l < g->NL; l++) {
            const dlayer& d = g->L[l];
            if (gsx_fits(d.gate, d.up, d.down))
                need += gsx_tiled_bytes(d.gate, g->E) + gsx_tiled_bytes(d.up, g->E) + gsx_tiled_bytes(d.down, g->E);
        }
        size_t fr = 0, tot = 0;
        if (hipMemGetInfo(&fr, &tot) == hipSuccess && need + ((size_t)1 << 30) <= fr) {
            if (!(dalloc(g, &g->gsx_toff, (g->E + 1) * sizeof(int), "scratch", err, err_len) &&
                  dalloc(g, &g->gsx_te, T * sizeof(int), "scratch", err, err_len) &&
                  dalloc(g, &g->gsx_img_in, 32 * T * H * 4, "scratch", err, err_len) &&
                  dalloc(g, &g->gsx_img_act, 32 * T * I * 4, "scratch", err, err_len) &&
                  dalloc(g, &g->gsx_s32, T * (W / 256) * 1536, "scratch", err, err_len) &&
                  dalloc(g, &g->gsx_s16, T * (W / 128) * 1536, "scratch", err, err_len) &&
                  dalloc(g, &g->gsx_act, 32 * T * I * 4, "scratch", err, err_len)))
                return false;
            for (int l = 0; l < g->NL; l++) {
                dlayer& d = g->L[l];
                if (!gsx_fits(d.gate, d.up, d.down)) continue;
                const qmat* sets[3] = {&d.gate, &d.up, &d.down};
                const uint8_t** dst[3] = {&d.sx_gate, &d.sx_up, &d.sx_down};
                for (int i = 0; i < 3; i++) {
                    uint8_t* t;
                    if (!dalloc(g, &t, gsx_tiled_bytes(*sets[i], g->E), "the experts' copy for crowded passes", err, err_len)) return false;
                    HIP_TRY(launch_gsx_tile(*sets[i], g->E, t, g->stream), "tiling the experts");
                    HIP_TRY(hipStreamSynchronize(g->stream), "tiling the experts");
                    *dst[i] = t;
                }
            }
        }
    }
    g->tiled_ready = true;
    return true;
}

extern "C" bool vitna_cuda_probe(char* err, size_t err_len) {
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return fail_hip(err, err_len, "the HIP runtime finds no device", e);
    if (n < 1) return fail(err, err_len, "the HIP runtime finds no device");
    return true;
}

extern "C" int vitna_cuda_devices(vitna_cuda_device_t* out, int max) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    int k = 0;
    for (int d = 0; d < n && k < max; d++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, d) != hipSuccess) continue;
        vitna_cuda_device_t* o = &out[k++];
        memset(o, 0, sizeof(*o));
        snprintf(o->name, sizeof(o->name), "%s (%s)", p.name, p.gcnArchName);
        o->total_bytes = p.totalGlobalMem;
        size_t fr = 0, tot = 0;
        if (hipSetDevice(d) == hipSuccess && hipMemGetInfo(&fr, &tot) == hipSuccess) o->free_bytes = fr;
        o->major = p.major;
        o->minor = p.minor;
    }
    return k;
}

static void drop_rows_graphs(vitna_cuda_model* g) {
    for (auto& r : g->rg) {
        if (!r.n) continue;
        (void)hipGraphExecDestroy(r.exec);
        (void)hipGraphDestroy(r.src);
        r.n = 0;
    }
}

extern "C" void vitna_cuda_free(struct vitna_cuda_model* g) {
    if (!g) return;
    (void)hipSetDevice(g->device);
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->graph_ready) {
        (void)hipGraphExecDestroy(g->step_graph);
        (void)hipGraphDestroy(g->step_graph_src);
    }
    drop_rows_graphs(g);
    for (void* p : g->allocs) (void)hipFree(p);
    for (void* p : g->pf_allocs) (void)hipFree(p);
    if (g->rows_host) (void)hipHostFree(g->rows_host);
    if (g->h_logits) (void)hipHostFree(g->h_logits);
    if (g->rows_copied) (void)hipEventDestroy(g->rows_copied);
    if (g->rt_host) (void)hipHostFree(g->rt_host);
    if (g->rt_copied) (void)hipEventDestroy(g->rt_copied);
    ec_destroy(g->ec);
    if (g->stream) (void)hipStreamDestroy(g->stream);
    delete g;
}

extern "C" struct vitna_cuda_model* vitna_cuda_create(const vitna_llama_t* m, const float* cos_tab, const float* sin_tab,
                                                      size_t expert_cache_bytes, char* err, size_t err_len) {
    if (!m) { fail(err, err_len, "no model"); return nullptr; }
    if (!check_shapes(m, err, err_len)) return nullptr;
    const vitna_llama_config_t* c = &m->cfg;
    if (c->n_heads && (!cos_tab || !sin_tab)) { fail(err, err_len, "the rotary tables are missing"); return nullptr; }
    if (!vitna_cuda_probe(err, err_len)) return nullptr;
    vitna_cuda_model* g = new vitna_cuda_model(); /* value-initialized: every plain member zero */
    g->device = 0;
    g->m = m;
    g->H = (int)c->hidden; g->I = (int)c->intermediate; g->E = (int)c->n_experts; g->K = (int)c->n_experts_used;
    g->NL = (int)c->n_layers; g->nh = (int)c->n_heads; g->nkv = (int)c->n_kv_heads; g->hd = (int)c->head_dim;
    g->V = (int)c->vocab; g->ctx = (int)m->ctx; g->seqs = (int)m->seqs; g->renorm = c->renormalize; g->attention = c->n_heads != 0;
    g->eps = c->rms_eps;
    g->fast = m->gpu_fast;
    g->fast_rows = FAST_ROWS;
    g->exact_rows = EXACT_ROWS;
    g->long_from = 1024;
    g->embed = {}; g->head = {};
    g->final_norm = nullptr;
    g->graph_ready = false;
    g->lost = false;
    g->rows_n = 0;
    auto bail = [&]() -> vitna_cuda_model* { vitna_cuda_free(g); return nullptr; };
    if (hipSetDevice(0) != hipSuccess) { fail(err, err_len, "cannot select device 0"); return bail(); }
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) == hipSuccess) snprintf(g->name, sizeof(g->name), "%s (%s)", p.name, p.gcnArchName);
    if (hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking) != hipSuccess) { fail(err, err_len, "cannot create a stream"); return bail(); }
    if (hipEventCreateWithFlags(&g->rows_copied, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&g->rt_copied, hipEventDisableTiming) != hipSuccess) {
        fail(err, err_len, "cannot create an event");
        return bail();
    }

    /* staging for the largest set of one layer's experts of one part */
    const vitna_llama_layer_t* L0 = &m->layers[0];
    size_t staging_bytes = 64u << 20;
    for (size_t l = 0; l < c->n_layers; l++) {
        const vitna_expert_t* x = &m->layers[l].experts[0];
        const size_t gb = vitna_matrix_row_bytes(x->gate.dtype, x->gate.cols) * x->gate.rows;
        const size_t db = vitna_matrix_row_bytes(x->down.dtype, x->down.cols) * x->down.rows;
        staging_bytes = std::max(staging_bytes, std::max(gb, db) * 16);
    }
    if (g->attention) {
        staging_bytes = std::max(staging_bytes, vitna_matrix_row_bytes(m->lm_head.dtype, m->lm_head.cols) * m->lm_head.rows);
        staging_bytes = std::max(staging_bytes, vitna_matrix_row_bytes(m->embed.dtype, m->embed.cols) * m->embed.rows);
    }
    (void)L0;
    uint8_t* staging = nullptr;
    if (hipMalloc(&staging, staging_bytes) != hipSuccess) { fail(err, err_len, "device memory for staging (%zu bytes)", staging_bytes); return bail(); }
    /* experts through a cache of slots when expert_cache_bytes holds fewer than all of them (expert_cache.h) */
    bool ok = ec_create(g->ec, m, expert_cache_bytes, err, err_len);
    if (!ok) { (void)hipFree(staging); return bail(); }
    g->L.resize(c->n_layers);
    std::vector<const vitna_matrix_t*> mats(c->n_experts);
    for (size_t l = 0; ok && l < c->n_layers; l++) {
        const vitna_llama_layer_t* L = &m->layers[l];
        dlayer& d = g->L[l];
        memset(&d, 0, sizeof(d));
        ok = upload_f32(g, &d.mlp_norm, L->mlp_norm, c->hidden, "the MLP norm", err, err_len) &&
             upload_f32(g, &d.router, (const float*)L->router.data, c->n_experts * c->hidden, "the router", err, err_len);
        const vitna_expert_t* x0 = &L->experts[0];
        const size_t E = c->n_experts;
        if (g->ec.on) {
            d.gate = ec_view(g->ec, (int)l, 0);
            d.up = ec_view(g->ec, (int)l, 1);
            d.down = ec_view(g->ec, (int)l, 2);
        } else {
            const size_t gbytes = set_bytes(x0->gate.dtype, x0->gate.rows, x0->gate.cols, E);
            const size_t dbytes = set_bytes(x0->down.dtype, x0->down.rows, x0->down.cols, E);
            uint8_t* mem = nullptr;
            ok = ok && dalloc(g, &mem, 2 * gbytes + dbytes, "a layer's experts", err, err_len);
            if (!ok) break;
            d.gate = place(mem, x0->gate.dtype, x0->gate.rows, x0->gate.cols, E);
            d.up = place(mem + gbytes, x0->up.dtype, x0->up.rows, x0->up.cols, E);
            d.down = place(mem + 2 * gbytes, x0->down.dtype, x0->down.rows, x0->down.cols, E);
            for (size_t e = 0; e < E; e++) mats[e] = &L->experts[e].gate;
            ok = upload_set(g, mats.data(), E, d.gate, staging, staging_bytes, err, err_len);
            for (size_t e = 0; ok && e < E; e++) mats[e] = &L->experts[e].up;
            ok = ok && upload_set(g, mats.data(), E, d.up, staging, staging_bytes, err, err_len);
            for (size_t e = 0; ok && e < E; e++) mats[e] = &L->experts[e].down;
            ok = ok && upload_set(g, mats.data(), E, d.down, staging, staging_bytes, err, err_len);
        }
        if (ok && g->attention) {
            ok = upload_matrix(g, &d.q, &L->q, staging, staging_bytes, "q", err, err_len) &&
                 upload_matrix(g, &d.k, &L->k, staging, staging_bytes, "k", err, err_len) &&
                 upload_matrix(g, &d.v, &L->v, staging, staging_bytes, "v", err, err_len) &&
                 upload_matrix(g, &d.o, &L->o, staging, staging_bytes, "o", err, err_len) &&
                 upload_f32(g, &d.attn_norm, L->attn_norm, c->hidden, "the attention norm", err, err_len);
            if (ok && c->qk_norm)
                ok = upload_f32(g, &d.q_norm, L->q_norm, c->head_dim, "the q norm", err, err_len) &&
                     upload_f32(g, &d.k_norm, L->k_norm, c->head_dim, "the k norm", err, err_len);
        }
    }
    if (ok && g->attention) {
        ok = upload_matrix(g, &g->embed, &m->embed, staging, staging_bytes, "the embedding", err, err_len) &&
             upload_matrix(g, &g->head, &m->lm_head, staging, staging_bytes, "the output projection", err, err_len) &&
             upload_f32(g, &g->final_norm, m->final_norm, c->hidden, "the final norm", err, err_len);
        const size_t half = c->head_dim / 2;
        ok = ok && upload_f32(g, &g->cos_tab, cos_tab, m->ctx * half, "the rotary cosines", err, err_len) &&
             upload_f32(g, &g->sin_tab, sin_tab, m->ctx * half, "the rotary sines", err, err_len);
    }
    (void)hipFree(staging);
    if (!ok) return bail();

    /* key-value cache and scratch */
    const size_t H = c->hidden, R = ROWS_MAX, E = c->n_experts, K = c->n_experts_used;
    const size_t qd = c->n_heads * c->head_dim, kd = c->n_kv_heads * c->head_dim;
    g->layer_kv = m->ctx * kd;
    g->splits_max = (int)((m->ctx + ATTN_CHUNK - 1) / ATTN_CHUNK);
    const size_t G = c->n_kv_heads ? c->n_heads / c->n_kv_heads : 1;
    ok = dalloc(g, &g->x, R * H * 4, "the residual", err, err_len) && dalloc(g, &g->xn, R * H * 4, "scratch", err, err_len) &&
         dalloc(g, &g->act, R * K * c->intermediate * 4, "scratch", err, err_len) &&
         dalloc(g, &g->ypart, R * K * H * 4, "scratch", err, err_len) &&
         dalloc(g, &g->sk_xh, R * std::max<size_t>(H, (size_t)c->n_heads * c->head_dim) * 2, "scratch", err, err_len) &&
         dalloc(g, &g->sk_xl, R * std::max<size_t>(H, (size_t)c->n_heads * c->head_dim) * 2, "scratch", err, err_len) &&
         dalloc(g, &g->sk_img[0], R * std::max<size_t>(H, qd) * 4, "scratch", err, err_len) &&
         dalloc(g, &g->sk_img[1], R * std::max<size_t>(H, qd) * 4, "scratch", err, err_len) &&
         /* a row's window of eight groups: three pieces of 8 bf16 */
         dalloc(g, &g->sk_img[2], R * std::max<size_t>(H, qd) / 256 * 48, "scratch", err, err_len) &&
         dalloc(g, &g->sk_img[3], R * std::max<size_t>(H, qd) / 128 * 48, "scratch", err, err_len) &&
         dalloc(g, &g->gm_xs, R * 2 * H * 2, "scratch", err, err_len) &&
         dalloc(g, &g->gm_as, R * K * 2 * c->intermediate * 2, "scratch", err, err_len) &&
         dalloc(g, &g->gm_xsum, R * (H / 16) * 4, "scratch", err, err_len) &&
         dalloc(g, &g->gm_asum, R * K * (c->intermediate / 16) * 4, "scratch", err, err_len) &&
         dalloc(g, &g->rlogits, 2 * R * E * 4, "scratch", err, err_len) && dalloc(g, &g->rt, R * sizeof(route_out), "scratch", err, err_len) &&
         dalloc(g, &g->rt_layers, c->n_layers * sizeof(route_out), "scratch", err, err_len) &&
         dalloc(g, &g->rows_rt, c->n_layers * R * sizeof(route_out), "the rows step's routing", err, err_len) &&
         dalloc(g, &g->rows_dev, R * sizeof(row_rec), "scratch", err, err_len) &&
         /* grouped by expert, or by slot when the experts pass through the cache */
         dalloc(g, &g->grp_count, std::max<size_t>(E, g->ec.n_slots) * sizeof(int), "scratch", err, err_len) &&
         dalloc(g, &g->grp_pairs, std::max<size_t>(E, g->ec.n_slots) * R * sizeof(int), "scratch", err, err_len);
    if (ok && g->attention) {
        ok = dalloc(g, &g->q, R * qd * 4, "scratch", err, err_len) && dalloc(g, &g->qp, R * qd * 4, "scratch", err, err_len) &&
             dalloc(g, &g->k, R * kd * 4, "scratch", err, err_len) && dalloc(g, &g->v, R * kd * 4, "scratch", err, err_len) &&
             dalloc(g, &g->att, R * qd * 4, "scratch", err, err_len) &&
             dalloc(g, &g->parts, (size_t)EXACT_ROWS * OPROJ_PARTS_MAX * c->hidden * 4, "scratch", err, err_len) &&
             dalloc(g, &g->vocab, R * c->vocab * 4, "the logits", err, err_len) &&
             dalloc(g, &g->partial, (size_t)R * c->n_kv_heads * g->splits_max * G * (c->head_dim + 4) * 4, "attention partials", err, err_len) &&
             dalloc(g, &g->k_cache, m->seqs * c->n_layers * g->layer_kv * 4, "the key cache", err, err_len) &&
             dalloc(g, &g->v_cache, m->seqs * c->n_layers * g->layer_kv * 4, "the value cache", err, err_len);
    }
    if (ok && g->attention) {
        /* the multi-row projections' split sums: per token tile, each 32-row tile of a launch (q/k/v, o, head)
           takes one counter and ceil(width / 2048) sums of 32 x 32 */
        const size_t mt = (R + 31) / 32, t32 = 32;
        const size_t lt[3] = {(qd + 2 * kd + 3 * (t32 - 1)) / t32, (H + t32 - 1) / t32, (c->vocab + t32 - 1) / t32};
        const size_t lw[3] = {H, qd, H};
        size_t cnt = 1, part = 1;
        for (int i = 0; i < 3; i++) {
            const size_t sp = (lw[i] / 256 + 7) / 8;
            if (sp > 1) {
                cnt = std::max(cnt, mt * lt[i]);
                part = std::max(part, mt * lt[i] * sp * 1024);
            }
        }
        g->sk_cnt_cap = cnt;
        g->sk_part_cap = part;
        ok = dalloc(g, &g->sk_part, part * 4, "scratch", err, err_len) && dalloc(g, &g->sk_cnt, cnt * 4, "scratch", err, err_len) &&
             hipMemset(g->sk_cnt, 0, cnt * 4) == hipSuccess;
    }
    if (!ok) return bail();
    if (hipMemset(g->x, 0, R * H * 4) != hipSuccess || hipMemset(g->rt, 0, R * sizeof(route_out)) != hipSuccess) {
        fail(err, err_len, "clearing device scratch failed");
        return bail();
    }
    if (hipHostMalloc((void**)&g->rows_host, R * sizeof(row_rec), 0) != hipSuccess ||
        hipHostMalloc((void**)&g->h_logits, 2 * R * E * 4, 0) != hipSuccess ||
        hipHostMalloc((void**)&g->rt_host, R * sizeof(route_out), 0) != hipSuccess) {
        fail(err, err_len, "page-locked host memory for the rows and logits");
        return bail();
    }
    if (hipDeviceSynchronize() != hipSuccess) { fail(err, err_len, "the device failed during upload"); return bail(); }
    return g;
}

/* ---- per-layer enqueues ---------------------------------------------- */

/* One row's attention and o-projection. Where the layer takes the merged o-projection its parts stay pending
   (g->parts_n) for the router and the experts' down kernel, which add them to x; vitna_hip_residual adds them when
   the residual is read before that. */
static hipError_t enqueue_attention(vitna_cuda_model* g, int layer, int n_rows, bool prepared) {
    const dlayer& d = g->L[layer];
    gemv_args ga;
    memset(&ga, 0, sizeof(ga));
    ga.w[0] = d.q; ga.w[1] = d.k; ga.w[2] = d.v;
    ga.y[0] = g->q; ga.y[1] = g->k; ga.y[2] = g->v;
    ga.n = 3;
    ga.x = g->x;
    ga.norm_w = d.attn_norm;
    ga.eps = g->eps;
    if (n_rows != 1) return hipErrorInvalidValue; /* several rows: enqueue_rows_attention */
    hipError_t e = launch_gemv(ga, g->stream);
    if (e != hipSuccess) return e;
    attn_args a;
    memset(&a, 0, sizeof(a));
    a.q_raw = g->q; a.k_raw = g->k; a.v_raw = g->v;
    a.q_norm = d.q_norm; a.k_norm = d.k_norm;
    a.cos_tab = g->cos_tab; a.sin_tab = g->sin_tab;
    a.k_cache = g->k_cache + (size_t)layer * g->layer_kv;
    a.v_cache = g->v_cache + (size_t)layer * g->layer_kv;
    a.seq_stride = (size_t)g->NL * g->layer_kv;
    a.rows = g->rows_dev;
    a.n_rows = 1;
    a.partial = g->partial;
    a.att = g->att;
    a.n_heads = g->nh; a.n_kv = g->nkv; a.hd = g->hd; a.ctx = g->ctx; a.splits_max = g->splits_max;
    a.splits_grid = g->splits_grid;
    a.eps = g->eps;
    a.prepared = prepared ? 1 : 0;
    a.mma = 1;
    e = launch_attention(a, g->stream);
    if (e != hipSuccess) return e;
    g->parts_n = 0;
    if (attention_oproj_fits(a, d.o)) {
        e = launch_attention_oproj(a, d.o, g->parts, g->stream);
        if (e != hipSuccess) return e;
        g->parts_n = g->nh / ATTN_OPROJ_HEADS;
        return hipSuccess;
    }
    e = launch_attention_merge(a, g->stream);
    if (e != hipSuccess) return e;
    gemv_args go;
    memset(&go, 0, sizeof(go));
    go.w[0] = d.o;
    go.y[0] = g->x;
    go.n = 1;
    go.x = g->att;
    go.add = 1;
    return launch_gemv(go, g->stream);
}

/* sp: the grouped experts' split of xn_out, run by the top-k kernel (several rows), or null */
static hipError_t enqueue_route(vitna_cuda_model* g, int layer, float* logits, int n_rows, const float* x, float* xn_out, bool topk,
                                const topk_split* sp = nullptr, route_out* rt = nullptr) {
    const dlayer& d = g->L[layer];
    route_args r;
    memset(&r, 0, sizeof(r));
    r.x = x;
    r.norm_w = d.mlp_norm;
    r.router = d.router;
    r.xn_out = xn_out;
    r.logits = logits;
    r.H = g->H; r.E = g->E; r.n_rows = n_rows;
    r.eps = g->eps;
    if (n_rows == 1 && x == g->x && g->parts_n) {
        r.parts = g->parts;
        r.n_parts = g->parts_n;
    }
    hipError_t e;
    if (n_rows >= ROUTE_WIDE_ROWS && xn_out && !r.parts) {
        /* many rows (a prompt's chunk): the prefill's norm, then its router over the normalized rows, eight rows by
           eight experts a lane group (the same sums in the same order as route_kernel's, so the same bits) */
        e = launch_prefill_norm(x, d.mlp_norm, xn_out, nullptr, n_rows, g->H, g->eps, g->stream);
        if (e == hipSuccess) e = launch_prefill_router(xn_out, d.router, logits, n_rows, g->E, g->H, g->stream);
    } else {
        e = launch_route(r, g->stream);
    }
    /* one token's top-k runs in the experts' prologue (enqueue_experts); several rows' in a kernel of its own */
    if (e == hipSuccess && topk && n_rows > 1) e = launch_topk(logits, n_rows, g->E, g->K, g->renorm, rt ? rt : g->rt, g->stream, sp);
    return e;
}

/* The experts of one token: routed from logits in the kernel's prologue when they are given, else as g->rt holds it. */
static hipError_t enqueue_experts(vitna_cuda_model* g, int layer, const float* logits, float* y, int add, route_out* rt = nullptr) {
    const dlayer& d = g->L[layer];
    if (!rt) rt = g->rt;
    experts_in_args ai;
    ai.gate = d.gate; ai.up = d.up; ai.xn = g->xn; ai.rt = rt; ai.logits = logits; ai.E = g->E; ai.renorm = g->renorm;
    ai.act = g->act; ai.K = g->K;
    hipError_t e = launch_experts_in(ai, g->stream);
    if (e != hipSuccess) return e;
    experts_down_args ad;
    ad.down = d.down; ad.act = g->act; ad.rt = rt; ad.y = y; ad.K = g->K; ad.add = add;
    ad.parts = nullptr; ad.n_parts = 0;
    if (add && y == g->x && g->parts_n) {
        /* the attention's parts go into the residual with the experts' sum; nothing reads them after */
        ad.parts = g->parts;
        ad.n_parts = g->parts_n;
        g->parts_n = 0;
    }
    return launch_experts_down(ad, g->stream);
}

static hipError_t enqueue_head(vitna_cuda_model* g) {
    if (g->parts_n) {
        /* a layer's attention whose experts never ran: its parts still belong in the residual */
        const hipError_t e = launch_attn_fold(g->x, g->parts, g->parts_n, g->H, g->stream);
        g->parts_n = 0;
        if (e != hipSuccess) return e;
    }
    gemv_args gh;
    memset(&gh, 0, sizeof(gh));
    gh.w[0] = g->head;
    gh.y[0] = g->vocab;
    gh.n = 1;
    gh.x = g->x;
    gh.norm_w = g->final_norm;
    gh.eps = g->eps;
    return launch_gemv(gh, g->stream);
}

static bool check_launch(vitna_cuda_model* g, hipError_t e, const char* what, char* err, size_t err_len) {
    if (e == hipSuccess) return true;
    if (e == hipErrorInvalidValue) return fail(err, err_len, "%s: a kernel was asked for a shape it does not take", what);
    (void)g;
    return fail_hip(err, err_len, what, e);
}

static int splits_bucket(const vitna_cuda_model* g, int max_pos) {
    const int need = max_pos / ATTN_CHUNK + 1;
    int b = 1;
    while (b < need) b <<= 1;
    return b < g->splits_max ? b : g->splits_max;
}

static bool set_row(vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, char* err, size_t err_len) {
    if (seq >= (size_t)g->seqs) return fail(err, err_len, "sequence %zu: the cache holds %d", seq, g->seqs);
    if (pos >= (size_t)g->ctx) return fail(err, err_len, "position %zu: the cache holds %d", pos, g->ctx);
    if (g->attention && (token < 0 || token >= g->V)) return fail(err, err_len, "token %d is outside the vocabulary of %d", token, g->V);
    const row_rec r = {token, (int32_t)pos, (int32_t)seq};
    g->splits_grid = splits_bucket(g, (int)pos);
    /* the layers of one token after the first find their row in place */
    if (g->row_set && g->row_last.token == r.token && g->row_last.pos == r.pos && g->row_last.seq == r.seq) return true;
    /* the previous copy out of the page-locked row must have run */
    HIP_TRY(hipEventSynchronize(g->rows_copied), "waiting for the previous row copy");
    g->rows_host[0] = r;
    HIP_TRY(hipMemcpyAsync(g->rows_dev, g->rows_host, sizeof(row_rec), hipMemcpyHostToDevice, g->stream), "copying the row");
    HIP_TRY(hipEventRecord(g->rows_copied, g->stream), "recording the row copy");
    g->row_last = r;
    g->row_set = true;
    return true;
}

/* ---- the reference's MoE ABI ----------------------------------------- */

extern "C" bool vitna_cuda_moe_route(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, size_t layer, float* logits,
                                     float* next, char* err, size_t err_len) {
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    if (!g->attention) return fail(err, err_len, "this model has no attention; use vitna_hip_moe_ffn");
    if (!set_row(g, seq, token, pos, err, err_len)) return false;
    g->last_step_mega = false;
    const bool nx = next && layer + 1 < (size_t)g->NL;
    /* embedding (layer 0), attention, router (and the next layer's router on the same residual, whose norm must
       not replace this layer's), the logits to the page-locked buffer. Launched one by one: a graph a layer was
       slower here (5.3-5.4 against 4.5-4.7 ms a token for configs[2]'s model). */
    hipError_t e = hipSuccess;
    if (layer == 0) e = launch_embed(g->embed, &g->rows_dev[0].token, 0, g->x, g->stream);
    if (e == hipSuccess) e = enqueue_attention(g, (int)layer, 1, false);
    if (e == hipSuccess) e = enqueue_route(g, (int)layer, g->rlogits, 1, g->x, g->xn, false);
    if (e == hipSuccess && nx) e = enqueue_route(g, (int)layer + 1, g->rlogits + g->E, 1, g->x, nullptr, false);
    if (!check_launch(g, e, "the layer up to its router", err, err_len)) return false;
    HIP_TRY(hipMemcpyAsync(g->h_logits, g->rlogits, (nx ? 2 : 1) * g->E * 4, hipMemcpyDeviceToHost, g->stream), "copying the router's logits");
    HIP_TRY(hipStreamSynchronize(g->stream), "running the layer up to its router");
    memcpy(logits, g->h_logits, g->E * 4);
    if (nx) memcpy(next, g->h_logits + g->E, g->E * 4);
    return true;
}

/* slots: where the experts are in the expert cache (the kernels' expert index), or null for resident experts */
/* at: the first of the rows (the routing goes to rt[at .. at + n)) */
static bool put_routing(vitna_cuda_model* g, size_t n, const int32_t* ids, const float* weights, size_t k, char* err, size_t err_len,
                        const int32_t* slots = nullptr, size_t at = 0) {
    if (k != (size_t)g->K) return fail(err, err_len, "%zu experts given; the model routes to %d", k, g->K);
    /* the previous routing's copy out of the page-locked buffer must have run */
    HIP_TRY(hipEventSynchronize(g->rt_copied), "waiting for the previous routing copy");
    route_out* ro = g->rt_host + at;
    for (size_t t = 0; t < n; t++) {
        memset(&ro[t], 0, sizeof(route_out));
        for (size_t i = 0; i < k; i++) {
            const int32_t e = ids[t * k + i];
            if (e < 0 || e >= g->E) return fail(err, err_len, "expert %d is outside the layer's %d", e, g->E);
            for (size_t j = 0; j < i; j++)
                if (ids[t * k + j] == e) return fail(err, err_len, "expert %d is named twice", e);
            ro[t].ids[i] = e;
            ro[t].weights[i] = weights[t * k + i];
            ro[t].chosen[i] = slots ? slots[t * k + i] : e;
            ro[t].cw[i] = weights[t * k + i];
        }
    }
    /* from page-locked memory, in stream order: the kernels after it read it, nothing waits on the host */
    HIP_TRY(hipMemcpyAsync(g->rt + at, ro, n * sizeof(route_out), hipMemcpyHostToDevice, g->stream), "copying the routing");
    HIP_TRY(hipEventRecord(g->rt_copied, g->stream), "recording the routing copy");
    return true;
}

/* One token's experts of layer as g->rt routes them, added into the residual. */
static bool run_experts(vitna_cuda_model* g, int layer, char* err, size_t err_len) {
    return check_launch(g, enqueue_experts(g, layer, nullptr, g->x, 1), "the experts", err, err_len);
}

extern "C" bool vitna_cuda_moe_experts(struct vitna_cuda_model* g, size_t layer, const int32_t* ids, const float* weights, size_t k,
                                       const int32_t* guess, char* err, size_t err_len) {
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    if (!g->ec.on) return put_routing(g, 1, ids, weights, k, err, err_len) && run_experts(g, (int)layer, err, err_len);
    /* through the expert cache (model_cuda.cu:4757-4913): the slots of this layer's experts, the routing naming the
       slots, the kernels after the copies into them, then the guess's copies behind the kernels */
    if (k != (size_t)g->K) return fail(err, err_len, "%zu experts given; the model routes to %d", k, g->K);
    for (size_t i = 0; i < k; i++) {
        if (ids[i] < 0 || ids[i] >= g->E) return fail(err, err_len, "expert %d is outside the layer's %d", ids[i], g->E);
        for (size_t j = 0; j < i; j++)
            if (ids[j] == ids[i]) return fail(err, err_len, "expert %d is named twice", ids[i]); /* before any slot is taken */
        if (guess && (guess[i] < 0 || guess[i] >= g->E)) return fail(err, err_len, "guessed expert %d is outside the layer's %d", guess[i], g->E);
    }
    int32_t slot_of[ROUTE_K_MAX];
    bool ok = ec_acquire(g->ec, (int)layer, ids, (int)k, g->stream, slot_of, err, err_len) &&
              put_routing(g, 1, ids, weights, k, err, err_len, slot_of) && ec_wait(g->ec, slot_of, (int)k, g->stream, err, err_len) &&
              run_experts(g, (int)layer, err, err_len);
    /* the holds are released whatever happened; the guess only after the kernels */
    const bool fin = ec_finish(g->ec, (int)layer, ok ? guess : nullptr, (int)k, err, err_len);
    return ok && fin;
}

extern "C" bool vitna_hip_expert_cache_state(const struct vitna_cuda_model* g, int32_t* where, size_t n_places, uint64_t* counters,
                                             char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    const expert_cache& c = g->ec;
    if (!c.on) return fail(err, err_len, "every expert of this model is resident on the device");
    if (where) {
        if (n_places != c.n_places) return fail(err, err_len, "%zu places given; the model has %zu", n_places, c.n_places);
        memcpy(where, c.where.data(), c.n_places * sizeof(int32_t));
    }
    if (counters) {
        const uint64_t v[10] = {(uint64_t)c.n_slots, c.slot_bytes, c.n.acquired, c.n.hits, c.n.in_flight, c.n.misses, c.n.prefetched,
                                c.n.prefetch_used, c.n.copies, c.n.bytes_copied};
        memcpy(counters, v, sizeof(v));
    }
    return true;
}

/* Paths that read every expert from where it rests on the device refuse a model whose experts pass through the
   cache. */
static bool experts_resident(const vitna_cuda_model* g, char* err, size_t err_len) {
    if (!g->ec.on) return true;
    return fail(err, err_len,
                "the experts pass through a cache of %d slots on the device; this path needs every expert resident "
                "(vitna_cuda_moe_route and vitna_cuda_moe_experts take the cache)",
                g->ec.n_slots);
}

extern "C" bool vitna_cuda_moe_head(struct vitna_cuda_model* g, float* logits, char* err, size_t err_len) {
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!g->attention) return fail(err, err_len, "this model has no output projection");
    if (!check_launch(g, enqueue_head(g), "the head", err, err_len)) return false;
    if (logits) HIP_TRY(hipMemcpyAsync(logits, g->vocab, (size_t)g->V * 4, hipMemcpyDeviceToHost, g->stream), "copying the logits");
    HIP_TRY(hipStreamSynchronize(g->stream), "running the head");
    return true;
}

extern "C" const char* vitna_cuda_moe_report(const struct vitna_cuda_model* g, char* buf, size_t len) {
    if (len == 0) return buf;
    if (!g) { buf[0] = 0; return buf; }
    if (g->ec.on) {
        ec_report(g->ec, buf, len);
        return buf;
    }
    snprintf(buf, len, "experts: all %d of each of %d layers resident on the device; nothing copied per token", g->E, g->NL);
    return buf;
}

extern "C" int vitna_cuda_kv_layers(const struct vitna_cuda_model* g) { return g ? g->NL : 0; }
extern "C" void vitna_cuda_test_long_from(struct vitna_cuda_model* g, size_t n) { if (g) g->long_from = n; }
/* model_cuda.cu:3517: on a fast model, passes of n rows or more (n under the default) take the grouped GEMM */
extern "C" void vitna_cuda_test_fast_rows(struct vitna_cuda_model* g, size_t n) {
    if (g && g->fast && n >= 1 && n < g->fast_rows) g->fast_rows = n;
}

extern "C" bool vitna_cuda_cpu_experts(struct vitna_cuda_model* g, size_t threads, char* err, size_t err_len) {
    (void)g; (void)threads;
    return fail(err, err_len, "every expert is resident on the device, so none run on the CPU beside it");
}

extern "C" bool vitna_cuda_step(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, float* logits, char* err, size_t err_len) {
    (void)g; (void)seq; (void)token; (void)pos; (void)logits;
    return fail(err, err_len, "a mixture of experts runs a layer at a time (vitna_cuda_moe_route and vitna_cuda_moe_experts)");
}

extern "C" size_t vitna_cuda_prompt_min(const struct vitna_cuda_model* g) { (void)g; return SIZE_MAX; }
extern "C" size_t vitna_cuda_prompt_piece_min(const struct vitna_cuda_model* g) { (void)g; return 1; }
extern "C" size_t vitna_cuda_exact_max(const struct vitna_cuda_model* g) { return g ? ROWS_MAX : 0; }

extern "C" bool vitna_cuda_rows(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t count, float* const* logits, char* err,
                                size_t err_len) {
    (void)g; (void)rows; (void)count; (void)logits;
    return fail(err, err_len, "a mixture of experts runs rows a layer at a time (vitna_cuda_moe_rows_*)");
}

extern "C" bool vitna_cuda_steps(struct vitna_cuda_model* g, size_t seq, const int32_t* tokens, size_t count, size_t pos, float* logits,
                                 size_t rows, char* err, size_t err_len) {
    (void)g; (void)seq; (void)tokens; (void)count; (void)pos; (void)logits; (void)rows;
    return fail(err, err_len, "a mixture of experts runs a prompt as rows (vitna_cuda_moe_rows_*)");
}

extern "C" const char* vitna_cuda_device_name(const struct vitna_cuda_model* g) { return g ? g->name : ""; }

extern "C" void vitna_cuda_wait(struct vitna_cuda_model* g) {
    if (g) (void)hipStreamSynchronize(g->stream);
}

extern "C" bool vitna_cuda_lost(struct vitna_cuda_model* g, char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no device model") || true;
    (void)hipGetLastError();
    const hipError_t e = hipStreamSynchronize(g->stream);
    if (e != hipSuccess) {
        g->lost = true;
        fail_hip(err, err_len, "the device", e);
        return true;
    }
    return false;
}

/* ---- checkers ---------------------------------------------------------- */

extern "C" bool vitna_cuda_widen(const vitna_matrix_t* w, float* out, char* err, size_t err_len) {
    if (!w || !w->data || !out) return fail(err, err_len, "no matrix");
    if (!quant_ok(w->dtype) && w->dtype != VITNA_DTYPE_F32) return fail(err, err_len, "%s is not read on the device", dtype_name(w->dtype));
    const size_t rb = vitna_matrix_row_bytes(w->dtype, w->cols);
    if (!rb) return fail(err, err_len, "%zu columns are not whole %s blocks", w->cols, dtype_name(w->dtype));
    const size_t bytes = rb * w->rows, n = w->rows * w->cols;
    uint8_t *src = nullptr, *planes = nullptr;
    float *o1 = nullptr, *o2 = nullptr;
    bool ok = true;
    const size_t pb = w->dtype == VITNA_DTYPE_F32 ? bytes : set_bytes(w->dtype, w->rows, w->cols, 1);
    if (hipMalloc(&src, bytes) != hipSuccess || hipMalloc(&planes, pb) != hipSuccess || hipMalloc(&o1, n * 4) != hipSuccess ||
        hipMalloc(&o2, n * 4) != hipSuccess)
        ok = fail(err, err_len, "device memory for widening %zu weights", n);
    if (ok && hipMemcpy(src, w->data, bytes, hipMemcpyHostToDevice) != hipSuccess) ok = fail(err, err_len, "copying the matrix");
    if (ok) {
        qmat q;
        if (w->dtype == VITNA_DTYPE_F32) {
            memset(&q, 0, sizeof(q));
            q.p[0] = src; q.rows = (int)w->rows; q.cols = (int)w->cols; q.dtype = VITNA_DTYPE_F32;
        } else {
            q = place(planes, w->dtype, w->rows, w->cols, 1);
            if (launch_repack(src, q, 0) != hipSuccess) ok = fail(err, err_len, "splitting the blocks");
        }
        if (ok && (launch_widen_planes(q, 0, o1, 0) != hipSuccess || launch_widen_blocks(src, w->dtype, w->rows, w->cols, o2, 0) != hipSuccess))
            ok = fail(err, err_len, "widening");
        if (ok && hipDeviceSynchronize() != hipSuccess) ok = fail(err, err_len, "the device failed widening");
    }
    std::vector<float> a, b;
    if (ok) {
        a.resize(n);
        b.resize(n);
        if (hipMemcpy(a.data(), o1, n * 4, hipMemcpyDeviceToHost) != hipSuccess || hipMemcpy(b.data(), o2, n * 4, hipMemcpyDeviceToHost) != hipSuccess)
            ok = fail(err, err_len, "copying the widened weights back");
    }
    if (ok && memcmp(a.data(), b.data(), n * 4) != 0) ok = fail(err, err_len, "the two ways of reading the blocks disagree");
    if (ok) memcpy(out, a.data(), n * 4);
    (void)hipFree(src); (void)hipFree(planes); (void)hipFree(o1); (void)hipFree(o2);
    return ok;
}

extern "C" bool vitna_cuda_expert_check(const vitna_matrix_t* gate, const vitna_matrix_t* up, const vitna_matrix_t* down, const float* norm_w,
                                        const float* x, float eps, float* xs, float* act, float* y, char* err, size_t err_len) {
    if (!gate || !up || !down || !norm_w || !x) return fail(err, err_len, "missing arguments");
    const size_t H = gate->cols, I = gate->rows;
    if (!matrix_ok(gate, I, H, "gate", err, err_len) || !matrix_ok(up, I, H, "up", err, err_len) ||
        !matrix_ok(down, H, I, "down", err, err_len, false))
        return false;
    if (gate->dtype != up->dtype) return fail(err, err_len, "gate and up must share a dtype");
    if (H % 16 || H > 8192) return fail(err, err_len, "width %zu", H);
    hipStream_t s = 0;
    std::vector<void*> mem;
    auto dm = [&](size_t b) -> void* { void* p = nullptr; if (hipMalloc(&p, b) != hipSuccess) return nullptr; mem.push_back(p); return p; };
    bool ok = true;
    uint8_t* gm = (uint8_t*)dm(set_bytes(gate->dtype, I, H, 1));
    uint8_t* um = (uint8_t*)dm(set_bytes(up->dtype, I, H, 1));
    uint8_t* dmem = (uint8_t*)dm(set_bytes(down->dtype, H, I, 1));
    const size_t stb = std::max(vitna_matrix_row_bytes(gate->dtype, H) * I, vitna_matrix_row_bytes(down->dtype, I) * H);
    uint8_t* st = (uint8_t*)dm(stb);
    float* dx = (float*)dm(H * 4);
    float* dw = (float*)dm(H * 4);
    float* dxn = (float*)dm(H * 4);
    float* dl = (float*)dm(4 * 4);
    float* drouter = (float*)dm(H * 4);
    float* dact = (float*)dm(I * 4);
    float* dy = (float*)dm(H * 4);
    route_out* drt = (route_out*)dm(sizeof(route_out));
    unsigned* dctr = (unsigned*)dm(16);
    for (void* p : mem) ok = ok && p;
    if (!ok) { for (void* p : mem) (void)hipFree(p); return fail(err, err_len, "device memory for the expert check"); }
    qmat qg = place(gm, gate->dtype, I, H, 1), qu = place(um, up->dtype, I, H, 1), qd = place(dmem, down->dtype, H, I, 1);
    auto up_one = [&](const vitna_matrix_t* w, const qmat& q) {
        const size_t b = vitna_matrix_row_bytes(w->dtype, w->cols) * w->rows;
        return hipMemcpy(st, w->data, b, hipMemcpyHostToDevice) == hipSuccess && launch_repack(st, q, s) == hipSuccess &&
               hipDeviceSynchronize() == hipSuccess;
    };
    ok = up_one(gate, qg) && up_one(up, qu) && up_one(down, qd);
    route_out r;
    memset(&r, 0, sizeof(r));
    r.weights[0] = 1.0f;
    r.cw[0] = 1.0f; /* expert 0, the only one: ids[0] = chosen[0] = 0 */
    ok = ok && hipMemcpy(dx, x, H * 4, hipMemcpyHostToDevice) == hipSuccess && hipMemcpy(dw, norm_w, H * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(drt, &r, sizeof(r), hipMemcpyHostToDevice) == hipSuccess && hipMemset(dctr, 0, 16) == hipSuccess &&
         hipMemset(drouter, 0, H * 4) == hipSuccess;
    if (ok) {
        /* the norm a step uses (the router kernel's, with a one-row router) */
        route_args ra;
        memset(&ra, 0, sizeof(ra));
        ra.x = dx; ra.norm_w = dw; ra.router = drouter; ra.xn_out = dxn; ra.logits = dl;
        ra.H = (int)H; ra.E = 1; ra.n_rows = 1; ra.eps = eps;
        experts_in_args ai;
        ai.gate = qg; ai.up = qu; ai.xn = dxn; ai.rt = drt; ai.logits = nullptr; ai.E = 1; ai.renorm = 0; ai.act = dact; ai.K = 1;
        experts_down_args ad;
        ad.down = qd; ad.act = dact; ad.rt = drt; ad.y = dy; ad.K = 1; ad.add = 0; ad.parts = nullptr; ad.n_parts = 0;
        ok = launch_route(ra, s) == hipSuccess && launch_experts_in(ai, s) == hipSuccess && launch_experts_down(ad, s) == hipSuccess &&
             hipDeviceSynchronize() == hipSuccess;
        if (!ok) fail(err, err_len, "the expert's kernels failed or do not take this shape");
    } else {
        fail(err, err_len, "uploading the expert failed");
    }
    if (ok) {
        ok = (!xs || hipMemcpy(xs, dxn, H * 4, hipMemcpyDeviceToHost) == hipSuccess) &&
             (!act || hipMemcpy(act, dact, I * 4, hipMemcpyDeviceToHost) == hipSuccess) &&
             (!y || hipMemcpy(y, dy, H * 4, hipMemcpyDeviceToHost) == hipSuccess);
        if (!ok) fail(err, err_len, "copying the expert's results back");
    }
    for (void* p : mem) (void)hipFree(p);
    return ok;
}

/* ---- extensions --------------------------------------------------------- */

/* The persistent step's resources, on first use: whether the model's shape takes it, the layer table, the
   activation buffers and the flags (zeroed: the first launch's epoch is 1). */
static bool ensure_step(vitna_cuda_model* g, char* err, size_t err_len) {
    if (g->step_state) return true;
    const int H = g->H, qd = g->nh * g->hd, kd = g->nkv * g->hd, G = g->nkv ? g->nh / g->nkv : 1;
    int nb = std::min(256, gemv_device_cus());
    /* the largest block count the o-projection's split divides */
    const char* why = nullptr;
    for (; nb >= 8; nb--)
        if (!(why = step_unsupported(H, g->I, g->E, g->K, g->nh, g->nkv, g->hd, nb, g->attention ? g->L[0].q.dtype : 0,
                                     g->attention ? g->L[0].k.dtype : 0, g->attention ? g->L[0].v.dtype : 0,
                                     g->attention ? g->L[0].o.dtype : 0, g->L[0].gate.dtype, g->L[0].down.dtype)))
            break;
    bool same = true;
    for (int l = 1; l < g->NL; l++)
        same &= g->L[l].gate.dtype == g->L[0].gate.dtype && g->L[l].down.dtype == g->L[0].down.dtype &&
                (!g->attention || (g->L[l].o.dtype == g->L[0].o.dtype && g->L[l].q.dtype == g->L[0].q.dtype &&
                                   g->L[l].k.dtype == g->L[0].k.dtype && g->L[l].v.dtype == g->L[0].v.dtype));
    if (why || nb < 8 || !same) {
        g->step_state = -1;
        g->step_reason = why ? why : "dtypes that differ between layers";
        return true;
    }
    const size_t prec = (size_t)g->hd + 4;
    step_args& a = g->step_base;
    memset(&a, 0, sizeof(a));
    a.s_qkv = (size_t)qd + 2 * kd;
    a.s_part = (size_t)nb * G * prec;
    a.s_opart = g->attention ? (size_t)(qd / 256) * H : 0;
    a.s_att = qd;
    a.s_xmid = H;
    a.s_logits = g->E;
    a.s_act = (size_t)g->K * g->I;
    auto al4 = [](size_t n) { return (n + 63) & ~(size_t)63; }; /* 256-byte aligned parts */
    a.s_qkv = al4(a.s_qkv); a.s_part = al4(a.s_part); a.s_opart = al4(a.s_opart); a.s_att = al4(a.s_att);
    a.s_xmid = al4(a.s_xmid); a.s_logits = al4(a.s_logits); a.s_act = al4(a.s_act);
    const size_t per_layer = a.s_qkv + a.s_part + a.s_opart + a.s_att + a.s_xmid + a.s_logits + a.s_act + al4(H);
    if (!dalloc(g, &g->step_buf, per_layer * g->NL * 4, "the step's activation buffers", err, err_len)) return false;
    const size_t nflags = (size_t)g->NL * STEP_PHASES * 256 + 64;
    if (!dalloc(g, &g->step_flags, nflags * 4, "the step's flags", err, err_len)) return false;
    if (!dalloc(g, &g->step_L, g->NL * sizeof(step_layer), "the step's layer table", err, err_len)) return false;
    HIP_TRY(hipMemset(g->step_flags, 0, nflags * 4), "clearing the step's flags");
    std::vector<step_layer> lt(g->NL);
    for (int l = 0; l < g->NL; l++) {
        const dlayer& d = g->L[l];
        step_layer& t = lt[l];
        memset(&t, 0, sizeof(t));
        t.q = d.q; t.k = d.k; t.v = d.v; t.o = d.o; t.gate = d.gate; t.up = d.up; t.down = d.down;
        t.attn_norm = d.attn_norm; t.mlp_norm = d.mlp_norm; t.q_norm = d.q_norm; t.k_norm = d.k_norm; t.router = d.router;
        if (g->attention) {
            t.k_cache = g->k_cache + (size_t)l * g->layer_kv;
            t.v_cache = g->v_cache + (size_t)l * g->layer_kv;
        }
    }
    HIP_TRY(hipMemcpy(g->step_L, lt.data(), g->NL * sizeof(step_layer), hipMemcpyHostToDevice), "uploading the layer table");
    float* p = g->step_buf;
    a.qkv = p; p += a.s_qkv * g->NL;
    a.part = p; p += a.s_part * g->NL;
    a.opart = p; p += a.s_opart * g->NL;
    a.att = p; p += a.s_att * g->NL;
    a.xmid = p; p += a.s_xmid * g->NL;
    a.logits = p; p += a.s_logits * g->NL;
    a.act = p; p += a.s_act * g->NL;
    a.xout = p;
    a.flags = g->step_flags;
    a.abort_word = g->step_flags + (size_t)g->NL * STEP_PHASES * 256;
    a.L = g->step_L;
    a.NL = g->NL;
    a.embed = g->embed;
    a.row = g->rows_dev;
    a.cos_tab = g->cos_tab;
    a.sin_tab = g->sin_tab;
    a.seq_stride = (size_t)g->NL * g->layer_kv;
    a.rt_layers = g->rt_layers;
    a.rt_last = g->rt;
    a.x0 = g->x;
    a.x_final = g->x;
    a.H = H; a.I = g->I; a.E = g->E; a.K = g->K; a.nh = g->nh; a.nkv = g->nkv; a.hd = g->hd;
    a.renorm = g->renorm; a.attention = g->attention ? 1 : 0;
    a.eps = g->eps;
    a.nb = nb;
    a.poll_nap = 1;
    if (const char* v = getenv("VITNA_STEP_NAP")) a.poll_nap = atoi(v);
    g->step_nb = nb;
    g->step_epoch = 0;
    g->step_state = 1;
    return true;
}

/* Whether this call runs the persistent step: asked for, and the model's shape takes it. */
static bool use_step(vitna_cuda_model* g, bool* mega, char* err, size_t err_len) {
    *mega = false;
    if (!g->step_want) return true;
    if (!ensure_step(g, err, err_len)) return false;
    *mega = g->step_state > 0;
    return true;
}

/* One launch of the persistent step over layers first .. first + n - 1 (the whole model, or one layer of a model
   without attention), on residual row 0. */
static hipError_t launch_step_layers(vitna_cuda_model* g, int first, int n, uint64_t* trace = nullptr, int trace_block = 0) {
    step_args a = g->step_base;
    a.trace = trace;
    a.trace_block = trace_block;
    g->last_step_mega = true;
    g->last_mega_n = n;
    a.L = g->step_L + first;
    a.NL = n;
    a.rt_layers = g->rt_layers + first;
    a.epoch = ++g->step_epoch;
    const dlayer& d = g->L[first];
    const int dts[5] = {d.gate.dtype, d.down.dtype, g->attention ? d.q.dtype : 0, g->attention ? d.v.dtype : 0,
                        g->attention ? d.o.dtype : 0};
    return launch_step(a, dts, g->stream);
}

/* After a synchronized persistent step: its abort word, cleared, as an error. */
static bool step_check(vitna_cuda_model* g, char* err, size_t err_len) {
    uint32_t ab = 0;
    HIP_TRY(hipMemcpy(&ab, g->step_base.abort_word, 4, hipMemcpyDeviceToHost), "reading the step's state");
    if (ab) {
        (void)hipMemset(g->step_base.abort_word, 0, 4);
        return fail(err, err_len, "the persistent step gave up waiting for a block (a block did not run or did not finish)");
    }
    return true;
}

static hipError_t enqueue_step_body(vitna_cuda_model* g) {
    hipError_t e = launch_embed(g->embed, &g->rows_dev[0].token, 0, g->x, g->stream);
    for (int l = 0; e == hipSuccess && l < g->NL; l++) {
        e = enqueue_attention(g, l, 1, false);
        if (e == hipSuccess) e = enqueue_route(g, l, g->rlogits, 1, g->x, g->xn, true);
        /* each layer's routing kept for the checkers; the last layer's where the rows' routing is read */
        if (e == hipSuccess) e = enqueue_experts(g, l, g->rlogits, g->x, 1, l + 1 < g->NL ? g->rt_layers + l : g->rt);
    }
    if (e == hipSuccess) e = enqueue_head(g);
    return e;
}

static bool ensure_graph(vitna_cuda_model* g, char* err, size_t err_len) {
    if (g->graph_ready && g->graph_splits == g->splits_grid) return true;
    HIP_TRY(hipStreamSynchronize(g->stream), "before capturing the step");
    if (g->graph_ready) {
        /* captured for another attention grid: captured again for this one */
        (void)hipGraphExecDestroy(g->step_graph);
        (void)hipGraphDestroy(g->step_graph_src);
        g->graph_ready = false;
    }
    HIP_TRY(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal), "capturing the step");
    const hipError_t e = enqueue_step_body(g);
    hipGraph_t graph = nullptr;
    const hipError_t e2 = hipStreamEndCapture(g->stream, &graph);
    if (e != hipSuccess) { if (graph) (void)hipGraphDestroy(graph); return check_launch(g, e, "capturing the step", err, err_len); }
    HIP_TRY(e2, "ending the capture of the step");
    const hipError_t e3 = hipGraphInstantiate(&g->step_graph, graph, nullptr, nullptr, 0);
    if (e3 != hipSuccess) (void)hipGraphDestroy(graph);
    HIP_TRY(e3, "instantiating the step's graph");
    g->step_graph_src = graph;
    g->graph_ready = true;
    g->graph_splits = g->splits_grid;
    return true;
}

extern "C" bool vitna_hip_moe_step_async(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!g->attention) return fail(err, err_len, "this model has no attention; use vitna_hip_moe_ffn");
    bool mega;
    if (!use_step(g, &mega, err, err_len)) return false;
    if (mega) {
        if (!set_row(g, seq, token, pos, err, err_len)) return false;
        hipError_t e = launch_step_layers(g, 0, g->NL);
        if (e == hipSuccess) e = enqueue_head(g);
        g->last_step_mega = true;
        return check_launch(g, e, "the step", err, err_len);
    }
    if (!set_row(g, seq, token, pos, err, err_len)) return false;
    if (!ensure_graph(g, err, err_len)) return false;
    HIP_TRY(hipGraphLaunch(g->step_graph, g->stream), "launching the step");
    g->last_step_mega = false;
    return true;
}

extern "C" bool vitna_hip_moe_step(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, float* logits, char* err,
                                   size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!vitna_hip_moe_step_async(g, seq, token, pos, err, err_len)) return false;
    if (logits) HIP_TRY(hipMemcpyAsync(logits, g->vocab, (size_t)g->V * 4, hipMemcpyDeviceToHost, g->stream), "copying the logits");
    HIP_TRY(hipStreamSynchronize(g->stream), "running the step");
    return !g->last_step_mega || step_check(g, err, err_len);
}

extern "C" bool vitna_hip_set_step_kernel(struct vitna_cuda_model* g, int on, int* taken, char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    g->step_want = on != 0;
    bool mega = false;
    if (!use_step(g, &mega, err, err_len)) return false;
    if (taken) *taken = mega ? 1 : 0;
    return true;
}

extern "C" bool vitna_hip_step_trace(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, int block, uint64_t* out, size_t n,
                                     char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!ensure_step(g, err, err_len)) return false;
    if (g->step_state < 1) return fail(err, err_len, "this model runs the per-layer kernels (%s)", g->step_reason);
    if (block < 0 || block >= g->step_nb) return fail(err, err_len, "block %d: the step runs %d", block, g->step_nb);
    const size_t need = (size_t)g->NL * STEP_TRACE_PER_LAYER;
    if (n < need) return fail(err, err_len, "the timeline takes %zu words", need);
    if (!g->step_trace && !dalloc(g, &g->step_trace, need * 8, "the step's timeline", err, err_len)) return false;
    HIP_TRY(hipMemset(g->step_trace, 0, need * 8), "clearing the timeline");
    if (g->attention && !set_row(g, seq, token, pos, err, err_len)) return false;
    if (!check_launch(g, launch_step_layers(g, 0, g->NL, g->step_trace, block), "the traced step", err, err_len)) return false;
    HIP_TRY(hipStreamSynchronize(g->stream), "running the traced step");
    if (!step_check(g, err, err_len)) return false;
    HIP_TRY(hipMemcpy(out, g->step_trace, need * 8, hipMemcpyDeviceToHost), "copying the timeline");
    return true;
}

extern "C" bool vitna_hip_moe_ffn(struct vitna_cuda_model* g, size_t layer, char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    bool mega = false;
    if (!g->attention && !use_step(g, &mega, err, err_len)) return false;
    if (mega) {
        /* the persistent step, one layer, no attention: route, experts, sum onto row 0 */
        if (!check_launch(g, launch_step_layers(g, (int)layer, 1), "the mixture of experts", err, err_len)) return false;
        HIP_TRY(hipStreamSynchronize(g->stream), "running the mixture of experts");
        return step_check(g, err, err_len);
    }
    g->last_step_mega = false;
    hipError_t e = enqueue_route(g, (int)layer, g->rlogits, 1, g->x, g->xn, true);
    if (e == hipSuccess) e = enqueue_experts(g, (int)layer, g->rlogits, g->x, 1);
    return check_launch(g, e, "the mixture of experts", err, err_len);
}

extern "C" bool vitna_hip_residual(struct vitna_cuda_model* g, size_t row, float* host, bool to_device, char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    if (row >= ROWS_MAX) return fail(err, err_len, "row %zu: at most %d", row, ROWS_MAX);
    float* d = g->x + row * g->H;
    if (row == 0 && g->parts_n) {
        /* the row's attention parts still pending: read, the residual has them; written, the new residual
           replaces what they would complete */
        if (!to_device) HIP_TRY(launch_attn_fold(g->x, g->parts, g->parts_n, g->H, g->stream), "adding the attention's parts");
        g->parts_n = 0;
    }
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    HIP_TRY(to_device ? hipMemcpy(d, host, g->H * 4, hipMemcpyHostToDevice) : hipMemcpy(host, d, g->H * 4, hipMemcpyDeviceToHost),
            "copying the residual");
    return true;
}

static hipError_t enqueue_multi(vitna_cuda_model* g, const gemv_multi_args& m, bool imaged);

extern "C" bool vitna_hip_rows_project(struct vitna_cuda_model* g, size_t layer, int which, const float* x, size_t n, float* y,
                                       char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    if (!ensure_tiled(g, err, err_len)) return false;
    if (!g->attention) return fail(err, err_len, "the model has no attention projections");
    if (n < 1 || n > ROWS_MAX) return fail(err, err_len, "%zu rows: 1 .. %d", n, ROWS_MAX);
    if (which < 0 || which > 4 || (which < 4 && layer >= (size_t)g->NL)) return fail(err, err_len, "no such projection");
    const qmat w = which == 0 ? g->L[layer].q : which == 1 ? g->L[layer].k : which == 2 ? g->L[layer].v : which == 3 ? g->L[layer].o : g->head;
    /* the input where the step keeps it (normed rows, or the attention output for o), the output in scratch of
       at least n x rows floats */
    float* dx = which == 3 ? g->att : g->xn;
    float* dy = which == 0 ? g->q : which == 1 ? g->k : which == 2 ? g->v : which == 3 ? g->ypart : g->vocab;
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    HIP_TRY(hipMemcpy(dx, x, n * w.cols * 4, hipMemcpyHostToDevice), "copying the rows");
    gemv_multi_args m;
    memset(&m, 0, sizeof(m));
    m.w[0] = w; m.y[0] = dy; m.nm = 1; m.x = dx; m.n = (int)n; m.xstride = w.cols;
    HIP_TRY(enqueue_multi(g, m, false), "the projection");
    HIP_TRY(hipStreamSynchronize(g->stream), "the projection");
    HIP_TRY(hipMemcpy(y, dy, n * w.rows * 4, hipMemcpyDeviceToHost), "copying the result");
    return true;
}

extern "C" bool vitna_hip_routing(struct vitna_cuda_model* g, size_t row, float* logits, int32_t* chosen, int32_t* ids, float* weights,
                                  char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    if (row >= ROWS_MAX) return fail(err, err_len, "row %zu: at most %d", row, ROWS_MAX);
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    route_out r;
    HIP_TRY(hipMemcpy(&r, g->rt + row, sizeof(r), hipMemcpyDeviceToHost), "copying the routing");
    const float* lsrc = g->rlogits + row * g->E;
    if (g->last_step_mega && row == 0) /* the persistent step keeps each layer's logits in its own buffer */
        lsrc = g->step_base.logits + (size_t)(g->last_mega_n - 1) * g->step_base.s_logits;
    if (logits) HIP_TRY(hipMemcpy(logits, lsrc, g->E * 4, hipMemcpyDeviceToHost), "copying the router's logits");
    for (int k = 0; k < g->K; k++) {
        if (chosen) chosen[k] = r.chosen[k];
        if (ids) ids[k] = r.ids[k];
        if (weights) weights[k] = r.weights[k];
    }
    return true;
}

extern "C" bool vitna_hip_step_routing(struct vitna_cuda_model* g, size_t layer, int32_t* chosen, int32_t* ids, float* weights,
                                       char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    route_out r;
    const route_out* src = layer + 1 < (size_t)g->NL ? g->rt_layers + layer : g->rt;
    HIP_TRY(hipMemcpy(&r, src, sizeof(r), hipMemcpyDeviceToHost), "copying the routing");
    for (int k = 0; k < g->K; k++) {
        if (chosen) chosen[k] = r.chosen[k];
        if (ids) ids[k] = r.ids[k];
        if (weights) weights[k] = r.weights[k];
    }
    return true;
}

extern "C" bool vitna_hip_rows_routing(struct vitna_cuda_model* g, size_t layer, size_t row, int32_t* chosen, int32_t* ids,
                                       float* weights, char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    if (row >= ROWS_MAX) return fail(err, err_len, "row %zu: at most %d", row, ROWS_MAX);
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    route_out r;
    const route_out* src = layer + 1 < (size_t)g->NL ? g->rows_rt + layer * ROWS_MAX + row : g->rt + row;
    HIP_TRY(hipMemcpy(&r, src, sizeof(r), hipMemcpyDeviceToHost), "copying the routing");
    for (int k = 0; k < g->K; k++) {
        if (chosen) chosen[k] = r.chosen[k];
        if (ids) ids[k] = r.ids[k];
        if (weights) weights[k] = r.weights[k];
    }
    return true;
}

extern "C" bool vitna_hip_attention_io(struct vitna_cuda_model* g, size_t row, float* q, float* att, char* err, size_t err_len) {
    if (!g || !g->attention) return fail(err, err_len, "no attention");
    if (row >= ROWS_MAX) return fail(err, err_len, "row %zu: at most %d", row, ROWS_MAX);
    const size_t qd = (size_t)g->nh * g->hd;
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    if (g->last_step_mega && row == 0) {
        /* the persistent step keeps each layer's q/k/v and attention output in its own buffers */
        const step_args& a = g->step_base;
        const size_t l = (size_t)g->NL - 1;
        if (q) HIP_TRY(hipMemcpy(q, a.qkv + l * a.s_qkv, qd * 4, hipMemcpyDeviceToHost), "copying q");
        if (att) HIP_TRY(hipMemcpy(att, a.att + l * a.s_att, qd * 4, hipMemcpyDeviceToHost), "copying the attention output");
        return true;
    }
    if (q) HIP_TRY(hipMemcpy(q, g->q + row * qd, qd * 4, hipMemcpyDeviceToHost), "copying q");
    if (att) HIP_TRY(hipMemcpy(att, g->att + row * qd, qd * 4, hipMemcpyDeviceToHost), "copying the attention output");
    return true;
}

extern "C" bool vitna_hip_kv(struct vitna_cuda_model* g, size_t seq, size_t layer, size_t pos0, size_t n, float* k, float* v, bool write,
                             char* err, size_t err_len) {
    if (!g || !g->attention) return fail(err, err_len, "no key-value cache");
    if (seq >= (size_t)g->seqs || layer >= (size_t)g->NL || pos0 + n > (size_t)g->ctx) return fail(err, err_len, "outside the cache");
    const size_t kd = (size_t)g->nkv * g->hd;
    const size_t off = ((size_t)seq * g->NL + layer) * g->layer_kv + pos0 * kd;
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting for the device");
    const hipMemcpyKind kind = write ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
    if (k) HIP_TRY(write ? hipMemcpy(g->k_cache + off, k, n * kd * 4, kind) : hipMemcpy(k, g->k_cache + off, n * kd * 4, kind), "copying keys");
    if (v) HIP_TRY(write ? hipMemcpy(g->v_cache + off, v, n * kd * 4, kind) : hipMemcpy(v, g->v_cache + off, n * kd * 4, kind), "copying values");
    return true;
}

extern "C" bool vitna_hip_kv_fill(struct vitna_cuda_model* g, uint64_t seed, const size_t* n_pos, char* err, size_t err_len) {
    if (!g || !g->attention) return fail(err, err_len, "no key-value cache");
    const size_t kd = (size_t)g->nkv * g->hd;
    for (int s = 0; s < g->seqs; s++) {
        const size_t n = std::min(n_pos[s], (size_t)g->ctx);
        for (int l = 0; l < g->NL; l++) {
            const size_t off = ((size_t)s * g->NL + l) * g->layer_kv;
            const uint64_t tag = (seed * 1000003ull + (uint64_t)s) * 1000003ull + (uint64_t)l;
            HIP_TRY(launch_fill_normal(g->k_cache + off, n * kd, 2 * tag + 1, g->stream), "filling keys");
            HIP_TRY(launch_fill_normal(g->v_cache + off, n * kd, 2 * tag + 2, g->stream), "filling values");
        }
    }
    HIP_TRY(hipStreamSynchronize(g->stream), "filling the cache");
    return true;
}

extern "C" bool vitna_hip_sync(struct vitna_cuda_model* g, char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    HIP_TRY(hipStreamSynchronize(g->stream), "the device");
    return true;
}

extern "C" void* vitna_hip_stream(struct vitna_cuda_model* g) { return g ? (void*)g->stream : nullptr; }
extern "C" const float* vitna_hip_logits_device(struct vitna_cuda_model* g) { return g ? g->vocab : nullptr; }

static double qmat_bytes(const qmat& q) {
    double b = 0;
    for (int i = 0; i < 4; i++) b += (double)plane_bytes(q.dtype, i, q.rows, q.cols);
    return b;
}

extern "C" bool vitna_hip_time_kernel(struct vitna_cuda_model* g, int which, int reps, int warmup, double* avg_us, double* bytes, char* err,
                                      size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if ((which >= 3 && which <= 6 && !g->attention) || which < 0 || which > 9)
        return fail(err, err_len, "no such kernel (%d) in this model", which);
    event_pair ev;
    HIP_TRY(ev.make(), "events");
    hipEvent_t t0 = ev.t0, t1 = ev.t1;
    double b = 0;
    const int H = g->H, K = g->K;
    auto one = [&](int i) -> hipError_t {
        const int l = i % g->NL;
        const dlayer& d = g->L[l];
        switch (which) {
            case 0: {
                experts_in_args ai;
                ai.gate = d.gate; ai.up = d.up; ai.xn = g->xn; ai.rt = g->rt; ai.logits = g->rlogits; ai.E = g->E;
                ai.renorm = g->renorm; ai.act = g->act; ai.K = K;
                b = 2.0 * K * qmat_bytes(d.gate) + H * 4.0 + K * (double)g->I * 4 + g->E * 4.0;
                return launch_experts_in(ai, g->stream);
            }
            case 8:
                /* the routing rule alone, one block */
                b = g->E * 4.0;
                return launch_route_check(g->rlogits, g->E, g->K, g->renorm, g->rt, g->stream);
            case 9:
                /* an empty launch: the floor of any kernel */
                b = 0;
                return launch_fill_normal(g->ypart, 0, 0, g->stream) == hipSuccess ? launch_route_check(g->rlogits, 4, 1, 0, g->rt + 1, g->stream)
                                                                                   : hipErrorInvalidValue;
            case 7:
                /* the router without the top-k */
                b = (double)g->E * H * 4 + H * 8.0 + g->E * 4.0;
                return enqueue_route(g, l, g->rlogits, 1, g->x, g->xn, false);
            case 1: {
                experts_down_args ad;
                ad.down = d.down; ad.act = g->act; ad.rt = g->rt; ad.y = g->ypart; ad.K = K; ad.add = 0; ad.parts = nullptr; ad.n_parts = 0;
                b = K * qmat_bytes(d.down) + K * (double)g->I * 4 + H * 4.0;
                return launch_experts_down(ad, g->stream);
            }
            case 2:
                b = (double)g->E * H * 4 + H * 8.0 + g->E * 4.0;
                return enqueue_route(g, l, g->rlogits, 1, g->x, g->xn, true);
            case 3: {
                gemv_args ga;
                memset(&ga, 0, sizeof(ga));
                ga.w[0] = d.q; ga.w[1] = d.k; ga.w[2] = d.v; ga.y[0] = g->q; ga.y[1] = g->k; ga.y[2] = g->v; ga.n = 3;
                ga.x = g->x; ga.norm_w = d.attn_norm; ga.eps = g->eps;
                b = qmat_bytes(d.q) + qmat_bytes(d.k) + qmat_bytes(d.v) + H * 8.0;
                return launch_gemv(ga, g->stream);
            }
            case 4: {
                attn_args a;
                memset(&a, 0, sizeof(a));
                a.q_raw = g->q; a.k_raw = g->k; a.v_raw = g->v; a.q_norm = d.q_norm; a.k_norm = d.k_norm;
                a.cos_tab = g->cos_tab; a.sin_tab = g->sin_tab;
                a.k_cache = g->k_cache + (size_t)l * g->layer_kv; a.v_cache = g->v_cache + (size_t)l * g->layer_kv;
                a.seq_stride = (size_t)g->NL * g->layer_kv; a.rows = g->rows_dev; a.n_rows = 1; a.partial = g->partial;
                a.att = g->att; a.n_heads = g->nh; a.n_kv = g->nkv; a.hd = g->hd; a.ctx = g->ctx;
                a.splits_max = g->splits_max; a.eps = g->eps; a.mma = 1;
                b = 0; /* set by the caller from the position */
                const hipError_t e = launch_attention(a, g->stream);
                if (e != hipSuccess) return e;
                /* as the step runs it: the merge with the o-projection where the layer takes it */
                if (attention_oproj_fits(a, d.o)) return launch_attention_oproj(a, d.o, g->parts, g->stream);
                return launch_attention_merge(a, g->stream);
            }
            case 5: {
                gemv_args go;
                memset(&go, 0, sizeof(go));
                go.w[0] = d.o; go.y[0] = g->ypart; go.n = 1; go.x = g->att;
                b = qmat_bytes(d.o) + (double)g->nh * g->hd * 4 + H * 4.0;
                return launch_gemv(go, g->stream);
            }
            default:
                b = qmat_bytes(g->head) + H * 8.0 + (double)g->V * 4;
                return enqueue_head(g);
        }
    };
    for (int i = 0; i < warmup; i++)
        if (!check_launch(g, one(i), "timing", err, err_len)) return false;
    HIP_TRY(hipEventRecord(t0, g->stream), "events");
    for (int i = 0; i < reps; i++)
        if (!check_launch(g, one(warmup + i), "timing", err, err_len)) return false;
    HIP_TRY(hipEventRecord(t1, g->stream), "events");
    HIP_TRY(hipEventSynchronize(t1), "timing");
    float ms = 0;
    HIP_TRY(hipEventElapsedTime(&ms, t0, t1), "events");
    if (avg_us) *avg_us = 1000.0 * ms / reps;
    if (bytes) *bytes = b;
    return true;
}

/* Rows and prefill: kernels_rows.hip. */

/* ---- prefill through one MoE layer: kernels_prefill.hip ---- */

static bool sync_stream(vitna_cuda_model* g, const char* what, char* err, size_t err_len) {
    HIP_TRY(hipStreamSynchronize(g->stream), what);
    return true;
}

/* The bytes a prefill of n rows needs for its working buffers; with base, the buffers' places in that region
   (each part 256-byte aligned). */
static size_t prefill_layout(const vitna_cuda_model* g, size_t n, char* base, pf_bufs* b) {
    const size_t H = g->H, E = g->E, K = g->K, I = g->I;
    const size_t tiles = (size_t)prefill_max_tiles((int)n, (int)K, (int)E) + 1;
    size_t at = 0;
    auto part = [&](auto** ptr, size_t bytes) {
        if (base) *ptr = reinterpret_cast<std::remove_reference_t<decltype(*ptr)>>(base + at);
        at += (bytes + 255) & ~(size_t)255;
    };
    pf_bufs dummy;
    pf_bufs& d = b ? *b : dummy;
    part(&d.xn, n * H * 4);
    part(&d.xb, n * H * 2);
    part(&d.logits, n * E * 4);
    part(&d.rt, n * sizeof(route_out));
    part(&d.count, E * 4);
    part(&d.pairs, E * n * 4);
    part(&d.off, E * 4);
    part(&d.tiles, tiles * 4);
    part(&d.ntiles, 4);
    part(&d.act, n * K * I * 2);
    part(&d.ypart, n * K * H * 2);
    return at;
}

static bool prefill_reserve(vitna_cuda_model* g, size_t n, char* err, size_t err_len) {
    /* the experts' tiled copy the prefill GEMM reads (made once) */
    if (!ensure_tiled(g, err, err_len)) return false;
    if (n <= g->pf_cap) return true;
    HIP_TRY(hipStreamSynchronize(g->stream), "waiting before the prefill buffers grow");
    /* a captured rows step of a fast pass reads these buffers: it is captured again on its next use */
    drop_rows_graphs(g);
    for (void* p : g->pf_allocs) (void)hipFree(p);
    g->pf_allocs.clear();
    g->pf_cap = 0;
    auto get = [&](void** ptr, size_t bytes) -> bool {
        void* p = nullptr;
        const hipError_t e = hipMalloc(&p, bytes ? bytes : 256);
        if (e != hipSuccess) return fail(err, err_len, "device memory for a prefill of %zu rows (%zu bytes): %s", n, bytes, hipGetErrorString(e));
        g->pf_allocs.push_back(p);
        *ptr = p;
        return true;
    };
    void *x = nullptr, *x0 = nullptr, *region = nullptr;
    if (!(get(&x, n * g->H * 4) && get(&x0, n * g->H * 4) && get(&region, prefill_layout(g, n, nullptr, nullptr)))) return false;
    g->pf_x = static_cast<float*>(x);
    g->pf_x0 = static_cast<float*>(x0);
    prefill_layout(g, n, static_cast<char*>(region), &g->pf);
    g->pf_cap = n;
    return true;
}

/* The phases of a prefill of the n rows at x (device), in place, on the working buffers b; ev (6 events or NULL)
   marks their boundaries: norm + router | routing + grouping + plan | gate/up GEMM | down GEMM | ordered sum. */
static hipError_t enqueue_prefill(vitna_cuda_model* g, int layer, int n, float* x, const pf_bufs& b, hipEvent_t* ev) {
    const dlayer& d = g->L[layer];
    hipStream_t s = g->stream;
    hipError_t e = hipSuccess;
    auto mark = [&](int i) { if (ev && e == hipSuccess) e = hipEventRecord(ev[i], s); };
    mark(0);
    if (e == hipSuccess) {
        e = launch_prefill_norm_router(x, d.mlp_norm, d.router, b.logits, b.xb, n, g->E, g->H, g->eps, s);
        if (e == hipErrorNotSupported) {
            e = launch_prefill_norm(x, d.mlp_norm, b.xn, b.xb, n, g->H, g->eps, s);
            if (e == hipSuccess) e = launch_prefill_router(b.xn, d.router, b.logits, n, g->E, g->H, s);
        }
    }
    mark(1);
    if (e == hipSuccess) e = launch_topk(b.logits, n, g->E, g->K, g->renorm, b.rt, s);
    if (e == hipSuccess) e = launch_group(b.rt, n, g->E, g->K, n, b.count, b.pairs, s);
    if (e == hipSuccess) e = launch_prefill_plan(b.count, g->E, b.off, b.tiles, b.ntiles, s);
    mark(2);
    prefill_args a;
    a.gate = d.gate; a.up = d.up; a.down = d.down;
    a.xb = b.xb; a.rt = b.rt; a.count = b.count; a.pairs = b.pairs; a.off = b.off;
    a.tiles = b.tiles; a.n_tiles = b.ntiles; a.act = b.act; a.ypart = b.ypart;
    a.E = g->E; a.K = g->K; a.cap = n; a.n = n;
    if (e == hipSuccess) e = launch_prefill_gemm(a, true, s);
    mark(3);
    if (e == hipSuccess) e = launch_prefill_gemm(a, false, s);
    mark(4);
    if (e == hipSuccess) e = launch_prefill_sum(b.ypart, x, n, g->K, g->H, s);
    mark(5);
    return e;
}

static bool prefill_check(vitna_cuda_model* g, size_t layer, size_t n, char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    if (g->lost) return fail(err, err_len, "the device was lost earlier");
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    if (n < 1 || n > 65536) return fail(err, err_len, "%zu rows: a prefill takes 1 to 65536", n);
    /* every expert set the model check accepts (Q8_0, Q4_K or Q6_K; widths multiples of 256) fits the GEMM */
    return true;
}

extern "C" bool vitna_hip_moe_prefill(struct vitna_cuda_model* g, size_t layer, float* x, size_t n, int32_t* chosen, char* err,
                                      size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!prefill_check(g, layer, n, err, err_len)) return false;
    if (!x) return fail(err, err_len, "no rows");
    HIP_TRY(hipSetDevice(g->device), "selecting the model's device");
    if (!prefill_reserve(g, n, err, err_len)) return false;
    HIP_TRY(hipMemcpyAsync(g->pf_x, x, n * g->H * 4, hipMemcpyHostToDevice, g->stream), "copying the rows to the device");
    if (!check_launch(g, enqueue_prefill(g, (int)layer, (int)n, g->pf_x, g->pf, nullptr), "the prefill", err, err_len)) return false;
    HIP_TRY(hipMemcpyAsync(x, g->pf_x, n * g->H * 4, hipMemcpyDeviceToHost, g->stream), "copying the rows back");
    if (chosen) {
        std::vector<route_out> rt(n);
        HIP_TRY(hipMemcpyAsync(rt.data(), g->pf.rt, n * sizeof(route_out), hipMemcpyDeviceToHost, g->stream), "copying the routing");
        if (!sync_stream(g, "the prefill", err, err_len)) return false;
        for (size_t i = 0; i < n; i++)
            for (int k = 0; k < g->K; k++) chosen[i * g->K + k] = rt[i].chosen[k];
        return true;
    }
    return sync_stream(g, "the prefill", err, err_len);
}

extern "C" bool vitna_hip_time_prefill(struct vitna_cuda_model* g, size_t layer, size_t n, uint64_t seed, int reps, double* us_total,
                                       double* us_phase, char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!prefill_check(g, layer, n, err, err_len)) return false;
    if (reps < 1) return fail(err, err_len, "reps must be positive");
    HIP_TRY(hipSetDevice(g->device), "selecting the model's device");
    if (!prefill_reserve(g, n, err, err_len)) return false;
    HIP_TRY(launch_fill_normal(g->pf_x0, n * g->H, seed, g->stream), "filling the rows");
    hipEvent_t ev[6];
    for (int i = 0; i < 6; i++) HIP_TRY(hipEventCreate(&ev[i]), "creating an event");
    double ph[5] = {0, 0, 0, 0, 0};
    bool ok = true;
    for (int r = -1; r < reps && ok; r++) { /* r = -1: warm-up */
        hipError_t e = hipMemcpyAsync(g->pf_x, g->pf_x0, n * g->H * 4, hipMemcpyDeviceToDevice, g->stream);
        if (e == hipSuccess) e = enqueue_prefill(g, (int)layer, (int)n, g->pf_x, g->pf, ev);
        if (e == hipSuccess) e = hipEventSynchronize(ev[5]);
        if (e != hipSuccess) { ok = fail_hip(err, err_len, "the timed prefill", e); break; }
        for (int i = 0; r >= 0 && i < 5; i++) {
            float ms = 0;
            if (hipEventElapsedTime(&ms, ev[i], ev[i + 1]) != hipSuccess) ms = 0;
            ph[i] += ms * 1000.0 / reps;
        }
    }
    for (int i = 0; i < 6; i++) (void)hipEventDestroy(ev[i]);
    if (!ok) return false;
    if (us_total) *us_total = ph[0] + ph[1] + ph[2] + ph[3] + ph[4];
    for (int i = 0; us_phase && i < 5; i++) us_phase[i] = ph[i];
    return true;
}

/* ---- the prefill without allocating ----
   The working buffers live in scratch, a file-scope device array of PREFILL_SCRATCH_BYTES that every GPU the
   library runs on holds until the process ends. Host code never passes the array's name to a kernel: on the host
   that name is a stand-in, not a device address. Its address on each device comes from hipGetSymbolAddress, taken
   once per device with that device current, and that pointer is what the kernels receive. Every call on one GPU
   shares the region, so calls that overlap on one GPU (two streams, two models on the same device) race. */
#define PREFILL_SCRATCH_BYTES ((size_t)128 << 20)
#define SCRATCH_DEVICES 64
static __device__ __align__(256) unsigned char scratch[PREFILL_SCRATCH_BYTES];
static std::mutex scratch_mu;
static char* scratch_at[SCRATCH_DEVICES];

static bool scratch_address(int device, char** out, char* err, size_t err_len) {
    if (device < 0 || device >= SCRATCH_DEVICES) return fail(err, err_len, "device %d: the static region serves devices 0..%d", device, SCRATCH_DEVICES - 1);
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_at[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return fail(err, err_len, "the static region's address on device %d: %s", device, hipGetErrorString(e));
        scratch_at[device] = static_cast<char*>(p);
    }
    *out = scratch_at[device];
    return true;
}

extern "C" bool vitna_hip_moe_prefill_noalloc(struct vitna_cuda_model* g, size_t layer, float* x, size_t n, int32_t* chosen, char* err,
                                              size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!prefill_check(g, layer, n, err, err_len)) return false;
    if (!x) return fail(err, err_len, "no rows");
    const size_t need = prefill_layout(g, n, nullptr, nullptr);
    if (need > PREFILL_SCRATCH_BYTES) {
        size_t lo = 0, hi = n; /* the most rows of this model the region holds */
        while (lo + 1 < hi) {
            const size_t mid = (lo + hi) / 2;
            (prefill_layout(g, mid, nullptr, nullptr) <= PREFILL_SCRATCH_BYTES ? lo : hi) = mid;
        }
        return fail(err, err_len, "%zu rows need %zu bytes of working memory; the static region holds %zu (%zu rows of this model)", n, need,
                    PREFILL_SCRATCH_BYTES, lo);
    }
    HIP_TRY(hipSetDevice(g->device), "selecting the model's device");
    char* base = nullptr;
    if (!scratch_address(g->device, &base, err, err_len)) return false;
    pf_bufs b;
    prefill_layout(g, n, base, &b);
    hipError_t e = enqueue_prefill(g, (int)layer, (int)n, x, b, nullptr);
    if (e == hipSuccess && chosen) e = launch_prefill_chosen(b.rt, (int)n, g->K, chosen, g->stream);
    g->last_step_mega = false;
    return check_launch(g, e, "the prefill", err, err_len);
}

/* The prefill's routing and output rows of the last timed or served prefill, to the host. */
extern "C" bool vitna_hip_prefill_rows(struct vitna_cuda_model* g, size_t n, float* x_in, float* x_out, int32_t* chosen, char* err,
                                       size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || n > g->pf_cap) return fail(err, err_len, "%zu rows: the last prefill held %zu", n, g ? g->pf_cap : 0);
    HIP_TRY(hipSetDevice(g->device), "selecting the model's device");
    if (x_in) HIP_TRY(hipMemcpyAsync(x_in, g->pf_x0, n * g->H * 4, hipMemcpyDeviceToHost, g->stream), "copying the input rows");
    if (x_out) HIP_TRY(hipMemcpyAsync(x_out, g->pf_x, n * g->H * 4, hipMemcpyDeviceToHost, g->stream), "copying the output rows");
    std::vector<route_out> rt(chosen ? n : 0);
    if (chosen) HIP_TRY(hipMemcpyAsync(rt.data(), g->pf.rt, n * sizeof(route_out), hipMemcpyDeviceToHost, g->stream), "copying the routing");
    if (!sync_stream(g, "copying the prefill", err, err_len)) return false;
    for (size_t i = 0; chosen && i < n; i++)
        for (int k = 0; k < g->K; k++) chosen[i * g->K + k] = rt[i].chosen[k];
    return true;
}

extern "C" bool vitna_hip_time_steps(struct vitna_cuda_model* g, size_t seq, int32_t token, size_t pos, int steps, double* ms_per_step,
                                     char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (steps < 1) return fail(err, err_len, "at least one step");
    bool mega;
    if (!use_step(g, &mega, err, err_len)) return false;
    /* every timed step decodes the same row, copied in once */
    if (!set_row(g, seq, token, pos, err, err_len)) return false;
    if (!mega && !ensure_graph(g, err, err_len)) return false;
    event_pair ev;
    HIP_TRY(ev.make(), "events");
    HIP_TRY(hipStreamSynchronize(g->stream), "before timing");
    HIP_TRY(hipEventRecord(ev.t0, g->stream), "events");
    for (int i = 0; i < steps; i++) {
        if (mega) {
            hipError_t e = launch_step_layers(g, 0, g->NL);
            if (e == hipSuccess) e = enqueue_head(g);
            if (!check_launch(g, e, "the step", err, err_len)) return false;
        } else {
            HIP_TRY(hipGraphLaunch(g->step_graph, g->stream), "launching the step");
        }
    }
    HIP_TRY(hipEventRecord(ev.t1, g->stream), "events");
    HIP_TRY(hipEventSynchronize(ev.t1), "timing the steps");
    if (mega && !step_check(g, err, err_len)) return false;
    g->last_step_mega = mega;
    float ms = 0;
    HIP_TRY(hipEventElapsedTime(&ms, ev.t0, ev.t1), "events");
    *ms_per_step = (double)ms / steps;
    return true;
}

extern "C" bool vitna_hip_time_ffn(struct vitna_cuda_model* g, int reps, double* us_per_layer, char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (reps < 1) return fail(err, err_len, "at least one repetition");
    bool mega = false;
    if (!g->attention && !use_step(g, &mega, err, err_len)) return false;
    if (mega) {
        /* the persistent step over every layer, without attention: one launch a repetition */
        event_pair ev;
        HIP_TRY(ev.make(), "events");
        for (int i = 0; i < 2; i++)
            if (!check_launch(g, launch_step_layers(g, 0, g->NL), "warming up", err, err_len)) return false;
        HIP_TRY(hipEventRecord(ev.t0, g->stream), "events");
        for (int i = 0; i < reps; i++)
            if (!check_launch(g, launch_step_layers(g, 0, g->NL), "timing the layers", err, err_len)) return false;
        HIP_TRY(hipEventRecord(ev.t1, g->stream), "events");
        HIP_TRY(hipEventSynchronize(ev.t1), "timing the layers");
        float ms = 0;
        HIP_TRY(hipEventElapsedTime(&ms, ev.t0, ev.t1), "events");
        if (!step_check(g, err, err_len)) return false;
        *us_per_layer = 1000.0 * ms / ((double)reps * g->NL);
        return true;
    }
    /* every layer's mixture-of-experts half on residual row 0, one after another, captured once */
    HIP_TRY(hipStreamSynchronize(g->stream), "before capturing the layers");
    HIP_TRY(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal), "capturing the layers");
    hipError_t e = hipSuccess;
    for (int l = 0; e == hipSuccess && l < g->NL; l++) {
        e = enqueue_route(g, l, g->rlogits, 1, g->x, g->xn, true);
        if (e == hipSuccess) e = enqueue_experts(g, l, g->rlogits, g->x, 1);
    }
    hipGraph_t graph = nullptr;
    const hipError_t e2 = hipStreamEndCapture(g->stream, &graph);
    if (e != hipSuccess) { if (graph) (void)hipGraphDestroy(graph); return check_launch(g, e, "capturing the layers", err, err_len); }
    HIP_TRY(e2, "ending the capture of the layers");
    hipGraphExec_t exec = nullptr;
    const hipError_t e3 = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HIP_TRY(e3, "instantiating the layers' graph");
    hipEvent_t t0 = nullptr, t1 = nullptr;
    bool ok = hipGraphLaunch(exec, g->stream) == hipSuccess && hipGraphLaunch(exec, g->stream) == hipSuccess &&
              hipEventCreate(&t0) == hipSuccess && hipEventCreate(&t1) == hipSuccess && hipEventRecord(t0, g->stream) == hipSuccess;
    for (int i = 0; ok && i < reps; i++) ok = hipGraphLaunch(exec, g->stream) == hipSuccess;
    float ms = 0;
    ok = ok && hipEventRecord(t1, g->stream) == hipSuccess && hipEventSynchronize(t1) == hipSuccess && hipEventElapsedTime(&ms, t0, t1) == hipSuccess;
    if (t0) (void)hipEventDestroy(t0);
    if (t1) (void)hipEventDestroy(t1);
    (void)hipGraphExecDestroy(exec);
    if (!ok) return fail(err, err_len, "timing the layers failed");
    *us_per_layer = 1000.0 * ms / ((double)reps * g->NL);
    return true;
}

extern "C" bool vitna_hip_route_check(const float* logits, int n_experts, int k, bool renormalize, int32_t* chosen, int32_t* ids,
                                      float* weights, char* err, size_t err_len) {
    if (!logits || n_experts < 1 || n_experts > ROUTE_E_MAX || n_experts % 4 || k < 1 || k > ROUTE_K_MAX || k > n_experts)
        return fail(err, err_len, "%d experts, %d a token: 1 to %d experts, a multiple of 4, and 1 to %d a token", n_experts, k,
                    ROUTE_E_MAX, ROUTE_K_MAX);
    float* dl = nullptr;
    route_out* dro = nullptr;
    bool ok = hipMalloc(&dl, n_experts * 4) == hipSuccess && hipMalloc(&dro, sizeof(route_out)) == hipSuccess;
    route_out r;
    ok = ok && hipMemcpy(dl, logits, n_experts * 4, hipMemcpyHostToDevice) == hipSuccess &&
         launch_route_check(dl, n_experts, k, renormalize ? 1 : 0, dro, 0) == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
         hipMemcpy(&r, dro, sizeof(r), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(dl);
    (void)hipFree(dro);
    if (!ok) return fail(err, err_len, "the device routing failed");
    for (int i = 0; i < k; i++) {
        if (chosen) chosen[i] = r.chosen[i];
        if (ids) ids[i] = r.ids[i];
        if (weights) weights[i] = r.weights[i];
    }
    return true;
}

/* The reference's host routing (engine/src/model.c:626-703, top_k and route), for callers of the layer-at-a-time ABI
   that have none of their own: K passes of argmax (strict >, so the first of equals; a NaN where a pass starts is
   kept), the chosen sorted by id, softmax in float32 (the max as scanned, the sum of expf(l - max) in index
   order), renormalized over the chosen with their total summed largest first. */
extern "C" bool vitna_hip_host_route(const float* logits, int n_experts, int k, bool renormalize, int32_t* chosen, int32_t* order,
                                     float* weights, char* err, size_t err_len) {
    if (!logits || n_experts < 1 || k < 1 || k > ROUTE_K_MAX || k > n_experts)
        return fail(err, err_len, "%d experts, %d a token: 1 to %d a token, no more than the experts", n_experts, k, ROUTE_K_MAX);
    int32_t ch[ROUTE_K_MAX], ord[ROUTE_K_MAX];
    float w[ROUTE_K_MAX];
    for (int i = 0; i < k; i++) {
        int best = -1;
        for (int e = 0; e < n_experts; e++) {
            bool taken = false;
            for (int j = 0; j < i; j++) taken |= ch[j] == e;
            if (!taken && (best < 0 || logits[e] > logits[best])) best = e;
        }
        ch[i] = best;
    }
    for (int i = 0; i < k; i++) ord[i] = ch[i];
    std::sort(ord, ord + k);
    float mx = logits[0];
    for (int e = 1; e < n_experts; e++)
        if (logits[e] > mx) mx = logits[e];
    float sum = 0.0f;
    for (int e = 0; e < n_experts; e++) sum += expf(logits[e] - mx);
    for (int i = 0; i < k; i++) w[i] = expf(logits[ord[i]] - mx) / sum;
    if (renormalize) {
        float share[ROUTE_K_MAX];
        for (int i = 0; i < k; i++) share[i] = w[i];
        std::stable_sort(share, share + k, [](float a, float b) { return a > b; });
        float total = 0.0f;
        for (int i = 0; i < k; i++) total += share[i];
        for (int i = 0; i < k; i++) w[i] /= total;
    }
    for (int i = 0; i < k; i++) {
        if (chosen) chosen[i] = ch[i];
        if (order) order[i] = ord[i];
        if (weights) weights[i] = w[i];
    }
    return true;
}

extern "C" bool vitna_hip_copy_probe(size_t bytes, int reps, double* avg_us, char* err, size_t err_len) {
    if (bytes % 16 || bytes == 0 || reps < 1) return fail(err, err_len, "a positive multiple of 16 bytes, at least one repetition");
    void *a = nullptr, *b = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    bool ok = hipMalloc(&a, bytes) == hipSuccess && hipMalloc(&b, bytes) == hipSuccess && hipMemset(a, 0, bytes) == hipSuccess &&
              hipEventCreate(&t0) == hipSuccess && hipEventCreate(&t1) == hipSuccess && launch_copy_probe(a, b, bytes, 0) == hipSuccess &&
              hipEventRecord(t0, 0) == hipSuccess;
    for (int i = 0; ok && i < reps; i++) ok = launch_copy_probe(a, b, bytes, 0) == hipSuccess;
    float ms = 0;
    ok = ok && hipEventRecord(t1, 0) == hipSuccess && hipEventSynchronize(t1) == hipSuccess && hipEventElapsedTime(&ms, t0, t1) == hipSuccess;
    if (t0) (void)hipEventDestroy(t0);
    if (t1) (void)hipEventDestroy(t1);
    (void)hipFree(a);
    (void)hipFree(b);
    if (!ok) return fail(err, err_len, "the copy probe failed");
    if (avg_us) *avg_us = 1000.0 * ms / reps;
    return true;
}

extern "C" bool vitna_hip_mfma_probe(int blocks, int iters, int reps, double* tflops, char* err, size_t err_len) {
    if (blocks < 1 || iters < 1 || reps < 1) return fail(err, err_len, "positive blocks, iterations and repetitions");
    float* out = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    bool ok = hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) == hipSuccess && hipEventCreate(&t0) == hipSuccess &&
              hipEventCreate(&t1) == hipSuccess && launch_mfma_probe(out, blocks, iters, 0) == hipSuccess &&
              hipEventRecord(t0, 0) == hipSuccess;
    for (int i = 0; ok && i < reps; i++) ok = launch_mfma_probe(out, blocks, iters, 0) == hipSuccess;
    float ms = 0;
    ok = ok && hipEventRecord(t1, 0) == hipSuccess && hipEventSynchronize(t1) == hipSuccess && hipEventElapsedTime(&ms, t0, t1) == hipSuccess;
    if (t0) (void)hipEventDestroy(t0);
    if (t1) (void)hipEventDestroy(t1);
    (void)hipFree(out);
    if (!ok) return fail(err, err_len, "the matrix-core probe failed");
    if (tflops) *tflops = mfma_probe_flops(blocks, iters) * reps / (ms * 1e-3) / 1e12;
    return true;
}

/* ---- several rows a layer at a time (model_cuda.h:124-161) -------------- */

extern "C" size_t vitna_cuda_moe_rows_max(const struct vitna_cuda_model* g) { return g ? ROWS_MAX : 0; }

/* Several rows times up to three matrices: from SKINNY_MIN rows on, on the matrix cores (kernels_skinny.hip),
   the rows split into bf16 hi and lo first; below, the multi-row GEMV. */
#define SKINNY_MIN 4
static bool multi_quant(const gemv_multi_args& m) {
    bool quant = true;
    for (int i = 0; i < m.nm; i++) quant &= m.w[i].dtype != VITNA_DTYPE_F32;
    return quant;
}
/* Whether launch_skinny takes its exact-integer path for m (the operand images then replace x's split). */
static bool multi_exact(const gemv_multi_args& m) {
    if (m.n < SKINNY_MIN || !multi_quant(m) || m.w[0].cols % 256 || m.xstride % 4 || (uintptr_t)m.x % 16) return false;
    for (int i = 0; i < m.nm; i++)
        if (!m.w[i].tiled || m.w[i].cols != m.w[0].cols) return false;
    return true;
}
static img_out model_img(const vitna_cuda_model* g) {
    return img_out{(u32x4*)g->sk_img[0], (u32x4*)g->sk_img[1], (uint16_t*)g->sk_img[2], (uint16_t*)g->sk_img[3]};
}

/* imaged: the producer of m.x wrote its operand images already (when multi_exact(m)). */
static hipError_t enqueue_multi(vitna_cuda_model* g, const gemv_multi_args& m, bool imaged) {
    if (m.n < SKINNY_MIN || !multi_quant(m)) return launch_gemv_multi(m, g->stream);
    const int K = m.w[0].cols;
    const bool exact = multi_exact(m);
    hipError_t e = hipSuccess;
    if (!exact || !imaged) e = launch_split_rows(m.x, m.n, K, m.xstride, g->sk_xh, g->sk_xl, exact ? g->sk_img : nullptr, g->stream);
    if (e != hipSuccess) return e;
    skinny_args a;
    memset(&a, 0, sizeof(a));
    for (int i = 0; i < m.nm; i++) { a.w[i] = m.w[i]; a.y[i] = m.y[i]; }
    a.nm = m.nm; a.xh = g->sk_xh; a.xl = g->sk_xl; a.n = m.n; a.add = m.add;
    if (exact) { a.img[0] = g->sk_img[0]; a.img[1] = g->sk_img[1]; a.s32 = g->sk_img[2]; a.s16 = g->sk_img[3]; }
    a.part = g->sk_part; a.cnt = g->sk_cnt; a.part_cap = g->sk_part_cap; a.cnt_cap = g->sk_cnt_cap;
    return launch_skinny(a, g->stream);
}

/* ypart: the previous layer's experts' outputs still to be added onto the residual rows (or null), added here
   in slot order by the kernel that normalizes the rows and writes the q/k/v operands. */
static hipError_t enqueue_rows_attention(vitna_cuda_model* g, int layer, int n, const float* ypart) {
    const dlayer& d = g->L[layer];
    gemv_multi_args ga;
    memset(&ga, 0, sizeof(ga));
    ga.w[0] = d.q; ga.w[1] = d.k; ga.w[2] = d.v;
    ga.y[0] = g->q; ga.y[1] = g->k; ga.y[2] = g->v;
    ga.nm = 3; ga.x = g->xn; ga.n = n; ga.xstride = g->H;
    const bool img = multi_exact(ga);
    hipError_t e = launch_residual_norm(g->x, ypart, g->K, d.attn_norm, g->xn, n, g->H, g->eps,
                                        img ? model_img(g) : img_out{nullptr, nullptr, nullptr, nullptr}, g->stream);
    if (e != hipSuccess) return e;
    e = enqueue_multi(g, ga, img);
    if (e != hipSuccess) return e;
    attn_args a;
    memset(&a, 0, sizeof(a));
    a.q_raw = g->q; a.k_raw = g->k; a.v_raw = g->v;
    a.q_norm = d.q_norm; a.k_norm = d.k_norm;
    a.cos_tab = g->cos_tab; a.sin_tab = g->sin_tab;
    a.k_cache = g->k_cache + (size_t)layer * g->layer_kv;
    a.v_cache = g->v_cache + (size_t)layer * g->layer_kv;
    a.seq_stride = (size_t)g->NL * g->layer_kv;
    a.rows = g->rows_dev;
    a.n_rows = n;
    a.partial = g->partial;
    a.att = g->att;
    a.n_heads = g->nh; a.n_kv = g->nkv; a.hd = g->hd; a.ctx = g->ctx; a.splits_max = g->splits_max;
    a.splits_grid = g->splits_grid;
    a.eps = g->eps;
    /* several rows: the score and value products on the matrix cores */
    a.mma = n > 1 ? 1 : 0;
    if (g->rows_shared_seq) {
        /* rows of one sequence see each other's keys: all of them stored before any attention reads */
        a.q_out = g->qp;
        e = launch_attention_prepare(a, g->stream);
        if (e != hipSuccess) return e;
        a.q_raw = g->qp;
        a.prepared = 1;
    }
    gemv_multi_args go;
    memset(&go, 0, sizeof(go));
    go.w[0] = d.o; go.y[0] = g->x; go.nm = 1; go.x = g->att; go.n = n; go.xstride = g->nh * g->hd; go.add = 1;
    /* the merge writes the o-projection's operands too */
    const bool oimg = multi_exact(go);
    if (g->rows_one_seq && n > 1 && attention_run_fits(a)) {
        /* a pass of one sequence (a prompt's chunk): tiles of rows, each chunk read once a tile, att written by the
           attention itself; the o-projection's operands split from it */
        e = launch_attention_flash(a, g->stream);
        return e == hipSuccess ? enqueue_multi(g, go, false) : e;
    }
    e = launch_attention(a, g->stream);
    if (oimg) a.img = model_img(g);
    if (e == hipSuccess) e = launch_attention_merge(a, g->stream);
    if (e != hipSuccess) return e;
    return enqueue_multi(g, go, oimg);
}

/* --precision fast (model_cuda.cu:5002-5022): a pass of fast_rows rows or more of a gpu_fast model runs its experts as
   a grouped GEMM on the matrix cores. Its sums run in another order, and its inputs in bf16, so its outputs are close
   to the exact kernels' but not their bits. */
static bool rows_fast(const vitna_cuda_model* g, int n) { return g->fast && (size_t)n >= g->fast_rows; }

/* The experts of a fast pass of n rows as rt[0..n) routes them: the normalized rows (g->xn) rounded to bf16, the
   (row, slot) pairs grouped by expert, the prefill's grouped GEMM (gate/up with SwiGLU, then down times the
   weight), each row's K parts added onto its residual row in slot order. The working buffers are the prefill's,
   reserved for n rows beforehand (prefill_reserve). */
static hipError_t enqueue_fast_experts(vitna_cuda_model* g, int layer, int n, const route_out* rt) {
    const dlayer& d = g->L[layer];
    const pf_bufs& b = g->pf;
    hipStream_t s = g->stream;
    if ((size_t)n > g->pf_cap) return hipErrorInvalidValue;
    hipError_t e = launch_prefill_bf16(g->xn, b.xb, (size_t)n * g->H, s);
    if (e == hipSuccess) e = launch_group(rt, n, g->E, g->K, n, b.count, b.pairs, s);
    if (e == hipSuccess) e = launch_prefill_plan(b.count, g->E, b.off, b.tiles, b.ntiles, s);
    prefill_args a;
    a.gate = d.gate; a.up = d.up; a.down = d.down;
    a.xb = b.xb; a.rt = rt; a.count = b.count; a.pairs = b.pairs; a.off = b.off;
    a.tiles = b.tiles; a.n_tiles = b.ntiles; a.act = b.act; a.ypart = b.ypart;
    a.E = g->E; a.K = g->K; a.cap = n; a.n = n;
    if (e == hipSuccess) e = launch_prefill_gemm(a, true, s);
    if (e == hipSuccess) e = launch_prefill_gemm(a, false, s);
    if (e == hipSuccess) e = launch_prefill_sum(b.ypart, g->x, n, g->K, g->H, s);
    return e;
}

/* The grouped experts of the pass's n rows, routed as g->rt[0..n) holds it, added onto the residual rows (or,
   defer_sum, left in g->ypart for the next kernel that reads the rows to add). */
static hipError_t enqueue_rows_experts(vitna_cuda_model* g, int layer, int n, bool defer_sum, bool split_done = false,
                                       const route_out* rt = nullptr) {
    const dlayer& d = g->L[layer];
    if (!rt) rt = g->rt;
    hipError_t e = launch_group(rt, n, g->E, g->K, ROWS_MAX, g->grp_count, g->grp_pairs, g->stream);
    if (e != hipSuccess) return e;
    if (n >= GSX_ROWS && d.sx_gate) {
        /* a crowded pass: tiles of 32 pairs of one expert */
        gsx_args x{};
        x.gate = d.gate; x.gate.tiled = d.sx_gate;
        x.up = d.up; x.up.tiled = d.sx_up;
        x.down = d.down; x.down.tiled = d.sx_down;
        x.xn = g->xn; x.rt = rt; x.count = g->grp_count; x.pairs = g->grp_pairs;
        x.E = g->E; x.K = g->K; x.cap = ROWS_MAX; x.n = n;
        x.toff = g->gsx_toff; x.te = g->gsx_te; x.max_tiles = gsx_max_tiles(ROWS_MAX, g->K, g->E);
        x.img_in = g->gsx_img_in; x.img_act = g->gsx_img_act; x.s32 = g->gsx_s32; x.s16 = g->gsx_s16;
        x.act = g->gsx_act; x.ypart = g->ypart;
        e = launch_gsx(x, g->stream);
        if (e == hipSuccess && !defer_sum) e = launch_reduce_rows(g->ypart, g->x, n, g->K, g->H, g->stream);
        return e;
    }
    /* every expert set check_shapes accepts (quantized, widths multiples of 256) fits the matrix-core kernels */
    if (!gmma_fits(d.gate, d.up, d.down)) return hipErrorInvalidValue;
    if (!split_done) e = launch_gmma_split(g->xn, n, g->H, g->H, gmma_gran(d.gate.dtype), g->gm_xs, g->gm_xsum, g->stream);
    gmma_args m{};
    m.gate = d.gate; m.up = d.up; m.down = d.down;
    m.xs = g->gm_xs; m.xsum = g->gm_xsum; m.as = g->gm_as; m.asum = g->gm_asum; m.rt = rt; m.count = g->grp_count; m.pairs = g->grp_pairs;
    m.E = g->E; m.K = g->K; m.cap = ROWS_MAX; m.n = n; m.ypart = g->ypart;
    if (e == hipSuccess) e = launch_gmma_in(m, g->stream);
    if (e == hipSuccess) e = launch_gmma_down(m, g->stream);
    if (e == hipSuccess && !defer_sum) e = launch_reduce_rows(g->ypart, g->x, n, g->K, g->H, g->stream);
    return e;
}

/* The head's rows: every row's, none (the final norm only, so the residual rows hold the pass's sums), or the one
   row a prompt's last chunk asks for (model.c:1011), the head then a single row's GEMM. */
#define HEAD_ALL (-1)
#define HEAD_NONE (-2)

static hipError_t enqueue_rows_head(vitna_cuda_model* g, int n, const float* ypart, int head = HEAD_ALL) {
    gemv_multi_args gh;
    memset(&gh, 0, sizeof(gh));
    gh.w[0] = g->head; gh.y[0] = g->vocab; gh.nm = 1; gh.x = g->xn; gh.n = n; gh.xstride = g->H;
    if (head >= 0) {
        gh.x = g->xn + (size_t)head * g->H;
        gh.y[0] = g->vocab + (size_t)head * g->V;
        gh.n = 1;
    }
    const bool img = head == HEAD_ALL && multi_exact(gh);
    hipError_t e = launch_residual_norm(g->x, ypart, g->K, g->final_norm, g->xn, n, g->H, g->eps,
                                        img ? model_img(g) : img_out{nullptr, nullptr, nullptr, nullptr}, g->stream);
    if (e != hipSuccess || head == HEAD_NONE) return e;
    return enqueue_multi(g, gh, img);
}

/* The head's rows a call's logits pointers ask for: none, the one (passes past the exact-rows limit, whose logits
   are not a step's bits anyway), or every row. */
static int head_rows(const vitna_cuda_model* g, size_t n, float* const* logits) {
    int asked = 0, last = -1;
    for (size_t i = 0; logits && i < n; i++)
        if (logits[i]) { asked++; last = (int)i; }
    if (!asked) return HEAD_NONE;
    return asked == 1 && n > (size_t)EXACT_ROWS ? last : HEAD_ALL;
}

/* ---- passes of few rows, each row with a single token's kernels (EXACT_ROWS) ---- */

static bool rows_exact(const vitna_cuda_model* g, int n) { return n <= g->exact_rows && !rows_fast(g, n); }

/* Layer's attention for the pass's n rows as enqueue_attention runs it for one: the q/k/v GEMV with its norm, the
   attention (rows of one sequence: each row's key and value stored first, with the same arithmetic), the merged
   o-projection when the layer takes it (its parts then folded into the rows, as the single token's router and
   experts add them) or else the merge and the o-projection GEMV. */
static hipError_t enqueue_exact_attention(vitna_cuda_model* g, int layer, int n) {
    const dlayer& d = g->L[layer];
    const int qd = g->nh * g->hd, kd = g->nkv * g->hd;
    gemv_args ga;
    memset(&ga, 0, sizeof(ga));
    ga.w[0] = d.q; ga.w[1] = d.k; ga.w[2] = d.v;
    ga.y[0] = g->q; ga.y[1] = g->k; ga.y[2] = g->v;
    ga.n = 3;
    ga.x = g->x;
    ga.norm_w = d.attn_norm;
    ga.eps = g->eps;
    ga.rows = n; ga.xstride = g->H; ga.ystride[0] = qd; ga.ystride[1] = kd; ga.ystride[2] = kd;
    hipError_t e = launch_gemv(ga, g->stream);
    if (e != hipSuccess) return e;
    attn_args a;
    memset(&a, 0, sizeof(a));
    a.q_raw = g->q; a.k_raw = g->k; a.v_raw = g->v;
    a.q_norm = d.q_norm; a.k_norm = d.k_norm;
    a.cos_tab = g->cos_tab; a.sin_tab = g->sin_tab;
    a.k_cache = g->k_cache + (size_t)layer * g->layer_kv;
    a.v_cache = g->v_cache + (size_t)layer * g->layer_kv;
    a.seq_stride = (size_t)g->NL * g->layer_kv;
    a.rows = g->rows_dev;
    a.n_rows = n;
    a.partial = g->partial;
    a.att = g->att;
    a.n_heads = g->nh; a.n_kv = g->nkv; a.hd = g->hd; a.ctx = g->ctx; a.splits_max = g->splits_max;
    a.splits_grid = g->splits_grid;
    a.eps = g->eps;
    a.mma = 1;
    if (g->rows_shared_seq) {
        a.q_out = g->qp;
        e = launch_attention_prepare(a, g->stream);
        if (e != hipSuccess) return e;
        a.q_raw = g->qp;
        a.prepared = 1;
    }
    e = launch_attention(a, g->stream);
    if (e != hipSuccess) return e;
    if (attention_oproj_fits(a, d.o)) {
        const int np = g->nh / ATTN_OPROJ_HEADS;
        e = launch_attention_oproj(a, d.o, g->parts, g->stream);
        return e == hipSuccess ? launch_attn_fold(g->x, g->parts, np, g->H, g->stream, n) : e;
    }
    e = launch_attention_merge(a, g->stream);
    if (e != hipSuccess) return e;
    gemv_args go;
    memset(&go, 0, sizeof(go));
    go.w[0] = d.o; go.y[0] = g->x; go.n = 1; go.x = g->att; go.add = 1;
    go.rows = n; go.xstride = qd; go.ystride[0] = g->H;
    return launch_gemv(go, g->stream);
}

/* The experts of the pass's rows at .. at + n - 1 as rt routes them (by slot on a cached model), each row as
   enqueue_experts runs one token's, added onto its residual row. */
static hipError_t enqueue_exact_experts(vitna_cuda_model* g, int layer, int n, int at = 0) {
    const dlayer& d = g->L[layer];
    const size_t act_row = (size_t)g->K * g->I;
    experts_in_args ai;
    ai.gate = d.gate; ai.up = d.up; ai.xn = g->xn + (size_t)at * g->H; ai.rt = g->rt + at; ai.logits = nullptr; ai.E = g->E;
    ai.renorm = g->renorm; ai.act = g->act + at * act_row; ai.K = g->K;
    hipError_t e = launch_experts_in(ai, g->stream, n);
    if (e != hipSuccess) return e;
    experts_down_args ad;
    ad.down = d.down; ad.act = g->act + at * act_row; ad.rt = g->rt + at; ad.y = g->x + (size_t)at * g->H; ad.K = g->K; ad.add = 1;
    ad.parts = nullptr; ad.n_parts = 0;
    return launch_experts_down(ad, g->stream, n);
}

/* The head of the pass's n rows as enqueue_head runs one row's. */
static hipError_t enqueue_exact_head(vitna_cuda_model* g, int n) {
    gemv_args gh;
    memset(&gh, 0, sizeof(gh));
    gh.w[0] = g->head;
    gh.y[0] = g->vocab;
    gh.n = 1;
    gh.x = g->x;
    gh.norm_w = g->final_norm;
    gh.eps = g->eps;
    gh.rows = n; gh.xstride = g->H; gh.ystride[0] = g->V;
    return launch_gemv(gh, g->stream);
}

extern "C" bool vitna_hip_set_exact_rows(struct vitna_cuda_model* g, size_t n, char* err, size_t err_len) {
    if (!g) return fail(err, err_len, "no model");
    if (n > EXACT_ROWS) return fail(err, err_len, "%zu rows: at most %d take the single-token kernels", n, EXACT_ROWS);
    g->exact_rows = (int)n;
    return true;
}

/* The pass's rows to the device, checked as a step checks its token (model.c:1190-1200). */
static bool set_rows(vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t n, char* err, size_t err_len) {
    if (n < 1 || n > ROWS_MAX) return fail(err, err_len, "%zu rows: 1 to %d a pass", n, ROWS_MAX);
    bool shared = false;
    for (size_t i = 0; i < n; i++) {
        const vitna_cuda_row_t r = rows[i];
        if (r.seq < 0 || r.seq >= g->seqs) return fail(err, err_len, "row %zu: sequence %d, the cache holds %d", i, r.seq, g->seqs);
        if (r.pos < 0 || r.pos >= g->ctx) return fail(err, err_len, "row %zu: position %d, the cache holds %d", i, r.pos, g->ctx);
        if (r.token < 0 || r.token >= g->V) return fail(err, err_len, "row %zu: token %d outside the vocabulary of %d", i, r.token, g->V);
        for (size_t j = 0; j < i; j++) shared |= rows[j].seq == r.seq;
    }
    HIP_TRY(hipEventSynchronize(g->rows_copied), "waiting for the previous row copy");
    g->row_set = false;
    int max_pos = 0;
    for (size_t i = 0; i < n; i++) {
        g->rows_host[i] = {rows[i].token, rows[i].pos, rows[i].seq};
        max_pos = std::max(max_pos, (int)rows[i].pos);
    }
    g->splits_grid = splits_bucket(g, max_pos);
    HIP_TRY(hipMemcpyAsync(g->rows_dev, g->rows_host, n * sizeof(row_rec), hipMemcpyHostToDevice, g->stream), "copying the rows");
    HIP_TRY(hipEventRecord(g->rows_copied, g->stream), "recording the row copy");
    g->rows_n = (int)n;
    g->rows_one_seq = true;
    for (size_t i = 1; i < n; i++) g->rows_one_seq &= rows[i].seq == rows[0].seq;
    g->pass_exact = false; /* vitna_cuda_moe_rows_route decides at layer 0 */
    g->parts_n = 0; /* a pass of rows owns x's rows: no one row's attention parts are pending any more */
    g->rows_shared_seq = shared;
    return true;
}

extern "C" bool vitna_cuda_moe_rows_route(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t n, size_t layer, float* logits,
                                          float* next, char* err, size_t err_len) {
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!ensure_tiled(g, err, err_len)) return false;
    if (!g->attention) return fail(err, err_len, "this model has no attention");
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    g->last_step_mega = false;
    if (layer == 0) {
        if (!set_rows(g, rows, n, err, err_len)) return false;
        g->pass_exact = rows_exact(g, (int)n);
        if (!check_launch(g, launch_embed_rows(g->embed, g->rows_dev, (int)n, g->x, g->stream), "the embeddings", err, err_len)) return false;
    } else if (n != (size_t)g->rows_n) {
        return fail(err, err_len, "%zu rows at layer %zu; the pass took %d at layer 0", n, layer, g->rows_n);
    }
    hipError_t e = g->pass_exact ? enqueue_exact_attention(g, (int)layer, (int)n) : enqueue_rows_attention(g, (int)layer, (int)n, nullptr);
    if (e == hipSuccess) e = enqueue_route(g, (int)layer, g->rlogits, (int)n, g->x, g->xn, false);
    const bool nx = next && layer + 1 < (size_t)g->NL;
    if (e == hipSuccess && nx) {
        const dlayer& d = g->L[layer + 1];
        route_args r;
        memset(&r, 0, sizeof(r));
        r.x = g->x; r.norm_w = d.mlp_norm; r.router = d.router; r.logits = g->rlogits + (size_t)ROWS_MAX * g->E;
        r.H = g->H; r.E = g->E; r.n_rows = (int)n; r.eps = g->eps;
        e = launch_route(r, g->stream);
    }
    if (!check_launch(g, e, "the rows up to their router", err, err_len)) return false;
    const size_t bytes = n * g->E * 4;
    HIP_TRY(hipMemcpyAsync(logits, g->rlogits, bytes, hipMemcpyDeviceToHost, g->stream), "copying the router's logits");
    if (nx) HIP_TRY(hipMemcpyAsync(next, g->rlogits + (size_t)ROWS_MAX * g->E, bytes, hipMemcpyDeviceToHost, g->stream), "copying the guess");
    HIP_TRY(hipStreamSynchronize(g->stream), "running the rows up to their router");
    return true;
}

/* The slots' tiled copies for layer's expert shapes: the areas made on the first pass of rows (each the largest
   any layer needs for every slot), and every copy forgotten when the layer's tile strides differ from those the
   copies were made with (the copies sit at slot * stride). */
static bool slot_tiles_for(vitna_cuda_model* g, const dlayer& d, char* err, size_t err_len) {
    const expert_cache& c = g->ec;
    if (!g->st_area[0]) {
        for (int p = 0; p < 3; p++) {
            size_t most = 0;
            for (int l = 0; l < g->NL; l++) {
                const qmat& m = p == 0 ? g->L[l].gate : p == 1 ? g->L[l].up : g->L[l].down;
                most = std::max(most, gmma_tiled_bytes(m, 1));
            }
            if (!dalloc(g, &g->st_area[p], most * c.n_slots, "the expert slots' tiled copy", err, err_len)) return false;
        }
        g->st_place.assign(c.n_slots, -1);
    }
    const size_t st[3] = {gmma_tiled_bytes(d.gate, 1), gmma_tiled_bytes(d.up, 1), gmma_tiled_bytes(d.down, 1)};
    if (st[0] != g->st_stride[0] || st[1] != g->st_stride[1] || st[2] != g->st_stride[2]) {
        for (int p = 0; p < 3; p++) g->st_stride[p] = st[p];
        std::fill(g->st_place.begin(), g->st_place.end(), -1);
    }
    return true;
}

/* A pass of rows through the expert cache (model_cuda.cu:5134-5386): the experts the rows want, in order of expert,
   in waves of at most n_slots - k; a wave's slots held, those lacking copied in, their tiled copies made where the
   slot's differs, then the grouped experts over the wave's (row, expert) pairs with the slots for experts. Each row's
   K outputs are summed once after the last wave, in the order of ids, as a resident pass sums them. Then the guess. */
static bool cached_rows_experts(vitna_cuda_model* g, int layer, int n, const int32_t* ids, const float* weights, int k,
                                const int32_t* guess, char* err, size_t err_len) {
    expert_cache& c = g->ec;
    const dlayer& d = g->L[layer];
    if (k != g->K) return fail(err, err_len, "%d experts given; the model routes to %d", k, g->K);
    std::vector<int32_t> cnt(g->E, 0);
    for (int t = 0; t < n; t++)
        for (int i = 0; i < k; i++) {
            const int32_t e = ids[(size_t)t * k + i];
            if (e < 0 || e >= g->E) return fail(err, err_len, "expert %d is outside the layer's %d", e, g->E);
            for (int j = 0; j < i; j++)
                if (ids[(size_t)t * k + j] == e) return fail(err, err_len, "expert %d is named twice", e);
            if (guess && (guess[(size_t)t * k + i] < 0 || guess[(size_t)t * k + i] >= g->E))
                return fail(err, err_len, "guessed expert %d is outside the layer's %d", guess[(size_t)t * k + i], g->E);
            cnt[e]++;
        }
    std::vector<int32_t> want, slot_of(g->E, -1);
    for (int x = 0; x < g->E; x++)
        if (cnt[x]) want.push_back(x);
    const int W = c.n_slots - c.K;
    if (g->pass_exact) {
        /* each row as a single token's step, from the slots: the rows in groups of consecutive rows whose experts
           take one wave of the rule (every row's k experts fit one: W >= k), each group a pass of the cache, so
           that the bits are those of every expert resident whatever the cache's size. A pass whose experts fit one
           wave is one group: the rule's own pass. */
        bool ok = true;
        std::vector<int32_t> gcnt(g->E), slots((size_t)n * k);
        for (int t0 = 0; ok && t0 < n;) {
            std::fill(gcnt.begin(), gcnt.end(), 0);
            int t1 = t0, distinct = 0;
            for (; t1 < n; t1++) {
                int fresh = 0;
                for (int i = 0; i < k; i++) fresh += gcnt[ids[(size_t)t1 * k + i]] == 0;
                if (t1 > t0 && distinct + fresh > W) break;
                distinct += fresh;
                for (int i = 0; i < k; i++) gcnt[ids[(size_t)t1 * k + i]]++;
            }
            std::vector<int32_t> gwant;
            for (int x = 0; x < g->E; x++)
                if (gcnt[x]) gwant.push_back(x);
            ec_rows_count(c, layer, gcnt.data());
            ok = ec_rows_wave(c, layer, gwant.data(), (int)gwant.size(), gcnt.data(), g->stream, slot_of.data(), err, err_len);
            for (size_t i = 0; ok && i < gwant.size(); i++) {
                const ec_slot& sl = c.slots[slot_of[gwant[i]]];
                if (sl.copying && hipStreamWaitEvent(g->stream, sl.landed, 0) != hipSuccess) ok = fail(err, err_len, "waiting for an expert's copy");
            }
            for (size_t i = (size_t)t0 * k; i < (size_t)t1 * k; i++) slots[i] = slot_of[ids[i]];
            ok = ok && put_routing(g, t1 - t0, ids + (size_t)t0 * k, weights + (size_t)t0 * k, k, err, err_len, slots.data() + (size_t)t0 * k, t0) &&
                 check_launch(g, enqueue_exact_experts(g, layer, t1 - t0, t0), "the rows' experts", err, err_len);
            /* the holds released whatever happened; the pass's guess after its last group's kernels */
            const bool last = t1 == n;
            const bool fin = ec_rows_finish(c, layer, ok && last ? guess : nullptr, last ? n : t1 - t0, k, err, err_len);
            ok = ok && fin;
            t0 = t1;
        }
        return ok;
    }
    if (!gmma_fits(d.gate, d.up, d.down)) return fail(err, err_len, "layer %d's experts do not fit the grouped kernels", layer);
    if (!slot_tiles_for(g, d, err, err_len)) return false;
    ec_rows_count(c, layer, cnt.data());
    gmma_args m{};
    m.gate = d.gate; m.up = d.up; m.down = d.down;
    m.gate.tiled = g->st_area[0]; m.up.tiled = g->st_area[1]; m.down.tiled = g->st_area[2];
    m.xs = g->gm_xs; m.xsum = g->gm_xsum; m.as = g->gm_as; m.asum = g->gm_asum; m.rt = g->rt; m.count = g->grp_count; m.pairs = g->grp_pairs;
    m.E = c.n_slots; m.K = g->K; m.cap = ROWS_MAX; m.n = n; m.ypart = g->ypart;
    hipError_t e = launch_gmma_split(g->xn, n, g->H, g->H, gmma_gran(d.gate.dtype), g->gm_xs, g->gm_xsum, g->stream);
    bool ok = check_launch(g, e, "the rows' split", err, err_len);
    std::vector<uint8_t> in_wave(g->E, 0);
    for (size_t w0 = 0; ok && w0 < want.size(); w0 += W) {
        const int nw = (int)std::min<size_t>(W, want.size() - w0);
        ok = ec_rows_wave(c, layer, want.data() + w0, nw, cnt.data(), g->stream, slot_of.data(), err, err_len);
        std::fill(in_wave.begin(), in_wave.end(), 0);
        for (int i = 0; ok && i < nw; i++) {
            const int x = want[w0 + i], s = slot_of[x];
            in_wave[x] = 1;
            const ec_slot& sl = c.slots[s];
            if (sl.copying && hipStreamWaitEvent(g->stream, sl.landed, 0) != hipSuccess) ok = fail(err, err_len, "waiting for an expert's copy");
            if (!ok || g->st_place[s] == sl.place) continue;
            /* the slot's tiled copy, on the compute stream: after the kernels that read the copy it replaces */
            const qmat* src[3] = {&d.gate, &d.up, &d.down};
            for (int p = 0; ok && p < 3; p++) {
                qmat one = *src[p];
                for (int q = 0; q < 4; q++)
                    if (one.p[q]) one.p[q] += (size_t)s * one.estride[q];
                e = launch_gmma_tile(one, 1, g->st_area[p] + (size_t)s * g->st_stride[p], g->stream);
                ok = check_launch(g, e, "tiling an expert slot", err, err_len);
            }
            if (ok) g->st_place[s] = sl.place;
        }
        if (!ok) break;
        /* the wave's routing: each pair's slot, or -1 for the experts of other waves */
        if (hipEventSynchronize(g->rt_copied) != hipSuccess) { ok = fail(err, err_len, "waiting for the previous routing copy"); break; }
        route_out* ro = g->rt_host;
        for (int t = 0; t < n; t++) {
            memset(&ro[t], 0, sizeof(route_out));
            for (int i = 0; i < k; i++) {
                const int32_t x = ids[(size_t)t * k + i];
                ro[t].ids[i] = in_wave[x] ? slot_of[x] : -1;
                ro[t].weights[i] = ro[t].cw[i] = weights[(size_t)t * k + i];
                ro[t].chosen[i] = ro[t].ids[i];
            }
        }
        e = hipMemcpyAsync(g->rt, ro, (size_t)n * sizeof(route_out), hipMemcpyHostToDevice, g->stream);
        if (e == hipSuccess) e = hipEventRecord(g->rt_copied, g->stream);
        if (e == hipSuccess) e = launch_group(g->rt, n, c.n_slots, g->K, ROWS_MAX, g->grp_count, g->grp_pairs, g->stream);
        if (e == hipSuccess) e = launch_gmma_in(m, g->stream);
        if (e == hipSuccess) e = launch_gmma_down(m, g->stream);
        ok = check_launch(g, e, "the rows' experts", err, err_len);
    }
    if (ok) ok = check_launch(g, launch_reduce_rows(g->ypart, g->x, n, g->K, g->H, g->stream), "the rows' sums", err, err_len);
    /* the holds are released whatever happened; the guess only after the kernels */
    const bool fin = ec_rows_finish(c, layer, ok ? guess : nullptr, n, k, err, err_len);
    return ok && fin;
}

extern "C" bool vitna_cuda_moe_rows_experts(struct vitna_cuda_model* g, size_t layer, size_t n, const int32_t* ids, const float* weights,
                                            size_t k, const int32_t* guess, char* err, size_t err_len) {
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!ensure_tiled(g, err, err_len)) return false;
    if (layer >= (size_t)g->NL) return fail(err, err_len, "layer %zu: the model has %d", layer, g->NL);
    if (n != (size_t)g->rows_n) return fail(err, err_len, "%zu rows; the pass has %d", n, g->rows_n);
    if (g->ec.on) return cached_rows_experts(g, (int)layer, (int)n, ids, weights, (int)k, guess, err, err_len);
    if (g->pass_exact)
        return put_routing(g, n, ids, weights, k, err, err_len) &&
               check_launch(g, enqueue_exact_experts(g, (int)layer, (int)n), "the rows' experts", err, err_len);
    if (rows_fast(g, (int)n)) {
        if (!prefill_reserve(g, n, err, err_len) || !put_routing(g, n, ids, weights, k, err, err_len)) return false;
        return check_launch(g, enqueue_fast_experts(g, (int)layer, (int)n, g->rt), "the rows' experts (grouped GEMM)", err, err_len);
    }
    if (!put_routing(g, n, ids, weights, k, err, err_len)) return false;
    return check_launch(g, enqueue_rows_experts(g, (int)layer, (int)n, false), "the rows' experts", err, err_len);
}

extern "C" bool vitna_cuda_moe_rows_head(struct vitna_cuda_model* g, size_t n, float* const* logits, char* err, size_t err_len) {
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!ensure_tiled(g, err, err_len)) return false;
    if (!g->attention) return fail(err, err_len, "this model has no output projection");
    if (n != (size_t)g->rows_n) return fail(err, err_len, "%zu rows; the pass has %d", n, g->rows_n);
    /* a prompt's chunks before its last ask no logits (model.c:1011): then the head has nothing to do */
    const int head = head_rows(g, n, logits);
    if (head == HEAD_NONE) return true;
    if (!check_launch(g, g->pass_exact ? enqueue_exact_head(g, (int)n) : enqueue_rows_head(g, (int)n, nullptr, head), "the head", err, err_len))
        return false;
    for (size_t i = 0; i < n; i++)
        if (logits && logits[i])
            HIP_TRY(hipMemcpyAsync(logits[i], g->vocab + i * g->V, (size_t)g->V * 4, hipMemcpyDeviceToHost, g->stream), "copying logits");
    HIP_TRY(hipStreamSynchronize(g->stream), "running the head");
    return true;
}

/* A whole decode step of n rows on the device, routing included. */
static hipError_t enqueue_rows_step_body(vitna_cuda_model* g, int n, int head) {
    hipError_t e = launch_embed_rows(g->embed, g->rows_dev, n, g->x, g->stream);
    const bool fast = rows_fast(g, n);
    /* each layer's experts' outputs are added onto the rows by the next layer's (or the head's) norm kernel; a fast
       pass adds them at once */
    const float* pending = nullptr;
    for (int l = 0; e == hipSuccess && l < g->NL; l++) {
        e = enqueue_rows_attention(g, l, n, pending);
        /* every layer's routing is kept (rows_rt, the last layer's in rt), the checkers read it */
        route_out* rt = l + 1 < g->NL ? g->rows_rt + (size_t)l * ROWS_MAX : g->rt;
        const dlayer& d = g->L[l];
        if (fast) {
            if (e == hipSuccess) e = enqueue_route(g, l, g->rlogits, n, g->x, g->xn, true, nullptr, rt);
            if (e == hipSuccess && n == 1) e = launch_topk(g->rlogits, 1, g->E, g->K, g->renorm, rt, g->stream);
            if (e == hipSuccess) e = enqueue_fast_experts(g, l, n, rt);
            pending = nullptr;
            continue;
        }
        /* several rows: the top-k kernel also splits the normed rows for the grouped experts */
        const bool fused_split = n > 1 && gmma_fits(d.gate, d.up, d.down);
        const topk_split sp = {g->xn, g->gm_xs, g->gm_xsum, (int)g->H, gmma_gran(d.gate.dtype)};
        if (e == hipSuccess) e = enqueue_route(g, l, g->rlogits, n, g->x, g->xn, true, fused_split ? &sp : nullptr, rt);
        if (e == hipSuccess && n == 1) e = launch_topk(g->rlogits, 1, g->E, g->K, g->renorm, rt, g->stream);
        if (e == hipSuccess) e = enqueue_rows_experts(g, l, n, true, fused_split, rt);
        pending = g->ypart;
    }
    if (e == hipSuccess) e = enqueue_rows_head(g, n, pending, head);
    return e;
}

static bool ensure_rows_graph(vitna_cuda_model* g, int n, int head, char* err, size_t err_len) {
    if (!ensure_tiled(g, err, err_len)) return false;
    /* a fast pass's working buffers exist before the capture (growing them later would free what the graph uses) */
    if (rows_fast(g, n) && !prefill_reserve(g, (size_t)n, err, err_len)) return false;
    const bool fast = rows_fast(g, n);
    int pick = 0;
    for (int i = 0; i < ROWS_GRAPHS; i++) {
        const auto& r = g->rg[i];
        if (r.n == n && r.shared == g->rows_shared_seq && r.fast == fast && r.splits == g->splits_grid && r.head == head) {
            g->rg[i].used = ++g->rg_clock;
            g->rg_cur = i;
            return true;
        }
        if (!r.n || (g->rg[pick].n && r.used < g->rg[pick].used)) pick = i;
    }
    auto& r = g->rg[pick];
    HIP_TRY(hipStreamSynchronize(g->stream), "before capturing the rows step");
    if (r.n) {
        (void)hipGraphExecDestroy(r.exec);
        (void)hipGraphDestroy(r.src);
        r.n = 0;
    }
    HIP_TRY(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal), "capturing the rows step");
    const hipError_t e = enqueue_rows_step_body(g, n, head);
    hipGraph_t graph = nullptr;
    const hipError_t e2 = hipStreamEndCapture(g->stream, &graph);
    if (e != hipSuccess) { if (graph) (void)hipGraphDestroy(graph); return check_launch(g, e, "capturing the rows step", err, err_len); }
    HIP_TRY(e2, "ending the capture of the rows step");
    const hipError_t e3 = hipGraphInstantiate(&r.exec, graph, nullptr, nullptr, 0);
    if (e3 != hipSuccess) (void)hipGraphDestroy(graph);
    HIP_TRY(e3, "instantiating the rows step's graph");
    r.src = graph;
    r.n = n;
    r.fast = fast;
    r.shared = g->rows_shared_seq;
    r.splits = g->splits_grid;
    r.head = head;
    r.used = ++g->rg_clock;
    g->rg_cur = pick;
    return true;
}

extern "C" bool vitna_hip_moe_rows_step(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t n, float* const* logits, char* err,
                                        size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!g->attention) return fail(err, err_len, "this model has no attention");
    if (!set_rows(g, rows, n, err, err_len)) return false;
    if (!ensure_rows_graph(g, (int)n, head_rows(g, n, logits), err, err_len)) return false;
    HIP_TRY(hipGraphLaunch(g->rg[g->rg_cur].exec, g->stream), "launching the rows step");
    g->last_step_mega = false;
    for (size_t i = 0; i < n; i++)
        if (logits && logits[i])
            HIP_TRY(hipMemcpyAsync(logits[i], g->vocab + i * g->V, (size_t)g->V * 4, hipMemcpyDeviceToHost, g->stream), "copying logits");
    if (logits) HIP_TRY(hipStreamSynchronize(g->stream), "running the rows step");
    return true;
}

extern "C" bool vitna_hip_time_rows(struct vitna_cuda_model* g, const vitna_cuda_row_t* rows, size_t n, int steps, double* ms_per_step,
                                    char* err, size_t err_len) {
    if (g && !experts_resident(g, err, err_len)) return false;
    if (!g || g->lost) return fail(err, err_len, "the device model is not usable");
    if (!g->attention) return fail(err, err_len, "this model has no attention");
    if (steps < 1) return fail(err, err_len, "at least one step");
    if (!set_rows(g, rows, n, err, err_len)) return false;
    if (!ensure_rows_graph(g, (int)n, HEAD_ALL, err, err_len)) return false;
    event_pair ev;
    HIP_TRY(ev.make(), "events");
    HIP_TRY(hipGraphLaunch(g->rg[g->rg_cur].exec, g->stream), "launching the rows step"); /* warm-up */
    HIP_TRY(hipStreamSynchronize(g->stream), "before timing");
    HIP_TRY(hipEventRecord(ev.t0, g->stream), "events");
    for (int i = 0; i < steps; i++) HIP_TRY(hipGraphLaunch(g->rg[g->rg_cur].exec, g->stream), "launching the rows step");
    HIP_TRY(hipEventRecord(ev.t1, g->stream), "events");
    HIP_TRY(hipEventSynchronize(ev.t1), "timing the rows steps");
    float ms = 0;
    HIP_TRY(hipEventElapsedTime(&ms, ev.t0, ev.t1), "events");
    *ms_per_step = (double)ms / steps;
    return true;
}
