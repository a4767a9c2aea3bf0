/**
 * vitna_kernels.h - Host-side launchers of libvitna_hip's kernels, shared by
 * the translation units (kernels_*.hip) and the engine (engine.hip). Every
 * launcher checks on the host that the shapes it is given are the shapes its
 * kernel assumes, and returns hipErrorInvalidValue otherwise, before anything
 * is launched.
 */

#ifndef VITNA_KERNELS_H
#define VITNA_KERNELS_H

#include "vitna_hip_internal.h"

#define ROUTE_K_MAX 16
#define ROUTE_E_MAX 512

/* A layer's routing on the device: the experts in order of id (ids), their
   weights, and the router's choice largest first (chosen). */
struct route_out {
    int32_t ids[ROUTE_K_MAX];     /* the chosen experts, ascending (the order the mixture is summed in) */
    float weights[ROUTE_K_MAX];   /* their weights, in the order of ids */
    int32_t chosen[ROUTE_K_MAX];  /* the chosen experts, largest logit first: the decode path's expert slots */
    float cw[ROUTE_K_MAX];        /* their weights, in the order of chosen */
};

/* ---- upload and checking ---- */

/* Split n_blocks GGUF blocks of dtype (AoS, as stored) at src into planes
   dst (plane pointers of one matrix, rows x nb). */
hipError_t launch_repack(const uint8_t* src, const qmat& dst, hipStream_t s);
/* Widen matrix m (expert e) into out, rows x cols, exactly: from the planes
   (way 0) or from the GGUF blocks at src (way 1). */
hipError_t launch_widen_planes(const qmat& m, int e, float* out, hipStream_t s);
hipError_t launch_widen_blocks(const uint8_t* src, int dtype, size_t rows, size_t cols, float* out, hipStream_t s);

/* ---- routing ---- */

/* RMSNorm of x (n_rows rows of H, row stride H) with norm_w, in the
   reference CPU's order, written to xn_out when it is not NULL, and the
   router's logits for each row (E of them, the router F32 [E x H]) in the
   reference CPU's order into logits (row stride E). The routing itself
   runs after it (launch_topk). */
/* The residual after a layer's attention while the o-projection's output is still in per-head-group parts
   (launch_attention_oproj): x + (((p_0 + p_1) + p_2) + ...), the parts summed in group order, then added. Every
   kernel that reads that residual forms it with this function, so all of them see the same bits. */
#define OPROJ_PARTS_MAX 8 /* n_heads / ATTN_OPROJ_HEADS at most: 32 query heads */
/* attn_resid in two steps, so that a kernel can request the parts early and add them late: the loads (every
   slot loaded, those past n_parts as the last part, unused; no branch), then the sum */
__device__ __forceinline__ void attn_parts_load(const float* __restrict__ parts, int n_parts, size_t stride, size_t i,
                                                float (&v)[OPROJ_PARTS_MAX]) {
#pragma unroll
    for (int p = 0; p < OPROJ_PARTS_MAX; p++) v[p] = parts[(size_t)min(p, n_parts - 1) * stride + i];
}
__device__ __forceinline__ float attn_parts_sum(float x, const float (&v)[OPROJ_PARTS_MAX], int n_parts) {
    float s = v[0];
#pragma unroll
    for (int p = 1; p < OPROJ_PARTS_MAX; p++) s = p < n_parts ? s + v[p] : s;
    return x + s;
}
__device__ __forceinline__ float attn_resid(float x, const float* __restrict__ parts, int n_parts, size_t stride, size_t i) {
    float v[OPROJ_PARTS_MAX];
    attn_parts_load(parts, n_parts, stride, i, v);
    return attn_parts_sum(x, v, n_parts);
}
#define ROUTE_PARTS_HMAX 2048 /* the widest rows the router takes with parts */

struct route_args {
    const float* x;
    const float* norm_w;
    const float* router;
    float* xn_out;
    float* logits;
    int H, E, n_rows;
    float eps;
    /* one row only: x's attention parts still to add (n_parts of H floats, part_stride apart), or null */
    const float* parts;
    int n_parts;
};
hipError_t launch_route(const route_args& a, hipStream_t s);

/* The device routing of one token's E logits (the rule every expert kernel
   applies), into *out: for checking it against the reference's rule. */
hipError_t launch_route_check(const float* logits, int E, int K, int renorm, route_out* out, hipStream_t s);

/* The routing of n_rows rows of logits (row stride E), one wave a row. */
/* The grouped experts' split of the routed rows (gmma_split.h), run by the routing kernel: x rows of H floats
   into xs and sums, runs of gran columns; xs null: none. */
struct topk_split {
    const float* x;
    uint16_t* xs;
    float* sums;
    int H, gran;
};
hipError_t launch_topk(const float* logits, int n_rows, int E, int K, int renorm, route_out* out, hipStream_t s,
                       const topk_split* sp = nullptr);

/* ---- experts, one token ---- */

/* act[k * I + r] = silu(gate_e[r] . xn) * (up_e[r] . xn) for e = ids[k].
   With logits set, every block first routes the token (the rule of
   engine/src/model.c:626-703 on its E router logits) and block 0 publishes
   the routing to rt; otherwise rt holds it already. */
struct experts_in_args {
    qmat gate, up;
    const float* xn;
    route_out* rt;
    const float* logits;
    int E, renorm;
    float* act;
    int K;
};
/* n_rows > 1: the same for each of n_rows tokens (xn rows of gate.cols, rt, act rows of K I, logits rows of E),
   each token's arithmetic that of a single token: its bits. */
hipError_t launch_experts_in(const experts_in_args& a, hipStream_t s, int n_rows = 1);

/* y[r] (+)= sum_k w_k (down_{ids[k]}[r] . act_k), into y or, with add,
   onto it. */
struct experts_down_args {
    qmat down;
    const float* act;
    const route_out* rt;
    float* y;
    int K, add;
    /* with add: the attention parts (attn_resid) added to y before the experts' sum, or null */
    const float* parts;
    int n_parts;
};
/* n_rows > 1 (without parts): the same for each of n_rows tokens (act rows of K cols, rt, y rows of down.rows). */
hipError_t launch_experts_down(const experts_down_args& a, hipStream_t s, int n_rows = 1);

/* ---- dense projections ---- */

/* Up to three matrices of the same width multiplied by one vector:
   y_i = W_i . xin, where xin = RMSNorm(x, norm_w) when norm_w is set (each
   block computes it) and x otherwise; with add, y_i += W_i . xin. With rows > 1, the same for each of rows
   vectors (x at xstride floats apart, y_i at ystride[i]): every row's sums in the order of a single vector's, so
   a row's result is the bits one call on it alone would give. */
struct gemv_args {
    qmat w[3];
    float* y[3];
    int n;          /* matrices */
    const float* x;
    const float* norm_w;
    float eps;
    int add;
    int rows;       /* 0 or 1: one vector */
    int xstride, ystride[3];
};
hipError_t launch_gemv(const gemv_args& a, hipStream_t s);

/* x = the embedding row of token (read from the device word *token when
   token_dev is set, else token), widened exactly. */
hipError_t launch_embed(const qmat& embed, const int32_t* token_dev, int token, float* x, hipStream_t s);

/* ---- attention (kernels_attn.hip) ---- */

/* A row of a pass: the token, its position, and the sequence whose cache it
   reads and writes (engine/include/model_cuda.h:21, vitna_cuda_row_t). */
struct row_rec {
    int32_t token, pos, seq;
};

/* Decode attention for n_rows rows, one layer: each row's q and k through the
   per-head RMSNorm (when q_norm is set) and the half-split RoPE at its
   position, its k and v written into its sequence's cache at that position,
   and softmax(q k^T / sqrt(hd)) v over positions 0..pos. Positions are split
   into chunks of ATTN_CHUNK, each block leaving its chunk's partial (max,
   sum, weighted values) in partial; launch_attention_merge combines them into
   att. */
#define ATTN_CHUNK 64
/* The most chunks a row's merge combines (its LDS holds one maximum and one sum a chunk): a context of at most
   ATTN_SPLITS_MAX * ATTN_CHUNK positions. */
#define ATTN_SPLITS_MAX 1024
/* Where a pass's operand images for the multi-row projections go (skinny_image.h); a null: none. */
struct img_out {
    u32x4* a;
    u32x4* b;
    uint16_t* s32;
    uint16_t* s16;
};

struct attn_args {
    const float* q_raw;    /* [n_rows][n_heads * hd] */
    const float* k_raw;    /* [n_rows][n_kv * hd] */
    const float* v_raw;
    const float* q_norm;   /* hd, or NULL */
    const float* k_norm;
    const float* cos_tab;  /* [ctx][hd/2] */
    const float* sin_tab;
    float* k_cache;        /* sequence 0 of this layer: [ctx][n_kv * hd] */
    float* v_cache;
    size_t seq_stride;     /* floats from one sequence's cache of this layer to the next's */
    const row_rec* rows;   /* device, n_rows */
    int n_rows;
    float* partial;        /* [n_rows][n_kv][splits_max][G][hd + 4]: values, max, sum, padding */
    float* att;            /* [n_rows][n_heads * hd] */
    int n_heads, n_kv, hd, ctx, splits_max;
    /* chunks the launch covers (the grid's first dimension): at least the most any row of the pass has, at most
       splits_max; 0: splits_max. Blocks past a row's last chunk return at once, but they still take a dispatch. */
    int splits_grid;
    float eps;
    /* 0: this kernel normalizes and rotates q and k and stores k and v at
       each row's position itself (rows of distinct sequences). 1: q_raw holds
       the prepared queries and the cache already holds every row's k and v
       (launch_attention_prepare ran first: rows may share a sequence). */
    int prepared;
    float* q_out;          /* prepare: where the prepared queries go */
    /* 1: the score and value products on the fp32 matrix cores (head dimension 128). 0: the fp32 vector
       kernel. */
    int mma;
    /* merge: att's operand images for the o-projection too, when img.a (n_heads * hd a multiple of 256) */
    img_out img;
};
hipError_t launch_attention(const attn_args& a, hipStream_t s);
/* Each row: the chunks' partials merged, as launch_attention_merge merges them (same bits in att), and the
   o-projection applied group by group: the n_heads / ATTN_OPROJ_HEADS groups of ATTN_OPROJ_HEADS query heads
   each leave parts[row][g][r] = o[r][the group's columns] . att[row][the group's columns]. The residual then is
   attn_resid(x, parts, n_heads / ATTN_OPROJ_HEADS, o.rows). A row of several gets the bits it gets alone. Each block merges one group's heads and
   multiplies them into a range of rows, so no kernel waits on another for att. attention_oproj_fits says
   whether a layer takes it (else: launch_attention_merge, then the o-projection GEMV). */
#define ATTN_OPROJ_HEADS 4
bool attention_oproj_fits(const attn_args& a, const qmat& o);
hipError_t launch_attention_oproj(const attn_args& a, const qmat& o, float* parts, hipStream_t s);
/* x[row][i] = attn_resid(x[row][i], parts[row], n_parts, H, i) for n_rows rows (parts n_parts H floats a row):
   the parts folded into the residual (for a reader of the residual between the attention and the experts). */
hipError_t launch_attn_fold(float* x, const float* parts, int n_parts, int H, hipStream_t s, int n_rows = 1);
/* Rows of ONE sequence (prepared: queries in q_raw, every row's key and value stored), head dimension 128: att of
   every (row, query head) from tiles of 4 * 16 / G rows, each block a tile's chunks in a loop with the softmax
   folded across them, each chunk's keys and values read once a tile (a prompt's passes). No partials, no merge;
   sums in another order than launch_attention's and the merge's. attention_run_fits says whether a pass takes it. */
bool attention_run_fits(const attn_args& a);
hipError_t launch_attention_flash(const attn_args& a, hipStream_t s);
/* The chunks' partials of every (row, query head) combined into att. */
hipError_t launch_attention_merge(const attn_args& a, hipStream_t s);
/* The prepare pass of prepared = 1: q normalized and rotated into q_out, k
   normalized and rotated and v stored into the cache at each row's position. */
hipError_t launch_attention_prepare(const attn_args& a, hipStream_t s);

/* ---- several rows (kernels_rows.hip) ---- */

hipError_t launch_embed_rows(const qmat& embed, const row_rec* rows, int n, float* x, hipStream_t s);
/* x[row] += the K parts of ypart in slot order (when ypart), y = RMSNorm(x) * w, and y's operand images when
   img.a (H a multiple of 256 then). */
hipError_t launch_residual_norm(float* x, const float* ypart, int K, const float* w, float* y, int n, int H, float eps,
                                const img_out& img, hipStream_t s);

/* y_i[row][r] (+)= W_i[r] . x[row] for n rows of x (row stride xstride); up to three matrices of one width. */
struct gemv_multi_args {
    qmat w[3];
    float* y[3];
    int nm;
    const float* x;
    int n, xstride, add;
};
hipError_t launch_gemv_multi(const gemv_multi_args& a, hipStream_t s);

/* Multi-row projections on the matrix cores (kernels_skinny.hip): y_i[t][r]
   (+)= W_i[r] . x[t] for t < n, to fp32 accuracy. launch_split_rows splits x
   into bf16 hi and lo parts: with img (widths a multiple of 256) into the
   operand images and group sums of the exact-integer kernels (img[0], img[1]:
   column orders A and B, [n / 32][cols / 256][2048] x 16 bytes each; img[2],
   img[3]: 32- and 16-column sums, [n / 32][cols / 256 or cols / 128][3][64]
   x 8 bytes), otherwise row-major into xh and xl ([n][cols] each), for the
   kernel that widens and splits each weight. */
struct skinny_args {
    qmat w[3];
    float* y[3];
    int nm;
    const uint16_t* xh;
    const uint16_t* xl;
    const uint32_t* img[2];
    const uint32_t *s32, *s16;
    int n, add;
    /* matrices wider than 2048 columns split across blocks: part (part_cap floats) holds each split's sum of a
       tile and cnt (cnt_cap ints, zero before the first call, left zero by every call) counts finished splits */
    float* part;
    int* cnt;
    size_t part_cap, cnt_cap;
    int splits[3], tiles, split_max; /* set by launch_skinny */
};
hipError_t launch_split_rows(const float* x, int n, int K, int xstride, uint16_t* xh, uint16_t* xl, uint32_t* const* img,
                             hipStream_t s);
hipError_t launch_skinny(const skinny_args& a, hipStream_t s);
/* The tiled copy of m (tile_bytes(dtype) x ceil(rows / 32) x cols / 256 bytes at dst) from its planes. */
hipError_t launch_tile(const qmat& m, uint8_t* dst, hipStream_t s);

/* The per-expert lists of (row, slot) pairs of n rows' routing: count[E],
   pairs[E][cap] = row * ROUTE_K_MAX + slot, in order of row. */
hipError_t launch_group(const route_out* rt, int n, int E, int K, int cap, int* count, int* pairs, hipStream_t s);

/* The grouped experts on the bf16 matrix cores (kernels_gmma.hip): activations split into bf16 hi/lo
   chunks with sums over runs of gmma_gran(dtype) columns (launch_gmma_split), gate/up writing the SwiGLU output
   split the same way, down into ypart. */
struct gmma_args {
    qmat gate, up, down;
    const uint16_t* xs;    /* the normalized rows, split [n][2H] */
    const float* xsum;     /* their sums [n][H / gmma_gran(gate)] */
    uint16_t* as;          /* the SwiGLU output, split [n * K][2I] */
    float* asum;           /* its sums [n * K][I / gmma_gran(down)] */
    const route_out* rt;   /* [n] */
    const int* count;      /* [E] */
    const int* pairs;      /* [E][cap] */
    int E, K, cap;
    int n;                 /* rows of the pass */
    float* ypart;          /* [n][K][H] */
};
/* The grouped experts' tiled copy of an expert set (kernels_gmma.hip): its size, and making it from the planes. */
size_t gmma_tiled_bytes(const qmat& m, int n_experts);
hipError_t launch_gmma_tile(const qmat& m, int n_experts, uint8_t* dst, hipStream_t s);
bool gmma_fits(const qmat& gate, const qmat& up, const qmat& down);
int gmma_gran(int dtype);
hipError_t launch_gmma_split(const float* x, int n, int K, int xstride, int gran, uint16_t* xs, float* sums, hipStream_t s);
hipError_t launch_gmma_in(const gmma_args& a, hipStream_t s);
hipError_t launch_gmma_down(const gmma_args& a, hipStream_t s);
/* The grouped experts of a crowded pass (kernels_skinny.hip): tiles of 32 pairs of one expert on the exact
   bf16 arithmetic of the multi-row projections. gate, up and down carry in .tiled their per-expert tiled copies
   (gsx_tiled_bytes, launch_gsx_tile); the pairs are launch_group's lists. Leaves ypart as launch_gmma_down does. */
struct gsx_args {
    qmat gate, up, down;
    const float* xn;       /* the normalized rows [n][H] */
    const route_out* rt;   /* [n] */
    const int* count;      /* [E] */
    const int* pairs;      /* [E][cap] */
    int E, K, cap, n;
    int *toff, *te;        /* [E + 1], [max_tiles] */
    int max_tiles;         /* at least gsx_max_tiles(n, K, E) */
    uint32_t* img_in;      /* operand images of the tiles' rows: 32 max_tiles x H x 4 bytes */
    uint32_t* img_act;     /* of the SwiGLU output: 32 max_tiles x I x 4 bytes */
    uint16_t *s32, *s16;   /* group sums: max_tiles x (max(H, I) / 256) x 1536 bytes, and twice that */
    float* act;            /* the SwiGLU output [32 max_tiles][I] */
    float* ypart;          /* [n][K][H] */
};
bool gsx_fits(const qmat& gate, const qmat& up, const qmat& down);
int gsx_max_tiles(int n, int K, int E);
size_t gsx_tiled_bytes(const qmat& m, int n_experts);
hipError_t launch_gsx_tile(const qmat& m, int n_experts, uint8_t* dst, hipStream_t s);
hipError_t launch_gsx(const gsx_args& a, hipStream_t s);

/* x[row] += the row's K outputs in ypart, added in slot order. */
hipError_t launch_reduce_rows(const float* ypart, float* x, int n, int K, int H, hipStream_t s);

/* ---- helpers ---- */
/* compute units of the current device (cached) */
int gemv_device_cus();
hipError_t launch_copy_probe(const void* src, void* dst, size_t bytes, hipStream_t s);
/* blocks x 256 threads of back-to-back bf16 MFMAs (out: blocks x 256 floats); the flops they do */
hipError_t launch_mfma_probe(float* out, int blocks, int iters, hipStream_t s);
double mfma_probe_flops(int blocks, int iters);
hipError_t launch_fill_normal(float* out, size_t n, uint64_t seed, hipStream_t s);


/* ---- prefill through one MoE layer (kernels_prefill.hip) ---- */
struct prefill_args {
    qmat gate, up, down;    /* Q8_0 experts of the layer */
    const uint16_t* xb;     /* bf16 normalized rows [n][H] */
    const route_out* rt;    /* [n] */
    const int* count;       /* [E] pairs of each expert */
    const int* pairs;       /* [E][cap] row * ROUTE_K_MAX + slot, rows ascending */
    const int* off;         /* [E] first pair of each expert in act */
    const int* tiles;       /* (expert << 16) | tile of 256 pairs */
    const int* n_tiles;
    uint16_t* act;          /* bf16 [n * K][I], pairs in expert order */
    uint16_t* ypart;        /* bf16 [n * K][H], row * K + slot: each pair's weighted expert output */
    int E, K, cap, n;
};
/* xn = RMSNorm(x) * w in the sixteen-chain order (route_kernel's, the same bits), and its bf16 rounding into xb
   unless xb is null. */
hipError_t launch_prefill_norm(const float* x, const float* w, float* xn, uint16_t* xb, int n, int H, float eps, hipStream_t s);
hipError_t launch_prefill_router(const float* xn, const float* R, float* logits, int n, int E, int H, hipStream_t s);
/* Both in one kernel, the fp32 normalized rows kept in LDS (hidden up to 2048; hipErrorNotSupported above). */
hipError_t launch_prefill_norm_router(const float* x, const float* nw, const float* R, float* logits, uint16_t* xb, int n, int E,
                                     int H, float eps, hipStream_t s);
/* xb = the bf16 rounding (to nearest even) of x, n values (n a multiple of 4). */
hipError_t launch_prefill_bf16(const float* x, uint16_t* xb, size_t n, hipStream_t s);
hipError_t launch_prefill_plan(const int* count, int E, int* off, int* tiles, int* n_tiles, hipStream_t s);
int prefill_max_tiles(int n, int K, int E);
/* x[row] += the sum over slots k (in order) of the bf16 parts ypart[row * K + k]. */
hipError_t launch_prefill_sum(const uint16_t* ypart, float* x, int n, int K, int H, hipStream_t s);
/* chosen[i * K + k] = rt[i].chosen[k]: each row's experts, largest logit first, as the caller's int32 array. */
hipError_t launch_prefill_chosen(const route_out* rt, int n, int K, int32_t* chosen, hipStream_t s);
hipError_t launch_prefill_gemm(const prefill_args& a, bool gate_up, hipStream_t s);

#endif
