/**
 * step_kernel.h - The persistent decode step (kernels_step.hip): its arguments
 * and launcher, shared with the engine.
 */

#ifndef VITNA_STEP_KERNEL_H
#define VITNA_STEP_KERNEL_H

#include "vitna_kernels.h"

/* the phases of a layer, each ending with every producing block's flag */
#define STEP_QKV 0
#define STEP_ATT 1
#define STEP_O 2
#define STEP_ROUTE 3
#define STEP_IN 4
#define STEP_DOWN 5
#define STEP_PHASES 6
#define STEP_OUT 2048 /* floats of a block's result staging in LDS */

/* One layer as the step reads it (device memory, one per layer). */
struct step_layer {
    qmat q, k, v, o, gate, up, down;
    const float *attn_norm, *mlp_norm, *q_norm, *k_norm, *router;
    float *k_cache, *v_cache; /* sequence 0 of this layer: [ctx][n_kv * hd] */
};

struct step_args {
    const step_layer* L;  /* NL layers */
    int NL;
    qmat embed;
    const row_rec* row;   /* the token, its position and sequence (device) */
    const float *cos_tab, *sin_tab;
    size_t seq_stride;    /* floats from one sequence's cache to the next's */
    /* per-layer buffers, layer l at base + l * stride (floats) */
    float *qkv, *part, *opart, *att, *xmid, *logits, *act, *xout;
    size_t s_qkv, s_part, s_opart, s_att, s_xmid, s_logits, s_act;
    uint32_t* flags;       /* [NL][STEP_PHASES][256] epochs */
    uint32_t* abort_word;  /* set when a wait runs out */
    route_out* rt_layers;  /* each layer's routing but the last */
    route_out* rt_last;    /* the last layer's */
    const float* x0;       /* models without attention: the input residual */
    float* x_final;        /* the last layer's output residual, also */
    int H, I, E, K, nh, nkv, hd, renorm, attention;
    float eps;
    uint32_t epoch;        /* this launch's flag value, larger than every earlier launch's */
    int nb;                /* blocks: one a compute unit */
    int poll_nap;          /* s_sleep 1 periods (64 clocks) between two polls of a flag set */
    uint64_t* trace;       /* or null: block trace_block's control wave stamps each phase (s_memrealtime, 100 MHz) */
    int trace_block;
};
#define STEP_TRACE_PER_LAYER 32

/* Why the persistent step cannot serve a model of this shape, or null. */
const char* step_unsupported(int H, int I, int E, int K, int nh, int nkv, int hd, int nb, int dt_q, int dt_k, int dt_v, int dt_o, int dt_gu,
                             int dt_dn);
size_t step_lds_bytes(int H, int hd, int nh, int nkv, int K, int I, int nb);
/* dts: the gate/up, down, q (and k), v and o dtypes */
hipError_t launch_step(const step_args& a, const int* dts, hipStream_t s);

#endif
