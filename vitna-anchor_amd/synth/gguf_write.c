/**
 * gguf_write.c - A synthetic model written as a GGUF checkpoint (version 3)
 * and the config.json the reference's loader reads beside it: workload
 * generation for the GGUF reader's tests (include/vitna_gguf.h). The bytes of
 * every tensor are the model's own, so a model read back from the file
 * computes exactly what the model in memory computes.
 *
 * Layout written (llama.cpp's naming and order): token_embd, output_norm,
 * output, then per layer attn_norm, attn_q, attn_k, attn_v, attn_output,
 * attn_q_norm, attn_k_norm, ffn_norm, ffn_gate_inp, ffn_gate_exps,
 * ffn_up_exps, ffn_down_exps; each expert stack [experts][rows][cols] in
 * expert order. Extents fastest first (columns, rows, experts); data offsets
 * multiples of the alignment. A few metadata entries the reader must step
 * over (a string, a string array, a bool) are written too.
 */

#include "vitna_synth.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { G_U32 = 4, G_F32 = 6, G_BOOL = 7, G_STR = 8, G_ARR = 9 };

typedef struct {
    FILE* f;
    int ok;
} out_t;

static void wr(out_t* o, const void* p, size_t n) {
    if (o->ok && n && fwrite(p, 1, n, o->f) != n) o->ok = 0;
}
static void w32(out_t* o, uint32_t v) {
    uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    wr(o, b, 4);
}
static void w64(out_t* o, uint64_t v) {
    w32(o, (uint32_t)v);
    w32(o, (uint32_t)(v >> 32));
}
static void wstr(out_t* o, const char* s) {
    w64(o, strlen(s));
    wr(o, s, strlen(s));
}
static void kv_u32(out_t* o, const char* arch, const char* key, uint32_t v) {
    char k[128];
    snprintf(k, sizeof(k), "%s.%s", arch, key);
    wstr(o, k);
    w32(o, G_U32);
    w32(o, v);
}
static void kv_f32(out_t* o, const char* arch, const char* key, float v) {
    char k[128];
    snprintf(k, sizeof(k), "%s.%s", arch, key);
    wstr(o, k);
    w32(o, G_F32);
    uint32_t b;
    memcpy(&b, &v, 4);
    w32(o, b);
}

static uint32_t ggml_type(int dtype) {
    switch (dtype) {
        case VITNA_DTYPE_F32: return 0;
        case VITNA_DTYPE_F16: return 1;
        case VITNA_DTYPE_Q8_0: return 8;
        case VITNA_DTYPE_Q4_K: return 12;
        case VITNA_DTYPE_Q6_K: return 14;
        case VITNA_DTYPE_BF16: return 30;
        default: return 0xffffffffu;
    }
}

/* One tensor of the file: up to 3 extents, and where its bytes come from (n_parts pieces of part_bytes each). */
typedef struct {
    char name[96];
    uint32_t dims;
    uint64_t ne[3];
    int dtype;
    uint64_t offset;
    uint64_t bytes;
    const void* parts[1024];
    size_t n_parts, part_bytes;
    const float* f32; /* a norm: float32 values written as dtype */
} tensor_t;

static size_t matrix_bytes(const vitna_matrix_t* m) { return vitna_matrix_row_bytes(m->dtype, m->cols) * m->rows; }

int vitna_synth_write_gguf(const vitna_llama_t* m, const char* dir, int norm_dtype, uint32_t alignment, char* err, size_t err_len) {
    const vitna_llama_config_t* c = &m->cfg;
    const char* arch = c->qwen3 ? "qwen3moe" : "olmoe";
    if (!c->n_heads || !c->n_experts || !m->embed.data || !c->qk_norm || c->qk_norm_per_head != c->qwen3 || c->n_experts > 1024 ||
        (norm_dtype != VITNA_DTYPE_F32 && norm_dtype != VITNA_DTYPE_F16 && norm_dtype != VITNA_DTYPE_BF16) || !alignment ||
        (alignment & (alignment - 1))) {
        if (err && err_len)
            snprintf(err, err_len, "the writer takes a mixture-of-experts model with attention and the QK-norm of its architecture "
                                   "(Qwen3's per head, OLMoE's whole), norms F32, F16 or BF16, a power-of-two alignment");
        return -1;
    }
    const size_t H = c->hidden, I = c->intermediate, E = c->n_experts, hd = c->head_dim;
    const size_t qd = c->n_heads * hd, kd = c->n_kv_heads * hd;
    const size_t n_t = 3 + c->n_layers * 12;
    tensor_t* T = (tensor_t*)calloc(n_t, sizeof(tensor_t));
    if (!T) return -1;
    size_t n = 0;
#define MAT(nm, mat)                                                                   \
    do {                                                                               \
        tensor_t* t = &T[n++];                                                         \
        snprintf(t->name, sizeof(t->name), "%s", nm);                                  \
        t->dims = 2; t->ne[0] = (mat).cols; t->ne[1] = (mat).rows; t->dtype = (mat).dtype; \
        t->parts[0] = (mat).data; t->n_parts = 1; t->part_bytes = matrix_bytes(&(mat)); \
    } while (0)
#define NORM(nm, vals, len)                                                           \
    do {                                                                              \
        tensor_t* t = &T[n++];                                                        \
        snprintf(t->name, sizeof(t->name), "%s", nm);                                 \
        t->dims = 1; t->ne[0] = (len); t->dtype = norm_dtype; t->f32 = (vals);        \
        t->n_parts = 1; t->part_bytes = (len) * (norm_dtype == VITNA_DTYPE_F32 ? 4 : 2); \
    } while (0)
    char nm[96];
    MAT("token_embd.weight", m->embed);
    NORM("output_norm.weight", m->final_norm, H);
    MAT("output.weight", m->lm_head);
    for (size_t l = 0; l < c->n_layers; l++) {
        const vitna_llama_layer_t* L = &m->layers[l];
        snprintf(nm, sizeof(nm), "blk.%zu.attn_norm.weight", l); NORM(nm, L->attn_norm, H);
        snprintf(nm, sizeof(nm), "blk.%zu.attn_q.weight", l); MAT(nm, L->q);
        snprintf(nm, sizeof(nm), "blk.%zu.attn_k.weight", l); MAT(nm, L->k);
        snprintf(nm, sizeof(nm), "blk.%zu.attn_v.weight", l); MAT(nm, L->v);
        snprintf(nm, sizeof(nm), "blk.%zu.attn_output.weight", l); MAT(nm, L->o);
        snprintf(nm, sizeof(nm), "blk.%zu.attn_q_norm.weight", l); NORM(nm, L->q_norm, c->qwen3 ? hd : qd);
        snprintf(nm, sizeof(nm), "blk.%zu.attn_k_norm.weight", l); NORM(nm, L->k_norm, c->qwen3 ? hd : kd);
        snprintf(nm, sizeof(nm), "blk.%zu.ffn_norm.weight", l); NORM(nm, L->mlp_norm, H);
        snprintf(nm, sizeof(nm), "blk.%zu.ffn_gate_inp.weight", l); MAT(nm, L->router);
        static const char* stacks[3] = {"gate", "up", "down"};
        for (int s = 0; s < 3; s++) {
            tensor_t* t = &T[n++];
            snprintf(t->name, sizeof(t->name), "blk.%zu.ffn_%s_exps.weight", l, stacks[s]);
            const vitna_matrix_t* x0 = s == 0 ? &L->experts[0].gate : s == 1 ? &L->experts[0].up : &L->experts[0].down;
            t->dims = 3; t->ne[0] = x0->cols; t->ne[1] = x0->rows; t->ne[2] = E; t->dtype = x0->dtype;
            t->n_parts = E; t->part_bytes = matrix_bytes(x0);
            for (size_t e = 0; e < E; e++)
                t->parts[e] = s == 0 ? L->experts[e].gate.data : s == 1 ? L->experts[e].up.data : L->experts[e].down.data;
        }
    }
#undef MAT
#undef NORM
    uint64_t off = 0;
    for (size_t i = 0; i < n; i++) {
        T[i].bytes = (uint64_t)T[i].n_parts * T[i].part_bytes;
        T[i].offset = off;
        off = (off + T[i].bytes + alignment - 1) / alignment * alignment;
    }
    char path[1024];
    snprintf(path, sizeof(path), "%s/model.gguf", dir);
    out_t o = {fopen(path, "wb"), 1};
    if (!o.f) {
        free(T);
        if (err && err_len) snprintf(err, err_len, "cannot write %s", path);
        return -1;
    }
    const uint32_t n_kv = 17;
    w32(&o, 0x46554747u);
    w32(&o, 3);
    w64(&o, n);
    w64(&o, n_kv);
    wstr(&o, "general.architecture"); w32(&o, G_STR); wstr(&o, arch);
    wstr(&o, "general.alignment"); w32(&o, G_U32); w32(&o, alignment);
    wstr(&o, "general.name"); w32(&o, G_STR); wstr(&o, "synthetic");
    wstr(&o, "tokenizer.ggml.tokens"); w32(&o, G_ARR); w32(&o, G_STR); w64(&o, 3); wstr(&o, "a"); wstr(&o, "bc"); wstr(&o, "");
    wstr(&o, "general.quantized"); w32(&o, G_BOOL); { const uint8_t one = 1; wr(&o, &one, 1); }
    kv_u32(&o, arch, "block_count", (uint32_t)c->n_layers);
    kv_u32(&o, arch, "context_length", (uint32_t)c->max_positions);
    kv_u32(&o, arch, "embedding_length", (uint32_t)H);
    kv_u32(&o, arch, c->qwen3 ? "expert_feed_forward_length" : "feed_forward_length", (uint32_t)I);
    kv_u32(&o, arch, "attention.head_count", (uint32_t)c->n_heads);
    kv_u32(&o, arch, "attention.head_count_kv", (uint32_t)c->n_kv_heads);
    kv_u32(&o, arch, "attention.key_length", (uint32_t)hd);
    kv_u32(&o, arch, "expert_count", (uint32_t)E);
    kv_u32(&o, arch, "expert_used_count", (uint32_t)c->n_experts_used);
    kv_f32(&o, arch, "attention.layer_norm_rms_epsilon", c->rms_eps);
    kv_f32(&o, arch, "rope.freq_base", c->rope_theta);
    kv_u32(&o, arch, "vocab_size", (uint32_t)c->vocab);
    for (size_t i = 0; i < n; i++) {
        wstr(&o, T[i].name);
        w32(&o, T[i].dims);
        for (uint32_t d = 0; d < T[i].dims; d++) w64(&o, T[i].ne[d]);
        w32(&o, ggml_type(T[i].dtype));
        w64(&o, T[i].offset);
    }
    long at = ftell(o.f);
    static const uint8_t zeros[1 << 12];
    const uint64_t start = ((uint64_t)at + alignment - 1) / alignment * alignment;
    wr(&o, zeros, (size_t)(start - (uint64_t)at));
    uint64_t pos = 0;
    for (size_t i = 0; i < n && o.ok; i++) {
        wr(&o, zeros, (size_t)(T[i].offset - pos));
        if (T[i].f32) {
            for (size_t j = 0; j < T[i].ne[0]; j++) {
                const float v = T[i].f32[j];
                if (T[i].dtype == VITNA_DTYPE_F32) {
                    wr(&o, &v, 4);
                } else if (T[i].dtype == VITNA_DTYPE_F16) {
                    const uint16_t h = vitna_synth_f32_to_f16(v);
                    wr(&o, &h, 2);
                } else {
                    uint32_t b;
                    memcpy(&b, &v, 4);
                    const uint16_t h = (uint16_t)((b + 0x7fffu + ((b >> 16) & 1)) >> 16); /* round to nearest even */
                    wr(&o, &h, 2);
                }
            }
        } else {
            for (size_t p = 0; p < T[i].n_parts; p++) wr(&o, T[i].parts[p], T[i].part_bytes);
        }
        pos = T[i].offset + T[i].bytes;
    }
    const int file_ok = o.ok && fclose(o.f) == 0;
    free(T);
    if (!file_ok) {
        if (err && err_len) snprintf(err, err_len, "writing %s failed", path);
        return -1;
    }
    /* config.json, the keys engine/src/model.c:54-137 reads */
    snprintf(path, sizeof(path), "%s/config.json", dir);
    FILE* f = fopen(path, "w");
    if (!f) {
        if (err && err_len) snprintf(err, err_len, "cannot write %s", path);
        return -1;
    }
    fprintf(f, "{\n  \"model_type\": \"%s\",\n  \"hidden_act\": \"silu\",\n", c->qwen3 ? "qwen3_moe" : "olmoe");
    fprintf(f, "  \"num_hidden_layers\": %zu,\n  \"hidden_size\": %zu,\n", c->n_layers, H);
    if (c->qwen3) fprintf(f, "  \"intermediate_size\": %zu,\n  \"moe_intermediate_size\": %zu,\n", 4 * H, I);
    else fprintf(f, "  \"intermediate_size\": %zu,\n", I);
    fprintf(f, "  \"num_attention_heads\": %zu,\n  \"num_key_value_heads\": %zu,\n  \"head_dim\": %zu,\n", c->n_heads, c->n_kv_heads, hd);
    fprintf(f, "  \"vocab_size\": %zu,\n  \"max_position_embeddings\": %zu,\n", c->vocab, c->max_positions);
    fprintf(f, "  \"num_experts\": %zu,\n  \"num_experts_per_tok\": %zu,\n  \"norm_topk_prob\": %s,\n", E, c->n_experts_used,
            c->renormalize ? "true" : "false");
    fprintf(f, "  \"rms_norm_eps\": %.9g,\n  \"rope_theta\": %.9g,\n  \"tie_word_embeddings\": false\n}\n", (double)c->rms_eps,
            (double)c->rope_theta);
    return fclose(f) == 0 ? 0 : -1;
}
