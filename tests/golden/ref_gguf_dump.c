/*
 * ref_gguf_dump.c - TEST INFRASTRUCTURE: drives the reference's own GGUF
 * reader and loader, compiled from /root/reference (oracle/Makefile target
 * ref, _ref/libvitna_ref.so), on a checkpoint directory, and prints what they
 * produce as JSON:
 *   dir      engine/src/gguf.c:229 vitna_gguf_open: the metadata it reads and
 *            every tensor it lists (name, dtype, shape, data offsets);
 *   model    engine/src/model.c:302 vitna_llama_load_ex(dir, dir/model.gguf):
 *            the config, every matrix's dtype, shape and byte offset in the
 *            data section, each norm's float bits hashed (FNV-1a 64), the
 *            rotary frequencies' bits, ctx and seqs.
 * The GGUF reader's tests compare vitna_hip_gguf_* against this output.
 *
 *   ref_gguf_dump <dir> <ctx> <seqs>
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gguf.h"
#include "model.h"

static unsigned long long fnv(const void* p, size_t n) {
    const unsigned char* b = (const unsigned char*)p;
    unsigned long long h = 1469598103934665603ull;
    for (size_t i = 0; i < n; i++) {
        h ^= b[i];
        h *= 1099511628211ull;
    }
    return h;
}

static const char* base;

static void mat(const char* name, const vitna_matrix_t* m, int comma) {
    printf("    \"%s\": [%d, %zu, %zu, %lld]%s\n", name, (int)m->dtype, m->rows, m->cols,
           m->data ? (long long)((const char*)m->data - base) : -1LL, comma ? "," : "");
}

static void vec(const char* name, const float* v, size_t n, int comma) {
    printf("    \"%s\": [%zu, \"%016llx\"]%s\n", name, n, v ? fnv(v, n * sizeof(float)) : 0ull, comma ? "," : "");
}

int main(int argc, char** argv) {
    if (argc != 4) {
        fprintf(stderr, "usage: %s <dir> <ctx> <seqs>\n", argv[0]);
        return 2;
    }
    char path[1024], err[512];
    snprintf(path, sizeof(path), "%s/model.gguf", argv[1]);
    vitna_safetensors_t st;
    vitna_gguf_info_t info;
    if (!vitna_gguf_open(path, &st, &info, err, sizeof(err))) {
        printf("{\"error\": \"%s\"}\n", err);
        return 1;
    }
    printf("{\n  \"info\": {\"arch\": \"%s\", \"version\": %u, \"alignment\": %llu, \"block_count\": %llu, "
           "\"embedding_length\": %llu, \"feed_forward_length\": %llu, \"expert_feed_forward_length\": %llu, "
           "\"head_count\": %llu, \"head_count_kv\": %llu, \"key_length\": %llu, \"context_length\": %llu, "
           "\"expert_count\": %llu, \"expert_used_count\": %llu, \"rms_eps\": %.17g, \"rope_freq_base\": %.17g, "
           "\"file_tensors\": %zu, \"data_offset\": %llu},\n",
           info.arch, info.version, (unsigned long long)info.alignment, (unsigned long long)info.block_count,
           (unsigned long long)info.embedding_length, (unsigned long long)info.feed_forward_length,
           (unsigned long long)info.expert_feed_forward_length, (unsigned long long)info.head_count,
           (unsigned long long)info.head_count_kv, (unsigned long long)info.key_length, (unsigned long long)info.context_length,
           (unsigned long long)info.expert_count, (unsigned long long)info.expert_used_count, info.rms_eps, info.rope_freq_base,
           info.file_tensors, (unsigned long long)st.data_base_offset);
    printf("  \"tensors\": [\n");
    for (size_t i = 0; i < st.tensor_count; i++) {
        const vitna_tensor_desc_t* t = &st.tensors[i];
        printf("    [\"%s\", %d, %zu, %zu, %zu, %llu, %llu]%s\n", t->name, (int)t->dtype, t->ndim, t->shape[0],
               t->ndim > 1 ? t->shape[1] : 0, (unsigned long long)t->offset_begin, (unsigned long long)t->offset_end,
               i + 1 < st.tensor_count ? "," : "");
    }
    printf("  ],\n");
    vitna_safetensors_close(&st);

    vitna_llama_t m;
    if (!vitna_llama_load_ex(&m, argv[1], path, (size_t)atol(argv[2]), (size_t)atol(argv[3]), err, sizeof(err))) {
        printf("  \"model_error\": \"%s\"\n}\n", err);
        return 1;
    }
    const vitna_llama_config_t* c = &m.cfg;
    base = (const char*)m.shards[0].mmap.data + m.shards[0].data_base_offset;
    printf("  \"model\": {\n");
    printf("    \"cfg\": [%zu, %zu, %zu, %zu, %zu, %zu, %zu, %zu, %.9g, %.9g, %d, %d, %d, %zu, %zu, %d, %d],\n", c->n_layers, c->hidden,
           c->intermediate, c->n_heads, c->n_kv_heads, c->head_dim, c->vocab, c->max_positions, (double)c->rms_eps,
           (double)c->rope_theta, c->tied_embeddings, c->qk_norm, c->qk_norm_per_head, c->n_experts, c->n_experts_used,
           c->renormalize, c->qwen3);
    printf("    \"ctx\": %zu,\n    \"seqs\": %zu,\n", m.ctx, m.seqs);
    mat("embed", &m.embed, 1);
    mat("lm_head", &m.lm_head, 1);
    vec("final_norm", m.final_norm, c->hidden, 1);
    vec("inv_freq", m.inv_freq, c->head_dim / 2, 1);
    char nm[128];
    for (size_t l = 0; l < c->n_layers; l++) {
        const vitna_llama_layer_t* L = &m.layers[l];
        snprintf(nm, sizeof(nm), "%zu.q", l); mat(nm, &L->q, 1);
        snprintf(nm, sizeof(nm), "%zu.k", l); mat(nm, &L->k, 1);
        snprintf(nm, sizeof(nm), "%zu.v", l); mat(nm, &L->v, 1);
        snprintf(nm, sizeof(nm), "%zu.o", l); mat(nm, &L->o, 1);
        snprintf(nm, sizeof(nm), "%zu.router", l); mat(nm, &L->router, 1);
        snprintf(nm, sizeof(nm), "%zu.attn_norm", l); vec(nm, L->attn_norm, c->hidden, 1);
        snprintf(nm, sizeof(nm), "%zu.mlp_norm", l); vec(nm, L->mlp_norm, c->hidden, 1);
        const size_t qn = c->qk_norm_per_head ? c->head_dim : c->n_heads * c->head_dim;
        const size_t kn = c->qk_norm_per_head ? c->head_dim : c->n_kv_heads * c->head_dim;
        snprintf(nm, sizeof(nm), "%zu.q_norm", l); vec(nm, L->q_norm, qn, 1);
        snprintf(nm, sizeof(nm), "%zu.k_norm", l); vec(nm, L->k_norm, kn, 1);
        for (size_t e = 0; e < c->n_experts; e++) {
            snprintf(nm, sizeof(nm), "%zu.%zu.gate", l, e); mat(nm, &L->experts[e].gate, 1);
            snprintf(nm, sizeof(nm), "%zu.%zu.up", l, e); mat(nm, &L->experts[e].up, 1);
            snprintf(nm, sizeof(nm), "%zu.%zu.down", l, e); mat(nm, &L->experts[e].down, 1);
        }
    }
    printf("    \"end\": 0\n  }\n}\n");
    vitna_llama_free(&m);
    return 0;
}
