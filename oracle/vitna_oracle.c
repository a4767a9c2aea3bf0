/**
 * vitna_oracle.c - TEST INFRASTRUCTURE ONLY: the parity checker, never the
 * product path (see vitna_oracle.h).
 *
 * A restatement, from the formulas, of the reference engine's CPU arithmetic
 * for the quantized mixture-of-experts decode path. Built with
 * -ffp-contract=off (oracle/Makefile), so a product is rounded before it is
 * added, exactly where the reference rounds it; fmaf() stands where the
 * reference uses _mm256_fmadd_ps, which rounds once, as fmaf does.
 *
 * Pinning (what checks each function; tests/test_oracle.py):
 *  - widening: the reference's own known answers (engine/tests/unit_tests.c
 *    test_quant), brute force over every byte value of each block field, and
 *    golden vectors written by the compiled reference (tests/golden/);
 *  - matvec, rmsnorm: golden vectors from the compiled reference, plus a
 *    double-precision bound;
 *  - top_k / route: closed-form cases (ties, renormalization order) and the
 *    compiled reference's traced router choice over whole steps;
 *  - moe / step: golden logits of the compiled reference's vitna_llama_step
 *    on seeded synthetic models.
 */

#include "vitna_oracle.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__GNUC__) && !defined(__clang__)
#pragma GCC optimize("fp-contract=off")
#endif

/* engine/src/ops.c:32-54 (vitna_f16_to_f32): exact half to float, subnormals
   normalized. */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, f = h & 0x3ffu, bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (f << 13);
    } else if (e == 0) {
        if (f == 0) {
            bits = sign;
        } else {
            /* value f * 2^-24: shift the leading one up to bit 10 */
            int shift = 0;
            while (!(f & 0x400u)) { f <<= 1; shift++; }
            bits = sign | ((uint32_t)(113 - shift) << 23) | ((f & 0x3ffu) << 13);
        }
    } else {
        bits = sign | ((e + 112u) << 23) | (f << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* engine/src/quant.c:40-44: w = (float)q * d, one rounding. */
void orc_dequant_q8_0(const uint8_t* b, float out[32]) {
    const float d = orc_f16_to_f32(rd16(b));
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)b[2 + i] * d;
}

/* engine/src/quant.c:115-142 (scale_min_k4, vitna_dequant_q4_k): group g of
   32 has a 6-bit scale and min; w = (d*sc)*q - (dmin*mn), each product
   rounded before the subtraction. */
void orc_dequant_q4_k(const uint8_t* b, float out[256]) {
    const float d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
    const uint8_t* s = b + 4;
    for (int g = 0; g < 8; g++) {
        int sc, mn;
        if (g < 4) {
            sc = s[g] & 63;
            mn = s[g + 4] & 63;
        } else {
            sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4);
            mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
        }
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        const uint8_t* q = b + 16 + 32 * (g >> 1);
        for (int l = 0; l < 32; l++) {
            const int v = (g & 1) ? (q[l] >> 4) : (q[l] & 15);
            const float p = d1 * (float)v;
            out[32 * g + l] = p - m1;
        }
    }
}

/* engine/src/quant.c:166-188: weight i = 128h + 32r + l takes its low four
   bits from ql[64h + 32(r&1) + l] (shift 4(r>>1)), its high two from
   qh[32h + l] (shift 2r); w = (d * sc[i/16]) * (q - 32). */
void orc_dequant_q6_k(const uint8_t* b, float out[256]) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = orc_f16_to_f32(rd16(b + 208));
    for (int i = 0; i < 256; i++) {
        const int h = i >> 7, r = (i >> 5) & 3, l = i & 31;
        const int lo = (ql[64 * h + 32 * (r & 1) + l] >> (4 * (r >> 1))) & 15;
        const int hi = (qh[32 * h + l] >> (2 * r)) & 3;
        const float ds = d * (float)sc[i >> 4];
        out[i] = ds * (float)((lo | (hi << 4)) - 32);
    }
}

/* engine/src/ops.c:56-71 (vitna_to_f32) and quant.c:344-377 (vitna_dequant). */
int orc_widen(const void* src, int dtype, float* dst, size_t n) {
    const uint8_t* b = (const uint8_t*)src;
    switch (dtype) {
        case VITNA_DTYPE_F32: memcpy(dst, src, n * 4); return 0;
        case VITNA_DTYPE_F16: for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(rd16(b + 2 * i)); return 0;
        case VITNA_DTYPE_BF16: for (size_t i = 0; i < n; i++) dst[i] = bf16_to_f32(rd16(b + 2 * i)); return 0;
        case VITNA_DTYPE_Q8_0: for (size_t i = 0; i < n; i += 32, b += 34) orc_dequant_q8_0(b, dst + i); return 0;
        case VITNA_DTYPE_Q4_K: for (size_t i = 0; i < n; i += 256, b += 144) orc_dequant_q4_k(b, dst + i); return 0;
        case VITNA_DTYPE_Q6_K: for (size_t i = 0; i < n; i += 256, b += 210) orc_dequant_q6_k(b, dst + i); return 0;
        default: return -1;
    }
}

/* engine/src/ops.c:163-170 (hsum256) applied to a0 + a1: the sixteen chains
   folded as the AVX2 path folds them. */
static float fold16(const float a[16]) {
    float v[8];
    for (int j = 0; j < 8; j++) v[j] = a[j] + a[j + 8];
    const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s2) + (s1 + s3);
}

/* engine/src/ops.c:212-229 (matvec_blocks_avx2) for block formats and
   ops.c:196-209 (matvec_f32_avx2) for F32: sixteen FMA chains over the row,
   folded; F32 rows not a multiple of 16 finish with mul-then-add. F16 takes
   ops.c:95-116's scalar path (vitna_matvec_scalar), a product then a sum per
   weight, in order. */
static void matvec_rows(const void* w, int dtype, const float* x, float* y, size_t r0, size_t r1, size_t cols) {
    const size_t be = vitna_block_elems((vitna_dtype_t)dtype), bb = vitna_block_bytes((vitna_dtype_t)dtype);
    const size_t rb = vitna_matrix_row_bytes((vitna_dtype_t)dtype, cols);
    float buf[256];
    for (size_t r = r0; r < r1; r++) {
        const uint8_t* row = (const uint8_t*)w + r * rb;
        if (dtype == VITNA_DTYPE_F16) {
            float s = 0.0f;
            for (size_t c = 0; c < cols; c++) {
                const float p = orc_f16_to_f32(rd16(row + 2 * c)) * x[c];
                s = s + p;
            }
            y[r] = s;
            continue;
        }
        float a[16] = {0};
        if (dtype == VITNA_DTYPE_F32 || dtype == VITNA_DTYPE_BF16) {
            size_t c = 0;
            for (; c + 16 <= cols; c += 16) {
                orc_widen(row + c * bb, dtype, buf, 16);
                for (int j = 0; j < 16; j++) a[j] = fmaf(buf[j], x[c + j], a[j]);
            }
            float s = fold16(a);
            for (; c < cols; c++) {
                orc_widen(row + c * bb, dtype, buf, 1);
                const float p = buf[0] * x[c];
                s = s + p;
            }
            y[r] = s;
            continue;
        }
        for (size_t c = 0; c < cols; c += be) {
            orc_widen(row + c / be * bb, dtype, buf, be);
            for (size_t i = 0; i < be; i += 16)
                for (int j = 0; j < 16; j++) a[j] = fmaf(buf[i + j], x[c + i + j], a[j]);
        }
        y[r] = fold16(a);
    }
}

static int matvec_ok(int dtype, size_t cols) {
    if (dtype == VITNA_DTYPE_F32 || dtype == VITNA_DTYPE_F16 || dtype == VITNA_DTYPE_BF16) return 1;
    if (dtype == VITNA_DTYPE_Q8_0 || dtype == VITNA_DTYPE_Q4_K || dtype == VITNA_DTYPE_Q6_K)
        return vitna_matrix_row_bytes((vitna_dtype_t)dtype, cols) != 0;
    return 0;
}

int orc_matvec(const void* w, int dtype, const float* x, float* y, size_t rows, size_t cols) {
    if (!matvec_ok(dtype, cols)) return -1;
    matvec_rows(w, dtype, x, y, 0, rows, cols);
    return 0;
}

typedef struct {
    const void* w;
    int dtype;
    const float* x;
    float* y;
    size_t r0, r1, cols;
} mv_job_t;

static void* mv_thread(void* p) {
    mv_job_t* j = (mv_job_t*)p;
    matvec_rows(j->w, j->dtype, j->x, j->y, j->r0, j->r1, j->cols);
    return NULL;
}

int orc_matvec_mt(const void* w, int dtype, const float* x, float* y, size_t rows, size_t cols, int threads) {
    if (!matvec_ok(dtype, cols)) return -1;
    if (threads <= 1 || rows < 64) {
        matvec_rows(w, dtype, x, y, 0, rows, cols);
        return 0;
    }
    if (threads > 256) threads = 256;
    pthread_t th[256];
    mv_job_t jobs[256];
    const size_t per = (rows + (size_t)threads - 1) / (size_t)threads;
    int started = 0;
    for (int t = 0; t < threads; t++) {
        const size_t r0 = (size_t)t * per, r1 = r0 + per < rows ? r0 + per : rows;
        if (r0 >= r1) break;
        jobs[t] = (mv_job_t){w, dtype, x, y, r0, r1, cols};
        if (pthread_create(&th[t], NULL, mv_thread, &jobs[t]) != 0) {
            matvec_rows(w, dtype, x, y, r0, r1, cols);
            jobs[t].y = NULL;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; t++)
        if (jobs[t].y) pthread_join(th[t], NULL);
    return 0;
}

/* engine/src/kernels.c:115-160 (vitna_rmsnorm_avx2): sum of squares in the
   AVX2 order (16 chains over 16-steps, a0 + a1, then an 8-wide tail into the
   combined chains, the fold, then a scalar tail), inv = 1 / sqrtf(ss/n + eps),
   y = (x * inv) * w. Safe in place. */
void orc_rmsnorm(const float* x, const float* w, float* y, size_t n, float eps) {
    if (!x || !w || !y || n == 0) return;
    float a[16] = {0};
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++) a[j] = fmaf(x[i + j], x[i + j], a[j]);
    float v[8];
    for (int j = 0; j < 8; j++) v[j] = a[j] + a[j + 8];
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) v[j] = fmaf(x[i + j], x[i + j], v[j]);
    const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    float ss = (s0 + s2) + (s1 + s3);
    for (; i < n; i++) {
        const float p = x[i] * x[i];
        ss = ss + p;
    }
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t k = 0; k < n; k++) {
        const float t = x[k] * inv;
        y[k] = t * w[k];
    }
}

/* engine/src/ops.c:283-288: (g / (1 + expf(-g))) * u, libm expf. */
void orc_silu_mul(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float g = gate[i];
        const float den = 1.0f + expf(-g);
        const float s = g / den;
        out[i] = s * up[i];
    }
}

/* engine/src/ops.c:273-281: half-split rotary pairs (j, j + half). */
void orc_rope_half(float* v, size_t hd, const float* c, const float* s) {
    const size_t half = hd / 2;
    for (size_t j = 0; j < half; j++) {
        const float a = v[j], b = v[j + half];
        const float ac = a * c[j], bs = b * s[j], bc = b * c[j], as = a * s[j];
        v[j] = ac - bs;
        v[j + half] = bc + as;
    }
}

/* engine/src/model.c:626-637: k passes of argmax over the experts not yet
   taken, strict >, so the lower index wins between equals. */
void orc_top_k(const float* logits, size_t n, size_t k, int32_t* out) {
    for (size_t i = 0; i < k; i++) {
        int32_t best = -1;
        for (size_t e = 0; e < n; e++) {
            int taken = 0;
            for (size_t j = 0; j < i; j++) taken |= out[j] == (int32_t)e;
            if (taken) continue;
            if (best < 0 || logits[e] > logits[best]) best = (int32_t)e;
        }
        out[i] = best;
    }
}

/* engine/src/model.c:667-703 (route): top-k; the chosen experts sorted by id
   into order; softmax over every expert in float32 (max, then the sum of
   expf(l - max) in index order); weight k = expf(l - max) / sum; with
   renormalize, each weight divided by the weights' total, summed largest
   first. */
void orc_route(const float* logits, size_t E, size_t K, bool renormalize, int32_t* chosen, int32_t* order, float* weights) {
    orc_top_k(logits, E, K, chosen);
    memcpy(order, chosen, K * sizeof(int32_t));
    for (size_t i = 1; i < K; i++) {
        const int32_t e = order[i];
        size_t j = i;
        while (j > 0 && order[j - 1] > e) { order[j] = order[j - 1]; j--; }
        order[j] = e;
    }
    float mx = logits[0];
    for (size_t e = 1; e < E; e++)
        if (logits[e] > mx) mx = logits[e];
    float sum = 0.0f;
    for (size_t e = 0; e < E; e++) sum += expf(logits[e] - mx);
    for (size_t k = 0; k < K; k++) weights[k] = expf(logits[order[k]] - mx) / sum;
    if (renormalize) {
        float share[VITNA_EXPERTS_USED_MAX];
        memcpy(share, weights, K * sizeof(float));
        for (size_t i = 1; i < K; i++) {
            const float s = share[i];
            size_t j = i;
            while (j > 0 && share[j - 1] < s) { share[j] = share[j - 1]; j--; }
            share[j] = s;
        }
        float total = 0.0f;
        for (size_t k = 0; k < K; k++) total += share[k];
        for (size_t k = 0; k < K; k++) weights[k] /= total;
    }
}

/* engine/src/model.c:723-764 (mixture_of_experts): router logits, route, and
   for each expert in order of id: gate, up, silu*up, down, then
   proj[i] = proj[i] + out[i]*w from zeros. */
int orc_moe(const vitna_llama_t* m, size_t l, const float* xn, float* logits, int32_t* chosen, int32_t* order, float* weights,
            float* proj, int threads) {
    const vitna_llama_config_t* c = &m->cfg;
    const vitna_llama_layer_t* L = &m->layers[l];
    const size_t E = c->n_experts, K = c->n_experts_used, H = c->hidden, I = c->intermediate;
    if (orc_matvec_mt(L->router.data, L->router.dtype, xn, logits, L->router.rows, L->router.cols, threads)) return -1;
    orc_route(logits, E, K, c->renormalize, chosen, order, weights);
    float* g = (float*)malloc(I * sizeof(float));
    float* u = (float*)malloc(I * sizeof(float));
    float* y = (float*)malloc(H * sizeof(float));
    if (!g || !u || !y) { free(g); free(u); free(y); return -1; }
    memset(proj, 0, H * sizeof(float));
    int rc = 0;
    for (size_t k = 0; k < K && !rc; k++) {
        const vitna_expert_t* x = &L->experts[order[k]];
        rc |= orc_matvec_mt(x->gate.data, x->gate.dtype, xn, g, x->gate.rows, x->gate.cols, threads);
        rc |= orc_matvec_mt(x->up.data, x->up.dtype, xn, u, x->up.rows, x->up.cols, threads);
        orc_silu_mul(g, u, g, I);
        rc |= orc_matvec_mt(x->down.data, x->down.dtype, g, y, x->down.rows, x->down.cols, threads);
        const float w = weights[k];
        for (size_t i = 0; i < H; i++) {
            const float scaled = y[i] * w;
            proj[i] = proj[i] + scaled;
        }
    }
    free(g);
    free(u);
    free(y);
    return rc;
}

/* engine/src/model.c:866-980 (vitna_llama_step, CPU branch). */
int orc_step(vitna_llama_t* m, size_t seq, int32_t token, size_t pos, float* logits, float* trace_logits, int32_t* trace_chosen,
             float* resid, int threads) {
    const vitna_llama_config_t* c = &m->cfg;
    const size_t H = c->hidden, hd = c->head_dim, half = hd / 2, E = c->n_experts, K = c->n_experts_used;
    const size_t kv_dim = c->n_kv_heads * hd, group = c->n_heads / c->n_kv_heads;
    if (seq >= m->seqs || pos >= m->ctx || token < 0 || (size_t)token >= c->vocab) return -1;
    const float scale = 1.0f / sqrtf((float)hd);
    float *x = m->x, *xn = m->xn;
    const size_t erb = vitna_matrix_row_bytes(m->embed.dtype, H);
    if (!erb || orc_widen((const uint8_t*)m->embed.data + (size_t)token * erb, m->embed.dtype, x, H)) return -1;
    for (size_t j = 0; j < half; j++) {
        const float angle = (float)pos * m->inv_freq[j];
        m->cos_t[j] = cosf(angle);
        m->sin_t[j] = sinf(angle);
    }
    float lg[512];
    int32_t ch[VITNA_EXPERTS_USED_MAX], ord[VITNA_EXPERTS_USED_MAX];
    float wts[VITNA_EXPERTS_USED_MAX];
    if (E > 512) return -1;
    for (size_t l = 0; l < c->n_layers; l++) {
        const vitna_llama_layer_t* L = &m->layers[l];
        float* kc = m->k_cache + (seq * c->n_layers + l) * m->ctx * kv_dim;
        float* vc = m->v_cache + (seq * c->n_layers + l) * m->ctx * kv_dim;
        orc_rmsnorm(x, L->attn_norm, xn, H, c->rms_eps);
        if (orc_matvec_mt(L->q.data, L->q.dtype, xn, m->q, L->q.rows, L->q.cols, threads) ||
            orc_matvec_mt(L->k.data, L->k.dtype, xn, m->k, L->k.rows, L->k.cols, threads) ||
            orc_matvec_mt(L->v.data, L->v.dtype, xn, m->v, L->v.rows, L->v.cols, threads))
            return -1;
        if (c->qk_norm && c->qk_norm_per_head) {
            for (size_t h = 0; h < c->n_heads; h++) orc_rmsnorm(m->q + h * hd, L->q_norm, m->q + h * hd, hd, c->rms_eps);
            for (size_t h = 0; h < c->n_kv_heads; h++) orc_rmsnorm(m->k + h * hd, L->k_norm, m->k + h * hd, hd, c->rms_eps);
        } else if (c->qk_norm) {
            orc_rmsnorm(m->q, L->q_norm, m->q, L->q.rows, c->rms_eps);
            orc_rmsnorm(m->k, L->k_norm, m->k, L->k.rows, c->rms_eps);
        }
        for (size_t h = 0; h < c->n_heads; h++) orc_rope_half(m->q + h * hd, hd, m->cos_t, m->sin_t);
        for (size_t h = 0; h < c->n_kv_heads; h++) orc_rope_half(m->k + h * hd, hd, m->cos_t, m->sin_t);
        memcpy(kc + pos * kv_dim, m->k, kv_dim * sizeof(float));
        memcpy(vc + pos * kv_dim, m->v, kv_dim * sizeof(float));
        for (size_t h = 0; h < c->n_heads; h++) {
            const float* qh = m->q + h * hd;
            const size_t kvh = h / group;
            float mx = -INFINITY;
            for (size_t t = 0; t <= pos; t++) {
                const float* kt = kc + t * kv_dim + kvh * hd;
                float s = 0.0f;
                for (size_t d = 0; d < hd; d++) {
                    const float p = qh[d] * kt[d];
                    s = s + p;
                }
                s *= scale;
                m->scores[t] = s;
                if (s > mx) mx = s;
            }
            float sum = 0.0f;
            for (size_t t = 0; t <= pos; t++) {
                m->scores[t] = expf(m->scores[t] - mx);
                sum += m->scores[t];
            }
            const float inv = 1.0f / sum;
            float* out = m->att + h * hd;
            memset(out, 0, hd * sizeof(float));
            for (size_t t = 0; t <= pos; t++) {
                const float p = m->scores[t] * inv;
                const float* vt = vc + t * kv_dim + kvh * hd;
                for (size_t d = 0; d < hd; d++) {
                    const float pv = p * vt[d];
                    out[d] = out[d] + pv;
                }
            }
        }
        if (orc_matvec_mt(L->o.data, L->o.dtype, m->att, m->proj, L->o.rows, L->o.cols, threads)) return -1;
        for (size_t i = 0; i < H; i++) x[i] = x[i] + m->proj[i];
        orc_rmsnorm(x, L->mlp_norm, xn, H, c->rms_eps);
        if (orc_moe(m, l, xn, lg, ch, ord, wts, m->proj, threads)) return -1;
        if (trace_logits) memcpy(trace_logits + l * E, lg, E * sizeof(float));
        if (trace_chosen) memcpy(trace_chosen + l * K, ch, K * sizeof(int32_t));
        for (size_t i = 0; i < H; i++) x[i] = x[i] + m->proj[i];
        if (resid) memcpy(resid + l * H, x, H * sizeof(float));
    }
    if (logits) {
        orc_rmsnorm(x, m->final_norm, xn, H, c->rms_eps);
        if (orc_matvec_mt(m->lm_head.data, m->lm_head.dtype, xn, logits, m->lm_head.rows, m->lm_head.cols, threads)) return -1;
    }
    return 0;
}
