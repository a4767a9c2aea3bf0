/**
 * kernels_attn.hip - Decode attention over the float32 key-value cache, for
 * one or many rows (tokens of possibly different sequences at their own
 * positions), with Qwen3's per-head QK RMSNorm and the half-split RoPE.
 *
 * Reference counterparts: qk_head_norm_rope_kernel model_cuda.cu:1514 and
 * attention_kernel model_cuda.cu:942 (split-K, last block merges); the CPU
 * arithmetic it is checked against is engine/src/model.c:909-957.
 *
 * Layout: the cache of a layer holds, for every sequence, ctx positions of
 * n_kv * hd floats (one position's heads back to back), as the reference's
 * [seq][layer][ctx][kv_dim]. A block takes ATTN_CHUNK positions of one kv
 * head of one row: four waves of 16 positions, four lanes a position in the
 * scores (hd / 4 dimensions a lane), a lane per dimension in the weighted sum
 * of values. Each of the G = n_heads / n_kv query heads sharing the kv head
 * is served by the same reads of the cache. Each block leaves its chunk's
 * (max, sum, weighted values) per query head; attention_merge_kernel, one
 * block per (row, query head), combines the chunks.
 */

#include "vitna_kernels.h"

#define GMAX 8

/* RMSNorm and RoPE of NV vectors of HD in LDS (v[i] at vecs + i * HD): the
   reference's per-head norm (engine/src/model.c:916-921) and vitna_rope_half
   (engine/src/ops.c:273-281). */
template <int HD>
__device__ void norm_rope(float* vecs, int nv, const float* wq, const float* wk, int k_from, float eps, const float* c,
                          const float* s, float* inv_s) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr int PL = HD / 64; /* elements a lane */
    if (wq) {
        /* a wave a vector: the sum of squares across the wave */
        for (int v = wave; v < nv; v += 4) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < PL; i++) {
                const float e = vecs[v * HD + lane + 64 * i];
                ss = fmaf(e, e, ss);
            }
            ss = wave_sum(ss);
            if (lane == 0) inv_s[v] = 1.0f / sqrtf(ss / (float)HD + eps);
        }
        __syncthreads();
        for (int i = tid; i < nv * HD; i += blockDim.x) {
            const int g = i / HD, d = i % HD;
            const float* w = g >= k_from ? wk : wq;
            vecs[i] = (vecs[i] * inv_s[g]) * w[d];
        }
        __syncthreads();
    }
    constexpr int HALF = HD / 2;
    for (int i = tid; i < nv * HALF; i += blockDim.x) {
        const int g = i / HALF, j = i % HALF;
        float* v = vecs + g * HD;
        const float a = v[j], b = v[j + HALF];
        const float ac = a * c[j], bs = b * s[j], bc = b * c[j], as = a * s[j];
        v[j] = ac - bs;
        v[j + HALF] = bc + as;
    }
    __syncthreads();
}

template <int HD>
__global__ __launch_bounds__(256) void attention_kernel(attn_args a) {
    constexpr int DPL = HD / 4;        /* dimensions a lane in the scores */
    constexpr int VPL = HD / 64;       /* dimensions a lane in the values */
    const int split = blockIdx.x, h = blockIdx.y, row = blockIdx.z;
    const row_rec rr = a.rows[row];
    const int pos = rr.pos, seq = rr.seq;
    const int n_act = pos / ATTN_CHUNK + 1;
    if (split >= n_act) return;
    const int G = a.n_heads / a.n_kv, kv_dim = a.n_kv * HD, half = HD / 2;
    float* kc = a.k_cache + (size_t)seq * a.seq_stride;
    float* vc = a.v_cache + (size_t)seq * a.seq_stride;
    __shared__ float sq[(GMAX + 1) * HD]; /* G query heads, then the new key */
    __shared__ float nv[HD];
    __shared__ float inv_s[GMAX + 1];
    __shared__ float sp[4][16][GMAX];
    __shared__ float wm[4][GMAX], wl[4][GMAX];
    __shared__ float wacc[4][GMAX][HD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float* nk = sq + G * HD;

    /* the chunk's keys and values, requested before anything waits on them: four lanes a position (hd / 4 keys
       a lane) and a lane a dimension across the wave's sixteen positions */
    const int p = lane >> 2, qd = lane & 3;
    const int t = split * ATTN_CHUNK + wave * 16 + p;
    const bool valid = t <= pos;
    const bool fresh = !a.prepared && t == pos; /* this row's own key: in LDS once normalized, not in the cache yet */
    float kr[DPL];
    if (valid && !fresh) {
        const float4* src = reinterpret_cast<const float4*>(kc + (size_t)t * kv_dim + (size_t)h * HD + qd * DPL);
#pragma unroll
        for (int i = 0; i < DPL / 4; i++) {
            const float4 u = src[i];
            kr[4 * i] = u.x; kr[4 * i + 1] = u.y; kr[4 * i + 2] = u.z; kr[4 * i + 3] = u.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < DPL; i++) kr[i] = 0.f;
    }
    const int t0 = split * ATTN_CHUNK + wave * 16;
    float vv[16][VPL];
#pragma unroll
    for (int pp = 0; pp < 16; pp++) {
        const int tt = t0 + pp;
        const bool ok = tt <= pos && !(!a.prepared && tt == pos);
        const float* vrow = vc + (size_t)(ok ? tt : 0) * kv_dim + (size_t)h * HD;
#pragma unroll
        for (int i = 0; i < VPL; i++) vv[pp][i] = ok ? vrow[lane + 64 * i] : 0.0f;
    }

    {
        /* the G query heads: G * HD / 4 <= 256 float4, one a thread */
        const float4* q4 = reinterpret_cast<const float4*>(a.q_raw + (size_t)row * a.n_heads * HD + (size_t)h * G * HD);
        if (tid < G * HD / 4) reinterpret_cast<float4*>(sq)[tid] = q4[tid];
    }
    if (a.prepared) {
        __syncthreads();
    } else {
        if (tid < HD) {
            nk[tid] = a.k_raw[(size_t)row * kv_dim + (size_t)h * HD + tid];
            nv[tid] = a.v_raw[(size_t)row * kv_dim + (size_t)h * HD + tid];
        }
        __syncthreads();
        norm_rope<HD>(sq, G + 1, a.q_norm, a.k_norm, G, a.eps, a.cos_tab + (size_t)pos * half, a.sin_tab + (size_t)pos * half, inv_s);
        if (split == n_act - 1 && tid < HD) {
            kc[(size_t)pos * kv_dim + (size_t)h * HD + tid] = nk[tid];
            vc[(size_t)pos * kv_dim + (size_t)h * HD + tid] = nv[tid];
        }
        if (fresh) {
#pragma unroll
            for (int i = 0; i < DPL; i++) kr[i] = nk[qd * DPL + i];
        }
#pragma unroll
        for (int pp = 0; pp < 16; pp++)
            if (t0 + pp == pos) {
#pragma unroll
                for (int i = 0; i < VPL; i++) vv[pp][i] = nv[lane + 64 * i];
            }
    }

    /* scores, and each head's max and sum over the wave's positions */
    const float scale = 1.0f / sqrtf((float)HD);
    float mw[GMAX], lw[GMAX], pe[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; g++) {
        if (g >= G) break;
        const float* qg = sq + g * HD + qd * DPL;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; i++) s = fmaf(qg[i], kr[i], s);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        s *= scale;
        float m = valid ? s : -INFINITY;
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float e = valid ? expf(s - m) : 0.0f;
        float l = e;
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) l += __shfl_xor(l, o, 64);
        mw[g] = m;
        lw[g] = l;
        pe[g] = e;
    }
    if (qd == 0) {
#pragma unroll
        for (int g = 0; g < GMAX; g++)
            if (g < G) sp[wave][p][g] = pe[g];
    }
    __syncthreads();

    /* values: a lane per dimension */
    float acc[GMAX][VPL];
#pragma unroll
    for (int g = 0; g < GMAX; g++)
#pragma unroll
        for (int i = 0; i < VPL; i++) acc[g][i] = 0.f;
#pragma unroll
    for (int pp = 0; pp < 16; pp++) {
#pragma unroll
        for (int g = 0; g < GMAX; g++) {
            if (g >= G) break;
            const float w = sp[wave][pp][g];
#pragma unroll
            for (int i = 0; i < VPL; i++) acc[g][i] = fmaf(w, vv[pp][i], acc[g][i]);
        }
    }
    if (lane == 0) {
        for (int g = 0; g < G; g++) { wm[wave][g] = mw[g]; wl[wave][g] = lw[g]; }
    }
#pragma unroll
    for (int g = 0; g < GMAX; g++) {
        if (g >= G) break;
#pragma unroll
        for (int i = 0; i < VPL; i++) wacc[wave][g][lane + 64 * i] = acc[g][i];
    }
    __syncthreads();

    /* this chunk's partial: the four waves merged */
    float* part = a.partial + (((size_t)row * a.n_kv + h) * a.splits_max + split) * G * (HD + 2);
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        float M = -INFINITY;
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][g]);
        float L = 0.f, o = 0.f;
        for (int w = 0; w < 4; w++) {
            const float f = wm[w][g] == -INFINITY ? 0.0f : expf(wm[w][g] - M);
            L = fmaf(wl[w][g], f, L);
            o = fmaf(wacc[w][g][d], f, o);
        }
        part[g * (HD + 2) + d] = o;
        if (d == 0) {
            part[g * (HD + 2) + HD] = M;
            part[g * (HD + 2) + HD + 1] = L;
        }
    }
}

/* The prepare pass: one block a (row, kv head), its G query heads and its key. */
template <int HD>
__global__ __launch_bounds__(256) void attention_prepare_kernel(attn_args a) {
    const int h = blockIdx.x, row = blockIdx.y;
    const row_rec rr = a.rows[row];
    const int pos = rr.pos, seq = rr.seq;
    const int G = a.n_heads / a.n_kv, kv_dim = a.n_kv * HD, half = HD / 2;
    __shared__ float sq[(GMAX + 1) * HD];
    __shared__ float inv_s[GMAX + 1];
    const int tid = threadIdx.x;
    float* nk = sq + G * HD;
    for (int i = tid; i < G * HD; i += 256) sq[i] = a.q_raw[(size_t)row * a.n_heads * HD + (size_t)h * G * HD + i];
    if (tid < HD) nk[tid] = a.k_raw[(size_t)row * kv_dim + (size_t)h * HD + tid];
    __syncthreads();
    norm_rope<HD>(sq, G + 1, a.q_norm, a.k_norm, G, a.eps, a.cos_tab + (size_t)pos * half, a.sin_tab + (size_t)pos * half, inv_s);
    for (int i = tid; i < G * HD; i += 256) a.q_out[(size_t)row * a.n_heads * HD + (size_t)h * G * HD + i] = sq[i];
    if (tid < HD) {
        float* kc = a.k_cache + (size_t)seq * a.seq_stride;
        float* vc = a.v_cache + (size_t)seq * a.seq_stride;
        kc[(size_t)pos * kv_dim + (size_t)h * HD + tid] = nk[tid];
        vc[(size_t)pos * kv_dim + (size_t)h * HD + tid] = a.v_raw[(size_t)row * kv_dim + (size_t)h * HD + tid];
    }
}


hipError_t launch_attention(const attn_args& a, hipStream_t s) {
    if (a.n_kv < 1 || a.n_heads % a.n_kv || a.n_heads / a.n_kv > GMAX || a.n_rows < 1) return hipErrorInvalidValue;
    if (a.splits_max * ATTN_CHUNK < a.ctx) return hipErrorInvalidValue;
    const dim3 grid(a.splits_max, a.n_kv, a.n_rows);
    if (a.hd == 128) attention_kernel<128><<<grid, 256, 0, s>>>(a);
    else if (a.hd == 64) attention_kernel<64><<<grid, 256, 0, s>>>(a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}


/* One block per (query head, row), a thread per dimension: the chunks'
   maxima and sums read in parallel, each chunk's scale exp(m_s - M) computed
   once, then each dimension's weighted values summed, eight chunks' loads in
   flight at a time. */
#define MERGE_MAX 256
__global__ void attention_merge_kernel(attn_args a) {
    const int hq = blockIdx.x, row = blockIdx.y, d = threadIdx.x;
    const int G = a.n_heads / a.n_kv, h = hq / G, g = hq % G, HD = a.hd;
    const int n_act = a.rows[row].pos / ATTN_CHUNK + 1;
    const float* base = a.partial + (((size_t)row * a.n_kv + h) * a.splits_max * G + g) * (HD + 2);
    const size_t stride = (size_t)G * (HD + 2);
    __shared__ float fm[MERGE_MAX], fl[MERGE_MAX];
    __shared__ float red[4];
    float m = -INFINITY;
    for (int s = d; s < n_act; s += blockDim.x) {
        fm[s] = base[s * stride + HD];
        fl[s] = base[s * stride + HD + 1];
        m = fmaxf(m, fm[s]);
    }
    m = wave_max(m);
    if ((d & 63) == 0) red[d >> 6] = m;
    __syncthreads();
    float M = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) M = fmaxf(M, red[w]);
    for (int s = d; s < n_act; s += blockDim.x) fm[s] = expf(fm[s] - M);
    __syncthreads();
    float L = 0.f, o = 0.f;
    int s = 0;
    for (; s + 8 <= n_act; s += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = base[(s + i) * stride + d];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            L = fmaf(fl[s + i], fm[s + i], L);
            o = fmaf(v[i], fm[s + i], o);
        }
    }
    for (; s < n_act; s++) {
        L = fmaf(fl[s], fm[s], L);
        o = fmaf(base[s * stride + d], fm[s], o);
    }
    a.att[(size_t)row * a.n_heads * HD + (size_t)hq * HD + d] = o / L;
}

hipError_t launch_attention_merge(const attn_args& a, hipStream_t s) {
    if (a.n_kv < 1 || a.n_heads % a.n_kv || a.n_rows < 1 || (a.hd != 64 && a.hd != 128) || a.splits_max > MERGE_MAX)
        return hipErrorInvalidValue;
    attention_merge_kernel<<<dim3(a.n_heads, a.n_rows), a.hd, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_attention_prepare(const attn_args& a, hipStream_t s) {
    if (a.n_kv < 1 || a.n_heads % a.n_kv || a.n_heads / a.n_kv > GMAX || a.n_rows < 1 || !a.q_out) return hipErrorInvalidValue;
    const dim3 grid(a.n_kv, a.n_rows);
    if (a.hd == 128) attention_prepare_kernel<128><<<grid, 256, 0, s>>>(a);
    else if (a.hd == 64) attention_prepare_kernel<64><<<grid, 256, 0, s>>>(a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}
