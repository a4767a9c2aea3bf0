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
#include "skinny_image.h"

#define GMAX 8

/* Sum over the lanes of one head's float4 group (HD / 4 consecutive lanes: a
   32-lane half for HD 128, a 16-lane row for HD 64), in every lane of it. */
template <int HD>
__device__ __forceinline__ float head_sum(float v) {
    if constexpr (HD == 128) {
        return half_sum_dpp(v);
    } else {
        v = row_scan_sum(v);
        const int r = (threadIdx.x >> 4) & 3;
        const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
        const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
        const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47));
        const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
        return r == 0 ? r0 : r == 1 ? r1 : r == 2 ? r2 : r3;
    }
}

/* The float4 of the RoPE partner (dimensions +- HD / 2) of this lane's float4. */
template <int HD>
__device__ __forceinline__ float4 rope_partner(float4 v) {
    float4 o;
    if constexpr (HD == 128) {
        o.x = swap16(v.x); o.y = swap16(v.y); o.z = swap16(v.z); o.w = swap16(v.w);
    } else { /* row_ror:8 within a 16-lane row swaps its halves */
        o.x = dpp_f<0x128, 0xf, 0xf>(v.x, 0.0f); o.y = dpp_f<0x128, 0xf, 0xf>(v.y, 0.0f);
        o.z = dpp_f<0x128, 0xf, 0xf>(v.z, 0.0f); o.w = dpp_f<0x128, 0xf, 0xf>(v.w, 0.0f);
    }
    return o;
}

/* The reference's per-head RMSNorm (engine/src/model.c:916-921) and
   vitna_rope_half (engine/src/ops.c:273-281) of one head's vector, held as
   float4 j of the head by HD / 4 consecutive lanes; every lane of the wave
   takes part (lanes outside a head pass zeros). */
template <int HD>
__device__ __forceinline__ float4 head_norm_rope(float4 v, int j, const float* w, float eps, const float* c, const float* s) {
    constexpr int QF4 = HD / 4, HALF = HD / 2;
    float ss = 0.0f;
    ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss); ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
    ss = head_sum<HD>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
    const float4 wv = reinterpret_cast<const float4*>(w)[j];
    v.x = (v.x * inv) * wv.x; v.y = (v.y * inv) * wv.y; v.z = (v.z * inv) * wv.z; v.w = (v.w * inv) * wv.w;
    const float4 pv = rope_partner<HD>(v);
    const bool first = j < QF4 / 2;
    const int d0 = 4 * (first ? j : j - QF4 / 2);
    const float4 cv = reinterpret_cast<const float4*>(c + d0)[0], sv = reinterpret_cast<const float4*>(s + d0)[0];
    (void)HALF;
    float4 o;
    if (first) { /* a = own, b = partner: a c - b s */
        o.x = v.x * cv.x - pv.x * sv.x; o.y = v.y * cv.y - pv.y * sv.y;
        o.z = v.z * cv.z - pv.z * sv.z; o.w = v.w * cv.w - pv.w * sv.w;
    } else { /* b = own, a = partner: b c + a s */
        o.x = v.x * cv.x + pv.x * sv.x; o.y = v.y * cv.y + pv.y * sv.y;
        o.z = v.z * cv.z + pv.z * sv.z; o.w = v.w * cv.w + pv.w * sv.w;
    }
    return o;
}

template <int HD, int G>
__global__ __launch_bounds__(256) void attention_kernel(attn_args a) {
    constexpr int DPL = HD / 4;  /* dimensions a lane in the scores */
    constexpr int VPL = HD / 64; /* dimensions a lane in the values */
    constexpr int QF4 = HD / 4;  /* float4 of a head */
    constexpr int PS = HD + 4;   /* floats of a (chunk, query head) partial */
    /* blocks go to the eight XCDs in turn by their linear index; the chunk a block takes is rotated by its
       (head, row) so that the leftover chunks of ragged rows do not all fall on the first XCDs */
    const int split = (int)((blockIdx.x + blockIdx.y + gridDim.y * blockIdx.z) % gridDim.x);
    const int h = blockIdx.y, row = blockIdx.z;
    const row_rec rr = a.rows[row];
    const int pos = rr.pos, seq = rr.seq;
    const int n_act = pos / ATTN_CHUNK + 1;
    if (split >= n_act) return;
    const int kv_dim = a.n_kv * HD, half = HD / 2;
    float* kc = a.k_cache + (size_t)seq * a.seq_stride;
    float* vc = a.v_cache + (size_t)seq * a.seq_stride;
    __shared__ __attribute__((aligned(16))) float sq[GMAX * HD]; /* the G query heads, normalized */
    __shared__ __attribute__((aligned(16))) float nk[HD];        /* this row's own key, normalized */
    __shared__ __attribute__((aligned(16))) float nvs[HD];       /* and value */
    __shared__ __attribute__((aligned(16))) float sp[4][16][GMAX];
    __shared__ float wm[4][GMAX], wl[4][GMAX];
    __shared__ __attribute__((aligned(16))) float wacc[4][GMAX][HD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const bool fresh_block = !a.prepared && split == n_act - 1; /* holds the row's own position */

    /* the chunk's keys and values, requested before anything waits on them: four lanes a position (hd / 4 keys
       a lane) and a lane a dimension across the wave's sixteen positions */
    const int p = lane >> 2, qd = lane & 3;
    const int t = split * ATTN_CHUNK + wave * 16 + p;
    const bool valid = t <= pos;
    const bool fresh = fresh_block && t == pos; /* this row's own key: in LDS once normalized, not in the cache yet */
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
    if (t0 + 15 < pos) { /* the wave's sixteen positions all before the row's own: no checks */
        const float* vrow = vc + (size_t)t0 * kv_dim + (size_t)h * HD + lane;
#pragma unroll
        for (int pp = 0; pp < 16; pp++)
#pragma unroll
            for (int i = 0; i < VPL; i++) vv[pp][i] = vrow[(size_t)pp * kv_dim + 64 * i];
    } else {
#pragma unroll
        for (int pp = 0; pp < 16; pp++) {
            const int tt = t0 + pp;
            const bool ok = tt <= pos && !(fresh_block && tt == pos);
            const float* vrow = vc + (size_t)(ok ? tt : 0) * kv_dim + (size_t)h * HD;
#pragma unroll
            for (int i = 0; i < VPL; i++) vv[pp][i] = ok ? vrow[lane + 64 * i] : 0.0f;
        }
    }

    /* the G query heads: thread tid holds float4 j of head g */
    {
        const int g = tid / QF4, j = tid % QF4;
        const bool qt = g < G;
        float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (qt) qv = reinterpret_cast<const float4*>(a.q_raw + (size_t)row * a.n_heads * HD + (size_t)(h * G + g) * HD)[j];
        if (!a.prepared) {
            const float* cs = a.cos_tab + (size_t)pos * half;
            const float* sn = a.sin_tab + (size_t)pos * half;
            if (g < GMAX) qv = head_norm_rope<HD>(qv, j, a.q_norm, a.eps, cs, sn);
            /* this row's own key and value, in the block that holds its position */
            if (fresh_block && wave == 0) {
                float4 kv4 = make_float4(0.f, 0.f, 0.f, 0.f);
                if (lane < QF4) kv4 = reinterpret_cast<const float4*>(a.k_raw + (size_t)row * kv_dim + (size_t)h * HD)[lane];
                kv4 = head_norm_rope<HD>(kv4, lane % QF4, a.k_norm, a.eps, cs, sn);
                if (lane < QF4) {
                    const float4 vn = reinterpret_cast<const float4*>(a.v_raw + (size_t)row * kv_dim + (size_t)h * HD)[lane];
                    reinterpret_cast<float4*>(nk)[lane] = kv4;
                    reinterpret_cast<float4*>(nvs)[lane] = vn;
                    reinterpret_cast<float4*>(kc + (size_t)pos * kv_dim + (size_t)h * HD)[lane] = kv4;
                    reinterpret_cast<float4*>(vc + (size_t)pos * kv_dim + (size_t)h * HD)[lane] = vn;
                }
            }
        }
        if (qt) reinterpret_cast<float4*>(sq)[tid] = qv;
    }
    __syncthreads();
    if (fresh) {
#pragma unroll
        for (int i = 0; i < DPL; i++) kr[i] = nk[qd * DPL + i];
    }
    if (fresh_block) {
#pragma unroll
        for (int pp = 0; pp < 16; pp++)
            if (t0 + pp == pos) {
#pragma unroll
                for (int i = 0; i < VPL; i++) vv[pp][i] = nvs[lane + 64 * i];
            }
    }

    /* scores, and each head's max and sum over the wave's positions; the G heads side by side, so their
       cross-lane steps interleave */
    const float scale = 1.0f / sqrtf((float)HD);
    float sc[G], mw[G], lw[G], pe[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float4* qg = reinterpret_cast<const float4*>(sq + g * HD + qd * DPL);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < DPL / 4; i++) {
            const float4 q4 = qg[i];
            acc = fmaf(q4.x, kr[4 * i], acc);
            acc = fmaf(q4.y, kr[4 * i + 1], acc);
            acc = fmaf(q4.z, kr[4 * i + 2], acc);
            acc = fmaf(q4.w, kr[4 * i + 3], acc);
        }
        sc[g] = acc;
    }
#pragma unroll
    for (int g = 0; g < G; g++) sc[g] = quad_sum(sc[g]) * scale;
#pragma unroll
    for (int g = 0; g < G; g++) mw[g] = wave_max_dpp(valid ? sc[g] : -INFINITY);
#pragma unroll
    for (int g = 0; g < G; g++) pe[g] = valid ? __expf(sc[g] - mw[g]) : 0.0f;
#pragma unroll
    for (int g = 0; g < G; g++) lw[g] = wave_sum_dpp(qd == 0 ? pe[g] : 0.0f);
    if (qd == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) sp[wave][p][g] = pe[g];
    }
    /* sp[wave] is this wave's own: LDS operations of one wave complete in order */
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");

    /* values: a lane per dimension */
    float acc[G][VPL];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < VPL; i++) acc[g][i] = 0.f;
#pragma unroll
    for (int pp = 0; pp < 16; pp++) {
        const float4 w0 = *reinterpret_cast<const float4*>(&sp[wave][pp][0]);
        const float4 w1 = *reinterpret_cast<const float4*>(&sp[wave][pp][4]);
        const float w[GMAX] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < VPL; i++) acc[g][i] = fmaf(w[g], vv[pp][i], acc[g][i]);
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) { wm[wave][g] = mw[g]; wl[wave][g] = lw[g]; }
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < VPL; i++) wacc[wave][g][lane + 64 * i] = acc[g][i];
    __syncthreads();

    /* this chunk's partial: the four waves merged, a float4 of one head a thread */
    {
        const int g = tid / QF4, j = tid % QF4;
        if (g < G) {
            float* part = a.partial + (((size_t)row * a.n_kv + h) * a.splits_max + split) * G * PS + (size_t)g * PS;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][g]);
            float L = 0.f;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float f = wm[w][g] == -INFINITY ? 0.0f : expf(wm[w][g] - M);
                const float4 x = reinterpret_cast<const float4*>(&wacc[w][g][0])[j];
                L = fmaf(wl[w][g], f, L);
                o.x = fmaf(x.x, f, o.x); o.y = fmaf(x.y, f, o.y); o.z = fmaf(x.z, f, o.z); o.w = fmaf(x.w, f, o.w);
            }
            reinterpret_cast<float4*>(part)[j] = o;
            if (j == 0) {
                part[HD] = M;
                part[HD + 1] = L;
            }
        }
    }
}

/* The prepare pass: one block a (row, kv head), its G query heads and its key, each through head_norm_rope with
   the lanes the attention kernels give it (thread t: float4 t % (HD / 4) of head t / (HD / 4); wave 0 the key), so
   that the prepared queries and the stored key are the bits those kernels compute for themselves (a pass of rows
   then gives each row what a step of that row alone gives). */
template <int HD>
__global__ __launch_bounds__(256) void attention_prepare_kernel(attn_args a) {
    constexpr int QF4 = HD / 4;
    const int h = blockIdx.x, row = blockIdx.y;
    const row_rec rr = a.rows[row];
    const int pos = rr.pos, seq = rr.seq;
    const int G = a.n_heads / a.n_kv, kv_dim = a.n_kv * HD, half = HD / 2;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float* cs = a.cos_tab + (size_t)pos * half;
    const float* sn = a.sin_tab + (size_t)pos * half;
    {
        const int g = tid / QF4, j = tid % QF4;
        const size_t at = (size_t)row * a.n_heads * HD + (size_t)(h * G + g) * HD;
        float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (g < G) qv = reinterpret_cast<const float4*>(a.q_raw + at)[j];
        if (g < GMAX) qv = head_norm_rope<HD>(qv, j, a.q_norm, a.eps, cs, sn);
        if (g < G) reinterpret_cast<float4*>(a.q_out + at)[j] = qv;
    }
    if (wave == 0) {
        float4 kv4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (lane < QF4) kv4 = reinterpret_cast<const float4*>(a.k_raw + (size_t)row * kv_dim + (size_t)h * HD)[lane];
        kv4 = head_norm_rope<HD>(kv4, lane % QF4, a.k_norm, a.eps, cs, sn);
        if (lane < QF4) {
            float* kc = a.k_cache + (size_t)seq * a.seq_stride;
            float* vc = a.v_cache + (size_t)seq * a.seq_stride;
            const float4 vn = reinterpret_cast<const float4*>(a.v_raw + (size_t)row * kv_dim + (size_t)h * HD)[lane];
            reinterpret_cast<float4*>(kc + (size_t)pos * kv_dim + (size_t)h * HD)[lane] = kv4;
            reinterpret_cast<float4*>(vc + (size_t)pos * kv_dim + (size_t)h * HD)[lane] = vn;
        }
    }
}


/* ---- the same attention on the matrix cores (head dimension 128, up to 8 query heads a kv head) ----
   The VALU kernel above spends most of its instructions on the products' reductions and addressing; here
   both products run on v_mfma_f32_16x16x4_f32, fp32 operands and products, fp32 accumulate. Per wave, its
   16 positions of the chunk:
     scores  S[16 positions][16 heads] = K . Q^T: step (t, m) takes dimension 32 t + 8 (l / 16) + m of
             position l % 16 (A) and of head l % 16 (B, zero past G); four chunk sums t < 4, added; lane l
             holds S[4 (l / 16) + r][l % 16];
     softmax per head over the wave's positions: a lane's four, then lanes l ^ 16, l ^ 32;
     values  O[16 heads][128] = P . V, eight tiles of 16 columns: step r takes position 4 (l / 16) + r, so A
             is the lane's own weight P[r] of head l % 16, and B its value of that position at dimension
             VDIM(j, l % 16) (the column-to-dimension map that makes a lane's loads two float4s a position);
             O lands in lanes l / 16 < 2 (heads 0..7).
   The cache reads (546 MB a layer at config 3) run at about 5.0 TB/s, near what this HBM streams (a copy
   runs at 5.1 TB/s), so the kernel is bound by them. The partial per (chunk, head) is the VALU kernel's,
   so the same merge follows. */
typedef float at_f4 __attribute__((ext_vector_type(4)));

#define ATTN_MMA_OCC 4 /* waves a SIMD: the kernel is held to 128 registers */
template <int G>
__global__ __launch_bounds__(256, ATTN_MMA_OCC) void attention_mma_kernel(attn_args a) {
    constexpr int HD = 128, QF4 = HD / 4, PS = HD + 4;
    /* blocks go to the eight XCDs in turn by their linear index; the chunk a block takes is rotated by its
       (head, row) so that the leftover chunks of ragged rows do not all fall on the first XCDs */
    const int split = (int)((blockIdx.x + blockIdx.y + gridDim.y * blockIdx.z) % gridDim.x);
    const int h = blockIdx.y, row = blockIdx.z;
    const row_rec rr = a.rows[row];
    const int pos = rr.pos, seq = rr.seq;
    const int n_act = pos / ATTN_CHUNK + 1;
    if (split >= n_act) return;
    const int kv_dim = a.n_kv * HD, half = HD / 2;
    float* kc = a.k_cache + (size_t)seq * a.seq_stride;
    float* vc = a.v_cache + (size_t)seq * a.seq_stride;
    __shared__ __attribute__((aligned(16))) float sq[GMAX * HD]; /* the G query heads, normalized, scaled */
    __shared__ __attribute__((aligned(16))) float nk[HD];
    __shared__ __attribute__((aligned(16))) float nvs[HD];
    __shared__ float wm[4][GMAX], wl[4][GMAX];
    __shared__ __attribute__((aligned(16))) float wacc[4][GMAX][HD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c16 = lane & 15, kq = lane >> 4;
    const bool fresh_block = !a.prepared && split == n_act - 1;
    const int t0 = split * ATTN_CHUNK + wave * 16;

    /* keys: position t0 + c16, dimensions 32 t + 8 kq .. + 7 */
    const int tk = t0 + c16;
    const bool kvalid = tk <= pos, kfresh = fresh_block && tk == pos;
    float4 kr[8];
    if (kvalid && !kfresh) {
        const float4* src = reinterpret_cast<const float4*>(kc + (size_t)tk * kv_dim + (size_t)h * HD + 8 * kq);
#pragma unroll
        for (int t = 0; t < 4; t++) { kr[2 * t] = src[8 * t]; kr[2 * t + 1] = src[8 * t + 1]; }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) kr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    /* values of positions t0 + 4 kq + i: column c16 of output tile j is dimension VDIM(j, c16), so a lane's
       dimensions of a position are two float4s and a wave's load reads whole lines (the columns of an MFMA
       are independent: which dimension each one carries is free) */
#define VDIM(j, c) (64 * ((j) >> 2) + 4 * (c) + ((j) & 3))
    float vv[8][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int tt = t0 + 4 * kq + i;
        const bool ok = tt <= pos && !(fresh_block && tt == pos);
        const float4* vrow = reinterpret_cast<const float4*>(vc + (size_t)(ok ? tt : 0) * kv_dim + (size_t)h * HD + 4 * c16);
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float4 f = ok ? vrow[16 * hh] : make_float4(0.f, 0.f, 0.f, 0.f);
            vv[4 * hh][i] = f.x;
            vv[4 * hh + 1][i] = f.y;
            vv[4 * hh + 2][i] = f.z;
            vv[4 * hh + 3][i] = f.w;
        }
    }

    /* the G query heads (normalized, rotated, scaled by 1 / sqrt(hd)); this row's own key and value */
    {
        const int g = tid / QF4, j = tid % QF4;
        const bool qt = g < G;
        float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (qt) qv = reinterpret_cast<const float4*>(a.q_raw + (size_t)row * a.n_heads * HD + (size_t)(h * G + g) * HD)[j];
        if (!a.prepared) {
            const float* cs = a.cos_tab + (size_t)pos * half;
            const float* sn = a.sin_tab + (size_t)pos * half;
            if (g < GMAX) qv = head_norm_rope<HD>(qv, j, a.q_norm, a.eps, cs, sn);
            if (fresh_block && wave == 0) {
                float4 kv4 = make_float4(0.f, 0.f, 0.f, 0.f);
                if (lane < QF4) kv4 = reinterpret_cast<const float4*>(a.k_raw + (size_t)row * kv_dim + (size_t)h * HD)[lane];
                kv4 = head_norm_rope<HD>(kv4, lane % QF4, a.k_norm, a.eps, cs, sn);
                if (lane < QF4) {
                    const float4 vn = reinterpret_cast<const float4*>(a.v_raw + (size_t)row * kv_dim + (size_t)h * HD)[lane];
                    reinterpret_cast<float4*>(nk)[lane] = kv4;
                    reinterpret_cast<float4*>(nvs)[lane] = vn;
                    reinterpret_cast<float4*>(kc + (size_t)pos * kv_dim + (size_t)h * HD)[lane] = kv4;
                    reinterpret_cast<float4*>(vc + (size_t)pos * kv_dim + (size_t)h * HD)[lane] = vn;
                }
            }
        }
        const float sc = 1.0f / sqrtf((float)HD);
        qv.x *= sc; qv.y *= sc; qv.z *= sc; qv.w *= sc;
        if (qt) reinterpret_cast<float4*>(sq)[tid] = qv;
    }
    __syncthreads();
    if (kfresh) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            kr[2 * t] = reinterpret_cast<const float4*>(nk + 32 * t + 8 * kq)[0];
            kr[2 * t + 1] = reinterpret_cast<const float4*>(nk + 32 * t + 8 * kq)[1];
        }
    }
    if (fresh_block && pos >= t0 + 4 * kq && pos < t0 + 4 * kq + 4) {
        const int i = pos - t0 - 4 * kq;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float nv = nvs[VDIM(j, c16)];
#pragma unroll
            for (int ii = 0; ii < 4; ii++)
                if (ii == i) vv[j][ii] = nv;
        }
    }

    /* scores on v_mfma_f32_16x16x4_f32, exact fp32 products: step (t, m) takes dimension 32 t + 8 kq + m of
       position c16 (A) and of head c16 (B); four independent sums, one a chunk t */
    at_f4 St[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        float4 q0 = make_float4(0.f, 0.f, 0.f, 0.f), q1 = q0;
        if (c16 < G) {
            q0 = reinterpret_cast<const float4*>(sq + c16 * HD + 32 * t + 8 * kq)[0];
            q1 = reinterpret_cast<const float4*>(sq + c16 * HD + 32 * t + 8 * kq)[1];
        }
        const float4 k0 = kr[2 * t], k1 = kr[2 * t + 1];
        const float ka[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        const float qa[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        at_f4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m8 = 0; m8 < 8; m8++) c = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[m8], qa[m8], c, 0, 0, 0);
        St[t] = c;
    }
    at_f4 S;
#pragma unroll
    for (int r = 0; r < 4; r++) S[r] = (St[0][r] + St[1][r]) + (St[2][r] + St[3][r]);
    /* softmax over the wave's positions, per head (lane l % 16): position 4 kq + r of the wave */
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const bool ok = t0 + 4 * kq + r <= pos;
        S[r] = ok ? S[r] : -INFINITY;
        m = fmaxf(m, S[r]);
    }
    m = fmaxf(m, __shfl_xor(m, 16, WAVE));
    m = fmaxf(m, __shfl_xor(m, 32, WAVE));
    float P[4], l = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        P[r] = S[r] == -INFINITY ? 0.0f : __expf(S[r] - m);
        l += P[r];
    }
    l += __shfl_xor(l, 16, WAVE);
    l += __shfl_xor(l, 32, WAVE);

    /* values: eight tiles of 16 dimensions (tile j, column c: dimension VDIM(j, c)) */
    at_f4 O[8];
    /* step r takes position 4 kq + r: A is the lane's own weight P[r] of head c16, B its value vv[j][r] */
#pragma unroll
    for (int j = 0; j < 8; j++) O[j] = at_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int j = 0; j < 8; j++) O[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(P[r], vv[j][r], O[j], 0, 0, 0);
    if (kq == 0 && c16 < G) {
        wm[wave][c16] = m;
        wl[wave][c16] = l;
    }
    if (kq < 2) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int g = 4 * kq + r;
            if (g < G) {
#pragma unroll
                for (int j = 0; j < 8; j++) wacc[wave][g][VDIM(j, c16)] = O[j][r];
            }
        }
    }
    __syncthreads();

    /* this chunk's partial: the four waves merged, a float4 of one head a thread */
    {
        const int g = tid / QF4, j = tid % QF4;
        if (g < G) {
            float* part = a.partial + (((size_t)row * a.n_kv + h) * a.splits_max + split) * G * PS + (size_t)g * PS;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][g]);
            float L = 0.f;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float f = wm[w][g] == -INFINITY ? 0.0f : expf(wm[w][g] - M);
                const float4 x = reinterpret_cast<const float4*>(&wacc[w][g][0])[j];
                L = fmaf(wl[w][g], f, L);
                o.x = fmaf(x.x, f, o.x); o.y = fmaf(x.y, f, o.y); o.z = fmaf(x.z, f, o.z); o.w = fmaf(x.w, f, o.w);
            }
            reinterpret_cast<float4*>(part)[j] = o;
            if (j == 0) {
                part[HD] = M;
                part[HD + 1] = L;
            }
        }
    }
}

hipError_t launch_attention(const attn_args& a, hipStream_t s) {
    if (a.n_kv < 1 || a.n_heads % a.n_kv || a.n_heads / a.n_kv > GMAX || a.n_rows < 1) return hipErrorInvalidValue;
    if (a.splits_max * ATTN_CHUNK < a.ctx || a.splits_grid < 0) return hipErrorInvalidValue;
    const dim3 grid(a.splits_grid > 0 && a.splits_grid < a.splits_max ? a.splits_grid : a.splits_max, a.n_kv, a.n_rows);
    const int G = a.n_heads / a.n_kv;
    if (a.mma && a.hd == 128) {
#define ATTN_MMA(GG) \
        if (G == GG) { attention_mma_kernel<GG><<<grid, 256, 0, s>>>(a); return hipGetLastError(); }
        ATTN_MMA(8) ATTN_MMA(4) ATTN_MMA(2) ATTN_MMA(1)
#undef ATTN_MMA
    }
#define ATTN_CASE(HD, GG) \
    if (a.hd == HD && G == GG) { attention_kernel<HD, GG><<<grid, 256, 0, s>>>(a); return hipGetLastError(); }
    ATTN_CASE(128, 8) ATTN_CASE(128, 4) ATTN_CASE(128, 2) ATTN_CASE(128, 1)
    ATTN_CASE(64, 8) ATTN_CASE(64, 4) ATTN_CASE(64, 2) ATTN_CASE(64, 1)
#undef ATTN_CASE
    return hipErrorInvalidValue;
}


/* ---- passes of many rows of one sequence (a prompt's chunks): a tile of rows a block ----
   The per-row kernels read a chunk's keys and values once for every row, so a prompt pass of 1024 rows of one
   sequence reads each chunk up to 1024 times (from the memory-side cache; the L2 of an XCD holds 4 MB of a layer's
   16 MB). Here a block takes one kv head for a tile of TQ = 4 * 16 / G rows and loops over the chunks up to the
   tile's last position: each chunk's keys and values go to LDS once (64 KB), and wave w takes 16 query columns,
   RW = 16 / G rows of the tile times the G heads, against the chunk's 64 positions, each row masked to the
   positions up to its own. The queries come prepared (launch_attention_prepare). The scores of each chunk fold
   into a running maximum and sum per column, the values into O rescaled as the maximum grows, and the block
   writes att itself (O / sum): no chunk leaves a partial and no merge runs. A chunk's keys and values are
   requested before the barrier that frees the LDS of the previous one; the other block of the CU covers the
   wait. Passes of more than 64 rows reach it (the exact-rows limit), so it is held to 1e-3, not to a step's
   bits.

   The products run on the bf16 matrix cores. Each operand is split into bf16 hi + lo (lo the rounding of what hi
   leaves) and each product taken as hi*hi + hi*lo + lo*hi on v_mfma_f32_16x16x32_bf16, summed in fp32: about
   2^-15 of |a||b| a product against fp32's 2^-24, at a sixteenth of the fp32 unit's cycles an operation. (The
   same loop on v_mfma_f32_16x16x4_f32 took a 4096-token prompt 255 ms exact and 212 ms fast, against 226 and 183
   here, same box, twice each.) The keys go to LDS split, position-major (16-byte chunks of eight dimensions,
   XOR-swizzled by position); the values split and transposed, dimension-major (8-byte chunks of four positions,
   swizzled by dimension), so that a lane's eight positions of one dimension are two reads. A thread of the fetch
   holds four consecutive positions of four dimensions, which it transposes in registers. The scores come out with
   lane (c16, kq) holding position 16 pt + 4 kq + i of column c16; the weighted values take positions
   16 pt + 4 kq + i of pt in {2 s, 2 s + 1} as the eight k-slots of MFMA s, on both operands. */
typedef __bf16 fl_bf8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t fl_pack(__bf16 a, __bf16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}
/* four floats as bf16 hi and lo, packed in order */
__device__ __forceinline__ void fl_split4(float x0, float x1, float x2, float x3, uint2& hi, uint2& lo) {
    const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1, h2 = (__bf16)x2, h3 = (__bf16)x3;
    hi = make_uint2(fl_pack(h0, h1), fl_pack(h2, h3));
    lo = make_uint2(fl_pack((__bf16)(x0 - (float)h0), (__bf16)(x1 - (float)h1)),
                    fl_pack((__bf16)(x2 - (float)h2), (__bf16)(x3 - (float)h3)));
}
__device__ __forceinline__ fl_bf8 fl_join(uint2 a, uint2 b) { return __builtin_bit_cast(fl_bf8, u32x4{a.x, a.y, b.x, b.y}); }
#define FL_MMA(A, B, C) __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, C, 0, 0, 0)

template <int G>
__global__ __launch_bounds__(256, 2) void attention_flash_kernel(attn_args a) {
    constexpr int HD = 128, RW = 16 / G, TQ = 4 * RW;
    /* a tile's work grows with its position; the second half of the grid takes the tiles in reverse, so the two
       blocks a compute unit holds together (blockIdx.y and blockIdx.y + half) pair a short tile with a long one
       (a 4096-token prompt 200.6-201.4 -> 199.6 ms) */
    const int half = (gridDim.y + 1) / 2;
    const int h = blockIdx.x, tile = (int)blockIdx.y < half ? (int)blockIdx.y : (int)gridDim.y - 1 - ((int)blockIdx.y - half);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c16 = lane & 15, kq = lane >> 4;
    const int r_first = tile * TQ, r_end = min(a.n_rows, r_first + TQ);
    int pmax = 0;
    for (int r = r_first; r < r_end; r++) pmax = max(pmax, a.rows[r].pos);
    const int nch = pmax / ATTN_CHUNK + 1;
    const int seq = a.rows[r_first].seq, kv_dim = a.n_kv * HD;
    const float* kc = a.k_cache + (size_t)seq * a.seq_stride;
    const float* vc = a.v_cache + (size_t)seq * a.seq_stride;
    /* keys [position][16 chunks of 8 dimensions], values [dimension][16 chunks of 4 positions], hi and lo */
    __shared__ __attribute__((aligned(16))) uint32_t skh[64 * 64], skl[64 * 64];
    __shared__ __attribute__((aligned(16))) uint32_t svh[128 * 32], svl[128 * 32];

    const int rr = r_first + wave * RW + c16 / G, g = c16 % G;
    const bool colv = rr < r_end;
    const int prow = colv ? a.rows[rr].pos : -1;
    /* the column's query, scaled: dimensions 32 s + 8 kq .. + 7 as the B operand of step s */
    fl_bf8 qh[4], ql[4];
    {
        const float sc = 1.0f / sqrtf((float)HD);
        const float4* q4 = reinterpret_cast<const float4*>(a.q_raw + (size_t)(colv ? rr : r_first) * a.n_heads * HD +
                                                           (size_t)(h * G + g) * HD);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 v0 = colv ? q4[8 * s + 2 * kq] : z, v1 = colv ? q4[8 * s + 2 * kq + 1] : z;
            uint2 h0, l0, h1, l1;
            fl_split4(v0.x * sc, v0.y * sc, v0.z * sc, v0.w * sc, h0, l0);
            fl_split4(v1.x * sc, v1.y * sc, v1.z * sc, v1.w * sc, h1, l1);
            qh[s] = fl_join(h0, h1);
            ql[s] = fl_join(l0, l1);
        }
    }
    /* a thread's fetch: positions 32 (i / 4) + 4 pg + i % 4 of the chunk, dimensions 4 cc .. 4 cc + 3 (a wave's
       load is two whole 512-byte rows) */
    const int pg = tid >> 5, cc = tid & 31;
    float4 kr[8], vr[8];
    auto fetch = [&](int c) {
        const int t0 = c * ATTN_CHUNK;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int p = 32 * (i >> 2) + 4 * pg + (i & 3), pos = t0 + p;
            const bool ok = pos <= pmax;
            const size_t at = (size_t)(ok ? pos : 0) * kv_dim + (size_t)h * HD + 4 * cc;
            kr[i] = ok ? *reinterpret_cast<const float4*>(kc + at) : make_float4(0.f, 0.f, 0.f, 0.f);
            vr[i] = ok ? *reinterpret_cast<const float4*>(vc + at) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    float m_run = -INFINITY, l_run = 0.0f;
    at_f4 O[8];
#pragma unroll
    for (int j = 0; j < 8; j++) O[j] = at_f4{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nch; c++) {
        fetch(c);
        __syncthreads(); /* the previous chunk's fragment reads are done */
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int p = 32 * (i >> 2) + 4 * pg + (i & 3);
            uint2 hh, ll;
            fl_split4(kr[i].x, kr[i].y, kr[i].z, kr[i].w, hh, ll);
            const int ka = (p * 16 + ((cc >> 1) ^ (p & 15))) * 4 + 2 * (cc & 1);
            *reinterpret_cast<uint2*>(&skh[ka]) = hh;
            *reinterpret_cast<uint2*>(&skl[ka]) = ll;
        }
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int pc = 8 * q + pg; /* the chunk of positions 32 q + 4 pg .. + 3 */
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const float4 *v = vr + 4 * q;
                const float x0 = d == 0 ? v[0].x : d == 1 ? v[0].y : d == 2 ? v[0].z : v[0].w;
                const float x1 = d == 0 ? v[1].x : d == 1 ? v[1].y : d == 2 ? v[1].z : v[1].w;
                const float x2 = d == 0 ? v[2].x : d == 1 ? v[2].y : d == 2 ? v[2].z : v[2].w;
                const float x3 = d == 0 ? v[3].x : d == 1 ? v[3].y : d == 2 ? v[3].z : v[3].w;
                uint2 hh, ll;
                fl_split4(x0, x1, x2, x3, hh, ll);
                const int dim = 4 * cc + d, va = (dim * 16 + (pc ^ (dim & 15))) * 2;
                *reinterpret_cast<uint2*>(&svh[va]) = hh;
                *reinterpret_cast<uint2*>(&svl[va]) = ll;
            }
        }
        __syncthreads();
        const int t0 = c * ATTN_CHUNK;
        at_f4 S[4];
#pragma unroll
        for (int pt = 0; pt < 4; pt++) {
            const int p = 16 * pt + c16;
            at_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int ka = (p * 16 + ((4 * s + kq) ^ (p & 15))) * 4;
                const fl_bf8 kh = *reinterpret_cast<const fl_bf8*>(&skh[ka]);
                const fl_bf8 kl = *reinterpret_cast<const fl_bf8*>(&skl[ka]);
                acc = FL_MMA(kh, qh[s], acc);
                acc = FL_MMA(kh, ql[s], acc);
                acc = FL_MMA(kl, qh[s], acc);
            }
            S[pt] = acc;
        }
        float m = m_run;
#pragma unroll
        for (int pt = 0; pt < 4; pt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const bool ok = t0 + 16 * pt + 4 * kq + i <= prow;
                S[pt][i] = ok ? S[pt][i] : -INFINITY;
                m = fmaxf(m, S[pt][i]);
            }
        m = fmaxf(m, __shfl_xor(m, 16, WAVE));
        m = fmaxf(m, __shfl_xor(m, 32, WAVE));
        const float f = m == -INFINITY || m_run == -INFINITY ? 0.0f : __expf(m_run - m);
        float l = 0.0f;
#pragma unroll
        for (int pt = 0; pt < 4; pt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                S[pt][i] = S[pt][i] == -INFINITY ? 0.0f : __expf(S[pt][i] - m);
                l += S[pt][i];
            }
        l += __shfl_xor(l, 16, WAVE);
        l += __shfl_xor(l, 32, WAVE);
        l_run = fmaf(l_run, f, l);
        m_run = m;
        float fo[4];
#pragma unroll
        for (int i = 0; i < 4; i++) fo[i] = __shfl(f, 4 * kq + i, WAVE);
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) O[j][i] *= fo[i];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            uint2 ph0, pl0, ph1, pl1;
            fl_split4(S[2 * s][0], S[2 * s][1], S[2 * s][2], S[2 * s][3], ph0, pl0);
            fl_split4(S[2 * s + 1][0], S[2 * s + 1][1], S[2 * s + 1][2], S[2 * s + 1][3], ph1, pl1);
            const fl_bf8 ph = fl_join(ph0, ph1), pl = fl_join(pl0, pl1);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int dim = 16 * j + c16;
                const int va0 = (dim * 16 + ((8 * s + kq) ^ (dim & 15))) * 2;
                const int va1 = (dim * 16 + ((8 * s + 4 + kq) ^ (dim & 15))) * 2;
                const fl_bf8 vh = fl_join(*reinterpret_cast<const uint2*>(&svh[va0]), *reinterpret_cast<const uint2*>(&svh[va1]));
                const fl_bf8 vl = fl_join(*reinterpret_cast<const uint2*>(&svl[va0]), *reinterpret_cast<const uint2*>(&svl[va1]));
                O[j] = FL_MMA(ph, vh, O[j]);
                O[j] = FL_MMA(ph, vl, O[j]);
                O[j] = FL_MMA(pl, vh, O[j]);
            }
        }
    }
    /* att = O / sum: column 4 kq + i of the lane's O, dimension 16 j + c16 */
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int ccol = 4 * kq + i, rw = r_first + wave * RW + ccol / G, gc = ccol % G;
        const float lsum = __shfl(l_run, ccol, WAVE);
        if (rw < r_end) {
            float* out = a.att + (size_t)rw * a.n_heads * HD + (size_t)(h * G + gc) * HD;
#pragma unroll
            for (int j = 0; j < 8; j++) out[16 * j + c16] = O[j][i] / lsum;
        }
    }
}

hipError_t launch_attention_flash(const attn_args& a, hipStream_t s) {
    if (!attention_run_fits(a) || a.n_rows < 1) return hipErrorInvalidValue;
    const int G = a.n_heads / a.n_kv, tq = 4 * (16 / G);
    const dim3 grid(a.n_kv, (a.n_rows + tq - 1) / tq);
    switch (G) {
        case 8: attention_flash_kernel<8><<<grid, 256, 0, s>>>(a); break;
        case 4: attention_flash_kernel<4><<<grid, 256, 0, s>>>(a); break;
        case 2: attention_flash_kernel<2><<<grid, 256, 0, s>>>(a); break;
        case 1: attention_flash_kernel<1><<<grid, 256, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool attention_run_fits(const attn_args& a) {
    return a.hd == 128 && a.prepared && a.n_kv >= 1 && a.n_heads % a.n_kv == 0 && 16 % (a.n_heads / a.n_kv) == 0 &&
           a.n_heads / a.n_kv <= GMAX;
}

/* One block per (query head, row): the chunks' maxima and sums read in parallel, each chunk's scale
   exp(m_s - M) computed once; then SP threads a dimension, thread (d, sp) summing the weighted values of chunks
   sp, sp + SP, ... (up to MERGE_PRE of them requested at once), and the SP partial sums added in sp order. SP
   grows with the chunks a row may have, so a long context is read in one or two rounds of loads rather than
   one round per eight chunks. */
#define MERGE_MAX ATTN_SPLITS_MAX
#define MERGE_PRE 32 /* chunks a thread requests before its first add */
template <int SP>
__global__ __launch_bounds__(SP > 1 ? 128 * SP : 1024) void attention_merge_kernel(attn_args a) {
    const int hq = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, HD = a.hd;
    /* (one thread a dimension: the block is the head's HD threads) */
    const int d = SP > 1 ? tid % HD : tid, sp = SP > 1 ? tid / HD : 0, nt = SP > 1 ? HD * SP : (int)blockDim.x;
    const int G = a.n_heads / a.n_kv, h = hq / G, g = hq % G;
    const int n_act = a.rows[row].pos / ATTN_CHUNK + 1;
    const float* base = a.partial + (((size_t)row * a.n_kv + h) * a.splits_max * G + g) * (HD + 4);
    const size_t stride = (size_t)G * (HD + 4);
    __shared__ float fm[MERGE_MAX], fl[MERGE_MAX];
    __shared__ float red[8];
    __shared__ float po[SP > 1 ? SP - 1 : 1][128], pl[SP > 1 ? SP - 1 : 1];
    /* this thread's first MERGE_PRE chunks' values, requested alongside the maxima */
    float v0[MERGE_PRE];
#pragma unroll
    for (int i = 0; i < MERGE_PRE; i++) {
        const int s = sp + SP * i;
        v0[i] = s < n_act ? base[s * stride + d] : 0.0f;
    }
    float m = -INFINITY;
    for (int s = tid; s < n_act; s += nt) {
        fm[s] = base[s * stride + HD];
        fl[s] = base[s * stride + HD + 1];
        m = fmaxf(m, fm[s]);
    }
    m = wave_max_dpp(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float M = red[0];
    for (int w = 1; w < nt / 64; w++) M = fmaxf(M, red[w]);
    for (int s = tid; s < n_act; s += nt) fm[s] = expf(fm[s] - M);
    __syncthreads();
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int i = 0; i < MERGE_PRE; i++) {
        const int s = sp + SP * i;
        if (s < n_act) {
            L = fmaf(fl[s], fm[s], L);
            o = fmaf(v0[i], fm[s], o);
        }
    }
    int s = sp + SP * MERGE_PRE;
    for (; s + 7 * SP < n_act; s += 8 * SP) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = base[(s + SP * i) * stride + d];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            L = fmaf(fl[s + SP * i], fm[s + SP * i], L);
            o = fmaf(v[i], fm[s + SP * i], o);
        }
    }
    for (; s < n_act; s += SP) {
        L = fmaf(fl[s], fm[s], L);
        o = fmaf(base[s * stride + d], fm[s], o);
    }
    if constexpr (SP > 1) {
        if (sp > 0) {
            po[sp - 1][d] = o;
            if (d == 0) pl[sp - 1] = L;
        }
        __syncthreads();
        if (sp > 0) return;
#pragma unroll
        for (int i = 0; i < SP - 1; i++) {
            o += po[i][d];
            L += pl[i];
        }
    }
    const float val = o / L;
    a.att[(size_t)row * a.n_heads * HD + (size_t)hq * HD + d] = val;
    if (a.img.a) {
        /* the head's HD columns of the row into the o-projection's operand images: 8 columns a thread. Only the
           waves of sp = 0 are left (whole waves returned above), and a barrier counts the waves still running. */
        __shared__ float sv[128];
        sv[d] = val;
        __syncthreads();
        if (d < HD / 8) {
            float e[8];
#pragma unroll
            for (int i = 0; i < 8; i++) e[i] = sv[8 * d + i];
            u32x4 vh, vl;
            float sum;
            img_split8(e, vh, vl, sum);
            const int K = a.n_heads * HD, c8 = hq * (HD / 8) + d;
            img_put(a.img.a, a.img.b, row, K, c8, vh, vl);
            const float t16 = sum + __shfl_xor(sum, 1, WAVE);
            const float t32 = t16 + __shfl_xor(t16, 2, WAVE);
            if (!(c8 & 1)) img_sum16(a.img.s16, row, K, c8 >> 1, t16);
            if (!(c8 & 3)) img_sum32(a.img.s32, row, K, c8 >> 2, t32);
        }
    }
}

hipError_t launch_attention_merge(const attn_args& a, hipStream_t s) {
    if (a.n_kv < 1 || a.n_heads % a.n_kv || a.n_rows < 1 || (a.hd != 64 && a.hd != 128) || a.splits_max > MERGE_MAX)
        return hipErrorInvalidValue;
    if (a.img.a && ((a.n_heads * a.hd) % 256 || !a.img.b || !a.img.s32 || !a.img.s16)) return hipErrorInvalidValue;
    const dim3 grid(a.n_heads, a.n_rows);
    /* threads a dimension: enough that a thread sums at most about MERGE_PRE chunks. A single row (batch-1
       decode) keeps one: its few blocks leave the device idle either way, and the wider form measured slower there. */
    if (a.n_rows > 1 && a.splits_max > 4 * MERGE_PRE) attention_merge_kernel<4><<<grid, 4 * a.hd, 0, s>>>(a);
    else if (a.n_rows > 1 && a.splits_max > 2 * MERGE_PRE) attention_merge_kernel<2><<<grid, 2 * a.hd, 0, s>>>(a);
    else attention_merge_kernel<1><<<grid, a.hd, 0, s>>>(a);
    return hipGetLastError();
}

/* The merge and the o-projection of one row, a group of HG = ATTN_OPROJ_HEADS query heads a block (blockIdx.x)
   and a range of 4 RPW U output rows (blockIdx.y). Its weights (the rows' CW = HG HD columns of the group) do not
   depend on anything before: every wave requests its U units of RPW rows at once. Wave w then merges head w of
   the group exactly as attention_merge_kernel<1> does (the maximum over the chunks, each chunk's scale
   exp(m_s - M), the sums in chunk order), so att is the same bits; the HG heads' outputs go to LDS, and each
   row's dot over the group's columns runs as the dense GEMV's does, LPR = CW / 32 lanes a row, one slice a lane.
   parts[g][r] holds row r's share of the group. Every block of a group merges the group's heads again (at
   configs[2], 32 blocks a group, 80 KB of partials each from L2): that costs less than the kernel boundary
   a separate merge kernel puts in front of the o-projection. More, smaller blocks than the GEMV would take
   (U = 4: 256 blocks at configs[2]) keep more of the weights in flight: with 128 blocks the pair took 1.4 us
   more. */
#define OPROJ_U 4 /* units of RPW rows a wave: 64 rows a block at head size 128, 256 blocks at config 2 */
#define OPROJ_PRE 36 /* (a multiple of 4) chunks whose values a lane requests in the first round (2,304 positions) */
template <int DT, int HD>
__global__ __launch_bounds__(256) void attention_oproj_kernel(attn_args a, qmat o, float* __restrict__ parts) {
    constexpr int HG = ATTN_OPROJ_HEADS, CW = HG * HD, LPR = CW / 32, RPW = WAVE / LPR, DPT = HD / 64;
    static_assert(HG == 4 && CW % 256 == 0 && LPR <= WAVE, "one wave a head, whole super-blocks a group");
    const int g = blockIdx.x, row = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane / LPR, al = lane % LPR;
    const int t_abs = g * (CW / 32) + al; /* the lane's slice of a row */
    if (row) {
        /* row blockIdx.z of a pass: its partials, att and parts; the arithmetic is a single row's */
        a.partial += (size_t)row * a.n_kv * a.splits_max * (a.n_heads / a.n_kv) * (HD + 4);
        a.att += (size_t)row * a.n_heads * HD;
        parts += (size_t)row * (a.n_heads / HG) * o.rows;
    }
    const int rbase = blockIdx.y * (4 * RPW * OPROJ_U) + wave * (RPW * OPROJ_U) + sub;
    /* the merge's loads first, none of them waiting for the position: wave w, head hq = g HG + w, DPT dimensions a
       lane, the values of chunks 0 .. OPROJ_PRE - 1 and the maxima and sums of chunks lane and lane + 64, read
       whatever the position (those past its last chunk, or past the buffer's chunks as its last, are not used) */
    __shared__ __attribute__((aligned(16))) float fm[HG][MERGE_MAX];
    __shared__ __attribute__((aligned(16))) float fl[HG][MERGE_MAX];
    __shared__ __attribute__((aligned(16))) float sx[CW];
    const int G = a.n_heads / a.n_kv, hq = g * HG + wave, h = hq / G, gi = hq % G;
    const float* base = a.partial + ((size_t)h * a.splits_max * G + gi) * (HD + 4);
    const size_t stride = (size_t)G * (HD + 4);
    const int d0 = lane * DPT, last = a.splits_max - 1;
    const int pos_v = gld<int>(&a.rows[row].pos);
    float v0[OPROJ_PRE][DPT];
#pragma unroll
    for (int i = 0; i < OPROJ_PRE; i++) {
        const float* p = base + (size_t)min(i, last) * stride + d0;
        if constexpr (DPT == 2) {
            const float2 t = *reinterpret_cast<const float2*>(p);
            v0[i][0] = t.x;
            v0[i][1] = t.y;
        } else {
            v0[i][0] = p[0];
        }
    }
    float2 ml[2];
#pragma unroll
    for (int i = 0; i < 2; i++) ml[i] = *reinterpret_cast<const float2*>(base + (size_t)min(lane + WAVE * i, last) * stride + HD);
    __builtin_amdgcn_sched_barrier(0);

    /* then the weights, which nothing before depends on either: U units of RPW rows a wave */
    qraw q[OPROJ_U];
#pragma unroll
    for (int u = 0; u < OPROJ_U; u++) {
        const int r = min(rbase + u * RPW, o.rows - 1);
        slice_load<DT>(o, 0, r, t_abs, q[u]);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int n_act = __builtin_amdgcn_readfirstlane(pos_v) / ATTN_CHUNK + 1;

    /* the merge, as attention_merge_kernel<1> computes it */
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int s = lane + WAVE * i;
        if (s < n_act) {
            fm[wave][s] = ml[i].x;
            fl[wave][s] = ml[i].y;
            m = fmaxf(m, ml[i].x);
        }
    }
    for (int s = lane + 2 * WAVE; s < n_act; s += WAVE) {
        fm[wave][s] = base[s * stride + HD];
        fl[wave][s] = base[s * stride + HD + 1];
        m = fmaxf(m, fm[wave][s]);
    }
    const float M = wave_max_dpp(m);
    for (int s = lane; s < n_act; s += WAVE) fm[wave][s] = expf(fm[wave][s] - M);
    __syncthreads();
    float L = 0.f, acc[DPT];
#pragma unroll
    for (int k = 0; k < DPT; k++) acc[k] = 0.f;
    {
        /* the first chunks' scales and sums, all read at once (entries past the last chunk are read, not used) */
        float sf[OPROJ_PRE], sl[OPROJ_PRE];
#pragma unroll
        for (int i = 0; i < OPROJ_PRE / 4; i++) {
            const float4 f4 = reinterpret_cast<const float4*>(fm[wave])[i], l4 = reinterpret_cast<const float4*>(fl[wave])[i];
            sf[4 * i] = f4.x; sf[4 * i + 1] = f4.y; sf[4 * i + 2] = f4.z; sf[4 * i + 3] = f4.w;
            sl[4 * i] = l4.x; sl[4 * i + 1] = l4.y; sl[4 * i + 2] = l4.z; sl[4 * i + 3] = l4.w;
        }
#pragma unroll
        for (int i = 0; i < OPROJ_PRE; i++)
            if (i < n_act) {
                L = fmaf(sl[i], sf[i], L);
#pragma unroll
                for (int k = 0; k < DPT; k++) acc[k] = fmaf(v0[i][k], sf[i], acc[k]);
            }
    }
    int s = OPROJ_PRE;
    for (; s + 7 < n_act; s += 8) {
        float v[8][DPT];
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int k = 0; k < DPT; k++) v[i][k] = base[(s + i) * stride + d0 + k];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            L = fmaf(fl[wave][s + i], fm[wave][s + i], L);
#pragma unroll
            for (int k = 0; k < DPT; k++) acc[k] = fmaf(v[i][k], fm[wave][s + i], acc[k]);
        }
    }
    for (; s < n_act; s++) {
        L = fmaf(fl[wave][s], fm[wave][s], L);
#pragma unroll
        for (int k = 0; k < DPT; k++) acc[k] = fmaf(base[s * stride + d0 + k], fm[wave][s], acc[k]);
    }
#pragma unroll
    for (int k = 0; k < DPT; k++) {
        const float val = acc[k] / L;
        sx[wave * HD + d0 + k] = val;
        if (blockIdx.y == 0) a.att[(size_t)hq * HD + d0 + k] = val;
    }
    __syncthreads();

    /* the rows: the lane's slice of the group's columns, then U units of RPW rows */
    xslice xs;
    load_xslice(DT, al, sx, xs);
#pragma unroll
    for (int u = 0; u < OPROJ_U; u++) {
        float p = slice_dot<DT>(q[u], t_abs, xs);
        p = row_sum<LPR>(p);
        const int r = rbase + u * RPW;
        if (al == LPR - 1 && r < o.rows) parts[(size_t)g * o.rows + r] = p;
    }
}

bool attention_oproj_fits(const attn_args& a, const qmat& o) {
    return a.n_rows >= 1 && (a.hd == 64 || a.hd == 128) && a.n_kv >= 1 && a.n_heads % a.n_kv == 0 &&
           a.n_heads % ATTN_OPROJ_HEADS == 0 && a.n_heads / ATTN_OPROJ_HEADS <= OPROJ_PARTS_MAX && a.splits_max <= MERGE_MAX &&
           o.cols == a.n_heads * a.hd && o.rows >= 256 && o.rows <= ROUTE_PARTS_HMAX &&
           (o.dtype == VITNA_DTYPE_Q4_K || o.dtype == VITNA_DTYPE_Q6_K || o.dtype == VITNA_DTYPE_Q8_0);
}

hipError_t launch_attention_oproj(const attn_args& a, const qmat& o, float* parts, hipStream_t s) {
    if (!attention_oproj_fits(a, o) || !parts) return hipErrorInvalidValue;
    const int rpw = WAVE / (ATTN_OPROJ_HEADS * a.hd / 32), per_block = 4 * rpw * OPROJ_U;
    const dim3 grid(a.n_heads / ATTN_OPROJ_HEADS, (o.rows + per_block - 1) / per_block, a.n_rows);
#define OPROJ_CASE(DT, HD) \
    if (o.dtype == DT && a.hd == HD) { attention_oproj_kernel<DT, HD><<<grid, 256, 0, s>>>(a, o, parts); return hipGetLastError(); }
    OPROJ_CASE(VITNA_DTYPE_Q4_K, 128) OPROJ_CASE(VITNA_DTYPE_Q6_K, 128) OPROJ_CASE(VITNA_DTYPE_Q8_0, 128)
    OPROJ_CASE(VITNA_DTYPE_Q4_K, 64) OPROJ_CASE(VITNA_DTYPE_Q6_K, 64) OPROJ_CASE(VITNA_DTYPE_Q8_0, 64)
#undef OPROJ_CASE
    return hipErrorInvalidValue;
}

__global__ __launch_bounds__(256) void attn_fold_kernel(float* __restrict__ x, const float* __restrict__ parts, int n_parts, int H) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    x += (size_t)blockIdx.y * H;
    parts += (size_t)blockIdx.y * n_parts * H;
    if (i < H) x[i] = attn_resid(x[i], parts, n_parts, (size_t)H, (size_t)i);
}

hipError_t launch_attn_fold(float* x, const float* parts, int n_parts, int H, hipStream_t s, int n_rows) {
    if (n_parts < 1 || n_parts > OPROJ_PARTS_MAX || H < 1 || n_rows < 1) return hipErrorInvalidValue;
    attn_fold_kernel<<<dim3((H + 255) / 256, n_rows), 256, 0, s>>>(x, parts, n_parts, H);
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
