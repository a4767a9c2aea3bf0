/**
 * kernels_rows.hip - Several rows at once (tokens of possibly different
 * sequences, each at its own position): the dense projections applied to
 * every row with one read of the weights, and the per-token expert grouping
 * that turns a ragged batch into grouped expert work, each selected expert's
 * weights read once for all the rows routed to it.
 *
 * Reference counterparts (engine/src/model_cuda.cu): the host counting sort
 * of (row, expert) pairs :5151-5176, add_rows_kernel :2120 and
 * norm_rows_kernel :2020 (residual_norm_kernel here), embed_multi_kernel
 * :1858, the *_multi kernels :1872-2006. The grouped experts themselves are kernels_gmma.hip's
 * (experts_in_rows_kernel :2071, experts_down_rows_kernel :2101).
 *
 * The grouping is built on the device (group_kernel): one block per expert
 * scans every row's routing and lists the (row, slot) pairs routed to it in
 * order of row, at a fixed capacity of ROWS_CAP pairs an expert, so no prefix
 * sum over experts is needed. Each pair's output is kept apart (ypart, one
 * hidden-wide row per pair) and reduce_rows_kernel adds a row's K outputs in
 * order of expert id, then onto the residual: the order the reference sums
 * in (engine/src/model.c:757-760).
 */

#include "vitna_kernels.h"
#include "skinny_image.h"
#include <algorithm>

template <int LPR>
__device__ __forceinline__ float rsum(float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

/* ---- embedding and norms ---------------------------------------------- */

__global__ void embed_rows_kernel(qmat m, const row_rec* __restrict__ rows, float* __restrict__ x, int H) {
    const int r = blockIdx.y;
    const int t = rows[r].token;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < H; c += gridDim.x * blockDim.x) x[(size_t)r * H + c] = widen_one(m, 0, t, c);
}

hipError_t launch_embed_rows(const qmat& embed, const row_rec* rows, int n, float* x, hipStream_t s) {
    if (n < 1) return hipErrorInvalidValue;
    embed_rows_kernel<<<dim3((embed.cols + 255) / 256, n), 256, 0, s>>>(embed, rows, x, embed.cols);
    return hipGetLastError();
}

/* One block a row: x += the K parts of the row in slot order (when ypart is given: the experts' outputs, as
   reduce_rows_kernel adds them), then y = RMSNorm(x) * w, and (when img.a is given) y split into the multi-row
   projections' operand images (skinny_image.h). Thread t takes the 8-column groups t + 256 j; the sum of
   squares runs over a thread's columns in order, then the block's threads in wave order. */
__global__ __launch_bounds__(256) void residual_norm_kernel(float* __restrict__ x, const float* __restrict__ ypart, int K,
                                                            const float* __restrict__ w, float* __restrict__ y, int H, float eps,
                                                            img_out img) {
    const int r = blockIdx.x, t = threadIdx.x, G8 = H / 8;
    float v[4][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c8 = t + 256 * j;
        if (c8 >= G8) continue;
        float4* xp = reinterpret_cast<float4*>(x + (size_t)r * H + 8 * c8);
        float4 a0 = xp[0], a1 = xp[1];
        if (ypart) {
            float s8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int k = 0; k < K; k++) {
                const float4* yp = reinterpret_cast<const float4*>(ypart + ((size_t)r * K + k) * H + 8 * c8);
                const float4 b0 = yp[0], b1 = yp[1];
                s8[0] = s8[0] + b0.x; s8[1] = s8[1] + b0.y; s8[2] = s8[2] + b0.z; s8[3] = s8[3] + b0.w;
                s8[4] = s8[4] + b1.x; s8[5] = s8[5] + b1.y; s8[6] = s8[6] + b1.z; s8[7] = s8[7] + b1.w;
            }
            a0.x = a0.x + s8[0]; a0.y = a0.y + s8[1]; a0.z = a0.z + s8[2]; a0.w = a0.w + s8[3];
            a1.x = a1.x + s8[4]; a1.y = a1.y + s8[5]; a1.z = a1.z + s8[6]; a1.w = a1.w + s8[7];
            xp[0] = a0;
            xp[1] = a1;
        }
        const float e[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[j][i] = e[i];
            ss = fmaf(e[i], e[i], ss);
        }
    }
    __shared__ float red[4];
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c8 = t + 256 * j;
        if (c8 >= G8) continue; /* G8 is a multiple of 32 when images are written: every shuffle partner is active */
        const float4* wp = reinterpret_cast<const float4*>(w + 8 * c8);
        const float4 w0 = wp[0], w1 = wp[1];
        const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = (v[j][i] * inv) * ww[i];
        float4* yp = reinterpret_cast<float4*>(y + (size_t)r * H + 8 * c8);
        yp[0] = make_float4(o[0], o[1], o[2], o[3]);
        yp[1] = make_float4(o[4], o[5], o[6], o[7]);
        if (img.a) {
            u32x4 vh, vl;
            float sum;
            img_split8(o, vh, vl, sum);
            img_put(img.a, img.b, r, H, c8, vh, vl);
            const float t16 = sum + __shfl_xor(sum, 1, WAVE);
            const float t32 = t16 + __shfl_xor(t16, 2, WAVE);
            if (!(c8 & 1)) img_sum16(img.s16, r, H, c8 >> 1, t16);
            if (!(c8 & 3)) img_sum32(img.s32, r, H, c8 >> 2, t32);
        }
    }
}

hipError_t launch_residual_norm(float* x, const float* ypart, int K, const float* w, float* y, int n, int H, float eps,
                                const img_out& img, hipStream_t s) {
    if (n < 1 || H % 8 || H > 8192 || (ypart && K < 1)) return hipErrorInvalidValue;
    if (img.a && (H % 256 || !img.b || !img.s32 || !img.s16)) return hipErrorInvalidValue;
    residual_norm_kernel<<<n, 256, 0, s>>>(x, ypart, K, w, y, H, eps, img);
    return hipGetLastError();
}

/* ---- dense projections of several rows -------------------------------- */

/* y_i[row][r] (+)= W_i[r] . x[row], row < n: a wave's slices of a weight row
   are read once and applied to every row's activations (x rows L2-resident). */
template <int DT, int LPR, int SPL>
__device__ __forceinline__ void gemv_multi_rows(const qmat& w, float* __restrict__ y, int add, const float* __restrict__ x, int n, int xstride,
                                                int unit0, int ustep, int lane) {
    constexpr int RPW = WAVE / LPR;
    const int sub = lane / LPR, al = lane % LPR;
    const int units = (w.rows + RPW - 1) / RPW;
    for (int u = unit0; u < units; u += ustep) {
        const int r = u * RPW + sub, rr = r < w.rows ? r : w.rows - 1;
        qraw q[SPL];
#pragma unroll
        for (int j = 0; j < SPL; j++) slice_load<DT>(w, 0, rr, al + LPR * j, q[j]);
        for (int t = 0; t < n; t++) {
            float p = 0.f;
#pragma unroll
            for (int j = 0; j < SPL; j++) {
                xslice xs;
                load_xslice(DT, al + LPR * j, x + (size_t)t * xstride, xs);
                p += slice_dot<DT>(q[j], al + LPR * j, xs);
            }
            p = rsum<LPR>(p);
            if (al == 0 && r < w.rows) {
                float* o = y + (size_t)t * w.rows + r;
                *o = add ? *o + p : p;
            }
        }
    }
}

template <int D0, int D1, int D2, int LPR, int SPL>
__global__ __launch_bounds__(256) void gemv_multi_kernel(gemv_multi_args a) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE, nwaves = gridDim.x * (blockDim.x / WAVE);
    constexpr int RPW = WAVE / LPR;
    int base = 0;
    for (int i = 0; i < a.nm; i++) {
        const int units = (a.w[i].rows + RPW - 1) / RPW;
        int first = (wave - base) % nwaves;
        if (first < 0) first += nwaves;
        if (first < units) {
            if (i == 0) gemv_multi_rows<D0, LPR, SPL>(a.w[0], a.y[0], a.add, a.x, a.n, a.xstride, first, nwaves, lane);
            else if (i == 1) gemv_multi_rows<D1, LPR, SPL>(a.w[1], a.y[1], a.add, a.x, a.n, a.xstride, first, nwaves, lane);
            else gemv_multi_rows<D2, LPR, SPL>(a.w[2], a.y[2], a.add, a.x, a.n, a.xstride, first, nwaves, lane);
        }
        base += units;
    }
}

template <int D0, int D1, int D2>
static hipError_t gemv_multi_width(const gemv_multi_args& a, hipStream_t s) {
    const int S = a.w[0].cols / 32;
    const int lpr = S < 64 ? S : 64, rpw = WAVE / lpr;
    int units = 0;
    for (int i = 0; i < a.nm; i++) units += (a.w[i].rows + rpw - 1) / rpw;
    int blocks = (units + 3) / 4;
    if (blocks > 2048) blocks = 2048;
    switch (S) {
        case 4: gemv_multi_kernel<D0, D1, D2, 4, 1><<<blocks, 256, 0, s>>>(a); break;
        case 8: gemv_multi_kernel<D0, D1, D2, 8, 1><<<blocks, 256, 0, s>>>(a); break;
        case 16: gemv_multi_kernel<D0, D1, D2, 16, 1><<<blocks, 256, 0, s>>>(a); break;
        case 32: gemv_multi_kernel<D0, D1, D2, 32, 1><<<blocks, 256, 0, s>>>(a); break;
        case 64: gemv_multi_kernel<D0, D1, D2, 64, 1><<<blocks, 256, 0, s>>>(a); break;
        case 128: gemv_multi_kernel<D0, D1, D2, 64, 2><<<blocks, 256, 0, s>>>(a); break;
        case 256: gemv_multi_kernel<D0, D1, D2, 64, 4><<<blocks, 256, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_multi(const gemv_multi_args& a, hipStream_t s) {
    if (a.nm < 1 || a.nm > 3 || a.n < 1) return hipErrorInvalidValue;
    for (int i = 1; i < a.nm; i++)
        if (a.w[i].cols != a.w[0].cols) return hipErrorInvalidValue;
    const int d0 = a.w[0].dtype, d1 = a.nm > 1 ? a.w[1].dtype : d0, d2 = a.nm > 2 ? a.w[2].dtype : d1;
    constexpr int Q8 = VITNA_DTYPE_Q8_0, Q4 = VITNA_DTYPE_Q4_K, Q6 = VITNA_DTYPE_Q6_K;
#define GM_CASE(A, B, C) \
    if (d0 == A && d1 == B && d2 == C) return gemv_multi_width<A, B, C>(a, s);
    GM_CASE(Q4, Q4, Q6)
    GM_CASE(Q4, Q4, Q4)
    GM_CASE(Q8, Q8, Q8)
    GM_CASE(Q6, Q6, Q6)
    GM_CASE(Q4, Q6, Q6)
    GM_CASE(Q6, Q6, Q4)
#undef GM_CASE
    return hipErrorInvalidValue;
}

/* ---- grouping --------------------------------------------------------- */

/* Block e lists the (row, slot) pairs whose routing names expert e, in order
   of row: pairs[e * cap + i] = row * ROUTE_K_MAX + slot, count[e] = how many.
   A thread a row, GROUP_T rows a pass. */
#define GROUP_T 1024
__global__ __launch_bounds__(GROUP_T) void group_kernel(const route_out* __restrict__ rt, int n, int K, int cap, int* __restrict__ count,
                                                        int* __restrict__ pairs) {
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ int wave_n[GROUP_T / WAVE];
    int base = 0;
    for (int r0 = 0; r0 < n; r0 += GROUP_T) {
        const int r = r0 + tid;
        int slot = -1;
        if (r < n) {
            const int4* ip = reinterpret_cast<const int4*>(rt[r].ids);
#pragma unroll
            for (int q = 0; q < ROUTE_K_MAX / 4; q++)
                if (4 * q < K) {
                    const int4 v = ip[q];
                    if (4 * q + 0 < K && v.x == e) slot = 4 * q + 0;
                    if (4 * q + 1 < K && v.y == e) slot = 4 * q + 1;
                    if (4 * q + 2 < K && v.z == e) slot = 4 * q + 2;
                    if (4 * q + 3 < K && v.w == e) slot = 4 * q + 3;
                }
        }
        const uint64_t b = __ballot(slot >= 0);
        const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
        if (lane == 0) wave_n[wave] = __popcll(b);
        __syncthreads();
        int before = base, total = 0;
#pragma unroll
        for (int w = 0; w < GROUP_T / WAVE; w++) {
            if (w < wave) before += wave_n[w];
            total += wave_n[w];
        }
        if (slot >= 0) {
            const int at = before + __popcll(b & below);
            if (at < cap) pairs[(size_t)e * cap + at] = r * ROUTE_K_MAX + slot;
        }
        base += total;
        __syncthreads();
    }
    if (tid == 0) count[e] = base < cap ? base : cap;
}

/* The same lists for passes of more than GROUP_T rows (a prefill): a thread takes GROUP_R consecutive rows,
   GROUP_T * GROUP_R rows a pass (4096 rows in one pass, where a row a thread took four passes of two barriers
   each: config 4's routing and grouping 28.5 -> 26 us; at 32 rows the ballot form above is 0.2 ms a step faster);
   each thread's matches go after those of the threads before it (a wave's inclusive scan, then the waves' totals
   in order). */
#define GROUP_R 4
__global__ __launch_bounds__(GROUP_T) void group_many_kernel(const route_out* __restrict__ rt, int n, int K, int cap, int* __restrict__ count,
                                                        int* __restrict__ pairs) {
    const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ int wave_n[GROUP_T / WAVE];
    int base = 0;
    for (int r0 = 0; r0 < n; r0 += GROUP_T * GROUP_R) {
        int slot[GROUP_R], mine = 0;
#pragma unroll
        for (int u = 0; u < GROUP_R; u++) {
            const int r = r0 + GROUP_R * tid + u;
            slot[u] = -1;
            if (r < n) {
                const int4* ip = reinterpret_cast<const int4*>(rt[r].ids);
#pragma unroll
                for (int q = 0; q < ROUTE_K_MAX / 4; q++)
                    if (4 * q < K) {
                        const int4 v = ip[q];
                        if (4 * q + 0 < K && v.x == e) slot[u] = 4 * q + 0;
                        if (4 * q + 1 < K && v.y == e) slot[u] = 4 * q + 1;
                        if (4 * q + 2 < K && v.z == e) slot[u] = 4 * q + 2;
                        if (4 * q + 3 < K && v.w == e) slot[u] = 4 * q + 3;
                    }
            }
            mine += slot[u] >= 0;
        }
        int incl = mine; /* inclusive scan of the matches across the wave */
#pragma unroll
        for (int d = 1; d < WAVE; d <<= 1) {
            const int o = __shfl_up(incl, d, WAVE);
            if (lane >= d) incl += o;
        }
        if (lane == WAVE - 1) wave_n[wave] = incl;
        __syncthreads();
        int before = base + incl - mine, total = 0;
#pragma unroll
        for (int w = 0; w < GROUP_T / WAVE; w++) {
            if (w < wave) before += wave_n[w];
            total += wave_n[w];
        }
#pragma unroll
        for (int u = 0; u < GROUP_R; u++)
            if (slot[u] >= 0) {
                if (before < cap) pairs[(size_t)e * cap + before] = (r0 + GROUP_R * tid + u) * ROUTE_K_MAX + slot[u];
                before++;
            }
        base += total;
        __syncthreads();
    }
    if (tid == 0) count[e] = base < cap ? base : cap;
}

hipError_t launch_group(const route_out* rt, int n, int E, int K, int cap, int* count, int* pairs, hipStream_t s) {
    if (n < 1 || n > cap || E < 1 || K < 1 || K > ROUTE_K_MAX) return hipErrorInvalidValue;
    if (n > GROUP_T) group_many_kernel<<<E, GROUP_T, 0, s>>>(rt, n, K, cap, count, pairs);
    else group_kernel<<<E, GROUP_T, 0, s>>>(rt, n, K, cap, count, pairs);
    return hipGetLastError();
}

/* x[row][r] = x[row][r] + sum over slots k (in order) of ypart[row * K + k][r]: a float4 of columns a thread,
   its K parts all requested before the first add. */
__global__ __launch_bounds__(256) void reduce_rows_kernel(const float* __restrict__ ypart, float* __restrict__ x, int n, int K, int H) {
    const int row = blockIdx.y, c4 = blockIdx.x * blockDim.x + threadIdx.x;
    if (c4 >= H / 4) return;
    const float4* yp = reinterpret_cast<const float4*>(ypart + (size_t)row * K * H) + c4;
    float4 p[ROUTE_K_MAX];
#pragma unroll
    for (int k = 0; k < ROUTE_K_MAX; k++)
        if (k < K) p[k] = yp[(size_t)k * (H / 4)];
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < ROUTE_K_MAX; k++)
        if (k < K) {
            sum.x = sum.x + p[k].x; sum.y = sum.y + p[k].y;
            sum.z = sum.z + p[k].z; sum.w = sum.w + p[k].w;
        }
    float4* xp = reinterpret_cast<float4*>(x + (size_t)row * H) + c4;
    float4 v = *xp;
    v.x = v.x + sum.x; v.y = v.y + sum.y; v.z = v.z + sum.z; v.w = v.w + sum.w;
    *xp = v;
}

hipError_t launch_reduce_rows(const float* ypart, float* x, int n, int K, int H, hipStream_t s) {
    if (n < 1 || K < 1 || K > ROUTE_K_MAX || H % 4) return hipErrorInvalidValue;
    reduce_rows_kernel<<<dim3((H / 4 + 255) / 256, n), 256, 0, s>>>(ypart, x, n, K, H);
    return hipGetLastError();
}
