/**
 * kernels_decode.hip - The batch-1 decode kernels of the quantized
 * mixture-of-experts path on gfx950: upload (GGUF blocks to planes), the
 * exact widening checker, the exact RMSNorm + router + top-k, the expert
 * GEMVs (gate/up with SiLU, down with the weighted sum and the residual add),
 * the dense projections and the embedding.
 *
 * Reference counterparts (engine/src/model_cuda.cu unless noted):
 *   route_kernel       router_kernel :1544 + model.c route :667-703 (on the device)
 *   experts_in_kernel  experts_in_kernel :1566
 *   experts_down_kernel experts_down_kernel :1591 (+ the residual add)
 *   gemv_kernel        attn_in_kernel :870 (norm + q/k/v), matvec_add_kernel :1430,
 *                      head_kernel :1459
 *   embed_kernel       embed_kernel :854
 *   widen kernels      vitna_cuda_widen :5441 (widen_rows_kernel :5419)
 */

#include "gemv_impl.h"
#include "gmma_split.h"
#include "route_impl.h"

/* ------------------------------------------------------------------ */
/* Upload: GGUF blocks into planes                                     */
/* ------------------------------------------------------------------ */

__global__ void repack_kernel(const uint8_t* __restrict__ src, qmat m, size_t n_blocks) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    uint8_t* P0 = const_cast<uint8_t*>(m.p[0]);
    uint8_t* P1 = const_cast<uint8_t*>(m.p[1]);
    uint8_t* P2 = const_cast<uint8_t*>(m.p[2]);
    uint8_t* P3 = const_cast<uint8_t*>(m.p[3]);
    if (m.dtype == VITNA_DTYPE_Q8_0) {
        const uint8_t* b = src + i * 34;
        P1[i * 2] = b[0];
        P1[i * 2 + 1] = b[1];
        for (int j = 0; j < 32; j++) P0[i * 32 + j] = b[2 + j];
    } else if (m.dtype == VITNA_DTYPE_Q4_K) {
        const uint8_t* b = src + i * 144;
        for (int j = 0; j < 16; j++) P1[i * 16 + j] = b[j];
        for (int j = 0; j < 128; j++) P0[i * 128 + j] = b[16 + j];
    } else if (m.dtype == VITNA_DTYPE_Q6_K) {
        const uint8_t* b = src + i * 210;
        for (int j = 0; j < 128; j++) P0[i * 128 + j] = b[j];
        for (int j = 0; j < 64; j++) P1[i * 64 + j] = b[128 + j];
        for (int j = 0; j < 16; j++) P2[i * 16 + j] = b[192 + j];
        P3[i * 2] = b[208];
        P3[i * 2 + 1] = b[209];
    }
}

hipError_t launch_repack(const uint8_t* src, const qmat& dst, hipStream_t s) {
    if (dst.dtype != VITNA_DTYPE_Q8_0 && dst.dtype != VITNA_DTYPE_Q4_K && dst.dtype != VITNA_DTYPE_Q6_K) return hipErrorInvalidValue;
    const size_t n = (size_t)dst.rows * dst.nb;
    if (n == 0) return hipSuccess;
    repack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(src, dst, n);
    return hipGetLastError();
}

__global__ void widen_planes_kernel(qmat m, int e, float* __restrict__ out) {
    const size_t n = (size_t)m.rows * m.cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = widen_one(m, e, (int)(i / m.cols), (int)(i % m.cols));
}

hipError_t launch_widen_planes(const qmat& m, int e, float* out, hipStream_t s) {
    const size_t n = (size_t)m.rows * m.cols;
    if (n == 0) return hipSuccess;
    const unsigned g = (unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    widen_planes_kernel<<<g, 256, 0, s>>>(m, e, out);
    return hipGetLastError();
}

/* The same weights straight from the GGUF blocks, by a second reading of the
   formats, so the checker compares two independent ways of reading. */
__device__ __forceinline__ float half_at(const uint8_t* p) { return f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

__global__ void widen_blocks_kernel(const uint8_t* __restrict__ src, int dtype, size_t rows, size_t cols, float* __restrict__ out) {
    const size_t n = rows * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t row = i / cols, col = i % cols;
        float w = 0.0f;
        if (dtype == VITNA_DTYPE_F32) {
            w = reinterpret_cast<const float*>(src)[i];
        } else if (dtype == VITNA_DTYPE_Q8_0) {
            const uint8_t* b = src + (row * (cols / 32) + col / 32) * 34;
            w = (float)(int8_t)b[2 + col % 32] * half_at(b);
        } else if (dtype == VITNA_DTYPE_Q4_K) {
            const uint8_t* b = src + (row * (cols / 256) + col / 256) * 144;
            const int k = (int)(col % 256), g = k / 32, l = k % 32;
            const uint8_t* s = b + 4;
            const int sc = g < 4 ? (s[g] & 63) : ((s[g + 4] & 15) | ((s[g - 4] >> 6) << 4));
            const int mn = g < 4 ? (s[g + 4] & 63) : ((s[g + 4] >> 4) | ((s[g] >> 6) << 4));
            const int q = (b[16 + 32 * (g / 2) + l] >> (4 * (g & 1))) & 15;
            const float d1 = half_at(b) * (float)sc, m1 = half_at(b + 2) * (float)mn;
            const float p = d1 * (float)q;
            w = p - m1;
        } else if (dtype == VITNA_DTYPE_Q6_K) {
            const uint8_t* b = src + (row * (cols / 256) + col / 256) * 210;
            const int k = (int)(col % 256), h = k / 128, r = (k % 128) / 32, l = k % 32;
            const int lo = (b[64 * h + 32 * (r & 1) + l] >> (4 * (r >> 1))) & 15;
            const int hi = (b[128 + 32 * h + l] >> (2 * r)) & 3;
            const float ds = half_at(b + 208) * (float)(int8_t)b[192 + k / 16];
            w = ds * (float)((lo | (hi << 4)) - 32);
        }
        out[i] = w;
    }
}

hipError_t launch_widen_blocks(const uint8_t* src, int dtype, size_t rows, size_t cols, float* out, hipStream_t s) {
    const size_t n = rows * cols;
    if (n == 0) return hipSuccess;
    const unsigned g = (unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    widen_blocks_kernel<<<g, 256, 0, s>>>(src, dtype, rows, cols, out);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ */
/* RMSNorm + router, in the reference CPU's order                      */
/* ------------------------------------------------------------------ */


/* Four router rows a block (sixteen lanes of wave 0 a row). NT threads: 64 (a pass of several rows), or 256 for
   one row: the other waves help load x (and its attention parts, route_args::parts), so that every load goes out
   in one round, ahead of wave 0's router weights. */
template <int NCH, int NT>
__global__ __launch_bounds__(NT) void route_kernel(route_args a) {
    extern __shared__ float sh[];
    float* sx = sh;             /* H: x */
    float* sxn = sh + a.H;      /* H: normalized */
    __shared__ float chains[16];
    __shared__ float inv_s;
    const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, rrow = blockIdx.x * 4 + (lane >> 4);
    const int tok = blockIdx.y;
    const float* x = a.x + (size_t)tok * a.H;
    constexpr int NF4 = NCH * 4, X4 = (NF4 + NT - 1) / NT; /* float4 of x, and a thread's share */
#define X4_OK(i) (NF4 % NT == 0 || tid + NT * (i) < NF4)
    /* wave 0's chains of router weights; with parts (NT = 256), after x and the parts, so that the norm, which
       waits for them, waits for no weight load (at NT = 64 that order leaves the registers short: spills) */
    float w[NCH];
    const bool has_row = tid < 64 && rrow < a.E;
    auto load_router = [&]() {
        if (tid < 64) {
            const float* wr = a.router + (size_t)(rrow < a.E ? rrow : 0) * a.H + j;
#pragma unroll
            for (int m = 0; m < NCH; m++) w[m] = wr[16 * m];
        }
    };
    if constexpr (NT == 64) load_router();
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4 xv[X4];
#pragma unroll
    for (int i = 0; i < X4; i++) xv[i] = x4[X4_OK(i) ? tid + NT * i : 0];
    constexpr int NP = NT > 64 ? OPROJ_PARTS_MAX : 1;
    float4 pv[NP][X4];
    const bool with_parts = NT > 64 && a.parts;
    if (with_parts) {
        /* (every slot loaded, those past n_parts as the last part, unused: no branch between the loads) */
        const float4* p4 = reinterpret_cast<const float4*>(a.parts);
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
            for (int i = 0; i < X4; i++) pv[p][i] = p4[(size_t)min(p, a.n_parts - 1) * (a.H / 4) + (X4_OK(i) ? tid + NT * i : 0)];
    }
    if constexpr (NT > 64) {
        __builtin_amdgcn_sched_barrier(0);
        load_router();
    }
    if (with_parts) {
#pragma unroll
        for (int i = 0; i < X4; i++) {
            /* attn_resid, a float4 at a time: the parts in group order, then x */
            float4 sum = pv[0][i];
#pragma unroll
            for (int p = 1; p < NP; p++) {
                const bool on = p < a.n_parts;
                sum.x = on ? sum.x + pv[p][i].x : sum.x; sum.y = on ? sum.y + pv[p][i].y : sum.y;
                sum.z = on ? sum.z + pv[p][i].z : sum.z; sum.w = on ? sum.w + pv[p][i].w : sum.w;
            }
            xv[i].x += sum.x; xv[i].y += sum.y; xv[i].z += sum.z; xv[i].w += sum.w;
        }
    }
#pragma unroll
    for (int i = 0; i < X4; i++)
        if (X4_OK(i)) reinterpret_cast<float4*>(sx)[tid + NT * i] = xv[i];
    __syncthreads();
    if (tid < 16) {
        /* engine/src/kernels.c:115-140: sixteen chains of squares (H a multiple of 16) */
        float acc = 0.0f;
#pragma unroll 16
        for (int m = 0; m < NCH; m++) acc = fmaf(sx[16 * m + tid], sx[16 * m + tid], acc);
        chains[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        float v[8];
        for (int q = 0; q < 8; q++) v[q] = chains[q] + chains[q + 8];
        const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
        const float ss = (s0 + s2) + (s1 + s3);
        /* kernels.c:146: 1 / sqrtf(ss / n + eps), each step correctly rounded */
        inv_s = 1.0f / sqrtf(ss / (float)a.H + a.eps);
    }
    __syncthreads();
    const float inv = inv_s;
    {
        const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
        float4 nw[X4];
#pragma unroll
        for (int i = 0; i < X4; i++) nw[i] = X4_OK(i) ? w4[tid + NT * i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < X4; i++) {
            if (!X4_OK(i)) continue;
            const float4 xv = reinterpret_cast<const float4*>(sx)[tid + NT * i];
            float4 o;
            o.x = (xv.x * inv) * nw[i].x; o.y = (xv.y * inv) * nw[i].y;
            o.z = (xv.z * inv) * nw[i].z; o.w = (xv.w * inv) * nw[i].w;
            reinterpret_cast<float4*>(sxn)[tid + NT * i] = o;
            if (a.xn_out && blockIdx.x == 0) reinterpret_cast<float4*>(a.xn_out + (size_t)tok * a.H)[tid + NT * i] = o;
        }
    }
    __syncthreads();
    if (tid >= 64) return;
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < NCH; m++) acc = fmaf(w[m], sxn[16 * m + j], acc);
    const float logit = fold16_lanes(acc);
    if (has_row && j == 0) a.logits[(size_t)tok * a.E + rrow] = logit;
#undef X4_OK
}

hipError_t launch_route(const route_args& a, hipStream_t s) {
    if (a.H % 256 || a.E < 1 || a.E > ROUTE_E_MAX || a.n_rows < 1) return hipErrorInvalidValue;
    if (a.parts && (a.n_rows != 1 || a.n_parts < 1 || a.n_parts > OPROJ_PARTS_MAX)) return hipErrorInvalidValue;
    const dim3 grid((a.E + 3) / 4, a.n_rows);
    const size_t lds = 2 * (size_t)a.H * sizeof(float);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    /* with parts: rows of at most ROUTE_PARTS_HMAX (wider ones would hold the router chain and every part's
       loads past the registers) */
    if (a.parts && a.H > ROUTE_PARTS_HMAX) return hipErrorInvalidValue;
#define ROUTE_CASE(N)                                                                   \
    case N:                                                                             \
        if (a.parts || a.n_rows == 1) route_kernel<N, 256><<<grid, 256, lds, s>>>(a);  \
        else route_kernel<N, 64><<<grid, 64, lds, s>>>(a);                              \
        break;
    switch (a.H / 16) {
        ROUTE_CASE(16) ROUTE_CASE(32) ROUTE_CASE(64) ROUTE_CASE(128)
        case 256: route_kernel<256, 64><<<grid, 64, lds, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
#undef ROUTE_CASE
    return hipGetLastError();
}

__global__ void route_check_kernel(const float* __restrict__ logits, int E, int K, int renorm, route_out* out) {
    __shared__ float slg[ROUTE_E_MAX];
    __shared__ route_out o;
    wave_route(logits, E, K, renorm, &o, slg);
    __syncthreads();
    if (threadIdx.x < sizeof(route_out) / 4) reinterpret_cast<int32_t*>(out)[threadIdx.x] = reinterpret_cast<const int32_t*>(&o)[threadIdx.x];
}

/* One wave a row: the routing of n_rows rows of logits (row stride E) into out; with sp.xs, then the row's
   split for the grouped experts (gmma_split.h, runs of G columns). */
template <int G>
__global__ __launch_bounds__(64) void topk_kernel(const float* __restrict__ logits, int E, int K, int renorm, route_out* out,
                                                  topk_split sp) {
    __shared__ float slg[ROUTE_E_MAX];
    const int r = blockIdx.x;
    wave_route(logits + (size_t)r * E, E, K, renorm, out + r, slg);
    if constexpr (G > 0)
        for (int g = threadIdx.x; g < sp.H / G; g += 64)
            gsplit_run<G>(sp.x + (size_t)r * sp.H, sp.H, g, sp.xs + (size_t)r * 2 * sp.H, sp.sums + (size_t)r * (sp.H / G));
}

hipError_t launch_topk(const float* logits, int n_rows, int E, int K, int renorm, route_out* out, hipStream_t s, const topk_split* sp) {
    if (n_rows < 1 || E < 1 || E > ROUTE_E_MAX || E % 4 || K < 1 || K > ROUTE_K_MAX || K > E) return hipErrorInvalidValue;
    const topk_split none = {nullptr, nullptr, nullptr, 0, 0};
    if (sp && sp->xs) {
        if (sp->H % sp->gran || (sp->gran != 16 && sp->gran != 32)) return hipErrorInvalidValue;
        if (sp->gran == 32) topk_kernel<32><<<n_rows, 64, 0, s>>>(logits, E, K, renorm, out, *sp);
        else topk_kernel<16><<<n_rows, 64, 0, s>>>(logits, E, K, renorm, out, *sp);
    } else {
        topk_kernel<0><<<n_rows, 64, 0, s>>>(logits, E, K, renorm, out, none);
    }
    return hipGetLastError();
}

hipError_t launch_route_check(const float* logits, int E, int K, int renorm, route_out* out, hipStream_t s) {
    if (E < 1 || E > ROUTE_E_MAX || E % 4 || K < 1 || K > ROUTE_K_MAX || K > E) return hipErrorInvalidValue;
    route_check_kernel<<<1, 64, 0, s>>>(logits, E, K, renorm, out);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ */
/* Experts, one token                                                  */
/* ------------------------------------------------------------------ */



/* The experts' gate and up rows against the normalized token: units (slot k, row r), k in the order of
   rt.chosen (largest logit first), act[k * I + r] = silu(gate . xn) * (up . xn). A wave takes 2 RPW
   consecutive units (one slot, except where a slot ends) and, when it routes the logits itself, runs only the
   selection rounds up to its slot before its loads go out. */
template <int DT, int LPR, int SPL, int NS>
__device__ __forceinline__ void experts_in_body(const experts_in_args& a, int wave, int lane) {
    constexpr int RPW = WAVE / LPR;
    const int sub = lane / LPR, al = lane % LPR, wib = threadIdx.x / WAVE;
    const int I = a.gate.rows, units = a.K * I;
    const int b = wave * 2 * RPW; /* this wave's first unit */
    xslice xs[SPL];
    __shared__ int wch[4][ROUTE_K_MAX];
    __shared__ route_out wrt[4];
    __shared__ float slg[4][NS * 64];
    int kmax = (min(b + 2 * RPW, units) - 1) / I;
    if (a.logits) {
        /* the selection rounds (the reference's passes, engine/src/model.c:626-650) up to slot kmax */
        float lg[NS];
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int e = lane + 64 * i;
            lg[i] = a.logits[e < a.E ? e : 0];
        }
        /* the token's activations requested right behind the logits: both were written by the router, and each
           round trip is long; the selection below waits for the logits only */
#pragma unroll
        for (int j = 0; j < SPL; j++) load_xslice(DT, lane % LPR + LPR * j, a.xn, xs[j]);
        bool nan = false;
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int e = lane + 64 * i;
            lg[i] = e < a.E ? lg[i] : -INFINITY;
            nan |= e < a.E && lg[i] != lg[i];
        }
        if (__any(nan)) {
            wave_route_n<NS>(a.logits, a.E, a.K, a.renorm, &wrt[wib], slg[wib]);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            if (lane < a.K) wch[wib][lane] = wrt[wib].chosen[lane];
        } else {
            uint32_t key[NS];
#pragma unroll
            for (int i = 0; i < NS; i++) key[i] = lane + 64 * i < a.E ? order_key(lg[i]) : 0u;
            for (int k = 0; k <= kmax; k++) {
                uint32_t m = key[0];
#pragma unroll
                for (int i = 1; i < NS; i++) m = max(m, key[i]);
                m = wave_max_u32(m);
                int pick = -1;
#pragma unroll
                for (int i = 0; i < NS; i++) {
                    const uint64_t bb = __ballot(key[i] == m);
                    if (pick < 0 && bb) pick = 64 * i + (int)__builtin_ctzll(bb);
                }
#pragma unroll
                for (int i = 0; i < NS; i++)
                    if (pick == lane + 64 * i) key[i] = 0u;
                if (lane == 0) wch[wib][k] = pick;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < SPL; j++) load_xslice(DT, lane % LPR + LPR * j, a.xn, xs[j]);
        if (lane < a.K) wch[wib][lane] = a.rt->chosen[lane];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    int u[2];
    qraw g[2][SPL], v[2][SPL];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        u[q] = b + q * RPW + sub;
        const int uu = u[q] < units ? u[q] : units - 1;
        const int k = uu / I, r = uu - k * I, e = wch[wib][k];
#pragma unroll
        for (int j = 0; j < SPL; j++) {
            slice_load<DT>(a.gate, e, r, al + LPR * j, g[q][j]);
            slice_load<DT>(a.up, e, r, al + LPR * j, v[q][j]);
        }
    }
#pragma unroll
    for (int q = 0; q < 2; q++) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < SPL; j++) {
            pg += slice_dot<DT>(g[q][j], al + LPR * j, xs[j]);
            pu += slice_dot<DT>(v[q][j], al + LPR * j, xs[j]);
        }
        pg = row_sum<LPR>(pg);
        pu = row_sum<LPR>(pu);
        if (al == LPR - 1 && u[q] < units) a.act[u[q]] = silu_mul(pg, pu);
    }
}

template <int DT, int LPR, int SPL>
__global__ __launch_bounds__(256) void experts_in_kernel(experts_in_args a) {
    constexpr int RPW = WAVE / LPR;
    const int lane = threadIdx.x & 63;
    if (blockIdx.y) {
        /* token blockIdx.y of several: its activations, routing (or logits) and outputs; a single token's arithmetic */
        const size_t r = blockIdx.y;
        a.xn += r * a.gate.cols;
        a.rt += r;
        a.act += r * a.K * a.gate.rows;
        if (a.logits) a.logits += r * a.E;
    }
    const int wave = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    const int uwaves = (a.K * a.gate.rows + 2 * RPW - 1) / (2 * RPW); /* waves with units */
    if (wave >= uwaves) {
        /* the wave past the units publishes the whole routing for the down projection */
        if (wave == uwaves && a.logits) {
            __shared__ float pslg[ROUTE_E_MAX];
            wave_route(a.logits, a.E, a.K, a.renorm, a.rt, pslg);
        }
        return;
    }
    if (!a.logits || a.E <= 64) experts_in_body<DT, LPR, SPL, 1>(a, wave, lane);
    else if (a.E <= 128) experts_in_body<DT, LPR, SPL, 2>(a, wave, lane);
    else if (a.E <= 256) experts_in_body<DT, LPR, SPL, 4>(a, wave, lane);
    else experts_in_body<DT, LPR, SPL, 8>(a, wave, lane);
}

template <int DT, int LPR, int SPL>
static hipError_t ein_launch(const experts_in_args& a, hipStream_t s, int n_rows) {
    constexpr int RPW = WAVE / LPR;
    const int units = a.K * a.gate.rows;
    const int waves = (units + 2 * RPW - 1) / (2 * RPW) + 1; /* the last one publishes the routing */
    const int blocks = (waves + 3) / 4;
    experts_in_kernel<DT, LPR, SPL><<<dim3(blocks, n_rows), 256, 0, s>>>(a);
    return hipGetLastError();
}

template <int DT>
static hipError_t ein_dispatch(const experts_in_args& a, hipStream_t s, int n) {
    switch (a.gate.cols / 32) {
        case 4: return ein_launch<DT, 4, 1>(a, s, n);
        case 8: return ein_launch<DT, 8, 1>(a, s, n);
        case 16: return ein_launch<DT, 16, 1>(a, s, n);
        case 32: return ein_launch<DT, 32, 1>(a, s, n);
        case 64: return ein_launch<DT, 64, 1>(a, s, n);
        case 128: return ein_launch<DT, 64, 2>(a, s, n);
        case 256: return ein_launch<DT, 64, 4>(a, s, n);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_experts_in(const experts_in_args& a, hipStream_t s, int n_rows) {
    if (a.gate.dtype != a.up.dtype || a.gate.rows != a.up.rows || a.gate.cols != a.up.cols || a.K < 1 || a.K > ROUTE_K_MAX ||
        n_rows < 1 || n_rows > 65535)
        return hipErrorInvalidValue;
    if (a.logits && (a.E < a.K || a.E > ROUTE_E_MAX || a.E % 4)) return hipErrorInvalidValue;
    switch (a.gate.dtype) {
        case VITNA_DTYPE_Q8_0: return ein_dispatch<VITNA_DTYPE_Q8_0>(a, s, n_rows);
        case VITNA_DTYPE_Q4_K: return ein_dispatch<VITNA_DTYPE_Q4_K>(a, s, n_rows);
        case VITNA_DTYPE_Q6_K: return ein_dispatch<VITNA_DTYPE_Q6_K>(a, s, n_rows);
        default: return hipErrorInvalidValue;
    }
}

/* One output row a wave: every (expert, slice) item of the row among the 64
   lanes, IPL items a lane, each lane's items fixed for every row, so its
   activations stay in registers. The weighted sum over experts is reduced
   across the wave. A wave has NR rows' weights in flight at once: two, or one
   where a lane's items are many (IPL 6 and more: two rows' weights and every
   item's activations would not fit the registers). */
template <int DT, int IPL>
__global__ __launch_bounds__(256) void experts_down_kernel(experts_down_args a) {
    constexpr int NR = IPL >= 6 ? 1 : 2;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE, nwaves = gridDim.x * (blockDim.x / WAVE);
    const int H = a.down.rows, I = a.down.cols, S = I / 32, N = a.K * S;
    if (blockIdx.y) {
        /* token blockIdx.y of several (no parts then): its activations, routing and output row */
        const size_t r = blockIdx.y;
        a.act += r * a.K * I;
        a.rt += r;
        a.y += r * H;
    }
    xslice xs[IPL];
    float wk[IPL];
    int ek[IPL], tk[IPL];
#pragma unroll
    for (int j = 0; j < IPL; j++) {
        const int i = lane + 64 * j;
        const bool ok = i < N;
        const int k = ok ? i / S : 0;
        tk[j] = ok ? i - k * S : 0;
        ek[j] = a.rt->chosen[k];
        wk[j] = ok ? a.rt->cw[k] : 0.0f;
        load_xslice(DT, tk[j], a.act + (size_t)k * I, xs[j]);
    }
    /* what the sums are added to (the residual, with the attention's parts), requested before the weights so that
       its loads land under them */
    __builtin_amdgcn_sched_barrier(0); /* the activations' sums first: their waits then count no later load */
    /* (without parts the loads read y again, unused: no branch, so the waits below count these loads exactly) */
    float yx[NR], yp[NR][OPROJ_PARTS_MAX];
    const float* pp = a.parts ? a.parts : a.y;
    const int np = a.parts ? a.n_parts : 1;
#pragma unroll
    for (int h = 0; h < NR; h++) {
        const int r = min(wave + h * nwaves, H - 1);
        yx[h] = a.y[r];
        attn_parts_load(pp, np, (size_t)H, (size_t)r, yp[h]);
    }
    for (int r0 = wave; r0 < H; r0 += NR * nwaves) {
        qraw q[NR][IPL];
#pragma unroll
        for (int h = 0; h < NR; h++) {
            const int r = r0 + h * nwaves < H ? r0 + h * nwaves : H - 1;
#pragma unroll
            for (int j = 0; j < IPL; j++) slice_load<DT, (IPL >= 6)>(a.down, ek[j], r, tk[j], q[h][j]);
        }
#pragma unroll
        for (int h = 0; h < NR; h++) {
            float p = 0.f;
#pragma unroll
            for (int j = 0; j < IPL; j++) p = fmaf(wk[j], slice_dot<DT, (IPL >= 6)>(q[h][j], tk[j], xs[j]), p);
            p = row_sum<64>(p);
            const int r = r0 + h * nwaves;
            if (lane == 63 && r < H) {
                if (!a.add) a.y[r] = p;
                else if (r0 == wave) {
                    /* (the empty asm keeps the compiler from summing before the loop, which would wait there) */
#pragma unroll
                    for (int i = 0; i < OPROJ_PARTS_MAX; i++) asm volatile("" : "+v"(yp[h][i]));
                    a.y[r] = (a.parts ? attn_parts_sum(yx[h], yp[h], a.n_parts) : yx[h]) + p;
                }
                else a.y[r] = (a.parts ? attn_resid(a.y[r], a.parts, a.n_parts, (size_t)H, (size_t)r) : a.y[r]) + p;
            }
        }
    }
}

template <int DT, int IPL>
static hipError_t edn_launch(const experts_down_args& a, hipStream_t s, int n_rows) {
    const int waves = IPL >= 6 ? a.down.rows : (a.down.rows + 1) / 2;
    experts_down_kernel<DT, IPL><<<dim3((waves + 3) / 4, n_rows), 256, 0, s>>>(a);
    return hipGetLastError();
}

template <int DT>
static hipError_t edn_dispatch(const experts_down_args& a, hipStream_t s, int n) {
    const int N = a.K * (a.down.cols / 32), ipl = (N + 63) / 64;
    switch (ipl) {
        case 1: return edn_launch<DT, 1>(a, s, n);
        case 2: return edn_launch<DT, 2>(a, s, n);
        case 3: return edn_launch<DT, 3>(a, s, n);
        case 4: return edn_launch<DT, 4>(a, s, n);
        case 5: return edn_launch<DT, 5>(a, s, n);
        case 6: return edn_launch<DT, 6>(a, s, n);
        case 8: return edn_launch<DT, 8>(a, s, n);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_experts_down(const experts_down_args& a, hipStream_t s, int n_rows) {
    if (a.K < 1 || a.K > ROUTE_K_MAX || a.down.cols % 32 || n_rows < 1 || n_rows > 65535 || (n_rows > 1 && a.parts))
        return hipErrorInvalidValue;
    switch (a.down.dtype) {
        case VITNA_DTYPE_Q8_0: return edn_dispatch<VITNA_DTYPE_Q8_0>(a, s, n_rows);
        case VITNA_DTYPE_Q4_K: return edn_dispatch<VITNA_DTYPE_Q4_K>(a, s, n_rows);
        case VITNA_DTYPE_Q6_K: return edn_dispatch<VITNA_DTYPE_Q6_K>(a, s, n_rows);
        default: return hipErrorInvalidValue;
    }
}

/* ------------------------------------------------------------------ */
/* Dense projections: gemv_impl.h, instantiated in gemv_q4/q6/q8.hip    */
/* ------------------------------------------------------------------ */

int gemv_device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) dev = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    }
    return cus;
}

hipError_t launch_gemv(const gemv_args& a, hipStream_t s) {
    if (a.n < 1 || a.n > 3) return hipErrorInvalidValue;
    for (int i = 1; i < a.n; i++)
        if (a.w[i].cols != a.w[0].cols) return hipErrorInvalidValue;
    const int d0 = a.w[0].dtype, d1 = a.n > 1 ? a.w[1].dtype : d0, d2 = a.n > 2 ? a.w[2].dtype : d1;
    bool served = false;
    hipError_t e = gemv_combo_q4(a, d0, d1, d2, s, &served);
    if (!served) e = gemv_combo_q6(a, d0, d1, d2, s, &served);
    if (!served) e = gemv_combo_q8(a, d0, d1, d2, s, &served);
    if (served || a.n == 1) return served ? e : hipErrorInvalidValue;
    /* a mix of dtypes no fused instantiation holds: one launch a matrix, each a single-dtype kernel */
    for (int i = 0; i < a.n; i++) {
        gemv_args one = a;
        one.n = 1;
        one.w[0] = a.w[i];
        one.y[0] = a.y[i];
        one.ystride[0] = a.ystride[i];
        e = launch_gemv(one, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

/* ------------------------------------------------------------------ */
/* Embedding                                                           */
/* ------------------------------------------------------------------ */

__global__ void embed_kernel(qmat m, const int32_t* token_dev, int token, float* __restrict__ x) {
    const int t = token_dev ? *token_dev : token;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < m.cols; c += gridDim.x * blockDim.x) x[c] = widen_one(m, 0, t, c);
}

hipError_t launch_embed(const qmat& embed, const int32_t* token_dev, int token, float* x, hipStream_t s) {
    embed_kernel<<<(embed.cols + 255) / 256, 256, 0, s>>>(embed, token_dev, token, x);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ */
/* Seeded N(0,1) fill (keys and values of a synthetic cache)           */
/* ------------------------------------------------------------------ */

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(float* __restrict__ out, size_t n, uint64_t seed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t h = mix64(seed * 0x9e3779b97f4a7c15ull + i);
        const float u1 = ((float)(uint32_t)(h >> 40) + 1.0f) * (1.0f / 16777217.0f);
        const float u2 = (float)(uint32_t)(h & 0xffffff) * (1.0f / 16777216.0f);
        out[i] = sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
    }
}

hipError_t launch_fill_normal(float* out, size_t n, uint64_t seed, hipStream_t s) {
    if (!n) return hipSuccess;
    fill_normal_kernel<<<4096, 256, 0, s>>>(out, n, seed);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ */
/* A plain copy of known size: the yardstick hardware counters of bytes  */
/* read and written are scaled by.                                       */
/* ------------------------------------------------------------------ */

__global__ void copy_probe_kernel(const float4* __restrict__ src, float4* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) dst[i] = src[i];
}

hipError_t launch_copy_probe(const void* src, void* dst, size_t bytes, hipStream_t s) {
    if (bytes % 16) return hipErrorInvalidValue;
    copy_probe_kernel<<<2048, 256, 0, s>>>(reinterpret_cast<const float4*>(src), reinterpret_cast<float4*>(dst), bytes / 16);
    return hipGetLastError();
}
