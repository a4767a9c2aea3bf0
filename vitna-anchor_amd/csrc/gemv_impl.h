/**
 * gemv_impl.h - The dense-projection GEMV (q/k/v with the RMSNorm prologue,
 * o-projection with the residual, LM head) as templates over the three
 * matrices' dtypes, the row width and the rows a wave takes at a time. Each
 * gemv_*.hip instantiates some dtype combinations, so they compile in
 * parallel; kernels_decode.hip's launch_gemv dispatches among them.
 */

#ifndef VITNA_GEMV_IMPL_H
#define VITNA_GEMV_IMPL_H

#include "vitna_kernels.h"

int gemv_device_cus();

/* ------------------------------------------------------------------ */
/* Dense projections                                                   */
/* ------------------------------------------------------------------ */

/* Units of RPW rows, U units in flight a wave: their loads all issued before
   any of their arithmetic. */
template <int DT, int LPR, int SPL, int U>
__device__ __forceinline__ void gemv_rows(const qmat& w, float* __restrict__ y, int add, const xslice* xs, int unit0, int ustep,
                                          int lane, int unit_end = 0x7fffffff) {
    constexpr int RPW = WAVE / LPR;
    const int sub = lane / LPR, al = lane % LPR;
    const int units = min((w.rows + RPW - 1) / RPW, unit_end);
    for (int u = unit0; u < units; u += U * ustep) {
        qraw q[U][SPL];
        int r[U];
#pragma unroll
        for (int h = 0; h < U; h++) {
            r[h] = (u + h * ustep) * RPW + sub;
            const int rr = r[h] < w.rows ? r[h] : w.rows - 1;
#pragma unroll
            for (int j = 0; j < SPL; j++) {
                if (DT == VITNA_DTYPE_F32) continue;
                slice_load<DT>(w, 0, rr, al + LPR * j, q[h][j]);
            }
        }
#pragma unroll
        for (int h = 0; h < U; h++) {
            const int rr = r[h] < w.rows ? r[h] : w.rows - 1;
            float p = 0.f;
#pragma unroll
            for (int j = 0; j < SPL; j++) {
                if (DT == VITNA_DTYPE_F32)
                    p += slice_dot_f32(reinterpret_cast<const float*>(w.p[0]) + (size_t)rr * w.cols, al + LPR * j, xs[j]);
                else
                    p += slice_dot<DT>(q[h][j], al + LPR * j, xs[j]);
            }
            p = row_sum<LPR>(p);
            if (al == LPR - 1 && r[h] < w.rows) y[r[h]] = add ? y[r[h]] + p : p;
        }
    }
}


template <int D0, int D1, int D2, int LPR, int SPL, bool NORM, int GEMV_U>
__global__ __launch_bounds__(256) void gemv_kernel(gemv_args a) {
    extern __shared__ float sh[];
    const int lane = threadIdx.x & 63;
    const int H = a.w[0].cols;
    if (blockIdx.y) {
        /* row blockIdx.y of several: its vector and outputs; the arithmetic is a single vector's */
        a.x += (size_t)blockIdx.y * a.xstride;
        for (int i = 0; i < 3; i++) a.y[i] += (size_t)blockIdx.y * a.ystride[i];
    }
    const float* xin = a.x;
    if (NORM) {
        /* up to eight float4 of x and of the weights a thread (H at most 8192, launch_gemv checks) */
        __shared__ float red[4];
        const int n4 = H / 4;
        float4 xv[8], wv[8];
        const float4* x4 = reinterpret_cast<const float4*>(a.x);
        const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
#pragma unroll
        for (int i = 0; i < 8; i++)
            if ((int)threadIdx.x + 256 * i < n4) { xv[i] = x4[threadIdx.x + 256 * i]; wv[i] = w4[threadIdx.x + 256 * i]; }
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if ((int)threadIdx.x + 256 * i < n4) {
                ss = fmaf(xv[i].x, xv[i].x, ss); ss = fmaf(xv[i].y, xv[i].y, ss);
                ss = fmaf(xv[i].z, xv[i].z, ss); ss = fmaf(xv[i].w, xv[i].w, ss);
            }
        ss = wave_sum(ss);
        if (lane == 0) red[threadIdx.x / WAVE] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = 1.0f / sqrtf(ss / (float)H + a.eps);
#pragma unroll
        for (int i = 0; i < 8; i++)
            if ((int)threadIdx.x + 256 * i < n4) {
                float4 o;
                o.x = (xv[i].x * inv) * wv[i].x; o.y = (xv[i].y * inv) * wv[i].y;
                o.z = (xv[i].z * inv) * wv[i].z; o.w = (xv[i].w * inv) * wv[i].w;
                reinterpret_cast<float4*>(sh)[threadIdx.x + 256 * i] = o;
            }
        __syncthreads();
        xin = sh;
    }
    xslice xs[SPL];
    const int wave = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE, nwaves = gridDim.x * (blockDim.x / WAVE);
    constexpr int RPW = WAVE / LPR;
    int units[3], batches = 0;
    for (int i = 0; i < 3; i++) {
        units[i] = i < a.n ? (a.w[i].rows + RPW - 1) / RPW : 0;
        batches += (units[i] + GEMV_U - 1) / GEMV_U;
    }
    if (nwaves >= batches) {
        /* one pass: wave w takes GEMV_U consecutive units of one matrix, so all its loads go out together */
        int wb = 0;
        for (int i = 0; i < a.n; i++) {
            const int nb = (units[i] + GEMV_U - 1) / GEMV_U;
            if (wave >= wb && wave < wb + nb) {
                const int u0 = (wave - wb) * GEMV_U;
                if (i == 0) {
#pragma unroll
                    for (int j = 0; j < SPL; j++) load_xslice(D0, lane % LPR + LPR * j, xin, xs[j]);
                    gemv_rows<D0, LPR, SPL, GEMV_U>(a.w[0], a.y[0], a.add, xs, u0, 1, lane, u0 + GEMV_U);
                } else if (i == 1) {
#pragma unroll
                    for (int j = 0; j < SPL; j++) load_xslice(D1, lane % LPR + LPR * j, xin, xs[j]);
                    gemv_rows<D1, LPR, SPL, GEMV_U>(a.w[1], a.y[1], a.add, xs, u0, 1, lane, u0 + GEMV_U);
                } else {
#pragma unroll
                    for (int j = 0; j < SPL; j++) load_xslice(D2, lane % LPR + LPR * j, xin, xs[j]);
                    gemv_rows<D2, LPR, SPL, GEMV_U>(a.w[2], a.y[2], a.add, xs, u0, 1, lane, u0 + GEMV_U);
                }
            }
            wb += nb;
        }
        return;
    }
    /* several passes: the matrices' units concatenated; wave w takes units w, w + nwaves, ... */
    int base = 0;
    for (int i = 0; i < a.n; i++) {
        int first = (wave - base) % nwaves;
        if (first < 0) first += nwaves;
        if (first < units[i]) {
            if (i == 0) {
#pragma unroll
                for (int j = 0; j < SPL; j++) load_xslice(D0, lane % LPR + LPR * j, xin, xs[j]);
                gemv_rows<D0, LPR, SPL, GEMV_U>(a.w[0], a.y[0], a.add, xs, first, nwaves, lane);
            } else if (i == 1) {
#pragma unroll
                for (int j = 0; j < SPL; j++) load_xslice(D1, lane % LPR + LPR * j, xin, xs[j]);
                gemv_rows<D1, LPR, SPL, GEMV_U>(a.w[1], a.y[1], a.add, xs, first, nwaves, lane);
            } else {
#pragma unroll
                for (int j = 0; j < SPL; j++) load_xslice(D2, lane % LPR + LPR * j, xin, xs[j]);
                gemv_rows<D2, LPR, SPL, GEMV_U>(a.w[2], a.y[2], a.add, xs, first, nwaves, lane);
            }
        }
        base += units[i];
    }
}

template <int D0, int D1, int D2, bool NORM, int U>
static hipError_t gemv_launch(const gemv_args& a, int blocks, size_t lds, hipStream_t s) {
    const dim3 grid(blocks, a.rows > 1 ? a.rows : 1);
    switch (a.w[0].cols / 32) {
        case 4: gemv_kernel<D0, D1, D2, 4, 1, NORM, U><<<grid, 256, lds, s>>>(a); break;
        case 8: gemv_kernel<D0, D1, D2, 8, 1, NORM, U><<<grid, 256, lds, s>>>(a); break;
        case 16: gemv_kernel<D0, D1, D2, 16, 1, NORM, U><<<grid, 256, lds, s>>>(a); break;
        case 32: gemv_kernel<D0, D1, D2, 32, 1, NORM, U><<<grid, 256, lds, s>>>(a); break;
        case 64: gemv_kernel<D0, D1, D2, 64, 1, NORM, U><<<grid, 256, lds, s>>>(a); break;
        case 128: gemv_kernel<D0, D1, D2, 64, 2, NORM, U><<<grid, 256, lds, s>>>(a); break;
        case 256: gemv_kernel<D0, D1, D2, 64, 4, NORM, U><<<grid, 256, lds, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

/* Rows a wave takes at a time (U): the most of 4, 2, 1 that still gives two waves a SIMD in one pass; when
   even U = 4 needs more than four blocks a CU, four blocks a CU loop over the rows. */
template <int D0, int D1, int D2, bool NORM>
static hipError_t gemv_by_width(const gemv_args& a, hipStream_t s) {
    const int S = a.w[0].cols / 32;
    const int lpr = S < 64 ? S : 64, rpw = WAVE / lpr;
    int units[3] = {0, 0, 0};
    for (int i = 0; i < a.n; i++) units[i] = (a.w[i].rows + rpw - 1) / rpw;
    auto batches = [&](int u) { return (units[0] + u - 1) / u + (units[1] + u - 1) / u + (units[2] + u - 1) / u; };
    const int cus = gemv_device_cus(), want = 8 * cus; /* waves: two a SIMD */
    const size_t lds = NORM ? (size_t)a.w[0].cols * sizeof(float) : 0;
    if (lds > 64 * 1024 || (NORM && a.w[0].cols > 8192)) return hipErrorInvalidValue;
    if (batches(4) >= want) {
        int blocks = (batches(4) + 3) / 4;
        blocks = blocks < 4 * cus ? blocks : 4 * cus;
        return gemv_launch<D0, D1, D2, NORM, 4>(a, blocks, lds, s);
    }
    if (batches(2) >= want) return gemv_launch<D0, D1, D2, NORM, 2>(a, (batches(2) + 3) / 4, lds, s);
    return gemv_launch<D0, D1, D2, NORM, 1>(a, (batches(1) + 3) / 4 > 0 ? (batches(1) + 3) / 4 : 1, lds, s);
}

template <int D0, int D1, int D2>
static hipError_t gemv_norm(const gemv_args& a, hipStream_t s) {
    return a.norm_w ? gemv_by_width<D0, D1, D2, true>(a, s) : gemv_by_width<D0, D1, D2, false>(a, s);
}

/* Instantiated in gemv_q4.hip, gemv_q6.hip, gemv_q8.hip: launch for dtypes (d0, d1, d2) when the file
   holds that combination (*served = true), else *served = false. */
hipError_t gemv_combo_q4(const gemv_args& a, int d0, int d1, int d2, hipStream_t s, bool* served);
hipError_t gemv_combo_q6(const gemv_args& a, int d0, int d1, int d2, hipStream_t s, bool* served);
hipError_t gemv_combo_q8(const gemv_args& a, int d0, int d1, int d2, hipStream_t s, bool* served);

#define GEMV_CASE(A, B, C)                 \
    if (d0 == A && d1 == B && d2 == C) {  \
        *served = true;                    \
        return gemv_norm<A, B, C>(a, s);  \
    }

#endif
