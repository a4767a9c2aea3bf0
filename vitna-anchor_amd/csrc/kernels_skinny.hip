/**
 * kernels_skinny.hip - Several token rows (up to 32 a tile) times a quantized
 * matrix on the bf16 matrix cores, to fp32 accuracy: the multi-row dense
 * projections of a ragged decode pass (q/k/v, o, LM head).
 *
 * Reference counterpart: rows_dot_multi model_cuda.cu:1826 and the *_multi
 * kernels :1872-2006 (the reference reads each weight row once for up to 8
 * rows, on the CUDA cores); the CPU arithmetic checked against is
 * engine/src/model.c:887-979, one row at a time.
 *
 * Each weight is widened as the reference widens it (engine/src/quant.c:40-188,
 * every product rounded) and split into bf16 hi + lo (hi = bf16(w),
 * lo = bf16(w - hi)); the activations come split the same way
 * (split_rows_kernel). A product is hi*hi + hi*lo + lo*hi on
 * v_mfma_f32_32x32x16_bf16 (three MFMAs, fp32 accumulate): the dropped lo*lo
 * term and the splits leave about 2^-16 relative error a product, far inside
 * the 1e-3 the decode path is held to.
 *
 * Tiling: a workgroup is KS waves over one tile of 32 token rows x (32 NT)
 * weight rows; wave w takes every KS-th 32-weight slice of K, and the waves'
 * accumulators are added through LDS in wave order. A lane supplies weight row
 * lane % 32 (tile k) and the k-octet lane / 32 of both runs of each slice, as
 * the activations' lanes do for token lane % 32: the MFMA's k order is the
 * slice's, the same on both sides.
 */

#include "vitna_kernels.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define SK_TOK 32

/* ---- activations, split ------------------------------------------------- */

__global__ void split_rows_kernel(const float* __restrict__ x, int n, int K, int xstride, uint16_t* __restrict__ xh,
                                  uint16_t* __restrict__ xl) {
    const int r = blockIdx.y;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < K; c += gridDim.x * blockDim.x) {
        const float v = x[(size_t)r * xstride + c];
        const __bf16 h = (__bf16)v;
        const __bf16 l = (__bf16)(v - (float)h);
        xh[(size_t)r * K + c] = __builtin_bit_cast(uint16_t, h);
        xl[(size_t)r * K + c] = __builtin_bit_cast(uint16_t, l);
    }
}

hipError_t launch_split_rows(const float* x, int n, int K, int xstride, uint16_t* xh, uint16_t* xl, hipStream_t s) {
    if (n < 1 || K < 1) return hipErrorInvalidValue;
    split_rows_kernel<<<dim3((K + 255) / 256, n), 256, 0, s>>>(x, n, K, xstride, xh, xl);
    return hipGetLastError();
}

/* ---- weights: one lane's octets of a slice, widened ----------------------- */

/* Elements 8 kq .. 8 kq + 7 of the slice's low run (lo) and high run (hi),
   widened exactly. */
template <int DT>
__device__ __forceinline__ void widen_octets(const qraw& r, int t, int kq, float lo[8], float hi[8]) {
    if (DT == VITNA_DTYPE_Q8_0) {
        const float d = f16_bits_to_f32(r.c);
        const uint32_t a0 = kq ? r.a.z : r.a.x, a1 = kq ? r.a.w : r.a.y, b0 = kq ? r.b.z : r.b.x, b1 = kq ? r.b.w : r.b.y;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = (float)(int8_t)((a0 >> (8 * i)) & 0xff) * d;
            lo[4 + i] = (float)(int8_t)((a1 >> (8 * i)) & 0xff) * d;
            hi[i] = (float)(int8_t)((b0 >> (8 * i)) & 0xff) * d;
            hi[4 + i] = (float)(int8_t)((b1 >> (8 * i)) & 0xff) * d;
        }
    } else if (DT == VITNA_DTYPE_Q4_K) {
        const uint32_t h0 = r.b.x, s03 = r.b.y, s47 = r.b.z, s8b = r.b.w;
        const float d = f16_bits_to_f32(h0 & 0xffffu), dmin = f16_bits_to_f32(h0 >> 16);
        const int c = (t & 7) >> 1;
        uint32_t sc0, mn0, sc1, mn1;
        if (c < 2) {
            const int g0 = 2 * c, g1 = g0 + 1;
            sc0 = (s03 >> (8 * g0)) & 63; mn0 = (s47 >> (8 * g0)) & 63;
            sc1 = (s03 >> (8 * g1)) & 63; mn1 = (s47 >> (8 * g1)) & 63;
        } else {
            const int j0 = 2 * c - 4, j1 = j0 + 1;
            sc0 = ((s8b >> (8 * j0)) & 15) | (((s03 >> (8 * j0 + 6)) & 3) << 4);
            mn0 = ((s8b >> (8 * j0 + 4)) & 15) | (((s47 >> (8 * j0 + 6)) & 3) << 4);
            sc1 = ((s8b >> (8 * j1)) & 15) | (((s03 >> (8 * j1 + 6)) & 3) << 4);
            mn1 = ((s8b >> (8 * j1 + 4)) & 15) | (((s47 >> (8 * j1 + 6)) & 3) << 4);
        }
        const float d10 = d * (float)sc0, m10 = dmin * (float)mn0, d11 = d * (float)sc1, m11 = dmin * (float)mn1;
        const uint32_t w0 = kq ? r.a.z : r.a.x, w1 = kq ? r.a.w : r.a.y;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = d10 * (float)((w0 >> (8 * i)) & 15) - m10;
            lo[4 + i] = d10 * (float)((w1 >> (8 * i)) & 15) - m10;
            hi[i] = d11 * (float)((w0 >> (8 * i + 4)) & 15) - m11;
            hi[4 + i] = d11 * (float)((w1 >> (8 * i + 4)) & 15) - m11;
        }
    } else { /* Q6_K */
        const int sh = (int)(r.c >> 16);
        const float d = f16_bits_to_f32(r.d);
        const float ds0 = d * (float)(int8_t)(r.c & 0xff), ds1 = d * (float)(int8_t)((r.c >> 8) & 0xff);
        const uint32_t l0 = kq ? r.a.z : r.a.x, l1 = kq ? r.a.w : r.a.y, q0h = kq ? r.b.z : r.b.x, q1h = kq ? r.b.w : r.b.y;
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t ql = w ? l1 : l0, hb = (w ? q1h : q0h) >> sh;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int qa = (int)(((ql >> (8 * i)) & 15) | (((hb >> (8 * i)) & 3) << 4)) - 32;
                const int qb = (int)(((ql >> (8 * i + 4)) & 15) | (((hb >> (8 * i + 4)) & 3) << 4)) - 32;
                lo[4 * w + i] = ds0 * (float)qa;
                hi[4 * w + i] = ds1 * (float)qb;
            }
        }
    }
}

__device__ __forceinline__ void split8(const float w[8], bf16x8& h, bf16x8& l) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const __bf16 b = (__bf16)w[i];
        h[i] = b;
        l[i] = (__bf16)(w[i] - (float)b);
    }
}

/* ---- the kernel --------------------------------------------------------- */

/* Block (blockIdx.x = weight-row block of matrix i, blockIdx.y = token tile). */
template <int NT>
__global__ __launch_bounds__(NT == 1 ? 1024 : 256) void skinny_kernel(skinny_args a) {
    extern __shared__ float red[]; /* [KS][NT][16][64] when KS > 1 */
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, KS = blockDim.x >> 6;
    const int l32 = lane & 31, kq = lane >> 5;
    constexpr int RB = 32 * NT; /* weight rows a block */
    int bx = blockIdx.x, mi = 0;
    for (; mi < a.nm - 1; mi++) {
        const int nb = (a.w[mi].rows + RB - 1) / RB;
        if (bx < nb) break;
        bx -= nb;
    }
    const qmat& w = a.w[mi];
    const int dt = w.dtype;
    const int row0 = bx * RB;
    const int tok0 = blockIdx.y * SK_TOK, tok = tok0 + l32;
    const bool tok_ok = tok < a.n;
    const int S = w.cols / 32;
    const uint16_t* xh = a.xh + (size_t)(tok_ok ? tok : 0) * w.cols;
    const uint16_t* xl = a.xl + (size_t)(tok_ok ? tok : 0) * w.cols;

    f32x16 acc[NT];
#pragma unroll
    for (int k = 0; k < NT; k++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[k][r] = 0.0f;

    /* one slice's operands: the activations (token tok, the lane's octet of both runs) and the NT weight rows */
    struct slice_ops {
        u32x4 ah0, al0, ah1, al1;
        qraw q[NT];
    };
    auto load = [&](int t, slice_ops& o) {
        int clo, chi;
        slice_cols(dt, t, &clo, &chi);
        o.ah0 = o.al0 = o.ah1 = o.al1 = u32x4{0, 0, 0, 0};
        if (tok_ok) {
            o.ah0 = *reinterpret_cast<const u32x4*>(xh + clo + 8 * kq);
            o.al0 = *reinterpret_cast<const u32x4*>(xl + clo + 8 * kq);
            o.ah1 = *reinterpret_cast<const u32x4*>(xh + chi + 8 * kq);
            o.al1 = *reinterpret_cast<const u32x4*>(xl + chi + 8 * kq);
        }
#pragma unroll
        for (int k = 0; k < NT; k++) {
            const int rr = min(row0 + 32 * k + l32, w.rows - 1);
            if (dt == VITNA_DTYPE_Q4_K) slice_load<VITNA_DTYPE_Q4_K>(w, 0, rr, t, o.q[k]);
            else if (dt == VITNA_DTYPE_Q6_K) slice_load<VITNA_DTYPE_Q6_K>(w, 0, rr, t, o.q[k]);
            else slice_load<VITNA_DTYPE_Q8_0>(w, 0, rr, t, o.q[k]);
        }
    };
    auto compute = [&](int t, const slice_ops& o) {
        const bf16x8 Ah0 = __builtin_bit_cast(bf16x8, o.ah0), Al0 = __builtin_bit_cast(bf16x8, o.al0);
        const bf16x8 Ah1 = __builtin_bit_cast(bf16x8, o.ah1), Al1 = __builtin_bit_cast(bf16x8, o.al1);
#pragma unroll
        for (int k = 0; k < NT; k++) {
            float wlo[8], whi[8];
            if (dt == VITNA_DTYPE_Q4_K) widen_octets<VITNA_DTYPE_Q4_K>(o.q[k], t, kq, wlo, whi);
            else if (dt == VITNA_DTYPE_Q6_K) widen_octets<VITNA_DTYPE_Q6_K>(o.q[k], t, kq, wlo, whi);
            else widen_octets<VITNA_DTYPE_Q8_0>(o.q[k], t, kq, wlo, whi);
            bf16x8 Bh0, Bl0, Bh1, Bl1;
            split8(wlo, Bh0, Bl0);
            split8(whi, Bh1, Bl1);
            acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Ah0, Bh0, acc[k], 0, 0, 0);
            acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Ah0, Bl0, acc[k], 0, 0, 0);
            acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Al0, Bh0, acc[k], 0, 0, 0);
            acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Ah1, Bh1, acc[k], 0, 0, 0);
            acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Ah1, Bl1, acc[k], 0, 0, 0);
            acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Al1, Bh1, acc[k], 0, 0, 0);
        }
    };
    /* slices wv, wv + KS, ...: the next one's loads in flight while this one computes */
    slice_ops o0, o1;
    if (wv < S) load(wv, o0);
    for (int t = wv; t < S; t += 2 * KS) {
        if (t + KS < S) load(t + KS, o1);
        compute(t, o0);
        if (t + KS >= S) break;
        if (t + 2 * KS < S) load(t + 2 * KS, o0);
        compute(t + KS, o1);
    }
    /* accumulator r of a lane: token 8 (r / 4) + 4 (lane / 32) + r % 4 of the tile, weight row lane % 32 */
    float* y = a.y[mi];
    auto put = [&](int k, int r, float v) {
        const int n = row0 + 32 * k + l32;
        const int tk = tok0 + 8 * (r >> 2) + 4 * kq + (r & 3);
        if (n < w.rows && tk < a.n) {
            float* o = y + (size_t)tk * w.rows + n;
            *o = a.add ? *o + v : v;
        }
    };
    if (KS == 1) {
#pragma unroll
        for (int k = 0; k < NT; k++)
#pragma unroll
            for (int r = 0; r < 16; r++) put(k, r, acc[k][r]);
        return;
    }
    /* the waves' sums: every wave's accumulators through LDS, then wave v adds up the registers r = v, v + KS,
       ... of every tile over the waves, in wave order */
#pragma unroll
    for (int k = 0; k < NT; k++)
#pragma unroll
        for (int r = 0; r < 16; r++) red[((wv * NT + k) * 16 + r) * 64 + lane] = acc[k][r];
    __syncthreads();
    for (int kr = wv; kr < NT * 16; kr += KS) {
        const int k = kr >> 4, r = kr & 15;
        float v = 0.0f;
        for (int u = 0; u < KS; u++) v += red[((u * NT + k) * 16 + r) * 64 + lane];
        put(k, r, v);
    }
}

hipError_t launch_skinny(const skinny_args& a, hipStream_t s) {
    if (a.nm < 1 || a.nm > 3 || a.n < 1 || !a.xh || !a.xl) return hipErrorInvalidValue;
    for (int i = 0; i < a.nm; i++) {
        const int d = a.w[i].dtype;
        if (a.w[i].cols != a.w[0].cols || a.w[i].cols % 32) return hipErrorInvalidValue;
        if (d != VITNA_DTYPE_Q8_0 && d != VITNA_DTYPE_Q4_K && d != VITNA_DTYPE_Q6_K) return hipErrorInvalidValue;
    }
    int cus = 0, dev = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    const int want = 8 * cus; /* two waves a SIMD */
    const int mt = (a.n + SK_TOK - 1) / SK_TOK;
    const int S = a.w[0].cols / 32;
    int rows = 0;
    for (int i = 0; i < a.nm; i++) rows += a.w[i].rows;
    /* wide matrices (the LM head) take four 32-row tiles a wave, so each token tile's activations are read
       a quarter as often; the rest one */
    const bool wide = rows >= 32768;
#ifndef SK_KS_MAX
#define SK_KS_MAX 16
#endif
    const int RB = wide ? 128 : 32, ks_max = wide ? 2 : SK_KS_MAX;
    int blocks = 0;
    for (int i = 0; i < a.nm; i++) blocks += (a.w[i].rows + RB - 1) / RB;
    int ks = 1;
    while (ks < ks_max && ks * 2 <= S && (size_t)blocks * mt * ks < (size_t)want) ks *= 2;
    const size_t lds = ks > 1 ? (size_t)ks * (wide ? 4 : 1) * 16 * 64 * sizeof(float) : 0;
    const dim3 grid(blocks, mt);
    if (wide) skinny_kernel<4><<<grid, 64 * ks, lds, s>>>(a);
    else skinny_kernel<1><<<grid, 64 * ks, lds, s>>>(a);
    return hipGetLastError();
}
