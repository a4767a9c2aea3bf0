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
 * Two kernels:
 *   skinny_exact_kernel / skinny_wide_kernel (widths a multiple of 256): the
 *     quants enter the MFMA as exact bf16 integers, each scale group keeps its
 *     own MFMA sum and its scale is applied in fp32 (the section "exact-integer
 *     quants" below); the operands come from images in MFMA lane order
 *     (skinny_image.h) and the weights from a tiled copy, so every load of a
 *     wave is 1 KB contiguous.
 *   skinny_kernel (other widths): each weight is widened as the reference
 *     widens it (engine/src/quant.c:40-188) and split into bf16 hi + lo, the
 *     activations likewise (split_rows_kernel), and a product is
 *     hi*hi + hi*lo + lo*hi on v_mfma_f32_32x32x16_bf16: about 2^-16 relative
 *     a product. A workgroup is KS waves over one tile of 32 token rows x
 *     (32 NT) weight rows; wave w takes every KS-th 32-weight slice of K, and
 *     the waves' accumulators are added through LDS in wave order. A lane
 *     supplies weight row lane % 32 and the k-octet lane / 32 of both runs of
 *     each slice, as the activations' lanes do for token lane % 32.
 * Both stay within 1e-3 of the CPU checker; each projection alone is held to
 * 2e-5 of max |ref| against the widened matrix in float64.
 *
 * The same exact arithmetic serves the grouped experts of crowded passes (64
 * rows and more) on tiles of 32 pairs of one expert (launch_gsx, at the end).
 */

#include "vitna_kernels.h"
#include "skinny_image.h"

#include <algorithm>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define SK_TOK 32
#define SK_NT 2 /* token tiles a block of the exact kernel takes when a pass has many */
#ifndef SK_NR
#define SK_NR 2
#endif

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

__device__ __forceinline__ uint16_t bf16_bits(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

/* The operand images of a pass (skinny_image.h): block (b, tt) takes superblock b of token tile tt, thread t
   its 8-column groups t + 256 j; rows past n repeat row n - 1. */
__global__ void split_image_kernel(const float* __restrict__ x, int n, int K, int xstride, u32x4* __restrict__ imga,
                                   u32x4* __restrict__ imgb, uint16_t* __restrict__ s32, uint16_t* __restrict__ s16) {
    const int b = blockIdx.x, tt = blockIdx.y;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int item = threadIdx.x + 256 * j, l = item >> 5, c8 = 32 * b + (item & 31);
        const int tok = min(32 * tt + l, n - 1), row = 32 * tt + l;
        const float4* src = reinterpret_cast<const float4*>(x + (size_t)tok * xstride + 8 * c8);
        const float4 v0 = src[0], v1 = src[1];
        const float e[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        u32x4 vh, vl;
        float sum;
        img_split8(e, vh, vl, sum);
        img_put(imga, imgb, row, K, c8, vh, vl);
        /* the 16- and 32-column sums (the pair's, then the quad's: lanes of consecutive c8, one token) */
        const float t16 = sum + __shfl_xor(sum, 1, WAVE);
        const float t32 = t16 + __shfl_xor(t16, 2, WAVE);
        if (!(c8 & 1)) img_sum16(s16, row, K, c8 >> 1, t16);
        if (!(c8 & 3)) img_sum32(s32, row, K, c8 >> 2, t32);
    }
}

hipError_t launch_split_rows(const float* x, int n, int K, int xstride, uint16_t* xh, uint16_t* xl, uint32_t* const* img,
                             hipStream_t s) {
    if (n < 1 || K < 1) return hipErrorInvalidValue;
    if (img) {
        if (K % 256 || xstride % 4 || (uintptr_t)x % 16) return hipErrorInvalidValue;
        split_image_kernel<<<dim3(K / 256, (n + 31) / 32), 256, 0, s>>>(x, n, K, xstride, (u32x4*)img[0], (u32x4*)img[1],
                                                                        (uint16_t*)img[2], (uint16_t*)img[3]);
    } else {
        split_rows_kernel<<<dim3((K + 255) / 256, n), 256, 0, s>>>(x, n, K, xstride, xh, xl);
    }
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

/* ---- exact-integer quants ------------------------------------------------ */
/*
 * Widths a multiple of 256 take this path. A wave owns one tile of 32 weight rows x 32 token rows over one
 * 256-column superblock (one Q4_K or Q6_K block, eight Q8_0 blocks), four units of 64 columns each: the
 * work is a few microseconds of loads a wave, so it is spread as wide as it goes and every load of the
 * wave's weights is issued at once. Within a unit every scale group (Q4_K 32 columns, Q6_K 16, Q8_0 32) keeps its own MFMA sum
 * P over its columns, and the group's scale is applied to P in fp32:
 *   Q8_0  bf16(q) exactly (signed):            acc += d P
 *   Q4_K  bf16(128 + q), q in 0..15:           acc += d sc P  -  (dmin m + 128 d sc) S
 *   Q6_K  bf16(128 + q6), q6 in 0..63:         acc += d sc P  -  160 d sc S
 * where S is the group's sum of the activations. 128 + q is the byte q under the exponent byte of 2^7 (two
 * v_perm_b32 for four weights). The S terms of eight groups go through the matrix cores too, as one
 * 32x32x8 product of the groups' sums (bf16 hi + lo, split on the host side of the pass) by their
 * coefficients, both as three bf16 pieces. S is the sum of the split activations hi + lo, so the offset
 * 128 S cancels exactly what the 128 in the weights added.
 *
 * A unit's k order: lane half kq (lane / 32) of each 16-column MFMA supplies 8 columns, and both operands
 * take them in the same order. Q4_K and Q8_0: the MFMAs of unit u cover columns 64 u + 16 kq + {0, 8} (the
 * first group) and + 32 (the second); Q4_K's byte 32 u + j holds columns 64 u + j (low nibble) and
 * 64 u + 32 + j (high). Q6_K unit u = (h, r0) = (u / 2, u % 2) covers the groups at columns
 * 128 h + 32 r + 16 s, r in {r0, r0 + 2}, s in {0, 1}, of which lane half kq takes columns + 8 kq .. + 8 kq + 7:
 * ql byte 64 h + 32 r0 + 16 s + j holds column 128 h + 32 r0 + 16 s + j (low nibble) and 128 h + 32 (r0 + 2)
 * + 16 s + j (high), qh byte 32 h + 16 s + j its high bits (bits 2 r).
 */

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sx_u2 __attribute__((ext_vector_type(2)));

/* four bytes (each below 128) as bf16 128 + byte */
__device__ __forceinline__ sx_u2 sx_mag4(uint32_t v) {
    return sx_u2{__builtin_amdgcn_perm(0x43434343u, v, 0x04010400u), __builtin_amdgcn_perm(0x43434343u, v, 0x04030402u)};
}
__device__ __forceinline__ bf16x8 sx_join(sx_u2 a, sx_u2 b) { return __builtin_bit_cast(bf16x8, u32x4{a.x, a.y, b.x, b.y}); }
/* eight signed bytes as bf16, exactly */
__device__ __forceinline__ bf16x8 sx_i8(uint32_t a, uint32_t b) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[i] = (__bf16)(float)(int8_t)(a >> (8 * i));
        r[4 + i] = (__bf16)(float)(int8_t)(b >> (8 * i));
    }
    return r;
}

/* One superblock of one 32-row tile: the lane's row's bytes for all four units. */
template <int DT> struct sx_w;
template <> struct sx_w<VITNA_DTYPE_Q4_K> { u32x4 q[4], h; };
template <> struct sx_w<VITNA_DTYPE_Q6_K> { sx_u2 ql[4][2], qh[2][2]; u32x4 sc; uint32_t d; };
template <> struct sx_w<VITNA_DTYPE_Q8_0> { u32x4 q[4][2], d; };

/* a unit's activations for the lane's token: four 8-column operands, hi and lo, and (when the unit applies
   S terms) the four group sums of the lane half */
struct sx_a {
    u32x4 h[4], l[4];
    sx_u2 sp[3];
};

/*
 * The tiled copy: per tile (32 rows; rows past the matrix repeat its last) and superblock, lane l = l32 + 32 kq
 * reads 16-byte pieces at lane-order offsets, so every load is 1 KB contiguous (512 bytes for the per-row
 * fields, which both lane halves read):
 *   Q4_K  [u][lane] q bytes 32 u + 16 kq + 0..15 (u < 4); at 4096 [l32] the 16-byte header
 *   Q6_K  [u][lane] ql bytes 64 (u / 2) + 32 (u % 2) + 16 s + 8 kq + 0..7 for s = 0, 1; at 4096 [h][lane] qh
 *         bytes 32 h + 16 s + 8 kq + 0..7 for s = 0, 1; at 6144 [l32] the 16 scales; at 6656 [l32] d
 *   Q8_0  [2 u + j][lane] q bytes 16 kq + 0..15 of block 8 b + 2 u + j; at 8192 [l32] the 8 blocks' d
 */
__device__ __forceinline__ uint32_t tile_src(const qmat& m, int tile, int b, int o) {
    /* the byte of the planes that byte o of tile / superblock b copies */
    const int S = m.cols / 256;
    (void)S;
    if (m.dtype == VITNA_DTYPE_Q4_K) {
        if (o < 4096) {
            const int u = o >> 10, lane = (o >> 4) & 63, j = o & 15;
            const size_t row = min(32 * tile + (lane & 31), m.rows - 1);
            return m.p[0][(row * m.nb + b) * 128 + 32 * u + 16 * (lane >> 5) + j];
        }
        const int l32 = (o - 4096) >> 4, j = o & 15;
        const size_t row = min(32 * tile + l32, m.rows - 1);
        return m.p[1][(row * m.nb + b) * 16 + j];
    } else if (m.dtype == VITNA_DTYPE_Q6_K) {
        if (o < 4096) {
            const int u = o >> 10, lane = (o >> 4) & 63, j = o & 15, sh = j >> 3, jj = j & 7;
            const size_t row = min(32 * tile + (lane & 31), m.rows - 1);
            return m.p[0][(row * m.nb + b) * 128 + 64 * (u >> 1) + 32 * (u & 1) + 16 * sh + 8 * (lane >> 5) + jj];
        }
        if (o < 6144) {
            const int q = o - 4096, h = q >> 10, lane = (q >> 4) & 63, j = q & 15, sh = j >> 3, jj = j & 7;
            const size_t row = min(32 * tile + (lane & 31), m.rows - 1);
            return m.p[1][(row * m.nb + b) * 64 + 32 * h + 16 * sh + 8 * (lane >> 5) + jj];
        }
        if (o < 6656) {
            const int l32 = (o - 6144) >> 4, j = o & 15;
            const size_t row = min(32 * tile + l32, m.rows - 1);
            return m.p[2][(row * m.nb + b) * 16 + j];
        }
        const int l32 = (o - 6656) >> 1, j = o & 1;
        const size_t row = min(32 * tile + l32, m.rows - 1);
        return m.p[3][(row * m.nb + b) * 2 + j];
    } else {
        if (o < 8192) {
            const int v = o >> 10, lane = (o >> 4) & 63, j = o & 15;
            const size_t row = min(32 * tile + (lane & 31), m.rows - 1);
            return m.p[0][(row * m.nb + 8 * b + v) * 32 + 16 * (lane >> 5) + j];
        }
        const int l32 = (o - 8192) >> 4, j = o & 15;
        const size_t row = min(32 * tile + l32, m.rows - 1);
        return m.p[1][(row * m.nb + 8 * b) * 2 + j];
    }
}

/* One block a tile / superblock, a thread a byte (the copy is made once, at upload). */
__global__ void tile_kernel(qmat m, uint8_t* __restrict__ dst) {
    const int S = m.cols / 256, tile = blockIdx.x / S, b = blockIdx.x % S;
    const int tb = (int)tile_bytes(m.dtype);
    uint8_t* out = dst + (size_t)blockIdx.x * tb;
    for (int o = threadIdx.x; o < tb; o += blockDim.x) out[o] = (uint8_t)tile_src(m, tile, b, o);
}

hipError_t launch_tile(const qmat& m, uint8_t* dst, hipStream_t s) {
    if (!tile_bytes(m.dtype) || m.cols % 256 || m.rows < 1) return hipErrorInvalidValue;
    tile_kernel<<<((m.rows + 31) / 32) * (m.cols / 256), 256, 0, s>>>(m, dst);
    return hipGetLastError();
}

/* The lane's bytes of tile / superblock b from the tiled copy: 1 KB (512-byte) loads in lane order. */
template <int DT>
__device__ __forceinline__ void sx_load_w(const qmat& w, int tile, int b, int lane, sx_w<DT>& o) {
    const uint8_t* T = w.tiled + ((size_t)tile * (w.cols / 256) + b) * (DT == VITNA_DTYPE_Q4_K ? 4608 : DT == VITNA_DTYPE_Q6_K ? 6720 : 8704);
    const int l32 = lane & 31;
    if constexpr (DT == VITNA_DTYPE_Q4_K) {
#pragma unroll
        for (int u = 0; u < 4; u++) o.q[u] = *reinterpret_cast<const u32x4*>(T + u * 1024 + lane * 16);
        o.h = *reinterpret_cast<const u32x4*>(T + 4096 + l32 * 16);
    } else if constexpr (DT == VITNA_DTYPE_Q6_K) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(T + u * 1024 + lane * 16);
            o.ql[u][0] = sx_u2{v.x, v.y};
            o.ql[u][1] = sx_u2{v.z, v.w};
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(T + 4096 + h * 1024 + lane * 16);
            o.qh[h][0] = sx_u2{v.x, v.y};
            o.qh[h][1] = sx_u2{v.z, v.w};
        }
        o.sc = *reinterpret_cast<const u32x4*>(T + 6144 + l32 * 16);
        o.d = *reinterpret_cast<const uint16_t*>(T + 6656 + l32 * 2);
    } else {
#pragma unroll
        for (int v = 0; v < 8; v++) o.q[v >> 1][v & 1] = *reinterpret_cast<const u32x4*>(T + v * 1024 + lane * 16);
        o.d = *reinterpret_cast<const u32x4*>(T + 8192 + l32 * 16);
    }
}

template <int DT> struct sx_unit_sums { static constexpr bool at(int U) { return DT == VITNA_DTYPE_Q4_K ? U == 3 : DT == VITNA_DTYPE_Q6_K ? (U & 1) : false; } };

/* Unit U's operands of token tile tt, superblock b (and the S-term sums when the unit applies them), from the
   images: every load is 1 KB (512 bytes for the sums) in lane order. */
template <int DT, int U>
__device__ __forceinline__ void sx_load_a(const skinny_args& a, int tt, int K, int b, int lane, sx_a& o) {
    const u32x4* img = reinterpret_cast<const u32x4*>(DT == VITNA_DTYPE_Q6_K ? a.img[1] : a.img[0]) +
                       ((size_t)tt * (K / 256) + b) * 2048 + (size_t)U * 512 + lane;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o.h[i] = img[i * 128];
        o.l[i] = img[i * 128 + 64];
    }
    if constexpr (sx_unit_sums<DT>::at(U)) {
        const sx_u2* sp = DT == VITNA_DTYPE_Q4_K
                              ? reinterpret_cast<const sx_u2*>(a.s32) + ((size_t)tt * (K / 256) + b) * 192 + lane
                              : reinterpret_cast<const sx_u2*>(a.s16) + ((size_t)tt * (K / 128) + 2 * b + (U >> 1)) * 192 + lane;
#pragma unroll
        for (int i = 0; i < 3; i++) o.sp[i] = sp[64 * i];
    }
}

__device__ __forceinline__ void sx_scale(f32x16& acc, float d, const f32x16& P) {
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = fmaf(d, P[r], acc[r]);
}
#define SX_MMA(A, B, C) __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, A), B, C, 0, 0, 0)

/* Q4_K scale and min of group g from the 12 scale bytes (header dwords 1..3) */
template <int G>
__device__ __forceinline__ void sx_q4k_sm(const u32x4& h, uint32_t& sc, uint32_t& mn) {
    if constexpr (G < 4) {
        sc = (h.y >> (8 * G)) & 63;
        mn = (h.z >> (8 * G)) & 63;
    } else {
        constexpr int j = G - 4;
        sc = ((h.w >> (8 * j)) & 15) | (((h.y >> (8 * j + 6)) & 3) << 4);
        mn = ((h.w >> (8 * j + 4)) & 15) | (((h.z >> (8 * j + 6)) & 3) << 4);
    }
}

/* the S terms of eight groups: the lane half's four sums times its four coefficients c, each as three bf16
   pieces, the six products down to 2^-24 of the largest (the offset part of c S cancels against the MFMA sums
   of 128 + q, so it is carried to fp32 accuracy) */
__device__ __forceinline__ void sx_sterm(const sx_a& x, const float c[4], f32x16& acc) {
    s16x4 cp[3];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const __bf16 p0 = (__bf16)c[i];
        const float r0 = c[i] - (float)p0;
        const __bf16 p1 = (__bf16)r0;
        cp[0][i] = __builtin_bit_cast(short, p0);
        cp[1][i] = __builtin_bit_cast(short, p1);
        cp[2][i] = __builtin_bit_cast(short, (__bf16)(r0 - (float)p1));
    }
    const s16x4 s0 = __builtin_bit_cast(s16x4, x.sp[0]), s1 = __builtin_bit_cast(s16x4, x.sp[1]), s2 = __builtin_bit_cast(s16x4, x.sp[2]);
    acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(s2, cp[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(s1, cp[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(s0, cp[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(s1, cp[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(s0, cp[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(s0, cp[0], acc, 0, 0, 0);
}

/* Unit U: its groups' sums and scales into acc; cs carries the superblock's S coefficients (Q4_K) from the
   units that make them to the unit that applies them. */
template <int DT, int U>
__device__ __forceinline__ void sx_compute(const sx_w<DT>& w, const sx_a& x, int kq, f32x16& acc, float cs[8]) {
    const f32x16 Z = {};
    if constexpr (DT == VITNA_DTYPE_Q4_K) {
        constexpr uint32_t M = 0x0f0f0f0fu;
        const u32x4 q = w.q[U];
        const bf16x8 a0 = sx_join(sx_mag4(q.x & M), sx_mag4(q.y & M)), a1 = sx_join(sx_mag4(q.z & M), sx_mag4(q.w & M));
        const bf16x8 b0 = sx_join(sx_mag4((q.x >> 4) & M), sx_mag4((q.y >> 4) & M));
        const bf16x8 b1 = sx_join(sx_mag4((q.z >> 4) & M), sx_mag4((q.w >> 4) & M));
        f32x16 P0 = SX_MMA(x.h[0], a0, Z), P1 = SX_MMA(x.h[2], b0, Z);
        P0 = SX_MMA(x.h[1], a1, P0);
        P1 = SX_MMA(x.h[3], b1, P1);
        P0 = SX_MMA(x.l[0], a0, P0);
        P1 = SX_MMA(x.l[2], b0, P1);
        P0 = SX_MMA(x.l[1], a1, P0);
        P1 = SX_MMA(x.l[3], b1, P1);
        const float d = f16_bits_to_f32(w.h.x & 0xffffu), dmin = f16_bits_to_f32(w.h.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        sx_q4k_sm<2 * U>(w.h, sc0, mn0);
        sx_q4k_sm<2 * U + 1>(w.h, sc1, mn1);
        const float d0 = d * (float)sc0, d1 = d * (float)sc1;
        sx_scale(acc, d0, P0);
        sx_scale(acc, d1, P1);
        cs[2 * U] = -fmaf(128.0f, d0, dmin * (float)mn0);
        cs[2 * U + 1] = -fmaf(128.0f, d1, dmin * (float)mn1);
        if constexpr (U == 3) {
            float c[4];
#pragma unroll
            for (int j = 0; j < 4; j++) c[j] = kq ? cs[4 + j] : cs[j];
            sx_sterm(x, c, acc);
        }
    } else if constexpr (DT == VITNA_DTYPE_Q6_K) {
        constexpr int h = U >> 1, r0 = U & 1;
        bf16x8 wq[4]; /* groups (r0, 0), (r0, 1), (r0 + 2, 0), (r0 + 2, 1) */
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = i & 1, hi = i >> 1, r = r0 + 2 * hi;
            uint32_t v[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t ql = hi ? (w.ql[U][s][j] >> 4) : w.ql[U][s][j];
                const uint32_t qh = w.qh[h][s][j];
                const uint32_t top = r == 0 ? qh << 4 : r == 1 ? qh << 2 : r == 2 ? qh : qh >> 2;
                v[j] = (ql & 0x0f0f0f0fu) | (top & 0x30303030u);
            }
            wq[i] = sx_join(sx_mag4(v[0]), sx_mag4(v[1]));
        }
        f32x16 P[4];
#pragma unroll
        for (int i = 0; i < 4; i++) P[i] = SX_MMA(x.h[i], wq[i], Z);
#pragma unroll
        for (int i = 0; i < 4; i++) P[i] = SX_MMA(x.l[i], wq[i], P[i]);
        const float d = f16_bits_to_f32(w.d);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = 8 * h + 2 * (r0 + 2 * (i >> 1)) + (i & 1); /* the group's scale index */
            sx_scale(acc, d * (float)(int8_t)(w.sc[g >> 2] >> (8 * (g & 3))), P[i]);
        }
        if constexpr (r0 == 1) {
            /* the S terms of groups 8 h .. 8 h + 7: lane half kq supplies 8 h + 4 kq .. + 3 */
            const uint32_t scw = kq ? w.sc[2 * h + 1] : w.sc[2 * h];
            const float m = -160.0f * d;
            float c[4];
#pragma unroll
            for (int j = 0; j < 4; j++) c[j] = m * (float)(int8_t)(scw >> (8 * j));
            sx_sterm(x, c, acc);
        }
    } else {
        const bf16x8 a0 = sx_i8(w.q[U][0].x, w.q[U][0].y), a1 = sx_i8(w.q[U][0].z, w.q[U][0].w);
        const bf16x8 b0 = sx_i8(w.q[U][1].x, w.q[U][1].y), b1 = sx_i8(w.q[U][1].z, w.q[U][1].w);
        f32x16 P0 = SX_MMA(x.h[0], a0, Z), P1 = SX_MMA(x.h[2], b0, Z);
        P0 = SX_MMA(x.h[1], a1, P0);
        P1 = SX_MMA(x.h[3], b1, P1);
        P0 = SX_MMA(x.l[0], a0, P0);
        P1 = SX_MMA(x.l[2], b0, P1);
        P0 = SX_MMA(x.l[1], a1, P0);
        P1 = SX_MMA(x.l[3], b1, P1);
        const uint32_t dw = w.d[U];
        sx_scale(acc, f16_bits_to_f32(dw & 0xffffu), P0);
        sx_scale(acc, f16_bits_to_f32(dw >> 16), P1);
    }
}

/* Superblock b of the lane's weight rows of NR consecutive 32-row tiles (those of them below nr) against NT
   token tiles tt0, tt0 + 1, ... (those below mt): every weight load issued first, then each token tile's
   activations two units ahead, each unit's activations used for all NR weight tiles; the weights stay in
   registers across the token tiles, and each (weight tile, token tile)'s sums run as they would alone. */
template <int DT, int NT, int NR>
__device__ __forceinline__ void sx_superblock(const skinny_args& a, const qmat& w, int tile, int nr, int tt0, int mt, int b,
                                              int lane, f32x16 (&acc)[NR][NT]) {
    const int kq = lane >> 5;
    const int K = w.cols;
    sx_w<DT> W[NR];
#pragma unroll
    for (int r = 0; r < NR; r++)
        if (r < nr) sx_load_w<DT>(w, tile + r, b, lane, W[r]);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tt = tt0 + t;
        if (tt >= mt) break;
        float cs[NR][8];
        sx_a x0, x1;
        sx_load_a<DT, 0>(a, tt, K, b, lane, x0);
        sx_load_a<DT, 1>(a, tt, K, b, lane, x1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < NR; r++)
            if (r < nr) sx_compute<DT, 0>(W[r], x0, kq, acc[r][t], cs[r]);
        sx_load_a<DT, 2>(a, tt, K, b, lane, x0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < NR; r++)
            if (r < nr) sx_compute<DT, 1>(W[r], x1, kq, acc[r][t], cs[r]);
        sx_load_a<DT, 3>(a, tt, K, b, lane, x1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < NR; r++)
            if (r < nr) sx_compute<DT, 2>(W[r], x0, kq, acc[r][t], cs[r]);
#pragma unroll
        for (int r = 0; r < NR; r++)
            if (r < nr) sx_compute<DT, 3>(W[r], x1, kq, acc[r][t], cs[r]);
    }
}

/*
 * Block (blockIdx.x = (32-row tile of matrix i, split), blockIdx.y = token tile): KS waves, wave v on superblock
 * 8 split + v. The waves' sums are added through LDS in wave order. A matrix wider than 8 superblocks takes
 * several splits: each block stores its tile's sum in part[], and the block that finishes a tile last (its
 * counter in cnt[]) adds the splits' sums in split order, writes the result and clears the counter, so the
 * result does not depend on which block finishes last.
 */
template <int NT, int NR>
__global__ __launch_bounds__(512) void skinny_exact_kernel(skinny_args a) {
    extern __shared__ float red[]; /* [KS][16][64] */
    __shared__ int last;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, KS = blockDim.x >> 6;
    const int l32 = lane & 31, kq = lane >> 5;
    int bx = blockIdx.x, mi = 0, tile0 = 0;
    for (; mi < a.nm - 1; mi++) {
        const int nb = ((a.w[mi].rows + 31) / 32 + NR - 1) / NR * a.splits[mi];
        if (bx < nb) break;
        bx -= nb;
        tile0 += (a.w[mi].rows + 31) / 32;
    }
    const qmat& w = a.w[mi];
    const int splits = a.splits[mi], sp = bx % splits, tile = bx / splits * NR;
    const int nr = min(NR, (w.rows + 31) / 32 - tile); /* this block's weight tiles */
    const int mt = (a.n + SK_TOK - 1) / SK_TOK, tt0 = blockIdx.y * NT;
    const int b = 8 * sp + wv;
    f32x16 acc[NR][NT];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[r][t] = f32x16{};
    if (b < w.cols / 256) {
        if (w.dtype == VITNA_DTYPE_Q4_K) sx_superblock<VITNA_DTYPE_Q4_K, NT, NR>(a, w, tile, nr, tt0, mt, b, lane, acc);
        else if (w.dtype == VITNA_DTYPE_Q6_K) sx_superblock<VITNA_DTYPE_Q6_K, NT, NR>(a, w, tile, nr, tt0, mt, b, lane, acc);
        /* (two Q8_0 weight tiles a block do not fit the registers: the launch keeps Q8_0 to one) */
        else if constexpr (NR == 1) sx_superblock<VITNA_DTYPE_Q8_0, NT, NR>(a, w, tile, nr, tt0, mt, b, lane, acc);
    }

    float* y = a.y[mi];
#pragma unroll
    for (int wr = 0; wr < NR; wr++) {
        if (wr >= nr) break;
        const int row0 = 32 * (tile + wr);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int tt = tt0 + t;
            if (tt >= mt) break;
            /* accumulator r of a lane: token 8 (r / 4) + 4 (lane / 32) + r % 4 of the tile, weight row lane % 32 */
            const int tok0 = tt * SK_TOK;
            auto put = [&](int r, float v) {
                const int n = row0 + l32;
                const int tk = tok0 + 8 * (r >> 2) + 4 * kq + (r & 3);
                if (n < w.rows && tk < a.n) {
                    float* o = y + (size_t)tk * w.rows + n;
                    *o = a.add ? *o + v : v;
                }
            };
            if (KS > 1) {
                if (t || wr) __syncthreads(); /* the previous tile's sums are read */
#pragma unroll
                for (int r = 0; r < 16; r++) red[(wv * 16 + r) * 64 + lane] = acc[wr][t][r];
                __syncthreads();
            }
            if (splits == 1) {
                if (KS == 1) {
#pragma unroll
                    for (int r = 0; r < 16; r++) put(r, acc[wr][t][r]);
                    continue;
                }
                for (int r = wv; r < 16; r += KS) {
                    float v = 0.0f;
                    for (int u = 0; u < KS; u++) v += red[(u * 16 + r) * 64 + lane];
                    put(r, v);
                }
                continue;
            }
            /* several splits: this block's sum of the tile into part[], then the last block of the tile adds them */
            const size_t slot = (size_t)tt * a.tiles + tile0 + tile + wr; /* the tile's counter */
            float* part = a.part + slot * a.split_max * 1024;
            /* The sums are stored as agent-scope atomics (written through this XCD's L2 to where every XCD reads);
               the counter's increment releases them and the last block's acquires them, at agent scope, so the last
               block reads every split's sums (the workgroup barrier carries thread 0's acquire to the others). */
            for (int r = wv; r < 16; r += KS) {
                float v = 0.0f;
                for (int u = 0; u < KS; u++) v += red[(u * 16 + r) * 64 + lane];
                __hip_atomic_store(part + (size_t)sp * 1024 + r * 64 + lane, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); /* every wave's stores complete before the barrier */
            __syncthreads();
            if (threadIdx.x == 0) last = __hip_atomic_fetch_add(a.cnt + slot, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
            __syncthreads();
            if (last) {
                for (int r = wv; r < 16; r += KS) {
                    float v = 0.0f;
                    for (int u = 0; u < splits; u++)
                        v += __hip_atomic_load(part + (size_t)u * 1024 + r * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    put(r, v);
                }
                if (threadIdx.x == 0) __hip_atomic_store(a.cnt + slot, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

/* ---- wide matrices (the LM head): activations staged in LDS ---------------- */

#define SXW_PIECES 2048

typedef __attribute__((address_space(3))) void* sx_lds_void;
typedef __attribute__((address_space(1))) void* sx_glb_void;

/* Superblock b's image of token tile tt, copied into LDS by global-to-LDS loads (lane l of a wave lands at the
   wave's base + 16 l: a straight copy). Counted by vmcnt. */
template <int DT, int NW>
__device__ __forceinline__ void sxw_fetch(const skinny_args& a, int K, int tt, int b, u32x4* img) {
    const int wv = threadIdx.x >> 6;
    const u32x4* src = reinterpret_cast<const u32x4*>(DT == VITNA_DTYPE_Q6_K ? a.img[1] : a.img[0]) + ((size_t)tt * (K / 256) + b) * 2048;
#pragma unroll
    for (int j = 0; j < SXW_PIECES / (64 * NW); j++) {
        const int p = threadIdx.x + 64 * NW * j;
        __builtin_amdgcn_global_load_lds((sx_glb_void)(src + p), (sx_lds_void)(img + wv * 64 + 64 * NW * j), 16, 0, 0);
    }
}

template <int DT, int U>
__device__ __forceinline__ void sxw_read(const u32x4* img, const skinny_args& a, int tt, int K, int b, int lane, sx_a& o) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o.h[i] = img[U * 512 + i * 128 + lane];
        o.l[i] = img[U * 512 + i * 128 + 64 + lane];
    }
    if constexpr (sx_unit_sums<DT>::at(U)) {
        const sx_u2* sp = DT == VITNA_DTYPE_Q4_K
                              ? reinterpret_cast<const sx_u2*>(a.s32) + ((size_t)tt * (K / 256) + b) * 192 + lane
                              : reinterpret_cast<const sx_u2*>(a.s16) + ((size_t)tt * (K / 128) + 2 * b + (U >> 1)) * 192 + lane;
#pragma unroll
        for (int i = 0; i < 3; i++) o.sp[i] = sp[64 * i];
    }
}

/* NW waves, wave v on tile NW blockIdx.x + v of the matrix, every superblock in turn: the block stages
   superblock b + 1's activations and each wave loads its weights for b + 1 while b computes. */
template <int DT, int NW>
__device__ __forceinline__ void sxw_body(const skinny_args& a, const qmat& w, int tile, int tt, u32x4* img, f32x16& acc) {
    const int lane = threadIdx.x & 63, kq = lane >> 5;
    const int K = w.cols, S = K / 256;

    sx_w<DT> W0, W1;
    float cs[8];
    sxw_fetch<DT, NW>(a, K, tt, 0, img);
    sx_load_w<DT>(w, tile, 0, lane, W0);
    auto step = [&](int b, const sx_w<DT>& W, sx_w<DT>& Wn) {
        /* image b landed (each wave waits for its own loads, the barrier for the others'); image b + 1's
           buffer was last read in step b - 1, which every wave has left */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const u32x4* cur = img + (b & 1) * SXW_PIECES;
        if (b + 1 < S) {
            sxw_fetch<DT, NW>(a, K, tt, b + 1, img + ((b + 1) & 1) * SXW_PIECES);
            sx_load_w<DT>(w, tile, b + 1, lane, Wn);
        }
        /* one unit's operands at a time (the barriers keep the scheduler from hoisting every unit's reads) */
        sx_a x;
        sxw_read<DT, 0>(cur, a, tt, K, b, lane, x);
        sx_compute<DT, 0>(W, x, kq, acc, cs);
        __builtin_amdgcn_sched_barrier(0);
        sxw_read<DT, 1>(cur, a, tt, K, b, lane, x);
        sx_compute<DT, 1>(W, x, kq, acc, cs);
        __builtin_amdgcn_sched_barrier(0);
        sxw_read<DT, 2>(cur, a, tt, K, b, lane, x);
        sx_compute<DT, 2>(W, x, kq, acc, cs);
        __builtin_amdgcn_sched_barrier(0);
        sxw_read<DT, 3>(cur, a, tt, K, b, lane, x);
        sx_compute<DT, 3>(W, x, kq, acc, cs);
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int b = 0; b < S; b += 2) {
        step(b, W0, W1);
        if (b + 1 < S) step(b + 1, W1, W0);
    }
}

/* Every matrix of the launch has dtype DT. */
template <int DT, int NW>
__global__ __launch_bounds__(64 * NW) void skinny_wide_kernel(skinny_args a) {
    __shared__ u32x4 img[2 * SXW_PIECES]; /* 64 KB */
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, l32 = lane & 31, kq = lane >> 5;
    int bx = blockIdx.x, mi = 0;
    for (; mi < a.nm - 1; mi++) {
        const int nb = ((a.w[mi].rows + 31) / 32 + NW - 1) / NW;
        if (bx < nb) break;
        bx -= nb;
    }
    const qmat& w = a.w[mi];
    const int tile = NW * bx + wv, tok0 = blockIdx.y * SK_TOK;
    f32x16 acc = {};
    sxw_body<DT, NW>(a, w, tile, blockIdx.y, img, acc);
    float* y = a.y[mi];
    const int n = 32 * tile + l32;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int tk = tok0 + 8 * (r >> 2) + 4 * kq + (r & 3);
        if (n < w.rows && tk < a.n) {
            float* o = y + (size_t)tk * w.rows + n;
            *o = a.add ? *o + acc[r] : acc[r];
        }
    }
}

static hipError_t launch_skinny_exact(const skinny_args& a0, hipStream_t s) {
    skinny_args a = a0;
    const int mt = (a.n + SK_TOK - 1) / SK_TOK;
    int blocks = 0, ks = 1, tiles = 0, split_max = 1;
    for (int i = 0; i < a.nm; i++) {
        const int S = a.w[i].cols / 256;
        a.splits[i] = (S + 7) / 8;
        ks = std::max(ks, std::min(S, 8));
        split_max = std::max(split_max, a.splits[i]);
        tiles += (a.w[i].rows + 31) / 32;
        blocks += (a.w[i].rows + 31) / 32 * a.splits[i];
    }
    a.tiles = tiles;
    a.split_max = split_max;
    bool one_dt = true;
    for (int i = 1; i < a.nm; i++) one_dt &= a.w[i].dtype == a.w[0].dtype;
    if (tiles >= 1024 && one_dt) {
        /* wide: NW tiles a block over the whole width, the activations shared through LDS (Q8_0 takes four
           waves a block: its two superblocks of weights in flight need more registers than eight allow) */
        const int dt = a.w[0].dtype, NW = dt == VITNA_DTYPE_Q8_0 ? 4 : 8;
        int wb = 0;
        for (int i = 0; i < a.nm; i++) wb += ((a.w[i].rows + 31) / 32 + NW - 1) / NW;
        const dim3 grid(wb, mt);
        if (dt == VITNA_DTYPE_Q4_K) skinny_wide_kernel<VITNA_DTYPE_Q4_K, 8><<<grid, 512, 0, s>>>(a);
        else if (dt == VITNA_DTYPE_Q6_K) skinny_wide_kernel<VITNA_DTYPE_Q6_K, 8><<<grid, 512, 0, s>>>(a);
        else skinny_wide_kernel<VITNA_DTYPE_Q8_0, 4><<<grid, 256, 0, s>>>(a);
        return hipGetLastError();
    }
    if (split_max > 1 && (!a.part || !a.cnt || (size_t)mt * tiles > a.cnt_cap || (size_t)mt * tiles * split_max * 1024 > a.part_cap))
        return hipErrorInvalidValue;
    /* many token tiles (a prompt's chunk): each block takes SK_NT of them, the weights loaded once for all, or
       two weight tiles against the same token tile, each unit's activations loaded once for both */
    const size_t lds = (size_t)ks * 16 * 64 * sizeof(float);
    if (mt >= 2 * SK_NT) {
        bool q8 = false;
        for (int i = 0; i < a.nm; i++) q8 |= a.w[i].dtype == VITNA_DTYPE_Q8_0;
        if (SK_NR == 2 && !q8) {
            int b2 = 0;
            for (int i = 0; i < a.nm; i++) b2 += ((a.w[i].rows + 31) / 32 + 1) / 2 * a.splits[i];
            skinny_exact_kernel<1, 2><<<dim3(b2, mt), 64 * ks, lds, s>>>(a);
        } else {
            skinny_exact_kernel<SK_NT, 1><<<dim3(blocks, (mt + SK_NT - 1) / SK_NT), 64 * ks, lds, s>>>(a);
        }
    } else {
        skinny_exact_kernel<1, 1><<<dim3(blocks, mt), 64 * ks, lds, s>>>(a);
    }
    return hipGetLastError();
}

hipError_t launch_skinny(const skinny_args& a, hipStream_t s) {
    if (a.nm < 1 || a.nm > 3 || a.n < 1) return hipErrorInvalidValue;
    for (int i = 0; i < a.nm; i++) {
        const int d = a.w[i].dtype;
        if (a.w[i].cols != a.w[0].cols || a.w[i].cols % 32) return hipErrorInvalidValue;
        if (d != VITNA_DTYPE_Q8_0 && d != VITNA_DTYPE_Q4_K && d != VITNA_DTYPE_Q6_K) return hipErrorInvalidValue;
    }
    bool exact = a.img[0] && a.img[1] && a.s16 && a.s32;
    for (int i = 0; i < a.nm; i++) exact &= a.w[i].cols % 256 == 0 && a.w[i].tiled;
    if (exact) return launch_skinny_exact(a, s);
    if (!a.xh || !a.xl) return hipErrorInvalidValue;
    int cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;
    const int want = 8 * cus; /* two waves a SIMD */
    const int mt = (a.n + SK_TOK - 1) / SK_TOK;
    const int S = a.w[0].cols / 32;
    int rows = 0;
    for (int i = 0; i < a.nm; i++) rows += a.w[i].rows;
    /* wide matrices (the LM head) take four 32-row tiles a wave, so each token tile's activations are read
       a quarter as often; the rest one */
    const bool wide = rows >= 32768;
    const int RB = wide ? 128 : 32, ks_max = wide ? 2 : 16;
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

/* ---- grouped experts of crowded passes ------------------------------------ */

/*
 * A pass whose experts hold many pairs each (a prompt's chunk: 1024 rows of top-8 over 128 experts, 64 pairs an
 * expert) runs its experts with the exact arithmetic above on tiles of 32 pairs of one expert, instead of the
 * four-pair tiles of kernels_gmma.hip, so that an expert's weights are read once per 32 pairs rather than once
 * per four. The pairs of each expert (launch_group's lists) are cut into tiles; tile t (of one expert, te[t])
 * is the virtual token tile t of the operand images, which a gather writes from the normalized rows. Gate and up
 * run in one block over the same activations; the block writes the SwiGLU output of its 32 x 32 (pair, row)
 * tile in fp32, whose images the same gather writes for down; down multiplies by the pair's weight into ypart,
 * as kernels_gmma.hip does. The weights come from a copy tiled as the dense matrices' are, experts back to back
 * (expert e's 32-row tile x is tile e I / 32 + x).
 *
 * Reference counterparts: experts_in_rows_kernel model_cuda.cu:2071 and experts_down_rows_kernel
 * model_cuda.cu:2101; the CPU arithmetic checked against is mixture_of_experts engine/src/model.c:745-761 and
 * vitna_silu_mul engine/src/ops.c:283, one row at a time.
 */

/* One block a (expert, 32-row tile, superblock): the expert's planes as a matrix of its own. */
__global__ void gsx_tile_kernel(qmat m, int tiles, uint8_t* __restrict__ dst) {
    const int S = m.cols / 256, b = blockIdx.x % S, tile = (blockIdx.x / S) % tiles, e = blockIdx.x / (S * tiles);
    qmat me = m;
#pragma unroll
    for (int i = 0; i < 4; i++) me.p[i] = m.p[i] ? m.p[i] + (size_t)e * m.estride[i] : nullptr;
    const int tb = (int)tile_bytes(m.dtype);
    uint8_t* out = dst + (size_t)blockIdx.x * tb;
    for (int o = threadIdx.x; o < tb; o += blockDim.x) out[o] = (uint8_t)tile_src(me, tile, b, o);
}

size_t gsx_tiled_bytes(const qmat& m, int n_experts) {
    return tile_bytes(m.dtype) * (size_t)(m.rows / 32) * (m.cols / 256) * n_experts;
}

hipError_t launch_gsx_tile(const qmat& m, int n_experts, uint8_t* dst, hipStream_t s) {
    if (!tile_bytes(m.dtype) || m.cols % 256 || m.rows % 32 || n_experts < 1) return hipErrorInvalidValue;
    const int tiles = m.rows / 32;
    gsx_tile_kernel<<<n_experts * tiles * (m.cols / 256), 256, 0, s>>>(m, tiles, dst);
    return hipGetLastError();
}

bool gsx_fits(const qmat& gate, const qmat& up, const qmat& down) {
    auto dt = [](int d) { return d == VITNA_DTYPE_Q8_0 || d == VITNA_DTYPE_Q4_K || d == VITNA_DTYPE_Q6_K; };
    const int H = gate.cols, I = gate.rows;
    /* whole superblocks, at most eight a row (one block's waves), whole 32-row tiles */
    return dt(gate.dtype) && up.dtype == gate.dtype && dt(down.dtype) && up.rows == I && up.cols == H && down.rows == H &&
           down.cols == I && H % 256 == 0 && I % 256 == 0 && H <= 2048 && I <= 2048;
}

int gsx_max_tiles(int n, int K, int E) { return (n * K + 31) / 32 + E; }

/* Tile offsets of the experts' pair lists (toff[E + 1]) and the expert of each tile (te[max_tiles], -1 past the
   last): one block, the first wave scanning the tile counts 64 experts at a time. */
__global__ __launch_bounds__(256) void gsx_plan_kernel(const int* __restrict__ count, int E, int* __restrict__ toff,
                                                       int* __restrict__ te, int max_tiles) {
    __shared__ int off[ROUTE_E_MAX + 1];
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        int run = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < E ? (count[e] + 31) / 32 : 0;
            int v = c; /* inclusive scan across the wave */
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int o = __shfl_up(v, d, WAVE);
                if (lane >= d) v += o;
            }
            if (e < E) off[e] = run + v - c;
            run += __shfl(v, 63, WAVE);
        }
        if (lane == 0) off[E] = run;
    }
    __syncthreads();
    for (int e = tid; e <= E; e += blockDim.x) toff[e] = off[e];
    for (int e = tid; e < E; e += blockDim.x)
        for (int t = off[e]; t < off[e + 1]; t++) te[t] = e;
    for (int t = off[E] + tid; t < max_tiles; t += blockDim.x) te[t] = -1;
}

/* The operand images (one column order) and group sums of the virtual token tiles: block (b, t) takes superblock
   b of tile t. With pairs, token l of tile t is pair toff-relative index 32 (t - toff[e]) + l of expert te[t]
   (past its count: the last pair again), read from row pair / ROUTE_K_MAX of x; without, it is row 32 t + l of x. */
__global__ void gsx_image_kernel(const float* __restrict__ x, int K, const int* __restrict__ pairs, const int* __restrict__ count,
                                 int cap, const int* __restrict__ toff, const int* __restrict__ te, u32x4* __restrict__ imga,
                                 u32x4* __restrict__ imgb, uint16_t* __restrict__ s32, uint16_t* __restrict__ s16) {
    const int b = blockIdx.x, t = blockIdx.y;
    const int e = te[t];
    if (e < 0) return;
    const int j0 = 32 * (t - toff[e]), c = count[e];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int item = threadIdx.x + 256 * j, l = item >> 5, c8 = 32 * b + (item & 31);
        const int row = 32 * t + l;
        size_t src_row = (size_t)row;
        if (pairs) src_row = (size_t)(pairs[(size_t)e * cap + min(j0 + l, c - 1)] / ROUTE_K_MAX);
        const float4* src = reinterpret_cast<const float4*>(x + src_row * K + 8 * c8);
        const float4 v0 = src[0], v1 = src[1];
        const float ev[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        u32x4 vh, vl;
        float sum;
        img_split8(ev, vh, vl, sum);
        img_put(imga, imgb, row, K, c8, vh, vl);
        const float t16 = sum + __shfl_xor(sum, 1, WAVE);
        const float t32 = t16 + __shfl_xor(t16, 2, WAVE);
        if (!(c8 & 1)) img_sum16(s16, row, K, c8 >> 1, t16);
        if (!(c8 & 3)) img_sum32(s32, row, K, c8 >> 2, t32);
    }
}

/* The KS waves' tiles added in wave order through red ([KS][16][64]); wave wv returns the sums of accumulators
   wv, wv + KS, ... in out[0], out[1], ... */
__device__ __forceinline__ void gsx_reduce(const f32x16& acc, float* red, int KS, int wv, int lane, float out[16]) {
    __syncthreads(); /* red is free */
#pragma unroll
    for (int r = 0; r < 16; r++) red[(wv * 16 + r) * 64 + lane] = acc[r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int r = wv + i * KS;
        if (r < 16) {
            float v = 0.0f;
            for (int u = 0; u < KS; u++) v += red[(u * 16 + r) * 64 + lane];
            out[i] = v;
        }
    }
}

/* act[32 t + token][32 x + row] = silu(gate . x) * (up . x) for virtual tile t (expert te[t]) and 32-row tile x
   (blockIdx.x) of the expert's I rows: KS = H / 256 waves, wave wv on superblock wv of both matrices, each unit's
   activations loaded once for both. */
template <int DT>
__global__ __launch_bounds__(512) void gsx_in_kernel(qmat gate, qmat up, skinny_args sa, const int* __restrict__ te,
                                                     float* __restrict__ act) {
    extern __shared__ float red[];
    const int t = blockIdx.y, e = te[t];
    if (e < 0) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, KS = blockDim.x >> 6, kq = lane >> 5, l32 = lane & 31;
    const int H = gate.cols, I = gate.rows, x = blockIdx.x, tile = e * (I / 32) + x, b = wv;
    f32x16 ag = {}, au = {};
    {
        sx_w<DT> Wg, Wu;
        sx_load_w<DT>(gate, tile, b, lane, Wg);
        sx_load_w<DT>(up, tile, b, lane, Wu);
        float cg[8], cu[8];
        sx_a x0, x1;
        sx_load_a<DT, 0>(sa, t, H, b, lane, x0);
        sx_load_a<DT, 1>(sa, t, H, b, lane, x1);
        __builtin_amdgcn_sched_barrier(0);
        sx_compute<DT, 0>(Wg, x0, kq, ag, cg);
        sx_compute<DT, 0>(Wu, x0, kq, au, cu);
        sx_load_a<DT, 2>(sa, t, H, b, lane, x0);
        __builtin_amdgcn_sched_barrier(0);
        sx_compute<DT, 1>(Wg, x1, kq, ag, cg);
        sx_compute<DT, 1>(Wu, x1, kq, au, cu);
        sx_load_a<DT, 3>(sa, t, H, b, lane, x1);
        __builtin_amdgcn_sched_barrier(0);
        sx_compute<DT, 2>(Wg, x0, kq, ag, cg);
        sx_compute<DT, 2>(Wu, x0, kq, au, cu);
        sx_compute<DT, 3>(Wg, x1, kq, ag, cg);
        sx_compute<DT, 3>(Wu, x1, kq, au, cu);
    }
    float g[16], u[16];
    gsx_reduce(ag, red, KS, wv, lane, g);
    gsx_reduce(au, red, KS, wv, lane, u);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int r = wv + i * KS;
        if (r < 16) {
            /* accumulator r: token 8 (r / 4) + 4 kq + r % 4 of the tile, row l32 of the tile */
            const int tok = 8 * (r >> 2) + 4 * kq + (r & 3);
            const float v = (g[i] / (1.0f + expf(-g[i]))) * u[i];
            act[(size_t)(32 * t + tok) * I + 32 * x + l32] = v;
        }
    }
}

/* ypart[(row K + slot) H + n] = w_slot (down_e[n] . act[pair]) for the pairs of virtual tile t (past the expert's
   count: none written) and NR 32-row tiles from NR x of the H rows (each unit's activations loaded once for
   them): KS = I / 256 waves, wave wv on superblock wv. */
template <int DT, int NR>
__global__ __launch_bounds__(512) void gsx_down_kernel(qmat down, skinny_args sa, const int* __restrict__ te,
                                                       const int* __restrict__ toff, const int* __restrict__ count,
                                                       const int* __restrict__ pairs, int cap, const route_out* __restrict__ rt,
                                                       int K, float* __restrict__ ypart) {
    extern __shared__ float red[];
    const int t = blockIdx.y, e = te[t];
    if (e < 0) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, KS = blockDim.x >> 6, kq = lane >> 5, l32 = lane & 31;
    const int H = down.rows, x0 = NR * blockIdx.x;
    f32x16 acc[NR][1];
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r][0] = f32x16{};
    sx_superblock<DT, 1, NR>(sa, down, e * (H / 32) + x0, NR, t, t + 1, wv, lane, acc);
    const int j0 = 32 * (t - toff[e]), c = count[e];
#pragma unroll
    for (int wr = 0; wr < NR; wr++) {
        float v[16];
        gsx_reduce(acc[wr][0], red, KS, wv, lane, v);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = wv + i * KS;
            if (r < 16) {
                const int j = j0 + 8 * (r >> 2) + 4 * kq + (r & 3);
                if (j < c) {
                    const int p = pairs[(size_t)e * cap + j], row = p / ROUTE_K_MAX, slot = p % ROUTE_K_MAX;
                    ypart[((size_t)row * K + slot) * H + 32 * (x0 + wr) + l32] = rt[row].weights[slot] * v[i];
                }
            }
        }
    }
}

hipError_t launch_gsx(const gsx_args& a, hipStream_t s) {
    if (!gsx_fits(a.gate, a.up, a.down) || !a.gate.tiled || !a.up.tiled || !a.down.tiled || a.K < 1 || a.K > ROUTE_K_MAX ||
        a.E < 1 || a.E > ROUTE_E_MAX || a.n < 1 || a.cap < a.n || a.max_tiles < gsx_max_tiles(a.n, a.K, a.E))
        return hipErrorInvalidValue;
    const int H = a.gate.cols, I = a.gate.rows, T = gsx_max_tiles(a.n, a.K, a.E);
    gsx_plan_kernel<<<1, 256, 0, s>>>(a.count, a.E, a.toff, a.te, T);
    const bool in_b = a.gate.dtype == VITNA_DTYPE_Q6_K, dn_b = a.down.dtype == VITNA_DTYPE_Q6_K;
    u32x4* ii = reinterpret_cast<u32x4*>(a.img_in);
    u32x4* ia = reinterpret_cast<u32x4*>(a.img_act);
    gsx_image_kernel<<<dim3(H / 256, T), 256, 0, s>>>(a.xn, H, a.pairs, a.count, a.cap, a.toff, a.te, in_b ? nullptr : ii,
                                                      in_b ? ii : nullptr, a.s32, a.s16);
    skinny_args si{};
    si.img[0] = si.img[1] = a.img_in;
    si.s32 = reinterpret_cast<const uint32_t*>(a.s32);
    si.s16 = reinterpret_cast<const uint32_t*>(a.s16);
    const int ksi = H / 256, ksd = I / 256;
    const dim3 gi(I / 32, T), gd(H / 32, T);
    switch (a.gate.dtype) {
    case VITNA_DTYPE_Q4_K: gsx_in_kernel<VITNA_DTYPE_Q4_K><<<gi, 64 * ksi, ksi * 4096, s>>>(a.gate, a.up, si, a.te, a.act); break;
    case VITNA_DTYPE_Q6_K: gsx_in_kernel<VITNA_DTYPE_Q6_K><<<gi, 64 * ksi, ksi * 4096, s>>>(a.gate, a.up, si, a.te, a.act); break;
    default: gsx_in_kernel<VITNA_DTYPE_Q8_0><<<gi, 64 * ksi, ksi * 4096, s>>>(a.gate, a.up, si, a.te, a.act); break;
    }
    gsx_image_kernel<<<dim3(I / 256, T), 256, 0, s>>>(a.act, I, nullptr, a.count, a.cap, a.toff, a.te, dn_b ? nullptr : ia,
                                                      dn_b ? ia : nullptr, a.s32, a.s16);
    skinny_args sd{};
    sd.img[0] = sd.img[1] = a.img_act;
    sd.s32 = reinterpret_cast<const uint32_t*>(a.s32);
    sd.s16 = reinterpret_cast<const uint32_t*>(a.s16);
    /* two 32-row tiles a block for K-quant down weights (Q8_0's two do not fit the registers) */
    const dim3 gd2(H / 64, T);
    switch (a.down.dtype) {
    case VITNA_DTYPE_Q4_K:
        gsx_down_kernel<VITNA_DTYPE_Q4_K, 2><<<gd2, 64 * ksd, ksd * 4096, s>>>(a.down, sd, a.te, a.toff, a.count, a.pairs, a.cap, a.rt, a.K, a.ypart);
        break;
    case VITNA_DTYPE_Q6_K:
        gsx_down_kernel<VITNA_DTYPE_Q6_K, 2><<<gd2, 64 * ksd, ksd * 4096, s>>>(a.down, sd, a.te, a.toff, a.count, a.pairs, a.cap, a.rt, a.K, a.ypart);
        break;
    default:
        gsx_down_kernel<VITNA_DTYPE_Q8_0, 1><<<gd, 64 * ksd, ksd * 4096, s>>>(a.down, sd, a.te, a.toff, a.count, a.pairs, a.cap, a.rt, a.K, a.ypart);
        break;
    }
    return hipGetLastError();
}
