/**
 * vitna_hip_internal.h - What the HIP translation units of libvitna_hip share:
 * the device layout of a quantized matrix, the per-slice dot products of the
 * decode GEMV, exact-order reductions, and launch helpers. gfx950 only.
 *
 * Compiled with -ffp-contract=off: no multiply is fused into an add unless
 * the code says fmaf, so the exact paths (RMSNorm, router, widening) round
 * where the reference's CPU code rounds, and the fast paths fuse where they
 * choose to.
 *
 * Device layout of a block-format matrix ("planes"). The host hands over
 * GGUF blocks (engine/include/quant.h, vitna_model.h); on upload each block is
 * split by field into planes, each plane row-major over (row, block), so that
 * every field a kernel reads is 16-byte aligned and a wavefront's loads are
 * contiguous. The bytes are the block's own, regrouped, no more and no fewer:
 *   Q8_0: P0 q     [rows][nb][32] int8    P1 d [rows][nb] f16
 *   Q4_K: P0 q     [rows][nb][128]        P1 hdr [rows][nb][16] = d, dmin, 12 scale bytes
 *   Q6_K: P0 ql    [rows][nb][128]        P1 qh [rows][nb][64]
 *         P2 sc    [rows][nb][16] int8    P3 d  [rows][nb] f16
 *   F32 : P0 the floats, rows x cols.
 * A set of experts of one part keeps each plane of every expert back to back,
 * expert e's plane i at p[i] + e * estride[i].
 *
 * The decode GEMV splits a row into slices of 32 weights, one per lane: slice
 * t of a row reads 16 bytes of P0 (Q8_0: 32), and its weights sit at two runs
 * of 16 columns, lo and hi (slice_cols). A lane keeps its slices' activations
 * in registers for every row it visits.
 */

#ifndef VITNA_HIP_INTERNAL_H
#define VITNA_HIP_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include "../../include/vitna_model.h"

#define WAVE 64

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


struct qmat {
    const uint8_t* p[4];
    uint64_t estride[4];  /* bytes between experts' planes; 0 for a single matrix */
    int rows, cols, nb;   /* nb: blocks a row */
    int dtype;
    /* A second copy of a dense matrix for the multi-row kernels, or null: per 32-row tile and 256-column
       superblock, tile_bytes() bytes in the order the MFMA lanes read them (kernels_skinny.hip). */
    const uint8_t* tiled;
};

/* Bytes of one 32-row tile's superblock in the tiled copy; 0 for a dtype without one. */
__host__ __device__ static inline size_t tile_bytes(int dtype) {
    return dtype == VITNA_DTYPE_Q4_K ? 4608 : dtype == VITNA_DTYPE_Q6_K ? 6720 : dtype == VITNA_DTYPE_Q8_0 ? 8704 : 0;
}

/* ---- host-side layout arithmetic, shared with the upload code ---- */

static inline size_t plane_bytes(int dtype, int plane, size_t rows, size_t cols) {
    const size_t nb = cols / (dtype == VITNA_DTYPE_Q8_0 ? 32 : 256);
    switch (dtype) {
        case VITNA_DTYPE_F32: return plane == 0 ? rows * cols * 4 : 0;
        case VITNA_DTYPE_Q8_0: return plane == 0 ? rows * nb * 32 : plane == 1 ? rows * nb * 2 : 0;
        case VITNA_DTYPE_Q4_K: return plane == 0 ? rows * nb * 128 : plane == 1 ? rows * nb * 16 : 0;
        case VITNA_DTYPE_Q6_K:
            return plane == 0 ? rows * nb * 128 : plane == 1 ? rows * nb * 64 : plane == 2 ? rows * nb * 16 : plane == 3 ? rows * nb * 2 : 0;
        default: return 0;
    }
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

/* ---- device helpers ---- */

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

/* The AVX2 horizontal tree over sixteen chain sums held by lanes j = 0..15 of
   a 16-lane group (engine/src/ops.c:165-170, kernels.c:140-146):
   v_j = a_j + a_{j+8}, then ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)).
   Valid in lane j = 0 of the group. */
__device__ __forceinline__ float fold16_lanes(float a);

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

/* Sum over the 32-lane halves of a wave separately. */
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

/* ---- cross-lane reductions on the DPP paths (no LDS traffic) ----
   A lane whose DPP source falls outside its row, or whose row or bank is
   masked off, reads `old`: the identity of the reduction. */
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v, float old) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}
#define DPP_ROW_SHR(n) (0x110 + (n))
#define DPP_ROW_BCAST15 0x142
#define DPP_ROW_BCAST31 0x143
#define DPP_QUAD_XOR1 0xB1 /* quad_perm [1,0,3,2] */
#define DPP_QUAD_XOR2 0x4E /* quad_perm [2,3,0,1] */

/* Sum over each group of four lanes, in every lane of the group. */
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f<DPP_QUAD_XOR1, 0xf, 0xf>(v, 0.0f);
    return v + dpp_f<DPP_QUAD_XOR2, 0xf, 0xf>(v, 0.0f);
}

/* Doubling scans within each 16-lane row: lane 15 of a row ends with the row's total. */
__device__ __forceinline__ float row_scan_sum(float v) {
    v += dpp_f<DPP_ROW_SHR(1), 0xf, 0xf>(v, 0.0f);
    v += dpp_f<DPP_ROW_SHR(2), 0xf, 0xf>(v, 0.0f);
    v += dpp_f<DPP_ROW_SHR(4), 0xf, 0xf>(v, 0.0f);
    return v + dpp_f<DPP_ROW_SHR(8), 0xf, 0xf>(v, 0.0f);
}
/* For a maximum a lane with no source reads its own value (max(v, v) = v), which lets the compiler fold
   the move into v_max_f32_dpp. */
__device__ __forceinline__ float row_scan_max(float v) {
    v = fmaxf(v, dpp_f<DPP_ROW_SHR(1), 0xf, 0xf>(v, v));
    v = fmaxf(v, dpp_f<DPP_ROW_SHR(2), 0xf, 0xf>(v, v));
    v = fmaxf(v, dpp_f<DPP_ROW_SHR(4), 0xf, 0xf>(v, v));
    return fmaxf(v, dpp_f<DPP_ROW_SHR(8), 0xf, 0xf>(v, v));
}

/* Sum of the wave, in every lane (the total gathers in lane 63, then a readlane). */
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = row_scan_sum(v);
    v += dpp_f<DPP_ROW_BCAST15, 0xa, 0xf>(v, 0.0f);
    v += dpp_f<DPP_ROW_BCAST31, 0xc, 0xf>(v, 0.0f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = row_scan_max(v);
    v = fmaxf(v, dpp_f<DPP_ROW_BCAST15, 0xa, 0xf>(v, v));
    v = fmaxf(v, dpp_f<DPP_ROW_BCAST31, 0xc, 0xf>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

/* Slices of one row split among LPR lanes: the sum over each group of LPR
   consecutive lanes, complete in the group's last lane (lane LPR - 1 of the
   group): doubling scans within 16-lane rows, then row broadcasts for groups
   of 32 and 64. */
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
    if constexpr (LPR >= 2) v += dpp_f<DPP_ROW_SHR(1), 0xf, 0xf>(v, 0.0f);
    if constexpr (LPR >= 4) v += dpp_f<DPP_ROW_SHR(2), 0xf, 0xf>(v, 0.0f);
    if constexpr (LPR >= 8) v += dpp_f<DPP_ROW_SHR(4), 0xf, 0xf>(v, 0.0f);
    if constexpr (LPR >= 16) v += dpp_f<DPP_ROW_SHR(8), 0xf, 0xf>(v, 0.0f);
    if constexpr (LPR >= 32) v += dpp_f<DPP_ROW_BCAST15, 0xa, 0xf>(v, 0.0f);
    if constexpr (LPR >= 64) v += dpp_f<DPP_ROW_BCAST31, 0xc, 0xf>(v, 0.0f);
    return v;
}

#define DPP_ROW_SHL(n) (0x100 + (n))
__device__ __forceinline__ float fold16_lanes(float a) {
    /* lane j adds lane j + 8 (row_shl reads the higher lane), then + 4, + 2, + 1 */
    const float v = a + dpp_f<DPP_ROW_SHL(8), 0xf, 0xf>(a, 0.0f);
    const float s = v + dpp_f<DPP_ROW_SHL(4), 0xf, 0xf>(v, 0.0f);
    const float u = s + dpp_f<DPP_ROW_SHL(2), 0xf, 0xf>(s, 0.0f);
    return u + dpp_f<DPP_ROW_SHL(1), 0xf, 0xf>(u, 0.0f);
}

/* Sum over each 32-lane half of the wave, in every lane of the half. */
__device__ __forceinline__ float half_sum_dpp(float v) {
    v = row_scan_sum(v);
    v += dpp_f<DPP_ROW_BCAST15, 0xa, 0xf>(v, 0.0f);
    const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return (threadIdx.x & 32) ? hi : lo;
}

/* The value of lane (this lane xor 16), within each 32-lane half (ds_swizzle, bit mode). */
__device__ __forceinline__ float swap16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}

/* Columns of slice t of a row: two runs of 16, starting at *lo and *hi. */
__device__ __forceinline__ void slice_cols(int dtype, int t, int* lo, int* hi) {
    if (dtype == VITNA_DTYPE_Q8_0) {
        *lo = 32 * t;
        *hi = 32 * t + 16;
    } else if (dtype == VITNA_DTYPE_Q4_K) {
        /* bytes 16p .. 16p+15 of the block's 128 q: chunk c = p/2 holds groups
           2c (low nibbles) and 2c+1 (high), at element 16(p&1) + i */
        const int b = t >> 3, p = t & 7, c = p >> 1;
        *lo = 256 * b + 64 * c + 16 * (p & 1);
        *hi = *lo + 32;
    } else if (dtype == VITNA_DTYPE_Q6_K) {
        /* u = 4h + 2r0 + s: ql bytes 64h + 32r0 + 16s + i carry weights
           128h + 32r0 + 16s + i (low nibble) and 128h + 32(r0+2) + 16s + i (high) */
        const int b = t >> 3, u = t & 7, h = u >> 2, r0 = (u >> 1) & 1, s = u & 1;
        *lo = 256 * b + 128 * h + 32 * r0 + 16 * s;
        *hi = *lo + 64;
    } else {
        *lo = 32 * t;
        *hi = 32 * t + 16;
    }
}

/* A lane's activations for one slice: the two runs, and their sums. */
struct xslice {
    float lo[16], hi[16];
    float slo, shi;
};

__device__ __forceinline__ void load_xslice(int dtype, int t, const float* __restrict__ x, xslice& xs) {
    int a, b;
    slice_cols(dtype, t, &a, &b);
    const float4* pa = reinterpret_cast<const float4*>(x + a);
    const float4* pb = reinterpret_cast<const float4*>(x + b);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 u = pa[i], v = pb[i];
        xs.lo[4 * i] = u.x; xs.lo[4 * i + 1] = u.y; xs.lo[4 * i + 2] = u.z; xs.lo[4 * i + 3] = u.w;
        xs.hi[4 * i] = v.x; xs.hi[4 * i + 1] = v.y; xs.hi[4 * i + 2] = v.z; xs.hi[4 * i + 3] = v.w;
    }
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) { s0 += xs.lo[i]; s1 += xs.hi[i]; }
    xs.slo = s0;
    xs.shi = s1;
}

/* The four bytes of w as floats, into f[0..3] (each one v_cvt_f32_ubyteN). */
#define BYTES_TO_F(w, f)                                    \
    do {                                                    \
        (f)[0] = (float)((w) & 0xffu);                      \
        (f)[1] = (float)(((w) >> 8) & 0xffu);               \
        (f)[2] = (float)(((w) >> 16) & 0xffu);              \
        (f)[3] = (float)((w) >> 24);                        \
    } while (0)

/* Raw bytes of one slice, loaded ahead of the arithmetic so a lane can keep
   several rows' loads in flight. */
struct qraw {
    u32x4 a;      /* Q8_0: q[0..15]; Q4_K: q bytes; Q6_K: ql bytes */
    u32x4 b;      /* Q8_0: q[16..31]; Q4_K: header; Q6_K: qh bytes */
    uint32_t c;   /* Q8_0: d; Q6_K: scale bytes 8h .. 8h + 3 of the block (h: the slice's half), or, picked at
                     the load (PICK), the slice's two (lo run | hi run << 8) */
    uint32_t d;   /* Q6_K: d */
    uint32_t e;   /* Q6_K: scale bytes 8h + 4 .. 8h + 7 (not PICK) */
};

/* A load from device memory through a global-address-space pointer: a global_load, counted by vmcnt alone (a
   flat load is counted by lgkmcnt too, so an LDS wait would also wait for it). */
template <typename T>
__device__ __forceinline__ T gld(const void* p) {
    typedef uint32_t w2 __attribute__((ext_vector_type(2)));
    if constexpr (sizeof(T) == 16) return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) u32x4*)p);
    else if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) w2*)p);
    else if constexpr (sizeof(T) == 4) return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) uint32_t*)p);
    else if constexpr (sizeof(T) == 2) return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) uint16_t*)p);
    else return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) uint8_t*)p);
}

/* PICK (Q6_K): the slice's two scale bytes picked as they are loaded, one register a slice instead of two, for
   kernels short of registers; otherwise the half's eight bytes are kept as loaded and picked by slice_dot (picking
   them at the load makes the wave wait for the load there, and a wait counts every load issued before it). */
template <int DT, bool PICK = false>
__device__ __forceinline__ void slice_load(const qmat& m, int e, int row, int t, qraw& r) {
    const size_t blk = (size_t)row * m.nb + (t >> (DT == VITNA_DTYPE_Q8_0 ? 0 : 3));
    if (DT == VITNA_DTYPE_Q8_0) {
        const uint8_t* q = m.p[0] + e * m.estride[0] + blk * 32;
        r.a = gld<u32x4>(q);
        r.b = gld<u32x4>(q + 16);
        r.c = gld<uint16_t>(m.p[1] + e * m.estride[1] + blk * 2);
    } else if (DT == VITNA_DTYPE_Q4_K) {
        r.a = gld<u32x4>(m.p[0] + e * m.estride[0] + blk * 128 + 16 * (t & 7));
        r.b = gld<u32x4>(m.p[1] + e * m.estride[1] + blk * 16);
    } else if (DT == VITNA_DTYPE_Q6_K) {
        const int u = t & 7, h = u >> 2, r0 = (u >> 1) & 1, s = u & 1;
        r.a = gld<u32x4>(m.p[0] + e * m.estride[0] + blk * 128 + 64 * h + 32 * r0 + 16 * s);
        r.b = gld<u32x4>(m.p[1] + e * m.estride[1] + blk * 64 + 32 * h + 16 * s);
        if constexpr (PICK) {
            /* scale of weights i: i / 16 = 8h + 2r + s, for r = r0 and r0 + 2 */
            const uint8_t* sc = m.p[2] + e * m.estride[2] + blk * 16;
            r.c = (uint32_t)gld<uint8_t>(sc + 8 * h + 2 * r0 + s) | ((uint32_t)gld<uint8_t>(sc + 8 * h + 2 * r0 + 4 + s) << 8);
        } else {
            /* the half's eight scale bytes as they lie (one 8-byte load; the planes are 8-byte aligned) */
            typedef uint32_t w2 __attribute__((ext_vector_type(2)));
            const w2 sc = gld<w2>(m.p[2] + e * m.estride[2] + blk * 16 + 8 * h);
            r.c = sc.x;
            r.e = sc.y;
        }
        r.d = gld<uint16_t>(m.p[3] + e * m.estride[3] + blk * 2);
    }
}

/* The slice's dot product with the lane's activations, fp32 accumulate. The
   per-weight widening w = f(q) is folded: sum (d1 q - m1) x = d1 sum(q x) -
   m1 sum(x), so the inner loop is a byte-to-float convert and one FMA. */
template <int DT, bool PICK = false>
__device__ __forceinline__ float slice_dot(const qraw& r, int t, const xslice& xs) {
    if (DT == VITNA_DTYPE_Q8_0) {
        /* q + 128 as unsigned bytes, the 128 x sum taken back out */
        const uint32_t w[8] = {r.a.x ^ 0x80808080u, r.a.y ^ 0x80808080u, r.a.z ^ 0x80808080u, r.a.w ^ 0x80808080u,
                               r.b.x ^ 0x80808080u, r.b.y ^ 0x80808080u, r.b.z ^ 0x80808080u, r.b.w ^ 0x80808080u};
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float f[4];
            BYTES_TO_F(w[j], f);
#pragma unroll
            for (int i = 0; i < 4; i++) acc0 = fmaf(f[i], xs.lo[4 * j + i], acc0);
            BYTES_TO_F(w[4 + j], f);
#pragma unroll
            for (int i = 0; i < 4; i++) acc1 = fmaf(f[i], xs.hi[4 * j + i], acc1);
        }
        const float d = f16_bits_to_f32(r.c);
        const float s = (acc0 + acc1) - 128.0f * (xs.slo + xs.shi);
        return d * s;
    } else if (DT == VITNA_DTYPE_Q4_K) {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t lo = w[j] & 0x0f0f0f0fu, hi = (w[j] >> 4) & 0x0f0f0f0fu;
            float f[4];
            BYTES_TO_F(lo, f);
#pragma unroll
            for (int i = 0; i < 4; i++) acc0 = fmaf(f[i], xs.lo[4 * j + i], acc0);
            BYTES_TO_F(hi, f);
#pragma unroll
            for (int i = 0; i < 4; i++) acc1 = fmaf(f[i], xs.hi[4 * j + i], acc1);
        }
        const uint32_t h0 = r.b.x, h1 = r.b.y, h2 = r.b.z, h3 = r.b.w;
        const float d = f16_bits_to_f32(h0 & 0xffffu), dmin = f16_bits_to_f32(h0 >> 16);
        /* scale bytes s[0..11] = bytes of h1, h2, h3; groups g0 = 2c, g1 = 2c + 1 */
        const int c = (t & 7) >> 1;
        const uint32_t s03 = h1, s47 = h2, s8b = h3;
        uint32_t sc0, mn0, sc1, mn1;
        if (c < 2) {
            const int g0 = 2 * c, g1 = g0 + 1;
            sc0 = (s03 >> (8 * g0)) & 63; mn0 = (s47 >> (8 * g0)) & 63;
            sc1 = (s03 >> (8 * g1)) & 63; mn1 = (s47 >> (8 * g1)) & 63;
        } else {
            const int j0 = 2 * c - 4, j1 = j0 + 1; /* g - 4 */
            sc0 = ((s8b >> (8 * j0)) & 15) | (((s03 >> (8 * j0 + 6)) & 3) << 4);
            mn0 = ((s8b >> (8 * j0 + 4)) & 15) | (((s47 >> (8 * j0 + 6)) & 3) << 4);
            sc1 = ((s8b >> (8 * j1)) & 15) | (((s03 >> (8 * j1 + 6)) & 3) << 4);
            mn1 = ((s8b >> (8 * j1 + 4)) & 15) | (((s47 >> (8 * j1 + 6)) & 3) << 4);
        }
        const float d0 = d * (float)sc0, m0 = dmin * (float)mn0, d1 = d * (float)sc1, m1 = dmin * (float)mn1;
        return fmaf(d0, acc0, fmaf(d1, acc1, -(m0 * xs.slo + m1 * xs.shi)));
    } else { /* Q6_K */
        const uint32_t ql[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, qh[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        /* slice u = 4h + 2r0 + s: its high bits shifted by 2 r0; weights i / 16 = 8h + 2r + s for r = r0 (scale byte
           2 r0 + s of the half's first four) and r0 + 2 (the same byte of the next four) */
        const int u = t & 7, r0 = (u >> 1) & 1, bi = 2 * r0 + (u & 1);
        const int sh = 2 * r0;
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t hb = qh[j] >> sh;
            const uint32_t q0 = (ql[j] & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4);
            const uint32_t q1 = ((ql[j] >> 4) & 0x0f0f0f0fu) | (((hb >> 4) & 0x03030303u) << 4);
            float f[4];
            BYTES_TO_F(q0, f);
#pragma unroll
            for (int i = 0; i < 4; i++) acc0 = fmaf(f[i], xs.lo[4 * j + i], acc0);
            BYTES_TO_F(q1, f);
#pragma unroll
            for (int i = 0; i < 4; i++) acc1 = fmaf(f[i], xs.hi[4 * j + i], acc1);
        }
        const float d = f16_bits_to_f32(r.d);
        const float s0 = (float)(int8_t)((PICK ? r.c : r.c >> (8 * bi)) & 0xff);
        const float s1 = (float)(int8_t)((PICK ? r.c >> 8 : r.e >> (8 * bi)) & 0xff);
        const float a0 = acc0 - 32.0f * xs.slo, a1 = acc1 - 32.0f * xs.shi;
        return d * fmaf(s0, a0, s1 * a1);
    }
}

/* F32 slice: 32 consecutive floats, the two runs. */
__device__ __forceinline__ float slice_dot_f32(const float* __restrict__ row, int t, const xslice& xs) {
    const float4* p = reinterpret_cast<const float4*>(row + 32 * t);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 u = p[i];
        acc = fmaf(u.x, xs.lo[4 * i], acc); acc = fmaf(u.y, xs.lo[4 * i + 1], acc);
        acc = fmaf(u.z, xs.lo[4 * i + 2], acc); acc = fmaf(u.w, xs.lo[4 * i + 3], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 u = p[4 + i];
        acc = fmaf(u.x, xs.hi[4 * i], acc); acc = fmaf(u.y, xs.hi[4 * i + 1], acc);
        acc = fmaf(u.z, xs.hi[4 * i + 2], acc); acc = fmaf(u.w, xs.hi[4 * i + 3], acc);
    }
    return acc;
}

/* Exact widening of one weight from the planes, as the reference's CPU code
   widens it (engine/src/quant.c:40-188): every product rounded on its own
   (the library is built without contraction). Used by the widen checker and
   the prefill GEMM's LDS staging. */
__device__ __forceinline__ float widen_one(const qmat& m, int e, int row, int col) {
    if (m.dtype == VITNA_DTYPE_F32) return reinterpret_cast<const float*>(m.p[0] + e * m.estride[0])[(size_t)row * m.cols + col];
    if (m.dtype == VITNA_DTYPE_Q8_0) {
        const size_t blk = (size_t)row * m.nb + (col >> 5);
        const int8_t q = (int8_t)m.p[0][e * m.estride[0] + blk * 32 + (col & 31)];
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(m.p[1] + e * m.estride[1] + blk * 2));
        return (float)q * d;
    }
    if (m.dtype == VITNA_DTYPE_Q4_K) {
        const size_t blk = (size_t)row * m.nb + (col >> 8);
        const int i = col & 255, g = i >> 5, l = i & 31;
        const uint8_t* h = m.p[1] + e * m.estride[1] + blk * 16;
        const uint8_t* s = h + 4;
        const float d = f16_bits_to_f32(h[0] | (h[1] << 8)), dmin = f16_bits_to_f32(h[2] | (h[3] << 8));
        int sc, mn;
        if (g < 4) { sc = s[g] & 63; mn = s[g + 4] & 63; }
        else { sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4); mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4); }
        const uint8_t qb = m.p[0][e * m.estride[0] + blk * 128 + 32 * (g >> 1) + l];
        const int q = (g & 1) ? (qb >> 4) : (qb & 15);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        const float p = d1 * (float)q;
        return p - m1;
    }
    if (m.dtype == VITNA_DTYPE_Q6_K) {
        const size_t blk = (size_t)row * m.nb + (col >> 8);
        const int i = col & 255, h = i >> 7, r = (i >> 5) & 3, l = i & 31;
        const uint8_t ql = m.p[0][e * m.estride[0] + blk * 128 + 64 * h + 32 * (r & 1) + l];
        const uint8_t qh = m.p[1][e * m.estride[1] + blk * 64 + 32 * h + l];
        const int q = (((ql >> (4 * (r >> 1))) & 15) | (((qh >> (2 * r)) & 3) << 4)) - 32;
        const int8_t sc = (int8_t)m.p[2][e * m.estride[2] + blk * 16 + (i >> 4)];
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(m.p[3] + e * m.estride[3] + blk * 2));
        const float ds = d * (float)sc;
        return ds * (float)q;
    }
    return 0.0f;
}

/* ---- kernels' launch entry points (host side, per translation unit) ---- */

struct ffn_args;  /* defined in the units that use it */

#endif
