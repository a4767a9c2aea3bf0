/**
 * kernels_gmma.hip - The grouped experts of a ragged decode pass on the bf16
 * matrix cores: every selected expert's gate/up and down rows are read once,
 * for all the tokens routed to it (four a tile), to fp32 accuracy.
 *
 * Reference counterparts: experts_in_rows_kernel model_cuda.cu:2071 and
 * experts_down_rows_kernel model_cuda.cu:2101 (each expert read once for up
 * to 8 rows, on the CUDA cores); the CPU arithmetic checked against is
 * mixture_of_experts engine/src/model.c:745-761 and vitna_silu_mul
 * engine/src/ops.c:283, one row at a time.
 *
 * Shape. A decode pass routes a handful of tokens to each expert (32 rows,
 * top-8 of 128: about 2.3 an expert), so the contraction is 4 tokens x many
 * weight rows. v_mfma_f32_4x4x4_16b_bf16 is sixteen 4x4x4 products; block b
 * (lanes 4b .. 4b + 3) takes its A rows (the tokens) from lanes 4 abid + i
 * when CBSZ = 4 broadcasts block abid's A to all blocks, and its B columns
 * from its own lanes 4b + j, leaving D[i][j] in lane 4b + j, register i. So
 * lane l owns weight row l of the wave's 64 and holds that row's results for
 * all four tokens. A 128-column step is 32 chunks of 4 columns; chunk t's
 * activations live in lanes 4 (t % 16) + i, register t / 16, and the MFMA of
 * chunk t names abid = t % 16: a lane holds 8 registers of activations a step.
 *
 * Arithmetic. Quants enter the MFMA as exact integers in bf16:
 *   Q4_K and Q6_K: 128 + q, the byte q under the exponent of 2^7 (0x43 in
 *     the high byte), two v_perm_b32 for four weights;
 *   Q8_0: q + 128 as an unsigned byte, converted.
 * Activations enter as bf16 hi + lo (x = hi + lo to about 2^-16 relative), so
 * each product is exact and the MFMA sums in fp32. Per block, in fp32:
 *   Q4_K (group of 32, w = d1 q - m1): d1 P - (m1 + 128 d1) S
 *   Q6_K (run of 16, w = ds (q6 - 32)): ds (P - 160 S)
 *   Q8_0 (block of 32, w = d q):        d (P - 128 S)
 * with P the MFMA sum of the offset quants times x and S the sum of x over
 * the block's columns (hi + lo, precomputed by whoever split the activations,
 * read by scalar loads). d1, m1 and ds are rounded as the reference widens
 * (engine/src/quant.c:40-188); the offsets cancel to about 2^-20 relative.
 *
 * Layouts. Split activations: rows of K / 4 chunks of 16 bytes, [4 hi bf16]
 * [4 lo bf16]; sums: rows of K / G floats, G = 16 for Q6_K and 32 otherwise.
 * Weights stream through registers one step ahead: a lane takes its own row's
 * 80 (Q4_K), 106 (Q6_K) or 136 (Q8_0) bytes a step, from the tiled copy (below),
 * where a wave's loads are contiguous.
 */

#include "vitna_kernels.h"
#include "gmma_split.h"

#include <type_traits>
#include <utility>

typedef short gm_bf4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int gm_int4 __attribute__((ext_vector_type(4)));

#define GM_TT 4 /* tokens a tile */

/* chunk t's product: A from block abid = t % 16 (activation register pair a), B the lane's four weights b */
template <int ABID>
__device__ __forceinline__ f32x4 mma4(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(gm_bf4, a), __builtin_bit_cast(gm_bf4, b), c, 4, ABID, 0);
}

/* f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>) */
template <typename F, int... T>
__device__ __forceinline__ void sfor_(F&& f, std::integer_sequence<int, T...>) {
    (f(std::integral_constant<int, T>()), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor(F&& f) {
    sfor_(f, std::make_integer_sequence<int, N>());
}

/* four bytes of v, each below 128, as bf16 128 + byte */
__device__ __forceinline__ u32x2 mag4(uint32_t v) {
    return u32x2{__builtin_amdgcn_perm(0x43434343u, v, 0x04010400u), __builtin_amdgcn_perm(0x43434343u, v, 0x04030402u)};
}
/* four unsigned bytes of v as bf16, converted */
__device__ __forceinline__ u32x2 cvt4(uint32_t v) {
    uint32_t o[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const __bf16 a = (__bf16)(float)((v >> (16 * h)) & 0xffu), b = (__bf16)(float)((v >> (16 * h + 8)) & 0xffu);
        o[h] = (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
    }
    return u32x2{o[0], o[1]};
}

/* Scalar (constant-space) reads: counted by lgkmcnt, uniform across the wave. */
__device__ __forceinline__ int sload(const int* p) { return *(const __attribute__((address_space(4))) int*)p; }
__device__ __forceinline__ gm_int4 sload4(const int* p) { return *(const __attribute__((address_space(4))) gm_int4*)p; }
typedef float gm_f4 __attribute__((ext_vector_type(4)));
typedef float gm_f8 __attribute__((ext_vector_type(8)));
template <int N>
struct svsel;
template <>
struct svsel<4> { typedef gm_f4 t; };
template <>
struct svsel<8> { typedef gm_f8 t; };
template <int N>
using sv = typename svsel<N>::t;
template <int N>
__device__ __forceinline__ sv<N> sloadf(const float* p) {
    return *(const __attribute__((address_space(4))) sv<N>*)p;
}

/* ---- activations, split ------------------------------------------------- */

/* x [n][K] -> xs [n][K/4 chunks of hi4 | lo4], sums [n][K/G]: one thread a run of G columns */
template <int G>
__global__ void gsplit_kernel(const float* __restrict__ x, int K, int xstride, uint16_t* __restrict__ xs, float* __restrict__ sums) {
    const int r = blockIdx.y, g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= K / G) return;
    gsplit_run<G>(x + (size_t)r * xstride, K, g, xs + (size_t)r * 2 * K, sums + (size_t)r * (K / G));
}

/* ---- one 128-column step of a lane's weight row ------------------------- */

template <int DT>
struct gstep;
template <>
struct gstep<VITNA_DTYPE_Q4_K> { /* the half block's 64 quant bytes, the block's header */
    u32x4 q[4];
    u32x4 h;
};
template <>
struct gstep<VITNA_DTYPE_Q6_K> { /* half h of the block: ql bytes 64h .., qh bytes 32h .., scales 8h .., d */
    u32x4 ql[4], qh[2];
    u32x2 sc;
    uint32_t d;
};
template <>
struct gstep<VITNA_DTYPE_Q8_0> { /* blocks 4 st .. 4 st + 3 */
    u32x4 q[8];
    uint32_t d[4];
};

/* ---- the tiled copy of an expert set ------------------------------------- */
/*
 * Per expert, per group of 64 rows (a wave's rows, lane l = row 64 g + l) and unit (Q4_K, Q6_K: a 256-column
 * block; Q8_0: a 128-column step), the bytes a lane's step loads, in 16-byte pieces in lane order, so that each
 * load of a wave is 1 KB contiguous (512 or 128 bytes for the small fields):
 *   Q4_K (9216): q half 0 [4][64] x 16, q half 1 [4][64] x 16, header [64] x 16
 *   Q6_K (13440): ql half 0, ql half 1 [4][64] x 16, qh half 0, half 1 [2][64] x 16, scales [2][64] x 8, d [64] x 2
 *   Q8_0 (8704): q [8][64] x 16 (the four blocks' 128 bytes), d [64] x 8
 * Experts back to back, gmma_tile_stride bytes apart.
 */
__host__ __device__ static inline size_t gmma_unit_bytes(int dtype) {
    return dtype == VITNA_DTYPE_Q4_K ? 9216 : dtype == VITNA_DTYPE_Q6_K ? 13440 : dtype == VITNA_DTYPE_Q8_0 ? 8704 : 0;
}
__host__ __device__ static inline size_t gmma_units(int dtype, int cols) { return dtype == VITNA_DTYPE_Q8_0 ? cols / 128 : cols / 256; }
__host__ __device__ static inline size_t gmma_tile_stride(const qmat& m) {
    return (size_t)(m.rows / 64) * gmma_units(m.dtype, m.cols) * gmma_unit_bytes(m.dtype);
}

/* the byte of expert e's planes that byte o of (group g, unit u) copies */
__device__ static uint32_t gtile_src(const qmat& m, int e, int g, int u, int o) {
    const uint8_t* P0 = m.p[0] + e * m.estride[0];
    const uint8_t* P1 = m.p[1] + e * m.estride[1];
    if (m.dtype == VITNA_DTYPE_Q4_K) {
        if (o < 8192) {
            const int half = o >> 12, i = (o >> 10) & 3, lane = (o >> 4) & 63, j = o & 15;
            return P0[((size_t)(64 * g + lane) * m.nb + u) * 128 + 64 * half + 16 * i + j];
        }
        const int lane = (o - 8192) >> 4, j = o & 15;
        return P1[((size_t)(64 * g + lane) * m.nb + u) * 16 + j];
    } else if (m.dtype == VITNA_DTYPE_Q6_K) {
        if (o < 8192) {
            const int h = o >> 12, i = (o >> 10) & 3, lane = (o >> 4) & 63, j = o & 15;
            return P0[((size_t)(64 * g + lane) * m.nb + u) * 128 + 64 * h + 16 * i + j];
        }
        if (o < 12288) {
            const int q = o - 8192, h = q >> 11, i = (q >> 10) & 1, lane = (q >> 4) & 63, j = q & 15;
            return P1[((size_t)(64 * g + lane) * m.nb + u) * 64 + 32 * h + 16 * i + j];
        }
        if (o < 13312) {
            const int q = o - 12288, h = q >> 9, lane = (q >> 3) & 63, j = q & 7;
            return (m.p[2] + e * m.estride[2])[((size_t)(64 * g + lane) * m.nb + u) * 16 + 8 * h + j];
        }
        const int q = o - 13312, lane = q >> 1, j = q & 1;
        return (m.p[3] + e * m.estride[3])[((size_t)(64 * g + lane) * m.nb + u) * 2 + j];
    } else {
        if (o < 8192) {
            const int i = o >> 10, lane = (o >> 4) & 63, j = o & 15;
            return P0[((size_t)(64 * g + lane) * m.nb + 4 * u) * 32 + 16 * i + j];
        }
        const int q = o - 8192, lane = q >> 3, b = (q & 7) >> 1, j = q & 1;
        return P1[((size_t)(64 * g + lane) * m.nb + 4 * u + b) * 2 + j];
    }
}

/* One block a (expert, group, unit), a thread a byte: made once, at upload. */
__global__ void gtile_kernel(qmat m, int groups, int units, uint8_t* __restrict__ dst) {
    const int u = blockIdx.x % units, g = (blockIdx.x / units) % groups, e = blockIdx.x / (units * groups);
    const int ub = (int)gmma_unit_bytes(m.dtype);
    uint8_t* out = dst + (size_t)blockIdx.x * ub;
    for (int o = threadIdx.x; o < ub; o += blockDim.x) out[o] = (uint8_t)gtile_src(m, e, g, u, o);
}

size_t gmma_tiled_bytes(const qmat& m, int n_experts) { return gmma_tile_stride(m) * n_experts; }

hipError_t launch_gmma_tile(const qmat& m, int n_experts, uint8_t* dst, hipStream_t s) {
    if (!gmma_unit_bytes(m.dtype) || m.rows % 64 || m.cols % 256 || n_experts < 1) return hipErrorInvalidValue;
    const int groups = m.rows / 64, units = (int)gmma_units(m.dtype, m.cols);
    gtile_kernel<<<n_experts * groups * units, 256, 0, s>>>(m, groups, units, dst);
    return hipGetLastError();
}

/* A lane's step from the tiled copy: every load of the wave 1 KB (or 512 / 128 bytes) contiguous. */
template <int DT>
__device__ __forceinline__ void gload(const qmat& m, int e, int row, int st, gstep<DT>& s) {
    const int g = row >> 6, lane = row & 63;
    const uint8_t* E = m.tiled + (size_t)e * gmma_tile_stride(m);
    if constexpr (DT == VITNA_DTYPE_Q4_K) {
        const uint8_t* T = E + ((size_t)g * (m.cols / 256) + (st >> 1)) * 9216;
#pragma unroll
        for (int i = 0; i < 4; i++) s.q[i] = *reinterpret_cast<const u32x4*>(T + (st & 1) * 4096 + i * 1024 + lane * 16);
        s.h = *reinterpret_cast<const u32x4*>(T + 8192 + lane * 16);
    } else if constexpr (DT == VITNA_DTYPE_Q6_K) {
        const uint8_t* T = E + ((size_t)g * (m.cols / 256) + (st >> 1)) * 13440;
        const int h = st & 1;
#pragma unroll
        for (int i = 0; i < 4; i++) s.ql[i] = *reinterpret_cast<const u32x4*>(T + h * 4096 + i * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < 2; i++) s.qh[i] = *reinterpret_cast<const u32x4*>(T + 8192 + h * 2048 + i * 1024 + lane * 16);
        s.sc = *reinterpret_cast<const u32x2*>(T + 12288 + h * 512 + lane * 8);
        s.d = *reinterpret_cast<const uint16_t*>(T + 13312 + lane * 2);
    } else {
        const uint8_t* T = E + ((size_t)g * (m.cols / 128) + st) * 8704;
#pragma unroll
        for (int i = 0; i < 8; i++) s.q[i] = *reinterpret_cast<const u32x4*>(T + i * 1024 + lane * 16);
        const u32x2 d = *reinterpret_cast<const u32x2*>(T + 8192 + lane * 8);
        s.d[0] = d.x & 0xffffu; s.d[1] = d.x >> 16; s.d[2] = d.y & 0xffffu; s.d[3] = d.y >> 16;
    }
}

template <int DT>
struct ggran {
    static constexpr int g = DT == VITNA_DTYPE_Q6_K ? 16 : 32; /* columns a scale */
    static constexpr int per = 128 / g;                        /* scale blocks a step */
};

/* Chunk T's four weights of matrix k of the step, as the MFMA's B operand. */
template <int DT, int T>
__device__ __forceinline__ u32x2 gweights(const gstep<DT>& s) {
    constexpr int G = ggran<DT>::g, B = T / (G / 4); /* scale block of the chunk */
    if constexpr (DT == VITNA_DTYPE_Q4_K) {
        /* group B of the step: pair B / 2, nibble B & 1; dword 8 (B / 2) + T % 8 */
        constexpr int dw = 8 * (B >> 1) + (T & 7);
        const uint32_t q = s.q[dw >> 2][dw & 3];
        return mag4((B & 1) ? (q >> 4) & 0x0f0f0f0fu : q & 0x0f0f0f0fu);
    } else if constexpr (DT == VITNA_DTYPE_Q6_K) {
        /* run B of the step: r = B / 2, l16 = B % 2; ql dword 8 (r & 1) + 4 l16 + T % 4, qh 4 l16 + T % 4 */
        constexpr int r = B >> 1, l16 = B & 1, qld = 8 * (r & 1) + 4 * l16 + (T & 3), qhd = 4 * l16 + (T & 3);
        const uint32_t ql = s.ql[qld >> 2][qld & 3] >> (4 * (r >> 1));
        const uint32_t qh = s.qh[qhd >> 2][qhd & 3];
        uint32_t hi;
        if constexpr (r < 2) hi = qh << (4 - 2 * r);
        else hi = qh >> (2 * r - 4);
        return mag4((ql & 0x0f0f0f0fu) | (hi & 0x30303030u));
    } else {
        constexpr int dw = 8 * B + (T & 7);
        return cvt4(s.q[dw >> 2][dw & 3] ^ 0x80808080u);
    }
}

/* Step st (HALF = st & 1) of NM matrices: av the lane's activation registers (chunks lane / 4 and 16 + lane / 4
   of its token lane % 4), S[i][b] the sum of token i over the step's scale block b. Every scale block of every
   matrix keeps its own MFMA sum through the step, so a chunk's MFMAs (block by block, hi parts then lo parts)
   never wait on one another. */
template <int DT, int NM, int HALF>
__device__ __forceinline__ void gcompute(const gstep<DT> s[NM], const u32x4 av[2], const sv<ggran<DT>::per> S[GM_TT],
                                         f32x4 acc[NM]) {
    constexpr int PER = ggran<DT>::per, CPB = ggran<DT>::g / 4; /* scale blocks a step, chunks a block */
    /* Scale blocks a pass: Q4_K takes its four at once; Q6_K (eight blocks of 16 columns) and Q8_0 (whose step holds
       36 registers of quants a matrix) take two at a time, which keeps their sums and weights within the register
       file (all at once they spilled 632 and 268 bytes a lane). The sums, and the order they are folded into acc,
       are the same either way. */
    constexpr int BP = DT == VITNA_DTYPE_Q4_K ? PER : 2;
    sfor<PER / BP>([&](auto gi) {
        constexpr int B0 = decltype(gi)::value * BP;
        f32x4 P[BP][NM];
#pragma unroll
        for (int b = 0; b < BP; b++)
#pragma unroll
            for (int k = 0; k < NM; k++) P[b][k] = f32x4{0.f, 0.f, 0.f, 0.f};
        sfor<CPB>([&](auto ui) {
            constexpr int U = decltype(ui)::value;
            u32x2 w[BP][NM];
            sfor<BP>([&](auto bi) {
                constexpr int B = B0 + decltype(bi)::value;
#pragma unroll
                for (int k = 0; k < NM; k++) w[B - B0][k] = gweights<DT, B * CPB + U>(s[k]);
            });
            sfor<BP>([&](auto bi) {
                constexpr int B = B0 + decltype(bi)::value, T = B * CPB + U;
                const u32x4 a = av[T >> 4];
#pragma unroll
                for (int k = 0; k < NM; k++) P[B - B0][k] = mma4<T & 15>(u32x2{a.x, a.y}, w[B - B0][k], P[B - B0][k]);
            });
            sfor<BP>([&](auto bi) {
                constexpr int B = B0 + decltype(bi)::value, T = B * CPB + U;
                const u32x4 a = av[T >> 4];
#pragma unroll
                for (int k = 0; k < NM; k++) P[B - B0][k] = mma4<T & 15>(u32x2{a.z, a.w}, w[B - B0][k], P[B - B0][k]);
            });
        });
        sfor<BP>([&](auto bi) {
            constexpr int B = B0 + decltype(bi)::value;
#pragma unroll
            for (int k = 0; k < NM; k++) {
                if constexpr (DT == VITNA_DTYPE_Q4_K) {
                    constexpr int g = 4 * HALF + B; /* group of the block */
                    const uint32_t h0 = s[k].h.x, s03 = s[k].h.y, s47 = s[k].h.z, s8b = s[k].h.w;
                    uint32_t sc, mn;
                    if constexpr (g < 4) {
                        sc = (s03 >> (8 * g)) & 63;
                        mn = (s47 >> (8 * g)) & 63;
                    } else {
                        constexpr int j = g - 4;
                        sc = ((s8b >> (8 * j)) & 15) | (((s03 >> (8 * j + 6)) & 3) << 4);
                        mn = ((s8b >> (8 * j + 4)) & 15) | (((s47 >> (8 * j + 6)) & 3) << 4);
                    }
                    const float d1 = f16_bits_to_f32(h0 & 0xffffu) * (float)sc;
                    const float m1 = f16_bits_to_f32(h0 >> 16) * (float)mn;
                    const float mp = m1 + 128.0f * d1;
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[k][i] = fmaf(-mp, S[i][B], fmaf(d1, P[B - B0][k][i], acc[k][i]));
                } else if constexpr (DT == VITNA_DTYPE_Q6_K) {
                    const uint32_t scw = B < 4 ? s[k].sc.x : s[k].sc.y;
                    const float ds = f16_bits_to_f32(s[k].d & 0xffffu) * (float)(int8_t)((scw >> (8 * (B & 3))) & 0xff);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[k][i] = fmaf(ds, fmaf(-160.0f, S[i][B], P[B - B0][k][i]), acc[k][i]);
                } else {
                    const float d = f16_bits_to_f32(s[k].d[B] & 0xffffu);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[k][i] = fmaf(d, fmaf(-128.0f, S[i][B], P[B - B0][k][i]), acc[k][i]);
                }
            }
        });
    });
}

/* One token tile: the lane's weight row (row) of NM matrices over steps s0 .. s1 - 1 (128 columns each) against
   tokens whose split activation rows start at arow (this lane's token, lane % 4) and whose sums rows start at
   srow[i], into acc. */
template <int DT, int NM>
__device__ __forceinline__ void grows(const qmat& m0, const qmat& m1, int e, int row, int s0, int s1, const u32x4* arow,
                                      const float* const srow[GM_TT], int lane, f32x4 acc[NM]) {
    constexpr int PER = ggran<DT>::per;
    const int c16 = lane >> 2;
    gstep<DT> b0[NM], b1[NM];
    u32x4 a0[2], a1[2];
    sv<PER> s0v[GM_TT], s1v[GM_TT];
    auto load = [&](int st, gstep<DT>* b, u32x4* av, sv<PER>* S) {
        gload<DT>(m0, e, row, st, b[0]);
        if constexpr (NM == 2) gload<DT>(m1, e, row, st, b[1]);
        av[0] = arow[32 * st + c16];
        av[1] = arow[32 * st + 16 + c16];
#pragma unroll
        for (int i = 0; i < GM_TT; i++) S[i] = sloadf<PER>(srow[i] + PER * st);
        /* the loads stay where they are, a step ahead of their use (the scheduler would otherwise sink them to
           their first use to save registers, leaving nothing in flight) */
        __builtin_amdgcn_sched_barrier(0);
    };
    /* steps in pairs from an even step (half 0, half 1 of a block); a range starting odd or ending early takes
       its lone step separately */
    int st = s0;
    if ((st & 1) && st < s1) {
        load(st, b1, a1, s1v);
        gcompute<DT, NM, 1>(b1, a1, s1v, acc);
        st++;
    }
    if (st + 1 < s1) {
        load(st, b0, a0, s0v);
        for (; st + 1 < s1; st += 2) {
            load(st + 1, b1, a1, s1v);
            gcompute<DT, NM, 0>(b0, a0, s0v, acc);
            if (st + 2 < s1) load(st + 2, b0, a0, s0v);
            gcompute<DT, NM, 1>(b1, a1, s1v, acc);
        }
    }
    if (st < s1) {
        load(st, b0, a0, s0v);
        gcompute<DT, NM, 0>(b0, a0, s0v, acc);
    }
}

/* The KS waves' sums of one 64-row group, added in wave order through LDS (red: KS x NM x 4 x 64 floats);
   every wave returns with the total in acc. */
template <int NM, int KS>
__device__ __forceinline__ void ksum(f32x4 acc[NM], float* red, int wv, int lane) {
    if constexpr (KS > 1) {
#pragma unroll
        for (int k = 0; k < NM; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[((wv * NM + k) * 4 + i) * 64 + lane] = acc[k][i];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < NM; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = red[(k * 4 + i) * 64 + lane];
                for (int w = 1; w < KS; w++) v += red[((w * NM + k) * 4 + i) * 64 + lane];
                acc[k][i] = v;
            }
        __syncthreads();
    }
}

/* ---- the kernels -------------------------------------------------------- */

/* The tile's pairs, past nt repeating the last. t0 is a multiple of 4 below the expert's capacity, itself a
   multiple of 4, so the four-entry read stays in the expert's list. */
__device__ __forceinline__ gm_int4 tile_pairs(const int* pr, int t0, int nt) {
    gm_int4 pv = sload4(pr + t0);
    pv.y = nt > 1 ? pv.y : pv.x;
    pv.z = nt > 2 ? pv.z : pv.y;
    pv.w = nt > 3 ? pv.w : pv.z;
    return pv;
}
__device__ __forceinline__ int pick(gm_int4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

/* act[row * K + slot][n] = silu(gate_e[n] . xn[row]) * (up_e[n] . xn[row]), written split, with its sums over
   runs of GO rows. A block: KS waves over one group of 64 weight rows of one expert, wave w taking the w-th
   of KS contiguous ranges of the columns; wave 0 writes. Q6_K and Q8_0 steps (27 and 36 registers a matrix, two
   matrices, two steps in flight) do not fit two waves a SIMD: held to that they spilled 548 and 204 bytes a lane
   inside the column loop; at one wave a SIMD the extra values sit in accumulator registers, and a rows step of
   32 sequences (8 layers) went 2.74 → 1.76 ms (Q6_K) and 2.10 → 1.94 ms (Q8_0), Q4_K unchanged. */
template <int DT, int GO, int KS>
__global__ __launch_bounds__(64 * KS, DT == VITNA_DTYPE_Q4_K ? 8 / KS : 1) void gmma_in_kernel(gmma_args a, int wpe, int ts_n) {
    __shared__ float red[KS > 1 ? KS * 2 * 4 * 64 : 1];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int per = a.E * wpe, ts = blockIdx.x / per, eb = blockIdx.x - ts * per;
    const int e = eb / wpe, rw = eb - e * wpe;
    const int c = sload(a.count + e);
    if (c <= ts * GM_TT) return;
    const int I = a.gate.rows, H = a.gate.cols;
    constexpr int GI = ggran<DT>::g;
    const int n = rw * 64 + lane;
    const int* pr = a.pairs + (size_t)e * a.cap;
    for (int t0 = ts * GM_TT; t0 < c; t0 += ts_n * GM_TT) {
        const int nt = min(GM_TT, c - t0);
        const gm_int4 pv = tile_pairs(pr, t0, nt);
        const u32x4* arow = reinterpret_cast<const u32x4*>(a.xs + (size_t)(pick(pv, lane & 3) / ROUTE_K_MAX) * 2 * H);
        const float* srow[GM_TT];
#pragma unroll
        for (int i = 0; i < GM_TT; i++) srow[i] = a.xsum + (size_t)(pick(pv, i) / ROUTE_K_MAX) * (H / GI);
        f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        const int ns = H / 128;
        grows<DT, 2>(a.gate, a.up, e, n, ns * wv / KS, ns * (wv + 1) / KS, arow, srow, lane, acc);
        ksum<2, KS>(acc, red, wv, lane);
        if (wv != 0) continue;
#pragma unroll
        for (int i = 0; i < GM_TT; i++) {
            if (i >= nt) break;
            const int p = pick(pv, i), pa = (p / ROUTE_K_MAX) * a.K + p % ROUTE_K_MAX;
            const float gv = acc[0][i], uv = acc[1][i];
            const float v = (gv / (1.0f + expf(-gv))) * uv;
            const __bf16 hb = (__bf16)v;
            const __bf16 lb = (__bf16)(v - (float)hb);
            uint16_t* o = a.as + (size_t)pa * 2 * I + 8 * (n >> 2) + (n & 3);
            o[0] = __builtin_bit_cast(uint16_t, hb);
            o[4] = __builtin_bit_cast(uint16_t, lb);
            const float sm = row_sum<GO>((float)hb + (float)lb);
            if ((lane & (GO - 1)) == GO - 1) a.asum[(size_t)pa * (I / GO) + n / GO] = sm;
        }
    }
}

/* ypart[row * K + slot][n] = w_slot * (down_e[n] . act[row * K + slot]) */
template <int DT, int KS>
__global__ __launch_bounds__(64 * KS, 8 / KS) void gmma_down_kernel(gmma_args a, int wpe, int ts_n) {
    __shared__ float red[KS > 1 ? KS * 1 * 4 * 64 : 1];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int per = a.E * wpe, ts = blockIdx.x / per, eb = blockIdx.x - ts * per;
    const int e = eb / wpe, rw = eb - e * wpe;
    const int c = sload(a.count + e);
    if (c <= ts * GM_TT) return;
    const int H = a.down.rows, I = a.down.cols;
    constexpr int GI = ggran<DT>::g;
    const int n = rw * 64 + lane;
    const int* pr = a.pairs + (size_t)e * a.cap;
    for (int t0 = ts * GM_TT; t0 < c; t0 += ts_n * GM_TT) {
        const int nt = min(GM_TT, c - t0);
        const gm_int4 pv = tile_pairs(pr, t0, nt);
        const int pl = pick(pv, lane & 3);
        const u32x4* arow = reinterpret_cast<const u32x4*>(a.as + (size_t)((pl / ROUTE_K_MAX) * a.K + pl % ROUTE_K_MAX) * 2 * I);
        const float* srow[GM_TT];
#pragma unroll
        for (int i = 0; i < GM_TT; i++) {
            const int p = pick(pv, i);
            srow[i] = a.asum + (size_t)((p / ROUTE_K_MAX) * a.K + p % ROUTE_K_MAX) * (I / GI);
        }
        f32x4 acc[1] = {{0.f, 0.f, 0.f, 0.f}};
        const int ns = I / 128;
        grows<DT, 1>(a.down, a.down, e, n, ns * wv / KS, ns * (wv + 1) / KS, arow, srow, lane, acc);
        ksum<1, KS>(acc, red, wv, lane);
        if (wv != 0) continue;
#pragma unroll
        for (int i = 0; i < GM_TT; i++) {
            if (i >= nt) break;
            const int p = pick(pv, i), row = p / ROUTE_K_MAX, slot = p % ROUTE_K_MAX;
            a.ypart[(size_t)(row * a.K + slot) * H + n] = a.rt[row].weights[slot] * acc[0][i];
        }
    }
}

/* ---- launches ------------------------------------------------------------ */

/* The most blocks an (expert, row group)'s tiles are spread over. The block index steps by experts x row groups
   from one share to the next (1536 at Qwen3's shape, a multiple of eight), so there every share of an (expert,
   row group) runs on the same XCD and reads its weights through the same L2. A prompt pass of 1024 rows (16 tiles an expert on average) took 472 ms a 4096-token prompt
   with at most 4 shares and 416 with 16 (32, or twice the average, measured the same). */
#define GM_TS_MAX 16
#define GIN_KS 4 /* gate/up: 2048 columns, four ranges of 512 */
#define GDN_KS 3 /* down: 768 columns, three ranges of 256 */

static bool gm_dtype(int d) { return d == VITNA_DTYPE_Q8_0 || d == VITNA_DTYPE_Q4_K || d == VITNA_DTYPE_Q6_K; }

bool gmma_fits(const qmat& gate, const qmat& up, const qmat& down) {
    /* whole 128-column steps in pairs, whole 64-row waves */
    return gm_dtype(gate.dtype) && up.dtype == gate.dtype && gm_dtype(down.dtype) && gate.cols % 256 == 0 &&
           down.cols % 256 == 0 && gate.rows % 64 == 0 && down.rows % 64 == 0 && up.rows == gate.rows &&
           up.cols == gate.cols && down.cols == gate.rows && down.rows == gate.cols;
}

int gmma_gran(int dtype) { return dtype == VITNA_DTYPE_Q6_K ? 16 : 32; }

hipError_t launch_gmma_split(const float* x, int n, int K, int xstride, int gran, uint16_t* xs, float* sums, hipStream_t s) {
    if (n < 1 || K < 1 || K % gran || (gran != 16 && gran != 32)) return hipErrorInvalidValue;
    const dim3 grid((K / gran + 63) / 64, n);
    if (gran == 32) gsplit_kernel<32><<<grid, 64, 0, s>>>(x, K, xstride, xs, sums);
    else gsplit_kernel<16><<<grid, 64, 0, s>>>(x, K, xstride, xs, sums);
    return hipGetLastError();
}

/* Blocks a (expert, row group): the expert's token tiles t, t + ts, ... go to block t of ts, so that an expert
   with more tiles than the average runs them side by side instead of one after another. Blocks past an expert's
   tiles return at once; they are dispatched after every first tile. Measured on 32 rows of top-8 over 128
   experts: gate/up gains from splitting even at two pairs an expert on average (its stragglers of five to eight
   pairs), down only when the experts are crowded (at two pairs an expert its extra blocks cost more). */
static int gmma_tile_split(const gmma_args& a, bool down) {
    const int pairs = a.n * a.K, tiles = (pairs + a.E * GM_TT - 1) / (a.E * GM_TT); /* tiles an expert on average */
    if (a.n <= GM_TT) return 1;
    if (down) return tiles <= 1 ? 1 : tiles < GM_TS_MAX ? tiles : GM_TS_MAX;
    return tiles <= 1 ? 2 : tiles < 4 ? 4 : tiles < GM_TS_MAX ? tiles : GM_TS_MAX;
}

hipError_t launch_gmma_in(const gmma_args& a, hipStream_t s) {
    if (!gmma_fits(a.gate, a.up, a.down) || !a.gate.tiled || !a.up.tiled || a.K < 1 || a.K > ROUTE_K_MAX || a.cap % 4 || a.n < 1)
        return hipErrorInvalidValue;
    /* KS waves split each row group's columns: enough waves to fill the SIMDs */
    const int wpe = a.gate.rows / 64, ts = gmma_tile_split(a, false), blocks = a.E * wpe * ts;
    const bool g16 = gmma_gran(a.down.dtype) == 16;
#define GI(D)                                                                                      \
    case D:                                                                                        \
        if (g16) gmma_in_kernel<D, 16, GIN_KS><<<blocks, 64 * GIN_KS, 0, s>>>(a, wpe, ts);             \
        else gmma_in_kernel<D, 32, GIN_KS><<<blocks, 64 * GIN_KS, 0, s>>>(a, wpe, ts);                 \
        return hipGetLastError();
    switch (a.gate.dtype) { GI(VITNA_DTYPE_Q4_K) GI(VITNA_DTYPE_Q6_K) GI(VITNA_DTYPE_Q8_0) }
#undef GI
    return hipErrorInvalidValue;
}

hipError_t launch_gmma_down(const gmma_args& a, hipStream_t s) {
    if (!gmma_fits(a.gate, a.up, a.down) || !a.down.tiled || a.K < 1 || a.K > ROUTE_K_MAX || a.cap % 4 || a.n < 1)
        return hipErrorInvalidValue;
    const int wpe = a.down.rows / 64, ts = gmma_tile_split(a, true), blocks = a.E * wpe * ts;
    switch (a.down.dtype) {
    case VITNA_DTYPE_Q4_K: gmma_down_kernel<VITNA_DTYPE_Q4_K, GDN_KS><<<blocks, 64 * GDN_KS, 0, s>>>(a, wpe, ts); return hipGetLastError();
    case VITNA_DTYPE_Q6_K: gmma_down_kernel<VITNA_DTYPE_Q6_K, GDN_KS><<<blocks, 64 * GDN_KS, 0, s>>>(a, wpe, ts); return hipGetLastError();
    case VITNA_DTYPE_Q8_0: gmma_down_kernel<VITNA_DTYPE_Q8_0, GDN_KS><<<blocks, 64 * GDN_KS, 0, s>>>(a, wpe, ts); return hipGetLastError();
    }
    return hipErrorInvalidValue;
}
