/**
 * kernels_prefill.hip - A prefill through one mixture-of-experts layer on
 * gfx950: n token rows are normalized, routed and run through their experts
 * as a grouped GEMM on the bf16 matrix cores.
 *
 * Reference counterparts (engine/src/model_cuda.cu): the counting sort of
 * (row, expert) pairs :5151-5176, tc_experts_gu_kernel :2288,
 * tc_experts_down_kernel :2321, experts_reduce_kernel :2343; the arithmetic
 * they approximate is the CPU's (engine/src/model.c:723-764).
 *
 * Routing is exact: RMSNorm and the router follow the reference CPU's
 * sixteen-chain order (engine/src/kernels.c:115-146, ops.c:212-229), so every
 * row chooses the experts the CPU chooses, with the same weights.
 *
 * The experts: each Q8_0 weight q * d (exact in fp32) is rounded to bf16 once a
 * workgroup (by the one wave that uses it, in registers, or into a bf16 stage in
 * LDS in the two-phase kernel); the normed rows and the SwiGLU output are rounded
 * to bf16 too; products accumulate in fp32 on the matrix cores.
 *
 * Pipeline, one stream:
 *   prefill_norm_router_kernel  exact RMSNorm and router logits in one pass (hidden up to 2048; wider rows
 *                               take prefill_norm_kernel, then prefill_router_kernel); bf16 rows for the GEMM
 *   topk_kernel                 the routing rule on every row (kernels_decode.hip)
 *   group_kernel                (row, slot) pairs of each expert in row order (kernels_rows.hip)
 *   prefill_plan_kernel         pair offsets of each expert; the list of 256-pair tiles
 *   prefill_wgemm_kernel<1>     act = silu(X_e G_e^T) * (X_e U_e^T), bf16, pairs in expert order
 *   prefill_wgemm_kernel<0>     ypart[row * K + slot] = w * (act_e D_e^T), bf16
 *   prefill_sum_kernel          x += the K parts of a row in slot order, summed in fp32
 *
 * The per-wave GEMM (prefill_wgemm_kernel, below) reads the experts' tiled copy; an expert set without it, or
 * with widths that are not multiples of 256, takes the two-phase prefill_gemm_kernel: a 512-thread workgroup
 * owns 256 pairs x 256 weight rows (for gate/up: 128 gate rows and the 128 up rows of the same columns, so
 * SwiGLU is local to a lane), each wave 64 x 128 as 2 x 4 tiles of v_mfma_f32_32x32x16_bf16, K advancing 64 a
 * stage (two Q8_0 blocks), the activations through a three-stage LDS ring filled by global-to-LDS loads two
 * stages ahead; waves 0-3 run their MFMAs while waves 4-7 dequantize and load, then the other way round. In
 * both, work items (tile, column block) are split into eight contiguous ranges, one per XCD (workgroup i runs
 * on XCD i mod 8), so the column blocks of one tile and the tiles of one expert share an L2.
 */

#include "vitna_kernels.h"

#include <algorithm>
#include <type_traits>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define PF_BM 256 /* pairs a tile */
#define PF_BN 256 /* weight rows a workgroup */
#define PF_THREADS 512
#define PF_BK 64  /* contraction a stage: two Q8_0 blocks */

/* The SwiGLU of the prefill GEMM, rounded to bf16 right after: silu(g) u with a hardware reciprocal (1 ulp),
   which the bf16 rounding dwarfs. Both GEMM kernels use this one form, so they give the same bits. */
__device__ __forceinline__ float pf_swiglu(float g, float u) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u; }

__device__ __forceinline__ uint32_t bf16_rne(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

/* ---- exact RMSNorm of every row --------------------------------------- */

/* One wave a row: the sum of squares in sixteen chains (kernels.c:115-140),
   the AVX2 fold, 1 / sqrtf(ss / H + eps), y = (x * inv) * w. Writes the fp32
   row and its bf16 rounding. */
__global__ __launch_bounds__(64) void prefill_norm_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ xn,
                                                          uint16_t* __restrict__ xb, int H, float eps) {
    extern __shared__ float sx[];
    __shared__ float inv_s;
    const int lane = threadIdx.x;
    const size_t r = blockIdx.x;
    const float4* x4 = reinterpret_cast<const float4*>(x + r * H);
    for (int i = lane; i < H / 4; i += 64) reinterpret_cast<float4*>(sx)[i] = x4[i];
    __syncthreads();
    if (lane < 16) {
        float acc = 0.0f;
        for (int m = 0; m < H / 16; m++) acc = fmaf(sx[16 * m + lane], sx[16 * m + lane], acc);
        const float ss = fold16_lanes(acc);
        if (lane == 0) inv_s = 1.0f / sqrtf(ss / (float)H + eps);
    }
    __syncthreads();
    const float inv = inv_s;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    for (int i = lane; i < H / 4; i += 64) {
        const float4 v = reinterpret_cast<const float4*>(sx)[i], nw = w4[i];
        float4 o;
        o.x = (v.x * inv) * nw.x; o.y = (v.y * inv) * nw.y;
        o.z = (v.z * inv) * nw.z; o.w = (v.w * inv) * nw.w;
        reinterpret_cast<float4*>(xn + r * H)[i] = o;
        if (!xb) continue;
        uint2 b;
        b.x = bf16_rne(o.x) | (bf16_rne(o.y) << 16);
        b.y = bf16_rne(o.z) | (bf16_rne(o.w) << 16);
        reinterpret_cast<uint2*>(xb + r * H)[i] = b;
    }
}

/* Column steps the routers unroll: the fused norm and router (two blocks a CU by LDS, two waves a SIMD) waits on
   its router loads, and eight steps in flight took it 73 -> 61 us at config 4; the plain router (many blocks, two
   experts a group) measured best at two. The same FMAs in the same order either way. */

/* ---- exact router logits of every row --------------------------------- */

/* logits[t][e] = router[e] . xn[t] in the AVX2 order: sixteen FMA chains
   (chain j: elements 16m + j, m ascending) and the fold. A 16-lane group
   holds the chains of RT rows x RE experts; a workgroup's 16 groups cover
   16 * RE experts. */
template <int RT, int RE>
__global__ __launch_bounds__(256) void prefill_router_kernel(const float* __restrict__ xn, const float* __restrict__ R, float* __restrict__ logits,
                                                            int n, int E, int H) {
    const int j = threadIdx.x & 15, grp = threadIdx.x >> 4;
    const int e0 = (blockIdx.x * 16 + grp) * RE, t0 = blockIdx.y * RT;
    if (e0 >= E) return; /* whole groups only: the fold stays within a group */
    const float* rp[RE];
    const float* xp[RT];
#pragma unroll
    for (int i = 0; i < RE; i++) rp[i] = R + (size_t)min(e0 + i, E - 1) * H + j;
#pragma unroll
    for (int t = 0; t < RT; t++) xp[t] = xn + (size_t)min(t0 + t, n - 1) * H + j;
    float acc[RE][RT];
#pragma unroll
    for (int i = 0; i < RE; i++)
#pragma unroll
        for (int t = 0; t < RT; t++) acc[i][t] = 0.0f;
    const int M = H / 16;
#pragma unroll 2
    for (int m = 0; m < M; m++) {
        float rv[RE], xv[RT];
#pragma unroll
        for (int i = 0; i < RE; i++) rv[i] = rp[i][16 * m];
#pragma unroll
        for (int t = 0; t < RT; t++) xv[t] = xp[t][16 * m];
#pragma unroll
        for (int i = 0; i < RE; i++)
#pragma unroll
            for (int t = 0; t < RT; t++) acc[i][t] = fmaf(rv[i], xv[t], acc[i][t]);
    }
#pragma unroll
    for (int i = 0; i < RE; i++)
#pragma unroll
        for (int t = 0; t < RT; t++) {
            const float v = fold16_lanes(acc[i][t]);
            if (j == 0 && e0 + i < E && t0 + t < n) logits[(size_t)(t0 + t) * E + e0 + i] = v;
        }
}

/* The norm and the router in one pass, for rows of up to NR_HMAX columns: a workgroup's RT rows are loaded into
   LDS once, normalized there exactly as prefill_norm_kernel does (sixteen lanes a row for the sum of squares),
   written out in bf16 for the GEMM, and read by the router's chains from LDS, so that the fp32 normalized rows
   never go to memory. The same arithmetic as the two kernels, so the same bits. */
#define NR_HMAX 2048
template <int RT, int RE>
__global__ __launch_bounds__(256) void prefill_norm_router_kernel(const float* __restrict__ x, const float* __restrict__ nw,
                                                                 const float* __restrict__ R, float* __restrict__ logits,
                                                                 uint16_t* __restrict__ xb, int n, int E, int H, float eps) {
    __shared__ __attribute__((aligned(16))) float sxn[RT * NR_HMAX];
    __shared__ float inv_s[RT];
    const int tid = threadIdx.x, j = tid & 15, grp = tid >> 4;
    const int t0 = blockIdx.y * RT, H4 = H / 4;
    for (int i = tid; i < RT * H4; i += 256) {
        const int t = i / H4, c = i - t * H4;
        reinterpret_cast<float4*>(sxn + t * H)[c] = reinterpret_cast<const float4*>(x + (size_t)min(t0 + t, n - 1) * H)[c];
    }
    __syncthreads();
    if (grp < RT) {
        /* engine/src/kernels.c:115-146: sixteen chains of squares, the fold, 1 / sqrtf(ss / n + eps) */
        const float* sr = sxn + grp * H;
        float acc = 0.0f;
        for (int m = 0; m < H / 16; m++) acc = fmaf(sr[16 * m + j], sr[16 * m + j], acc);
        const float ss = fold16_lanes(acc);
        if (j == 0) inv_s[grp] = 1.0f / sqrtf(ss / (float)H + eps);
    }
    __syncthreads();
    const float4* w4 = reinterpret_cast<const float4*>(nw);
    for (int i = tid; i < RT * H4; i += 256) {
        const int t = i / H4, c = i - t * H4;
        const float inv = inv_s[t];
        float4* p = reinterpret_cast<float4*>(sxn + t * H) + c;
        const float4 v = *p, w = w4[c];
        float4 o;
        o.x = (v.x * inv) * w.x; o.y = (v.y * inv) * w.y;
        o.z = (v.z * inv) * w.z; o.w = (v.w * inv) * w.w;
        *p = o;
        if (blockIdx.x == 0 && t0 + t < n) {
            uint2 b;
            b.x = bf16_rne(o.x) | (bf16_rne(o.y) << 16);
            b.y = bf16_rne(o.z) | (bf16_rne(o.w) << 16);
            reinterpret_cast<uint2*>(xb + (size_t)(t0 + t) * H)[c] = b;
        }
    }
    __syncthreads();
    const int e0 = (blockIdx.x * 16 + grp) * RE;
    if (e0 >= E) return; /* whole groups only: the fold stays within a group */
    const float* rp[RE];
#pragma unroll
    for (int i = 0; i < RE; i++) rp[i] = R + (size_t)min(e0 + i, E - 1) * H + j;
    float acc[RE][RT];
#pragma unroll
    for (int i = 0; i < RE; i++)
#pragma unroll
        for (int t = 0; t < RT; t++) acc[i][t] = 0.0f;
    const int M = H / 16;
#pragma unroll 8
    for (int m = 0; m < M; m++) {
        float rv[RE], xv[RT];
#pragma unroll
        for (int i = 0; i < RE; i++) rv[i] = rp[i][16 * m];
#pragma unroll
        for (int t = 0; t < RT; t++) xv[t] = sxn[t * H + 16 * m + j];
#pragma unroll
        for (int i = 0; i < RE; i++)
#pragma unroll
            for (int t = 0; t < RT; t++) acc[i][t] = fmaf(rv[i], xv[t], acc[i][t]);
    }
#pragma unroll
    for (int i = 0; i < RE; i++)
#pragma unroll
        for (int t = 0; t < RT; t++) {
            const float v = fold16_lanes(acc[i][t]);
            if (j == 0 && e0 + i < E && t0 + t < n) logits[(size_t)(t0 + t) * E + e0 + i] = v;
        }
}

/* ---- plan: offsets and tiles ------------------------------------------ */

__global__ __launch_bounds__(256) void prefill_plan_kernel(const int* __restrict__ count, int E, int* __restrict__ off, int* __restrict__ tiles,
                                                          int* __restrict__ n_tiles) {
    __shared__ int s_off[ROUTE_E_MAX], s_toff[ROUTE_E_MAX];
    if (threadIdx.x == 0) {
        int o = 0, t = 0;
        for (int e = 0; e < E; e++) {
            const int c = count[e];
            s_off[e] = o;
            s_toff[e] = t;
            o += c;
            t += (c + PF_BM - 1) / PF_BM;
        }
        *n_tiles = t;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        off[e] = s_off[e];
        const int nt = (count[e] + PF_BM - 1) / PF_BM;
        for (int i = 0; i < nt; i++) tiles[s_toff[e] + i] = (e << 16) | i;
    }
}

/* ---- the grouped GEMM --------------------------------------------------- */

typedef __attribute__((address_space(3))) void* lds_void;
typedef __attribute__((address_space(1))) void* glb_void;

/* LDS of a workgroup (160 KiB, gfx950's limit):
     A ring, 3 stages of 256 rows x 128 B (bf16, K = 64), filled by
       global-to-LDS loads two stages ahead of use;
     B pair, 2 stages of 256 rows x 128 B (bf16), written by the workgroup's
       own threads: each thread loads 32 quants and their scale of the stage
       two ahead into registers, and one stage ahead dequantizes them (q * d in
       fp32, rounded to bf16) into the B stage. Every weight is dequantized
       once a workgroup.
   Rows of both hold 16-byte chunk c at position c ^ ((row >> 1) & 7): the
   fragment reads (sixteen consecutive rows at one chunk) then cover all 64
   banks without conflict. Each thread issues the same seven loads a stage
   (three for B, then four for A), so the vmcnt waits count stages. */
#define PF_A_STAGES 3
#define PF_TILE_BYTES (PF_BM * 128)

__device__ __forceinline__ int chunk_pos(int row, int c) { return c ^ ((row >> 1) & 7); }

/* 16 int8 quants (four dwords) times d, rounded to bf16, as two 16-byte chunks */
__device__ __forceinline__ void dequant16(const u32x4 q, float d, u32x4& lo, u32x4& hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    uint32_t o[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t v = q[w];
        const bf16x2 p0 = {(__bf16)((float)(int8_t)(v & 0xff) * d), (__bf16)((float)(int8_t)((v >> 8) & 0xff) * d)};
        const bf16x2 p1 = {(__bf16)((float)(int8_t)((v >> 16) & 0xff) * d), (__bf16)((float)(int8_t)(v >> 24) * d)};
        o[2 * w] = __builtin_bit_cast(uint32_t, p0);
        o[2 * w + 1] = __builtin_bit_cast(uint32_t, p1);
    }
    lo = u32x4{o[0], o[1], o[2], o[3]};
    hi = u32x4{o[4], o[5], o[6], o[7]};
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 p = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, p);
}

/* One thread's share of a stage's weights in the shared-stage kernel: 32 consecutive weights of one row (the
   32-column group g of the row), loaded from the planes a stage ahead and widened into four 16-byte chunks of
   bf16 (eight weights each, in column order). The widening is the reference's, each weight rounded once more,
   to bf16, at the end (engine/src/quant.c:40-188):
     Q8_0  q * d;
     Q4_K  (d * sc) * q - dmin * mn, the product rounded before the subtraction;
     Q6_K  (d * sc) * q, q = (low | high << 4) - 32, a scale every 16 weights.
   Every thread issues the same number of loads a stage (LOADS), which the stage's wait counts. */
template <int DT>
struct pf_bgroup;

template <>
struct pf_bgroup<VITNA_DTYPE_Q8_0> {
    static constexpr int LOADS = 3;
    u32x4 q0, q1;
    uint32_t d;
    __device__ __forceinline__ void load(const qmat& m, int e, int row, int g) {
        const u32x4* src = reinterpret_cast<const u32x4*>(m.p[0] + (size_t)e * m.estride[0] + ((size_t)row * m.nb + g) * 32);
        q0 = src[0];
        q1 = src[1];
        d = reinterpret_cast<const uint16_t*>(m.p[1] + (size_t)e * m.estride[1])[(size_t)row * m.nb + g];
    }
    __device__ __forceinline__ void widen(u32x4 (&c)[4]) const {
        const float df = f16_bits_to_f32(d);
        dequant16(q0, df, c[0], c[1]);
        dequant16(q1, df, c[2], c[3]);
    }
};

template <>
struct pf_bgroup<VITNA_DTYPE_Q4_K> {
    static constexpr int LOADS = 3;
    u32x4 q0, q1, hd; /* the group's 32 quant bytes (one nibble each), the super-block's header */
    int gi;
    __device__ __forceinline__ void load(const qmat& m, int e, int row, int g) {
        const size_t blk = (size_t)row * m.nb + (g >> 3);
        gi = g & 7;
        const u32x4* src = reinterpret_cast<const u32x4*>(m.p[0] + (size_t)e * m.estride[0] + blk * 128 + 32 * (gi >> 1));
        q0 = src[0];
        q1 = src[1];
        hd = *reinterpret_cast<const u32x4*>(m.p[1] + (size_t)e * m.estride[1] + blk * 16);
    }
    __device__ __forceinline__ void widen(u32x4 (&c)[4]) const {
        /* header: d, dmin (f16), then twelve bytes of 6-bit scales and mins (quant.c:115) */
        const uint32_t s03 = hd[1], s47 = hd[2], s8b = hd[3];
        auto byte = [](uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); };
        int sc, mn;
        if (gi < 4) {
            sc = byte(s03, gi) & 63;
            mn = byte(s47, gi) & 63;
        } else {
            sc = (byte(s8b, gi - 4) & 15) | ((byte(s03, gi - 4) >> 6) << 4);
            mn = (byte(s8b, gi - 4) >> 4) | ((byte(s47, gi - 4) >> 6) << 4);
        }
        const float d1 = f16_bits_to_f32(hd[0] & 0xffffu) * (float)sc, m1 = f16_bits_to_f32(hd[0] >> 16) * (float)mn;
        const int sh = 4 * (gi & 1);
        const uint32_t w[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            uint32_t o[4];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t v = (w[2 * ch + h] >> sh) & 0x0f0f0f0fu;
                float f[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float prod = d1 * (float)((v >> (8 * i)) & 0xffu);
                    f[i] = prod - m1;
                }
                o[2 * h] = pack_bf16(f[0], f[1]);
                o[2 * h + 1] = pack_bf16(f[2], f[3]);
            }
            c[ch] = u32x4{o[0], o[1], o[2], o[3]};
        }
    }
};

template <>
struct pf_bgroup<VITNA_DTYPE_Q6_K> {
    static constexpr int LOADS = 6;
    u32x4 l0, l1, h0, h1; /* the group's 32 low-nibble bytes and 32 high-bit bytes */
    uint32_t sc, d;       /* its two 16-weight scales (int8), the super-block's d (f16) */
    int r;
    __device__ __forceinline__ void load(const qmat& m, int e, int row, int g) {
        const size_t blk = (size_t)row * m.nb + (g >> 3);
        const int gi = g & 7, h = gi >> 2;
        r = gi & 3;
        const u32x4* ql = reinterpret_cast<const u32x4*>(m.p[0] + (size_t)e * m.estride[0] + blk * 128 + 64 * h + 32 * (r & 1));
        const u32x4* qh = reinterpret_cast<const u32x4*>(m.p[1] + (size_t)e * m.estride[1] + blk * 64 + 32 * h);
        l0 = ql[0];
        l1 = ql[1];
        h0 = qh[0];
        h1 = qh[1];
        sc = *reinterpret_cast<const uint16_t*>(m.p[2] + (size_t)e * m.estride[2] + blk * 16 + 8 * h + 2 * r);
        d = reinterpret_cast<const uint16_t*>(m.p[3] + (size_t)e * m.estride[3])[blk];
    }
    __device__ __forceinline__ void widen(u32x4 (&c)[4]) const {
        const float dd = f16_bits_to_f32(d);
        const float ds[2] = {dd * (float)(int8_t)(sc & 0xffu), dd * (float)(int8_t)(sc >> 8)};
        const int sl = 4 * (r >> 1), shh = 2 * r;
        const uint32_t lw[8] = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
        const uint32_t hw[8] = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            const float s = ds[ch >> 1];
            uint32_t o[4];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t lo = (lw[2 * ch + h] >> sl) & 0x0f0f0f0fu, hi = (hw[2 * ch + h] >> shh) & 0x03030303u;
                const uint32_t q = lo | (hi << 4);
                float f[4];
#pragma unroll
                for (int i = 0; i < 4; i++) f[i] = s * (float)((int)((q >> (8 * i)) & 0xffu) - 32);
                o[2 * h] = pack_bf16(f[0], f[1]);
                o[2 * h + 1] = pack_bf16(f[2], f[3]);
            }
            c[ch] = u32x4{o[0], o[1], o[2], o[3]};
        }
    }
};

template <bool GU, int DT>
__global__ __launch_bounds__(PF_THREADS) void prefill_gemm_kernel(prefill_args a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[(PF_A_STAGES + 2) * PF_TILE_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int H = a.gate.cols, I = a.gate.rows;
    const int NT = GU ? I / (PF_BN / 2) : H / PF_BN; /* column blocks a tile */
    const int KD = GU ? H : I;                       /* contraction length */
    const int nwork = *a.n_tiles * NT;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per = (nwork + 7) >> 3;
    const int w = xcd * per + slot;
    if (slot >= per || w >= nwork) return;
    const int tl = a.tiles[w / NT], nt = w - (w / NT) * NT;
    const int e = tl >> 16, m0 = (tl & 0xffff) * PF_BM;
    const int cnt = a.count[e];
    const int pbase = a.off[e];

    /* A: this lane's four 16-byte global-to-LDS loads a stage */
    const uint8_t* asrc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int sl = (wv * 4 + i) * 64 + lane, r = sl >> 3, c = chunk_pos(r, sl & 7);
        const int pa = min(m0 + r, cnt - 1);
        const uint16_t* row = GU ? a.xb + (size_t)(a.pairs[(size_t)e * a.cap + pa] / ROUTE_K_MAX) * H : a.act + (size_t)(pbase + pa) * I;
        asrc[i] = reinterpret_cast<const uint8_t*>(row) + 16 * c;
    }
    /* B: this thread's weight row bn and 32-column half bh of the stage */
    const int bn = tid >> 1, bh = tid & 1;
    const qmat& wmat = GU ? (bn < PF_BN / 2 ? a.gate : a.up) : a.down;
    const int wrow = GU ? nt * (PF_BN / 2) + (bn % (PF_BN / 2)) : nt * PF_BN + bn;

    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    const uint32_t bstage0 = lds0 + PF_A_STAGES * PF_TILE_BYTES;
    auto issue_a = [&](int s) {
        uint8_t* base = lds + (s % PF_A_STAGES) * PF_TILE_BYTES;
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_global_load_lds((glb_void)(asrc[i] + (size_t)s * 128), (lds_void)(base + (wv * 4 + i) * 1024), 16, 0, 0);
    };
    pf_bgroup<DT> bw;
    auto load_b = [&](int s) { bw.load(wmat, e, wrow, 2 * s + bh); };
    /* widen the loaded stage into B stage buffer s & 1: row bn, chunks 4 bh .. 4 bh + 3 */
    auto store_b = [&](int s) {
        u32x4 c[4];
        bw.widen(c);
        const uint32_t rowb = bstage0 + (s & 1) * PF_TILE_BYTES + bn * 128;
#pragma unroll
        for (int j = 0; j < 4; j++)
            asm volatile("ds_write_b128 %0, %1" ::"v"(rowb + (chunk_pos(bn, 4 * bh + j) << 4)), "v"(c[j]) : "memory");
    };

    /* this wave's 64 x 128: A rows wmi * 64 + 32 i + lane % 32; B rows brow[k] (for gate/up: k = 0, 1 gate
       columns, k = 2, 3 the up rows of the same columns); the lane's k-octet kq */
    const int wmi = wv >> 1, wni = wv & 1, l32 = lane & 31, kq = lane >> 5;
    uint32_t aoff[2], boff[4];
#pragma unroll
    for (int i = 0; i < 2; i++) aoff[i] = (wmi * 64 + i * 32 + l32) * 128;
#pragma unroll
    for (int k = 0; k < 4; k++) boff[k] = (GU ? (k >> 1) * (PF_BN / 2) + wni * 64 + (k & 1) * 32 + l32 : wni * 128 + k * 32 + l32) * 128;
    /* (row >> 1) & 7 of every fragment row this lane reads: the rows differ by multiples of 32 */
    const int swz = (l32 >> 1) & 7;
    /* 32-row subtiles past the expert's last pair do no MFMA work */
    const bool live0 = m0 + wmi * 64 < cnt, live1 = m0 + wmi * 64 + 32 < cnt;

    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][k][r] = 0.0f;

    const int S = KD / PF_BK;
    /* prologue: B of stage 0 dequantized, B of stage 1 in registers, A of stages 0 and 1 in flight */
    load_b(0);
    issue_a(0);
    store_b(0);
    if (S > 1) { load_b(1); issue_a(1); }
    /* Two phases a stage, split by a barrier. Waves 0-3 (one on each SIMD) read their fragments and run their
       MFMAs in the first phase while waves 4-7 dequantize their share of the next stage and issue their loads;
       in the second phase the two groups swap. So each SIMD's matrix core works in both phases while the other
       wave uses the VALU and the LDS. */
    const bool first = wv < 4;
    auto mma = [&](int s) {
        if (!live0) return;
        /* Fragment reads are ds_read instructions of our own: the compiler would otherwise wait for every
           global-to-LDS load in flight (vmcnt(0)) before any LDS read. */
        const uint32_t abase = lds0 + (s % PF_A_STAGES) * PF_TILE_BYTES, bbase = bstage0 + (s & 1) * PF_TILE_BYTES;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            u32x4 af[2][2], bf[4][2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int c = 4 * b + 2 * h + kq; /* chunk of k = 32 b + 16 h + 8 kq */
                const uint32_t cp = (uint32_t)((c ^ swz) << 4);
#pragma unroll
                for (int i = 0; i < 2; i++) asm volatile("ds_read_b128 %0, %1" : "=v"(af[i][h]) : "v"(abase + aoff[i] + cp));
#pragma unroll
                for (int k = 0; k < 4; k++) asm volatile("ds_read_b128 %0, %1" : "=v"(bf[k][h]) : "v"(bbase + boff[k] + cp));
            }
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(af[0][0]), "+v"(af[0][1]), "+v"(af[1][0]), "+v"(af[1][1]), "+v"(bf[0][0]), "+v"(bf[0][1]), "+v"(bf[1][0]),
                           "+v"(bf[1][1]), "+v"(bf[2][0]), "+v"(bf[2][1]), "+v"(bf[3][0]), "+v"(bf[3][1]));
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const bf16x8 b0 = __builtin_bit_cast(bf16x8, bf[k][0]), b1 = __builtin_bit_cast(bf16x8, bf[k][1]);
                acc[0][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[0][0]), b0, acc[0][k], 0, 0, 0);
                acc[0][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[0][1]), b1, acc[0][k], 0, 0, 0);
                if (live1) {
                    acc[1][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[1][0]), b0, acc[1][k], 0, 0, 0);
                    acc[1][k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[1][1]), b1, acc[1][k], 0, 0, 0);
                }
            }
        }
    };
    auto feed = [&](int s) {
        if (s + 1 < S) store_b(s + 1);
        if (s + 2 < S) { load_b(s + 2); issue_a(s + 2); }
    };
    for (int s = 0; s < S; s++) {
        /* A of stage s landed (the seven loads of stage s + 1 may be in flight); this thread's B writes done */
        if (s + 1 < S) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(pf_bgroup<DT>::LOADS + 4) : "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (first) mma(s);
        else feed(s);
        __builtin_amdgcn_s_barrier();
        if (first) feed(s);
        else mma(s);
    }

    /* accumulator r of a lane: row 8 (r / 4) + 4 (lane / 32) + r % 4 of the 32 x 32 tile, column lane % 32 */
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int p = m0 + wmi * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (p >= cnt) continue;
            if (GU) {
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const float gt = acc[i][k][r], up = acc[i][k + 2][r];
                    const float v = pf_swiglu(gt, up);
                    a.act[(size_t)(pbase + p) * I + nt * (PF_BN / 2) + wni * 64 + k * 32 + l32] = (uint16_t)bf16_rne(v);
                }
            } else {
                const int pr = a.pairs[(size_t)e * a.cap + p], row = pr / ROUTE_K_MAX, sl = pr % ROUTE_K_MAX;
                const float wt = a.rt[row].weights[sl];
                uint16_t* y = a.ypart + ((size_t)row * a.K + sl) * H + nt * PF_BN + wni * 128 + l32;
#pragma unroll
                for (int k = 0; k < 4; k++) y[32 * k] = (uint16_t)bf16_rne(acc[i][k][r] * wt);
            }
        }
}

/* ---- the grouped GEMM, each wave converting its own weights ------------------------------------------

   A 256-thread workgroup (one wave a SIMD) owns one tile (up to 256 pairs) and 256 weight rows; wave w owns 64 of
   them (gate/up: 32 gate rows and the 32 up rows of the same columns, so SwiGLU stays in a lane; down: 64 rows)
   against every pair of the tile, as ML x 2 tiles of v_mfma_f32_32x32x16_bf16. The waves share only the
   activations, which arrive in an LDS ring (four stages of K = 64, 256 rows x 128 bytes) by global-to-LDS
   loads three stages ahead; one barrier a stage. The weights never pass through LDS: each lane loads the Q8_0
   bytes its own B fragments need, three stages ahead, and widens them itself (q * d exact in fp32, rounded to
   bf16, as before) just before its MFMAs, on the VALU while the matrix core works. Every weight is read and
   widened once a workgroup, by the one wave that uses it.

   A lane (l32, kq) of a 32-row weight tile needs, for K step j (16 columns), row l32's 8 quants at 16 j + 8 kq;
   the experts' tiled copy holds each K step's 16 bytes of 64 rows together, so each weight load of a wave is
   512 contiguous bytes (a wave's loads of the row-major planes, 32 rows 2 KB apart, ran at a fraction of that).

   Loads a stage, in this order: the activations of stage s + 3 (NA = ML a lane: the live rows) after the barrier, the weights of
   stage s + 3 (NB a lane: eight 8-byte quant loads, two scale loads) after the MFMAs, every stage past the end a
   repeat of the last. At the top of stage s the youngest 2 NA + 2 NB loads may still run: those of stages s + 1
   and s + 2; everything stage s reads is older. The loads stay in flight for about three stages, which the
   activation and weight streams need: with two, the stage time was the memory latency over two. */

/* The workgroup barrier of the pipeline: this wave's LDS accesses done, then s_barrier. Not a fence: a
   workgroup release fence would also wait for every global-to-LDS load in flight (vmcnt(0)), which the
   pipeline keeps in flight across barriers on purpose. The memory clobber keeps the compiler from moving
   memory accesses across it. */
__device__ __forceinline__ void wg_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void vm_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p;
}

/* A global-to-LDS load of 16 bytes a lane: lane L's bytes land at lds + 16 L. M0 is set here and nowhere else
   in these kernels. */
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

#define PW_THREADS 256
#define PW_NB 10
#define PW_AST 4 /* activation stages in the LDS ring */

typedef __attribute__((ext_vector_type(2))) uint32_t pw_u32x2;

/* eight int8 quants (lo, hi) times d, rounded to bf16: (u - 128) d with u = q + 128 as a byte, exact in fp32 */
__device__ __forceinline__ u32x4 pw_widen8(uint32_t lo, uint32_t hi, float d, float nd128) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const uint32_t v[2] = {lo ^ 0x80808080u, hi ^ 0x80808080u};
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 2; w++) {
        const float f0 = fmaf((float)(v[w] & 0xffu), d, nd128), f1 = fmaf((float)((v[w] >> 8) & 0xffu), d, nd128);
        const float f2 = fmaf((float)((v[w] >> 16) & 0xffu), d, nd128), f3 = fmaf((float)(v[w] >> 24), d, nd128);
        const bf16x2 p0 = {(__bf16)f0, (__bf16)f1}, p1 = {(__bf16)f2, (__bf16)f3};
        o[2 * w] = __builtin_bit_cast(uint32_t, p0);
        o[2 * w + 1] = __builtin_bit_cast(uint32_t, p1);
    }
    return u32x4{o[0], o[1], o[2], o[3]};
}

/* A stage's weights of one lane: quants q[t][j] (tile t, K step j: its 8 bytes), scales d[t] (the stage's two
   blocks, f16) */
struct pw_bset {
    pw_u32x2 q[2][4];
    uint32_t d[2];
};

template <bool GU, int ML>
__device__ __forceinline__ void pw_body(const prefill_args& a, int e, int m0, int nt, int cnt, uint8_t* lds, int* yrow, float* ywt) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, l32 = lane & 31, kq = lane >> 5;
    const int H = a.gate.cols, I = a.gate.rows;
    const int KD = GU ? H : I, nb = KD / 32, S = KD / PF_BK;
    const int pbase = a.off[e];

    /* activations, only the tile's 32 ML live rows: DMA i of this lane fills 16-byte slot (wv * NA + i) * 64 + lane
       of a stage: row slot / 8, position slot % 8, which holds chunk position ^ ((row >> 1) & 7) */
    constexpr int NA = ML;
    const uint8_t* abase = reinterpret_cast<const uint8_t*>(GU ? a.xb : a.act);
    uint32_t aoff[NA]; /* byte offsets from abase: the activations are under 4 GiB (launch_prefill_gemm) */
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int sl = (wv * NA + i) * 64 + lane, r = sl >> 3, c = chunk_pos(r, sl & 7);
        const int pa = min(m0 + r, cnt - 1);
        const size_t row = GU ? (size_t)(a.pairs[(size_t)e * a.cap + pa] / ROUTE_K_MAX) * H : (size_t)(pbase + pa) * I;
        aoff[i] = (uint32_t)(row * 2 + 16 * c);
    }
    /* weights from the experts' tiled copy (gtile_kernel): per 64-row group and 128-column unit, eight 1 KB
       chunks [64 rows][16 columns], then the rows' four scales each. Tile t of this wave is a 32-row half of a
       group. */
    const uint8_t *wq[2], *wd[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const qmat& W = GU ? (t ? a.up : a.gate) : a.down;
        const int r0 = GU ? nt * 128 + wv * 32 : nt * 256 + wv * 64 + t * 32;
        const size_t units = (size_t)W.cols / 128, stride = (size_t)(W.rows / 64) * units * 8704;
        const uint8_t* g0 = W.tiled + (size_t)e * stride + (size_t)(r0 >> 6) * units * 8704;
        const int rin = (r0 & 32) + l32; /* row in the 64-row group */
        wq[t] = g0 + rin * 16 + 8 * kq;
        wd[t] = g0 + 8192 + rin * 8;
    }
    const uint32_t lds0 = lds_addr(lds);
    if (!GU && tid < PF_BM && m0 + tid < cnt) {
        /* the tile's pairs: where each one's part goes and its weight (read by the epilogue, after the barriers) */
        const int pr = a.pairs[(size_t)e * a.cap + m0 + tid], row = pr / ROUTE_K_MAX, sl = pr % ROUTE_K_MAX;
        yrow[tid] = row * a.K + sl;
        ywt[tid] = a.rt[row].weights[sl];
    }

    auto issue_a = [&](int x) {
        x = min(x, S - 1);
        const uint32_t base = lds0 + (uint32_t)(x % PW_AST) * PF_TILE_BYTES + (uint32_t)wv * NA * 1024;
#pragma unroll
        for (int i = 0; i < NA; i++) dma16(abase + aoff[i] + (size_t)x * 128, __builtin_amdgcn_readfirstlane(base + i * 1024));
    };
    /* The weight loads are asm of our own, like the activations', and waited for by count: the compiler would
       count only its own loads and so wait for younger global-to-LDS loads too. Nothing touches a set's
       registers between its loads and the wait that names them (the stage's "+v" wait below). */
    auto issue_b = [&](int x, pw_bset& b) {
        x = min(x, S - 1);
        const size_t u = (size_t)(x >> 1) * 8704;
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                asm volatile("global_load_dwordx2 %0, %1, off" : "=&v"(b.q[t][j]) : "v"(wq[t] + u + (4 * (x & 1) + j) * 1024) : "memory");
            asm volatile("global_load_dword %0, %1, off" : "=&v"(b.d[t]) : "v"(wd[t] + u + 4 * (x & 1)) : "memory");
        }
    };

    f32x16 acc[ML][2];
#pragma unroll
    for (int m = 0; m < ML; m++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[m][t][r] = 0.0f;

    /* fragment reads: row 32 m + l32 of the stage, chunk 2 j + kq */
    const int swz = (l32 >> 1) & 7;
    /* Fragment reads are plain LDS loads: the compiler sees no global-to-LDS load (they are asm of our own), so it
       waits only for its LDS reads, and it can interleave them, the widening and the MFMAs. The barrier's memory
       clobber keeps them inside their stage. */
    typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
    auto read_a = [&](uint32_t base, int j, u32x4 (&f)[ML]) {
        const uint32_t p = base + (uint32_t)l32 * 128 + (uint32_t)(((2 * j + kq) ^ swz) << 4);
#pragma unroll
        for (int m = 0; m < ML; m++) f[m] = *(lds_u32x4*)(uintptr_t)(p + m * 4096);
    };

    pw_bset bs[4];
    auto stage = [&](int s, pw_bset& b) {
        /* the activations of stage s in LDS (every wave's own loads, then the barrier), this lane's weights */
        asm volatile("s_waitcnt vmcnt(%10)"
                     : "+v"(b.q[0][0]), "+v"(b.q[0][1]), "+v"(b.q[0][2]), "+v"(b.q[0][3]), "+v"(b.q[1][0]), "+v"(b.q[1][1]),
                       "+v"(b.q[1][2]), "+v"(b.q[1][3]), "+v"(b.d[0]), "+v"(b.d[1])
                     : "n"(2 * NA + 2 * PW_NB)
                     : "memory");
        wg_barrier();
        issue_a(s + 3);
        const uint32_t abase = lds0 + (uint32_t)(s % PW_AST) * PF_TILE_BYTES;
        u32x4 fa[2][ML];
        read_a(abase, 0, fa[0]);
        float dd[2][2], nd[2][2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                dd[t][h] = f16_bits_to_f32(h ? b.d[t] >> 16 : b.d[t] & 0xffffu);
                nd[t][h] = -128.0f * dd[t][h];
            }
        /* the next stage's weight set is free once this stage has widened its own: issue it at the end */
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (j < 3) read_a(abase, j + 1, fa[(j + 1) & 1]);
            u32x4 bw[2];
#pragma unroll
            for (int t = 0; t < 2; t++) bw[t] = pw_widen8(b.q[t][j].x, b.q[t][j].y, dd[t][j >> 1], nd[t][j >> 1]);
#pragma unroll
            for (int m = 0; m < ML; m++)
#pragma unroll
                for (int t = 0; t < 2; t++)
                    acc[m][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[j & 1][m]),
                                                                       __builtin_bit_cast(bf16x8, bw[t]), acc[m][t], 0, 0, 0);
        }
    };

    /* prologue: A(0) B(0) A(1) B(1) B(2); stage s then issues A(s + 2) and B(s + 3) */
    vm_wait<0>();
    issue_a(0);
    issue_b(0, bs[0]);
    issue_a(1);
    issue_b(1, bs[1]);
    issue_a(2);
    issue_b(2, bs[2]);
    /* S is a multiple of 4 (launch_prefill_gemm): the body has no branch, so the compiler's waits for the
       weight registers count the loads of the straight line */
    for (int s0 = 0; s0 < S; s0 += 4) {
        stage(s0, bs[0]);
        issue_b(s0 + 3, bs[3]);
        stage(s0 + 1, bs[1]);
        issue_b(s0 + 4, bs[0]);
        stage(s0 + 2, bs[2]);
        issue_b(s0 + 5, bs[1]);
        stage(s0 + 3, bs[3]);
        issue_b(s0 + 6, bs[2]);
    }
    /* every load done: none into LDS outlives the workgroup, and the weight sets loaded past the end (bs[0..2]; the
       last stage consumed bs[3]) stay live until here, so the compiler gives their registers to nothing else while
       their loads may still land */
#pragma unroll
    for (int i = 0; i < 3; i++)
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+v"(bs[i].q[0][0]), "+v"(bs[i].q[0][1]), "+v"(bs[i].q[0][2]), "+v"(bs[i].q[0][3]), "+v"(bs[i].q[1][0]),
                       "+v"(bs[i].q[1][1]), "+v"(bs[i].q[1][2]), "+v"(bs[i].q[1][3]), "+v"(bs[i].d[0]), "+v"(bs[i].d[1])
                     :
                     : "memory");

    /* accumulator r of a lane: row 8 (r / 4) + 4 kq + r % 4 of the 32 x 32 tile, column l32 */
#pragma unroll
    for (int m = 0; m < ML; m++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int p = m0 + 32 * m + 8 * (r >> 2) + 4 * kq + (r & 3);
            if (p >= cnt) continue;
            if (GU) {
                const float gt = acc[m][0][r], up = acc[m][1][r];
                const float v = pf_swiglu(gt, up);
                a.act[(size_t)(pbase + p) * I + nt * 128 + wv * 32 + l32] = (uint16_t)bf16_rne(v);
            } else {
                const int q = p - m0;
                const float wt = ywt[q];
                uint16_t* y = a.ypart + (size_t)yrow[q] * H + nt * 256 + wv * 64 + l32;
#pragma unroll
                for (int t = 0; t < 2; t++) y[32 * t] = (uint16_t)bf16_rne(acc[m][t][r] * wt);
            }
        }
}


template <bool GU>
__global__ __launch_bounds__(PW_THREADS, 1) void prefill_wgemm_kernel(prefill_args a) {

    __shared__ __attribute__((aligned(1024))) uint8_t lds[PW_AST * PF_TILE_BYTES];
    __shared__ int yrow[PF_BM];
    __shared__ float ywt[PF_BM];
    const int H = a.gate.cols, I = a.gate.rows;
    const int NT = GU ? I / 128 : H / 256;
    const int nwork = *a.n_tiles * NT;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per = (nwork + 7) >> 3;
    const int w = xcd * per + slot;
    if (slot >= per || w >= nwork) return;
    const int tl = a.tiles[w / NT], nt = w - (w / NT) * NT;
    const int e = tl >> 16, m0 = (tl & 0xffff) * PF_BM;
    const int cnt = a.count[e];
    const int rows = cnt - m0;
    if (rows > 128) pw_body<GU, 8>(a, e, m0, nt, cnt, lds, yrow, ywt);
    else if (rows > 64) pw_body<GU, 4>(a, e, m0, nt, cnt, lds, yrow, ywt);
    else pw_body<GU, 2>(a, e, m0, nt, cnt, lds, yrow, ywt);
}

/* ---- the matrix cores' yardstick ------------------------------------------ */

/* Nothing but v_mfma_f32_32x32x16_bf16 on eight independent accumulators a wave, one wave a SIMD: what the
   matrix cores of this device sustain, as the copy probe is what its memory streams. */
__global__ __launch_bounds__(256, 1) void mfma_probe_kernel(float* __restrict__ out, int iters, float seed) {
    f32x16 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;
    bf16x8 x, w;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        x[k] = (__bf16)(seed * (float)(threadIdx.x + k));
        w[k] = (__bf16)(seed * (float)(k + 1));
    }
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, w, acc[i], 0, 0, 0);
    }
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) sum += acc[i][r];
    out[blockIdx.x * 256 + threadIdx.x] = sum; /* kept, so the products are not optimized away */
}

hipError_t launch_mfma_probe(float* out, int blocks, int iters, hipStream_t s) {
    if (blocks < 1 || iters < 1) return hipErrorInvalidValue;
    mfma_probe_kernel<<<blocks, 256, 0, s>>>(out, iters, 1e-3f);
    return hipGetLastError();
}

double mfma_probe_flops(int blocks, int iters) { return (double)blocks * 4 * iters * 8 * (2.0 * 32 * 32 * 16); }

/* ---- launches ----------------------------------------------------------- */

/* Experts a 16-lane group of the routers. At 128 experts the plain router's groups of 8 left one block column:
   1024 rows were 128 blocks (a prompt of 4096 tokens 210.6 -> 208.4 ms exact with 2). The fused kernel
   normalizes its rows in every block of a row tile, so it keeps 8 (config 4: 73 us, against 101 with 4 and 155
   with 2). Each (row, expert) chain runs the same either way: the same bits. */
#define PR_RE 2
#define NR_RE 8

hipError_t launch_prefill_norm(const float* x, const float* w, float* xn, uint16_t* xb, int n, int H, float eps, hipStream_t s) {
    if (n < 1 || H % 16 || H > 8192) return hipErrorInvalidValue;
    prefill_norm_kernel<<<n, 64, H * 4, s>>>(x, w, xn, xb, H, eps);
    return hipGetLastError();
}

hipError_t launch_prefill_router(const float* xn, const float* R, float* logits, int n, int E, int H, hipStream_t s) {
    if (n < 1 || E < 1 || H % 16) return hipErrorInvalidValue;
    constexpr int RT = 8, RE = PR_RE;
    prefill_router_kernel<RT, RE><<<dim3((E + 16 * RE - 1) / (16 * RE), (n + RT - 1) / RT), 256, 0, s>>>(xn, R, logits, n, E, H);
    return hipGetLastError();
}

hipError_t launch_prefill_norm_router(const float* x, const float* nw, const float* R, float* logits, uint16_t* xb, int n, int E,
                                     int H, float eps, hipStream_t s) {
    if (n < 1 || E < 1 || H % 16) return hipErrorInvalidValue;
    if (H > NR_HMAX) return hipErrorNotSupported; /* the two-kernel form */
    constexpr int RT = 8, RE = NR_RE;
    prefill_norm_router_kernel<RT, RE><<<dim3((E + 16 * RE - 1) / (16 * RE), (n + RT - 1) / RT), 256, 0, s>>>(x, nw, R, logits, xb, n, E, H, eps);
    return hipGetLastError();
}

/* The bf16 rounding of n fp32 values (the normalized rows a pass of rows hands the grouped GEMM), four a thread. */
__global__ __launch_bounds__(256) void prefill_bf16_kernel(const float4* __restrict__ x, uint2* __restrict__ xb, size_t n4) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        const float4 v = x[i];
        xb[i] = uint2{bf16_rne(v.x) | (bf16_rne(v.y) << 16), bf16_rne(v.z) | (bf16_rne(v.w) << 16)};
    }
}

hipError_t launch_prefill_bf16(const float* x, uint16_t* xb, size_t n, hipStream_t s) {
    if (!n || n % 4) return hipErrorInvalidValue;
    const size_t n4 = n / 4, blocks = std::min<size_t>((n4 + 255) / 256, 4096);
    prefill_bf16_kernel<<<(unsigned)blocks, 256, 0, s>>>(reinterpret_cast<const float4*>(x), reinterpret_cast<uint2*>(xb), n4);
    return hipGetLastError();
}

hipError_t launch_prefill_plan(const int* count, int E, int* off, int* tiles, int* n_tiles, hipStream_t s) {
    if (E < 1 || E > ROUTE_E_MAX) return hipErrorInvalidValue;
    prefill_plan_kernel<<<1, 256, 0, s>>>(count, E, off, tiles, n_tiles);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void prefill_chosen_kernel(const route_out* __restrict__ rt, int n, int K, int32_t* __restrict__ chosen) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n * K) chosen[i] = rt[i / K].chosen[i % K];
}

hipError_t launch_prefill_chosen(const route_out* rt, int n, int K, int32_t* chosen, hipStream_t s) {
    if (n < 1 || K < 1 || K > ROUTE_K_MAX) return hipErrorInvalidValue;
    prefill_chosen_kernel<<<(n * K + 255) / 256, 256, 0, s>>>(rt, n, K, chosen);
    return hipGetLastError();
}

/* x[row][c] += sum over slots k, in order, of the bf16 parts: eight columns a thread, the K parts all requested
   before the first add */
__global__ __launch_bounds__(256) void prefill_sum_kernel(const uint16_t* __restrict__ ypart, float* __restrict__ x, int K, int H) {
    const int row = blockIdx.y, c8 = blockIdx.x * blockDim.x + threadIdx.x;
    if (c8 >= H / 8) return;
    const uint4* yp = reinterpret_cast<const uint4*>(ypart + (size_t)row * K * H) + c8;
    uint4 p[ROUTE_K_MAX];
#pragma unroll
    for (int k = 0; k < ROUTE_K_MAX; k++)
        if (k < K) p[k] = yp[(size_t)k * (H / 8)];
    float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < ROUTE_K_MAX; k++)
        if (k < K) {
            const uint32_t w[4] = {p[k].x, p[k].y, p[k].z, p[k].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sum[2 * i] = sum[2 * i] + __uint_as_float(w[i] << 16);
                sum[2 * i + 1] = sum[2 * i + 1] + __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    float4* xp = reinterpret_cast<float4*>(x + (size_t)row * H) + 2 * c8;
    float4 v0 = xp[0], v1 = xp[1];
    v0.x = v0.x + sum[0]; v0.y = v0.y + sum[1]; v0.z = v0.z + sum[2]; v0.w = v0.w + sum[3];
    v1.x = v1.x + sum[4]; v1.y = v1.y + sum[5]; v1.z = v1.z + sum[6]; v1.w = v1.w + sum[7];
    xp[0] = v0;
    xp[1] = v1;
}

hipError_t launch_prefill_sum(const uint16_t* ypart, float* x, int n, int K, int H, hipStream_t s) {
    if (n < 1 || K < 1 || K > ROUTE_K_MAX || H % 8) return hipErrorInvalidValue;
    prefill_sum_kernel<<<dim3((H / 8 + 255) / 256, n), 256, 0, s>>>(ypart, x, K, H);
    return hipGetLastError();
}

int prefill_max_tiles(int n, int K, int E) { return (n * K + PF_BM - 1) / PF_BM + E; }

template <bool GU>
static hipError_t launch_shared_stage(const prefill_args& a, int dt, unsigned blocks, hipStream_t s) {
    switch (dt) {
        case VITNA_DTYPE_Q8_0: prefill_gemm_kernel<GU, VITNA_DTYPE_Q8_0><<<blocks, PF_THREADS, 0, s>>>(a); break;
        case VITNA_DTYPE_Q4_K: prefill_gemm_kernel<GU, VITNA_DTYPE_Q4_K><<<blocks, PF_THREADS, 0, s>>>(a); break;
        case VITNA_DTYPE_Q6_K: prefill_gemm_kernel<GU, VITNA_DTYPE_Q6_K><<<blocks, PF_THREADS, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_prefill_gemm(const prefill_args& a, bool gate_up, hipStream_t s) {
    const int H = a.gate.cols, I = a.gate.rows;
    auto quant = [](int t) { return t == VITNA_DTYPE_Q8_0 || t == VITNA_DTYPE_Q4_K || t == VITNA_DTYPE_Q6_K; };
    if (!quant(a.gate.dtype) || a.up.dtype != a.gate.dtype || !quant(a.down.dtype)) return hipErrorInvalidValue;
    if (H % PF_BN || I % (PF_BN / 2) || a.up.rows != I || a.up.cols != H || a.down.rows != H || a.down.cols != I) return hipErrorInvalidValue;
    /* a K-quant stage (64 columns) lies within one 256-column super-block */
    if ((a.gate.dtype != VITNA_DTYPE_Q8_0 && H % 256) || (a.down.dtype != VITNA_DTYPE_Q8_0 && I % 256)) return hipErrorInvalidValue;
    if (a.K < 1 || a.K > ROUTE_K_MAX || a.cap > 65536 * PF_BM || a.E > ROUTE_E_MAX) return hipErrorInvalidValue;
    const int NT = gate_up ? I / (PF_BN / 2) : H / PF_BN;
    const size_t blocks = ((size_t)NT * prefill_max_tiles(a.n, a.K, a.E) + 7) / 8 * 8;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    /* Q8_0 experts with their tiled copy (made by the allocating entry points) take the kernel that widens each
       wave's own weights; K-quant experts, and Q8_0 ones without the copy (the no-allocation entry point before any
       allocating one ran), the shared-stage kernel, which reads the planes. On Q8_0 the two give the same bits: the
       same products, summed in the same order. */
    const bool q8 = a.gate.dtype == VITNA_DTYPE_Q8_0 && a.down.dtype == VITNA_DTYPE_Q8_0;
    const bool wide = q8 && a.gate.tiled && a.up.tiled && a.down.tiled && H % 256 == 0 && I % 256 == 0 &&
                      (size_t)a.n * a.K * I * 2 < ((size_t)1 << 32) && (size_t)a.n * H * 2 < ((size_t)1 << 32);
    if (wide && gate_up) prefill_wgemm_kernel<true><<<(unsigned)blocks, PW_THREADS, 0, s>>>(a);
    else if (wide) prefill_wgemm_kernel<false><<<(unsigned)blocks, PW_THREADS, 0, s>>>(a);
    else if (gate_up) return launch_shared_stage<true>(a, a.gate.dtype, (unsigned)blocks, s);
    else return launch_shared_stage<false>(a, a.down.dtype, (unsigned)blocks, s);
    return hipGetLastError();
}
