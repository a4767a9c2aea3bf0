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
 * The experts: Q8_0 quants (|q| <= 127) are exact in bf16, so they enter the
 * MFMA unscaled; each 32-weight block's fp32 scale d multiplies that block's
 * fp32 partial product on the accumulators. The only rounding beyond fp32 is
 * that of the activations (normed rows, then the SwiGLU output) to bf16.
 *
 * Pipeline, one stream:
 *   prefill_norm_kernel     exact RMSNorm; fp32 rows for the router, bf16 for the GEMM
 *   prefill_router_kernel   exact router logits, 8 rows x 8 experts a thread
 *   topk_kernel             the routing rule on every row (kernels_decode.hip)
 *   group_kernel            (row, slot) pairs of each expert in row order (kernels_rows.hip)
 *   prefill_plan_kernel     pair offsets of each expert; the list of 128-pair tiles
 *   prefill_gemm_kernel<1>  act = silu(X_e G_e^T) * (X_e U_e^T), bf16, pairs in expert order
 *   prefill_gemm_kernel<0>  ypart[row * K + slot] = w * (act_e D_e^T)
 *   reduce_rows_kernel      x += the K parts of a row in slot order (kernels_rows.hip)
 *
 * GEMM tiling: a 256-thread workgroup owns 128 pairs x 128 weight rows (for
 * gate/up: 64 gate rows and the 64 up rows of the same columns, so SwiGLU is
 * local to a lane). Each wave owns 64 x 64 as 2 x 2 tiles of
 * v_mfma_f32_32x32x16_bf16. K advances 64 a stage (two Q8_0 blocks) through
 * a three-stage LDS ring filled by global-to-LDS loads, two stages ahead. Work items (tile, column block) are split into eight
 * contiguous ranges, one per XCD (workgroup i runs on XCD i mod 8), so the
 * column blocks of one tile and the tiles of one expert share an L2.
 */

#include "vitna_kernels.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define PF_BM 128 /* pairs a tile */
#define PF_BN 128 /* weight rows a workgroup */
#define PF_BK 64  /* contraction a stage: two Q8_0 blocks */

__device__ __forceinline__ uint32_t bf16_rne(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

/* two small integers (exact in bf16: the top half of the float) packed low, high */
__device__ __forceinline__ uint32_t pack_int_bf16(int lo, int hi) {
    return (__float_as_uint((float)lo) >> 16) | (__float_as_uint((float)hi) & 0xffff0000u);
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
        uint2 b;
        b.x = bf16_rne(o.x) | (bf16_rne(o.y) << 16);
        b.y = bf16_rne(o.z) | (bf16_rne(o.w) << 16);
        reinterpret_cast<uint2*>(xb + r * H)[i] = b;
    }
}

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

/* LDS ring of PF_STAGES stages; a stage holds K = 64 of the tile:
     A  128 rows x 128 B (bf16), 16-byte chunk c of row r at position c ^ (r & 7)
     B  128 rows x  64 B (int8 quants), chunk c of row n at position c ^ ((n >> 2) & 3)
     D  128 rows x 2 f16 scales, each in the low half of a dword (a 2-byte
        global-to-LDS load fills 4 bytes of LDS a lane)
   The swizzles keep the fragment reads (eight or sixteen consecutive rows at
   one chunk) on distinct banks. Global-to-LDS loads (global_load_lds) fill
   them without passing through registers; each wave issues the same seven
   loads a stage, so "stage s has landed" is vmcnt <= 7 x (stages in flight
   after s), followed by a barrier for the other waves' parts. */
#define PF_STAGES 3
#define PF_A_BYTES (PF_BM * 128)
#define PF_B_BYTES (PF_BN * 64)
#define PF_D_BYTES (PF_BN * 8)
#define PF_STAGE_BYTES (PF_A_BYTES + PF_B_BYTES + PF_D_BYTES)

/* 8 int8 quants (two dwords) as 8 bf16 */
__device__ __forceinline__ bf16x8 widen_q8(uint32_t w0, uint32_t w1) {
    u32x4 o;
    o[0] = pack_int_bf16((int)(int8_t)(w0 & 0xff), (int)(int8_t)((w0 >> 8) & 0xff));
    o[1] = pack_int_bf16((int)(int8_t)((w0 >> 16) & 0xff), (int)(int8_t)(w0 >> 24));
    o[2] = pack_int_bf16((int)(int8_t)(w1 & 0xff), (int)(int8_t)((w1 >> 8) & 0xff));
    o[3] = pack_int_bf16((int)(int8_t)((w1 >> 16) & 0xff), (int)(int8_t)(w1 >> 24));
    return __builtin_bit_cast(bf16x8, o);
}

template <bool GU>
__global__ __launch_bounds__(256, 2) void prefill_gemm_kernel(prefill_args a) {
    __shared__ __attribute__((aligned(1024))) uint8_t ring[PF_STAGES * PF_STAGE_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int H = a.gate.cols, I = a.gate.rows;
    const int NT = GU ? I / 64 : H / PF_BN; /* column blocks a tile */
    const int KD = GU ? H : I;              /* contraction length */
    const int nwork = *a.n_tiles * NT;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per = (nwork + 7) >> 3;
    const int w = xcd * per + slot;
    if (slot >= per || w >= nwork) return;
    const int tl = a.tiles[w / NT], nt = w - (w / NT) * NT;
    const int e = tl >> 16, m0 = (tl & 0xffff) * PF_BM;
    const int cnt = a.count[e];
    const int pbase = a.off[e];
    const int nb = KD / 32;

    /* global sources of this lane's seven loads a stage (advanced by the stage) */
    const uint8_t* asrc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int sl = (wv * 4 + i) * 64 + lane, r = sl >> 3, c = (sl & 7) ^ (r & 7);
        const int pa = min(m0 + r, cnt - 1);
        const uint16_t* row = GU ? a.xb + (size_t)(a.pairs[(size_t)e * a.cap + pa] / ROUTE_K_MAX) * H : a.act + (size_t)(pbase + pa) * I;
        asrc[i] = reinterpret_cast<const uint8_t*>(row) + 16 * c;
    }
    const uint8_t* bsrc[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int sl = (wv * 2 + i) * 64 + lane, n = sl >> 2, c = (sl & 3) ^ ((n >> 2) & 3);
        const qmat& wm = GU ? (n < 64 ? a.gate : a.up) : a.down;
        const int wrow = GU ? nt * 64 + (n & 63) : nt * PF_BN + n;
        bsrc[i] = wm.p[0] + (size_t)e * wm.estride[0] + (size_t)wrow * nb * 32 + 16 * c;
    }
    const uint8_t* dsrc;
    {
        const int sl = wv * 64 + lane, n = sl >> 1, blk = sl & 1;
        const qmat& wm = GU ? (n < 64 ? a.gate : a.up) : a.down;
        const int wrow = GU ? nt * 64 + (n & 63) : nt * PF_BN + n;
        dsrc = wm.p[1] + (size_t)e * wm.estride[1] + ((size_t)wrow * nb + blk) * 2;
    }
    auto issue = [&](int s, int buf) {
        uint8_t* base = ring + buf * PF_STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_global_load_lds((glb_void)(asrc[i] + (size_t)s * 128), (lds_void)(base + (wv * 4 + i) * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_global_load_lds((glb_void)(bsrc[i] + (size_t)s * 64), (lds_void)(base + PF_A_BYTES + (wv * 2 + i) * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((glb_void)(dsrc + (size_t)s * 4), (lds_void)(base + PF_A_BYTES + PF_B_BYTES + wv * 256), 2, 0, 0);
    };

    /* this wave's 64 x 64: A rows wmi * 64 + 32 i + lane % 32, B rows brow[k]; the lane's k-octet kq */
    const int wmi = wv >> 1, wni = wv & 1, l32 = lane & 31, kq = lane >> 5;
    int aoff[2], boff[2], brow[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = wmi * 64 + i * 32 + l32;
        aoff[i] = r * 128;
        brow[i] = GU ? i * 64 + wni * 32 + l32 : wni * 64 + i * 32 + l32;
        boff[i] = brow[i] * 64 ;
    }
    const int aswz[2] = {(wmi * 64 + l32) & 7, (wmi * 64 + 32 + l32) & 7};
    const int bswz[2] = {(brow[0] >> 2) & 3, (brow[1] >> 2) & 3};

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][k][r] = 0.0f;
    const f32x16 zero = {};

    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;
    const int S = KD / PF_BK;
    issue(0, 0);
    if (S > 1) issue(1, 1);
    for (int s = 0; s < S; s++) {
        if (s + 1 < S) asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (s + 2 < S) issue(s + 2, (s + 2) % PF_STAGES);
        /* Fragment reads are issued as ds_read instructions of our own: the compiler would otherwise wait for
           every global-to-LDS load in flight (vmcnt(0)) before any LDS read, the stage being filled included. */
        const uint32_t base = ring_lds + (s % PF_STAGES) * PF_STAGE_BYTES;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            u32x4 af[2][2];
            uint2 bq[2][2];
            uint32_t dr[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int c = 4 * b + 2 * h + kq; /* A chunk: k = 32 b + 16 h + 8 kq */
                    asm volatile("ds_read_b128 %0, %1" : "=v"(af[i][h]) : "v"(base + aoff[i] + ((c ^ aswz[i]) << 4)));
                    const int cb = 2 * b + h; /* B chunk: the same k, 16 quants a chunk */
                    asm volatile("ds_read_b64 %0, %1" : "=v"(bq[i][h]) : "v"(base + PF_A_BYTES + boff[i] + ((cb ^ bswz[i]) << 4) + 8 * kq));
                }
#pragma unroll
            for (int i = 0; i < 2; i++)
                asm volatile("ds_read_u16 %0, %1" : "=v"(dr[i]) : "v"(base + PF_A_BYTES + PF_B_BYTES + (brow[i] * 2 + b) * 4));
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(af[0][0]), "+v"(af[0][1]), "+v"(af[1][0]), "+v"(af[1][1]), "+v"(bq[0][0]), "+v"(bq[0][1]), "+v"(bq[1][0]),
                           "+v"(bq[1][1]), "+v"(dr[0]), "+v"(dr[1]));
            bf16x8 bfr[2][2];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int h = 0; h < 2; h++) bfr[i][h] = widen_q8(bq[i][h].x, bq[i][h].y);
            const float dd[2] = {f16_bits_to_f32(dr[0] & 0xffff), f16_bits_to_f32(dr[1] & 0xffff)};
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    f32x16 t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[i][0]), bfr[k][0], zero, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af[i][1]), bfr[k][1], t, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][k][r] = fmaf(dd[k], t[r], acc[i][k][r]);
                }
        }
    }

    /* accumulator r of a lane: row 8 (r / 4) + 4 (lane / 32) + r % 4 of the 32 x 32 tile, column lane % 32 */
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int p = m0 + wmi * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (p >= cnt) continue;
            if (GU) {
                const float gt = acc[i][0][r], up = acc[i][1][r];
                const float v = gt / (1.0f + __expf(-gt)) * up;
                a.act[(size_t)(pbase + p) * I + nt * 64 + wni * 32 + l32] = (uint16_t)bf16_rne(v);
            } else {
                const int pr = a.pairs[(size_t)e * a.cap + p], row = pr / ROUTE_K_MAX, sl = pr % ROUTE_K_MAX;
                const float wt = a.rt[row].weights[sl];
                float* y = a.ypart + ((size_t)row * a.K + sl) * H + nt * PF_BN + wni * 64 + l32;
                y[0] = acc[i][0][r] * wt;
                y[32] = acc[i][1][r] * wt;
            }
        }
}

/* ---- launches ----------------------------------------------------------- */

hipError_t launch_prefill_norm(const float* x, const float* w, float* xn, uint16_t* xb, int n, int H, float eps, hipStream_t s) {
    if (n < 1 || H % 16 || H > 8192) return hipErrorInvalidValue;
    prefill_norm_kernel<<<n, 64, H * 4, s>>>(x, w, xn, xb, H, eps);
    return hipGetLastError();
}

hipError_t launch_prefill_router(const float* xn, const float* R, float* logits, int n, int E, int H, hipStream_t s) {
    if (n < 1 || E < 1 || H % 16) return hipErrorInvalidValue;
    constexpr int RT = 8, RE = 8;
    prefill_router_kernel<RT, RE><<<dim3((E + 16 * RE - 1) / (16 * RE), (n + RT - 1) / RT), 256, 0, s>>>(xn, R, logits, n, E, H);
    return hipGetLastError();
}

hipError_t launch_prefill_plan(const int* count, int E, int* off, int* tiles, int* n_tiles, hipStream_t s) {
    if (E < 1 || E > ROUTE_E_MAX) return hipErrorInvalidValue;
    prefill_plan_kernel<<<1, 256, 0, s>>>(count, E, off, tiles, n_tiles);
    return hipGetLastError();
}

int prefill_max_tiles(int n, int K, int E) { return (n * K + PF_BM - 1) / PF_BM + E; }

hipError_t launch_prefill_gemm(const prefill_args& a, bool gate_up, hipStream_t s) {
    const int H = a.gate.cols, I = a.gate.rows;
    const qmat* parts[3] = {&a.gate, &a.up, &a.down};
    for (const qmat* q : parts)
        if (q->dtype != VITNA_DTYPE_Q8_0) return hipErrorInvalidValue;
    if (H % PF_BN || I % PF_BK || a.up.rows != I || a.up.cols != H || a.down.rows != H || a.down.cols != I) return hipErrorInvalidValue;
    if (a.K < 1 || a.K > ROUTE_K_MAX || a.cap > 65536 * PF_BM || a.E > ROUTE_E_MAX) return hipErrorInvalidValue;
    const int NT = gate_up ? I / 64 : H / PF_BN;
    const size_t blocks = ((size_t)NT * prefill_max_tiles(a.n, a.K, a.E) + 7) / 8 * 8;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (gate_up) prefill_gemm_kernel<true><<<(unsigned)blocks, 256, 0, s>>>(a);
    else prefill_gemm_kernel<false><<<(unsigned)blocks, 256, 0, s>>>(a);
    return hipGetLastError();
}
