/**
 * kernels_step.hip - The batch-1 decode step (every layer of one token) as
 * one persistent kernel on gfx950: the path the reference runs as a chain of
 * kernels per layer (engine/src/model_cuda.cu attn_in_kernel :870,
 * attention_kernel :942, matvec_add_kernel :1430, router_kernel :1544,
 * experts_in_kernel :1566, experts_down_kernel :1591), with the CPU order
 * of engine/src/model.c:887-979 where parity needs it.
 *
 * One block a CU, eight waves a block. Wave 0 of each block is its control
 * wave: it waits for the inputs of the block's next piece of work, brings them
 * into LDS, and publishes the block's results. Waves 1-7 are workers: they
 * request the weights of their next piece of work as soon as its addresses are
 * known, before its inputs exist, so the weight stream overlaps the wait; a
 * worker never waits on a global load it did not need, because every
 * cross-block value goes through the control wave.
 *
 * A layer is six phases; each ends with every block's flag:
 *   QKV    RMSNorm (the reference's sixteen-chain order) + q, k, v GEMV rows
 *   ATT    attention over one chunk of positions of one key-value head, for
 *          the G query heads that share it: partial (max, sum, values);
 *          the chunk holding the new position also stores its k and v
 *   O      the chunks of two query heads merged, times those heads' 256
 *          columns of the o-projection, for 1/RG of its rows (a split over
 *          columns: the router phase adds the splits in a fixed order)
 *   ROUTE  (a few blocks) the residual after attention, its RMSNorm and the
 *          router's logits, all in the reference's order (bit-exact)
 *   IN     every block routes the token (the reference's rule), then the
 *          chosen experts' gate and up rows and SiLU
 *   DOWN   the experts' down rows, their weighted sum, the residual
 * A mixture-of-experts model without attention runs ROUTE, IN and DOWN.
 *
 * Cross-block data moves through device-coherent memory: buffer stores and
 * loads with the sc1 bit (device scope), which write through and read past
 * the per-XCD L2. A block's results are stored by its control wave, which
 * waits for the stores to complete (vmcnt) before it stores its flag; a
 * reader polls the producers' flags with the same device-scope loads. The
 * flags of one step carry the step's epoch, so nothing is cleared between
 * steps. Every wait is bounded: a wait that runs out sets the abort word,
 * every other wait sees it, and the kernel drains; the host reports the
 * failure.
 */

#include "route_impl.h"
#include "step_kernel.h"

#include <mutex>

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;


#define SC1 16 /* the cache-policy bits of a device-scope buffer access */
#define STEP_SPIN_MAX (1u << 22)

__device__ __forceinline__ rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f4 ld4c(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, SC1));
}
__device__ __forceinline__ u32x4 ld4u(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, SC1); }
__device__ __forceinline__ float ld1c(rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, SC1));
}
__device__ __forceinline__ void st1c(float v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, SC1);
}
__device__ __forceinline__ void st4c(f4 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)off, 0, SC1);
}
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

/* Waves of the block meet; LDS writes before are seen by LDS reads after. Global loads in flight stay in flight. */
__device__ __forceinline__ void bar() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* ---- dtype dispatch of the slice helpers (a wave-uniform switch) ---- */
__device__ __forceinline__ void qload(int dt, const qmat& m, int e, int row, int t, qraw& r) {
    if (dt == VITNA_DTYPE_Q4_K) slice_load<VITNA_DTYPE_Q4_K>(m, e, row, t, r);
    else if (dt == VITNA_DTYPE_Q6_K) slice_load<VITNA_DTYPE_Q6_K>(m, e, row, t, r);
    else slice_load<VITNA_DTYPE_Q8_0>(m, e, row, t, r);
}
__device__ __forceinline__ float qdot(int dt, const qraw& r, int t, const xslice& xs) {
    if (dt == VITNA_DTYPE_Q4_K) return slice_dot<VITNA_DTYPE_Q4_K>(r, t, xs);
    if (dt == VITNA_DTYPE_Q6_K) return slice_dot<VITNA_DTYPE_Q6_K>(r, t, xs);
    return slice_dot<VITNA_DTYPE_Q8_0>(r, t, xs);
}
/* The lane's activations for slice t of a row whose columns start at base (LDS). */
__device__ __forceinline__ void lds_xslice(int dt, int t, const float* base, xslice& xs) {
    int a, b;
    slice_cols(dt, t, &a, &b);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 u = reinterpret_cast<const float4*>(base + a)[i], v = reinterpret_cast<const float4*>(base + b)[i];
        xs.lo[4 * i] = u.x; xs.lo[4 * i + 1] = u.y; xs.lo[4 * i + 2] = u.z; xs.lo[4 * i + 3] = u.w;
        xs.hi[4 * i] = v.x; xs.hi[4 * i + 1] = v.y; xs.hi[4 * i + 2] = v.z; xs.hi[4 * i + 3] = v.w;
    }
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) { s0 += xs.lo[i]; s1 += xs.hi[i]; }
    xs.slo = s0;
    xs.shi = s1;
}

/* ---- the control wave's waits ---- */

/* Until flags[0 .. n) all hold epoch or later (n <= 256). False when the step is aborted. */
__device__ bool wait_flags(const uint32_t* flags, int n, uint32_t epoch, uint32_t* abort_word, int lane, int nap) {
    const rsrc_t rf = rsrc(flags, 1024), ra = rsrc(abort_word, 4);
    for (uint32_t it = 0;; it++) {
        const u32x4 v = ld4u(rf, lane * 16);
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (4 * lane + i < n) ok &= (int32_t)(v[i] - epoch) >= 0;
        if (__all(ok)) return true;
        if ((it & 63) == 63) {
            if (__builtin_amdgcn_raw_buffer_load_b32(ra, 0, 0, SC1)) return false;
            if (it > STEP_SPIN_MAX) {
                if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(1u, ra, 0, 0, SC1);
                return false;
            }
        }
        for (int i = 0; i < nap; i++) __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ void set_flag(uint32_t* flags, int b, uint32_t epoch, int lane) {
    stores_done();
    if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(epoch, rsrc(flags, 1024), b * 4, 0, SC1);
}

/* The reference's RMSNorm of the H floats at x (LDS) with weights w (global), into out (LDS), by one wave:
   sixteen chains of squares (engine/src/kernels.c:115-140), the AVX2 fold, 1 / sqrtf(ss / H + eps), then
   (x * inv) * w, each step rounded. */
__device__ void norm_exact(const float* x, const float* __restrict__ w, float* out, int H, float eps, int lane) {
    float acc = 0.0f;
    if (lane < 16)
        for (int m0 = 0; m0 < H / 16; m0 += 16) {
            /* sixteen of the chain's values from LDS at once, then their FMAs in order */
            float xv[16];
#pragma unroll
            for (int i = 0; i < 16; i++) xv[i] = x[16 * (m0 + i) + lane];
#pragma unroll
            for (int i = 0; i < 16; i++) acc = fmaf(xv[i], xv[i], acc);
        }
    float ch[16];
#pragma unroll
    for (int q = 0; q < 16; q++) ch[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), q));
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] = ch[q] + ch[q + 8];
    const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    const float ss = (s0 + s2) + (s1 + s3);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = lane; i < H / 4; i += 64) {
        const float4 xv = reinterpret_cast<const float4*>(x)[i], wv = gld<float4>(w + 4 * i);
        float4 o;
        o.x = (xv.x * inv) * wv.x; o.y = (xv.y * inv) * wv.y; o.z = (xv.z * inv) * wv.z; o.w = (xv.w * inv) * wv.w;
        reinterpret_cast<float4*>(out)[i] = o;
    }
}

/* RMSNorm (fp32, for the per-head QK-norm) then the half-split RoPE at the table row, of hd floats at v (LDS) in
   place, by one wave: engine/src/model.c:919-928 (vitna_rmsnorm, vitna_rope_half, ops.c:273-281). */
__device__ void head_norm_rope(float* v, const float* __restrict__ nw, const float* __restrict__ cs, const float* __restrict__ sn, int hd,
                               float eps, int lane) {
    const int half = hd / 2;
    float ss = 0.0f;
    for (int d = lane; d < hd; d += 64) ss = fmaf(v[d], v[d], ss);
    ss = wave_sum_dpp(ss);
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    float a = 0.f, b = 0.f;
    if (lane < half) {
        a = v[lane];
        b = v[lane + half];
        if (nw) {
            a = (a * inv) * nw[lane];
            b = (b * inv) * nw[lane + half];
        }
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < half) {
        const float c = cs[lane], s = sn[lane];
        v[lane] = a * c - b * s;
        v[lane + half] = b * c + a * s;
    }
    __builtin_amdgcn_wave_barrier();
}

/* ---- the kernel ---- */

#define NW 7        /* worker waves a block: with the control wave, two waves a SIMD */
#define MAX0 3      /* q/k/v row groups a worker */
#define MAXO 4      /* o-projection row groups a worker */
#define MAX5 5      /* gate/up units a worker */
#define MAXD 2      /* down rows a worker */
#define SUB 64      /* positions an attention pass stages in LDS */
#define ATTN_PF 10  /* key-value rows a worker stages (ceil(SUB / NW)) */

/* HS: the hidden width in slices of 32; DGU, DDN: the experts' gate/up and down dtypes; IPL: down slices a lane
   (the K chosen experts' slices of one down row over 64 lanes). */
template <int HS, int DGU, int DDN, int IPL, bool ATT, int DQK, int DV, int DO>
__global__ __launch_bounds__(64 * (NW + 1)) void step_kernel(step_args a, const step_layer* __restrict__ LT) {
    constexpr int LPR = HS < 64 ? HS : 64, SPL = HS / LPR, RPW = 64 / LPR, H = HS * 32;
    extern __shared__ float lds[];
    __shared__ route_out srt;
    __shared__ float slg[ROUTE_E_MAX];
    __shared__ int sgo;
    /* the wave index is uniform within a wave: said so, the branches on it are scalar and the control and worker
       paths share registers */
    const int tid = threadIdx.x, lane0 = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool ctl = wv == 0;
    const int wk = wv - 1, NB = gridDim.x, b = blockIdx.x, GW = NB * NW, gw = b * NW + wk;
    float* sx = lds;              /* the layer's residual, then the residual after attention */
    float* sxn = sx + H;          /* its RMSNorm */
    float* sout = sxn + H;        /* results on their way out (STEP_OUT floats) */
    float* W = sout + STEP_OUT;   /* per-phase staging */

    const int pos = a.row->pos, seq = a.row->seq, token = a.row->token;
    const int hd = a.hd, G = a.nh > 0 ? a.nh / a.nkv : 1, qd = a.nh * hd, kd = a.nkv * hd, R0 = qd + 2 * kd;
    const uint32_t ep = a.epoch;
    /* attention chunks: nkv * nch units, one a block */
    const int npos = pos + 1;
    /* chunks a key-value head: a block each, at most 64 (the merge takes a chunk a lane) */
    const int per_head = a.nkv ? min(64, NB / a.nkv > 0 ? NB / a.nkv : 1) : 1;
    const int CHP = (npos + per_head - 1) / per_head, nch = (npos + CHP - 1) / CHP, U1 = a.nkv * nch;
    /* o-projection split: CG column groups of 256 (HPC heads each), RG row groups of RR rows */
    const int CG = qd / 256, RG = CG ? NB / CG : 1, RR = H / RG, HPC = 256 / (hd ? hd : 256);
    const int RB = (a.E + NW - 1) / NW; /* router blocks: a row a worker */
    const int S6 = a.I / 32, N6 = a.K * S6;         /* down slices a row */
    const size_t prec = (size_t)hd + 4;             /* a partial record: values, max, sum, two pads */

    /* LT (the layer table, a.L) is a restrict, read-only kernel argument: its uniform reads are scalar loads
       (counted by lgkmcnt), so reading a descriptor never waits for the workers' weight loads in flight. */
    auto fl = [&](int l, int ph) { return a.flags + ((size_t)l * STEP_PHASES + ph) * 256; };

    for (int l = 0; l < a.NL; l++) {
        /* the lane's index, passed through an opaque move at every phase: what is derived from it is computed in the
           phase that uses it, rather than hoisted or shared across phases and held in registers throughout */
        int lane, sub, al, rq_j, rq_s, lp;
        /* lp: the layer index, passed through an opaque move at every phase like the lane's, so each phase reads the
           layer descriptors it needs (scalar loads) instead of every descriptor staying in registers all layer */
#define FRESH_LANE()                                                       \
    do {                                                                   \
        asm volatile("v_mov_b32 %0, %1" : "=v"(lane) : "v"(lane0));        \
        lp = l;                                                            \
        asm volatile("" : "+s"(lp));                                       \
        sub = lane / LPR;                                                  \
        al = lane % LPR;                                                   \
        rq_j = 4 * (lane >> 4) + ((lane >> 2) & 3);                        \
        rq_s = lane & 3;                                                   \
    } while (0)
        FRESH_LANE();
#define L (LT[lp])
        /* ---- a worker's weight loads for its share of a phase (issued right after the phase's inputs are in LDS;
           each phase's registers are its own) ---- */
        auto load_qkv = [&](int li, qraw (&p0)[MAX0][SPL]) {
            const step_layer& Ld = LT[li];
    #pragma unroll
            for (int i = 0; i < MAX0; i++) {
                const int u = gw + GW * i, row = u * RPW + sub;
                if (row < R0) {
                    const qmat& m = row < qd ? Ld.q : row < qd + kd ? Ld.k : Ld.v;
                    const int r = row < qd ? row : row < qd + kd ? row - qd : row - qd - kd;
    #pragma unroll
                    for (int j = 0; j < SPL; j++) {
                        if (row < qd + kd) slice_load<DQK>(m, 0, r, al + LPR * j, p0[i][j]);
                        else slice_load<DV>(m, 0, r, al + LPR * j, p0[i][j]);
                    }
                }
            }
        };
        auto load_attn = [&](int l, float2 (&pk)[ATTN_PF], float2 (&pv)[ATTN_PF]) {
            if (b >= U1) return;
            const int h = b / nch, c = b % nch, t0 = c * CHP, t1 = min(t0 + CHP, npos), te = min(t0 + SUB, t1);
            const float* kc = LT[l].k_cache + (size_t)seq * a.seq_stride + (size_t)h * hd;
            const float* vc = LT[l].v_cache + (size_t)seq * a.seq_stride + (size_t)h * hd;
    #pragma unroll
            for (int i = 0; i < ATTN_PF; i++) {
                const int t = t0 + wk + NW * i;
                if (t < te && t != pos && 2 * lane < hd) {
                    pk[i] = gld<float2>(kc + (size_t)t * kd + 2 * lane);
                    pv[i] = gld<float2>(vc + (size_t)t * kd + 2 * lane);
                }
            }
        };
        auto load_o = [&](int l, qraw (&po)[MAXO]) {
            const qmat& m = LT[l].o;
            const int hp = b % CG, rgi = b / CG, q8 = lane >> 3, t = hp * 8 + (lane & 7);
    #pragma unroll
            for (int i = 0; i < MAXO; i++) {
                const int pass = wk + NW * i, r = pass * 8 + q8;
                if (r < RR) slice_load<DO>(m, 0, rgi * RR + r, t, po[i]);
            }
        };
        /* One router row a worker wave; the row's sixteen chains (chain j: columns j, j + 16, ...) each split in
           four consecutive quarters over four lanes: lane 16q + 4jj + s holds quarter s of chain 4q + jj. */
        auto load_router = [&](int l, float (&pr)[HS / 2]) {
            if (gw >= a.E) return;
            const float* wr = LT[l].router + (size_t)gw * H + rq_j + 16 * (HS / 2) * rq_s;
    #pragma unroll
            for (int m = 0; m < HS / 2; m++) pr[m] = gld<float>(wr + 16 * m);
        };
        auto load_down = [&](int l, qraw (&pd)[MAXD][IPL]) {
            const qmat& m = LT[l].down;
    #pragma unroll
            for (int i = 0; i < MAXD; i++) {
                const int r = gw + GW * i;
                if (r < H) {
    #pragma unroll
                    for (int j = 0; j < IPL; j++) {
                        const int it = lane + 64 * j;
                        if (it < N6) {
                            const int k = it / S6, t = it - k * S6;
                            slice_load<DDN>(m, srt.chosen[k], r, t, pd[i][j]);
                        }
                    }
                }
            }
        };

        /* the control wave's stop: every wave of the block returns at the same barrier */
        auto go = [&](bool ok) {
            if (ctl && lane == 0) sgo = ok ? 1 : 0;
        };

        const bool last = l + 1 == a.NL;
        /* the phase timeline of one block, for measurement */
        auto stamp = [&](int i) {
            if (a.trace && ctl && b == a.trace_block && lane == 0)
                a.trace[(size_t)l * STEP_TRACE_PER_LAYER + i] = __builtin_amdgcn_s_memrealtime();
        };
        if constexpr (ATT) {
            /* ================= QKV ================= */
            FRESH_LANE();
            stamp(0);
            if (ctl) {
                bool ok = true;
                if (l == 0) {
                    for (int c = lane; c < H; c += 64) sx[c] = widen_one(a.embed, 0, token, c);
                } else {
                    ok = wait_flags(fl(l - 1, STEP_DOWN), NB, ep, a.abort_word, lane, a.poll_nap);
                    const rsrc_t rx = rsrc(a.xout + (size_t)(l - 1) * H, H * 4);
                    for (int i = lane; i < H / 4; i += 64) reinterpret_cast<f4*>(sx)[i] = ld4c(rx, i * 16);
                }
                __builtin_amdgcn_wave_barrier();
                norm_exact(sx, L.attn_norm, sxn, H, a.eps, lane);
                go(ok);
                stamp(1);
            }
            bar();
            if (!sgo) return;
            if (!ctl) {
                qraw p0[MAX0][SPL] = {}; /* every register defined: no value of an earlier layer stays live */
                load_qkv(lp, p0);
#pragma unroll
                for (int i = 0; i < MAX0; i++) {
                    const int u = gw + GW * i, row = u * RPW + sub;
                    if (u * RPW < R0) {
                        __builtin_amdgcn_sched_barrier(0); /* one unit's activations in registers at a time */
                        float p = 0.f;
#pragma unroll
                        for (int j = 0; j < SPL; j++) {
                            xslice xs;
                            if (u * RPW < qd + kd) {
                                lds_xslice(DQK, al + LPR * j, sxn, xs);
                                p += slice_dot<DQK>(p0[i][j], al + LPR * j, xs);
                            } else {
                                lds_xslice(DV, al + LPR * j, sxn, xs);
                                p += slice_dot<DV>(p0[i][j], al + LPR * j, xs);
                            }
                        }
                        p = row_sum<LPR>(p);
                        if (al == LPR - 1 && row < R0) sout[(wk * MAX0 + i) * RPW + sub] = p;
                    }
                }
            }
            bar();
            if (ctl) {
                const rsrc_t rq = rsrc(a.qkv + (size_t)l * a.s_qkv, R0 * 4);
                for (int s = lane; s < NW * MAX0 * RPW; s += 64) {
                    const int w = s / (MAX0 * RPW), i = (s / RPW) % MAX0, sb = s % RPW;
                    const int row = (b * NW + w + GW * i) * RPW + sb;
                    if (row < R0) st1c(sout[s], rq, row * 4);
                }
                set_flag(fl(l, STEP_QKV), b, ep, lane);
                stamp(2);
            }

            /* ================= ATT ================= */
            FRESH_LANE();
            float* Ks = W;                          /* [SUB][hd + 4] */
            float* Vs = Ks + SUB * (hd + 4);        /* [SUB][hd + 4] */
            float* qs = Vs + SUB * (hd + 4);        /* [G][hd] */
            float* ps = qs + 8 * 128;               /* [G][SUB] */
            const int h = b / (nch ? nch : 1), c = b % (nch ? nch : 1), t0 = c * CHP, t1 = min(t0 + CHP, npos);
            const bool unit = b < U1;
            stamp(3);
            if (ctl) {
                bool ok = wait_flags(fl(l, STEP_QKV), NB, ep, a.abort_word, lane, a.poll_nap);
                if (unit) {
                    const rsrc_t rq = rsrc(a.qkv + (size_t)l * a.s_qkv, R0 * 4);
                    for (int i = lane; i < G * hd / 4; i += 64) reinterpret_cast<f4*>(qs)[i] = ld4c(rq, (h * G * hd) * 4 + i * 16);
                    float* kn = ps;             /* the new k and v, staged */
                    float* vn = ps + hd;
                    for (int i = lane; i < hd; i += 64) {
                        kn[i] = ld1c(rq, (qd + h * hd + i) * 4);
                        vn[i] = ld1c(rq, (qd + kd + h * hd + i) * 4);
                    }
                    __builtin_amdgcn_wave_barrier();
                    const float* cs = a.cos_tab + (size_t)pos * (hd / 2);
                    const float* sn = a.sin_tab + (size_t)pos * (hd / 2);
                    for (int g = 0; g < G; g++) head_norm_rope(qs + g * hd, L.q_norm, cs, sn, hd, a.eps, lane);
                    head_norm_rope(kn, L.k_norm, cs, sn, hd, a.eps, lane);
                    if (pos >= t0 && pos < t1) {
                        /* this unit holds the new position: its k and v into the cache (for later steps) and LDS */
                        float* kc = L.k_cache + (size_t)seq * a.seq_stride + (size_t)pos * kd + (size_t)h * hd;
                        float* vc = L.v_cache + (size_t)seq * a.seq_stride + (size_t)pos * kd + (size_t)h * hd;
                        for (int i = lane; i < hd; i += 64) {
                            kc[i] = kn[i];
                            vc[i] = vn[i];
                            if (pos - t0 < SUB) {
                                Ks[(pos - t0) * (hd + 4) + i] = kn[i];
                                Vs[(pos - t0) * (hd + 4) + i] = vn[i];
                            }
                        }
                    }
                }
                go(ok);
                stamp(4);
            }
            bar();
            if (!sgo) return;
            if (!ctl && unit) {
                const int te = min(t0 + SUB, t1);
                float2 pk[ATTN_PF] = {}, pv[ATTN_PF] = {};
                load_attn(lp, pk, pv);
#pragma unroll
                for (int i = 0; i < ATTN_PF; i++) {
                    const int t = t0 + wk + NW * i;
                    if (t < te && t != pos && 2 * lane < hd) {
                        *reinterpret_cast<float2*>(Ks + (t - t0) * (hd + 4) + 2 * lane) = pk[i];
                        *reinterpret_cast<float2*>(Vs + (t - t0) * (hd + 4) + 2 * lane) = pv[i];
                    }
                }
            }
            bar();
            if (!ctl && unit) {
                const float scale = 1.0f / sqrtf((float)hd);
                /* the worker's heads: g = wk, wk + NW */
                float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
                float2 o_run[2] = {{0.f, 0.f}, {0.f, 0.f}};
                const float* kcb = L.k_cache + (size_t)seq * a.seq_stride + (size_t)h * hd;
                const float* vcb = L.v_cache + (size_t)seq * a.seq_stride + (size_t)h * hd;
                for (int s0 = t0; s0 < t1; s0 += SUB) {
                    const int n = min(SUB, t1 - s0);
                    if (s0 > t0) {
                        /* a later pass over the unit: its rows staged here (none prefetched); the control wave meets
                           these two barriers too */
                        bar(); /* every worker is past the previous pass's reads */
                        for (int t = s0 + wk; t < s0 + n; t += NW) {
                            if (2 * lane < hd) {
                                const float2 kk = t == pos ? make_float2(ps[2 * lane], ps[2 * lane + 1])
                                                           : gld<float2>(kcb + (size_t)t * kd + 2 * lane);
                                const float2 vv = t == pos ? make_float2(ps[hd + 2 * lane], ps[hd + 2 * lane + 1])
                                                           : gld<float2>(vcb + (size_t)t * kd + 2 * lane);
                                *reinterpret_cast<float2*>(Ks + (t - s0) * (hd + 4) + 2 * lane) = kk;
                                *reinterpret_cast<float2*>(Vs + (t - s0) * (hd + 4) + 2 * lane) = vv;
                            }
                        }
                        bar();
                    }
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int g = wk + NW * q;
                        if (g < G) {
                            float s = -INFINITY;
                            if (lane < n) {
                                const float4* kr = reinterpret_cast<const float4*>(Ks + lane * (hd + 4));
                                const float4* qr = reinterpret_cast<const float4*>(qs + g * hd);
                                float acc = 0.f;
                                for (int d0 = 0; d0 < hd / 4; d0 += 8) {
                                    /* eight float4 of the key and the query from LDS at once, then the FMAs */
                                    float4 kk[8], qq[8];
#pragma unroll
                                    for (int i = 0; i < 8; i++) { kk[i] = kr[d0 + i]; qq[i] = qr[d0 + i]; }
#pragma unroll
                                    for (int i = 0; i < 8; i++) {
                                        acc = fmaf(qq[i].x, kk[i].x, acc); acc = fmaf(qq[i].y, kk[i].y, acc);
                                        acc = fmaf(qq[i].z, kk[i].z, acc); acc = fmaf(qq[i].w, kk[i].w, acc);
                                    }
                                }
                                s = acc * scale;
                            }
                            const float mx = fmaxf(m_run[q], wave_max_dpp(s));
                            const float p = lane < n ? expf(s - mx) : 0.f;
                            const float corr = expf(m_run[q] - mx);
                            l_run[q] = l_run[q] * corr + wave_sum_dpp(p);
                            o_run[q].x *= corr;
                            o_run[q].y *= corr;
                            m_run[q] = mx;
                            const int dl = 2 * lane < hd ? 2 * lane : 0;
                            for (int t0p = 0; t0p < n; t0p += 8) {
                                /* eight positions' values from LDS at once; positions past n weigh 0 */
                                float2 vv[8];
#pragma unroll
                                for (int i = 0; i < 8; i++) vv[i] = *reinterpret_cast<const float2*>(Vs + (t0p + i) * (hd + 4) + dl);
#pragma unroll
                                for (int i = 0; i < 8; i++) {
                                    const int t = t0p + i;
                                    const float pt = t < n ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), t)) : 0.0f;
                                    const float2 v = t < n ? vv[i] : make_float2(0.f, 0.f);
                                    o_run[q].x = fmaf(pt, v.x, o_run[q].x);
                                    o_run[q].y = fmaf(pt, v.y, o_run[q].y);
                                }
                            }
                        }
                    }
                }
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int g = wk + NW * q;
                    if (g < G) {
                        float* rec = sout + g * prec;
                        if (2 * lane < hd) *reinterpret_cast<float2*>(rec + 2 * lane) = o_run[q];
                        if (lane == 0) {
                            rec[hd] = m_run[q];
                            rec[hd + 1] = l_run[q];
                        }
                    }
                }
            }
            if (ctl && unit)
                for (int s0 = t0 + SUB; s0 < t1; s0 += SUB) {
                    bar();
                    bar();
                }
            bar();
            if (ctl) {
                if (unit) {
                    const rsrc_t rp = rsrc(a.part + (size_t)l * a.s_part, (uint32_t)(U1 * G * prec * 4));
                    for (int i = lane; i < (int)(G * prec / 4); i += 64)
                        st4c(reinterpret_cast<const f4*>(sout)[i], rp, (uint32_t)((size_t)b * G * prec * 4 + i * 16));
                }
                set_flag(fl(l, STEP_ATT), b, ep, lane);
                stamp(5);
            }

            /* ================= O ================= */
            FRESH_LANE();
            {
                const int hp = b % CG, rgi = b / CG;
                float* sp = W;                          /* [HPC][nch][prec] */
                float* satt = W + HPC * nch * prec;     /* [256] */
                stamp(6);
                if (ctl) {
                    const bool ok = wait_flags(fl(l, STEP_ATT), NB, ep, a.abort_word, lane, a.poll_nap);
                    const rsrc_t rp = rsrc(a.part + (size_t)l * a.s_part, (uint32_t)(U1 * G * prec * 4));
                    const int per = (int)(prec / 4);
                    for (int s = lane; s < HPC * nch * per; s += 64) {
                        const int i = s / (nch * per), cc = (s / per) % nch, f = s % per;
                        const int hq = hp * HPC + i, hh = hq / G, g = hq % G;
                        const size_t rec = ((size_t)(hh * nch + cc) * G + g) * prec;
                        reinterpret_cast<f4*>(sp)[s] = ld4c(rp, (uint32_t)(rec * 4 + f * 16));
                    }
                    go(ok);
                    stamp(7);
                }
                bar();
                if (!sgo) return;
                qraw po[MAXO] = {};
                if (!ctl) load_o(lp, po);
                if (!ctl && wk < HPC) {
                    /* merge head hp * HPC + wk: the chunks' maxima, then the scaled sums */
                    const float* base = sp + (size_t)wk * nch * prec;
                    /* the chunks' maxima and sums, a chunk a lane, then the scale of each chunk in every lane */
                    float mc = -INFINITY, lc = 0.f;
                    if (lane < nch) {
                        mc = base[lane * prec + hd];
                        lc = base[lane * prec + hd + 1];
                    }
                    const float M = wave_max_dpp(mc);
                    const float scl = lane < nch ? expf(mc - M) : 0.f;
                    const float Lsum = wave_sum_dpp(lc * scl);
                    float2 o = {0.f, 0.f};
                    const int dl = 2 * lane < hd ? 2 * lane : 0;
                    for (int c0 = 0; c0 < nch; c0 += 8) {
                        float2 vv[8];
#pragma unroll
                        for (int i = 0; i < 8; i++) vv[i] = *reinterpret_cast<const float2*>(base + (c0 + i) * prec + dl);
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            const int cc = c0 + i;
                            const float sc = cc < nch ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scl), cc)) : 0.0f;
                            const float2 v = cc < nch ? vv[i] : make_float2(0.f, 0.f);
                            o.x = fmaf(v.x, sc, o.x);
                            o.y = fmaf(v.y, sc, o.y);
                        }
                    }
                    if (2 * lane < hd) {
                        satt[wk * hd + 2 * lane] = o.x / Lsum;
                        satt[wk * hd + 2 * lane + 1] = o.y / Lsum;
                    }
                }
                bar();
                if (!ctl) {
                    const qmat& m = L.o;
                    const int q8 = lane >> 3, t = hp * 8 + (lane & 7);
                    xslice xs; /* the same slice of the heads' outputs for every row */
                    lds_xslice(DO, t, satt - hp * 256, xs);
#pragma unroll
                    for (int i = 0; i < MAXO; i++) {
                        const int pass = wk + NW * i, r = pass * 8 + q8;
                        if (pass * 8 < RR) {
                            float p = slice_dot<DO>(po[i], t, xs);
                            p = row_sum<8>(p);
                            if ((lane & 7) == 7 && r < RR) sout[r] = p;
                        }
                    }
                }
                bar();
                if (ctl) {
                    const rsrc_t ro = rsrc(a.opart + (size_t)l * a.s_opart, (uint32_t)(CG * H * 4));
                    for (int r = lane; r < RR; r += 64) st1c(sout[r], ro, (uint32_t)((hp * H + rgi * RR + r) * 4));
                    if (rgi == 0) {
                        const rsrc_t rt = rsrc(a.att + (size_t)l * a.s_att, (uint32_t)(qd * 4));
                        for (int i = lane; i < 256; i += 64) st1c(satt[i], rt, (uint32_t)((hp * 256 + i) * 4));
                    }
                    set_flag(fl(l, STEP_O), b, ep, lane);
                    stamp(8);
                }
            }
        }

        /* ================= ROUTE (blocks 0 .. RB - 1) ================= */
        FRESH_LANE();
        if (b < RB) {
            stamp(9);
            if (ctl) {
                bool ok = true;
                if constexpr (ATT) {
                    ok = wait_flags(fl(l, STEP_O), NB, ep, a.abort_word, lane, a.poll_nap);
                } else if (l == 0) {
                    for (int i = lane; i < H / 4; i += 64) reinterpret_cast<float4*>(sx)[i] = reinterpret_cast<const float4*>(a.x0)[i];
                } else {
                    ok = wait_flags(fl(l - 1, STEP_DOWN), NB, ep, a.abort_word, lane, a.poll_nap);
                    const rsrc_t rx = rsrc(a.xout + (size_t)(l - 1) * H, H * 4);
                    for (int i = lane; i < H / 4; i += 64) reinterpret_cast<f4*>(sx)[i] = ld4c(rx, i * 16);
                }
                go(ok);
            }
            bar();
            if (!sgo) return;
            float pr[HS / 2] = {}; /* a router lane's quarter of one chain: H / 64 weights */
            if (!ctl) load_router(lp, pr);
            if constexpr (ATT) {
                /* the residual after attention, x + o, o's column splits added in order; each wave a slice */
                const rsrc_t ro = rsrc(a.opart + (size_t)l * a.s_opart, (uint32_t)(CG * H * 4));
                for (int c4 = wv * 64 + lane; c4 < H / 4; c4 += (NW + 1) * 64) {
                    f4 o = ld4c(ro, c4 * 16);
                    for (int hp = 1; hp < CG; hp++) o += ld4c(ro, (uint32_t)((hp * H) * 4 + c4 * 16));
                    f4 x = reinterpret_cast<f4*>(sx)[c4];
                    reinterpret_cast<f4*>(sx)[c4] = x + o;
                }
                bar();
            }
            if (ctl) {
                stamp(10);
                norm_exact(sx, L.mlp_norm, sxn, H, a.eps, lane);
            }
            bar();
            if (!ctl) {
                /* the row's sixteen chains in the reference's order (engine/src/ops.c:212-229): each chain's four
                   quarters in turn, the running sum handed one lane on between quarters; then the AVX2 fold */
                float xq[HS / 2]; /* the lane's quarter of the normed row, from LDS at once */
#pragma unroll
                for (int m = 0; m < HS / 2; m++) xq[m] = sxn[16 * (rq_s * (HS / 2) + m) + rq_j];
                float acc = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (rq_s == q) {
#pragma unroll
                        for (int m = 0; m < HS / 2; m++) acc = fmaf(pr[m], xq[m], acc);
                    }
                    if (q < 3) {
                        const float prev = dpp_f<DPP_ROW_SHR(1), 0xf, 0xf>(acc, 0.0f);
                        if (rq_s == q + 1) acc = prev;
                    }
                }
                float ch[16];
#pragma unroll
                for (int j = 0; j < 16; j++)
                    ch[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 16 * (j >> 2) + 4 * (j & 3) + 3));
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = ch[j] + ch[j + 8];
                const float logit = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
                if (lane == 0 && gw < a.E) sout[wk] = logit;
            }
            bar();
            if (ctl) {
                const rsrc_t rl = rsrc(a.logits + (size_t)l * a.s_logits, a.E * 4);
                for (int s = lane; s < NW; s += 64) {
                    const int rrow = b * NW + s;
                    if (rrow < a.E) st1c(sout[s], rl, rrow * 4);
                }
                if (b == 0) {
                    const rsrc_t rm = rsrc(a.xmid + (size_t)l * a.s_xmid, H * 4);
                    for (int i = lane; i < H / 4; i += 64) st4c(reinterpret_cast<const f4*>(sx)[i], rm, i * 16);
                }
                set_flag(fl(l, STEP_ROUTE), b, ep, lane);
                stamp(11);
            }
        }

        /* ================= IN ================= */
        FRESH_LANE();
        stamp(12);
        if (ctl) {
            const bool ok = wait_flags(fl(l, STEP_ROUTE), RB, ep, a.abort_word, lane, a.poll_nap);
            const rsrc_t rl = rsrc(a.logits + (size_t)l * a.s_logits, a.E * 4);
            for (int e = lane; e < a.E; e += 64) slg[e] = ld1c(rl, e * 4);
            const rsrc_t rm = rsrc(a.xmid + (size_t)l * a.s_xmid, H * 4);
            for (int i = lane; i < H / 4; i += 64) reinterpret_cast<f4*>(sx)[i] = ld4c(rm, i * 16);
            __builtin_amdgcn_wave_barrier();
            norm_exact(sx, L.mlp_norm, sxn, H, a.eps, lane);
            __shared__ float scratch[ROUTE_E_MAX];
            wave_route(slg, a.E, a.K, a.renorm, &srt, scratch);
            __builtin_amdgcn_wave_barrier();
            if (b == 0 && lane < (int)(sizeof(route_out) / 4)) {
                route_out* dst = last ? a.rt_last : a.rt_layers + l;
                reinterpret_cast<int32_t*>(dst)[lane] = reinterpret_cast<const int32_t*>(&srt)[lane];
            }
            go(ok);
            stamp(13);
        }
        bar();
        if (!sgo) return;
        if (!ctl) {
            const qmat& mg = L.gate;
            const qmat& mu = L.up;
            const int units = a.K * a.I;
            qraw gq[MAX5][SPL] = {}, uq[MAX5][SPL] = {};
#pragma unroll
            for (int i = 0; i < MAX5; i++) {
                const int u = (gw + GW * i) * RPW + sub;
                if (u < units) {
                    const int k = u / a.I, r = u - k * a.I, e = srt.chosen[k];
#pragma unroll
                    for (int j = 0; j < SPL; j++) {
                        slice_load<DGU>(mg, e, r, al + LPR * j, gq[i][j]);
                        slice_load<DGU>(mu, e, r, al + LPR * j, uq[i][j]);
                    }
                }
            }
            xslice xs[SPL]; /* the lane's slices of the normed token: the same for every unit */
#pragma unroll
            for (int j = 0; j < SPL; j++) lds_xslice(DGU, al + LPR * j, sxn, xs[j]);
#pragma unroll
            for (int i = 0; i < MAX5; i++) {
                const int u0 = (gw + GW * i) * RPW, u = u0 + sub;
                if (u0 < units) {
                    float pg = 0.f, pu = 0.f;
#pragma unroll
                    for (int j = 0; j < SPL; j++) {
                        pg += slice_dot<DGU>(gq[i][j], al + LPR * j, xs[j]);
                        pu += slice_dot<DGU>(uq[i][j], al + LPR * j, xs[j]);
                    }
                    pg = row_sum<LPR>(pg);
                    pu = row_sum<LPR>(pu);
                    if (al == LPR - 1 && u < units) sout[(wk * MAX5 + i) * RPW + sub] = silu_mul(pg, pu);
                }
            }
        }
        bar();
        if (ctl) {
            const int units = a.K * a.I;
            const rsrc_t ra = rsrc(a.act + (size_t)l * a.s_act, units * 4);
            for (int s = lane; s < NW * MAX5 * RPW; s += 64) {
                const int w = s / (MAX5 * RPW), i = (s / RPW) % MAX5, sb = s % RPW;
                const int u = (b * NW + w + GW * i) * RPW + sb;
                if (u < units) st1c(sout[s], ra, u * 4);
            }
            set_flag(fl(l, STEP_IN), b, ep, lane);
            stamp(14);
        }

        /* ================= DOWN ================= */
        FRESH_LANE();
        float* sact = W; /* [K][I] */
        stamp(15);
        if (ctl) {
            const bool ok = wait_flags(fl(l, STEP_IN), NB, ep, a.abort_word, lane, a.poll_nap);
            const int units = a.K * a.I;
            const rsrc_t ra = rsrc(a.act + (size_t)l * a.s_act, units * 4);
            for (int i = lane; i < units / 4; i += 64) reinterpret_cast<f4*>(sact)[i] = ld4c(ra, i * 16);
            go(ok);
            stamp(16);
        }
        bar();
        if (!sgo) return;
        if (!ctl) {
            qraw pd[MAXD][IPL] = {};
            load_down(lp, pd);
            const qmat& m = L.down;
#pragma unroll
            for (int i = 0; i < MAXD; i++) {
                const int r = gw + GW * i;
                if (gw + GW * i < H) {
                    float p = 0.f;
#pragma unroll
                    for (int j = 0; j < IPL; j++) {
                        const int it = lane + 64 * j;
                        if (it < N6) {
                            const int k = it / S6, t = it - k * S6;
                            __builtin_amdgcn_sched_barrier(0); /* one item's activations in registers at a time */
                            xslice xs;
                            lds_xslice(DDN, t, sact + (size_t)k * a.I, xs);
                            p = fmaf(srt.cw[k], slice_dot<DDN>(pd[i][j], t, xs), p);
                        }
                    }
                    p = row_sum<64>(p);
                    if (lane == 63) sout[wk * MAXD + i] = sx[r] + p;
                }
            }
        }
        bar();
        if (ctl) {
            const rsrc_t rx = rsrc(a.xout + (size_t)l * H, H * 4);
            const rsrc_t rf = rsrc(a.x_final, H * 4);
            for (int s = lane; s < NW * MAXD; s += 64) {
                const int w = s / MAXD, i = s % MAXD, r = b * NW + w + GW * i;
                if (r < H) {
                    st1c(sout[s], rx, r * 4);
                    if (last) st1c(sout[s], rf, r * 4);
                }
            }
            set_flag(fl(l, STEP_DOWN), b, ep, lane);
            stamp(17);
        }
    }
}

#undef FRESH_LANE
#undef L

/* ---- host side ---- */

size_t step_lds_bytes(int H, int hd, int nh, int nkv, int K, int I, int nb) {
    size_t w = 0;
    if (nh) {
        const int G = nh / nkv;
        const size_t att = 2 * (size_t)SUB * (hd + 4) + 8 * 128 + (size_t)8 * SUB;
        const int per_head = std::min(64, nb / nkv > 0 ? nb / nkv : 1);
        const size_t merge = (size_t)(256 / hd) * per_head * (hd + 4) + 256;
        w = att > merge ? att : merge;
        (void)G;
    }
    const size_t act = (size_t)K * I;
    if (act > w) w = act;
    return (2 * (size_t)H + STEP_OUT + w) * sizeof(float);
}

/* The instantiations (hidden slices, gate/up dtype, down dtype, down slices a lane) the library carries:
   Qwen3-30B-A3B's shape (configs 1-3), OLMoE-1B-7B's (config 0), and the test models' hidden 512 Q4_K_M. */
#define STEP_FOREACH(X)                                                                                     \
    X(64, VITNA_DTYPE_Q4_K, VITNA_DTYPE_Q6_K, 3, true, VITNA_DTYPE_Q4_K, VITNA_DTYPE_Q6_K, VITNA_DTYPE_Q4_K) \
    X(64, VITNA_DTYPE_Q4_K, VITNA_DTYPE_Q6_K, 3, false, 0, 0, 0)                                            \
    X(64, VITNA_DTYPE_Q8_0, VITNA_DTYPE_Q8_0, 4, false, 0, 0, 0)                                            \
    X(16, VITNA_DTYPE_Q4_K, VITNA_DTYPE_Q6_K, 1, true, VITNA_DTYPE_Q4_K, VITNA_DTYPE_Q6_K, VITNA_DTYPE_Q4_K)

/* the attention dtypes (q and k, v, o) of a model; 0 for a model without attention */
static const void* step_fn(int H, int dgu, int ddn, int K, int I, bool att, int dqk, int dv, int dout) {
    const int ipl = (K * (I / 32) + 63) / 64;
#define STEP_MATCH(hs, gu, dn, ip, at, qk, v, o)                                                                      \
    if (H / 32 == hs && dgu == gu && ddn == dn && ipl == ip && att == at && (!at || (dqk == qk && dv == v && dout == o))) \
        return (const void*)step_kernel<hs, gu, dn, ip, at, qk, v, o>;
    STEP_FOREACH(STEP_MATCH)
#undef STEP_MATCH
    return nullptr;
}

/* Whether the persistent step takes this model (else the per-layer kernels serve it), with the reason. */
const char* step_unsupported(int H, int I, int E, int K, int nh, int nkv, int hd, int nb, int dt_q, int dt_k, int dt_v, int dt_o, int dt_gu,
                             int dt_dn) {
    if (H % 256) return "hidden width";
    if (nb < 8 || nb > 256) return "compute units";
    if (I % 32 || (K * I) % 4) return "expert width";
    if (nh && dt_q != dt_k) return "q and k of different dtypes";
    if (!step_fn(H, dt_gu, dt_dn, K, I, nh != 0, dt_q, dt_v, dt_o)) return "a shape or dtype mix the persistent step is not built for";
    const int HS = H / 32, GW = nb * NW, LPR = HS < 64 ? HS : 64, RPW = 64 / LPR;
    if ((size_t)K * I > (size_t)MAX5 * GW * RPW) return "expert rows";
    if (H > MAXD * GW) return "residual rows";
    if (E > ROUTE_E_MAX || K > ROUTE_K_MAX) return "experts";
    if ((E + NW - 1) / NW > nb) return "router rows";
    if (nh) {
        const int qd = nh * hd, kd = nkv * hd, G = nh / nkv;
        if (hd != 64 && hd != 128) return "head width";
        if (G > 8 || G * hd > 8 * 128) return "query heads a key-value head";
        if (qd % 256 || nb % (qd / 256) || H % (nb / (qd / 256))) return "o-projection split";
        const int RR = H / (nb / (qd / 256));
        if ((RR + 7) / 8 > MAXO * NW || RR > STEP_OUT) return "o-projection rows";
        if (dt_o != VITNA_DTYPE_Q4_K && dt_o != VITNA_DTYPE_Q6_K && dt_o != VITNA_DTYPE_Q8_0) return "o-projection dtype";
        if ((qd + 2 * kd + RPW - 1) / RPW > MAX0 * GW) return "q/k/v rows";
        if (nb / nkv < 1) return "key-value heads";
        if ((size_t)G * (hd + 4) > STEP_OUT) return "attention records";
    }
    if (step_lds_bytes(H, hd, nh, nkv, K, I, nb) > 150 * 1024) return "LDS";
    return nullptr;
}

hipError_t launch_step(const step_args& a, const int* dts, hipStream_t s) {
    const void* fn = step_fn(a.H, dts[0], dts[1], a.K, a.I, a.attention != 0, dts[2], dts[3], dts[4]);
    if (!fn) return hipErrorInvalidValue;
    const size_t lds = step_lds_bytes(a.H, a.hd, a.nh, a.nkv, a.K, a.I, a.nb);
    /* the functions whose dynamic LDS limit is already raised: shared by every model of the process, so
       guarded against two host threads launching at once */
    static std::mutex attr_mu;
    static const void* attr_done[8];
    static size_t attr_lds[8];
    std::lock_guard<std::mutex> lock(attr_mu);
    int slot = 0;
    while (slot < 8 && attr_done[slot] && attr_done[slot] != fn) slot++;
    if (slot == 8 || attr_done[slot] != fn || attr_lds[slot] < lds) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        if (slot < 8) {
            attr_done[slot] = fn;
            attr_lds[slot] = lds;
        }
    }
    const step_layer* L = a.L;
    void* args[] = {const_cast<step_args*>(&a), &L};
    return hipLaunchCooperativeKernel(fn, dim3(a.nb), dim3(64 * (NW + 1)), args, (unsigned)lds, s);
}
