/**
 * route_impl.h - The device form of the reference's routing rule and SwiGLU,
 * shared by the decode kernels (kernels_decode.hip) and the persistent
 * decode step (kernels_step.hip).
 */

#ifndef VITNA_ROUTE_IMPL_H
#define VITNA_ROUTE_IMPL_H

#include "vitna_kernels.h"

/* The reference's routing (engine/src/model.c:626-703) of one token by one
   wave: the K largest of E logits, largest first, the lower index first
   between equals; the chosen sorted by id; softmax weights over every
   expert; renormalized over the chosen, summed largest first, when renorm.
   Lanes write *o. slg: ROUTE_E_MAX floats of LDS.

   Without NaNs each pass of argmax is a wave-wide maximum of order-preserving
   32-bit keys (-0 keyed as +0, since the passes compare with >) followed by
   the lowest index holding it. With a NaN among the logits the passes are run as the
   reference runs them (a NaN where a pass starts is kept, since x > NaN is
   false; a later one never wins). */

__device__ __forceinline__ uint32_t order_key(float v) {
    uint32_t u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0; /* -0 == +0 */
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* The largest of the wave's values, in every lane: row shifts then row broadcasts (DPP), read from lane 63. */
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false)); /* row_shr:1 */
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false)); /* row_shr:2 */
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false)); /* row_shr:4 */
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false)); /* row_shr:8 */
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xa, 0xf, false)); /* row_bcast:15 */
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xc, 0xf, false)); /* row_bcast:31 */
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

/* order_key's inverse (a key from -0 comes back as +0, which exp(l - max) cannot tell apart). */
__device__ __forceinline__ float key_value(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k); }

/* NS logits a lane (E <= 64 NS). */
template <int NS>
__device__ __forceinline__ void wave_route_n(const float* __restrict__ lg_in, int E, int K, int renorm, route_out* o, float* slg) {
    const int lane = threadIdx.x & 63;
    float lg[NS];
    bool nan = false;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int e = lane + 64 * i;
        lg[i] = e < E ? lg_in[e] : -INFINITY;
        nan |= e < E && lg[i] != lg[i];
    }
    int e_mine = 0;       /* lane k < K: the k-th chosen, largest first */
    float v_mine = 0.0f;  /* and its logit */
    float mx;             /* the max as the CPU scans it */
    if (__any(nan)) {
        __shared__ int chosen_s[ROUTE_K_MAX];
#pragma unroll
        for (int i = 0; i < NS; i++)
            if (lane + 64 * i < E) slg[lane + 64 * i] = lg[i];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        unsigned taken = 0;
        for (int k = 0; k < K; k++) {
            int first = 0x7fffffff, bi = 0x7fffffff;
            float bv = 0.0f;
#pragma unroll
            for (int i = 0; i < NS; i++) {
                const int e = lane + 64 * i;
                if (e < E && !(taken >> i & 1)) {
                    first = min(first, e);
                    const float v = lg[i];
                    if (v == v && (bi == 0x7fffffff || v > bv)) { bv = v; bi = e; }
                }
            }
            for (int off = 32; off > 0; off >>= 1) {
                const int of = __shfl_xor(first, off, 64), oi = __shfl_xor(bi, off, 64);
                const float ov = __shfl_xor(bv, off, 64);
                first = min(first, of);
                const bool take = oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi));
                if (take) { bv = ov; bi = oi; }
            }
            const float fv = slg[first];
            const int pick = (fv != fv || bi == 0x7fffffff) ? first : bi;
            if ((pick & 63) == lane) taken |= 1u << (pick >> 6);
            if (lane == 0) chosen_s[k] = pick;
        }
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < NS; i++)
            if (lane + 64 * i < E) m = fmaxf(m, lg[i]);
        mx = wave_max(m);
        if (slg[0] != slg[0]) mx = slg[0]; /* a NaN first stays the max */
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (lane < K) {
            e_mine = chosen_s[lane];
            v_mine = slg[e_mine];
        }
    } else {
        /* K rounds: the largest remaining key over the wave, then the lowest index holding it, which is
           the pass's argmax (strict >: the first of equals wins). Keys of absent or taken experts are 0,
           below every logit's key (order_key(-inf) > 0). The first round's key is the max. */
        uint32_t key[NS];
#pragma unroll
        for (int i = 0; i < NS; i++) key[i] = lane + 64 * i < E ? order_key(lg[i]) : 0u;
        mx = 0.0f;
        for (int k = 0; k < K; k++) {
            uint32_t m = key[0];
#pragma unroll
            for (int i = 1; i < NS; i++) m = max(m, key[i]);
            m = wave_max_u32(m);
            if (k == 0) mx = key_value(m);
            int pick = -1;
#pragma unroll
            for (int i = 0; i < NS; i++) {
                const uint64_t b = __ballot(key[i] == m);
                if (pick < 0 && b) pick = 64 * i + (int)__builtin_ctzll(b);
            }
            float sel = lg[0];
#pragma unroll
            for (int i = 1; i < NS; i++)
                if ((pick >> 6) == i) sel = lg[i];
            const float pv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sel), pick & 63));
            if (lane == k) { e_mine = pick; v_mine = pv; }
#pragma unroll
            for (int i = 0; i < NS; i++)
                if (pick == lane + 64 * i) key[i] = 0u;
        }
    }
    /* softmax over every expert: the sum of exp(l - max) */
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NS; i++)
        if (lane + 64 * i < E) sum += expf(lg[i] - mx);
    sum = wave_sum_dpp(sum);
    const float share = lane < K ? expf(v_mine - mx) / sum : 0.0f;
    float total = 1.0f;
    if (renorm) {
        /* the chosen are largest first, so their shares are too: the total in that order */
        total = 0.0f;
        for (int j = 0; j < K; j++) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(share), j));
    }
    int at = 0; /* where the lane's expert falls in order of id */
    for (int j = 0; j < K; j++) at += __builtin_amdgcn_readlane(e_mine, j) < e_mine;
    if (lane < K) {
        const float wt = renorm ? share / total : share;
        o->chosen[lane] = e_mine;
        o->cw[lane] = wt;
        o->ids[at] = e_mine;
        o->weights[at] = wt;
    }
}

__device__ __forceinline__ void wave_route(const float* __restrict__ lg_in, int E, int K, int renorm, route_out* o, float* slg) {
    if (E <= 64) wave_route_n<1>(lg_in, E, K, renorm, o, slg);
    else if (E <= 128) wave_route_n<2>(lg_in, E, K, renorm, o, slg);
    else if (E <= 256) wave_route_n<4>(lg_in, E, K, renorm, o, slg);
    else wave_route_n<8>(lg_in, E, K, renorm, o, slg);
}


__device__ __forceinline__ float silu_mul(float g, float u) {
    /* engine/src/ops.c:283-288: (g / (1 + exp(-g))) * u */
    const float den = 1.0f + expf(-g);
    return (g / den) * u;
}

#endif
