/**
 * gmma_split.h - The grouped experts' activation split (kernels_gmma.hip),
 * shared with the routing kernel that runs it on its own row.
 *
 * Row r of x (K floats) becomes xs row r: K / 4 chunks of 16 bytes, [4 hi
 * bf16][4 lo bf16] (hi = bf16(x), lo = bf16(x - hi)), and sums row r: K / G
 * floats, the sum of hi + lo over each run of G columns, in column order.
 */
#ifndef VITNA_GMMA_SPLIT_H
#define VITNA_GMMA_SPLIT_H

#include "vitna_hip_internal.h"

/* run g (columns G g .. G g + G - 1) of one row: src the row of x, xs and sums the row's outputs */
template <int G>
__device__ __forceinline__ void gsplit_run(const float* __restrict__ src, int K, int g, uint16_t* __restrict__ xs,
                                           float* __restrict__ sums) {
    const float* p = src + g * G;
    uint16_t* dst = xs + 2 * G * g;
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < G / 4; c++) {
        const float4 v = reinterpret_cast<const float4*>(p)[c];
        const float e[4] = {v.x, v.y, v.z, v.w};
        uint32_t hb[4], lb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const __bf16 h = (__bf16)e[i];
            const __bf16 l = (__bf16)(e[i] - (float)h);
            hb[i] = __builtin_bit_cast(uint16_t, h);
            lb[i] = __builtin_bit_cast(uint16_t, l);
            s += (float)h + (float)l;
        }
        reinterpret_cast<u32x4*>(dst)[c] = u32x4{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16), lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16)};
    }
    sums[g] = s;
}

#endif
