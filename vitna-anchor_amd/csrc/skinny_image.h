/**
 * skinny_image.h - Writing the operand images of the multi-row projections
 * (kernels_skinny.hip), shared by the kernels that produce their inputs.
 *
 * For token tile tt = row / 32 and 256-column superblock b, an image is 2048
 * pieces of 16 bytes: piece ((U * 4 + i) * 2 + hl) * 64 + lane holds 8 bf16,
 * hi (hl 0) or lo (1), of token 32 tt + lane % 32 at the columns of MFMA
 * operand i of unit U for lane half kq = lane / 32:
 *   order A (Q4_K, Q8_0): 64 U + 16 kq + 8 (i % 2) + 32 (i / 2)
 *   order B (Q6_K):       128 (U / 2) + 32 (U % 2) + 8 kq + 16 (i % 2) + 64 (i / 2)
 * Group sums of the split values (hi + lo), as three bf16 pieces, in the lane
 * order of the S-term operand: window w of eight groups, piece p, lane l =
 * token % 32 + 32 (g % 8 / 4): [tt][w][p][64] x 4 bf16, group g % 4 of the
 * four. s32 has one window of 32-column groups a superblock, s16 two windows
 * of 16-column groups.
 */
#ifndef VITNA_SKINNY_IMAGE_H
#define VITNA_SKINNY_IMAGE_H

#include "vitna_hip_internal.h"

/* the eight floats e as bf16 hi and lo (hi = bf16(x), lo = bf16(x - hi)), and the sum of hi + lo in order */
__device__ __forceinline__ void img_split8(const float e[8], u32x4& vh, u32x4& vl, float& sum) {
    uint32_t h[4], lo[4];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const __bf16 h0 = (__bf16)e[2 * k], h1 = (__bf16)e[2 * k + 1];
        const __bf16 l0 = (__bf16)(e[2 * k] - (float)h0), l1 = (__bf16)(e[2 * k + 1] - (float)h1);
        h[k] = __builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        lo[k] = __builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        s += (float)h0 + (float)l0;
        s += (float)h1 + (float)l1;
    }
    vh = u32x4{h[0], h[1], h[2], h[3]};
    vl = u32x4{lo[0], lo[1], lo[2], lo[3]};
    sum = s;
}

/* columns 8 c8 .. 8 c8 + 7 of row `row` (a row K columns wide) into both images (or the one that is not null) */
__device__ __forceinline__ void img_put(u32x4* imga, u32x4* imgb, int row, int K, int c8, const u32x4& vh, const u32x4& vl) {
    const int tt = row >> 5, l = row & 31, b = c8 >> 5, c = 8 * (c8 & 31);
    const size_t base = ((size_t)tt * (K / 256) + b) * 2048;
    if (imga) {
        const int U = c >> 6, r = c & 63, i = ((r >> 5) << 1) | ((r >> 3) & 1), kq = (r >> 4) & 1;
        const size_t q = base + (size_t)((U * 4 + i) * 2) * 64 + l + 32 * kq;
        imga[q] = vh;
        imga[q + 64] = vl;
    }
    if (imgb) {
        const int r = c & 127, U = 2 * (c >> 7) + ((r >> 5) & 1), i = ((r >> 4) & 1) + 2 * (r >> 6), kq = (r >> 3) & 1;
        const size_t q = base + (size_t)((U * 4 + i) * 2) * 64 + l + 32 * kq;
        imgb[q] = vh;
        imgb[q + 64] = vl;
    }
}

/* S as three bf16 pieces, stride apart: S = p0 + p1 + p2 to about 2^-24 relative */
__device__ __forceinline__ void img_bf16x3(float S, uint16_t* d, size_t stride) {
    const __bf16 p0 = (__bf16)S;
    const float r0 = S - (float)p0;
    const __bf16 p1 = (__bf16)r0;
    d[0] = __builtin_bit_cast(uint16_t, p0);
    d[stride] = __builtin_bit_cast(uint16_t, p1);
    d[2 * stride] = __builtin_bit_cast(uint16_t, (__bf16)(r0 - (float)p1));
}

/* the sum of 16-column group g16 (columns 16 g16 ..) of row `row` */
__device__ __forceinline__ void img_sum16(uint16_t* s16, int row, int K, int g16, float S) {
    const int tt = row >> 5, l = row & 31, w = g16 >> 3, gi = g16 & 7;
    img_bf16x3(S, s16 + (((size_t)tt * (K / 128) + w) * 3 * 64 + l + 32 * (gi >> 2)) * 4 + (gi & 3), 256);
}

/* the sum of 32-column group g32 of row `row` */
__device__ __forceinline__ void img_sum32(uint16_t* s32, int row, int K, int g32, float S) {
    const int tt = row >> 5, l = row & 31, w = g32 >> 3, gi = g32 & 7;
    img_bf16x3(S, s32 + (((size_t)tt * (K / 256) + w) * 3 * 64 + l + 32 * (gi >> 2)) * 4 + (gi & 3), 256);
}

#endif
