// Device-side multiresolution hash-grid corner math shared by the encode,
// fused encode+MLP and scatter kernels.  The arithmetic follows
// modules/TinyMLP/networkFusionHashtable.cu:458-548 (forward) and
// networkFusionBackwardHashtable.cu:805-907 (scatter) operation by operation,
// so that it is bit-identical to the CPU oracle given the same scale table.
// All HIP sources are built with -ffp-contract=off: an FMA appears only where
// fmaf() is written.
#pragma once

#include "common.h"

namespace graft {

struct Corners {
    uint32_t idx[8];  // element offset of feature 0 within the level slice
    float w[8];       // order 000,100,010,110,001,101,011,111
};

// BWD = false: x0 clamped to [0, N_l]   (forward kernels)
// BWD = true:  x0 clamped to [0, N_l-1] (gradient scatter)
template <bool BWD>
__device__ __forceinline__ void level_corners(float px, float py, float pz, float s, int N_l,
                                              bool dense, uint32_t mask, Corners& c)
{
    const float x_l = px * s;
    const float y_l = py * s;
    const float z_l = pz * s;
    const float fx = floorf(x_l), fy = floorf(y_l), fz = floorf(z_l);
    const int hi = BWD ? N_l - 1 : N_l;
    int x0 = max(0, min((int)fx, hi));
    int y0 = max(0, min((int)fy, hi));
    int z0 = max(0, min((int)fz, hi));
    const int x1 = min(x0 + 1, N_l);
    const int y1 = min(y0 + 1, N_l);
    const int z1 = min(z0 + 1, N_l);

    const float wx1 = (1.0f - x_l) + fx;
    const float wy1 = (1.0f - y_l) + fy;
    const float wz1 = (1.0f - z_l) + fz;
    const float ux = 1.0f - wx1, uy = 1.0f - wy1, uz = 1.0f - wz1;
    c.w[0] = (wx1 * wy1) * wz1;
    c.w[1] = (ux * wy1) * wz1;
    c.w[2] = (wx1 * uy) * wz1;
    c.w[3] = (ux * uy) * wz1;
    c.w[4] = (wx1 * wy1) * uz;
    c.w[5] = (ux * wy1) * uz;
    c.w[6] = (wx1 * uy) * uz;
    c.w[7] = (ux * uy) * uz;

    if (dense) {
        const int st = N_l + 1;
        const int b00 = y0 * st + z0 * st * st;
        const int b10 = y1 * st + z0 * st * st;
        const int b01 = y0 * st + z1 * st * st;
        const int b11 = y1 * st + z1 * st * st;
        c.idx[0] = (uint32_t)(x0 + b00) * 2u;
        c.idx[1] = (uint32_t)(x1 + b00) * 2u;
        c.idx[2] = (uint32_t)(x0 + b10) * 2u;
        c.idx[3] = (uint32_t)(x1 + b10) * 2u;
        c.idx[4] = (uint32_t)(x0 + b01) * 2u;
        c.idx[5] = (uint32_t)(x1 + b01) * 2u;
        c.idx[6] = (uint32_t)(x0 + b11) * 2u;
        c.idx[7] = (uint32_t)(x1 + b11) * 2u;
    } else {
        const uint32_t hy0 = (uint32_t)y0 * 2654435761u, hy1 = (uint32_t)y1 * 2654435761u;
        const uint32_t hz0 = (uint32_t)z0 * 805459861u, hz1 = (uint32_t)z1 * 805459861u;
        const uint32_t ux0 = (uint32_t)x0, ux1 = (uint32_t)x1;
        c.idx[0] = ((ux0 ^ hy0 ^ hz0) & mask) * 2u;
        c.idx[1] = ((ux1 ^ hy0 ^ hz0) & mask) * 2u;
        c.idx[2] = ((ux0 ^ hy1 ^ hz0) & mask) * 2u;
        c.idx[3] = ((ux1 ^ hy1 ^ hz0) & mask) * 2u;
        c.idx[4] = ((ux0 ^ hy0 ^ hz1) & mask) * 2u;
        c.idx[5] = ((ux1 ^ hy0 ^ hz1) & mask) * 2u;
        c.idx[6] = ((ux0 ^ hy1 ^ hz1) & mask) * 2u;
        c.idx[7] = ((ux1 ^ hy1 ^ hz1) & mask) * 2u;
    }
}

// One level of the forward encode: 8 half2 gathers, fp32 fmaf chain from
// corner 111 outwards (networkFusionHashtable.cu:185-201).
__device__ __forceinline__ float2 encode_level(float px, float py, float pz, float s, int N_l,
                                               bool dense, uint32_t mask,
                                               const _Float16* __restrict__ lvl)
{
    Corners c;
    level_corners<false>(px, py, pz, s, N_l, dense, mask, c);
    h2 f[8];
#pragma unroll
    for (int k = 0; k < 8; k++) f[k] = *reinterpret_cast<const h2*>(lvl + c.idx[k]);
    float ax = (float)f[7].x * c.w[7];
    float ay = (float)f[7].y * c.w[7];
#pragma unroll
    for (int k = 6; k >= 0; k--) {
        ax = fmaf((float)f[k].x, c.w[k], ax);
        ay = fmaf((float)f[k].y, c.w[k], ay);
    }
    return make_float2(ax, ay);
}

}  // namespace graft
