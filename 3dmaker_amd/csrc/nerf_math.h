// Scalar math shared by the NeRF-side kernels (ray setup, DDA, compositing,
// gradient glue).  Every routine is plain IEEE fp32 arithmetic (the library is
// built with -ffp-contract=off and correctly rounded division), so the
// kernels' results are reproducible operation by operation.
#pragma once

#include "common.h"

namespace graft {

constexpr int kMaxHits = 1024;             // per-ray sample cap (InstantNerf.h:24)
constexpr int kMaxMarchIters = 1 << 20;    // DDA iteration bound per ray (see march loop)

// e^x by Cody & Waite range reduction (x = k ln2 + r, |r| <= ln2/2, with ln2
// split into a 16-bit head and a tail so that k * ln2_hi is exact) and the
// degree-7 Taylor polynomial of e^r in Horner form (truncation error below
// 6e-9 relative), scaled exactly by 2^k.  Max error 1.2 ulp on [-87, 88].
// Results below FLT_MIN are flushed to 0; overflow gives +inf; NaN stays NaN.
__host__ __device__ __forceinline__ float nerf_expf(float x)
{
    if (x != x) return x;
    if (x > 89.0f) return __builtin_huge_valf();
    if (x < -87.0f) return 0.0f;
    const float kf = rintf(x * 1.44269504f);
    const int k = (int)kf;
    const float r = (x - kf * 0.693145751953125f) - kf * 1.428606765330187e-06f;
    float p = 1.98412698e-4f;
    p = p * r + 1.38888889e-3f;
    p = p * r + 8.33333333e-3f;
    p = p * r + 4.16666667e-2f;
    p = p * r + 1.66666667e-1f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, k);
}

// max(0, min((int)f, hi)) with the saturating float->int conversion of the
// hardware spelled out (NaN and negatives -> 0, f >= hi -> hi).
__host__ __device__ __forceinline__ int clamp_floor_idx(float f, int hi)
{
    // branch-free: fmaxf turns NaN and negatives into 0, fminf caps at hi (exact: hi < 2^24)
    return (int)fminf(fmaxf(f, 0.0f), (float)hi);
}

// get_cascade (processRays.cu:11-19): the smallest cascade c whose box
// aabb * 2^c contains pos, i.e. ceil(log2(max_k pos_k / bound_k)) clamped to
// [0, C-1].  The ceil(log2) is exact (frexp) rather than a log2f evaluation.
__host__ __device__ __forceinline__ int get_cascade(float px, float py, float pz, float3 mn, float3 mx, int C)
{
    const float rx = fmaxf(px / mx.x, px / mn.x);
    const float ry = fmaxf(py / mx.y, py / mn.y);
    const float rz = fmaxf(pz / mx.z, pz / mn.z);
    const float s = fmaxf(rx, fmaxf(ry, rz));
    if (s <= 1.0f) return 0;
    int e = 0;
    const float m = frexpf(s, &e);
    const int c = (m == 0.5f) ? e - 1 : e;
    return c < 0 ? 0 : (c > C - 1 ? C - 1 : c);
}

// contract_pos (processRays.cu:21-46): scene box -> [0.25, 0.75], the outside
// contracted towards [0, 1].
__host__ __device__ __forceinline__ float contract_axis(float p, float mn, float mx)
{
    const float ext = mx - mn;
    const float rel = (p - mn) / ext;
    const float n = rel * 2.0f - 1.0f;
    const float c = fabsf(n) <= 1.0f ? n : (2.0f - 1.0f / fabsf(n)) * copysignf(1.0f, n);
    return fmaxf(0.0f, fminf((c + 2.0f) * 0.25f, 1.0f));
}

// Cells of the mip pyramid below `level` (get_mipmap_offset, processRays.cu:83-93).
__host__ __device__ __forceinline__ uint32_t mip_offset(uint3 res, int level)
{
    uint32_t off = 0, rx = res.x, ry = res.y, rz = res.z;
    for (int l = 0; l < level; l++) {
        off += rx * ry * rz;
        rx >>= 1;
        ry >>= 1;
        rz >>= 1;
    }
    return off;
}

__host__ __device__ __forceinline__ float clamp_half_range(float v) { return fmaxf(-65504.0f, fminf(65504.0f, v)); }

// Density logit as the colour head sees it (otherKernels.cu:208-211): clamped
// to [-64, 64], NaN -> 0.
__host__ __device__ __forceinline__ float sanitize_logit(float v)
{
    v = fmaxf(-64.0f, fminf(64.0f, v));
    return (v != v) ? 0.0f : v;
}

// Real spherical harmonics of degree <= 3 at a unit direction, with the
// published constants (Sloan, "Stupid Spherical Harmonics Tricks") in the
// reference's sign convention and order (otherKernels.cu:182-200).
__host__ __device__ __forceinline__ void sh_basis16(float x, float y, float z, float (&sh)[16])
{
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    sh[0] = 0.28209479f;
    sh[1] = -0.48860251f * y;
    sh[2] = 0.48860251f * z;
    sh[3] = -0.48860251f * x;
    sh[4] = 1.09254843f * x * y;
    sh[5] = -1.09254843f * y * z;
    sh[6] = 0.31539156f * (3.0f * z2 - 1.0f);
    sh[7] = -1.09254843f * x * z;
    sh[8] = 0.54627421f * (x2 - y2);
    sh[9] = -0.59004359f * y * (3.0f * x2 - y2);
    sh[10] = 2.89061144f * x * y * z;
    sh[11] = -0.45704580f * y * (5.0f * z2 - 1.0f);
    sh[12] = 0.37317633f * z * (5.0f * z2 - 3.0f);
    sh[13] = -0.45704580f * x * (5.0f * z2 - 1.0f);
    sh[14] = 1.44530572f * z * (x2 - y2);
    sh[15] = -0.59004359f * x * (x2 - 3.0f * y2);
}

}  // namespace graft
