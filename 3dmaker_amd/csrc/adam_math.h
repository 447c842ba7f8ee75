// The Adam update of one parameter (optimizerKernel.cu:16-167), shared by the
// optimizer kernels and the binned scatter's fused table update.  Written
// operation by operation (no FP contraction, IEEE division and square root):
// every kernel that applies it produces the same bits.
#pragma once

#include "optimizer.h"

namespace graft {

__device__ __forceinline__ float finite_or_zero(float x) { return isfinite(x) ? x : 0.0f; }

__device__ __forceinline__ void adam_update(float graw, float& m, float& v, float& w, const AdamArgs& a)
{
    const float g = finite_or_zero(graw * a.inv_scale);
    const float mv = a.b1 * finite_or_zero(m) + (1.0f - a.b1) * g;
    const float vv = a.b2 * finite_or_zero(v) + ((1.0f - a.b2) * g) * g;
    const float mh = mv / a.bc1;
    const float vh = vv / a.bc2;
    float wv = isfinite(w) ? w : 0.0f;
    wv = wv - ((a.lr * mh) / (sqrtf(vh) + a.eps));
    if (!isfinite(wv)) wv = 0.0f;
    m = mv;
    v = vv;
    w = wv;
}

}  // namespace graft
