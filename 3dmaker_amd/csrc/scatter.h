// Internal interface of the binned hash-grid gradient scatter (hash_scatter.hip).
#pragma once

#include "common.h"
#include "optimizer.h"

namespace graft {

// Device scratch of the binned scatter, sized once for a grid configuration
// and a maximum sample count; one per owner (a TinyMLPHashGrid instance, or
// the launchers' per-stream cache), so that scatters driven from different
// owners never share it.
struct ScatterPlan;

// nullptr when the configuration is outside the binned path's limits (then
// hash_scatter falls back to the per-corner atomic kernel).
ScatterPlan* scatter_plan_create(const GridMeta& m, int maxN);
void scatter_plan_destroy(ScatterPlan* p);
int scatter_plan_max_samples(const ScatterPlan* p);

// grads [L][T][2] += scatter of denc [N x 2L] (backward clamp), as the
// atomic hash_scatter, with the table sums formed in fixed point (exact
// integer addition, one rounding to fp32 per entry): deterministic.
// grads_zero: the caller guarantees that grads is all zero on entry (the
// training step: Adam clears every gradient it consumes); the entries of the
// bins the batch touches are then stored instead of read-modify-written.
void hash_scatter_binned(ScatterPlan* p, const GridMeta& m, const __half* denc, const float* pos,
                         int pos_stride, float* grads, int N, hipStream_t stream, const uint32_t* d_n,
                         bool grads_zero);

// The table half of the training step's optimizer step fused into the
// scatter: every table entry [L][T][2] the scatter of denc reaches takes its
// Adam update (adam_hash's arithmetic) from the gradient hash_scatter_binned
// with grads_zero would have stored, in the same pass; no gradient array is
// read or written, entries the batch does not reach keep every word (the
// zero gradients adam_hash skips).  The update waits for wait_before_update
// (nullable) after the sorting passes, before its first table read.
// tile_live (nullable): per 16-sample tile of denc, 0 where every value of
// the tile is +-0 (nerf_heads_dx's flags); those rows are not read.
struct TableAdam {
    float* w;       // fp32 master table
    __half* w16;    // fp16 copy the encode reads
    float* m;
    float* v;
    AdamArgs a;
};
void hash_scatter_adam(ScatterPlan* p, const GridMeta& m, const __half* denc, const float* pos, int pos_stride, int N,
                       const TableAdam& t, hipStream_t stream, const uint32_t* d_n = nullptr,
                       hipEvent_t wait_before_update = nullptr, const uint32_t* tile_live = nullptr);

// hash_scatter_binned's sum (grads +=) with the scratch in a fixed static
// device array instead of allocated memory: no allocation on any call.  The
// batch runs in sub-batches that fit the array; grids beyond its bin capacity
// throw.  Calls that overlap on one GPU race (they share the array).
void hash_scatter_noalloc(const GridMeta& m, const __half* denc, const float* pos, int pos_stride, float* grads,
                          int N, hipStream_t stream);
size_t scatter_noalloc_bytes();

}  // namespace graft
