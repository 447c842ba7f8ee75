// Internal interface of the NeRF-side kernels (raymarch.hip, render.hip).
//
// Counts that the previous kernel produced on the device (active rays,
// compacted samples) are passed as `const uint32_t* d_n` next to a host upper
// bound `n_max`: a kernel processes min(*d_n, n_max) items when d_n is set and
// n_max otherwise, so a training step never has to read a count back to the
// host to size its launches.
#pragma once

#include "common.h"
#include "nerf_math.h"

namespace graft {

struct OccGrid {
    const uint8_t* bits;   // [C * S] bits, LSB-first, per cascade a mip pyramid
    uint3 res;             // level-0 resolution
    float3 aabb_min, aabb_max;
    int cascades, mip_levels;
};

// compute_ray_aabb_inv_kernel (otherKernels.cu:91-154).
void ray_aabb_inv(uint32_t R, const float3* o, const float3* d, float3 aabb_min, float3 aabb_max, int cascades,
                  float3* d_inv, float* nears, float* fars, hipStream_t s);

// Device scratch of one compaction: per-256-ray block sums and result[2] =
// {active rays, compacted samples}.
struct MarchScratch {
    uint32_t* block_sums;  // >= ceil(R / 256)
    uint32_t* result;      // [2]
};
size_t march_scratch_words(uint32_t R);

// processRaysHitLinear (processRays.cu:931-1040) without host round trips, in
// two halves so that a caller can re-compact one window of rays several times
// (one hit batch after the other) on an unchanged grid: march_store marches
// every ray once (march_rays_dda_calc_hits, :626-737) and keeps sample k of ray
// i (the t value march_rays_dda_offset writes, :896-909) in the march store at
// march_store_index(i, k); march_compact_stored scans the counts, applies the
// cutoff (find_cutoff_ray_kernel, :739-769) and gathers the samples, one thread
// per sample.  counts, offsets [R]; t_out, ray_idx, pos_out [batch]; the active
// ray and sample counts stay on the device in scratch.result.
//
// Store layout: tiles of 64 rays (one wave of the march) x kMaxHits, hit-major
// inside a tile, so lanes that emit their k-th sample together write one
// contiguous 256-byte row and a tile's rows fill up in L2 before they leave it.
__host__ __device__ inline size_t march_store_index(uint32_t ray, uint32_t k)
{
    return (size_t)(ray >> 6) * (64 * kMaxHits) + (size_t)k * 64 + (ray & 63);
}
inline size_t march_store_floats(uint32_t R) { return (size_t)((R + 63) / 64) * 64 * kMaxHits; }
void march_store(uint32_t R, const float3* o, const float3* d, const float3* d_inv, const float* nears,
                 const float* fars, const OccGrid& g, int K, uint32_t* counts, float* t_scratch, hipStream_t s);
// Compacts rays [ray_base, ray_base + R) of the stored march (counts already
// offset to the window's first ray; o, d too).  counts_out (nullable)
// receives a copy of the R counts, so that the step can read them after the
// march store has been overwritten.
void march_compact_stored(uint32_t R, const float3* o, const float3* d, const OccGrid& g, uint32_t batch,
                          const uint32_t* counts, const float* t_scratch, uint32_t ray_base, uint32_t* offsets,
                          float* t_out, uint32_t* ray_idx, float4* pos_out, const MarchScratch& scratch,
                          hipStream_t s, uint32_t* counts_out = nullptr);

// march_rays_dda_calc_hits (processRays.cu:626-737): per-ray sample counts only.
void march_count(uint32_t R, const float3* o, const float3* d, const float3* d_inv, const float* nears,
                 const float* fars, const OccGrid& g, int K, uint32_t* counts, hipStream_t s);
// march_rays_dda_kernel (processRays.cu:96-226): the per-ray ("sparse")
// layout, sample k of ray i at t_sparse[i * kMaxHits + k] and, when morton is
// set, the 30-bit Morton code of its level-0 cell at morton[i * kMaxHits + k].
void march_sparse(uint32_t R, const float3* o, const float3* d, const float3* d_inv, const float* nears,
                  const float* fars, const OccGrid& g, int K, uint32_t* counts, float* t_sparse, uint32_t* morton,
                  hipStream_t s);
// Exclusive scan of counts [R] into offsets (uint32 wrap-around, as
// custom_exclusive_sum, processRays.cu:486-549) and the cutoff at batch:
// scratch.result = {rays whose samples fit in batch, their samples}; batch =
// UINT32_MAX gives {R, all samples}.
void scan_counts(uint32_t R, const uint32_t* counts, uint32_t batch, uint32_t* offsets, const MarchScratch& scratch,
                 hipStream_t s, uint32_t* counts_out = nullptr);
// find_cutoff_ray_from_kernel (processRays.cu:771-799) over rays [rays_done,
// R): result[4] = {batch rays, their samples, base = offsets[rays_done],
// rays_done + batch rays}, all zero (and *next_done zero) when the first ray
// does not fit or rays_done >= R; *next_done (nullable) = result[3].
void cutoff_from(uint32_t R, const uint32_t* offsets, const uint32_t* counts, uint32_t batch, uint32_t rays_done,
                 uint32_t* next_done, uint32_t* result, hipStream_t s);
// Samples j < result[1] of rays [0, result[0]) whose samples start at
// offsets[i] - base, from a march store holding those rays from row 0:
// t_out[j], ray_idx[j] (ray-local), pos_out[j] (contracted, w = 0).
void gather_stored(uint32_t max_samples, const float3* o, const float3* d, const OccGrid& g, const uint32_t* offsets,
                   uint32_t base, const float* t_scratch, const uint32_t* result, float* t_out, uint32_t* ray_idx,
                   float4* pos_out, hipStream_t s);
// compact_hits(_linear)_kernel (processRays.cu:297-318, 466-483) over the
// result[1] samples of rays [0, R): sparse_idx[j] = ray * kMaxHits + k, keys[j]
// (nullable) = morton[sparse_idx[j]].
void compact_sparse(uint32_t R, const uint32_t* offsets, const uint32_t* result, uint32_t max_samples,
                    const uint32_t* morton, uint32_t* keys, uint32_t* sparse_idx, hipStream_t s);
// generate_mlp_batch_kernel (processRays.cu:320-356) over result[1] samples.
void sparse_batch(const uint32_t* result, uint32_t max_samples, const uint32_t* sparse_idx, const float* t_sparse,
                  const float3* o, const float3* d, float3 aabb_min, float3 aabb_max, float4* pos_out,
                  uint32_t* ray_idx, float* t_out, hipStream_t s);
// compute_real_sh_degree_3_kernel (otherKernels.cu:18-64): out [n][16]
// (16-byte aligned).
void sh_degree3(uint32_t n, const float3* dirs, float* out, hipStream_t s);
// Stable ascending sort of n (key, value) pairs of 32-bit keys (rocPRIM's
// LSD radix sort; library-owned temporary storage grown on demand).  Blocks
// until the sort has finished.
void sort_pairs_u32(const uint32_t* keys_in, uint32_t* keys_out, const uint32_t* values_in, uint32_t* values_out,
                    uint32_t n, hipStream_t s);

// compute_SH_gather (otherKernels.cu:156-273).
void sh_gather(const float3* dirs, const uint32_t* ray_idx, const uint32_t* d_n, uint32_t n_max, float bias,
               const float* density_out, __half* color_in, float* sigma, hipStream_t s);

// render_rays_distortion_kernel (compositing.cu:84-213).
struct CompositeArgs {
    const uint32_t* offsets;
    const uint32_t* counts;
    const float* t;
    const float* sigma;
    const float* depth_prior;   // nullable
    const float* sigma_prior;   // nullable
    const float* rgb;           // [N x rgb_stride], rgb in the first 3 columns
    int rgb_stride;             // 3 in the reference layout
    const float* rgb_true;      // nullable
    float* final_rgb;
    float* final_depth;
    float* phi;                 // nullable
    float* dw;
    float* weight_sum;
    float lambda_dist, lambda_depth;
    float3 bg;
};
void composite(const CompositeArgs& a, const uint32_t* d_rays, uint32_t rays_max, hipStream_t s);

// render_rays_kernel (compositing.cu:5-78), the inference compositor: ray r's
// samples start at offsets[r + rays_done] - base, counts[r] of them; early stop
// once T < 1e-4.  Uses offsets, counts, t, sigma, rgb (rgb_stride), rgb_true
// and phi (nullable), final_rgb, final_depth, bg of CompositeArgs.
void composite_infer(const CompositeArgs& a, uint32_t base, uint32_t rays_done, const uint32_t* d_rays,
                     uint32_t rays_max, hipStream_t s);

// compute_color_grad (otherKernels.cu:303-409).
struct ColorGradArgs {
    uint32_t initial_offset;
    const uint32_t* counts;
    const uint32_t* offsets;
    const float* t;
    const float* density_out;   // [N x density_stride]: the density logit 0 first
    int density_stride = 16;    // 16 in the reference layout; 1: the logit alone
    const float* color_out;     // [N x color_stride]
    int color_stride;           // 3 in the reference layout
    const float* phi;
    const float* final_rgb;
    const float* dw;
    const float* weight_sum;
    __half* color_grad;         // [N x grad_stride]: 3 gradients, then zeros
    int grad_stride;            // 3 in the reference layout
    float* dsigma;
    float loss_scale, bias;
    uint32_t total_rays;
};
void color_grad(const ColorGradArgs& a, const uint32_t* d_rays, uint32_t rays_max, hipStream_t s);

// composite() followed by color_grad() with initial_offset 0, fused: one wave
// per ray, bit-identical outputs (compositing.cu:84-213, otherKernels.cu:303-409).
// The colour-gradient arguments read the weights' gradients from a.dw and
// final colours, phi and weight sums from the compositing results.
void render_grad(const CompositeArgs& a, const ColorGradArgs& g, const uint32_t* d_rays, uint32_t rays_max,
                 hipStream_t s);

// compute_density_grad (otherKernels.cu:506-562).
void density_grad(const uint32_t* d_n, uint32_t n_max, const float* dsigma, const __half* color_dx,
                  __half* density_grad, hipStream_t s);

// Occupancy (otherKernels.cu:677-807; InstantNerf.cu:1177-1204).
void update_master_grid(const float* tmp, float* master, float decay, uint32_t n, hipStream_t s);
// out[0] = sum of in[0..n) in a fixed order (two passes, partials in scratch [>= 1024 floats]).
void reduce_sum(const float* in, uint32_t n, float* partials, float* out, hipStream_t s);
void update_occupancy_bits(uint32_t* bits32, const float* master, const float* d_sum, int total, int G, int S,
                           float min_optical, float base_voxel, hipStream_t s);
void build_mipmaps(uint8_t* bits, uint3 res, int mip_levels, int cascades, hipStream_t s);

// extractOccupancyGrid (InstantNerf.cu:882-939): pos [n x 3]; out [ceil(n / 32)]
// words, bit k of word i for point 32 i + k (exact cascade index).
void query_occupancy(const float* master, const float* pos, uint32_t* out, uint3 res, float3 mn, float3 mx,
                     float min_optical, int cascades, int n, hipStream_t s);
// out[i] = src[i * stride], i < n.
void extract_column(const float* src, int stride, float* out, int n, hipStream_t s);

}  // namespace graft
