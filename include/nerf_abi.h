/*
 * C-ABI of the MI355X (gfx950) NeRF-side hot path: the reference's extern "C"
 * launchers of modules/NeRF (InstantNerf.h:385-568) for the training path, and
 * launchers for the kernels the reference launches inline from
 * InstantNerf.cu.  cudaStream_t is replaced by hipStream_t; float3 / uint3 are
 * HIP's (12 bytes, 4-byte aligned, like CUDA's).  Pointers are device
 * pointers unless stated.  Failures set tinymlp_last_error() (tinymlp_abi.h)
 * instead of printing and returning silently.
 *
 * Arithmetic deviations from the reference's fast-math device code, shared
 * with the CPU oracle the tests compare against: e^x is one fixed
 * Cody-Waite/Taylor routine (max 1.2 ulp), the cascade index uses an exact
 * ceil(log2), division and square root are correctly rounded.
 */
#ifndef GRAFT_NERF_ABI_H
#define GRAFT_NERF_ABI_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "tinymlp_abi.h"

#ifdef __cplusplus
#include <hip/hip_vector_types.h>
/* the reference's default arguments (C++ callers only) */
#define GRAFT_DEFAULT(v) = v
extern "C" {
#else
#define GRAFT_DEFAULT(v)
#endif

/* ---- the hierarchical DDA march and its compactions ----
 * Every march below is the reference's (march_rays_dda_calc_hits /
 * march_rays_dda_offset / march_rays_dda_kernel, processRays.cu:96-226,
 * 626-737, 801-929): the same cells, sample t values and per-ray cap of 1024
 * samples (MAX_HITS, InstantNerf.h:24), bit for bit.  Positions are written as
 * float4 (x, y, z, 0) and need 16-byte alignment. */

/* launchMarchRaysDDA (processRays.cu:228-265, declared InstantNerf.h:385-403).
 * The per-ray layout: sample k of ray i at t_hits_out[i * 1024 + k], the
 * 30-bit Morton code of its level-0 cell (coordinates mod 1024) at
 * packed_coords_out[i * 1024 + k] (nullable here), the count at
 * num_steps_per_ray[i]. */
void launchMarchRaysDDA(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                        const float3* rays_d_inv, const float* nears, const float* fars,
                        const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                        const float3 aabb_max, const int numCascades, const int mipmapLevels,
                        const int samplesPerVoxel, uint32_t* packed_coords_out, float* t_hits_out,
                        uint32_t* num_steps_per_ray, hipStream_t stream);

/* processRaysChunk (processRays.cu:357-464, declared InstantNerf.h:405-434).
 * launchMarchRaysDDA into d_sparse_*, exclusive scan of the counts into
 * d_ray_offsets, then every sample of every ray compacted (no batch cutoff:
 * the outputs hold all samples) and stably sorted by Morton code: keys_in /
 * indices_in hold the ray-major compaction, keys_out / indices_out the sorted
 * one (index = ray * 1024 + k), and positions, ray indices and t follow the
 * sorted order.  Blocks the calling thread (one read of the sample count,
 * and the sort). */
void processRaysChunk(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                      const float3* rays_d_inv, const float* nears, const float* fars,
                      const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                      const float3 aabb_max, const int numCascades, const int mipmapLevels,
                      const int samplesPerVoxel, uint32_t* d_sparse_morton, float* d_sparse_ts,
                      uint32_t* d_num_steps, uint32_t* d_ray_offsets, uint32_t* d_dense_morton_keys_in,
                      uint32_t* d_dense_sparse_indices_in, uint32_t* d_dense_morton_keys_out,
                      uint32_t* d_dense_sparse_indices_out, float* d_mlp_positions_batch,
                      uint32_t* d_ray_indices, float* d_t_sorted, hipStream_t stream);

/* processRaysChunkLinear (processRays.cu:551-624, declared InstantNerf.h:436-460):
 * processRaysChunk without the Morton keys and the sort; the outputs are in
 * ray-major order.  Blocks the calling thread (one read of the sample count). */
void processRaysChunkLinear(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                            const float3* rays_d_inv, const float* nears, const float* fars,
                            const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                            const float3 aabb_max, const int numCascades, const int mipmapLevels,
                            const int samplesPerVoxel, float* d_sparse_ts, uint32_t* d_num_steps,
                            uint32_t* d_ray_offsets, uint32_t* d_dense_sparse_indices,
                            float* d_mlp_positions_batch, uint32_t* d_ray_indices, float* d_t_sorted,
                            hipStream_t stream);

/* processRaysHitData (processRays.cu:1042-1081, declared InstantNerf.h:521-539).
 * Per-ray sample counts into d_num_steps and their exclusive scan (uint32
 * wrap-around) into d_ray_offsets; asynchronous.  d_block_sums is accepted
 * for signature compatibility and not used; it may be NULL. */
void processRaysHitData(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                        const float3* rays_d_inv, const float* nears, const float* fars,
                        const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                        const float3 aabb_max, const int numCascades, const int mipmapLevels,
                        const int samplesPerVoxel, uint32_t* d_num_steps, uint32_t* d_ray_offsets,
                        uint32_t* d_block_sums, hipStream_t stream);

/* processRaysHitPositions (processRays.cu:1083-1174, declared InstantNerf.h:541-568).
 * After processRaysHitData on the same rays and grid: the rays from rays_done
 * whose samples fit in batchSize (find_cutoff_ray_from_kernel, :771-799).
 * Returns their number B (0 when the first does not fit or no rays are left),
 * writes rays_done + B to *d_active_rays_count (0 in those cases),
 * offsets[rays_done] to *out_base and their sample count to *totalHits
 * (host pointers; *out_base is left alone when B is 0), and fills sample j of
 * the batch at index d_ray_offsets[rays_done + r] - base + k: t, the
 * batch-local ray index r, the contracted position.  Blocks the calling thread
 * for the cutoff; the fill is asynchronous.  d_block_sums is not used. */
int processRaysHitPositions(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                            const float3* rays_d_inv, const float* nears, const float* fars,
                            const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                            const float3 aabb_max, const int numCascades, const int mipmapLevels,
                            const int samplesPerVoxel, const uint32_t rays_done, const int batchSize,
                            uint32_t* totalHits, uint32_t* out_base, uint32_t* d_num_steps,
                            uint32_t* d_ray_offsets, float* d_mlp_positions_batch, uint32_t* d_ray_indices,
                            uint32_t* d_active_rays_count, float* d_t_sorted, uint32_t* d_block_sums,
                            hipStream_t stream);

/* launchComputeRealSHDegree3 (otherKernels.cu:66-83, declared InstantNerf.h:491-496).
 * d_out_sh [total_hits][16] (16-byte aligned): the real spherical harmonics
 * of degree <= 3 of each direction (taken as given, not normalised), in the
 * order and sign convention of the colour head's input. */
void launchComputeRealSHDegree3(const uint32_t total_hits, const float3* d_directions, float* d_out_sh,
                                hipStream_t stream GRAFT_DEFAULT(0));

/* processRays.cu:931-1040 (declared InstantNerf.h:509-533).  Count pass,
 * exclusive scan and cutoff at batchSize, fill pass; returns the number of
 * active rays and writes the compacted sample count to *totalHits (host).
 * The three blocking round trips of the reference become one read at the end,
 * and the second march of the fill pass becomes a gather: the rays are marched
 * once into a library-owned store of 4 KiB per ray (grown on demand, kept
 * until the process ends).  d_block_sums is accepted for signature
 * compatibility and not used; it may be NULL. */
int processRaysHitLinear(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                         const float3* rays_d_inv, const float* nears, const float* fars,
                         const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                         const float3 aabb_max, const int numCascades, const int mipmapLevels,
                         const int samplesPerVoxel, const int batchSize, uint32_t* totalHits,
                         uint32_t* d_active_rays_count, uint32_t* d_num_steps, uint32_t* d_ray_offsets,
                         float* d_mlp_positions_batch, uint32_t* d_ray_indices, float* d_t_sorted,
                         uint32_t* d_block_sums, hipStream_t stream);

/* compositing.cu:215-279 (declared InstantNerf.h:444-465).  d_dw_out set: the
 * training compositor with the distortion loss (render_rays_distortion_kernel;
 * base and raysDone unused, the training path passes 0).  d_dw_out NULL: the
 * inference compositor (render_rays_kernel, compositing.cu:5-78): ray r's
 * samples start at d_ray_offsets[r + raysDone] - base, d_num_steps[r] of them,
 * early stop once transmittance < 1e-4; d_rgb_true / d_phi_out nullable. */
void launchVolumeRendering(const uint32_t num_rays, const uint32_t* d_ray_offsets, const uint32_t* d_num_steps,
                           const float* d_t_sorted, const float* d_density_sigma, const float* d_depth_chunk,
                           const float* d_sigma_chunk, const float* d_rgb_output, const float* d_rgb_true,
                           float* d_render_rgb, float* d_render_depth, float* d_phi_out, float* d_dw_out,
                           float* d_weight_sum, float lambda_dist, float lambda_depth,
                           float3 bg_color GRAFT_DEFAULT(make_float3(1.0f, 1.0f, 1.0f)),
                           uint32_t base GRAFT_DEFAULT(0), uint32_t raysDone GRAFT_DEFAULT(0),
                           hipStream_t stream GRAFT_DEFAULT(0));

/* fetchRayChunkStreamingKernel (DataLoader.cu:548-661) as launched by
 * DataLoader::fetchRayChunk (:663-679): size rays from offset (randomize = 0)
 * or drawn with pcg_hash from seed, skipping every holdout_every-th image,
 * with depth-prior rays for dense_fraction of them when num_records > 0 (rec_*
 * nullable otherwise); RGBA8 pixels composited over bg_color.  d_transforms:
 * [images][16] row-major camera-to-world; d_images_rgba: [images][h][w][4];
 * total_rays = images * w * h.  d_chunk_dense / d_chunk_sigma nullable. */
void launchFetchRayChunk(int offset, int size, int total_rays, uint32_t seed, int randomize, int width, int height,
                         float focal_length, const float* d_transforms, const uint8_t* d_images_rgba,
                         float3* d_chunk_rays_o, float3* d_chunk_rays_d, float* d_chunk_rgb, float* d_chunk_dense,
                         float* d_chunk_sigma, const int* rec_frame, const float* rec_u, const float* rec_v,
                         const float* rec_D, const float* rec_sigma, uint32_t num_records, float dense_fraction,
                         float uv_scale_x, float uv_scale_y, float3 bg_color, int holdout_every, hipStream_t stream);

/* ---- kernels the reference launches inline (no extern "C" counterpart) ---- */

/* compute_ray_aabb_inv_kernel (otherKernels.cu:91-154), launched at InstantNerf.cu:391-398. */
void launchComputeRayAabbInv(uint32_t num_rays, const float3* rays_o, const float3* rays_d, float3 aabb_min,
                             float3 aabb_max, int num_cascades, float3* rays_d_inv, float* nears, float* fars,
                             hipStream_t stream);

/* compute_SH_gather (otherKernels.cu:156-273), launched at InstantNerf.cu:444-450, 512-517. */
void launchComputeSHGather(const float3* d_chunk_d, const uint32_t* d_ray_indices, int offset, int batchSize,
                           float densityBias, float* d_density_out, GRAFT_HALF* d_color_in, float* d_density_sigma,
                           hipStream_t stream);

/* compute_color_grad (otherKernels.cu:303-409), launched at InstantNerf.cu:526-543. */
void launchComputeColorGrad(uint32_t numRays, uint32_t initialOffset, const uint32_t* num_steps,
                            const uint32_t* ray_offsets, const float* t_sorted, const float* density_mlp_out,
                            const float* color_mlp_out, const float* phi_chunk, const float* final_rgb,
                            const float* dw_out, const float* weight_sum, GRAFT_HALF* custom_color_grad,
                            float* tmp_dsigma, float loss_scale, float densityBias, uint32_t totalRaysBatch,
                            hipStream_t stream);

/* launchVolumeRendering (training compositor, d_dw_out set) followed by
 * launchComputeColorGrad with initialOffset 0, as one kernel with one wave per
 * ray (InstantNerf.cu:463-481 then 526-543; no single reference counterpart).
 * Outputs are bit-identical to the two launches; colour gradients are written
 * with row pitch grad_stride (3 in the reference layout, extra columns zeroed)
 * and colours read with row pitch rgb_stride. */
void launchVolumeRenderingColorGrad(uint32_t num_rays, const uint32_t* d_ray_offsets, const uint32_t* d_num_steps,
                                    const float* d_t_sorted, const float* d_density_sigma, const float* d_depth_chunk,
                                    const float* d_sigma_chunk, const float* d_rgb_output, int rgb_stride,
                                    const float* d_rgb_true, float* d_render_rgb, float* d_render_depth,
                                    float* d_phi_out, float* d_dw_out, float* d_weight_sum, float lambda_dist,
                                    float lambda_depth, float3 bg_color, const float* density_mlp_out,
                                    GRAFT_HALF* custom_color_grad, int grad_stride, float* tmp_dsigma,
                                    float loss_scale, float densityBias, uint32_t totalRaysBatch, hipStream_t stream);

/* compute_density_grad (otherKernels.cu:506-562), launched at InstantNerf.cu:552-557. */
void launchComputeDensityGrad(uint32_t batch_size, const float* tmp_dsigma, const GRAFT_HALF* custom_dx_out,
                              GRAFT_HALF* custom_density_grad, hipStream_t stream);

/* updateMasterGrid (otherKernels.cu:677-690). */
void launchUpdateMasterGrid(const float* tmpGrid, float* masterGrid, float decayValue, int N, hipStream_t stream);

/* Sum of d_in[0..n) into d_out[0], fixed summation order (replaces the CUB
 * DeviceReduce::Sum of otherKernels.cu:696-698). */
void launchReduceSum(const float* d_in, int n, float* d_out, hipStream_t stream);

/* updateOccupancyGrid (otherKernels.cu:700-750): level-0 bits from the master
 * grid; G = cells per cascade, S = cells of one cascade's mip pyramid. */
void launchUpdateOccupancyGrid(uint32_t* d_occupancy_grid, const float* d_master_grid, const float* d_sum,
                               int total_cells, int cells_per_cascade, int pyramid_cells_per_cascade,
                               float min_optical_thickness, float base_voxel, hipStream_t stream);

/* InstantNerf::buildMipmaps + bitfield_max_pool (InstantNerf.cu:1177-1204,
 * otherKernels.cu:752-807). */
void launchBuildMipmaps(uint8_t* d_grid, uint3 grid_resolution, int mipmapLevels, int numCascades,
                        hipStream_t stream);

/* ---- the NeRF step's two heads on the 16x16x32 fp16 MFMA (no single
 * reference counterpart: the reference runs each head's forward and backward
 * as separate launches, networkFusionHashtable.cu:441-682,
 * networkFusion.cu:197-355, networkFusionBackward.cu:49-646,
 * networkFusionBackwardHashtable.cu:71-781, with compute_SH_gather and
 * compute_density_grad between them).  Shapes: density 32-64-16 and colour
 * 32-64-64-8 (TinyMLP's hardware shapes of the 32-64-64-3 head), ReLU.
 * Weights are device arrays of per-layer device pointers as the TinyMLP
 * classes keep them (fp16 W [out][in], fp32 b).  Encodings are level-major:
 * d_enc[l][enc_plane] fp16 feature pairs, l < levels <= 16, enc_plane >=
 * num_samples.  Unsupported shapes are reported through tinymlp_last_error. */

/* Bytes of the packed-weight buffer the launchers below take. */
size_t nerfHeadsPackedBytes(void);

/* Packs both heads' current weights and biases into d_packed. */
void launchNerfHeadsPack(const GRAFT_HALF* const* d_density_w, const float* const* d_density_b,
                         const GRAFT_HALF* const* d_color_w, const float* const* d_color_b, void* d_packed,
                         hipStream_t stream);

/* Density head -> sigma = e^min(sanitised logit 0 - density_bias, 8), the
 * colour input [logits sanitised to +-64, NaN -> 0 | SH of the sample's ray
 * direction] (fp16 [N][32], d_color_in; the backward's input), colour head
 * (sigmoid when color_activation = 1) -> d_color_out fp32 [N][8];
 * d_density_out (fp32 [N][16], the logits before sanitising) is nullable. */
void launchNerfHeadsForward(const void* d_packed, const GRAFT_HALF* d_enc, int enc_plane, int levels,
                            const float3* d_dirs, const uint32_t* d_ray_indices, int num_samples,
                            float density_bias, int color_activation, float* d_sigma, float* d_density_out,
                            float* d_color_out, GRAFT_HALF* d_color_in, hipStream_t stream);

/* Recomputes the heads' hidden layers from d_enc and d_color_in, then the
 * colour dX chain from d_color_dy (fp16 [N][8]), the density-gradient glue
 * with d_dsigma and the density dX chain: d_denc fp16 [N][32] = dL/d(encoding);
 * d_density_dy (fp16 [N][16]) and d_color_dx (fp16 [N][32], the logit
 * features; the SH features are written as 0) are nullable.  16-sample tiles
 * whose colour dL/dy is zero and whose density dL/dy rounds to +-0 skip the
 * chain (their outputs are the chain's: zeros and the glue of +0);
 * d_tile_live (nullable, uint32 [ceil(N / 16)]) receives 1 for the others. */
void launchNerfHeadsBackward(const void* d_packed, const GRAFT_HALF* d_enc, int enc_plane, int levels,
                             const GRAFT_HALF* d_color_in, const GRAFT_HALF* d_color_dy, const float* d_dsigma,
                             int num_samples, GRAFT_HALF* d_denc, GRAFT_HALF* d_density_dy, GRAFT_HALF* d_color_dx,
                             uint32_t* d_tile_live, hipStream_t stream);

/* The weight gradients of every layer of both heads for the same inputs,
 * stored (not added) into the per-layer fp32 arrays (device arrays of device
 * pointers); the block partials are summed in a fixed order.  d_density_dy
 * (nullable) is the density dL/dy launchNerfHeadsBackward stored for the same
 * inputs: given, the density head's gradients start from it instead of
 * running the colour dX chain again (same values).  d_tile_live (nullable)
 * is that call's tile flags: only the flagged tiles are visited (the others
 * add nothing). */
void launchNerfHeadsWeightGrads(const void* d_packed, const GRAFT_HALF* d_enc, int enc_plane, int levels,
                                const GRAFT_HALF* d_color_in, const GRAFT_HALF* d_color_dy, const float* d_dsigma,
                                const GRAFT_HALF* d_density_dy, const uint32_t* d_tile_live, int num_samples,
                                float* const* d_density_dw, float* const* d_density_db, float* const* d_color_dw,
                                float* const* d_color_db, hipStream_t stream);

/* ABI self-check (no reference counterpart): writes a.xyz, b.xyz to out[0..6). */
void nerf_abi_echo_vec(float3 a, uint3 b, float* out);

#ifdef __cplusplus
}
#endif
#undef GRAFT_DEFAULT
#endif
