/*
 * CPU oracle for the NeRF side of the 3DMaker training hot path: ray/AABB
 * setup, cascaded-occupancy DDA with hit-centric compaction, spherical-harmonic
 * gather, volume compositing with the distortion loss, the color/density
 * gradient glue and the occupancy bitfield.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against
 * (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg).  Never linked
 * into or used as a fallback of the product library.
 *
 * Every function restates one reference kernel (file:line relative to the
 * reference checkout) in IEEE-754 fp32, round-to-nearest-even, no FP
 * contraction, operation by operation in the reference's order.  Two
 * deliberate, documented deviations from the reference's device fast-math:
 *  - e^x is orc_expf() below (Cody-Waite reduction + degree-7 Taylor
 *    polynomial), the same method the HIP kernels use, instead of CUDA __expf;
 *  - the cascade index ceil(log2(s)) is taken exactly from frexpf() instead of
 *    fast-math log2f (processRays.cu:17).
 * Float3 arrays are tightly packed x,y,z (12-byte stride, like CUDA float3).
 */
#ifndef GRAFT_NERF_ORACLE_H
#define GRAFT_NERF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_MAX_HITS 1024 /* InstantNerf.h:24 */

/* e^x: x < -87.33654 -> 0 (no subnormal results), NaN -> NaN, overflow -> inf. */
float orc_expf(float x);
void orc_expf_array(const float* x, float* y, size_t n);

/* get_cascade (processRays.cu:11-19) with exact ceil(log2). */
int orc_get_cascade(const float* pos3, const float* aabb_min, const float* aabb_max, int num_cascades);

/* contract_pos (processRays.cu:21-46). */
void orc_contract_pos(const float* pos3, const float* aabb_min, const float* aabb_max, float* out3);

/* Cells of one cascade's mip pyramid (InstantNerf.cu:286-299): sum over l<levels of (res>>l)^3. */
uint32_t orc_pyramid_cells(const uint32_t* res3, int levels);

/* compute_ray_aabb_inv_kernel (otherKernels.cu:91-154). */
void orc_ray_aabb_inv(uint32_t R, const float* rays_o, const float* rays_d,
                      const float* aabb_min, const float* aabb_max, int num_cascades,
                      float* d_inv, float* nears, float* fars);

/* march_rays_dda_calc_hits (processRays.cu:626-737): per-ray sample counts. */
void orc_march_count(uint32_t R, const float* rays_o, const float* rays_d, const float* d_inv,
                     const float* nears, const float* fars, const uint8_t* bits,
                     const uint32_t* res3, const float* aabb_min, const float* aabb_max,
                     int num_cascades, int mip_levels, int K, uint32_t* counts);

/* processRaysHitLinear (processRays.cu:931-1040): count, exclusive scan, cutoff
 * at batch_size (find_cutoff_ray_kernel :739-769), fill (march_rays_dda_offset
 * :801-929).  Returns the active ray count; *total_hits receives the number of
 * compacted samples.  offsets [R] is the exclusive scan of counts over ALL rays.
 * t_out/ray_idx_out/pos_out (float4 x,y,z,0) are written for the active rays. */
uint32_t orc_march_hits(uint32_t R, const float* rays_o, const float* rays_d, const float* d_inv,
                        const float* nears, const float* fars, const uint8_t* bits,
                        const uint32_t* res3, const float* aabb_min, const float* aabb_max,
                        int num_cascades, int mip_levels, int K, uint32_t batch_size,
                        uint32_t* counts, uint32_t* offsets, uint32_t* total_hits,
                        float* t_out, uint32_t* ray_idx_out, float* pos_out);

/* processRaysHitPositions' fill (march_rays_dda_offset, processRays.cu:801-929,
 * called at :1150-1170 on the batch's rays): ray i of the R given (pointers
 * already offset to the batch's first ray) writes its samples at
 * out_base[i] + k with the ray index i (batch-local). */
void orc_march_fill(uint32_t R, const float* rays_o, const float* rays_d, const float* d_inv,
                    const float* nears, const float* fars, const uint8_t* bits,
                    const uint32_t* res3, const float* aabb_min, const float* aabb_max,
                    int num_cascades, int mip_levels, int K, const uint32_t* out_base, float* t_out,
                    uint32_t* ray_idx_out, float* pos_out);

/* march_rays_dda_kernel (processRays.cu:96-226): the per-ray layout, sample k
 * of ray i at t_sparse[i * ORC_MAX_HITS + k] and, when morton is set, the
 * Morton code of its level-0 cell at morton[i * ORC_MAX_HITS + k]; counts [R]. */
void orc_march_sparse(uint32_t R, const float* rays_o, const float* rays_d, const float* d_inv,
                      const float* nears, const float* fars, const uint8_t* bits,
                      const uint32_t* res3, const float* aabb_min, const float* aabb_max,
                      int num_cascades, int mip_levels, int K, uint32_t* counts, float* t_sparse,
                      uint32_t* morton);

/* generate_mlp_batch_kernel (processRays.cu:320-356): sample j is sparse
 * sample sparse_idx[j] of ray sparse_idx[j] / ORC_MAX_HITS: its contracted
 * position (float4, w = 0), ray index and t. */
void orc_sparse_batch(uint32_t N, const uint32_t* sparse_idx, const float* t_sparse, const float* rays_o,
                      const float* rays_d, const float* aabb_min, const float* aabb_max, float* pos_out,
                      uint32_t* ray_idx_out, float* t_out);

/* morton3d / expand_bits_3d (processRays.cu:71-82): 30-bit interleave of the
 * low 10 bits of x (bit 3b), y (3b + 1), z (3b + 2). */
uint32_t orc_morton30(uint32_t x, uint32_t y, uint32_t z);

/* compute_real_sh_degree_3_kernel (otherKernels.cu:18-64): out [N][16], the
 * basis of compute_SH_gather below at each direction as given. */
void orc_sh_degree3(uint32_t N, const float* dirs, float* out);

/* compute_SH_gather (otherKernels.cu:156-273): color input fp16 [N][32] =
 * [16 sanitised density logits | 16 real SH (degree <= 3) of the ray direction],
 * sigma [N] = exp(min(logit0 - bias, 8)). */
void orc_sh_gather(uint32_t N, const float* dirs, const uint32_t* ray_idx, float density_bias,
                   const float* density_out, uint16_t* color_in, float* sigma);

/* render_rays_distortion_kernel (compositing.cu:84-213).  depth_prior and
 * sigma_prior are nullable (depth supervision off); rgb_true and phi nullable. */
void orc_composite_distortion(uint32_t R, const uint32_t* offsets, const uint32_t* counts,
                              const float* t, const float* sigma, const float* depth_prior,
                              const float* sigma_prior, const float* rgb, const float* rgb_true,
                              float* final_rgb, float* final_depth, float* phi, float* dw,
                              float* weight_sum, float lambda_dist, float lambda_depth,
                              const float* bg3);

/* render_rays_kernel (compositing.cu:5-78), the inference compositor: sample
 * i of ray r sits at offsets[r + rays_done] - base + i, the last sample's
 * delta is 1e-3, rays stop early once T < 1e-4; rgb has rgb_stride floats per
 * sample (3 in the reference).  rgb_true and phi are nullable. */
void orc_composite_infer(uint32_t R, uint32_t base, uint32_t rays_done, const uint32_t* offsets,
                         const uint32_t* counts, const float* t, const float* sigma, const float* rgb,
                         int rgb_stride, const float* rgb_true, float* final_rgb, float* final_depth, float* phi,
                         const float* bg3);

/* compute_color_grad (otherKernels.cu:303-409) with initialOffset = 0:
 * fp16 dL/dc [N][3] and fp32 dsigma [N]. */
void orc_color_grad(uint32_t R, const uint32_t* counts, const uint32_t* offsets, const float* t,
                    const float* density_out, const float* color_out, const float* phi,
                    const float* final_rgb, const float* dw, const float* weight_sum,
                    uint16_t* color_grad, float* dsigma, float loss_scale, float density_bias,
                    uint32_t total_rays);

/* compute_density_grad (otherKernels.cu:506-562): fp16 [N][16] from the color
 * head's dL/dinput fp16 [N][32] (first 16) plus dsigma into slot 0. */
void orc_density_grad(uint32_t N, const float* dsigma, const uint16_t* color_dx, uint16_t* density_grad);

/* updateMasterGrid (otherKernels.cu:677-690): EMA-max with decay. */
void orc_update_master_grid(const float* tmp, float* master, float decay, uint32_t n);

/* updateOccupancyGrid (otherKernels.cu:700-750): level-0 bits of every cascade
 * from the master grid; sum is the reduction of master over all cells. */
void orc_update_occupancy_bits(uint8_t* bits, const float* master, float sum, int total_cells,
                               int cells_per_cascade, int pyramid_cells, float min_optical_thickness,
                               float base_voxel);

/* buildMipmaps + bitfield_max_pool (InstantNerf.cu:1177-1204, otherKernels.cu:752-807). */
void orc_build_mipmaps(uint8_t* bits, const uint32_t* res3, int mip_levels, int num_cascades);

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11, "Parallel random numbers:
 * as easy as 1, 2, 3"): the occupancy refresh's generator in this build (the
 * reference draws from cuRAND's Philox state, whose counter/key use is not
 * reproducible here).  c[4] is the counter in, the block out. */
void orc_philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1);

/* sampleAABB (otherKernels.cu:591-648; modes 1 every cell of
 * [cell_offset, cell_offset + N), 2 a random cell of [cell_offset,
 * cell_offset + total_cells)) and sampleOccupiedAABB (:852-888; mode 0, a
 * random entry of list[0, list_count)) with this build's draws: sample idx
 * takes the Philox4x32-10 block of counter (idx, 0, seed lo, seed hi) under key
 * (0x3DA3ACB5, 0xA79C5F42), each output u as (u >> 8) 2^-24 + 2^-25; out4
 * [N][4] = contracted position, cell id (int bits). */
void orc_occ_sample(float* out4, int N, int mode, int total_cells, int cell_offset, const int* list, int list_count,
                    uint64_t seed, const uint32_t* res3, const float* mn, const float* mx);

/* updateTmpGrid (otherKernels.cu:650-675): tmp[cell] = max(tmp[cell],
 * e^min(logit - bias, 8)) with logit = density_out[16 idx] (orc_expf). */
void orc_occ_tmp_max(const float* samples4, const float* density_out, float* tmp, float bias, int N);

/* pcg_hash (DataLoader.cu:542-546). */
uint32_t orc_pcg_hash(uint32_t input);

/* fetchRayChunkStreamingKernel (DataLoader.cu:548-661) for rays [0, size) of
 * a chunk: transforms [images][16] row-major, images_rgba [images][h][w][4];
 * outputs rays_o/rays_d [size][3], rgb [size][3], dense/sigma [size].  The
 * direction is normalised with a correctly rounded 1/sqrt (the reference uses
 * fast-math rsqrtf).  rec_* may be NULL when num_records == 0. */
void orc_fetch_ray_chunk(int offset, int size, int total_rays, uint32_t seed, int randomize, int width, int height,
                         float focal, const float* transforms, const uint8_t* images_rgba, float* rays_o,
                         float* rays_d, float* rgb, float* dense, float* sigma, const int* rec_frame,
                         const float* rec_u, const float* rec_v, const float* rec_D, const float* rec_sigma,
                         uint32_t num_records, float dense_fraction, float uv_scale_x, float uv_scale_y,
                         const float* bg3, int holdout_every);

#ifdef __cplusplus
}
#endif
#endif
