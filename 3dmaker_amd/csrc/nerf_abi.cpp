// extern "C" surface of the NeRF side: the reference's launchers
// (modules/NeRF/InstantNerf.h:385-568), launchers for the kernels the
// reference launches inline, and the flat handle API over InstantNerf.
// Exceptions never cross this boundary (abi_error.h).
#include "InstantNerf.h"
#include "nerf_abi.h"
#include "nerf_capi.h"

#include "abi_error.h"
#include "capi_handles.h"
#include "nerf.h"
#include "nerf_heads.h"
#include "nerf_math.h"
#include "occupancy.h"

#include <cstddef>
#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>

using graft::guarded;

static_assert(sizeof(InerfOptions) == sizeof(NerfOptions), "InerfOptions must mirror NerfOptions");
static_assert(offsetof(InerfOptions, levelsMipmap) == offsetof(NerfOptions, levelsMipmap), "layout");
static_assert(offsetof(InerfOptions, growthFactor) == offsetof(NerfOptions, growthFactor), "layout");
static_assert(offsetof(InerfOptions, lossScale) == offsetof(NerfOptions, lossScale), "layout");
static_assert(offsetof(InerfOptions, bgColor) == offsetof(NerfOptions, bgColor), "layout");
static_assert(offsetof(InerfOptions, densityBias) == offsetof(NerfOptions, densityBias), "layout");
static_assert(offsetof(InerfOptions, isProfiling) == offsetof(NerfOptions, isProfiling), "layout");

namespace {

// Scratch of the launchers, one set per (device, stream): the compactions'
// block sums and results, the march store (kMaxHits floats per ray) and the
// sum's partials; grown on demand, kept until the process ends.  Calls on one
// stream run in order and share a set; calls on different streams never do.
struct LauncherScratch {
    graft::Workspace words, tstore, partials;
};

std::mutex g_mu;

LauncherScratch& scratch_of(hipStream_t s)
{
    int dev = 0;
    GRAFT_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    static auto* sets = new std::map<std::pair<int, hipStream_t>, std::unique_ptr<LauncherScratch>>();
    auto& p = (*sets)[{dev, s}];
    if (!p) p.reset(new LauncherScratch());
    return *p;
}

uint32_t* march_scratch(hipStream_t s, size_t words)
{
    return static_cast<uint32_t*>(scratch_of(s).words.get(words * sizeof(uint32_t)));
}

float* march_tstore(hipStream_t s, size_t floats)
{
    return static_cast<float*>(scratch_of(s).tstore.get(floats * sizeof(float)));
}

graft::OccGrid occ_grid(const uint8_t* bits, uint3 res, float3 mn, float3 mx, int cascades, int mips)
{
    graft::OccGrid g{};
    g.bits = bits;
    g.res = res;
    g.aabb_min = mn;
    g.aabb_max = mx;
    g.cascades = cascades;
    g.mip_levels = mips;
    return g;
}

// float4 stores need 16-byte alignment (the reference's vector stores do too).
void require_aligned16(const void* p, const char* what)
{
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
        throw std::runtime_error(std::string(what) + " must be 16-byte aligned");
}

// Exclusive scan of counts into offsets with the library's scratch; returns
// the scratch (result = {R, total samples}) and writes the total to *total.
graft::MarchScratch scan_all(uint32_t R, const uint32_t* counts, uint32_t* offsets, hipStream_t s, uint32_t* total)
{
    const size_t words = graft::march_scratch_words(R);
    uint32_t* sc = march_scratch(s, words);
    graft::MarchScratch ms{sc, sc + (words - 2)};
    graft::scan_counts(R, counts, 0xffffffffu, offsets, ms, s);
    if (total) {
        uint32_t h[2] = {0, 0};
        GRAFT_HIP_CHECK(hipMemcpyAsync(h, ms.result, sizeof(h), hipMemcpyDeviceToHost, s));
        GRAFT_HIP_CHECK(hipStreamSynchronize(s));
        *total = h[1];
    }
    return ms;
}

// processRaysChunk / processRaysChunkLinear (processRays.cu:357-464, 551-624):
// sparse march, scan, compaction (Morton-sorted when keys are given), batch.
void chunk_pipeline(uint32_t R, const float3* o, const float3* d, const float3* di, const float* nears,
                    const float* fars, const graft::OccGrid& g, int K, uint32_t* morton, float* t_sparse,
                    uint32_t* counts, uint32_t* offsets, uint32_t* keys_in, uint32_t* idx_in, uint32_t* keys_out,
                    uint32_t* idx_out, float* pos, uint32_t* ridx, float* t_sorted, hipStream_t s)
{
    if (R == 0) return;
    require_aligned16(pos, "d_mlp_positions_batch");
    graft::march_sparse(R, o, d, di, nears, fars, g, K, counts, t_sparse, morton, s);
    uint32_t total = 0;
    const graft::MarchScratch ms = scan_all(R, counts, offsets, s, &total);
    if (total == 0) return;
    graft::compact_sparse(R, offsets, ms.result, total, morton, keys_in, idx_in, s);
    const uint32_t* order = idx_in;
    if (keys_in) {
        graft::sort_pairs_u32(keys_in, keys_out, idx_in, idx_out, total, s);
        order = idx_out;
    }
    graft::sparse_batch(ms.result, total, order, t_sparse, o, d, g.aabb_min, g.aabb_max,
                        reinterpret_cast<float4*>(pos), ridx, t_sorted, s);
}

float* reduce_partials(hipStream_t s)
{
    return static_cast<float*>(scratch_of(s).partials.get(1024 * sizeof(float)));
}

}  // namespace

struct Inerf {
    InstantNerf nerf;
    TmlpGrid density{nullptr, false};
    TmlpNet color{nullptr, false};
};

extern "C" {

int processRaysHitLinear(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                         const float3* rays_d_inv, const float* nears, const float* fars,
                         const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                         const float3 aabb_max, const int numCascades, const int mipmapLevels,
                         const int samplesPerVoxel, const int batchSize, uint32_t* totalHits,
                         uint32_t* d_active_rays_count, uint32_t* d_num_steps, uint32_t* d_ray_offsets,
                         float* d_mlp_positions_batch, uint32_t* d_ray_indices, float* d_t_sorted,
                         uint32_t* d_block_sums, hipStream_t stream)
{
    int active = 0;
    guarded("processRaysHitLinear", [&] {
        if (batchSize < 0) throw std::runtime_error("batchSize must be >= 0");
        require_aligned16(d_mlp_positions_batch, "d_mlp_positions_batch");
        const graft::OccGrid g =
            occ_grid(occupancy_grid, grid_resolution, aabb_min, aabb_max, numCascades, mipmapLevels);
        const size_t words = graft::march_scratch_words(num_rays);
        (void)d_block_sums;  // sized (R + 1023) / 1024 by reference callers: too small, not used
        uint32_t* sc = march_scratch(stream, words);
        graft::MarchScratch ms{sc, sc + (words - 2)};
        float* ts = march_tstore(stream, graft::march_store_floats(std::max<uint32_t>(num_rays, 1)));
        graft::march_store(num_rays, rays_o, rays_d, rays_d_inv, nears, fars, g, samplesPerVoxel, d_num_steps, ts,
                           stream);
        graft::march_compact_stored(num_rays, rays_o, rays_d, g, (uint32_t)batchSize, d_num_steps, ts, 0, d_ray_offsets,
                                    d_t_sorted, d_ray_indices, reinterpret_cast<float4*>(d_mlp_positions_batch), ms,
                                    stream);
        uint32_t h[2] = {0, 0};
        GRAFT_HIP_CHECK(hipMemcpyAsync(h, ms.result, sizeof(h), hipMemcpyDeviceToHost, stream));
        GRAFT_HIP_CHECK(hipStreamSynchronize(stream));
        if (d_active_rays_count)
            GRAFT_HIP_CHECK(hipMemcpy(d_active_rays_count, &h[0], sizeof(uint32_t), hipMemcpyHostToDevice));
        if (totalHits) *totalHits = h[1];
        active = (int)h[0];
    });
    return active;
}

void processRaysHitData(const uint32_t num_rays, const float3* rays_o, const float3* rays_d, const float3* rays_d_inv,
                        const float* nears, const float* fars, const uint8_t* occupancy_grid,
                        const uint3 grid_resolution, const float3 aabb_min, const float3 aabb_max,
                        const int numCascades, const int mipmapLevels, const int samplesPerVoxel,
                        uint32_t* d_num_steps, uint32_t* d_ray_offsets, uint32_t* d_block_sums, hipStream_t stream)
{
    guarded("processRaysHitData", [&] {
        (void)d_block_sums;  // sized (R + 1023) / 1024 by reference callers; the library's scratch is used
        if (num_rays == 0) return;
        const graft::OccGrid g =
            occ_grid(occupancy_grid, grid_resolution, aabb_min, aabb_max, numCascades, mipmapLevels);
        graft::march_count(num_rays, rays_o, rays_d, rays_d_inv, nears, fars, g, samplesPerVoxel, d_num_steps,
                           stream);
        scan_all(num_rays, d_num_steps, d_ray_offsets, stream, nullptr);
    });
}

int processRaysHitPositions(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                            const float3* rays_d_inv, const float* nears, const float* fars,
                            const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                            const float3 aabb_max, const int numCascades, const int mipmapLevels,
                            const int samplesPerVoxel, const uint32_t rays_done, const int batchSize,
                            uint32_t* totalHits, uint32_t* out_base, uint32_t* d_num_steps, uint32_t* d_ray_offsets,
                            float* d_mlp_positions_batch, uint32_t* d_ray_indices, uint32_t* d_active_rays_count,
                            float* d_t_sorted, uint32_t* d_block_sums, hipStream_t stream)
{
    int active = 0;
    guarded("processRaysHitPositions", [&] {
        (void)d_block_sums;
        if (batchSize < 0) throw std::runtime_error("batchSize must be >= 0");
        if (!totalHits || !out_base) throw std::runtime_error("totalHits and out_base must not be NULL");
        require_aligned16(d_mlp_positions_batch, "d_mlp_positions_batch");
        const graft::OccGrid g =
            occ_grid(occupancy_grid, grid_resolution, aabb_min, aabb_max, numCascades, mipmapLevels);
        const uint32_t left = rays_done < num_rays ? num_rays - rays_done : 0u;
        // scratch: the re-marched rays' counts [left], then the cutoff result [4]
        uint32_t* sc = march_scratch(stream, (size_t)left + 4);
        uint32_t* res = sc + left;
        graft::cutoff_from(num_rays, d_ray_offsets, d_num_steps, (uint32_t)batchSize, rays_done,
                           d_active_rays_count, res, stream);
        uint32_t h[4] = {0, 0, 0, 0};
        GRAFT_HIP_CHECK(hipMemcpyAsync(h, res, sizeof(h), hipMemcpyDeviceToHost, stream));
        GRAFT_HIP_CHECK(hipStreamSynchronize(stream));
        if (h[3] <= rays_done) {  // the first ray does not fit (or no rays are left)
            *totalHits = 0;
            return;
        }
        const uint32_t batch_rays = h[0], total = h[1], base = h[2];
        *out_base = base;
        *totalHits = total;
        // march_rays_dda_offset (processRays.cu:801-929) re-marches the batch's
        // rays; here they are marched into the store and gathered per sample
        float* ts = march_tstore(stream, graft::march_store_floats(batch_rays));
        const size_t r0 = rays_done;
        graft::march_store(batch_rays, rays_o + r0, rays_d + r0, rays_d_inv + r0, nears + r0, fars + r0, g,
                           samplesPerVoxel, sc, ts, stream);
        graft::gather_stored(total, rays_o + r0, rays_d + r0, g, d_ray_offsets + r0, base, ts, res, d_t_sorted,
                             d_ray_indices, reinterpret_cast<float4*>(d_mlp_positions_batch), stream);
        active = (int)batch_rays;
    });
    return active;
}

void launchMarchRaysDDA(const uint32_t num_rays, const float3* rays_o, const float3* rays_d, const float3* rays_d_inv,
                        const float* nears, const float* fars, const uint8_t* occupancy_grid,
                        const uint3 grid_resolution, const float3 aabb_min, const float3 aabb_max,
                        const int numCascades, const int mipmapLevels, const int samplesPerVoxel,
                        uint32_t* packed_coords_out, float* t_hits_out, uint32_t* num_steps_per_ray,
                        hipStream_t stream)
{
    guarded("launchMarchRaysDDA", [&] {
        const graft::OccGrid g =
            occ_grid(occupancy_grid, grid_resolution, aabb_min, aabb_max, numCascades, mipmapLevels);
        graft::march_sparse(num_rays, rays_o, rays_d, rays_d_inv, nears, fars, g, samplesPerVoxel,
                            num_steps_per_ray, t_hits_out, packed_coords_out, stream);
    });
}

void processRaysChunk(const uint32_t num_rays, const float3* rays_o, const float3* rays_d, const float3* rays_d_inv,
                      const float* nears, const float* fars, const uint8_t* occupancy_grid,
                      const uint3 grid_resolution, const float3 aabb_min, const float3 aabb_max,
                      const int numCascades, const int mipmapLevels, const int samplesPerVoxel,
                      uint32_t* d_sparse_morton, float* d_sparse_ts, uint32_t* d_num_steps, uint32_t* d_ray_offsets,
                      uint32_t* d_dense_morton_keys_in, uint32_t* d_dense_sparse_indices_in,
                      uint32_t* d_dense_morton_keys_out, uint32_t* d_dense_sparse_indices_out,
                      float* d_mlp_positions_batch, uint32_t* d_ray_indices, float* d_t_sorted, hipStream_t stream)
{
    guarded("processRaysChunk", [&] {
        if (!d_sparse_morton || !d_dense_morton_keys_in || !d_dense_morton_keys_out || !d_dense_sparse_indices_out)
            throw std::runtime_error("the Morton key and sorted index buffers must not be NULL");
        const graft::OccGrid g =
            occ_grid(occupancy_grid, grid_resolution, aabb_min, aabb_max, numCascades, mipmapLevels);
        chunk_pipeline(num_rays, rays_o, rays_d, rays_d_inv, nears, fars, g, samplesPerVoxel, d_sparse_morton,
                       d_sparse_ts, d_num_steps, d_ray_offsets, d_dense_morton_keys_in, d_dense_sparse_indices_in,
                       d_dense_morton_keys_out, d_dense_sparse_indices_out, d_mlp_positions_batch, d_ray_indices,
                       d_t_sorted, stream);
    });
}

void processRaysChunkLinear(const uint32_t num_rays, const float3* rays_o, const float3* rays_d,
                            const float3* rays_d_inv, const float* nears, const float* fars,
                            const uint8_t* occupancy_grid, const uint3 grid_resolution, const float3 aabb_min,
                            const float3 aabb_max, const int numCascades, const int mipmapLevels,
                            const int samplesPerVoxel, float* d_sparse_ts, uint32_t* d_num_steps,
                            uint32_t* d_ray_offsets, uint32_t* d_dense_sparse_indices, float* d_mlp_positions_batch,
                            uint32_t* d_ray_indices, float* d_t_sorted, hipStream_t stream)
{
    guarded("processRaysChunkLinear", [&] {
        const graft::OccGrid g =
            occ_grid(occupancy_grid, grid_resolution, aabb_min, aabb_max, numCascades, mipmapLevels);
        chunk_pipeline(num_rays, rays_o, rays_d, rays_d_inv, nears, fars, g, samplesPerVoxel, nullptr, d_sparse_ts,
                       d_num_steps, d_ray_offsets, nullptr, d_dense_sparse_indices, nullptr, nullptr,
                       d_mlp_positions_batch, d_ray_indices, d_t_sorted, stream);
    });
}

void launchComputeRealSHDegree3(const uint32_t total_hits, const float3* d_directions, float* d_out_sh,
                                hipStream_t stream)
{
    guarded("launchComputeRealSHDegree3", [&] {
        if (total_hits == 0) return;
        require_aligned16(d_out_sh, "d_out_sh");
        graft::sh_degree3(total_hits, d_directions, d_out_sh, stream);
    });
}

size_t nerfHeadsPackedBytes(void) { return graft::nerf_heads_packed_bytes(); }

void launchNerfHeadsPack(const GRAFT_HALF* const* d_density_w, const float* const* d_density_b,
                         const GRAFT_HALF* const* d_color_w, const float* const* d_color_b, void* d_packed,
                         hipStream_t stream)
{
    guarded("launchNerfHeadsPack", [&] {
        if (!d_density_w || !d_density_b || !d_color_w || !d_color_b || !d_packed)
            throw std::runtime_error("null argument");
        graft::nerf_heads_pack(graft::NerfHeadsWeights{d_density_w, d_density_b, d_color_w, d_color_b}, d_packed,
                               stream);
    });
}

void launchNerfHeadsForward(const void* d_packed, const GRAFT_HALF* d_enc, int enc_plane, int levels,
                            const float3* d_dirs, const uint32_t* d_ray_indices, int num_samples,
                            float density_bias, int color_activation, float* d_sigma, float* d_density_out,
                            float* d_color_out, GRAFT_HALF* d_color_in, hipStream_t stream)
{
    guarded("launchNerfHeadsForward", [&] {
        if (num_samples < 0) throw std::runtime_error("num_samples must be >= 0");
        if (!d_packed || !d_enc || !d_dirs || !d_ray_indices || !d_sigma || !d_color_out)
            throw std::runtime_error("null argument");
        graft::NerfHeadsFwd h;
        h.packed = d_packed;
        h.enc = d_enc;
        h.enc_plane = enc_plane;
        h.levels = levels;
        h.dirs = d_dirs;
        h.ray_idx = d_ray_indices;
        h.density_bias = density_bias;
        h.out_act = color_activation;
        h.sigma = d_sigma;
        h.density_out = d_density_out;
        h.color_out = d_color_out;
        h.color_in = d_color_in;
        graft::nerf_heads_forward(h, num_samples, stream);
    });
}

static graft::NerfHeadsBwd heads_bwd(const void* d_packed, const GRAFT_HALF* d_enc, int enc_plane, int levels,
                                     const GRAFT_HALF* d_color_in, const GRAFT_HALF* d_color_dy, const float* d_dsigma)
{
    if (!d_packed || !d_enc || !d_color_in || !d_color_dy || !d_dsigma) throw std::runtime_error("null argument");
    graft::NerfHeadsBwd h;
    h.packed = d_packed;
    h.enc = d_enc;
    h.enc_plane = enc_plane;
    h.levels = levels;
    h.color_in = d_color_in;
    h.color_dy = d_color_dy;
    h.dsigma = d_dsigma;
    return h;
}

void launchNerfHeadsBackward(const void* d_packed, const GRAFT_HALF* d_enc, int enc_plane, int levels,
                             const GRAFT_HALF* d_color_in, const GRAFT_HALF* d_color_dy, const float* d_dsigma,
                             int num_samples, GRAFT_HALF* d_denc, GRAFT_HALF* d_density_dy, GRAFT_HALF* d_color_dx,
                             uint32_t* d_tile_live, hipStream_t stream)
{
    guarded("launchNerfHeadsBackward", [&] {
        if (num_samples < 0) throw std::runtime_error("num_samples must be >= 0");
        if (!d_denc) throw std::runtime_error("null argument");
        graft::NerfHeadsBwd h = heads_bwd(d_packed, d_enc, enc_plane, levels, d_color_in, d_color_dy, d_dsigma);
        h.denc = d_denc;
        h.density_dy = d_density_dy;
        h.color_dx = d_color_dx;
        h.tile_live = d_tile_live;
        graft::nerf_heads_dx(h, num_samples, stream);
    });
}

void launchNerfHeadsWeightGrads(const void* d_packed, const GRAFT_HALF* d_enc, int enc_plane, int levels,
                                const GRAFT_HALF* d_color_in, const GRAFT_HALF* d_color_dy, const float* d_dsigma,
                                const GRAFT_HALF* d_density_dy, const uint32_t* d_tile_live, int num_samples,
                                float* const* d_density_dw, float* const* d_density_db, float* const* d_color_dw,
                                float* const* d_color_db, hipStream_t stream)
{
    guarded("launchNerfHeadsWeightGrads", [&] {
        if (num_samples < 0) throw std::runtime_error("num_samples must be >= 0");
        if (!d_density_dw || !d_density_db || !d_color_dw || !d_color_db) throw std::runtime_error("null argument");
        graft::NerfHeadsBwd h = heads_bwd(d_packed, d_enc, enc_plane, levels, d_color_in, d_color_dy, d_dsigma);
        // read only: the density dL/dy launchNerfHeadsBackward stored for these inputs
        h.density_dy = const_cast<__half*>(reinterpret_cast<const __half*>(d_density_dy));
        h.tile_live = const_cast<uint32_t*>(d_tile_live);  // read only here
        // the whole GPU: two blocks per CU (one of each head)
        h.dw_blocks = graft::num_cus();
        graft::nerf_heads_dw(h, graft::NerfHeadsGrads{d_density_dw, d_density_db, d_color_dw, d_color_db},
                             num_samples, stream);
    });
}

void launchVolumeRendering(const uint32_t num_rays, const uint32_t* d_ray_offsets, const uint32_t* d_num_steps,
                           const float* d_t_sorted, const float* d_density_sigma, const float* d_depth_chunk,
                           const float* d_sigma_chunk, const float* d_rgb_output, const float* d_rgb_true,
                           float* d_render_rgb, float* d_render_depth, float* d_phi_out, float* d_dw_out,
                           float* d_weight_sum, float lambda_dist, float lambda_depth, float3 bg_color,
                           uint32_t base, uint32_t raysDone, hipStream_t stream)
{
    guarded("launchVolumeRendering", [&] {
        if (!d_dw_out) {  // render_rays_kernel (compositing.cu:5-78)
            graft::CompositeArgs a{};
            a.offsets = d_ray_offsets;
            a.counts = d_num_steps;
            a.t = d_t_sorted;
            a.sigma = d_density_sigma;
            a.rgb = d_rgb_output;
            a.rgb_stride = 3;
            a.rgb_true = d_rgb_true;
            a.final_rgb = d_render_rgb;
            a.final_depth = d_render_depth;
            a.phi = d_phi_out;
            a.bg = bg_color;
            graft::composite_infer(a, base, raysDone, nullptr, num_rays, stream);
            return;
        }
        graft::CompositeArgs a{};
        a.offsets = d_ray_offsets;
        a.counts = d_num_steps;
        a.t = d_t_sorted;
        a.sigma = d_density_sigma;
        a.depth_prior = d_depth_chunk;
        a.sigma_prior = d_sigma_chunk;
        a.rgb = d_rgb_output;
        a.rgb_stride = 3;
        a.rgb_true = d_rgb_true;
        a.final_rgb = d_render_rgb;
        a.final_depth = d_render_depth;
        a.phi = d_phi_out;
        a.dw = d_dw_out;
        a.weight_sum = d_weight_sum;
        a.lambda_dist = lambda_dist;
        a.lambda_depth = lambda_depth;
        a.bg = bg_color;
        graft::composite(a, nullptr, num_rays, stream);
    });
}

void launchComputeRayAabbInv(uint32_t num_rays, const float3* rays_o, const float3* rays_d, float3 aabb_min,
                             float3 aabb_max, int num_cascades, float3* rays_d_inv, float* nears, float* fars,
                             hipStream_t stream)
{
    guarded("launchComputeRayAabbInv", [&] {
        graft::ray_aabb_inv(num_rays, rays_o, rays_d, aabb_min, aabb_max, num_cascades, rays_d_inv, nears, fars,
                            stream);
    });
}

void launchComputeSHGather(const float3* d_chunk_d, const uint32_t* d_ray_indices, int offset, int batchSize,
                           float densityBias, float* d_density_out, GRAFT_HALF* d_color_in, float* d_density_sigma,
                           hipStream_t stream)
{
    guarded("launchComputeSHGather", [&] {
        if (batchSize < 0 || offset < 0) throw std::runtime_error("negative size");
        graft::sh_gather(d_chunk_d, d_ray_indices + offset, nullptr, (uint32_t)batchSize, densityBias, d_density_out,
                         d_color_in, d_density_sigma, stream);
    });
}

void launchComputeColorGrad(uint32_t numRays, uint32_t initialOffset, const uint32_t* num_steps,
                            const uint32_t* ray_offsets, const float* t_sorted, const float* density_mlp_out,
                            const float* color_mlp_out, const float* phi_chunk, const float* final_rgb,
                            const float* dw_out, const float* weight_sum, GRAFT_HALF* custom_color_grad,
                            float* tmp_dsigma, float loss_scale, float densityBias, uint32_t totalRaysBatch,
                            hipStream_t stream)
{
    guarded("launchComputeColorGrad", [&] {
        graft::ColorGradArgs a{};
        a.initial_offset = initialOffset;
        a.counts = num_steps;
        a.offsets = ray_offsets;
        a.t = t_sorted;
        a.density_out = density_mlp_out;
        a.color_out = color_mlp_out;
        a.color_stride = 3;
        a.phi = phi_chunk;
        a.final_rgb = final_rgb;
        a.dw = dw_out;
        a.weight_sum = weight_sum;
        a.color_grad = custom_color_grad;
        a.grad_stride = 3;
        a.dsigma = tmp_dsigma;
        a.loss_scale = loss_scale;
        a.bias = densityBias;
        a.total_rays = totalRaysBatch;
        graft::color_grad(a, nullptr, numRays, stream);
    });
}

void launchVolumeRenderingColorGrad(uint32_t num_rays, const uint32_t* d_ray_offsets, const uint32_t* d_num_steps,
                                    const float* d_t_sorted, const float* d_density_sigma, const float* d_depth_chunk,
                                    const float* d_sigma_chunk, const float* d_rgb_output, int rgb_stride,
                                    const float* d_rgb_true, float* d_render_rgb, float* d_render_depth,
                                    float* d_phi_out, float* d_dw_out, float* d_weight_sum, float lambda_dist,
                                    float lambda_depth, float3 bg_color, const float* density_mlp_out,
                                    GRAFT_HALF* custom_color_grad, int grad_stride, float* tmp_dsigma,
                                    float loss_scale, float densityBias, uint32_t totalRaysBatch, hipStream_t stream)
{
    guarded("launchVolumeRenderingColorGrad", [&] {
        if (rgb_stride < 3 || grad_stride < 3) throw std::runtime_error("row pitches must be >= 3");
        graft::CompositeArgs a{};
        a.offsets = d_ray_offsets;
        a.counts = d_num_steps;
        a.t = d_t_sorted;
        a.sigma = d_density_sigma;
        a.depth_prior = d_depth_chunk;
        a.sigma_prior = d_sigma_chunk;
        a.rgb = d_rgb_output;
        a.rgb_stride = rgb_stride;
        a.rgb_true = d_rgb_true;
        a.final_rgb = d_render_rgb;
        a.final_depth = d_render_depth;
        a.phi = d_phi_out;
        a.dw = d_dw_out;
        a.weight_sum = d_weight_sum;
        a.lambda_dist = lambda_dist;
        a.lambda_depth = lambda_depth;
        a.bg = bg_color;
        graft::ColorGradArgs g{};
        g.initial_offset = 0;
        g.counts = d_num_steps;
        g.offsets = d_ray_offsets;
        g.t = d_t_sorted;
        g.density_out = density_mlp_out;
        g.color_out = d_rgb_output;
        g.color_stride = rgb_stride;
        g.phi = d_phi_out;
        g.final_rgb = d_render_rgb;
        g.dw = d_dw_out;
        g.weight_sum = d_weight_sum;
        g.color_grad = custom_color_grad;
        g.grad_stride = grad_stride;
        g.dsigma = tmp_dsigma;
        g.loss_scale = loss_scale;
        g.bias = densityBias;
        g.total_rays = totalRaysBatch;
        graft::render_grad(a, g, nullptr, num_rays, stream);
    });
}

void launchComputeDensityGrad(uint32_t batch_size, const float* tmp_dsigma, const GRAFT_HALF* custom_dx_out,
                              GRAFT_HALF* custom_density_grad, hipStream_t stream)
{
    guarded("launchComputeDensityGrad", [&] {
        graft::density_grad(nullptr, batch_size, tmp_dsigma, custom_dx_out, custom_density_grad, stream);
    });
}

void launchUpdateMasterGrid(const float* tmpGrid, float* masterGrid, float decayValue, int N, hipStream_t stream)
{
    guarded("launchUpdateMasterGrid", [&] {
        if (N < 0) throw std::runtime_error("negative size");
        graft::update_master_grid(tmpGrid, masterGrid, decayValue, (uint32_t)N, stream);
    });
}

void launchReduceSum(const float* d_in, int n, float* d_out, hipStream_t stream)
{
    guarded("launchReduceSum", [&] {
        if (n < 0) throw std::runtime_error("negative size");
        graft::reduce_sum(d_in, (uint32_t)n, reduce_partials(stream), d_out, stream);
    });
}

void launchUpdateOccupancyGrid(uint32_t* d_occupancy_grid, const float* d_master_grid, const float* d_sum,
                               int total_cells, int cells_per_cascade, int pyramid_cells_per_cascade,
                               float min_optical_thickness, float base_voxel, hipStream_t stream)
{
    guarded("launchUpdateOccupancyGrid", [&] {
        graft::update_occupancy_bits(d_occupancy_grid, d_master_grid, d_sum, total_cells, cells_per_cascade,
                                     pyramid_cells_per_cascade, min_optical_thickness, base_voxel, stream);
    });
}

void launchBuildMipmaps(uint8_t* d_grid, uint3 grid_resolution, int mipmapLevels, int numCascades,
                        hipStream_t stream)
{
    guarded("launchBuildMipmaps",
            [&] { graft::build_mipmaps(d_grid, grid_resolution, mipmapLevels, numCascades, stream); });
}

void nerf_abi_echo_vec(float3 a, uint3 b, float* out)
{
    out[0] = a.x;
    out[1] = a.y;
    out[2] = a.z;
    out[3] = (float)b.x;
    out[4] = (float)b.y;
    out[5] = (float)b.z;
}

// ---- flat handle API ----

void inerf_default_options(InerfOptions* out)
{
    const NerfOptions d{};
    std::memcpy(out, &d, sizeof(d));
}

size_t inerf_options_size(void) { return sizeof(NerfOptions); }

Inerf* inerf_create(const InerfOptions* opts)
{
    Inerf* h = nullptr;
    guarded("inerf_create", [&] {
        NerfOptions o;
        std::memcpy(&o, opts, sizeof(o));
        h = new Inerf();
        try {
            h->nerf.init(o, TRAINING);
        } catch (...) {
            delete h;
            h = nullptr;
            throw;
        }
        h->density.g = h->nerf.densityMLP();
        h->color.n = h->nerf.colorMLP();
    });
    return h;
}

void inerf_destroy(Inerf* h) { delete h; }

#define NERF_CALL(name, body) guarded(name, [&] { if (!h) throw std::runtime_error("null handle"); body; })

int inerf_train(Inerf* h, const float* rays_o, const float* rays_d, const float* rays_depth, const float* rays_sigma,
                const float* rgb_true, uint32_t num_rays, int* train_step_count, uint32_t* hit_counts,
                float* rgb_out, hipStream_t stream)
{
    return NERF_CALL("inerf_train", {
        int dummy = 0;
        h->nerf.trainWithRaysHit(reinterpret_cast<const float3*>(rays_o), reinterpret_cast<const float3*>(rays_d),
                                 rays_depth, rays_sigma, rgb_true, num_rays,
                                 train_step_count ? *train_step_count : dummy, hit_counts, rgb_out, stream);
    });
}

int inerf_set_learning_rate(Inerf* h, float lr) { return NERF_CALL("inerf_set_learning_rate", h->nerf.setLearningRate(lr)); }
int inerf_set_next_rays(Inerf* h, const float* rays_o, const float* rays_d, uint32_t num_rays)
{
    return NERF_CALL("inerf_set_next_rays",
                     h->nerf.setNextRays(reinterpret_cast<const float3*>(rays_o),
                                         reinterpret_cast<const float3*>(rays_d), num_rays));
}
int inerf_set_step_limit(Inerf* h, int max_steps)
{
    return NERF_CALL("inerf_set_step_limit", h->nerf.setStepLimit(max_steps));
}
uint32_t inerf_last_rays_trained(Inerf* h) { return h ? h->nerf.lastRaysTrained() : 0u; }
int inerf_set_keep_color_dx(Inerf* h, int on)
{
    return NERF_CALL("inerf_set_keep_color_dx", h->nerf.setKeepColorDx(on != 0));
}
int inerf_set_bg_color(Inerf* h, float r, float g, float b)
{
    return NERF_CALL("inerf_set_bg_color", h->nerf.setBgColor(make_float3(r, g, b)));
}
int inerf_set_profiling(Inerf* h, int on) { return NERF_CALL("inerf_set_profiling", h->nerf.setProfiling(on != 0)); }
int inerf_print_stats(Inerf* h) { return NERF_CALL("inerf_print_stats", h->nerf.printStats()); }
int inerf_stats(Inerf* h, char* buf, int len)
{
    if (!h) return 0;
    const std::string s = h->nerf.statsString();
    if (buf && len > 0) {
        const size_t n = std::min(s.size(), (size_t)len - 1);
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return (int)s.size();
}
int inerf_reset_stats(Inerf* h) { return NERF_CALL("inerf_reset_stats", h->nerf.resetStats()); }
int inerf_set_memory_mode(Inerf* h, int inference)
{
    return NERF_CALL("inerf_set_memory_mode", h->nerf.setMemoryMode(inference ? INFERENCE : TRAINING));
}
int inerf_render(Inerf* h, const float* rays_o, const float* rays_d, uint32_t num_rays, float* rgb_out,
                 hipStream_t stream)
{
    return NERF_CALL("inerf_render",
                     h->nerf.renderImageHit(reinterpret_cast<const float3*>(rays_o),
                                            reinterpret_cast<const float3*>(rays_d), num_rays, rgb_out, stream));
}
int inerf_query_occupancy(Inerf* h, const float* pos, int n, uint32_t* words_out, float min_optical,
                          hipStream_t stream)
{
    return NERF_CALL("inerf_query_occupancy", h->nerf.queryOccupancyGrid(pos, n, words_out, min_optical, stream));
}
int inerf_query_density_logit(Inerf* h, const float* pos, int n, float* logit_out, hipStream_t stream)
{
    return NERF_CALL("inerf_query_density_logit", h->nerf.queryDensityLogit(pos, n, logit_out, stream));
}
int inerf_query_radiance(Inerf* h, const float* pos, int n, float dx, float dy, float dz, float* rgb_out,
                         hipStream_t stream)
{
    return NERF_CALL("inerf_query_radiance",
                     h->nerf.queryRadiance(pos, n, make_float3(dx, dy, dz), rgb_out, stream));
}
int inerf_build_occupancy_bitgrid(Inerf* h, uint8_t* bits_out, float min_density, hipStream_t stream)
{
    return NERF_CALL("inerf_build_occupancy_bitgrid", h->nerf.buildOccupancyBitgrid(bits_out, min_density, stream));
}

int inerf_update_occupancy(Inerf* h, hipStream_t stream)
{
    return NERF_CALL("inerf_update_occupancy", h->nerf.updateOccupancy(stream));
}
size_t inerf_occupancy_bytes(Inerf* h) { return h ? h->nerf.occupancyBytes() : 0; }
int inerf_get_occupancy(Inerf* h, uint8_t* host_bits)
{
    return NERF_CALL("inerf_get_occupancy", {
        GRAFT_HIP_CHECK(hipDeviceSynchronize());
        GRAFT_HIP_CHECK(hipMemcpy(host_bits, h->nerf.occupancyGrid(), h->nerf.occupancyBytes(), hipMemcpyDeviceToHost));
    });
}
int inerf_set_occupancy(Inerf* h, const uint8_t* host_bits)
{
    return NERF_CALL("inerf_set_occupancy", h->nerf.setOccupancyBits(host_bits));
}
int inerf_get_master_grid(Inerf* h, float* host_cells)
{
    return NERF_CALL("inerf_get_master_grid", {
        const NerfOptions& o = h->nerf.options();
        const size_t n = (size_t)o.numCascades * o.gridResolution.x * o.gridResolution.y * o.gridResolution.z;
        GRAFT_HIP_CHECK(hipDeviceSynchronize());
        GRAFT_HIP_CHECK(hipMemcpy(host_cells, h->nerf.masterOccupancyGrid(), n * sizeof(float), hipMemcpyDeviceToHost));
    });
}
int inerf_refresh_buffers(Inerf* h, InerfRefreshBuffers* out)
{
    return NERF_CALL("inerf_refresh_buffers", {
        const InstantNerf::RefreshBuffers r = h->nerf.refreshBuffers();
        out->samples = reinterpret_cast<float*>(r.samples);
        out->density_out = r.density_out;
        out->tmp_grid = r.tmp_grid;
        out->active_list = r.active_list;
        out->active_count = r.active_count;
        out->last_count = r.lastCount;
        out->density_stride = r.densityStride;
        out->density_order = r.densityOrder;
    });
}
int inerf_step_buffers(Inerf* h, InerfStepBuffers* out)
{
    return NERF_CALL("inerf_step_buffers", {
        const InstantNerf::StepBuffers b = h->nerf.stepBuffers();
        out->num_steps = b.num_steps;
        out->ray_offsets = b.ray_offsets;
        out->positions = reinterpret_cast<float*>(b.positions);
        out->ray_indices = b.ray_indices;
        out->t_sorted = b.t_sorted;
        out->density_out = b.density_out;
        out->color_input = b.color_input;
        out->color_output = b.color_output;
        out->sigma = b.sigma;
        out->render_rgb = b.render_rgb;
        out->phi = b.phi;
        out->dw = b.dw;
        out->weight_sum = b.weight_sum;
        out->dsigma = b.dsigma;
        out->color_dx = b.color_dx;
        out->density_grad = b.density_grad;
        out->result = b.result;
        out->trainSteps = b.trainSteps;
        out->windowStart = b.windowStart;
        out->encodings = b.encodings;
        out->encodingPlane = b.encodingPlane;
        out->activationsSaved = b.activationsSaved;
        out->density_stride = b.densityStride;
    });
}
int inerf_save(Inerf* h, const char* path)
{
    return NERF_CALL("inerf_save", {
        if (!path) throw std::runtime_error("null path");
        h->nerf.save(path);
    });
}
int inerf_load(Inerf* h, const char* path)
{
    return NERF_CALL("inerf_load", {
        if (!path) throw std::runtime_error("null path");
        h->nerf.load(path);
        h->density.g = h->nerf.densityMLP();  // load() rebuilt both heads
        h->color.n = h->nerf.colorMLP();
    });
}
int inerf_get_options(Inerf* h, InerfOptions* out)
{
    return NERF_CALL("inerf_get_options", {
        if (!out) throw std::runtime_error("null output");
        std::memcpy(out, &h->nerf.options(), sizeof(NerfOptions));
    });
}

TmlpGrid* inerf_density(Inerf* h) { return h ? &h->density : nullptr; }
TmlpNet* inerf_color(Inerf* h) { return h ? &h->color : nullptr; }

void inerf_philox4x32_10(uint32_t* ctr, uint32_t k0, uint32_t k1) { graft::philox4x32_10_host(ctr, k0, k1); }

}  // extern "C"
