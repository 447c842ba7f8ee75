/*
 * Flat C handle API over InstantNerf (include/InstantNerf.h), for callers
 * that cannot use C++ (ctypes, cgo, JNI).  Each function mirrors one method of
 * the reference class modules/NeRF/InstantNerf.h:279-335; C++ exceptions are
 * caught and reported as a non-zero return plus tinymlp_last_error_message().
 * No counterpart exists in the reference, which is C++-only.
 */
#ifndef GRAFT_NERF_CAPI_H
#define GRAFT_NERF_CAPI_H

#include "nerf_abi.h"
#include "tinymlp_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Byte-for-byte the layout of NerfOptions (InstantNerf.h:35-76); C has no
 * default member values, so start from inerf_default_options(). */
typedef struct InerfOptions {
    uint32_t gridResolution[3];
    float aabbMin[3];
    float aabbMax[3];
    int levelsMipmap, numCascades, samplesPerVoxel;
    int densityHiddenDim, densityNumLayers;
    int colorHiddenDim, colorNumLayers;
    int hashTableSize, numLevels;
    float growthFactor;
    int baseResolution, featuresPerLevel;
    int renderBatchSize, batchSize, rayChunkSize;
    float lambdaDepth, lambdaDist, learningRate, beta1, beta2, epsilon, lossScale;
    float bgColor[3];
    float minDensityThreshold, decayValue, densityBias;
    uint8_t legacyRenderFlag, isProfiling;
} InerfOptions;

typedef struct Inerf Inerf;

/* Device pointers of the last training step (see InstantNerf::StepBuffers). */
typedef struct InerfStepBuffers {
    uint32_t* num_steps;
    uint32_t* ray_offsets;
    float* positions;       /* float4 [batch] */
    uint32_t* ray_indices;
    float* t_sorted;
    float* density_out;     /* [batch x density_stride]: density logit 0 first */
    GRAFT_HALF* color_input;
    float* color_output;    /* [batch x 8] */
    float* sigma;
    float* render_rgb;
    float* phi;
    float* dw;
    float* weight_sum;
    float* dsigma;
    GRAFT_HALF* color_dx;
    GRAFT_HALF* density_grad;
    uint32_t* result;       /* [2] active rays, compacted samples */
    int trainSteps;
    uint32_t windowStart;   /* first ray of the last step within the last call's rays */
    GRAFT_HALF* encodings;  /* [numLevels][encodingPlane] feature pairs of the last step */
    uint32_t encodingPlane;
    int activationsSaved;   /* 0: hidden activations recomputed, not stored; color_dx holds the logit features only,
                               and only after inerf_set_keep_color_dx(h, 1) */
    int density_stride;     /* 16, or 1 (the logit alone) */
} InerfStepBuffers;

/* InstantNerf::refreshBuffers (introspection, no reference counterpart). */
typedef struct InerfRefreshBuffers {
    float* samples;         /* float4 [last_count]: contracted position, cell id bits */
    float* density_out;     /* [last_count x density_stride]: density logit 0 first */
    float* tmp_grid;        /* [cascades x cells] */
    int* active_list;
    int* active_count;
    int last_count;
    int density_stride;     /* 1 or 16 */
    const uint32_t* density_order; /* nullable: density_out row j is sample density_order[j] */
} InerfRefreshBuffers;

void inerf_default_options(InerfOptions* out);
size_t inerf_options_size(void);
Inerf* inerf_create(const InerfOptions* opts);
void inerf_destroy(Inerf* h);
int inerf_train(Inerf* h, const float* rays_o, const float* rays_d, const float* rays_depth, const float* rays_sigma,
                const float* rgb_true, uint32_t num_rays, int* train_step_count, uint32_t* hit_counts,
                float* rgb_out, hipStream_t stream);
int inerf_set_learning_rate(Inerf* h, float lr);
/* InstantNerf::setNextRays (no reference counterpart): rays of the next
 * inerf_train call, compacted beside the current call's last step. */
int inerf_set_next_rays(Inerf* h, const float* rays_o, const float* rays_d, uint32_t num_rays);
int inerf_set_bg_color(Inerf* h, float r, float g, float b);
/* InstantNerf::setStepLimit / lastRaysTrained (no reference counterpart): at
 * most max_steps optimizer steps per inerf_train call (0: no limit). */
int inerf_set_step_limit(Inerf* h, int max_steps);
uint32_t inerf_last_rays_trained(Inerf* h);
/* InstantNerf::setKeepColorDx (no reference counterpart; introspection for
 * tests): on != 0 keeps each step's colour dL/d(input) in the step buffers'
 * color_dx, which the step with recomputed activations otherwise does not
 * store. */
int inerf_set_keep_color_dx(Inerf* h, int on);
int inerf_set_profiling(Inerf* h, int on);
int inerf_print_stats(Inerf* h);
/* Per-stage profiling means as "stage:mean_ms:calls;..." into buf (NUL-terminated,
 * truncated to len); returns the full length.  inerf_reset_stats clears them. */
int inerf_stats(Inerf* h, char* buf, int len);
int inerf_reset_stats(Inerf* h);
/* InstantNerf::setMemoryMode (InstantNerf.h:294): 0 TRAINING, 1 INFERENCE. */
int inerf_set_memory_mode(Inerf* h, int inference);
/* InstantNerf::renderImageHit (InstantNerf.h:317-323): rays as float3 [n],
 * rgb_out [n x 3] device pointers. */
int inerf_render(Inerf* h, const float* rays_o, const float* rays_d, uint32_t num_rays, float* rgb_out,
                 hipStream_t stream);
/* InstantNerf::queryOccupancyGrid / queryDensityLogit / queryRadiance /
 * buildOccupancyBitgrid (InstantNerf.h:325-328); pos is [n x 3] on the device. */
int inerf_query_occupancy(Inerf* h, const float* pos, int n, uint32_t* words_out, float min_optical,
                          hipStream_t stream);
int inerf_query_density_logit(Inerf* h, const float* pos, int n, float* logit_out, hipStream_t stream);
int inerf_query_radiance(Inerf* h, const float* pos, int n, float dx, float dy, float dz, float* rgb_out,
                         hipStream_t stream);
int inerf_build_occupancy_bitgrid(Inerf* h, uint8_t* bits_out, float min_density, hipStream_t stream);
int inerf_update_occupancy(Inerf* h, hipStream_t stream);
size_t inerf_occupancy_bytes(Inerf* h);
int inerf_get_occupancy(Inerf* h, uint8_t* host_bits);
int inerf_set_occupancy(Inerf* h, const uint8_t* host_bits);
int inerf_get_master_grid(Inerf* h, float* host_cells);
int inerf_step_buffers(Inerf* h, InerfStepBuffers* out);
int inerf_refresh_buffers(Inerf* h, InerfRefreshBuffers* out);
/* InstantNerf::save / load (InstantNerf.h:333-334): the reference's .inerf
 * format ("INERF1", raw NerfOptions, hash table, density and colour weights,
 * master occupancy grid, bitfield).  load re-initialises the model with the
 * file's options; inerf_get_options reads them back. */
int inerf_save(Inerf* h, const char* path);
int inerf_load(Inerf* h, const char* path);
int inerf_get_options(Inerf* h, InerfOptions* out);
/* Non-owning views of the two heads (tmlp_*_destroy on them is a no-op); they
 * stay valid across inerf_load. */
TmlpGrid* inerf_density(Inerf* h);
TmlpNet* inerf_color(Inerf* h);

/* Philox4x32-10 of the occupancy sampler on the host: ctr[4] in, out. */
void inerf_philox4x32_10(uint32_t* ctr, uint32_t k0, uint32_t k1);

#ifdef __cplusplus
}
#endif
#endif
