// InstantNerf: the NeRF training engine of the MI355X (gfx950) hot path.
// Drop-in for modules/NeRF/InstantNerf.h:35-335 of the reference: same
// NerfOptions layout (field order and types), MemoryMode, class name and
// training entry point, with cudaStream_t replaced by hipStream_t.
//
// What one trainWithRaysHit() step does (InstantNerf.cu:359-583) and how it
// differs from the reference:
//  - ray/AABB setup, DDA count + scan + cutoff + fill without host round
//    trips; the compacted sample and active-ray counts stay on the device and
//    every later kernel of the step reads them there;
//  - the ray window is marched once per call (and again after each occupancy
//    refresh), keeping every sample's t in a rayChunkSize x 1024 scratch
//    (4 KiB per ray); later hit batches of the window re-scan the stored
//    counts and gather their samples instead of re-marching the window;
//  - ONE forward of each MLP with activation saves (the reference runs an
//    inference pre-pass and then the training forward on identical inputs);
//  - the only device->host read per step is the active-ray count, which the
//    host needs to advance its ray cursor; it is issued right after the
//    compaction and waited for only after the whole step has been enqueued;
//  - batchSize must be >= 1024 (one ray's maximum sample count), so a step can
//    never end up with zero active rays (the reference prints and returns);
//  - occupancy refresh uses this library's own Philox4x32-10 stream and a
//    fixed-order sum, so its random samples are not the reference's.
// Rendering (renderImageHit, InstantNerf.cu:713-864; renderImage behind
// legacyRenderFlag) marches each ray chunk once and composites every hit
// batch with the inference compositor (compositing.cu:5-78).  MemoryMode only
// selects the render hit batch (renderBatchSize in INFERENCE, batchSize in
// TRAINING); training state stays allocated, and trainWithRaysHit requires
// TRAINING.  save/load write and read the reference's .inerf format
// (InstantNerf.cu:1206-1352) byte for byte; load re-initialises the model with
// the file's options.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>
#include <hip/hip_vector_types.h>

#include <cstdint>
#include <string>

#include "TinyMLP.h"
#include "TinyMLPHashGrid.h"

#ifndef MAX_HITS
#define MAX_HITS 1024  // per-ray sample cap (InstantNerf.h:24)
#endif

// InstantNerf.h:27-30
enum MemoryMode { TRAINING, INFERENCE };

// InstantNerf.h:35-76 (same field order, types and defaults).
struct NerfOptions {
    uint3 gridResolution = make_uint3(128, 128, 128);
    float3 aabbMin = make_float3(-1.0f, -1.0f, -1.0f);
    float3 aabbMax = make_float3(1.0f, 1.0f, 1.0f);
    int levelsMipmap = 4;
    int numCascades = 1;
    int samplesPerVoxel = 1;

    int densityHiddenDim = 64;
    int densityNumLayers = 2;

    int colorHiddenDim = 64;
    int colorNumLayers = 2;

    int hashTableSize = 1 << 19;
    int numLevels = 16;
    float growthFactor = 1.3819f;
    int baseResolution = 16;
    int featuresPerLevel = 2;

    int renderBatchSize = 2048 * 1024;
    int batchSize = 256 * 1024;
    int rayChunkSize = 256 * 1024;

    float lambdaDepth = 0.02882f;
    float lambdaDist = 0.0362781f;
    float learningRate = 1e-3f;
    float beta1 = 0.9f;
    float beta2 = 0.999f;
    float epsilon = 1e-8f;
    float lossScale = 1.0f;

    float3 bgColor = make_float3(1.0f, 1.0f, 1.0f);
    float minDensityThreshold = 0.01;
    float decayValue = 0.95f;
    float densityBias = 1.0f;

    bool legacyRenderFlag = false;
    bool isProfiling = false;
};

class InstantNerf {
public:
    InstantNerf() = default;
    ~InstantNerf();

    InstantNerf(const InstantNerf&) = delete;
    InstantNerf& operator=(const InstantNerf&) = delete;

    // InstantNerf.cu:282-339
    void init(const NerfOptions& opts, MemoryMode memMode = TRAINING);
    void printStats();
    void resetStats();
    void setLearningRate(float lr) { m_opts.learningRate = lr; }
    void setBgColor(float3 c) { m_opts.bgColor = c; }
    void setProfiling(bool p) { m_opts.isProfiling = p; }
    void setMemoryMode(MemoryMode mode);
    // Addition (no reference counterpart): the rays of the NEXT
    // trainWithRaysHit call, already written (queued on that call's stream)
    // before the current call.  The current call then compacts their first
    // hit batch on its side stream beside its last step, and the next call
    // with exactly these buffers and count starts training at once instead of
    // marching first.  The buffers must stay unchanged until that call; a call
    // with other rays, a render or an occupancy change in between discards the
    // prefetch (the call compacts as usual).  numRays = 0 clears.
    void setNextRays(const float3* d_rays_o, const float3* d_rays_d, uint32_t numRays);
    // Addition: at most maxSteps optimizer steps per trainWithRaysHit call
    // (0: no limit, the reference's behaviour); the call then returns after
    // training the rays [0, lastRaysTrained()), and the caller continues with
    // the rest.
    void setStepLimit(int maxSteps) { m_stepLimit = maxSteps > 0 ? maxSteps : 0; }
    uint32_t lastRaysTrained() const { return m_lastRaysTrained; }
    // Addition (introspection): keep the colour head's dL/d(input) of each
    // step in stepBuffers().color_dx.  The step with recomputed activations
    // (activationsSaved 0) reads none of it and stores it only when this is
    // on (off by default); the other path always stores it (its density
    // gradient glue reads it).
    void setKeepColorDx(bool keep) { m_keepColorDx = keep; }

    // InstantNerf.cu:359-583.  d_rays_depth / d_rays_sigma may be null (depth
    // supervision off), d_rgb_true must be set, hitCounts (host, nullable)
    // receives the compacted sample count of every step, d_rgb_out (nullable)
    // the composited colour of every ray.
    void trainWithRaysHit(const float3* d_rays_o, const float3* d_rays_d, const float* d_rays_depth,
                          const float* d_rays_sigma, const float* d_rgb_true, uint32_t numRays, int& trainStepCount,
                          uint32_t* hitCounts, float* d_rgb_out, hipStream_t stream);

    void renderImage(const float3* d_rays_o, const float3* d_rays_d, uint32_t numRays, float* d_rgb_out = nullptr,
                     hipStream_t stream = 0);
    void renderImageHit(const float3* d_rays_o, const float3* d_rays_d, uint32_t numRays, float* d_rgb_out,
                        hipStream_t stream);
    // InstantNerf.cu:941-984.  d_pos holds n contracted positions as x,y,z
    // triples; density/radiance queries need n % 16 == 0.
    void queryOccupancyGrid(const float* d_pos, int n, uint32_t* d_data_out, float minOpticalThreshold,
                            hipStream_t stream = 0);
    void queryDensityLogit(const float* d_pos, int n, float* d_logit_out, hipStream_t stream = 0);
    void queryRadiance(const float* d_pos, int n, float3 viewDir, float* d_rgb_out, hipStream_t stream = 0);
    void buildOccupancyBitgrid(uint8_t* d_out, float minDensityThreshold, hipStream_t stream = 0);

    const NerfOptions& options() const { return m_opts; }
    const uint8_t* occupancyGrid() { return d_occupancyGrid; }
    size_t occupancyBytes() { return m_occupancyBytes; }

    void save(const std::string& filename);
    void load(const std::string& filename);

    // ---- additions (no reference counterpart) ----
    TinyMLPHashGrid* densityMLP() { return m_densityMLP; }
    TinyMLP* colorMLP() { return m_colorMLP; }
    float* masterOccupancyGrid() { return d_masterOccupancyGrid; }
    // Overwrite the occupancy bitfield (host bytes, occupancyBytes() long).
    void setOccupancyBits(const uint8_t* host_bits);
    // Profiling results as "stage:mean_ms:calls;" entries (setProfiling(true)).
    std::string statsString() const;
    // Refresh the occupancy grid now (the step loop does it every 16 steps).
    void updateOccupancy(hipStream_t stream = 0);
    // Device buffers of the last step (introspection for tests).
    struct StepBuffers {
        uint32_t* num_steps;      // [rayChunkSize]
        uint32_t* ray_offsets;    // [rayChunkSize]
        float4* positions;        // [batchSize]
        uint32_t* ray_indices;    // [batchSize]
        float* t_sorted;          // [batchSize]
        float* density_out;       // [batchSize x densityStride]: density logit 0 first
        half* color_input;        // [batchSize x 32]
        float* color_output;      // [batchSize x 8] (padded head output)
        float* sigma;             // [batchSize]
        float* render_rgb;        // [rayChunkSize x 3]
        float* phi;               // [rayChunkSize x 3]
        float* dw;                // [batchSize]
        float* weight_sum;        // [rayChunkSize]
        float* dsigma;            // [batchSize]
        half* color_dx;           // [batchSize x 32]; with activationsSaved 0 only after setKeepColorDx(true)
        half* density_grad;       // [batchSize x 16]
        uint32_t* result;         // [2]: active rays, compacted samples of the last step
        int trainSteps;
        uint32_t windowStart;     // index of the last step's first ray in the last call's rays
        half* encodings;          // [numLevels][encodingPlane] feature pairs of the last step
        uint32_t encodingPlane;
        int activationsSaved;     // 0: the heads' hidden activations are recomputed, not kept in
                                  // the TinyMLP activation buffers; color_dx then holds only the
                                  // logit features (the SH features are 0)
        int densityStride;        // 16 (the density head's whole output) or 1 (the 16x16x32 heads:
                                  // the logit alone; the others are in color_input, sanitised)
    };
    StepBuffers stepBuffers() const;

    // Buffers of the last occupancy refresh (introspection for tests): the
    // sample buffer holds its last chunk (lastCount samples: the last cascade
    // of an early refresh, the last cascade chunk of a late one).
    struct RefreshBuffers {
        float4* samples;          // [lastCount]: contracted position, cell id (int bits)
        float* density_out;       // [lastCount x densityStride]: density logit 0 first
        float* tmp_grid;          // [numCascades x cells]
        int* active_list;         // occupied cells in cell order (late refresh)
        int* active_count;        // [1]
        int lastCount;
        int densityStride;        // 1 (the logit alone) or 16 (the density head's whole output)
        const uint32_t* densityOrder;  // nullable: density_out row j is sample densityOrder[j]
    };
    RefreshBuffers refreshBuffers() const;

private:
    void allocate();
    void freeBuffers();
    void earlyOccupancyGridUpdate(hipStream_t stream);
    void lateOccupancyGridUpdate(hipStream_t stream);
    void drawLateRefresh(long steps, hipStream_t stream);
    void finishOccupancyUpdate(hipStream_t stream);
    uint32_t renderHitBatch() const;

    NerfOptions m_opts{};
    MemoryMode m_memMode = TRAINING;
    TinyMLP* m_colorMLP = nullptr;
    TinyMLPHashGrid* m_densityMLP = nullptr;
    bool m_init = false;
    int m_trainSteps = 0;
    long m_gridVersion = 0;  // bumped whenever the occupancy bitfield changes
    uint32_t m_windowStart = 0;
    int m_stepLimit = 0;
    uint32_t m_lastRaysTrained = 0;
    bool m_keepColorDx = false;

    uint8_t* d_occupancyGrid = nullptr;
    size_t m_occupancyBytes = 0;
    float* d_masterOccupancyGrid = nullptr;
    void* m_buf = nullptr;  // opaque device buffer set
};
