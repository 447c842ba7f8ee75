// InstantNerf training engine on gfx950 (declared in include/InstantNerf.h).
//
// The step loop follows InstantNerf::trainWithRaysHit (InstantNerf.cu:359-583)
// stage by stage; the occupancy refresh follows earlyOccupancyGridUpdate /
// lateOccupancyGridUpdate (InstantNerf.cu:1009-1171).  Every launch of a step
// is sized for the step's upper bounds (rayChunkSize rays, batchSize samples)
// and reads the actual counts the compaction left in device memory.
#include "InstantNerf.h"

#include "hashgrid.h"
#include "scatter.h"
#include "mlp.h"
#include "nerf.h"
#include "nerf_heads.h"
#include "nerf_math.h"
#include "occupancy.h"
#include "optimizer.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <stdexcept>
#include <vector>

namespace {

// Events that only order streams on this device: a device-scope release is
// enough (the host never inspects them), and avoids the system-scope cache
// writeback of a default event between the kernels it separates.
constexpr unsigned kStreamEvent = hipEventDisableTiming | hipEventReleaseToDevice;

struct StageTimer {
    const char* name;
    hipEvent_t a, b;
};

// What one compaction produces.  Two sets alternate, so the compaction of the
// next hit batch can run on the side stream while the current step still
// reads its own set.
struct StepSet {
    uint32_t* offsets = nullptr;   // [rayChunkSize] per-ray sample offsets
    uint32_t* counts = nullptr;    // [rayChunkSize] per-ray sample counts (copied from the march store)
    float4* positions = nullptr;   // [batchSize]
    uint32_t* ray_idx = nullptr;   // [batchSize]
    float* t_sorted = nullptr;     // [batchSize]
    uint32_t* result = nullptr;    // [2] active rays, compacted samples
    uint32_t* h_result = nullptr;  // pinned copy of result
    hipEvent_t ev_result = nullptr, ev_ready = nullptr;
    uint32_t raysDone = 0;         // first ray of the batch in the call's rays
};

// A marched window of rays: ray setup, per-ray sample counts and the march
// store (march_store_floats(rayChunkSize)) of rays [c0, c1) of the buffers o, d.
struct MarchStore {
    float3* d_inv = nullptr;
    float* nears = nullptr;
    float* fars = nullptr;
    uint32_t* counts = nullptr;
    float* t = nullptr;
    uint32_t c0 = 0, c1 = 0;
    long version = -1;               // grid version it was marched on (-1: nothing)
    const float3* o = nullptr;
    const float3* d = nullptr;
};

struct NerfBuffers {
    // per step, rays: the current call's marched window, and the next call's
    // first window marched ahead (setNextRays) in the other store
    MarchStore ms[2];
    int cur = 0;                     // store of the current call
    uint32_t* block_sums = nullptr;
    StepSet set[2];
    int last_set = 0;                // set of the last training step
    // Rays of the next trainWithRaysHit call (setNextRays), and the first hit
    // batch of those rays, compacted beside the last step of the call before.
    struct Ahead {
        const float3* o = nullptr;
        const float3* d = nullptr;
        uint32_t n = 0;
    } next;
    struct Prefetched {
        bool valid = false;
        const float3* o = nullptr;
        const float3* d = nullptr;
        uint32_t n = 0;
        int set = 0;
        int store = 0;               // march store of its window
        long version = -1;           // grid version it was marched on
    } pre;
    float* render_rgb = nullptr;
    float* render_depth = nullptr;
    float* phi = nullptr;
    float* weight_sum = nullptr;
    // per step, samples
    float* density_out = nullptr;
    float* sigma = nullptr;
    float* dw = nullptr;
    float* dsigma = nullptr;
    __half* color_dx = nullptr;
    __half* enc_planar = nullptr;    // [L][Bn] feature pairs: the step's encodings, level-major
    void* heads_packed = nullptr;    // both heads' weights packed for nerf_heads.hip (null: other shapes)
    uint32_t* tile_live = nullptr;   // [Bn / 16 + 1]: 16-sample tiles with a nonzero gradient (dX -> dW)
    // occupancy
    float* tmp_grid = nullptr;
    float4* occ_samples = nullptr;
    float* occ_density = nullptr;
    __half* occ_enc = nullptr;       // [capacity x 2L] encodings of the refresh samples (level-major with the heads)
    // the refresh with the 16x16x32 density head: its own packed fragments
    // (packed at the refresh's start), the samples in spatial order
    void* occ_packed = nullptr;
    float4* occ_sorted = nullptr;
    uint32_t* occ_perm = nullptr;
    graft::OccSortScratch occ_sort{};
    bool occ_last_sorted = false;  // the last chunk's densities are in occ_perm's order
    float* partials = nullptr;
    float* sum = nullptr;
    int* active_list = nullptr;
    int* active_count = nullptr;
    uint32_t* list_scratch = nullptr;
    int occ_capacity = 0;
    int occ_last_count = 0;   // samples of the last refresh's last chunk
    // a late refresh's samples drawn a step ahead (one cascade): the step
    // count and grid version they were drawn for (-1: none)
    long drawn_steps = -1;
    long drawn_version = -1;
    // inference render / queries (allocated on first use, sized to the hit batch)
    struct Render {
        uint32_t cap = 0;
        float4* positions = nullptr;
        uint32_t* ray_idx = nullptr;
        float* t = nullptr;
        float* density_out = nullptr;  // [cap x 16]
        __half* color_in = nullptr;    // [cap x 32]
        float* sigma = nullptr;
        float* rgb = nullptr;          // [cap x colour head width] (padded)
        float3* dir = nullptr;         // one view direction (queryRadiance)
    } render;
    // model views
    __half* color_in = nullptr;      // TinyMLP activation 0
    graft::GridMeta meta{};
    // Beside the main stream: `side` runs the ray setup, march and compaction
    // of the next hit batch and the MLP weight gradients and Adam updates;
    // `occ` runs the occupancy refresh.
    hipStream_t side = nullptr, occ = nullptr;
    hipStream_t cmp = nullptr;  // ray setup, march and compaction of the next hit batch
    hipEvent_t ev_fork = nullptr, ev_join = nullptr, ev_done = nullptr, ev_done_occ = nullptr;
    hipEvent_t ev_done_cmp = nullptr;
    hipEvent_t ev_dl = nullptr;      // main: this step's MLP output gradients are written
    hipEvent_t ev_occ_fork = nullptr;  // main: a refresh step's parameters are final (step start)
    hipEvent_t ev_opt = nullptr;       // side: the step's MLP Adam updates are done
    std::vector<StageTimer> pending;
    std::map<std::string, std::pair<double, long>> stats;
};

template <class T>
T* dalloc(size_t n)
{
    void* p = nullptr;
    if (n) GRAFT_HIP_CHECK(hipMalloc(&p, n * sizeof(T)));
    return static_cast<T*>(p);
}

template <class T>
void dfree(T*& p)
{
    if (p) (void)hipFree(p);
    p = nullptr;
}

int grid_cells(const NerfOptions& o) { return (int)(o.gridResolution.x * o.gridResolution.y * o.gridResolution.z); }

NerfBuffers& B(void* p) { return *static_cast<NerfBuffers*>(p); }

graft::OccGrid occ_grid(const NerfOptions& o, const uint8_t* bits)
{
    graft::OccGrid g{};
    g.bits = bits;
    g.res = o.gridResolution;
    g.aabb_min = o.aabbMin;
    g.aabb_max = o.aabbMax;
    g.cascades = o.numCascades;
    g.mip_levels = o.levelsMipmap;
    return g;
}

graft::MlpShape shape_of(const MLPOption& o) { return graft::MlpShape{o.inputDim, o.hiddenDim, o.outputDim, o.numLayers}; }

}  // namespace

InstantNerf::~InstantNerf() { freeBuffers(); }

void InstantNerf::freeBuffers()
{
    if (m_buf) {
        NerfBuffers& b = B(m_buf);
        for (MarchStore& M : b.ms) {
            dfree(M.d_inv);
            dfree(M.nears);
            dfree(M.fars);
            dfree(M.counts);
            dfree(M.t);
        }
        dfree(b.block_sums);
        for (StepSet& S : b.set) {
            dfree(S.offsets);
            dfree(S.counts);
            dfree(S.positions);
            dfree(S.ray_idx);
            dfree(S.t_sorted);
            dfree(S.result);
            if (S.h_result) (void)hipHostFree(S.h_result);
            if (S.ev_result) (void)hipEventDestroy(S.ev_result);
            if (S.ev_ready) (void)hipEventDestroy(S.ev_ready);
        }
        dfree(b.render_rgb);
        dfree(b.render_depth);
        dfree(b.phi);
        dfree(b.weight_sum);
        dfree(b.density_out);
        dfree(b.sigma);
        dfree(b.dw);
        dfree(b.dsigma);
        dfree(b.color_dx);
        dfree(b.enc_planar);
        dfree(b.heads_packed);
        dfree(b.tile_live);
        dfree(b.tmp_grid);
        dfree(b.occ_samples);
        dfree(b.occ_density);
        dfree(b.occ_enc);
        dfree(b.occ_packed);
        dfree(b.occ_sorted);
        dfree(b.occ_perm);
        dfree(b.occ_sort.counts);
        dfree(b.occ_sort.offsets);
        dfree(b.occ_sort.block_sums);
        dfree(b.occ_sort.result);
        dfree(b.occ_sort.rank);
        dfree(b.partials);
        dfree(b.sum);
        dfree(b.active_list);
        dfree(b.active_count);
        dfree(b.list_scratch);
        dfree(b.render.positions);
        dfree(b.render.ray_idx);
        dfree(b.render.t);
        dfree(b.render.density_out);
        dfree(b.render.color_in);
        dfree(b.render.sigma);
        dfree(b.render.rgb);
        dfree(b.render.dir);
        if (b.ev_fork) (void)hipEventDestroy(b.ev_fork);
        if (b.ev_join) (void)hipEventDestroy(b.ev_join);
        if (b.ev_done) (void)hipEventDestroy(b.ev_done);
        if (b.ev_done_occ) (void)hipEventDestroy(b.ev_done_occ);
        if (b.ev_dl) (void)hipEventDestroy(b.ev_dl);
        if (b.ev_occ_fork) (void)hipEventDestroy(b.ev_occ_fork);
        if (b.ev_opt) (void)hipEventDestroy(b.ev_opt);
        if (b.ev_done_cmp) (void)hipEventDestroy(b.ev_done_cmp);
        if (b.occ) (void)hipStreamDestroy(b.occ);
        if (b.side) (void)hipStreamDestroy(b.side);
        if (b.cmp) (void)hipStreamDestroy(b.cmp);
        for (auto& t : b.pending) {
            (void)hipEventDestroy(t.a);
            (void)hipEventDestroy(t.b);
        }
        delete &b;
        m_buf = nullptr;
    }
    dfree(d_occupancyGrid);
    dfree(d_masterOccupancyGrid);
    delete m_colorMLP;
    delete m_densityMLP;
    m_colorMLP = nullptr;
    m_densityMLP = nullptr;
    m_init = false;
}

// InstantNerf.cu:282-339
void InstantNerf::init(const NerfOptions& opts, MemoryMode memMode)
{
    freeBuffers();
    if (opts.batchSize < MAX_HITS)
        throw std::runtime_error("InstantNerf: batchSize must be >= 1024 (one ray's maximum sample count)");
    if (opts.rayChunkSize <= 0 || opts.rayChunkSize % 16)
        throw std::runtime_error("InstantNerf: rayChunkSize must be a positive multiple of 16");
    if (opts.featuresPerLevel != 2) throw std::runtime_error("InstantNerf: featuresPerLevel must be 2");
    m_opts = opts;
    m_memMode = memMode;
    m_trainSteps = 0;

    const int G = grid_cells(opts);
    const int N = opts.numCascades * G;
    const uint32_t S = graft::mip_offset(opts.gridResolution, opts.levelsMipmap);
    if (G % 32 || S % 32) throw std::runtime_error("InstantNerf: grid cells per cascade must be multiples of 32");
    m_occupancyBytes = ((size_t)S * opts.numCascades + 7) / 8;
    d_occupancyGrid = dalloc<uint8_t>(m_occupancyBytes);
    GRAFT_HIP_CHECK(hipMemset(d_occupancyGrid, 0, m_occupancyBytes));
    d_masterOccupancyGrid = dalloc<float>((size_t)N);
    GRAFT_HIP_CHECK(hipMemset(d_masterOccupancyGrid, 0, (size_t)N * sizeof(float)));

    MLPGridOptions dopt{};
    dopt.vectorDim = 4;
    dopt.hiddenDim = opts.densityHiddenDim;
    dopt.outputDim = 16;
    dopt.numLayers = opts.densityNumLayers;
    dopt.activationType = ACT_RELU;
    dopt.tableSize = opts.hashTableSize;
    dopt.numLevels = opts.numLevels;
    dopt.b = opts.growthFactor;
    dopt.lowestSize = opts.baseResolution;
    dopt.featuresLevel = opts.featuresPerLevel;
    const int densityInfer = std::max(G, opts.renderBatchSize);
    m_densityMLP = new TinyMLPHashGrid(dopt, opts.batchSize, densityInfer);

    MLPOption copt{};
    copt.inputDim = 32;
    copt.hiddenDim = opts.colorHiddenDim;
    copt.outputDim = 3;
    copt.numLayers = opts.colorNumLayers;
    copt.activationType = ACT_RELU;
    copt.outputActivation = OUT_ACT_SIGMOID;
    m_colorMLP = new TinyMLP(copt, opts.batchSize, opts.renderBatchSize);

    m_buf = new NerfBuffers();
    allocate();
    m_init = true;
    earlyOccupancyGridUpdate(0);
    GRAFT_HIP_CHECK(hipDeviceSynchronize());
}

void InstantNerf::allocate()
{
    NerfBuffers& b = B(m_buf);
    const size_t R = (size_t)m_opts.rayChunkSize, Bn = (size_t)m_opts.batchSize;
    const int G = grid_cells(m_opts);
    const int N = m_opts.numCascades * G;
    for (MarchStore& M : b.ms) {
        M.d_inv = dalloc<float3>(R);
        M.nears = dalloc<float>(R);
        M.fars = dalloc<float>(R);
        M.counts = dalloc<uint32_t>(R);
        M.t = dalloc<float>(graft::march_store_floats((uint32_t)R));
    }
    b.block_sums = dalloc<uint32_t>(graft::march_scratch_words((uint32_t)R));
    for (StepSet& S : b.set) {
        S.offsets = dalloc<uint32_t>(R);
        S.counts = dalloc<uint32_t>(R);
        S.positions = dalloc<float4>(Bn);
        S.ray_idx = dalloc<uint32_t>(Bn);
        S.t_sorted = dalloc<float>(Bn);
        S.result = dalloc<uint32_t>(2);
        GRAFT_HIP_CHECK(hipMemset(S.result, 0, 2 * sizeof(uint32_t)));
        GRAFT_HIP_CHECK(hipHostMalloc((void**)&S.h_result, 2 * sizeof(uint32_t), hipHostMallocDefault));
        GRAFT_HIP_CHECK(hipEventCreateWithFlags(&S.ev_result, hipEventDisableTiming));
        GRAFT_HIP_CHECK(hipEventCreateWithFlags(&S.ev_ready, kStreamEvent));
    }
    b.render_rgb = dalloc<float>(3 * R);
    b.render_depth = dalloc<float>(R);
    b.phi = dalloc<float>(3 * R);
    b.weight_sum = dalloc<float>(R);
    b.density_out = dalloc<float>(16 * Bn);
    b.sigma = dalloc<float>(Bn);
    b.dw = dalloc<float>(Bn);
    b.dsigma = dalloc<float>(Bn);
    b.color_dx = dalloc<__half>(32 * Bn);
    b.tmp_grid = dalloc<float>((size_t)N);
    const int halfN = N / 2;
    b.occ_capacity = std::max(G, halfN / std::max(1, m_opts.numCascades));
    b.occ_samples = dalloc<float4>((size_t)b.occ_capacity);
    // a late refresh with no occupied cell leaves its list samples as they
    // were: zeros here (cell 0) until a refresh writes them
    GRAFT_HIP_CHECK(hipMemset(b.occ_samples, 0, (size_t)b.occ_capacity * sizeof(float4)));
    b.occ_density = dalloc<float>((size_t)b.occ_capacity * 16);
    b.occ_enc = dalloc<__half>((size_t)b.occ_capacity * 2 * m_opts.numLevels);
    b.partials = dalloc<float>(1024);
    b.sum = dalloc<float>(1);
    b.active_list = dalloc<int>((size_t)N);
    b.active_count = dalloc<int>(1);
    b.list_scratch = dalloc<uint32_t>(graft::occ_list_scratch_words(N));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_fork, kStreamEvent));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_join, kStreamEvent));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_done, kStreamEvent));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_done_occ, kStreamEvent));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_dl, kStreamEvent));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_occ_fork, kStreamEvent));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_opt, kStreamEvent));
    GRAFT_HIP_CHECK(hipEventCreateWithFlags(&b.ev_done_cmp, kStreamEvent));
    GRAFT_HIP_CHECK(hipStreamCreateWithFlags(&b.occ, hipStreamNonBlocking));
    GRAFT_HIP_CHECK(hipStreamCreateWithFlags(&b.side, hipStreamNonBlocking));
    GRAFT_HIP_CHECK(hipStreamCreateWithFlags(&b.cmp, hipStreamNonBlocking));

    // The color head's activation-0 buffer receives the SH gather output directly.
    const TinyMLP::Buffers cb = m_colorMLP->buffers();
    __half* acts0 = nullptr;
    GRAFT_HIP_CHECK(hipMemcpy(&acts0, cb.activations, sizeof(acts0), hipMemcpyDeviceToHost));
    b.color_in = acts0;
    b.meta = graft::make_grid_meta(m_opts.hashTableSize, m_opts.numLevels, m_opts.growthFactor, m_opts.baseResolution);
    b.enc_planar = dalloc<__half>((size_t)2 * b.meta.numLevels * Bn);
    const TinyMLPHashGrid::Buffers dbuf = m_densityMLP->buffers();
    const graft::MlpShape dsh{2 * m_opts.numLevels, dbuf.hw.hiddenDim, dbuf.hw.outputDim, dbuf.hw.numLayers};
    const graft::MlpShape csh = shape_of(cb.hw);
    if (graft::nerf_heads_supported(dsh, csh)) {
        b.heads_packed = dalloc<unsigned char>(graft::nerf_heads_packed_bytes());
        b.tile_live = dalloc<uint32_t>((size_t)Bn / 16 + 1);
        b.occ_packed = dalloc<unsigned char>(graft::nerf_heads_packed_bytes());
        b.occ_sorted = dalloc<float4>((size_t)b.occ_capacity);
        b.occ_perm = dalloc<uint32_t>((size_t)b.occ_capacity);
        const size_t keys = graft::occ_sort_keys(m_opts.numCascades, m_opts.gridResolution);
        b.occ_sort.counts = dalloc<uint32_t>(keys);
        b.occ_sort.offsets = dalloc<uint32_t>(keys);
        b.occ_sort.block_sums = dalloc<uint32_t>(graft::march_scratch_words((uint32_t)keys));
        b.occ_sort.result = dalloc<uint32_t>(2);
        b.occ_sort.rank = dalloc<uint32_t>((size_t)b.occ_capacity);
    }
}

// InstantNerf.cu:341-359.  The mode picks the hit batch of the render path
// (renderBatchSize in INFERENCE, batchSize in TRAINING); training state stays
// allocated (the reference frees it), and training requires TRAINING mode.
void InstantNerf::setMemoryMode(MemoryMode mode)
{
    if (!m_init) return;
    m_memMode = mode;
}

void InstantNerf::setNextRays(const float3* d_rays_o, const float3* d_rays_d, uint32_t numRays)
{
    if (!m_init) throw std::runtime_error("InstantNerf: init() must be called before setNextRays()");
    if (numRays && (!d_rays_o || !d_rays_d)) throw std::runtime_error("InstantNerf: setNextRays needs ray buffers");
    B(m_buf).next = numRays ? NerfBuffers::Ahead{d_rays_o, d_rays_d, numRays} : NerfBuffers::Ahead{};
}

// InstantNerf.cu:359-583
void InstantNerf::trainWithRaysHit(const float3* d_rays_o, const float3* d_rays_d, const float* d_rays_depth,
                                   const float* d_rays_sigma, const float* d_rgb_true, uint32_t numRays,
                                   int& trainStepCount, uint32_t* hitCounts, float* d_rgb_out, hipStream_t stream)
{
    if (!m_init) throw std::runtime_error("InstantNerf: init() must be called before trainWithRaysHit()");
    if (!d_rgb_true) throw std::runtime_error("InstantNerf: trainWithRaysHit needs ground-truth colours");
    if (m_memMode != TRAINING) throw std::runtime_error("InstantNerf: trainWithRaysHit needs setMemoryMode(TRAINING)");
    if (numRays == 0) return;
    NerfBuffers& b = B(m_buf);
    const NerfOptions& o = m_opts;
    const uint32_t Bn = (uint32_t)o.batchSize;
    const graft::OccGrid g = occ_grid(o, d_occupancyGrid);
    const TinyMLPHashGrid::Buffers db = m_densityMLP->buffers();
    const TinyMLP::Buffers cb = m_colorMLP->buffers();
    const graft::MlpShape dshape{2 * o.numLevels, db.hw.hiddenDim, db.hw.outputDim, db.hw.numLayers};
    const graft::MlpShape cshape = shape_of(cb.hw);
    const int cstride = cb.hw.outputDim;

    auto stage_on = [&](hipStream_t s, const char* name, auto&& fn) {
        if (!o.isProfiling) {
            fn();
            return;
        }
        StageTimer t{name, nullptr, nullptr};
        GRAFT_HIP_CHECK(hipEventCreate(&t.a));
        GRAFT_HIP_CHECK(hipEventCreate(&t.b));
        GRAFT_HIP_CHECK(hipEventRecord(t.a, s));
        fn();
        GRAFT_HIP_CHECK(hipEventRecord(t.b, s));
        b.pending.push_back(t);
    };
    auto stage = [&](const char* name, auto&& fn) { stage_on(stream, name, fn); };

    // processRaysHitLinear (processRays.cu:931-1040) for the hit batch that
    // starts at ray raysDone, into step set k, on the compaction stream: the
    // window is marched only when it is not covered by the cached march on the
    // current grid.  The set's previous step has finished reading it by
    // then: the compaction stream waits for a later step's ev_dl first.
    // the window of rays [raysDone, raysDone + rayChunkSize) marched into
    // store si on the current grid, unless that store holds it already
    auto march_window = [&](int si, uint32_t raysDone, const float3* rays_o, const float3* rays_d, uint32_t nRays) {
        MarchStore& M = b.ms[si];
        const uint32_t R = std::min<uint32_t>((uint32_t)o.rayChunkSize, nRays - raysDone);
        if (M.version == m_gridVersion && M.o == rays_o && M.d == rays_d && raysDone >= M.c0 &&
            raysDone + R <= M.c1)
            return;
        const float3* co = rays_o + raysDone;
        const float3* cd = rays_d + raysDone;
        stage_on(b.cmp, "rayAabb", [&] {
            graft::ray_aabb_inv(R, co, cd, o.aabbMin, o.aabbMax, o.numCascades, M.d_inv, M.nears, M.fars, b.cmp);
        });
        stage_on(b.cmp, "march", [&] {
            graft::march_store(R, co, cd, M.d_inv, M.nears, M.fars, g, o.samplesPerVoxel, M.counts, M.t, b.cmp);
        });
        M.c0 = raysDone;
        M.c1 = raysDone + R;
        M.version = m_gridVersion;
        M.o = rays_o;
        M.d = rays_d;
    };
    auto compact_rays = [&](int k, int si, uint32_t raysDone, const float3* rays_o, const float3* rays_d,
                            uint32_t nRays) {
        StepSet& S = b.set[k];
        const uint32_t R = std::min<uint32_t>((uint32_t)o.rayChunkSize, nRays - raysDone);
        const float3* co = rays_o + raysDone;
        const float3* cd = rays_d + raysDone;
        march_window(si, raysDone, rays_o, rays_d, nRays);
        const MarchStore& M = b.ms[si];
        const uint32_t woff = raysDone - M.c0;
        stage_on(b.cmp, "compaction", [&] {
            graft::march_compact_stored(R, co, cd, g, Bn, M.counts + woff, M.t, woff, S.offsets, S.t_sorted,
                                        S.ray_idx, S.positions, graft::MarchScratch{b.block_sums, S.result}, b.cmp,
                                        S.counts);
        });
        // the main stream needs the set on the device only: ready before the
        // 8-byte copy to the host, whose latency stays off the step's path
        GRAFT_HIP_CHECK(hipEventRecord(S.ev_ready, b.cmp));
        GRAFT_HIP_CHECK(hipMemcpyAsync(S.h_result, S.result, 2 * sizeof(uint32_t), hipMemcpyDeviceToHost, b.cmp));
        GRAFT_HIP_CHECK(hipEventRecord(S.ev_result, b.cmp));
        S.raysDone = raysDone;
    };
    auto compact = [&](int k, uint32_t raysDone) { compact_rays(k, b.cur, raysDone, d_rays_o, d_rays_d, numRays); };

    // the side streams start after everything the caller queued (rays, grid)
    GRAFT_HIP_CHECK(hipEventRecord(b.ev_fork, stream));
    GRAFT_HIP_CHECK(hipStreamWaitEvent(b.side, b.ev_fork, 0));
    GRAFT_HIP_CHECK(hipStreamWaitEvent(b.cmp, b.ev_fork, 0));
    GRAFT_HIP_CHECK(hipStreamWaitEvent(b.occ, b.ev_fork, 0));
    // The first hit batch: compacted beside the previous call's last step
    // when that call was told these rays (same buffers, same grid), else now.
    const bool prefetched = b.pre.valid && b.pre.o == d_rays_o && b.pre.d == d_rays_d && b.pre.n == numRays &&
                            b.pre.version == m_gridVersion;
    b.pre.valid = false;
    const NerfBuffers::Ahead next = b.next;
    b.next = NerfBuffers::Ahead{};
    int k = 0, i = 0;
    bool opt_recorded = false;  // ev_opt holds a step of this call
    // A store is valid only for rays not rewritten since it was marched:
    // within a call, or from the call before under the setNextRays contract.
    // Callers refill ray buffers between calls (two feed slots taking turns),
    // so the same pointers may hold other rays now.
    if (prefetched) {
        k = b.pre.set;
        b.cur = b.pre.store;
        b.ms[b.cur ^ 1].version = -1;
    } else {
        b.ms[0].version = b.ms[1].version = -1;
        compact(k, 0);
    }
    // The next call's first window, marched ahead into the other store on
    // the grid of now (again after every refresh of this call): its first
    // hit batch, compacted beside this call's last step, then needs no march
    // at the end of the call unless the grid changed after the last one.
    // (Not now when the first step refreshes the grid.)
    const bool ahead = next.n && next.o != d_rays_o && next.d != d_rays_d;
    auto march_next = [&] {
        if (ahead) march_window(b.cur ^ 1, 0, next.o, next.d, next.n);
    };
    if (m_trainSteps % 16 != 0) march_next();
    // both heads' current weights (they may have been loaded or changed
    // since the last call) for the first step's forward
    auto pack_heads = [&](hipStream_t s) {
        graft::nerf_heads_pack(
            graft::NerfHeadsWeights{db.fwd_weights, db.master_biases, cb.fwd_weights, cb.master_biases},
            b.heads_packed, s);
    };
    if (b.heads_packed) pack_heads(stream);
    while (true) {
        StepSet& S = b.set[k];
        const uint32_t raysDone = S.raysDone;
        const float3* cd = d_rays_d + raysDone;
        const float* cdep = d_rays_depth ? d_rays_depth + raysDone : nullptr;
        const float* csig = d_rays_sigma ? d_rays_sigma + raysDone : nullptr;
        const uint32_t R = std::min<uint32_t>((uint32_t)o.rayChunkSize, numRays - raysDone);
        const uint32_t* d_rays = S.result;      // active rays of this step
        const uint32_t* d_hits = S.result + 1;  // compacted samples of this step
        m_windowStart = raysDone;
        b.last_set = k;

        // S was compacted on the side stream after the previous step's MLP
        // S on the device, and the previous step's MLP Adam (side stream):
        // then the weights this forward uses are updated
        GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, S.ev_ready, 0));
        if (opt_recorded) GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_opt, 0));
        // InstantNerf.cu:488-494: the refresh reads only the density head's
        // parameters -- the ones this step's forward reads, final once S is
        // ready -- and changes only the grid that later batches march, so it
        // runs on its own stream beside the whole step: forward, backward and
        // scatter.  The density head's Adam updates and the next batch's march
        // wait for it, so every kernel sees the parameters and grid of the
        // serial order.
        const bool refresh = (m_trainSteps % 16 == 0);
        if (refresh) GRAFT_HIP_CHECK(hipEventRecord(b.ev_occ_fork, stream));
        // The refresh's launches are enqueued after the forward and the dX
        // chain (the host's launch time then overlaps them), forked from the
        // step's start all the same.
        auto enqueue_refresh = [&] {
            if (!refresh) return;
            GRAFT_HIP_CHECK(hipStreamWaitEvent(b.occ, b.ev_occ_fork, 0));
            stage_on(b.occ, "occupancy", [&] {
                if (m_trainSteps < 256) earlyOccupancyGridUpdate(b.occ);
                else lateOccupancyGridUpdate(b.occ);
            });
            GRAFT_HIP_CHECK(hipEventRecord(b.ev_join, b.occ));
        };
        // hash encode (its own stage with the 16x16x32 heads), then density
        // head, SH gather and colour head
        if (b.heads_packed)
            stage("encode", [&] {
                graft::hash_encode_planar(b.meta, db.fwd_hashtable, reinterpret_cast<const float*>(S.positions), 4,
                                          b.enc_planar, (int)Bn, (int)Bn, stream, d_hits);
            });
        stage("forward", [&] {
            graft::NerfFwdArgs fa;
            fa.dshape = dshape;
            fa.pos = reinterpret_cast<const float*>(S.positions);
            fa.pos_stride = 4;
            fa.table = db.fwd_hashtable;
            fa.meta = &b.meta;
            fa.dW = db.fwd_weights;
            fa.dB = db.master_biases;
            // the 16x16x32 heads store no activations: the backward recomputes them
            fa.dacts = b.heads_packed ? nullptr : db.activations;
            fa.density_out = b.density_out;
            // the heads store the density logit 0 alone (all the step reads of it)
            fa.density_stride = b.heads_packed ? 1 : 16;
            fa.dirs = cd;
            fa.ray_idx = S.ray_idx;
            fa.density_bias = o.densityBias;
            fa.sigma = b.sigma;
            fa.cshape = cshape;
            fa.out_act = cb.hw.outputActivation;
            fa.cW = cb.fwd_weights;
            fa.cB = cb.master_biases;
            fa.cacts = b.heads_packed ? nullptr : cb.activations;
            fa.color_in = b.color_in;
            fa.color_out = cb.padded_outputs;
            fa.enc_scratch = b.enc_planar;
            fa.enc_plane = (int)Bn;
            fa.heads_packed = b.heads_packed;
            fa.heads_prepacked = true;  // packed at the call's start and after every step's layer Adam
            fa.enc_ready = b.heads_packed != nullptr;
            graft::nerf_forward(fa, (int)Bn, stream, d_hits);
        });
        // The next step's late refresh (one cascade): its samples are drawn
        // beside the rest of this step, from the step after the forward.
        if (!refresh && m_opts.numCascades == 1 && (m_trainSteps + 1) % 16 == 0 && m_trainSteps + 1 >= 256) {
            GRAFT_HIP_CHECK(hipEventRecord(b.ev_occ_fork, stream));
            GRAFT_HIP_CHECK(hipStreamWaitEvent(b.occ, b.ev_occ_fork, 0));
            stage_on(b.occ, "occupancyDraw", [&] { drawLateRefresh((long)m_trainSteps + 1, b.occ); });
        }

        float* final_rgb = d_rgb_out ? d_rgb_out + (size_t)raysDone * 3 : b.render_rgb;
        stage("renderGrad", [&] {
            graft::CompositeArgs ca{};
            ca.offsets = S.offsets;
            ca.counts = S.counts;
            ca.t = S.t_sorted;
            ca.sigma = b.sigma;
            ca.depth_prior = cdep;
            ca.sigma_prior = csig;
            ca.rgb = cb.padded_outputs;
            ca.rgb_stride = cstride;
            ca.rgb_true = d_rgb_true + (size_t)raysDone * 3;
            ca.final_rgb = final_rgb;
            ca.final_depth = b.render_depth;
            ca.phi = b.phi;
            ca.dw = b.dw;
            ca.weight_sum = b.weight_sum;
            ca.lambda_dist = o.lambdaDist;
            ca.lambda_depth = o.lambdaDepth;
            ca.bg = o.bgColor;
            graft::ColorGradArgs ga{};
            ga.initial_offset = 0;
            ga.counts = S.counts;
            ga.offsets = S.offsets;
            ga.t = S.t_sorted;
            ga.density_out = b.density_out;
            ga.density_stride = b.heads_packed ? 1 : 16;
            ga.color_out = cb.padded_outputs;
            ga.color_stride = cstride;
            ga.phi = b.phi;
            ga.final_rgb = final_rgb;
            ga.dw = b.dw;
            ga.weight_sum = b.weight_sum;
            ga.color_grad = cb.dloss;
            ga.grad_stride = cstride;
            ga.dsigma = b.dsigma;
            ga.loss_scale = o.lossScale;
            ga.bias = o.densityBias;
            ga.total_rays = numRays;
            graft::render_grad(ca, ga, d_rays, R, stream);
        });
        // The hash scatter waits only for dL/d(encoding): the main stream runs
        // the dX chain of both heads (dX-only kernels for the NeRF shapes) and
        // the side stream the weight gradients and MLP Adam beside the scatter.
        graft::NerfBwdDxArgs bx;
        bx.cshape = cshape;
        bx.dshape = dshape;
        bx.color_dy = cb.dloss;
        bx.cacts = cb.activations;
        bx.cW = cb.fwd_weights;
        bx.dsigma = b.dsigma;
        bx.dacts = db.activations;
        bx.dW = db.fwd_weights;
        bx.color_dx = b.color_dx;
        bx.density_dy = db.dloss;
        bx.denc = db.dx_out;
        graft::NerfHeadsBwd hb;
        hb.packed = b.heads_packed;
        hb.enc = b.enc_planar;
        hb.enc_plane = (int)Bn;
        hb.levels = b.meta.numLevels;
        hb.color_in = b.color_in;
        hb.color_dy = cb.dloss;
        hb.dsigma = b.dsigma;
        hb.denc = db.dx_out;
        hb.density_dy = db.dloss;
        hb.color_dx = m_keepColorDx ? b.color_dx : nullptr;  // read by nothing in the step
        hb.tile_live = b.tile_live;
        const bool heads = b.heads_packed != nullptr;
        const bool fused_dx = !heads && graft::nerf_backward_dx(bx, 0, stream);  // shape check only (N = 0)
        const bool dx_only = !heads && graft::mlp_has_dx_kernel(cshape) && graft::mlp_has_dx_kernel(dshape);
        if (heads) {
            // recomputed activations: colour dX chain, glue, density dX chain
            stage("backwardDx", [&] { graft::nerf_heads_dx(hb, (int)Bn, stream, d_hits); });
        } else if (fused_dx || dx_only) {
            if (fused_dx) {
                // colour dX chain, density-gradient glue, density dX chain: one launch
                stage("backwardDx", [&] { graft::nerf_backward_dx(bx, (int)Bn, stream, d_hits); });
            } else {
                stage("colorDx", [&] {
                    graft::mlp_backward_dx(cshape, cb.dloss, cb.activations, cb.fwd_weights, b.color_dx, (int)Bn,
                                           stream, d_hits);
                });
                stage("densityGrad",
                      [&] { graft::density_grad(d_hits, Bn, b.dsigma, b.color_dx, db.dloss, stream); });
                stage("densityDx", [&] {
                    graft::mlp_backward_dx(dshape, db.dloss, db.activations, db.fwd_weights, db.dx_out, (int)Bn,
                                           stream, d_hits);
                });
            }
        } else {
            stage("colorBwd", [&] {
                graft::mlp_backward(cshape, cb.dloss, cb.activations, cb.fwd_weights, cb.w_grad, cb.b_grad,
                                    b.color_dx, (int)Bn, stream, d_hits, /*accumulate=*/false,
                                    static_cast<graft::Workspace*>(cb.workspace));
            });
            stage("densityGrad", [&] { graft::density_grad(d_hits, Bn, b.dsigma, b.color_dx, db.dloss, stream); });
            stage("densityBwd", [&] {
                graft::mlp_backward(dshape, db.dloss, db.activations, db.fwd_weights, db.w_grad, db.b_grad,
                                    db.dx_out, (int)Bn, stream, d_hits, /*accumulate=*/false,
                                    static_cast<graft::Workspace*>(db.workspace));
            });
        }
        GRAFT_HIP_CHECK(hipEventRecord(b.ev_dl, stream));
        enqueue_refresh();
        // The scatter is the step's critical path: it is enqueued before the
        // side streams' work, so that the host's launches of that work never
        // delay it.
        // With the binned scatter the table's Adam update is fused into it
        // (every entry the batch reaches is updated as its sum completes; no
        // gradient array).  The update waits for a refresh of this step, which
        // reads the table.
        const bool fused_table = db.scatter_plan != nullptr;
        // Profiling: the wait for the refresh comes before the stage's timer
        // (then the whole scatter waits, not only its update), so that the
        // stage times the scatter's kernels and not the refresh beside them.
        hipEvent_t update_wait = refresh ? b.ev_join : nullptr;
        if (o.isProfiling && update_wait) {
            GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, update_wait, 0));
            update_wait = nullptr;
        }
        stage("hashScatter", [&] {
            if (fused_table)
                m_densityMLP->scatterAdamTable(db.dx_out, reinterpret_cast<const float*>(S.positions), 4, (int)Bn,
                                               d_hits, o.learningRate, o.beta1, o.beta2, o.epsilon, o.lossScale,
                                               stream, update_wait, heads ? b.tile_live : nullptr);
            else
                // the table gradient is all zero here: the previous step's
                // Adam cleared every entry it consumed
                graft::hash_scatter_atomic(b.meta, db.dx_out, reinterpret_cast<const float*>(S.positions), 4,
                                           db.hashtable_grads, (int)Bn, stream, d_hits);
        });
        // Beside it: the weight gradients (this step's gradient overwrites the
        // last one: no zero_grad pass).  The side stream's wait on ev_dl also
        // orders every read of this step set by the main stream before the
        // compaction that refills the set two steps later (it is enqueued on
        // the side stream after the next step's wait on ev_dl).
        GRAFT_HIP_CHECK(hipStreamWaitEvent(b.side, b.ev_dl, 0));

        // The only host read of the step: its active-ray count (computed a
        // step ago), to advance the cursor.  The next batch is compacted on
        // the side stream first, beside this step's scatter (after the
        // refresh instead when this step refreshes the grid).
        GRAFT_HIP_CHECK(hipEventSynchronize(S.ev_result));
        const uint32_t active = S.h_result[0], hits = S.h_result[1];
        if (active == 0) {
            // unreachable with batchSize >= one ray's sample cap; leave no work
            // of this call on the side streams and no timers behind
            GRAFT_HIP_CHECK(hipEventRecord(b.ev_done, b.side));
            GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_done, 0));
            GRAFT_HIP_CHECK(hipEventRecord(b.ev_done_occ, b.occ));
            GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_done_occ, 0));
            GRAFT_HIP_CHECK(hipEventRecord(b.ev_done_cmp, b.cmp));
            GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_done_cmp, 0));
            GRAFT_HIP_CHECK(hipStreamSynchronize(stream));
            for (auto& t : b.pending) {
                (void)hipEventDestroy(t.a);
                (void)hipEventDestroy(t.b);
            }
            b.pending.clear();
            b.pre.valid = false;
            throw std::runtime_error("InstantNerf: no ray fits the batch");
        }
        if (hitCounts) hitCounts[i] = hits;
        i++;
        m_lastRaysTrained = raysDone + active;
        const bool all_rays = raysDone + active >= numRays;
        const bool stop = all_rays || (m_stepLimit > 0 && i >= m_stepLimit);
        // the compaction stream: after this step's reads of the set it refills
        // (ev_dl) and, on a refresh step, after the refresh (ev_join)
        GRAFT_HIP_CHECK(hipStreamWaitEvent(b.cmp, b.ev_dl, 0));
        if (refresh) GRAFT_HIP_CHECK(hipStreamWaitEvent(b.cmp, b.ev_join, 0));
        if (!stop) compact(k ^ 1, raysDone + active);
        if (refresh && !stop) march_next();

        if (heads) {
            stage_on(b.side, "headsBwd", [&] {
                graft::nerf_heads_dw(hb, graft::NerfHeadsGrads{db.w_grad, db.b_grad, cb.w_grad, cb.b_grad}, (int)Bn,
                                     b.side, d_hits, static_cast<graft::Workspace*>(db.workspace));
            });
        } else if (fused_dx || dx_only) {
            stage_on(b.side, "colorBwd", [&] {
                graft::mlp_backward(cshape, cb.dloss, cb.activations, cb.fwd_weights, cb.w_grad, cb.b_grad, nullptr,
                                    (int)Bn, b.side, d_hits, /*accumulate=*/false,
                                    static_cast<graft::Workspace*>(cb.workspace));
            });
            stage_on(b.side, "densityBwd", [&] {
                graft::mlp_backward(dshape, db.dloss, db.activations, db.fwd_weights, db.w_grad, db.b_grad, nullptr,
                                    (int)Bn, b.side, d_hits, /*accumulate=*/false,
                                    static_cast<graft::Workspace*>(db.workspace));
            });
        }
        // Adam: MLP layers of both heads on the side stream, the hash table on
        // the main stream (in the scatter above when that is the binned one).
        // The colour head's needs nothing of the refresh;
        // the density head's (and, after it on the side stream, the next
        // batch's march) waits until the refresh has read the parameters and
        // written the grid.
        stage_on(b.side, "colorOpt", [&] {
            m_colorMLP->step(o.learningRate, o.beta1, o.beta2, o.epsilon, o.lossScale, b.side);
        });
        if (refresh) {
            GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_join, 0));
            GRAFT_HIP_CHECK(hipStreamWaitEvent(b.side, b.ev_join, 0));
        }
        if (fused_table)
            stage_on(b.side, "densityOpt", [&] {
                m_densityMLP->stepMlp(o.learningRate, o.beta1, o.beta2, o.epsilon, o.lossScale, b.side);
            });
        else
            stage("densityOpt", [&] {
                m_densityMLP->stepSplit(o.learningRate, o.beta1, o.beta2, o.epsilon, o.lossScale, b.side, stream);
            });
        // the next step's weights, packed beside this step's scatter
        if (b.heads_packed) pack_heads(b.side);
        GRAFT_HIP_CHECK(hipEventRecord(b.ev_opt, b.side));
        opt_recorded = true;

        trainStepCount++;
        m_trainSteps++;
        if (stop) {
            // the next call's rays are compacted ahead only when they are
            // other buffers than this call's (a caller refilling these buffers
            // in place for the next call would otherwise train on stale rays)
            if (all_rays && ahead) {
                // the next call's first hit batch, beside this last step, from
                // the other store (marched ahead unless the grid has changed)
                k ^= 1;
                compact_rays(k, b.cur ^ 1, 0, next.o, next.d, next.n);
                b.pre = NerfBuffers::Prefetched{true, next.o, next.d, next.n, k, b.cur ^ 1, m_gridVersion};
            }
            break;
        }
        k ^= 1;
    }
    // nothing of this call stays on the side streams past the return
    GRAFT_HIP_CHECK(hipEventRecord(b.ev_done, b.side));
    GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_done, 0));
    GRAFT_HIP_CHECK(hipEventRecord(b.ev_done_occ, b.occ));
    GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_done_occ, 0));
    GRAFT_HIP_CHECK(hipEventRecord(b.ev_done_cmp, b.cmp));
    GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, b.ev_done_cmp, 0));

    if (o.isProfiling && !b.pending.empty()) {
        for (auto& t : b.pending) {
            // stages on the side streams may end after the last one recorded
            GRAFT_HIP_CHECK(hipEventSynchronize(t.b));
            float ms = 0.f;
            GRAFT_HIP_CHECK(hipEventElapsedTime(&ms, t.a, t.b));
            auto& s = b.stats[t.name];
            s.first += ms;
            s.second += 1;
            (void)hipEventDestroy(t.a);
            (void)hipEventDestroy(t.b);
        }
        b.pending.clear();
    }
}

// InstantNerf.cu:82-148 (flat table instead of the reference's tree).
void InstantNerf::printStats()
{
    if (!m_buf) return;
    NerfBuffers& b = B(m_buf);
    std::printf("%-18s %10s %8s\n", "stage", "mean ms", "calls");
    for (const auto& kv : b.stats)
        std::printf("%-18s %10.4f %8ld\n", kv.first.c_str(), kv.second.first / std::max(1L, kv.second.second),
                    kv.second.second);
}

void InstantNerf::resetStats()
{
    if (m_buf) B(m_buf).stats.clear();
}

std::string InstantNerf::statsString() const
{
    std::string out;
    if (!m_buf) return out;
    const NerfBuffers& b = *static_cast<const NerfBuffers*>(m_buf);
    char line[160];
    for (const auto& kv : b.stats) {
        std::snprintf(line, sizeof(line), "%s:%.6f:%ld;", kv.first.c_str(),
                      kv.second.first / std::max(1L, kv.second.second), kv.second.second);
        out += line;
    }
    return out;
}

void InstantNerf::updateOccupancy(hipStream_t stream)
{
    if (!m_init) throw std::runtime_error("InstantNerf: init() first");
    if (m_trainSteps < 256) earlyOccupancyGridUpdate(stream);
    else lateOccupancyGridUpdate(stream);
}

namespace {

// The per-cell maximum of sigma over the n refresh samples in b.occ_samples,
// into b.tmp_grid, with each sample's density logit 0 in b.occ_density
// (stride refresh_density_stride; in b.occ_perm's order when sorted).  The encode runs as its own launch (each
// XCD's L2 holding only its levels' tables; the samples are spread over the
// whole grid, so an encode fused with the head would cycle all 32 MiB of table
// through every L2).  With the 16x16x32 heads: samples spread at random are
// evaluated in the spatial order late_refresh_draw put them in (sorted: in
// b.occ_sorted), so that a wave's gathers share table lines; the density
// head runs on the level-major encodings with the maximum fused in
// (b.occ_packed holds the density head's fragments, packed at the refresh's
// start); otherwise the TinyMLP density forward, then the maximum.
void occupancy_density_max(NerfBuffers& b, const TinyMLPHashGrid::Buffers& db, const graft::MlpShape& dshape, int n,
                           bool sorted, bool one_per_cell, const NerfOptions& o, hipStream_t stream)
{
    if (b.occ_packed) {
        const float4* src = sorted ? b.occ_sorted : b.occ_samples;
        graft::hash_encode_planar(b.meta, db.fwd_hashtable, reinterpret_cast<const float*>(src), 4, b.occ_enc, n, n,
                                  stream);
        graft::NerfDensityMax a;
        a.packed = b.occ_packed;
        a.enc = b.occ_enc;
        a.enc_plane = n;
        a.levels = b.meta.numLevels;
        a.samples = src;
        a.density_bias = o.densityBias;
        a.logit = b.occ_density;
        a.tmp = b.tmp_grid;
        a.one_per_cell = one_per_cell;
        graft::nerf_density_max(a, n, stream);
        b.occ_last_sorted = sorted;
        return;
    }
    b.occ_last_sorted = false;
    graft::hash_encode(b.meta, db.fwd_hashtable, reinterpret_cast<const float*>(b.occ_samples), 4, b.occ_enc, n,
                       stream);
    graft::FwdInput in;
    in.x = b.occ_enc;
    graft::mlp_forward(dshape, in, db.fwd_weights, db.master_biases, nullptr, b.occ_density, n, OUT_ACT_NONE, stream);
    graft::occ_tmp_max(b.occ_samples, b.occ_density, b.tmp_grid, o.densityBias, n, stream);
}

int refresh_density_stride(const NerfBuffers& b) { return b.occ_packed ? 1 : 16; }

// the density head's current weights for the refresh's own fragments
void pack_refresh(NerfBuffers& b, const TinyMLPHashGrid::Buffers& db, hipStream_t stream)
{
    if (b.occ_packed)
        graft::nerf_heads_pack_density(graft::NerfHeadsWeights{db.fwd_weights, db.master_biases, nullptr, nullptr},
                                       b.occ_packed, stream);
}

// Samples of a late refresh's chunk ch (InstantNerf.cu:1009-1106): half from
// the occupied-cell list in b.active_list, half uniform over all cells,
// seeded by the refresh's step count; with the 16x16x32 heads also put in a
// spatial order (b.occ_sorted, b.occ_perm).  They depend on the grid and the
// step count only, not on any parameter.
void late_refresh_draw(NerfBuffers& b, const NerfOptions& o, long steps, int ch, hipStream_t stream)
{
    const int N = o.numCascades * grid_cells(o);
    const int chunks = o.numCascades;
    const int perChunk = (N / 2) / chunks;
    const int occPer = perChunk / 2;
    const int uniPer = perChunk - occPer;
    const uint64_t seed = (uint64_t)steps * (2ULL * chunks) + 2ULL * ch;
    graft::occ_sample(b.occ_samples, occPer, graft::kSampleFromList, 0, 0, b.active_list, b.active_count, seed,
                      o.gridResolution, o.aabbMin, o.aabbMax, stream);
    graft::occ_sample(b.occ_samples + occPer, uniPer, graft::kSampleRandomCell, N, 0, nullptr, nullptr, seed + 1,
                      o.gridResolution, o.aabbMin, o.aabbMax, stream);
    if (b.occ_packed)
        graft::occ_sort_samples(b.occ_samples, perChunk, o.numCascades, o.gridResolution, b.occ_sort, b.occ_sorted,
                                b.occ_perm, stream);
}

// the occupied-cell list of the grid (its pass over every cell also clears
// the tmp grid)
void late_refresh_list(NerfBuffers& b, const NerfOptions& o, const uint8_t* grid, hipStream_t stream)
{
    const int G = grid_cells(o);
    const int S = (int)graft::mip_offset(o.gridResolution, o.levelsMipmap);
    graft::occ_active_list(grid, o.numCascades * G, G, S, b.active_list, b.active_count, b.list_scratch, stream,
                           b.tmp_grid);
}
}  // namespace

// InstantNerf.cu:1108-1171: one jittered sample per cell of every cascade.
void InstantNerf::earlyOccupancyGridUpdate(hipStream_t stream)
{
    NerfBuffers& b = B(m_buf);
    const int G = grid_cells(m_opts);
    const int N = m_opts.numCascades * G;
    const TinyMLPHashGrid::Buffers db = m_densityMLP->buffers();
    const graft::MlpShape dshape{2 * m_opts.numLevels, db.hw.hiddenDim, db.hw.outputDim, db.hw.numLayers};
    // with the density head of the 16x16x32 heads, each cell's one sample
    // stores its sigma; else the maximum starts from zero
    if (!b.occ_packed) GRAFT_HIP_CHECK(hipMemsetAsync(b.tmp_grid, 0, (size_t)N * sizeof(float), stream));
    pack_refresh(b, db, stream);
    for (int c = 0; c < m_opts.numCascades; ++c) {
        graft::occ_sample(b.occ_samples, G, graft::kSampleEveryCell, G, c * G, nullptr, nullptr,
                          (uint64_t)m_trainSteps + (uint64_t)c, m_opts.gridResolution, m_opts.aabbMin, m_opts.aabbMax,
                          stream);
        // every cell in cell order: already spatial
        occupancy_density_max(b, db, dshape, G, /*sorted=*/false, true, m_opts, stream);
    }
    b.occ_last_count = G;
    finishOccupancyUpdate(stream);
}

// InstantNerf.cu:1009-1106: half the cells' worth of samples, per cascade
// chunk half from occupied cells and half uniform over all cells.
void InstantNerf::lateOccupancyGridUpdate(hipStream_t stream)
{
    NerfBuffers& b = B(m_buf);
    const int N = m_opts.numCascades * grid_cells(m_opts);
    const TinyMLPHashGrid::Buffers db = m_densityMLP->buffers();
    const graft::MlpShape dshape{2 * m_opts.numLevels, db.hw.hiddenDim, db.hw.outputDim, db.hw.numLayers};
    pack_refresh(b, db, stream);
    // the samples of a one-chunk refresh may have been drawn a step ahead
    // (drawLateRefresh) for this step count on this grid
    const bool drawn = b.drawn_steps == (long)m_trainSteps && b.drawn_version == m_gridVersion;
    b.drawn_steps = b.drawn_version = -1;
    if (!drawn) late_refresh_list(b, m_opts, d_occupancyGrid, stream);
    const int chunks = m_opts.numCascades;
    const int perChunk = (N / 2) / chunks;
    for (int ch = 0; ch < chunks; ++ch) {
        if (!drawn) late_refresh_draw(b, m_opts, (long)m_trainSteps, ch, stream);
        occupancy_density_max(b, db, dshape, perChunk, /*sorted=*/b.occ_packed != nullptr, false, m_opts, stream);
        b.occ_last_count = perChunk;
    }
    finishOccupancyUpdate(stream);
}

// The sample draw of the late refresh at step count `steps`, a step ahead of
// it: the occupied-cell list, the samples and their spatial sort read only
// the grid and the step count, so with one cascade (one chunk, whose samples
// the refresh's density head then evaluates) they run beside the step before
// the refresh instead of on the refresh's own path.  The refresh uses them
// only if the grid has not changed since (m_gridVersion).
void InstantNerf::drawLateRefresh(long steps, hipStream_t stream)
{
    NerfBuffers& b = B(m_buf);
    if (m_opts.numCascades != 1 || steps < 256 || steps % 16 != 0) return;
    late_refresh_list(b, m_opts, d_occupancyGrid, stream);
    late_refresh_draw(b, m_opts, steps, 0, stream);
    b.drawn_steps = steps;
    b.drawn_version = m_gridVersion;
}

// EMA-max into the master grid, mean, level-0 bits, mip pyramid (InstantNerf.cu:1150-1171).
void InstantNerf::finishOccupancyUpdate(hipStream_t stream)
{
    m_gridVersion++;
    NerfBuffers& b = B(m_buf);
    const int G = grid_cells(m_opts);
    const int N = m_opts.numCascades * G;
    const int S = (int)graft::mip_offset(m_opts.gridResolution, m_opts.levelsMipmap);
    graft::update_master_grid(b.tmp_grid, d_masterOccupancyGrid, m_opts.decayValue, (uint32_t)N, stream);
    graft::reduce_sum(d_masterOccupancyGrid, (uint32_t)N, b.partials, b.sum, stream);
    const float base_voxel = (m_opts.aabbMax.x - m_opts.aabbMin.x) / (float)m_opts.gridResolution.x;
    graft::update_occupancy_bits(reinterpret_cast<uint32_t*>(d_occupancyGrid), d_masterOccupancyGrid, b.sum, N, G, S,
                                 m_opts.minDensityThreshold, base_voxel, stream);
    graft::build_mipmaps(d_occupancyGrid, m_opts.gridResolution, m_opts.levelsMipmap, m_opts.numCascades, stream);
}

void InstantNerf::setOccupancyBits(const uint8_t* host_bits)
{
    if (!m_init) throw std::runtime_error("InstantNerf: init() first");
    GRAFT_HIP_CHECK(hipMemcpy(d_occupancyGrid, host_bits, m_occupancyBytes, hipMemcpyHostToDevice));
    m_gridVersion++;
}

InstantNerf::RefreshBuffers InstantNerf::refreshBuffers() const
{
    if (!m_buf) throw std::runtime_error("InstantNerf: init() first");
    const NerfBuffers& b = *static_cast<const NerfBuffers*>(m_buf);
    RefreshBuffers r{};
    r.samples = b.occ_samples;
    r.density_out = b.occ_density;
    r.densityStride = refresh_density_stride(b);
    r.densityOrder = b.occ_last_sorted ? b.occ_perm : nullptr;
    r.tmp_grid = b.tmp_grid;
    r.active_list = b.active_list;
    r.active_count = b.active_count;
    r.lastCount = b.occ_last_count;
    return r;
}

InstantNerf::StepBuffers InstantNerf::stepBuffers() const
{
    if (!m_buf) throw std::runtime_error("InstantNerf: init() first");
    const NerfBuffers& b = *static_cast<const NerfBuffers*>(m_buf);
    StepBuffers s{};
    const StepSet& S = b.set[b.last_set];
    s.num_steps = S.counts;
    s.ray_offsets = S.offsets;
    s.positions = S.positions;
    s.ray_indices = S.ray_idx;
    s.t_sorted = S.t_sorted;
    s.density_out = b.density_out;
    s.densityStride = b.heads_packed ? 1 : 16;
    s.color_input = b.color_in;
    s.color_output = m_colorMLP->buffers().padded_outputs;
    s.sigma = b.sigma;
    s.render_rgb = b.render_rgb;
    s.phi = b.phi;
    s.dw = b.dw;
    s.weight_sum = b.weight_sum;
    s.dsigma = b.dsigma;
    s.color_dx = b.color_dx;
    s.density_grad = m_densityMLP->buffers().dloss;
    s.result = S.result;
    s.trainSteps = m_trainSteps;
    s.windowStart = m_windowStart;
    s.encodings = reinterpret_cast<half*>(b.enc_planar);
    s.encodingPlane = (uint32_t)std::max(1, m_opts.batchSize);
    s.activationsSaved = b.heads_packed ? 0 : 1;
    return s;
}

// ---- inference render and queries ----

namespace {

void ensure_render(NerfBuffers& b, uint32_t cap, int color_width)
{
    if (b.render.cap >= cap) return;
    dfree(b.render.positions);
    dfree(b.render.ray_idx);
    dfree(b.render.t);
    dfree(b.render.density_out);
    dfree(b.render.color_in);
    dfree(b.render.sigma);
    dfree(b.render.rgb);
    b.render.positions = dalloc<float4>(cap);
    b.render.ray_idx = dalloc<uint32_t>(cap);
    b.render.t = dalloc<float>(cap);
    b.render.density_out = dalloc<float>((size_t)cap * 16);
    b.render.color_in = dalloc<__half>((size_t)cap * 32);
    b.render.sigma = dalloc<float>(cap);
    b.render.rgb = dalloc<float>((size_t)cap * color_width);
    b.render.cap = cap;
}

}  // namespace

uint32_t InstantNerf::renderHitBatch() const
{
    const int hb = (m_memMode == INFERENCE) ? m_opts.renderBatchSize : m_opts.batchSize;
    return (uint32_t)std::max(hb, MAX_HITS) & ~15u;
}

// renderImageHit (InstantNerf.cu:713-864): per chunk of rayChunkSize rays,
// march once, then per hit batch: compaction from the first unrendered ray,
// density inference, SH gather, colour inference, inference compositing
// (compositing.cu:5-78) straight into d_rgb_out.  One host read per hit batch
// (its active-ray count); the reference makes three blocking ones.
void InstantNerf::renderImageHit(const float3* d_rays_o, const float3* d_rays_d, uint32_t numRays, float* d_rgb_out,
                                 hipStream_t stream)
{
    if (!m_init) throw std::runtime_error("InstantNerf: init() must be called before renderImageHit()");
    NerfBuffers& b = B(m_buf);
    const NerfOptions& o = m_opts;
    const uint32_t hitBatch = renderHitBatch();
    const TinyMLPHashGrid::Buffers db = m_densityMLP->buffers();
    const TinyMLP::Buffers cb = m_colorMLP->buffers();
    const graft::MlpShape dshape{2 * o.numLevels, db.hw.hiddenDim, db.hw.outputDim, db.hw.numLayers};
    const graft::MlpShape cshape = shape_of(cb.hw);
    ensure_render(b, hitBatch, cshape.out);
    const graft::OccGrid g = occ_grid(o, d_occupancyGrid);
    StepSet& S = b.set[0];  // the render path runs on the caller's stream only
    const uint32_t* d_rays = S.result;
    const uint32_t* d_hits = S.result + 1;
    MarchStore& M = b.ms[b.cur];
    b.ms[0].version = b.ms[1].version = -1;  // the march store is reused below
    b.pre.valid = false;                     // and so is step set 0

    for (uint32_t c0 = 0; c0 < numRays; c0 += (uint32_t)o.rayChunkSize) {
        const uint32_t R = std::min<uint32_t>((uint32_t)o.rayChunkSize, numRays - c0);
        const float3* co = d_rays_o + c0;
        const float3* cd = d_rays_d + c0;
        graft::ray_aabb_inv(R, co, cd, o.aabbMin, o.aabbMax, o.numCascades, M.d_inv, M.nears, M.fars, stream);
        graft::march_store(R, co, cd, M.d_inv, M.nears, M.fars, g, o.samplesPerVoxel, M.counts, M.t, stream);
        uint32_t done = 0;
        while (done < R) {
            graft::march_compact_stored(R - done, co + done, cd + done, g, hitBatch, M.counts + done, M.t, done,
                                        S.offsets, b.render.t, b.render.ray_idx, b.render.positions,
                                        graft::MarchScratch{b.block_sums, S.result}, stream);
            GRAFT_HIP_CHECK(hipMemcpyAsync(S.h_result, S.result, 2 * sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
            GRAFT_HIP_CHECK(hipEventRecord(S.ev_result, stream));
            graft::NerfFwdArgs fa;
            fa.dshape = dshape;
            fa.pos = reinterpret_cast<const float*>(b.render.positions);
            fa.pos_stride = 4;
            fa.table = db.fwd_hashtable;
            fa.meta = &b.meta;
            fa.dW = db.fwd_weights;
            fa.dB = db.master_biases;
            fa.dirs = cd + done;
            fa.ray_idx = b.render.ray_idx;
            fa.density_bias = o.densityBias;
            fa.sigma = b.render.sigma;
            fa.cshape = cshape;
            fa.out_act = cb.hw.outputActivation;
            fa.cW = cb.fwd_weights;
            fa.cB = cb.master_biases;
            fa.color_out = b.render.rgb;
            graft::nerf_forward(fa, (int)hitBatch, stream, d_hits);
            graft::CompositeArgs ca{};
            ca.offsets = S.offsets;
            ca.counts = M.counts + done;
            ca.t = b.render.t;
            ca.sigma = b.render.sigma;
            ca.rgb = b.render.rgb;
            ca.rgb_stride = cshape.out;
            ca.final_rgb = d_rgb_out ? d_rgb_out + (size_t)(c0 + done) * 3 : b.render_rgb;
            ca.final_depth = b.render_depth;
            ca.bg = o.bgColor;
            graft::composite_infer(ca, 0, 0, d_rays, R - done, stream);
            GRAFT_HIP_CHECK(hipEventSynchronize(S.ev_result));
            const uint32_t active = S.h_result[0];
            if (active == 0) throw std::runtime_error("InstantNerf: the render hit batch cannot hold one ray");
            done += active;
        }
    }
}

// renderImage (InstantNerf.cu:585-711), the legacy path behind legacyRenderFlag:
// every ray's samples, MLP outputs and composite are those of renderImageHit.
void InstantNerf::renderImage(const float3* d_rays_o, const float3* d_rays_d, uint32_t numRays, float* d_rgb_out,
                              hipStream_t stream)
{
    if (!m_opts.legacyRenderFlag)
        throw std::runtime_error("InstantNerf: renderImage() requires legacyRenderFlag=true; use renderImageHit()");
    renderImageHit(d_rays_o, d_rays_d, numRays, d_rgb_out, stream);
}

// queryOccupancyGrid (InstantNerf.cu:941-946): d_pos [n x 3].
void InstantNerf::queryOccupancyGrid(const float* d_pos, int n, uint32_t* d_data_out, float minOpticalThreshold,
                                     hipStream_t stream)
{
    if (!m_init) throw std::runtime_error("InstantNerf: init() must be called before queryOccupancyGrid()");
    graft::query_occupancy(d_masterOccupancyGrid, d_pos, d_data_out, m_opts.gridResolution, m_opts.aabbMin,
                           m_opts.aabbMax, minOpticalThreshold, m_opts.numCascades, n, stream);
}

// queryDensityLogit (InstantNerf.cu:948-961): raw density logit (output 0 of
// the density head) of contracted positions d_pos [n x 3]; n % 16 == 0.
void InstantNerf::queryDensityLogit(const float* d_pos, int n, float* d_logit_out, hipStream_t stream)
{
    if (n <= 0) return;
    if (n % 16 != 0) throw std::runtime_error("queryDensityLogit: n must be a multiple of 16 (caller pads)");
    if (!m_init) throw std::runtime_error("InstantNerf: query before init()");
    NerfBuffers& b = B(m_buf);
    const TinyMLPHashGrid::Buffers db = m_densityMLP->buffers();
    const graft::MlpShape dshape{2 * m_opts.numLevels, db.hw.hiddenDim, db.hw.outputDim, db.hw.numLayers};
    const uint32_t cap = renderHitBatch();
    ensure_render(b, cap, m_colorMLP->buffers().hw.outputDim);
    for (int off = 0; off < n; off += (int)cap) {
        const int cn = std::min<int>((int)cap, n - off);
        graft::FwdInput in;
        in.pos = d_pos + (size_t)off * 3;
        in.pos_stride = 3;
        in.table = db.fwd_hashtable;
        in.meta = &b.meta;
        graft::mlp_forward(dshape, in, db.fwd_weights, db.master_biases, nullptr, b.render.density_out, cn,
                           OUT_ACT_NONE, stream);
        graft::extract_column(b.render.density_out, 16, d_logit_out + off, cn, stream);
    }
}

// queryRadiance (InstantNerf.cu:963-984): colour of contracted positions
// d_pos [n x 3] seen along viewDir; d_rgb_out [n x 3]; n % 16 == 0.
void InstantNerf::queryRadiance(const float* d_pos, int n, float3 viewDir, float* d_rgb_out, hipStream_t stream)
{
    if (n <= 0) return;
    if (n % 16 != 0) throw std::runtime_error("queryRadiance: n must be a multiple of 16 (caller pads)");
    if (!m_init) throw std::runtime_error("InstantNerf: query before init()");
    NerfBuffers& b = B(m_buf);
    const TinyMLPHashGrid::Buffers db = m_densityMLP->buffers();
    const TinyMLP::Buffers cb = m_colorMLP->buffers();
    const graft::MlpShape dshape{2 * m_opts.numLevels, db.hw.hiddenDim, db.hw.outputDim, db.hw.numLayers};
    const graft::MlpShape cshape = shape_of(cb.hw);
    const uint32_t cap = renderHitBatch();
    ensure_render(b, cap, cshape.out);
    if (!b.render.dir) b.render.dir = dalloc<float3>(1);
    GRAFT_HIP_CHECK(hipMemcpyAsync(b.render.dir, &viewDir, sizeof(float3), hipMemcpyHostToDevice, stream));
    GRAFT_HIP_CHECK(hipMemsetAsync(b.render.ray_idx, 0, (size_t)std::min<int>((int)cap, n) * sizeof(uint32_t), stream));
    for (int off = 0; off < n; off += (int)cap) {
        const int cn = std::min<int>((int)cap, n - off);
        graft::FwdInput in;
        in.pos = d_pos + (size_t)off * 3;
        in.pos_stride = 3;
        in.table = db.fwd_hashtable;
        in.meta = &b.meta;
        graft::mlp_forward(dshape, in, db.fwd_weights, db.master_biases, nullptr, b.render.density_out, cn,
                           OUT_ACT_NONE, stream);
        graft::sh_gather(b.render.dir, b.render.ray_idx, nullptr, (uint32_t)cn, m_opts.densityBias,
                         b.render.density_out, b.render.color_in, b.render.sigma, stream);
        graft::FwdInput ci;
        ci.x = b.render.color_in;
        graft::mlp_forward(cshape, ci, cb.fwd_weights, cb.master_biases, nullptr, b.render.rgb, cn,
                           cb.hw.outputActivation, stream);
        graft::unpad_f32(b.render.rgb, d_rgb_out + (size_t)off * 3, cn, cshape.out, 3, stream);
    }
    GRAFT_HIP_CHECK(hipStreamSynchronize(stream));  // viewDir is a host value
}

// buildOccupancyBitgrid (InstantNerf.cu:986-1007): bits from the master grid
// with the per-cascade threshold only (no mean floor), then the mip pyramid.
void InstantNerf::buildOccupancyBitgrid(uint8_t* d_out, float minDensityThreshold, hipStream_t stream)
{
    if (!m_init) throw std::runtime_error("InstantNerf: buildOccupancyBitgrid before init()");
    NerfBuffers& b = B(m_buf);
    const int G = grid_cells(m_opts);
    const int N = m_opts.numCascades * G;
    const int S = (int)graft::mip_offset(m_opts.gridResolution, m_opts.levelsMipmap);
    static const float kNoFloor = 1e30f;
    GRAFT_HIP_CHECK(hipMemcpyAsync(b.sum, &kNoFloor, sizeof(float), hipMemcpyHostToDevice, stream));
    const float base_voxel = (m_opts.aabbMax.x - m_opts.aabbMin.x) / (float)m_opts.gridResolution.x;
    graft::update_occupancy_bits(reinterpret_cast<uint32_t*>(d_out), d_masterOccupancyGrid, b.sum, N, G, S,
                                 minDensityThreshold, base_voxel, stream);
    graft::build_mipmaps(d_out, m_opts.gridResolution, m_opts.levelsMipmap, m_opts.numCascades, stream);
}

// ---- .inerf files (InstantNerf.cu:1206-1352) ----
//
// "INERF1", the raw NerfOptions (152 bytes, the CUDA layout), the fp32 master
// hash table [L][T][F], density weights then biases (every layer, hardware
// shapes, output 16), colour weights then biases sized as if the colour head
// had 16 outputs (the hardware head has 8: the rest is zero), the fp32 master
// occupancy grid [C][res^3] and the occupancy bitfield.
static_assert(sizeof(NerfOptions) == 152, "NerfOptions must keep the reference's 152-byte layout (.inerf header)");

namespace {

struct InerfLayout {
    size_t hash, dW, dB, cW, cB, master, bits;
};

InerfLayout inerf_layout(const NerfOptions& o)
{
    InerfLayout s{};
    s.hash = (size_t)o.numLevels * (size_t)o.hashTableSize * (size_t)o.featuresPerLevel;
    const int d_in = o.numLevels * o.featuresPerLevel;
    for (int l = 0; l < o.densityNumLayers; l++) {
        const int in = l == 0 ? d_in : o.densityHiddenDim, out = l == o.densityNumLayers - 1 ? 16 : o.densityHiddenDim;
        s.dW += (size_t)in * out;
        s.dB += (size_t)out;
    }
    for (int l = 0; l < o.colorNumLayers; l++) {
        const int in = l == 0 ? 32 : o.colorHiddenDim, out = l == o.colorNumLayers - 1 ? 16 : o.colorHiddenDim;
        s.cW += (size_t)in * out;
        s.cB += (size_t)out;
    }
    const size_t G = (size_t)o.gridResolution.x * o.gridResolution.y * o.gridResolution.z;
    s.master = (size_t)o.numCascades * G;
    s.bits = ((size_t)graft::mip_offset(o.gridResolution, o.levelsMipmap) * o.numCascades + 7) / 8;
    return s;
}

template <class T>
void write_block(std::FILE* f, const std::vector<T>& v)
{
    if (!v.empty() && std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size())
        throw std::runtime_error("InstantNerf::save: write failed");
}

template <class T>
void read_block(std::FILE* f, std::vector<T>& v)
{
    if (!v.empty() && std::fread(v.data(), sizeof(T), v.size(), f) != v.size())
        throw std::runtime_error("InstantNerf::load: truncated .inerf file");
}

struct FileCloser {
    std::FILE* f;
    ~FileCloser()
    {
        if (f) std::fclose(f);
    }
};

}  // namespace

void InstantNerf::save(const std::string& filename)
{
    if (!m_init) throw std::runtime_error("InstantNerf not initialized, cannot save.");
    GRAFT_HIP_CHECK(hipDeviceSynchronize());
    const InerfLayout L = inerf_layout(m_opts);
    std::vector<float> hash(L.hash), dW(L.dW, 0.f), dB(L.dB, 0.f), cW(L.cW, 0.f), cB(L.cB, 0.f), master(L.master);
    std::vector<uint8_t> bits(L.bits);
    m_densityMLP->saveHashgrid(hash.data());
    m_densityMLP->saveWeights(dW.data(), dB.data());
    m_colorMLP->saveWeights(cW.data(), cB.data());
    GRAFT_HIP_CHECK(hipMemcpy(master.data(), d_masterOccupancyGrid, L.master * sizeof(float), hipMemcpyDeviceToHost));
    GRAFT_HIP_CHECK(hipMemcpy(bits.data(), d_occupancyGrid, L.bits, hipMemcpyDeviceToHost));
    FileCloser fc{std::fopen(filename.c_str(), "wb")};
    if (!fc.f) throw std::runtime_error("Cannot open file for saving: " + filename);
    static const char magic[6] = {'I', 'N', 'E', 'R', 'F', '1'};
    NerfOptions header;
    std::memset(static_cast<void*>(&header), 0, sizeof(header));  // deterministic padding bytes
    header = m_opts;
    if (std::fwrite(magic, 1, 6, fc.f) != 6 || std::fwrite(&header, sizeof(header), 1, fc.f) != 1)
        throw std::runtime_error("InstantNerf::save: write failed");
    write_block(fc.f, hash);
    write_block(fc.f, dW);
    write_block(fc.f, dB);
    write_block(fc.f, cW);
    write_block(fc.f, cB);
    write_block(fc.f, master);
    write_block(fc.f, bits);
}

void InstantNerf::load(const std::string& filename)
{
    FileCloser fc{std::fopen(filename.c_str(), "rb")};
    if (!fc.f) throw std::runtime_error("Cannot open file for loading: " + filename);
    char magic[6];
    if (std::fread(magic, 1, 6, fc.f) != 6 || std::string(magic, 6) != "INERF1")
        throw std::runtime_error("Invalid INERF file format");
    NerfOptions o;
    if (std::fread(&o, sizeof(o), 1, fc.f) != 1) throw std::runtime_error("InstantNerf::load: truncated .inerf file");
    if (o.numLevels <= 0 || o.numLevels > 32 || o.hashTableSize <= 0 || o.featuresPerLevel != 2 ||
        o.numCascades <= 0 || o.numCascades > 16 || o.levelsMipmap <= 0 || o.densityNumLayers <= 0 ||
        o.colorNumLayers <= 0 || o.gridResolution.x == 0 || o.gridResolution.x > 1024 ||
        o.gridResolution.y == 0 || o.gridResolution.y > 1024 || o.gridResolution.z == 0 || o.gridResolution.z > 1024)
        throw std::runtime_error("InstantNerf::load: implausible options in .inerf header");
    const InerfLayout L = inerf_layout(o);
    std::vector<float> hash(L.hash), dW(L.dW), dB(L.dB), cW(L.cW), cB(L.cB), master(L.master);
    std::vector<uint8_t> bits(L.bits);
    read_block(fc.f, hash);
    read_block(fc.f, dW);
    read_block(fc.f, dB);
    read_block(fc.f, cW);
    read_block(fc.f, cB);
    read_block(fc.f, master);
    read_block(fc.f, bits);
    o.isProfiling = false;
    init(o, m_memMode);
    m_densityMLP->loadHashgrid(hash.data());
    m_densityMLP->loadWeights(dW.data(), dB.data());
    m_colorMLP->loadWeights(cW.data(), cB.data());
    GRAFT_HIP_CHECK(hipMemcpy(d_masterOccupancyGrid, master.data(), L.master * sizeof(float), hipMemcpyHostToDevice));
    GRAFT_HIP_CHECK(hipMemcpy(d_occupancyGrid, bits.data(), L.bits, hipMemcpyHostToDevice));
    m_gridVersion++;
}
