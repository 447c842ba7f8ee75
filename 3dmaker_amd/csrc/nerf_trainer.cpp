// INerfTrainer (include/NerfTrainer.h): the reference's training driver
// (modules/NeRF/NerfTrainer.cu) over InstantNerf and the device-resident
// DataLoader.  Host logic only; every device step is a library kernel.
#include "NerfTrainer.h"

#include "dataloader.h"
#include "nerf.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>

namespace {

constexpr float kPI = 3.14159265359f;
constexpr char kSceneMagic[4] = {'S', 'C', 'N', '1'};

template <class T>
T* dalloc(size_t n)
{
    void* p = nullptr;
    GRAFT_HIP_CHECK(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    return static_cast<T*>(p);
}

// Peak signal-to-noise ratio of a mean squared error on [0, 1] colours, with
// the error floored at 1e-8 (80 dB).
float psnr_db(float mse) { return -10.0f * log10f(fmaxf(mse, 1e-8f)); }

// Smoothed wall time per step: the first measurement as is, each later one
// pulls the estimate 30 % of the way towards itself.
double smoothed_ms(double estimate, double measured)
{
    return estimate > 0.0 ? estimate + 0.30 * (measured - estimate) : measured;
}

// The scene footer appended to a saved model: "SCN1", then the scene centre,
// up vector, scale and horizontal field of view (radians) as 8 floats.
struct SceneFooter {
    float center[3];
    float up[3];
    float scale;
    float angle_x;
};
static_assert(sizeof(SceneFooter) == 8 * sizeof(float), "footer layout");
constexpr std::streamoff kSceneFooterBytes = sizeof(kSceneMagic) + sizeof(SceneFooter);

bool read_scene_footer(const std::string& path, SceneFooter& f)
{
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) return false;
    const std::streamoff bytes = in.tellg();
    if (bytes < kSceneFooterBytes) return false;
    char tail[kSceneFooterBytes];
    in.seekg(bytes - kSceneFooterBytes);
    if (!in.read(tail, kSceneFooterBytes)) return false;
    if (std::memcmp(tail, kSceneMagic, sizeof(kSceneMagic)) != 0) return false;
    std::memcpy(&f, tail + sizeof(kSceneMagic), sizeof(f));
    return true;
}

}  // namespace

// NerfTrainer.cu:49-93: the trainer's fixed model (density 64 x 2, colour
// 32 x 3, T = 2^19, 16 levels, b = 1.3819, 128^3 grid, AABB +-1.5).
void INerfTrainer::init(const NerfConfig& config)
{
    m_config = config;
    NerfOptions& o = m_masterConfig;
    o = NerfOptions{};
    o.gridResolution = make_uint3(128, 128, 128);
    o.aabbMin = make_float3(-1.5f, -1.5f, -1.5f);
    o.aabbMax = make_float3(1.5f, 1.5f, 1.5f);
    o.levelsMipmap = 4;
    o.numCascades = config.numCascades > 0 ? config.numCascades : 1;
    o.samplesPerVoxel = config.sampleK;
    o.densityHiddenDim = 64;
    o.densityNumLayers = 2;
    o.colorHiddenDim = 32;
    o.colorNumLayers = 3;
    o.hashTableSize = 1 << 19;
    o.numLevels = 16;
    o.growthFactor = 1.3819f;
    o.baseResolution = 16;
    o.featuresPerLevel = 2;
    o.renderBatchSize = config.renderBatchSize;
    o.batchSize = config.batchSize;
    o.rayChunkSize = config.batchSize / 4;
    o.lambdaDepth = config.lambdaDepth;
    o.lambdaDist = config.lambdaDist;
    o.learningRate = config.maxLR;
    o.beta1 = 0.9f;
    o.beta2 = 0.999f;
    o.epsilon = 1e-8f;
    o.lossScale = 128.0f;
    o.bgColor = make_float3(1.0f, 1.0f, 1.0f);
    o.minDensityThreshold = config.minDensityThreshold;
    o.decayValue = 0.95f;
    o.densityBias = 0.0f;
    o.legacyRenderFlag = false;
    o.isProfiling = false;
    m_holdout_every = config.shouldValidate ? 8 : 0;

    if (!m_d_loss) m_d_loss = dalloc<float>(1);
    GRAFT_HIP_CHECK(hipFree(m_d_chunkRgb));
    GRAFT_HIP_CHECK(hipFree(m_d_err));
    GRAFT_HIP_CHECK(hipFree(m_d_partials));
    m_d_chunkRgb = dalloc<float>((size_t)o.rayChunkSize * 3);
    m_d_err = dalloc<float>((size_t)o.rayChunkSize);
    m_d_partials = dalloc<float>(1024);
}

INerfTrainer::~INerfTrainer()
{
    delete m_nerf;
    delete m_dataloader;
    (void)hipFree(m_d_loss);
    (void)hipFree(m_d_chunkRgb);
    (void)hipFree(m_d_err);
    (void)hipFree(m_d_partials);
}

void INerfTrainer::buildModel()
{
    if (m_nerf) return;
    m_nerf = new InstantNerf();
    m_nerf->init(m_masterConfig, TRAINING);
}

void INerfTrainer::loadDataset(const std::string& path)
{
    throw std::logic_error("INerfTrainer::loadDataset(" + path +
                           "): dataset files are not read by this build; pass the images in memory");
}

void INerfTrainer::loadDataset(const uint8_t* host_rgba, const float* host_transforms, int numImages, int width,
                               int height, float focal)
{
    if (m_masterConfig.rayChunkSize <= 0) throw std::runtime_error("INerfTrainer: init() first");
    dropAheadChunk();
    delete m_dataloader;
    m_dataloader = nullptr;
    m_dataloader = new DataLoader(host_rgba, host_transforms, numImages, width, height, focal,
                                  (uint32_t)m_masterConfig.rayChunkSize, true, m_config.depthFraction);
    m_total_rays = m_dataloader->getTotalRays();
    // NerfTrainer.cu:113-114: numCascades 0 takes the loader's pose estimate
    // (before the model exists; a model built by an earlier call keeps its grid)
    if (m_config.numCascades <= 0) m_masterConfig.numCascades = std::max(1, m_dataloader->getNumCascades());
    buildModel();
    float3 c, up;
    m_dataloader->getSceneOrientation(c, up);
    m_sceneCenter = {0.0f, 0.0f, 0.0f};
    m_sceneUp = {up.x, up.y, up.z};
    m_sceneScale = 1.0f;
    m_cameraAngleX = m_dataloader->getCameraAngleX();
    m_globalStep = 0;
    m_rayCursor = 0;
    m_lossHistory.clear();
}

// NerfTrainer.cu:131-135
float INerfTrainer::currentLR() const
{
    const int anneal = (m_config.annealSteps > 0) ? m_config.annealSteps : std::max(1, m_targetSteps);
    const float progress = fminf((float)m_globalStep / (float)anneal, 1.0f);
    return m_config.minLR + 0.5f * (m_config.maxLR - m_config.minLR) * (1.0f + cosf(kPI * progress));
}

float INerfTrainer::chunkMse(const float* d_pred, const float* d_target, int n)
{
    graft::ray_sq_err(d_pred, d_target, m_d_err, n, 0);
    graft::reduce_sum(m_d_err, (uint32_t)n, m_d_partials, m_d_loss, 0);
    float h = 0.0f;
    GRAFT_HIP_CHECK(hipMemcpy(&h, m_d_loss, sizeof(float), hipMemcpyDeviceToHost));
    return h;
}

// The chunk fetched ahead is not used (the cursor moved or the data changed):
// forget it and rewind the draws made for it, so that the chunk sequence stays
// the one of the serial driver.
void INerfTrainer::dropAheadChunk()
{
    if (!m_ahead.valid) return;
    m_rng = m_ahead.rng_before;
    m_ahead.valid = false;
}

// NerfTrainer.cu:137-179: one ray chunk from the epoch's seed with a random
// background, all of its hit batches, optionally the chunk's colour MSE.
// The next chunk is drawn (epoch seed when the cursor wraps, then the
// background: the order the next call would draw them in) and fetched into
// the loader's second slot before this one trains, so that its first hit
// batch is compacted beside this chunk's last step.
float INerfTrainer::trainOneChunk(bool computeLoss)
{
    const uint32_t rayChunk = (uint32_t)m_masterConfig.rayChunkSize;
    if (m_rayCursor >= m_total_rays) m_rayCursor = 0;
    int chunkSize = 0;
    float3 bg{};
    if (m_ahead.valid && m_ahead.cursor == m_rayCursor) {
        m_dataloader->advanceChunk();
        m_epochSeed = m_ahead.seed;
        chunkSize = m_ahead.size;
        bg = m_ahead.bg;
        m_ahead.valid = false;
    } else {
        dropAheadChunk();
        if (m_rayCursor == 0) m_epochSeed = m_seed_dist(m_rng);
        chunkSize = (int)std::min(rayChunk, m_total_rays - m_rayCursor);
        bg = make_float3(m_dist(m_rng), m_dist(m_rng), m_dist(m_rng));
        m_dataloader->fetchRayChunk((int)m_rayCursor, chunkSize, m_epochSeed, bg, 0, false, (int)m_holdout_every);
    }

    AheadChunk next;
    next.rng_before = m_rng;
    next.cursor = m_rayCursor + (uint32_t)chunkSize;
    if (next.cursor >= m_total_rays) next.cursor = 0;
    next.seed = (next.cursor == 0) ? m_seed_dist(m_rng) : m_epochSeed;
    next.size = (int)std::min(rayChunk, m_total_rays - next.cursor);
    next.bg = make_float3(m_dist(m_rng), m_dist(m_rng), m_dist(m_rng));
    next.valid = true;
    m_dataloader->fetchRayChunkAhead((int)next.cursor, next.size, next.seed, next.bg, 0, false,
                                     (int)m_holdout_every);
    m_ahead = next;

    m_nerf->setLearningRate(currentLR());
    m_nerf->setMemoryMode(TRAINING);
    m_nerf->setBgColor(bg);
    m_nerf->setNextRays(m_dataloader->getAheadRaysO(), m_dataloader->getAheadRaysD(), (uint32_t)next.size);

    std::vector<uint32_t> hitCounts((size_t)chunkSize, 0);
    m_nerf->trainWithRaysHit(m_dataloader->getChunkRaysO(), m_dataloader->getChunkRaysD(),
                             m_dataloader->getChunkRaysDense(), m_dataloader->getChunkRaysSigma(),
                             m_dataloader->getChunkRgbTrue(), (uint32_t)chunkSize, m_globalStep, hitCounts.data(),
                             computeLoss ? m_d_chunkRgb : nullptr, 0);
    m_rayCursor += (uint32_t)chunkSize;
    m_raysSeen += chunkSize;
    if (!computeLoss) return -1.0f;
    return chunkMse(m_d_chunkRgb, m_dataloader->getChunkRgbTrue(), chunkSize) / (float)std::max(1, chunkSize);
}

// Starts a schedule of totalSteps (at least 1) optimizer steps from step 0,
// the first ray of the feed and no loss or timing history
// (NerfTrainer.cu:181-188).
void INerfTrainer::beginTraining(int totalSteps)
{
    dropAheadChunk();
    m_lossHistory.clear();
    m_emaMsPerStep = 0.0;
    m_raysSeen = 0.0;
    m_rayCursor = 0;
    m_globalStep = 0;
    m_targetSteps = totalSteps > 1 ? totalSteps : 1;
}

// Trains whole ray chunks until at least nSteps more optimizer steps have run
// or the schedule is complete (a 20000-step schedule is begun when none was);
// the first chunk of the call also measures its colour MSE
// (NerfTrainer.cu:190-225).  Without a model and dataset it does nothing and
// returns zeroed stats.
TrainStats INerfTrainer::trainSteps(int nSteps)
{
    if (!m_nerf || !m_dataloader || m_total_rays == 0) return TrainStats{};
    if (m_targetSteps == 0) beginTraining(20000);
    const int from = m_globalStep;
    const int until = std::min(m_targetSteps, from + std::max(nSteps, 1));
    const auto started = std::chrono::high_resolution_clock::now();
    float measured = -1.0f;  // this call's chunk MSE, when one was measured
    for (int chunk = 0; m_globalStep < until; chunk++) {
        const float mse = trainOneChunk(chunk == 0);
        if (mse > 0.0f) measured = mse;
    }
    GRAFT_HIP_CHECK(hipDeviceSynchronize());
    const double wall_ms =
        std::chrono::duration<double, std::milli>(std::chrono::high_resolution_clock::now() - started).count();
    if (m_globalStep > from) m_emaMsPerStep = smoothed_ms(m_emaMsPerStep, wall_ms / (m_globalStep - from));
    if (measured > 0.0f) m_lossHistory.push_back(measured);

    TrainStats st;
    st.step = m_globalStep;
    st.targetSteps = m_targetSteps;
    st.loss = measured > 0.0f ? measured : (m_lossHistory.empty() ? 0.0f : m_lossHistory.back());
    st.psnr = st.loss > 0.0f ? psnr_db(st.loss) : 0.0f;
    st.lr = currentLR();
    st.epochs = epochs();
    st.msPerStep = (float)m_emaMsPerStep;
    st.etaSeconds = (float)(m_emaMsPerStep * 1e-3 * std::max(0, m_targetSteps - m_globalStep));
    return st;
}

// NerfTrainer.cu:228-252: progress bar on stdout.
void INerfTrainer::train(int maxSteps, int maxEpochs)
{
    (void)maxEpochs;
    if (!m_nerf || !m_dataloader || m_total_rays == 0)
        throw std::runtime_error("INerfTrainer: train() called before loadDataset()");
    beginTraining(maxSteps);
    const int tick = std::max(1, maxSteps / 100);
    while (!isTrainingDone()) {
        const TrainStats s = trainSteps(tick);
        const float frac = s.targetSteps > 0 ? std::min(1.0f, (float)s.step / (float)s.targetSteps) : 0.0f;
        const int filled = (int)(frac * 28 + 0.5f);
        std::printf("\r[%s%s] %d/%d steps | epoch %.2f | %.2f ms/step | PSNR %.1f   ",
                    std::string((size_t)filled, '#').c_str(), std::string((size_t)(28 - filled), ' ').c_str(), s.step,
                    s.targetSteps, s.epochs, s.msPerStep, s.psnr);
        std::fflush(stdout);
    }
    std::printf("\n");
}

// NerfTrainer.cu:302-327
Image INerfTrainer::renderC2W(const float c2w[16], float focal, int width, int height)
{
    Image img;
    img.width = width;
    img.height = height;
    img.rgb.assign((size_t)width * height * 3, 0.0f);
    if (!m_nerf || width <= 0 || height <= 0) return img;
    const int numRays = width * height;
    float3* d_o = dalloc<float3>((size_t)numRays);
    float3* d_d = dalloc<float3>((size_t)numRays);
    float* d_rgb = dalloc<float>((size_t)numRays * 3);
    try {
        graft::pinhole_rays(width, height, focal, c2w, d_o, d_d, 0);
        m_nerf->setMemoryMode(INFERENCE);
        m_nerf->renderImageHit(d_o, d_d, (uint32_t)numRays, d_rgb, 0);
        GRAFT_HIP_CHECK(hipMemcpy(img.rgb.data(), d_rgb, (size_t)numRays * 3 * sizeof(float), hipMemcpyDeviceToHost));
    } catch (...) {
        (void)hipFree(d_o);
        (void)hipFree(d_d);
        (void)hipFree(d_rgb);
        throw;
    }
    (void)hipFree(d_o);
    (void)hipFree(d_d);
    (void)hipFree(d_rgb);
    return img;
}

// NerfTrainer.cu:329-360: camera on a sphere around the scene centre, looking at it.
Image INerfTrainer::renderOrbit(float azimuthDeg, float elevationDeg, float radius, float fovDeg, int width,
                                int height)
{
    if (!m_nerf) return Image{};
    const float cx = m_sceneCenter.x, cy = m_sceneCenter.y, cz = m_sceneCenter.z;
    float ux = m_sceneUp.x, uy = m_sceneUp.y, uz = m_sceneUp.z;
    const float ul = std::sqrt(ux * ux + uy * uy + uz * uz);
    if (ul > 0) {
        ux /= ul;
        uy /= ul;
        uz /= ul;
    }
    // a, b: an orthonormal basis of the plane normal to up
    const float rx = std::fabs(uy) < 0.9f ? 0.0f : 1.0f, ry = std::fabs(uy) < 0.9f ? 1.0f : 0.0f, rz = 0.0f;
    float ax = uy * rz - uz * ry, ay = uz * rx - ux * rz, az_ = ux * ry - uy * rx;
    const float al = std::sqrt(ax * ax + ay * ay + az_ * az_);
    ax /= al;
    ay /= al;
    az_ /= al;
    const float bx = uy * az_ - uz * ay, by = uz * ax - ux * az_, bz = ux * ay - uy * ax;
    const float az = azimuthDeg * kPI / 180.0f, el = elevationDeg * kPI / 180.0f;
    const float px = std::cos(az) * ax + std::sin(az) * bx, py = std::cos(az) * ay + std::sin(az) * by;
    const float pz = std::cos(az) * az_ + std::sin(az) * bz;
    const float dx = std::cos(el) * px + std::sin(el) * ux, dy = std::cos(el) * py + std::sin(el) * uy;
    const float dz = std::cos(el) * pz + std::sin(el) * uz;
    const float ex = cx + radius * dx, ey = cy + radius * dy, ez = cz + radius * dz;
    float fx = cx - ex, fy = cy - ey, fz = cz - ez;
    const float fl = std::sqrt(fx * fx + fy * fy + fz * fz);
    fx /= fl;
    fy /= fl;
    fz /= fl;
    float sx = fy * uz - fz * uy, sy = fz * ux - fx * uz, sz = fx * uy - fy * ux;
    const float sl = std::sqrt(sx * sx + sy * sy + sz * sz);
    sx /= sl;
    sy /= sl;
    sz /= sl;
    const float vx = sy * fz - sz * fy, vy = sz * fx - sx * fz, vz = sx * fy - sy * fx;
    const float c2w[16] = {sx, vx, -fx, ex, sy, vy, -fy, ey, sz, vz, -fz, ez, 0.0f, 0.0f, 0.0f, 1.0f};
    const float focal = 0.5f * (float)width / std::tan(0.5f * fovDeg * kPI / 180.0f);
    return renderC2W(c2w, focal, width, height);
}

// NerfTrainer.cu:362-371
Image INerfTrainer::renderTrainView(int index, int width, int height)
{
    if (!m_nerf || !m_dataloader) return Image{};
    if (width <= 0) width = m_dataloader->getWidth();
    if (height <= 0) height = m_dataloader->getHeight();
    float c2w[16];
    m_dataloader->getFramePose(index, c2w);
    const float focal = 0.5f * (float)width / std::tan(0.5f * m_dataloader->getCameraAngleX());
    return renderC2W(c2w, focal, width, height);
}

// PSNR over the held-out views (the images training skips: every 8th),
// rendered in tiles of rayChunkSize rays against ground truth composited
// over white, from the per-pixel error (r^2 + g^2 + b^2) / 3 averaged over
// all their pixels (NerfTrainer.cu:378-409).  The model keeps its current
// background colour, the last training chunk's.
float INerfTrainer::validate()
{
    if (!m_nerf || !m_dataloader) return 0.0f;
    const long long pixels = (long long)m_dataloader->getWidth() * m_dataloader->getHeight();
    if (pixels <= 0) return 0.0f;
    constexpr int kHeldOutEvery = 8;
    const long long tile = m_masterConfig.rayChunkSize;
    const float3 white = make_float3(1.0f, 1.0f, 1.0f);
    double squared = 0.0;
    long long seen = 0;
    m_nerf->setMemoryMode(INFERENCE);
    for (int view = 0; view < m_dataloader->getNumImages(); view += kHeldOutEvery) {
        for (long long px = 0; px < pixels; px += tile) {
            const int n = (int)std::min(tile, pixels - px);
            m_dataloader->fetchRayChunk((int)(view * pixels + px), n, 0, white, 0, true, 0);
            m_nerf->renderImageHit(m_dataloader->getChunkRaysO(), m_dataloader->getChunkRaysD(), (uint32_t)n,
                                   m_d_chunkRgb, 0);
            squared += chunkMse(m_d_chunkRgb, m_dataloader->getChunkRgbTrue(), n);
            seen += n;
        }
    }
    m_nerf->setMemoryMode(TRAINING);
    return psnr_db((float)(squared / (double)(seen > 0 ? seen : 1)));
}

// Views in the feed: its rays over the pixels of one view.
int INerfTrainer::numTrainViews() const
{
    if (!m_dataloader) return 0;
    const uint32_t per_view = (uint32_t)std::max(0, m_dataloader->getWidth() * m_dataloader->getHeight());
    return per_view ? (int)(m_total_rays / per_view) : 0;
}

// The model file (InstantNerf::save), then the scene footer (NerfTrainer.cu:262-278).
void INerfTrainer::save(const std::string& path)
{
    if (!m_nerf) return;
    m_nerf->save(path);
    SceneFooter f{{m_sceneCenter.x, m_sceneCenter.y, m_sceneCenter.z},
                  {m_sceneUp.x, m_sceneUp.y, m_sceneUp.z},
                  m_sceneScale,
                  m_cameraAngleX};
    std::ofstream out(path, std::ios::binary | std::ios::app);
    out.write(kSceneMagic, sizeof(kSceneMagic));
    out.write(reinterpret_cast<const char*>(&f), sizeof(f));
    if (!out) throw std::runtime_error("INerfTrainer::save: cannot append the scene footer to " + path);
}

// The model (its options become the trainer's), and the scene fields when the
// file ends with a footer (NerfTrainer.cu:280-300).
void INerfTrainer::load(const std::string& path)
{
    if (!m_nerf) m_nerf = new InstantNerf();
    m_nerf->load(path);
    m_masterConfig = m_nerf->options();
    const size_t chunk = (size_t)m_masterConfig.rayChunkSize;
    (void)hipFree(m_d_chunkRgb);
    (void)hipFree(m_d_err);
    m_d_chunkRgb = dalloc<float>(chunk * 3);
    m_d_err = dalloc<float>(chunk);
    if (!m_d_loss) m_d_loss = dalloc<float>(1);
    if (!m_d_partials) m_d_partials = dalloc<float>(1024);
    SceneFooter f;
    if (!read_scene_footer(path, f)) return;
    m_sceneCenter = {f.center[0], f.center[1], f.center[2]};
    m_sceneUp = {f.up[0], f.up[1], f.up[2]};
    m_sceneScale = f.scale;
    m_cameraAngleX = f.angle_x;
}
