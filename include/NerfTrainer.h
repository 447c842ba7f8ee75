// INerfTrainer: the training driver of 3DMaker on MI355X (gfx950).
// Drop-in for modules/NeRF/NerfTrainer.h:1-112 of the reference: same
// NerfConfig / TrainStats / Image / Vec3 types and the same training,
// validation, rendering and file entry points over InstantNerf and DataLoader.
//
// Not part of this build: loadDataset(path) (transforms.json parsing, image
// decoding and scene normalisation) throws; the dataset is handed over in
// memory through the loadDataset overload below instead.
#pragma once

#include <cstdint>
#include <random>
#include <string>
#include <vector>

#include "DataLoader.h"
#include "InstantNerf.h"

struct Vec3 {
    float x, y, z;
};

struct Image {
    int width = 0, height = 0;
    std::vector<float> rgb;
};

// NerfTrainer.h:16-25
struct TrainStats {
    int step = 0;
    int targetSteps = 0;
    float loss = 0.0f;
    float psnr = 0.0f;
    float lr = 0.0f;
    float epochs = 0.0f;
    float msPerStep = 0.0f;
    float etaSeconds = 0.0f;
};

// NerfTrainer.h:27-41 (same fields and defaults)
struct NerfConfig {
    float lambdaDepth = 0.01f;
    float lambdaDist = 0.1f;
    int numCascades = 0;
    float minDensityThreshold = 0.01f;
    int sampleK = 1;
    int batchSize = 256 * 1024;
    int renderBatchSize = 256 * 1024;
    float depthFraction = 12.5f / 100.0f;
    bool shouldValidate = false;

    float maxLR = 1e-2f;
    float minLR = 1e-3f;
    int annealSteps = 0;
};

class INerfTrainer {
public:
    INerfTrainer() = default;
    ~INerfTrainer();

    INerfTrainer(const INerfTrainer&) = delete;
    INerfTrainer& operator=(const INerfTrainer&) = delete;

    // NerfTrainer.cu:49-93
    void init(const NerfConfig& config);
    // NerfTrainer.cu:107-129; throws: dataset files are not read by this build.
    void loadDataset(const std::string& path);
    // The dataset in memory: numImages RGBA8 images (host, [n][h][w][4]) and
    // camera-to-world matrices (host, [n][16] row-major), focal in pixels.
    // numCascades 0 in the config takes the loader's estimate from the poses
    // (DataLoader::getNumCascades), as NerfTrainer.cu:113-114 does.
    void loadDataset(const uint8_t* host_rgba, const float* host_transforms, int numImages, int width, int height,
                     float focal);

    // NerfTrainer.cu:241-252
    void train(int maxSteps, int maxEpochs = 0);

    // NerfTrainer.cu:181-227
    void beginTraining(int totalSteps);
    TrainStats trainSteps(int nSteps);
    bool isTrainingDone() const { return m_targetSteps > 0 && m_globalStep >= m_targetSteps; }
    const std::vector<float>& lossHistory() const { return m_lossHistory; }
    int step() const { return m_globalStep; }
    int targetSteps() const { return m_targetSteps; }
    float epochs() const { return (m_total_rays > 0) ? (float)(m_raysSeen / (double)m_total_rays) : 0.0f; }
    float msPerStep() const { return (float)m_emaMsPerStep; }

    // NerfTrainer.cu:373-408: PSNR over every 8th view (holdout), INFERENCE mode.
    float validate();

    // NerfTrainer.cu:269-300: .inerf file plus the "SCN1" scene footer.
    void save(const std::string& path);
    void load(const std::string& path);

    Vec3 sceneCenter() const { return m_sceneCenter; }
    Vec3 sceneUp() const { return m_sceneUp; }

    // NerfTrainer.cu:302-371
    Image renderOrbit(float azimuthDeg, float elevationDeg, float radius, float fovDeg = 50.0f, int width = 800,
                      int height = 800);
    Image renderTrainView(int index, int width = 0, int height = 0);
    int numTrainViews() const;

    // ---- additions (no reference counterpart) ----
    InstantNerf* nerf() { return m_nerf; }
    int numCascades() const { return m_masterConfig.numCascades; }
    DataLoader* dataloader() { return m_dataloader; }

private:
    void buildModel();
    float trainOneChunk(bool computeLoss);
    void dropAheadChunk();
    float currentLR() const;
    Image renderC2W(const float c2w[16], float focal, int width, int height);
    float chunkMse(const float* d_pred, const float* d_target, int n);

    NerfConfig m_config;
    NerfOptions m_masterConfig;
    InstantNerf* m_nerf = nullptr;
    DataLoader* m_dataloader = nullptr;

    uint32_t m_holdout_every = 0;
    uint32_t m_total_rays = 0;

    Vec3 m_sceneCenter = {0.0f, 0.0f, 0.0f};
    Vec3 m_sceneUp = {0.0f, 1.0f, 0.0f};
    float m_sceneScale = 1.0f;
    float m_cameraAngleX = 0.0f;

    int m_globalStep = 0;
    int m_targetSteps = 0;
    uint32_t m_rayCursor = 0;
    uint32_t m_epochSeed = 0;
    std::vector<float> m_lossHistory;

    double m_raysSeen = 0.0;
    double m_emaMsPerStep = 0.0;

    float* m_d_err = nullptr;       // per-ray squared error of a chunk
    float* m_d_partials = nullptr;  // fixed-order reduction scratch
    float* m_d_loss = nullptr;
    float* m_d_chunkRgb = nullptr;

    std::mt19937 m_rng{42};
    std::uniform_real_distribution<float> m_dist{0.0f, 1.0f};
    std::uniform_int_distribution<uint32_t> m_seed_dist{0u, 0xFFFFFFFFu};

    // The next chunk, drawn and fetched into the loader's second slot while
    // the current one trains (InstantNerf::setNextRays compacts its first hit
    // batch beside the current chunk's last step).  rng_before is the draw
    // state before its draws, restored when the chunk is dropped unused.
    struct AheadChunk {
        bool valid = false;
        uint32_t cursor = 0;
        int size = 0;
        uint32_t seed = 0;
        float3 bg{};
        std::mt19937 rng_before;
    } m_ahead;
};
