// Flat C handle API over INerfTrainer (include/trainer_capi.h).
#include "DataLoader.h"
#include "NerfTrainer.h"
#include "abi_error.h"
#include "trainer_capi.h"

#include <cstring>
#include <stdexcept>

using graft::guarded;

struct Ntr {
    INerfTrainer t;
};

namespace {

NerfConfig to_config(const NtrConfig& c)
{
    NerfConfig n;
    n.lambdaDepth = c.lambdaDepth;
    n.lambdaDist = c.lambdaDist;
    n.numCascades = c.numCascades;
    n.minDensityThreshold = c.minDensityThreshold;
    n.sampleK = c.sampleK;
    n.batchSize = c.batchSize;
    n.renderBatchSize = c.renderBatchSize;
    n.depthFraction = c.depthFraction;
    n.shouldValidate = c.shouldValidate != 0;
    n.maxLR = c.maxLR;
    n.minLR = c.minLR;
    n.annealSteps = c.annealSteps;
    return n;
}

int copy_image(const Image& img, int width, int height, float* host_rgb)
{
    if (img.width != width || img.height != height) throw std::runtime_error("render: no image");
    std::memcpy(host_rgb, img.rgb.data(), img.rgb.size() * sizeof(float));
    return 0;
}

}  // namespace

#define NTR_CALL(name, body) guarded(name, [&] { if (!h) throw std::runtime_error("null handle"); body; })

extern "C" {

void ntr_default_config(NtrConfig* out)
{
    const NerfConfig d{};
    out->lambdaDepth = d.lambdaDepth;
    out->lambdaDist = d.lambdaDist;
    out->numCascades = d.numCascades;
    out->minDensityThreshold = d.minDensityThreshold;
    out->sampleK = d.sampleK;
    out->batchSize = d.batchSize;
    out->renderBatchSize = d.renderBatchSize;
    out->depthFraction = d.depthFraction;
    out->shouldValidate = d.shouldValidate ? 1 : 0;
    out->maxLR = d.maxLR;
    out->minLR = d.minLR;
    out->annealSteps = d.annealSteps;
}

Ntr* ntr_create(const NtrConfig* config)
{
    Ntr* h = nullptr;
    guarded("ntr_create", [&] {
        if (!config) throw std::runtime_error("null config");
        Ntr* n = new Ntr();
        try {
            n->t.init(to_config(*config));
        } catch (...) {
            delete n;
            throw;
        }
        h = n;
    });
    return h;
}

void ntr_destroy(Ntr* h) { delete h; }

int ntr_load_dataset(Ntr* h, const uint8_t* host_rgba, const float* host_transforms, int num_images, int width,
                     int height, float focal)
{
    return NTR_CALL("ntr_load_dataset", h->t.loadDataset(host_rgba, host_transforms, num_images, width, height, focal));
}
int ntr_begin_training(Ntr* h, int total_steps) { return NTR_CALL("ntr_begin_training", h->t.beginTraining(total_steps)); }
int ntr_train_steps(Ntr* h, int n_steps, NtrStats* out)
{
    return NTR_CALL("ntr_train_steps", {
        const TrainStats s = h->t.trainSteps(n_steps);
        if (out) {
            out->step = s.step;
            out->targetSteps = s.targetSteps;
            out->loss = s.loss;
            out->psnr = s.psnr;
            out->lr = s.lr;
            out->epochs = s.epochs;
            out->msPerStep = s.msPerStep;
            out->etaSeconds = s.etaSeconds;
        }
    });
}
int ntr_validate(Ntr* h, float* psnr_out)
{
    return NTR_CALL("ntr_validate", {
        const float p = h->t.validate();
        if (psnr_out) *psnr_out = p;
    });
}
int ntr_save(Ntr* h, const char* path)
{
    return NTR_CALL("ntr_save", {
        if (!path) throw std::runtime_error("null path");
        h->t.save(path);
    });
}
int ntr_load(Ntr* h, const char* path)
{
    return NTR_CALL("ntr_load", {
        if (!path) throw std::runtime_error("null path");
        h->t.load(path);
    });
}
int ntr_render_orbit(Ntr* h, float azimuth_deg, float elevation_deg, float radius, float fov_deg, int width,
                     int height, float* host_rgb)
{
    return NTR_CALL("ntr_render_orbit", {
        copy_image(h->t.renderOrbit(azimuth_deg, elevation_deg, radius, fov_deg, width, height), width, height,
                   host_rgb);
    });
}
int ntr_render_train_view(Ntr* h, int index, int width, int height, float* host_rgb)
{
    return NTR_CALL("ntr_render_train_view", {
        copy_image(h->t.renderTrainView(index, width, height), width, height, host_rgb);
    });
}
int ntr_num_train_views(Ntr* h) { return h ? h->t.numTrainViews() : 0; }
int ntr_step(Ntr* h) { return h ? h->t.step() : 0; }
int ntr_num_cascades(Ntr* h) { return h ? h->t.numCascades() : 0; }
int ntr_estimate_num_cascades(const float* host_transforms, int n)
{
    return DataLoader::estimateNumCascades(host_transforms, n);
}

}  // extern "C"
