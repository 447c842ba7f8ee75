/*
 * Flat C handle API over INerfTrainer (include/NerfTrainer.h), for callers
 * that cannot use C++ (ctypes, cgo, JNI).  Each function mirrors one method of
 * modules/NeRF/NerfTrainer.h:43-112; errors return non-zero with the message
 * in tinymlp_last_error_message().  No counterpart exists in the reference,
 * which is C++-only.
 */
#ifndef GRAFT_TRAINER_CAPI_H
#define GRAFT_TRAINER_CAPI_H

#include <stdint.h>

#include "tinymlp_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* NerfConfig (NerfTrainer.h:27-41) field by field; shouldValidate as a byte. */
typedef struct NtrConfig {
    float lambdaDepth, lambdaDist;
    int numCascades;
    float minDensityThreshold;
    int sampleK, batchSize, renderBatchSize;
    float depthFraction;
    uint8_t shouldValidate;
    float maxLR, minLR;
    int annealSteps;
} NtrConfig;

/* TrainStats (NerfTrainer.h:16-25). */
typedef struct NtrStats {
    int step, targetSteps;
    float loss, psnr, lr, epochs, msPerStep, etaSeconds;
} NtrStats;

typedef struct Ntr Ntr;

void ntr_default_config(NtrConfig* out);
Ntr* ntr_create(const NtrConfig* config);
void ntr_destroy(Ntr* h);
/* host_rgba [n][h][w][4] bytes, host_transforms [n][16] row-major c2w, focal in pixels. */
int ntr_load_dataset(Ntr* h, const uint8_t* host_rgba, const float* host_transforms, int num_images, int width,
                     int height, float focal);
int ntr_begin_training(Ntr* h, int total_steps);
int ntr_train_steps(Ntr* h, int n_steps, NtrStats* out);
int ntr_validate(Ntr* h, float* psnr_out);
int ntr_save(Ntr* h, const char* path);
int ntr_load(Ntr* h, const char* path);
/* Host rgb [height][width][3] floats. */
int ntr_render_orbit(Ntr* h, float azimuth_deg, float elevation_deg, float radius, float fov_deg, int width,
                     int height, float* host_rgb);
int ntr_render_train_view(Ntr* h, int index, int width, int height, float* host_rgb);
int ntr_num_train_views(Ntr* h);
int ntr_step(Ntr* h);
/* Occupancy cascades of the trainer's model (its config's, or the loader's
 * estimate when the config asks for 0). */
int ntr_num_cascades(Ntr* h);
/* DataLoader::getNumCascades (DataLoader.h:70) on n row-major camera-to-world
 * matrices, without a loader or a GPU: 1, 3 or 4. */
int ntr_estimate_num_cascades(const float* host_transforms, int n);

#ifdef __cplusplus
}
#endif
#endif
