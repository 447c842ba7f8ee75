// Internal interface of the training ray feed (dataloader.hip).
#pragma once

#include "common.h"

namespace graft {

// pcg_hash (DataLoader.cu:542-546): PCG-RXS-M-XS 32-bit output permutation.
__host__ __device__ __forceinline__ uint32_t pcg_hash(uint32_t input)
{
    const uint32_t state = input * 747796405u + 2891336453u;
    const uint32_t word = ((state >> ((state >> 28u) + 4u)) ^ state) * 277803737u;
    return (word >> 22u) ^ word;
}

// Arguments of fetchRayChunkStreamingKernel (DataLoader.cu:548-563).
struct RayFeedArgs {
    int offset, size, total_rays;
    uint32_t seed;
    int randomize;
    int width, height;
    float focal;
    const float* transforms;     // [images][16] row-major camera-to-world
    const uint8_t* images_rgba;  // [images][height][width][4]
    float3* rays_o;
    float3* rays_d;
    float* rgb;                  // [size][3]
    float* dense;                // nullable [size]: depth prior D, -1 = none
    float* sigma;                // nullable [size]: depth prior sigma, -1 = none
    const int* rec_frame;        // depth-prior records (nullable when num_records == 0)
    const float* rec_u;
    const float* rec_v;
    const float* rec_D;
    const float* rec_sigma;
    uint32_t num_records;
    float dense_fraction, uv_scale_x, uv_scale_y;
    float3 bg;
    int holdout_every;
};

void fetch_ray_chunk(const RayFeedArgs& a, hipStream_t s);

struct PinholeCam {
    float m[12];  // rows of the camera-to-world 3x4
};
// generate_custom_rays_kernel (NerfTrainer.cu:25-47): width x height pinhole
// rays, pixel (px, py) -> ((px - w/2)/f, -(py - h/2)/f, -1) rotated by c2w12.
void pinhole_rays(int width, int height, float focal, const float* c2w12, float3* o, float3* d, hipStream_t s);
// out[i] = |pred_i - target_i|^2 / 3 over rgb triples.
void ray_sq_err(const float* pred, const float* target, float* out, int n, hipStream_t s);

}  // namespace graft
