// Training ray feed for gfx950: fetchRayChunkStreamingKernel of the reference
// (modules/NeRF/DataLoader.cu:542-679) with the images resident in HBM.
//
// One thread per ray of the chunk: draw an image pixel with pcg_hash (skipping
// every holdout_every-th image), optionally replace it by a depth-prior ray,
// build the pinhole ray from the camera-to-world matrix, and composite the
// RGBA8 pixel over the chunk's background colour.  Integer draws are bit-exact
// with the reference; the direction is normalised with a correctly rounded
// 1 / sqrt (the reference uses fast-math rsqrtf), divisions are correctly rounded.
#include "dataloader.h"

#include <algorithm>

namespace graft {

namespace {

__global__ __launch_bounds__(256) void fetch_ray_chunk_kernel(const RayFeedArgs a)
{
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.size) return;
    const int pixels = a.width * a.height;
    uint32_t global_idx;
    if (a.randomize) {
        const uint32_t rand_val = pcg_hash((uint32_t)(a.offset + idx) + a.seed);
        const int num_imgs = a.total_rays / pixels;
        const int num_test = a.holdout_every >= 2 ? (num_imgs + a.holdout_every - 1) / a.holdout_every : 0;
        const int num_train = num_imgs - num_test;
        if (a.holdout_every >= 2 && num_train >= 1) {
            const int slot = (int)(rand_val % (uint32_t)num_train);
            const int img = (slot / (a.holdout_every - 1)) * a.holdout_every + slot % (a.holdout_every - 1) + 1;
            const uint32_t pix = pcg_hash(rand_val) % (uint32_t)pixels;
            global_idx = (uint32_t)img * (uint32_t)pixels + pix;
        } else {
            global_idx = rand_val % (uint32_t)a.total_rays;
        }
    } else {
        global_idx = (uint32_t)(a.offset + idx) % (uint32_t)a.total_rays;
    }
    int img_idx = (int)(global_idx / (uint32_t)pixels);
    const int pixel_idx = (int)(global_idx % (uint32_t)pixels);
    float px = (float)(pixel_idx % a.width);
    float py = (float)(pixel_idx / a.width);

    float out_D = -1.0f, out_sigma = -1.0f;
    if (a.randomize && a.dense_fraction > 0.0f && a.num_records > 0) {
        const uint32_t hsel = pcg_hash(((uint32_t)idx + 0x9E3779B9u) ^ (a.seed * 2654435761u));
        if ((float)hsel * (1.0f / 4294967296.0f) < a.dense_fraction) {
            const uint32_t r = pcg_hash(hsel) % a.num_records;
            const int f = a.rec_frame[r];
            if (!(a.holdout_every >= 2 && f % a.holdout_every == 0)) {
                img_idx = f;
                px = a.rec_u[r] * a.uv_scale_x;
                py = a.rec_v[r] * a.uv_scale_y;
                out_D = a.rec_D[r];
                out_sigma = a.rec_sigma[r];
                const int pxi = min(max((int)(px + 0.5f), 0), a.width - 1);
                const int pyi = min(max((int)(py + 0.5f), 0), a.height - 1);
                global_idx = (uint32_t)img_idx * (uint32_t)pixels + (uint32_t)(pyi * a.width + pxi);
            }
        }
    }

    float dx = (px - (float)a.width * 0.5f) / a.focal;
    float dy = -(py - (float)a.height * 0.5f) / a.focal;
    float dz = -1.0f;
    const float inv_norm = 1.0f / sqrtf(dx * dx + dy * dy + dz * dz);
    dx *= inv_norm;
    dy *= inv_norm;
    dz *= inv_norm;
    const float* m = a.transforms + (size_t)img_idx * 16;
    a.rays_o[idx] = make_float3(m[3], m[7], m[11]);
    a.rays_d[idx] = make_float3(m[0] * dx + m[1] * dy + m[2] * dz, m[4] * dx + m[5] * dy + m[6] * dz,
                                m[8] * dx + m[9] * dy + m[10] * dz);

    const uchar4 px4 = reinterpret_cast<const uchar4*>(a.images_rgba)[global_idx];
    const float fa = (float)px4.w / 255.0f;
    const float fr = (float)px4.x / 255.0f * fa + a.bg.x * (1.0f - fa);
    const float fg = (float)px4.y / 255.0f * fa + a.bg.y * (1.0f - fa);
    const float fb = (float)px4.z / 255.0f * fa + a.bg.z * (1.0f - fa);
    a.rgb[3 * idx] = fr;
    a.rgb[3 * idx + 1] = fg;
    a.rgb[3 * idx + 2] = fb;
    if (a.dense) a.dense[idx] = out_D;
    if (a.sigma) a.sigma[idx] = out_sigma;
}

// generate_custom_rays_kernel (NerfTrainer.cu:25-47): one pinhole ray per
// pixel (px, py) of a width x height image, c2w row-major 3x4.
__global__ __launch_bounds__(256) void pinhole_rays_kernel(int width, int height, float focal, PinholeCam cam,
                                                           float3* __restrict__ o, float3* __restrict__ d)
{
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= width * height) return;
    const float px = (float)(idx % width), py = (float)(idx / width);
    float dx = (px - (float)width * 0.5f) / focal;
    float dy = -(py - (float)height * 0.5f) / focal;
    float dz = -1.0f;
    const float inv = 1.0f / sqrtf(dx * dx + dy * dy + dz * dz);
    dx *= inv;
    dy *= inv;
    dz *= inv;
    const float* m = cam.m;
    o[idx] = make_float3(m[3], m[7], m[11]);
    d[idx] = make_float3(m[0] * dx + m[1] * dy + m[2] * dz, m[4] * dx + m[5] * dy + m[6] * dz,
                         m[8] * dx + m[9] * dy + m[10] * dz);
}

// Per-ray squared error (r^2 + g^2 + b^2) / 3 of mse_kernel (NerfTrainer.cu:15-23).
__global__ __launch_bounds__(256) void ray_sq_err_kernel(const float* __restrict__ pred,
                                                         const float* __restrict__ target, float* __restrict__ out,
                                                         int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float r = pred[3 * i] - target[3 * i], g = pred[3 * i + 1] - target[3 * i + 1];
    const float b = pred[3 * i + 2] - target[3 * i + 2];
    out[i] = (r * r + g * g + b * b) / 3.0f;
}

}  // namespace

void pinhole_rays(int width, int height, float focal, const float* c2w12, float3* o, float3* d, hipStream_t s)
{
    const int n = width * height;
    if (n <= 0) return;
    PinholeCam cam{};
    for (int k = 0; k < 12; k++) cam.m[k] = c2w12[k];
    hipLaunchKernelGGL(pinhole_rays_kernel, dim3((n + 255) / 256), dim3(256), 0, s, width, height, focal, cam, o, d);
    GRAFT_LAUNCH_CHECK();
}

void ray_sq_err(const float* pred, const float* target, float* out, int n, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(ray_sq_err_kernel, dim3((n + 255) / 256), dim3(256), 0, s, pred, target, out, n);
    GRAFT_LAUNCH_CHECK();
}

void fetch_ray_chunk(const RayFeedArgs& a, hipStream_t s)
{
    if (a.size <= 0) return;
    if (a.width <= 0 || a.height <= 0 || a.total_rays <= 0 || a.total_rays % (a.width * a.height))
        throw std::runtime_error("fetchRayChunk: total_rays must be a positive multiple of width * height");
    if (!a.transforms || !a.images_rgba || !a.rays_o || !a.rays_d || !a.rgb)
        throw std::runtime_error("fetchRayChunk: null buffer");
    if (a.num_records > 0 && (!a.rec_frame || !a.rec_u || !a.rec_v || !a.rec_D || !a.rec_sigma))
        throw std::runtime_error("fetchRayChunk: depth-prior records missing");
    hipLaunchKernelGGL(fetch_ray_chunk_kernel, dim3((a.size + 255) / 256), dim3(256), 0, s, a);
    GRAFT_LAUNCH_CHECK();
}

}  // namespace graft
