// DataLoader: the training ray feed of 3DMaker on MI355X (gfx950).
// Drop-in for the ray-fetch part of modules/NeRF/DataLoader.h:8-103 of the
// reference: same fetchRayChunk() signature and chunk getters, with
// cudaStream_t replaced by hipStream_t.  Images live in device memory
// (RGBA8, [image][row][column][4]) instead of mapped pinned host memory.
//
// Not part of this build: the path constructors (transforms.json parsing,
// image decoding, scene recentring / bounds derivation, DataLoader.cu:1-530);
// the dataset is handed over in memory instead.
#pragma once

#include <hip/hip_runtime_api.h>
#include <hip/hip_vector_types.h>

#include <cstdint>
#include <vector>

class DataLoader {
public:
    // host_rgba: numImages x height x width x 4 bytes; host_transforms:
    // numImages x 16 floats, row-major camera-to-world (NeRF convention,
    // camera looking down -z); focal in pixels.  dense_fraction as in the
    // reference constructor (fraction of depth-prior rays per chunk).
    DataLoader(const uint8_t* host_rgba, const float* host_transforms, int numImages, int width, int height,
               float focal, uint32_t ray_chunk_size, bool is_training = true, float dense_fraction = 0.0f);
    ~DataLoader();

    DataLoader(const DataLoader&) = delete;
    DataLoader& operator=(const DataLoader&) = delete;

    const float3* getChunkRaysO() const { return d_chunk_rays_o; }
    const float3* getChunkRaysD() const { return d_chunk_rays_d; }
    const float* getChunkRgbTrue() const { return d_chunk_rgb_true; }
    const float* getChunkRaysDense() const { return d_chunk_rays_dense; }
    const float* getChunkRaysSigma() const { return d_chunk_rays_sigma; }

    void setDenseRaysFraction(float f) { m_dense_fraction = f; }
    float getDenseRaysFraction() const { return m_dense_fraction; }
    uint32_t getNumDepthRecords() const { return m_num_records; }
    // Depth priors (host arrays of n records): frame index, pixel (u, v) in a
    // depth_width x depth_height image, along-ray depth D and its sigma.
    void setDepthPriors(const int* frame, const float* u, const float* v, const float* D, const float* sigma,
                        uint32_t n, int depth_width, int depth_height);

    // DataLoader.cu:663-679: size rays from offset (sequential) or drawn with
    // pcg_hash from seed (training), skipping every holdout_every-th image.
    void fetchRayChunk(int offset, int size, uint32_t seed, float3 bg_color = make_float3(1.0f, 1.0f, 1.0f),
                       hipStream_t stream = 0, bool forceSequential = false, int holdout_every = 0);
    // Additions (no reference counterpart): a second chunk slot, so the next
    // chunk can be fetched while the current one trains.  fetchRayChunkAhead
    // fills the second slot (allocated on first use); advanceChunk swaps the
    // slots, making the fetched-ahead chunk the current one.
    void fetchRayChunkAhead(int offset, int size, uint32_t seed, float3 bg_color = make_float3(1.0f, 1.0f, 1.0f),
                            hipStream_t stream = 0, bool forceSequential = false, int holdout_every = 0);
    void advanceChunk();
    const float3* getAheadRaysO() const { return d_ahead_rays_o; }
    const float3* getAheadRaysD() const { return d_ahead_rays_d; }
    void freeVRAM();

    uint32_t getTotalRays() const { return total_rays; }
    int getWidth() const { return width; }
    int getHeight() const { return height; }
    float getFocal() const { return focal; }
    int getNumImages() const { return num_images; }
    // DataLoader.h:69: horizontal field of view, 2 atan(w / (2 focal)).
    float getCameraAngleX() const;
    // DataLoader.h:89-92: camera-to-world of frame i (row-major 4x4), zeros when out of range.
    void getFramePose(int i, float out[16]) const;
    // DataLoader.h:49-68: mean camera position and normalised mean camera up axis.
    void getSceneOrientation(float3& center, float3& up) const;
    // DataLoader.h:70: occupancy cascades for this pose set, from the
    // reference's pose-only heuristic (DataLoader.cu:213-271, 367-377); see
    // estimateNumCascades.
    int getNumCascades() const { return estimateNumCascades(h_transforms.data(), num_images); }
    // The heuristic on n row-major camera-to-world matrices: 4 where the view
    // directions are (nearly) parallel and neither converge nor diverge
    // (forward-facing), 3 where the cameras look away from the point their
    // view rays pass closest to (outward panorama), else 1 (bounded: orbit or
    // nadir).  Fewer than 4 poses: 1, the reference loader's default.
    static int estimateNumCascades(const float* transforms, int n);

private:
    int width = 0, height = 0, num_images = 0;
    float focal = 0.0f;
    uint32_t total_rays = 0, m_chunk = 0, m_num_records = 0;
    bool m_is_training = true;
    float m_dense_fraction = 0.0f;
    int m_depth_width = 0, m_depth_height = 0;
    std::vector<float> h_transforms;  // [images][16]
    uint8_t* d_images_rgba = nullptr;
    float* d_transforms = nullptr;
    float3* d_chunk_rays_o = nullptr;
    float3* d_chunk_rays_d = nullptr;
    float* d_chunk_rgb_true = nullptr;
    float* d_chunk_rays_dense = nullptr;
    float* d_chunk_rays_sigma = nullptr;
    float3* d_ahead_rays_o = nullptr;
    float3* d_ahead_rays_d = nullptr;
    float* d_ahead_rgb_true = nullptr;
    float* d_ahead_rays_dense = nullptr;
    float* d_ahead_rays_sigma = nullptr;
    void fetch_into(float3* o, float3* d, float* rgb, float* dense, float* sigma, int offset, int size, uint32_t seed,
                    float3 bg_color, hipStream_t stream, bool forceSequential, int holdout_every);
    int* d_rec_frame = nullptr;
    float* d_rec_u = nullptr;
    float* d_rec_v = nullptr;
    float* d_rec_D = nullptr;
    float* d_rec_sigma = nullptr;
};
