// DataLoader (include/DataLoader.h): device-resident dataset + ray feed, and
// the launchFetchRayChunk C-ABI entry point.
#include "DataLoader.h"

#include "abi_error.h"
#include "dataloader.h"
#include "nerf_abi.h"

#include <cmath>
#include <stdexcept>
#include <utility>

namespace {

template <class T>
T* dcopy(const T* host, size_t n)
{
    void* p = nullptr;
    GRAFT_HIP_CHECK(hipMalloc(&p, n * sizeof(T)));
    if (host) GRAFT_HIP_CHECK(hipMemcpy(p, host, n * sizeof(T), hipMemcpyHostToDevice));
    return static_cast<T*>(p);
}

template <class T>
void dfree(T*& p)
{
    if (p) (void)hipFree(p);
    p = nullptr;
}

}  // namespace

DataLoader::DataLoader(const uint8_t* host_rgba, const float* host_transforms, int numImages, int w, int h, float f,
                       uint32_t ray_chunk_size, bool is_training, float dense_fraction)
    : width(w), height(h), num_images(numImages), focal(f), m_chunk(ray_chunk_size), m_is_training(is_training),
      m_dense_fraction(dense_fraction)
{
    if (!host_rgba || !host_transforms || numImages <= 0 || w <= 0 || h <= 0 || ray_chunk_size == 0)
        throw std::runtime_error("DataLoader: empty dataset or chunk");
    const size_t pixels = (size_t)w * (size_t)h * (size_t)numImages;
    if (pixels > 0xffffffffull) throw std::runtime_error("DataLoader: more than 2^32 pixels");
    total_rays = (uint32_t)pixels;
    h_transforms.assign(host_transforms, host_transforms + (size_t)numImages * 16);
    d_images_rgba = dcopy(host_rgba, pixels * 4);
    d_transforms = dcopy(host_transforms, (size_t)numImages * 16);
    d_chunk_rays_o = dcopy<float3>(nullptr, m_chunk);
    d_chunk_rays_d = dcopy<float3>(nullptr, m_chunk);
    d_chunk_rgb_true = dcopy<float>(nullptr, (size_t)m_chunk * 3);
    d_chunk_rays_dense = dcopy<float>(nullptr, m_chunk);
    d_chunk_rays_sigma = dcopy<float>(nullptr, m_chunk);
}

DataLoader::~DataLoader() { freeVRAM(); }

float DataLoader::getCameraAngleX() const { return 2.0f * std::atan(0.5f * (float)width / focal); }

void DataLoader::getFramePose(int i, float out[16]) const
{
    for (int k = 0; k < 16; ++k) out[k] = (i >= 0 && i < num_images) ? h_transforms[(size_t)i * 16 + k] : 0.0f;
}

void DataLoader::getSceneOrientation(float3& center, float3& up) const
{
    if (num_images == 0) {
        center = make_float3(0, 0, 0);
        up = make_float3(0, 0, 1);
        return;
    }
    float px = 0, py = 0, pz = 0, ux = 0, uy = 0, uz = 0;
    for (int i = 0; i < num_images; i++) {
        const float* m = &h_transforms[(size_t)i * 16];
        px += m[3];
        py += m[7];
        pz += m[11];
        ux += m[1];
        uy += m[5];
        uz += m[9];
    }
    center = make_float3(px / num_images, py / num_images, pz / num_images);
    const float len = std::sqrt(ux * ux + uy * uy + uz * uz);
    up = len > 0 ? make_float3(ux / len, uy / len, uz / len) : make_float3(0, 0, 1);
}

namespace {

double det3x3(const double (&m)[3][3])
{
    return m[0][0] * (m[1][1] * m[2][2] - m[1][2] * m[2][1]) - m[0][1] * (m[1][0] * m[2][2] - m[1][2] * m[2][0]) +
           m[0][2] * (m[1][0] * m[2][1] - m[1][1] * m[2][0]);
}

float norm3f(float x, float y, float z) { return std::sqrt(x * x + y * y + z * z); }

}  // namespace

// DataLoader.cu:213-271 (the regime signals) and 367-377 (the estimate), with
// the reference's precisions: view directions and the inwardness mean in
// fp32, the normal equations in fp64.
int DataLoader::estimateNumCascades(const float* tf, int n)
{
    if (!tf || n < 4) return 1;
    std::vector<float3> dir((size_t)n), eye((size_t)n);
    float3 mean_eye = make_float3(0, 0, 0);
    // normal equations of the point nearest to every view ray:
    // sum_i (I - f_i f_i^T) p = sum_i (I - f_i f_i^T) c_i
    double A[3][3] = {{0, 0, 0}, {0, 0, 0}, {0, 0, 0}}, rhs[3] = {0, 0, 0};
    for (int i = 0; i < n; i++) {
        const float* m = tf + (size_t)i * 16;
        float3 f = make_float3(-m[2], -m[6], -m[10]);  // the camera looks down its -z column
        const float len = norm3f(f.x, f.y, f.z);
        if (len > 1e-8f) f = make_float3(f.x / len, f.y / len, f.z / len);
        const float3 c = make_float3(m[3], m[7], m[11]);
        dir[(size_t)i] = f;
        eye[(size_t)i] = c;
        mean_eye = make_float3(mean_eye.x + c.x, mean_eye.y + c.y, mean_eye.z + c.z);
        const double fv[3] = {f.x, f.y, f.z}, cv[3] = {c.x, c.y, c.z};
        for (int r = 0; r < 3; r++)
            for (int k = 0; k < 3; k++) {
                const double a = (r == k ? 1.0 : 0.0) - fv[r] * fv[k];
                A[r][k] += a;
                rhs[r] += a * cv[k];
            }
    }
    mean_eye = make_float3(mean_eye.x / n, mean_eye.y / n, mean_eye.z / n);
    // (sum_i (I - f_i f_i^T)) / n loses an eigenvalue when the view directions
    // are parallel: a determinant below 0.02 (about 0.3 for spread directions)
    double An[3][3];
    for (int r = 0; r < 3; r++)
        for (int k = 0; k < 3; k++) An[r][k] = A[r][k] / n;
    const bool parallel = std::fabs(det3x3(An)) < 0.02;
    float3 p = mean_eye;  // where the rays do not converge: the mean camera position
    const double d = det3x3(A);
    if (!parallel && std::fabs(d) >= 1e-12) {
        double x[3];
        for (int col = 0; col < 3; col++) {  // Cramer's rule
            double Ac[3][3];
            for (int r = 0; r < 3; r++)
                for (int k = 0; k < 3; k++) Ac[r][k] = k == col ? rhs[r] : A[r][k];
            x[col] = det3x3(Ac) / d;
        }
        p = make_float3((float)x[0], (float)x[1], (float)x[2]);
    }
    // mean cosine between each view direction and the direction to p
    float inward = 0.0f;
    for (int i = 0; i < n; i++) {
        float gx = p.x - eye[(size_t)i].x, gy = p.y - eye[(size_t)i].y, gz = p.z - eye[(size_t)i].z;
        const float gl = norm3f(gx, gy, gz);
        if (gl > 1e-8f) {
            gx /= gl;
            gy /= gl;
            gz /= gl;
        }
        inward += dir[(size_t)i].x * gx + dir[(size_t)i].y * gy + dir[(size_t)i].z * gz;
    }
    inward /= (float)n;
    if (parallel && std::fabs(inward) < 0.3f) return 4;  // forward-facing
    if (inward < -0.3f) return 3;                         // outward panorama
    return 1;                                             // bounded
}

void DataLoader::freeVRAM()
{
    dfree(d_images_rgba);
    dfree(d_transforms);
    dfree(d_chunk_rays_o);
    dfree(d_chunk_rays_d);
    dfree(d_chunk_rgb_true);
    dfree(d_chunk_rays_dense);
    dfree(d_chunk_rays_sigma);
    dfree(d_ahead_rays_o);
    dfree(d_ahead_rays_d);
    dfree(d_ahead_rgb_true);
    dfree(d_ahead_rays_dense);
    dfree(d_ahead_rays_sigma);
    dfree(d_rec_frame);
    dfree(d_rec_u);
    dfree(d_rec_v);
    dfree(d_rec_D);
    dfree(d_rec_sigma);
    m_num_records = 0;
}

void DataLoader::setDepthPriors(const int* frame, const float* u, const float* v, const float* D, const float* sigma,
                                uint32_t n, int depth_width, int depth_height)
{
    dfree(d_rec_frame);
    dfree(d_rec_u);
    dfree(d_rec_v);
    dfree(d_rec_D);
    dfree(d_rec_sigma);
    m_num_records = 0;
    if (n == 0) return;
    for (uint32_t i = 0; i < n; i++)
        if (frame[i] < 0 || frame[i] >= num_images) throw std::runtime_error("DataLoader: depth prior frame out of range");
    d_rec_frame = dcopy(frame, n);
    d_rec_u = dcopy(u, n);
    d_rec_v = dcopy(v, n);
    d_rec_D = dcopy(D, n);
    d_rec_sigma = dcopy(sigma, n);
    m_num_records = n;
    m_depth_width = depth_width;
    m_depth_height = depth_height;
}

void DataLoader::fetchRayChunk(int offset, int size, uint32_t seed, float3 bg_color, hipStream_t stream,
                               bool forceSequential, int holdout_every)
{
    fetch_into(d_chunk_rays_o, d_chunk_rays_d, d_chunk_rgb_true, d_chunk_rays_dense, d_chunk_rays_sigma, offset, size,
               seed, bg_color, stream, forceSequential, holdout_every);
}

void DataLoader::fetchRayChunkAhead(int offset, int size, uint32_t seed, float3 bg_color, hipStream_t stream,
                                    bool forceSequential, int holdout_every)
{
    if (!d_images_rgba) throw std::runtime_error("DataLoader: data freed");
    if (!d_ahead_rays_o) {
        d_ahead_rays_o = dcopy<float3>(nullptr, m_chunk);
        d_ahead_rays_d = dcopy<float3>(nullptr, m_chunk);
        d_ahead_rgb_true = dcopy<float>(nullptr, (size_t)m_chunk * 3);
        d_ahead_rays_dense = dcopy<float>(nullptr, m_chunk);
        d_ahead_rays_sigma = dcopy<float>(nullptr, m_chunk);
    }
    fetch_into(d_ahead_rays_o, d_ahead_rays_d, d_ahead_rgb_true, d_ahead_rays_dense, d_ahead_rays_sigma, offset, size,
               seed, bg_color, stream, forceSequential, holdout_every);
}

void DataLoader::advanceChunk()
{
    if (!d_ahead_rays_o) throw std::runtime_error("DataLoader: no chunk fetched ahead");
    std::swap(d_chunk_rays_o, d_ahead_rays_o);
    std::swap(d_chunk_rays_d, d_ahead_rays_d);
    std::swap(d_chunk_rgb_true, d_ahead_rgb_true);
    std::swap(d_chunk_rays_dense, d_ahead_rays_dense);
    std::swap(d_chunk_rays_sigma, d_ahead_rays_sigma);
}

void DataLoader::fetch_into(float3* o, float3* d, float* rgb, float* dense, float* sigma, int offset, int size,
                            uint32_t seed, float3 bg_color, hipStream_t stream, bool forceSequential,
                            int holdout_every)
{
    if (!d_images_rgba) throw std::runtime_error("DataLoader: data freed");
    if (size < 0 || (uint32_t)size > m_chunk) throw std::runtime_error("DataLoader: chunk larger than ray_chunk_size");
    graft::RayFeedArgs a{};
    a.offset = offset;
    a.size = size;
    a.total_rays = (int)total_rays;
    a.seed = seed;
    a.randomize = (m_is_training && !forceSequential) ? 1 : 0;
    a.width = width;
    a.height = height;
    a.focal = focal;
    a.transforms = d_transforms;
    a.images_rgba = d_images_rgba;
    a.rays_o = o;
    a.rays_d = d;
    a.rgb = rgb;
    a.dense = dense;
    a.sigma = sigma;
    a.rec_frame = d_rec_frame;
    a.rec_u = d_rec_u;
    a.rec_v = d_rec_v;
    a.rec_D = d_rec_D;
    a.rec_sigma = d_rec_sigma;
    a.num_records = m_num_records;
    a.dense_fraction = m_dense_fraction;
    a.uv_scale_x = m_depth_width > 0 ? (float)width / (float)m_depth_width : 1.0f;
    a.uv_scale_y = m_depth_height > 0 ? (float)height / (float)m_depth_height : 1.0f;
    a.bg = bg_color;
    a.holdout_every = holdout_every;
    graft::fetch_ray_chunk(a, stream);
}

extern "C" void launchFetchRayChunk(int offset, int size, int total_rays, uint32_t seed, int randomize, int width,
                                    int height, float focal_length, const float* d_transforms,
                                    const uint8_t* d_images_rgba, float3* d_chunk_rays_o, float3* d_chunk_rays_d,
                                    float* d_chunk_rgb, float* d_chunk_dense, float* d_chunk_sigma,
                                    const int* rec_frame, const float* rec_u, const float* rec_v, const float* rec_D,
                                    const float* rec_sigma, uint32_t num_records, float dense_fraction,
                                    float uv_scale_x, float uv_scale_y, float3 bg_color, int holdout_every,
                                    hipStream_t stream)
{
    graft::guarded("launchFetchRayChunk", [&] {
        graft::RayFeedArgs a{offset, size, total_rays, seed, randomize, width, height, focal_length, d_transforms,
                             d_images_rgba, d_chunk_rays_o, d_chunk_rays_d, d_chunk_rgb, d_chunk_dense,
                             d_chunk_sigma, rec_frame, rec_u, rec_v, rec_D, rec_sigma, num_records, dense_fraction,
                             uv_scale_x, uv_scale_y, bg_color, holdout_every};
        graft::fetch_ray_chunk(a, stream);
    });
}
