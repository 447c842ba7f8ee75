// Shared device/host helpers for the gfx950 kernels of the TinyMLP / NeRF
// training hot path.  CDNA4 only: 64-wide wavefronts, fp16 MFMA 16x16x16.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#define GRAFT_HIP_CHECK(expr)                                                          \
    do {                                                                               \
        hipError_t _e = (expr);                                                        \
        if (_e != hipSuccess)                                                          \
            throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(_e) + \
                                     " at " __FILE__ ":" + std::to_string(__LINE__));   \
    } while (0)

// Kernel launches report through hipGetLastError right after the launch, so a
// bad configuration surfaces as an exception instead of a silent no-op.
#define GRAFT_LAUNCH_CHECK() GRAFT_HIP_CHECK(hipGetLastError())

namespace graft {

constexpr int kWave = 64;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// D = A(16x16) * B(16x16) + C, fp16 inputs, fp32 accumulation.
// Lane l holds A[l%16][4*(l/16)+j], B[4*(l/16)+j][l%16], D[4*(l/16)+j][l%16].
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 f4zero() { return f4{0.f, 0.f, 0.f, 0.f}; }
__device__ __forceinline__ h4 h4zero() { return h4{(_Float16)0.f, (_Float16)0.f, (_Float16)0.f, (_Float16)0.f}; }

// fp32 -> fp16 round-to-nearest-even (v_cvt_f16_f32 under the default mode).
__device__ __forceinline__ _Float16 to_h(float x) { return (_Float16)x; }

// 8-byte global load/store of four fp16 values.
__device__ __forceinline__ h4 ld_h4(const _Float16* p) { return *reinterpret_cast<const h4*>(p); }
__device__ __forceinline__ void st_h4(_Float16* p, h4 v) { *reinterpret_cast<h4*>(p) = v; }

// Fire-and-forget fp32 atomic add (global_atomic_add_f32 without return).
__device__ __forceinline__ void atomic_add_f32(float* p, float v)
{
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-level grid metadata of a multiresolution hash grid.  The per-level scale
// is one host-computed table, scale[l] = (float)(base * b^l) evaluated in fp64,
// shared with the CPU oracle; res[l] = floor(scale[l]).
constexpr int kMaxLevels = 64;
struct GridMeta {
    float scale[kMaxLevels];
    int res[kMaxLevels];
    int numLevels;
    int tableSize;
    int denseLevelStart;
    int pad_;
};

GridMeta make_grid_meta(int tableSize, int numLevels, float b, int lowestSize);
int dense_level_start(int tableSize, int lowestSize, float b, int numLevels);

// Spatial hash of a lattice corner (prime XOR, uint32 wrap) masked to T.
__device__ __forceinline__ uint32_t hash_coords(int cx, int cy, int cz, uint32_t mask)
{
    return (((uint32_t)cx) ^ ((uint32_t)cy * 2654435761u) ^ ((uint32_t)cz * 805459861u)) & mask;
}

__device__ __forceinline__ uint32_t dense_index(int cx, int cy, int cz, int N_l)
{
    return (uint32_t)(cx + cy * (N_l + 1) + cz * (N_l + 1) * (N_l + 1));
}

// Device scratch of one owner (an MLP instance, or one stream of the
// extern "C" launchers): grown on demand, never shrunk, freed with the owner.
// Kernels of one owner run in stream order, so they never share it with
// another owner's work in flight.  Growing frees the old buffer with
// hipFree, which waits for the device first.
class Workspace {
public:
    Workspace() = default;
    ~Workspace();
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    void* get(size_t bytes);
    size_t size() const { return bytes_; }

private:
    void* p_ = nullptr;
    size_t bytes_ = 0;
};

// The workspace of (current device, stream), for callers without an owner of
// their own (the extern "C" launchers); kept until the process ends.
Workspace& stream_workspace(hipStream_t s);

int num_cus();

// Largest dynamic LDS allocation one workgroup may request on the current
// device (160 KiB on gfx950).
int max_lds_per_block();

}  // namespace graft
