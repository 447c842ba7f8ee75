// Multiresolution hash grid on gfx950: standalone encode and the gradient
// scatter, plus the host-side level table shared with the fused forward.
//
//   encode   networkFusionHashtable.cu:441-551 (encode block of the fused kernel)
//   scatter  networkFusionBackwardHashtable.cu:783-910 (hashTableScatter_Backward)
//
// Thread mapping: one thread per (sample, group of 4 levels), group fastest,
// so the per-sample row of the encoding / its gradient (4 levels x 2 features
// = 16 B per thread) is read and written with contiguous 16-byte accesses,
// and the level metadata comes from LDS.
#include "hashgrid.h"

#include "hash_encode.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <memory>
#include <mutex>

namespace graft {

int dense_level_start(int tableSize, int lowestSize, float b, int numLevels)
{
    // networkFusionHashtable.cu:367-377, host float arithmetic (libm).
    float inner = (std::cbrt(static_cast<float>(tableSize)) - 1.0f) / (float)lowestSize;
    float cont = std::log2(inner) / std::log2(b);
    int d = static_cast<int>(std::floor(cont)) + 1;
    return std::max(0, std::min(d, numLevels));
}

GridMeta make_grid_meta(int tableSize, int numLevels, float b, int lowestSize)
{
    if (numLevels < 1 || numLevels > kMaxLevels)
        throw std::runtime_error("TinyMLPHashGrid: numLevels must be in [1, 64]");
    if (tableSize < 2 || (tableSize & (tableSize - 1)))
        throw std::runtime_error("TinyMLPHashGrid: tableSize must be a power of two");
    GridMeta m{};
    m.numLevels = numLevels;
    m.tableSize = tableSize;
    m.denseLevelStart = dense_level_start(tableSize, lowestSize, b, numLevels);
    for (int l = 0; l < numLevels; l++) {
        m.scale[l] = (float)((double)lowestSize * std::pow((double)b, (double)l));
        m.res[l] = (int)std::floor(m.scale[l]);
        if (l < m.denseLevelStart) {
            const double cells = std::pow((double)m.res[l] + 1.0, 3.0);
            if (cells > (double)tableSize)
                throw std::runtime_error("TinyMLPHashGrid: dense level exceeds the table size");
        }
    }
    return m;
}

namespace {

struct GridKernelArgs {
    const uint32_t* d_n;   // nullable device-side sample count (<= N)
    int L, T, dense_start, pos_stride, N;
    float scale[kMaxLevels];
    int res[kMaxLevels];
};

__device__ __forceinline__ void stage_meta(const GridKernelArgs& a, float* ss, int* sr)
{
    for (int e = threadIdx.x; e < a.L; e += blockDim.x) {
        ss[e] = a.scale[e];
        sr[e] = a.res[e];
    }
    __syncthreads();
}

// gfx950 dispatches workgroup i to XCD i mod 8, and each XCD has its own 4 MB
// L2.  The encode gives each XCD its own levels, so that its L2 holds only
// those levels' fp16 tables (2 MiB per hashed level at T = 2^19) instead of
// cycling all 32 MiB through every L2: levels are dealt to XCDs in snake
// order, l -> l mod 8 for even l / 8 and 7 - l mod 8 for odd, which pairs
// level l with level 15 - l (a small dense level with a hashed one).
constexpr int kXcds = 8;

// Each workgroup encodes, for every sample of its stride, the levels of its
// XCD, 16 k + x and 16 k + 15 - x; both are computed unconditionally (an
// out-of-range level reads level 0 and is not stored) so that their gathers
// are in flight together.  Output: PLANAR, enc[l][plane] feature pairs; else
// row-major enc[n][2L].
template <bool PLANAR>
__global__ __launch_bounds__(256) void hash_encode_kernel(const GridKernelArgs a, const float* __restrict__ pos,
                                                          const _Float16* __restrict__ table,
                                                          _Float16* __restrict__ enc, int plane)
{
    __shared__ float ss[kMaxLevels];
    __shared__ int sr[kMaxLevels];
    stage_meta(a, ss, sr);
    const uint32_t mask = (uint32_t)a.T - 1u;
    const int N = a.d_n ? min((int)*a.d_n, a.N) : a.N;
    const int x = blockIdx.x % kXcds, nb = gridDim.x / kXcds;
    const int D = 2 * a.L;
    for (int n = (blockIdx.x / kXcds) * blockDim.x + threadIdx.x; n < N; n += nb * blockDim.x) {
        const float* pp = pos + (size_t)n * a.pos_stride;
        const float px = pp[0], py = pp[1], pz = pp[2];
        for (int base = 0; base < a.L; base += 2 * kXcds) {
            const int la = base + x, lb = base + 2 * kXcds - 1 - x;
            const bool va = la < a.L, vb = lb < a.L;
            const int ca = va ? la : 0, cb = vb ? lb : 0;
            const float2 ea = encode_level(px, py, pz, ss[ca], sr[ca], ca < a.dense_start, mask,
                                           table + (size_t)ca * a.T * 2);
            const float2 eb = encode_level(px, py, pz, ss[cb], sr[cb], cb < a.dense_start, mask,
                                           table + (size_t)cb * a.T * 2);
            const h2 ha{to_h(ea.x), to_h(ea.y)}, hb{to_h(eb.x), to_h(eb.y)};
            if constexpr (PLANAR) {
                if (va) *reinterpret_cast<h2*>(enc + ((size_t)la * plane + n) * 2) = ha;
                if (vb) *reinterpret_cast<h2*>(enc + ((size_t)lb * plane + n) * 2) = hb;
            } else {
                if (va) *reinterpret_cast<h2*>(enc + (size_t)n * D + 2 * la) = ha;
                if (vb) *reinterpret_cast<h2*>(enc + (size_t)n * D + 2 * lb) = hb;
            }
        }
    }
}

// grads[l][idx][f] += dL/denc[n][2l+f] * w_c for the 8 corners (scatter clamp).
//
// fp32 atomics on gfx950 are priced per cache-line request rather than per
// lane (measured: 4 atomics into one line cost about as much as one), so:
//  - a wave covers 16 consecutive samples at one level, four lanes per sample
//    for (x-corner xs, feature f).  The two x-neighbour corners of a level
//    differ only in the low bits of their index (dense: adjacent entries;
//    hashed: x0 ^ (x0 + 1) touches the low bits only, inside one 16-entry =
//    128-byte block 15 times in 16), so the quad's 4 atomics per y/z corner
//    usually share a line and each lane issues 4 atomics instead of 16;
//  - samples arrive ray by ray, closely spaced, so at coarse levels
//    consecutive samples share corners: a segmented sum over the 16 samples
//    merges equal addresses and only the last lane of each run issues the
//    atomic.  The products g_f * w_c are unchanged; only the order of the
//    fp32 additions differs (the reference's red.add order is unspecified).
__global__ __launch_bounds__(256) void hash_scatter_kernel(const GridKernelArgs a,
                                                           const float* __restrict__ pos,
                                                           const _Float16* __restrict__ denc,
                                                           float* __restrict__ grads)
{
    // This kernel's waves issue ahead of other kernels' waves on the same
    // SIMD (the side stream's work runs beside it): its atomic stream is the
    // step's critical path.
    __builtin_amdgcn_s_setprio(3);
    __shared__ float ss[kMaxLevels];
    __shared__ int sr[kMaxLevels];
    stage_meta(a, ss, sr);
    const uint32_t mask = (uint32_t)a.T - 1u;
    const int D = 2 * a.L;
    const int N = a.d_n ? min((int)*a.d_n, a.N) : a.N;
    const int lane = threadIdx.x & 63;
    const int s = lane >> 2, xs = (lane >> 1) & 1, f = lane & 1;
    const long long nwaves = (long long)((N + 15) / 16) * a.L;
    const long long wstride = ((long long)gridDim.x * blockDim.x) >> 6;
    for (long long w = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6; w < nwaves; w += wstride) {
        const int l = (int)(w % a.L);
        const int n = (int)((w / a.L) * 16 + s);
        const bool valid = n < N;
        Corners c;
        float gv = 0.0f;
        if (valid) {
            const float* pp = pos + (size_t)n * a.pos_stride;
            gv = (float)denc[(size_t)n * D + 2 * l + f];
            level_corners<true>(pp[0], pp[1], pp[2], ss[l], sr[l], l < a.dense_start, mask, c);
        }
        float* lvl = grads + (size_t)l * a.T * 2;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t A = valid ? c.idx[xs + 2 * q] + (uint32_t)f : 0xffffffffu;
            float v = valid ? gv * c.w[xs + 2 * q] : 0.0f;
            const uint32_t A_prev = __shfl_up(A, 4, 64);
            bool seen = (s == 0) || (A != A_prev);  // run head
            const bool head = seen;
#pragma unroll
            for (int d = 1; d < 16; d <<= 1) {
                const float vp = __shfl_up(v, 4 * d, 64);
                const int sp = __shfl_up((int)seen, 4 * d, 64);
                if (s >= d && !seen) {
                    v += vp;
                    seen = sp != 0;
                }
            }
            const int next_head = __shfl_down((int)head, 4, 64);
            const bool tail = (s == 15) || next_head;
            if (valid && tail) atomic_add_f32(lvl + A, v);
        }
    }
}

GridKernelArgs grid_args(const GridMeta& m, int N, int pos_stride)
{
    GridKernelArgs a{};
    a.L = m.numLevels;
    a.T = m.tableSize;
    a.dense_start = m.denseLevelStart;
    a.pos_stride = pos_stride;
    a.N = N;
    for (int l = 0; l < m.numLevels; l++) {
        a.scale[l] = m.scale[l];
        a.res[l] = m.res[l];
    }
    return a;
}

// kXcds workgroups per 256 samples, at most 256 per XCD; at least one per XCD
// so that every level has a workgroup.
int encode_blocks(int N)
{
    return kXcds * std::max(1, std::min((N + 255) / 256, 256));
}

}  // namespace

void hash_encode(const GridMeta& m, const __half* table, const float* pos, int pos_stride,
                 __half* enc, int N, hipStream_t stream, const uint32_t* d_n)
{
    if (N <= 0) return;
    if (pos_stride < 3) throw std::runtime_error("hash encode: position stride must be >= 3");
    GridKernelArgs a = grid_args(m, N, pos_stride);
    a.d_n = d_n;
    hipLaunchKernelGGL(hash_encode_kernel<false>, dim3(encode_blocks(N)), dim3(256), 0, stream, a, pos,
                       reinterpret_cast<const _Float16*>(table), reinterpret_cast<_Float16*>(enc), 0);
    GRAFT_LAUNCH_CHECK();
}

void hash_encode_planar(const GridMeta& m, const __half* table, const float* pos, int pos_stride,
                        __half* enc, int plane, int N, hipStream_t stream, const uint32_t* d_n)
{
    if (N <= 0) return;
    if (pos_stride < 3) throw std::runtime_error("hash encode: position stride must be >= 3");
    if (plane < N) throw std::runtime_error("hash encode: plane stride below the sample count");
    GridKernelArgs a = grid_args(m, N, pos_stride);
    a.d_n = d_n;
    hipLaunchKernelGGL(hash_encode_kernel<true>, dim3(encode_blocks(N)), dim3(256), 0, stream, a, pos,
                       reinterpret_cast<const _Float16*>(table), reinterpret_cast<_Float16*>(enc), plane);
    GRAFT_LAUNCH_CHECK();
}

void hash_scatter_atomic(const GridMeta& m, const __half* denc, const float* pos, int pos_stride,
                         float* grads, int N, hipStream_t stream, const uint32_t* d_n)
{
    if (N <= 0) return;
    if (pos_stride < 3) throw std::runtime_error("hash scatter: position stride must be >= 3");
    GridKernelArgs a = grid_args(m, N, pos_stride);
    a.d_n = d_n;
    // One workgroup per CU: the memory-side atomic rate, not the number of
    // waves issuing atomics, bounds this kernel (measured on a training step:
    // 1 block per CU is as fast as 16), and the idle CU slots then run the
    // side stream's work (next batch's compaction, occupancy refresh).
    const long long threads = (long long)((N + 15) / 16) * m.numLevels * 64;
    const int blocks = (int)std::max(1LL, std::min((threads + 255) / 256, (long long)num_cus()));
    hipLaunchKernelGGL(hash_scatter_kernel, dim3(blocks), dim3(256), 0, stream, a,
                       pos, reinterpret_cast<const _Float16*>(denc), grads);
    GRAFT_LAUNCH_CHECK();
}

// ---------------------------------------------------------------------------
// process-wide helpers
// ---------------------------------------------------------------------------

namespace {
std::mutex g_ws_mu;
int g_cus = 0;
int g_lds = 0;
}  // namespace

int max_lds_per_block()
{
    if (g_lds == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && n > 0)
            g_lds = n;
        else
            g_lds = 64 * 1024;
    }
    return g_lds;
}

Workspace::~Workspace()
{
    if (p_) (void)hipFree(p_);
}

void* Workspace::get(size_t bytes)
{
    if (bytes > bytes_) {
        if (p_) GRAFT_HIP_CHECK(hipFree(p_));
        p_ = nullptr;
        bytes_ = 0;
        const size_t nb = std::max(bytes, (size_t)1 << 16);
        GRAFT_HIP_CHECK(hipMalloc(&p_, nb));
        bytes_ = nb;
    }
    return p_;
}

Workspace& stream_workspace(hipStream_t s)
{
    int dev = 0;
    GRAFT_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_ws_mu);
    static std::map<std::pair<int, hipStream_t>, std::unique_ptr<Workspace>>* cache =
        new std::map<std::pair<int, hipStream_t>, std::unique_ptr<Workspace>>();  // outlives static destructors
    auto& w = (*cache)[{dev, s}];
    if (!w) w.reset(new Workspace());
    return *w;
}

int num_cus()
{
    if (g_cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cus = n;
        else
            g_cus = 256;
    }
    return g_cus;
}

}  // namespace graft
