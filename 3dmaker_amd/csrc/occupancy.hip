// Occupancy-grid refresh kernels for gfx950: cell sampling, the per-cell
// max of sampled densities, and the list of occupied cells.
//
//   sampling     sampleAABB / sampleOccupiedAABB   otherKernels.cu:591-648, 852-888
//   tmp max      updateTmpGrid                     otherKernels.cu:650-675
//   active list  extractActiveCells                otherKernels.cu:809-834
//
// Random numbers: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11): 10 rounds of the two 32x32->64
// multiplies with M0 = 0xD2511F53, M1 = 0xCD9E8D57 and the Weyl key schedule
// W0 = 0x9E3779B9, W1 = 0xBB67AE85.  Counter = (sample index, 0, seed lo,
// seed hi), key = (0x3DA3ACB5, 0xA79C5F42).  A 32-bit output u maps to the
// float (u >> 8) * 2^-24 + 2^-25, the centre of one of 2^24 equal bins of
// (0, 1).  This is this library's own stream: the reference draws from
// cuRAND, so sampled cells and jitters are not the reference's.
//
// The occupied-cell list is built in cell order (count, scan, write), so it is
// identical from run to run; the reference appends with an atomic counter.
#include "nerf.h"
#include "nerf_math.h"
#include "occupancy.h"

#include <algorithm>

namespace graft {

namespace {

__host__ __device__ __forceinline__ void philox_round(uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3,
                                                      uint32_t k0, uint32_t k1)
{
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c1 ^ k0;
    const uint32_t n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
}

__host__ __device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1)
{
#pragma unroll
    for (int r = 0; r < 10; r++) {
        philox_round(c[0], c[1], c[2], c[3], k0, k1);
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

__device__ __forceinline__ float u01(uint32_t u) { return (float)(u >> 8) * 5.9604645e-8f + 2.9802322e-8f; }

struct SampleArgs {
    float4* out;
    int N, mode, total_cells, cell_offset;
    const int* list;
    const int* d_list_count;
    uint32_t seed_lo, seed_hi;
    uint3 res;
    float3 mn, mx;
};

__global__ __launch_bounds__(256) void occ_sample_kernel(const SampleArgs a)
{
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.N) return;
    uint32_t c[4] = {(uint32_t)idx, 0u, a.seed_lo, a.seed_hi};
    philox4x32_10(c, 0x3DA3ACB5u, 0xA79C5F42u);
    const float rx = u01(c[0]), ry = u01(c[1]), rz = u01(c[2]), rw = u01(c[3]);
    int cell;
    if (a.mode == kSampleFromList) {
        const int n = *a.d_list_count;
        if (n == 0) return;
        cell = a.list[min((int)(rw * (float)n), n - 1)];
    } else if (a.mode == kSampleEveryCell) {
        cell = a.cell_offset + idx;
    } else {
        cell = a.cell_offset + min((int)(rw * (float)a.total_cells), a.total_cells - 1);
    }
    const int G = (int)(a.res.x * a.res.y * a.res.z);
    const int cascade = cell / G, local = cell % G;
    const int gx = local % (int)a.res.x;
    const int gy = (local / (int)a.res.x) % (int)a.res.y;
    const int gz = local / (int)(a.res.x * a.res.y);
    const float cs = ldexpf(1.0f, cascade);
    const float lx = a.mn.x * cs, ly = a.mn.y * cs, lz = a.mn.z * cs;
    const float hx = a.mx.x * cs, hy = a.mx.y * cs, hz = a.mx.z * cs;
    const float sx = (hx - lx) / (float)a.res.x, sy = (hy - ly) / (float)a.res.y, sz = (hz - lz) / (float)a.res.z;
    const float px = lx + ((float)gx + rx) * sx;
    const float py = ly + ((float)gy + ry) * sy;
    const float pz = lz + ((float)gz + rz) * sz;
    a.out[idx] = make_float4(contract_axis(px, a.mn.x, a.mx.x), contract_axis(py, a.mn.y, a.mx.y),
                             contract_axis(pz, a.mn.z, a.mx.z), __int_as_float(cell));
}

// sigma = e^min(logit - bias, 8) >= 0, so an integer max over the float bits
// is the float max, and the result does not depend on the order of updates.
__global__ __launch_bounds__(256) void occ_tmp_max_kernel(const float4* __restrict__ samples,
                                                          const float* __restrict__ dout, float* __restrict__ tmp,
                                                          float bias, int N)
{
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N) return;
    const int cell = __float_as_int(samples[idx].w);
    const float sigma = nerf_expf(fminf(dout[16 * (size_t)idx] - bias, 8.0f));
    atomicMax(reinterpret_cast<int*>(tmp) + cell, __float_as_int(sigma));
}

__device__ __forceinline__ bool cell_occupied(const uint8_t* bits, int cell, int G, int S)
{
    const int c = cell / G;
    const int pos = c * S + (cell - c * G);
    return (bits[pos >> 3] >> (pos & 7)) & 1;
}

__global__ __launch_bounds__(256) void occ_count_kernel(const uint8_t* __restrict__ bits, int total, int G, int S,
                                                        uint32_t* __restrict__ block_counts, float* __restrict__ zero)
{
    const int cell = blockIdx.x * 256 + threadIdx.x;
    if (zero && cell < total) zero[cell] = 0.0f;
    const bool occ = cell < total && cell_occupied(bits, cell, G, S);
    const int n = __syncthreads_count(occ);
    if (threadIdx.x == 0) block_counts[blockIdx.x] = (uint32_t)n;
}

// One workgroup: exclusive scan of nb block counts in place; *total = sum.
__global__ __launch_bounds__(1024) void occ_scan_kernel(uint32_t* __restrict__ v, int nb, int* __restrict__ total)
{
    __shared__ uint32_t s[1024];
    __shared__ uint32_t s_carry;
    if (threadIdx.x == 0) s_carry = 0;
    __syncthreads();
    for (int base = 0; base < nb; base += 1024) {
        const int i = base + threadIdx.x;
        const uint32_t x = i < nb ? v[i] : 0u;
        s[threadIdx.x] = x;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const uint32_t y = threadIdx.x >= (unsigned)o ? s[threadIdx.x - o] : 0u;
            __syncthreads();
            s[threadIdx.x] += y;
            __syncthreads();
        }
        const uint32_t carry = s_carry;
        if (i < nb) v[i] = carry + s[threadIdx.x] - x;
        __syncthreads();
        if (threadIdx.x == 1023) s_carry = carry + s[1023];
        __syncthreads();
    }
    if (threadIdx.x == 0) *total = (int)s_carry;
}

__global__ __launch_bounds__(256) void occ_write_kernel(const uint8_t* __restrict__ bits, int total, int G, int S,
                                                        const uint32_t* __restrict__ block_offsets,
                                                        int* __restrict__ list)
{
    __shared__ uint32_t s_wave[4];
    const int cell = blockIdx.x * 256 + threadIdx.x;
    const bool occ = cell < total && cell_occupied(bits, cell, G, S);
    const uint64_t m = __ballot(occ);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) s_wave[wave] = (uint32_t)__popcll(m);
    __syncthreads();
    uint32_t before = block_offsets[blockIdx.x];
    for (int w = 0; w < wave; w++) before += s_wave[w];
    const uint64_t below = lane ? (m & ((~0ull) >> (64 - lane))) : 0ull;
    if (occ) list[before + (uint32_t)__popcll(below)] = cell;
}

// Spatial key of a sample's cell for the refresh's evaluation order: the
// cascade, then the Morton code of the cell's 4x4x4 block (bit b of the block
// coordinates x, y, z at bits 3b, 3b + 1, 3b + 2).
struct SortKeyArgs {
    int G;
    uint3 res;
    uint32_t per_cascade;  // P^3, P = blocks per axis rounded up to a power of two
};

__device__ __forceinline__ uint32_t spread3(uint32_t v)
{
    uint32_t m = 0;
#pragma unroll
    for (int b = 0; b < 10; b++) m |= ((v >> b) & 1u) << (3 * b);
    return m;
}

__device__ __forceinline__ uint32_t occ_sort_key(const SortKeyArgs& k, int cell)
{
    const int cascade = cell / k.G, local = cell - cascade * k.G;
    const uint32_t gx = (uint32_t)(local % (int)k.res.x);
    const uint32_t gy = (uint32_t)((local / (int)k.res.x) % (int)k.res.y);
    const uint32_t gz = (uint32_t)(local / (int)(k.res.x * k.res.y));
    return (uint32_t)cascade * k.per_cascade + (spread3(gx >> 2) | (spread3(gy >> 2) << 1) | (spread3(gz >> 2) << 2));
}

// The counting key of sample i: its spatial key in one of kSortCopies key
// ranges, picked by the sample index, so that the many samples of one block
// of occupied cells spread their counter atomics over that many cache lines.
// The order is then (copy, cascade, block): a handful of spatial sweeps.
constexpr uint32_t kSortCopies = 8;

__device__ __forceinline__ uint32_t occ_count_key(const SortKeyArgs& k, uint32_t keys, int i, int cell)
{
    return ((uint32_t)i & (kSortCopies - 1)) * keys + occ_sort_key(k, cell);
}

// rank[i] = the sample's place among the samples of its key (in the order the
// atomics land: any order serves, the per-cell maximum does not depend on it)
__global__ __launch_bounds__(256) void occ_rank_kernel(const float4* __restrict__ samples, int N, const SortKeyArgs k,
                                                       uint32_t keys, uint32_t* __restrict__ counts,
                                                       uint32_t* __restrict__ rank)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= N) return;
    rank[i] = atomicAdd(counts + occ_count_key(k, keys, i, __float_as_int(samples[i].w)), 1u);
}

__global__ __launch_bounds__(256) void occ_place_kernel(const float4* __restrict__ samples, int N, const SortKeyArgs k,
                                                        uint32_t keys, const uint32_t* __restrict__ offsets,
                                                        const uint32_t* __restrict__ rank, float4* __restrict__ sorted,
                                                        uint32_t* __restrict__ perm)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= N) return;
    const float4 v = samples[i];
    const uint32_t j = offsets[occ_count_key(k, keys, i, __float_as_int(v.w))] + rank[i];
    sorted[j] = v;
    perm[j] = (uint32_t)i;
}

int nblocks(int n) { return std::max(1, (n + 255) / 256); }

SortKeyArgs sort_key_args(int cascades, uint3 res, uint32_t* keys)
{
    uint32_t P = 1;
    const uint32_t m = std::max({(res.x + 3) / 4, (res.y + 3) / 4, (res.z + 3) / 4});
    while (P < m) P <<= 1;
    SortKeyArgs k{(int)(res.x * res.y * res.z), res, P * P * P};
    if (keys) *keys = (uint32_t)cascades * k.per_cascade;
    return k;
}

}  // namespace

void occ_sample(float4* out, int N, int mode, int total_cells, int cell_offset, const int* list,
                const int* d_list_count, uint64_t seed, uint3 res, float3 mn, float3 mx, hipStream_t s)
{
    if (N <= 0) return;
    SampleArgs a{};
    a.out = out;
    a.N = N;
    a.mode = mode;
    a.total_cells = total_cells;
    a.cell_offset = cell_offset;
    a.list = list;
    a.d_list_count = d_list_count;
    a.seed_lo = (uint32_t)seed;
    a.seed_hi = (uint32_t)(seed >> 32);
    a.res = res;
    a.mn = mn;
    a.mx = mx;
    hipLaunchKernelGGL(occ_sample_kernel, dim3(nblocks(N)), dim3(256), 0, s, a);
    GRAFT_LAUNCH_CHECK();
}

void occ_tmp_max(const float4* samples, const float* density_out, float* tmp, float bias, int N, hipStream_t s)
{
    if (N <= 0) return;
    hipLaunchKernelGGL(occ_tmp_max_kernel, dim3(nblocks(N)), dim3(256), 0, s, samples, density_out, tmp, bias, N);
    GRAFT_LAUNCH_CHECK();
}

size_t occ_list_scratch_words(int total) { return (size_t)nblocks(total); }

size_t occ_sort_keys(int cascades, uint3 res)
{
    uint32_t keys = 0;
    sort_key_args(cascades, res, &keys);
    return (size_t)keys * kSortCopies;
}

void occ_sort_samples(const float4* samples, int N, int cascades, uint3 res, const OccSortScratch& sc, float4* sorted,
                      uint32_t* perm, hipStream_t s)
{
    if (N <= 0) return;
    uint32_t keys = 0;
    const SortKeyArgs k = sort_key_args(cascades, res, &keys);
    const uint32_t all = keys * kSortCopies;
    GRAFT_HIP_CHECK(hipMemsetAsync(sc.counts, 0, (size_t)all * sizeof(uint32_t), s));
    hipLaunchKernelGGL(occ_rank_kernel, dim3(nblocks(N)), dim3(256), 0, s, samples, N, k, keys, sc.counts, sc.rank);
    GRAFT_LAUNCH_CHECK();
    scan_counts(all, sc.counts, 0xffffffffu, sc.offsets, MarchScratch{sc.block_sums, sc.result}, s);
    hipLaunchKernelGGL(occ_place_kernel, dim3(nblocks(N)), dim3(256), 0, s, samples, N, k, keys, sc.offsets, sc.rank,
                       sorted, perm);
    GRAFT_LAUNCH_CHECK();
}

void occ_active_list(const uint8_t* bits, int total, int G, int S, int* list, int* d_count, uint32_t* scratch,
                     hipStream_t s, float* zero)
{
    const int nb = nblocks(total);
    hipLaunchKernelGGL(occ_count_kernel, dim3(nb), dim3(256), 0, s, bits, total, G, S, scratch, zero);
    GRAFT_LAUNCH_CHECK();
    hipLaunchKernelGGL(occ_scan_kernel, dim3(1), dim3(1024), 0, s, scratch, nb, d_count);
    GRAFT_LAUNCH_CHECK();
    hipLaunchKernelGGL(occ_write_kernel, dim3(nb), dim3(256), 0, s, bits, total, G, S, scratch, list);
    GRAFT_LAUNCH_CHECK();
}

void philox4x32_10_host(uint32_t ctr[4], uint32_t k0, uint32_t k1) { philox4x32_10(ctr, k0, k1); }

}  // namespace graft
