// Cascaded-occupancy DDA raymarch with hit-centric compaction for gfx950.
//
//   ray setup   compute_ray_aabb_inv_kernel   otherKernels.cu:91-154
//   count pass  march_rays_dda_calc_hits      processRays.cu:626-737
//   scan+cutoff custom_exclusive_sum, find_cutoff_ray_kernel  processRays.cu:486-549, 739-769
//   fill pass   march_rays_dda_offset         processRays.cu:801-929
//
// The reference orchestrates these with three blocking device->host reads per
// step (processRays.cu:979-1013) and marches every ray twice (count, fill).
// Here the compaction runs without any host round trip and marches once:
//   1. store: one thread per ray marches and keeps its sample t values in a
//      rays x 1024 store (4 KiB per ray: HBM capacity traded for the second
//      march; tiles of 64 rays, hit-major, see march_store_index) and its
//      sample count;
//   2. block sums: each 256-ray workgroup reduces its counts;
//   3. scan: one workgroup of 1024 threads scans the block sums and, since the
//      inclusive prefix of counts is monotone, finds the one block holding the
//      cutoff and resolves it ray by ray: active rays = the longest ray prefix
//      whose samples fit in the batch, exactly the reference rule;
//   4. offsets: each workgroup rescans its 256 counts in LDS and writes the
//      exclusive offsets of its rays;
//   5. gather: one thread per compacted sample finds its ray by binary search
//      over the offsets, copies its t and contracts o + t d, writing the
//      samples ray-major (the reference order).
// The march performs the reference's fp32 operations in the reference's
// order, so counts, t values and positions are bit-identical to its count and
// fill passes.  A training step re-compacts the rest of its ray window after
// every hit batch (processRays.cu:931-1040 runs once per optimizer step); the
// counts depend only on the occupancy grid, so a caller re-runs steps 2-5 on
// the stored march until the grid changes.
#include "nerf.h"
#include "nerf_math.h"

#include <algorithm>

namespace graft {

namespace {

constexpr int kMaxMip = 16;

struct MarchArgs {
    const float3* o;
    const float3* d;
    const float3* di;
    const float* nears;
    const float* fars;
    const uint8_t* bits;
    uint3 res;
    float3 mn, mx;
    int C, L, K;
    uint32_t R;
    uint32_t total_cells;        // cells of one cascade pyramid
    uint32_t mip_off[kMaxMip];   // cells below level l
    float3 vs0[kMaxMip];         // cascade-0 voxel size of level l: extent / (res >> l)
    int shift_levels;            // res divisible by 2^(L-1): level-l cells are level-0 cells >> l
};

// Marches ray i, hands sample k (its t value and the level-0 cell it lies in)
// to sink(k, t, ix, iy, iz), and returns the sample count.
//
// The reference loop (processRays.cu:660-733) spends one iteration per mip
// level: at a t it starts at level L-1 and descends while the cell is
// occupied, recomputing the position, cascade and cell coordinates each time
// although t does not change.  Here everything that depends only on t is
// computed once per t, the L cell bytes are loaded together, and the level the
// reference would stop at (the first unoccupied level from the top, else 0) is
// read off the loaded bits.  The operations that produce each value are the
// reference's, so t, the cell indices and the sample t values are
// bit-identical; `it` counts the reference's iterations, descents included.
// The voxel size uses (e * 2^c) / r == 2^c * (e / r), exact for powers of two,
// with e / r precomputed per level.
template <int MAXL, class Sink>
__device__ uint32_t march_ray(const MarchArgs& a, uint32_t i, Sink&& sink)
{
    const float3 o = a.o[i], d = a.d[i], di = a.di[i];
    float t = a.nears[i];
    const float t_max = a.fars[i];
    const float ex = a.mx.x - a.mn.x, ey = a.mx.y - a.mn.y, ez = a.mx.z - a.mn.z;
    const float sx = d.x >= 0.0f ? 1.0f : 0.0f, sy = d.y >= 0.0f ? 1.0f : 0.0f, sz = d.z >= 0.0f ? 1.0f : 0.0f;
    const int L = a.L;  // <= MAXL
    uint32_t hit = 0;
    for (int it = 0; t < t_max && hit < (uint32_t)kMaxHits && it < kMaxMarchIters;) {
        const float px = o.x + t * d.x, py = o.y + t * d.y, pz = o.z + t * d.z;
        int c = 0;
        if (a.C > 1) c = get_cascade(px, py, pz, a.mn, a.mx, a.C);  // one cascade: always 0
        const float cs = ldexpf(1.0f, c);
        const float cminx = a.mn.x * cs, cminy = a.mn.y * cs, cminz = a.mn.z * cs;
        const float cextx = ex * cs, cexty = ey * cs, cextz = ez * cs;
        const float rx = (px - cminx) / cextx, ry = (py - cminy) / cexty, rz = (pz - cminz) / cextz;
        const uint32_t cbase = (uint32_t)c * a.total_cells;
        // every level's byte is loaded without a branch (levels >= L read
        // byte 0 and are ignored), so the loads issue together and the
        // iteration waits for memory once
        uint32_t bit[MAXL], flat[MAXL];
        int ix[MAXL], iy[MAXL], iz[MAXL];
        if (a.shift_levels) {
            // floor(r * (res >> l)) = floor(r * res) >> l when 2^l divides res:
            // the scaling by 2^-l is exact, and so is the clamp's upper end
            const int x0 = clamp_floor_idx(floorf(rx * (float)a.res.x), (int)a.res.x - 1);
            const int y0 = clamp_floor_idx(floorf(ry * (float)a.res.y), (int)a.res.y - 1);
            const int z0 = clamp_floor_idx(floorf(rz * (float)a.res.z), (int)a.res.z - 1);
#pragma unroll
            for (int l = 0; l < MAXL; l++) {
                ix[l] = x0 >> l;
                iy[l] = y0 >> l;
                iz[l] = z0 >> l;
            }
        } else {
#pragma unroll
            for (int l = 0; l < MAXL; l++) {
                const uint32_t rlx = a.res.x >> l, rly = a.res.y >> l, rlz = a.res.z >> l;
                ix[l] = clamp_floor_idx(floorf(rx * (float)rlx), (int)rlx - 1);
                iy[l] = clamp_floor_idx(floorf(ry * (float)rly), (int)rly - 1);
                iz[l] = clamp_floor_idx(floorf(rz * (float)rlz), (int)rlz - 1);
            }
        }
#pragma unroll
        for (int l = 0; l < MAXL; l++) {
            const uint32_t rlx = a.res.x >> l, rly = a.res.y >> l;
            flat[l] = l < L ? cbase + a.mip_off[l] + __umul24((uint32_t)iz[l], rlx * rly) +
                                  __umul24((uint32_t)iy[l], rlx) + (uint32_t)ix[l]
                            : 0u;
        }
        uint8_t byte[MAXL];
#pragma unroll
        for (int l = 0; l < MAXL; l++) byte[l] = a.bits[flat[l] >> 3];
#pragma unroll
        for (int l = 0; l < MAXL; l++) bit[l] = ((uint32_t)byte[l] >> (flat[l] & 7)) & 1u;
        // the reference's level sequence L-1, L-2, ... stops at the first
        // unoccupied level, or at level 0
        int level = L - 1, vix = 0, viy = 0, viz = 0;
        float3 v0 = a.vs0[0];
        bool occ = false;
#pragma unroll
        for (int l = MAXL - 1; l >= 0; l--) {
            if (l == level) {
                vix = ix[l];
                viy = iy[l];
                viz = iz[l];
                v0 = a.vs0[l];
                occ = bit[l] != 0;
                if (occ && l > 0) level = l - 1;
            }
        }
        it += L - level;
        const float vsx = v0.x * cs, vsy = v0.y * cs, vsz = v0.z * cs;
        const float nbx = cminx + ((float)vix + sx) * vsx;
        const float nby = cminy + ((float)viy + sy) * vsy;
        const float nbz = cminz + ((float)viz + sz) * vsz;
        const float next_t = fminf(fminf((nbx - o.x) * di.x, (nby - o.y) * di.y), (nbz - o.z) * di.z);
        if (occ) {  // occupied at level 0: K samples over the voxel, whose exit is next_t
            const float span = next_t - t;
            for (int k = 0; k < a.K; ++k) {
                if (hit >= (uint32_t)kMaxHits) break;
                sink(hit, t + ((float)k + 0.5f) / (float)a.K * span, vix, viy, viz);
                hit++;
            }
        }
        t = fmaxf(t + 1e-5f, next_t + 1e-6f);
    }
    return hit;
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    return v;
}

// Inclusive scan over the workgroup (NW waves of 64); every thread must call.
template <int NW>
__device__ __forceinline__ uint32_t block_incl_scan(uint32_t v, uint32_t* s_wave /* [NW] */)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = wave_incl_scan(v);
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        uint32_t w = lane < NW ? s_wave[lane] : 0u;
        w = wave_incl_scan(w);
        if (lane < NW) s_wave[lane] = w;
    }
    __syncthreads();
    const uint32_t before = wave > 0 ? s_wave[wave - 1] : 0u;
    __syncthreads();
    return incl + before;
}

__global__ __launch_bounds__(256) void ray_aabb_kernel(uint32_t R, const float3* __restrict__ O,
                                                       const float3* __restrict__ D, float3 lo, float3 hi,
                                                       float3* __restrict__ DI, float* __restrict__ nears,
                                                       float* __restrict__ fars)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= R) return;
    const float3 o = O[i];
    float3 d = D[i];
    if (fabsf(d.x) < 1e-8f) d.x = 1e-8f;
    if (fabsf(d.y) < 1e-8f) d.y = 1e-8f;
    if (fabsf(d.z) < 1e-8f) d.z = 1e-8f;
    const float3 inv = make_float3(1.0f / d.x, 1.0f / d.y, 1.0f / d.z);
    DI[i] = inv;
    float t1x = (lo.x - o.x) * inv.x, t2x = (hi.x - o.x) * inv.x;
    if (t1x > t2x) { const float q = t1x; t1x = t2x; t2x = q; }
    float t1y = (lo.y - o.y) * inv.y, t2y = (hi.y - o.y) * inv.y;
    if (t1y > t2y) { const float q = t1y; t1y = t2y; t2y = q; }
    float t1z = (lo.z - o.z) * inv.z, t2z = (hi.z - o.z) * inv.z;
    if (t1z > t2z) { const float q = t1z; t1z = t2z; t2z = q; }
    const float te = fmaxf(fmaxf(t1x, t1y), t1z);
    const float tx = fminf(fminf(t2x, t2y), t2z);
    if (te > tx || tx < 0.0f) {
        nears[i] = 0.0f;
        fars[i] = 0.0f;
    } else {
        nears[i] = fmaxf(te, 0.0f);
        fars[i] = tx;
    }
}

// One workgroup: block_sums (in) -> exclusive block offsets (out, in place);
// result = {active rays, compacted samples}.
__global__ __launch_bounds__(1024) void march_scan_kernel(const uint32_t* __restrict__ counts,
                                                          uint32_t* __restrict__ block_sums, uint32_t nb,
                                                          uint32_t R, uint32_t batch, uint32_t* __restrict__ result)
{
    __shared__ uint32_t s_wave[16];
    __shared__ uint32_t s_carry, s_bstar;
    const uint32_t tid = threadIdx.x;
    if (tid == 0) {
        s_carry = 0;
        s_bstar = 0xffffffffu;
    }
    __syncthreads();
    for (uint32_t base = 0; base < nb; base += 1024) {
        const uint32_t b = base + tid;
        const uint32_t v = b < nb ? block_sums[b] : 0u;
        const uint32_t carry = s_carry;
        const uint32_t incl = carry + block_incl_scan<16>(v, s_wave);
        const uint32_t excl = incl - v;
        if (b < nb) {
            block_sums[b] = excl;
            if (excl <= batch && incl > batch) s_bstar = b;  // unique: prefixes are monotone
        }
        __syncthreads();
        if (tid == 1023) s_carry = incl;
        __syncthreads();
    }
    const uint32_t bstar = s_bstar;
    if (bstar == 0xffffffffu) {
        if (tid == 0) {
            result[0] = R;
            result[1] = s_carry;
        }
        return;
    }
    const uint32_t excl_b = block_sums[bstar];
    const uint32_t i = bstar * 256 + tid;
    const uint32_t c = (tid < 256 && i < R) ? counts[i] : 0u;
    const uint32_t incl = block_incl_scan<16>(c, s_wave);
    const bool ok = tid < 256 && i < R && excl_b + incl <= batch;
    const int n_ok = __syncthreads_count(ok);
    if (n_ok == 0) {
        if (tid == 0) {
            result[0] = bstar * 256;
            result[1] = excl_b;
        }
    } else if ((int)tid == n_ok - 1) {
        result[0] = bstar * 256 + (uint32_t)n_ok;
        result[1] = excl_b + incl;
    }
}

template <int MAXL>
__global__ __launch_bounds__(256) void march_store_kernel(const MarchArgs a, uint32_t* __restrict__ counts,
                                                          float* __restrict__ t_scratch)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.R)
        counts[i] = march_ray<MAXL>(a, i, [&](uint32_t k, float t, int, int, int) {
            t_scratch[march_store_index(i, k)] = t;
        });
}

// march_rays_dda_calc_hits (processRays.cu:626-737): counts only.
template <int MAXL>
__global__ __launch_bounds__(256) void march_count_kernel(const MarchArgs a, uint32_t* __restrict__ counts)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.R) counts[i] = march_ray<MAXL>(a, i, [](uint32_t, float, int, int, int) {});
}

// 30-bit Morton code of a cell: bit b of x, y, z goes to bit 3b, 3b + 1,
// 3b + 2; coordinates are taken mod 2^10 (expand_bits_3d / morton3d,
// processRays.cu:71-82).
__device__ __forceinline__ uint32_t morton30(uint32_t x, uint32_t y, uint32_t z)
{
    uint32_t m = 0;
#pragma unroll
    for (int b = 0; b < 10; b++)
        m |= (((x >> b) & 1u) << (3 * b)) | (((y >> b) & 1u) << (3 * b + 1)) | (((z >> b) & 1u) << (3 * b + 2));
    return m;
}

// march_rays_dda_kernel (processRays.cu:96-226): sample k of ray i at
// t_sparse[i * kMaxHits + k], its cell's Morton code at the same index of
// morton (nullable).
template <int MAXL>
__global__ __launch_bounds__(256) void march_sparse_kernel(const MarchArgs a, uint32_t* __restrict__ counts,
                                                           float* __restrict__ t_sparse,
                                                           uint32_t* __restrict__ morton)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.R) return;
    const size_t row = (size_t)i * kMaxHits;
    counts[i] = march_ray<MAXL>(a, i, [&](uint32_t k, float t, int x, int y, int z) {
        t_sparse[row + k] = t;
        if (morton != nullptr) morton[row + k] = morton30((uint32_t)x, (uint32_t)y, (uint32_t)z);
    });
}

__global__ __launch_bounds__(256) void block_sums_kernel(const uint32_t* __restrict__ counts, uint32_t n,
                                                         uint32_t* __restrict__ block_sums)
{
    __shared__ uint32_t s_wave[4];
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    uint32_t v = i < n ? counts[i] : 0u;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) s_wave[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) block_sums[blockIdx.x] = (s_wave[0] + s_wave[1]) + (s_wave[2] + s_wave[3]);
}

__global__ __launch_bounds__(256) void offsets_kernel(const uint32_t* __restrict__ counts, uint32_t n,
                                                      const uint32_t* __restrict__ block_excl,
                                                      uint32_t* __restrict__ offsets, uint32_t* __restrict__ counts_out)
{
    __shared__ uint32_t s_wave[4];
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t c = i < n ? counts[i] : 0u;
    const uint32_t incl = block_incl_scan<4>(c, s_wave);
    if (i < n) {
        offsets[i] = block_excl[blockIdx.x] + (incl - c);
        if (counts_out != nullptr) counts_out[i] = c;
    }
}

// The ray of compacted sample j: the last of rays [0, active) whose offset
// (less base) is <= j; rays without samples share the next ray's offset.
__device__ __forceinline__ uint32_t ray_of_sample(const uint32_t* __restrict__ offsets, uint32_t base,
                                                  uint32_t active, uint32_t j)
{
    uint32_t lo = 0, hi = active - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        if (offsets[mid] - base <= j) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// One thread per compacted sample j < result[1] of rays [0, result[0]); t
// comes from the stored march, the position is contracted as in the fill.
// The sample index within the ray is clamped to the store's row, so offsets
// that disagree with the stored march cannot read outside it.
struct GatherArgs {
    const float3* o;
    const float3* d;
    float3 mn, mx;
    const uint32_t* offsets;
    uint32_t base;           // subtracted from every offset
    const float* t_scratch;
    uint32_t ray_base;
    const uint32_t* result;
    float* t_out;
    uint32_t* ridx;
    float4* pos_out;
};

__global__ __launch_bounds__(256) void gather_samples_kernel(const GatherArgs g)
{
    const uint32_t active = g.result[0], total = g.result[1];
    for (uint32_t j = blockIdx.x * 256 + threadIdx.x; j < total; j += gridDim.x * 256) {
        const uint32_t lo = ray_of_sample(g.offsets, g.base, active, j);
        const uint32_t k = min(j - (g.offsets[lo] - g.base), (uint32_t)kMaxHits - 1u);
        const float tk = g.t_scratch[march_store_index(g.ray_base + lo, k)];
        const float3 o = g.o[lo], d = g.d[lo];
        g.t_out[j] = tk;
        g.ridx[j] = lo;
        g.pos_out[j] = make_float4(contract_axis(o.x + tk * d.x, g.mn.x, g.mx.x),
                                   contract_axis(o.y + tk * d.y, g.mn.y, g.mx.y),
                                   contract_axis(o.z + tk * d.z, g.mn.z, g.mx.z), 0.0f);
    }
}

// find_cutoff_ray_from_kernel (processRays.cu:771-799): the rays from
// rays_done whose samples fit in batch.  The boundary ray i (the last that
// fits) writes result = {i + 1 - rays_done, its inclusive sample count past
// base, base, i + 1} and *next_done = i + 1; result and *next_done stay zero
// when the first ray does not fit.
__global__ __launch_bounds__(256) void cutoff_from_kernel(uint32_t R, const uint32_t* __restrict__ offsets,
                                                          const uint32_t* __restrict__ counts, uint32_t batch,
                                                          uint32_t rays_done, uint32_t* __restrict__ next_done,
                                                          uint32_t* __restrict__ result)
{
    const uint32_t base = offsets[rays_done];
    for (uint32_t i = rays_done + blockIdx.x * 256 + threadIdx.x; i < R; i += gridDim.x * 256) {
        const uint32_t incl = offsets[i] + counts[i] - base;
        if (incl > batch) continue;
        if (i + 1 < R && offsets[i + 1] + counts[i + 1] - base <= batch) continue;
        result[0] = i + 1 - rays_done;
        result[1] = incl;
        result[2] = base;
        result[3] = i + 1;
        if (next_done != nullptr) *next_done = i + 1;
    }
}

// compact_hits_kernel / compact_hits_linear_kernel (processRays.cu:297-318,
// 466-483), one thread per compacted sample j < result[1] of rays [0, R):
// sparse_idx[j] = ray * kMaxHits + k for sample k of its ray, keys[j] (nullable)
// that sample's Morton code.
__global__ __launch_bounds__(256) void compact_sparse_kernel(uint32_t R, const uint32_t* __restrict__ offsets,
                                                             const uint32_t* __restrict__ result,
                                                             const uint32_t* __restrict__ morton,
                                                             uint32_t* __restrict__ keys,
                                                             uint32_t* __restrict__ sparse_idx)
{
    const uint32_t total = result[1];
    for (uint32_t j = blockIdx.x * 256 + threadIdx.x; j < total; j += gridDim.x * 256) {
        const uint32_t ray = ray_of_sample(offsets, 0u, R, j);
        const uint32_t k = min(j - offsets[ray], (uint32_t)kMaxHits - 1u);
        const uint32_t idx = ray * (uint32_t)kMaxHits + k;
        sparse_idx[j] = idx;
        if (keys != nullptr) keys[j] = morton[idx];
    }
}

// generate_mlp_batch_kernel (processRays.cu:320-356): sample j < result[1]
// is sparse sample sparse_idx[j] of ray sparse_idx[j] / kMaxHits.
__global__ __launch_bounds__(256) void sparse_batch_kernel(const uint32_t* __restrict__ result,
                                                           const uint32_t* __restrict__ sparse_idx,
                                                           const float* __restrict__ t_sparse,
                                                           const float3* __restrict__ O, const float3* __restrict__ D,
                                                           float3 mn, float3 mx, float4* __restrict__ pos_out,
                                                           uint32_t* __restrict__ ridx, float* __restrict__ t_out)
{
    const uint32_t total = result[1];
    for (uint32_t j = blockIdx.x * 256 + threadIdx.x; j < total; j += gridDim.x * 256) {
        const uint32_t idx = sparse_idx[j];
        const uint32_t ray = idx / (uint32_t)kMaxHits;
        const float tk = t_sparse[idx];
        const float3 o = O[ray], d = D[ray];
        pos_out[j] = make_float4(contract_axis(o.x + tk * d.x, mn.x, mx.x), contract_axis(o.y + tk * d.y, mn.y, mx.y),
                                 contract_axis(o.z + tk * d.z, mn.z, mx.z), 0.0f);
        ridx[j] = ray;
        t_out[j] = tk;
    }
}

// compute_real_sh_degree_3_kernel (otherKernels.cu:18-64): out[n][16].
__global__ __launch_bounds__(256) void sh_degree3_kernel(uint32_t n, const float3* __restrict__ dirs,
                                                         float4* __restrict__ out)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float3 d = dirs[i];
    float sh[16];
    sh_basis16(d.x, d.y, d.z, sh);
#pragma unroll
    for (int q = 0; q < 4; q++) out[4 * (size_t)i + q] = make_float4(sh[4 * q], sh[4 * q + 1], sh[4 * q + 2], sh[4 * q + 3]);
}

MarchArgs march_args(uint32_t R, const float3* o, const float3* d, const float3* di, const float* nears,
                     const float* fars, const OccGrid& g, int K)
{
    if (g.mip_levels < 1 || g.mip_levels > kMaxMip) throw std::runtime_error("raymarch: mip levels must be in [1, 16]");
    if (g.cascades < 1) throw std::runtime_error("raymarch: need at least one cascade");
    if (K < 1) throw std::runtime_error("raymarch: samplesPerVoxel must be >= 1");
    if ((g.res.x >> (g.mip_levels - 1)) == 0 || (g.res.y >> (g.mip_levels - 1)) == 0 ||
        (g.res.z >> (g.mip_levels - 1)) == 0)
        throw std::runtime_error("raymarch: grid resolution too small for the mip levels");
    if ((uint64_t)g.res.x * g.res.y >= (1ull << 24) || g.res.z >= (1u << 24))
        throw std::runtime_error("raymarch: grid resolution too large (res.x * res.y must be < 2^24)");
    MarchArgs a{};
    a.o = o;
    a.d = d;
    a.di = di;
    a.nears = nears;
    a.fars = fars;
    a.bits = g.bits;
    a.res = g.res;
    a.mn = g.aabb_min;
    a.mx = g.aabb_max;
    a.C = g.cascades;
    a.L = g.mip_levels;
    a.K = K;
    a.R = R;
    const float ex = g.aabb_max.x - g.aabb_min.x, ey = g.aabb_max.y - g.aabb_min.y, ez = g.aabb_max.z - g.aabb_min.z;
    for (int l = 0; l < g.mip_levels; l++) {
        a.mip_off[l] = mip_offset(g.res, l);
        a.vs0[l] = make_float3(ex / (float)(g.res.x >> l), ey / (float)(g.res.y >> l), ez / (float)(g.res.z >> l));
    }
    a.total_cells = mip_offset(g.res, g.mip_levels);
    const uint32_t m = (1u << (g.mip_levels - 1)) - 1u;
    a.shift_levels = ((g.res.x | g.res.y | g.res.z) & m) == 0 ? 1 : 0;
    return a;
}

}  // namespace

void ray_aabb_inv(uint32_t R, const float3* o, const float3* d, float3 mn, float3 mx, int cascades,
                  float3* d_inv, float* nears, float* fars, hipStream_t s)
{
    if (R == 0) return;
    const float scale = ldexpf(1.0f, cascades - 1);
    const float3 lo = make_float3(mn.x * scale, mn.y * scale, mn.z * scale);
    const float3 hi = make_float3(mx.x * scale, mx.y * scale, mx.z * scale);
    hipLaunchKernelGGL(ray_aabb_kernel, dim3((R + 255) / 256), dim3(256), 0, s, R, o, d, lo, hi, d_inv, nears, fars);
    GRAFT_LAUNCH_CHECK();
}

size_t march_scratch_words(uint32_t R) { return (size_t)(R + 255) / 256 + 2; }

// Launches kernel<MAXL> for the smallest MAXL >= the mip level count.
#define GRAFT_MARCH_LAUNCH(kernel, a, s, ...)                                                               \
    do {                                                                                                    \
        const dim3 grid_((a.R + 255) / 256);                                                                \
        if (a.L <= 4) hipLaunchKernelGGL(kernel<4>, grid_, dim3(256), 0, s, a, __VA_ARGS__);                \
        else if (a.L <= 8) hipLaunchKernelGGL(kernel<8>, grid_, dim3(256), 0, s, a, __VA_ARGS__);           \
        else hipLaunchKernelGGL(kernel<kMaxMip>, grid_, dim3(256), 0, s, a, __VA_ARGS__);                   \
        GRAFT_LAUNCH_CHECK();                                                                               \
    } while (0)

void march_store(uint32_t R, const float3* o, const float3* d, const float3* d_inv, const float* nears,
                 const float* fars, const OccGrid& g, int K, uint32_t* counts, float* t_scratch, hipStream_t s)
{
    if (R == 0) return;
    const MarchArgs a = march_args(R, o, d, d_inv, nears, fars, g, K);
    GRAFT_MARCH_LAUNCH(march_store_kernel, a, s, counts, t_scratch);
}

void march_count(uint32_t R, const float3* o, const float3* d, const float3* d_inv, const float* nears,
                 const float* fars, const OccGrid& g, int K, uint32_t* counts, hipStream_t s)
{
    if (R == 0) return;
    const MarchArgs a = march_args(R, o, d, d_inv, nears, fars, g, K);
    GRAFT_MARCH_LAUNCH(march_count_kernel, a, s, counts);
}

void march_sparse(uint32_t R, const float3* o, const float3* d, const float3* d_inv, const float* nears,
                  const float* fars, const OccGrid& g, int K, uint32_t* counts, float* t_sparse, uint32_t* morton,
                  hipStream_t s)
{
    if (R == 0) return;
    const MarchArgs a = march_args(R, o, d, d_inv, nears, fars, g, K);
    GRAFT_MARCH_LAUNCH(march_sparse_kernel, a, s, counts, t_sparse, morton);
}

void scan_counts(uint32_t R, const uint32_t* counts, uint32_t batch, uint32_t* offsets, const MarchScratch& sc,
                 hipStream_t s, uint32_t* counts_out)
{
    if (R == 0) {
        GRAFT_HIP_CHECK(hipMemsetAsync(sc.result, 0, 2 * sizeof(uint32_t), s));
        return;
    }
    const uint32_t nb = (R + 255) / 256;
    hipLaunchKernelGGL(block_sums_kernel, dim3(nb), dim3(256), 0, s, counts, R, sc.block_sums);
    GRAFT_LAUNCH_CHECK();
    hipLaunchKernelGGL(march_scan_kernel, dim3(1), dim3(1024), 0, s, counts, sc.block_sums, nb, R, batch, sc.result);
    GRAFT_LAUNCH_CHECK();
    hipLaunchKernelGGL(offsets_kernel, dim3(nb), dim3(256), 0, s, counts, R, sc.block_sums, offsets, counts_out);
    GRAFT_LAUNCH_CHECK();
}

static int sample_blocks(uint32_t n) { return (int)std::max<uint32_t>(1, std::min<uint32_t>((n + 255) / 256, 4096)); }

void march_compact_stored(uint32_t R, const float3* o, const float3* d, const OccGrid& g, uint32_t batch,
                          const uint32_t* counts, const float* t_scratch, uint32_t ray_base, uint32_t* offsets,
                          float* t_out, uint32_t* ray_idx, float4* pos_out, const MarchScratch& sc, hipStream_t s,
                          uint32_t* counts_out)
{
    scan_counts(R, counts, batch, offsets, sc, s, counts_out);
    if (R == 0) return;
    GatherArgs ga{o, d, g.aabb_min, g.aabb_max, offsets, 0u, t_scratch, ray_base, sc.result, t_out, ray_idx, pos_out};
    hipLaunchKernelGGL(gather_samples_kernel, dim3(sample_blocks(batch)), dim3(256), 0, s, ga);
    GRAFT_LAUNCH_CHECK();
}

void cutoff_from(uint32_t R, const uint32_t* offsets, const uint32_t* counts, uint32_t batch, uint32_t rays_done,
                 uint32_t* next_done, uint32_t* result, hipStream_t s)
{
    GRAFT_HIP_CHECK(hipMemsetAsync(result, 0, 4 * sizeof(uint32_t), s));
    if (next_done) GRAFT_HIP_CHECK(hipMemsetAsync(next_done, 0, sizeof(uint32_t), s));
    if (rays_done >= R) return;
    const int blocks = (int)std::min<uint32_t>((R - rays_done + 255) / 256, 1024);
    hipLaunchKernelGGL(cutoff_from_kernel, dim3(blocks), dim3(256), 0, s, R, offsets, counts, batch, rays_done,
                       next_done, result);
    GRAFT_LAUNCH_CHECK();
}

void gather_stored(uint32_t max_samples, const float3* o, const float3* d, const OccGrid& g, const uint32_t* offsets,
                   uint32_t base, const float* t_scratch, const uint32_t* result, float* t_out, uint32_t* ray_idx,
                   float4* pos_out, hipStream_t s)
{
    if (max_samples == 0) return;
    GatherArgs ga{o, d, g.aabb_min, g.aabb_max, offsets, base, t_scratch, 0u, result, t_out, ray_idx, pos_out};
    hipLaunchKernelGGL(gather_samples_kernel, dim3(sample_blocks(max_samples)), dim3(256), 0, s, ga);
    GRAFT_LAUNCH_CHECK();
}

void compact_sparse(uint32_t R, const uint32_t* offsets, const uint32_t* result, uint32_t max_samples,
                    const uint32_t* morton, uint32_t* keys, uint32_t* sparse_idx, hipStream_t s)
{
    if (R == 0 || max_samples == 0) return;
    hipLaunchKernelGGL(compact_sparse_kernel, dim3(sample_blocks(max_samples)), dim3(256), 0, s, R, offsets, result,
                       morton, keys, sparse_idx);
    GRAFT_LAUNCH_CHECK();
}

void sparse_batch(const uint32_t* result, uint32_t max_samples, const uint32_t* sparse_idx, const float* t_sparse,
                  const float3* o, const float3* d, float3 aabb_min, float3 aabb_max, float4* pos_out,
                  uint32_t* ray_idx, float* t_out, hipStream_t s)
{
    if (max_samples == 0) return;
    hipLaunchKernelGGL(sparse_batch_kernel, dim3(sample_blocks(max_samples)), dim3(256), 0, s, result, sparse_idx,
                       t_sparse, o, d, aabb_min, aabb_max, pos_out, ray_idx, t_out);
    GRAFT_LAUNCH_CHECK();
}

void sh_degree3(uint32_t n, const float3* dirs, float* out, hipStream_t s)
{
    if (n == 0) return;
    hipLaunchKernelGGL(sh_degree3_kernel, dim3((n + 255) / 256), dim3(256), 0, s, n, dirs,
                       reinterpret_cast<float4*>(out));
    GRAFT_LAUNCH_CHECK();
}

}  // namespace graft
