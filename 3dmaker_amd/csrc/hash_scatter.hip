// Binned hash-grid gradient scatter for gfx950: the table gradient of
// hashTableScatter_Backward (networkFusionBackwardHashtable.cu:783-910),
// grads[l][idx][f] += dL/denc[n][2l+f] * w_c over the 8 corners of every
// (sample, level), backward clamp.
//
// The reference issues one global fp32 atomic per product.  On gfx950 those
// atomics execute beyond the L2 and are priced per 64-byte line request, so a
// 2^18-sample batch at T = 2^19 is bound by about 10 M line requests.  This
// path sorts the products by table slice instead and sums every slice in LDS:
//
//  count       per round of kRound samples: how many corner-pair records fall
//              into each bin (level, kSlice-entry slice of the level) and the
//              largest |dL/denc| of each level;
//  prefix      per bin: exclusive prefix of the counts over the rounds, and
//              the bin's total;
//  distribute  per round: every corner pair becomes one 16-byte record
//              {x0 slot | x1 slot << 16, (g0, g1) as fp16, w of the x0 corner,
//              w of the x1 corner} written at its bin's cursor (bin base +
//              round prefix + LDS rank); workgroup 0 also writes the chunk
//              table (bins of more than kSplit records cut into chunks of
//              kChunk) and the list of bins of several chunks.  The weights are the reference's products
//              (wx * wy) * wz, so every product g * w is the reference's fp32
//              product bit for bit;
//  accumulate  per chunk: the slice's sums in LDS as int64 fixed point
//              (ds_add_u64), then one store per table entry.  A chunk of a
//              bin of several stores its sums as an int64 partial slice
//              instead;
//  merge       per bin of several chunks: the sum of its partial slices, then
//              the same stores.
//              The training step's variant applies Adam to every entry the
//              sums reach instead of storing a gradient (the table half of
//              the optimizer step, optimizerKernel.cu:16-167, fused in): the
//              update sees the gradient the stored path would have stored.
//
// A corner pair is the two x-neighbour corners of one (y, z) corner.  Dense
// levels index them x0 and x0 + 1 of one (y, z) row, and a dense slice is a
// whole number of rows; hashed levels index them x0 ^ H and (x0 + 1) ^ H,
// which differ only below bit bitlen(x0 + 1) <= 12, so both lie in one
// 4096-entry aligned slice.
//
// Fixed point: a product c of level l has |c| <= max|g| of the level
// < 2^(E+1) (the corner weights are <= 1); it adds rint(c * 2^e) with
// e = min(49, 60 - ceil(log2(records of the bin))) - E, so every product is
// below 2^50 (the fp64 rounding trick of fixed_of needs < 2^51) and no
// partial or total sum of the bin reaches 2^62.  Integer addition is exact and order-free: the result
// is the exactly summed fixed-point products rounded once to fp32, whatever
// the record order, chunking or scheduling (deterministic).  Non-finite
// products take an fp32 atomic instead, so NaN/Inf reach the entry as they do
// through the reference's atomics.
//
// Refinement: the level's quantum 2^-e is absolute, so a gradient whose sum
// is tiny against the level's largest gradient keeps few significant bits, and
// one whose products are each below half a quantum, or cancel at that
// resolution, sums to 0 (and the fused update would skip it, where the
// reference's fp32 sum is nonzero and Adam moves the entry).  In a training
// step about a sixth of the touched gradients are such.  A gradient that took
// a product below 2^24 quanta and whose sum is below 2^24 quanta is summed
// again from the bin's records, 2^s times finer (s = min(26, 38 - lg): every
// such product stays below 2^50 units and a sum of 2^lg of them below 2^62).
// Rare cases take further passes: a gradient that also took a product of
// 2^24 quanta or more (products cancelling) is summed at e again; one whose
// finer sum is still below 2^24 units is summed at the scale its largest
// |product| sets, the way the level maximum sets e.  Every other sum is at
// least 2^24 units of its scale (each product within 2^-25 of the sum) or made
// of products of at least 2^24 quanta (each within 2^-25 of the smallest).
#include "scatter.h"

#include "adam_math.h"
#include "hashgrid.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <utility>

namespace graft {

namespace {

constexpr int kSlice = 4096;  // table entries (feature pairs) per bin
constexpr int kSliceShift = 12;
constexpr int kBinThreads = 512;
constexpr int kSamplesPerThread = 1;
constexpr int kRound = kBinThreads * kSamplesPerThread;
// Accumulate chunks: a bin of more than kSplit records is cut into chunks of
// kChunk records, summed by as many workgroups and merged after (the heaviest
// bins, those of the coarse dense levels in a training step, then run on many
// CUs at once); other bins are one chunk each.  The allocation-free entry
// point splits bins of more than kChunkNoAlloc records into chunks of that
// size (fewer partial slices).
constexpr uint32_t kChunk = 8192;
constexpr uint32_t kSplit = 3 * kChunk;
constexpr uint32_t kChunkNoAlloc = 32768;
constexpr int kMaxBins = 8192;
constexpr int kDenseBins = 64;  // target bins per dense level
// word offset of a dense slice's finer sums (a dense slice holds at most
// kSlice / 2 entries, so its 2 * entries words and their finer twins share
// the LDS slice)
constexpr int kFine = kSlice;

struct ScatterArgs {
    const uint32_t* d_n;  // nullable device-side sample count (<= N)
    // nullable, per 16-sample tile: 0 where every dL/denc of the tile is +-0
    // (they add no record; their rows are not read)
    const uint32_t* tile_live;
    int L, T, dense_start, pos_stride, N, bins, rounds;
    uint32_t mask;
    uint32_t chunk;  // records per accumulate chunk of a split bin
    uint32_t split;  // bins of more records are split into chunks
    float scale[kMaxLevels];
    int res[kMaxLevels];
    int bin_base[kMaxLevels + 1];   // bins of level l: [bin_base[l], bin_base[l + 1])
    int rows_per_slice[kMaxLevels]; // dense levels: (y, z) rows of N_l + 1 entries per slice
};

// The four (y, z) corner pairs of one sample at level l, with the backward
// clamp and the weights of level_corners<true> (hash_encode.h); pair q holds
// corners (y_{q&1}, z_{q>>1}).
struct Pairs {
    int bin[4];
    uint32_t key[4];  // slot of x0 within the slice | slot of x1 << 16
    float w0[4];      // weight of the x0 corner, (wx * wy) * wz
    float w1[4];      // weight of the x1 corner, ((1 - wx) * wy) * wz
};

__device__ __forceinline__ void level_pairs(const ScatterArgs& a, int l, float px, float py, float pz, Pairs& p)
{
    const float s = a.scale[l];
    const int N_l = a.res[l];
    const float x_l = px * s, y_l = py * s, z_l = pz * s;
    const float fx = floorf(x_l), fy = floorf(y_l), fz = floorf(z_l);
    const int hi = N_l - 1;
    const int x0 = max(0, min((int)fx, hi));
    const int y0 = max(0, min((int)fy, hi));
    const int z0 = max(0, min((int)fz, hi));
    const int x1 = min(x0 + 1, N_l), y1 = min(y0 + 1, N_l), z1 = min(z0 + 1, N_l);
    const float wx1 = (1.0f - x_l) + fx;
    const float wy1 = (1.0f - y_l) + fy;
    const float wz1 = (1.0f - z_l) + fz;
    const float ux = 1.0f - wx1, uy = 1.0f - wy1, uz = 1.0f - wz1;
    // networkFusionBackwardHashtable.cu:836-839: w = (x-factor * y-factor) * z-factor
    const float ys[2] = {wy1, uy}, zs[2] = {wz1, uz};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        p.w0[q] = (wx1 * ys[q & 1]) * zs[q >> 1];
        p.w1[q] = (ux * ys[q & 1]) * zs[q >> 1];
    }
    const int base = a.bin_base[l];
    if (l < a.dense_start) {
        const int st = N_l + 1;
        const int rps = a.rows_per_slice[l];
        const int rows[4] = {y0 + z0 * st, y1 + z0 * st, y0 + z1 * st, y1 + z1 * st};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int sl = rows[q] / rps;
            const uint32_t s0 = (uint32_t)((rows[q] - sl * rps) * st + x0);
            p.bin[q] = base + sl;
            p.key[q] = s0 | ((s0 + (uint32_t)(x1 - x0)) << 16);
        }
    } else {
        const uint32_t hy0 = (uint32_t)y0 * 2654435761u, hy1 = (uint32_t)y1 * 2654435761u;
        const uint32_t hz0 = (uint32_t)z0 * 805459861u, hz1 = (uint32_t)z1 * 805459861u;
        const uint32_t h[4] = {hy0 ^ hz0, hy1 ^ hz0, hy0 ^ hz1, hy1 ^ hz1};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t s0 = ((uint32_t)x0 ^ h[q]) & a.mask;
            const uint32_t s1 = ((uint32_t)x1 ^ h[q]) & a.mask;
            p.bin[q] = base + (int)(s0 >> kSliceShift);
            p.key[q] = (s0 & (kSlice - 1)) | ((s1 & (kSlice - 1)) << 16);
        }
    }
}

__device__ __forceinline__ int sample_count(const ScatterArgs& a) { return a.d_n ? min((int)*a.d_n, a.N) : a.N; }

// |dL/denc| of a level's feature pair: the larger fp16 magnitude, as bits.
__device__ __forceinline__ uint32_t pair_mag(uint32_t gb) { return max(gb & 0x7fffu, (gb >> 16) & 0x7fffu); }

// dL/denc of levels [l0, l0 + kLevelGroup) of one sample's row, loaded
// together (16-byte loads when the row is 16-byte aligned); zero past L.
constexpr int kLevelGroup = 16;

__device__ __forceinline__ void load_levels(const uint32_t* grow, int l0, int L, bool vec,
                                            uint32_t (&g)[kLevelGroup])
{
    if (vec && l0 + kLevelGroup <= L) {
        const uint4* v = reinterpret_cast<const uint4*>(grow + l0);
#pragma unroll
        for (int j = 0; j < kLevelGroup / 4; j++) {
            const uint4 t = v[j];
            g[4 * j] = t.x;
            g[4 * j + 1] = t.y;
            g[4 * j + 2] = t.z;
            g[4 * j + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < kLevelGroup; j++) g[j] = l0 + j < L ? grow[l0 + j] : 0u;
    }
}

// Lanes whose bin equals the first active lane's add together (one LDS
// atomic): dense levels map most of a wave's samples to a handful of bins.
__device__ __forceinline__ void bin_add(uint32_t* hist, int bin)
{
    const uint64_t act = __ballot(1);
    const int first = __ffsll((unsigned long long)act) - 1;
    const int b0 = __shfl(bin, first, 64);
    const uint64_t same = __ballot(bin == b0);
    if (bin != b0)
        atomicAdd(&hist[bin], 1u);
    else if ((int)(threadIdx.x & 63) == first)
        atomicAdd(&hist[b0], (uint32_t)__popcll(same));
}

// The same with each lane's rank: the slot it takes at its bin's cursor.
__device__ __forceinline__ uint32_t bin_take(uint32_t* cur, int bin)
{
    const uint64_t act = __ballot(1);
    const int first = __ffsll((unsigned long long)act) - 1;
    const int b0 = __shfl(bin, first, 64);
    const uint64_t same = __ballot(bin == b0);
    uint32_t at = 0;
    if (bin != b0) {
        at = atomicAdd(&cur[bin], 1u);
    } else {
        if ((int)(threadIdx.x & 63) == first) at = atomicAdd(&cur[b0], (uint32_t)__popcll(same));
        at = __shfl(at, first, 64) + (uint32_t)__popcll(same & __lanemask_lt());
    }
    return at;
}

__global__ __launch_bounds__(kBinThreads) void scatter_count_kernel(const ScatterArgs a, const float* __restrict__ pos,
                                                                    const _Float16* __restrict__ denc,
                                                                    uint32_t* __restrict__ counts,
                                                                    uint32_t* __restrict__ lvlmax)
{
    extern __shared__ uint32_t sh[];
    uint32_t* hist = sh;
    uint32_t* lmax = sh + a.bins;
    for (int i = threadIdx.x; i < a.bins + a.L; i += kBinThreads) sh[i] = 0u;
    __syncthreads();
    const int N = sample_count(a);
    const bool vec = (a.L & 3) == 0;
    for (int k = 0; k < kSamplesPerThread; k++) {
        const int n = blockIdx.x * kRound + k * kBinThreads + threadIdx.x;
        const bool valid = n < N && (!a.tile_live || a.tile_live[n >> 4] != 0u);
        float px = 0.f, py = 0.f, pz = 0.f;
        const uint32_t* grow = reinterpret_cast<const uint32_t*>(denc + (size_t)(valid ? n : 0) * 2 * a.L);
        if (valid) {
            const float* pp = pos + (size_t)n * a.pos_stride;
            px = pp[0];
            py = pp[1];
            pz = pp[2];
        }
        for (int l0 = 0; l0 < a.L; l0 += kLevelGroup) {
            uint32_t gv[kLevelGroup];
            load_levels(grow, l0, a.L, vec, gv);
#pragma unroll
            for (int j = 0; j < kLevelGroup; j++) {
                const int l = l0 + j;
                if (l >= a.L) break;
                const uint32_t gb = valid ? gv[j] : 0u;
                const bool live = (gb & 0x7fff7fffu) != 0u;  // else both features +-0: no product is nonzero
                const uint32_t m = __ockl_wfred_max_u32(pair_mag(gb));
                if ((threadIdx.x & 63) == 0 && m) atomicMax(&lmax[l], m);
                if (!live) continue;
                Pairs p;
                level_pairs(a, l, px, py, pz, p);
                if (l < a.dense_start) {
#pragma unroll
                    for (int q = 0; q < 4; q++) bin_add(hist, p.bin[q]);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) atomicAdd(&hist[p.bin[q]], 1u);
                }
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.bins; i += kBinThreads) counts[(size_t)blockIdx.x * a.bins + i] = hist[i];
    for (int i = threadIdx.x; i < a.L; i += kBinThreads) lvlmax[(size_t)blockIdx.x * a.L + i] = lmax[i];
}

// Block x: bins [64 x, 64 x + 64), one per lane, and kPrefixWaves waves, each
// over a contiguous range of rounds (every wave load is one 256-byte row
// segment).  counts[r][b] <- sum over r' < r of counts[r'][b]; totals[b].
// Block x < L also reduces level x's per-round maxima.
constexpr int kPrefixWaves = 16;
constexpr int kPrefixThreads = 64 * kPrefixWaves;
constexpr int kPrefixUnroll = 4;  // loads in flight per thread (2, 3, 8 and 16 measured slower)
constexpr int kPrefixBins = 32;  // bins per workgroup (a divisor of 64; 16 and 8 measured slower)

__global__ __launch_bounds__(kPrefixThreads) void scatter_prefix_kernel(const ScatterArgs a, uint32_t* __restrict__ counts,
                                                              uint32_t* __restrict__ totals,
                                                              const uint32_t* __restrict__ lvlmax,
                                                              uint32_t* __restrict__ lvlmax_out)
{
    // kPrefixBins bins per workgroup, the rounds cut into kRanges ranges (one
    // per group of kPrefixBins lanes): short dependent load chains per thread
    constexpr int kSplit = 64 / kPrefixBins;
    constexpr int kRanges = kSplit * kPrefixWaves;
    __shared__ uint32_t part[kRanges][kPrefixBins];
    __shared__ uint32_t wmax[kPrefixWaves];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int q = kSplit * w + lane / kPrefixBins;  // this lane group's range of rounds
    const int bl = lane % kPrefixBins;
    const int b = blockIdx.x * kPrefixBins + bl;
    const int R = a.rounds;
    const int per = (R + kRanges - 1) / kRanges;
    const int r0 = min(R, q * per), r1 = min(R, r0 + per);
    const bool vb = b < a.bins;
    uint32_t s = 0;
    if (vb) {
        int r = r0;
        for (; r + kPrefixUnroll <= r1; r += kPrefixUnroll) {
            uint32_t c[kPrefixUnroll];
#pragma unroll
            for (int k = 0; k < kPrefixUnroll; k++) c[k] = counts[(size_t)(r + k) * a.bins + b];
#pragma unroll
            for (int k = 0; k < kPrefixUnroll; k++) s += c[k];
        }
        for (; r < r1; r++) s += counts[(size_t)r * a.bins + b];
    }
    part[q][bl] = s;
    if ((int)blockIdx.x < a.L) {
        uint32_t m = 0;
        for (int r = threadIdx.x; r < R; r += kPrefixThreads) m = max(m, lvlmax[(size_t)r * a.L + blockIdx.x]);
        m = __ockl_wfred_max_u32(m);
        if (lane == 0) wmax[w] = m;
    }
    __syncthreads();
    if ((int)blockIdx.x < a.L && threadIdx.x == 0) {
        uint32_t m = 0;
        for (int k = 0; k < kPrefixWaves; k++) m = max(m, wmax[k]);
        lvlmax_out[blockIdx.x] = m;
    }
    uint32_t run = 0;
    for (int k = 0; k < q; k++) run += part[k][bl];
    if (vb) {
        int r = r0;
        for (; r + kPrefixUnroll <= r1; r += kPrefixUnroll) {
            uint32_t c[kPrefixUnroll];
#pragma unroll
            for (int k = 0; k < kPrefixUnroll; k++) c[k] = counts[(size_t)(r + k) * a.bins + b];
#pragma unroll
            for (int k = 0; k < kPrefixUnroll; k++) {
                counts[(size_t)(r + k) * a.bins + b] = run;
                run += c[k];
            }
        }
        for (; r < r1; r++) {
            const size_t i = (size_t)r * a.bins + b;
            const uint32_t c = counts[i];
            counts[i] = run;
            run += c;
        }
        if (q == kRanges - 1) totals[b] = run;
    }
}

// Exclusive prefix sum of in[0, n) into out[0, n) (in == out allowed: every
// thread reads and writes only its own segment); returns the total.  Every
// thread of the kBinThreads-thread block calls it; wsum is kBinThreads / 64
// words of LDS.  T: uint32_t, or uint64_t for several counters packed in
// bit fields that cannot carry into each other.
template <class T>
__device__ T block_exclusive_scan(const T* in, T* out, int n, T* wsum)
{
    constexpr int kWaves = kBinThreads / 64;
    const int per = (n + kBinThreads - 1) / kBinThreads;
    const int b0 = min(n, (int)threadIdx.x * per), b1 = min(n, b0 + per);
    T s = 0;
    for (int i = b0; i < b1; i++) s += in[i];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    T x = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const T y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    T run = x - s, total = 0;
    for (int k = 0; k < kWaves; k++) {
        if (k < w) run += wsum[k];
        total += wsum[k];
    }
    for (int i = b0; i < b1; i++) {
        const T v = in[i];
        out[i] = run;
        run += v;
    }
    __syncthreads();
    return total;
}

// Chunk table entries (uint4): bin, first record, end record, and the
// chunk's partial slice, or kSoleOwner for a bin of one chunk.  Merge list
// entries: bin, the bin's first record, its first partial slice, its chunk
// count.
constexpr uint32_t kSoleOwner = 0xffffffffu;

// Bins of one chunk finished in the accumulate's second phase, beside the
// merges (about one block per block slot of the GPU, two per CU).
constexpr uint32_t kLateChunks = 448;

// Workgroup 0 also writes the chunk table and the merge list of the
// accumulate pass (the heaviest work first): the chunks of the bins of more
// than a.split records (cut into chunks of a.chunk records), then the other
// bins of more than a.chunk records, then the remaining bins with records,
// last level first (the fine levels' bins take the longest to finish);
// nchunks[0] = chunks of the first phase, [1] = bins to merge, [2] = chunks
// (the last min(kLateChunks, bins of at most a.chunk records) run in the
// second phase).
__global__ __launch_bounds__(kBinThreads) void scatter_distribute_kernel(
    const ScatterArgs a, const float* __restrict__ pos, const _Float16* __restrict__ denc,
    const uint32_t* __restrict__ prefix, const uint32_t* __restrict__ totals, float4* __restrict__ rec,
    uint32_t cap, uint4* __restrict__ chunks, uint4* __restrict__ merges, uint32_t* __restrict__ nchunks)
{
    extern __shared__ uint32_t sh[];
    uint32_t* cur = sh;                        // [bins]
    uint32_t* aux = sh + ((a.bins + 1) & ~1);  // [2 bins], 8-byte aligned (block 0: chunk table positions)
    __shared__ uint32_t wsum[kBinThreads / 64];
    __shared__ uint64_t wsum64[kBinThreads / 64];
    block_exclusive_scan(totals, cur, a.bins, wsum);
    if (blockIdx.x == 0) {
        const uint32_t C = a.chunk, S = a.split;
        // per bin, four counters packed in one word and scanned together (no
        // field's total carries into the next: chunks of split bins < 2^18,
        // bins <= kMaxBins < 2^14): the chunks of a split bin (bits 0-17: its
        // first chunk, also its first partial slice) and 1 for its merge entry
        // (bits 46-59), or 1 for a large bin of one chunk (bits 18-31), or 1
        // for a small one (bits 32-45)
        uint64_t* pk = reinterpret_cast<uint64_t*>(aux);
        for (int b = threadIdx.x; b < a.bins; b += kBinThreads) {
            const uint32_t t = totals[b];
            uint64_t v = 0;
            if (t > S) v = (uint64_t)((t + C - 1) / C) | (1ull << 46);
            else if (t > C) v = 1ull << 18;
            else if (t != 0u) v = 1ull << 32;
            pk[b] = v;
        }
        __syncthreads();
        const uint64_t tot = block_exclusive_scan(pk, pk, a.bins, wsum64);
        const uint32_t nsplit = (uint32_t)(tot & 0x3ffffu), nlarge = (uint32_t)(tot >> 18) & 0x3fffu,
                       nsmall = (uint32_t)(tot >> 32) & 0x3fffu, nmerge = (uint32_t)(tot >> 46) & 0x3fffu;
        for (int b = threadIdx.x; b < a.bins; b += kBinThreads) {
            const uint32_t t = totals[b];
            const uint64_t v = pk[b];
            if (t > S) {
                const uint32_t first = (uint32_t)(v & 0x3ffffu), k = (t + C - 1) / C;
                for (uint32_t j = 0; j < k; j++)
                    chunks[first + j] = make_uint4((uint32_t)b, cur[b] + j * C, cur[b] + min((j + 1) * C, t), first + j);
                merges[(uint32_t)(v >> 46) & 0x3fffu] = make_uint4((uint32_t)b, cur[b], first, k);
            } else if (t > C) {
                chunks[nsplit + ((uint32_t)(v >> 18) & 0x3fffu)] = make_uint4((uint32_t)b, cur[b], cur[b] + t, kSoleOwner);
            } else if (t != 0u) {
                const uint32_t back = nsmall - 1u - ((uint32_t)(v >> 32) & 0x3fffu);
                chunks[nsplit + nlarge + back] = make_uint4((uint32_t)b, cur[b], cur[b] + t, kSoleOwner);
            }
        }
        if (threadIdx.x == 0) {
            const uint32_t all = nsplit + nlarge + nsmall;
            nchunks[0] = all - min(nsmall, kLateChunks);
            nchunks[1] = nmerge;
            nchunks[2] = all;
        }
    }
    for (int b = threadIdx.x; b < a.bins; b += kBinThreads) cur[b] += prefix[(size_t)blockIdx.x * a.bins + b];
    __syncthreads();
    const int N = sample_count(a);
    const bool vec = (a.L & 3) == 0;
    for (int k = 0; k < kSamplesPerThread; k++) {
        const int n = blockIdx.x * kRound + k * kBinThreads + threadIdx.x;
        if (n >= N) break;
        if (a.tile_live && a.tile_live[n >> 4] == 0u) continue;  // no record: every product is +-0
        const float* pp = pos + (size_t)n * a.pos_stride;
        const float px = pp[0], py = pp[1], pz = pp[2];
        const uint32_t* grow = reinterpret_cast<const uint32_t*>(denc + (size_t)n * 2 * a.L);
        for (int l0 = 0; l0 < a.L; l0 += kLevelGroup) {
            uint32_t gv[kLevelGroup];
            load_levels(grow, l0, a.L, vec, gv);
#pragma unroll
            for (int j = 0; j < kLevelGroup; j++) {
                const int l = l0 + j;
                if (l >= a.L) break;
                const uint32_t gb = gv[j];
                if ((gb & 0x7fff7fffu) == 0u) continue;
                Pairs p;
                level_pairs(a, l, px, py, pz, p);
                const bool dense = l < a.dense_start;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t at = dense ? bin_take(cur, p.bin[q]) : atomicAdd(&cur[p.bin[q]], 1u);
                    if (at < cap)
                        rec[at] = make_float4(__uint_as_float(p.key[q]), __uint_as_float(gb), p.w0[q], p.w1[q]);
                }
            }
        }
    }
}

// rint(c * 2^e) as an int64 for |c * 2^e| < 2^51: adding 1.5 * 2^52 to the
// fp64 value leaves the rounded integer (two's complement) in the low
// mantissa bits.
__device__ __forceinline__ long long fixed_of(float c, int e)
{
    const double y = ldexp((double)c, e) + 6755399441055744.0;
    return __double_as_longlong(y) - 0x4338000000000000LL;
}

__device__ __forceinline__ void lds_add(unsigned long long* acc, int i, long long q)
{
    __hip_atomic_fetch_add(acc + i, (unsigned long long)q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A product that may be non-finite: fixed point if finite, else an fp32
// atomic on the table entry (and the slice is then flushed with atomics).
__device__ __forceinline__ void add_checked(unsigned long long* acc, float* gl, int i, float c, int e, int* flag)
{
    if (isfinite(c)) {
        lds_add(acc, i, fixed_of(c, e));
    } else {
        atomic_add_f32(gl + i, c);
        *flag = 1;
    }
}

// The fused update's form: a non-finite product marks its gradient
// non-finite (one bit per gradient of the slice) instead of adding.  Adam
// takes any non-finite gradient as 0 (finite_or_zero), and the sum the
// stored path forms from such a product is non-finite whatever else it adds,
// so the bit is all the update needs.
__device__ __forceinline__ void add_or_mark(unsigned long long* acc, uint32_t* nf, int i, float c, int e)
{
    if (isfinite(c)) lds_add(acc, i, fixed_of(c, e));
    else atomicOr(&nf[i >> 5], 1u << (i & 31));
}

__device__ __forceinline__ bool finite_bits(float x) { return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u; }

// 0 < |c| < 2^(24 - e): a nonzero product of fewer than 2^24 quanta; thr_bits
// is the fp32 pattern of 2^(24 - e) (the unsigned wrap excludes |c| == 0, and
// non-finite patterns lie above every threshold).
__device__ __forceinline__ bool small_product(float c, uint32_t thr_bits)
{
    return (__float_as_uint(c) & 0x7fffffffu) - 1u < thr_bits - 1u;
}

__device__ __forceinline__ void set_bit(uint32_t* w, int i) { atomicOr(&w[i >> 5], 1u << (i & 31)); }
__device__ __forceinline__ bool get_bit(const uint32_t* w, int i) { return (w[i >> 5] >> (i & 31)) & 1u; }

// Sums below this many quanta carry fewer significant bits than fp32 and are
// summed again at the entry's own scale.
constexpr long long kFewBits = 1LL << 24;

// The four products of a corner-pair record and the gradient words they add
// to: g_f * w of the x0 corner, then of the x1 corner (the reference's
// valX / valY = grads * weight, networkFusionBackwardHashtable.cu:864-865).
struct RecProducts {
    float c[4];
    int at[4];
};

__device__ __forceinline__ RecProducts rec_products(const float4& r)
{
    const uint32_t key = __float_as_uint(r.x);
    const int s0 = (int)(key & 0xffffu), s1 = (int)(key >> 16);
    const h2 gh = __builtin_bit_cast(h2, __float_as_uint(r.y));
    const float g0 = (float)gh.x, g1 = (float)gh.y, w0 = r.z, w1 = r.w;
    return RecProducts{{g0 * w0, g1 * w0, g0 * w1, g1 * w1}, {2 * s0, 2 * s0 + 1, 2 * s1, 2 * s1 + 1}};
}

// Every product of the record is finite: both fp16 gradients and both weights
// are (|g| <= 65504, weights in [0, 1]).
__device__ __forceinline__ bool rec_finite(const float4& r)
{
    const uint32_t gb = __float_as_uint(r.y);
    return ((gb & 0x7c00u) != 0x7c00u) & ((gb & 0x7c000000u) != 0x7c000000u) & finite_bits(r.z) & finite_bits(r.w);
}

constexpr int kAccThreads = 512;

// f(i) for every set bit i < nbits of an LDS bitmap, each word visited by one
// thread of the block.
template <class F>
__device__ __forceinline__ void for_each_bit(const uint32_t* w, int nbits, F&& f)
{
    const int nwords = (nbits + 31) >> 5;
    for (int wi = threadIdx.x; wi < nwords; wi += kAccThreads) {
        uint32_t m = w[wi];
        while (m) {
            const int b = __ffs(m) - 1;
            m &= m - 1;
            f(wi * 32 + b);
        }
    }
}


// f(products) over records [r0, r1) step kAccThreads, kRescan loads in flight
// per thread (a dependent load per record would wait out the memory latency
// each time).
constexpr int kRescan = 8;

template <class F>
__device__ __forceinline__ void for_each_record(const float4* __restrict__ rec, uint32_t r0, uint32_t r1, F&& f)
{
    for (uint32_t i0 = r0 + threadIdx.x; i0 < r1; i0 += kRescan * kAccThreads) {
        float4 r[kRescan];
#pragma unroll
        for (int k = 0; k < kRescan; k++) {
            const uint32_t i = i0 + k * kAccThreads;
            r[k] = i < r1 ? rec[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < kRescan; k++)
            if (i0 + k * kAccThreads < r1) f(rec_products(r[k]));
    }
}


// Parameters of the fused table update (ADAM): the table [L][T][2] (fp32
// master, fp16 copy) and its moments.
struct TableAdamArgs {
    float* w;
    _Float16* w16;
    float* m;
    float* v;
    AdamArgs a;
};

constexpr int kNfWords = 2 * kSlice / 32;  // non-finite bits of one slice

// Adam on entries [s0, s0 + kAdamBatch * kAccThreads) step kAccThreads of one
// slice (entry elem = base + s): gradient f of entry s is grad_of(2 s + f)
// (which also says whether its sum is nonzero), or non-finite where its bit
// is set; entries with neither a nonzero sum nor the bit keep every word (the
// stored path's zero gradients, which Adam skips).  Only touched features'
// words are stored.
constexpr int kAdamBatch = 8;  // entries per thread in flight in the update pass (4 measured slower)

template <class G>
__device__ __forceinline__ void table_adam_batch(const TableAdamArgs& t, size_t base, int s0, int slots,
                                                 G&& grad_of, const uint32_t* nfw)
{
    constexpr int kBatch = kAdamBatch;
    bool t0[kBatch], t1[kBatch];
    float g0[kBatch], g1[kBatch];
    float2 w[kBatch], m[kBatch], v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; k++) {
        const int s = s0 + k * kAccThreads;
        t0[k] = t1[k] = false;
        g0[k] = g1[k] = 0.f;
        if (s < slots) {
            float a0, a1;
            const bool z0 = grad_of(2 * s, a0), z1 = grad_of(2 * s + 1, a1);
            const uint32_t bits = nfw[(2 * s) >> 5] >> ((2 * s) & 31);  // 2 s even: both bits in one word
            const bool n0 = bits & 1u, n1 = (bits >> 1) & 1u;
            t0[k] = z0 | n0;
            t1[k] = z1 | n1;
            g0[k] = n0 ? __builtin_nanf("") : a0;
            g1[k] = n1 ? __builtin_nanf("") : a1;
        }
        if (t0[k] | t1[k]) {
            const size_t i = base + (size_t)s;
            w[k] = reinterpret_cast<const float2*>(t.w)[i];
            m[k] = reinterpret_cast<const float2*>(t.m)[i];
            v[k] = reinterpret_cast<const float2*>(t.v)[i];
        }
    }
    // every update before the first store: a store between two entries'
    // updates would make the next entry's wait for its loads also wait for
    // that store to complete (one counter covers loads and stores)
#pragma unroll
    for (int k = 0; k < kBatch; k++) {
        if (t0[k]) adam_update(g0[k], m[k].x, v[k].x, w[k].x, t.a);
        if (t1[k]) adam_update(g1[k], m[k].y, v[k].y, w[k].y, t.a);
    }
#pragma unroll
    for (int k = 0; k < kBatch; k++) {
        if (!(t0[k] | t1[k])) continue;
        const size_t i = base + (size_t)(s0 + k * kAccThreads);
        reinterpret_cast<float2*>(t.w)[i] = w[k];
        reinterpret_cast<float2*>(t.m)[i] = m[k];
        reinterpret_cast<float2*>(t.v)[i] = v[k];
        if (t0[k] & t1[k]) {
            reinterpret_cast<h2*>(t.w16)[i] = h2{to_h(w[k].x), to_h(w[k].y)};
        } else {
            t.w16[2 * i + (t0[k] ? 0 : 1)] = to_h(t0[k] ? w[k].x : w[k].y);
        }
    }
}

// The slice of one bin: its level, its first table entry and entry count,
// and the fixed-point scales of its sums.
struct SliceCtx {
    int l, slots, e, E, sfine;
    bool dense;
    uint32_t thr, tot;
    size_t ebase;  // first table entry of the slice ([L][T] numbering)
    // gradient words in use: [0, 2 slots), and for a dense slice (at most
    // kSlice / 2 entries) the finer sums of its small products at
    // [kFine, kFine + 2 slots)
    __device__ int used() const { return dense ? 4 * slots : 2 * slots; }
    __device__ int word(int k) const { return k < 2 * slots ? k : kFine + (k - 2 * slots); }
};

__device__ __forceinline__ SliceCtx slice_ctx(const ScatterArgs& a, int bin, const uint32_t* __restrict__ totals,
                                              const uint32_t* __restrict__ lvlmax)
{
    SliceCtx c;
    int l = 0;
    while (l + 1 < a.L && a.bin_base[l + 1] <= bin) l++;
    c.l = l;
    const int sl = bin - a.bin_base[l];
    c.dense = l < a.dense_start;
    int elem0;
    if (c.dense) {
        const int st = a.res[l] + 1, rps = a.rows_per_slice[l];
        const int row0 = sl * rps;
        elem0 = row0 * st;
        c.slots = min(rps, st * st - row0) * st;
    } else {
        elem0 = sl * kSlice;
        c.slots = min(kSlice, a.T);
    }
    c.ebase = (size_t)l * a.T + elem0;
    const uint32_t hb = lvlmax[l];
    const int ex = (int)((hb >> 10) & 31u);
    c.E = ex == 0 ? -15 : min(ex - 15, 15);
    c.tot = totals[bin];
    const int lg = c.tot <= 1u ? 0 : 32 - __clz(c.tot - 1u);
    c.e = min(49, 60 - lg) - c.E;
    c.thr = (uint32_t)(127 + 24 - c.e) << 23;  // 2^(24 - e), 24 - e in [-40, 9]
    // the finer scale e + sfine of small products: below 2^(24 + sfine) <= 2^50
    // units each, 2^lg of them below 2^62
    c.sfine = min(26, 38 - lg);
    return c;
}

// A slice's sums in LDS (two blocks per CU: at most 80 KiB each).
template <bool ADAM>
struct SliceLds {
    unsigned long long acc[2 * kSlice];
    uint32_t nf[ADAM ? kNfWords : 1];  // non-finite products (fused update)
    uint32_t sus[kNfWords];            // gradients that took a small product (summed again at a finer scale)
    uint32_t aux[kNfWords];            // gradients with products cancelling
    uint32_t tny[kNfWords];            // gradients still below 2^24 units
    uint8_t ex_off[2 * kSlice];        // the refined gradients' exponent above e
    int flag;                          // stored path: non-finite products went to the entries by fp32 atomics
};

// Sums of the records [r0, r1) of one bin into the cleared slice; ends with a
// block barrier.  gl: the slice's gradient words (stored path), for the fp32
// atomics of non-finite products.
template <bool ADAM>
__device__ __forceinline__ void sum_records(SliceLds<ADAM>& S, const SliceCtx& c, const float4* __restrict__ rec,
                                            uint32_t r0, uint32_t r1, float* gl)
{
    const uint32_t thr = c.thr;
    const int e = c.e, sfine = c.sfine;
    // the gradients a record adds a small product to (refined if their sums stay small)
    auto mark_small = [&](const float (&cc)[4], const int (&at)[4]) {
        if (small_product(cc[0], thr) | small_product(cc[1], thr) | small_product(cc[2], thr) |
            small_product(cc[3], thr)) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (small_product(cc[j], thr)) set_bit(S.sus, at[j]);
        }
    };
    // records per thread in flight before their LDS adds (hashed bins)
    constexpr int kBatch = 8;
    if (c.dense) {
        // Dense bins: the distribute pass leaves the records of consecutive
        // samples of a ray in consecutive slots, and those share corner
        // pairs.  Each lane takes kRun consecutive records (one 64-byte
        // piece of the wave's contiguous span) and adds the fixed-point
        // values of a run of equal keys in registers (exact: integer sums in
        // any order), with one LDS add per run it holds: products below 2^24
        // quanta at the finer scale into acc[kFine + i], the others at e.
        constexpr int kRun = 4;
        constexpr int kGroups = 2;  // runs per lane in flight (4 and 6 measured slower)
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        constexpr int kWaveSpan = 64 * kRun;
        for (uint32_t b0 = r0 + (uint32_t)wv * kWaveSpan; b0 < r1; b0 += (uint32_t)kGroups * kAccThreads * kRun) {
            float4 r[kGroups][kRun];
#pragma unroll
            for (int gi = 0; gi < kGroups; gi++)
#pragma unroll
                for (int k = 0; k < kRun; k++) {
                    const uint32_t i = b0 + (uint32_t)gi * kAccThreads * kRun + (uint32_t)(lane * kRun + k);
                    r[gi][k] = i < r1 ? rec[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
            for (int gi = 0; gi < kGroups; gi++) {
                uint32_t cur = 0xffffffffu;
                long long q[4] = {0, 0, 0, 0}, qf[4] = {0, 0, 0, 0};
                uint32_t sm = 0;  // gradients of the run that took a small product
                auto flush = [&]() {
                    if (cur == 0xffffffffu) return;
                    const int s0 = (int)(cur & 0xffffu), s1 = (int)(cur >> 16);
                    const int at[4] = {2 * s0, 2 * s0 + 1, 2 * s1, 2 * s1 + 1};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if (q[j]) lds_add(S.acc, at[j], q[j]);
                        if (qf[j]) lds_add(S.acc, kFine + at[j], qf[j]);
                        if (sm & (1u << j)) set_bit(S.sus, at[j]);
                    }
                };
#pragma unroll
                for (int k = 0; k < kRun; k++) {
                    const uint32_t i = b0 + (uint32_t)gi * kAccThreads * kRun + (uint32_t)(lane * kRun + k);
                    if (i >= r1) break;
                    const uint32_t key = __float_as_uint(r[gi][k].x);
                    if (key != cur) {
                        flush();
                        cur = key;
                        q[0] = q[1] = q[2] = q[3] = 0;
                        qf[0] = qf[1] = qf[2] = qf[3] = 0;
                        sm = 0;
                    }
                    const RecProducts rp = rec_products(r[gi][k]);
                    const bool fin = rec_finite(r[gi][k]);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const bool small = small_product(rp.c[j], thr);
                        sm |= small ? 1u << j : 0u;
                        if (small) {
                            qf[j] += fixed_of(rp.c[j], e + sfine);
                        } else if (fin || isfinite(rp.c[j])) {
                            q[j] += fixed_of(rp.c[j], e);
                        } else if constexpr (ADAM) {
                            set_bit(S.nf, rp.at[j]);
                        } else {
                            atomic_add_f32(gl + rp.at[j], rp.c[j]);
                            S.flag = 1;
                        }
                    }
                }
                flush();
            }
        }
    } else {
        for (uint32_t i0 = r0 + threadIdx.x; i0 < r1; i0 += kBatch * kAccThreads) {
            float4 r[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; k++) {
                const uint32_t i = i0 + k * kAccThreads;
                r[k] = i < r1 ? rec[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < kBatch; k++) {
                if (i0 + k * kAccThreads >= r1) break;
                const RecProducts rp = rec_products(r[k]);
                if (rec_finite(r[k])) {
#pragma unroll
                    for (int j = 0; j < 4; j++) lds_add(S.acc, rp.at[j], fixed_of(rp.c[j], e));
                } else if constexpr (ADAM) {
#pragma unroll
                    for (int j = 0; j < 4; j++) add_or_mark(S.acc, S.nf, rp.at[j], rp.c[j], e);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++) add_checked(S.acc, gl, rp.at[j], rp.c[j], e, &S.flag);
                }
                mark_small(rp.c, rp.at);
            }
        }
    }
    __syncthreads();
}

// The sole owner of a bin's sums (every record [r0, r1) of the bin summed
// into S): the refinement passes (see the file comment) over the records,
// then the table update (ADAM) or the gradient store.
template <bool ADAM>
__device__ __forceinline__ void finish_slice(SliceLds<ADAM>& S, const SliceCtx& c, const float4* __restrict__ rec,
                                             uint32_t r0, uint32_t r1, float* gl, int grads_zero,
                                             const TableAdamArgs& ta)
{
    const int slots = c.slots, e = c.e, E = c.E, sfine = c.sfine;
    const uint32_t thr = c.thr;
    const bool dense = c.dense;
    bool refine = false;  // hashed slice: some gradients summed again (pass 1)
    bool tiny = false;    // gradients below 2^24 units of their finer scale
    if (dense) {
        // the two scales together, in units of the finer one
        for_each_bit(S.sus, 2 * slots, [&](int i) {
            const double v = ldexp((double)(long long)S.acc[i], sfine) + (double)(long long)S.acc[kFine + i];
            if (fabs(v) < 0x1p24) {
                set_bit(S.tny, i);
                tiny = true;
            }
        });
    } else {
        // keep the marks of gradients whose sums stayed below 2^24 quanta
        // (each mark word owned by one thread)
        bool few = false;
        for (int wi = threadIdx.x; wi < (2 * slots + 31) >> 5; wi += kAccThreads) {
            uint32_t m = S.sus[wi], keep = m;
            while (m) {
                const int b = __ffs(m) - 1;
                m &= m - 1;
                const long long q = (long long)S.acc[wi * 32 + b];
                if (q > -kFewBits && q < kFewBits) few = true;
                else keep &= ~(1u << b);
            }
            S.sus[wi] = keep;
        }
        refine = __syncthreads_or(few);
    }
    if (refine) {
        // pass 1: the marked gradients' small products at scale e + sfine; a
        // product of 2^24 quanta or more marks its gradient for pass 2
        for_each_bit(S.sus, 2 * slots, [&](int i) {
            S.acc[i] = 0ull;
            S.ex_off[i] = (uint8_t)sfine;
        });
        __syncthreads();
        bool big = false;
        for_each_record(rec, r0, r1, [&](const RecProducts& rp) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (finite_bits(rp.c[j]) && rp.c[j] != 0.f && get_bit(S.sus, rp.at[j])) {
                    if (small_product(rp.c[j], thr)) {
                        lds_add(S.acc, rp.at[j], fixed_of(rp.c[j], e + sfine));
                    } else {
                        set_bit(S.aux, rp.at[j]);
                        big = true;
                    }
                }
        });
        if (__syncthreads_or(big)) {
            // pass 2 (products cancelling): those gradients at scale e again
            for (int wi = threadIdx.x; wi < (2 * slots + 31) >> 5; wi += kAccThreads) S.sus[wi] &= ~S.aux[wi];
            for_each_bit(S.aux, 2 * slots, [&](int i) { S.acc[i] = 0ull; });
            __syncthreads();
            for_each_record(rec, r0, r1, [&](const RecProducts& rp) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (finite_bits(rp.c[j]) && get_bit(S.aux, rp.at[j])) lds_add(S.acc, rp.at[j], fixed_of(rp.c[j], e));
            });
            __syncthreads();
        }
        // gradients whose finer sums stay below 2^24 units (products of a few
        // quanta at most)
        for_each_bit(S.sus, 2 * slots, [&](int i) {
            const long long q = (long long)S.acc[i];
            if (q > -kFewBits && q < kFewBits) {
                set_bit(S.tny, i);
                tiny = true;
            }
        });
    }
    const bool any_tiny = __syncthreads_or(tiny);
    if (any_tiny) {
        // passes 3 and 4: the largest |product| of each (fp32 bit patterns of
        // non-negative values order as the values), then the sums at the
        // exponent it sets: |product| < 2^(Es + 1) gives min(49, 60 - lg) - Es,
        // Es <= E, an offset over e of E - Es in [0, 164]; the sum lands in
        // acc[i] (a dense slice's finer sum cleared)
        for_each_bit(S.tny, 2 * slots, [&](int i) {
            S.acc[i] = 0ull;
            if (dense) S.acc[kFine + i] = 0ull;
        });
        __syncthreads();
        for_each_record(rec, r0, r1, [&](const RecProducts& rp) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (finite_bits(rp.c[j]) && rp.c[j] != 0.f && get_bit(S.tny, rp.at[j]))
                    __hip_atomic_fetch_max(S.acc + rp.at[j], (unsigned long long)(__float_as_uint(rp.c[j]) & 0x7fffffffu),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        });
        __syncthreads();
        for_each_bit(S.tny, 2 * slots, [&](int i) {
            const uint32_t mb = (uint32_t)S.acc[i];
            const int Es = mb >= 0x800000u ? (int)(mb >> 23) - 127 : (mb ? 31 - __clz(mb) - 149 : E);
            S.ex_off[i] = (uint8_t)min(255, max(0, E - Es));
            S.acc[i] = 0ull;
        });
        __syncthreads();
        for_each_record(rec, r0, r1, [&](const RecProducts& rp) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (finite_bits(rp.c[j]) && rp.c[j] != 0.f && get_bit(S.tny, rp.at[j]))
                    lds_add(S.acc, rp.at[j], fixed_of(rp.c[j], e + S.ex_off[rp.at[j]]));
        });
        __syncthreads();
    }
    // gradient word i: its fp32 value (the exact fixed-point sum rounded once;
    // a dense slice's two scales combined in fp64 first) and whether its sum
    // is nonzero
    auto grad_of = [&](int i, float& g) -> bool {
        const long long q = (long long)S.acc[i];
        if ((refine || any_tiny) && (get_bit(S.tny, i) || (refine && get_bit(S.sus, i)))) {
            g = ldexpf((float)q, -(e + (int)S.ex_off[i]));
            return q != 0;
        }
        if (dense) {
            const long long f = (long long)S.acc[kFine + i];
            if (f == 0) g = ldexpf((float)q, -e);
            else if (q == 0) g = ldexpf((float)f, -(e + sfine));
            else g = (float)(ldexp((double)q, -e) + ldexp((double)f, -(e + sfine)));
            return (q | f) != 0;
        }
        g = ldexpf((float)q, -e);
        return q != 0;
    };
    if constexpr (ADAM) {
        // update every entry the sums reached
        for (int s0 = threadIdx.x; s0 < slots; s0 += kAdamBatch * kAccThreads)
            table_adam_batch(ta, c.ebase, s0, slots, grad_of, S.nf);
        return;
    }
    {
        // non-finite products went to the entries by fp32 atomics: then the
        // sums follow by atomics too
        const bool atomic = S.flag != 0;
        float2* g2 = reinterpret_cast<float2*>(gl);
        if (atomic || grads_zero) {
            for (int s = threadIdx.x; s < slots; s += kAccThreads) {
                float v0, v1;
                const bool z0 = grad_of(2 * s, v0), z1 = grad_of(2 * s + 1, v1);
                if (atomic) {
                    if (z0) atomic_add_f32(gl + 2 * s, v0);
                    if (z1) atomic_add_f32(gl + 2 * s + 1, v1);
                } else {
                    g2[s] = make_float2(v0, v1);
                }
            }
        } else {
            // read-modify-write, kBatch entries per thread in flight
            constexpr int kBatch = 8;
            for (int s0 = threadIdx.x; s0 < slots; s0 += kBatch * kAccThreads) {
                float2 o[kBatch];
#pragma unroll
                for (int k = 0; k < kBatch; k++) {
                    const int s = s0 + k * kAccThreads;
                    o[k] = s < slots ? g2[s] : make_float2(0.f, 0.f);
                }
#pragma unroll
                for (int k = 0; k < kBatch; k++) {
                    const int s = s0 + k * kAccThreads;
                    if (s >= slots) break;
                    float v0, v1;
                    const bool z0 = grad_of(2 * s, v0), z1 = grad_of(2 * s + 1, v1);
                    if (z0 | z1) g2[s] = make_float2(o[k].x + v0, o[k].y + v1);
                }
            }
        }
    }
}

// Parameters shared by the two accumulate launches.
struct AccArgs {
    const float4* rec;
    const uint4* chunks;
    const uint4* merges;
    const uint32_t* nchunks;  // [3]: first phase's chunks, bins to merge, all chunks
    const uint32_t* totals;
    const uint32_t* lvlmax;
    float* grads;             // stored path
    unsigned long long* part;
    uint32_t* part_nf;
    uint32_t* part_sus;
    uint32_t* part_flag;
    int grads_zero;
};

// One chunk: its sums in LDS (int64 fixed point, ds_add_u64).  A bin of one
// chunk is finished here (refinement, then the table update or the gradient
// store); a chunk of a bin of several stores its sums and marks as its
// partial slice for the bin's merge.
template <bool ADAM>
__device__ __forceinline__ void do_chunk(SliceLds<ADAM>& S, const ScatterArgs& a, const AccArgs& g, uint32_t ci,
                                         const TableAdamArgs& ta)
{
    const uint4 ch = g.chunks[ci];
    const SliceCtx c = slice_ctx(a, (int)ch.x, g.totals, g.lvlmax);
    float* gl = ADAM ? nullptr : g.grads + c.ebase * 2;
    const int nu = c.used();
    for (int k = threadIdx.x; k < nu; k += kAccThreads) S.acc[c.word(k)] = 0ull;
    for (int i = threadIdx.x; i < kNfWords; i += kAccThreads) {
        S.sus[i] = S.aux[i] = S.tny[i] = 0u;
        if constexpr (ADAM) S.nf[i] = 0u;
    }
    if (threadIdx.x == 0) S.flag = 0;
    __syncthreads();
    sum_records(S, c, g.rec, ch.y, ch.z, gl);
    if (ch.w != kSoleOwner) {
        unsigned long long* mine = g.part + (size_t)ch.w * (2 * kSlice);
        for (int k = threadIdx.x; k < nu; k += kAccThreads) mine[k] = S.acc[c.word(k)];
        for (int i = threadIdx.x; i < kNfWords; i += kAccThreads) {
            g.part_sus[(size_t)ch.w * kNfWords + i] = S.sus[i];
            if constexpr (ADAM) g.part_nf[(size_t)ch.w * kNfWords + i] = S.nf[i];
        }
        if (!ADAM && threadIdx.x == 0) g.part_flag[ch.w] = (uint32_t)S.flag;
        return;
    }
    finish_slice(S, c, g.rec, ch.y, ch.z, gl, g.grads_zero, ta);
}

// One bin of several chunks (its partial slices are complete): the exact sum
// of the partial slices, then the sole owner's finish over all the bin's
// records.  Each thread adds the words it owns, two slices' loads in flight.
template <bool ADAM>
__device__ __forceinline__ void do_merge(SliceLds<ADAM>& S, const ScatterArgs& a, const AccArgs& g, uint32_t mi,
                                         const TableAdamArgs& ta)
{
    const uint4 mg = g.merges[mi];  // bin, first record, first partial slice, chunks
    const SliceCtx c = slice_ctx(a, (int)mg.x, g.totals, g.lvlmax);
    float* gl = ADAM ? nullptr : g.grads + c.ebase * 2;
    const uint32_t p0 = mg.z, kb = mg.w;
    const int nu = c.used();
    constexpr int kWords = 2 * kSlice / kAccThreads;  // words per thread
    unsigned long long sum[kWords];
#pragma unroll
    for (int k = 0; k < kWords; k++) sum[k] = 0ull;
    for (uint32_t j = 0; j < kb; j += 2) {
        const unsigned long long* o0 = g.part + (size_t)(p0 + j) * (2 * kSlice);
        const unsigned long long* o1 = g.part + (size_t)(p0 + min(j + 1, kb - 1)) * (2 * kSlice);
        const bool two = j + 1 < kb;
        unsigned long long t0[kWords], t1[kWords];
#pragma unroll
        for (int k = 0; k < kWords; k++) {
            const int w = threadIdx.x + k * kAccThreads;
            t0[k] = w < nu ? o0[w] : 0ull;
            t1[k] = (two && w < nu) ? o1[w] : 0ull;
        }
#pragma unroll
        for (int k = 0; k < kWords; k++) sum[k] += t0[k] + t1[k];
    }
#pragma unroll
    for (int k = 0; k < kWords; k++) {
        const int w = threadIdx.x + k * kAccThreads;
        if (w < nu) S.acc[c.word(w)] = sum[k];
    }
    for (int i = threadIdx.x; i < kNfWords; i += kAccThreads) {
        uint32_t su = 0u, n = 0u;
        for (uint32_t j = 0; j < kb; j++) {
            su |= g.part_sus[(size_t)(p0 + j) * kNfWords + i];
            if constexpr (ADAM) n |= g.part_nf[(size_t)(p0 + j) * kNfWords + i];
        }
        S.sus[i] = su;
        S.aux[i] = S.tny[i] = 0u;
        if constexpr (ADAM) S.nf[i] = n;
    }
    if (threadIdx.x == 0) {
        uint32_t f = 0u;
        if (!ADAM)
            for (uint32_t j = 0; j < kb; j++) f |= g.part_flag[p0 + j];
        S.flag = (int)f;
    }
    __syncthreads();
    finish_slice(S, c, g.rec, mg.y, mg.y + c.tot, gl, g.grads_zero, ta);
}

// The accumulate pass in two launches.  Phase 1: chunks [0, nchunks[0]) --
// every chunk of the bins of several chunks (first: the heaviest work), then
// bins of one chunk.  Phase 2 (after phase 1: the kernel boundary orders the
// partial slices, no device-scope fence or counter is needed): the merges of
// the bins of several chunks, beside the last bins of one chunk (chunks
// [nchunks[0], nchunks[2])), so that the merges run on a busy GPU.  Two
// blocks per CU (the LDS holds two slices): at most 128 VGPRs.
template <bool ADAM, bool PHASE2>
__global__ __launch_bounds__(kAccThreads) __attribute__((amdgpu_waves_per_eu(4))) void scatter_accumulate_kernel(
    const ScatterArgs a, const AccArgs g, const TableAdamArgs ta)
{
    __shared__ SliceLds<ADAM> S;
    if constexpr (!PHASE2) {
        if (blockIdx.x < g.nchunks[0]) do_chunk(S, a, g, blockIdx.x, ta);
    } else {
        const uint32_t nm = g.nchunks[1];
        if (blockIdx.x < nm) {
            do_merge(S, a, g, blockIdx.x, ta);
        } else {
            const uint32_t ci = g.nchunks[0] + (blockIdx.x - nm);
            if (ci < g.nchunks[2]) do_chunk(S, a, g, ci, ta);
        }
    }
}

}  // namespace

struct ScatterPlan {
    int maxN = 0;
    int max_chunks = 0;
    int max_multi = 0;
    GridMeta meta{};
    ScatterArgs args{};
    void* mem = nullptr;
    float4* rec = nullptr;
    uint32_t* counts = nullptr;
    uint32_t* totals = nullptr;
    uint32_t* lvlmax = nullptr;
    uint32_t* lvlmax_final = nullptr;
    uint4* chunks = nullptr;
    uint4* merges = nullptr;             // bins of several chunks
    uint32_t* nchunks = nullptr;         // [3]: first phase's chunks, bins to merge, chunks
    unsigned long long* part = nullptr;  // partial slices of the chunks of multi-chunk bins
    uint32_t* part_nf = nullptr;         // non-finite bits of the partial slices (fused table update)
    uint32_t* part_sus = nullptr;        // small-product marks of the partial slices
    uint32_t* part_flag = nullptr;       // per partial slice: non-finite products went by atomics (stored path)
};

namespace {

bool same_meta(const GridMeta& a, const GridMeta& b)
{
    if (a.numLevels != b.numLevels || a.tableSize != b.tableSize || a.denseLevelStart != b.denseLevelStart)
        return false;
    for (int l = 0; l < a.numLevels; l++)
        if (a.scale[l] != b.scale[l] || a.res[l] != b.res[l]) return false;
    return true;
}

// Bins of every level; false if the configuration is outside the binned
// path's limits.
bool layout(const GridMeta& m, ScatterArgs& a)
{
    a = ScatterArgs{};
    a.L = m.numLevels;
    a.T = m.tableSize;
    a.dense_start = m.denseLevelStart;
    a.mask = (uint32_t)m.tableSize - 1u;
    int bins = 0;
    for (int l = 0; l < m.numLevels; l++) {
        a.scale[l] = m.scale[l];
        a.res[l] = m.res[l];
        a.bin_base[l] = bins;
        if (m.res[l] < 1) return false;
        if (l < m.denseLevelStart) {
            const long long st = (long long)m.res[l] + 1;
            if (st > kSlice / 2) return false;
            // about kDenseBins bins per level (at most kSlice / 2 entries each,
            // the other half of the LDS slice holding their finer sums): a
            // coarse level's few entries take a contribution from nearly
            // every sample, so its records are spread over as many blocks
            // as a fine level's
            const long long rows = st * st;
            const int rps =
                (int)std::max(1LL, std::min((long long)(kSlice / 2 / st), (rows + kDenseBins - 1) / kDenseBins));
            a.rows_per_slice[l] = rps;
            bins += (int)((st * st + rps - 1) / rps);
        } else {
            // x0 and x0 + 1 <= N_l must differ only below bit 12
            if (m.res[l] >= kSlice) return false;
            bins += std::max(1, m.tableSize / kSlice);
        }
        if (bins > kMaxBins) return false;
    }
    a.bin_base[m.numLevels] = bins;
    a.bins = bins;
    return true;
}

size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

namespace {

// Byte offsets of a plan's buffers (every call rewrites what it reads: no
// buffer needs to start zero).
struct PlanLayout {
    size_t o_prt, o_pnf, o_psu, o_pfl, o_rec, o_cnt, o_tot, o_lmx, o_lmf, o_chk, o_mrg, o_nch, bytes;
};

// Partial slices: every chunk of a split bin has one; a bin of t > split
// records has ceil(t / C) < t / C + 1 chunks (C = chunk) and there are fewer
// than recs / split <= recs / C such bins, so 2 recs / C + 1 slices suffice.  with_nf: room
// for the fused table update's non-finite bits of every partial slice (plans
// of the training step; the allocation-free plan has none).
bool plan_shape(const GridMeta& m, int maxN, ScatterPlan& p, PlanLayout& lay, uint32_t chunk, uint32_t split,
                int max_multi_cap = 0, bool with_nf = false)
{
    ScatterArgs a;
    if (maxN < 1 || !layout(m, a)) return false;
    const unsigned long long recs = 4ull * (unsigned long long)m.numLevels * (unsigned long long)maxN;
    // record indices fit 32 bits, chunks of split bins (< recs / chunk + bins)
    // the chunk table's 18-bit counters
    if (recs >= (1ull << 30) || chunk < 8192u || split < chunk) return false;
    a.rounds = (maxN + kRound - 1) / kRound;
    a.chunk = chunk;
    a.split = split;
    p.maxN = maxN;
    p.meta = m;
    p.args = a;
    p.max_chunks = (int)(recs / chunk) + a.bins + 1;
    p.max_multi = (int)(2 * (recs / chunk) + 1);
    const int multi = std::max(p.max_multi, max_multi_cap);
    const size_t max_merges = (size_t)std::min<unsigned long long>(recs / chunk + 1, (unsigned long long)a.bins);
    size_t off = 0;
    lay.o_prt = off; off = align_up(off + (size_t)multi * 2 * kSlice * 8);
    lay.o_pnf = off; off = align_up(off + (with_nf ? (size_t)multi * kNfWords * 4 : 0));
    lay.o_psu = off; off = align_up(off + (size_t)multi * kNfWords * 4);
    lay.o_pfl = off; off = align_up(off + (size_t)multi * 4);
    lay.o_rec = off; off = align_up(off + recs * sizeof(float4));
    lay.o_cnt = off; off = align_up(off + (size_t)a.rounds * a.bins * 4);
    lay.o_tot = off; off = align_up(off + (size_t)a.bins * 4);
    lay.o_lmx = off; off = align_up(off + (size_t)a.rounds * a.L * 4);
    lay.o_lmf = off; off = align_up(off + (size_t)a.L * 4);
    lay.o_chk = off; off = align_up(off + (size_t)p.max_chunks * sizeof(uint4));
    lay.o_mrg = off; off = align_up(off + max_merges * sizeof(uint4));
    lay.o_nch = off; off = align_up(off + 3 * 4);
    lay.bytes = off;
    return true;
}

void plan_bind(ScatterPlan& p, char* base, const PlanLayout& lay)
{
    p.mem = base;
    p.rec = reinterpret_cast<float4*>(base + lay.o_rec);
    p.counts = reinterpret_cast<uint32_t*>(base + lay.o_cnt);
    p.totals = reinterpret_cast<uint32_t*>(base + lay.o_tot);
    p.lvlmax = reinterpret_cast<uint32_t*>(base + lay.o_lmx);
    p.lvlmax_final = reinterpret_cast<uint32_t*>(base + lay.o_lmf);
    p.chunks = reinterpret_cast<uint4*>(base + lay.o_chk);
    p.merges = reinterpret_cast<uint4*>(base + lay.o_mrg);
    p.nchunks = reinterpret_cast<uint32_t*>(base + lay.o_nch);
    p.part = reinterpret_cast<unsigned long long*>(base + lay.o_prt);
    p.part_nf = lay.o_pnf < lay.o_psu ? reinterpret_cast<uint32_t*>(base + lay.o_pnf) : nullptr;
    p.part_sus = reinterpret_cast<uint32_t*>(base + lay.o_psu);
    p.part_flag = reinterpret_cast<uint32_t*>(base + lay.o_pfl);
}

}  // namespace

ScatterPlan* scatter_plan_create(const GridMeta& m, int maxN)
{
    auto* p = new ScatterPlan();
    PlanLayout lay;
    if (!plan_shape(m, maxN, *p, lay, kChunk, kSplit, 0, /*with_nf=*/true)) {
        delete p;
        return nullptr;
    }
    void* mem = nullptr;
    hipError_t e = hipMalloc(&mem, lay.bytes);
    if (e != hipSuccess) {
        delete p;
        GRAFT_HIP_CHECK(e);
    }
    plan_bind(*p, static_cast<char*>(mem), lay);
    return p;
}

void scatter_plan_destroy(ScatterPlan* p)
{
    if (!p) return;
    if (p->mem) (void)hipFree(p->mem);
    delete p;
}

int scatter_plan_max_samples(const ScatterPlan* p) { return p ? p->maxN : 0; }

namespace {

// count, prefix, distribute, then (after wait_before, when given) accumulate:
// into grads, or (ta) as the fused table update.
void scatter_launch(ScatterPlan* p, const GridMeta& m, const __half* denc, const float* pos, int pos_stride,
                    float* grads, int N, hipStream_t stream, const uint32_t* d_n, bool grads_zero,
                    const TableAdamArgs* ta, hipEvent_t wait_before, const uint32_t* tile_live = nullptr)
{
    if (N <= 0) return;
    if (!p) throw std::runtime_error("hash scatter: no scatter plan");
    if (pos_stride < 3) throw std::runtime_error("hash scatter: position stride must be >= 3");
    if (N > p->maxN) throw std::runtime_error("hash scatter: batch exceeds the plan's sample capacity");
    if (!same_meta(p->meta, m)) throw std::runtime_error("hash scatter: plan built for another grid");
    if (ta && !p->part_nf) throw std::runtime_error("hash scatter: plan without the fused update's scratch");
    ScatterArgs a = p->args;
    a.d_n = d_n;
    a.tile_live = tile_live;
    a.N = N;
    a.pos_stride = pos_stride;
    a.rounds = (N + kRound - 1) / kRound;
    const auto* dh = reinterpret_cast<const _Float16*>(denc);
    const size_t lds_count = (size_t)(a.bins + a.L) * 4;
    const size_t lds_dist = (size_t)(((a.bins + 1) & ~1) + 2 * a.bins) * 4;
    hipLaunchKernelGGL(scatter_count_kernel, dim3(a.rounds), dim3(kBinThreads), lds_count, stream, a, pos, dh,
                       p->counts, p->lvlmax);
    GRAFT_LAUNCH_CHECK();
    const int prefix_blocks = std::max((a.bins + kPrefixBins - 1) / kPrefixBins, a.L);
    hipLaunchKernelGGL(scatter_prefix_kernel, dim3(prefix_blocks), dim3(kPrefixThreads), 0, stream, a, p->counts, p->totals,
                       p->lvlmax, p->lvlmax_final);
    GRAFT_LAUNCH_CHECK();
    const uint32_t cap = (uint32_t)(4ull * (unsigned long long)a.L * (unsigned long long)p->maxN);
    hipLaunchKernelGGL(scatter_distribute_kernel, dim3(a.rounds), dim3(kBinThreads), lds_dist, stream, a, pos, dh,
                       p->counts, p->totals, p->rec, cap, p->chunks, p->merges, p->nchunks);
    GRAFT_LAUNCH_CHECK();
    if (wait_before) GRAFT_HIP_CHECK(hipStreamWaitEvent(stream, wait_before, 0));
    const unsigned long long recs = 4ull * (unsigned long long)a.L * (unsigned long long)N;
    const int grid = (int)std::min<unsigned long long>(recs / a.chunk + a.bins + 1, (unsigned long long)p->max_chunks);
    const int mgrid = (int)std::min<unsigned long long>(recs / a.chunk + 1, (unsigned long long)a.bins);
    AccArgs g{p->rec, p->chunks, p->merges, p->nchunks, p->totals, p->lvlmax_final, grads, p->part, p->part_nf,
              p->part_sus, p->part_flag, grads_zero ? 1 : 0};
    const int grid2 = mgrid + (int)std::min<unsigned long long>(kLateChunks, (unsigned long long)a.bins);
    if (ta) {
        hipLaunchKernelGGL((scatter_accumulate_kernel<true, false>), dim3(grid), dim3(kAccThreads), 0, stream, a, g,
                           *ta);
        GRAFT_LAUNCH_CHECK();
        hipLaunchKernelGGL((scatter_accumulate_kernel<true, true>), dim3(grid2), dim3(kAccThreads), 0, stream, a, g,
                           *ta);
    } else {
        hipLaunchKernelGGL((scatter_accumulate_kernel<false, false>), dim3(grid), dim3(kAccThreads), 0, stream, a, g,
                           TableAdamArgs{});
        GRAFT_LAUNCH_CHECK();
        hipLaunchKernelGGL((scatter_accumulate_kernel<false, true>), dim3(grid2), dim3(kAccThreads), 0, stream, a, g,
                           TableAdamArgs{});
    }
    GRAFT_LAUNCH_CHECK();
}

}  // namespace

void hash_scatter_binned(ScatterPlan* p, const GridMeta& m, const __half* denc, const float* pos, int pos_stride,
                         float* grads, int N, hipStream_t stream, const uint32_t* d_n, bool grads_zero)
{
    scatter_launch(p, m, denc, pos, pos_stride, grads, N, stream, d_n, grads_zero, nullptr, nullptr);
}

void hash_scatter_adam(ScatterPlan* p, const GridMeta& m, const __half* denc, const float* pos, int pos_stride, int N,
                       const TableAdam& t, hipStream_t stream, const uint32_t* d_n, hipEvent_t wait_before_update,
                       const uint32_t* tile_live)
{
    if (!t.w || !t.w16 || !t.m || !t.v) throw std::runtime_error("hash scatter: null table or moment array");
    const TableAdamArgs ta{t.w, reinterpret_cast<_Float16*>(t.w16), t.m, t.v, t.a};
    scatter_launch(p, m, denc, pos, pos_stride, nullptr, N, stream, d_n, false, &ta, wait_before_update, tile_live);
}

namespace {

// Scratch of the stateless launchers, one plan per (device, stream): two
// streams never share one.  A plan is replaced (after its stream drains) when
// a call needs more samples or another grid.  Plans live until the process
// ends.
std::mutex g_plans_mu;
std::map<std::pair<int, hipStream_t>, ScatterPlan*> g_plans;

ScatterPlan* plan_for_stream(const GridMeta& m, int N, hipStream_t stream)
{
    int dev = 0;
    GRAFT_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_plans_mu);
    ScatterPlan*& p = g_plans[{dev, stream}];
    if (p && (p->maxN < N || !same_meta(p->meta, m))) {
        GRAFT_HIP_CHECK(hipStreamSynchronize(stream));
        scatter_plan_destroy(p);
        p = nullptr;
    }
    if (!p) p = scatter_plan_create(m, N);
    return p;
}

}  // namespace

void hash_scatter(const GridMeta& m, const __half* denc, const float* pos, int pos_stride, float* grads, int N,
                  hipStream_t stream, const uint32_t* d_n)
{
    if (N <= 0) return;
    ScatterPlan* p = plan_for_stream(m, N, stream);
    if (p)
        hash_scatter_binned(p, m, denc, pos, pos_stride, grads, N, stream, d_n, /*grads_zero=*/false);
    else
        hash_scatter_atomic(m, denc, pos, pos_stride, grads, N, stream, d_n);
}

// ---------------------------------------------------------------------------
// Allocation-free variant.  The scratch is one file-scope device array per
// GPU (kNoAllocBytes; each GPU the library runs on keeps it until the process
// ends).  Every call rewrites what it reads of it (nothing needs to start
// zero).  Batches above one sub-batch run as consecutive sub-batches on the
// caller's stream.  All calls on one GPU share the array:
// calls that overlap on one GPU (two streams, or two threads) race.
// ---------------------------------------------------------------------------

namespace {

constexpr size_t kNoAllocBytes = (size_t)48 << 20;
constexpr unsigned long long kNoAllocRecords = 1ull << 21;  // corner-pair records per sub-batch
constexpr size_t kNoAllocCountWords = (size_t)1 << 20;       // rounds x bins per sub-batch
constexpr int kNoAllocMulti = (int)(2 * (kNoAllocRecords / kChunkNoAlloc)) + 1;  // partial slices per sub-batch
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

char* g_noalloc_base[kMaxDevices];
std::mutex g_noalloc_mu;

// The array's device address on the current GPU (looked up on the first call
// on each GPU).
char* noalloc_base()
{
    int dev = 0;
    GRAFT_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("hash scatter (no-alloc): device index out of range");
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_base[dev]) {
        void* ptr = nullptr;
        GRAFT_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) throw std::runtime_error("hash scatter (no-alloc): no device address for the scratch array");
        g_noalloc_base[dev] = static_cast<char*>(ptr);
    }
    return g_noalloc_base[dev];
}

}  // namespace

size_t scatter_noalloc_bytes() { return kNoAllocBytes; }

void hash_scatter_noalloc(const GridMeta& m, const __half* denc, const float* pos, int pos_stride, float* grads,
                          int N, hipStream_t stream)
{
    if (N <= 0) return;
    if (pos_stride < 3) throw std::runtime_error("hash scatter: position stride must be >= 3");
    ScatterArgs a;
    if (!layout(m, a))
        throw std::runtime_error("hash scatter (no-alloc): grid beyond the fixed scratch (more than 8192 bins of "
                                 "4096 entries, or a hashed level's resolution above 4095)");
    const long long by_rec = (long long)(kNoAllocRecords / (4ull * (unsigned long long)m.numLevels));
    const long long by_cnt = (long long)(kNoAllocCountWords / (size_t)a.bins) * kRound;
    const int sub = (int)(std::min(by_rec, by_cnt) / kRound * kRound);
    if (sub < kRound) throw std::runtime_error("hash scatter (no-alloc): grid beyond the fixed scratch");
    ScatterPlan plan;
    PlanLayout lay;
    if (!plan_shape(m, sub, plan, lay, kChunkNoAlloc, kChunkNoAlloc, kNoAllocMulti) || plan.max_multi > kNoAllocMulti ||
        lay.bytes > kNoAllocBytes)
        throw std::runtime_error("hash scatter (no-alloc): grid beyond the fixed scratch");
    plan_bind(plan, noalloc_base(), lay);
    const int D = 2 * m.numLevels;
    for (int off = 0; off < N; off += sub) {
        const int n = std::min(sub, N - off);
        hash_scatter_binned(&plan, m, denc + (size_t)off * D, pos + (size_t)off * pos_stride, pos_stride, grads, n,
                            stream, nullptr, /*grads_zero=*/false);
    }
}

}  // namespace graft
