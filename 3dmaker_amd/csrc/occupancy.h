// Internal interface of occupancy.hip (occupancy-grid refresh).
#pragma once

#include "common.h"

namespace graft {

enum SampleMode {
    kSampleEveryCell = 0,  // sample idx -> cell cell_offset + idx (N == total_cells)
    kSampleRandomCell = 1, // uniform cell in [cell_offset, cell_offset + total_cells)
    kSampleFromList = 2,   // uniform entry of list[0 .. *d_list_count)
};

// samples [N] float4: contracted position, w = cell index (int bits).
void occ_sample(float4* out, int N, int mode, int total_cells, int cell_offset, const int* list,
                const int* d_list_count, uint64_t seed, uint3 res, float3 aabb_min, float3 aabb_max, hipStream_t s);

// tmp[cell] = max(tmp[cell], e^min(density_out[16 i] - bias, 8)) for every sample i.
void occ_tmp_max(const float4* samples, const float* density_out, float* tmp, float bias, int N, hipStream_t s);

// Occupied level-0 cells in increasing cell order; *d_count = their number.
// zero (nullable): a [total] array cleared on the way (the refresh's tmp grid).
size_t occ_list_scratch_words(int total);
void occ_active_list(const uint8_t* bits, int total, int G, int S, int* list, int* d_count, uint32_t* scratch,
                     hipStream_t s, float* zero = nullptr);

// The refresh's samples in a spatial order (a few sweeps, each by cascade,
// then the Morton code of the cell's 4x4x4 block), so that a wave's encode
// gathers share table lines: sorted[j] = samples[perm[j]].  Only the evaluation order changes: the
// per-cell maximum of the densities does not depend on it.
struct OccSortScratch {
    uint32_t* counts;      // [occ_sort_keys]
    uint32_t* offsets;     // [occ_sort_keys]
    uint32_t* block_sums;  // [march_scratch_words(occ_sort_keys)]
    uint32_t* result;      // [2]
    uint32_t* rank;        // [samples]
};
size_t occ_sort_keys(int cascades, uint3 res);
void occ_sort_samples(const float4* samples, int N, int cascades, uint3 res, const OccSortScratch& scratch,
                      float4* sorted, uint32_t* perm, hipStream_t s);

// Host evaluation of the generator (known-answer tests).
void philox4x32_10_host(uint32_t ctr[4], uint32_t k0, uint32_t k1);

}  // namespace graft
