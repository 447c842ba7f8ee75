// Internal interface of the hash-grid kernels (hashgrid.hip).
#pragma once

#include "common.h"

namespace graft {

// enc [N x 2L] fp16 from positions [N x pos_stride] (x, y, z, ...).
// d_n (nullable): device-side sample count (<= N), as for the MLP kernels.
void hash_encode(const GridMeta& m, const __half* table, const float* pos, int pos_stride,
                 __half* enc, int N, hipStream_t stream, const uint32_t* d_n = nullptr);

// The same encodings level-major: level l of sample n at enc[(l * plane + n) * 2],
// its two features adjacent (plane >= N).
void hash_encode_planar(const GridMeta& m, const __half* table, const float* pos, int pos_stride,
                        __half* enc, int plane, int N, hipStream_t stream, const uint32_t* d_n = nullptr);

// grads [L][T][2] += scatter of denc [N x 2L] (backward clamp).
// d_n (nullable): device-side sample count (<= N), as for the MLP kernels.
// The binned path (scatter.h) with scratch cached per (device, stream), or,
// for configurations outside its limits, hash_scatter_atomic.
void hash_scatter(const GridMeta& m, const __half* denc, const float* pos, int pos_stride,
                  float* grads, int N, hipStream_t stream, const uint32_t* d_n = nullptr);

// The same sum with one fp32 global atomic per run of equal corners.
void hash_scatter_atomic(const GridMeta& m, const __half* denc, const float* pos, int pos_stride,
                         float* grads, int N, hipStream_t stream, const uint32_t* d_n = nullptr);

}  // namespace graft
