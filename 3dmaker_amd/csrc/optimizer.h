// Internal interface of optimizer.hip.
#pragma once

#include "common.h"

namespace graft {

struct AdamArgs {
    float lr, b1, b2, eps, bc1, bc2, inv_scale;
};

constexpr int kMaxLayerCount = 16;
struct LayerSizes {
    int n[kMaxLayerCount];
};

// Hash-table Adam (skip g == 0, zero consumed g, fp16 copy).  n % 4 == 0.
void adam_hash(float* w, __half* w16, float* g, float* m, float* v, size_t n, const AdamArgs& a,
               hipStream_t stream);

// Per-layer dense Adam over device arrays of pointers; w16 may be nullptr.
void adam_layers(float* const* w, __half* const* w16, float* const* g, float* const* m,
                 float* const* v, const LayerSizes& sz, int layers, const AdamArgs& a,
                 hipStream_t stream);

// adam_layers over the weights (with fp16 copy) and the biases in one launch.
void adam_dense(float* const* wW, __half* const* w16, float* const* gW, float* const* mW, float* const* vW,
                const LayerSizes& szW, float* const* wB, float* const* gB, float* const* mB, float* const* vB,
                const LayerSizes& szB, int layers, const AdamArgs& a, hipStream_t stream);

void zero_layers(float* const* a, float* const* b, const LayerSizes& sa, const LayerSizes& sb, int layers,
                 hipStream_t stream);

// *total += sum of squared error; dloss = fp16(diff * 2/(N*valid) * scale [* sigmoid']).
// ws holds the per-block partial sums (nullptr: the stream's workspace).
void mse_loss_grad(const float* pred, const __half* tgt, __half* dloss, float* total, int N, int padded,
                   int valid, float loss_scale, int out_act, hipStream_t stream, Workspace* ws = nullptr);

void pad_f32(const float* src, float* dst, long long rows, int udim, int pdim, hipStream_t s);
void pad_f16(const __half* src, __half* dst, long long rows, int udim, int pdim, hipStream_t s);
void f32_to_f16(const float* src, __half* dst, long long n, hipStream_t s);
void unpad_f32(const float* src, float* dst, long long rows, int pdim, int udim, hipStream_t s);

}  // namespace graft
