// The NeRF training step's two heads (density 32-64-16, colour 32-64-64-8) on
// the 16x16x32 fp16 MFMA (nerf_heads.hip).  The forward stores only sigma,
// the density output, the colour output and the colour input; both backward
// kernels recompute a tile's hidden activations from the encodings and the
// colour input.
#pragma once

#include "common.h"
#include "mlp.h"

namespace graft {

// Device arrays of per-layer device pointers, as TinyMLP keeps them.
struct NerfHeadsWeights {
    const __half* const* dW;
    const float* const* dB;
    const __half* const* cW;
    const float* const* cB;
};

struct NerfHeadsFwd {
    const void* packed;            // nerf_heads_pack output
    const __half* enc;             // [levels][enc_plane] feature pairs (hash_encode_planar)
    int enc_plane = 0;
    int levels = 16;
    const float3* dirs = nullptr;  // per ray
    const uint32_t* ray_idx = nullptr;
    float density_bias = 0.0f;
    int out_act = 1;               // colour output: 0 none, 1 sigmoid
    float* sigma = nullptr;        // [N]
    float* density_out = nullptr;  // nullable [N x density_stride] (logits + bias, before sanitising)
    int density_stride = 16;       // 16: the density head's whole output; 1: its logit 0 alone
    float* color_out = nullptr;    // [N x 8]
    __half* color_in = nullptr;    // [N x 32]: sanitised logits | SH (the backward's input; nullable
                                   // for an inference caller)
};

struct NerfHeadsBwd {
    const void* packed;
    const __half* enc;
    int enc_plane = 0;
    int levels = 16;
    const __half* color_in = nullptr;  // [N x 32] the colour input nerf_heads_forward stored
    const __half* color_dy = nullptr;  // [N x 8] colour dL/dy
    const float* dsigma = nullptr;     // [N]
    __half* denc = nullptr;            // [N x 32] dL/d(encoding) (nerf_heads_dx)
    __half* density_dy = nullptr;      // nullable [N x 16]
    __half* color_dx = nullptr;        // nullable [N x 32]: logit features; the SH features are not computed (0)
    // nullable [ceil(N / 16)]: nerf_heads_dx stores per 16-sample tile whether
    // any gradient through the heads is nonzero; nerf_heads_dw given the same
    // array (of the same inputs) skips the others (they add nothing)
    uint32_t* tile_live = nullptr;
    int dw_blocks = 0;                 // weight-gradient blocks per head (0: half the CUs each, so that the
                                       // kernel leaves room beside the scatter it runs with)
};

// Per-layer fp32 gradient arrays (device arrays of device pointers); the
// weight-gradient kernel overwrites them.
struct NerfHeadsGrads {
    float* const* dW;
    float* const* dB;
    float* const* cW;
    float* const* cB;
};

// The occupancy refresh's use of the density head: per sample j of samples[]
// (w = cell index bits) sigma = e^min(logit 0 - density_bias, 8) maxed into
// tmp[cell] (integer max on the float bits) and, when logit is given, logit 0
// stored at logit[j].
struct NerfDensityMax {
    const void* packed;            // nerf_heads_pack or nerf_heads_pack_density output
    const __half* enc = nullptr;   // [levels][enc_plane] feature pairs of samples[] (hash_encode_planar)
    int enc_plane = 0;
    int levels = 16;
    const float4* samples = nullptr;
    float density_bias = 0.0f;
    float* logit = nullptr;
    float* tmp = nullptr;
    // the samples cover every cell they reach exactly once (the early refresh):
    // sigma is stored, which is the maximum over a zeroed cell
    bool one_per_cell = false;
};

bool nerf_heads_supported(const MlpShape& density, const MlpShape& color);
size_t nerf_heads_packed_bytes();
// Packs both heads' fp16 weights and fp32 biases for the kernels below.
void nerf_heads_pack(const NerfHeadsWeights& w, void* packed, hipStream_t s);
// The density head's fragments and biases only (the colour head's are left as they are).
void nerf_heads_pack_density(const NerfHeadsWeights& w, void* packed, hipStream_t s);
void nerf_density_max(const NerfDensityMax& a, int N, hipStream_t s);
void nerf_heads_forward(const NerfHeadsFwd& a, int N, hipStream_t s, const uint32_t* d_n = nullptr);
// dL/d(encoding) (and the optional density / colour dL arrays).
void nerf_heads_dx(const NerfHeadsBwd& a, int N, hipStream_t s, const uint32_t* d_n = nullptr);
// Every layer's dW and db of both heads, overwriting out; the block partials
// live in ws (nullptr: the stream's workspace).
void nerf_heads_dw(const NerfHeadsBwd& a, const NerfHeadsGrads& out, int N, hipStream_t s,
                   const uint32_t* d_n = nullptr, Workspace* ws = nullptr);

}  // namespace graft
