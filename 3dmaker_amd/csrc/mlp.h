// Internal interface of the fused MLP kernels (mlp.hip).
#pragma once

#include "common.h"

namespace graft {

constexpr int kMaxLayers = 16;

// Hardware shape of a TinyMLP: layer l maps in_l -> out_l.
struct MlpShape {
    int in, hid, out, layers;
    int in_l(int l) const { return l == 0 ? in : hid; }
    int out_l(int l) const { return l == layers - 1 ? out : hid; }
    int maxd() const { return std::max(in, std::max(hid, out)); }
    void validate() const;
};

// Layer-0 input: either fp16 features x [N x in], or positions + hash table
// (then the encoding is computed on the fly and saved to acts[0]).
struct FwdInput {
    const __half* x = nullptr;
    bool save_x0 = false;   // plain input: also write x into acts[0]
    const float* pos = nullptr;
    int pos_stride = 4;
    const __half* table = nullptr;
    const GridMeta* meta = nullptr;
};

// W, B, acts are DEVICE arrays of per-layer device pointers.  acts == nullptr
// selects the inference kernel (no activation saves).
// d_n (nullable): device-side sample count; the kernels then process
// min(*d_n, N) samples, N being the host upper bound the launch is sized for.
void mlp_forward(const MlpShape& s, const FwdInput& in, const __half* const* W,
                 const float* const* B, __half* const* acts, float* out, int N, int out_act,
                 hipStream_t stream, const uint32_t* d_n = nullptr);

// dW/dB (device arrays of per-layer pointers) are accumulated (+=), or
// overwritten with this batch's gradient when accumulate is false; dx may be
// nullptr (then layer 0's dX is skipped).  ws holds the per-block partial
// sums (nullptr: the stream's workspace).
void mlp_backward(const MlpShape& s, const __half* dy, const __half* const* acts,
                  const __half* const* W, float* const* dW, float* const* dB, __half* dx, int N,
                  hipStream_t stream, const uint32_t* d_n = nullptr, bool accumulate = true,
                  Workspace* ws = nullptr);

// dx = dL/dx alone, bitwise the dx of mlp_backward, for the NeRF head shapes
// (32-64-16, 2 layers; 32-64-8, 3 layers); returns false for other shapes.
// mlp_backward(..., dx = nullptr) then yields the weight gradients.
bool mlp_backward_dx(const MlpShape& s, const __half* dy, const __half* const* acts, const __half* const* W,
                     __half* dx, int N, hipStream_t stream, const uint32_t* d_n = nullptr);
bool mlp_has_dx_kernel(const MlpShape& s);

// Fixed-order sum of nparts block partials ws [nparts][P] of one net's
// gradients (W of every layer row-major [out][in], then b of every layer)
// into dW / dB (device arrays of per-layer pointers), added when accumulate.
void mlp_grad_reduce(const MlpShape& s, const float* ws, int nparts, float* const* dW, float* const* dB,
                     bool accumulate, hipStream_t stream);

// The forward of a NeRF step (hash encode + density head, SH gather, colour
// head) in one launch; bitwise equal to mlp_forward(density), sh_gather,
// mlp_forward(colour).  dacts / density_out / cacts / color_in may be null
// (inference); sigma and color_out are always written.
struct NerfFwdArgs {
    MlpShape dshape;                 // density head, out == 16
    const float* pos = nullptr;      // [N x pos_stride] contracted positions
    int pos_stride = 4;
    const __half* table = nullptr;   // fp16 hash table [L][T][2]
    const GridMeta* meta = nullptr;
    const __half* const* dW = nullptr;
    const float* const* dB = nullptr;
    __half* const* dacts = nullptr;  // device array: encodings, hidden activations
    float* density_out = nullptr;    // [N x density_stride]
    int density_stride = 16;         // 1 (the 16x16x32 heads only): the density logit 0 alone, [N]
    const float3* dirs = nullptr;    // per ray
    const uint32_t* ray_idx = nullptr;
    float density_bias = 0.0f;
    float* sigma = nullptr;          // [N]
    MlpShape cshape;                 // colour head, in == 32
    int out_act = 1;                 // colour output activation (0 none, 1 sigmoid)
    const __half* const* cW = nullptr;
    const float* const* cB = nullptr;
    __half* const* cacts = nullptr;  // device array; entries 1.. receive the hidden activations
    __half* color_in = nullptr;      // [N x 32] logits | SH (the colour head's activation 0)
    float* color_out = nullptr;      // [N x cshape.out]
    // Nullable: [L][enc_plane] feature pairs (enc_plane >= N).  When set, the
    // encode runs first as its own launch (hash_encode_planar, each XCD's L2
    // holding only its levels' tables) and the network kernel reads it.
    __half* enc_scratch = nullptr;
    int enc_plane = 0;
    bool enc_ready = false;  // enc_scratch already holds these positions' encodings: no encode launch
    // Nullable: a buffer of nerf_heads_packed_bytes().  With it, the planar
    // encodings and the head shapes nerf_heads_supported() accepts, and no
    // activations asked for (dacts, cacts null), the heads run as the
    // 16x16x32 MFMA kernels of nerf_heads.hip after packing the weights into
    // this buffer (heads_prepacked: the caller packed the current weights).
    void* heads_packed = nullptr;
    bool heads_prepacked = false;
};
void nerf_forward(const NerfFwdArgs& a, int N, hipStream_t stream, const uint32_t* d_n = nullptr);

// The dX part of a NeRF step's backward in one launch: colour dL/dinput,
// density dL/dy (colour dL/dinput[0..15] + d sigma on the logit, clamped) and
// dL/d(encoding); bitwise equal to mlp_backward_dx(colour), density_grad,
// mlp_backward_dx(density).  Only for the head shapes 32-64-64-8 and
// 32-64-16; returns false for others.
struct NerfBwdDxArgs {
    MlpShape cshape, dshape;
    const __half* color_dy = nullptr;       // [N x 8]
    const __half* const* cacts = nullptr;
    const __half* const* cW = nullptr;
    const float* dsigma = nullptr;          // [N]
    const __half* const* dacts = nullptr;
    const __half* const* dW = nullptr;
    __half* color_dx = nullptr;             // [N x 32]
    __half* density_dy = nullptr;           // [N x 16]
    __half* denc = nullptr;                 // [N x 32]
};
bool nerf_backward_dx(const NerfBwdDxArgs& a, int N, hipStream_t stream, const uint32_t* d_n = nullptr);

}  // namespace graft
