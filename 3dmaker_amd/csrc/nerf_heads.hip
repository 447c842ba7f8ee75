// The two NeRF heads of the training step on gfx950's 16x16x32 fp16 MFMA:
// density 32-64-16 (ReLU) and colour 32-64-64-8 (ReLU, sigmoid output), the
// shapes of InstantNerf (networkFusionHashtable.cu:441-682,
// networkFusion.cu:197-355, networkFusionBackward.cu:49-646,
// networkFusionBackwardHashtable.cu:71-781).
//
// Layout.  Samples run along N (lane % 16) and features along K.  A
// 32-feature K block of v_mfma_f32_16x16x32_f16 holds, in lane (n, g = lane /
// 16), slots j = 0..7; slot j stands for feature
//     kslot(kb, g, j) = 32 kb + (j < 4 ? 4 g + j : 16 + 4 g + j - 4).
// That is the D layout of the two 16-row output blocks 2 kb, 2 kb + 1 of a
// layer (lane (n, g) holds rows 4 g .. 4 g + 3 of each), so a layer's output,
// biased, activated and rounded to fp16, is the next layer's B operand as it
// stands.  The weights are the A operand, packed once per step with the same
// slot order (the order of K inside one MFMA is free as long as A and B agree).
//
// The forward stores its outputs and the colour input (logits | SH, 64 B per
// sample) and no hidden activation: the backward kernels recompute each
// 16-sample tile's hidden layers from the encodings and that colour input.
// nerf_heads_dx (critical path) runs the colour dX chain, the
// density-gradient glue (compute_density_grad, otherKernels.cu:506-562) and
// the density dX chain down to dL/d(encoding); nerf_heads_dw (beside the hash
// scatter) runs the same chains and accumulates every layer's dW and db over
// its tiles in registers: dW_l = sum_n dY_l[n] X_l[n]^T needs samples along
// K, so each 16x16 block of X_l and dY_l is transposed by one 16x16x16 MFMA
// against the identity (exact: one non-zero product per output), and two
// tiles' transposed blocks make one 16x16x32 dW update.  Block partials go to
// the caller's workspace and mlp_grad_reduce sums them in a fixed order.
#include "nerf_heads.h"

#include "mlp.h"
#include "nerf_math.h"

#include <algorithm>

namespace graft {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int DIN = 32, DHID = 64, DOUT = 16;  // density head
constexpr int CIN = 32, CHID = 64, COUT = 8;   // colour head (hardware output width)

// forward fragments (A = W, rows = outputs, slots = inputs)
constexpr int FD0 = 0;   // density L0: mt 0..3
constexpr int FD1 = 4;   // density L1: kb 0..1
constexpr int FC0 = 6;   // colour L0: mt 0..3
constexpr int FC1 = 10;  // colour L1: 2 mt + kb
constexpr int FC2 = 18;  // colour L2: kb 0..1
constexpr int kFwdFrags = 20;
// transposed fragments (A = W^T, rows = inputs, slots = outputs)
constexpr int TC2 = 0;   // colour L2^T: mt 0..3 (inputs 0..63), outputs 0..7
constexpr int TC1 = 4;   // colour L1^T: 2 mt + kb
constexpr int TC0 = 12;  // colour L0^T, logit inputs 0..15 only: kb 0..1
constexpr int TD1 = 14;  // density L1^T: mt 0..3, outputs 0..15
constexpr int TD0 = 18;  // density L0^T: 2 mt + kb (mt 0..1)
constexpr int kTrFrags = 22;
// bias blocks (rows 16 mt + 4 g + j in lane group g)
constexpr int BD0 = 0, BD1 = 4, BC0 = 5, BC1 = 9, BC2 = 13;
constexpr int kBiasBlocks = 14;

constexpr size_t kFwdBytes = (size_t)kFwdFrags * 64 * 16;
constexpr size_t kTrBytes = (size_t)kTrFrags * 64 * 16;
constexpr size_t kBiasBytes = (size_t)kBiasBlocks * 4 * 16;

// parameters of each head in mlp_grad_reduce's order: W of every layer
// (row-major [out][in]), then b of every layer
constexpr int PD_W0 = 0, PD_W1 = PD_W0 + DHID * DIN, PD_B0 = PD_W1 + DOUT * DHID, PD_B1 = PD_B0 + DHID;
constexpr int PD = PD_B1 + DOUT;  // 3152
constexpr int PC_W0 = 0, PC_W1 = PC_W0 + CHID * CIN, PC_W2 = PC_W1 + CHID * CHID, PC_B0 = PC_W2 + COUT * CHID;
constexpr int PC_B1 = PC_B0 + CHID, PC_B2 = PC_B1 + CHID;
constexpr int PC = PC_B2 + COUT;  // 6792

__host__ __device__ constexpr int kslot(int kb, int g, int j) { return 32 * kb + (j < 4 ? 4 * g + j : 12 + 4 * g + j); }

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

__device__ __forceinline__ h8 cat(h4 lo, h4 hi) { return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}; }
__device__ __forceinline__ h4 lo4(h8 v) { return h4{v[0], v[1], v[2], v[3]}; }
__device__ __forceinline__ h4 hi4(h8 v) { return h4{v[4], v[5], v[6], v[7]}; }

typedef short s4 __attribute__((ext_vector_type(4)));

// four fp32 values rounded to fp16 (to nearest even), two per instruction
__device__ __forceinline__ h4 round_h4(f4 d) { return __builtin_convertvector(d, h4); }

// ReLU of one output block whose accumulator started from the bias, rounded
// to fp16: rounding first, then the integer max of the fp16 bits with 0, which
// turns every negative value and -0 into +0 and keeps the others.
__device__ __forceinline__ h4 relu_h4(f4 acc)
{
    const s4 b = __builtin_bit_cast(s4, round_h4(acc));
    return __builtin_bit_cast(h4, __builtin_elementwise_max(b, (s4)0));
}

// Two halves of v (fp16 bits) kept where the matching half of x (the fp16
// bits of a ReLU output: +0 or positive) is not 0, else 0: min(x, 1) per
// half is the 0/1 mask and the 16-bit integer product applies it.  The mask
// instruction is written out so that the compiler does not trace it back to
// a float compare and select per half; the product stays compiler-visible
// (it feeds MFMAs, whose operand hazards the compiler tracks).
__device__ __forceinline__ uint32_t keep_where_positive(uint32_t v, uint32_t x)
{
    typedef unsigned short u2 __attribute__((ext_vector_type(2)));
    uint32_t m;
    __asm__("v_pk_min_u16 %0, %1, 1 op_sel_hi:[1,0]" : "=v"(m) : "v"(x));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u2, v) * __builtin_bit_cast(u2, m));
}

// dX block rounded to fp16, zero where the layer's input activation is not > 0
__device__ __forceinline__ h4 mask_h4(f4 d, h4 x)
{
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 m = __builtin_bit_cast(u32x2, x);
    const u32x2 v = __builtin_bit_cast(u32x2, round_h4(d));
    return __builtin_bit_cast(h4, u32x2{keep_where_positive(v[0], m[0]), keep_where_positive(v[1], m[1])});
}

// Placed at the top of a tile loop: the LDS-staged fragments and biases are
// read where they are used instead of being hoisted into registers for the
// whole loop (which would cost a wave's occupancy).
__device__ __forceinline__ void reload_fence() { __asm__ volatile("" ::: "memory"); }

// ---------------------------------------------------------------------------
// packing: W (row-major fp16 [out][in]) and b (fp32) of both heads -> slots
// ---------------------------------------------------------------------------

struct PackParams {
    const _Float16* const* dW;
    const float* const* dB;
    const _Float16* const* cW;
    const float* const* cB;
    h8* fwd;   // [kFwdFrags][64]
    h8* tr;    // [kTrFrags][64]
    f4* bias;  // [kBiasBlocks][4]
    bool density_only;  // the density head's forward fragments and biases only
};

// element (row, col) of W_l [out][in], 0 outside
__device__ __forceinline__ _Float16 wat(const _Float16* W, int out, int in, int row, int col)
{
    return (row < out && col < in) ? W[row * in + col] : (_Float16)0.f;
}

__global__ __launch_bounds__(256) void pack_kernel(const PackParams p)
{
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int nf = (kFwdFrags + kTrFrags) * 64;
    if (p.density_only && (t < nf ? (t >> 6) >= FC0 : ((t - nf) >> 2) >= BC0)) return;
    if (t < nf) {
        const int lane = t & 63, f = t >> 6, m = lane & 15, g = lane >> 4;
        h8 v;
        if (f < kFwdFrags) {
            const _Float16* W;
            int out, in, mt, kb;
            if (f < FD1) { W = p.dW[0]; out = DHID; in = DIN; mt = f - FD0; kb = 0; }
            else if (f < FC0) { W = p.dW[1]; out = DOUT; in = DHID; mt = 0; kb = f - FD1; }
            else if (f < FC1) { W = p.cW[0]; out = CHID; in = CIN; mt = f - FC0; kb = 0; }
            else if (f < FC2) { W = p.cW[1]; out = CHID; in = CHID; mt = (f - FC1) >> 1; kb = (f - FC1) & 1; }
            else { W = p.cW[2]; out = COUT; in = CHID; mt = 0; kb = f - FC2; }
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = wat(W, out, in, 16 * mt + m, kslot(kb, g, j));
            p.fwd[f * 64 + lane] = v;
        } else {
            const int q = f - kFwdFrags;
            const _Float16* W;
            int out, in, mt, kb;
            if (q < TC1) { W = p.cW[2]; out = COUT; in = CHID; mt = q - TC2; kb = 0; }
            else if (q < TC0) { W = p.cW[1]; out = CHID; in = CHID; mt = (q - TC1) >> 1; kb = (q - TC1) & 1; }
            else if (q < TD1) { W = p.cW[0]; out = CHID; in = CIN; mt = 0; kb = q - TC0; }
            else if (q < TD0) { W = p.dW[1]; out = DOUT; in = DHID; mt = q - TD1; kb = 0; }
            else { W = p.dW[0]; out = DHID; in = DIN; mt = (q - TD0) >> 1; kb = (q - TD0) & 1; }
            // rows = inputs, slots = outputs
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = wat(W, out, in, kslot(kb, g, j), 16 * mt + m);
            p.tr[q * 64 + lane] = v;
        }
        return;
    }
    const int u = t - nf;
    if (u < kBiasBlocks * 4) {
        const int b = u >> 2, g = u & 3;
        const float* B;
        int out, mt;
        if (b < BD1) { B = p.dB[0]; out = DHID; mt = b - BD0; }
        else if (b < BC0) { B = p.dB[1]; out = DOUT; mt = 0; }
        else if (b < BC1) { B = p.cB[0]; out = CHID; mt = b - BC0; }
        else if (b < BC2) { B = p.cB[1]; out = CHID; mt = b - BC1; }
        else { B = p.cB[2]; out = COUT; mt = 0; }
        f4 v;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = 16 * mt + 4 * g + j;
            v[j] = row < out ? B[row] : 0.f;
        }
        p.bias[u] = v;
    }
}

// ---------------------------------------------------------------------------
// one tile through both heads
// ---------------------------------------------------------------------------

struct Weights {
    h8 F[kFwdFrags];
};

// The forward fragments staged in LDS, read where they are used.
struct LdsWeights {
    struct Ref {
        const h8* base;
        int lane;
        __device__ h8 operator[](int q) const { return base[q * 64 + lane]; }
    } F;
};

// The forward values of one tile the backward needs.
struct Acts {
    h8 enc;      // density input (kslot order)
    h8 hd[2];    // density hidden
    f4 y;        // density output block (pre-sanitise logits, fp32, + bias)
    h8 cin;      // colour input: sanitised logits | SH
    h8 h1[2];    // colour hidden 1
    h8 h2[2];    // colour hidden 2
    f4 rgb[1];   // colour output rows 4 g .. 4 g + 3 (pre-activation), lanes g < 2
};

struct TileIn {
    h8 enc;
    float dx, dy, dz;
};

// encodings of lane (n, g): levels 2g, 2g+1 (slots 0..3) and 8+2g, 9+2g
// (slots 4..7) from the level-major pairs enc[l][plane]
__device__ __forceinline__ TileIn load_tile(const _Float16* __restrict__ enc, int plane, int L,
                                            const float3* __restrict__ dirs, const uint32_t* __restrict__ ridx,
                                            int n, bool valid, int g)
{
    TileIn t;
    t.dx = t.dy = t.dz = 0.f;
    h2 e[4];
#pragma unroll
    for (int q = 0; q < 4; q++) e[q] = h2{(_Float16)0.f, (_Float16)0.f};
    if (valid) {
        const int lv[4] = {2 * g, 2 * g + 1, 8 + 2 * g, 9 + 2 * g};
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (lv[q] < L) e[q] = *reinterpret_cast<const h2*>(enc + ((size_t)lv[q] * plane + n) * 2);
        const float3 d = dirs[ridx[n]];
        t.dx = d.x;
        t.dy = d.y;
        t.dz = d.z;
    }
    t.enc = h8{e[0].x, e[0].y, e[1].x, e[1].y, e[2].x, e[2].y, e[3].x, e[3].y};
    return t;
}

// SH coefficients 4 g .. 4 g + 3 of a unit direction (sh_basis16's
// expressions, the ones of compute_SH_gather)
__device__ __forceinline__ h4 sh_quad(float x, float y, float z, int g)
{
    float sh[16];
    sh_basis16(x, y, z, sh);
    h4 s;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float v = g == 0 ? sh[j] : g == 1 ? sh[4 + j] : g == 2 ? sh[8 + j] : sh[12 + j];
        s[j] = to_h(v);
    }
    return s;
}

__device__ __forceinline__ void forward_tile(const Weights& w, const f4* __restrict__ sbias, const TileIn& in,
                                             int g, Acts& a)
{
    a.enc = in.enc;
    // density L0 (32 -> 64)
    f4 d0[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) d0[mt] = mfma32(w.F[FD0 + mt], in.enc, sbias[(BD0 + mt) * 4 + g]);
    a.hd[0] = cat(relu_h4(d0[0]), relu_h4(d0[1]));
    a.hd[1] = cat(relu_h4(d0[2]), relu_h4(d0[3]));
    // density L1 (64 -> 16)
    f4 y = mfma32(w.F[FD1 + 0], a.hd[0], sbias[BD1 * 4 + g]);
    y = mfma32(w.F[FD1 + 1], a.hd[1], y);
    a.y = y;
    h4 lg;
#pragma unroll
    for (int j = 0; j < 4; j++) lg[j] = to_h(sanitize_logit(y[j]));
    a.cin = cat(lg, sh_quad(in.dx, in.dy, in.dz, g));
    // colour L0 (32 -> 64)
    f4 c0[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) c0[mt] = mfma32(w.F[FC0 + mt], a.cin, sbias[(BC0 + mt) * 4 + g]);
    a.h1[0] = cat(relu_h4(c0[0]), relu_h4(c0[1]));
    a.h1[1] = cat(relu_h4(c0[2]), relu_h4(c0[3]));
    // colour L1 (64 -> 64)
    f4 c1[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        c1[mt] = mfma32(w.F[FC1 + 2 * mt], a.h1[0], sbias[(BC1 + mt) * 4 + g]);
        c1[mt] = mfma32(w.F[FC1 + 2 * mt + 1], a.h1[1], c1[mt]);
    }
    a.h2[0] = cat(relu_h4(c1[0]), relu_h4(c1[1]));
    a.h2[1] = cat(relu_h4(c1[2]), relu_h4(c1[3]));
    // colour L2 (64 -> 8)
    f4 o = mfma32(w.F[FC2 + 0], a.h2[0], sbias[BC2 * 4 + g]);
    o = mfma32(w.F[FC2 + 1], a.h2[1], o);
    a.rgb[0] = o;
}

// The activations the backward needs, from the tile's encodings and the
// colour input the forward stored: the density hidden layer and both colour
// hidden layers (the same operations as forward_tile, so the same bits).
// FW: the forward fragments, w.F[q] -> h8 (registers or LDS)
template <class FW>
__device__ __forceinline__ void recompute_tile(const FW& w, const f4* __restrict__ sbias, h8 enc, h8 cin, int g,
                                               Acts& a)
{
    a.enc = enc;
    a.cin = cin;
    f4 d0[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) d0[mt] = mfma32(w.F[FD0 + mt], enc, sbias[(BD0 + mt) * 4 + g]);
    a.hd[0] = cat(relu_h4(d0[0]), relu_h4(d0[1]));
    a.hd[1] = cat(relu_h4(d0[2]), relu_h4(d0[3]));
    f4 c0[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) c0[mt] = mfma32(w.F[FC0 + mt], cin, sbias[(BC0 + mt) * 4 + g]);
    a.h1[0] = cat(relu_h4(c0[0]), relu_h4(c0[1]));
    a.h1[1] = cat(relu_h4(c0[2]), relu_h4(c0[3]));
    f4 c1[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        c1[mt] = mfma32(w.F[FC1 + 2 * mt], a.h1[0], sbias[(BC1 + mt) * 4 + g]);
        c1[mt] = mfma32(w.F[FC1 + 2 * mt + 1], a.h1[1], c1[mt]);
    }
    a.h2[0] = cat(relu_h4(c1[0]), relu_h4(c1[1]));
    a.h2[1] = cat(relu_h4(c1[2]), relu_h4(c1[3]));
}

// The inputs of one tile's backward, all indexed by the sample.
struct BwdIn {
    h8 enc, cin, cdy;
    float ds;
};

// The dL/dy blocks of every layer of one tile (fp16, masked as the dX chain
// passes them on) and dL/d(encoding).
struct Grads {
    h8 c2;       // colour L2 output (cdy, slots 0..3 of lane groups 0, 1)
    h4 c1[4];    // colour L1 output
    h4 c0[4];    // colour L0 output
    h4 d1;       // density L1 output (dL/dy of the density head)
    h4 d0[4];    // density L0 output
    h4 cx;       // colour dL/d(input) for the logit features 4 g .. 4 g + 3
    h4 denc[2];  // dL/d(encoding), blocks 0..1
};

// T: the transposed fragments staged in LDS ([kTrFrags][64] h8)
template <bool FULL_DENC>
__device__ __forceinline__ void backward_tile(const h8* T, int lane, const Acts& a, h8 cdy, float ds, Grads& gr)
{
    const int g = lane >> 4;
    const f4 z = f4zero();
    auto TF = [&](int q) { return T[q * 64 + lane]; };
    gr.c2 = cdy;
    // colour L2^T: dX2 (64) masked by h2 > 0 -> dY1
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        const f4 d = mfma32(TF(TC2 + mt), cdy, z);
        gr.c1[mt] = mask_h4(d, (mt & 1) ? hi4(a.h2[mt >> 1]) : lo4(a.h2[mt >> 1]));
    }
    const h8 g1[2] = {cat(gr.c1[0], gr.c1[1]), cat(gr.c1[2], gr.c1[3])};
    // colour L1^T: dX1 masked by h1 > 0 -> dY0
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        f4 d = mfma32(TF(TC1 + 2 * mt), g1[0], z);
        d = mfma32(TF(TC1 + 2 * mt + 1), g1[1], d);
        gr.c0[mt] = mask_h4(d, (mt & 1) ? hi4(a.h1[mt >> 1]) : lo4(a.h1[mt >> 1]));
    }
    const h8 g0[2] = {cat(gr.c0[0], gr.c0[1]), cat(gr.c0[2], gr.c0[3])};
    // colour L0^T for the logit inputs: dL/dlogit (fp16)
    f4 cx = mfma32(TF(TC0 + 0), g0[0], z);
    cx = mfma32(TF(TC0 + 1), g0[1], cx);
    gr.cx = round_h4(cx);
    // glue: + d sigma on logit 0, clamped to the fp16 range, NaN -> 0
    h4 dd;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float f = (float)gr.cx[j];
        if (g == 0 && j == 0) f += ds;
        f = clamp_half_range(f);
        if (f != f) f = 0.0f;
        dd[j] = to_h(f);
    }
    gr.d1 = dd;
    const h8 gd1 = cat(dd, h4zero());
    // density L1^T: dX (64) masked by hd > 0 -> dY0
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        const f4 d = mfma32(TF(TD1 + mt), gd1, z);
        gr.d0[mt] = mask_h4(d, (mt & 1) ? hi4(a.hd[mt >> 1]) : lo4(a.hd[mt >> 1]));
    }
    if constexpr (FULL_DENC) {
        const h8 gd0[2] = {cat(gr.d0[0], gr.d0[1]), cat(gr.d0[2], gr.d0[3])};
        // density L0^T: dL/d(encoding)
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            f4 d = mfma32(TF(TD0 + 2 * mt), gd0[0], z);
            d = mfma32(TF(TD0 + 2 * mt + 1), gd0[1], d);
            gr.denc[mt] = round_h4(d);
        }
    }
}

__device__ __forceinline__ void load_weights(Weights& w, const h8* __restrict__ F, int lane)
{
#pragma unroll
    for (int f = 0; f < kFwdFrags; f++) w.F[f] = F[f * 64 + lane];
}

// biases into LDS (kBiasBlocks x 4 lane groups x f4)
__device__ __forceinline__ void stage_bias(f4* sbias, const f4* __restrict__ bias)
{
    for (int e = threadIdx.x; e < kBiasBlocks * 4; e += blockDim.x) sbias[e] = bias[e];
    __syncthreads();
}

// transposed fragments into LDS; the caller synchronises
__device__ __forceinline__ void stage_tr(h8* str, const h8* __restrict__ tr)
{
    for (int e = threadIdx.x; e < kTrFrags * 64; e += blockDim.x) str[e] = tr[e];
}

__device__ __forceinline__ h8 load_cdy(const _Float16* __restrict__ cdy, int n, bool valid, int g)
{
    h4 v = h4zero();
    if (valid && g < 2) v = ld_h4(cdy + (size_t)n * COUT + 4 * g);
    return cat(v, h4zero());
}

__device__ __forceinline__ h8 load_enc(const _Float16* __restrict__ enc, int plane, int L, int n, bool valid, int g)
{
    h2 e[4];
#pragma unroll
    for (int q = 0; q < 4; q++) e[q] = h2{(_Float16)0.f, (_Float16)0.f};
    if (valid) {
        const int lv[4] = {2 * g, 2 * g + 1, 8 + 2 * g, 9 + 2 * g};
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (lv[q] < L) e[q] = *reinterpret_cast<const h2*>(enc + ((size_t)lv[q] * plane + n) * 2);
    }
    return h8{e[0].x, e[0].y, e[1].x, e[1].y, e[2].x, e[2].y, e[3].x, e[3].y};
}

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

struct FwdParams {
    const h8* fwd;
    const f4* bias;
    const _Float16* enc;
    int plane, L;
    const float3* dirs;
    const uint32_t* ray_idx;
    const uint32_t* d_n;
    int N;
    float density_bias;
    float* sigma;     // [N]
    float* dout;      // nullable [N x 16], or [N] (logit 0 alone) when dout_full is false
    bool dout_full;
    float* cout;      // [N x COUT]
    _Float16* cin;    // nullable [N x 32]
};

template <int OUT_ACT>
__global__ __launch_bounds__(256) void heads_fwd_kernel(const FwdParams p)
{
    __shared__ f4 sbias[kBiasBlocks * 4];
    stage_bias(sbias, p.bias);
    const int lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15;
    Weights w;
    load_weights(w, p.fwd, lane);
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int ntiles = (N + 15) >> 4;
    const int nw = gridDim.x * (blockDim.x >> 6);
    for (int tile = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); tile < ntiles; tile += nw) {
        reload_fence();
        const int n = tile * 16 + r;
        const bool valid = n < N;
        const TileIn in = load_tile(p.enc, p.plane, p.L, p.dirs, p.ray_idx, n, valid, g);
        Acts a;
        forward_tile(w, sbias, in, g, a);
        if (!valid) continue;
        if (p.dout) {
            if (p.dout_full) *reinterpret_cast<f4*>(p.dout + (size_t)n * DOUT + 4 * g) = a.y;
            else if (g == 0) p.dout[n] = a.y[0];
        }
        if (g == 0) p.sigma[n] = nerf_expf(fminf(sanitize_logit(a.y[0]) - p.density_bias, 8.0f));
        if (p.cin) {
            st_h4(p.cin + (size_t)n * 32 + 4 * g, lo4(a.cin));
            st_h4(p.cin + (size_t)n * 32 + 16 + 4 * g, hi4(a.cin));
        }
        if (g < 2) {
            f4 v = a.rgb[0];
            if (OUT_ACT == 1) {
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = 1.0f / (1.0f + expf(-v[j]));
            }
            *reinterpret_cast<f4*>(p.cout + (size_t)n * COUT + 4 * g) = v;
        }
    }
}

// The density head alone over samples in an arbitrary order (the occupancy
// refresh): sigma = e^min(logit 0 - bias, 8) of each sample maxed into its
// cell of tmp as an integer max on the float bits (sigma >= 0: the float max,
// whatever the order), and logit 0 stored in the same order.
struct DensityMaxParams {
    const h8* fwd;
    const f4* bias;
    const _Float16* enc;
    int plane, L;
    const float4* samples;  // w = cell index bits
    int N;
    float density_bias;
    float* logit;           // nullable [N]
    float* tmp;
    bool one_per_cell;      // every cell of tmp gets exactly one sample: stored, not maxed
};

__global__ __launch_bounds__(256) void density_max_kernel(const DensityMaxParams p)
{
    __shared__ f4 sbias[kBiasBlocks * 4];
    stage_bias(sbias, p.bias);
    const int lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15;
    h8 F[6];
#pragma unroll
    for (int q = 0; q < 6; q++) F[q] = p.fwd[(FD0 + q) * 64 + lane];
    const int ntiles = (p.N + 15) >> 4;
    const int nw = gridDim.x * (blockDim.x >> 6);
    int tile = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    // the next tile's encodings and cell are in flight while this one computes
    auto load = [&](int t, h8& enc, int& cell) {
        const int n = t * 16 + r;
        const bool valid = t < ntiles && n < p.N;
        enc = load_enc(p.enc, p.plane, p.L, n, valid, g);
        cell = (valid && g == 0) ? __float_as_int(p.samples[n].w) : 0;
    };
    h8 enc;
    int cell;
    load(tile, enc, cell);
    for (; tile < ntiles; tile += nw) {
        h8 enc_n;
        int cell_n;
        load(tile + nw, enc_n, cell_n);
        const int n = tile * 16 + r;
        f4 d0[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) d0[mt] = mfma32(F[mt], enc, sbias[(BD0 + mt) * 4 + g]);
        const h8 hd0 = cat(relu_h4(d0[0]), relu_h4(d0[1]));
        const h8 hd1 = cat(relu_h4(d0[2]), relu_h4(d0[3]));
        f4 y = mfma32(F[4], hd0, sbias[BD1 * 4 + g]);
        y = mfma32(F[5], hd1, y);
        if (n < p.N && g == 0) {
            const float sigma = nerf_expf(fminf(y[0] - p.density_bias, 8.0f));
            int* dst = reinterpret_cast<int*>(p.tmp) + cell;
            if (p.one_per_cell) *dst = __float_as_int(sigma);  // the max over one sample
            else atomicMax(dst, __float_as_int(sigma));
            if (p.logit) p.logit[n] = y[0];
        }
        enc = enc_n;
        cell = cell_n;
    }
}

struct BwdParams {
    const h8* fwd;
    const h8* tr;
    const f4* bias;
    const _Float16* enc;
    int plane, L;
    const _Float16* cin;   // [N x 32] colour input stored by the forward
    const uint32_t* d_n;
    int N;
    const _Float16* cdy;   // [N x COUT] colour dL/dy
    const float* dsigma;   // [N]
    _Float16* denc;        // [N x 32]
    _Float16* dloss;       // nullable [N x 16] density dL/dy
    _Float16* cdx;         // nullable [N x 32] colour dL/d(input): logit features, SH features 0
    float* ws_d;           // [gridDim.x][PD] (weight-gradient kernel)
    float* ws_c;           // [gridDim.x][PC]
    uint32_t* tile_live;   // nullable [tiles]: the dX kernel stores which tiles have a nonzero gradient, the
                           // weight-gradient kernel then visits only those
};

__device__ __forceinline__ BwdIn load_bwd(const BwdParams& p, int n, bool valid, int g)
{
    BwdIn in;
    in.enc = load_enc(p.enc, p.plane, p.L, n, valid, g);
    h4 c0 = h4zero(), c1 = h4zero();
    if (valid) {
        c0 = ld_h4(p.cin + (size_t)n * 32 + 4 * g);
        c1 = ld_h4(p.cin + (size_t)n * 32 + 16 + 4 * g);
    }
    in.cin = cat(c0, c1);
    in.cdy = load_cdy(p.cdy, n, valid, g);
    in.ds = (valid && g == 0) ? p.dsigma[n] : 0.0f;
    return in;
}

// A tile whose colour dL/dy is zero in every sample, and whose density dL/dy
// (the glue of a zero colour dL/dx and d sigma) rounds to zero as well, has
// zero gradients through both heads: every dL/d(encoding), dW and db term of
// it is 0 (samples past a ray's saturated transmittance; about half the tiles
// of a converged scene).  The kernels below skip such tiles wave-uniformly;
// the dX kernel stores what the chain would (zeros, and the glue of +0).

// density dL/dy slot 0 of a sample whose colour dL/dx is +0 (the glue)
__device__ __forceinline__ _Float16 glue_of_zero(float ds)
{
    float f = 0.0f + ds;
    f = clamp_half_range(f);
    if (f != f) f = 0.0f;
    return to_h(f);
}

__device__ __forceinline__ bool h8_nonzero(h8 v)
{
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 b = __builtin_bit_cast(u32x4, v);
    return ((b[0] | b[1] | b[2] | b[3]) & 0x7fff7fffu) != 0u;
}

__device__ __forceinline__ bool h4_nonzero(h4 v)
{
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 b = __builtin_bit_cast(u32x2, v);
    return ((b[0] | b[1]) & 0x7fff7fffu) != 0u;
}

// the whole wave's tile has some nonzero colour dL/dy or density dL/dy
__device__ __forceinline__ bool tile_live(h8 cdy, float ds, int g)
{
    const bool mine = h8_nonzero(cdy) || (g == 0 && (__builtin_bit_cast(uint16_t, glue_of_zero(ds)) & 0x7fffu) != 0u);
    return __ballot(mine) != 0ull;
}

__global__ __launch_bounds__(256) void heads_dx_kernel(const BwdParams p)
{
    __shared__ f4 sbias[kBiasBlocks * 4];
    __shared__ h8 str[kTrFrags * 64];
    stage_tr(str, p.tr);
    stage_bias(sbias, p.bias);
    const int lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15;
    Weights w;
    load_weights(w, p.fwd, lane);
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int ntiles = (N + 15) >> 4;
    const int nw = gridDim.x * (blockDim.x >> 6);
    int tile = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    BwdIn cur = load_bwd(p, tile * 16 + r, tile < ntiles && tile * 16 + r < N, g);
    for (; tile < ntiles; tile += nw) {
        reload_fence();
        const int n = tile * 16 + r;
        const bool valid = n < N;
        // the next tile's inputs are in flight while this one computes
        const int nt = tile + nw;
        const BwdIn nxt = load_bwd(p, nt * 16 + r, nt < ntiles && nt * 16 + r < N, g);
        Grads gr;
        const bool live = tile_live(cur.cdy, cur.ds, g);
        if (p.tile_live && lane == 0) p.tile_live[tile] = live ? 1u : 0u;
        if (live) {
            Acts a;
            recompute_tile(w, sbias, cur.enc, cur.cin, g, a);
            backward_tile<true>(str, lane, a, cur.cdy, cur.ds, gr);
        } else {
            gr.denc[0] = gr.denc[1] = gr.cx = h4zero();
            gr.d1 = h4zero();
            if (g == 0) gr.d1[0] = glue_of_zero(cur.ds);
        }
        if (valid) {
            st_h4(p.denc + (size_t)n * DIN + 4 * g, gr.denc[0]);
            st_h4(p.denc + (size_t)n * DIN + 16 + 4 * g, gr.denc[1]);
            if (p.dloss) st_h4(p.dloss + (size_t)n * DOUT + 4 * g, gr.d1);
            if (p.cdx) {
                st_h4(p.cdx + (size_t)n * 32 + 4 * g, gr.cx);
                st_h4(p.cdx + (size_t)n * 32 + 16 + 4 * g, h4zero());
            }
        }
        cur = nxt;
    }
}

// One 16x16 block in the D layout (lane (n, g): features 4 g + j of sample n)
// -> lane (feature f, g): samples 4 g + j of feature f (fp32, exact).
__device__ __forceinline__ f4 transpose16(h4 blk, h4 ident)
{
    return __builtin_amdgcn_mfma_f32_16x16x16f16(blk, ident, f4zero(), 0, 0, 0);
}

// One block transposed and rounded to fp16 (exact); *colsum (nullable) adds
// its 4 values (a partial of the feature's db).
__device__ __forceinline__ h4 tblk(h4 b, h4 ident, float* colsum = nullptr)
{
    const f4 t = transpose16(b, ident);
    if (colsum) *colsum += (t[0] + t[1]) + (t[2] + t[3]);
    return round_h4(t);
}

__device__ __forceinline__ h4 blk(const h8* v, int b) { return (b & 1) ? hi4(v[b >> 1]) : lo4(v[b >> 1]); }

__device__ __forceinline__ f4 mfma16t(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// Accumulators of the weight-gradient kernel, per head: dW blocks [out
// block][in block] and db partials.
struct ColorAcc {
    f4 c0[4][2], c1[4][4], c2[4];
    float b0[4], b1[4], b2;
};
struct DensityAcc {
    f4 d0[4][2], d1[4];
    float b0[4], b1;
};

// The colour head's dW / db of one tile: dY2 = cdy, dY1 and dY0 from the
// colour dX chain (backward_tile's operations, so the same bits); each
// layer's update follows as soon as its dL/dy exists.
__device__ __forceinline__ void color_dw_tile(ColorAcc& A, const h8* T, int lane, const Acts& a, h4 cdy, h4 ident)
{
    const f4 z = f4zero();
    auto TF = [&](int q) { return T[q * 64 + lane]; };
    const h8 g2 = cat(cdy, h4zero());
    {  // L2: cdy x h2
        const h4 Y = tblk(cdy, ident, &A.b2);
#pragma unroll
        for (int mi = 0; mi < 4; mi++) A.c2[mi] = mfma16t(Y, tblk(blk(a.h2, mi), ident), A.c2[mi]);
    }
    h4 c1[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) c1[mt] = mask_h4(mfma32(TF(TC2 + mt), g2, z), blk(a.h2, mt));
    {  // L1: dY1 x h1
        h4 X[4];
#pragma unroll
        for (int mi = 0; mi < 4; mi++) X[mi] = tblk(blk(a.h1, mi), ident);
#pragma unroll
        for (int mo = 0; mo < 4; mo++) {
            const h4 Y = tblk(c1[mo], ident, &A.b1[mo]);
#pragma unroll
            for (int mi = 0; mi < 4; mi++) A.c1[mo][mi] = mfma16t(Y, X[mi], A.c1[mo][mi]);
        }
    }
    const h8 g1[2] = {cat(c1[0], c1[1]), cat(c1[2], c1[3])};
    const h4 X0 = tblk(lo4(a.cin), ident), X1 = tblk(hi4(a.cin), ident);
#pragma unroll
    for (int mo = 0; mo < 4; mo++) {  // L0: dY0 x cin
        f4 d = mfma32(TF(TC1 + 2 * mo), g1[0], z);
        d = mfma32(TF(TC1 + 2 * mo + 1), g1[1], d);
        const h4 Y = tblk(mask_h4(d, blk(a.h1, mo)), ident, &A.b0[mo]);
        A.c0[mo][0] = mfma16t(Y, X0, A.c0[mo][0]);
        A.c0[mo][1] = mfma16t(Y, X1, A.c0[mo][1]);
    }
}

// The density head's dW / db of one tile from its dL/dy (d1) and hidden
// layer (hd): dY0 = (W1^T d1 masked by hd > 0), then the two updates.
__device__ __forceinline__ void density_dw_update(DensityAcc& A, const h8* T, int lane, const h8* hd, h8 enc, h4 d1,
                                                  h4 ident)
{
    const f4 z = f4zero();
    const h8 gd1 = cat(d1, h4zero());
    h4 d0[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) d0[mt] = mask_h4(mfma32(T[(TD1 + mt) * 64 + lane], gd1, z), blk(hd, mt));
    {  // L1: dY1 x hd
        const h4 Y = tblk(d1, ident, &A.b1);
#pragma unroll
        for (int mi = 0; mi < 4; mi++) A.d1[mi] = mfma16t(Y, tblk(blk(hd, mi), ident), A.d1[mi]);
    }
    const h4 X0 = tblk(lo4(enc), ident), X1 = tblk(hi4(enc), ident);
#pragma unroll
    for (int mo = 0; mo < 4; mo++) {  // L0: dY0 x enc
        const h4 Y = tblk(d0[mo], ident, &A.b0[mo]);
        A.d0[mo][0] = mfma16t(Y, X0, A.d0[mo][0]);
        A.d0[mo][1] = mfma16t(Y, X1, A.d0[mo][1]);
    }
}

// The density head's dW / db of one tile when its dL/dy is not stored: the
// whole dX chain down to it (backward_tile's operations, so the same bits).
__device__ __forceinline__ void density_dw_tile(DensityAcc& A, const h8* T, int lane, const Acts& a, h4 cdy, float ds,
                                                h4 ident)
{
    Grads gr;
    backward_tile<false>(T, lane, a, cat(cdy, h4zero()), ds, gr);
    density_dw_update(A, T, lane, a.hd, a.enc, gr.d1, ident);
}

// The density hidden layer of one tile (recompute_tile's operations for it)
template <class FW>
__device__ __forceinline__ void recompute_density(const FW& w, const f4* __restrict__ sbias, h8 enc, int g, h8* hd)
{
    f4 d0[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) d0[mt] = mfma32(w.F[FD0 + mt], enc, sbias[(BD0 + mt) * 4 + g]);
    hd[0] = cat(relu_h4(d0[0]), relu_h4(d0[1]));
    hd[1] = cat(relu_h4(d0[2]), relu_h4(d0[3]));
}

// db: the four lane groups of a feature hold partial sums
__device__ __forceinline__ float gsum(float v)
{
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// lane (i = r, g) of dW block (mo, mi) holds rows 16 mo + 4 g + j, column
// 16 mi + r; the waves of a block add theirs in wave order (first: store)
__device__ __forceinline__ void put_w(float* s, int wofs, int in, int mo, int mi, f4 v, int rows, bool first, int g,
                                      int r)
{
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int o = 16 * mo + 4 * g + j;
        if (o < rows) {
            float& d = s[wofs + o * in + 16 * mi + r];
            d = first ? v[j] : d + v[j];
        }
    }
}
__device__ __forceinline__ void put_b(float* s, int bofs, int mo, float v, int rows, bool first, int g, int r)
{
    const int o = 16 * mo + r;
    if (g == 0 && o < rows) {
        float& d = s[bofs + o];
        d = first ? v : d + v;
    }
}

// Blocks [0, color_blocks) accumulate the colour head's gradients over every
// tile, the others the density head's: each block partial is one head's row
// of the workspace.
// A wave's live tiles among t0, t0 + stride, t0 + 2 stride, ... in order
// (wave-uniform): the flags of 64 candidates are loaded at once, one per lane,
// and kept as a mask, so that finding the next tile waits for no load (a wave
// of the step visits at most 64 candidates).
struct LiveTiles {
    const uint32_t* live;
    int base, stride, ntiles, lane;
    uint64_t mask;
    __device__ LiveTiles(const uint32_t* __restrict__ l, int t0, int st, int nt, int ln)
        : live(l), base(t0), stride(st), ntiles(nt), lane(ln)
    {
        load();
    }
    __device__ void load()
    {
        const int c = base + lane * stride;
        mask = __ballot(c < ntiles && live[c] != 0u);
    }
    // the next live tile, ntiles once there is none
    __device__ int next()
    {
        while (mask == 0ull) {
            base += 64 * stride;
            if (base >= ntiles) return ntiles;
            load();
        }
        const int i = __ffsll((unsigned long long)mask) - 1;
        mask &= mask - 1ull;
        return base + i * stride;
    }
};

// LIVE: p.tile_live holds the dX kernel's flags and only live tiles are visited
template <bool LIVE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void heads_dw_kernel(const BwdParams p,
                                                                                               int color_blocks)
{
    __shared__ f4 sbias[kBiasBlocks * 4];
    // the fragments during the tile loop, then the block partial of one head
    extern __shared__ __align__(16) unsigned char smem[];
    h8* str = reinterpret_cast<h8*>(smem);
    h8* sfw = str + kTrFrags * 64;
    float* sred = reinterpret_cast<float*>(smem);
    stage_tr(str, p.tr);
    for (int e = threadIdx.x; e < kFwdFrags * 64; e += blockDim.x) sfw[e] = p.fwd[e];
    stage_bias(sbias, p.bias);
    const int lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15, wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    const LdsWeights w{{sfw, lane}};
    h4 ident;
#pragma unroll
    for (int j = 0; j < 4; j++) ident[j] = (_Float16)(4 * g + j == r ? 1.0f : 0.0f);
    const bool color = (int)blockIdx.x < color_blocks;
    const int rb = color ? blockIdx.x : blockIdx.x - color_blocks;        // block index within the role
    const int nb = color ? color_blocks : (int)gridDim.x - color_blocks;  // blocks of the role
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int ntiles = (N + 15) >> 4;
    if (color) {
        ColorAcc A;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            A.c0[i][0] = A.c0[i][1] = A.c2[i] = f4zero();
#pragma unroll
            for (int k = 0; k < 4; k++) A.c1[i][k] = f4zero();
            A.b0[i] = A.b1[i] = 0.f;
        }
        A.b2 = 0.f;
        const int stride = nb * waves;
        if constexpr (LIVE) {
            // this wave's live tiles (every stride-th tile; the dead ones add
            // nothing), in order
            // invalid samples: zero dL/dy; the next live tile's inputs are in
            // flight while this one computes
            LiveTiles lt(p.tile_live, rb * waves + wave, stride, ntiles, lane);
            int tile = lt.next();
            BwdIn in = load_bwd(p, tile * 16 + r, tile < ntiles && tile * 16 + r < N, g);
            while (tile < ntiles) {
                reload_fence();
                const int nt = lt.next();
                const BwdIn nxt = load_bwd(p, nt * 16 + r, nt < ntiles && nt * 16 + r < N, g);
                Acts a;
                recompute_tile(w, sbias, in.enc, in.cin, g, a);
                color_dw_tile(A, str, lane, a, lo4(in.cdy), ident);
                in = nxt;
                tile = nt;
            }
        } else {
            int tile = rb * waves + wave;
            // invalid samples: zero dL/dy; the next tile's inputs are in
            // flight while this one computes
            BwdIn in = load_bwd(p, tile * 16 + r, tile < ntiles && tile * 16 + r < N, g);
            for (; tile < ntiles; tile += stride) {
                reload_fence();
                const int nt = tile + stride;
                const BwdIn nxt = load_bwd(p, nt * 16 + r, nt < ntiles && nt * 16 + r < N, g);
                Acts a;
                recompute_tile(w, sbias, in.enc, in.cin, g, a);
                color_dw_tile(A, str, lane, a, lo4(in.cdy), ident);
                in = nxt;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            A.b0[i] = gsum(A.b0[i]);
            A.b1[i] = gsum(A.b1[i]);
        }
        A.b2 = gsum(A.b2);
        __syncthreads();  // every wave is done with the fragments
        for (int wv = 0; wv < waves; wv++) {
            if (wave == wv) {
                const bool first = wv == 0;
#pragma unroll
                for (int mo = 0; mo < 4; mo++) {
                    put_w(sred, PC_W0, CIN, mo, 0, A.c0[mo][0], CHID, first, g, r);
                    put_w(sred, PC_W0, CIN, mo, 1, A.c0[mo][1], CHID, first, g, r);
                    put_b(sred, PC_B0, mo, A.b0[mo], CHID, first, g, r);
#pragma unroll
                    for (int mi = 0; mi < 4; mi++) put_w(sred, PC_W1, CHID, mo, mi, A.c1[mo][mi], CHID, first, g, r);
                    put_b(sred, PC_B1, mo, A.b1[mo], CHID, first, g, r);
                    put_w(sred, PC_W2, CHID, 0, mo, A.c2[mo], COUT, first, g, r);
                }
                put_b(sred, PC_B2, 0, A.b2, COUT, first, g, r);
            }
            __syncthreads();
        }
        for (int e = threadIdx.x; e < PC; e += blockDim.x) p.ws_c[(size_t)rb * PC + e] = sred[e];
    } else {
        DensityAcc A;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            A.d0[i][0] = A.d0[i][1] = A.d1[i] = f4zero();
            A.b0[i] = 0.f;
        }
        A.b1 = 0.f;
        const int stride = nb * waves;
        int tile = rb * waves + wave;
        if (p.dloss) {
            // the density dL/dy the dX kernel stored for these inputs: no
            // colour chain; the next tile's inputs are in flight while this
            // one computes
            auto load = [&](int t, h8& enc, h4& d1) {
                const int n = t * 16 + r;
                const bool valid = t < ntiles && n < N;
                enc = load_enc(p.enc, p.plane, p.L, n, valid, g);
                d1 = valid ? ld_h4(p.dloss + (size_t)n * DOUT + 4 * g) : h4zero();
            };
            if constexpr (LIVE) {
                LiveTiles lt(p.tile_live, tile, stride, ntiles, lane);
                int t = lt.next();
                h8 enc;
                h4 d1;
                load(t, enc, d1);
                while (t < ntiles) {
                    reload_fence();
                    const int nt = lt.next();
                    h8 enc_n;
                    h4 d1_n;
                    load(nt, enc_n, d1_n);
                    h8 hd[2];
                    recompute_density(w, sbias, enc, g, hd);
                    density_dw_update(A, str, lane, hd, enc, d1, ident);
                    enc = enc_n;
                    d1 = d1_n;
                    t = nt;
                }
            } else {
                h8 enc;
                h4 d1;
                load(tile, enc, d1);
                for (; tile < ntiles; tile += stride) {
                    reload_fence();
                    h8 enc_n;
                    h4 d1_n;
                    load(tile + stride, enc_n, d1_n);
                    h8 hd[2];
                    recompute_density(w, sbias, enc, g, hd);
                    density_dw_update(A, str, lane, hd, enc, d1, ident);
                    enc = enc_n;
                    d1 = d1_n;
                }
            }
        } else {
            BwdIn in = load_bwd(p, tile * 16 + r, tile < ntiles && tile * 16 + r < N, g);
            for (; tile < ntiles; tile += stride) {
                reload_fence();
                const int nt = tile + stride;
                const BwdIn nxt = load_bwd(p, nt * 16 + r, nt < ntiles && nt * 16 + r < N, g);
                Acts a;
                recompute_tile(w, sbias, in.enc, in.cin, g, a);
                density_dw_tile(A, str, lane, a, lo4(in.cdy), in.ds, ident);
                in = nxt;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) A.b0[i] = gsum(A.b0[i]);
        A.b1 = gsum(A.b1);
        __syncthreads();  // every wave is done with the fragments
        for (int wv = 0; wv < waves; wv++) {
            if (wave == wv) {
                const bool first = wv == 0;
#pragma unroll
                for (int mo = 0; mo < 4; mo++) {
                    put_w(sred, PD_W0, DIN, mo, 0, A.d0[mo][0], DHID, first, g, r);
                    put_w(sred, PD_W0, DIN, mo, 1, A.d0[mo][1], DHID, first, g, r);
                    put_b(sred, PD_B0, mo, A.b0[mo], DHID, first, g, r);
                    put_w(sred, PD_W1, DHID, 0, mo, A.d1[mo], DOUT, first, g, r);
                }
                put_b(sred, PD_B1, 0, A.b1, DOUT, first, g, r);
            }
            __syncthreads();
        }
        for (int e = threadIdx.x; e < PD; e += blockDim.x) p.ws_d[(size_t)rb * PD + e] = sred[e];
    }
}

bool shapes_ok(const MlpShape& d, const MlpShape& c)
{
    return d.in == DIN && d.hid == DHID && d.out == DOUT && d.layers == 2 && c.in == CIN && c.hid == CHID &&
           c.out == COUT && c.layers == 3;
}

int grid_for(const void* kern, int lds, int ntiles, int per_block_tiles)
{
    int per_cu = 0;
    GRAFT_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds));
    const int want = (ntiles + per_block_tiles - 1) / per_block_tiles;
    return std::max(1, std::min(want, num_cus() * std::max(1, per_cu)));
}

}  // namespace

bool nerf_heads_supported(const MlpShape& density, const MlpShape& color)
{
    return shapes_ok(density, color);
}

size_t nerf_heads_packed_bytes() { return kFwdBytes + kTrBytes + kBiasBytes; }

void nerf_heads_pack(const NerfHeadsWeights& w, void* packed, hipStream_t s)
{
    PackParams p{};
    p.dW = reinterpret_cast<const _Float16* const*>(w.dW);
    p.dB = w.dB;
    p.cW = reinterpret_cast<const _Float16* const*>(w.cW);
    p.cB = w.cB;
    unsigned char* base = static_cast<unsigned char*>(packed);
    p.fwd = reinterpret_cast<h8*>(base);
    p.tr = reinterpret_cast<h8*>(base + kFwdBytes);
    p.bias = reinterpret_cast<f4*>(base + kFwdBytes + kTrBytes);
    const int threads = (kFwdFrags + kTrFrags) * 64 + kBiasBlocks * 4;
    hipLaunchKernelGGL(pack_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, p);
    GRAFT_LAUNCH_CHECK();
}

void nerf_heads_pack_density(const NerfHeadsWeights& w, void* packed, hipStream_t s)
{
    PackParams p{};
    p.dW = reinterpret_cast<const _Float16* const*>(w.dW);
    p.dB = w.dB;
    unsigned char* base = static_cast<unsigned char*>(packed);
    p.fwd = reinterpret_cast<h8*>(base);
    p.tr = reinterpret_cast<h8*>(base + kFwdBytes);
    p.bias = reinterpret_cast<f4*>(base + kFwdBytes + kTrBytes);
    p.density_only = true;
    const int threads = (kFwdFrags + kTrFrags) * 64 + kBiasBlocks * 4;
    hipLaunchKernelGGL(pack_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, p);
    GRAFT_LAUNCH_CHECK();
}

void nerf_density_max(const NerfDensityMax& a, int N, hipStream_t s)
{
    if (N <= 0) return;
    if (a.enc_plane < N) throw std::runtime_error("NeRF heads: encoding plane stride below the sample count");
    if (a.levels < 1 || a.levels > 16) throw std::runtime_error("NeRF heads: the density input is 16 levels x 2");
    DensityMaxParams p{};
    const unsigned char* base = static_cast<const unsigned char*>(a.packed);
    p.fwd = reinterpret_cast<const h8*>(base);
    p.bias = reinterpret_cast<const f4*>(base + kFwdBytes + kTrBytes);
    p.enc = reinterpret_cast<const _Float16*>(a.enc);
    p.plane = a.enc_plane;
    p.L = a.levels;
    p.samples = a.samples;
    p.N = N;
    p.density_bias = a.density_bias;
    p.logit = a.logit;
    p.tmp = a.tmp;
    p.one_per_cell = a.one_per_cell;
    const int blocks = grid_for((const void*)density_max_kernel, 0, (N + 15) / 16, 4);
    hipLaunchKernelGGL(density_max_kernel, dim3(blocks), dim3(256), 0, s, p);
    GRAFT_LAUNCH_CHECK();
}

void nerf_heads_forward(const NerfHeadsFwd& a, int N, hipStream_t s, const uint32_t* d_n)
{
    if (N <= 0) return;
    if (a.out_act != 0 && a.out_act != 1) throw std::runtime_error("NeRF heads: unsupported output activation");
    if (a.enc_plane < N) throw std::runtime_error("NeRF heads: encoding plane stride below the sample count");
    if (a.levels < 1 || a.levels > 16) throw std::runtime_error("NeRF heads: the density input is 16 levels x 2");
    FwdParams p{};
    const unsigned char* base = static_cast<const unsigned char*>(a.packed);
    p.fwd = reinterpret_cast<const h8*>(base);
    p.bias = reinterpret_cast<const f4*>(base + kFwdBytes + kTrBytes);
    p.enc = reinterpret_cast<const _Float16*>(a.enc);
    p.plane = a.enc_plane;
    p.L = a.levels;
    p.dirs = a.dirs;
    p.ray_idx = a.ray_idx;
    p.d_n = d_n;
    p.N = N;
    p.density_bias = a.density_bias;
    p.sigma = a.sigma;
    if (a.density_stride != 16 && a.density_stride != 1)
        throw std::runtime_error("NeRF heads: the density output stride must be 16 or 1");
    p.dout = a.density_out;
    p.dout_full = a.density_stride == 16;
    p.cout = a.color_out;
    p.cin = reinterpret_cast<_Float16*>(a.color_in);
    const int ntiles = (N + 15) / 16;
    const void* kern = a.out_act == 1 ? (const void*)heads_fwd_kernel<1> : (const void*)heads_fwd_kernel<0>;
    const int blocks = grid_for(kern, 0, ntiles, 4);
    if (a.out_act == 1) hipLaunchKernelGGL(heads_fwd_kernel<1>, dim3(blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL(heads_fwd_kernel<0>, dim3(blocks), dim3(256), 0, s, p);
    GRAFT_LAUNCH_CHECK();
}

static BwdParams bwd_params(const NerfHeadsBwd& a, int N, const uint32_t* d_n)
{
    if (a.enc_plane < N) throw std::runtime_error("NeRF heads: encoding plane stride below the sample count");
    if (a.levels < 1 || a.levels > 16) throw std::runtime_error("NeRF heads: the density input is 16 levels x 2");
    if (!a.color_in) throw std::runtime_error("NeRF heads: the backward reads the colour input the forward stored");
    BwdParams p{};
    const unsigned char* base = static_cast<const unsigned char*>(a.packed);
    p.fwd = reinterpret_cast<const h8*>(base);
    p.tr = reinterpret_cast<const h8*>(base + kFwdBytes);
    p.bias = reinterpret_cast<const f4*>(base + kFwdBytes + kTrBytes);
    p.enc = reinterpret_cast<const _Float16*>(a.enc);
    p.plane = a.enc_plane;
    p.L = a.levels;
    p.cin = reinterpret_cast<const _Float16*>(a.color_in);
    p.d_n = d_n;
    p.N = N;
    p.cdy = reinterpret_cast<const _Float16*>(a.color_dy);
    p.dsigma = a.dsigma;
    p.denc = reinterpret_cast<_Float16*>(a.denc);
    p.dloss = reinterpret_cast<_Float16*>(a.density_dy);
    p.cdx = reinterpret_cast<_Float16*>(a.color_dx);
    p.tile_live = a.tile_live;
    return p;
}

void nerf_heads_dx(const NerfHeadsBwd& a, int N, hipStream_t s, const uint32_t* d_n)
{
    if (N <= 0) return;
    const BwdParams p = bwd_params(a, N, d_n);
    const int ntiles = (N + 15) / 16;
    const int blocks = grid_for((const void*)heads_dx_kernel, 0, ntiles, 4);
    hipLaunchKernelGGL(heads_dx_kernel, dim3(blocks), dim3(256), 0, s, p);
    GRAFT_LAUNCH_CHECK();
}

void nerf_heads_dw(const NerfHeadsBwd& a, const NerfHeadsGrads& out, int N, hipStream_t s, const uint32_t* d_n,
                   Workspace* ws)
{
    // N = 0 still runs: the gradients are overwritten with zeros
    if (N < 0) return;
    BwdParams p = bwd_params(a, N, d_n);
    const int lds = (int)std::max(kTrBytes + kFwdBytes, (size_t)PC * sizeof(float));
    const int per_head = a.dw_blocks > 0 ? a.dw_blocks : std::max(1, num_cus() / 2);
    // an even split also when the density dL/dy is stored (measured against
    // 70/30, 40/60 and 30/70 colour/density splits beside the scatter)
    const int cb = per_head, db = per_head;
    Workspace& w = ws ? *ws : stream_workspace(s);
    float* part = static_cast<float*>(w.get(((size_t)cb * PC + (size_t)db * PD) * sizeof(float)));
    p.ws_c = part;
    p.ws_d = part + (size_t)cb * PC;
    if (p.tile_live) hipLaunchKernelGGL(heads_dw_kernel<true>, dim3(cb + db), dim3(256), lds, s, p, cb);
    else hipLaunchKernelGGL(heads_dw_kernel<false>, dim3(cb + db), dim3(256), lds, s, p, cb);
    GRAFT_LAUNCH_CHECK();
    const MlpShape ds{DIN, DHID, DOUT, 2}, cs{CIN, CHID, COUT, 3};
    mlp_grad_reduce(ds, p.ws_d, db, out.dW, out.dB, false, s);
    mlp_grad_reduce(cs, p.ws_c, cb, out.cW, out.cB, false, s);
}

}  // namespace graft
