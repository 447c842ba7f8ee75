// Fully-fused TinyMLP forward/backward for gfx950 (CDNA4), fp16 MFMA with fp32
// accumulation.
//
// Layout idea: activations travel as the B operand of v_mfma_f32_16x16x16f16
// with samples along N and features along K.  The D layout of one 16x16 MFMA
// (lane l holds rows 4*(l/16)..+3 of column l%16) is exactly the B layout of
// the next layer's K-block, so a 16-sample tile walks through every layer in
// registers: bias, ReLU and the fp16 rounding happen in place, and weights are
// the A operand, pre-swizzled into LDS once per block.
//
// Semantics follow the reference kernels:
//   forward  networkFusion.cu:197-355, networkFusionHashtable.cu:408-682
//   backward networkFusionBackward.cu:49-646,
//            networkFusionBackwardHashtable.cu:71-781 (COMPUTE_HASHGRAD = 0)
// Rounding points: hidden activations -> fp16 after bias+ReLU, the last layer
// stays fp32 (optional sigmoid); each dX -> fp16, then masked where the saved
// activation <= 0.  dW/db are fp32 sums.  Unlike the reference, dW/db are not
// fp32 atomics: every block writes a partial into a workspace and a second
// kernel reduces the partials in a fixed order (bitwise-repeatable grads).
#include "mlp.h"

#include "hash_encode.h"
#include "mlp_device.h"

#include <algorithm>
#include <vector>

namespace graft {

namespace {

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------

struct FwdParams {
    const float* pos;             // HASH: [N x pos_stride] positions
    const _Float16* table;        // HASH: [L][T][2]
    const _Float16* x;            // plain: [N x in]
    _Float16* const* acts;        // SAVE: device array of per-layer activations
    const _Float16* const* W;     // device array, W_l row-major [out_l][in_l]
    const float* const* B;        // device array, b_l [out_l]
    float* out;                   // [N x out]
    const uint32_t* d_n;          // nullable device-side sample count (<= N)
    int N, in, hid, out_dim, layers, pos_stride, save_x0;
    int frag_off[kMaxLayers];     // in halves
    int bias_off[kMaxLayers];     // in floats from bias_base
    int bias_base, meta_base;     // byte offsets into dynamic LDS
    int L, T, dense_start;
    float scale[kMaxLevels];
    int res[kMaxLevels];
};

template <int MAXD, bool HASH, bool SAVE, int OUT_ACT>
__global__ __launch_bounds__(256) void mlp_fwd_kernel(const FwdParams p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* sfrag = reinterpret_cast<_Float16*>(smem);
    float* sbias = reinterpret_cast<float*>(smem + p.bias_base);
    float* sscale = reinterpret_cast<float*>(smem + p.meta_base);
    int* sres = reinterpret_cast<int*>(smem + p.meta_base + 4 * kMaxLevels);
    const int tid = threadIdx.x;

    stage_biases(sbias, p.B, p.bias_off, p.hid, p.out_dim, p.layers);
    if constexpr (HASH) {
        for (int e = tid; e < p.L; e += blockDim.x) {
            sscale[e] = p.scale[e];
            sres[e] = p.res[e];
        }
    }
    stage_fragments<false>(sfrag, p.W, p.in, p.hid, p.out_dim, p.layers);
    const NetView net{sfrag, sbias, p.frag_off, p.bias_off, p.in, p.hid, p.out_dim, p.layers};

    constexpr int NT = MAXD / 16;
    const int lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int ntiles = (N + 15) >> 4;
    const int KS0 = tiles16(p.in);
    _Float16* act0 = nullptr;
    if constexpr (SAVE) act0 = p.acts[0];

    for (int tile = blockIdx.x * 4 + wave; tile < ntiles; tile += gridDim.x * 4) {
        const int n = tile * 16 + r;
        const bool valid = n < N;
        h4 X[NT];
        if constexpr (HASH) {
            float px = 0.f, py = 0.f, pz = 0.f;
            if (valid) {
                const float* pp = p.pos + (size_t)n * p.pos_stride;
                px = pp[0];
                py = pp[1];
                pz = pp[2];
            }
            encode_tile<NT>(X, px, py, pz, sscale, sres, p.L, p.T, p.dense_start, p.table, p.in, act0, n, valid, g);
        } else {
#pragma unroll
            for (int ks = 0; ks < NT; ks++) {
                const int col = 16 * ks + 4 * g;
                const bool in_range = valid && ks < KS0 && col < p.in;
                X[ks] = in_range ? ld_h4(p.x + (size_t)n * p.in + col) : h4zero();
                if (SAVE && in_range && p.save_x0) st_h4(act0 + (size_t)n * p.in + col, X[ks]);
            }
        }
        net_tile<NT>(X, net, SAVE ? p.acts : nullptr, n, valid, lane, [&](int mt, f4 y) {
            if (!valid) return;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int col = 16 * mt + 4 * g + j;
                float v = y[j];
                if (OUT_ACT == 1) v = 1.0f / (1.0f + expf(-v));
                if (col < p.out_dim) p.out[(size_t)n * p.out_dim + col] = v;
            }
        });
    }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------

constexpr int kBwdTilesPerWave = 2;                   // 16-sample tiles per wave per chunk
constexpr int kBwdChunk = 4 * 16 * kBwdTilesPerWave;  // samples per block-chunk
constexpr int kBwdPitch = kBwdChunk + 8;              // LDS row pitch (halves), +16 B against bank conflicts

struct BwdParams {
    const _Float16* dy;             // [N x out]
    const _Float16* const* acts;    // device array: acts[0] = layer-0 input, acts[l] = H_l
    const _Float16* const* W;       // device array
    float* ws;                      // [gridDim.x][P] partial dW (all layers) then db
    _Float16* dx;                   // nullable [N x in]
    const uint32_t* d_n;            // nullable device-side sample count (<= N)
    int N, in, hid, out_dim, layers;
    int fragT_off[kMaxLayers];      // halves
    int wofs[kMaxLayers], bofs[kMaxLayers];
    int P;
    int gt_base, xt_base, acc_base; // byte offsets into dynamic LDS
    int nchunks;
};

// LMAX > 0: at most LMAX layers and every wave keeps the dW tiles it owns
// (tile q of a layer belongs to wave q % 4 in every chunk) and one db per
// thread in registers; the LDS then holds only the weights and one chunk's
// transposed activations, so several blocks share a CU.  LMAX == 0: any
// depth, block partials accumulated in LDS.  Both add each chunk's sums in the
// same order, so their partials are bitwise equal.
template <int MAXD, int LMAX>
__global__ __launch_bounds__(256) void mlp_bwd_kernel(const BwdParams p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* sfrag = reinterpret_cast<_Float16*>(smem);
    _Float16* Gt = reinterpret_cast<_Float16*>(smem + p.gt_base);
    _Float16* Xt = reinterpret_cast<_Float16*>(smem + p.xt_base);
    float* sacc = reinterpret_cast<float*>(smem + p.acc_base);
    const int tid = threadIdx.x;

    // Transposed fragments for dX = W^T G
    if constexpr (LMAX == 0)
        for (int e = tid; e < p.P; e += blockDim.x) sacc[e] = 0.f;
    stage_fragments<true>(sfrag, p.W, p.in, p.hid, p.out_dim, p.layers);

    constexpr int NT = MAXD / 16;
    constexpr int TPW = kBwdTilesPerWave;
    constexpr int QW = (NT * NT + 3) / 4;  // dW tiles a wave owns per layer
    constexpr int LR = LMAX > 0 ? LMAX : 1;
    const int lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int nchunks = (N + kBwdChunk - 1) / kBwdChunk;
    f4 dwacc[LR][QW];
    float dbacc[LR];
#pragma unroll
    for (int a = 0; a < LR; a++) {
        dbacc[a] = 0.f;
#pragma unroll
        for (int k = 0; k < QW; k++) dwacc[a][k] = f4zero();
    }

    for (int chunk = blockIdx.x; chunk < nchunks; chunk += gridDim.x) {
        const int s0 = chunk * kBwdChunk;
        h4 G[TPW][NT];
        {
            const int KSo = tiles16(p.out_dim);
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const int n = s0 + (wave * TPW + t) * 16 + r;
#pragma unroll
                for (int ks = 0; ks < NT; ks++) {
                    const int col = 16 * ks + 4 * g;
                    G[t][ks] = (n < N && ks < KSo && col < p.out_dim)
                                   ? ld_h4(p.dy + (size_t)n * p.out_dim + col)
                                   : h4zero();
                }
            }
        }

        // One layer of the backward; dw/db: this wave's register accumulators
        // of layer l (LMAX > 0) or nullptr (LDS partials).
        auto layer = [&](int l, f4* dw, float* db) {
            const int in_l = l == 0 ? p.in : p.hid;
            const int out_l = l == p.layers - 1 ? p.out_dim : p.hid;
            const int KSo = tiles16(out_l), MTi = tiles16(in_l);
            const _Float16* xl = p.acts[l];

            // Layer input activations in B layout, and both operands of dW into LDS (feature-major).
            h4 X[TPW][NT];
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const int sl = (wave * TPW + t) * 16 + r;
                const int n = s0 + sl;
#pragma unroll
                for (int mt = 0; mt < NT; mt++) {
                    const int col = 16 * mt + 4 * g;
                    X[t][mt] = (n < N && mt < MTi && col < in_l) ? ld_h4(xl + (size_t)n * in_l + col) : h4zero();
                    if (mt < MTi) {
#pragma unroll
                        for (int j = 0; j < 4; j++) Xt[(col + j) * kBwdPitch + sl] = X[t][mt][j];
                    }
                }
#pragma unroll
                for (int ks = 0; ks < NT; ks++) {
                    if (ks < KSo) {
                        const int row = 16 * ks + 4 * g;
#pragma unroll
                        for (int j = 0; j < 4; j++) Gt[(row + j) * kBwdPitch + sl] = G[t][ks][j];
                    }
                }
            }

            // dX = W^T G, rounded to fp16, ReLU-masked by the saved activation.
            if (l > 0 || p.dx != nullptr) {
                const _Float16* fr = sfrag + p.fragT_off[l] + lane * 4;
#pragma unroll
                for (int t = 0; t < TPW; t++) {
                    const int n = s0 + (wave * TPW + t) * 16 + r;
                    h4 Gn[NT];
#pragma unroll
                    for (int mt = 0; mt < NT; mt++) {
                        Gn[mt] = h4zero();
                        if (mt < MTi) {
                            f4 acc = f4zero();
#pragma unroll
                            for (int ks = 0; ks < NT; ks++)
                                if (ks < KSo)
                                    acc = mfma16(*reinterpret_cast<const h4*>(fr + (mt * KSo + ks) * 256), G[t][ks], acc);
                            h4 h;
#pragma unroll
                            for (int j = 0; j < 4; j++) h[j] = to_h(acc[j]);
                            if (l > 0) {
#pragma unroll
                                for (int j = 0; j < 4; j++)
                                    if (!((float)X[t][mt][j] > 0.f)) h[j] = (_Float16)0.f;
                            } else {
                                const int col = 16 * mt + 4 * g;
                                if (n < N && col < in_l) st_h4(p.dx + (size_t)n * in_l + col, h);
                            }
                            Gn[mt] = h;
                        }
                    }
#pragma unroll
                    for (int mt = 0; mt < NT; mt++) G[t][mt] = Gn[mt];
                }
            }
            __syncthreads();

            // dW_l[o][i] += sum_s Gt[o][s] * Xt[i][s]; tile q = (mo, mi) belongs to wave q % 4.
            const int ntile = KSo * MTi;
#pragma unroll
            for (int k = 0; k < QW; k++) {
                const int q = wave + 4 * k;
                if (q < ntile) {
                    const int mo = q / MTi, mi = q - mo * MTi;
                    const _Float16* ga = Gt + (16 * mo + r) * kBwdPitch + 4 * g;
                    const _Float16* xb = Xt + (16 * mi + r) * kBwdPitch + 4 * g;
                    f4 acc = f4zero();
#pragma unroll
                    for (int kk = 0; kk < kBwdChunk / 16; kk++)
                        acc = mfma16(*reinterpret_cast<const h4*>(ga + 16 * kk),
                                     *reinterpret_cast<const h4*>(xb + 16 * kk), acc);
                    if (dw) {
#pragma unroll
                        for (int j = 0; j < 4; j++) dw[k][j] += acc[j];
                    } else {
                        const int i = 16 * mi + r;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int o = 16 * mo + 4 * g + j;
                            if (o < out_l && i < in_l) sacc[p.wofs[l] + o * in_l + i] += acc[j];
                        }
                    }
                }
            }
            // db_l[o] += sum_s Gt[o][s] (fp32 sum of fp16 values), o = tid
            for (int o = tid; o < out_l; o += blockDim.x) {
                const _Float16* row = Gt + o * kBwdPitch;
                float s = 0.f;
                for (int k = 0; k < kBwdChunk; k += 4) {
                    const h4 v = *reinterpret_cast<const h4*>(row + k);
                    s += ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
                }
                if (db) *db += s;
                else sacc[p.bofs[l] + o] += s;
            }
            __syncthreads();
        };

        if constexpr (LMAX > 0) {
#pragma unroll
            for (int l = LMAX - 1; l >= 0; l--)
                if (l < p.layers) layer(l, dwacc[l], &dbacc[l]);
        } else {
            for (int l = p.layers - 1; l >= 0; l--) layer(l, nullptr, nullptr);
        }
    }

    float* dst = p.ws + (size_t)blockIdx.x * p.P;
    if constexpr (LMAX > 0) {
#pragma unroll
        for (int l = 0; l < LMAX; l++) {
            if (l >= p.layers) continue;
            const int in_l = l == 0 ? p.in : p.hid;
            const int out_l = l == p.layers - 1 ? p.out_dim : p.hid;
            const int MTi = tiles16(in_l), ntile = tiles16(out_l) * MTi;
#pragma unroll
            for (int k = 0; k < QW; k++) {
                const int q = wave + 4 * k;
                if (q >= ntile) continue;
                const int mo = q / MTi, mi = q - mo * MTi, i = 16 * mi + r;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int o = 16 * mo + 4 * g + j;
                    if (o < out_l && i < in_l) dst[p.wofs[l] + o * in_l + i] = dwacc[l][k][j];
                }
            }
            if (tid < out_l) dst[p.bofs[l] + tid] = dbacc[l];
        }
    } else {
        for (int e = tid; e < p.P; e += blockDim.x) dst[e] = sacc[e];
    }
}

// ---------------------------------------------------------------------------
// backward for the NeRF head shapes, all in registers
// ---------------------------------------------------------------------------
//
// dW = sum_s G[o][s] X[i][s] needs both operands with the sample index along
// K, while the MFMA chain of the layers holds every 16-sample tile with the
// sample along N ("S layout": lane l has features 4(l/16)..+3 of sample l%16).
// One MFMA against the identity, D = T * I, moves a 16x16 tile from A layout
// to D layout, which for these tiles is exactly S -> "F layout" (lane l has
// feature l%16 of samples 4(l/16)..+3); it is exact for every finite fp16
// (a -0 becomes +0, which no sum or mask here can see).  A tile holding inf or
// NaN would spread it through the 0 * x products, so such a tile is moved with
// lane shuffles instead.  Each wave then runs its tiles layer by layer with no
// LDS traffic but the weights, keeps its dW/db in registers, and the four waves
// of a block add their partials in a fixed order at the end.

__device__ __forceinline__ h4 ident_h4(int lane)
{
    const int g = lane >> 4, r = lane & 15;
    h4 v;
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = (4 * g + j == r) ? (_Float16)1.0f : (_Float16)0.0f;
    return v;
}

__device__ __forceinline__ bool h4_nonfinite(h4 v)
{
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; j++) bad |= (__builtin_bit_cast(uint16_t, v[j]) & 0x7c00u) == 0x7c00u;
    return bad;
}

// S layout -> F layout of one 16x16 tile.
__device__ __forceinline__ h4 tile_transpose(h4 v, h4 id, bool exact_slow, int lane)
{
    if (!exact_slow) {
        const f4 d = mfma16(v, id, f4zero());
        return h4{(_Float16)d[0], (_Float16)d[1], (_Float16)d[2], (_Float16)d[3]};
    }
    // element (row 4g + j, col r) lives in lane (4g + j) + 16 (r / 4), component r % 4
    const int g = lane >> 4, r = lane & 15;
    const uint32_t w0 = __builtin_bit_cast(uint32_t, h2{v[0], v[1]});
    const uint32_t w1 = __builtin_bit_cast(uint32_t, h2{v[2], v[3]});
    h4 out;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int src = 4 * g + j + 16 * (r >> 2);
        const uint32_t a = (uint32_t)__shfl((int)w0, src, 64), b = (uint32_t)__shfl((int)w1, src, 64);
        const uint32_t w = (r & 2) ? b : a;
        out[j] = __builtin_bit_cast(_Float16, (uint16_t)((r & 1) ? (w >> 16) : (w & 0xffffu)));
    }
    return out;
}


template <int IN, int HID, int OUT, int LAYERS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mlp_bwd_head_kernel(const BwdParams p)
{
    using S = HeadShape<IN, HID, OUT, LAYERS>;
    constexpr int MB = 4;  // max 16-wide blocks per layer (width <= 64)
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* sfrag = reinterpret_cast<_Float16*>(smem);
    float* sred = reinterpret_cast<float*>(smem + p.acc_base);  // [P] block partial
    const int tid = threadIdx.x;

    // Transposed fragments for dX = W^T G (as mlp_bwd_kernel).
    stage_fragments<true>(sfrag, p.W, IN, HID, OUT, LAYERS);

    const int lane = tid & 63, wave = tid >> 6, g = lane >> 4, r = lane & 15;
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int ntiles = (N + 15) >> 4;
    const h4 id = ident_h4(lane);
    f4 acc[S::nacc()];
    float dbs[S::ndb()];
#pragma unroll
    for (int a = 0; a < S::nacc(); a++) acc[a] = f4zero();
#pragma unroll
    for (int a = 0; a < S::ndb(); a++) dbs[a] = 0.f;

    for (int tile = blockIdx.x * 4 + wave; tile < ntiles; tile += gridDim.x * 4) {
        const int n = tile * 16 + r;
        const bool valid = n < N;
        h4 G[MB];
#pragma unroll
        for (int ob = 0; ob < MB; ob++) {
            const int col = 16 * ob + 4 * g;
            G[ob] = (ob < S::ob(LAYERS - 1) && valid && col < OUT) ? ld_h4(p.dy + (size_t)n * OUT + col) : h4zero();
        }
#pragma unroll
        for (int l = LAYERS - 1; l >= 0; l--) {
            const int in_l = S::in_l(l);
            h4 X[MB];
#pragma unroll
            for (int ib = 0; ib < MB; ib++) {
                const int col = 16 * ib + 4 * g;
                X[ib] = (ib < S::ib(l) && valid) ? ld_h4(p.acts[l] + (size_t)n * in_l + col) : h4zero();
            }
            // exact-slow transposes only for a tile holding inf / NaN
            bool bad = false;
#pragma unroll
            for (int b = 0; b < MB; b++) bad |= h4_nonfinite(G[b]) | h4_nonfinite(X[b]);
            const bool slow = __ballot(bad) != 0;
            h4 GF[MB], XF[MB];
#pragma unroll
            for (int ob = 0; ob < MB; ob++)
                if (ob < S::ob(l)) GF[ob] = tile_transpose(G[ob], id, slow, lane);
#pragma unroll
            for (int ib = 0; ib < MB; ib++)
                if (ib < S::ib(l)) XF[ib] = tile_transpose(X[ib], id, slow, lane);
            // dW[o][i] += G_F(o) X_F(i); db[o] += sum of this lane's 4 samples
#pragma unroll
            for (int ob = 0; ob < MB; ob++) {
                if (ob >= S::ob(l)) continue;
#pragma unroll
                for (int ib = 0; ib < MB; ib++)
                    if (ib < S::ib(l)) {
                        f4& a = acc[S::acc_off(l) + ob * S::ib(l) + ib];
                        a = mfma16(GF[ob], XF[ib], a);
                    }
                const h4 v = GF[ob];
                dbs[S::db_off(l) + ob] += ((float)v[0] + (float)v[1]) + ((float)v[2] + (float)v[3]);
            }
            // dX = W^T G, rounded to fp16, ReLU-masked by this layer's input
            if (l > 0 || p.dx != nullptr) {
                const _Float16* fr = sfrag + p.fragT_off[l] + lane * 4;
                h4 Gn[MB];
#pragma unroll
                for (int ib = 0; ib < MB; ib++) {
                    Gn[ib] = h4zero();
                    if (ib >= S::ib(l)) continue;
                    f4 d = f4zero();
#pragma unroll
                    for (int ob = 0; ob < MB; ob++)
                        if (ob < S::ob(l))
                            d = mfma16(*reinterpret_cast<const h4*>(fr + (ib * S::ob(l) + ob) * 256), G[ob], d);
                    h4 h;
#pragma unroll
                    for (int j = 0; j < 4; j++) h[j] = to_h(d[j]);
                    if (l > 0) {
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            if (!((float)X[ib][j] > 0.f)) h[j] = (_Float16)0.f;
                    } else {
                        const int col = 16 * ib + 4 * g;
                        if (valid && col < IN) st_h4(p.dx + (size_t)n * IN + col, h);
                    }
                    Gn[ib] = h;
                }
#pragma unroll
                for (int b = 0; b < MB; b++) G[b] = Gn[b];
            }
        }
    }

    // db: the 4 lanes of a feature (g = 0..3) in a fixed order
#pragma unroll
    for (int a = 0; a < S::ndb(); a++) {
        const float v0 = __shfl(dbs[a], r, 64), v1 = __shfl(dbs[a], r + 16, 64);
        const float v2 = __shfl(dbs[a], r + 32, 64), v3 = __shfl(dbs[a], r + 48, 64);
        dbs[a] = (v0 + v1) + (v2 + v3);
    }
    // block partial: wave 0 writes, waves 1..3 add in order
    for (int w = 0; w < 4; w++) {
        if (wave == w) {
#pragma unroll
            for (int l = 0; l < LAYERS; l++) {
                const int in_l = S::in_l(l), out_l = S::out_l(l);
#pragma unroll
                for (int ob = 0; ob < MB; ob++) {
                    if (ob >= S::ob(l)) continue;
#pragma unroll
                    for (int ib = 0; ib < MB; ib++) {
                        if (ib >= S::ib(l)) continue;
                        const f4 a = acc[S::acc_off(l) + ob * S::ib(l) + ib];
                        const int i = 16 * ib + r;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int o = 16 * ob + 4 * g + j;
                            if (o < out_l && i < in_l) {
                                float* dst = sred + p.wofs[l] + o * in_l + i;
                                *dst = (w == 0) ? a[j] : *dst + a[j];
                            }
                        }
                    }
                    const int o = 16 * ob + r;
                    if (g == 0 && o < out_l) {
                        float* dst = sred + p.bofs[l] + o;
                        *dst = (w == 0) ? dbs[S::db_off(l) + ob] : *dst + dbs[S::db_off(l) + ob];
                    }
                }
            }
        }
        __syncthreads();
    }
    float* dstp = p.ws + (size_t)blockIdx.x * p.P;
    for (int e = tid; e < p.P; e += blockDim.x) dstp[e] = sred[e];
}

// dL/dx alone (no dW/db) for the NeRF head shapes: the same chain of MFMAs
// as mlp_bwd_head_kernel's dX in the same order, so the result is bitwise its
// dx.  A caller that needs dx first (the hash scatter waits for it) runs this,
// and the weight gradients later with mlp_backward(dx = nullptr), which
// recomputes the chain beside other work.
template <int IN, int HID, int OUT, int LAYERS>
__global__ __launch_bounds__(256) void mlp_bwd_dx_kernel(const BwdParams p)
{
    using S = HeadShape<IN, HID, OUT, LAYERS>;
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* sfrag = reinterpret_cast<_Float16*>(smem);
    stage_fragments<true>(sfrag, p.W, IN, HID, OUT, LAYERS);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, r = lane & 15;
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int ntiles = (N + 15) >> 4;
    for (int tile = blockIdx.x * 4 + wave; tile < ntiles; tile += gridDim.x * 4) {
        const int n = tile * 16 + r;
        const bool valid = n < N;
        h4 G[4];
#pragma unroll
        for (int ob = 0; ob < 4; ob++) {
            const int col = 16 * ob + 4 * g;
            G[ob] = (ob < S::ob(LAYERS - 1) && valid && col < OUT) ? ld_h4(p.dy + (size_t)n * OUT + col) : h4zero();
        }
        dx_chain<IN, HID, OUT, LAYERS>(G, sfrag, p.fragT_off, p.acts, n, valid, lane);
#pragma unroll
        for (int ib = 0; ib < S::ib(0); ib++) {
            const int col = 16 * ib + 4 * g;
            if (valid && col < IN) st_h4(p.dx + (size_t)n * IN + col, G[ib]);
        }
    }
}

// grad[p] += sum over blocks of ws[b][p], summed in block order.
struct ReduceParams {
    const float* ws;
    float* const* dW;
    float* const* dB;
    int nparts, P, layers, wtot, accumulate;
    int wofs[kMaxLayers], bofs[kMaxLayers];
};

// 64 parameters x 16 row groups per 1024-thread block: group q sums partial
// rows q, q + 16, ... (eight independent loads in flight per thread), then the
// 16 group sums are added in a fixed tree, so the result is bitwise
// repeatable.  accumulate = 0 stores the sum (the gradients need no zeroing).
__global__ __launch_bounds__(1024) void mlp_grad_reduce_kernel(const ReduceParams p)
{
    constexpr int kGroups = 16;
    __shared__ float part[kGroups][64];
    const int pl = threadIdx.x & 63, grp = threadIdx.x >> 6;
    const int idx = blockIdx.x * 64 + pl;
    float s = 0.f;
    if (idx < p.P) {
        const float* src = p.ws + idx;
        int b = grp;
        for (; b + 7 * kGroups < p.nparts; b += 8 * kGroups) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = src[(size_t)(b + u * kGroups) * p.P];
#pragma unroll
            for (int u = 0; u < 8; u++) s += v[u];
        }
        for (; b < p.nparts; b += kGroups) s += src[(size_t)b * p.P];
    }
    part[grp][pl] = s;
    __syncthreads();
#pragma unroll
    for (int h = kGroups / 2; h > 0; h >>= 1) {
        if (grp < h) part[grp][pl] += part[grp + h][pl];
        __syncthreads();
    }
    if (grp == 0 && idx < p.P) {
        const float tot = part[0][pl];
        float* dst;
        if (idx < p.wtot) {
            int l = 0;
            while (l + 1 < p.layers && idx >= p.wofs[l + 1]) l++;
            dst = p.dW[l] + (idx - p.wofs[l]);
        } else {
            const int k = idx - p.wtot;
            int l = 0;
            while (l + 1 < p.layers && k >= p.bofs[l + 1] - p.wtot) l++;
            dst = p.dB[l] + (k - (p.bofs[l] - p.wtot));
        }
        *dst = p.accumulate ? *dst + tot : tot;
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

void MlpShape::validate() const
{
    if (layers < 1 || layers > kMaxLayers)
        throw std::runtime_error("TinyMLP: numLayers must be in [1, " + std::to_string(kMaxLayers) + "]");
    if (in < 1 || hid < 1 || out < 1)
        throw std::runtime_error("TinyMLP: dimensions must be positive");
    if (in % 4 || hid % 4 || out % 4)
        throw std::runtime_error("TinyMLP: in/hidden/out dims must be multiples of 4");
    if (maxd() > 128) throw std::runtime_error("TinyMLP: max(in, hidden, out) must be <= 128");
}

static int pick_maxd(int d)
{
    if (d <= 16) return 16;
    if (d <= 32) return 32;
    if (d <= 64) return 64;
    return 128;
}

static void fill_layer_offsets(const MlpShape& s, bool transposed, int* frag_off, int* bias_off,
                               int& frag_halves, int& bias_floats)
{
    frag_halves = 0;
    bias_floats = 0;
    for (int l = 0; l < s.layers; l++) {
        const int a = tiles16(s.out_l(l)), b = tiles16(s.in_l(l));
        frag_off[l] = frag_halves;
        frag_halves += a * b * 256;
        (void)transposed;
        if (bias_off) {
            bias_off[l] = bias_floats;
            bias_floats += a * 16;
        }
    }
}


void mlp_forward(const MlpShape& s, const FwdInput& in, const __half* const* W,
                 const float* const* B, __half* const* acts, float* out, int N, int out_act,
                 hipStream_t stream, const uint32_t* d_n)
{
    s.validate();
    if (N <= 0) return;
    FwdParams p{};
    p.pos = in.pos;
    p.pos_stride = in.pos_stride;
    p.table = reinterpret_cast<const _Float16*>(in.table);
    p.x = reinterpret_cast<const _Float16*>(in.x);
    p.acts = reinterpret_cast<_Float16* const*>(acts);
    p.W = reinterpret_cast<const _Float16* const*>(W);
    p.B = B;
    p.out = out;
    p.d_n = d_n;
    p.N = N;
    p.in = s.in;
    p.hid = s.hid;
    p.out_dim = s.out;
    p.layers = s.layers;
    p.save_x0 = in.save_x0 ? 1 : 0;
    int frag_halves = 0, bias_floats = 0;
    fill_layer_offsets(s, false, p.frag_off, p.bias_off, frag_halves, bias_floats);
    p.bias_base = (frag_halves * 2 + 15) & ~15;
    p.meta_base = (p.bias_base + bias_floats * 4 + 15) & ~15;
    const bool hash = in.table != nullptr;
    int lds = p.meta_base + (hash ? 8 * kMaxLevels : 0);
    if (lds > max_lds_per_block()) throw std::runtime_error("TinyMLP: network too large for the fused kernel LDS budget");
    if (hash) {
        const GridMeta& m = *in.meta;
        p.L = m.numLevels;
        p.T = m.tableSize;
        p.dense_start = m.denseLevelStart;
        for (int l = 0; l < m.numLevels; l++) {
            p.scale[l] = m.scale[l];
            p.res[l] = m.res[l];
        }
        if (2 * p.L != s.in) throw std::runtime_error("TinyMLPHashGrid: inputDim must equal 2 * numLevels");
    }
    const bool save = acts != nullptr;
    const int ntiles = (N + 15) / 16;
    const int blocks = std::max(1, std::min((ntiles + 3) / 4, num_cus() * 8));
    const int maxd = pick_maxd(s.maxd());

#define GRAFT_FWD_LAUNCH(MD)                                                                       \
    do {                                                                                           \
        if (hash) {                                                                                \
            if (save) hipLaunchKernelGGL((mlp_fwd_kernel<MD, true, true, 0>), dim3(blocks), dim3(256), lds, stream, p); \
            else hipLaunchKernelGGL((mlp_fwd_kernel<MD, true, false, 0>), dim3(blocks), dim3(256), lds, stream, p);     \
        } else if (out_act == 1) {                                                                 \
            if (save) hipLaunchKernelGGL((mlp_fwd_kernel<MD, false, true, 1>), dim3(blocks), dim3(256), lds, stream, p); \
            else hipLaunchKernelGGL((mlp_fwd_kernel<MD, false, false, 1>), dim3(blocks), dim3(256), lds, stream, p);     \
        } else {                                                                                   \
            if (save) hipLaunchKernelGGL((mlp_fwd_kernel<MD, false, true, 0>), dim3(blocks), dim3(256), lds, stream, p); \
            else hipLaunchKernelGGL((mlp_fwd_kernel<MD, false, false, 0>), dim3(blocks), dim3(256), lds, stream, p);     \
        }                                                                                          \
    } while (0)

    switch (maxd) {
        case 16: GRAFT_FWD_LAUNCH(16); break;
        case 32: GRAFT_FWD_LAUNCH(32); break;
        case 64: GRAFT_FWD_LAUNCH(64); break;
        default: GRAFT_FWD_LAUNCH(128); break;
    }
#undef GRAFT_FWD_LAUNCH
    GRAFT_LAUNCH_CHECK();
}

bool mlp_has_dx_kernel(const MlpShape& s)
{
    return s.in == 32 && s.hid == 64 && (s.out == 16 && s.layers == 2 || s.out == 8 && s.layers == 3);
}

bool mlp_backward_dx(const MlpShape& s, const __half* dy, const __half* const* acts, const __half* const* W,
                     __half* dx, int N, hipStream_t stream, const uint32_t* d_n)
{
    s.validate();
    if (!mlp_has_dx_kernel(s)) return false;
    const bool density_head = s.out == 16;
    if (dx == nullptr) throw std::runtime_error("TinyMLP: dX-only backward needs dx");
    if (N <= 0) return true;
    BwdParams p{};
    p.dy = reinterpret_cast<const _Float16*>(dy);
    p.acts = reinterpret_cast<const _Float16* const*>(acts);
    p.W = reinterpret_cast<const _Float16* const*>(W);
    p.dx = reinterpret_cast<_Float16*>(dx);
    p.d_n = d_n;
    p.N = N;
    p.in = s.in;
    p.hid = s.hid;
    p.out_dim = s.out;
    p.layers = s.layers;
    int frag_halves = 0, unused = 0;
    fill_layer_offsets(s, true, p.fragT_off, nullptr, frag_halves, unused);
    const int lds = frag_halves * 2;
    const auto kern = density_head ? mlp_bwd_dx_kernel<32, 64, 16, 2> : mlp_bwd_dx_kernel<32, 64, 8, 3>;
    int per_cu = 0;
    GRAFT_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds));
    const int ntiles = (N + 15) / 16;
    const int blocks = std::max(1, std::min((ntiles + 3) / 4, num_cus() * std::max(1, per_cu)));
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, stream, p);
    GRAFT_LAUNCH_CHECK();
    return true;
}

void mlp_backward(const MlpShape& s, const __half* dy, const __half* const* acts,
                  const __half* const* W, float* const* dW, float* const* dB, __half* dx, int N,
                  hipStream_t stream, const uint32_t* d_n, bool accumulate, Workspace* ws)
{
    s.validate();
    if (N <= 0) return;
    BwdParams p{};
    p.dy = reinterpret_cast<const _Float16*>(dy);
    p.acts = reinterpret_cast<const _Float16* const*>(acts);
    p.W = reinterpret_cast<const _Float16* const*>(W);
    p.dx = reinterpret_cast<_Float16*>(dx);
    p.d_n = d_n;
    p.N = N;
    p.in = s.in;
    p.hid = s.hid;
    p.out_dim = s.out;
    p.layers = s.layers;
    int frag_halves = 0, unused = 0;
    fill_layer_offsets(s, true, p.fragT_off, nullptr, frag_halves, unused);
    int wtot = 0;
    for (int l = 0; l < s.layers; l++) {
        p.wofs[l] = wtot;
        wtot += s.in_l(l) * s.out_l(l);
    }
    int btot = wtot;
    for (int l = 0; l < s.layers; l++) {
        p.bofs[l] = btot;
        btot += s.out_l(l);
    }
    p.P = btot;
    const int maxd = pick_maxd(s.maxd());
    // the two NeRF heads: registers only, transposes on the MFMA unit
    const bool density_head = s.in == 32 && s.hid == 64 && s.out == 16 && s.layers == 2;
    const bool color_head = s.in == 32 && s.hid == 64 && s.out == 8 && s.layers == 3;
    if (density_head || color_head) {
        p.acc_base = (frag_halves * 2 + 15) & ~15;
        const int lds = p.acc_base + p.P * 4;
        if (lds > max_lds_per_block()) throw std::runtime_error("TinyMLP: backward LDS budget");
        const int ntiles = (N + 15) / 16;
        const auto kern = density_head ? mlp_bwd_head_kernel<32, 64, 16, 2> : mlp_bwd_head_kernel<32, 64, 8, 3>;
        // one block per resident slot: the grid-stride split then ends in a
        // single wave of blocks (a second, partial wave would run alone)
        int per_cu = 0;
        GRAFT_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds));
        const int blocks = std::max(1, std::min((ntiles + 3) / 4, num_cus() * std::max(1, per_cu)));
        p.ws = static_cast<float*>((ws ? *ws : stream_workspace(stream)).get((size_t)blocks * p.P * sizeof(float)));
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, stream, p);
        GRAFT_LAUNCH_CHECK();
        ReduceParams rp{};
        rp.ws = p.ws;
        rp.dW = dW;
        rp.dB = dB;
        rp.nparts = blocks;
        rp.P = p.P;
        rp.layers = s.layers;
        rp.wtot = wtot;
        rp.accumulate = accumulate ? 1 : 0;
        for (int l = 0; l < s.layers; l++) {
            rp.wofs[l] = p.wofs[l];
            rp.bofs[l] = p.bofs[l];
        }
        hipLaunchKernelGGL(mlp_grad_reduce_kernel, dim3((p.P + 63) / 64), dim3(1024), 0, stream, rp);
        GRAFT_LAUNCH_CHECK();
        return;
    }
    // register accumulators for nets of up to 4 layers of width <= 64
    const bool reg = maxd <= 64 && s.layers <= 4;
    p.gt_base = (frag_halves * 2 + 15) & ~15;
    p.xt_base = p.gt_base + maxd * kBwdPitch * 2;
    p.acc_base = p.xt_base + maxd * kBwdPitch * 2;
    const int lds = p.acc_base + (reg ? 0 : p.P * 4);
    if (lds > max_lds_per_block()) throw std::runtime_error("TinyMLP: network too large for the fused backward LDS budget");
    p.nchunks = (N + kBwdChunk - 1) / kBwdChunk;
    const int per_cu = reg ? std::max(1, std::min(4, max_lds_per_block() / std::max(lds, 1))) : 2;
    const int blocks = std::max(1, std::min(p.nchunks, num_cus() * per_cu));
    p.ws = static_cast<float*>((ws ? *ws : stream_workspace(stream)).get((size_t)blocks * p.P * sizeof(float)));

    if (reg) {
        switch (maxd) {
            case 16: hipLaunchKernelGGL((mlp_bwd_kernel<16, 4>), dim3(blocks), dim3(256), lds, stream, p); break;
            case 32: hipLaunchKernelGGL((mlp_bwd_kernel<32, 4>), dim3(blocks), dim3(256), lds, stream, p); break;
            default: hipLaunchKernelGGL((mlp_bwd_kernel<64, 4>), dim3(blocks), dim3(256), lds, stream, p); break;
        }
    } else {
        switch (maxd) {
            case 16: hipLaunchKernelGGL((mlp_bwd_kernel<16, 0>), dim3(blocks), dim3(256), lds, stream, p); break;
            case 32: hipLaunchKernelGGL((mlp_bwd_kernel<32, 0>), dim3(blocks), dim3(256), lds, stream, p); break;
            case 64: hipLaunchKernelGGL((mlp_bwd_kernel<64, 0>), dim3(blocks), dim3(256), lds, stream, p); break;
            default: hipLaunchKernelGGL((mlp_bwd_kernel<128, 0>), dim3(blocks), dim3(256), lds, stream, p); break;
        }
    }
    GRAFT_LAUNCH_CHECK();

    ReduceParams rp{};
    rp.ws = p.ws;
    rp.dW = dW;
    rp.dB = dB;
    rp.nparts = blocks;
    rp.P = p.P;
    rp.layers = s.layers;
    rp.wtot = wtot;
    rp.accumulate = accumulate ? 1 : 0;
    for (int l = 0; l < s.layers; l++) {
        rp.wofs[l] = p.wofs[l];
        rp.bofs[l] = p.bofs[l];
    }
    hipLaunchKernelGGL(mlp_grad_reduce_kernel, dim3((p.P + 63) / 64), dim3(1024), 0, stream, rp);
    GRAFT_LAUNCH_CHECK();
}

void mlp_grad_reduce(const MlpShape& s, const float* ws, int nparts, float* const* dW, float* const* dB,
                     bool accumulate, hipStream_t stream)
{
    s.validate();
    ReduceParams rp{};
    rp.ws = ws;
    rp.dW = dW;
    rp.dB = dB;
    rp.nparts = nparts;
    rp.layers = s.layers;
    rp.accumulate = accumulate ? 1 : 0;
    int tot = 0;
    for (int l = 0; l < s.layers; l++) {
        rp.wofs[l] = tot;
        tot += s.in_l(l) * s.out_l(l);
    }
    rp.wtot = tot;
    for (int l = 0; l < s.layers; l++) {
        rp.bofs[l] = tot;
        tot += s.out_l(l);
    }
    rp.P = tot;
    hipLaunchKernelGGL(mlp_grad_reduce_kernel, dim3((rp.P + 63) / 64), dim3(1024), 0, stream, rp);
    GRAFT_LAUNCH_CHECK();
}

}  // namespace graft
