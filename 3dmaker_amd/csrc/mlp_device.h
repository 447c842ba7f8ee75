// Device building blocks of the fused MLP kernels (mlp.hip, nerf_fused.hip).
//
// Layout: activations travel as the B operand of v_mfma_f32_16x16x16f16 with
// samples along N and features along K.  The D layout of one 16x16 MFMA (lane
// l holds rows 4(l/16)..+3 of column l%16) is exactly the B layout of the next
// layer's K-block, so a 16-sample tile walks through every layer in
// registers; weights are the A operand, pre-swizzled into LDS once per block.
#pragma once

#include "common.h"
#include "hash_encode.h"
#include "mlp.h"

namespace graft {

__host__ __device__ inline int tiles16(int d) { return (d + 15) / 16; }

// Stages the fp16 weights of every layer into LDS as MFMA A-operand
// fragments, one quad of 4 halves per (layer, 16x16 block, lane):
//   forward     frag(l, mt, ks)[lane][j] = W_l[16 mt + lane%16][16 ks + 4 (lane/16) + j]
//   transposed fragT(l, mt, ks)[lane][j] = W_l[16 ks + 4 (lane/16) + j][16 mt + lane%16]
// Blocks are stored mt-major (ks fastest), layer after layer, with zeros
// outside the matrix.  Every thread issues the global loads of kStageBatch
// quads before it stores any, so a block waits about one memory latency per
// batch instead of one per element.  Ends with a barrier.
constexpr int kStageBatch = 8;

template <bool TRANSPOSED>
__device__ void stage_fragments(_Float16* __restrict__ sfrag, const _Float16* const* W, int in, int hid, int out,
                                int layers)
{
    __shared__ const _Float16* sW[kMaxLayers];
    const int tid = threadIdx.x;
    __syncthreads();  // sW may still be read by an earlier call
    if (tid < layers) sW[tid] = W[tid];
    __syncthreads();
    auto quads = [&](int l) {
        const int in_l = l == 0 ? in : hid, out_l = l == layers - 1 ? out : hid;
        return tiles16(out_l) * tiles16(in_l) * 64;
    };
    int total = 0;
    for (int l = 0; l < layers; l++) total += quads(l);
    for (int base = 0; base < total; base += kStageBatch * (int)blockDim.x) {
        h4 v[kStageBatch];
#pragma unroll
        for (int k = 0; k < kStageBatch; k++) {
            const int q = base + k * (int)blockDim.x + tid;
            v[k] = h4zero();
            if (q >= total) continue;
            int l = 0, q0 = 0;
            while (q >= q0 + quads(l)) q0 += quads(l++);
            const int in_l = l == 0 ? in : hid, out_l = l == layers - 1 ? out : hid;
            const int f = (q - q0) >> 6, ln = (q - q0) & 63;
            const _Float16* w = sW[l];
            // in_l and out_l are multiples of 4: a quad is wholly inside or outside
            if constexpr (!TRANSPOSED) {
                const int KS = tiles16(in_l), mt = f / KS, ks = f - mt * KS;
                const int row = 16 * mt + (ln & 15), col = 16 * ks + 4 * (ln >> 4);
                if (row < out_l && col < in_l) {
                    const _Float16* src = w + row * in_l + col;
                    if ((reinterpret_cast<uintptr_t>(src) & 7u) == 0) v[k] = ld_h4(src);
                    else v[k] = h4{src[0], src[1], src[2], src[3]};
                }
            } else {
                const int KS = tiles16(out_l), mt = f / KS, ks = f - mt * KS;
                const int i = 16 * mt + (ln & 15), o = 16 * ks + 4 * (ln >> 4);
                if (i < in_l && o < out_l)
                    v[k] = h4{w[o * in_l + i], w[(o + 1) * in_l + i], w[(o + 2) * in_l + i], w[(o + 3) * in_l + i]};
            }
        }
#pragma unroll
        for (int k = 0; k < kStageBatch; k++) {
            const int q = base + k * (int)blockDim.x + tid;
            if (q < total) st_h4(sfrag + 4 * q, v[k]);
        }
    }
    __syncthreads();
}

// Biases of every layer, zero-padded to whole 16-blocks, at bias_off[l]
// floats.  The caller synchronises before use.
__device__ __forceinline__ void stage_biases(float* __restrict__ sbias, const float* const* B, const int* bias_off,
                                             int hid, int out, int layers)
{
    for (int l = 0; l < layers; l++) {
        const int out_l = l == layers - 1 ? out : hid;
        for (int e = threadIdx.x; e < tiles16(out_l) * 16; e += blockDim.x)
            sbias[bias_off[l] + e] = e < out_l ? B[l][e] : 0.f;
    }
}

// Compile-time layer shapes of a net whose widths are all <= 64 (at most four
// 16-wide blocks per layer): ib/ob = input/output blocks of layer l.
template <int IN, int HID, int OUT, int LAYERS>
struct HeadShape {
    static constexpr int in_l(int l) { return l == 0 ? IN : HID; }
    static constexpr int out_l(int l) { return l == LAYERS - 1 ? OUT : HID; }
    static constexpr int ib(int l) { return (in_l(l) + 15) / 16; }
    static constexpr int ob(int l) { return (out_l(l) + 15) / 16; }
    static constexpr int acc_off(int l) { return l == 0 ? 0 : acc_off(l - 1) + ob(l - 1) * ib(l - 1); }
    static constexpr int nacc() { return acc_off(LAYERS - 1) + ob(LAYERS - 1) * ib(LAYERS - 1); }
    static constexpr int db_off(int l) { return l == 0 ? 0 : db_off(l - 1) + ob(l - 1); }
    static constexpr int ndb() { return db_off(LAYERS - 1) + ob(LAYERS - 1); }
};

// The dX chain of one 16-sample tile through a net whose transposed weight
// fragments are staged (stage_fragments<true>): G holds dL/dy of the last
// layer (S layout: lane (r, g) has features 4 g .. 4 g + 3 of K-block b of
// sample r); on return G holds dL/dx of layer 0's input.  Each layer's dX is
// rounded to fp16 and masked where that layer's input activation is <= 0
// (not at layer 0).  acts is the device array of per-layer activations.
template <int IN, int HID, int OUT, int LAYERS>
__device__ __forceinline__ void dx_chain(h4 (&G)[4], const _Float16* sfrag, const int* fragT_off,
                                         const _Float16* const* acts, int n, bool valid, int lane)
{
    using S = HeadShape<IN, HID, OUT, LAYERS>;
    const int g = lane >> 4;
#pragma unroll
    for (int l = LAYERS - 1; l >= 0; l--) {
        const int in_l = S::in_l(l);
        const _Float16* fr = sfrag + fragT_off[l] + lane * 4;
        h4 Gn[4];
#pragma unroll
        for (int ib = 0; ib < 4; ib++) {
            Gn[ib] = h4zero();
            if (ib >= S::ib(l)) continue;
            f4 d = f4zero();
#pragma unroll
            for (int ob = 0; ob < 4; ob++)
                if (ob < S::ob(l)) d = mfma16(*reinterpret_cast<const h4*>(fr + (ib * S::ob(l) + ob) * 256), G[ob], d);
            h4 h;
#pragma unroll
            for (int j = 0; j < 4; j++) h[j] = to_h(d[j]);
            if (l > 0) {
                const int col = 16 * ib + 4 * g;
                const h4 X = valid ? ld_h4(acts[l] + (size_t)n * in_l + col) : h4zero();
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (!((float)X[j] > 0.f)) h[j] = (_Float16)0.f;
            }
            Gn[ib] = h;
        }
#pragma unroll
        for (int b = 0; b < 4; b++) G[b] = Gn[b];
    }
}

// Per-block view of one staged network.
struct NetView {
    const _Float16* frag;  // staged A fragments (stage_fragments<false>)
    const float* bias;     // staged biases (stage_biases)
    const int* frag_off;   // per layer, halves
    const int* bias_off;   // per layer, floats
    int in, hid, out, layers;
};

// Row n of the layer-0 activation [N x in]: the lane's 4 features of K-block
// ks (2 when the row ends mid-quad).
__device__ __forceinline__ void store_act0(_Float16* act0, int in, int n, int ks, int g, h4 x)
{
    const int col = 16 * ks + 4 * g;
    _Float16* dst = act0 + (size_t)n * in + col;
    if (col + 4 <= in) st_h4(dst, x);
    else if (col + 2 <= in) *reinterpret_cast<h2*>(dst) = h2{x.x, x.y};
}

// Hash encode of one 16-sample tile straight into the layer-0 B operand:
// lane (r = sample, g) holds levels 8 ks + 2 g and 8 ks + 2 g + 1 of K-block
// ks.  act0 (nullable) receives the fp16 encoding [N x in].
template <int NT>
__device__ __forceinline__ void encode_tile(h4 (&X)[NT], float px, float py, float pz, const float* sscale,
                                            const int* sres, int L, int T, int dense_start, const _Float16* table,
                                            int in, _Float16* act0, int n, bool valid, int g)
{
    const uint32_t mask = (uint32_t)T - 1u;
    const int KS0 = tiles16(in);
#pragma unroll
    for (int ks = 0; ks < NT; ks++) {
        X[ks] = h4zero();
        if (ks < KS0) {
            const int la = 8 * ks + 2 * g, lb = la + 1;
            float2 ea = make_float2(0.f, 0.f), eb = make_float2(0.f, 0.f);
            if (valid && la < L)
                ea = encode_level(px, py, pz, sscale[la], sres[la], la < dense_start, mask, table + (size_t)la * T * 2);
            if (valid && lb < L)
                eb = encode_level(px, py, pz, sscale[lb], sres[lb], lb < dense_start, mask, table + (size_t)lb * T * 2);
            X[ks] = h4{to_h(ea.x), to_h(ea.y), to_h(eb.x), to_h(eb.y)};
            if (act0 != nullptr && valid) store_act0(act0, in, n, ks, g, X[ks]);
        }
    }
}

// The same operand from encodings stored level-major, enc[l][plane] feature
// pairs (hash_encode_planar): lane (r, g) loads levels 8 ks + 2 g and
// 8 ks + 2 g + 1 of its sample; the 16 lanes of a level read 64 contiguous
// bytes.  act0 (nullable) receives the row-major encoding as above.
template <int NT>
__device__ __forceinline__ void load_encoded_tile(h4 (&X)[NT], const _Float16* __restrict__ enc, int plane, int L,
                                                  int in, _Float16* act0, int n, bool valid, int g)
{
    const int KS0 = tiles16(in);
#pragma unroll
    for (int ks = 0; ks < NT; ks++) {
        X[ks] = h4zero();
        if (ks < KS0) {
            const int la = 8 * ks + 2 * g, lb = la + 1;
            h2 ea{(_Float16)0.f, (_Float16)0.f}, eb{(_Float16)0.f, (_Float16)0.f};
            if (valid && la < L) ea = *reinterpret_cast<const h2*>(enc + ((size_t)la * plane + n) * 2);
            if (valid && lb < L) eb = *reinterpret_cast<const h2*>(enc + ((size_t)lb * plane + n) * 2);
            X[ks] = h4{ea.x, ea.y, eb.x, eb.y};
            if (act0 != nullptr && valid) store_act0(act0, in, n, ks, g, X[ks]);
        }
    }
}

// One 16-sample tile through every layer of a staged network.  X is the
// layer-0 input (B layout); hidden activations are bias + ReLU rounded to
// fp16 and, when acts is set, saved to acts[l + 1][n][*] (acts is a device
// array of per-layer pointers).  The last layer's pre-activation (fp32,
// acc + bias) goes to emit(mt, y) for every output block mt, in D layout:
// lane (r, g) has columns 16 mt + 4 g + j of sample r.
template <int NT, typename Emit>
__device__ __forceinline__ void net_tile(h4 (&X)[NT], const NetView& v, _Float16* const* acts, int n, bool valid,
                                         int lane, Emit&& emit)
{
    const int g = lane >> 4;
    for (int l = 0; l < v.layers; l++) {
        const int in_l = l == 0 ? v.in : v.hid;
        const int out_l = l == v.layers - 1 ? v.out : v.hid;
        const int KS = tiles16(in_l), MT = tiles16(out_l);
        const _Float16* fr = v.frag + v.frag_off[l] + lane * 4;
        const float* bl = v.bias + v.bias_off[l];
        f4 acc[NT];
#pragma unroll
        for (int mt = 0; mt < NT; mt++) {
            acc[mt] = f4zero();
            if (mt < MT) {
#pragma unroll
                for (int ks = 0; ks < NT; ks++)
                    if (ks < KS) acc[mt] = mfma16(*reinterpret_cast<const h4*>(fr + (mt * KS + ks) * 256), X[ks], acc[mt]);
            }
        }
        if (l < v.layers - 1) {
            _Float16* act = acts != nullptr ? acts[l + 1] : nullptr;
#pragma unroll
            for (int mt = 0; mt < NT; mt++) {
                h4 h = h4zero();
                if (mt < MT) {
                    const f4 bv = *reinterpret_cast<const f4*>(bl + 16 * mt + 4 * g);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float x = acc[mt][j] + bv[j];
                        h[j] = to_h(x > 0.f ? x : 0.f);
                    }
                    const int col = 16 * mt + 4 * g;
                    if (act != nullptr && valid && col < out_l) st_h4(act + (size_t)n * out_l + col, h);
                }
                X[mt] = h;
            }
        } else {
#pragma unroll
            for (int mt = 0; mt < NT; mt++) {
                if (mt < MT) {
                    const f4 bv = *reinterpret_cast<const f4*>(bl + 16 * mt + 4 * g);
                    f4 y;
#pragma unroll
                    for (int j = 0; j < 4; j++) y[j] = acc[mt][j] + bv[j];
                    emit(mt, y);
                }
            }
        }
    }
}

}  // namespace graft
