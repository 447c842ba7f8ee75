// The two halves of a NeRF step that run per sample in one kernel each.
//
// Forward: hash encode + density MLP, SH gather, colour MLP, per 16-sample
// tile in registers.  The reference runs it as three launches with two HBM
// round trips (networkFusionHashtable.cu:441-682, compute_SH_gather
// otherKernels.cu:156-273, networkFusion.cu:197-355).  Here the density
// head's output block, already in the MFMA D layout that is the colour head's
// B layout for input features 0..15, is sanitised and rounded to fp16 in
// place; each lane adds the 4 SH coefficients of its sample it holds as
// features 16..31.  Every value is produced by the same fp32 operations in the
// same order as the three-launch chain, so the outputs are bitwise those of
// that chain.  The saved buffers (density output, sigma, both heads'
// activations) are the ones the backward reads; an inference caller passes
// nulls and keeps only sigma and the colour output.
//
// Backward, dX part: the colour head's dX chain, the density-gradient glue
// (compute_density_grad, otherKernels.cu:506-562) and the density head's dX
// chain, down to dL/d(encoding) for the hash scatter; bitwise the outputs of
// the dX-only head kernels and density_grad_kernel.  The weight gradients are
// computed apart (mlp_backward with dx = nullptr).
#include "hashgrid.h"
#include "mlp_device.h"
#include "nerf.h"
#include "nerf_heads.h"

#include <algorithm>

namespace graft {

namespace {

struct NerfFwdParams {
    const float* pos;
    const _Float16* table;
    const _Float16* enc;      // level-major encodings (PLANAR kernels)
    int plane;
    const _Float16* const* dW;
    const float* const* dB;
    _Float16* const* dacts;   // nullable
    float* dout;              // nullable [N x 16]
    const float3* dirs;
    const uint32_t* ray_idx;
    float* sigma;             // [N]
    const _Float16* const* cW;
    const float* const* cB;
    _Float16* const* cacts;   // nullable (hidden activations of the colour head)
    _Float16* cin;            // nullable [N x 32]
    float* cout;              // [N x c_out]
    const uint32_t* d_n;
    float density_bias;
    int N, pos_stride;
    int L, T, dense_start;
    int d_in, d_hid, d_layers;
    int c_hid, c_out, c_layers;
    int d_frag_off[kMaxLayers], d_bias_off[kMaxLayers];
    int c_frag_off[kMaxLayers], c_bias_off[kMaxLayers];
    int c_frag_base, d_bias_base, c_bias_base, meta_base;  // LDS byte offsets
    float scale[kMaxLevels];
    int res[kMaxLevels];
};

template <int NT, int OUT_ACT, bool PLANAR>
__global__ __launch_bounds__(256) void nerf_fwd_kernel(const NerfFwdParams p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* dfrag = reinterpret_cast<_Float16*>(smem);
    _Float16* cfrag = reinterpret_cast<_Float16*>(smem + p.c_frag_base);
    float* dbias = reinterpret_cast<float*>(smem + p.d_bias_base);
    float* cbias = reinterpret_cast<float*>(smem + p.c_bias_base);
    float* sscale = reinterpret_cast<float*>(smem + p.meta_base);
    int* sres = reinterpret_cast<int*>(smem + p.meta_base + 4 * kMaxLevels);
    const int tid = threadIdx.x;

    stage_biases(dbias, p.dB, p.d_bias_off, p.d_hid, 16, p.d_layers);
    stage_biases(cbias, p.cB, p.c_bias_off, p.c_hid, p.c_out, p.c_layers);
    for (int e = tid; e < p.L; e += blockDim.x) {
        sscale[e] = p.scale[e];
        sres[e] = p.res[e];
    }
    stage_fragments<false>(dfrag, p.dW, p.d_in, p.d_hid, 16, p.d_layers);
    stage_fragments<false>(cfrag, p.cW, 32, p.c_hid, p.c_out, p.c_layers);
    const NetView dnet{dfrag, dbias, p.d_frag_off, p.d_bias_off, p.d_in, p.d_hid, 16, p.d_layers};
    const NetView cnet{cfrag, cbias, p.c_frag_off, p.c_bias_off, 32, p.c_hid, p.c_out, p.c_layers};

    const int lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
    const int N = p.d_n ? min((int)*p.d_n, p.N) : p.N;
    const int ntiles = (N + 15) >> 4;
    _Float16* act0 = p.dacts != nullptr ? p.dacts[0] : nullptr;

    for (int tile = blockIdx.x * 4 + wave; tile < ntiles; tile += gridDim.x * 4) {
        const int n = tile * 16 + r;
        const bool valid = n < N;
        float3 dir = make_float3(0.f, 0.f, 0.f);
        if (valid) dir = p.dirs[p.ray_idx[n]];
        h4 X[NT];
        if constexpr (PLANAR) {
            load_encoded_tile<NT>(X, p.enc, p.plane, p.L, p.d_in, act0, n, valid, g);
        } else {
            float px = 0.f, py = 0.f, pz = 0.f;
            if (valid) {
                const float* pp = p.pos + (size_t)n * p.pos_stride;
                px = pp[0];
                py = pp[1];
                pz = pp[2];
            }
            encode_tile<NT>(X, px, py, pz, sscale, sres, p.L, p.T, p.dense_start, p.table, p.d_in, act0, n, valid, g);
        }

        // density head -> colour input features 0..15 (sanitised logits), sigma
        h4 C[NT];
#pragma unroll
        for (int k = 0; k < NT; k++) C[k] = h4zero();
        net_tile<NT>(X, dnet, p.dacts, n, valid, lane, [&](int mt, f4 y) {
            if (mt != 0) return;
            if (valid && p.dout != nullptr) *reinterpret_cast<f4*>(p.dout + (size_t)n * 16 + 4 * g) = y;
            float lg[4];
#pragma unroll
            for (int j = 0; j < 4; j++) lg[j] = sanitize_logit(y[j]);
            C[0] = h4{to_h(lg[0]), to_h(lg[1]), to_h(lg[2]), to_h(lg[3])};
            if (valid && g == 0) p.sigma[n] = nerf_expf(fminf(lg[0] - p.density_bias, 8.0f));
        });
        // features 16..31: SH coefficients 4 g .. 4 g + 3 of this lane's sample
        {
            float sh[16];
            sh_basis16(dir.x, dir.y, dir.z, sh);
            h4 s;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float v = g == 0 ? sh[j] : g == 1 ? sh[4 + j] : g == 2 ? sh[8 + j] : sh[12 + j];
                s[j] = to_h(v);
            }
            if constexpr (NT > 1) C[1] = s;
        }
        if (valid && p.cin != nullptr) {
            st_h4(p.cin + (size_t)n * 32 + 4 * g, C[0]);
            if constexpr (NT > 1) st_h4(p.cin + (size_t)n * 32 + 16 + 4 * g, C[1]);
        }

        // colour head
        net_tile<NT>(C, cnet, p.cacts, n, valid, lane, [&](int mt, f4 y) {
            const int col = 16 * mt + 4 * g;
            if (!valid || col >= p.c_out) return;
            f4 v = y;
            if (OUT_ACT == 1) {
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = 1.0f / (1.0f + expf(-v[j]));
            }
            *reinterpret_cast<f4*>(p.cout + (size_t)n * p.c_out + col) = v;
        });
    }
}

struct NerfBwdDxParams {
    const _Float16* cdy;              // [N x COUT] colour dL/dy (fp16)
    const _Float16* const* cacts;     // colour activations
    const _Float16* const* cW;
    const float* dsigma;              // [N]
    const _Float16* const* dacts;     // density activations
    const _Float16* const* dW;
    _Float16* cdx;                    // [N x 32] colour dL/dinput
    _Float16* dloss;                  // [N x 16] density dL/dy
    _Float16* denc;                   // [N x DIN] dL/d(encoding)
    const uint32_t* d_n;
    int N;
    int c_fragT_off[kMaxLayers], d_fragT_off[kMaxLayers];
    int d_frag_base;                  // LDS byte offset of the density fragments
};

template <int CIN, int CHID, int COUT, int CL, int DIN, int DHID, int DL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void nerf_bwd_dx_kernel(const NerfBwdDxParams p)
{
    using CS = HeadShape<CIN, CHID, COUT, CL>;
    using DS = HeadShape<DIN, DHID, 16, DL>;
    extern __shared__ __align__(16) unsigned char smem[];
    _Float16* cfrag = reinterpret_cast<_Float16*>(smem);
    _Float16* dfrag = reinterpret_cast<_Float16*>(smem + p.d_frag_base);
    stage_fragments<true>(cfrag, p.cW, CIN, CHID, COUT, CL);
    stage_fragments<true>(dfrag, p.dW, DIN, DHID, 16, DL);

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
            G[ob] = (ob < CS::ob(CL - 1) && valid && col < COUT) ? ld_h4(p.cdy + (size_t)n * COUT + col) : h4zero();
        }
        dx_chain<CIN, CHID, COUT, CL>(G, cfrag, p.c_fragT_off, p.cacts, n, valid, lane);
        if (valid) {
#pragma unroll
            for (int ib = 0; ib < CS::ib(0); ib++) st_h4(p.cdx + (size_t)n * CIN + 16 * ib + 4 * g, G[ib]);
        }
        // density dL/dy = colour dL/dinput[0..15] with d sigma added to the
        // logit, clamped to the fp16 range, NaN -> 0 (density_grad_kernel)
        h4 D;
        const float ds = (valid && g == 0) ? p.dsigma[n] : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float f = (float)G[0][j];
            if (g == 0 && j == 0) f += ds;
            f = clamp_half_range(f);
            if (f != f) f = 0.0f;
            D[j] = to_h(f);
        }
        if (valid) st_h4(p.dloss + (size_t)n * 16 + 4 * g, D);
        h4 E[4] = {D, h4zero(), h4zero(), h4zero()};
        dx_chain<DIN, DHID, 16, DL>(E, dfrag, p.d_fragT_off, p.dacts, n, valid, lane);
        if (valid) {
#pragma unroll
            for (int ib = 0; ib < DS::ib(0); ib++) st_h4(p.denc + (size_t)n * DIN + 16 * ib + 4 * g, E[ib]);
        }
    }
}

int pick_nt(int d)
{
    if (d <= 32) return 2;  // the colour input alone is 32 wide
    if (d <= 64) return 4;
    return 8;
}

}  // namespace

void nerf_forward(const NerfFwdArgs& a, int N, hipStream_t stream, const uint32_t* d_n)
{
    a.dshape.validate();
    a.cshape.validate();
    if (N <= 0) return;
    if (a.dshape.out != 16) throw std::runtime_error("NeRF forward: the density head must have 16 outputs");
    if (a.cshape.in != 32) throw std::runtime_error("NeRF forward: the colour head must take 32 inputs");
    if (a.out_act != 0 && a.out_act != 1) throw std::runtime_error("NeRF forward: unsupported output activation");
    if (a.pos_stride < 3) throw std::runtime_error("NeRF forward: position stride must be >= 3");
    const GridMeta& m = *a.meta;
    if (2 * m.numLevels != a.dshape.in) throw std::runtime_error("NeRF forward: density input must be 2 * numLevels");

    const bool planar = a.enc_scratch != nullptr;
    if (planar) {
        if (a.enc_plane < N) throw std::runtime_error("NeRF forward: encoding plane stride below the sample count");
        if (!a.enc_ready) hash_encode_planar(m, a.table, a.pos, a.pos_stride, a.enc_scratch, a.enc_plane, N, stream, d_n);
    }
    if (planar && a.heads_packed != nullptr && a.dacts == nullptr && a.cacts == nullptr &&
        nerf_heads_supported(a.dshape, a.cshape)) {
        if (!a.heads_prepacked) nerf_heads_pack(NerfHeadsWeights{a.dW, a.dB, a.cW, a.cB}, a.heads_packed, stream);
        NerfHeadsFwd h;
        h.packed = a.heads_packed;
        h.enc = a.enc_scratch;
        h.enc_plane = a.enc_plane;
        h.levels = m.numLevels;
        h.dirs = a.dirs;
        h.ray_idx = a.ray_idx;
        h.density_bias = a.density_bias;
        h.out_act = a.out_act;
        h.sigma = a.sigma;
        h.density_out = a.density_out;
        h.density_stride = a.density_stride;
        h.color_out = a.color_out;
        h.color_in = a.color_in;
        nerf_heads_forward(h, N, stream, d_n);
        return;
    }
    if (a.density_stride != 16) throw std::runtime_error("NeRF forward: a compact density output needs the MFMA heads");
    NerfFwdParams p{};
    p.pos = a.pos;
    p.pos_stride = a.pos_stride;
    p.table = reinterpret_cast<const _Float16*>(a.table);
    p.enc = reinterpret_cast<const _Float16*>(a.enc_scratch);
    p.plane = a.enc_plane;
    p.dW = reinterpret_cast<const _Float16* const*>(a.dW);
    p.dB = a.dB;
    p.dacts = reinterpret_cast<_Float16* const*>(a.dacts);
    p.dout = a.density_out;
    p.dirs = a.dirs;
    p.ray_idx = a.ray_idx;
    p.sigma = a.sigma;
    p.density_bias = a.density_bias;
    p.cW = reinterpret_cast<const _Float16* const*>(a.cW);
    p.cB = a.cB;
    p.cacts = reinterpret_cast<_Float16* const*>(a.cacts);
    p.cin = reinterpret_cast<_Float16*>(a.color_in);
    p.cout = a.color_out;
    p.d_n = d_n;
    p.N = N;
    p.L = m.numLevels;
    p.T = m.tableSize;
    p.dense_start = m.denseLevelStart;
    for (int l = 0; l < m.numLevels; l++) {
        p.scale[l] = m.scale[l];
        p.res[l] = m.res[l];
    }
    p.d_in = a.dshape.in;
    p.d_hid = a.dshape.hid;
    p.d_layers = a.dshape.layers;
    p.c_hid = a.cshape.hid;
    p.c_out = a.cshape.out;
    p.c_layers = a.cshape.layers;

    auto offsets = [](const MlpShape& s, int* frag_off, int* bias_off, int& halves, int& floats) {
        halves = floats = 0;
        for (int l = 0; l < s.layers; l++) {
            frag_off[l] = halves;
            bias_off[l] = floats;
            halves += tiles16(s.out_l(l)) * tiles16(s.in_l(l)) * 256;
            floats += tiles16(s.out_l(l)) * 16;
        }
    };
    int dh = 0, df = 0, ch = 0, cf = 0;
    offsets(a.dshape, p.d_frag_off, p.d_bias_off, dh, df);
    offsets(a.cshape, p.c_frag_off, p.c_bias_off, ch, cf);
    p.c_frag_base = (dh * 2 + 15) & ~15;
    p.d_bias_base = (p.c_frag_base + ch * 2 + 15) & ~15;
    p.c_bias_base = (p.d_bias_base + df * 4 + 15) & ~15;
    p.meta_base = (p.c_bias_base + cf * 4 + 15) & ~15;
    const int lds = p.meta_base + 8 * kMaxLevels;
    if (lds > max_lds_per_block()) throw std::runtime_error("NeRF forward: networks too large for the LDS budget");

    const int ntiles = (N + 15) / 16;
    // 4 workgroups per CU: each wave takes several tiles, so the per-workgroup
    // staging of both heads' weights into LDS is amortised (measured: 2 per CU
    // 126 us, 4 per CU 111 us, 8 per CU 121 us for a 236 K-sample step)
    const int blocks = std::max(1, std::min((ntiles + 3) / 4, num_cus() * 4));
    const int nt = pick_nt(std::max(a.dshape.maxd(), a.cshape.maxd()));
#define GRAFT_NERF_FWD_P(NTV, PL)                                                                             \
    do {                                                                                                      \
        if (a.out_act == 1)                                                                                   \
            hipLaunchKernelGGL((nerf_fwd_kernel<NTV, 1, PL>), dim3(blocks), dim3(256), lds, stream, p);       \
        else                                                                                                  \
            hipLaunchKernelGGL((nerf_fwd_kernel<NTV, 0, PL>), dim3(blocks), dim3(256), lds, stream, p);       \
    } while (0)
#define GRAFT_NERF_FWD(NTV)                                                                                   \
    do {                                                                                                      \
        if (planar) GRAFT_NERF_FWD_P(NTV, true);                                                              \
        else GRAFT_NERF_FWD_P(NTV, false);                                                                    \
    } while (0)
    switch (nt) {
        case 2: GRAFT_NERF_FWD(2); break;
        case 4: GRAFT_NERF_FWD(4); break;
        default: GRAFT_NERF_FWD(8); break;
    }
#undef GRAFT_NERF_FWD
#undef GRAFT_NERF_FWD_P
    GRAFT_LAUNCH_CHECK();
}

bool nerf_backward_dx(const NerfBwdDxArgs& a, int N, hipStream_t stream, const uint32_t* d_n)
{
    const bool shapes = a.cshape.in == 32 && a.cshape.hid == 64 && a.cshape.out == 8 && a.cshape.layers == 3 &&
                        a.dshape.in == 32 && a.dshape.hid == 64 && a.dshape.out == 16 && a.dshape.layers == 2;
    if (!shapes) return false;
    if (N <= 0) return true;
    NerfBwdDxParams p{};
    p.cdy = reinterpret_cast<const _Float16*>(a.color_dy);
    p.cacts = reinterpret_cast<const _Float16* const*>(a.cacts);
    p.cW = reinterpret_cast<const _Float16* const*>(a.cW);
    p.dsigma = a.dsigma;
    p.dacts = reinterpret_cast<const _Float16* const*>(a.dacts);
    p.dW = reinterpret_cast<const _Float16* const*>(a.dW);
    p.cdx = reinterpret_cast<_Float16*>(a.color_dx);
    p.dloss = reinterpret_cast<_Float16*>(a.density_dy);
    p.denc = reinterpret_cast<_Float16*>(a.denc);
    p.d_n = d_n;
    p.N = N;
    int ch = 0, dh = 0;
    for (int l = 0; l < a.cshape.layers; l++) {
        p.c_fragT_off[l] = ch;
        ch += tiles16(a.cshape.out_l(l)) * tiles16(a.cshape.in_l(l)) * 256;
    }
    for (int l = 0; l < a.dshape.layers; l++) {
        p.d_fragT_off[l] = dh;
        dh += tiles16(a.dshape.out_l(l)) * tiles16(a.dshape.in_l(l)) * 256;
    }
    p.d_frag_base = (ch * 2 + 15) & ~15;
    const int lds = p.d_frag_base + dh * 2;
    const auto kern = nerf_bwd_dx_kernel<32, 64, 8, 3, 32, 64, 2>;
    int per_cu = 0;
    GRAFT_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds));
    const int ntiles = (N + 15) / 16;
    const int blocks = std::max(1, std::min((ntiles + 3) / 4, num_cus() * std::max(1, per_cu)));
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, stream, p);
    GRAFT_LAUNCH_CHECK();
    return true;
}

}  // namespace graft
