// Fused Adam, MSE loss/grad, gradient zeroing and the small layout kernels of
// the TinyMLP host classes, for gfx950.
//
//   Adam      optimizerKernel.cu:16-167 (weights, biases, hash table)
//   MSE       optimizerKernel.cu:169-224, grad scale :388
//   zero      optimizerKernel.cu:226-239
//
// The Adam update is written operation by operation (no FP contraction, IEEE
// division and square root) so that it is bit-identical to the CPU oracle.
// The hash-table pass is one HBM stream over 16-byte vectors: gradients of
// exactly 0.0f skip the m/v/w reads, every consumed gradient is zeroed.
#include "optimizer.h"

#include "adam_math.h"

#include <algorithm>

namespace graft {

namespace {

__global__ __launch_bounds__(256) void adam_hash_kernel(float* __restrict__ w, _Float16* __restrict__ w16,
                                                        float* __restrict__ g, float* __restrict__ m,
                                                        float* __restrict__ v, size_t n4, AdamArgs a)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        const f4 gr = reinterpret_cast<const f4*>(g)[i];
        const bool nz0 = gr[0] != 0.0f, nz1 = gr[1] != 0.0f, nz2 = gr[2] != 0.0f, nz3 = gr[3] != 0.0f;
        if (!(nz0 | nz1 | nz2 | nz3)) continue;
        f4 mv = reinterpret_cast<const f4*>(m)[i];
        f4 vv = reinterpret_cast<const f4*>(v)[i];
        f4 wv = reinterpret_cast<const f4*>(w)[i];
        const bool nz[4] = {nz0, nz1, nz2, nz3};
        f4 gz = gr;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (nz[j]) {
                float mj = mv[j], vj = vv[j], wj = wv[j];
                adam_update(gr[j], mj, vj, wj, a);
                mv[j] = mj;
                vv[j] = vj;
                wv[j] = wj;
                gz[j] = 0.0f;
            }
        }
        reinterpret_cast<f4*>(g)[i] = gz;
        reinterpret_cast<f4*>(m)[i] = mv;
        reinterpret_cast<f4*>(v)[i] = vv;
        reinterpret_cast<f4*>(w)[i] = wv;
        if (nz0 & nz1 & nz2 & nz3) {
            reinterpret_cast<h4*>(w16)[i] = h4{to_h(wv[0]), to_h(wv[1]), to_h(wv[2]), to_h(wv[3])};
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (nz[j]) w16[4 * i + j] = to_h(wv[j]);
        }
    }
}

// Dense per-layer Adam (weights with fp16 copy, or biases without).
__global__ __launch_bounds__(256) void adam_layers_kernel(float* const* w, _Float16* const* w16,
                                                          float* const* g, float* const* m,
                                                          float* const* v, LayerSizes sz, AdamArgs a)
{
    const int l = blockIdx.y;
    const int n = sz.n[l];
    float* wl = w[l];
    float* gl = g[l];
    float* ml = m[l];
    float* vl = v[l];
    _Float16* hl = w16 ? w16[l] : nullptr;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float mi = ml[i], vi = vl[i], wi = wl[i];
        adam_update(gl[i], mi, vi, wi, a);
        ml[i] = mi;
        vl[i] = vi;
        wl[i] = wi;
        if (hl) hl[i] = to_h(wi);
    }
}

// Weights (with fp16 copy) and biases of every layer in one launch:
// blockIdx.y < layers -> weights of layer y, else biases of layer y - layers.
struct DenseGroup {
    float* const* w;
    _Float16* const* w16;  // nullable
    float* const* g;
    float* const* m;
    float* const* v;
    LayerSizes sz;
};

__global__ __launch_bounds__(256) void adam_dense_kernel(const DenseGroup W, const DenseGroup B, int layers,
                                                         AdamArgs a)
{
    const bool is_w = (int)blockIdx.y < layers;
    const DenseGroup& G = is_w ? W : B;
    const int l = is_w ? blockIdx.y : blockIdx.y - layers;
    const int n = G.sz.n[l];
    float* wl = G.w[l];
    float* gl = G.g[l];
    float* ml = G.m[l];
    float* vl = G.v[l];
    _Float16* hl = G.w16 ? G.w16[l] : nullptr;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float mi = ml[i], vi = vl[i], wi = wl[i];
        adam_update(gl[i], mi, vi, wi, a);
        ml[i] = mi;
        vl[i] = vi;
        wl[i] = wi;
        if (hl) hl[i] = to_h(wi);
    }
}

__global__ __launch_bounds__(256) void zero_layers_kernel(float* const* a, float* const* b, LayerSizes sa,
                                                          LayerSizes sb)
{
    const int l = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < sa.n[l]; i += gridDim.x * blockDim.x) a[l][i] = 0.0f;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < sb.n[l]; i += gridDim.x * blockDim.x) b[l][i] = 0.0f;
}

// Two elements per thread as half2 pairs; padded columns carry zero gradient.
template <int OUT_ACT>
__global__ __launch_bounds__(256) void mse_kernel(const float* __restrict__ pred, const _Float16* __restrict__ tgt,
                                                  _Float16* __restrict__ dloss, float* __restrict__ partials,
                                                  long long n2, int padded, int valid, float grad_scale)
{
    __shared__ float red[4];
    float local = 0.0f;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n2; i += (long long)gridDim.x * blockDim.x) {
        const long long e = 2 * i;
        const int c0 = (int)(e % padded), c1 = c0 + 1;
        const float2 p = *reinterpret_cast<const float2*>(pred + e);
        const h2 t = *reinterpret_cast<const h2*>(tgt + e);
        const float dx = c0 < valid ? p.x - (float)t.x : 0.0f;
        const float dy = c1 < valid ? p.y - (float)t.y : 0.0f;
        local += dx * dx + dy * dy;
        float gx = dx * grad_scale, gy = dy * grad_scale;
        if (OUT_ACT == 1) {
            gx *= p.x * (1.0f - p.x);
            gy *= p.y * (1.0f - p.y);
        }
        *reinterpret_cast<h2*>(dloss + e) = h2{to_h(gx), to_h(gy)};
    }
    for (int o = 32; o > 0; o >>= 1) local += __shfl_down(local, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = local;
    __syncthreads();
    if (threadIdx.x == 0) partials[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// *total += the block partials of mse_kernel, summed in a fixed order (one
// block; a same-address atomic per block would serialise thousands of adds).
__global__ __launch_bounds__(1024) void sum_into_kernel(const float* __restrict__ partials, int n,
                                                        float* __restrict__ total)
{
    __shared__ float red[16];
    float v = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) v += partials[i];
    for (int o = 32; o > 0; o >>= 1) v += __shfl_down(v, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += red[w];
        *total += t;
    }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void pad_cast_kernel(const TI* __restrict__ src, TO* __restrict__ dst,
                                                       long long rows, int udim, int pdim)
{
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < rows * pdim;
         i += (long long)gridDim.x * blockDim.x) {
        const long long r = i / pdim;
        const int c = (int)(i - r * pdim);
        dst[i] = c < udim ? (TO)src[r * udim + c] : (TO)0;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void unpad_kernel(const T* __restrict__ src, T* __restrict__ dst, long long rows,
                                                    int pdim, int udim)
{
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < rows * udim;
         i += (long long)gridDim.x * blockDim.x) {
        const long long r = i / udim;
        const int c = (int)(i - r * udim);
        dst[i] = src[r * pdim + c];
    }
}

int blocks_for(long long n)
{
    return (int)std::max(1LL, std::min((n + 255) / 256, (long long)num_cus() * 16));
}

}  // namespace

void adam_hash(float* w, __half* w16, float* g, float* m, float* v, size_t n, const AdamArgs& a,
               hipStream_t stream)
{
    if (n == 0) return;
    if (n % 4) throw std::runtime_error("hash Adam: parameter count must be a multiple of 4");
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(adam_hash_kernel, dim3(blocks_for((long long)n4)), dim3(256), 0, stream, w,
                       reinterpret_cast<_Float16*>(w16), g, m, v, n4, a);
    GRAFT_LAUNCH_CHECK();
}

void adam_layers(float* const* w, __half* const* w16, float* const* g, float* const* m,
                 float* const* v, const LayerSizes& sz, int layers, const AdamArgs& a,
                 hipStream_t stream)
{
    int mx = 0;
    for (int l = 0; l < layers; l++) mx = std::max(mx, sz.n[l]);
    if (mx == 0) return;
    hipLaunchKernelGGL(adam_layers_kernel, dim3((mx + 255) / 256, layers), dim3(256), 0, stream, w,
                       reinterpret_cast<_Float16* const*>(w16), g, m, v, sz, a);
    GRAFT_LAUNCH_CHECK();
}

void adam_dense(float* const* wW, __half* const* w16, float* const* gW, float* const* mW, float* const* vW,
                const LayerSizes& szW, float* const* wB, float* const* gB, float* const* mB, float* const* vB,
                const LayerSizes& szB, int layers, const AdamArgs& a, hipStream_t stream)
{
    int mx = 0;
    for (int l = 0; l < layers; l++) mx = std::max(mx, std::max(szW.n[l], szB.n[l]));
    if (mx == 0) return;
    const DenseGroup W{wW, reinterpret_cast<_Float16* const*>(w16), gW, mW, vW, szW};
    const DenseGroup B{wB, nullptr, gB, mB, vB, szB};
    hipLaunchKernelGGL(adam_dense_kernel, dim3((mx + 255) / 256, 2 * layers), dim3(256), 0, stream, W, B, layers, a);
    GRAFT_LAUNCH_CHECK();
}

void zero_layers(float* const* a, float* const* b, const LayerSizes& sa, const LayerSizes& sb, int layers,
                 hipStream_t stream)
{
    int mx = 0;
    for (int l = 0; l < layers; l++) mx = std::max(mx, std::max(sa.n[l], sb.n[l]));
    if (mx == 0) return;
    hipLaunchKernelGGL(zero_layers_kernel, dim3((mx + 255) / 256, layers), dim3(256), 0, stream, a, b, sa, sb);
    GRAFT_LAUNCH_CHECK();
}

void mse_loss_grad(const float* pred, const __half* tgt, __half* dloss, float* total, int N, int padded,
                   int valid, float loss_scale, int out_act, hipStream_t stream, Workspace* ws)
{
    if (N <= 0) return;
    if (padded % 2) throw std::runtime_error("MSE: padded dimension must be even");
    const float grad_scale = (2.0f / (float)(N * valid)) * loss_scale;
    const long long n2 = (long long)N * padded / 2;
    const int blocks = blocks_for(n2);
    const _Float16* t = reinterpret_cast<const _Float16*>(tgt);
    _Float16* d = reinterpret_cast<_Float16*>(dloss);
    float* partials = static_cast<float*>((ws ? *ws : stream_workspace(stream)).get((size_t)blocks * sizeof(float)));
    if (out_act == 1)
        hipLaunchKernelGGL(mse_kernel<1>, dim3(blocks), dim3(256), 0, stream, pred, t, d, partials, n2, padded, valid,
                           grad_scale);
    else
        hipLaunchKernelGGL(mse_kernel<0>, dim3(blocks), dim3(256), 0, stream, pred, t, d, partials, n2, padded, valid,
                           grad_scale);
    GRAFT_LAUNCH_CHECK();
    hipLaunchKernelGGL(sum_into_kernel, dim3(1), dim3(1024), 0, stream, partials, blocks, total);
    GRAFT_LAUNCH_CHECK();
}

void pad_f32(const float* src, float* dst, long long rows, int udim, int pdim, hipStream_t s)
{
    if (rows <= 0) return;
    hipLaunchKernelGGL((pad_cast_kernel<float, float>), dim3(blocks_for(rows * pdim)), dim3(256), 0, s, src, dst, rows, udim, pdim);
    GRAFT_LAUNCH_CHECK();
}

void pad_f16(const __half* src, __half* dst, long long rows, int udim, int pdim, hipStream_t s)
{
    if (rows <= 0) return;
    hipLaunchKernelGGL((pad_cast_kernel<_Float16, _Float16>), dim3(blocks_for(rows * pdim)), dim3(256), 0, s,
                       reinterpret_cast<const _Float16*>(src), reinterpret_cast<_Float16*>(dst), rows, udim, pdim);
    GRAFT_LAUNCH_CHECK();
}

void f32_to_f16(const float* src, __half* dst, long long n, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL((pad_cast_kernel<float, _Float16>), dim3(blocks_for(n)), dim3(256), 0, s, src,
                       reinterpret_cast<_Float16*>(dst), n, 1, 1);
    GRAFT_LAUNCH_CHECK();
}

void unpad_f32(const float* src, float* dst, long long rows, int pdim, int udim, hipStream_t s)
{
    if (rows <= 0) return;
    hipLaunchKernelGGL((unpad_kernel<float>), dim3(blocks_for(rows * udim)), dim3(256), 0, s, src, dst, rows, pdim, udim);
    GRAFT_LAUNCH_CHECK();
}

}  // namespace graft
