// Per-sample and per-ray kernels around the two MLPs, plus the occupancy
// bitfield, for gfx950.
//
//   sh_gather       compute_SH_gather              otherKernels.cu:156-273
//   composite       render_rays_distortion_kernel  compositing.cu:80-213
//   composite_infer render_rays_kernel             compositing.cu:5-78
//   color_grad      compute_color_grad             otherKernels.cu:303-409
//   density_grad    compute_density_grad           otherKernels.cu:497-562
//   master grid     updateMasterGrid               otherKernels.cu:677-690
//   occupancy bits  updateOccupancyGrid            otherKernels.cu:700-750
//   mip pyramid     bitfield_max_pool / buildMipmaps  otherKernels.cu:752-807, InstantNerf.cu:1177-1204
//
// Arithmetic follows the reference kernels operation by operation (fp32,
// no contraction, correctly rounded division); e^x is nerf_expf.  Sample and
// ray counts may come from device memory (see nerf.h).
#include "nerf.h"
#include "nerf_math.h"

#include <algorithm>
#include <type_traits>

namespace graft {

namespace {

__device__ __forceinline__ uint32_t dev_count(const uint32_t* d_n, uint32_t n_max)
{
    return d_n ? min(*d_n, n_max) : n_max;
}


// One sample per thread: 64 B of density logits in, 64 B of fp16 color input
// and the sigma out, all as 16-byte vectors.
__global__ __launch_bounds__(256) void sh_gather_kernel(const float3* __restrict__ dirs,
                                                        const uint32_t* __restrict__ ray_idx,
                                                        const uint32_t* __restrict__ d_n, uint32_t n_max, float bias,
                                                        const float* __restrict__ dout, _Float16* __restrict__ cin,
                                                        float* __restrict__ sigma)
{
    const uint32_t N = dev_count(d_n, n_max);
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const float3 d = dirs[ray_idx[n]];
    float sh[16];
    sh_basis16(d.x, d.y, d.z, sh);
    const f4* src = reinterpret_cast<const f4*>(dout + 16 * (size_t)n);
    float lg[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const f4 v = src[q];
#pragma unroll
        for (int j = 0; j < 4; j++) lg[4 * q + j] = sanitize_logit(v[j]);
    }
    sigma[n] = nerf_expf(fminf(lg[0] - bias, 8.0f));
    h4* dst = reinterpret_cast<h4*>(cin + 32 * (size_t)n);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        dst[q] = h4{to_h(lg[4 * q]), to_h(lg[4 * q + 1]), to_h(lg[4 * q + 2]), to_h(lg[4 * q + 3])};
        dst[4 + q] = h4{to_h(sh[4 * q]), to_h(sh[4 * q + 1]), to_h(sh[4 * q + 2]), to_h(sh[4 * q + 3])};
    }
}

__device__ __forceinline__ float disparity_warp(float t, float t_near, float inv_g_range)
{
    return (1.0f - t_near / fmaxf(t, 1e-4f)) * inv_g_range;
}

__global__ __launch_bounds__(256) void composite_kernel(const CompositeArgs a, const uint32_t* __restrict__ d_rays,
                                                        uint32_t rays_max)
{
    const uint32_t R = dev_count(d_rays, rays_max);
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= R) return;
    const uint32_t off = a.offsets[r], cnt = a.counts[r];
    const float d_prior = a.depth_prior ? a.depth_prior[r] : -1.0f;
    const float s_prior = a.sigma_prior ? a.sigma_prior[r] : -1.0f;
    const float dwl = (d_prior >= 0) ? a.lambda_depth : 0.0f;
    const float t_near = (cnt > 0) ? fmaxf(a.t[off], 1e-4f) : 1.0f;
    const float t_far = (cnt > 0) ? a.t[off + cnt - 1] : 1.0f;
    const float g_far = 1.0f - t_near / fmaxf(t_far, t_near + 1e-4f);
    const float inv_g = (g_far > 1e-6f) ? (1.0f / g_far) : 0.0f;
    float T = 1.0f, rc = 0.0f, gc = 0.0f, bc = 0.0f, depth = 0.0f;
    const float c = 2.0f / 3;
    float dw_g = 0.0f, dwm_g = 0.0f, dw_s = 0.0f, dwm_s = 0.0f, dls = 0.0f;
    for (uint32_t i = 0; i < cnt; i++) {
        const uint32_t idx = off + i;
        const float t = a.t[idx];
        float t_next = (i < cnt - 1) ? a.t[idx + 1] : (t + 1e-3f);
        float delta = t_next - t;
        if (delta < 0.0f) {
            delta = 0.0f;
            t_next = t;
        }
        const float s = disparity_warp(t, t_near, inv_g);
        const float s_next = disparity_warp(t_next, t_near, inv_g);
        const float m = 0.5f * (s + s_next);
        const float alpha = 1.0f - nerf_expf(-a.sigma[idx] * delta);
        const float w = alpha * T;
        const float* cc = a.rgb + (size_t)a.rgb_stride * idx;
        rc += w * cc[0];
        gc += w * cc[1];
        bc += w * cc[2];
        depth += w * t;
        T *= (1.0f - alpha);
        dw_g += w;
        dwm_g += w * m;
        const float tx = (t - d_prior) / s_prior;
        dls += nerf_expf(-0.5f * tx * tx) * delta;
        a.dw[idx] = w;
    }
    dls = 1.0f / fmaxf(dls, 1e-8f);
    float wgs = 0.0f;
    for (uint32_t i = 0; i < cnt; i++) {
        const uint32_t idx = off + i;
        const float t = a.t[idx];
        float t_next = (i < cnt - 1) ? a.t[idx + 1] : (t + 1e-3f);
        float delta = t_next - t;
        if (delta < 0.0f) {
            delta = 0.0f;
            t_next = t;
        }
        const float s = disparity_warp(t, t_near, inv_g);
        const float s_next = disparity_warp(t_next, t_near, inv_g);
        const float m = 0.5f * (s + s_next);
        float ds = s_next - s;
        if (ds < 0.0f) ds = 0.0f;
        const float w = a.dw[idx];
        const float tx = (t - d_prior) / s_prior;
        const float dwt = nerf_expf(-0.5f * tx * tx) * delta * dls;
        const float dloss = -dwt * (1.0f / fmaxf(w, 1e-6f));
        const float bil = m * (2 * dw_s - dw_g) + (dwm_g - 2 * dwm_s);
        const float g = a.lambda_dist * (2 * (bil) + c * w * ds) + dwl * dloss;
        a.dw[idx] = g;
        wgs += w * g;
        dw_s += w;
        dwm_s += w * m;
    }
    a.weight_sum[r] = wgs;
    rc += T * a.bg.x;
    gc += T * a.bg.y;
    bc += T * a.bg.z;
    a.final_rgb[3 * r] = rc;
    a.final_rgb[3 * r + 1] = gc;
    a.final_rgb[3 * r + 2] = bc;
    a.final_depth[r] = depth;
    if (a.rgb_true && a.phi) {
        a.phi[3 * r] = 2.0f * (rc - a.rgb_true[3 * r]);
        a.phi[3 * r + 1] = 2.0f * (gc - a.rgb_true[3 * r + 1]);
        a.phi[3 * r + 2] = 2.0f * (bc - a.rgb_true[3 * r + 2]);
    }
}

__global__ __launch_bounds__(256) void composite_infer_kernel(const CompositeArgs a, uint32_t base,
                                                              uint32_t rays_done, const uint32_t* __restrict__ d_rays,
                                                              uint32_t rays_max)
{
    const uint32_t R = dev_count(d_rays, rays_max);
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= R) return;
    const uint32_t off = a.offsets[r + rays_done] - base, cnt = a.counts[r];
    float T = 1.0f, rc = 0.0f, gc = 0.0f, bc = 0.0f, depth = 0.0f;
    for (uint32_t i = 0; i < cnt; i++) {
        const uint32_t idx = off + i;
        const float t = a.t[idx];
        float delta = (i < cnt - 1) ? a.t[idx + 1] - t : 1e-3f;
        if (delta < 0.0f) delta = 0.0f;
        const float alpha = 1.0f - nerf_expf(-a.sigma[idx] * delta);
        const float w = alpha * T;
        const float* c = a.rgb + (size_t)a.rgb_stride * idx;
        rc += w * c[0];
        gc += w * c[1];
        bc += w * c[2];
        depth += w * t;
        T *= (1.0f - alpha);
        if (T < 1e-4f) break;
    }
    rc += T * a.bg.x;
    gc += T * a.bg.y;
    bc += T * a.bg.z;
    a.final_rgb[3 * r] = rc;
    a.final_rgb[3 * r + 1] = gc;
    a.final_rgb[3 * r + 2] = bc;
    if (a.final_depth) a.final_depth[r] = depth;
    if (a.rgb_true && a.phi) {
        a.phi[3 * r] = 2.0f * (rc - a.rgb_true[3 * r]);
        a.phi[3 * r + 1] = 2.0f * (gc - a.rgb_true[3 * r + 1]);
        a.phi[3 * r + 2] = 2.0f * (bc - a.rgb_true[3 * r + 2]);
    }
}

__global__ __launch_bounds__(256) void color_grad_kernel(const ColorGradArgs a, const uint32_t* __restrict__ d_rays,
                                                         uint32_t rays_max)
{
    const uint32_t R = dev_count(d_rays, rays_max);
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= R) return;
    const uint32_t r = idx + a.initial_offset;
    float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f, wg = 0.0f;
    const uint32_t base = a.offsets[r];
    const float wgs = a.weight_sum[r];
    const uint32_t cnt = a.counts[r];
    const float pr = a.phi[3 * r], pg = a.phi[3 * r + 1], pb = a.phi[3 * r + 2];
    const float fr = a.final_rgb[3 * r], fg = a.final_rgb[3 * r + 1], fb = a.final_rgb[3 * r + 2];
    const uint32_t start = a.offsets[a.initial_offset];
    const float bs = 1.0f / (float)a.total_rays;
    for (uint32_t j = 0; j < cnt; j++) {
        const uint32_t gi = base + j;
        const size_t i = gi - start;
        const float tc = a.t[gi];
        const float delta = (j == cnt - 1) ? 1e-3f : fmaxf(a.t[gi + 1] - tc, 0.0f);
        const float sigma = nerf_expf(fminf(a.density_out[(size_t)a.density_stride * i] - a.bias, 8.0f));
        const float alpha = 1.0f - nerf_expf(-sigma * delta);
        const float w = T * alpha;
        const float* co = a.color_out + (size_t)a.color_stride * i;
        const float c_r = co[0], c_g = co[1], c_b = co[2];
        cr += w * c_r;
        cg += w * c_g;
        cb += w * c_b;
        float g_r = pr * w * c_r * (1.0f - c_r) * a.loss_scale * bs;
        float g_g = pg * w * c_g * (1.0f - c_g) * a.loss_scale * bs;
        float g_b = pb * w * c_b * (1.0f - c_b) * a.loss_scale * bs;
        g_r = clamp_half_range(g_r);
        g_g = clamp_half_range(g_g);
        g_b = clamp_half_range(g_b);
        if (g_r != g_r || g_g != g_g || g_b != g_b) g_r = g_g = g_b = 0.0f;
        _Float16* cgo = reinterpret_cast<_Float16*>(a.color_grad) + (size_t)a.grad_stride * i;
        cgo[0] = to_h(g_r);
        cgo[1] = to_h(g_g);
        cgo[2] = to_h(g_b);
        for (int k = 3; k < a.grad_stride; k++) cgo[k] = (_Float16)0.0f;
        const float sr = fr - cr, sg = fg - cg, sb = fb - cb;
        const float dr = T * c_r * (1.0f - alpha) - sr;
        const float dg = T * c_g * (1.0f - alpha) - sg;
        const float db = T * c_b * (1.0f - alpha) - sb;
        const float gw = a.dw[i];
        wg += w * gw;
        const float suffix = wgs - wg;
        float dsi = delta * (dr * pr + dg * pg + db * pb);
        dsi += delta * (gw * T * (1.0f - alpha) - suffix);
        float ds = dsi * sigma * a.loss_scale * bs;
        ds = clamp_half_range(ds);
        if (ds != ds) ds = 0.0f;
        a.dsigma[i] = ds;
        T = T * (1.0f - alpha);
    }
}

// ---------------------------------------------------------------------------
// Fused compositing + distortion gradient + colour gradient, one wave per ray.
//
// The reference runs two thread-per-ray kernels whose loops walk a ray's
// samples in order (compositing.cu:131-196, otherKernels.cu:346-407).  A step
// holds a few hundred to a few thousand rays of up to 1024 samples, so such
// loops are bound by the longest ray: one load latency and a chain of
// dependent fp32 operations per sample.
//
// Here one wave takes one ray and every lane owns a run of n = ceil(cnt / 64)
// consecutive samples.  The running transmittance T and the running sums of
// the reference loops become two-level scans: each lane folds its own run
// (products of 1 - alpha, sums of weight x value relative to its run's start),
// a 64-lane scan combines the runs, and a second pass over the run emits the
// per-sample results from the lane's prefix.  Four passes over the run:
//   A  T and the weighted sums of the compositing (colour, depth, sum w,
//      sum w m, sum of depth-prior terms);
//   B  the distortion (+ depth-prior) gradient per weight, from exclusive
//      prefix sums of w and w m (compositing.cu:177-195);
//   C  the colour gradient's own transmittance and the weighted sums of
//      colour and of w g (otherKernels.cu:346-366);
//   D  colour gradient and d sigma per sample (otherKernels.cu:367-407).
// The arithmetic per sample is the reference's; only the association of the
// products and sums differs (scans instead of left-to-right folds), so
// results agree with the serial kernels above to fp32 rounding.
// Wave-wide sums and scans on DPP moves (row shifts and rotations within the
// 16-lane rows, then the four row totals through v_readlane): no LDS
// permutes.  bound_ctrl off: a lane whose source lies outside its row keeps
// `old` (the identity).
template <int CTRL>
__device__ __forceinline__ float dpp(float old, float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowRor1 = 0x121, kRowRor2 = 0x122, kRowRor4 = 0x124, kRowRor8 = 0x128;
constexpr int kWaveShr1 = 0x138;

__device__ __forceinline__ float lane_value(float v, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// the sum over the wave, identical in every lane: each row's sum by rotations
// (every lane of a row adds the same pairs, commutatively), then the rows'
__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp<kRowRor8>(0.0f, v);
    v += dpp<kRowRor4>(0.0f, v);
    v += dpp<kRowRor2>(0.0f, v);
    v += dpp<kRowRor1>(0.0f, v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// exclusive prefix sum / product over the lanes
__device__ __forceinline__ float wave_excl_sum(float v, int lane)
{
    v += dpp<kRowShr1>(0.0f, v);
    v += dpp<kRowShr2>(0.0f, v);
    v += dpp<kRowShr4>(0.0f, v);
    v += dpp<kRowShr8>(0.0f, v);
    const float r0 = lane_value(v, 15), r1 = lane_value(v, 31), r2 = lane_value(v, 47);
    const int row = lane >> 4;
    const float below = row == 0 ? 0.0f : row == 1 ? r0 : row == 2 ? r0 + r1 : (r0 + r1) + r2;
    if (row != 0) v = below + v;
    return dpp<kWaveShr1>(0.0f, v);
}

__device__ __forceinline__ float wave_excl_prod(float v, int lane)
{
    v *= dpp<kRowShr1>(1.0f, v);
    v *= dpp<kRowShr2>(1.0f, v);
    v *= dpp<kRowShr4>(1.0f, v);
    v *= dpp<kRowShr8>(1.0f, v);
    const float r0 = lane_value(v, 15), r1 = lane_value(v, 31), r2 = lane_value(v, 47);
    const int row = lane >> 4;
    const float below = row == 0 ? 1.0f : row == 1 ? r0 : row == 2 ? r0 * r1 : (r0 * r1) * r2;
    if (row != 0) v = below * v;
    return dpp<kWaveShr1>(1.0f, v);
}

// Per-sample terms of the compositing pass (compositing.cu:131-160).
struct CompSample {
    float t, delta, m, ds, alpha, e;
};

// From its loaded inputs: the sample's t, the next sample's t (read only when
// i < cnt - 1) and sigma.
__device__ __forceinline__ CompSample comp_terms(float t, float t_next_in, float sigma, uint32_t i, uint32_t cnt,
                                                 float t_near, float inv_g, float d_prior, float s_prior)
{
    CompSample c;
    c.t = t;
    float t_next = (i < cnt - 1) ? t_next_in : (c.t + 1e-3f);
    c.delta = t_next - c.t;
    if (c.delta < 0.0f) {
        c.delta = 0.0f;
        t_next = c.t;
    }
    const float s = disparity_warp(c.t, t_near, inv_g);
    const float s_next = disparity_warp(t_next, t_near, inv_g);
    c.m = 0.5f * (s + s_next);
    c.ds = s_next - s;
    if (c.ds < 0.0f) c.ds = 0.0f;
    c.alpha = 1.0f - nerf_expf(-sigma * c.delta);
    const float tx = (c.t - d_prior) / s_prior;
    c.e = nerf_expf(-0.5f * tx * tx) * c.delta;
    return c;
}

__device__ __forceinline__ CompSample comp_sample(const CompositeArgs& a, uint32_t idx, uint32_t i, uint32_t cnt,
                                                  float t_near, float inv_g, float d_prior, float s_prior)
{
    const float t = a.t[idx];
    const float t_next = (i < cnt - 1) ? a.t[idx + 1] : 0.0f;
    return comp_terms(t, t_next, a.sigma[idx], i, cnt, t_near, inv_g, d_prior, s_prior);
}

// Per-sample terms of the colour-gradient pass (otherKernels.cu:349-356).
struct GradSample {
    float delta, sigma, alpha;
};

// From its loaded inputs: the sample's t, the next one's (read only when
// j < cnt - 1) and the density output.
__device__ __forceinline__ GradSample grad_terms(float tc, float t_next, float density, float bias, uint32_t j,
                                                 uint32_t cnt)
{
    GradSample s;
    s.delta = (j == cnt - 1) ? 1e-3f : fmaxf(t_next - tc, 0.0f);
    s.sigma = nerf_expf(fminf(density - bias, 8.0f));
    s.alpha = 1.0f - nerf_expf(-s.sigma * s.delta);
    return s;
}

__device__ __forceinline__ GradSample grad_sample(const ColorGradArgs& g, uint32_t gi, size_t i, uint32_t j,
                                                  uint32_t cnt)
{
    const float tc = g.t[gi];
    const float t_next = (j == cnt - 1) ? 0.0f : g.t[gi + 1];
    return grad_terms(tc, t_next, g.density_out[(size_t)g.density_stride * i], g.bias, j, cnt);
}

// One ray of the fused render gradient.  NC > 0: every lane holds at most NC
// samples (cnt <= 64 NC), kept in registers from pass A to B and from C to D
// (the loads and exponentials of B and D are not repeated), and pass C takes
// pass A's colours and pass B's dL/dw from registers (the caller checks that
// they are the same arrays), and every load of the ray (its samples' t, next
// t, sigma, colour and density output, the ray's first and last t and target
// colour) is issued at once before pass A; NC == 0: any count, each pass
// reloads its samples.  A ray without samples writes what the passes would
// (their sums are +0 and the transmittance 1) and nothing else.
template <int NC>
__device__ __forceinline__ void render_grad_ray(const CompositeArgs& a, const ColorGradArgs& gr, uint32_t r,
                                                int lane, uint32_t start, float bs)
{
    constexpr int M = NC > 0 ? NC : 1;
    const float c23 = 2.0f / 3;
    const uint32_t off = a.offsets[r], cnt = a.counts[r];
    const float true_r = a.rgb_true[3 * r], true_g = a.rgb_true[3 * r + 1], true_b = a.rgb_true[3 * r + 2];
    if (cnt == 0) {  // wave-uniform
        if (lane == 0) {
            const float t_end = 1.0f, zero = 0.0f;
            float rc = zero, gc = zero, bc = zero;
            rc += t_end * a.bg.x;
            gc += t_end * a.bg.y;
            bc += t_end * a.bg.z;
            a.weight_sum[r] = zero;
            a.final_rgb[3 * r] = rc;
            a.final_rgb[3 * r + 1] = gc;
            a.final_rgb[3 * r + 2] = bc;
            a.final_depth[r] = zero;
            a.phi[3 * r] = 2.0f * (rc - true_r);
            a.phi[3 * r + 1] = 2.0f * (gc - true_g);
            a.phi[3 * r + 2] = 2.0f * (bc - true_b);
        }
        return;
    }
    const uint32_t run = (cnt + 63) / 64;
    const uint32_t k0 = min((uint32_t)lane * run, cnt), k1 = min(k0 + run, cnt);
    // NC > 0: the lane's samples' inputs (a lane without a sample in a slot
    // reads the ray's last sample and ignores it)
    float in_t[M], in_tn[M], in_sig[M], in_c0[M], in_c1[M], in_c2[M], in_den[M];
    if constexpr (NC > 0) {
#pragma unroll
        for (int q = 0; q < NC; q++) {
            const uint32_t i = min(k0 + (uint32_t)q, cnt - 1), idx = off + i;
            in_t[q] = a.t[idx];
            in_tn[q] = a.t[i < cnt - 1 ? idx + 1 : idx];
            in_sig[q] = a.sigma[idx];
            const float* cc = a.rgb + (size_t)a.rgb_stride * idx;
            in_c0[q] = cc[0];
            in_c1[q] = cc[1];
            in_c2[q] = cc[2];
            in_den[q] = gr.density_out[(size_t)gr.density_stride * idx];
        }
    }
    const float d_prior = a.depth_prior ? a.depth_prior[r] : -1.0f;
    const float s_prior = a.sigma_prior ? a.sigma_prior[r] : -1.0f;
    const float dwl = (d_prior >= 0) ? a.lambda_depth : 0.0f;
    const float t_near = (cnt > 0) ? fmaxf(a.t[off], 1e-4f) : 1.0f;
    const float t_far = (cnt > 0) ? a.t[off + cnt - 1] : 1.0f;
    const float g_far = 1.0f - t_near / fmaxf(t_far, t_near + 1e-4f);
    const float inv_g = (g_far > 1e-6f) ? (1.0f / g_far) : 0.0f;
    // f(sample index, cache slot) over the lane's run; the slot is a
    // compile-time constant, so the caches stay in registers
    static_assert(NC <= 2, "at most two cached samples per lane");
    auto each = [&](auto&& f) {
        if constexpr (NC > 0) {
            if (k0 < k1) f(k0, std::integral_constant<int, 0>{});
            if constexpr (NC > 1)
                if (k0 + 1 < k1) f(k0 + 1, std::integral_constant<int, 1>{});
        } else {
            for (uint32_t i = k0; i < k1; i++) f(i, std::integral_constant<int, 0>{});
        }
    };
    CompSample cs[M];
    GradSample gs[M];
    float cg_w[M], co_r[M], co_g[M], co_b[M];  // pass A's colours and pass B's dL/dw
    float d_w[M], d_r[M], d_g[M], d_b[M];      // pass C's, for pass D

    // ---- A: transmittance and weighted sums of the compositing ----
    float tl = 1.0f, sr = 0.f, sg = 0.f, sb = 0.f, sd = 0.f, sw = 0.f, swm = 0.f, se = 0.f;
    each([&](uint32_t i, int q) {
        const uint32_t idx = off + i;
        CompSample c;
        float c0, c1, c2;
        if constexpr (NC > 0) {
            c = comp_terms(in_t[q], in_tn[q], in_sig[q], i, cnt, t_near, inv_g, d_prior, s_prior);
            c0 = in_c0[q];
            c1 = in_c1[q];
            c2 = in_c2[q];
        } else {
            c = comp_sample(a, idx, i, cnt, t_near, inv_g, d_prior, s_prior);
            const float* cc = a.rgb + (size_t)a.rgb_stride * idx;
            c0 = cc[0];
            c1 = cc[1];
            c2 = cc[2];
        }
        const float w = c.alpha * tl;
        sr += w * c0;
        sg += w * c1;
        sb += w * c2;
        sd += w * c.t;
        sw += w;
        swm += w * c.m;
        se += c.e;
        tl *= (1.0f - c.alpha);
        if constexpr (NC > 0) {
            cs[q] = c;
            co_r[q] = c0;
            co_g[q] = c1;
            co_b[q] = c2;
        }
    });
    const float tj = wave_excl_prod(tl, lane);
    const float t_end = __shfl(tj * tl, 63, 64);
    const float lw = tj * sw, lwm = tj * swm;
    float rc = wave_sum(tj * sr), gc = wave_sum(tj * sg), bc = wave_sum(tj * sb);
    const float depth = wave_sum(tj * sd);
    const float dw_g = wave_sum(lw), dwm_g = wave_sum(lwm);
    const float dls = 1.0f / fmaxf(wave_sum(se), 1e-8f);
    float dw_s = wave_excl_sum(lw, lane), dwm_s = wave_excl_sum(lwm, lane);

    // ---- B: distortion (+ depth prior) gradient per weight ----
    float tr = tj, wgl = 0.0f;
    each([&](uint32_t i, int q) {
        const uint32_t idx = off + i;
        CompSample c;
        if constexpr (NC > 0) c = cs[q];
        else c = comp_sample(a, idx, i, cnt, t_near, inv_g, d_prior, s_prior);
        const float w = c.alpha * tr;
        tr *= (1.0f - c.alpha);
        const float dloss = -(c.e * dls) * (1.0f / fmaxf(w, 1e-6f));
        const float bil = c.m * (2 * dw_s - dw_g) + (dwm_g - 2 * dwm_s);
        const float g = a.lambda_dist * (2 * (bil) + c23 * w * c.ds) + dwl * dloss;
        a.dw[idx] = g;
        if constexpr (NC > 0) cg_w[q] = g;
        wgl += w * g;
        dw_s += w;
        dwm_s += w * c.m;
    });
    const float wgs = wave_sum(wgl);
    rc += t_end * a.bg.x;
    gc += t_end * a.bg.y;
    bc += t_end * a.bg.z;
    const float pr = 2.0f * (rc - true_r);
    const float pg = 2.0f * (gc - true_g);
    const float pb = 2.0f * (bc - true_b);
    if (lane == 0) {
        a.weight_sum[r] = wgs;
        a.final_rgb[3 * r] = rc;
        a.final_rgb[3 * r + 1] = gc;
        a.final_rgb[3 * r + 2] = bc;
        a.final_depth[r] = depth;
        a.phi[3 * r] = pr;
        a.phi[3 * r + 1] = pg;
        a.phi[3 * r + 2] = pb;
    }

    // ---- C: the colour gradient's transmittance and weighted sums ----
    // (the colour outputs and dL/dw of pass A and B when they are the same
    // arrays, else loaded)
    float tl2 = 1.0f, qr = 0.f, qg = 0.f, qb = 0.f, qw = 0.f;
    each([&](uint32_t j, int q) {
        const uint32_t gi = off + j;
        const size_t i = (size_t)gi - start;
        GradSample s;
        if constexpr (NC > 0) s = grad_terms(in_t[q], in_tn[q], in_den[q], gr.bias, j, cnt);
        else s = grad_sample(gr, gi, i, j, cnt);
        float c0, c1, c2, gw;
        if constexpr (NC > 0) {
            c0 = co_r[q];
            c1 = co_g[q];
            c2 = co_b[q];
            gw = cg_w[q];
        } else {
            const float* co = gr.color_out + (size_t)gr.color_stride * i;
            c0 = co[0];
            c1 = co[1];
            c2 = co[2];
            gw = gr.dw[i];
        }
        const float w = tl2 * s.alpha;
        qr += w * c0;
        qg += w * c1;
        qb += w * c2;
        qw += w * gw;
        tl2 *= (1.0f - s.alpha);
        if constexpr (NC > 0) {
            gs[q] = s;
            d_r[q] = c0;
            d_g[q] = c1;
            d_b[q] = c2;
            d_w[q] = gw;
        }
    });
    const float tj2 = wave_excl_prod(tl2, lane);
    float cr2 = wave_excl_sum(tj2 * qr, lane), cg2 = wave_excl_sum(tj2 * qg, lane);
    float cb2 = wave_excl_sum(tj2 * qb, lane), wg = wave_excl_sum(tj2 * qw, lane);

    // ---- D: colour gradient and d sigma per sample ----
    float T2 = tj2;
    each([&](uint32_t j, int q) {
        const uint32_t gi = off + j;
        const size_t i = (size_t)gi - start;
        GradSample s;
        float c_r, c_g, c_b, gw;
        if constexpr (NC > 0) {
            s = gs[q];
            c_r = d_r[q];
            c_g = d_g[q];
            c_b = d_b[q];
            gw = d_w[q];
        } else {
            s = grad_sample(gr, gi, i, j, cnt);
            const float* co = gr.color_out + (size_t)gr.color_stride * i;
            c_r = co[0];
            c_g = co[1];
            c_b = co[2];
            gw = gr.dw[i];
        }
        const float w = T2 * s.alpha;
        cr2 += w * c_r;
        cg2 += w * c_g;
        cb2 += w * c_b;
        wg += w * gw;
        float g_r = pr * w * c_r * (1.0f - c_r) * gr.loss_scale * bs;
        float g_g = pg * w * c_g * (1.0f - c_g) * gr.loss_scale * bs;
        float g_b = pb * w * c_b * (1.0f - c_b) * gr.loss_scale * bs;
        g_r = clamp_half_range(g_r);
        g_g = clamp_half_range(g_g);
        g_b = clamp_half_range(g_b);
        if (g_r != g_r || g_g != g_g || g_b != g_b) g_r = g_g = g_b = 0.0f;
        _Float16* cgo = reinterpret_cast<_Float16*>(gr.color_grad) + (size_t)gr.grad_stride * i;
        cgo[0] = to_h(g_r);
        cgo[1] = to_h(g_g);
        cgo[2] = to_h(g_b);
        for (int k = 3; k < gr.grad_stride; k++) cgo[k] = (_Float16)0.0f;
        const float dr = T2 * c_r * (1.0f - s.alpha) - (rc - cr2);
        const float dg = T2 * c_g * (1.0f - s.alpha) - (gc - cg2);
        const float db = T2 * c_b * (1.0f - s.alpha) - (bc - cb2);
        const float suffix = wgs - wg;
        float dsi = s.delta * (dr * pr + dg * pg + db * pb);
        dsi += s.delta * (gw * T2 * (1.0f - s.alpha) - suffix);
        float dsv = dsi * s.sigma * gr.loss_scale * bs;
        dsv = clamp_half_range(dsv);
        if (dsv != dsv) dsv = 0.0f;
        gr.dsigma[i] = dsv;
        T2 = T2 * (1.0f - s.alpha);
    });
}

__global__ __launch_bounds__(256) void render_grad_kernel(const CompositeArgs a, const ColorGradArgs gr,
                                                          const uint32_t* __restrict__ d_rays, uint32_t rays_max)
{
    const uint32_t R = dev_count(d_rays, rays_max);
    const int lane = threadIdx.x & 63;
    const uint32_t nwaves = gridDim.x * 4;
    const uint32_t start = gr.offsets[0];
    const float bs = 1.0f / (float)gr.total_rays;
    // pass B's dL/dw and pass A's colours are pass C's when the arrays, their
    // numbering (a batch starting at sample 0) and the sample times are the
    // same (the training step's case)
    const bool same = start == 0u && gr.initial_offset == 0u && a.dw == gr.dw && a.rgb == gr.color_out &&
                      a.rgb_stride == gr.color_stride && a.t == gr.t && a.offsets == gr.offsets &&
                      a.counts == gr.counts;
    for (uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < R; r += nwaves) {  // wave-uniform
        if (same && a.counts[r] <= 128u) render_grad_ray<2>(a, gr, r, lane, start, bs);
        else render_grad_ray<0>(a, gr, r, lane, start, bs);
    }
}

__global__ __launch_bounds__(256) void density_grad_kernel(const uint32_t* __restrict__ d_n, uint32_t n_max,
                                                           const float* __restrict__ dsigma,
                                                           const _Float16* __restrict__ cdx,
                                                           _Float16* __restrict__ dgrad)
{
    const uint32_t N = dev_count(d_n, n_max);
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const h4* src = reinterpret_cast<const h4*>(cdx + 32 * (size_t)n);
    h4* dst = reinterpret_cast<h4*>(dgrad + 16 * (size_t)n);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const h4 v = src[q];
        h4 o;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float f = (float)v[j];
            if (q == 0 && j == 0) f += dsigma[n];
            f = clamp_half_range(f);
            if (f != f) f = 0.0f;
            o[j] = to_h(f);
        }
        dst[q] = o;
    }
}

__global__ __launch_bounds__(256) void master_grid_kernel(const float* __restrict__ tmp, float* __restrict__ master,
                                                          float decay, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float prev = master[i];
    master[i] = (prev < 0.f) ? prev : fmaxf(prev * decay, tmp[i]);
}

// Fixed-order sum: block b sums elements b, b + gridDim, ... per thread, then
// a fixed tree over the workgroup; the second pass sums the partials likewise.
__global__ __launch_bounds__(256) void reduce_sum_kernel(const float* __restrict__ in, uint32_t n,
                                                         float* __restrict__ out)
{
    __shared__ float s[256];
    float acc = 0.0f;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) acc += in[i];
    s[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) s[threadIdx.x] += s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = s[0];
}

// 64 cells per wave -> one ballot -> two 32-bit words (cells 32k..32k+31 in
// word k, LSB = lowest cell), at the cascade's pyramid offset.
__global__ __launch_bounds__(256) void occupancy_bits_kernel(uint32_t* __restrict__ bits32,
                                                             const float* __restrict__ master,
                                                             const float* __restrict__ d_sum, int total, int G, int S,
                                                             float min_optical, float base_voxel)
{
    const int cell = blockIdx.x * blockDim.x + threadIdx.x;
    bool active = false;
    if (cell < total) {
        const float mean = d_sum[0] / (float)total;
        const int c = cell / G;
        const float thr = fminf((min_optical / base_voxel) / ldexpf(1.0f, c), mean);
        active = master[cell] > thr;
    }
    const uint64_t m = __ballot(active);
    const int lane = threadIdx.x & 63;
    if ((lane & 31) == 0 && cell < total) {
        const int c = cell / G;
        const int bitpos = c * S + (cell - c * G);
        bits32[bitpos >> 5] = (uint32_t)(m >> lane);
    }
}

// extractOccupancyGrid (InstantNerf.cu:882-939): one bit per query point, set
// when the master-grid cell holding it exceeds the cascade's threshold; 32
// points per output word (bit k of word i = point 32 i + k).
__global__ __launch_bounds__(256) void query_occupancy_kernel(const float* __restrict__ master,
                                                              const float* __restrict__ pos,
                                                              uint32_t* __restrict__ out, uint3 res, float3 mn,
                                                              float3 mx, float min_optical, int C, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    bool active = false;
    if (i < n) {
        const float px = pos[3 * i], py = pos[3 * i + 1], pz = pos[3 * i + 2];
        const int c = get_cascade(px, py, pz, mn, mx, C);
        const float cs = ldexpf(1.0f, c);
        const float ex = mx.x - mn.x, ey = mx.y - mn.y, ez = mx.z - mn.z;
        const float rx = (px - mn.x * cs) / (ex * cs), ry = (py - mn.y * cs) / (ey * cs);
        const float rz = (pz - mn.z * cs) / (ez * cs);
        const int vx = clamp_floor_idx(floorf(rx * (float)res.x), (int)res.x - 1);
        const int vy = clamp_floor_idx(floorf(ry * (float)res.y), (int)res.y - 1);
        const int vz = clamp_floor_idx(floorf(rz * (float)res.z), (int)res.z - 1);
        const uint32_t flat = (uint32_t)c * (res.x * res.y * res.z) + (uint32_t)vz * (res.x * res.y) +
                              (uint32_t)vy * res.x + (uint32_t)vx;
        const float base_voxel = ex / (float)res.x;
        active = master[flat] > (min_optical / base_voxel) / cs;
    }
    const uint64_t m = __ballot(active);
    const int lane = threadIdx.x & 63;
    if ((lane & 31) == 0 && i < n) out[i >> 5] = (uint32_t)(m >> lane);
}

// out[i] = src[i * stride] (k_extractDensityLogit, InstantNerf.cu:866-870).
__global__ __launch_bounds__(256) void column_kernel(const float* __restrict__ src, int stride,
                                                     float* __restrict__ out, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = src[(size_t)i * stride];
}

__global__ __launch_bounds__(256) void mip_pool_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                       uint3 ro)
{
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    const int total = (int)(ro.x * ro.y * ro.z);
    bool occ = false;
    if (o < total) {
        const int x = o % (int)ro.x, y = (o / (int)ro.x) % (int)ro.y, z = o / (int)(ro.x * ro.y);
        const int rix = 2 * (int)ro.x, riy = 2 * (int)ro.y;
#pragma unroll
        for (int dz = 0; dz < 2; ++dz)
#pragma unroll
            for (int dy = 0; dy < 2; ++dy)
#pragma unroll
                for (int dx = 0; dx < 2; ++dx) {
                    const int idx = (2 * z + dz) * (rix * riy) + (2 * y + dy) * rix + (2 * x + dx);
                    occ = occ || ((in[idx >> 3] >> (idx & 7)) & 1);
                }
    }
    const uint64_t m = __ballot(occ);
    const int lane = threadIdx.x & 63;
    if (total >= 32) {
        if ((lane & 31) == 0 && o < total) reinterpret_cast<uint32_t*>(out)[o >> 5] = (uint32_t)(m >> lane);
    } else if (threadIdx.x == 0) {
        for (int b = 0; b < (total + 7) / 8; ++b) out[b] = (uint8_t)((m >> (8 * b)) & 0xFF);
    }
}

inline int blocks_for(uint32_t n) { return (int)std::max<uint32_t>(1, (n + 255) / 256); }

}  // namespace

void sh_gather(const float3* dirs, const uint32_t* ray_idx, const uint32_t* d_n, uint32_t n_max, float bias,
               const float* density_out, __half* color_in, float* sigma, hipStream_t s)
{
    if (n_max == 0) return;
    hipLaunchKernelGGL(sh_gather_kernel, dim3(blocks_for(n_max)), dim3(256), 0, s, dirs, ray_idx, d_n, n_max, bias,
                       density_out, reinterpret_cast<_Float16*>(color_in), sigma);
    GRAFT_LAUNCH_CHECK();
}

void composite(const CompositeArgs& a, const uint32_t* d_rays, uint32_t rays_max, hipStream_t s)
{
    if (rays_max == 0) return;
    hipLaunchKernelGGL(composite_kernel, dim3(blocks_for(rays_max)), dim3(256), 0, s, a, d_rays, rays_max);
    GRAFT_LAUNCH_CHECK();
}

void composite_infer(const CompositeArgs& a, uint32_t base, uint32_t rays_done, const uint32_t* d_rays,
                     uint32_t rays_max, hipStream_t s)
{
    if (rays_max == 0) return;
    hipLaunchKernelGGL(composite_infer_kernel, dim3(blocks_for(rays_max)), dim3(256), 0, s, a, base, rays_done,
                       d_rays, rays_max);
    GRAFT_LAUNCH_CHECK();
}

void color_grad(const ColorGradArgs& a, const uint32_t* d_rays, uint32_t rays_max, hipStream_t s)
{
    if (rays_max == 0) return;
    if (a.total_rays == 0) throw std::runtime_error("color grad: totalRaysBatch must be > 0");
    if (a.density_stride < 1) throw std::runtime_error("color grad: density output stride must be >= 1");
    hipLaunchKernelGGL(color_grad_kernel, dim3(blocks_for(rays_max)), dim3(256), 0, s, a, d_rays, rays_max);
    GRAFT_LAUNCH_CHECK();
}

void render_grad(const CompositeArgs& a, const ColorGradArgs& g, const uint32_t* d_rays, uint32_t rays_max,
                 hipStream_t s)
{
    if (rays_max == 0) return;
    if (g.total_rays == 0) throw std::runtime_error("color grad: totalRaysBatch must be > 0");
    if (g.density_stride < 1) throw std::runtime_error("color grad: density output stride must be >= 1");
    if (!a.rgb_true || !a.phi) throw std::runtime_error("render_grad: needs ground truth and phi");
    const int blocks = (int)std::min<uint32_t>((rays_max + 3) / 4, (uint32_t)num_cus() * 8);
    hipLaunchKernelGGL(render_grad_kernel, dim3(blocks), dim3(256), 0, s, a, g, d_rays, rays_max);
    GRAFT_LAUNCH_CHECK();
}

void density_grad(const uint32_t* d_n, uint32_t n_max, const float* dsigma, const __half* color_dx,
                  __half* dgrad, hipStream_t s)
{
    if (n_max == 0) return;
    hipLaunchKernelGGL(density_grad_kernel, dim3(blocks_for(n_max)), dim3(256), 0, s, d_n, n_max, dsigma,
                       reinterpret_cast<const _Float16*>(color_dx), reinterpret_cast<_Float16*>(dgrad));
    GRAFT_LAUNCH_CHECK();
}

void update_master_grid(const float* tmp, float* master, float decay, uint32_t n, hipStream_t s)
{
    if (n == 0) return;
    hipLaunchKernelGGL(master_grid_kernel, dim3(blocks_for(n)), dim3(256), 0, s, tmp, master, decay, n);
    GRAFT_LAUNCH_CHECK();
}

void reduce_sum(const float* in, uint32_t n, float* partials, float* out, hipStream_t s)
{
    const int nb = std::min(1024, blocks_for(n));
    hipLaunchKernelGGL(reduce_sum_kernel, dim3(nb), dim3(256), 0, s, in, n, partials);
    GRAFT_LAUNCH_CHECK();
    hipLaunchKernelGGL(reduce_sum_kernel, dim3(1), dim3(256), 0, s, partials, (uint32_t)nb, out);
    GRAFT_LAUNCH_CHECK();
}

void update_occupancy_bits(uint32_t* bits32, const float* master, const float* d_sum, int total, int G, int S,
                           float min_optical, float base_voxel, hipStream_t s)
{
    if (total <= 0) return;
    if (G % 32 || S % 32) throw std::runtime_error("occupancy: cells per cascade must be multiples of 32");
    hipLaunchKernelGGL(occupancy_bits_kernel, dim3(blocks_for((uint32_t)total)), dim3(256), 0, s, bits32, master,
                       d_sum, total, G, S, min_optical, base_voxel);
    GRAFT_LAUNCH_CHECK();
}

void query_occupancy(const float* master, const float* pos, uint32_t* out, uint3 res, float3 mn, float3 mx,
                     float min_optical, int C, int n, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(query_occupancy_kernel, dim3(blocks_for((uint32_t)n)), dim3(256), 0, s, master, pos, out, res,
                       mn, mx, min_optical, C, n);
    GRAFT_LAUNCH_CHECK();
}

void extract_column(const float* src, int stride, float* out, int n, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(column_kernel, dim3(blocks_for((uint32_t)n)), dim3(256), 0, s, src, stride, out, n);
    GRAFT_LAUNCH_CHECK();
}

void build_mipmaps(uint8_t* bits, uint3 res, int L, int C, hipStream_t s)
{
    const uint32_t S = mip_offset(res, L);
    if (S % 8) throw std::runtime_error("occupancy: pyramid cells per cascade must be a multiple of 8");
    for (int c = 0; c < C; ++c) {
        uint8_t* cur = bits + (size_t)c * (S / 8);
        uint3 r = res;
        for (int l = 0; l < L - 1; ++l) {
            const uint3 ro = make_uint3(r.x / 2, r.y / 2, r.z / 2);
            const uint32_t cells = ro.x * ro.y * ro.z;
            if (cells == 0) break;
            if (cells >= 32 && cells % 32) throw std::runtime_error("occupancy: mip level cells must be a multiple of 32");
            uint8_t* nxt = cur + (r.x * r.y * r.z) / 8;
            hipLaunchKernelGGL(mip_pool_kernel, dim3(blocks_for(cells)), dim3(256), 0, s, cur, nxt, ro);
            GRAFT_LAUNCH_CHECK();
            cur = nxt;
            r = ro;
        }
    }
}

}  // namespace graft
