/*
 * CPU oracle for the NeRF side of the hot path (declarations and the
 * documented deviations from the reference in nerf_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels; never part of the
 * product library.  IEEE fp32, round-to-nearest-even, built with
 * -ffp-contract=off; each function follows the cited reference kernel
 * operation by operation.
 */
#include "nerf_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* Upper bound on DDA iterations per ray.  The reference loop has none; a ray
 * only gets near it when t grows past 256, where t + 1e-5f stops advancing
 * (processRays.cu:731).  The HIP kernels use the same bound. */
#define ORC_MAX_MARCH_ITERS (1 << 20)

/* ---- e^x ------------------------------------------------------------------
 * Cody & Waite range reduction (x = k ln2 + r, |r| <= ln2/2, ln2 split into a
 * 16-bit head and a tail so k*ln2_hi is exact) and the degree-7 Taylor
 * polynomial of e^r in Horner form (truncation error < 6e-9 relative), then an
 * exact scaling by 2^k.  Results below FLT_MIN are flushed to zero. */
float orc_expf(float x)
{
    if (x != x) return x;
    if (x > 89.0f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    const float kf = rintf(x * 1.44269504f);
    const int k = (int)kf;
    const float r = (x - kf * 0.693145751953125f) - kf * 1.428606765330187e-06f;
    float p = 1.98412698e-4f;
    p = p * r + 1.38888889e-3f;
    p = p * r + 8.33333333e-3f;
    p = p * r + 4.16666667e-2f;
    p = p * r + 1.66666667e-1f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, k);
}

void orc_expf_array(const float* x, float* y, size_t n)
{
    for (size_t i = 0; i < n; i++) y[i] = orc_expf(x[i]);
}

/* ---- geometry helpers (processRays.cu:11-46, 83-93) ----------------------- */

int orc_get_cascade(const float* p, const float* mn, const float* mx, int C)
{
    const float rx = fmaxf(p[0] / mx[0], p[0] / mn[0]);
    const float ry = fmaxf(p[1] / mx[1], p[1] / mn[1]);
    const float rz = fmaxf(p[2] / mx[2], p[2] / mn[2]);
    const float s = fmaxf(rx, fmaxf(ry, rz));
    if (s <= 1.0f) return 0;
    int e = 0;
    const float m = frexpf(s, &e); /* s = m * 2^e, m in [0.5, 1) */
    const int c = (m == 0.5f) ? e - 1 : e;
    return c < 0 ? 0 : (c > C - 1 ? C - 1 : c);
}

void orc_contract_pos(const float* p, const float* mn, const float* mx, float* out)
{
    for (int k = 0; k < 3; k++) {
        const float ext = mx[k] - mn[k];
        const float rel = (p[k] - mn[k]) / ext;
        const float n = rel * 2.0f - 1.0f;
        const float c = fabsf(n) <= 1.0f ? n : (2.0f - 1.0f / fabsf(n)) * copysignf(1.0f, n);
        out[k] = fmaxf(0.0f, fminf((c + 2.0f) * 0.25f, 1.0f));
    }
}

static uint32_t mip_offset(const uint32_t* res, int level)
{
    uint32_t off = 0, rx = res[0], ry = res[1], rz = res[2];
    for (int l = 0; l < level; l++) {
        off += rx * ry * rz;
        rx >>= 1;
        ry >>= 1;
        rz >>= 1;
    }
    return off;
}

uint32_t orc_pyramid_cells(const uint32_t* res, int levels) { return mip_offset(res, levels); }

/* max(0, min((int)f, hi)) with the GPU's saturating float->int conversion. */
static int clamp_floor_idx(float f, int hi)
{
    if (!(f >= 0.0f)) return 0;
    if (f >= (float)hi) return hi;
    return (int)f;
}

/* ---- compute_ray_aabb_inv_kernel (otherKernels.cu:91-154) ---------------- */
void orc_ray_aabb_inv(uint32_t R, const float* O, const float* D, const float* mn, const float* mx,
                      int C, float* DI, float* nears, float* fars)
{
    const float scale = ldexpf(1.0f, C - 1);
    float lo[3], hi[3];
    for (int k = 0; k < 3; k++) {
        lo[k] = mn[k] * scale;
        hi[k] = mx[k] * scale;
    }
    for (uint32_t i = 0; i < R; i++) {
        const float* o = O + 3 * i;
        float d[3] = {D[3 * i], D[3 * i + 1], D[3 * i + 2]};
        float t1[3], t2[3];
        for (int k = 0; k < 3; k++) {
            if (fabsf(d[k]) < 1e-8f) d[k] = 1e-8f;
            const float inv = 1.0f / d[k];
            DI[3 * i + k] = inv;
            t1[k] = (lo[k] - o[k]) * inv;
            t2[k] = (hi[k] - o[k]) * inv;
            if (t1[k] > t2[k]) {
                const float tmp = t1[k];
                t1[k] = t2[k];
                t2[k] = tmp;
            }
        }
        const float te = fmaxf(fmaxf(t1[0], t1[1]), t1[2]);
        const float tx = fminf(fminf(t2[0], t2[1]), t2[2]);
        if (te > tx || tx < 0.0f) {
            nears[i] = 0.0f;
            fars[i] = 0.0f;
        } else {
            nears[i] = fmaxf(te, 0.0f);
            fars[i] = tx;
        }
    }
}

/* expand_bits_3d / morton3d (processRays.cu:71-82): bit b of x, y, z to bits
 * 3b, 3b+1, 3b+2 of the result, coordinates taken mod 2^10. */
uint32_t orc_morton30(uint32_t x, uint32_t y, uint32_t z)
{
    uint32_t m = 0;
    for (int b = 0; b < 10; b++) {
        m |= ((x >> b) & 1u) << (3 * b);
        m |= ((y >> b) & 1u) << (3 * b + 1);
        m |= ((z >> b) & 1u) << (3 * b + 2);
    }
    return m;
}

/* ---- the hierarchical DDA of march_rays_dda_calc_hits / _offset / _kernel -
 * processRays.cu:626-737 (count), 801-929 (fill) and 96-226 (per-ray
 * layout).  fill = 0 counts only; fill = 1 writes sample `hit` at
 * out_base + hit (t, ray index i, contracted position); fill = 2 writes it at
 * i * ORC_MAX_HITS + hit (t, and the Morton code of its level-0 cell when
 * morton is set). */
static uint32_t march_one(uint32_t i, const float* O, const float* D, const float* DI, float t_min,
                          float t_max, const uint8_t* bits, const uint32_t* res, const float* mn,
                          const float* mx, int C, int L, int K, int fill, uint32_t out_base,
                          float* t_out, uint32_t* ridx, float* pos_out, uint32_t* morton)
{
    const float* o = O + 3 * i;
    const float* d = D + 3 * i;
    const float* di = DI + 3 * i;
    float ext[3];
    int stp[3];
    for (int k = 0; k < 3; k++) {
        ext[k] = mx[k] - mn[k];
        stp[k] = d[k] >= 0.0f ? 1 : -1;
    }
    const uint32_t total_cells = mip_offset(res, L);
    uint32_t hit = 0;
    float t = t_min;
    int level = L - 1;
    for (int it = 0; t < t_max && hit < ORC_MAX_HITS && it < ORC_MAX_MARCH_ITERS; it++) {
        float p[3];
        for (int k = 0; k < 3; k++) p[k] = o[k] + t * d[k];
        const int c = orc_get_cascade(p, mn, mx, C);
        const float cs = ldexpf(1.0f, c);
        float cmin[3], cext[3], vs[3];
        uint32_t rl[3];
        int vi[3];
        for (int k = 0; k < 3; k++) {
            cmin[k] = mn[k] * cs;
            cext[k] = ext[k] * cs;
            rl[k] = res[k] >> level;
            vs[k] = cext[k] / (float)rl[k];
            const float rel = (p[k] - cmin[k]) / cext[k];
            vi[k] = clamp_floor_idx(floorf(rel * (float)rl[k]), (int)rl[k] - 1);
        }
        const uint32_t flat = (uint32_t)c * total_cells + mip_offset(res, level) +
                              (uint32_t)vi[2] * (rl[0] * rl[1]) + (uint32_t)vi[1] * rl[0] + (uint32_t)vi[0];
        const int occ = (bits[flat >> 3] >> (flat & 7)) & 1;
        if (occ) {
            if (level > 0) {
                level--;
                continue;
            }
            if (!fill) {
                int n = K;
                const int rem = ORC_MAX_HITS - (int)hit;
                if (n > rem) n = rem;
                hit += (uint32_t)n;
            } else {
                float eb[3];
                for (int k = 0; k < 3; k++) eb[k] = cmin[k] + ((float)vi[k] + (stp[k] > 0 ? 1.0f : 0.0f)) * vs[k];
                const float exit_t =
                    fminf(fminf((eb[0] - o[0]) * di[0], (eb[1] - o[1]) * di[1]), (eb[2] - o[2]) * di[2]);
                const float span = exit_t - t;
                for (int k = 0; k < K; ++k) {
                    if (hit >= ORC_MAX_HITS) break;
                    const float tk = t + ((float)k + 0.5f) / (float)K * span;
                    if (fill == 2) {
                        const size_t w = (size_t)i * ORC_MAX_HITS + hit;
                        t_out[w] = tk;
                        if (morton) morton[w] = orc_morton30((uint32_t)vi[0], (uint32_t)vi[1], (uint32_t)vi[2]);
                        hit++;
                        continue;
                    }
                    const uint32_t w = out_base + hit;
                    t_out[w] = tk;
                    ridx[w] = i;
                    float q[3], cq[3];
                    for (int a = 0; a < 3; a++) q[a] = o[a] + tk * d[a];
                    orc_contract_pos(q, mn, mx, cq);
                    pos_out[4 * (size_t)w] = cq[0];
                    pos_out[4 * (size_t)w + 1] = cq[1];
                    pos_out[4 * (size_t)w + 2] = cq[2];
                    pos_out[4 * (size_t)w + 3] = 0.0f;
                    hit++;
                }
            }
        }
        float nb[3], ta[3];
        for (int k = 0; k < 3; k++) {
            nb[k] = cmin[k] + ((float)vi[k] + (stp[k] > 0 ? 1.0f : 0.0f)) * vs[k];
            ta[k] = (nb[k] - o[k]) * di[k];
        }
        const float next_t = fminf(fminf(ta[0], ta[1]), ta[2]);
        t = fmaxf(t + 1e-5f, next_t + 1e-6f);
        level = L - 1;
    }
    return hit;
}

void orc_march_count(uint32_t R, const float* O, const float* D, const float* DI, const float* nears,
                     const float* fars, const uint8_t* bits, const uint32_t* res, const float* mn,
                     const float* mx, int C, int L, int K, uint32_t* counts)
{
#pragma omp parallel for schedule(dynamic, 256)
    for (long long i = 0; i < (long long)R; i++)
        counts[i] = march_one((uint32_t)i, O, D, DI, nears[i], fars[i], bits, res, mn, mx, C, L, K, 0, 0,
                              NULL, NULL, NULL, NULL);
}

uint32_t orc_march_hits(uint32_t R, const float* O, const float* D, const float* DI, const float* nears,
                        const float* fars, const uint8_t* bits, const uint32_t* res, const float* mn,
                        const float* mx, int C, int L, int K, uint32_t batch, uint32_t* counts,
                        uint32_t* offsets, uint32_t* total_hits, float* t_out, uint32_t* ridx,
                        float* pos_out)
{
    orc_march_count(R, O, D, DI, nears, fars, bits, res, mn, mx, C, L, K, counts);
    /* custom_exclusive_sum (processRays.cu:486-549): uint32 wrap-around sums */
    uint32_t run = 0;
    for (uint32_t i = 0; i < R; i++) {
        offsets[i] = run;
        run += counts[i];
    }
    *total_hits = 0;
    if (R == 0) return 0;
    if (run == 0) return R; /* processRays.cu:984-987 */
    /* find_cutoff_ray_kernel: largest i+1 with offsets[i] + counts[i] <= batch */
    uint32_t active = 0;
    for (uint32_t i = 0; i < R; i++) {
        if (offsets[i] + counts[i] <= batch) active = i + 1;
        else break;
    }
    if (active == 0) return 0;
    *total_hits = offsets[active - 1] + counts[active - 1];
#pragma omp parallel for schedule(dynamic, 256)
    for (long long i = 0; i < (long long)active; i++)
        march_one((uint32_t)i, O, D, DI, nears[i], fars[i], bits, res, mn, mx, C, L, K, 1, offsets[i], t_out,
                  ridx, pos_out, NULL);
    return active;
}

void orc_march_fill(uint32_t R, const float* O, const float* D, const float* DI, const float* nears,
                    const float* fars, const uint8_t* bits, const uint32_t* res, const float* mn,
                    const float* mx, int C, int L, int K, const uint32_t* out_base, float* t_out,
                    uint32_t* ridx, float* pos_out)
{
#pragma omp parallel for schedule(dynamic, 256)
    for (long long i = 0; i < (long long)R; i++)
        march_one((uint32_t)i, O, D, DI, nears[i], fars[i], bits, res, mn, mx, C, L, K, 1, out_base[i], t_out,
                  ridx, pos_out, NULL);
}

void orc_sparse_batch(uint32_t N, const uint32_t* sparse_idx, const float* t_sparse, const float* O,
                      const float* D, const float* mn, const float* mx, float* pos_out, uint32_t* ridx,
                      float* t_out)
{
#pragma omp parallel for schedule(static)
    for (long long j = 0; j < (long long)N; j++) {
        const uint32_t idx = sparse_idx[j];
        const uint32_t ray = idx / ORC_MAX_HITS;
        const float t = t_sparse[idx];
        float q[3], cq[3];
        for (int a = 0; a < 3; a++) q[a] = O[3 * (size_t)ray + a] + t * D[3 * (size_t)ray + a];
        orc_contract_pos(q, mn, mx, cq);
        for (int a = 0; a < 3; a++) pos_out[4 * (size_t)j + a] = cq[a];
        pos_out[4 * (size_t)j + 3] = 0.0f;
        ridx[j] = ray;
        t_out[j] = t;
    }
}

void orc_march_sparse(uint32_t R, const float* O, const float* D, const float* DI, const float* nears,
                      const float* fars, const uint8_t* bits, const uint32_t* res, const float* mn,
                      const float* mx, int C, int L, int K, uint32_t* counts, float* t_sparse, uint32_t* morton)
{
#pragma omp parallel for schedule(dynamic, 256)
    for (long long i = 0; i < (long long)R; i++)
        counts[i] = march_one((uint32_t)i, O, D, DI, nears[i], fars[i], bits, res, mn, mx, C, L, K, 2, 0, t_sparse,
                              NULL, NULL, morton);
}

/* ---- compute_SH_gather (otherKernels.cu:156-273) -------------------------- */
static float sanitize_logit(float v)
{
    v = fmaxf(-64.0f, fminf(64.0f, v));
    return (v != v) ? 0.0f : v;
}

/* The 16 real SH of compute_SH_gather and compute_real_sh_degree_3_kernel
 * (otherKernels.cu:24-51, 182-200; one expression list in both). */
static void sh16(const float* d, float* sh)
{
    const float x = d[0], y = d[1], z = d[2];
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    sh[0] = 0.28209479f;
    sh[1] = -0.48860251f * y;
    sh[2] = 0.48860251f * z;
    sh[3] = -0.48860251f * x;
    sh[4] = 1.09254843f * x * y;
    sh[5] = -1.09254843f * y * z;
    sh[6] = 0.31539156f * (3.0f * z2 - 1.0f);
    sh[7] = -1.09254843f * x * z;
    sh[8] = 0.54627421f * (x2 - y2);
    sh[9] = -0.59004359f * y * (3.0f * x2 - y2);
    sh[10] = 2.89061144f * x * y * z;
    sh[11] = -0.45704580f * y * (5.0f * z2 - 1.0f);
    sh[12] = 0.37317633f * z * (5.0f * z2 - 3.0f);
    sh[13] = -0.45704580f * x * (5.0f * z2 - 1.0f);
    sh[14] = 1.44530572f * z * (x2 - y2);
    sh[15] = -0.59004359f * x * (x2 - 3.0f * y2);
}

/* compute_real_sh_degree_3_kernel (otherKernels.cu:18-64): out [N][16]. */
void orc_sh_degree3(uint32_t N, const float* dirs, float* out)
{
#pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; n++) sh16(dirs + 3 * (size_t)n, out + 16 * (size_t)n);
}

void orc_sh_gather(uint32_t N, const float* dirs, const uint32_t* ray_idx, float bias, const float* dout,
                   uint16_t* color_in, float* sigma)
{
#pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; n++) {
        float sh[16];
        sh16(dirs + 3 * (size_t)ray_idx[n], sh);
        float lg[16];
        for (int k = 0; k < 16; k++) lg[k] = sanitize_logit(dout[16 * (size_t)n + k]);
        sigma[n] = orc_expf(fminf(lg[0] - bias, 8.0f));
        for (int k = 0; k < 16; k++) {
            color_in[32 * (size_t)n + k] = orc_f32_to_f16(lg[k]);
            color_in[32 * (size_t)n + 16 + k] = orc_f32_to_f16(sh[k]);
        }
    }
}

/* ---- render_rays_distortion_kernel (compositing.cu:80-213) ---------------- */
static float disparity_warp(float t, float t_near, float inv_g_range)
{
    return (1.0f - t_near / fmaxf(t, 1e-4f)) * inv_g_range;
}

void orc_composite_infer(uint32_t R, uint32_t base, uint32_t rays_done, const uint32_t* offsets,
                         const uint32_t* counts, const float* ts, const float* sig, const float* rgb,
                         int rgb_stride, const float* rgb_true, float* final_rgb, float* final_depth, float* phi,
                         const float* bg)
{
#pragma omp parallel for schedule(dynamic, 256)
    for (long long r = 0; r < (long long)R; r++) {
        const uint32_t off = offsets[r + rays_done] - base, cnt = counts[r];
        float T = 1.0f, rc = 0.0f, gc = 0.0f, bc = 0.0f, depth = 0.0f;
        for (uint32_t i = 0; i < cnt; i++) {
            const uint32_t idx = off + i;
            const float t = ts[idx];
            float delta = (i < cnt - 1) ? ts[idx + 1] - t : 1e-3f;
            if (delta < 0.0f) delta = 0.0f;
            const float alpha = 1.0f - orc_expf(-sig[idx] * delta);
            const float w = alpha * T;
            const float* c = rgb + (size_t)rgb_stride * idx;
            rc += w * c[0];
            gc += w * c[1];
            bc += w * c[2];
            depth += w * t;
            T *= (1.0f - alpha);
            if (T < 1e-4f) break;
        }
        rc += T * bg[0];
        gc += T * bg[1];
        bc += T * bg[2];
        final_rgb[3 * r] = rc;
        final_rgb[3 * r + 1] = gc;
        final_rgb[3 * r + 2] = bc;
        final_depth[r] = depth;
        if (rgb_true && phi) {
            phi[3 * r] = 2.0f * (rc - rgb_true[3 * r]);
            phi[3 * r + 1] = 2.0f * (gc - rgb_true[3 * r + 1]);
            phi[3 * r + 2] = 2.0f * (bc - rgb_true[3 * r + 2]);
        }
    }
}

void orc_composite_distortion(uint32_t R, const uint32_t* offsets, const uint32_t* counts, const float* ts,
                              const float* sig, const float* depth_prior, const float* sigma_prior,
                              const float* rgb, const float* rgb_true, float* final_rgb, float* final_depth,
                              float* phi, float* dw, float* weight_sum, float lambda_dist, float lambda_depth,
                              const float* bg)
{
#pragma omp parallel for schedule(dynamic, 256)
    for (long long r = 0; r < (long long)R; r++) {
        const uint32_t off = offsets[r], cnt = counts[r];
        const float d_prior = depth_prior ? depth_prior[r] : -1.0f;
        const float s_prior = sigma_prior ? sigma_prior[r] : -1.0f;
        const float dwl = (d_prior >= 0) ? lambda_depth : 0.0f;
        const float t_near = (cnt > 0) ? fmaxf(ts[off], 1e-4f) : 1.0f;
        const float t_far = (cnt > 0) ? ts[off + cnt - 1] : 1.0f;
        const float g_far = 1.0f - t_near / fmaxf(t_far, t_near + 1e-4f);
        const float inv_g = (g_far > 1e-6f) ? (1.0f / g_far) : 0.0f;
        float T = 1.0f, rc = 0.0f, gc = 0.0f, bc = 0.0f, depth = 0.0f;
        const float c = 2.0f / 3;
        float dw_g = 0.0f, dwm_g = 0.0f, dw_s = 0.0f, dwm_s = 0.0f, dls = 0.0f;
        for (uint32_t i = 0; i < cnt; i++) {
            const uint32_t idx = off + i;
            const float t = ts[idx];
            float t_next = (i < cnt - 1) ? ts[idx + 1] : (t + 1e-3f);
            float delta = t_next - t;
            if (delta < 0.0f) {
                delta = 0.0f;
                t_next = t;
            }
            const float s = disparity_warp(t, t_near, inv_g);
            const float s_next = disparity_warp(t_next, t_near, inv_g);
            const float m = 0.5f * (s + s_next);
            const float alpha = 1.0f - orc_expf(-sig[idx] * delta);
            const float w = alpha * T;
            rc += w * rgb[3 * (size_t)idx];
            gc += w * rgb[3 * (size_t)idx + 1];
            bc += w * rgb[3 * (size_t)idx + 2];
            depth += w * t;
            T *= (1.0f - alpha);
            dw_g += w;
            dwm_g += w * m;
            const float tx = (t - d_prior) / s_prior;
            dls += orc_expf(-0.5f * tx * tx) * delta;
            dw[idx] = w;
        }
        dls = 1.0f / fmaxf(dls, 1e-8f);
        float wgs = 0.0f;
        for (uint32_t i = 0; i < cnt; i++) {
            const uint32_t idx = off + i;
            const float t = ts[idx];
            float t_next = (i < cnt - 1) ? ts[idx + 1] : (t + 1e-3f);
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
            const float w = dw[idx];
            const float tx = (t - d_prior) / s_prior;
            const float dwt = orc_expf(-0.5f * tx * tx) * delta * dls;
            const float dloss = -dwt * (1.0f / fmaxf(w, (float)1e-6));
            const float bil = m * (2 * dw_s - dw_g) + (dwm_g - 2 * dwm_s);
            const float g = lambda_dist * (2 * (bil) + c * w * ds) + dwl * dloss;
            dw[idx] = g;
            wgs += w * g;
            dw_s += w;
            dwm_s += w * m;
        }
        weight_sum[r] = wgs;
        rc += T * bg[0];
        gc += T * bg[1];
        bc += T * bg[2];
        final_rgb[3 * r] = rc;
        final_rgb[3 * r + 1] = gc;
        final_rgb[3 * r + 2] = bc;
        final_depth[r] = depth;
        if (rgb_true && phi) {
            phi[3 * r] = 2.0f * (rc - rgb_true[3 * r]);
            phi[3 * r + 1] = 2.0f * (gc - rgb_true[3 * r + 1]);
            phi[3 * r + 2] = 2.0f * (bc - rgb_true[3 * r + 2]);
        }
    }
}

/* ---- compute_color_grad (otherKernels.cu:303-409), initialOffset = 0 ------ */
static float clamp_half_range(float v) { return fmaxf(-65504.0f, fminf(65504.0f, v)); }

void orc_color_grad(uint32_t R, const uint32_t* counts, const uint32_t* offsets, const float* ts,
                    const float* dout, const float* cout, const float* phi, const float* final_rgb,
                    const float* dw, const float* weight_sum, uint16_t* cgrad, float* dsigma, float loss_scale,
                    float bias, uint32_t total_rays)
{
    const uint32_t start = R ? offsets[0] : 0;
#pragma omp parallel for schedule(dynamic, 256)
    for (long long r = 0; r < (long long)R; r++) {
        float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f, wg = 0.0f;
        const uint32_t base = offsets[r];
        const float wgs = weight_sum[r];
        const uint32_t cnt = counts[r];
        const float pr = phi[3 * r], pg = phi[3 * r + 1], pb = phi[3 * r + 2];
        const float fr = final_rgb[3 * r], fg = final_rgb[3 * r + 1], fb = final_rgb[3 * r + 2];
        for (uint32_t j = 0; j < cnt; j++) {
            const uint32_t gi = base + j;
            const size_t i = gi - start;
            const float tc = ts[gi];
            const float delta = (j == cnt - 1) ? 1e-3f : fmaxf(ts[gi + 1] - tc, 0.0f);
            const float sigma = orc_expf(fminf(dout[16 * i] - bias, 8.0f));
            const float alpha = 1.0f - orc_expf(-sigma * delta);
            const float w = T * alpha;
            const float c_r = cout[3 * i], c_g = cout[3 * i + 1], c_b = cout[3 * i + 2];
            cr += w * c_r;
            cg += w * c_g;
            cb += w * c_b;
            const float bs = 1.0f / (float)total_rays;
            float g_r = pr * w * c_r * (1.0f - c_r) * loss_scale * bs;
            float g_g = pg * w * c_g * (1.0f - c_g) * loss_scale * bs;
            float g_b = pb * w * c_b * (1.0f - c_b) * loss_scale * bs;
            g_r = clamp_half_range(g_r);
            g_g = clamp_half_range(g_g);
            g_b = clamp_half_range(g_b);
            if (g_r != g_r || g_g != g_g || g_b != g_b) g_r = g_g = g_b = 0.0f;
            cgrad[3 * i] = orc_f32_to_f16(g_r);
            cgrad[3 * i + 1] = orc_f32_to_f16(g_g);
            cgrad[3 * i + 2] = orc_f32_to_f16(g_b);
            const float sr = fr - cr, sg = fg - cg, sb = fb - cb;
            const float dr = T * c_r * (1.0f - alpha) - sr;
            const float dg = T * c_g * (1.0f - alpha) - sg;
            const float db = T * c_b * (1.0f - alpha) - sb;
            const float gw = dw[i];
            wg += w * gw;
            const float suffix = wgs - wg;
            float dsi = delta * (dr * pr + dg * pg + db * pb);
            dsi += delta * (gw * T * (1.0f - alpha) - suffix);
            float ds = dsi * sigma * loss_scale * bs;
            ds = clamp_half_range(ds);
            if (ds != ds) ds = 0.0f;
            dsigma[i] = ds;
            T = T * (1.0f - alpha);
        }
    }
}

/* ---- compute_density_grad (otherKernels.cu:497-562) ----------------------- */
void orc_density_grad(uint32_t N, const float* dsigma, const uint16_t* cdx, uint16_t* dgrad)
{
#pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; n++) {
        for (int k = 0; k < 16; k++) {
            float v = orc_f16_to_f32(cdx[32 * (size_t)n + k]);
            if (k == 0) v += dsigma[n];
            v = clamp_half_range(v);
            if (v != v) v = 0.0f;
            dgrad[16 * (size_t)n + k] = orc_f32_to_f16(v);
        }
    }
}

/* ---- occupancy (otherKernels.cu:677-807, InstantNerf.cu:1177-1204) -------- */
void orc_update_master_grid(const float* tmp, float* master, float decay, uint32_t n)
{
    for (uint32_t i = 0; i < n; i++) {
        const float prev = master[i];
        master[i] = (prev < 0.f) ? prev : fmaxf(prev * decay, tmp[i]);
    }
}

static void set_bit(uint8_t* bits, uint32_t pos, int v)
{
    if (v) bits[pos >> 3] |= (uint8_t)(1u << (pos & 7));
    else bits[pos >> 3] &= (uint8_t)~(1u << (pos & 7));
}

void orc_update_occupancy_bits(uint8_t* bits, const float* master, float sum, int total, int G, int S,
                               float min_optical, float base_voxel)
{
    const float mean = sum / (float)total;
    for (int cell = 0; cell < total; cell++) {
        const int c = cell / G;
        const float thr = fminf((min_optical / base_voxel) / ldexpf(1.0f, c), mean);
        set_bit(bits, (uint32_t)(c * S + cell % G), master[cell] > thr);
    }
}

void orc_build_mipmaps(uint8_t* bits, const uint32_t* res, int L, int C)
{
    const uint32_t S = mip_offset(res, L);
    for (int c = 0; c < C; c++) {
        uint8_t* cur = bits + (size_t)c * (S / 8);
        uint32_t rx = res[0], ry = res[1], rz = res[2];
        for (int l = 0; l < L - 1; l++) {
            const uint32_t ox = rx / 2, oy = ry / 2, oz = rz / 2;
            const uint32_t out_cells = ox * oy * oz;
            uint8_t* nxt = cur + (rx * ry * rz) / 8;
            /* words of 32 cells when out_cells >= 32, else whole bytes */
            const uint32_t written = out_cells >= 32 ? out_cells : ((out_cells + 7) / 8) * 8;
            for (uint32_t o = 0; o < written; o++) {
                int occ = 0;
                if (o < out_cells) {
                    const uint32_t x = o % ox, y = (o / ox) % oy, z = o / (ox * oy);
                    for (int dz = 0; dz < 2; dz++)
                        for (int dy = 0; dy < 2; dy++)
                            for (int dx = 0; dx < 2; dx++) {
                                const uint32_t in = (2 * z + dz) * (2 * ox * 2 * oy) + (2 * y + dy) * (2 * ox) + (2 * x + dx);
                                occ |= (cur[in >> 3] >> (in & 7)) & 1;
                            }
                }
                set_bit(nxt, o, occ);
            }
            cur = nxt;
            rx = ox;
            ry = oy;
            rz = oz;
        }
    }
}

/* ---- occupancy refresh sampling (otherKernels.cu:591-675, 852-888) ---- */
void orc_philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1)
{
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        c[1] = (uint32_t)p1;
        c[3] = (uint32_t)p0;
        c[0] = n0;
        c[2] = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

static float unit_of(uint32_t u) { return (float)(u >> 8) * 5.9604645e-8f + 2.9802322e-8f; }

void orc_occ_sample(float* out4, int N, int mode, int total_cells, int cell_offset, const int* list, int list_count,
                    uint64_t seed, const uint32_t* res3, const float* mn, const float* mx)
{
    const int G = (int)(res3[0] * res3[1] * res3[2]);
    for (int idx = 0; idx < N; idx++) {
        uint32_t c[4] = {(uint32_t)idx, 0u, (uint32_t)seed, (uint32_t)(seed >> 32)};
        orc_philox4x32_10(c, 0x3DA3ACB5u, 0xA79C5F42u);
        const float r[3] = {unit_of(c[0]), unit_of(c[1]), unit_of(c[2])};
        const float rw = unit_of(c[3]);
        int cell;
        if (mode == 0) {
            if (list_count == 0) continue;
            int k = (int)(rw * (float)list_count);
            cell = list[k < list_count - 1 ? k : list_count - 1];
        } else if (mode == 1) {
            cell = cell_offset + idx;
        } else {
            int k = (int)(rw * (float)total_cells);
            cell = cell_offset + (k < total_cells - 1 ? k : total_cells - 1);
        }
        const int cas = cell / G, local = cell % G;
        const int g[3] = {local % (int)res3[0], (local / (int)res3[0]) % (int)res3[1],
                          local / (int)(res3[0] * res3[1])};
        const float cs = ldexpf(1.0f, cas);
        float p[3], q[3];
        for (int k = 0; k < 3; k++) {
            const float lo = mn[k] * cs, hi = mx[k] * cs;
            const float size = (hi - lo) / (float)res3[k];
            p[k] = lo + ((float)g[k] + r[k]) * size;
        }
        orc_contract_pos(p, mn, mx, q);
        out4[4 * (size_t)idx] = q[0];
        out4[4 * (size_t)idx + 1] = q[1];
        out4[4 * (size_t)idx + 2] = q[2];
        memcpy(&out4[4 * (size_t)idx + 3], &cell, 4);
    }
}

void orc_occ_tmp_max(const float* samples4, const float* density_out, float* tmp, float bias, int N)
{
    for (int idx = 0; idx < N; idx++) {
        int cell;
        memcpy(&cell, &samples4[4 * (size_t)idx + 3], 4);
        const float sigma = orc_expf(fminf(density_out[16 * (size_t)idx] - bias, 8.0f));
        if (sigma > tmp[cell]) tmp[cell] = sigma;
    }
}

/* ---- training ray feed (DataLoader.cu:542-661) ---- */

uint32_t orc_pcg_hash(uint32_t input)
{
    const uint32_t state = input * 747796405u + 2891336453u;
    const uint32_t word = ((state >> ((state >> 28u) + 4u)) ^ state) * 277803737u;
    return (word >> 22u) ^ word;
}

void orc_fetch_ray_chunk(int offset, int size, int total_rays, uint32_t seed, int randomize, int width, int height,
                         float focal, const float* transforms, const uint8_t* images_rgba, float* rays_o,
                         float* rays_d, float* rgb, float* dense, float* sigma, const int* rec_frame,
                         const float* rec_u, const float* rec_v, const float* rec_D, const float* rec_sigma,
                         uint32_t num_records, float dense_fraction, float uv_scale_x, float uv_scale_y,
                         const float* bg, int holdout_every)
{
    const int pixels = width * height;
    for (int idx = 0; idx < size; idx++) {
        uint32_t global_idx;
        if (randomize) {
            const uint32_t rand_val = orc_pcg_hash((uint32_t)(offset + idx) + seed);
            if (holdout_every >= 2) {
                const int num_imgs = total_rays / pixels;
                const int num_test = (num_imgs + holdout_every - 1) / holdout_every;
                const int num_train = num_imgs - num_test;
                if (num_train < 1) {
                    global_idx = rand_val % (uint32_t)total_rays;
                } else {
                    const int train_slot = (int)(rand_val % (uint32_t)num_train);
                    const int block = train_slot / (holdout_every - 1);
                    const int within = train_slot % (holdout_every - 1);
                    const int img_idx = block * holdout_every + within + 1;
                    const uint32_t r2 = orc_pcg_hash(rand_val);
                    const int pixel_idx = (int)(r2 % (uint32_t)pixels);
                    global_idx = (uint32_t)img_idx * (uint32_t)pixels + (uint32_t)pixel_idx;
                }
            } else {
                global_idx = rand_val % (uint32_t)total_rays;
            }
        } else {
            global_idx = (uint32_t)((offset + idx) % total_rays);
        }
        int img_idx = (int)(global_idx / (uint32_t)pixels);
        const int pixel_idx = (int)(global_idx % (uint32_t)pixels);
        float px = (float)(pixel_idx % width);
        float py = (float)(pixel_idx / width);
        float out_D = -1.0f, out_sigma = -1.0f;
        if (randomize && dense_fraction > 0.0f && num_records > 0) {
            const uint32_t hsel = orc_pcg_hash(((uint32_t)idx + 0x9E3779B9u) ^ (seed * 2654435761u));
            if ((float)hsel * (1.0f / 4294967296.0f) < dense_fraction) {
                const uint32_t r = orc_pcg_hash(hsel) % num_records;
                const int f = rec_frame[r];
                if (!(holdout_every >= 2 && (f % holdout_every == 0))) {
                    img_idx = f;
                    px = rec_u[r] * uv_scale_x;
                    py = rec_v[r] * uv_scale_y;
                    out_D = rec_D[r];
                    out_sigma = rec_sigma[r];
                    int px_i = (int)(px + 0.5f), py_i = (int)(py + 0.5f);
                    px_i = px_i < 0 ? 0 : (px_i > width - 1 ? width - 1 : px_i);
                    py_i = py_i < 0 ? 0 : (py_i > height - 1 ? height - 1 : py_i);
                    global_idx = (uint32_t)img_idx * (uint32_t)pixels + (uint32_t)(py_i * width + px_i);
                }
            }
        }
        float dx = (px - (float)width * 0.5f) / focal;
        float dy = -(py - (float)height * 0.5f) / focal;
        float dz = -1.0f;
        const float inv = 1.0f / sqrtf(dx * dx + dy * dy + dz * dz);
        dx *= inv;
        dy *= inv;
        dz *= inv;
        const float* c2w = transforms + (size_t)img_idx * 16;
        rays_d[3 * idx] = c2w[0] * dx + c2w[1] * dy + c2w[2] * dz;
        rays_d[3 * idx + 1] = c2w[4] * dx + c2w[5] * dy + c2w[6] * dz;
        rays_d[3 * idx + 2] = c2w[8] * dx + c2w[9] * dy + c2w[10] * dz;
        rays_o[3 * idx] = c2w[3];
        rays_o[3 * idx + 1] = c2w[7];
        rays_o[3 * idx + 2] = c2w[11];
        const uint8_t* p = images_rgba + (size_t)global_idx * 4;
        float fr = p[0] / 255.0f, fg = p[1] / 255.0f, fb = p[2] / 255.0f;
        const float fa = p[3] / 255.0f;
        fr = fr * fa + bg[0] * (1.0f - fa);
        fg = fg * fa + bg[1] * (1.0f - fa);
        fb = fb * fa + bg[2] * (1.0f - fa);
        rgb[3 * idx] = fr;
        rgb[3 * idx + 1] = fg;
        rgb[3 * idx + 2] = fb;
        if (dense) dense[idx] = out_D;
        if (sigma) sigma[idx] = out_sigma;
    }
}
