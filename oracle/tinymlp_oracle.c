/*
 * CPU oracle: hash grid, fused MLPs, MSE and Adam of the reference's TinyMLP
 * module.  TEST INFRASTRUCTURE ONLY -- see oracle.h.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off, no fast-math).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* binary16 conversion                                                      */
/* ------------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) {                     /* Inf / NaN */
        if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> Inf */
    if (a < 0x38800000u) {                      /* result is subnormal or zero */
        if (a < 0x33000000u) return (uint16_t)sign;          /* < 2^-25 */
        uint32_t e = a >> 23;
        uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;              /* 14..24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (a - 0x38000000u) >> 13;       /* rebias 127 -> 15 */
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {                                /* subnormal: normalise */
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            m &= 0x3ffu;
            x = sign | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------ */
/* hash grid indexing                                                        */
/* ------------------------------------------------------------------------ */

/* networkFusionHashtable.cu:62-66 -- prime-XOR spatial hash, uint32 wrap. */
uint32_t orc_hash_coords(int cx, int cy, int cz, int T)
{
    return (((uint32_t)cx * 1u) ^ ((uint32_t)cy * 2654435761u) ^ ((uint32_t)cz * 805459861u))
           & (uint32_t)(T - 1);
}

/* networkFusionHashtable.cu:68-70 -- 1:1 lattice index for dense levels. */
uint32_t orc_dense_index(int cx, int cy, int cz, int N_l)
{
    return (uint32_t)(cx + cy * (N_l + 1) + cz * (N_l + 1) * (N_l + 1));
}

/* networkFusionHashtable.cu:367-377 -- host float arithmetic, libm. */
int orc_dense_level_start(int T, int lowestSize, float b, int numLevels)
{
    float inner = (cbrtf((float)T) - 1.0f) / (float)lowestSize;
    float cont = log2f(inner) / log2f(b);
    int d = (int)floorf(cont) + 1;
    if (d < 0) d = 0;
    if (d > numLevels) d = numLevels;
    return d;
}

void orc_level_scales(int lowestSize, float b, int numLevels, float* scale, int* res)
{
    for (int l = 0; l < numLevels; l++) {
        float s = (float)((double)lowestSize * pow((double)b, (double)l));
        if (scale) scale[l] = s;
        if (res) res[l] = (int)floorf(s);
    }
}

/* One (sample, level) corner set.  networkFusionHashtable.cu:458-498 (fwd clamp)
 * and networkFusionBackwardHashtable.cu:805-842 (bwd clamp). */
static void corners_one(const float* p, float s, int N_l, int l, int T, int dense, int bwd_clamp,
                        uint32_t idx[8], float w[8])
{
    float x_l = p[0] * s;
    float y_l = p[1] * s;
    float z_l = p[2] * s;
    float fx = floorf(x_l), fy = floorf(y_l), fz = floorf(z_l);
    int x0 = (int)fx, y0 = (int)fy, z0 = (int)fz;
    int hi = bwd_clamp ? N_l - 1 : N_l;
    x0 = x0 < hi ? x0 : hi; x0 = x0 > 0 ? x0 : 0;
    y0 = y0 < hi ? y0 : hi; y0 = y0 > 0 ? y0 : 0;
    z0 = z0 < hi ? z0 : hi; z0 = z0 > 0 ? z0 : 0;
    int x1 = x0 + 1 < N_l ? x0 + 1 : N_l;
    int y1 = y0 + 1 < N_l ? y0 + 1 : N_l;
    int z1 = z0 + 1 < N_l ? z0 + 1 : N_l;

    float wx1 = (1.0f - x_l) + fx;
    float wy1 = (1.0f - y_l) + fy;
    float wz1 = (1.0f - z_l) + fz;
    float ux = 1.0f - wx1, uy = 1.0f - wy1, uz = 1.0f - wz1;

    w[0] = (wx1 * wy1) * wz1;
    w[1] = (ux * wy1) * wz1;
    w[2] = (wx1 * uy) * wz1;
    w[3] = (ux * uy) * wz1;
    w[4] = (wx1 * wy1) * uz;
    w[5] = (ux * wy1) * uz;
    w[6] = (wx1 * uy) * uz;
    w[7] = (ux * uy) * uz;

    const int cx[8] = {x0, x1, x0, x1, x0, x1, x0, x1};
    const int cy[8] = {y0, y0, y1, y1, y0, y0, y1, y1};
    const int cz[8] = {z0, z0, z0, z0, z1, z1, z1, z1};
    uint32_t base = (uint32_t)l * (uint32_t)T * 2u;
    for (int c = 0; c < 8; c++) {
        uint32_t t = dense ? orc_dense_index(cx[c], cy[c], cz[c], N_l)
                           : orc_hash_coords(cx[c], cy[c], cz[c], T);
        idx[c] = base + t * 2u;
    }
}

void orc_hash_corners(const float* pos, int pos_stride, int N, int T, int L,
                      int lowestSize, float b, int bwd_clamp,
                      uint32_t* idx_out, float* w_out)
{
    float scale[64];
    int res[64];
    orc_level_scales(lowestSize, b, L, scale, res);
    int dls = orc_dense_level_start(T, lowestSize, b, L);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int l = 0; l < L; l++) {
            corners_one(pos + (size_t)n * pos_stride, scale[l], res[l], l, T, l < dls, bwd_clamp,
                        idx_out + ((size_t)n * L + l) * 8, w_out + ((size_t)n * L + l) * 8);
        }
    }
}

/* networkFusionHashtable.cu:441-551: __fmaf_rn chain from corner 111 outwards,
 * one RNE rounding to fp16 per feature. */
void orc_hash_encode_fwd(const float* pos, int pos_stride, int N,
                         const uint16_t* table, int T, int L, int lowestSize, float b,
                         uint16_t* enc_out)
{
    float scale[64];
    int res[64];
    orc_level_scales(lowestSize, b, L, scale, res);
    int dls = orc_dense_level_start(T, lowestSize, b, L);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int l = 0; l < L; l++) {
            uint32_t idx[8];
            float w[8];
            corners_one(pos + (size_t)n * pos_stride, scale[l], res[l], l, T, l < dls, 0, idx, w);
            for (int f = 0; f < 2; f++) {
                float acc = orc_f16_to_f32(table[idx[7] + f]) * w[7];
                for (int c = 6; c >= 0; c--) acc = fmaf(orc_f16_to_f32(table[idx[c] + f]), w[c], acc);
                enc_out[(size_t)n * 2 * L + 2 * l + f] = orc_f32_to_f16(acc);
            }
        }
    }
}

/* networkFusionBackwardHashtable.cu:783-910 (hashTableScatter_Backward).
 * Levels own disjoint slices of the table, so they run in parallel without
 * atomics; samples are summed in order in fp64. */
void orc_hash_scatter_bwd(const float* pos, int pos_stride, int N,
                          const uint16_t* denc, int T, int L, int lowestSize, float b,
                          float* grads)
{
    float scale[64];
    int res[64];
    orc_level_scales(lowestSize, b, L, scale, res);
    int dls = orc_dense_level_start(T, lowestSize, b, L);
#pragma omp parallel for schedule(dynamic, 1)
    for (int l = 0; l < L; l++) {
        size_t lev = (size_t)T * 2;
        double* acc = (double*)calloc(lev, sizeof(double));
        unsigned char* touched = (unsigned char*)calloc(lev, 1);
        for (int n = 0; n < N; n++) {
            uint32_t idx[8];
            float w[8];
            corners_one(pos + (size_t)n * pos_stride, scale[l], res[l], l, T, l < dls, 1, idx, w);
            float gx = orc_f16_to_f32(denc[(size_t)n * 2 * L + 2 * l]);
            float gy = orc_f16_to_f32(denc[(size_t)n * 2 * L + 2 * l + 1]);
            for (int c = 0; c < 8; c++) {
                size_t o = idx[c] - (size_t)l * lev;
                acc[o] += (double)(gx * w[c]);
                acc[o + 1] += (double)(gy * w[c]);
                touched[o] = touched[o + 1] = 1;
            }
        }
        float* g = grads + (size_t)l * lev;
        for (size_t i = 0; i < lev; i++)
            if (touched[i]) g[i] = (float)((double)g[i] + acc[i]);
        free(acc);
        free(touched);
    }
}

/* The same sums as orc_hash_scatter_bwd (grads written, not added to) plus,
 * per gradient word, the sum of the products' magnitudes (fp64 rounded to
 * fp32) and the number of products (zero ones included): what an error bound
 * of a reordered or fixed-point sum needs. */
void orc_hash_scatter_stats(const float* pos, int pos_stride, int N,
                            const uint16_t* denc, int T, int L, int lowestSize, float b,
                            float* grads, float* gabs, uint32_t* count)
{
    float scale[64];
    int res[64];
    orc_level_scales(lowestSize, b, L, scale, res);
    int dls = orc_dense_level_start(T, lowestSize, b, L);
    /* fp64 sums of every level, kept between calls (repeated test calls
     * would otherwise pay the first touch of fresh pages every time) */
    static double* ws = NULL;
    static size_t ws_words = 0;
    size_t need = (size_t)L * T * 4;
    if (need > ws_words) {
        free(ws);
        ws = (double*)malloc(need * sizeof(double));
        ws_words = ws ? need : 0;
        if (!ws) return;
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (int l = 0; l < L; l++) {
        size_t lev = (size_t)T * 2;
        double* acc = ws + (size_t)l * 2 * lev;
        memset(acc, 0, 2 * lev * sizeof(double));
        double* aab = acc + lev;
        uint32_t* cnt = count + (size_t)l * lev;
        memset(cnt, 0, lev * sizeof(uint32_t));
        for (int n = 0; n < N; n++) {
            uint32_t idx[8];
            float w[8];
            corners_one(pos + (size_t)n * pos_stride, scale[l], res[l], l, T, l < dls, 1, idx, w);
            float gx = orc_f16_to_f32(denc[(size_t)n * 2 * L + 2 * l]);
            float gy = orc_f16_to_f32(denc[(size_t)n * 2 * L + 2 * l + 1]);
            for (int c = 0; c < 8; c++) {
                size_t o = idx[c] - (size_t)l * lev;
                float px = gx * w[c], py = gy * w[c];
                acc[o] += (double)px;
                acc[o + 1] += (double)py;
                aab[o] += fabs((double)px);
                aab[o + 1] += fabs((double)py);
                cnt[o]++;
                cnt[o + 1]++;
            }
        }
        for (size_t i = 0; i < lev; i++) {
            grads[(size_t)l * lev + i] = (float)acc[i];
            gabs[(size_t)l * lev + i] = (float)aab[i];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* fused MLP                                                                 */
/* ------------------------------------------------------------------------ */

static inline int layer_in(int l, int inDim, int hidDim) { return l == 0 ? inDim : hidDim; }
static inline int layer_out(int l, int L, int hidDim, int outDim) { return l == L - 1 ? outDim : hidDim; }

/* networkFusion.cu:262-352 / networkFusionHashtable.cu:572-682: per layer,
 * fp32 accumulation of exact fp16 products (taken in fp64 here), + fp32 bias,
 * ReLU and fp16 rounding for hidden layers; the last layer stays fp32 with an
 * optional sigmoid 1/(1+exp(-v)) (networkFusion.cu:322-324). */
void orc_mlp_forward(const uint16_t* x, int N, int inDim, int hidDim, int outDim,
                     int numLayers, const uint16_t* W, const float* B, int out_act,
                     uint16_t* acts, float* y)
{
    int maxd = inDim > hidDim ? inDim : hidDim;
    if (outDim > maxd) maxd = outDim;
#pragma omp parallel
    {
        float* cur = (float*)malloc(sizeof(float) * maxd);
        float* nxt = (float*)malloc(sizeof(float) * maxd);
        float* wf = NULL;
        size_t wtot = 0;
        for (int l = 0; l < numLayers; l++)
            wtot += (size_t)layer_in(l, inDim, hidDim) * layer_out(l, numLayers, hidDim, outDim);
        wf = (float*)malloc(sizeof(float) * wtot);
        orc_f16_to_f32_array(W, wf, wtot);
#pragma omp for schedule(static)
        for (int n = 0; n < N; n++) {
            for (int k = 0; k < inDim; k++) cur[k] = orc_f16_to_f32(x[(size_t)n * inDim + k]);
            size_t woff = 0, boff = 0;
            for (int l = 0; l < numLayers; l++) {
                int in_l = layer_in(l, inDim, hidDim);
                int out_l = layer_out(l, numLayers, hidDim, outDim);
                for (int o = 0; o < out_l; o++) {
                    const float* wr = wf + woff + (size_t)o * in_l;
                    double acc = 0.0;
                    for (int k = 0; k < in_l; k++) acc += (double)cur[k] * (double)wr[k];
                    float v = (float)acc + B[boff + o];
                    if (l < numLayers - 1) {
                        v = v > 0.0f ? v : 0.0f;
                        uint16_t h = orc_f32_to_f16(v);
                        if (acts) acts[(size_t)(l) * N * hidDim + (size_t)n * hidDim + o] = h;
                        nxt[o] = orc_f16_to_f32(h);
                    } else {
                        if (out_act == 1) v = 1.0f / (1.0f + expf(-v));
                        y[(size_t)n * outDim + o] = v;
                    }
                }
                woff += (size_t)in_l * out_l;
                boff += out_l;
                float* t = cur; cur = nxt; nxt = t;
            }
        }
        free(cur); free(nxt); free(wf);
    }
}

/* networkFusionBackward.cu:49-646 and networkFusionBackwardHashtable.cu:71-781.
 * Rounding points: G_l is fp16 (input dy, then every dX), dW/db are fp32 sums
 * (fp64 here), dX is rounded to fp16 before the ReLU mask of the saved
 * activation (mask where act <= 0, networkFusionBackwardHashtable.cu:286-297). */
void orc_mlp_backward(const uint16_t* dy, const uint16_t* x0, const uint16_t* acts,
                      int N, int inDim, int hidDim, int outDim, int numLayers,
                      const uint16_t* W, float* dW, float* dB, uint16_t* dx)
{
    int maxd = inDim > hidDim ? inDim : hidDim;
    if (outDim > maxd) maxd = outDim;
    size_t wtot = 0, btot = 0;
    size_t woffs[16], boffs[16];
    for (int l = 0; l < numLayers; l++) {
        woffs[l] = wtot;
        boffs[l] = btot;
        wtot += (size_t)layer_in(l, inDim, hidDim) * layer_out(l, numLayers, hidDim, outDim);
        btot += layer_out(l, numLayers, hidDim, outDim);
    }
    float* wf = (float*)malloc(sizeof(float) * wtot);
    orc_f16_to_f32_array(W, wf, wtot);
    int nth = orc_num_threads();
    double* accW = (double*)calloc((size_t)nth * wtot, sizeof(double));
    double* accB = (double*)calloc((size_t)nth * btot, sizeof(double));
#pragma omp parallel
    {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        double* aW = accW + (size_t)tid * wtot;
        double* aB = accB + (size_t)tid * btot;
        float* g = (float*)malloc(sizeof(float) * maxd);
        float* gn = (float*)malloc(sizeof(float) * maxd);
        float* xin = (float*)malloc(sizeof(float) * maxd);
#pragma omp for schedule(static)
        for (int n = 0; n < N; n++) {
            for (int o = 0; o < outDim; o++) g[o] = orc_f16_to_f32(dy[(size_t)n * outDim + o]);
            for (int l = numLayers - 1; l >= 0; l--) {
                int in_l = layer_in(l, inDim, hidDim);
                int out_l = layer_out(l, numLayers, hidDim, outDim);
                /* layer input activation */
                for (int i = 0; i < in_l; i++) {
                    uint16_t h = (l == 0) ? x0[(size_t)n * inDim + i]
                                          : acts[(size_t)(l - 1) * N * hidDim + (size_t)n * hidDim + i];
                    xin[i] = orc_f16_to_f32(h);
                }
                const float* wl = wf + woffs[l];
                double* aw = aW + woffs[l];
                for (int o = 0; o < out_l; o++) {
                    double go = g[o];
                    aB[boffs[l] + o] += go;
                    if (go != 0.0)
                        for (int i = 0; i < in_l; i++) aw[(size_t)o * in_l + i] += go * (double)xin[i];
                }
                for (int i = 0; i < in_l; i++) {
                    double acc = 0.0;
                    for (int o = 0; o < out_l; o++) acc += (double)g[o] * (double)wl[(size_t)o * in_l + i];
                    uint16_t h = orc_f32_to_f16((float)acc);
                    if (l == 0) {
                        if (dx) dx[(size_t)n * inDim + i] = h;
                    } else {
                        gn[i] = (xin[i] <= 0.0f) ? 0.0f : orc_f16_to_f32(h);
                    }
                }
                float* t = g; g = gn; gn = t;
            }
        }
        free(g); free(gn); free(xin);
    }
    for (size_t j = 0; j < wtot; j++) {
        double s = 0.0;
        for (int t = 0; t < nth; t++) s += accW[(size_t)t * wtot + j];
        dW[j] = (float)((double)dW[j] + s);
    }
    for (size_t j = 0; j < btot; j++) {
        double s = 0.0;
        for (int t = 0; t < nth; t++) s += accB[(size_t)t * btot + j];
        dB[j] = (float)((double)dB[j] + s);
    }
    free(accW); free(accB); free(wf);
}

/* ------------------------------------------------------------------------ */
/* loss and optimizer                                                        */
/* ------------------------------------------------------------------------ */

/* optimizerKernel.cu:169-224 with grad_scale from :388. */
double orc_mse_loss_grad(const float* pred, const uint16_t* tgt, uint16_t* dloss,
                         int N, int paddedDim, int validDim, float loss_scale, int out_act)
{
    float grad_scale = (2.0f / (float)(N * validDim)) * loss_scale;
    size_t ne = (size_t)N * paddedDim;
    double total = 0.0;
#pragma omp parallel for reduction(+ : total) schedule(static)
    for (long long i = 0; i < (long long)ne; i++) {
        int col = (int)(i % paddedDim);
        float p = pred[i];
        float t = orc_f16_to_f32(tgt[i]);
        float diff = (col < validDim) ? (p - t) : 0.0f;
        total += (double)(diff * diff);
        float gr = diff * grad_scale;
        if (out_act == 1) gr *= p * (1.0f - p);
        dloss[i] = orc_f32_to_f16(gr);
    }
    return total;
}

static inline float finite_or_zero(float x) { return isfinite(x) ? x : 0.0f; }

/* optimizerKernel.cu:16-64 (weights; the bias kernel :66-113 is the same
 * update without the fp16 copy). */
void orc_adam_dense(float* w, uint16_t* w16, const float* g, float* m, float* v, size_t n,
                    float lr, float beta1, float beta2, float eps,
                    float bc1, float bc2, float inv_loss_scale)
{
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) {
        float gg = finite_or_zero(g[i] * inv_loss_scale);
        float mv = finite_or_zero(m[i]);
        float vv = finite_or_zero(v[i]);
        float wv = w[i];
        if (!isfinite(wv)) wv = 0.0f;
        mv = beta1 * mv + (1.0f - beta1) * gg;
        vv = beta2 * vv + ((1.0f - beta2) * gg) * gg;
        float mh = mv / bc1;
        float vh = vv / bc2;
        wv = wv - ((lr * mh) / (sqrtf(vh) + eps));
        if (!isfinite(wv)) wv = 0.0f;
        m[i] = mv;
        v[i] = vv;
        w[i] = wv;
        if (w16) w16[i] = orc_f32_to_f16(wv);
    }
}

/* optimizerKernel.cu:116-167. */
void orc_adam_hash(float* w, uint16_t* w16, float* g, float* m, float* v, size_t n,
                   float lr, float beta1, float beta2, float eps,
                   float bc1, float bc2, float inv_loss_scale)
{
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) {
        float graw = g[i];
        if (graw == 0.0f) continue;
        g[i] = 0.0f;
        float gg = finite_or_zero(graw * inv_loss_scale);
        float mv = beta1 * finite_or_zero(m[i]) + (1.0f - beta1) * gg;
        float vv = beta2 * finite_or_zero(v[i]) + ((1.0f - beta2) * gg) * gg;
        float mh = mv / bc1;
        float vh = vv / bc2;
        float wv = w[i];
        if (!isfinite(wv)) wv = 0.0f;
        wv = wv - ((lr * mh) / (sqrtf(vh) + eps));
        if (!isfinite(wv)) wv = 0.0f;
        m[i] = mv;
        v[i] = vv;
        w[i] = wv;
        if (w16) w16[i] = orc_f32_to_f16(wv);
    }
}

/* TinyMLP.cu:392-404: step capped at 50,000; corrections in float via powf. */
void orc_adam_bias_corrections(float beta1, float beta2, int step, float* bc1, float* bc2)
{
    if (step > 50000) step = 50000;
    *bc1 = 1.0f - powf(beta1, (float)step);
    *bc2 = 1.0f - powf(beta2, (float)step);
}

int orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
