/*
 * CPU oracle for the 3DMaker per-sample training hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline
 * leg).  It is never linked into, loaded by, or used as a fallback of the
 * product library (3dmaker_amd/).
 *
 * Every function restates the arithmetic of one reference kernel, cited as
 * file:line relative to the reference checkout.  Arithmetic is IEEE-754 fp32
 * with round-to-nearest-even, built with -ffp-contract=off so that an FMA
 * appears only where the reference writes __fmaf_rn.  Sums whose order the
 * reference leaves to hardware (WMMA accumulation, fp32 atomics) are taken in
 * fp64 here and rounded once: the HIP path is compared to them by tolerance.
 *
 * fp16 values are passed as raw IEEE binary16 bit patterns (uint16_t).
 */
#ifndef GRAFT_ORACLE_H
#define GRAFT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- binary16 <-> binary32, round-to-nearest-even (IEEE 754-2008 5.4.2) -- */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);
void     orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void     orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* ---- hash grid indexing (networkFusionHashtable.cu:62-70, 367-377) ------- */
uint32_t orc_hash_coords(int cx, int cy, int cz, int T);
uint32_t orc_dense_index(int cx, int cy, int cz, int N_l);
int      orc_dense_level_start(int T, int lowestSize, float b, int numLevels);
/* Canonical per-level scale: scale[l] = (float)(lowestSize * pow((double)b, l)),
 * res[l] = floor(scale[l]).  Both the oracle and the HIP kernels read this one
 * table (the reference derives it on device with fast-math __powf). */
void     orc_level_scales(int lowestSize, float b, int numLevels, float* scale, int* res);

/* Per (sample, level): the 8 corner element offsets (l*T*F + idx*F) and the 8
 * trilinear weights, in the reference corner order 000,100,010,110,001,101,011,111.
 * bwd_clamp = 0: forward clamp x0 in [0, N_l] (networkFusionHashtable.cu:458-474)
 * bwd_clamp = 1: scatter clamp x0 in [0, N_l-1] (networkFusionBackwardHashtable.cu:805-833)
 * idx_out/w_out: [N][L][8]. */
void orc_hash_corners(const float* pos, int pos_stride, int N, int T, int L,
                      int lowestSize, float b, int bwd_clamp,
                      uint32_t* idx_out, float* w_out);

/* Encode forward (networkFusionHashtable.cu:441-551): enc fp16 [N][2L]. */
void orc_hash_encode_fwd(const float* pos, int pos_stride, int N,
                         const uint16_t* table, int T, int L, int lowestSize, float b,
                         uint16_t* enc_out);

/* Scatter backward (networkFusionBackwardHashtable.cu:783-910):
 * grads[L*T*2] += sum over samples of g_f * w_c.  Products are fp32 as in the
 * reference; the sum over colliding samples is taken in fp64. */
void orc_hash_scatter_bwd(const float* pos, int pos_stride, int N,
                          const uint16_t* denc, int T, int L, int lowestSize, float b,
                          float* grads);

/* The same sums written to grads (not added), with per gradient word the sum
 * of the products' magnitudes and the number of products: the inputs of an
 * error bound for a reordered or fixed-point sum (test infrastructure). */
void orc_hash_scatter_stats(const float* pos, int pos_stride, int N,
                            const uint16_t* denc, int T, int L, int lowestSize, float b,
                            float* grads, float* gabs, uint32_t* count);

/* ---- fused MLP (networkFusion.cu:197-355, networkFusionHashtable.cu:572-682) --
 * Layer l maps in_l -> out_l with W_l fp16 row-major [out_l][in_l] and b_l fp32.
 * in_0 = inDim, out_{L-1} = outDim, all others hidDim.  Hidden activations are
 * ReLU'd and rounded to fp16; the last layer is fp32 (+ sigmoid if out_act=1).
 * W and B are flat concatenations of the layers in order.
 * acts (nullable): fp16 [N][hid] per hidden layer, concatenated (L-1 blocks). */
void orc_mlp_forward(const uint16_t* x, int N, int inDim, int hidDim, int outDim,
                     int numLayers, const uint16_t* W, const float* B, int out_act,
                     uint16_t* acts, float* y);

/* MLP backward (networkFusionBackward.cu:49-646,
 * networkFusionBackwardHashtable.cu:71-781 with COMPUTE_HASHGRAD=0):
 *   dW_l += G_l^T X_l, db_l += colsum(G_l), G_{l-1} = fp16(G_l W_l) masked
 *   where the saved activation X_l <= 0 (l >= 1); dx = fp16(G_0 W_0) unmasked.
 * dy fp16 [N][outDim]; x0 fp16 [N][inDim]; acts as written by orc_mlp_forward.
 * dW, dB flat like W, B (accumulated +=).  dx (nullable) fp16 [N][inDim]. */
void orc_mlp_backward(const uint16_t* dy, const uint16_t* x0, const uint16_t* acts,
                      int N, int inDim, int hidDim, int outDim, int numLayers,
                      const uint16_t* W, float* dW, float* dB, uint16_t* dx);

/* ---- loss and optimizer (optimizerKernel.cu) ----------------------------- */
/* fusedMSELossGrad_Kernel (optimizerKernel.cu:169-224, launcher :369-401).
 * Returns the summed squared error (the value the kernel atomically adds). */
double orc_mse_loss_grad(const float* pred, const uint16_t* tgt, uint16_t* dloss,
                         int N, int paddedDim, int validDim, float loss_scale, int out_act);

/* fusedAdamWeightsOptim / fusedAdamBiasOptim (optimizerKernel.cu:16-113):
 * dense update of n parameters; w16 (nullable) receives the fp16 copy. */
void orc_adam_dense(float* w, uint16_t* w16, const float* g, float* m, float* v, size_t n,
                    float lr, float beta1, float beta2, float eps,
                    float bc1, float bc2, float inv_loss_scale);

/* fusedAdamHashGridOptim (optimizerKernel.cu:116-167): skips entries whose raw
 * gradient is exactly 0.0f and zeroes the gradient after use. */
void orc_adam_hash(float* w, uint16_t* w16, float* g, float* m, float* v, size_t n,
                   float lr, float beta1, float beta2, float eps,
                   float bc1, float bc2, float inv_loss_scale);

/* Host-side bias corrections of TinyMLP::step (TinyMLP.cu:392-404). */
void orc_adam_bias_corrections(float beta1, float beta2, int step, float* bc1, float* bc2);

/* ---- utilities ------------------------------------------------------------ */
int orc_num_threads(void);
void orc_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
