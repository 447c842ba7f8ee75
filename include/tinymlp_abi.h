/*
 * C-ABI of the MI355X (gfx950) TinyMLP hot path: the extern "C" kernel
 * launchers of the reference's modules/TinyMLP, with cudaStream_t replaced by
 * hipStream_t.  Pointers are device pointers unless stated; per-layer tensors
 * are passed, as in the reference, as DEVICE arrays of device pointers.
 *
 * Differences from the reference, all strictly safer:
 *  - an unsupported shape (e.g. maxDim > 128) or a failed launch returns a
 *    non-zero status through tinymlp_last_error() instead of a silent no-op
 *    (the launchers themselves keep the reference's void return type);
 *  - per-level hash-grid scales come from one host table (float)(base*b^l)
 *    evaluated in fp64, not from device fast-math powf.
 *
 * Usable from C (ctypes, cgo) and C++: `half` is uint16_t storage in C.
 */
#ifndef GRAFT_TINYMLP_ABI_H
#define GRAFT_TINYMLP_ABI_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
#include <hip/hip_fp16.h>
#define GRAFT_HALF half
#define GRAFT_DEFAULT(x) = x
extern "C" {
#else
#define GRAFT_HALF uint16_t
#define GRAFT_DEFAULT(x)
#endif

#define ACT_RELU 0
#define OUT_ACT_NONE 0
#define OUT_ACT_SIGMOID 1

/* modules/TinyMLP/TinyMLP.h:26-33 (same field order and sizes). */
typedef struct MLPOption {
    int inputDim;
    int hiddenDim;
    int outputDim;
    int numLayers;
    int activationType;
    int outputActivation GRAFT_DEFAULT(OUT_ACT_NONE);
} MLPOption;

/* modules/TinyMLP/TinyMLPHashGrid.h:11-23 (same field order and sizes). */
typedef struct MLPGridOptions {
    int vectorDim;
    int hiddenDim;
    int outputDim;
    int numLayers;
    int activationType;
    int tableSize;
    int numLevels;
    float b;
    int lowestSize;
    int featuresLevel;
} MLPGridOptions;

/* ---- plain fused MLP (modules/TinyMLP/TinyMLP.h:171-263) ---------------- */

/* TinyMLP.h:171-180: inference forward, no activation saves. */
void launchNetworkFusionKernel(MLPOption* opt, GRAFT_HALF* d_inputs, GRAFT_HALF** d_weights_array,
                               float** d_biases_array, float* d_outputs, int batchSize,
                               hipStream_t stream);

/* TinyMLP.h:183-194: backward; dW/db accumulated (+=); d_dx_out (nullable)
 * receives dL/dinput as fp16. */
void launchNetworkFusionBackwardKernel(MLPOption* opt, GRAFT_HALF* d_loss_output,
                                       GRAFT_HALF** d_weights_array, float** d_biases_array,
                                       GRAFT_HALF** d_activations, float** d_grad_weights,
                                       float** d_grad_biases, GRAFT_HALF* d_dx_out, int batchSize,
                                       hipStream_t stream);

/* TinyMLP.h:197-206: training forward; writes d_activations[1..numLayers-1]
 * (d_activations[0] is the caller's copy of the input). */
void launchNetworkFusionGradKernel(MLPOption* opt, GRAFT_HALF* d_inputs, GRAFT_HALF** d_activations,
                                   GRAFT_HALF** d_weights_array, float** d_biases_array,
                                   float* d_outputs, int batchSize, hipStream_t stream);

/* TinyMLP.h:209-224 */
void launchAdamWeightsOptim(MLPOption* opt, float** master_weights, GRAFT_HALF** fwd_weights,
                            float** gradients, float** m, float** v, float lr, float beta1,
                            float beta2, float epsilon, float bias_correction1,
                            float bias_correction2, float inv_loss_scale, hipStream_t stream);

/* TinyMLP.h:227-241 */
void launchAdamBiasOptim(MLPOption* opt, float** biases, float** gradients, float** m, float** v,
                         float lr, float beta1, float beta2, float epsilon,
                         float bias_correction1, float bias_correction2, float inv_loss_scale,
                         hipStream_t stream);

/* TinyMLP.h:244-255: MSE loss (+= into *total_loss) and fp16 dLoss. */
void launchMSELossGrad(const float* predictions, const GRAFT_HALF* targets, GRAFT_HALF* dLoss_out,
                       float* total_loss, int batchSize, int paddedDim, int validDim,
                       float loss_scale, hipStream_t stream,
                       int outputActivation GRAFT_DEFAULT(OUT_ACT_NONE));

/* TinyMLP.h:258-263 */
void launchZeroGradients(MLPOption* opt, float** w_grads, float** b_grads, hipStream_t stream);

/* ---- hash grid + fused MLP (modules/TinyMLP/TinyMLPHashGrid.h:172-256) -- */

/* TinyMLPHashGrid.h:172-181: inference.  d_inputs is [batch x 4] float
 * (x, y, z, pad) in [0,1]. */
void launchNetworkFusionHashTableKernel(MLPGridOptions* opt, GRAFT_HALF* d_hashtable,
                                        float* d_inputs, GRAFT_HALF** d_weights_array,
                                        float** d_biases_array, float* d_outputs, int batchSize,
                                        hipStream_t stream);

/* TinyMLPHashGrid.h:184-194: training forward; d_activations[0] receives the
 * fp16 encoding [batch x 2L], d_activations[1..] the hidden activations. */
void launchNetworkFusionHashTableGradKernel(MLPGridOptions* opt, GRAFT_HALF* d_hashtable,
                                            float* d_inputs, GRAFT_HALF** d_activations,
                                            GRAFT_HALF** d_weights_array, float** d_biases_array,
                                            float* d_outputs, int batchSize, hipStream_t stream);

/* TinyMLPHashGrid.h:196-209: backward with the hash-gradient scatter fused
 * behind the MLP backward (d_dx_out is used as scratch). */
void launchNetworkFusionHashTableBackwardKernel(MLPGridOptions* opt, GRAFT_HALF* d_loss_output,
                                                GRAFT_HALF** d_weights_array,
                                                float** d_biases_array, GRAFT_HALF** d_activations,
                                                float* d_inputs, float** d_grad_weights,
                                                float** d_grad_biases, float* d_hashtable_grads,
                                                GRAFT_HALF* d_dx_out, int batchSize,
                                                hipStream_t stream);

/* TinyMLPHashGrid.h:213-226: split path -- MLP backward writes dL/d(encoding)
 * to d_dx_out, then a scatter kernel adds into d_hashtable_grads. */
void launchNetworkFusionScatterBackwardKernel(MLPGridOptions* opt, GRAFT_HALF* d_loss_output,
                                              GRAFT_HALF** d_weights_array, float** d_biases_array,
                                              GRAFT_HALF** d_activations, float* d_inputs,
                                              float** d_grad_weights, float** d_grad_biases,
                                              float* d_hashtable_grads, GRAFT_HALF* d_dx_out,
                                              int batchSize, hipStream_t stream);

/* TinyMLPHashGrid.h:228-239 (declared, never defined in the reference):
 * here the standalone scatter of d_dx_out [batch x 2L] into the grads. */
void launchHashTableBackwardKernel(GRAFT_HALF* d_dx_out, float* d_inputs, float* d_hashtable_grads,
                                   int batchSize, int tableSize, int numLevels, float b,
                                   int lowestSize, int featuresLevel, hipStream_t stream);

/* No counterpart in the reference.  launchHashTableBackwardKernel for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): the same sum
 * (d_hashtable_grads += scatter of d_dx_out, within the scatter's tolerance)
 * with its scratch in a fixed 48 MiB static device array instead of
 * library-allocated memory; it calls no hipMalloc/hipFree.  Any batch size
 * (large batches run as consecutive sub-batches on `stream`); grids with more
 * than 8192 slices of 4096 entries, or a hashed level's resolution above 4095,
 * are rejected through tinymlp_last_error().  All calls on one GPU share the
 * array: calls that overlap on one GPU race. */
void launchHashTableBackwardKernelNoAlloc(GRAFT_HALF* d_dx_out, float* d_inputs, float* d_hashtable_grads,
                                          int batchSize, int tableSize, int numLevels, float b,
                                          int lowestSize, int featuresLevel, hipStream_t stream);

/* TinyMLPHashGrid.h:241-255: Adam over the fp32 master table; skips entries
 * whose gradient is exactly 0 and zeroes each gradient it consumes. */
void launchAdamHashGridOptim(MLPGridOptions* opt, float* master_hash, GRAFT_HALF* fwd_hash,
                             float* gradients, float* m, float* v, float lr, float beta1,
                             float beta2, float epsilon, float bias_correction1,
                             float bias_correction2, float inv_loss_scale, hipStream_t stream);

/* ---- additions with no reference counterpart ----------------------------- */

/* Standalone hash encode (no MLP): d_inputs [batch x inputStride] float,
 * d_enc_out fp16 [batch x 2L].  For encode-only callers and measurement. */
void launchHashEncodeKernel(MLPGridOptions* opt, GRAFT_HALF* d_hashtable, const float* d_inputs,
                            int inputStride, GRAFT_HALF* d_enc_out, int batchSize,
                            hipStream_t stream);

/* Status of the last launcher call on this thread: 0 = ok.  The message stays
 * valid until the next call. */
int tinymlp_last_error(void);
const char* tinymlp_last_error_message(void);

#ifdef __cplusplus
}
#endif

#undef GRAFT_DEFAULT
#endif
