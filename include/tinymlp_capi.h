/*
 * Flat C handle API over the TinyMLP / TinyMLPHashGrid classes, for callers
 * that cannot use C++ (ctypes, cgo, JNI).  Each function mirrors one method of
 * the reference classes (modules/TinyMLP/TinyMLP.h:35-84,
 * modules/TinyMLP/TinyMLPHashGrid.h:33-85); C++ exceptions are caught and
 * reported as a non-zero return plus tinymlp_last_error_message().
 * No counterpart exists in the reference, which is C++-only.
 */
#ifndef GRAFT_TINYMLP_CAPI_H
#define GRAFT_TINYMLP_CAPI_H

#include "tinymlp_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct TmlpNet TmlpNet;        /* TinyMLP */
typedef struct TmlpGrid TmlpGrid;      /* TinyMLPHashGrid */

/* Device pointers of the internal buffers (introspection for tests). */
typedef struct TmlpGridBuffers {
    float* master_hashtable;
    GRAFT_HALF* fwd_hashtable;
    float* hashtable_grads;
    float* hash_m;
    float* hash_v;
    float** master_weights;
    float** master_biases;
    GRAFT_HALF** fwd_weights;
    float** w_grad;
    float** b_grad;
    GRAFT_HALF** activations;
    GRAFT_HALF* dx_out;
    GRAFT_HALF* dloss;
    float* padded_inputs;
    float* padded_outputs;
    MLPGridOptions hw;
    int step;
    float** w_m;            /* MLP Adam moments, per layer */
    float** w_v;
    float** b_m;
    float** b_v;
} TmlpGridBuffers;

typedef struct TmlpNetBuffers {
    float** master_weights;
    float** master_biases;
    GRAFT_HALF** fwd_weights;
    float** w_grad;
    float** b_grad;
    GRAFT_HALF** activations;
    GRAFT_HALF* dloss;
    float* padded_outputs;
    MLPOption hw;
    int step;
    float** w_m;            /* Adam moments, per layer */
    float** w_v;
    float** b_m;
    float** b_v;
} TmlpNetBuffers;

/* ---- TinyMLPHashGrid ---- */
TmlpGrid* tmlp_grid_create(const MLPGridOptions* opt, int maxBatchSize, int inferBatchSize, unsigned seed,
                           int isTraining);
void tmlp_grid_destroy(TmlpGrid* h);
int tmlp_grid_switch_mode(TmlpGrid* h, int training);
int tmlp_grid_zero_grad(TmlpGrid* h, hipStream_t s);
int tmlp_grid_forward(TmlpGrid* h, const float* in, float* out, int batch, hipStream_t s);
int tmlp_grid_inference(TmlpGrid* h, const float* in, float* out, int batch, hipStream_t s);
/* returns 0 on success; *loss receives the mean loss when fetch != 0 */
int tmlp_grid_loss(TmlpGrid* h, const GRAFT_HALF* targets, int batch, float loss_scale, int fetch, float* loss,
                   hipStream_t s);
int tmlp_grid_backward(TmlpGrid* h, const GRAFT_HALF* custom_grad /* nullable */, int batch, hipStream_t s);
int tmlp_grid_set_split_scatter(TmlpGrid* h, int enabled);
int tmlp_grid_step(TmlpGrid* h, float lr, float b1, float b2, float eps, float loss_scale, hipStream_t s);
/* TinyMLPHashGrid::scatterAdamTable (no reference counterpart): scatter of dx [N x 2L] at positions
 * (pos_stride floats each) with the table's Adam update of the next step fused in; then
 * tmlp_grid_step_mlp (TinyMLPHashGrid::stepMlp) advances the step and updates the MLP layers.
 * tile_live (nullable, uint32 per 16 rows of dx): 0 where all 16 rows are +-0 (skipped). */
int tmlp_grid_scatter_adam_table(TmlpGrid* h, const GRAFT_HALF* dx, const float* positions, int pos_stride, int N,
                                 float lr, float b1, float b2, float eps, float loss_scale, const uint32_t* tile_live,
                                 hipStream_t s);
int tmlp_grid_step_mlp(TmlpGrid* h, float lr, float b1, float b2, float eps, float loss_scale, hipStream_t s);
int tmlp_grid_reset_step(TmlpGrid* h);
int tmlp_grid_load_weights(TmlpGrid* h, const float* host_w, const float* host_b);
int tmlp_grid_save_weights(TmlpGrid* h, float* host_w, float* host_b);
int tmlp_grid_load_hashgrid(TmlpGrid* h, const float* host_table);
int tmlp_grid_save_hashgrid(TmlpGrid* h, float* host_table);
int tmlp_grid_load_file(TmlpGrid* h, const char* path);
int tmlp_grid_save_file(TmlpGrid* h, const char* path);
int tmlp_grid_buffers(TmlpGrid* h, TmlpGridBuffers* out);

/* ---- TinyMLP ---- */
TmlpNet* tmlp_net_create(const MLPOption* opt, int maxBatchSize, int inferBatchSize, unsigned seed, int isTraining);
void tmlp_net_destroy(TmlpNet* h);
int tmlp_net_switch_mode(TmlpNet* h, int training);
int tmlp_net_zero_grad(TmlpNet* h, hipStream_t s);
int tmlp_net_forward(TmlpNet* h, const GRAFT_HALF* in, float* out, int batch, hipStream_t s);
int tmlp_net_inference(TmlpNet* h, const GRAFT_HALF* in, float* out, int batch, hipStream_t s);
int tmlp_net_loss(TmlpNet* h, const GRAFT_HALF* targets, int batch, float loss_scale, int fetch, float* loss,
                  hipStream_t s);
/* custom_grad and dx_out are nullable: the four reference overloads */
int tmlp_net_backward(TmlpNet* h, const GRAFT_HALF* custom_grad, GRAFT_HALF* dx_out, int batch, hipStream_t s);
int tmlp_net_step(TmlpNet* h, float lr, float b1, float b2, float eps, float loss_scale, hipStream_t s);
int tmlp_net_reset_step(TmlpNet* h);
int tmlp_net_load_weights(TmlpNet* h, const float* host_w, const float* host_b);
int tmlp_net_save_weights(TmlpNet* h, float* host_w, float* host_b);
int tmlp_net_load_file(TmlpNet* h, const char* path);
int tmlp_net_save_file(TmlpNet* h, const char* path);
int tmlp_net_buffers(TmlpNet* h, TmlpNetBuffers* out);

/* ---- misc ---- */
int tmlp_device_synchronize(void);
const char* tmlp_version(void);

#ifdef __cplusplus
}
#endif
#endif
