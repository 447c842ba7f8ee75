// extern "C" surface: the reference's TinyMLP kernel launchers
// (modules/TinyMLP/TinyMLP.h:171-263, TinyMLPHashGrid.h:172-256) and the flat
// handle API over the classes.  Exceptions never cross this boundary: they
// become a non-zero tinymlp_last_error() and a message on stderr.
#include "TinyMLP.h"
#include "TinyMLPHashGrid.h"
#include "tinymlp_abi.h"
#include "tinymlp_capi.h"

#include "abi_error.h"
#include "capi_handles.h"
#include "common.h"
#include "hashgrid.h"
#include "mlp.h"
#include "optimizer.h"
#include "scatter.h"

#include <cstdio>
#include <string>

namespace {

using graft::guarded;

graft::MlpShape shape(const MLPOption* o)
{
    return graft::MlpShape{o->inputDim, o->hiddenDim, o->outputDim, o->numLayers};
}

graft::MlpShape shape(const MLPGridOptions* o)
{
    return graft::MlpShape{o->numLevels * o->featuresLevel, o->hiddenDim, o->outputDim, o->numLayers};
}

graft::GridMeta meta(const MLPGridOptions* o)
{
    if (o->featuresLevel != 2) throw std::runtime_error("featuresLevel must be 2");
    return graft::make_grid_meta(o->tableSize, o->numLevels, o->b, o->lowestSize);
}

graft::LayerSizes wsizes(const MLPOption* o)
{
    graft::LayerSizes s{};
    for (int l = 0; l < o->numLayers; l++)
        s.n[l] = (l == 0 ? o->inputDim : o->hiddenDim) * (l == o->numLayers - 1 ? o->outputDim : o->hiddenDim);
    return s;
}

graft::LayerSizes bsizes(const MLPOption* o)
{
    graft::LayerSizes s{};
    for (int l = 0; l < o->numLayers; l++) s.n[l] = l == o->numLayers - 1 ? o->outputDim : o->hiddenDim;
    return s;
}

graft::AdamArgs adam(float lr, float b1, float b2, float eps, float bc1, float bc2, float ils)
{
    return graft::AdamArgs{lr, b1, b2, eps, bc1, bc2, ils};
}

thread_local int t_err = 0;
thread_local std::string t_msg;

}  // namespace

void graft::set_last_error(int code, const std::string& msg)
{
    t_err = code;
    t_msg = msg;
    if (code) std::fprintf(stderr, "[tinymlp] %s\n", msg.c_str());
}

extern "C" {

int tinymlp_last_error(void) { return t_err; }
const char* tinymlp_last_error_message(void) { return t_msg.c_str(); }

// ---------------------------------------------------------------------------
// plain MLP launchers
// ---------------------------------------------------------------------------

void launchNetworkFusionKernel(MLPOption* opt, half* d_inputs, half** W, float** B, float* d_outputs, int batchSize,
                               hipStream_t stream)
{
    guarded("launchNetworkFusionKernel", [&] {
        graft::FwdInput in;
        in.x = d_inputs;
        graft::mlp_forward(shape(opt), in, W, B, nullptr, d_outputs, batchSize, opt->outputActivation, stream);
    });
}

void launchNetworkFusionGradKernel(MLPOption* opt, half* d_inputs, half** acts, half** W, float** B,
                                   float* d_outputs, int batchSize, hipStream_t stream)
{
    guarded("launchNetworkFusionGradKernel", [&] {
        graft::FwdInput in;
        in.x = d_inputs;
        graft::mlp_forward(shape(opt), in, W, B, acts, d_outputs, batchSize, opt->outputActivation, stream);
    });
}

void launchNetworkFusionBackwardKernel(MLPOption* opt, half* d_loss_output, half** W, float** /*B*/, half** acts,
                                       float** dW, float** dB, half* d_dx_out, int batchSize, hipStream_t stream)
{
    guarded("launchNetworkFusionBackwardKernel", [&] {
        graft::mlp_backward(shape(opt), d_loss_output, acts, W, dW, dB, d_dx_out, batchSize, stream);
    });
}

void launchAdamWeightsOptim(MLPOption* opt, float** master_weights, half** fwd_weights, float** gradients,
                            float** m, float** v, float lr, float beta1, float beta2, float epsilon, float bc1,
                            float bc2, float inv_loss_scale, hipStream_t stream)
{
    guarded("launchAdamWeightsOptim", [&] {
        graft::adam_layers(master_weights, fwd_weights, gradients, m, v, wsizes(opt), opt->numLayers,
                           adam(lr, beta1, beta2, epsilon, bc1, bc2, inv_loss_scale), stream);
    });
}

void launchAdamBiasOptim(MLPOption* opt, float** biases, float** gradients, float** m, float** v, float lr,
                         float beta1, float beta2, float epsilon, float bc1, float bc2, float inv_loss_scale,
                         hipStream_t stream)
{
    guarded("launchAdamBiasOptim", [&] {
        graft::adam_layers(biases, nullptr, gradients, m, v, bsizes(opt), opt->numLayers,
                           adam(lr, beta1, beta2, epsilon, bc1, bc2, inv_loss_scale), stream);
    });
}

void launchMSELossGrad(const float* predictions, const half* targets, half* dLoss_out, float* total_loss,
                       int batchSize, int paddedDim, int validDim, float loss_scale, hipStream_t stream,
                       int outputActivation)
{
    guarded("launchMSELossGrad", [&] {
        graft::mse_loss_grad(predictions, targets, dLoss_out, total_loss, batchSize, paddedDim, validDim, loss_scale,
                             outputActivation, stream);
    });
}

void launchZeroGradients(MLPOption* opt, float** w_grads, float** b_grads, hipStream_t stream)
{
    guarded("launchZeroGradients", [&] {
        graft::zero_layers(w_grads, b_grads, wsizes(opt), bsizes(opt), opt->numLayers, stream);
    });
}

// ---------------------------------------------------------------------------
// hash grid launchers
// ---------------------------------------------------------------------------

void launchNetworkFusionHashTableKernel(MLPGridOptions* opt, half* d_hashtable, float* d_inputs, half** W,
                                        float** B, float* d_outputs, int batchSize, hipStream_t stream)
{
    guarded("launchNetworkFusionHashTableKernel", [&] {
        const graft::GridMeta m = meta(opt);
        graft::FwdInput in;
        in.pos = d_inputs;
        in.pos_stride = 4;
        in.table = d_hashtable;
        in.meta = &m;
        graft::mlp_forward(shape(opt), in, W, B, nullptr, d_outputs, batchSize, OUT_ACT_NONE, stream);
    });
}

void launchNetworkFusionHashTableGradKernel(MLPGridOptions* opt, half* d_hashtable, float* d_inputs, half** acts,
                                            half** W, float** B, float* d_outputs, int batchSize,
                                            hipStream_t stream)
{
    guarded("launchNetworkFusionHashTableGradKernel", [&] {
        const graft::GridMeta m = meta(opt);
        graft::FwdInput in;
        in.pos = d_inputs;
        in.pos_stride = 4;
        in.table = d_hashtable;
        in.meta = &m;
        graft::mlp_forward(shape(opt), in, W, B, acts, d_outputs, batchSize, OUT_ACT_NONE, stream);
    });
}

static void hash_backward(MLPGridOptions* opt, half* dloss, half** W, half** acts, float* d_inputs, float** dW,
                          float** dB, float* grads, half* dx, int batchSize, hipStream_t stream)
{
    const graft::GridMeta m = meta(opt);
    if (!dx) throw std::runtime_error("d_dx_out must not be null");
    graft::mlp_backward(shape(opt), dloss, acts, W, dW, dB, dx, batchSize, stream);
    graft::hash_scatter(m, dx, d_inputs, 4, grads, batchSize, stream);
}

void launchNetworkFusionHashTableBackwardKernel(MLPGridOptions* opt, half* d_loss_output, half** W, float** /*B*/,
                                                half** acts, float* d_inputs, float** dW, float** dB,
                                                float* d_hashtable_grads, half* d_dx_out, int batchSize,
                                                hipStream_t stream)
{
    guarded("launchNetworkFusionHashTableBackwardKernel", [&] {
        hash_backward(opt, d_loss_output, W, acts, d_inputs, dW, dB, d_hashtable_grads, d_dx_out, batchSize, stream);
    });
}

void launchNetworkFusionScatterBackwardKernel(MLPGridOptions* opt, half* d_loss_output, half** W, float** /*B*/,
                                              half** acts, float* d_inputs, float** dW, float** dB,
                                              float* d_hashtable_grads, half* d_dx_out, int batchSize,
                                              hipStream_t stream)
{
    guarded("launchNetworkFusionScatterBackwardKernel", [&] {
        hash_backward(opt, d_loss_output, W, acts, d_inputs, dW, dB, d_hashtable_grads, d_dx_out, batchSize, stream);
    });
}

void launchHashTableBackwardKernel(half* d_dx_out, float* d_inputs, float* d_hashtable_grads, int batchSize,
                                   int tableSize, int numLevels, float b, int lowestSize, int featuresLevel,
                                   hipStream_t stream)
{
    guarded("launchHashTableBackwardKernel", [&] {
        if (featuresLevel != 2) throw std::runtime_error("featuresLevel must be 2");
        const graft::GridMeta m = graft::make_grid_meta(tableSize, numLevels, b, lowestSize);
        graft::hash_scatter(m, d_dx_out, d_inputs, 4, d_hashtable_grads, batchSize, stream);
    });
}

void launchHashTableBackwardKernelNoAlloc(half* d_dx_out, float* d_inputs, float* d_hashtable_grads, int batchSize,
                                          int tableSize, int numLevels, float b, int lowestSize, int featuresLevel,
                                          hipStream_t stream)
{
    guarded("launchHashTableBackwardKernelNoAlloc", [&] {
        if (featuresLevel != 2) throw std::runtime_error("featuresLevel must be 2");
        const graft::GridMeta m = graft::make_grid_meta(tableSize, numLevels, b, lowestSize);
        graft::hash_scatter_noalloc(m, d_dx_out, d_inputs, 4, d_hashtable_grads, batchSize, stream);
    });
}

void launchAdamHashGridOptim(MLPGridOptions* opt, float* master_hash, half* fwd_hash, float* gradients, float* m,
                             float* v, float lr, float beta1, float beta2, float epsilon, float bc1, float bc2,
                             float inv_loss_scale, hipStream_t stream)
{
    guarded("launchAdamHashGridOptim", [&] {
        const size_t n = (size_t)opt->numLevels * opt->tableSize * opt->featuresLevel;
        graft::adam_hash(master_hash, fwd_hash, gradients, m, v, n,
                         adam(lr, beta1, beta2, epsilon, bc1, bc2, inv_loss_scale), stream);
    });
}

void launchHashEncodeKernel(MLPGridOptions* opt, half* d_hashtable, const float* d_inputs, int inputStride,
                            half* d_enc_out, int batchSize, hipStream_t stream)
{
    guarded("launchHashEncodeKernel", [&] {
        const graft::GridMeta m = meta(opt);
        graft::hash_encode(m, d_hashtable, d_inputs, inputStride, d_enc_out, batchSize, stream);
    });
}

// ---------------------------------------------------------------------------
// flat handle API
// ---------------------------------------------------------------------------


TmlpGrid* tmlp_grid_create(const MLPGridOptions* opt, int maxBatchSize, int inferBatchSize, unsigned seed,
                           int isTraining)
{
    TmlpGrid* h = nullptr;
    guarded("tmlp_grid_create", [&] {
        h = new TmlpGrid{new TinyMLPHashGrid(*opt, maxBatchSize, inferBatchSize, seed, isTraining != 0), true};
    });
    return h;
}

void tmlp_grid_destroy(TmlpGrid* h)
{
    if (!h || !h->owned) return;
    delete h->g;
    delete h;
}

#define GRID_CALL(name, body) guarded(name, [&] { if (!h) throw std::runtime_error("null handle"); body; })

int tmlp_grid_switch_mode(TmlpGrid* h, int training)
{
    return GRID_CALL("switch_mode", training ? h->g->switchToTrainingMode() : h->g->switchToInferenceMode());
}
int tmlp_grid_zero_grad(TmlpGrid* h, hipStream_t s) { return GRID_CALL("zero_grad", h->g->zero_grad(s)); }
int tmlp_grid_forward(TmlpGrid* h, const float* in, float* out, int batch, hipStream_t s)
{
    return GRID_CALL("forward", h->g->forward(in, out, batch, s));
}
int tmlp_grid_inference(TmlpGrid* h, const float* in, float* out, int batch, hipStream_t s)
{
    return GRID_CALL("inference", h->g->inference(in, out, batch, s));
}
int tmlp_grid_loss(TmlpGrid* h, const half* targets, int batch, float loss_scale, int fetch, float* loss,
                   hipStream_t s)
{
    return GRID_CALL("calculate_loss_and_grad", {
        const float v = h->g->calculate_loss_and_grad(targets, batch, loss_scale, fetch != 0, s);
        if (loss) *loss = v;
    });
}
int tmlp_grid_backward(TmlpGrid* h, const half* custom, int batch, hipStream_t s)
{
    return GRID_CALL("backward", custom ? h->g->backward(custom, batch, s) : h->g->backward(batch, s));
}
int tmlp_grid_set_split_scatter(TmlpGrid* h, int enabled) { return GRID_CALL("setSplitScatter", h->g->setSplitScatter(enabled != 0)); }
int tmlp_grid_step(TmlpGrid* h, float lr, float b1, float b2, float eps, float loss_scale, hipStream_t s)
{
    return GRID_CALL("step", h->g->step(lr, b1, b2, eps, loss_scale, s));
}
int tmlp_grid_scatter_adam_table(TmlpGrid* h, const GRAFT_HALF* dx, const float* positions, int pos_stride, int N,
                                 float lr, float b1, float b2, float eps, float loss_scale, const uint32_t* tile_live,
                                 hipStream_t s)
{
    return GRID_CALL("scatterAdamTable", {
        if (N < 0) throw std::runtime_error("N must be >= 0");
        if (N > 0 && (!dx || !positions)) throw std::runtime_error("null argument");
        h->g->scatterAdamTable(reinterpret_cast<const half*>(dx), positions, pos_stride, N, nullptr, lr, b1, b2, eps,
                               loss_scale, s, nullptr, tile_live);
    });
}
int tmlp_grid_step_mlp(TmlpGrid* h, float lr, float b1, float b2, float eps, float loss_scale, hipStream_t s)
{
    return GRID_CALL("stepMlp", h->g->stepMlp(lr, b1, b2, eps, loss_scale, s));
}
int tmlp_grid_reset_step(TmlpGrid* h) { return GRID_CALL("reset_step", h->g->reset_step()); }
int tmlp_grid_load_weights(TmlpGrid* h, const float* w, const float* b) { return GRID_CALL("loadWeights", h->g->loadWeights(w, b)); }
int tmlp_grid_save_weights(TmlpGrid* h, float* w, float* b) { return GRID_CALL("saveWeights", h->g->saveWeights(w, b)); }
int tmlp_grid_load_hashgrid(TmlpGrid* h, const float* t) { return GRID_CALL("loadHashgrid", h->g->loadHashgrid(t)); }
int tmlp_grid_save_hashgrid(TmlpGrid* h, float* t) { return GRID_CALL("saveHashgrid", h->g->saveHashgrid(t)); }
int tmlp_grid_load_file(TmlpGrid* h, const char* p) { return GRID_CALL("loadWeights(file)", h->g->loadWeights(std::string(p))); }
int tmlp_grid_save_file(TmlpGrid* h, const char* p) { return GRID_CALL("saveWeights(file)", h->g->saveWeights(std::string(p))); }
int tmlp_grid_buffers(TmlpGrid* h, TmlpGridBuffers* out)
{
    return GRID_CALL("buffers", {
        const TinyMLPHashGrid::Buffers b = h->g->buffers();
        out->master_hashtable = b.master_hashtable;
        out->fwd_hashtable = b.fwd_hashtable;
        out->hashtable_grads = b.hashtable_grads;
        out->hash_m = b.hash_m;
        out->hash_v = b.hash_v;
        out->master_weights = b.master_weights;
        out->master_biases = b.master_biases;
        out->fwd_weights = b.fwd_weights;
        out->w_grad = b.w_grad;
        out->b_grad = b.b_grad;
        out->activations = b.activations;
        out->dx_out = b.dx_out;
        out->dloss = b.dloss;
        out->padded_inputs = b.padded_inputs;
        out->padded_outputs = b.padded_outputs;
        out->hw = b.hw;
        out->step = b.step;
        out->w_m = b.w_m;
        out->w_v = b.w_v;
        out->b_m = b.b_m;
        out->b_v = b.b_v;
    });
}

TmlpNet* tmlp_net_create(const MLPOption* opt, int maxBatchSize, int inferBatchSize, unsigned seed, int isTraining)
{
    TmlpNet* h = nullptr;
    guarded("tmlp_net_create", [&] { h = new TmlpNet{new TinyMLP(*opt, maxBatchSize, inferBatchSize, seed, isTraining != 0)}; });
    return h;
}

void tmlp_net_destroy(TmlpNet* h)
{
    if (!h || !h->owned) return;
    delete h->n;
    delete h;
}

int tmlp_net_switch_mode(TmlpNet* h, int training)
{
    return GRID_CALL("switch_mode", training ? h->n->switchToTrainingMode() : h->n->switchToInferenceMode());
}
int tmlp_net_zero_grad(TmlpNet* h, hipStream_t s) { return GRID_CALL("zero_grad", h->n->zero_grad(s)); }
int tmlp_net_forward(TmlpNet* h, const half* in, float* out, int batch, hipStream_t s)
{
    return GRID_CALL("forward", h->n->forward(in, out, batch, s));
}
int tmlp_net_inference(TmlpNet* h, const half* in, float* out, int batch, hipStream_t s)
{
    return GRID_CALL("inference", h->n->inference(in, out, batch, s));
}
int tmlp_net_loss(TmlpNet* h, const half* targets, int batch, float loss_scale, int fetch, float* loss, hipStream_t s)
{
    return GRID_CALL("calculate_loss_and_grad", {
        const float v = h->n->calculate_loss_and_grad(targets, batch, loss_scale, fetch != 0, s);
        if (loss) *loss = v;
    });
}
int tmlp_net_backward(TmlpNet* h, const half* custom, half* dx, int batch, hipStream_t s)
{
    return GRID_CALL("backward", {
        if (custom && dx) h->n->backward(custom, dx, batch, s);
        else if (custom) h->n->backward(custom, batch, s);
        else if (dx) h->n->backward(dx, batch, s);
        else h->n->backward(batch, s);
    });
}
int tmlp_net_step(TmlpNet* h, float lr, float b1, float b2, float eps, float loss_scale, hipStream_t s)
{
    return GRID_CALL("step", h->n->step(lr, b1, b2, eps, loss_scale, s));
}
int tmlp_net_reset_step(TmlpNet* h) { return GRID_CALL("reset_step", h->n->reset_step()); }
int tmlp_net_load_weights(TmlpNet* h, const float* w, const float* b) { return GRID_CALL("loadWeights", h->n->loadWeights(w, b)); }
int tmlp_net_save_weights(TmlpNet* h, float* w, float* b) { return GRID_CALL("saveWeights", h->n->saveWeights(w, b)); }
int tmlp_net_load_file(TmlpNet* h, const char* p) { return GRID_CALL("loadWeights(file)", h->n->loadWeights(std::string(p))); }
int tmlp_net_save_file(TmlpNet* h, const char* p) { return GRID_CALL("saveWeights(file)", h->n->saveWeights(std::string(p))); }
int tmlp_net_buffers(TmlpNet* h, TmlpNetBuffers* out)
{
    return GRID_CALL("buffers", {
        const TinyMLP::Buffers b = h->n->buffers();
        out->master_weights = b.master_weights;
        out->master_biases = b.master_biases;
        out->fwd_weights = b.fwd_weights;
        out->w_grad = b.w_grad;
        out->b_grad = b.b_grad;
        out->activations = b.activations;
        out->dloss = b.dloss;
        out->padded_outputs = b.padded_outputs;
        out->hw = b.hw;
        out->step = b.step;
        out->w_m = b.w_m;
        out->w_v = b.w_v;
        out->b_m = b.b_m;
        out->b_v = b.b_v;
    });
}

int tmlp_device_synchronize(void)
{
    return guarded("hipDeviceSynchronize", [&] { GRAFT_HIP_CHECK(hipDeviceSynchronize()); });
}

const char* tmlp_version(void) { return "3dmaker_amd tinymlp gfx950 0.1"; }

}  // extern "C"
