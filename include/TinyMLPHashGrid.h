// TinyMLPHashGrid: multiresolution hash-grid encoding fused with a TinyMLP
// (the NeRF density head) for MI355X / gfx950.  Drop-in for
// modules/TinyMLP/TinyMLPHashGrid.h:33-165 of the reference: same class name,
// constructor, methods and default arguments, with cudaStream_t replaced by
// hipStream_t.
//
// Behavioural differences (all strictly safer than the reference):
//  - backward() before any forward() throws std::runtime_error (the reference
//    dereferences an unset input pointer, TinyMLPHashGrid.cu:258,343);
//  - unsupported shapes throw at construction instead of silent no-ops;
//  - per-level scales come from one fp64-evaluated host table
//    (float)(lowestSize * b^l) instead of device fast-math __powf/exp2f;
//  - MLP weight gradients are reduced deterministically.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <string>

#include "TinyMLP.h"
#include "tinymlp_abi.h"

// TinyMLPHashGrid.h:25-27
inline int inputDim(MLPGridOptions& opt) { return opt.featuresLevel * opt.numLevels; }

class TinyMLPHashGrid {
public:
    // TinyMLPHashGrid.h:35
    explicit TinyMLPHashGrid(const MLPGridOptions& options, int maxBatchSize, int inferBatchSize = 0,
                             unsigned int seed = 42, bool isTraining = true);
    ~TinyMLPHashGrid();

    TinyMLPHashGrid(const TinyMLPHashGrid&) = delete;
    TinyMLPHashGrid& operator=(const TinyMLPHashGrid&) = delete;

    void switchToInferenceMode();
    void switchToTrainingMode();

    void zero_grad(hipStream_t stream = 0);

    // d_unpadded_inputs: [batchSize x vectorDim] float positions in [0,1].
    void forward(const float* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream = 0);

    float calculate_loss_and_grad(const half* d_unpadded_targets, int batchSize, float loss_scale = 65536.0f,
                                  bool fetch_loss = false, hipStream_t stream = 0);

    void backward(int batchSize, hipStream_t stream = 0);
    void backward(const half* custom_loss_grad, int batchSize, hipStream_t stream = 0);

    void setSplitScatter(bool enabled) { m_useSplitScatter = enabled; }
    bool getSplitScatter() const { return m_useSplitScatter; }

    void step(float lr = 3e-4f, float beta1 = 0.9f, float beta2 = 0.999f, float epsilon = 1e-8f,
              float loss_scale = 65536.0f, hipStream_t stream = 0);
    void reset_step();

    void inference(const float* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream = 0);

    void loadWeights(const std::string& filename);
    void saveWeights(const std::string& filename);
    void loadWeights(const float* host_weights, const float* host_biases);
    void saveWeights(float* host_weights, float* host_biases);
    void loadHashgrid(const float* host_hashgrid);
    void saveHashgrid(float* host_hashgrid);

    // ---- additions (no reference counterpart) ----
    // step() with its two updates on two streams: the MLP layers on
    // mlp_stream, the hash table on hash_stream (one Adam step count for both).
    void stepSplit(float lr, float beta1, float beta2, float epsilon, float loss_scale, hipStream_t mlp_stream,
                   hipStream_t hash_stream);
    // The table half of the next step() fused into the scatter of the
    // backward: d_dx_out [N x 2L] (N, or *d_n when given, samples at
    // d_positions with pos_stride floats each) is scattered and every table
    // entry it reaches takes that step's Adam update in the same pass, with
    // the gradient the scatter would have stored (no gradient array).  The
    // step count is not advanced: stepMlp(), which follows, does that.
    // wait_before_update (nullable) is waited on before the first table
    // write.  Needs the binned scatter (scatter_plan non-null).  d_tile_live
    // (nullable): per 16-sample tile of d_dx_out, 0 where the whole tile is
    // +-0 (those rows are skipped: they add nothing).
    void scatterAdamTable(const half* d_dx_out, const float* d_positions, int pos_stride, int N, const uint32_t* d_n,
                          float lr, float beta1, float beta2, float epsilon, float loss_scale, hipStream_t stream,
                          hipEvent_t wait_before_update, const uint32_t* d_tile_live = nullptr);
    // The MLP half of step(): advances the step count, updates the layers.
    void stepMlp(float lr, float beta1, float beta2, float epsilon, float loss_scale, hipStream_t stream);

    // introspection for tests
    struct Buffers {
        float* master_hashtable;
        half* fwd_hashtable;
        float* hashtable_grads;
        float* hash_m;
        float* hash_v;
        float** master_weights;   // device arrays of per-layer pointers
        float** master_biases;
        half** fwd_weights;
        float** w_grad;
        float** b_grad;
        half** activations;       // [0] = encoding [maxBatch x 2L]
        half* dx_out;             // dL/d(encoding) [maxBatch x 2L]
        half* dloss;
        float* padded_inputs;     // [maxBatch x 4]
        float* padded_outputs;
        MLPGridOptions hw;
        int step;
        void* scatter_plan;       // binned-scatter scratch (opaque); null: per-corner atomic scatter
        float** w_m;              // MLP Adam moments (device arrays of per-layer pointers)
        float** w_v;
        float** b_m;
        float** b_v;
        void* workspace;          // partial-sum workspace of this instance (opaque)
    };
    Buffers buffers() const;

private:
    MLPGridOptions user_opt;
    MLPGridOptions hw_opt;
    MLPOption mlp_opt;
    int m_maxBatchSize;
    int m_inferBatchSize;
    int current_step;
    bool m_isTraining;
    bool m_useSplitScatter = true;

    float* d_padded_inputs = nullptr;
    const float* d_current_inputs_backward = nullptr;
    half* d_padded_targets = nullptr;
    float* d_padded_outputs_float = nullptr;
    half* d_dLoss_internal = nullptr;
    float* d_total_loss = nullptr;

    float* d_master_hashtable = nullptr;
    half* d_fwd_hashtable = nullptr;
    float* d_hashtable_grads = nullptr;
    float* d_hash_m = nullptr;
    float* d_hash_v = nullptr;
    int m_totalHashElements;

    float** d_master_weights = nullptr;
    float** d_master_biases = nullptr;
    half** d_fwd_weights = nullptr;
    half** d_activations = nullptr;
    half* d_dx_out = nullptr;
    float** d_w_grad = nullptr;
    float** d_b_grad = nullptr;
    float** d_w_m = nullptr;
    float** d_w_v = nullptr;
    float** d_b_m = nullptr;
    float** d_b_v = nullptr;
    void* h_ptrs = nullptr;
    void* m_meta = nullptr;   // hash-grid level table (opaque)
    void* m_scatter = nullptr; // binned-scatter scratch of this instance (opaque)
    void* m_workspace = nullptr;  // partial-sum workspace of the loss and backward (opaque)

    void allocate_memory();
    void free_training_state();
    void run_backward(int batchSize, hipStream_t stream);
};
