// TinyMLP: fully-fused MLP (fp16 MFMA, fp32 master weights, fused Adam) for
// MI355X / gfx950.  Drop-in for modules/TinyMLP/TinyMLP.h:35-154 of the
// reference: same class name, constructor, methods and default arguments,
// with cudaStream_t replaced by hipStream_t.
//
// Behavioural differences (all strictly safer than the reference):
//  - unsupported shapes (max dim > 128, numLayers > 16) throw
//    std::runtime_error at construction instead of making every launch a
//    silent no-op (TinyMLP.cu / networkFusion.cu:389);
//  - HIP errors throw std::runtime_error instead of abort();
//  - weight gradients are reduced deterministically (no fp32 atomics).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <string>

#include "tinymlp_abi.h"

class TinyMLP {
public:
    // TinyMLP.h:38
    explicit TinyMLP(const MLPOption& options, int maxBatchSize, int inferBatchSize = 0,
                     unsigned int seed = 42, bool isTraining = true);
    ~TinyMLP();

    TinyMLP(const TinyMLP&) = delete;
    TinyMLP& operator=(const TinyMLP&) = delete;

    void switchToInferenceMode();
    void switchToTrainingMode();

    void zero_grad(hipStream_t stream = 0);

    // Training forward: saves activations; writes UNPADDED fp32 outputs (d_outputs may be null).
    void forward(const half* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream = 0);

    float calculate_loss_and_grad(const half* d_unpadded_targets, int batchSize, float loss_scale = 65536.0f,
                                  bool fetch_loss = false, hipStream_t stream = 0);

    void backward(int batchSize, hipStream_t stream = 0);
    void backward(const half* custom_loss_grad, int batchSize, hipStream_t stream = 0);
    void backward(half* out_d_dx_out, int batchSize, hipStream_t stream = 0);
    void backward(const half* custom_loss_grad, half* out_d_dx_out, int batchSize, hipStream_t stream = 0);

    void step(float lr = 3e-4f, float beta1 = 0.9f, float beta2 = 0.999f, float epsilon = 1e-8f,
              float loss_scale = 65536.0f, hipStream_t stream = 0);
    void reset_step();

    void inference(const half* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream = 0);

    void loadWeights(const std::string& filename);
    void saveWeights(const std::string& filename);
    void loadWeights(const float* host_weights, const float* host_biases);
    void saveWeights(float* host_weights, float* host_biases);

    // ---- additions (no reference counterpart): introspection for tests ----
    struct Buffers {
        float** master_weights;   // device arrays of per-layer pointers
        float** master_biases;
        half** fwd_weights;
        float** w_grad;
        float** b_grad;
        half** activations;       // [0] = padded input snapshot
        half* dloss;              // fp16 dL/dout [maxBatch x hw out]
        float* padded_outputs;    // fp32 [maxBatch x hw out]
        MLPOption hw;
        int step;
        float** w_m;              // Adam moments (device arrays of per-layer pointers)
        float** w_v;
        float** b_m;
        float** b_v;
        void* workspace;          // partial-sum workspace of this instance (opaque)
    };
    Buffers buffers() const;

private:
    MLPOption user_opt;
    MLPOption hw_opt;
    int m_maxBatchSize;
    int m_inferBatchSize;
    int current_step;
    bool m_isTraining;

    half* d_padded_inputs = nullptr;
    half* d_padded_targets = nullptr;
    float* d_padded_outputs_float = nullptr;
    half* d_dLoss_internal = nullptr;
    float* d_total_loss = nullptr;

    // Host mirrors of the per-layer device pointers; the device arrays
    // (d_*) hold the same pointers for the launch ABI.
    float** d_master_weights = nullptr;
    float** d_master_biases = nullptr;
    half** d_fwd_weights = nullptr;
    half** d_activations = nullptr;
    float** d_w_grad = nullptr;
    float** d_b_grad = nullptr;
    float** d_w_m = nullptr;
    float** d_w_v = nullptr;
    float** d_b_m = nullptr;
    float** d_b_v = nullptr;
    void* h_ptrs = nullptr;   // host-side pointer tables (opaque)
    void* m_workspace = nullptr;  // partial-sum workspace of the loss and backward (opaque)

    void allocate_memory();
    void free_training_state();
    void run_backward(const half* custom, bool have_custom, half* dx, int batchSize, hipStream_t s);
};
