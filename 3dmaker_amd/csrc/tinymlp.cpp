// Host classes TinyMLP and TinyMLPHashGrid (the reference's modules/TinyMLP
// C++ API) on top of the gfx950 kernels.  Lifecycle, buffer ownership, mode
// switches, padding rules and initialisation order follow
// TinyMLP.cu:75-481 and TinyMLPHashGrid.cu:36-455.
#include "TinyMLP.h"
#include "TinyMLPHashGrid.h"

#include "common.h"
#include "hashgrid.h"
#include "mlp.h"
#include "optimizer.h"
#include "scatter.h"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <random>
#include <vector>

using graft::AdamArgs;
using graft::LayerSizes;
using graft::MlpShape;

namespace {

// TinyMLP.h:144-153: next power of two, at least 8.
int nextPowerOf2(int n)
{
    if (n <= 8) return 8;
    n--;
    n |= n >> 1;
    n |= n >> 2;
    n |= n >> 4;
    n |= n >> 8;
    n |= n >> 16;
    return n + 1;
}

template <class T>
T* dalloc(size_t n, bool zero = false)
{
    T* p = nullptr;
    if (n == 0) return nullptr;
    GRAFT_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&p), n * sizeof(T)));
    if (zero) GRAFT_HIP_CHECK(hipMemset(p, 0, n * sizeof(T)));
    return p;
}

void dfree(void* p)
{
    if (p) (void)hipFree(p);
}

// Per-layer device buffers plus the device array of their pointers.
struct LayerTable {
    std::vector<void*> h;
    void** d = nullptr;

    void create(const std::vector<size_t>& bytes, bool zero, void* first = nullptr)
    {
        h.assign(bytes.size(), nullptr);
        for (size_t l = 0; l < bytes.size(); l++) {
            if (l == 0 && first) {
                h[l] = first;
                continue;
            }
            GRAFT_HIP_CHECK(hipMalloc(&h[l], std::max<size_t>(bytes[l], 4)));
            if (zero) GRAFT_HIP_CHECK(hipMemset(h[l], 0, std::max<size_t>(bytes[l], 4)));
        }
        GRAFT_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&d), h.size() * sizeof(void*)));
        GRAFT_HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(void*), hipMemcpyHostToDevice));
    }
    void destroy(bool skip_first = false)
    {
        for (size_t l = skip_first ? 1 : 0; l < h.size(); l++) dfree(h[l]);
        h.clear();
        dfree(d);
        d = nullptr;
    }
    bool alive() const { return d != nullptr; }
    template <class T>
    T** dev() const { return reinterpret_cast<T**>(d); }
    template <class T>
    T* at(int l) const { return reinterpret_cast<T*>(h[l]); }
};

struct Tables {
    LayerTable mw, mb, fw, wg, bg, wm, wv, bm, bv, acts;
};

struct Dims {
    int in, hid, out, layers;
    int in_l(int l) const { return l == 0 ? in : hid; }
    int out_l(int l) const { return l == layers - 1 ? out : hid; }
    std::vector<size_t> wbytes(size_t es) const
    {
        std::vector<size_t> v;
        for (int l = 0; l < layers; l++) v.push_back((size_t)in_l(l) * out_l(l) * es);
        return v;
    }
    std::vector<size_t> bbytes(size_t es) const
    {
        std::vector<size_t> v;
        for (int l = 0; l < layers; l++) v.push_back((size_t)out_l(l) * es);
        return v;
    }
    LayerSizes wsizes() const
    {
        LayerSizes s{};
        for (int l = 0; l < layers; l++) s.n[l] = in_l(l) * out_l(l);
        return s;
    }
    LayerSizes bsizes() const
    {
        LayerSizes s{};
        for (int l = 0; l < layers; l++) s.n[l] = out_l(l);
        return s;
    }
};

// LeCun-uniform weights U(-1/sqrt(in), 1/sqrt(in)), zero biases, drawn layer by
// layer from one mt19937 stream (TinyMLP.cu:86-104, TinyMLPHashGrid.cu:68-82).
void init_layers(const Dims& d, std::mt19937& gen, Tables& t)
{
    for (int l = 0; l < d.layers; l++) {
        const int in_d = d.in_l(l), out_d = d.out_l(l);
        const float bound = 1.0f / std::sqrt((float)in_d);
        std::uniform_real_distribution<float> dist(-bound, bound);
        std::vector<float> hw((size_t)in_d * out_d), hb(out_d, 0.0f);
        for (auto& v : hw) v = dist(gen);
        GRAFT_HIP_CHECK(hipMemcpy(t.mw.h[l], hw.data(), hw.size() * 4, hipMemcpyHostToDevice));
        GRAFT_HIP_CHECK(hipMemcpy(t.mb.h[l], hb.data(), hb.size() * 4, hipMemcpyHostToDevice));
        graft::f32_to_f16(t.mw.at<float>(l), t.fw.at<__half>(l), (long long)hw.size(), 0);
    }
    GRAFT_HIP_CHECK(hipDeviceSynchronize());
}

void load_layers(const Dims& d, Tables& t, const float* hw, const float* hb)
{
    size_t wo = 0, bo = 0;
    for (int l = 0; l < d.layers; l++) {
        const size_t we = (size_t)d.in_l(l) * d.out_l(l), be = d.out_l(l);
        GRAFT_HIP_CHECK(hipMemcpy(t.mw.h[l], hw + wo, we * 4, hipMemcpyHostToDevice));
        GRAFT_HIP_CHECK(hipMemcpy(t.mb.h[l], hb + bo, be * 4, hipMemcpyHostToDevice));
        graft::f32_to_f16(t.mw.at<float>(l), t.fw.at<__half>(l), (long long)we, 0);
        wo += we;
        bo += be;
    }
    GRAFT_HIP_CHECK(hipDeviceSynchronize());
}

void save_layers(const Dims& d, const Tables& t, float* hw, float* hb)
{
    size_t wo = 0, bo = 0;
    for (int l = 0; l < d.layers; l++) {
        const size_t we = (size_t)d.in_l(l) * d.out_l(l), be = d.out_l(l);
        GRAFT_HIP_CHECK(hipMemcpy(hw + wo, t.mw.h[l], we * 4, hipMemcpyDeviceToHost));
        GRAFT_HIP_CHECK(hipMemcpy(hb + bo, t.mb.h[l], be * 4, hipMemcpyDeviceToHost));
        wo += we;
        bo += be;
    }
}

void create_training_tables(const Dims& d, Tables& t)
{
    if (!t.wg.alive()) t.wg.create(d.wbytes(4), true);
    if (!t.bg.alive()) t.bg.create(d.bbytes(4), true);
    if (!t.wm.alive()) t.wm.create(d.wbytes(4), true);
    if (!t.bm.alive()) t.bm.create(d.bbytes(4), true);
    if (!t.wv.alive()) t.wv.create(d.wbytes(4), true);
    if (!t.bv.alive()) t.bv.create(d.bbytes(4), true);
}

void destroy_training_tables(Tables& t)
{
    t.wg.destroy();
    t.bg.destroy();
    t.wm.destroy();
    t.bm.destroy();
    t.wv.destroy();
    t.bv.destroy();
}

AdamArgs adam_args(int step, float lr, float b1, float b2, float eps, float loss_scale)
{
    AdamArgs a{};
    a.lr = lr;
    a.b1 = b1;
    a.b2 = b2;
    a.eps = eps;
    a.bc1 = 1.0f - std::pow(b1, (float)step);
    a.bc2 = 1.0f - std::pow(b2, (float)step);
    a.inv_scale = 1.0f / loss_scale;
    return a;
}

}  // namespace

// ===========================================================================
// TinyMLP
// ===========================================================================

#define TT (*static_cast<Tables*>(h_ptrs))

static Dims dims_of(const MLPOption& o) { return Dims{o.inputDim, o.hiddenDim, o.outputDim, o.numLayers}; }

static MlpShape shape_of(const MLPOption& o) { return MlpShape{o.inputDim, o.hiddenDim, o.outputDim, o.numLayers}; }

TinyMLP::TinyMLP(const MLPOption& options, int maxBatchSize, int inferBatchSize, unsigned int seed, bool isTraining)
    : user_opt(options),
      m_maxBatchSize(maxBatchSize),
      m_inferBatchSize(inferBatchSize <= 0 ? maxBatchSize : inferBatchSize),
      current_step(0),
      m_isTraining(isTraining)
{
    hw_opt = options;
    hw_opt.inputDim = nextPowerOf2(user_opt.inputDim);
    hw_opt.hiddenDim = nextPowerOf2(user_opt.hiddenDim);
    hw_opt.outputDim = nextPowerOf2(user_opt.outputDim);
    shape_of(hw_opt).validate();
    if (maxBatchSize <= 0) throw std::runtime_error("TinyMLP: maxBatchSize must be positive");
    h_ptrs = new Tables();
    const Dims d = dims_of(hw_opt);
    TT.mw.create(d.wbytes(4), false);
    TT.mb.create(d.bbytes(4), false);
    TT.fw.create(d.wbytes(2), false);
    allocate_memory();
    std::mt19937 gen(seed);
    init_layers(d, gen, TT);
    d_master_weights = TT.mw.dev<float>();
    d_master_biases = TT.mb.dev<float>();
    d_fwd_weights = TT.fw.dev<half>();
}

TinyMLP::~TinyMLP()
{
    if (!h_ptrs) return;
    free_training_state();
    dfree(d_padded_inputs);
    dfree(d_padded_outputs_float);
    TT.mw.destroy();
    TT.mb.destroy();
    TT.fw.destroy();
    delete static_cast<Tables*>(h_ptrs);
    h_ptrs = nullptr;
}

// TinyMLP.cu:157-222
void TinyMLP::allocate_memory()
{
    const int max_pad = std::max(m_maxBatchSize, m_inferBatchSize);
    const bool needs_in_pad = user_opt.inputDim != hw_opt.inputDim;
    const bool needs_out_pad = user_opt.outputDim != hw_opt.outputDim;
    if ((m_isTraining || needs_in_pad) && !d_padded_inputs)
        d_padded_inputs = dalloc<half>((size_t)max_pad * hw_opt.inputDim);
    if (m_isTraining && !d_padded_targets) d_padded_targets = dalloc<half>((size_t)m_maxBatchSize * hw_opt.outputDim);
    if ((m_isTraining || needs_out_pad) && !d_padded_outputs_float)
        d_padded_outputs_float = dalloc<float>((size_t)max_pad * hw_opt.outputDim);
    if (m_isTraining) {
        if (!d_dLoss_internal) d_dLoss_internal = dalloc<half>((size_t)m_maxBatchSize * hw_opt.outputDim);
        if (!d_total_loss) d_total_loss = dalloc<float>(1, true);
        const Dims d = dims_of(hw_opt);
        create_training_tables(d, TT);
        if (!TT.acts.alive()) {
            std::vector<size_t> ab(hw_opt.numLayers, (size_t)m_maxBatchSize * hw_opt.hiddenDim * 2);
            TT.acts.create(ab, false, d_padded_inputs);  // [0] aliases the padded input (TinyMLP.cu:212)
        }
        d_w_grad = TT.wg.dev<float>();
        d_b_grad = TT.bg.dev<float>();
        d_w_m = TT.wm.dev<float>();
        d_w_v = TT.wv.dev<float>();
        d_b_m = TT.bm.dev<float>();
        d_b_v = TT.bv.dev<float>();
        d_activations = TT.acts.dev<half>();
        if (!m_workspace) m_workspace = new graft::Workspace();
    }
}

void TinyMLP::free_training_state()
{
    delete static_cast<graft::Workspace*>(m_workspace);
    m_workspace = nullptr;
    dfree(d_padded_targets);
    d_padded_targets = nullptr;
    dfree(d_dLoss_internal);
    d_dLoss_internal = nullptr;
    dfree(d_total_loss);
    d_total_loss = nullptr;
    destroy_training_tables(TT);
    TT.acts.destroy(true);
    d_w_grad = d_b_grad = d_w_m = d_w_v = d_b_m = d_b_v = nullptr;
    d_activations = nullptr;
}

// TinyMLP.cu:224-254
void TinyMLP::switchToInferenceMode()
{
    if (!m_isTraining) return;
    if (user_opt.inputDim == hw_opt.inputDim && d_padded_inputs) {
        dfree(d_padded_inputs);
        d_padded_inputs = nullptr;
    }
    if (user_opt.outputDim == hw_opt.outputDim && d_padded_outputs_float) {
        dfree(d_padded_outputs_float);
        d_padded_outputs_float = nullptr;
    }
    free_training_state();
    m_isTraining = false;
}

void TinyMLP::switchToTrainingMode()
{
    if (m_isTraining) return;
    m_isTraining = true;
    allocate_memory();
}

void TinyMLP::zero_grad(hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("zero_grad called while in inference mode!");
    const Dims d = dims_of(hw_opt);
    graft::zero_layers(d_w_grad, d_b_grad, d.wsizes(), d.bsizes(), d.layers, stream);
}

// TinyMLP.cu:261-285
void TinyMLP::forward(const half* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("forward called while in inference mode!");
    if (batchSize > m_maxBatchSize) throw std::runtime_error("Batch size exceeds maxBatchSize");
    if (batchSize <= 0) return;
    graft::FwdInput in;
    if (user_opt.inputDim != hw_opt.inputDim) {
        graft::pad_f16(d_unpadded_inputs, d_padded_inputs, batchSize, user_opt.inputDim, hw_opt.inputDim, stream);
        in.x = d_padded_inputs;
    } else {
        // The activation-0 snapshot is written by the fused kernel itself.
        in.x = d_unpadded_inputs;
        in.save_x0 = true;
    }
    graft::mlp_forward(shape_of(hw_opt), in, d_fwd_weights, d_master_biases, d_activations, d_padded_outputs_float,
                       batchSize, hw_opt.outputActivation, stream);
    if (d_outputs) {
        if (user_opt.outputDim == hw_opt.outputDim)
            GRAFT_HIP_CHECK(hipMemcpyAsync(d_outputs, d_padded_outputs_float,
                                           (size_t)batchSize * hw_opt.outputDim * sizeof(float),
                                           hipMemcpyDeviceToDevice, stream));
        else
            graft::unpad_f32(d_padded_outputs_float, d_outputs, batchSize, hw_opt.outputDim, user_opt.outputDim,
                             stream);
    }
}

// TinyMLP.cu:287-318
void TinyMLP::inference(const half* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream)
{
    if (batchSize > m_inferBatchSize) {
        for (int off = 0; off < batchSize; off += m_inferBatchSize) {
            const int cur = std::min(m_inferBatchSize, batchSize - off);
            inference(d_unpadded_inputs + (size_t)off * user_opt.inputDim,
                      d_outputs ? d_outputs + (size_t)off * user_opt.outputDim : nullptr, cur, stream);
        }
        return;
    }
    if (batchSize <= 0) return;
    graft::FwdInput in;
    in.x = d_unpadded_inputs;
    if (user_opt.inputDim != hw_opt.inputDim) {
        graft::pad_f16(d_unpadded_inputs, d_padded_inputs, batchSize, user_opt.inputDim, hw_opt.inputDim, stream);
        in.x = d_padded_inputs;
    }
    if (user_opt.outputDim == hw_opt.outputDim) {
        if (d_outputs)
            graft::mlp_forward(shape_of(hw_opt), in, d_fwd_weights, d_master_biases, nullptr, d_outputs, batchSize,
                               hw_opt.outputActivation, stream);
    } else {
        graft::mlp_forward(shape_of(hw_opt), in, d_fwd_weights, d_master_biases, nullptr, d_padded_outputs_float,
                           batchSize, hw_opt.outputActivation, stream);
        if (d_outputs)
            graft::unpad_f32(d_padded_outputs_float, d_outputs, batchSize, hw_opt.outputDim, user_opt.outputDim,
                             stream);
    }
}

// TinyMLP.cu:320-352
float TinyMLP::calculate_loss_and_grad(const half* d_unpadded_targets, int batchSize, float loss_scale, bool fetch_loss,
                                       hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("calculate_loss_and_grad called while in inference mode!");
    GRAFT_HIP_CHECK(hipMemsetAsync(d_total_loss, 0, sizeof(float), stream));
    const half* tg = d_unpadded_targets;
    if (user_opt.outputDim != hw_opt.outputDim) {
        graft::pad_f16(d_unpadded_targets, d_padded_targets, batchSize, user_opt.outputDim, hw_opt.outputDim, stream);
        tg = d_padded_targets;
    }
    graft::mse_loss_grad(d_padded_outputs_float, tg, d_dLoss_internal, d_total_loss, batchSize, hw_opt.outputDim,
                         user_opt.outputDim, loss_scale, hw_opt.outputActivation, stream,
                         static_cast<graft::Workspace*>(m_workspace));
    if (fetch_loss) {
        float h = 0.f;
        GRAFT_HIP_CHECK(hipMemcpyAsync(&h, d_total_loss, sizeof(float), hipMemcpyDeviceToHost, stream));
        GRAFT_HIP_CHECK(hipStreamSynchronize(stream));
        return h / (float)(batchSize * user_opt.outputDim);
    }
    return 0.0f;
}

void TinyMLP::run_backward(const half* custom, bool have_custom, half* dx, int batchSize, hipStream_t s)
{
    if (!m_isTraining) throw std::runtime_error("backward called while in inference mode!");
    if (batchSize > m_maxBatchSize) throw std::runtime_error("Batch size exceeds maxBatchSize");
    if (batchSize <= 0) return;
    if (have_custom) {
        if (user_opt.outputDim != hw_opt.outputDim)
            graft::pad_f16(custom, d_dLoss_internal, batchSize, user_opt.outputDim, hw_opt.outputDim, s);
        else
            GRAFT_HIP_CHECK(hipMemcpyAsync(d_dLoss_internal, custom, (size_t)batchSize * hw_opt.outputDim * sizeof(half),
                                           hipMemcpyDeviceToDevice, s));
    }
    graft::mlp_backward(shape_of(hw_opt), d_dLoss_internal, d_activations, d_fwd_weights, d_w_grad, d_b_grad, dx,
                        batchSize, s, nullptr, true, static_cast<graft::Workspace*>(m_workspace));
}

// TinyMLP.cu:354-390
void TinyMLP::backward(int batchSize, hipStream_t stream) { run_backward(nullptr, false, nullptr, batchSize, stream); }
void TinyMLP::backward(const half* g, int batchSize, hipStream_t stream) { run_backward(g, true, nullptr, batchSize, stream); }
void TinyMLP::backward(half* dx, int batchSize, hipStream_t stream) { run_backward(nullptr, false, dx, batchSize, stream); }
void TinyMLP::backward(const half* g, half* dx, int batchSize, hipStream_t stream) { run_backward(g, true, dx, batchSize, stream); }

void TinyMLP::reset_step() { current_step = 0; }

// TinyMLP.cu:392-404
void TinyMLP::step(float lr, float beta1, float beta2, float epsilon, float loss_scale, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("step called while in inference mode!");
    if (current_step < 50000) current_step++;
    const AdamArgs a = adam_args(current_step, lr, beta1, beta2, epsilon, loss_scale);
    const Dims d = dims_of(hw_opt);
    graft::adam_dense(d_master_weights, d_fwd_weights, d_w_grad, d_w_m, d_w_v, d.wsizes(), d_master_biases,
                      d_b_grad, d_b_m, d_b_v, d.bsizes(), d.layers, a, stream);
}

// TinyMLP.cu:406-481: raw MLPOption header, then per layer W then B (fp32).
void TinyMLP::loadWeights(const std::string& filename)
{
    std::ifstream in(filename, std::ios::binary);
    if (!in.is_open()) throw std::runtime_error("Cannot open file for loading weights: " + filename);
    MLPOption fo;
    in.read(reinterpret_cast<char*>(&fo), sizeof(MLPOption));
    if (fo.inputDim != hw_opt.inputDim || fo.hiddenDim != hw_opt.hiddenDim || fo.outputDim != hw_opt.outputDim ||
        fo.numLayers != hw_opt.numLayers)
        throw std::runtime_error("Weight file dimension mismatch!");
    const Dims d = dims_of(hw_opt);
    std::vector<float> w, b;
    for (int l = 0; l < d.layers; l++) {
        const size_t we = (size_t)d.in_l(l) * d.out_l(l), be = d.out_l(l);
        std::vector<float> lw(we), lb(be);
        in.read(reinterpret_cast<char*>(lw.data()), we * 4);
        in.read(reinterpret_cast<char*>(lb.data()), be * 4);
        if (!in) throw std::runtime_error("Weight file truncated: " + filename);
        w.insert(w.end(), lw.begin(), lw.end());
        b.insert(b.end(), lb.begin(), lb.end());
    }
    load_layers(d, TT, w.data(), b.data());
}

void TinyMLP::saveWeights(const std::string& filename)
{
    std::ofstream out(filename, std::ios::binary);
    if (!out.is_open()) throw std::runtime_error("Cannot open file for saving weights: " + filename);
    out.write(reinterpret_cast<const char*>(&hw_opt), sizeof(MLPOption));
    const Dims d = dims_of(hw_opt);
    for (int l = 0; l < d.layers; l++) {
        const size_t we = (size_t)d.in_l(l) * d.out_l(l), be = d.out_l(l);
        std::vector<float> lw(we), lb(be);
        GRAFT_HIP_CHECK(hipMemcpy(lw.data(), TT.mw.h[l], we * 4, hipMemcpyDeviceToHost));
        GRAFT_HIP_CHECK(hipMemcpy(lb.data(), TT.mb.h[l], be * 4, hipMemcpyDeviceToHost));
        out.write(reinterpret_cast<const char*>(lw.data()), we * 4);
        out.write(reinterpret_cast<const char*>(lb.data()), be * 4);
    }
}

void TinyMLP::loadWeights(const float* hw, const float* hb) { load_layers(dims_of(hw_opt), TT, hw, hb); }
void TinyMLP::saveWeights(float* hw, float* hb) { save_layers(dims_of(hw_opt), TT, hw, hb); }

TinyMLP::Buffers TinyMLP::buffers() const
{
    Buffers b{};
    b.master_weights = d_master_weights;
    b.master_biases = d_master_biases;
    b.fwd_weights = d_fwd_weights;
    b.w_grad = d_w_grad;
    b.b_grad = d_b_grad;
    b.activations = d_activations;
    b.dloss = d_dLoss_internal;
    b.padded_outputs = d_padded_outputs_float;
    b.hw = hw_opt;
    b.step = current_step;
    b.w_m = d_w_m;
    b.w_v = d_w_v;
    b.b_m = d_b_m;
    b.b_v = d_b_v;
    b.workspace = m_workspace;
    return b;
}

// ===========================================================================
// TinyMLPHashGrid
// ===========================================================================

#define META (*static_cast<graft::GridMeta*>(m_meta))

TinyMLPHashGrid::TinyMLPHashGrid(const MLPGridOptions& options, int maxBatchSize, int inferBatchSize,
                                 unsigned int seed, bool isTraining)
    : user_opt(options),
      m_maxBatchSize(maxBatchSize),
      m_inferBatchSize(inferBatchSize <= 0 ? maxBatchSize : inferBatchSize),
      current_step(0),
      m_isTraining(isTraining)
{
    // TinyMLPHashGrid.cu:38-39
    if (options.vectorDim != 3 && options.vectorDim != 4)
        throw std::runtime_error("TinyMLPHashGrid: vectorDim must be 3 or 4");
    if (options.featuresLevel != 2) throw std::runtime_error("TinyMLPHashGrid: featuresLevel must be 2");
    if (maxBatchSize <= 0) throw std::runtime_error("TinyMLPHashGrid: maxBatchSize must be positive");
    hw_opt = options;
    hw_opt.hiddenDim = nextPowerOf2(options.hiddenDim);
    hw_opt.outputDim = nextPowerOf2(options.outputDim);
    mlp_opt = MLPOption{};
    mlp_opt.inputDim = hw_opt.numLevels * hw_opt.featuresLevel;
    mlp_opt.hiddenDim = hw_opt.hiddenDim;
    mlp_opt.outputDim = hw_opt.outputDim;
    mlp_opt.numLayers = hw_opt.numLayers;
    mlp_opt.activationType = hw_opt.activationType;
    mlp_opt.outputActivation = OUT_ACT_NONE;
    shape_of(mlp_opt).validate();
    m_meta = new graft::GridMeta(graft::make_grid_meta(hw_opt.tableSize, hw_opt.numLevels, hw_opt.b, hw_opt.lowestSize));
    m_totalHashElements = hw_opt.numLevels * hw_opt.tableSize * hw_opt.featuresLevel;

    h_ptrs = new Tables();
    const Dims d = dims_of(mlp_opt);
    TT.mw.create(d.wbytes(4), false);
    TT.mb.create(d.bbytes(4), false);
    TT.fw.create(d.wbytes(2), false);
    d_master_hashtable = dalloc<float>(m_totalHashElements);
    d_fwd_hashtable = dalloc<half>(m_totalHashElements);
    allocate_memory();

    // TinyMLPHashGrid.cu:52-84: table U(-0.1, 0.1) first, then the layers, one stream.
    std::mt19937 gen(seed);
    std::uniform_real_distribution<float> hash_dist(-0.1f, 0.1f);
    std::vector<float> hh(m_totalHashElements);
    for (auto& v : hh) v = hash_dist(gen);
    GRAFT_HIP_CHECK(hipMemcpy(d_master_hashtable, hh.data(), hh.size() * 4, hipMemcpyHostToDevice));
    graft::f32_to_f16(d_master_hashtable, d_fwd_hashtable, m_totalHashElements, 0);
    init_layers(d, gen, TT);
    d_master_weights = TT.mw.dev<float>();
    d_master_biases = TT.mb.dev<float>();
    d_fwd_weights = TT.fw.dev<half>();
}

TinyMLPHashGrid::~TinyMLPHashGrid()
{
    if (!h_ptrs) return;
    free_training_state();
    dfree(d_padded_inputs);
    dfree(d_padded_outputs_float);
    dfree(d_master_hashtable);
    dfree(d_fwd_hashtable);
    TT.mw.destroy();
    TT.mb.destroy();
    TT.fw.destroy();
    delete static_cast<Tables*>(h_ptrs);
    delete static_cast<graft::GridMeta*>(m_meta);
    h_ptrs = nullptr;
}

// TinyMLPHashGrid.cu:110-202
void TinyMLPHashGrid::allocate_memory()
{
    const int inDim = mlp_opt.inputDim, outDim = mlp_opt.outputDim, hidDim = mlp_opt.hiddenDim;
    const int max_pad = std::max(m_maxBatchSize, m_inferBatchSize);
    const bool needs_in_pad = user_opt.vectorDim != 4;
    const bool needs_out_pad = user_opt.outputDim != hw_opt.outputDim;
    if ((m_isTraining || needs_in_pad) && !d_padded_inputs) d_padded_inputs = dalloc<float>((size_t)max_pad * 4);
    if (m_isTraining && !d_padded_targets) d_padded_targets = dalloc<half>((size_t)m_maxBatchSize * outDim);
    if ((m_isTraining || needs_out_pad) && !d_padded_outputs_float)
        d_padded_outputs_float = dalloc<float>((size_t)max_pad * outDim);
    if (m_isTraining) {
        if (!d_dLoss_internal) d_dLoss_internal = dalloc<half>((size_t)m_maxBatchSize * outDim);
        if (!d_total_loss) d_total_loss = dalloc<float>(1, true);
        if (!d_dx_out) d_dx_out = dalloc<half>((size_t)m_maxBatchSize * inDim);
        if (!d_hashtable_grads) d_hashtable_grads = dalloc<float>(m_totalHashElements, true);
        if (!d_hash_m) d_hash_m = dalloc<float>(m_totalHashElements, true);
        if (!d_hash_v) d_hash_v = dalloc<float>(m_totalHashElements, true);
        const Dims d = dims_of(mlp_opt);
        create_training_tables(d, TT);
        if (!TT.acts.alive()) {
            std::vector<size_t> ab(mlp_opt.numLayers, (size_t)m_maxBatchSize * hidDim * 2);
            ab[0] = (size_t)m_maxBatchSize * inDim * 2;
            TT.acts.create(ab, false);
        }
        d_w_grad = TT.wg.dev<float>();
        d_b_grad = TT.bg.dev<float>();
        d_w_m = TT.wm.dev<float>();
        d_w_v = TT.wv.dev<float>();
        d_b_m = TT.bm.dev<float>();
        d_b_v = TT.bv.dev<float>();
        d_activations = TT.acts.dev<half>();
        if (!m_scatter) m_scatter = graft::scatter_plan_create(META, m_maxBatchSize);
        if (!m_workspace) m_workspace = new graft::Workspace();
    }
}

void TinyMLPHashGrid::free_training_state()
{
    for (void** p : {reinterpret_cast<void**>(&d_padded_targets), reinterpret_cast<void**>(&d_dLoss_internal),
                     reinterpret_cast<void**>(&d_total_loss), reinterpret_cast<void**>(&d_dx_out),
                     reinterpret_cast<void**>(&d_hashtable_grads), reinterpret_cast<void**>(&d_hash_m),
                     reinterpret_cast<void**>(&d_hash_v)}) {
        dfree(*p);
        *p = nullptr;
    }
    destroy_training_tables(TT);
    TT.acts.destroy();
    graft::scatter_plan_destroy(static_cast<graft::ScatterPlan*>(m_scatter));
    m_scatter = nullptr;
    delete static_cast<graft::Workspace*>(m_workspace);
    m_workspace = nullptr;
    d_w_grad = d_b_grad = d_w_m = d_w_v = d_b_m = d_b_v = nullptr;
    d_activations = nullptr;
    d_current_inputs_backward = nullptr;
}

// TinyMLPHashGrid.cu:204-232
void TinyMLPHashGrid::switchToInferenceMode()
{
    if (!m_isTraining) return;
    if (user_opt.vectorDim == 4 && d_padded_inputs) {
        dfree(d_padded_inputs);
        d_padded_inputs = nullptr;
    }
    if (user_opt.outputDim == hw_opt.outputDim && d_padded_outputs_float) {
        dfree(d_padded_outputs_float);
        d_padded_outputs_float = nullptr;
    }
    free_training_state();
    m_isTraining = false;
}

void TinyMLPHashGrid::switchToTrainingMode()
{
    if (m_isTraining) return;
    m_isTraining = true;
    allocate_memory();
}

// TinyMLPHashGrid.cu:240-244: the hash grads are zeroed by the Adam pass itself.
void TinyMLPHashGrid::zero_grad(hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("zero_grad called while in inference mode!");
    const Dims d = dims_of(mlp_opt);
    graft::zero_layers(d_w_grad, d_b_grad, d.wsizes(), d.bsizes(), d.layers, stream);
}

// TinyMLPHashGrid.cu:246-273
void TinyMLPHashGrid::forward(const float* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("forward called while in inference mode!");
    if (batchSize > m_maxBatchSize) throw std::runtime_error("batchSize exceeds maxBatchSize");
    if (batchSize <= 0) return;
    const float* inp = d_unpadded_inputs;
    if (user_opt.vectorDim == 3) {
        graft::pad_f32(d_unpadded_inputs, d_padded_inputs, batchSize, 3, 4, stream);
        inp = d_padded_inputs;
    }
    d_current_inputs_backward = inp;
    graft::FwdInput in;
    in.pos = inp;
    in.pos_stride = 4;
    in.table = d_fwd_hashtable;
    in.meta = &META;
    graft::mlp_forward(shape_of(mlp_opt), in, d_fwd_weights, d_master_biases, d_activations, d_padded_outputs_float,
                       batchSize, OUT_ACT_NONE, stream);
    if (d_outputs) {
        if (user_opt.outputDim == hw_opt.outputDim)
            GRAFT_HIP_CHECK(hipMemcpyAsync(d_outputs, d_padded_outputs_float,
                                           (size_t)batchSize * hw_opt.outputDim * sizeof(float),
                                           hipMemcpyDeviceToDevice, stream));
        else
            graft::unpad_f32(d_padded_outputs_float, d_outputs, batchSize, hw_opt.outputDim, user_opt.outputDim,
                             stream);
    }
}

// TinyMLPHashGrid.cu:275-308
void TinyMLPHashGrid::inference(const float* d_unpadded_inputs, float* d_outputs, int batchSize, hipStream_t stream)
{
    if (batchSize > m_inferBatchSize) {
        for (int off = 0; off < batchSize; off += m_inferBatchSize) {
            const int cur = std::min(m_inferBatchSize, batchSize - off);
            inference(d_unpadded_inputs + (size_t)off * user_opt.vectorDim,
                      d_outputs ? d_outputs + (size_t)off * user_opt.outputDim : nullptr, cur, stream);
        }
        return;
    }
    if (batchSize <= 0) return;
    graft::FwdInput in;
    in.pos = d_unpadded_inputs;
    in.pos_stride = user_opt.vectorDim;
    in.table = d_fwd_hashtable;
    in.meta = &META;
    if (user_opt.outputDim == hw_opt.outputDim) {
        if (d_outputs)
            graft::mlp_forward(shape_of(mlp_opt), in, d_fwd_weights, d_master_biases, nullptr, d_outputs, batchSize,
                               OUT_ACT_NONE, stream);
    } else {
        graft::mlp_forward(shape_of(mlp_opt), in, d_fwd_weights, d_master_biases, nullptr, d_padded_outputs_float,
                           batchSize, OUT_ACT_NONE, stream);
        if (d_outputs)
            graft::unpad_f32(d_padded_outputs_float, d_outputs, batchSize, hw_opt.outputDim, user_opt.outputDim,
                             stream);
    }
}

// TinyMLPHashGrid.cu:310-334
float TinyMLPHashGrid::calculate_loss_and_grad(const half* d_unpadded_targets, int batchSize, float loss_scale,
                                               bool fetch_loss, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("calculate_loss_and_grad called while in inference mode!");
    GRAFT_HIP_CHECK(hipMemsetAsync(d_total_loss, 0, sizeof(float), stream));
    const half* tg = d_unpadded_targets;
    if (user_opt.outputDim != hw_opt.outputDim) {
        graft::pad_f16(d_unpadded_targets, d_padded_targets, batchSize, user_opt.outputDim, hw_opt.outputDim, stream);
        tg = d_padded_targets;
    }
    graft::mse_loss_grad(d_padded_outputs_float, tg, d_dLoss_internal, d_total_loss, batchSize, hw_opt.outputDim,
                         user_opt.outputDim, loss_scale, OUT_ACT_NONE, stream,
                         static_cast<graft::Workspace*>(m_workspace));
    if (fetch_loss) {
        float h = 0.f;
        GRAFT_HIP_CHECK(hipMemcpyAsync(&h, d_total_loss, sizeof(float), hipMemcpyDeviceToHost, stream));
        GRAFT_HIP_CHECK(hipStreamSynchronize(stream));
        return h / (float)(batchSize * user_opt.outputDim);
    }
    return 0.0f;
}

void TinyMLPHashGrid::run_backward(int batchSize, hipStream_t stream)
{
    if (!d_current_inputs_backward) throw std::runtime_error("backward called before forward");
    if (batchSize > m_maxBatchSize) throw std::runtime_error("batchSize exceeds maxBatchSize");
    if (batchSize <= 0) return;
    graft::mlp_backward(shape_of(mlp_opt), d_dLoss_internal, d_activations, d_fwd_weights, d_w_grad, d_b_grad,
                        d_dx_out, batchSize, stream, nullptr, true, static_cast<graft::Workspace*>(m_workspace));
    if (m_scatter)
        graft::hash_scatter_binned(static_cast<graft::ScatterPlan*>(m_scatter), META, d_dx_out,
                                   d_current_inputs_backward, 4, d_hashtable_grads, batchSize, stream, nullptr,
                                   /*grads_zero=*/false);
    else
        graft::hash_scatter_atomic(META, d_dx_out, d_current_inputs_backward, 4, d_hashtable_grads, batchSize,
                                   stream);
}

// TinyMLPHashGrid.cu:336-377 (split and fused scatter are one path here).
void TinyMLPHashGrid::backward(int batchSize, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("backward called while in inference mode!");
    run_backward(batchSize, stream);
}

void TinyMLPHashGrid::backward(const half* custom_loss_grad, int batchSize, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("backward called while in inference mode!");
    if (batchSize > m_maxBatchSize) throw std::runtime_error("batchSize exceeds maxBatchSize");
    if (batchSize <= 0) return;
    if (user_opt.outputDim != hw_opt.outputDim)
        graft::pad_f16(custom_loss_grad, d_dLoss_internal, batchSize, user_opt.outputDim, hw_opt.outputDim, stream);
    else
        GRAFT_HIP_CHECK(hipMemcpyAsync(d_dLoss_internal, custom_loss_grad,
                                       (size_t)batchSize * hw_opt.outputDim * sizeof(half), hipMemcpyDeviceToDevice,
                                       stream));
    run_backward(batchSize, stream);
}

void TinyMLPHashGrid::reset_step() { current_step = 0; }

// TinyMLPHashGrid.cu:379-392
void TinyMLPHashGrid::step(float lr, float beta1, float beta2, float epsilon, float loss_scale, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("step called while in inference mode!");
    if (current_step < 50000) current_step++;
    const AdamArgs a = adam_args(current_step, lr, beta1, beta2, epsilon, loss_scale);
    const Dims d = dims_of(mlp_opt);
    graft::adam_dense(d_master_weights, d_fwd_weights, d_w_grad, d_w_m, d_w_v, d.wsizes(), d_master_biases,
                      d_b_grad, d_b_m, d_b_v, d.bsizes(), d.layers, a, stream);
    graft::adam_hash(d_master_hashtable, d_fwd_hashtable, d_hashtable_grads, d_hash_m, d_hash_v,
                     (size_t)m_totalHashElements, a, stream);
}

void TinyMLPHashGrid::stepSplit(float lr, float beta1, float beta2, float epsilon, float loss_scale,
                                hipStream_t mlp_stream, hipStream_t hash_stream)
{
    if (!m_isTraining) throw std::runtime_error("step called while in inference mode!");
    if (current_step < 50000) current_step++;
    const AdamArgs a = adam_args(current_step, lr, beta1, beta2, epsilon, loss_scale);
    const Dims d = dims_of(mlp_opt);
    graft::adam_dense(d_master_weights, d_fwd_weights, d_w_grad, d_w_m, d_w_v, d.wsizes(), d_master_biases,
                      d_b_grad, d_b_m, d_b_v, d.bsizes(), d.layers, a, mlp_stream);
    graft::adam_hash(d_master_hashtable, d_fwd_hashtable, d_hashtable_grads, d_hash_m, d_hash_v,
                     (size_t)m_totalHashElements, a, hash_stream);
}

void TinyMLPHashGrid::scatterAdamTable(const half* d_dx_out, const float* d_positions, int pos_stride, int N,
                                       const uint32_t* d_n, float lr, float beta1, float beta2, float epsilon,
                                       float loss_scale, hipStream_t stream, hipEvent_t wait_before_update,
                                       const uint32_t* d_tile_live)
{
    if (!m_isTraining) throw std::runtime_error("step called while in inference mode!");
    if (!m_scatter) throw std::runtime_error("scatterAdamTable: this grid has no binned scatter");
    // the step count the next stepMlp() takes
    const int next = current_step < 50000 ? current_step + 1 : current_step;
    const graft::TableAdam t{d_master_hashtable, d_fwd_hashtable, d_hash_m, d_hash_v,
                             adam_args(next, lr, beta1, beta2, epsilon, loss_scale)};
    graft::hash_scatter_adam(static_cast<graft::ScatterPlan*>(m_scatter), META, d_dx_out, d_positions, pos_stride, N,
                             t, stream, d_n, wait_before_update, d_tile_live);
}

void TinyMLPHashGrid::stepMlp(float lr, float beta1, float beta2, float epsilon, float loss_scale, hipStream_t stream)
{
    if (!m_isTraining) throw std::runtime_error("step called while in inference mode!");
    if (current_step < 50000) current_step++;
    const AdamArgs a = adam_args(current_step, lr, beta1, beta2, epsilon, loss_scale);
    const Dims d = dims_of(mlp_opt);
    graft::adam_dense(d_master_weights, d_fwd_weights, d_w_grad, d_w_m, d_w_v, d.wsizes(), d_master_biases,
                      d_b_grad, d_b_m, d_b_v, d.bsizes(), d.layers, a, stream);
}

// TinyMLPHashGrid.cu:394-455: raw MLPGridOptions header, fp32 table, then W, B per layer.
void TinyMLPHashGrid::loadWeights(const std::string& filename)
{
    std::ifstream in(filename, std::ios::binary);
    if (!in.is_open()) throw std::runtime_error("Cannot open: " + filename);
    MLPGridOptions fo;
    in.read(reinterpret_cast<char*>(&fo), sizeof(MLPGridOptions));
    if (fo.numLevels != hw_opt.numLevels || fo.tableSize != hw_opt.tableSize ||
        fo.featuresLevel != hw_opt.featuresLevel || fo.hiddenDim != hw_opt.hiddenDim ||
        fo.outputDim != hw_opt.outputDim || fo.numLayers != hw_opt.numLayers)
        throw std::runtime_error("Weight file dimension mismatch");
    std::vector<float> hh(m_totalHashElements);
    in.read(reinterpret_cast<char*>(hh.data()), hh.size() * 4);
    const Dims d = dims_of(mlp_opt);
    std::vector<float> w, b;
    for (int l = 0; l < d.layers; l++) {
        const size_t we = (size_t)d.in_l(l) * d.out_l(l), be = d.out_l(l);
        std::vector<float> lw(we), lb(be);
        in.read(reinterpret_cast<char*>(lw.data()), we * 4);
        in.read(reinterpret_cast<char*>(lb.data()), be * 4);
        w.insert(w.end(), lw.begin(), lw.end());
        b.insert(b.end(), lb.begin(), lb.end());
    }
    if (!in) throw std::runtime_error("Weight file truncated: " + filename);
    loadHashgrid(hh.data());
    load_layers(d, TT, w.data(), b.data());
}

void TinyMLPHashGrid::saveWeights(const std::string& filename)
{
    std::ofstream out(filename, std::ios::binary);
    if (!out.is_open()) throw std::runtime_error("Cannot open: " + filename);
    out.write(reinterpret_cast<const char*>(&hw_opt), sizeof(MLPGridOptions));
    std::vector<float> hh(m_totalHashElements);
    saveHashgrid(hh.data());
    out.write(reinterpret_cast<const char*>(hh.data()), hh.size() * 4);
    const Dims d = dims_of(mlp_opt);
    for (int l = 0; l < d.layers; l++) {
        const size_t we = (size_t)d.in_l(l) * d.out_l(l), be = d.out_l(l);
        std::vector<float> lw(we), lb(be);
        GRAFT_HIP_CHECK(hipMemcpy(lw.data(), TT.mw.h[l], we * 4, hipMemcpyDeviceToHost));
        GRAFT_HIP_CHECK(hipMemcpy(lb.data(), TT.mb.h[l], be * 4, hipMemcpyDeviceToHost));
        out.write(reinterpret_cast<const char*>(lw.data()), we * 4);
        out.write(reinterpret_cast<const char*>(lb.data()), be * 4);
    }
}

void TinyMLPHashGrid::loadWeights(const float* hw, const float* hb) { load_layers(dims_of(mlp_opt), TT, hw, hb); }
void TinyMLPHashGrid::saveWeights(float* hw, float* hb) { save_layers(dims_of(mlp_opt), TT, hw, hb); }

void TinyMLPHashGrid::loadHashgrid(const float* host_hashgrid)
{
    GRAFT_HIP_CHECK(hipMemcpy(d_master_hashtable, host_hashgrid, (size_t)m_totalHashElements * 4, hipMemcpyHostToDevice));
    graft::f32_to_f16(d_master_hashtable, d_fwd_hashtable, m_totalHashElements, 0);
    GRAFT_HIP_CHECK(hipDeviceSynchronize());
}

void TinyMLPHashGrid::saveHashgrid(float* host_hashgrid)
{
    GRAFT_HIP_CHECK(hipMemcpy(host_hashgrid, d_master_hashtable, (size_t)m_totalHashElements * 4, hipMemcpyDeviceToHost));
}

TinyMLPHashGrid::Buffers TinyMLPHashGrid::buffers() const
{
    Buffers b{};
    b.master_hashtable = d_master_hashtable;
    b.fwd_hashtable = d_fwd_hashtable;
    b.hashtable_grads = d_hashtable_grads;
    b.hash_m = d_hash_m;
    b.hash_v = d_hash_v;
    b.master_weights = d_master_weights;
    b.master_biases = d_master_biases;
    b.fwd_weights = d_fwd_weights;
    b.w_grad = d_w_grad;
    b.b_grad = d_b_grad;
    b.activations = d_activations;
    b.dx_out = d_dx_out;
    b.dloss = d_dLoss_internal;
    b.padded_inputs = d_padded_inputs;
    b.padded_outputs = d_padded_outputs_float;
    b.hw = hw_opt;
    b.step = current_step;
    b.scatter_plan = m_scatter;
    b.workspace = m_workspace;
    b.w_m = d_w_m;
    b.w_v = d_w_v;
    b.b_m = d_b_m;
    b.b_v = d_b_v;
    return b;
}
