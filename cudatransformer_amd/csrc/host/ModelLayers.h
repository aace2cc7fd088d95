// The layers a NanoGPT training step stacks around AttentionLayer, with the reference's
// Layer<DType> interface and semantics, computing in libctattn.so:
//   LinearLayer            LinearLayer.cu:13-223 (y = x W^T + b, W [out][in])
//   LayerNormLayer         LayerNorm.cu:13-165 (gamma = 1, beta = 0, eps 1e-5)
//   ActivationLayer        ActivationLayer.cu:13-151 (ReLU, GELU tanh form, Sigmoid, Tanh)
//   MLPLayer               MLPLayer.cu:13-172 (a sequence of layers)
//   TransformerBlockLayer  TransformerBlockLayer.cu:13-220 (LayerNorm -> Attention ->
//                          LayerNorm -> MLP, no residual connections, as the reference has it)
//   TransformerLayer       TransformerLayer.cu:13-249 (a stack of blocks)
//   CheckpointLayer        CheckpointLayer.cu:10-58 (keeps its input, identity)
//   SGDOptimizer           SGDOptimizer.cu (over parameter / gradient maps)
//   AdamOptimizer          AdamOptimizer.cu:21-140 (over parameter / gradient maps)
//   AdamWOptimizer         AdamOptimizer.cu:142-233
// Same conventions as the reference: weights start at zero (cudaMakeShared zero-fills,
// LinearLayer.cu:28), LayerNorm at (1, 0); gradients accumulate across backward calls until
// zeroGrad; backward(input, gradOutput) works for any `input`.  Differences: the reference
// recomputes every activation in backward (TransformerBlockLayer.cu backward,
// TransformerLayer.cu:78-140).  Here LayerNorm, MLP, block and transformer layers keep the
// activations of their last forward and their backward reuses them when it is given that
// forward's input tensor (the same device buffer and shape); any other input is recomputed
// as the reference does.  The kept activations are released by the backward that consumes
// them, by the next forward, or by clear().  The results are the same either way; the kept
// activations cost HBM (about 0.6 GB for the 6-layer d384 B16 T256 model) and save the
// recomputation.  Also: gradient buffers are allocated on the first backward; setParameters
// copies into the layer's buffers (the attention layer's setters adopt the buffer, as the
// reference's do); Adam advances its step once per step (the reference advances it twice,
// AdamOptimizer.cu:75,95).
#pragma once

#include <cmath>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "AttentionLayer.h"
#include "ModuleLayer.h"
#include "ProjectionLayers.h"
#include "Tensor.h"

namespace ct {

// The reference's ActivationType (ActivationLayer.cu).
enum class ActivationType { ReLU = CTATTN_ACT_RELU, GELU = CTATTN_ACT_GELU, Sigmoid = CTATTN_ACT_SIGMOID, Tanh = CTATTN_ACT_TANH };

namespace detail {

template <typename DType>
inline std::shared_ptr<DType[]> filled(size_t n, float value) {
    return Tensor<DType>(std::vector<size_t>{n}, value).dataPtr();
}

template <typename DType>
inline void copyInto(const std::shared_ptr<DType[]> &dst, const Tensor<DType> &src, size_t n, const std::string &what) {
    if (src.size() != n)
        throw std::invalid_argument(what + ": expected " + std::to_string(n) + " elements, got " +
                                    std::to_string(src.size()));
    if (n > 0)
        hipCheck(hipMemcpyAsync(dst.get(), src.get(), n * sizeof(DType), hipMemcpyDeviceToDevice, Runtime::stream()),
                 "hipMemcpyAsync D2D");
}

template <typename DType>
inline std::shared_ptr<DType[]> cloneBuffer(const std::shared_ptr<DType[]> &src, size_t n) {
    auto dst = deviceAlloc<DType>(n);
    if (n > 0)
        hipCheck(hipMemcpyAsync(dst.get(), src.get(), n * sizeof(DType), hipMemcpyDeviceToDevice, Runtime::stream()),
                 "hipMemcpyAsync D2D");
    return dst;
}

template <typename DType>
inline void zeroBuffer(const std::shared_ptr<DType[]> &g, size_t n) {
    if (g != nullptr && n > 0)
        hipCheck(hipMemsetAsync(g.get(), 0, n * sizeof(DType), Runtime::stream()), "hipMemsetAsync");
}

template <typename DType>
inline void sgdStep(const std::shared_ptr<DType[]> &p, const std::shared_ptr<DType[]> &g, double lr, size_t n) {
    if (g == nullptr) return;
    ctattnCheck(ctattn_sgd_update(DTypeCode<DType>::value, p.get(), g.get(), lr, int64_t(n), Runtime::stream()),
                "ctattn_sgd_update");
}

// Rows of an activation [..., dim] (its element count over the last dimension).
template <typename DType>
inline size_t rowsOf(const Tensor<DType> &t, size_t dim, const char *what) {
    if (t.nDim() < 1 || t.shape(t.nDim() - 1) != dim)
        throw std::invalid_argument(std::string(what) + ": last dimension must be " + std::to_string(dim));
    return t.size() / dim;
}

inline std::string prefixed(const std::string &prefix, const std::string &name) { return prefix + "." + name; }

// Whether `a` is the tensor `b` (same device buffer and shape): the test for reusing the
// activations a forward on `b` kept.
template <typename DType>
inline bool sameTensor(const Tensor<DType> &a, const Tensor<DType> &b) {
    return !a.empty() && a.get() == b.get() && a.shape() == b.shape();
}

// Splits a prefixed map: entries "prefix.rest" -> "rest".
template <typename DType>
inline std::map<std::string, Tensor<DType>> sub(const std::map<std::string, Tensor<DType>> &m, const std::string &prefix) {
    std::map<std::string, Tensor<DType>> out;
    const std::string p = prefix + ".";
    for (const auto &[k, v] : m)
        if (k.compare(0, p.size(), p) == 0) out[k.substr(p.size())] = v;
    return out;
}

template <typename DType>
inline void merge(std::map<std::string, Tensor<DType>> &into, const std::string &prefix,
                  const std::map<std::string, Tensor<DType>> &from) {
    for (const auto &[k, v] : from) into[prefixed(prefix, k)] = v;
}

}  // namespace detail

template <typename DType = float>
struct LinearLayer : public Layer<DType> {
    int inputDim = 1;
    int outputDim = 1;
    bool useBias = true;
    std::shared_ptr<DType[]> weights, biases, weightsGrad, biasesGrad;

    LinearLayer(int inputDim, int outputDim, bool useBias = true)
        : inputDim(inputDim), outputDim(outputDim), useBias(useBias) {
        if (inputDim < 1 || outputDim < 1) throw std::invalid_argument("LinearLayer: dimensions must be >= 1");
        weights = detail::zeros<DType>(weightSize());
        if (useBias) biases = detail::zeros<DType>(size_t(outputDim));
    }

    size_t weightSize() const { return size_t(inputDim) * outputDim; }

    std::shared_ptr<Layer<DType>> clone() override {
        auto c = std::make_shared<LinearLayer<DType>>(inputDim, outputDim, useBias);
        c->weights = detail::cloneBuffer(weights, weightSize());
        if (useBias) c->biases = detail::cloneBuffer(biases, size_t(outputDim));
        return c;
    }

    // [..., inputDim] -> [..., outputDim] (LinearLayer.cu forward).
    Tensor<DType> forward(Tensor<DType> input) override {
        const size_t rows = detail::rowsOf(input, size_t(inputDim), "LinearLayer input");
        std::vector<size_t> shape = input.shape();
        shape.back() = size_t(outputDim);
        Tensor<DType> out = Tensor<DType>::empty(shape);
        ctattnCheck(ctattn_linear_fwd(DTypeCode<DType>::value, input.get(), weights.get(),
                                      useBias ? biases.get() : nullptr, out.get(), int64_t(rows), outputDim, inputDim,
                                      Runtime::stream()),
                    "ctattn_linear_fwd");
        return out;
    }

    // forward() followed by an activation, in one launch (ctattn_linear_act_fwd): returns the
    // pre-activation (the activation layer's input) and the activated output.
    std::pair<Tensor<DType>, Tensor<DType>> forwardAct(const Tensor<DType> &input, int act) {
        const size_t rows = detail::rowsOf(input, size_t(inputDim), "LinearLayer input");
        std::vector<size_t> shape = input.shape();
        shape.back() = size_t(outputDim);
        Tensor<DType> pre = Tensor<DType>::empty(shape), out = Tensor<DType>::empty(shape);
        ctattnCheck(ctattn_linear_act_fwd(DTypeCode<DType>::value, act, input.get(), weights.get(),
                                          useBias ? biases.get() : nullptr, pre.get(), out.get(), int64_t(rows),
                                          outputDim, inputDim, Runtime::stream()),
                    "ctattn_linear_act_fwd");
        return {pre, out};
    }

    // backward() whose dInput also goes through the preceding activation (input = act(pre)):
    // returns the gradient of pre (ctattn_linear_act_bwd).
    Tensor<DType> backwardAct(const Tensor<DType> &input, const Tensor<DType> &gradOutput, const Tensor<DType> &pre,
                              int act) {
        const size_t rows = detail::rowsOf(input, size_t(inputDim), "LinearLayer input");
        if (detail::rowsOf(gradOutput, size_t(outputDim), "LinearLayer grad_output") != rows ||
            pre.size() != input.size())
            throw std::invalid_argument("LinearLayer: grad_output / pre-activation shape");
        ensureGrads();
        Tensor<DType> preGrad = Tensor<DType>::empty(input.shape());
        const int dt = DTypeCode<DType>::value;
        const int64_t wsBytes = ctattn_linear_bwd_workspace_bytes(dt, int64_t(rows), outputDim, inputDim);
        auto ws = detail::workspace(wsBytes, "ctattn_linear_bwd_workspace_bytes");
        ctattnCheck(ctattn_linear_act_bwd(dt, act, input.get(), weights.get(), gradOutput.get(), pre.get(),
                                          preGrad.get(), weightsGrad.get(), useBias ? biasesGrad.get() : nullptr,
                                          ws.get(), wsBytes, int64_t(rows), outputDim, inputDim, Runtime::stream()),
                    "ctattn_linear_act_bwd");
        return preGrad;
    }

    // Accumulates dW (and dB), returns dInput (LinearLayer.cu backward).
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override {
        const size_t rows = detail::rowsOf(input, size_t(inputDim), "LinearLayer input");
        if (detail::rowsOf(gradOutput, size_t(outputDim), "LinearLayer grad_output") != rows)
            throw std::invalid_argument("LinearLayer: grad_output rows do not match the input");
        ensureGrads();
        Tensor<DType> inputGrad = Tensor<DType>::empty(input.shape());
        const int dt = DTypeCode<DType>::value;
        const int64_t wsBytes = ctattn_linear_bwd_workspace_bytes(dt, int64_t(rows), outputDim, inputDim);
        auto ws = detail::workspace(wsBytes, "ctattn_linear_bwd_workspace_bytes");
        ctattnCheck(ctattn_linear_bwd(dt, input.get(), weights.get(), gradOutput.get(), inputGrad.get(),
                                      weightsGrad.get(), useBias ? biasesGrad.get() : nullptr, ws.get(), wsBytes,
                                      int64_t(rows), outputDim, inputDim, Runtime::stream()),
                    "ctattn_linear_bwd");
        return inputGrad;
    }

    std::map<std::string, Tensor<DType>> getParameters() override {
        std::map<std::string, Tensor<DType>> m{{"weights", Tensor<DType>(weights, weightShape())}};
        if (useBias) m["biases"] = Tensor<DType>(biases, {size_t(outputDim)});
        return m;
    }
    void setParameters(const std::map<std::string, Tensor<DType>> &p) override {
        if (p.count("weights")) detail::copyInto(weights, p.at("weights"), weightSize(), "LinearLayer weights");
        if (useBias && p.count("biases")) detail::copyInto(biases, p.at("biases"), size_t(outputDim), "LinearLayer biases");
    }
    std::map<std::string, Tensor<DType>> getGradients() override {
        ensureGrads();
        std::map<std::string, Tensor<DType>> m{{"weights", Tensor<DType>(weightsGrad, weightShape())}};
        if (useBias) m["biases"] = Tensor<DType>(biasesGrad, {size_t(outputDim)});
        return m;
    }
    void zeroGrad() override {
        detail::zeroBuffer(weightsGrad, weightSize());
        detail::zeroBuffer(biasesGrad, size_t(outputDim));
    }
    void sgdUpdate(double lr) override {
        detail::sgdStep(weights, weightsGrad, lr, weightSize());
        if (useBias) detail::sgdStep(biases, biasesGrad, lr, size_t(outputDim));
    }

    // Shallow accessors (LinearLayer.cu:140-223): getters share the buffer, setters adopt it.
    Tensor<DType> getWeights() { return Tensor<DType>(weights, weightShape()); }
    void setWeights(const Tensor<DType> &t) { weights = adopt(t, weightSize(), "weights"); }
    Tensor<DType> getBiases() { return useBias ? Tensor<DType>(biases, {size_t(outputDim)}) : Tensor<DType>(); }
    void setBiases(const Tensor<DType> &t) { biases = adopt(t, useBias ? size_t(outputDim) : 0, "biases"); }
    Tensor<DType> getWeightGrad() {
        ensureGrads();
        return Tensor<DType>(weightsGrad, weightShape());
    }
    void setWeightGrad(const Tensor<DType> &t) { weightsGrad = adopt(t, weightSize(), "weight gradient"); }
    Tensor<DType> getBiasGrad() {
        ensureGrads();
        return useBias ? Tensor<DType>(biasesGrad, {size_t(outputDim)}) : Tensor<DType>();
    }
    void setBiasGrad(const Tensor<DType> &t) { biasesGrad = adopt(t, useBias ? size_t(outputDim) : 0, "bias gradient"); }

private:
    static std::shared_ptr<DType[]> adopt(const Tensor<DType> &t, size_t n, const char *what) {
        if (n == 0) throw std::invalid_argument(std::string("LinearLayer has no ") + what);
        if (t.size() != n)
            throw std::invalid_argument(std::string("LinearLayer ") + what + ": expected " + std::to_string(n) +
                                        " elements, got " + std::to_string(t.size()));
        return t.dataPtr();
    }
    std::vector<size_t> weightShape() const { return {size_t(outputDim), size_t(inputDim)}; }
    void ensureGrads() {
        if (weightsGrad == nullptr) weightsGrad = detail::zeros<DType>(weightSize());
        if (useBias && biasesGrad == nullptr) biasesGrad = detail::zeros<DType>(size_t(outputDim));
    }
};

template <typename DType = float>
struct LayerNormLayer : public Layer<DType> {
    int inputDim = 1;
    double epsilon = 1e-5;
    std::shared_ptr<DType[]> weights, biases, weightsGrad, biasesGrad;

    LayerNormLayer(int inputDim, double epsilon = 1e-5) : inputDim(inputDim), epsilon(epsilon) {
        if (inputDim < 1) throw std::invalid_argument("LayerNormLayer: inputDim must be >= 1");
        weights = detail::filled<DType>(size_t(inputDim), 1.f);
        biases = detail::zeros<DType>(size_t(inputDim));
    }

    std::shared_ptr<Layer<DType>> clone() override {
        auto c = std::make_shared<LayerNormLayer<DType>>(inputDim, epsilon);
        c->weights = detail::cloneBuffer(weights, size_t(inputDim));
        c->biases = detail::cloneBuffer(biases, size_t(inputDim));
        return c;
    }

    Tensor<DType> forward(Tensor<DType> input) override {
        auto [out, stats] = run(input);
        cachedInput = input;
        cachedStats = stats;
        return out;
    }

    // dX and the accumulated dGamma / dBeta (LayerNorm.cu:143), from the row statistics the
    // last forward kept when `input` is its input, else recomputed from `input`.
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override {
        const size_t rows = detail::rowsOf(input, size_t(inputDim), "LayerNormLayer input");
        if (gradOutput.size() != input.size()) throw std::invalid_argument("LayerNormLayer: grad_output shape");
        auto stats = detail::sameTensor(cachedInput, input) ? cachedStats : run(input).second;
        clear();
        ensureGrads();
        Tensor<DType> inputGrad = Tensor<DType>::empty(input.shape());
        const int dt = DTypeCode<DType>::value;
        const int64_t wsBytes = ctattn_layernorm_bwd_workspace_bytes(dt, int64_t(rows), inputDim);
        auto ws = detail::workspace(wsBytes, "ctattn_layernorm_bwd_workspace_bytes");
        ctattnCheck(ctattn_layernorm_bwd(dt, input.get(), weights.get(), gradOutput.get(), stats.get(),
                                         stats.get() + rows, inputGrad.get(), weightsGrad.get(), biasesGrad.get(),
                                         ws.get(), wsBytes, int64_t(rows), inputDim, Runtime::stream()),
                    "ctattn_layernorm_bwd");
        return inputGrad;
    }

    std::map<std::string, Tensor<DType>> getParameters() override {
        return {{"weights", Tensor<DType>(weights, {size_t(inputDim)})}, {"biases", Tensor<DType>(biases, {size_t(inputDim)})}};
    }
    void setParameters(const std::map<std::string, Tensor<DType>> &p) override {
        if (p.count("weights")) detail::copyInto(weights, p.at("weights"), size_t(inputDim), "LayerNorm weights");
        if (p.count("biases")) detail::copyInto(biases, p.at("biases"), size_t(inputDim), "LayerNorm biases");
    }
    std::map<std::string, Tensor<DType>> getGradients() override {
        ensureGrads();
        return {{"weights", Tensor<DType>(weightsGrad, {size_t(inputDim)})},
                {"biases", Tensor<DType>(biasesGrad, {size_t(inputDim)})}};
    }
    void zeroGrad() override {
        detail::zeroBuffer(weightsGrad, size_t(inputDim));
        detail::zeroBuffer(biasesGrad, size_t(inputDim));
    }
    void sgdUpdate(double lr) override {
        detail::sgdStep(weights, weightsGrad, lr, size_t(inputDim));
        detail::sgdStep(biases, biasesGrad, lr, size_t(inputDim));
    }
    void clear() override {
        cachedInput = Tensor<DType>();
        cachedStats = nullptr;
    }

private:
    Tensor<DType> cachedInput;
    std::shared_ptr<StatOf<DType>[]> cachedStats;

    // Output and the row statistics [mean (rows) | rstd (rows)] (fp64 for double, else fp32).
    std::pair<Tensor<DType>, std::shared_ptr<StatOf<DType>[]>> run(const Tensor<DType> &input) {
        const size_t rows = detail::rowsOf(input, size_t(inputDim), "LayerNormLayer input");
        Tensor<DType> out = Tensor<DType>::empty(input.shape());
        auto stats = deviceAlloc<StatOf<DType>>(2 * rows);
        ctattnCheck(ctattn_layernorm_fwd(DTypeCode<DType>::value, input.get(), weights.get(), biases.get(), out.get(),
                                         stats.get(), stats.get() + rows, int64_t(rows), inputDim, epsilon,
                                         Runtime::stream()),
                    "ctattn_layernorm_fwd");
        return {out, stats};
    }
    void ensureGrads() {
        if (weightsGrad == nullptr) weightsGrad = detail::zeros<DType>(size_t(inputDim));
        if (biasesGrad == nullptr) biasesGrad = detail::zeros<DType>(size_t(inputDim));
    }
};

template <typename DType = float>
struct ActivationLayer : public Layer<DType> {
    int inputDim = 1;
    ActivationType activationType = ActivationType::ReLU;

    ActivationLayer(int inputDim, ActivationType type) : inputDim(inputDim), activationType(type) {}

    std::shared_ptr<Layer<DType>> clone() override {
        return std::make_shared<ActivationLayer<DType>>(inputDim, activationType);
    }
    Tensor<DType> forward(Tensor<DType> input) override {
        Tensor<DType> out = Tensor<DType>::empty(input.shape());
        ctattnCheck(ctattn_activation_fwd(DTypeCode<DType>::value, int(activationType), input.get(), out.get(),
                                          int64_t(input.size()), Runtime::stream()),
                    "ctattn_activation_fwd");
        return out;
    }
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override {
        if (gradOutput.size() != input.size()) throw std::invalid_argument("ActivationLayer: grad_output shape");
        Tensor<DType> inputGrad = Tensor<DType>::empty(input.shape());
        ctattnCheck(ctattn_activation_bwd(DTypeCode<DType>::value, int(activationType), input.get(), gradOutput.get(),
                                          inputGrad.get(), int64_t(input.size()), Runtime::stream()),
                    "ctattn_activation_bwd");
        return inputGrad;
    }
};

// A sequence of layers; parameters are keyed "layer_<index>.<name>" (MLPLayer.cu:105-146).
template <typename DType = float>
struct MLPLayer : public Layer<DType> {
    std::vector<Module<DType>> layers;

    explicit MLPLayer(std::vector<Module<DType>> layers) : layers(std::move(layers)) {}

    std::shared_ptr<Layer<DType>> clone() override {
        std::vector<Module<DType>> c;
        for (auto &l : layers) c.push_back(l->clone());
        return std::make_shared<MLPLayer<DType>>(c);
    }
    // A linear layer followed by an activation runs as one GEMM launch (its epilogue applies
    // the activation); the activation's input, the pre-activation, is kept like any layer input.
    Tensor<DType> forward(Tensor<DType> input) override {
        cachedInputs.clear();
        for (size_t i = 0; i < layers.size(); ++i) {
            cachedInputs.push_back(input);
            if (auto *act = activationAfterLinear(i)) {
                auto po = static_cast<LinearLayer<DType> *>(layers[i].get())->forwardAct(input, int(act->activationType));
                cachedInputs.push_back(po.first);
                input = po.second;
                ++i;
                continue;
            }
            input = layers[i]->forward(input);
        }
        return input;
    }
    // Backpropagates through the layers in reverse, from the layer inputs the last forward
    // kept when `input` is its input, else from inputs recomputed from `input`.
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override {
        std::vector<Tensor<DType>> inputs;
        if (!cachedInputs.empty() && detail::sameTensor(cachedInputs.front(), input)) {
            inputs.swap(cachedInputs);
        } else {
            clear();
            inputs.push_back(input);
            for (size_t i = 0; i + 1 < layers.size(); ++i) inputs.push_back(layers[i]->forward(inputs.back()));
        }
        for (size_t i = layers.size(); i-- > 0;) {
            auto *lin = dynamic_cast<LinearLayer<DType> *>(layers[i].get());
            auto *act = i > 0 ? dynamic_cast<ActivationLayer<DType> *>(layers[i - 1].get()) : nullptr;
            if (lin != nullptr && act != nullptr) {
                // The linear layer's dX and the preceding activation's backward in one launch.
                gradOutput = lin->backwardAct(inputs[i], gradOutput, inputs[i - 1], int(act->activationType));
                inputs[i] = inputs[i - 1] = Tensor<DType>();
                --i;
                continue;
            }
            gradOutput = layers[i]->backward(inputs[i], gradOutput);
            inputs[i] = Tensor<DType>();
        }
        return gradOutput;
    }
    void clear() override {
        cachedInputs.clear();
        for (auto &l : layers) l->clear();
    }
    std::map<std::string, Tensor<DType>> getParameters() override {
        std::map<std::string, Tensor<DType>> m;
        for (size_t i = 0; i < layers.size(); ++i) detail::merge(m, key(i), layers[i]->getParameters());
        return m;
    }
    void setParameters(const std::map<std::string, Tensor<DType>> &p) override {
        for (size_t i = 0; i < layers.size(); ++i) layers[i]->setParameters(detail::sub(p, key(i)));
    }
    std::map<std::string, Tensor<DType>> getGradients() override {
        std::map<std::string, Tensor<DType>> m;
        for (size_t i = 0; i < layers.size(); ++i) detail::merge(m, key(i), layers[i]->getGradients());
        return m;
    }
    void zeroGrad() override {
        for (auto &l : layers) l->zeroGrad();
    }
    void sgdUpdate(double lr) override {
        for (auto &l : layers) l->sgdUpdate(lr);
    }

private:
    std::vector<Tensor<DType>> cachedInputs;  // each layer's input in the last forward
    static std::string key(size_t i) { return "layer_" + std::to_string(i); }
    // The activation layer at i + 1 when layer i is a linear layer, else null.
    ActivationLayer<DType> *activationAfterLinear(size_t i) const {
        if (i + 1 >= layers.size() || dynamic_cast<LinearLayer<DType> *>(layers[i].get()) == nullptr) return nullptr;
        return dynamic_cast<ActivationLayer<DType> *>(layers[i + 1].get());
    }
};

template <typename DType = float>
struct TransformerBlockLayer : public Layer<DType> {
    std::shared_ptr<LayerNormLayer<DType>> firstNorm;
    std::shared_ptr<AttentionLayer<DType>> attention;
    std::shared_ptr<LayerNormLayer<DType>> secondNorm;
    std::shared_ptr<MLPLayer<DType>> mlp;
    int inputDim = 1, numHeads = 1, headDim = 1, mlpDim = 1;
    ActivationType activationType = ActivationType::ReLU;

    TransformerBlockLayer(int inputDim, int numHeads, int headDim, int mlpDim,
                          ActivationType activationType = ActivationType::ReLU, bool causal = false)
        : inputDim(inputDim), numHeads(numHeads), headDim(headDim), mlpDim(mlpDim), activationType(activationType) {
        firstNorm = std::make_shared<LayerNormLayer<DType>>(inputDim);
        attention = std::make_shared<AttentionLayer<DType>>(inputDim, numHeads, headDim, causal);
        secondNorm = std::make_shared<LayerNormLayer<DType>>(inputDim);
        mlp = std::make_shared<MLPLayer<DType>>(std::vector<Module<DType>>{
            std::make_shared<LinearLayer<DType>>(inputDim, mlpDim),
            std::make_shared<ActivationLayer<DType>>(mlpDim, activationType),
            std::make_shared<LinearLayer<DType>>(mlpDim, inputDim)});
    }

    std::shared_ptr<Layer<DType>> clone() override {
        auto c = std::make_shared<TransformerBlockLayer<DType>>(inputDim, numHeads, headDim, mlpDim, activationType,
                                                                attention->causal());
        c->firstNorm = std::static_pointer_cast<LayerNormLayer<DType>>(firstNorm->clone());
        c->attention = std::static_pointer_cast<AttentionLayer<DType>>(attention->clone());
        c->secondNorm = std::static_pointer_cast<LayerNormLayer<DType>>(secondNorm->clone());
        c->mlp = std::static_pointer_cast<MLPLayer<DType>>(mlp->clone());
        return c;
    }

    // LayerNorm -> Attention -> LayerNorm -> MLP (TransformerBlockLayer.cu:60-66), keeping
    // the activations and attention states for backward.
    Tensor<DType> forward(Tensor<DType> input) override {
        Kept k = run(input);
        Tensor<DType> out = mlp->forward(k.normed2);
        kept = std::move(k);
        return out;
    }

    // Backpropagates through MLP, LayerNorm, attention and LayerNorm
    // (TransformerBlockLayer.cu:74-87), from the last forward's activations when `input` is
    // its input, else from activations recomputed from `input`.
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override {
        Kept k;
        if (detail::sameTensor(kept.input, input)) {
            std::swap(k, kept);
        } else {
            clear();
            k = run(input);
        }
        Tensor<DType> g = mlp->backward(k.normed2, gradOutput);
        k.normed2 = Tensor<DType>();
        g = secondNorm->backward(k.attn, g);
        k.attn = Tensor<DType>();
        g = attention->backward(k.normed, g, k.states.data());
        return firstNorm->backward(input, g);
    }
    void clear() override {
        kept = Kept();
        firstNorm->clear();
        secondNorm->clear();
        mlp->clear();
        attention->flashAttn.clearCache();
    }

    std::map<std::string, Tensor<DType>> getParameters() override { return collect(false); }
    std::map<std::string, Tensor<DType>> getGradients() override { return collect(true); }
    void setParameters(const std::map<std::string, Tensor<DType>> &p) override {
        firstNorm->setParameters(detail::sub(p, "firstNorm"));
        attention->setParameters(detail::sub(p, "attention"));
        secondNorm->setParameters(detail::sub(p, "secondNorm"));
        mlp->setParameters(detail::sub(p, "mlp"));
    }
    void zeroGrad() override {
        firstNorm->zeroGrad();
        attention->zeroGrad();
        secondNorm->zeroGrad();
        mlp->zeroGrad();
    }
    void sgdUpdate(double lr) override {
        firstNorm->sgdUpdate(lr);
        attention->sgdUpdate(lr);
        secondNorm->sgdUpdate(lr);
        mlp->sgdUpdate(lr);
    }

private:
    struct Kept {
        Tensor<DType> input, normed, attn, normed2;
        std::array<Tensor<DType>, 4> states;  // attention's [Q, K, V, attention output]
    };
    Kept kept;

    // The activations up to the MLP's input.
    Kept run(const Tensor<DType> &input) {
        Kept k;
        k.input = input;
        k.normed = firstNorm->forward(input);
        k.attn = attention->forward(k.normed, k.states.data());
        k.normed2 = secondNorm->forward(k.attn);
        return k;
    }

    std::map<std::string, Tensor<DType>> collect(bool grads) {
        std::map<std::string, Tensor<DType>> m;
        auto get = [grads](Layer<DType> &l) { return grads ? l.getGradients() : l.getParameters(); };
        detail::merge(m, "firstNorm", get(*firstNorm));
        detail::merge(m, "attention", get(*attention));
        detail::merge(m, "secondNorm", get(*secondNorm));
        detail::merge(m, "mlp", get(*mlp));
        return m;
    }
};

// A stack of numLayers blocks (TransformerLayer.cu:29-41).  Parameters are keyed
// "layer_<slot>.<name>" where slot is the block's position in the reference's layer list,
// which holds a CheckpointLayer before every checkpointGap-th block (checkpointGap > 0), so
// the keys match the reference's for every checkpointGap.  backward backpropagates block by
// block; the gradients equal the reference's for any checkpointGap (its checkpoints only
// change what it keeps in memory).
template <typename DType = float>
struct TransformerLayer : public Layer<DType> {
    std::vector<std::shared_ptr<TransformerBlockLayer<DType>>> blocks;
    int inputDim = 1, numHeads = 1, headDim = 1, mlpDim = 1, numLayers = 1, checkpointGap = 0;
    ActivationType activationType = ActivationType::ReLU;

    TransformerLayer(int inputDim, int numHeads, int headDim, int mlpDim, int numLayers, int checkpointGap = 0,
                     ActivationType activationType = ActivationType::ReLU, bool causal = false)
        : inputDim(inputDim), numHeads(numHeads), headDim(headDim), mlpDim(mlpDim), numLayers(numLayers),
          checkpointGap(checkpointGap), activationType(activationType) {
        if (numLayers < 1) throw std::invalid_argument("TransformerLayer: numLayers must be >= 1");
        if (checkpointGap < 0) throw std::invalid_argument("TransformerLayer: checkpointGap must be >= 0");
        for (int i = 0; i < numLayers; ++i)
            blocks.push_back(std::make_shared<TransformerBlockLayer<DType>>(inputDim, numHeads, headDim, mlpDim,
                                                                           activationType, causal));
    }

    bool causal() const { return blocks.front()->attention->causal(); }

    std::shared_ptr<Layer<DType>> clone() override {
        auto c = std::make_shared<TransformerLayer<DType>>(*this);
        c->blockInputs.clear();
        for (auto &b : c->blocks) b = std::static_pointer_cast<TransformerBlockLayer<DType>>(b->clone());
        return c;
    }
    Tensor<DType> forward(Tensor<DType> input) override {
        blockInputs.clear();
        for (auto &b : blocks) {
            blockInputs.push_back(input);
            input = b->forward(input);
        }
        return input;
    }
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override {
        std::vector<Tensor<DType>> inputs;
        if (!blockInputs.empty() && detail::sameTensor(blockInputs.front(), input)) {
            inputs.swap(blockInputs);
        } else {
            clear();
            inputs.push_back(input);
            for (size_t i = 0; i + 1 < blocks.size(); ++i) inputs.push_back(blocks[i]->forward(inputs.back()));
        }
        for (size_t i = blocks.size(); i-- > 0;) {
            gradOutput = blocks[i]->backward(inputs[i], gradOutput);
            inputs[i] = Tensor<DType>();
        }
        return gradOutput;
    }
    void clear() override {
        blockInputs.clear();
        for (auto &b : blocks) b->clear();
    }
    std::map<std::string, Tensor<DType>> getParameters() override {
        std::map<std::string, Tensor<DType>> m;
        for (size_t i = 0; i < blocks.size(); ++i) detail::merge(m, key(i), blocks[i]->getParameters());
        return m;
    }
    void setParameters(const std::map<std::string, Tensor<DType>> &p) override {
        for (size_t i = 0; i < blocks.size(); ++i) blocks[i]->setParameters(detail::sub(p, key(i)));
    }
    std::map<std::string, Tensor<DType>> getGradients() override {
        std::map<std::string, Tensor<DType>> m;
        for (size_t i = 0; i < blocks.size(); ++i) detail::merge(m, key(i), blocks[i]->getGradients());
        return m;
    }
    void zeroGrad() override {
        for (auto &b : blocks) b->zeroGrad();
    }
    void sgdUpdate(double lr) override {
        for (auto &b : blocks) b->sgdUpdate(lr);
    }

private:
    std::vector<Tensor<DType>> blockInputs;  // each block's input in the last forward

    std::string key(size_t i) const {
        const size_t slot = i + (checkpointGap > 0 ? i / size_t(checkpointGap) : 0);
        return "layer_" + std::to_string(slot);
    }
};

// Gradient-checkpoint marker (CheckpointLayer.cu:10-58): forward keeps its input and
// returns it, backward passes the gradient through, clear() drops the kept input.
template <typename DType = float>
struct CheckpointLayer : public Layer<DType> {
    Tensor<DType> activationStorage;

    std::shared_ptr<Layer<DType>> clone() override {
        auto c = std::make_shared<CheckpointLayer<DType>>();
        if (activationStorage.size() > 0) c->activationStorage = activationStorage.clone();
        return c;
    }
    Tensor<DType> forward(Tensor<DType> input) override {
        activationStorage = input;
        return input;
    }
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override { return gradOutput; }
    void clear() override { activationStorage = Tensor<DType>(); }
};

namespace detail {
// The checks every optimizer's step makes before updating anything (AdamOptimizer.cu step,
// SGDOptimizer.cu step): each parameter has a gradient of its size.
template <typename DType>
inline void checkGrads(const std::map<std::string, Tensor<DType>> &params,
                       const std::map<std::string, Tensor<DType>> &grads) {
    for (const auto &[name, p] : params) {
        auto g = grads.find(name);
        if (g == grads.end())
            throw std::invalid_argument("Gradient for parameter '" + name + "' not found in gradients map.");
        if (g->second.size() != p.size())
            throw std::invalid_argument("Size mismatch between parameter '" + name + "' and its gradient.");
    }
}
}  // namespace detail

// SGD over a parameter map (SGDOptimizer.cu): step(grads) does params[k] -= lr * grads[k] for
// every parameter, after checking that each has a gradient of its size.
template <typename DType = float>
struct SGDOptimizer {
    std::map<std::string, Tensor<DType>> parameters;
    double learningRate;

    SGDOptimizer(std::map<std::string, Tensor<DType>> params, double lr)
        : parameters(std::move(params)), learningRate(lr) {}

    void step(const std::map<std::string, Tensor<DType>> &grads) {
        detail::checkGrads(parameters, grads);
        for (const auto &[name, p] : parameters)
            detail::sgdStep(p.dataPtr(), grads.at(name).dataPtr(), learningRate, p.size());
    }
    double getLearningRate() const { return learningRate; }
    void setLearningRate(double lr) { learningRate = lr; }
};

// Adam / AdamW over a parameter map (AdamOptimizer.cu:21-140 AdamOptimizer, :142-233
// AdamWOptimizer): step(grads) updates every parameter (one launch per 32 tensors), and
// throws if `grads` lacks one or a size differs, as the reference does.  The moments (fp64
// for double parameters, fp32 otherwise) are zero at construction; the step counter advances
// once per step (the reference advances it twice).  decoupled = false is the reference's
// AdamOptimizer (decay folded into the gradient), true its AdamWOptimizer.
template <typename DType = float>
struct AdamOptimizer {
    using Stat = StatOf<DType>;
    std::map<std::string, Tensor<DType>> parameters;
    double learningRate, beta1, beta2, epsilon, decay;
    bool decoupled = false;
    int timeStep = 0;
    std::map<std::string, std::pair<std::shared_ptr<Stat[]>, std::shared_ptr<Stat[]>>> moments;

    explicit AdamOptimizer(std::map<std::string, Tensor<DType>> params, double lr = 1e-3, double b1 = 0.9,
                           double b2 = 0.999, double eps = 1e-8, double decay = 0.0, bool decoupled = false)
        : parameters(std::move(params)), learningRate(lr), beta1(b1), beta2(b2), epsilon(eps), decay(decay),
          decoupled(decoupled) {
        for (const auto &[name, p] : parameters)
            moments[name] = {detail::zeros<Stat>(p.size()), detail::zeros<Stat>(p.size())};
    }

    void step(const std::map<std::string, Tensor<DType>> &grads) {
        detail::checkGrads(parameters, grads);
        ++timeStep;
        std::vector<void *> ps;
        std::vector<const void *> gs;
        std::vector<void *> ms, vs;
        std::vector<int64_t> ns;
        for (const auto &[name, p] : parameters) {
            auto &mv = moments[name];
            ps.push_back(p.get());
            gs.push_back(grads.at(name).get());
            ms.push_back(mv.first.get());
            vs.push_back(mv.second.get());
            ns.push_back(int64_t(p.size()));
        }
        ctattnCheck(ctattn_adam_update_multi(DTypeCode<DType>::value, int(ps.size()), ps.data(), gs.data(), ms.data(),
                                             vs.data(), ns.data(), learningRate, beta1, beta2, epsilon, decay,
                                             timeStep, decoupled ? 1 : 0, Runtime::stream()),
                    "ctattn_adam_update_multi");
    }

    double getLearningRate() const { return learningRate; }
    void setLearningRate(double lr) { learningRate = lr; }
    int getTimeStep() const { return timeStep; }
    void setTimeStep(int t) { timeStep = t; }
};

// AdamW: the decoupled-decay variant (AdamOptimizer.cu:142-233).
template <typename DType = float>
struct AdamWOptimizer : public AdamOptimizer<DType> {
    explicit AdamWOptimizer(std::map<std::string, Tensor<DType>> params, double lr = 1e-3, double b1 = 0.9,
                            double b2 = 0.999, double eps = 1e-8, double decay = 0.0)
        : AdamOptimizer<DType>(std::move(params), lr, b1, b2, eps, decay, true) {}
};

}  // namespace ct
