// AttentionLayer<DType>: QKV projection -> flash attention -> output projection, the
// reference's master attention layer (AttentionLayer.cu:13-407) as a Layer<DType>.
//
// Same interface and semantics: forward / backward with and without the cached states
// [Q, K, V, attention output], shallow weight getters and setters, zeroGrad, sgdUpdate,
// parameter and gradient maps, clone.  Differences, all deliberate:
//   * the attention output is kept in the states and used by the output projection's
//     backward (the reference clears states[3] before its backward reads it,
//     AttentionLayer.cu:98-100,137);
//   * an optional causal mask (the reference has none; default off);
//   * the weight getters report the shape the data has, [H*d, E] for Q/K/V and
//     [E, H*d] for the output projection; the reference labels the Q/K/V weights
//     [E, H*d] (AttentionLayer.cu:168) while its kernels index [H*d][E]; the two agree
//     whenever E == H*d;
//   * setters check the adopted buffer's element count.
#pragma once

#include <array>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "FlashAttentionLayer.h"
#include "ModuleLayer.h"
#include "ProjectionLayers.h"

namespace ct {

template <typename DType = float>
struct AttentionLayer : public Layer<DType> {
    QKVProjectionLayer<DType> qkvProj;
    FlashAttentionLayer<DType> flashAttn;
    OutputProjectionLayer<DType> outProj;
    int inputDim = 1;
    int numHeads = 1;
    int headDim = 1;

    AttentionLayer(int inputDim, int numHeads, int headDim, bool causal = false)
        : qkvProj(inputDim, numHeads, headDim),
          flashAttn(headDim, numHeads, causal),
          outProj(inputDim, headDim, numHeads),
          inputDim(inputDim),
          numHeads(numHeads),
          headDim(headDim) {}

    bool causal() const { return flashAttn.causal; }

    // Deep copy of all eight parameter buffers (AttentionLayer.cu:37-58).
    std::shared_ptr<Layer<DType>> clone() override {
        auto c = std::make_shared<AttentionLayer<DType>>(inputDim, numHeads, headDim, flashAttn.causal);
        auto q = qkvProj.clone();
        auto o = outProj.clone();
        c->qkvProj.weightsQuery = q->weightsQuery;
        c->qkvProj.weightsKey = q->weightsKey;
        c->qkvProj.weightsValue = q->weightsValue;
        c->qkvProj.biasesQuery = q->biasesQuery;
        c->qkvProj.biasesKey = q->biasesKey;
        c->qkvProj.biasesValue = q->biasesValue;
        c->outProj.weightsProj = o->weightsProj;
        c->outProj.biasesProj = o->biasesProj;
        return c;
    }

    Tensor<DType> forward(Tensor<DType> input) override { return forward(input, nullptr); }

    // outStates (4 tensors, optional) receives [Q, K, V, attention output] for backward
    // (AttentionLayer.cu:75-102).
    Tensor<DType> forward(Tensor<DType> input, Tensor<DType> *outStates) {
        std::array<Tensor<DType>, 3> qkv = qkvProj.computeQKV(input);
        Tensor<DType> attn = flashAttn.computeAttention(qkv[0], qkv[1], qkv[2], outStates != nullptr);
        if (outStates != nullptr) {
            outStates[0] = qkv[0];
            outStates[1] = qkv[1];
            outStates[2] = qkv[2];
            outStates[3] = attn;
        }
        return outProj.forward(attn);
    }

    // Recomputes the forward states, then backpropagates (AttentionLayer.cu:112-117).
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) override {
        std::array<Tensor<DType>, 4> states;
        forward(input, states.data());
        return backward(input, gradOutput, states.data());
    }

    // Backpropagates with the cached states; accumulates every parameter gradient and returns
    // dInput (AttentionLayer.cu:127-158).  The states are released as they are consumed.
    Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput, Tensor<DType> *states) {
        if (states == nullptr) throw std::invalid_argument("backward: states must not be null");
        for (int i = 0; i < 4; ++i)
            if (states[i].empty()) throw std::invalid_argument("backward: states must hold [Q, K, V, attention output]");
        Tensor<DType> attnGrad = outProj.backward(states[3], gradOutput);
        states[3] = Tensor<DType>();
        std::array<Tensor<DType>, 3> qkvGrads = flashAttn.computeBackward(states[0], states[1], states[2], attnGrad);
        states[0] = states[1] = states[2] = Tensor<DType>();
        attnGrad = Tensor<DType>();
        Tensor<DType> inputGrad = qkvProj.computeBackward(input, qkvGrads[0], qkvGrads[1], qkvGrads[2]);
        flashAttn.clearCache();
        return inputGrad;
    }

    // ---- shallow parameter access (AttentionLayer.cu:160-269) ----
    Tensor<DType> getQueryWeights() { return Tensor<DType>(qkvProj.weightsQuery, qkvWeightShape()); }
    Tensor<DType> getKeyWeights() { return Tensor<DType>(qkvProj.weightsKey, qkvWeightShape()); }
    Tensor<DType> getValueWeights() { return Tensor<DType>(qkvProj.weightsValue, qkvWeightShape()); }
    Tensor<DType> getQueryBiases() { return Tensor<DType>(qkvProj.biasesQuery, {qkvProj.biasSize()}); }
    Tensor<DType> getKeyBiases() { return Tensor<DType>(qkvProj.biasesKey, {qkvProj.biasSize()}); }
    Tensor<DType> getValueBiases() { return Tensor<DType>(qkvProj.biasesValue, {qkvProj.biasSize()}); }
    Tensor<DType> getOutputWeights() { return Tensor<DType>(outProj.weightsProj, outWeightShape()); }
    Tensor<DType> getOutputBiases() { return Tensor<DType>(outProj.biasesProj, {size_t(inputDim)}); }

    void setQueryWeights(Tensor<DType> t) { qkvProj.weightsQuery = adopt(t, qkvProj.projSize(), "query weights"); }
    void setKeyWeights(Tensor<DType> t) { qkvProj.weightsKey = adopt(t, qkvProj.projSize(), "key weights"); }
    void setValueWeights(Tensor<DType> t) { qkvProj.weightsValue = adopt(t, qkvProj.projSize(), "value weights"); }
    void setQueryBiases(Tensor<DType> t) { qkvProj.biasesQuery = adopt(t, qkvProj.biasSize(), "query biases"); }
    void setKeyBiases(Tensor<DType> t) { qkvProj.biasesKey = adopt(t, qkvProj.biasSize(), "key biases"); }
    void setValueBiases(Tensor<DType> t) { qkvProj.biasesValue = adopt(t, qkvProj.biasSize(), "value biases"); }
    void setOutputWeights(Tensor<DType> t) { outProj.weightsProj = adopt(t, outProj.weightSize(), "output weights"); }
    void setOutputBiases(Tensor<DType> t) { outProj.biasesProj = adopt(t, size_t(inputDim), "output biases"); }

    // Zeroes every gradient buffer that exists (AttentionLayer.cu:275-300).
    void zeroGrad() override {
        for (auto *g : {&qkvProj.weightsQueryGrad, &qkvProj.weightsKeyGrad, &qkvProj.weightsValueGrad})
            zeroBuffer(*g, qkvProj.projSize());
        for (auto *g : {&qkvProj.biasesQueryGrad, &qkvProj.biasesKeyGrad, &qkvProj.biasesValueGrad})
            zeroBuffer(*g, qkvProj.biasSize());
        zeroBuffer(outProj.weightsProjGrad, outProj.weightSize());
        zeroBuffer(outProj.biasesProjGrad, size_t(inputDim));
    }

    // p -= lr * grad on all eight buffers; gradient buffers are allocated (zero) if backward
    // never ran (AttentionLayer.cu:302-334).
    void sgdUpdate(double lr) override {
        ensureGrads();
        sgd(qkvProj.weightsQuery, qkvProj.weightsQueryGrad, lr, qkvProj.projSize());
        sgd(qkvProj.biasesQuery, qkvProj.biasesQueryGrad, lr, qkvProj.biasSize());
        sgd(qkvProj.weightsKey, qkvProj.weightsKeyGrad, lr, qkvProj.projSize());
        sgd(qkvProj.biasesKey, qkvProj.biasesKeyGrad, lr, qkvProj.biasSize());
        sgd(qkvProj.weightsValue, qkvProj.weightsValueGrad, lr, qkvProj.projSize());
        sgd(qkvProj.biasesValue, qkvProj.biasesValueGrad, lr, qkvProj.biasSize());
        sgd(outProj.weightsProj, outProj.weightsProjGrad, lr, outProj.weightSize());
        sgd(outProj.biasesProj, outProj.biasesProjGrad, lr, size_t(inputDim));
    }

    // Parameter map with the reference's keys (AttentionLayer.cu:340-356).
    std::map<std::string, Tensor<DType>> getParameters() override {
        return {{"query.weights", getQueryWeights()}, {"query.biases", getQueryBiases()},
                {"key.weights", getKeyWeights()},     {"key.biases", getKeyBiases()},
                {"value.weights", getValueWeights()}, {"value.biases", getValueBiases()},
                {"output.weights", getOutputWeights()}, {"output.biases", getOutputBiases()}};
    }

    void setParameters(const std::map<std::string, Tensor<DType>> &params) override {
        if (params.count("query.weights")) setQueryWeights(params.at("query.weights"));
        if (params.count("query.biases")) setQueryBiases(params.at("query.biases"));
        if (params.count("key.weights")) setKeyWeights(params.at("key.weights"));
        if (params.count("key.biases")) setKeyBiases(params.at("key.biases"));
        if (params.count("value.weights")) setValueWeights(params.at("value.weights"));
        if (params.count("value.biases")) setValueBiases(params.at("value.biases"));
        if (params.count("output.weights")) setOutputWeights(params.at("output.weights"));
        if (params.count("output.biases")) setOutputBiases(params.at("output.biases"));
    }

    // Gradient map (same keys), allocating zero buffers if backward never ran
    // (AttentionLayer.cu:373-405).
    std::map<std::string, Tensor<DType>> getGradients() override {
        ensureGrads();
        return {{"query.weights", Tensor<DType>(qkvProj.weightsQueryGrad, qkvWeightShape())},
                {"query.biases", Tensor<DType>(qkvProj.biasesQueryGrad, {qkvProj.biasSize()})},
                {"key.weights", Tensor<DType>(qkvProj.weightsKeyGrad, qkvWeightShape())},
                {"key.biases", Tensor<DType>(qkvProj.biasesKeyGrad, {qkvProj.biasSize()})},
                {"value.weights", Tensor<DType>(qkvProj.weightsValueGrad, qkvWeightShape())},
                {"value.biases", Tensor<DType>(qkvProj.biasesValueGrad, {qkvProj.biasSize()})},
                {"output.weights", Tensor<DType>(outProj.weightsProjGrad, outWeightShape())},
                {"output.biases", Tensor<DType>(outProj.biasesProjGrad, {size_t(inputDim)})}};
    }

private:
    std::vector<size_t> qkvWeightShape() const { return {size_t(headDim) * numHeads, size_t(inputDim)}; }
    std::vector<size_t> outWeightShape() const { return {size_t(inputDim), size_t(headDim) * numHeads}; }

    static std::shared_ptr<DType[]> adopt(const Tensor<DType> &t, size_t n, const char *what) {
        if (t.size() != n)
            throw std::invalid_argument(std::string(what) + ": expected " + std::to_string(n) + " elements, got " +
                                        std::to_string(t.size()));
        return t.dataPtr();
    }

    void ensureGrads() {
        qkvProj.ensureGrads();
        if (outProj.weightsProjGrad == nullptr) outProj.weightsProjGrad = detail::zeros<DType>(outProj.weightSize());
        if (outProj.biasesProjGrad == nullptr) outProj.biasesProjGrad = detail::zeros<DType>(size_t(inputDim));
    }

    static void zeroBuffer(const std::shared_ptr<DType[]> &g, size_t n) {
        if (g != nullptr)
            hipCheck(hipMemsetAsync(g.get(), 0, n * sizeof(DType), Runtime::stream()), "hipMemsetAsync");
    }

    static void sgd(const std::shared_ptr<DType[]> &p, const std::shared_ptr<DType[]> &g, double lr, size_t n) {
        ctattnCheck(ctattn_sgd_update(DTypeCode<DType>::value, p.get(), g.get(), lr, int64_t(n), Runtime::stream()),
                    "ctattn_sgd_update");
    }
};

}  // namespace ct
