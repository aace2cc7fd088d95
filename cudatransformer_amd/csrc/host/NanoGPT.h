// NanoGPT<DType>: the reference's language model (NanoGPT.cu:25-470) and the layers only it
// uses (Embedding.cu TokenEmbedding / PositionEmbedding / UnEmbedding, SoftmaxLoss.cu Softmax /
// CrossEntropyLoss), on libctattn.so.
//
// Same API and semantics as the reference: token + position embedding -> TransformerLayer ->
// un-embedding (no bias) -> softmax with temperature; forward returns the probabilities
// [..., T, vocab]; loss(probs, target) is the per-position cross-entropy -log p[target] / N
// (N = number of positions, so the losses sum to the mean); backward(input, probs, target)
// accumulates every parameter gradient from the activation checkpointed before the
// un-embedding; parameter keys "tokenEmbedding", "positionEmbedding", "unEmbedding" and the
// transformer's "layer_<i>.…"; weights start at zero; greedy / random / nucleus / top-k
// sampling on the host.  Differences, all deliberate:
//   * forward keeps its embedding and every layer's activations; a backward given that
//     forward's ids tensor reuses them instead of recomputing (same result, see
//     ModelLayers.h), any other ids are recomputed as the reference does;
//   * the softmax and cross-entropy backward are one kernel, dz = (p - onehot) / (N temp),
//     from the probabilities passed to backward (the reference chains the two backward passes
//     and re-derives p from a recomputed un-embedding, NanoGPT.cu:365-368; same result);
//   * the position embedding is indexed by position t (the reference's kernel uses b*T + t);
//   * an optional causal mask on every attention layer (default off, as in the reference);
//   * generate() feeds at most the last maxSeqLen tokens back (the reference overruns its
//     position table past maxSeqLen); top-k clamps K to the vocabulary.
// Every class is instantiated for float, bfloat16, half and double storage; losses are fp64
// for double and fp32 otherwise.
#pragma once

#include <algorithm>
#include <map>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "ModelLayers.h"

namespace ct {

// The reference's SamplingMode (NanoGPT.cu).
enum class SamplingMode { Greedy, Random, Nucleus, TopK };

namespace detail {

// (rows, T) of an id tensor [..., T].
inline std::pair<size_t, size_t> idRows(const Tensor<int32_t> &ids, const char *what) {
    if (ids.nDim() < 1) throw std::invalid_argument(std::string(what) + ": ids need at least one dimension");
    const size_t T = ids.shape(ids.nDim() - 1);
    return {T == 0 ? 0 : ids.size() / T, T};
}

inline std::vector<size_t> withLast(const std::vector<size_t> &shape, size_t last) {
    std::vector<size_t> s = shape;
    s.push_back(last);
    return s;
}

}  // namespace detail

// A [rows][embeddingDim] lookup table with its gradient (the state TokenEmbedding and
// PositionEmbedding share, Embedding.cu:13-170).
template <typename DType = float>
struct EmbeddingTable {
    int tableRows = 1;
    int embeddingDim = 1;
    std::shared_ptr<DType[]> embeddingMatrix, gradEmbeddingMatrix;

    EmbeddingTable(int rows, int dim) : tableRows(rows), embeddingDim(dim) {
        if (rows < 1 || dim < 1) throw std::invalid_argument("embedding sizes must be >= 1");
        embeddingMatrix = detail::zeros<DType>(elements());
        gradEmbeddingMatrix = detail::zeros<DType>(elements());
    }

    size_t elements() const { return size_t(tableRows) * embeddingDim; }
    std::vector<size_t> tableShape() const { return {size_t(tableRows), size_t(embeddingDim)}; }

    Tensor<DType> getParameters() { return Tensor<DType>(embeddingMatrix, tableShape()); }
    void setParameters(const Tensor<DType> &t) { detail::copyInto(embeddingMatrix, t, elements(), "embedding table"); }
    Tensor<DType> getGradients() { return Tensor<DType>(gradEmbeddingMatrix, tableShape()); }
    void zeroGrad() { detail::zeroBuffer(gradEmbeddingMatrix, elements()); }
    void sgdUpdate(double lr) { detail::sgdStep(embeddingMatrix, gradEmbeddingMatrix, lr, elements()); }

protected:
    void copyFrom(const EmbeddingTable &o) {
        embeddingMatrix = detail::cloneBuffer(o.embeddingMatrix, elements());
        gradEmbeddingMatrix = detail::cloneBuffer(o.gradEmbeddingMatrix, elements());
    }

    // out[..., T, E] from the token table, the position table, or both.
    Tensor<DType> lookup(const Tensor<int32_t> &ids, const DType *tok, const DType *pos, int vocab, int maxLen) const {
        auto [B, T] = detail::idRows(ids, "embedding");
        Tensor<DType> out = Tensor<DType>::empty(detail::withLast(ids.shape(), size_t(embeddingDim)));
        ctattnCheck(ctattn_embedding_fwd(DTypeCode<DType>::value, ids.get(), tok, pos, out.get(), int64_t(B),
                                         int64_t(T), embeddingDim, vocab, maxLen, Runtime::stream()),
                    "ctattn_embedding_fwd");
        return out;
    }
};

// Token embedding (Embedding.cu:13-170): out[b][t] = table[ids[b][t]]; ids outside the
// vocabulary give zero rows.
template <typename DType = float>
struct TokenEmbedding : public EmbeddingTable<DType> {
    int vocabSize = 1;

    TokenEmbedding(int vocabSize, int embeddingDim) : EmbeddingTable<DType>(vocabSize, embeddingDim), vocabSize(vocabSize) {}

    Tensor<DType> forward(const Tensor<int32_t> &ids) const {
        const size_t T = detail::idRows(ids, "TokenEmbedding").second;
        return this->lookup(ids, this->embeddingMatrix.get(), nullptr, vocabSize, int(std::max<size_t>(T, 1)));
    }
    Tensor<DType> operator()(const Tensor<int32_t> &ids) const { return forward(ids); }

    // table[ids[b][t]] += gradOutput[b][t] (Embedding.cu:82).
    void backward(const Tensor<int32_t> &ids, const Tensor<DType> &gradOutput) {
        auto [B, T] = detail::idRows(ids, "TokenEmbedding");
        if (gradOutput.size() != B * T * size_t(this->embeddingDim))
            throw std::invalid_argument("TokenEmbedding: grad_output shape does not match the ids");
        ctattnCheck(ctattn_embedding_bwd(DTypeCode<DType>::value, ids.get(), gradOutput.get(),
                                         this->gradEmbeddingMatrix.get(), nullptr, int64_t(B), int64_t(T),
                                         this->embeddingDim, vocabSize, Runtime::stream()),
                    "ctattn_embedding_bwd");
    }

    TokenEmbedding clone() const {
        TokenEmbedding c(vocabSize, this->embeddingDim);
        c.copyFrom(*this);
        return c;
    }
};

// Learned position embedding (Embedding.cu:172-318): out[b][t] = table[t], T <= blockSize.
template <typename DType = float>
struct PositionEmbedding : public EmbeddingTable<DType> {
    int blockSize = 1;

    PositionEmbedding(int blockSize, int embeddingDim) : EmbeddingTable<DType>(blockSize, embeddingDim), blockSize(blockSize) {}

    Tensor<DType> forward(const Tensor<int32_t> &ids) const {
        return this->lookup(ids, nullptr, this->embeddingMatrix.get(), 1, blockSize);
    }
    Tensor<DType> operator()(const Tensor<int32_t> &ids) const { return forward(ids); }

    // table[t] += sum_b gradOutput[b][t] (Embedding.cu:234).
    void backward(const Tensor<int32_t> &ids, const Tensor<DType> &gradOutput) {
        auto [B, T] = detail::idRows(ids, "PositionEmbedding");
        if (T > size_t(blockSize)) throw std::invalid_argument("PositionEmbedding: sequence longer than blockSize");
        if (gradOutput.size() != B * T * size_t(this->embeddingDim))
            throw std::invalid_argument("PositionEmbedding: grad_output shape does not match the ids");
        ctattnCheck(ctattn_embedding_bwd(DTypeCode<DType>::value, ids.get(), gradOutput.get(), nullptr,
                                         this->gradEmbeddingMatrix.get(), int64_t(B), int64_t(T), this->embeddingDim,
                                         1, Runtime::stream()),
                    "ctattn_embedding_bwd");
    }

    PositionEmbedding clone() const {
        PositionEmbedding c(blockSize, this->embeddingDim);
        c.copyFrom(*this);
        return c;
    }
};

// Un-embedding (Embedding.cu:320-470): a bias-free projection [..., E] -> [..., vocab] with
// weights [vocab][E].
template <typename DType = float>
struct UnEmbedding {
    int vocabSize = 1;
    int embeddingDim = 1;
    std::shared_ptr<LinearLayer<DType>> proj;

    UnEmbedding(int vocabSize, int embeddingDim)
        : vocabSize(vocabSize), embeddingDim(embeddingDim),
          proj(std::make_shared<LinearLayer<DType>>(embeddingDim, vocabSize, false)) {}

    Tensor<DType> forward(const Tensor<DType> &input) { return proj->forward(input); }
    Tensor<DType> operator()(const Tensor<DType> &input) { return forward(input); }
    Tensor<DType> backward(const Tensor<DType> &input, const Tensor<DType> &gradOutput) {
        return proj->backward(input, gradOutput);
    }
    Tensor<DType> getParameters() { return proj->getParameters().at("weights"); }
    void setParameters(const Tensor<DType> &t) { proj->setParameters({{"weights", t}}); }
    Tensor<DType> getGradients() { return proj->getGradients().at("weights"); }
    void zeroGrad() { proj->zeroGrad(); }
    void sgdUpdate(double lr) { proj->sgdUpdate(lr); }
    UnEmbedding clone() const {
        UnEmbedding c(vocabSize, embeddingDim);
        c.proj = std::static_pointer_cast<LinearLayer<DType>>(proj->clone());
        return c;
    }
};

// Softmax over the last dimension with temperature (SoftmaxLoss.cu:13-95).
template <typename DType = float>
struct Softmax {
    double temperature = 1.0;

    explicit Softmax(double temperature = 1.0) : temperature(temperature) {}

    Tensor<DType> forward(const Tensor<DType> &input) const {
        const size_t V = lastDim(input);
        Tensor<DType> out = Tensor<DType>::empty(input.shape());
        ctattnCheck(ctattn_softmax_fwd(DTypeCode<DType>::value, input.get(), out.get(), int64_t(input.size() / V),
                                       int64_t(V), temperature, Runtime::stream()),
                    "ctattn_softmax_fwd");
        return out;
    }
    Tensor<DType> operator()(const Tensor<DType> &input) const { return forward(input); }

    // Gradient with respect to the softmax input, from that input (SoftmaxLoss.cu:58-75).
    Tensor<DType> backward(const Tensor<DType> &input, const Tensor<DType> &gradOutput) const {
        if (gradOutput.size() != input.size()) throw std::invalid_argument("Softmax: grad_output shape");
        const size_t V = lastDim(input);
        Tensor<DType> p = forward(input);
        Tensor<DType> dz = Tensor<DType>::empty(input.shape());
        ctattnCheck(ctattn_softmax_bwd(DTypeCode<DType>::value, p.get(), gradOutput.get(), dz.get(),
                                       int64_t(input.size() / V), int64_t(V), temperature, Runtime::stream()),
                    "ctattn_softmax_bwd");
        return dz;
    }

private:
    static size_t lastDim(const Tensor<DType> &t) {
        if (t.nDim() < 1 || t.shape(t.nDim() - 1) == 0) throw std::invalid_argument("Softmax: empty last dimension");
        return t.shape(t.nDim() - 1);
    }
};

// Cross-entropy on probabilities (SoftmaxLoss.cu:150-215): loss has the shape of `target`
// (the positions), loss[r] = -log p[r][target[r]] / N.
template <typename DType = float>
struct CrossEntropyLoss {
    Tensor<StatOf<DType>> forward(const Tensor<DType> &input, const Tensor<int32_t> &target) const {
        const size_t V = checkShapes(input, target);
        auto loss = Tensor<StatOf<DType>>::empty(target.shape());
        ctattnCheck(ctattn_cross_entropy_fwd(DTypeCode<DType>::value, input.get(), target.get(), loss.get(),
                                             int64_t(target.size()), int64_t(V), Runtime::stream()),
                    "ctattn_cross_entropy_fwd");
        return loss;
    }
    Tensor<StatOf<DType>> operator()(const Tensor<DType> &input, const Tensor<int32_t> &target) const {
        return forward(input, target);
    }
    Tensor<DType> backward(const Tensor<DType> &input, const Tensor<int32_t> &target) const {
        const size_t V = checkShapes(input, target);
        Tensor<DType> grad = Tensor<DType>::empty(input.shape());
        ctattnCheck(ctattn_cross_entropy_bwd(DTypeCode<DType>::value, input.get(), target.get(), grad.get(),
                                             int64_t(target.size()), int64_t(V), Runtime::stream()),
                    "ctattn_cross_entropy_bwd");
        return grad;
    }

    static size_t checkShapes(const Tensor<DType> &input, const Tensor<int32_t> &target) {
        if (input.nDim() < 1 || input.shape(input.nDim() - 1) == 0)
            throw std::invalid_argument("CrossEntropyLoss: empty class dimension");
        const size_t V = input.shape(input.nDim() - 1);
        if (target.size() * V != input.size())
            throw std::invalid_argument("CrossEntropyLoss: target must hold one class id per row of the input");
        return V;
    }
};

// Mean squared error per row (SoftmaxLoss.cu:214-272): loss[..] = sum_j (x - y)^2 / D over
// the last dimension, shaped like the input without it (the reference allocates only
// shape[0] entries, SoftmaxLoss.cu:234, and writes every row); backward = 2 (x - y) / D.
template <typename DType = float>
struct MSELoss {
    Tensor<StatOf<DType>> forward(const Tensor<DType> &input, const Tensor<DType> &target) const {
        const size_t D = checkShapes(input, target);
        std::vector<size_t> shape(input.shape().begin(), input.shape().end() - 1);
        if (shape.empty()) shape.push_back(1);
        auto loss = Tensor<StatOf<DType>>::empty(shape);
        ctattnCheck(ctattn_mse_loss_fwd(DTypeCode<DType>::value, input.get(), target.get(), loss.get(),
                                        int64_t(input.size() / D), int64_t(D), Runtime::stream()),
                    "ctattn_mse_loss_fwd");
        return loss;
    }
    Tensor<StatOf<DType>> operator()(const Tensor<DType> &input, const Tensor<DType> &target) const {
        return forward(input, target);
    }
    Tensor<DType> backward(const Tensor<DType> &input, const Tensor<DType> &target) const {
        const size_t D = checkShapes(input, target);
        Tensor<DType> grad = Tensor<DType>::empty(input.shape());
        ctattnCheck(ctattn_mse_loss_bwd(DTypeCode<DType>::value, input.get(), target.get(), grad.get(),
                                        int64_t(input.size() / D), int64_t(D), Runtime::stream()),
                    "ctattn_mse_loss_bwd");
        return grad;
    }

    static size_t checkShapes(const Tensor<DType> &input, const Tensor<DType> &target) {
        if (input.nDim() < 1 || input.shape(input.nDim() - 1) == 0)
            throw std::invalid_argument("MSELoss: empty last dimension");
        if (input.shape() != target.shape()) throw std::invalid_argument("MSELoss: input and target shapes differ");
        return input.shape(input.nDim() - 1);
    }
};

template <typename DType = float>
struct NanoGPT {
    TokenEmbedding<DType> tokenEmbedding;
    PositionEmbedding<DType> positionEmbedding;
    TransformerLayer<DType> transformerLayer;
    UnEmbedding<DType> unEmbedding;
    Tensor<DType> preUnembeddingCheckpoint;  // the transformer output of the last forward
    Softmax<DType> softmax;
    CrossEntropyLoss<DType> crossEntropyLoss;

    NanoGPT(int vocabSize, int maxSeqLen, int embeddingDim, int numHeads, int headDim, int mlpDim, int numLayers,
            int checkpointGap = 0, double temperature = 1.0, ActivationType activationType = ActivationType::ReLU,
            bool causal = false)
        : tokenEmbedding(vocabSize, embeddingDim),
          positionEmbedding(maxSeqLen, embeddingDim),
          transformerLayer(embeddingDim, numHeads, headDim, mlpDim, numLayers, checkpointGap, activationType, causal),
          unEmbedding(vocabSize, embeddingDim),
          softmax(temperature) {}

    int vocabSize() const { return tokenEmbedding.vocabSize; }
    int maxSeqLen() const { return positionEmbedding.blockSize; }
    int embeddingDim() const { return transformerLayer.inputDim; }
    int numHeads() const { return transformerLayer.numHeads; }
    int headDim() const { return transformerLayer.headDim; }
    int mlpDim() const { return transformerLayer.mlpDim; }
    int numLayers() const { return transformerLayer.numLayers; }
    int checkpointGap() const { return transformerLayer.checkpointGap; }
    ActivationType activationType() const { return transformerLayer.activationType; }
    bool causal() const { return transformerLayer.causal(); }
    double getTemperature() const { return softmax.temperature; }
    void setTemperature(double t) {
        if (!(t > 0.0)) throw std::invalid_argument("temperature must be > 0");
        softmax.temperature = t;
    }

    // ids [..., T] (T <= maxSeqLen) -> probabilities [..., T, vocab] (NanoGPT.cu:83-94).
    Tensor<DType> forward(const Tensor<int32_t> &ids) {
        keptIds = ids;
        keptEmbedding = embed(ids);
        Tensor<DType> x = transformerLayer.forward(keptEmbedding);
        preUnembeddingCheckpoint = x;
        return softmax.forward(unEmbedding.forward(x)).reshape(detail::withLast(ids.shape(), size_t(vocabSize())));
    }
    Tensor<DType> operator()(const Tensor<int32_t> &ids) { return forward(ids); }
    Tensor<DType> forward(const std::vector<int32_t> &ids) {
        return forward(Tensor<int32_t>::fromPointer({ids.size()}, ids.data()));
    }

    // Per-position cross-entropy [..., T] (NanoGPT.cu:345-347).
    Tensor<StatOf<DType>> loss(const Tensor<DType> &probs, const Tensor<int32_t> &target) const {
        return crossEntropyLoss.forward(probs, target);
    }

    // Accumulates every parameter gradient of the mean cross-entropy (NanoGPT.cu:357-377).
    // `probs` are forward(input)'s output; the transformer output comes from the checkpoint
    // that forward left, or is recomputed when it does not match `input`.  When `input` is
    // the ids tensor of the last forward, the embedding and the transformer's activations
    // that forward kept are reused instead of recomputed.
    void backward(const Tensor<int32_t> &input, const Tensor<DType> &probs, const Tensor<int32_t> &target) {
        auto [B, T] = detail::idRows(input, "NanoGPT.backward");
        const size_t rows = B * T, V = size_t(vocabSize()), E = size_t(embeddingDim());
        if (probs.size() != rows * V) throw std::invalid_argument("NanoGPT.backward: probs must be [..., T, vocab]");
        if (target.size() != rows) throw std::invalid_argument("NanoGPT.backward: target must match the input");
        Tensor<DType> embedded = detail::sameTensor(keptIds, input) ? keptEmbedding : embed(input);
        keptIds = Tensor<int32_t>();
        keptEmbedding = Tensor<DType>();
        Tensor<DType> x = preUnembeddingCheckpoint;
        if (x.empty() || x.size() != rows * E) x = transformerLayer.forward(embedded);
        x = x.reshape({B, T, E});
        Tensor<DType> dz = Tensor<DType>::empty({B, T, V});
        ctattnCheck(ctattn_softmax_cross_entropy_bwd(DTypeCode<DType>::value, probs.get(), target.get(), dz.get(),
                                                     int64_t(rows), int64_t(V), softmax.temperature,
                                                     Runtime::stream()),
                    "ctattn_softmax_cross_entropy_bwd");
        Tensor<DType> g = unEmbedding.backward(x, dz);
        x = Tensor<DType>();
        dz = Tensor<DType>();
        g = transformerLayer.backward(embedded, g);
        ctattnCheck(ctattn_embedding_bwd(DTypeCode<DType>::value, input.get(), g.get(),
                                         tokenEmbedding.gradEmbeddingMatrix.get(),
                                         positionEmbedding.gradEmbeddingMatrix.get(), int64_t(B), int64_t(T),
                                         int64_t(E), vocabSize(), Runtime::stream()),
                    "ctattn_embedding_bwd");
    }

    // Drops the checkpointed and kept activations (NanoGPT.cu:466).
    void clear() {
        preUnembeddingCheckpoint = Tensor<DType>();
        keptIds = Tensor<int32_t>();
        keptEmbedding = Tensor<DType>();
        transformerLayer.clear();
    }

    // Zeroes every gradient buffer in one launch per 32 buffers (allocating those that do not
    // exist yet), instead of one fill per buffer.
    void zeroGrad() {
        std::vector<void *> ptrs;
        std::vector<int64_t> bytes;
        for (auto &[name, g] : getGradients()) {
            ptrs.push_back(g.get());
            bytes.push_back(int64_t(g.size() * sizeof(DType)));
        }
        ctattnCheck(ctattn_zero_multi(int(ptrs.size()), ptrs.data(), bytes.data(), Runtime::stream()),
                    "ctattn_zero_multi");
    }
    void sgdUpdate(double lr) {
        tokenEmbedding.sgdUpdate(lr);
        positionEmbedding.sgdUpdate(lr);
        transformerLayer.sgdUpdate(lr);
        unEmbedding.sgdUpdate(lr);
    }

    NanoGPT clone() {
        NanoGPT c = *this;
        c.tokenEmbedding = tokenEmbedding.clone();
        c.positionEmbedding = positionEmbedding.clone();
        c.transformerLayer = *std::static_pointer_cast<TransformerLayer<DType>>(transformerLayer.clone());
        c.unEmbedding = unEmbedding.clone();
        c.preUnembeddingCheckpoint = Tensor<DType>();
        c.keptIds = Tensor<int32_t>();
        c.keptEmbedding = Tensor<DType>();
        return c;
    }

    std::map<std::string, Tensor<DType>> getParameters() {
        auto m = transformerLayer.getParameters();
        m["tokenEmbedding"] = tokenEmbedding.getParameters();
        m["positionEmbedding"] = positionEmbedding.getParameters();
        m["unEmbedding"] = unEmbedding.getParameters();
        return m;
    }
    void setParameters(const std::map<std::string, Tensor<DType>> &p) {
        if (p.count("tokenEmbedding")) tokenEmbedding.setParameters(p.at("tokenEmbedding"));
        if (p.count("positionEmbedding")) positionEmbedding.setParameters(p.at("positionEmbedding"));
        if (p.count("unEmbedding")) unEmbedding.setParameters(p.at("unEmbedding"));
        transformerLayer.setParameters(p);
    }
    std::map<std::string, Tensor<DType>> getGradients() {
        auto m = transformerLayer.getGradients();
        m["tokenEmbedding"] = tokenEmbedding.getGradients();
        m["positionEmbedding"] = positionEmbedding.getGradients();
        m["unEmbedding"] = unEmbedding.getGradients();
        return m;
    }

    // Next token from probabilities [T, vocab] (their last row), NanoGPT.cu:154-200:
    // Greedy = argmax; Random = draw in proportion to p; Nucleus = draw among the tokens with
    // p > P (argmax if none); TopK = draw among the K most probable.
    int32_t predict(const Tensor<DType> &probs, SamplingMode mode, int K = 10, double P = 0.1) const {
        if (probs.nDim() != 2) throw std::invalid_argument("predict: probabilities must be [seqLen, vocab]");
        const size_t T = probs.shape(0), V = probs.shape(1);
        if (T == 0 || V == 0) throw std::invalid_argument("predict: empty probabilities");
        std::vector<float> all = probs.toFloats();
        std::vector<float> last(all.end() - std::ptrdiff_t(V), all.end());
        const int32_t argmax = int32_t(std::max_element(last.begin(), last.end()) - last.begin());
        if (mode == SamplingMode::Greedy) return argmax;
        std::vector<int32_t> ids;
        std::vector<double> w;
        if (mode == SamplingMode::Random) {
            for (size_t i = 0; i < V; ++i) ids.push_back(int32_t(i)), w.push_back(last[i]);
        } else if (mode == SamplingMode::Nucleus) {
            for (size_t i = 0; i < V; ++i)
                if (last[i] > P) ids.push_back(int32_t(i)), w.push_back(last[i]);
        } else {
            std::vector<int32_t> order(V);
            for (size_t i = 0; i < V; ++i) order[i] = int32_t(i);
            const size_t k = size_t(std::clamp(K, 1, int(V)));
            std::partial_sort(order.begin(), order.begin() + std::ptrdiff_t(k), order.end(),
                              [&](int32_t a, int32_t b) { return last[size_t(a)] > last[size_t(b)]; });
            for (size_t i = 0; i < k; ++i) ids.push_back(order[i]), w.push_back(last[size_t(order[i])]);
        }
        double total = 0.0;
        for (double x : w) total += x;
        if (ids.empty() || !(total > 0.0)) return argmax;
        std::mt19937 gen(std::random_device{}());
        std::discrete_distribution<size_t> dist(w.begin(), w.end());
        return ids[dist(gen)];
    }

    int32_t sample(const std::vector<int32_t> &input, SamplingMode mode, int K = 10, double P = 0.1) {
        return predict(forward(context(input)), mode, K, P);
    }

    // Appends numTokens sampled tokens to `input` (NanoGPT.cu:266-280).
    std::vector<int32_t> generate(std::vector<int32_t> input, int numTokens, SamplingMode mode, int K = 10,
                                  double P = 0.1) {
        if (input.empty()) throw std::invalid_argument("generate: empty prompt");
        for (int i = 0; i < numTokens; ++i) input.push_back(sample(input, mode, K, P));
        return input;
    }

private:
    Tensor<int32_t> keptIds;      // the ids of the last forward
    Tensor<DType> keptEmbedding;  // and their embedding

    Tensor<DType> embed(const Tensor<int32_t> &ids) {
        auto [B, T] = detail::idRows(ids, "NanoGPT");
        if (T > size_t(maxSeqLen()))
            throw std::invalid_argument("NanoGPT: sequence length " + std::to_string(T) + " exceeds maxSeqLen " +
                                        std::to_string(maxSeqLen()));
        const size_t E = size_t(embeddingDim());
        Tensor<DType> out = Tensor<DType>::empty({B, T, E});
        ctattnCheck(ctattn_embedding_fwd(DTypeCode<DType>::value, ids.get(), tokenEmbedding.embeddingMatrix.get(),
                                         positionEmbedding.embeddingMatrix.get(), out.get(), int64_t(B), int64_t(T),
                                         int64_t(E), vocabSize(), maxSeqLen(), Runtime::stream()),
                    "ctattn_embedding_fwd");
        return out;
    }

    std::vector<int32_t> context(const std::vector<int32_t> &ids) const {
        const size_t n = std::min(ids.size(), size_t(maxSeqLen()));
        return std::vector<int32_t>(ids.end() - std::ptrdiff_t(n), ids.end());
    }
};

}  // namespace ct
