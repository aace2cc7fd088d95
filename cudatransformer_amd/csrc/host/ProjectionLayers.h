// QKVProjectionLayer<DType> and OutputProjectionLayer<DType>: the two projections around the
// attention core, with the reference's state and method shapes (QKVProjectionLayer.cu:8-141,
// OutputProjectionLayer.cu:8-97), computing on the MFMA GEMMs of libctattn.so.
//
// Same semantics as the reference: weights start at zero (cudaMakeShared zero-fills,
// QKVProjectionLayer.cu:46-53), Q/K/V come out in [B, H, T, d], gradient buffers are
// allocated lazily on the first backward and accumulate across backward calls until
// zeroGrad (the reference atomically adds into them).  Differences: the bias gradients sum
// every row (the reference's kernels sum one row per 32-row tile), the weight gradients are
// deterministic, and nothing synchronises the device.
#pragma once

#include <array>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "Tensor.h"

namespace ct {

namespace detail {

// (batch, sequence length) of an activation [..., T, E] whose last dim is `inner`
// (QKVProjectionLayer.cu:74-75: T = shape[nDim-2], B = size / (T * inputDim)).
template <typename DType>
inline std::pair<size_t, size_t> batchSeq(const Tensor<DType> &t, size_t inner, const char *what) {
    if (t.nDim() < 2 || t.shape(t.nDim() - 1) != inner)
        throw std::invalid_argument(std::string(what) + ": last dimension must be " + std::to_string(inner));
    const size_t T = t.shape(t.nDim() - 2);
    const size_t B = T == 0 ? 0 : t.size() / (T * inner);
    return {B, T};
}

inline std::shared_ptr<uint8_t[]> workspace(int64_t bytes, const char *fn) {
    if (bytes < 0) ctattnCheck(int(hipErrorInvalidValue), fn);
    return deviceAlloc<uint8_t>(size_t(bytes > 0 ? bytes : 1));
}

template <typename DType>
inline std::shared_ptr<DType[]> zeros(size_t n) {
    return Tensor<DType>(std::vector<size_t>{n}).dataPtr();
}

}  // namespace detail

template <typename DType = float>
struct QKVProjectionLayer {
    std::shared_ptr<DType[]> weightsQuery, weightsQueryGrad, biasesQuery, biasesQueryGrad;
    std::shared_ptr<DType[]> weightsKey, weightsKeyGrad, biasesKey, biasesKeyGrad;
    std::shared_ptr<DType[]> weightsValue, weightsValueGrad, biasesValue, biasesValueGrad;
    int inputDim = 1;
    int numHeads = 1;
    int headDim = 1;

    QKVProjectionLayer(int inputDim, int numHeads, int headDim)
        : inputDim(inputDim), numHeads(numHeads), headDim(headDim) {
        if (inputDim < 1 || numHeads < 1 || headDim < 1)
            throw std::invalid_argument("inputDim, numHeads and headDim must be >= 1");
        weightsQuery = detail::zeros<DType>(projSize());
        weightsKey = detail::zeros<DType>(projSize());
        weightsValue = detail::zeros<DType>(projSize());
        biasesQuery = detail::zeros<DType>(biasSize());
        biasesKey = detail::zeros<DType>(biasSize());
        biasesValue = detail::zeros<DType>(biasSize());
    }

    size_t projSize() const { return size_t(inputDim) * headDim * numHeads; }
    size_t biasSize() const { return size_t(headDim) * numHeads; }

    // Deep copy of the weights (QKVProjectionLayer.cu:57-69).
    std::shared_ptr<QKVProjectionLayer<DType>> clone() const {
        auto c = std::make_shared<QKVProjectionLayer<DType>>(inputDim, numHeads, headDim);
        copyInto(c->weightsQuery, weightsQuery, projSize());
        copyInto(c->weightsKey, weightsKey, projSize());
        copyInto(c->weightsValue, weightsValue, projSize());
        copyInto(c->biasesQuery, biasesQuery, biasSize());
        copyInto(c->biasesKey, biasesKey, biasSize());
        copyInto(c->biasesValue, biasesValue, biasSize());
        return c;
    }

    // Q, K, V [B, H, T, d] of input [..., T, E] (QKVProjectionLayer.cu:73-94).
    std::array<Tensor<DType>, 3> computeQKV(const Tensor<DType> &input) {
        const auto [B, T] = detail::batchSeq(input, size_t(inputDim), "QKVProjectionLayer input");
        const std::vector<size_t> shape = {B, size_t(numHeads), T, size_t(headDim)};
        std::array<Tensor<DType>, 3> qkv = {Tensor<DType>::empty(shape), Tensor<DType>::empty(shape),
                                            Tensor<DType>::empty(shape)};
        ctattnCheck(ctattn_qkv_proj_fwd(DTypeCode<DType>::value, input.get(), weightsQuery.get(), weightsKey.get(),
                                        weightsValue.get(), biasesQuery.get(), biasesKey.get(), biasesValue.get(),
                                        qkv[0].get(), qkv[1].get(), qkv[2].get(), int64_t(B), int64_t(T), inputDim,
                                        numHeads, headDim, Runtime::stream()),
                    "ctattn_qkv_proj_fwd");
        return qkv;
    }

    // Accumulates the weight / bias gradients and returns dInput (QKVProjectionLayer.cu:100-141).
    Tensor<DType> computeBackward(const Tensor<DType> &input, const Tensor<DType> &queryGrad,
                                  const Tensor<DType> &keyGrad, const Tensor<DType> &valueGrad) {
        const auto [B, T] = detail::batchSeq(input, size_t(inputDim), "QKVProjectionLayer input");
        const std::vector<size_t> shape = {B, size_t(numHeads), T, size_t(headDim)};
        for (const Tensor<DType> *g : {&queryGrad, &keyGrad, &valueGrad})
            if (g->shape() != shape) throw std::invalid_argument("QKV gradients must be [B, H, T, d]");
        ensureGrads();
        Tensor<DType> inputGrad = Tensor<DType>::empty(input.shape());
        const int dt = DTypeCode<DType>::value;
        const int64_t wsBytes =
            ctattn_qkv_proj_bwd_workspace_bytes(dt, int64_t(B), int64_t(T), inputDim, numHeads, headDim);
        auto ws = detail::workspace(wsBytes, "ctattn_qkv_proj_bwd_workspace_bytes");
        ctattnCheck(ctattn_qkv_proj_bwd(dt, input.get(), queryGrad.get(), keyGrad.get(), valueGrad.get(),
                                        weightsQuery.get(), weightsKey.get(), weightsValue.get(),
                                        weightsQueryGrad.get(), weightsKeyGrad.get(), weightsValueGrad.get(),
                                        biasesQueryGrad.get(), biasesKeyGrad.get(), biasesValueGrad.get(),
                                        inputGrad.get(), ws.get(), wsBytes, int64_t(B), int64_t(T), inputDim,
                                        numHeads, headDim, Runtime::stream()),
                    "ctattn_qkv_proj_bwd");
        return inputGrad;
    }

    void ensureGrads() {
        if (weightsQueryGrad == nullptr) weightsQueryGrad = detail::zeros<DType>(projSize());
        if (weightsKeyGrad == nullptr) weightsKeyGrad = detail::zeros<DType>(projSize());
        if (weightsValueGrad == nullptr) weightsValueGrad = detail::zeros<DType>(projSize());
        if (biasesQueryGrad == nullptr) biasesQueryGrad = detail::zeros<DType>(biasSize());
        if (biasesKeyGrad == nullptr) biasesKeyGrad = detail::zeros<DType>(biasSize());
        if (biasesValueGrad == nullptr) biasesValueGrad = detail::zeros<DType>(biasSize());
    }

    static void copyInto(const std::shared_ptr<DType[]> &dst, const std::shared_ptr<DType[]> &src, size_t n) {
        hipCheck(hipMemcpyAsync(dst.get(), src.get(), n * sizeof(DType), hipMemcpyDeviceToDevice, Runtime::stream()),
                 "hipMemcpyAsync D2D");
    }
};

template <typename DType = float>
struct OutputProjectionLayer {
    std::shared_ptr<DType[]> weightsProj, weightsProjGrad, biasesProj, biasesProjGrad;
    int inputDim = 1;
    int headDim = 1;
    int numHeads = 1;

    OutputProjectionLayer(int inputDim, int headDim, int numHeads)
        : inputDim(inputDim), headDim(headDim), numHeads(numHeads) {
        if (inputDim < 1 || numHeads < 1 || headDim < 1)
            throw std::invalid_argument("inputDim, numHeads and headDim must be >= 1");
        weightsProj = detail::zeros<DType>(weightSize());
        biasesProj = detail::zeros<DType>(size_t(inputDim));
    }

    size_t weightSize() const { return size_t(inputDim) * headDim * numHeads; }

    std::shared_ptr<OutputProjectionLayer<DType>> clone() const {
        auto c = std::make_shared<OutputProjectionLayer<DType>>(inputDim, headDim, numHeads);
        QKVProjectionLayer<DType>::copyInto(c->weightsProj, weightsProj, weightSize());
        QKVProjectionLayer<DType>::copyInto(c->biasesProj, biasesProj, size_t(inputDim));
        return c;
    }

    // y [B, T, E] from the attention output [B, H, T, d] (OutputProjectionLayer.cu:52-66).
    Tensor<DType> forward(const Tensor<DType> &input) {
        const auto [B, T] = attnShape(input);
        Tensor<DType> output = Tensor<DType>::empty({B, T, size_t(inputDim)});
        ctattnCheck(ctattn_out_proj_fwd(DTypeCode<DType>::value, input.get(), weightsProj.get(), biasesProj.get(),
                                        output.get(), int64_t(B), int64_t(T), inputDim, numHeads, headDim,
                                        Runtime::stream()),
                    "ctattn_out_proj_fwd");
        return output;
    }

    // Accumulates dWo / dbo and returns d(attention output) (OutputProjectionLayer.cu:69-97).
    Tensor<DType> backward(const Tensor<DType> &input, const Tensor<DType> &gradOutput) {
        const auto [B, T] = attnShape(input);
        if (gradOutput.size() != B * T * size_t(inputDim))
            throw std::invalid_argument("gradOutput must be [B, T, inputDim]");
        if (weightsProjGrad == nullptr) weightsProjGrad = detail::zeros<DType>(weightSize());
        if (biasesProjGrad == nullptr) biasesProjGrad = detail::zeros<DType>(size_t(inputDim));
        Tensor<DType> inputGrad = Tensor<DType>::empty(input.shape());
        const int dt = DTypeCode<DType>::value;
        const int64_t wsBytes =
            ctattn_out_proj_bwd_workspace_bytes(dt, int64_t(B), int64_t(T), inputDim, numHeads, headDim);
        auto ws = detail::workspace(wsBytes, "ctattn_out_proj_bwd_workspace_bytes");
        ctattnCheck(ctattn_out_proj_bwd(dt, input.get(), gradOutput.get(), weightsProj.get(), weightsProjGrad.get(),
                                        biasesProjGrad.get(), inputGrad.get(), ws.get(), wsBytes, int64_t(B),
                                        int64_t(T), inputDim, numHeads, headDim, Runtime::stream()),
                    "ctattn_out_proj_bwd");
        return inputGrad;
    }

private:
    std::pair<size_t, size_t> attnShape(const Tensor<DType> &t) const {
        if (t.nDim() != 4 || int(t.shape(1)) != numHeads || int(t.shape(3)) != headDim)
            throw std::invalid_argument("attention output must be [batch, " + std::to_string(numHeads) +
                                        ", seq_len, " + std::to_string(headDim) + "]");
        return {t.shape(0), t.shape(2)};
    }
};

}  // namespace ct
