// Layer<DType>: the reference's layer interface (ModuleLayer.cu:15-91), unchanged in shape:
// virtual clone / forward / backward, operator(), parameter and gradient maps, zeroGrad,
// sgdUpdate, and Module<DType> = shared_ptr<Layer<DType>>; plus clear().
#pragma once

#include <map>
#include <memory>
#include <string>

#include "Tensor.h"

namespace ct {

template <typename DType = float>
struct Layer {
    Layer() = default;
    virtual ~Layer() = default;

    virtual std::shared_ptr<Layer<DType>> clone() = 0;
    virtual Tensor<DType> forward(Tensor<DType> input) = 0;
    virtual Tensor<DType> backward(Tensor<DType> input, Tensor<DType> gradOutput) = 0;

    Tensor<DType> operator()(Tensor<DType> input) { return this->forward(input); }

    virtual std::map<std::string, Tensor<DType>> getParameters() { return {}; }
    virtual void setParameters(const std::map<std::string, Tensor<DType>> &) {}
    virtual std::map<std::string, Tensor<DType>> getGradients() { return {}; }
    virtual void zeroGrad() {}
    virtual void sgdUpdate(double) {}
    // Drops the activations a layer keeps from its last forward for its backward (the
    // reference's TransformerLayer / MLPLayer::clear free their checkpoints).
    virtual void clear() {}
};

template <typename DType = float>
using Module = std::shared_ptr<Layer<DType>>;

}  // namespace ct
