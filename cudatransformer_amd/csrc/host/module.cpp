// pybind11 module `cuda_transformer`: the attention-path part of the reference's Python API
// (cuda_transformer.cu:22-119 declare_tensor, :147-157 the Module base, :257-324 the
// attention layer bindings, :437 and :825 the Attention factories), on the MI355X kernels
// behind include/ctattn.h.
//
// Names follow the reference: FloatTensor / BFloatTensor with fromNumpy, numpy, shape,
// clone, item, fill, reshape; FloatModule / BFloatModule (the Layer base: forward, backward,
// getParameters, setParameters, getGradients, zeroGrad, sgdUpdate, __call__);
// FloatAttentionLayer / BFloatAttentionLayer (forward, forward_caching, backward,
// backward_caching, sgdUpdate, the get/set{Query,Key,Value,Output}{Weights,Biases} pairs,
// __call__) and the factories AttentionFloat / AttentionBFloat / Attention(input_dim,
// num_heads, head_dim).  The reference does not bind FlashAttentionLayer itself (it is
// reached only through AttentionLayer); here it is bound as well, as
// FloatFlashAttentionLayer / BFloatFlashAttentionLayer with the C++ method names
// (computeAttention, computeBackward, clearCache, clone) and the factories FlashAttention /
// FlashAttentionFloat / FlashAttentionBFloat.  Attention factories take an extra
// causal=False.  bf16 tensors take and return float32 numpy arrays (numpy has no bfloat16;
// values are rounded to nearest even on upload).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "AttentionLayer.h"
#include "FlashAttentionLayer.h"
#include "ModuleLayer.h"
#include "Tensor.h"

namespace py = pybind11;
using namespace ct;

namespace {

template <typename DType>
Tensor<DType> tensorFromNumpy(const py::array_t<float, py::array::c_style | py::array::forcecast> &arr) {
    std::vector<size_t> shape(arr.shape(), arr.shape() + arr.ndim());
    if (shape.size() > 8) throw std::invalid_argument("Tensor dimension exceeds 8");
    return Tensor<DType>::fromFloats(shape, arr.data());
}

template <typename DType>
py::array_t<float> tensorToNumpy(const Tensor<DType> &t) {
    std::vector<float> host = t.toFloats();
    std::vector<py::ssize_t> shape(t.shape().begin(), t.shape().end());
    py::array_t<float> out(shape);
    if (!host.empty()) std::memcpy(out.mutable_data(), host.data(), host.size() * sizeof(float));
    return out;
}

template <typename DType>
void declareTensor(py::module_ &m, const std::string &suffix) {
    py::class_<Tensor<DType>>(m, (suffix + "Tensor").c_str(),
                              "N-dimensional GPU tensor. Assignments and copies are shallow (shared buffer); "
                              "call clone() to obtain an independent copy.")
        .def(py::init<>(), "Constructs an empty tensor with no allocated memory.")
        .def(py::init([](const std::vector<size_t> &shape) { return Tensor<DType>(shape); }), py::arg("shape"),
             "Constructs a zero-initialised tensor with the given shape on the GPU.")
        .def_static("fromNumpy", &tensorFromNumpy<DType>, py::arg("array"),
                    "Copies a NumPy array (cast to float32, C order) to a new GPU tensor.")
        .def("numpy", &tensorToNumpy<DType>, "Copies the tensor to the CPU and returns it as a float32 NumPy array.")
        .def("shape", [](const Tensor<DType> &t) { return t.shape(); }, "Returns the tensor shape as a list of ints.")
        .def("size", &Tensor<DType>::size, "Number of elements.")
        .def("clone", &Tensor<DType>::clone, "Returns a deep copy with its own GPU buffer.")
        .def("item", &Tensor<DType>::item, "Returns the value of a single-element tensor.")
        .def("fill", &Tensor<DType>::fill, py::arg("value"), "Fills every element in place.")
        .def("reshape", &Tensor<DType>::reshape, py::arg("shape"),
             "Returns a view with a new shape (same element count, shared buffer).")
        .def("__repr__", [suffix](const Tensor<DType> &t) {
            std::string s = suffix + "Tensor(shape=[";
            for (size_t i = 0; i < t.nDim(); ++i) s += (i ? ", " : "") + std::to_string(t.shape(i));
            return s + "])";
        });
}

template <typename DType>
void declareFlashAttention(py::module_ &m, const std::string &suffix) {
    using FA = FlashAttentionLayer<DType>;
    py::class_<FA, std::shared_ptr<FA>>(m, (suffix + "FlashAttentionLayer").c_str(),
                                        "Scaled-dot-product attention core on [batch, heads, seq, head_dim] "
                                        "tensors (MI355X kernels), with the forward state cached for backward.")
        .def(py::init<int, int, bool>(), py::arg("head_dim"), py::arg("num_heads"), py::arg("causal") = false)
        .def_readonly("headDim", &FA::headDim)
        .def_readonly("numHeads", &FA::numHeads)
        .def_readwrite("causal", &FA::causal, "Mask key j > query i (default False: the reference's behaviour).")
        .def("computeAttention", &FA::computeAttention, py::arg("queries"), py::arg("keys"), py::arg("values"),
             py::arg("save_states") = false,
             "Returns O = softmax(Q K^T / sqrt(d)) V; with save_states=True the forward state is cached.")
        .def("computeBackward",
             [](FA &self, const Tensor<DType> &q, const Tensor<DType> &k, const Tensor<DType> &v,
                const Tensor<DType> &dout) {
                 auto g = self.computeBackward(q, k, v, dout);
                 return py::make_tuple(g[0], g[1], g[2]);
             },
             py::arg("queries"), py::arg("keys"), py::arg("values"), py::arg("grad_output"),
             "Returns (dQ, dK, dV); reuses the cached forward state or recomputes it.")
        .def("clearCache", &FA::clearCache, "Drops the cached forward state.")
        .def("hasCache", [](const FA &self) { return !self.cachedLse.empty(); })
        .def("clone", &FA::clone, "A new layer with the same configuration and no cache.");
}

// The Layer base class (ModuleLayer.cu:15-91), bound as <suffix>Module.
template <typename DType>
void declareModule(py::module_ &m, const std::string &suffix) {
    using L = Layer<DType>;
    py::class_<L, std::shared_ptr<L>>(m, (suffix + "Module").c_str(),
                                      "Abstract layer: forward, backward, parameters, gradients, SGD.")
        .def("forward", &L::forward, py::arg("input"), "Runs the layer on `input`.")
        .def("backward", &L::backward, py::arg("input"), py::arg("grad_output"),
             "Backpropagates `grad_output`, accumulating parameter gradients; returns the input gradient.")
        .def("getParameters", &L::getParameters, "Parameter tensors by name (shared buffers).")
        .def("setParameters", &L::setParameters, py::arg("params"), "Adopts the given parameter tensors.")
        .def("getGradients", &L::getGradients, "Gradient tensors by name (shared buffers).")
        .def("zeroGrad", &L::zeroGrad, "Zeroes the accumulated gradients.")
        .def("sgdUpdate", &L::sgdUpdate, py::arg("lr"), "param -= lr * grad for every parameter.")
        .def("clone", &L::clone, "Deep copy of the layer's parameters.")
        .def("__call__", &L::operator(), py::arg("input"), "Shorthand for forward(input).");
}

// AttentionLayer (cuda_transformer.cu:257-324).
template <typename DType>
void declareAttention(py::module_ &m, const std::string &suffix) {
    using A = AttentionLayer<DType>;
    using T = Tensor<DType>;
    py::class_<A, Layer<DType>, std::shared_ptr<A>>(
        m, (suffix + "AttentionLayer").c_str(),
        "Multi-head attention: QKV projection -> flash attention -> output projection.\n"
        "All get/set methods are shallow (shared GPU buffer).  Q/K/V weight shape [headDim*numHeads, inputDim]\n"
        "(row j = output feature j); output weight shape [inputDim, headDim*numHeads].")
        .def(py::init<int, int, int, bool>(), py::arg("input_dim"), py::arg("num_heads"), py::arg("head_dim"),
             py::arg("causal") = false)
        .def_readonly("inputDim", &A::inputDim)
        .def_readonly("numHeads", &A::numHeads)
        .def_readonly("headDim", &A::headDim)
        .def_property_readonly("causal", &A::causal)
        .def("forward", static_cast<T (A::*)(T)>(&A::forward), py::arg("input"),
             "QKV projection -> attention -> output projection; returns [batch, seq, inputDim].")
        .def("forward_caching",
             [](A &layer, T input) {
                 std::array<T, 4> states;
                 T out = layer.forward(input, states.data());
                 py::list py_states;
                 for (auto &st : states) py_states.append(st);
                 return py::make_tuple(out, py_states);
             },
             py::arg("input"), "Returns (output, [Q, K, V, attention output]).")
        .def("backward", static_cast<T (A::*)(T, T)>(&A::backward), py::arg("input"), py::arg("grad_output"),
             "Recomputes the forward, backpropagates, accumulates every parameter gradient; returns dInput.")
        .def("backward_caching",
             [](A &layer, T input, T gradOutput, py::list py_states) {
                 if (py_states.size() != 4) throw std::runtime_error("States list must have exactly 4 Tensors");
                 std::array<T, 4> states;
                 for (size_t i = 0; i < 4; ++i) states[i] = py_states[i].cast<T>();
                 return layer.backward(input, gradOutput, states.data());
             },
             py::arg("input"), py::arg("grad_output"), py::arg("states"),
             "Backpropagates using the states [Q, K, V, attention output] from forward_caching.")
        .def("sgdUpdate", &A::sgdUpdate, py::arg("lr"), "SGD on all eight parameter buffers.")
        .def("zeroGrad", &A::zeroGrad, "Zeroes the accumulated gradients.")
        .def("getQueryWeights", &A::getQueryWeights)
        .def("setQueryWeights", &A::setQueryWeights, py::arg("tensor"))
        .def("getQueryBiases", &A::getQueryBiases)
        .def("setQueryBiases", &A::setQueryBiases, py::arg("tensor"))
        .def("getKeyWeights", &A::getKeyWeights)
        .def("setKeyWeights", &A::setKeyWeights, py::arg("tensor"))
        .def("getKeyBiases", &A::getKeyBiases)
        .def("setKeyBiases", &A::setKeyBiases, py::arg("tensor"))
        .def("getValueWeights", &A::getValueWeights)
        .def("setValueWeights", &A::setValueWeights, py::arg("tensor"))
        .def("getValueBiases", &A::getValueBiases)
        .def("setValueBiases", &A::setValueBiases, py::arg("tensor"))
        .def("getOutputWeights", &A::getOutputWeights)
        .def("setOutputWeights", &A::setOutputWeights, py::arg("tensor"))
        .def("getOutputBiases", &A::getOutputBiases)
        .def("setOutputBiases", &A::setOutputBiases, py::arg("tensor"))
        .def("__call__", &A::operator(), py::arg("input"), "Shorthand for forward(input).");
    m.def(("Attention" + suffix).c_str(),
          [](int inputDim, int numHeads, int headDim, bool causal) {
              return std::make_shared<A>(inputDim, numHeads, headDim, causal);
          },
          py::arg("input_dim"), py::arg("num_heads"), py::arg("head_dim"), py::arg("causal") = false,
          "Creates a multi-head AttentionLayer (QKV projection + flash attention + output projection).");
}

}  // namespace

PYBIND11_MODULE(cuda_transformer, m) {
    m.doc() =
        "cuda_transformer (MI355X): the flash-attention path of CudaTransformer on gfx950 HIP kernels.\n"
        "Tensors: FloatTensor, BFloatTensor.  Layers: FloatModule / BFloatModule (base),\n"
        "FloatAttentionLayer / BFloatAttentionLayer (AttentionFloat, AttentionBFloat, Attention),\n"
        "FloatFlashAttentionLayer / BFloatFlashAttentionLayer (FlashAttention(head_dim, num_heads,\n"
        "causal=False)).";

    declareTensor<float>(m, "Float");
    declareTensor<bf16>(m, "BFloat");
    declareFlashAttention<float>(m, "Float");
    declareFlashAttention<bf16>(m, "BFloat");
    declareModule<float>(m, "Float");
    declareModule<bf16>(m, "BFloat");
    declareAttention<float>(m, "Float");
    declareAttention<bf16>(m, "BFloat");
    m.def("Attention",
          [](int inputDim, int numHeads, int headDim, bool causal) {
              return std::make_shared<AttentionLayer<float>>(inputDim, numHeads, headDim, causal);
          },
          py::arg("input_dim"), py::arg("num_heads"), py::arg("head_dim"), py::arg("causal") = false,
          "Creates a float multi-head AttentionLayer.");

    auto makeFloat = [](int headDim, int numHeads, bool causal) {
        return std::make_shared<FlashAttentionLayer<float>>(headDim, numHeads, causal);
    };
    m.def("FlashAttention", makeFloat, py::arg("head_dim"), py::arg("num_heads"), py::arg("causal") = false,
          "Creates a float FlashAttentionLayer.");
    m.def("FlashAttentionFloat", makeFloat, py::arg("head_dim"), py::arg("num_heads"), py::arg("causal") = false,
          "Creates a float FlashAttentionLayer.");
    m.def("FlashAttentionBFloat",
          [](int headDim, int numHeads, bool causal) {
              return std::make_shared<FlashAttentionLayer<bf16>>(headDim, numHeads, causal);
          },
          py::arg("head_dim"), py::arg("num_heads"), py::arg("causal") = false,
          "Creates a bfloat16 FlashAttentionLayer (fp32 accumulation).");
    m.def("synchronize", &Runtime::synchronize, "Waits for all work queued by this module.");
    m.def("set_policy", &ctattn_set_policy, py::arg("policy"),
          "Kernel selection policy: 0 = MFMA (fastest), 1 = generic kernels, 2 = MFMA with a "
          "deterministic dQ reduction.  Returns the previous policy.");
    m.def("version", &ctattn_version, "Version of the attention kernel library.");
}
