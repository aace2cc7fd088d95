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
//
// Around attention, with the reference's names (cuda_transformer.cu:178-370, 372-410,
// 495-787), for every <T> in Float, BFloat, Half, Double: <T>LayerNormLayer, <T>LinearLayer,
// <T>ActivationLayer, <T>MLPLayer, <T>CheckpointLayer, <T>TransformerBlockLayer,
// <T>TransformerLayer and their factories (LayerNorm, Linear, Activation, ReLU, GELU, Sigmoid,
// Tanh, MLP, Checkpoint, TransformerBlock, Transformer; with the <T> suffix, float without
// one), <T>Softmax, <T>CrossEntropyLoss, <T>MSELoss, <T>TokenEmbedding, <T>PositionEmbedding,
// <T>UnEmbedding, <T>NanoGPT, <T>SGDOptimizer, <T>AdamOptimizer, <T>AdamWOptimizer;
// IntTensor for ids; enums ActivationType and SamplingMode.  Id arguments accept an
// IntTensor, a NumPy array or a list.  Half and Double tensors take float32 / float64 numpy
// arrays.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <type_traits>

#include "AttentionLayer.h"
#include "FlashAttentionLayer.h"
#include "ModelLayers.h"
#include "ModuleLayer.h"
#include "NanoGPT.h"
#include "Tensor.h"
#include "TensorOps.h"

namespace py = pybind11;
using namespace ct;

namespace {

// NumPy element type of a tensor: its own type, except float32 for the bf16 and f16 tensors
// (numpy has no bfloat16; both are rounded to nearest even on upload).
template <typename DType> using NpType = std::conditional_t<kHalfLike<DType>, float, DType>;
template <typename DType> constexpr bool kRawNumpy = !kHalfLike<DType>;
using IdArray = py::array_t<int32_t, py::array::c_style | py::array::forcecast>;

template <typename DType>
Tensor<DType> tensorFromNumpy(const py::array_t<NpType<DType>, py::array::c_style | py::array::forcecast> &arr) {
    std::vector<size_t> shape(arr.shape(), arr.shape() + arr.ndim());
    if (shape.size() > 8) throw std::invalid_argument("Tensor dimension exceeds 8");
    if constexpr (kRawNumpy<DType>)
        return Tensor<DType>::fromPointer(shape, arr.data());
    else
        return Tensor<DType>::fromFloats(shape, arr.data());
}

template <typename DType>
py::array_t<NpType<DType>> tensorToNumpy(const Tensor<DType> &t) {
    std::vector<py::ssize_t> shape(t.shape().begin(), t.shape().end());
    py::array_t<NpType<DType>> out(shape);
    if constexpr (kRawNumpy<DType>) {
        std::vector<HostElem<DType>> host = t.toHost();
        if (!host.empty()) std::memcpy(out.mutable_data(), host.data(), host.size() * sizeof(DType));
    } else {
        std::vector<float> host = t.toFloats();
        if (!host.empty()) std::memcpy(out.mutable_data(), host.data(), host.size() * sizeof(float));
    }
    return out;
}

// An id argument given as an IntTensor, a NumPy array or a list.
Tensor<int32_t> idsFrom(const py::object &o) {
    if (py::isinstance<Tensor<int32_t>>(o)) return o.cast<Tensor<int32_t>>();
    return tensorFromNumpy<int32_t>(o.cast<IdArray>());
}

std::vector<int32_t> idVector(const py::object &o) {
    if (py::isinstance<Tensor<int32_t>>(o)) return o.cast<Tensor<int32_t>>().toHost();
    IdArray a = o.cast<IdArray>();
    return std::vector<int32_t>(a.data(), a.data() + a.size());
}

// The reference's Tensor methods beyond storage (cuda_transformer.cu:40-119): conversions,
// arithmetic and comparison operators with tensors or Python numbers, reductions,
// transpose, kron, matmul.
template <typename DType>
void declareTensorOps(py::class_<Tensor<DType>> &c) {
    using T = Tensor<DType>;
    c.def("float", [](const T &t) { return ops::cast<float>(t); }, "Casts to 32-bit float.")
        .def("half", [](const T &t) { return ops::cast<f16>(t); }, "Casts to 16-bit float (FP16).")
        .def("bfloat", [](const T &t) { return ops::cast<bf16>(t); }, "Casts to bfloat16.")
        .def("double", [](const T &t) { return ops::cast<double>(t); }, "Casts to 64-bit float.")
        .def("int", [](const T &t) { return ops::cast<int32_t>(t); }, "Casts to 32-bit int.")
        .def("long", [](const T &t) { return ops::cast<int64_t>(t); }, "Casts to 64-bit int.")
        .def("short", [](const T &t) { return ops::cast<int16_t>(t); }, "Casts to 16-bit int.")
        .def("byte", [](const T &t) { return ops::cast<int8_t>(t); }, "Casts to 8-bit int (ByteTensor).")
        .def("bool", [](const T &t) { return ops::cast<bool>(t); }, "Casts to boolean (x != 0).");
    struct Arith {
        const char *name, *rname;
        int op;
    };
    for (const Arith a : {Arith{"__add__", "__radd__", CTATTN_OP_ADD}, Arith{"__sub__", "__rsub__", CTATTN_OP_SUB},
                          Arith{"__mul__", "__rmul__", CTATTN_OP_MUL}, Arith{"__truediv__", "__rtruediv__", CTATTN_OP_DIV},
                          Arith{"__mod__", "__rmod__", CTATTN_OP_MOD}}) {
        const int op = a.op;
        c.def(a.name, [op](const T &x, const T &y) { return ops::binary<DType>(x, y, op); }, py::is_operator());
        c.def(a.name, [op](const T &x, double s) { return ops::scalar<DType>(x, s, op); }, py::is_operator());
        c.def(a.rname, [op](const T &x, double s) { return ops::scalar<DType>(x, s, op, true); }, py::is_operator());
    }
    struct Cmp {
        const char *name;
        int op;
    };
    for (const Cmp a : {Cmp{"__eq__", CTATTN_OP_EQ}, Cmp{"__ne__", CTATTN_OP_NE}, Cmp{"__lt__", CTATTN_OP_LT},
                        Cmp{"__le__", CTATTN_OP_LE}, Cmp{"__gt__", CTATTN_OP_GT}, Cmp{"__ge__", CTATTN_OP_GE}}) {
        const int op = a.op;
        c.def(a.name, [op](const T &x, const T &y) { return ops::binary<bool>(x, y, op); }, py::is_operator());
        c.def(a.name, [op](const T &x, double s) { return ops::scalar<bool>(x, s, op); }, py::is_operator());
    }
    c.def("__neg__", [](const T &t) { return ops::unary(t, CTATTN_UN_NEG); }, py::is_operator())
        .def("__matmul__", [](const T &a, const T &b) { return ops::matmul(a, b); }, py::is_operator())
        .def("__rmatmul__", [](const T &a, const T &b) { return ops::matmul(b, a); }, py::is_operator())
        .def("matmul", [](const T &a, const T &b) { return ops::matmul(a, b); }, py::arg("other"),
             "Matrix product over the last two dimensions (batched over the leading ones).")
        .def("kron", [](const T &a, const T &b) { return ops::kron(a, b); }, py::arg("other"),
             "Kronecker product with a tensor of the same number of dimensions.")
        .def("transpose", [](const T &t, const std::vector<size_t> &perm) { return ops::permute(t, perm); },
             py::arg("perm"), "Returns a tensor with axes permuted according to perm.")
        .def("transpose", [](const T &t, size_t a1, size_t a2) { return ops::transpose(t, a1, a2); },
             py::arg("axis1"), py::arg("axis2"), "Returns a tensor with axis1 and axis2 swapped.")
        .def("reduce", [](const T &t, const std::vector<size_t> &axes, ReductionOp op) { return ops::reduce(t, axes, op); },
             py::arg("axes"), py::arg("op"), "Reduces the given axes with a ReductionOp.");
    struct Red {
        const char *name;
        ReductionOp op;
        const char *doc;
    };
    for (const Red r : {Red{"sum", ReductionOp::SUM, "Sums elements."}, Red{"mean", ReductionOp::MEAN, "Computes the mean."},
                        Red{"max", ReductionOp::MAX, "Computes the maximum."},
                        Red{"min", ReductionOp::MIN, "Computes the minimum."},
                        Red{"manhattan", ReductionOp::NORM_L1, "L1 (Manhattan) norm; alias of norm_l1."},
                        Red{"norm_l1", ReductionOp::NORM_L1, "L1 norm (sum of absolute values)."},
                        Red{"norm", ReductionOp::NORM_L2, "L2 (Euclidean) norm; alias of norm_l2."},
                        Red{"norm_l2", ReductionOp::NORM_L2, "L2 norm (square root of the sum of squares)."}}) {
        const ReductionOp op = r.op;
        c.def(r.name, [op](const T &t, int dim) { return ops::reduceDim(t, dim, op); }, py::arg("dim") = -1,
              (std::string(r.doc) + " dim=-1 reduces the whole tensor to a one-element tensor.").c_str());
    }
    c.def("cpu",
          [](const T &t) {
              py::list out;
              if constexpr (kHalfLike<DType>) {
                  for (float v : t.toFloats()) out.append(v);
              } else {
                  for (auto v : t.toHost()) out.append(py::cast(DType(v)));
              }
              return out;
          },
          "Copies the tensor to the CPU and returns its values as a flat list.");
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
                    "Copies a NumPy array (cast to the tensor's NumPy type, C order) to a new GPU tensor.")
        .def("numpy", &tensorToNumpy<DType>,
             "Copies the tensor to the CPU and returns it as a NumPy array (its own type; float32 for the "
             "BFloat and Half tensors).")
        .def("shape", [](const Tensor<DType> &t) { return t.shape(); }, "Returns the tensor shape as a list of ints.")
        .def("size", &Tensor<DType>::size, "Number of elements.")
        .def("clone", &Tensor<DType>::clone, "Returns a deep copy with its own GPU buffer.")
        .def("item",
             [](const Tensor<DType> &t) -> py::object {
                 if (t.size() != 1) throw std::invalid_argument("Tensor is not a scalar");
                 if constexpr (kHalfLike<DType>) return py::float_(t.item());
                 else return py::cast(DType(t.toHost()[0]));
             },
             "Returns the value of a single-element tensor.")
        .def("fill", &Tensor<DType>::fill, py::arg("value"), "Fills every element in place.")
        .def("reshape", &Tensor<DType>::reshape, py::arg("shape"),
             "Returns a view with a new shape (same element count, shared buffer).")
        .def("__repr__", [suffix](const Tensor<DType> &t) {
            std::string s = suffix + "Tensor(shape=[";
            for (size_t i = 0; i < t.nDim(); ++i) s += (i ? ", " : "") + std::to_string(t.shape(i));
            return s + "])";
        });
}

// Adds the operators after every tensor class exists, so that signatures name the Python
// classes they return (BoolTensor for comparisons, the cast targets).
template <typename DType>
void addTensorOps(py::module_ &m, const std::string &suffix) {
    auto cls = py::reinterpret_borrow<py::class_<Tensor<DType>>>(m.attr((suffix + "Tensor").c_str()));
    declareTensorOps<DType>(cls);
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
        .def("clear", &L::clear, "Drops the activations kept from the last forward for backward.")
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

// The layers around attention (cuda_transformer.cu:178-370 and the factories :411-444).
template <typename DType>
void declareLayers(py::module_ &m, const std::string &suffix) {
    using L = Layer<DType>;
    using LN = LayerNormLayer<DType>;
    using LIN = LinearLayer<DType>;
    using ACT = ActivationLayer<DType>;
    using MLP = MLPLayer<DType>;
    using TB = TransformerBlockLayer<DType>;
    using TR = TransformerLayer<DType>;

    py::class_<LN, L, std::shared_ptr<LN>>(m, (suffix + "LayerNormLayer").c_str(),
                                           "Layer normalisation over the last dimension with learnable scale "
                                           "(weights, initially 1) and shift (biases, initially 0).")
        .def(py::init<int, double>(), py::arg("input_dim"), py::arg("epsilon") = 1e-5)
        .def_readonly("inputDim", &LN::inputDim)
        .def_readonly("epsilon", &LN::epsilon);
    py::class_<CheckpointLayer<DType>, L, std::shared_ptr<CheckpointLayer<DType>>>(
        m, (suffix + "CheckpointLayer").c_str(),
        "Gradient-checkpoint marker: forward stores its input and returns it, backward passes the gradient.")
        .def(py::init<>())
        .def("clear", &CheckpointLayer<DType>::clear, "Drops the stored activation.");
    py::class_<ACT, L, std::shared_ptr<ACT>>(m, (suffix + "ActivationLayer").c_str(),
                                             "Elementwise ReLU / GELU (tanh form) / Sigmoid / Tanh.")
        .def(py::init<int, ActivationType>(), py::arg("input_dim"), py::arg("activation_type"))
        .def_readonly("activationType", &ACT::activationType);
    py::class_<LIN, L, std::shared_ptr<LIN>>(m, (suffix + "LinearLayer").c_str(),
                                             "Fully connected layer y = x W^T + b, W [output_dim, input_dim]; "
                                             "get/set methods are shallow (shared GPU buffer).")
        .def(py::init<int, int, bool>(), py::arg("input_dim"), py::arg("output_dim"), py::arg("use_bias") = true)
        .def_readonly("inputDim", &LIN::inputDim)
        .def_readonly("outputDim", &LIN::outputDim)
        .def("getWeights", &LIN::getWeights)
        .def("setWeights", &LIN::setWeights, py::arg("tensor"))
        .def("getBiases", &LIN::getBiases)
        .def("setBiases", &LIN::setBiases, py::arg("tensor"))
        .def("getWeightGrad", &LIN::getWeightGrad)
        .def("setWeightGrad", &LIN::setWeightGrad, py::arg("tensor"))
        .def("getBiasGrad", &LIN::getBiasGrad)
        .def("setBiasGrad", &LIN::setBiasGrad, py::arg("tensor"));
    py::class_<MLP, L, std::shared_ptr<MLP>>(m, (suffix + "MLPLayer").c_str(),
                                             "Sequential container; parameters keyed 'layer_<i>.<name>'.")
        .def(py::init<std::vector<Module<DType>>>(), py::arg("layers"))
        .def_readonly("layers", &MLP::layers);
    py::class_<TB, L, std::shared_ptr<TB>>(m, (suffix + "TransformerBlockLayer").c_str(),
                                           "LayerNorm -> Attention -> LayerNorm -> MLP (Linear, Activation, "
                                           "Linear), without residual connections.")
        .def(py::init<int, int, int, int, ActivationType, bool>(), py::arg("input_dim"), py::arg("num_heads"),
             py::arg("head_dim"), py::arg("mlp_dim"), py::arg("activation_type") = ActivationType::ReLU,
             py::arg("causal") = false)
        .def_readonly("firstNorm", &TB::firstNorm)
        .def_readonly("attention", &TB::attention)
        .def_readonly("secondNorm", &TB::secondNorm)
        .def_readonly("mlp", &TB::mlp);
    py::class_<TR, L, std::shared_ptr<TR>>(m, (suffix + "TransformerLayer").c_str(),
                                           "A stack of transformer blocks; parameters keyed 'layer_<i>.<name>'.")
        .def(py::init<int, int, int, int, int, int, ActivationType, bool>(), py::arg("input_dim"),
             py::arg("num_heads"), py::arg("head_dim"), py::arg("mlp_dim"), py::arg("num_layers"),
             py::arg("checkpoint_gap") = 0, py::arg("activation_type") = ActivationType::ReLU,
             py::arg("causal") = false)
        .def_readonly("blocks", &TR::blocks)
        .def_readonly("numLayers", &TR::numLayers)
        .def_readonly("checkpointGap", &TR::checkpointGap);

}

// Factories LayerNorm<suffix>, Linear<suffix>, … (cuda_transformer.cu:411-444; the
// un-suffixed float names, :811-836, come from suffix "").
template <typename DType>
void declareFactories(py::module_ &m, const std::string &suffix) {
    using LN = LayerNormLayer<DType>;
    using LIN = LinearLayer<DType>;
    using ACT = ActivationLayer<DType>;
    using MLP = MLPLayer<DType>;
    using TB = TransformerBlockLayer<DType>;
    using TR = TransformerLayer<DType>;
    auto def = [&](const std::string &name, auto fn, auto... args) { m.def((name + suffix).c_str(), fn, args...); };
    def("LayerNorm", [](int d, double eps) { return std::make_shared<LN>(d, eps); }, py::arg("input_dim"),
        py::arg("epsilon") = 1e-5);
    def("Checkpoint", [] { return std::make_shared<CheckpointLayer<DType>>(); });
    def("Linear", [](int i, int o, bool b) { return std::make_shared<LIN>(i, o, b); }, py::arg("input_dim"),
        py::arg("output_dim"), py::arg("use_bias") = true);
    def("Activation", [](int d, ActivationType t) { return std::make_shared<ACT>(d, t); }, py::arg("input_dim"),
        py::arg("activation_type"));
    def("ReLU", [](int d) { return std::make_shared<ACT>(d, ActivationType::ReLU); }, py::arg("input_dim"));
    def("GELU", [](int d) { return std::make_shared<ACT>(d, ActivationType::GELU); }, py::arg("input_dim"));
    def("Sigmoid", [](int d) { return std::make_shared<ACT>(d, ActivationType::Sigmoid); }, py::arg("input_dim"));
    def("Tanh", [](int d) { return std::make_shared<ACT>(d, ActivationType::Tanh); }, py::arg("input_dim"));
    def("MLP", [](std::vector<Module<DType>> layers) { return std::make_shared<MLP>(layers); }, py::arg("layers"));
    def("TransformerBlock",
        [](int e, int h, int d, int mlp, ActivationType a, bool c) { return std::make_shared<TB>(e, h, d, mlp, a, c); },
        py::arg("input_dim"), py::arg("num_heads"), py::arg("head_dim"), py::arg("mlp_dim"),
        py::arg("activation_type") = ActivationType::ReLU, py::arg("causal") = false);
    def("Transformer",
        [](int e, int h, int d, int mlp, int n, int gap, ActivationType a, bool c) {
            return std::make_shared<TR>(e, h, d, mlp, n, gap, a, c);
        },
        py::arg("input_dim"), py::arg("num_heads"), py::arg("head_dim"), py::arg("mlp_dim"), py::arg("num_layers"),
        py::arg("checkpoint_gap") = 0, py::arg("activation_type") = ActivationType::ReLU, py::arg("causal") = false);
}

// Softmax and cross-entropy (cuda_transformer.cu:579-633).
template <typename DType>
void declareLosses(py::module_ &m, const std::string &suffix) {
    using T = Tensor<DType>;
    py::class_<Softmax<DType>>(m, (suffix + "Softmax").c_str(), "Softmax over the last dimension with temperature.")
        .def(py::init<double>(), py::arg("temperature") = 1.0)
        .def_readwrite("temperature", &Softmax<DType>::temperature)
        .def("forward", &Softmax<DType>::forward, py::arg("input"))
        .def("__call__", &Softmax<DType>::forward, py::arg("input"))
        .def("backward", &Softmax<DType>::backward, py::arg("input"), py::arg("grad_output"),
             "Gradient with respect to the softmax input, given that input.");
    py::class_<CrossEntropyLoss<DType>>(m, (suffix + "CrossEntropyLoss").c_str(),
                                        "-log p[target] / N per row, on probabilities (loss tensor in fp32, "
                                        "fp64 for Double).")
        .def(py::init<>())
        .def("forward", [](const CrossEntropyLoss<DType> &l, const T &p, py::object t) { return l.forward(p, idsFrom(t)); },
             py::arg("input"), py::arg("target"))
        .def("__call__", [](const CrossEntropyLoss<DType> &l, const T &p, py::object t) { return l.forward(p, idsFrom(t)); },
             py::arg("input"), py::arg("target"))
        .def("backward", [](const CrossEntropyLoss<DType> &l, const T &p, py::object t) { return l.backward(p, idsFrom(t)); },
             py::arg("input"), py::arg("target"));
    py::class_<MSELoss<DType>>(m, (suffix + "MSELoss").c_str(),
                               "Mean squared error per row, sum_j (x - y)^2 / D over the last dimension (loss tensor "
                               "in fp32, fp64 for Double).")
        .def(py::init<>())
        .def("forward", &MSELoss<DType>::forward, py::arg("input"), py::arg("target"))
        .def("__call__", &MSELoss<DType>::forward, py::arg("input"), py::arg("target"))
        .def("backward", &MSELoss<DType>::backward, py::arg("input"), py::arg("target"),
             "Gradient 2 (x - y) / D with respect to the input.");
}

// Embeddings, NanoGPT and the optimizers (cuda_transformer.cu:372-410, 495-578, 634-787).
template <typename DType>
void declareNanoGPT(py::module_ &m, const std::string &suffix) {
    using T = Tensor<DType>;
    using G = NanoGPT<DType>;
    using TE = TokenEmbedding<DType>;
    using PE = PositionEmbedding<DType>;
    using UE = UnEmbedding<DType>;
    using ADAM = AdamOptimizer<DType>;
    using ADAMW = AdamWOptimizer<DType>;
    using SGD = SGDOptimizer<DType>;
    const auto name = [&](const char *n) { return suffix + n; };
    py::class_<TE>(m, name("TokenEmbedding").c_str(), "Token id -> embedding row lookup.")
        .def(py::init<int, int>(), py::arg("vocab_size"), py::arg("embedding_dim"))
        .def("forward", [](const TE &e, py::object ids) { return e.forward(idsFrom(ids)); },
             py::arg("input"))
        .def("__call__", [](const TE &e, py::object ids) { return e.forward(idsFrom(ids)); },
             py::arg("input"))
        .def("backward", [](TE &e, py::object ids, const T &g) { e.backward(idsFrom(ids), g); },
             py::arg("input"), py::arg("grad_output"))
        .def("getParameters", &TE::getParameters)
        .def("setParameters", &TE::setParameters, py::arg("tensor"))
        .def("getGradients", &TE::getGradients)
        .def("zeroGrad", &TE::zeroGrad)
        .def("sgdUpdate", &TE::sgdUpdate, py::arg("lr"))
        .def("clone", &TE::clone);
    py::class_<PE>(m, name("PositionEmbedding").c_str(), "Learned position embedding [max_seq_len, E].")
        .def(py::init<int, int>(), py::arg("max_seq_len"), py::arg("embedding_dim"))
        .def("forward", [](const PE &e, py::object ids) { return e.forward(idsFrom(ids)); },
             py::arg("input"))
        .def("__call__", [](const PE &e, py::object ids) { return e.forward(idsFrom(ids)); },
             py::arg("input"))
        .def("backward", [](PE &e, py::object ids, const T &g) { e.backward(idsFrom(ids), g); },
             py::arg("input"), py::arg("grad_output"))
        .def("getParameters", &PE::getParameters)
        .def("setParameters", &PE::setParameters, py::arg("tensor"))
        .def("getGradients", &PE::getGradients)
        .def("zeroGrad", &PE::zeroGrad)
        .def("sgdUpdate", &PE::sgdUpdate, py::arg("lr"))
        .def("clone", &PE::clone);
    py::class_<UE>(m, name("UnEmbedding").c_str(), "Bias-free projection [..., E] -> [..., vocab].")
        .def(py::init<int, int>(), py::arg("vocab_size"), py::arg("embedding_dim"))
        .def("forward", &UE::forward, py::arg("input"))
        .def("__call__", &UE::forward, py::arg("input"))
        .def("backward", &UE::backward, py::arg("input"), py::arg("grad_output"))
        .def("getParameters", &UE::getParameters)
        .def("setParameters", &UE::setParameters, py::arg("tensor"))
        .def("getGradients", &UE::getGradients)
        .def("zeroGrad", &UE::zeroGrad)
        .def("sgdUpdate", &UE::sgdUpdate, py::arg("lr"))
        .def("clone", &UE::clone);

    auto generate = [](G &g, py::object input, int n, SamplingMode mode, int K, double P) -> py::object {
        std::vector<int32_t> out = g.generate(idVector(input), n, mode, K, P);
        if (py::isinstance<Tensor<int32_t>>(input)) return py::cast(Tensor<int32_t>::fromPointer({out.size()}, out.data()));
        if (py::isinstance<py::list>(input)) return py::cast(out);
        IdArray a(py::ssize_t(out.size()));
        std::copy(out.begin(), out.end(), a.mutable_data());
        return std::move(a);
    };
    py::class_<G>(m, name("NanoGPT").c_str(),
                  "GPT language model: token + position embedding -> Transformer -> un-embedding -> softmax.\n"
                  "forward returns probabilities [..., T, vocab]; backward(input, probs, target) accumulates the\n"
                  "gradients of the mean cross-entropy.  Weights start at zero (set them with setParameters).")
        .def(py::init<int, int, int, int, int, int, int, int, double, ActivationType, bool>(), py::arg("vocab_size"),
             py::arg("max_seq_len"), py::arg("embedding_dim"), py::arg("num_heads"), py::arg("head_dim"),
             py::arg("mlp_dim"), py::arg("num_layers"), py::arg("checkpoint_gap") = 0, py::arg("temperature") = 1.0,
             py::arg("activation_type") = ActivationType::ReLU, py::arg("causal") = false)
        .def("vocabSize", &G::vocabSize)
        .def("maxSeqLen", &G::maxSeqLen)
        .def("embeddingDim", &G::embeddingDim)
        .def("numHeads", &G::numHeads)
        .def("headDim", &G::headDim)
        .def("mlpDim", &G::mlpDim)
        .def("numLayers", &G::numLayers)
        .def("checkpointGap", &G::checkpointGap)
        .def("activationType", &G::activationType)
        .def("causal", &G::causal)
        .def("getTemperature", &G::getTemperature)
        .def("setTemperature", &G::setTemperature, py::arg("temperature"))
        .def("forward", [](G &g, py::object ids) { return g.forward(idsFrom(ids)); }, py::arg("input"),
             "Token ids [..., T] (IntTensor, NumPy array or list) -> probabilities [..., T, vocab].")
        .def("__call__", [](G &g, py::object ids) { return g.forward(idsFrom(ids)); }, py::arg("input"))
        .def("loss", [](const G &g, const T &probs, py::object target) { return g.loss(probs, idsFrom(target)); },
             py::arg("logits"), py::arg("target"), "Per-position cross-entropy -log p[target] / N (sums to the mean).")
        .def("backward",
             [](G &g, py::object input, const T &probs, py::object target) {
                 g.backward(idsFrom(input), probs, idsFrom(target));
             },
             py::arg("input"), py::arg("logits"), py::arg("target"),
             "Accumulates all parameter gradients; call with forward's input and output.")
        .def("predict", &G::predict, py::arg("logits"), py::arg("mode"), py::arg("K") = 10, py::arg("P") = 0.1,
             "Next token from probabilities [seqLen, vocab] (last row).")
        .def("sample",
             [](G &g, py::object input, SamplingMode mode, int K, double P) {
                 return g.sample(idVector(input), mode, K, P);
             },
             py::arg("input"), py::arg("mode"), py::arg("K") = 10, py::arg("P") = 0.1)
        .def("generate", generate, py::arg("input"), py::arg("num_tokens"), py::arg("mode"), py::arg("K") = 10,
             py::arg("P") = 0.1, "Appends num_tokens sampled tokens; returns the input's type.")
        .def("zeroGrad", &G::zeroGrad)
        .def("sgdUpdate", &G::sgdUpdate, py::arg("lr"))
        .def("clone", &G::clone)
        .def("clear", &G::clear, "Drops the checkpointed activation and the activations kept for backward.")
        .def("getParameters", &G::getParameters)
        .def("setParameters", &G::setParameters, py::arg("params"))
        .def("getGradients", &G::getGradients)
        .def_readonly("transformerLayer", &G::transformerLayer);

    py::class_<SGD>(m, name("SGDOptimizer").c_str(), "SGD over a parameter map: params[k] -= lr * grads[k].")
        .def(py::init<std::map<std::string, T>, double>(), py::arg("params"), py::arg("lr"))
        .def("step", &SGD::step, py::arg("grads"), "One update of every parameter from `grads`.")
        .def("getLearningRate", &SGD::getLearningRate)
        .def("setLearningRate", &SGD::setLearningRate, py::arg("lr"));
    py::class_<ADAM>(m, name("AdamOptimizer").c_str(), "Adam over a parameter map (decay folded into the gradient).")
        .def(py::init<std::map<std::string, T>, double, double, double, double, double, bool>(), py::arg("params"),
             py::arg("lr") = 0.001, py::arg("b1") = 0.9, py::arg("b2") = 0.999, py::arg("eps") = 1e-8,
             py::arg("decay") = 0.0, py::arg("decoupled") = false)
        .def("step", &ADAM::step, py::arg("grads"), "One update of every parameter from `grads`.")
        .def("getLearningRate", &ADAM::getLearningRate)
        .def("setLearningRate", &ADAM::setLearningRate, py::arg("lr"))
        .def("getTimeStep", &ADAM::getTimeStep)
        .def("setTimeStep", &ADAM::setTimeStep, py::arg("t"));
    py::class_<ADAMW, ADAM>(m, name("AdamWOptimizer").c_str(), "AdamW over a parameter map (decoupled decay).")
        .def(py::init<std::map<std::string, T>, double, double, double, double, double>(), py::arg("params"),
             py::arg("lr") = 0.001, py::arg("b1") = 0.9, py::arg("b2") = 0.999, py::arg("eps") = 1e-8,
             py::arg("decay") = 0.0);
}

}  // namespace

PYBIND11_MODULE(cuda_transformer, m) {
    m.doc() =
        "cuda_transformer (MI355X): CudaTransformer's Python API on gfx950 HIP kernels.\n"
        "<T> is Float, BFloat, Half or Double.  Tensors: <T>Tensor, IntTensor (token ids).\n"
        "Layers: <T>Module (base), <T>AttentionLayer (Attention<T>, Attention), <T>FlashAttentionLayer\n"
        "(FlashAttention<T>, FlashAttention(head_dim, num_heads, causal=False)), <T>LayerNormLayer,\n"
        "<T>LinearLayer, <T>ActivationLayer, <T>MLPLayer, <T>CheckpointLayer, <T>TransformerBlockLayer,\n"
        "<T>TransformerLayer (factories LayerNorm, Linear, Activation, ReLU, GELU, Sigmoid, Tanh, MLP,\n"
        "Checkpoint, TransformerBlock, Transformer, with a <T> suffix, float without one).\n"
        "Losses: <T>Softmax, <T>CrossEntropyLoss, <T>MSELoss.  Model: <T>TokenEmbedding,\n"
        "<T>PositionEmbedding, <T>UnEmbedding, <T>NanoGPT.  Optimizers: <T>SGDOptimizer,\n"
        "<T>AdamOptimizer, <T>AdamWOptimizer.  Enums ActivationType, SamplingMode.";

    py::enum_<ActivationType>(m, "ActivationType", "Activation of the MLP sub-layers.")
        .value("ReLU", ActivationType::ReLU)
        .value("GELU", ActivationType::GELU, "tanh approximation")
        .value("Sigmoid", ActivationType::Sigmoid)
        .value("Tanh", ActivationType::Tanh);
    py::enum_<ReductionOp>(m, "ReductionOp", "Reduction of Tensor.reduce.")
        .value("SUM", ReductionOp::SUM)
        .value("MEAN", ReductionOp::MEAN)
        .value("MAX", ReductionOp::MAX)
        .value("MIN", ReductionOp::MIN)
        .value("NORM_L1", ReductionOp::NORM_L1)
        .value("NORM_L2", ReductionOp::NORM_L2);
    py::enum_<SamplingMode>(m, "SamplingMode", "Next-token choice of NanoGPT.predict / sample / generate.")
        .value("Greedy", SamplingMode::Greedy)
        .value("Random", SamplingMode::Random)
        .value("Nucleus", SamplingMode::Nucleus)
        .value("TopK", SamplingMode::TopK);

    declareTensor<float>(m, "Float");
    declareTensor<bf16>(m, "BFloat");
    declareTensor<f16>(m, "Half");
    declareTensor<double>(m, "Double");
    declareTensor<int32_t>(m, "Int");
    declareTensor<int64_t>(m, "Long");
    declareTensor<int16_t>(m, "Short");
    declareTensor<int8_t>(m, "Byte");
    declareTensor<bool>(m, "Bool");
    addTensorOps<float>(m, "Float");
    addTensorOps<bf16>(m, "BFloat");
    addTensorOps<f16>(m, "Half");
    addTensorOps<double>(m, "Double");
    addTensorOps<int32_t>(m, "Int");
    addTensorOps<int64_t>(m, "Long");
    addTensorOps<int16_t>(m, "Short");
    addTensorOps<int8_t>(m, "Byte");
    addTensorOps<bool>(m, "Bool");
    declareFlashAttention<float>(m, "Float");
    declareFlashAttention<bf16>(m, "BFloat");
    declareFlashAttention<f16>(m, "Half");
    declareFlashAttention<double>(m, "Double");
    declareModule<float>(m, "Float");
    declareModule<bf16>(m, "BFloat");
    declareModule<f16>(m, "Half");
    declareModule<double>(m, "Double");
    declareAttention<float>(m, "Float");
    declareAttention<bf16>(m, "BFloat");
    declareAttention<f16>(m, "Half");
    declareAttention<double>(m, "Double");
    declareLayers<float>(m, "Float");
    declareLayers<bf16>(m, "BFloat");
    declareLayers<f16>(m, "Half");
    declareLayers<double>(m, "Double");
    declareFactories<float>(m, "Float");
    declareFactories<bf16>(m, "BFloat");
    declareFactories<f16>(m, "Half");
    declareFactories<double>(m, "Double");
    declareFactories<float>(m, "");
    declareLosses<float>(m, "Float");
    declareLosses<bf16>(m, "BFloat");
    declareLosses<f16>(m, "Half");
    declareLosses<double>(m, "Double");
    declareNanoGPT<float>(m, "Float");
    declareNanoGPT<bf16>(m, "BFloat");
    declareNanoGPT<f16>(m, "Half");
    declareNanoGPT<double>(m, "Double");
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
    m.def("FlashAttentionHalf",
          [](int headDim, int numHeads, bool causal) {
              return std::make_shared<FlashAttentionLayer<f16>>(headDim, numHeads, causal);
          },
          py::arg("head_dim"), py::arg("num_heads"), py::arg("causal") = false,
          "Creates a float16 FlashAttentionLayer (generic kernels, fp32 accumulation).");
    m.def("FlashAttentionDouble",
          [](int headDim, int numHeads, bool causal) {
              return std::make_shared<FlashAttentionLayer<double>>(headDim, numHeads, causal);
          },
          py::arg("head_dim"), py::arg("num_heads"), py::arg("causal") = false,
          "Creates a float64 FlashAttentionLayer (generic kernels, fp64 arithmetic and LSE).");
    m.def("synchronize", &Runtime::synchronize, "Waits for all work queued by this module.");
    m.def("empty_cache", [] { BlockCache::instance().emptyCache(); },
          "Returns the device memory cached for reuse by this module's tensors to the driver.");
    m.def("memory_cached", [] { return BlockCache::instance().cachedBytes(); },
          "Bytes of freed tensor memory held for reuse.");
    m.def("memory_reserved", [] { return BlockCache::instance().reservedBytes(); },
          "Bytes of device memory this module's allocator holds (in use or cached).");
    m.def("set_policy", &ctattn_set_policy, py::arg("policy"),
          "Kernel selection policy: 0 = MFMA (fastest), 1 = generic kernels, 2 = MFMA with a "
          "deterministic dQ reduction.  Returns the previous policy.");
    m.def("version", &ctattn_version, "Version of the attention kernel library.");
}
