// pybind11 module `cuda_transformer`: the attention-path part of the reference's Python API
// (cuda_transformer.cu:22-119 declare_tensor, :257-324 the attention bindings), on the
// MI355X kernels behind include/ctattn.h.
//
// Names follow the reference: FloatTensor / BFloatTensor with fromNumpy, numpy, shape,
// clone, item, fill, reshape.  The reference does not bind FlashAttentionLayer itself (it is
// reached only through AttentionLayer); here it is bound as FloatFlashAttentionLayer /
// BFloatFlashAttentionLayer with the C++ method names (computeAttention, computeBackward,
// clearCache, clone), plus the factories FlashAttention / FlashAttentionFloat /
// FlashAttentionBFloat.  bf16 tensors take and return float32 numpy arrays (numpy has no
// bfloat16; values are rounded to nearest even on upload).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

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

}  // namespace

PYBIND11_MODULE(cuda_transformer, m) {
    m.doc() =
        "cuda_transformer (MI355X): the flash-attention path of CudaTransformer on gfx950 HIP kernels.\n"
        "Tensors: FloatTensor, BFloatTensor.  Attention core: FloatFlashAttentionLayer,\n"
        "BFloatFlashAttentionLayer, FlashAttention(head_dim, num_heads, causal=False).";

    declareTensor<float>(m, "Float");
    declareTensor<bf16>(m, "BFloat");
    declareFlashAttention<float>(m, "Float");
    declareFlashAttention<bf16>(m, "BFloat");

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
