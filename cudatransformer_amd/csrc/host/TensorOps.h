// Tensor<DType> operations of the reference's Tensor class (Tensor.cu:267-950): dtype casts,
// broadcasting arithmetic and comparisons, unary maps, reductions, transpose, Kronecker and
// matrix products.  Each computes in libctattn.so (ctattn_tensor_* in include/ctattn.h) and
// returns a new tensor; shape errors throw std::invalid_argument (ValueError in Python) before
// anything is launched.  Differences from the reference: broadcasting and reduction axes are
// checked on the host; reducing an empty axis gives 0 (SUM, MEAN of integers, norms), NaN
// (MEAN of floating types) or an error (MAX, MIN); matmul requires b's batch to be 1 or a's.
#pragma once

#include <algorithm>
#include <limits>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "Tensor.h"

namespace ct {

// The reference's ReductionOp (headers.cu).
enum class ReductionOp {
    SUM = CTATTN_RED_SUM,
    MEAN = CTATTN_RED_MEAN,
    MAX = CTATTN_RED_MAX,
    MIN = CTATTN_RED_MIN,
    NORM_L1 = CTATTN_RED_NORM_L1,
    NORM_L2 = CTATTN_RED_NORM_L2
};

namespace ops {

inline std::vector<int64_t> dims64(const std::vector<size_t> &s) { return std::vector<int64_t>(s.begin(), s.end()); }

inline size_t product(const std::vector<size_t> &s, size_t from, size_t to) {
    size_t n = 1;
    for (size_t k = from; k < to; ++k) n *= s[k];
    return n;
}

// Tensor::to<To>() (Tensor.cu:267): a new tensor of the converted values.
template <typename To, typename From>
Tensor<To> cast(const Tensor<From> &t) {
    if constexpr (std::is_same_v<To, From>) {
        return t.clone();
    } else {
        Tensor<To> out = Tensor<To>::empty(t.shape());
        ctattnCheck(ctattn_tensor_cast(DTypeCode<From>::value, t.get(), DTypeCode<To>::value, out.get(),
                                       int64_t(t.size()), Runtime::stream()),
                    "ctattn_tensor_cast");
        return out;
    }
}

inline std::vector<size_t> broadcastShape(const std::vector<size_t> &a, const std::vector<size_t> &b) {
    const size_t n = std::max(a.size(), b.size());
    if (n > 8) throw std::invalid_argument("Tensor dimension exceeds 8");
    std::vector<size_t> out(n);
    for (size_t i = 0; i < n; ++i) {
        const size_t da = i < a.size() ? a[a.size() - 1 - i] : 1, db = i < b.size() ? b[b.size() - 1 - i] : 1;
        if (da != db && da != 1 && db != 1) throw std::invalid_argument("Broadcasting failed: shapes do not match");
        out[n - 1 - i] = da == 1 ? db : da;  // a 1 stretches to the other extent, 0 included
    }
    return out;
}

// a op b with broadcasting (Tensor.cu:650-740); Out is bool for the comparisons.
template <typename Out, typename DType>
Tensor<Out> binary(const Tensor<DType> &a, const Tensor<DType> &b, int op) {
    Tensor<Out> out = Tensor<Out>::empty(broadcastShape(a.shape(), b.shape()));
    const auto sa = dims64(a.shape()), sb = dims64(b.shape());
    ctattnCheck(ctattn_tensor_binary(DTypeCode<DType>::value, op, a.get(), int(sa.size()), sa.data(), b.get(),
                                     int(sb.size()), sb.data(), out.get(), Runtime::stream()),
                "ctattn_tensor_binary");
    return out;
}

// a op s, or s op a with scalarLeft (Tensor.cu:742-790).
template <typename Out, typename DType>
Tensor<Out> scalar(const Tensor<DType> &a, double s, int op, bool scalarLeft = false) {
    Tensor<Out> out = Tensor<Out>::empty(a.shape());
    ctattnCheck(ctattn_tensor_scalar(DTypeCode<DType>::value, op, a.get(), s, scalarLeft ? 1 : 0, out.get(),
                                     int64_t(a.size()), Runtime::stream()),
                "ctattn_tensor_scalar");
    return out;
}

template <typename DType>
Tensor<DType> unary(const Tensor<DType> &a, int op) {
    Tensor<DType> out = Tensor<DType>::empty(a.shape());
    ctattnCheck(ctattn_tensor_unary(DTypeCode<DType>::value, op, a.get(), out.get(), int64_t(a.size()),
                                    Runtime::stream()),
                "ctattn_tensor_unary");
    return out;
}

// Axes permuted: output axis k is input axis perm[k] (Tensor.cu:577-601).
template <typename DType>
Tensor<DType> permute(const Tensor<DType> &a, const std::vector<size_t> &perm) {
    if (perm.size() != a.nDim()) throw std::invalid_argument("transpose: perm must name every axis once");
    std::vector<size_t> shape(perm.size());
    std::vector<int32_t> p(perm.size());
    for (size_t k = 0; k < perm.size(); ++k) {
        if (perm[k] >= a.nDim()) throw std::invalid_argument("transpose: axis out of range");
        shape[k] = a.shape(perm[k]);
        p[k] = int32_t(perm[k]);
    }
    std::vector<size_t> sorted(perm);
    std::sort(sorted.begin(), sorted.end());
    if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end())
        throw std::invalid_argument("transpose: perm must name every axis once");
    Tensor<DType> out = Tensor<DType>::empty(shape);
    const auto s = dims64(a.shape());
    ctattnCheck(ctattn_tensor_permute(DTypeCode<DType>::value, a.get(), int(s.size()), s.data(), p.data(), out.get(),
                                      Runtime::stream()),
                "ctattn_tensor_permute");
    return out;
}

// Two axes swapped (Tensor.cu:607-616).
template <typename DType>
Tensor<DType> transpose(const Tensor<DType> &a, size_t axis1, size_t axis2) {
    if (axis1 >= a.nDim() || axis2 >= a.nDim()) throw std::invalid_argument("transpose: axis out of range");
    std::vector<size_t> p(a.nDim());
    std::iota(p.begin(), p.end(), size_t(0));
    std::swap(p[axis1], p[axis2]);
    return permute(a, p);
}

// a viewed as [outer][R][inner] reduced over R.
template <typename DType>
Tensor<DType> reduce3(const Tensor<DType> &a, size_t outer, size_t R, size_t inner, ReductionOp op,
                      const std::vector<size_t> &outShape) {
    Tensor<DType> out = Tensor<DType>::empty(outShape);
    if (outer * inner == 0) return out;
    if (R == 0) {
        if (op == ReductionOp::MAX || op == ReductionOp::MIN)
            throw std::invalid_argument("reduce: max / min of an empty axis");
        out.fill(op == ReductionOp::MEAN && !std::is_integral_v<DType> ? std::numeric_limits<double>::quiet_NaN() : 0.0);
        return out;
    }
    const int dt = DTypeCode<DType>::value;
    const int64_t wsBytes = ctattn_tensor_reduce_workspace_bytes(dt, int64_t(outer), int64_t(R), int64_t(inner));
    if (wsBytes < 0) ctattnCheck(1, "ctattn_tensor_reduce_workspace_bytes");
    auto ws = deviceAlloc<uint8_t>(size_t(wsBytes));
    ctattnCheck(ctattn_tensor_reduce(dt, int(op), a.get(), int64_t(outer), int64_t(R), int64_t(inner), out.get(),
                                     ws.get(), wsBytes, Runtime::stream()),
                "ctattn_tensor_reduce");
    return out;
}

// Reduction over `axes` (Tensor.cu:807-845): the result keeps the other axes in order, or is
// [1] when every axis is reduced.
template <typename DType>
Tensor<DType> reduce(const Tensor<DType> &a, std::vector<size_t> axes, ReductionOp op) {
    const size_t nd = a.nDim();
    std::sort(axes.begin(), axes.end());
    axes.erase(std::unique(axes.begin(), axes.end()), axes.end());
    for (size_t ax : axes)
        if (ax >= nd) throw std::invalid_argument("reduce: axis out of range");
    std::vector<size_t> kept, outShape;
    for (size_t k = 0; k < nd; ++k)
        if (!std::binary_search(axes.begin(), axes.end(), k)) {
            kept.push_back(k);
            outShape.push_back(a.shape(k));
        }
    if (outShape.empty()) outShape.push_back(1);
    if (axes.empty()) return a.clone();
    const auto &s = a.shape();
    // One axis: [outer][R][inner] in place (columns need outer <= 65535).
    if (axes.size() == 1) {
        const size_t ax = axes[0], outer = product(s, 0, ax), inner = product(s, ax + 1, nd);
        if (inner == 1 || outer <= 65535) return reduce3(a, outer, s[ax], inner, op, outShape);
    }
    size_t R = 1;
    for (size_t ax : axes) R *= s[ax];
    const size_t outer = product(outShape, 0, outShape.size());
    // Reduced axes already trailing: rows of the trailing block; otherwise move them last.
    bool trailing = true;
    for (size_t j = 0; j < axes.size(); ++j) trailing = trailing && axes[j] == nd - axes.size() + j;
    if (trailing) return reduce3(a, outer, R, 1, op, outShape);
    std::vector<size_t> perm(kept);
    perm.insert(perm.end(), axes.begin(), axes.end());
    return reduce3(permute(a, perm), outer, R, 1, op, outShape);
}

// dim < 0 reduces every axis (Tensor.cu:865-870).
template <typename DType>
Tensor<DType> reduceDim(const Tensor<DType> &a, int dim, ReductionOp op) {
    if (dim < 0) {
        std::vector<size_t> all(a.nDim());
        std::iota(all.begin(), all.end(), size_t(0));
        return reduce(a, all, op);
    }
    return reduce(a, {size_t(dim)}, op);
}

// Kronecker product of two tensors of equal rank (Tensor.cu:877-905).
template <typename DType>
Tensor<DType> kron(const Tensor<DType> &a, const Tensor<DType> &b) {
    if (a.nDim() != b.nDim()) throw std::invalid_argument("kron: tensors must have the same number of dimensions");
    std::vector<size_t> shape(a.nDim());
    for (size_t k = 0; k < a.nDim(); ++k) shape[k] = a.shape(k) * b.shape(k);
    Tensor<DType> out = Tensor<DType>::empty(shape);
    const auto sa = dims64(a.shape()), sb = dims64(b.shape());
    ctattnCheck(ctattn_tensor_kron(DTypeCode<DType>::value, a.get(), b.get(), int(sa.size()), sa.data(), sb.data(),
                                   out.get(), Runtime::stream()),
                "ctattn_tensor_kron");
    return out;
}

// Batched matrix product over the last two axes (Tensor.cu:912-950): a [..., M, K] times
// b [..., K, N] -> [..., M, N] with a's leading axes; b holds one matrix or one per batch.
template <typename DType>
Tensor<DType> matmul(const Tensor<DType> &a, const Tensor<DType> &b) {
    if (a.nDim() < 2 || b.nDim() < 2) throw std::invalid_argument("matmul: both tensors need at least 2 dimensions");
    const size_t M = a.shape(a.nDim() - 2), K = a.shape(a.nDim() - 1);
    const size_t K2 = b.shape(b.nDim() - 2), N = b.shape(b.nDim() - 1);
    if (K != K2) throw std::invalid_argument("matmul: inner dimensions differ");
    const size_t batch = M * K == 0 ? product(a.shape(), 0, a.nDim() - 2) : a.size() / (M * K);
    const size_t batchB = K * N == 0 ? product(b.shape(), 0, b.nDim() - 2) : b.size() / (K * N);
    if (batchB != 1 && batchB != batch)
        throw std::invalid_argument("matmul: b must hold one matrix or one per batch of a");
    std::vector<size_t> shape(a.shape().begin(), a.shape().end() - 2);
    shape.push_back(M);
    shape.push_back(N);
    Tensor<DType> out = Tensor<DType>::empty(shape);
    ctattnCheck(ctattn_tensor_matmul(DTypeCode<DType>::value, a.get(), b.get(), out.get(), int64_t(batch),
                                     int64_t(batchB), int64_t(M), int64_t(K), int64_t(N), Runtime::stream()),
                "ctattn_tensor_matmul");
    return out;
}

}  // namespace ops
}  // namespace ct
