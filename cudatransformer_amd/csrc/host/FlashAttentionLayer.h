// FlashAttentionLayer<DType>: the reference's attention-core utility
// (FlashAttentionLayer.cu:13-150) over the ctattn C-ABI.
//
// Same members and calls: FlashAttentionLayer(headDim, numHeads), clone(),
// computeAttention(q, k, v, saveStates), computeBackward(q, k, v, outputGrad), clearCache(),
// with the forward state cached by computeAttention(..., true) and recomputed by
// computeBackward when absent (FlashAttentionLayer.cu:114-127).  Differences, all deliberate:
//   * a `causal` member (default false = the reference's unmasked attention);
//   * the cached state is the fp32 logsumexp [B, H, T] instead of (max, denominator);
//   * the cached output shares the returned tensor's buffer instead of a D2D copy
//     (FlashAttentionLayer.cu:81-84), together with the tensor's version count: when the
//     returned O was written in place through the Tensor API (fill, mutable data()) before
//     computeBackward, the backward recomputes the forward instead of using the changed O,
//     which gives the reference's result (it kept a private copy) without the copy;
//   * the cache is only used when its batch size and sequence length match the call;
//   * shapes are validated ([B, numHeads, T, headDim]) and every launch is checked.
#pragma once

#include <array>
#include <type_traits>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "Tensor.h"

namespace ct {

template <typename DType = float>
struct FlashAttentionLayer {
    using Stat = StatOf<DType>;  // LSE element type
    int headDim = 1;
    int numHeads = 1;
    bool causal = false;

    // Cached forward state (FlashAttentionLayer.cu:18-22).
    Tensor<Stat> cachedLse;  // LSE [B, H, T]: fp64 for double, fp32 otherwise
    Tensor<DType> cachedOutput;
    uint64_t cachedOutputVersion = 0;  // cachedOutput.version() when it was cached
    int cachedBatchSize = 0;
    int cachedSequenceLength = 0;

    FlashAttentionLayer(int headDim, int numHeads, bool causal = false)
        : headDim(headDim), numHeads(numHeads), causal(causal) {
        if (headDim < 1 || headDim > 256) throw std::invalid_argument("headDim must be in [1, 256]");
        if (numHeads < 1) throw std::invalid_argument("numHeads must be >= 1");
    }

    // Copies the configuration only (FlashAttentionLayer.cu:34-36).
    std::shared_ptr<FlashAttentionLayer<DType>> clone() const {
        return std::make_shared<FlashAttentionLayer<DType>>(headDim, numHeads, causal);
    }

    // O = softmax(Q K^T / sqrt(d)) V for [B, H, T, d] inputs (FlashAttentionLayer.cu:45-87).
    Tensor<DType> computeAttention(const Tensor<DType> &queries, const Tensor<DType> &keys,
                                   const Tensor<DType> &values, bool saveStates = false) {
        check(queries, "queries");
        check(keys, "keys");
        check(values, "values");
        sameShape(queries, keys, "keys");
        sameShape(queries, values, "values");
        const size_t B = queries.shape(0), T = queries.shape(2);
        Tensor<DType> output = Tensor<DType>::empty(queries.shape());  // fully written by the kernel
        Tensor<Stat> lse = Tensor<Stat>::empty({B, size_t(numHeads), T});
        forward(queries, keys, values, output, lse);
        if (saveStates) {
            cachedLse = lse;
            cachedOutput = output;
            cachedOutputVersion = output.version();
            cachedBatchSize = int(B);
            cachedSequenceLength = int(T);
        }
        return output;
    }

    // {dQ, dK, dV} for upstream gradient dO (FlashAttentionLayer.cu:97-142).
    std::array<Tensor<DType>, 3> computeBackward(const Tensor<DType> &queries, const Tensor<DType> &keys,
                                                 const Tensor<DType> &values,
                                                 const Tensor<DType> &outputGrad) {
        check(queries, "queries");
        sameShape(queries, keys, "keys");
        sameShape(queries, values, "values");
        sameShape(queries, outputGrad, "outputGrad");
        const size_t B = queries.shape(0), T = queries.shape(2);
        Tensor<Stat> lse = cachedLse;
        Tensor<DType> output = cachedOutput;
        if (lse.empty() || output.empty() || cachedBatchSize != int(B) || cachedSequenceLength != int(T) ||
            output.version() != cachedOutputVersion) {
            // No usable cached forward (none, another shape, or the returned O was written in
            // place since): recompute it (FlashAttentionLayer.cu:114-127).
            lse = Tensor<Stat>::empty({B, size_t(numHeads), T});
            output = Tensor<DType>::empty(queries.shape());
            forward(queries, keys, values, output, lse);
        }
        // Fully overwritten by ctattn_bwd (the reference zero-fills and accumulates atomically).
        // The default workspace is linear in B * H * T, like the reference's backward memory.
        std::array<Tensor<DType>, 3> grads = {Tensor<DType>::empty(queries.shape()),
                                              Tensor<DType>::empty(queries.shape()),
                                              Tensor<DType>::empty(queries.shape())};
        const int64_t wsBytes = ctattn_bwd_workspace_bytes(DTypeCode<DType>::value, int64_t(B), numHeads,
                                                           int64_t(T), headDim, causal ? 1 : 0);
        if (wsBytes < 0) ctattnCheck(int(hipErrorInvalidValue), "ctattn_bwd_workspace_bytes");
        std::shared_ptr<uint8_t[]> workspace = deviceAlloc<uint8_t>(size_t(wsBytes > 0 ? wsBytes : 1));
        ctattnCheck(ctattn_bwd(DTypeCode<DType>::value, queries.get(), keys.get(), values.get(), output.get(),
                               outputGrad.get(), lse.get(), grads[0].get(), grads[1].get(), grads[2].get(),
                               workspace.get(), wsBytes, int64_t(B), numHeads, int64_t(T), headDim,
                               causal ? 1 : 0, Runtime::stream()),
                    "ctattn_bwd");
        return grads;
    }

    // Drops the cached forward state (FlashAttentionLayer.cu:145-149).
    void clearCache() {
        cachedLse = Tensor<Stat>();
        cachedOutput = Tensor<DType>();
        cachedOutputVersion = 0;
        cachedBatchSize = 0;
        cachedSequenceLength = 0;
    }

private:
    // ctattn_fwd_ws with a workspace from the caching allocator (non-empty only for head dims
    // that run padded), so the library itself allocates nothing.
    void forward(const Tensor<DType> &queries, const Tensor<DType> &keys, const Tensor<DType> &values,
                 Tensor<DType> &output, Tensor<Stat> &lse) const {
        const int64_t B = int64_t(queries.shape(0)), T = int64_t(queries.shape(2));
        const int64_t wsBytes = ctattn_fwd_workspace_bytes(DTypeCode<DType>::value, B, numHeads, T, headDim);
        if (wsBytes < 0) ctattnCheck(int(hipErrorInvalidValue), "ctattn_fwd_workspace_bytes");
        std::shared_ptr<uint8_t[]> workspace;
        if (wsBytes > 0) workspace = deviceAlloc<uint8_t>(size_t(wsBytes));
        ctattnCheck(ctattn_fwd_ws(DTypeCode<DType>::value, queries.get(), keys.get(), values.get(), output.get(),
                                  lse.get(), workspace.get(), wsBytes, B, numHeads, T, headDim, causal ? 1 : 0,
                                  Runtime::stream()),
                    "ctattn_fwd_ws");
    }

    void check(const Tensor<DType> &t, const char *name) const {
        if (t.nDim() != 4 || int(t.shape(1)) != numHeads || int(t.shape(3)) != headDim)
            throw std::invalid_argument(std::string(name) + " must be [batch, " + std::to_string(numHeads) +
                                        ", seq_len, " + std::to_string(headDim) + "]");
    }
    static void sameShape(const Tensor<DType> &a, const Tensor<DType> &b, const char *name) {
        if (a.shape() != b.shape()) throw std::invalid_argument(std::string(name) + " shape differs from queries");
    }
};

}  // namespace ct
