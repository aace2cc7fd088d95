// Elementwise activations and their derivatives (relu_/gelu_/sigmoid_/tanh_kernels.cu),
// shared by the activation kernels (model_ops.hip) and the GEMM epilogues that fuse them
// (linear_gemm.hip), so both paths compute the same values.  `kind` is enum ctattn_activation;
// GELU is the tanh form.
#pragma once

#include "attn_common.h"
#include "ctattn.h"

namespace ctattn {

constexpr double kGeluC = 0.7978845608028654;  // sqrt(2 / pi)
constexpr double kGeluA = 0.044715;

// Contraction into fused multiply-adds is off in both functions, so each call site (the
// elementwise kernels, every GEMM epilogue instantiation) evaluates them as written and the
// fused and separate paths agree bit for bit.
template <typename A> __device__ __forceinline__ A act_fwd(int kind, A x) {
#pragma clang fp contract(off)
    switch (kind) {
        case CTATTN_ACT_RELU: return x > A(0) ? x : A(0);
        case CTATTN_ACT_GELU: return A(0.5) * x * (A(1) + acc_tanh(A(kGeluC) * (x + A(kGeluA) * x * x * x)));
        case CTATTN_ACT_SIGMOID: return A(1) / (A(1) + acc_exp(-x));
        default: return acc_tanh(x);
    }
}

template <typename A> __device__ __forceinline__ A act_grad(int kind, A x) {
#pragma clang fp contract(off)
    switch (kind) {
        case CTATTN_ACT_RELU: return x > A(0) ? A(1) : A(0);
        case CTATTN_ACT_GELU: {
            const A t = acc_tanh(A(kGeluC) * (x + A(kGeluA) * x * x * x));
            return A(0.5) * (A(1) + t) + A(0.5) * x * (A(1) - t * t) * A(kGeluC) * (A(1) + A(3) * A(kGeluA) * x * x);
        }
        case CTATTN_ACT_SIGMOID: {
            const A s = A(1) / (A(1) + acc_exp(-x));
            return s * (A(1) - s);
        }
        default: {
            const A t = acc_tanh(x);
            return A(1) - t * t;
        }
    }
}

// act'(x) * dy, rounded to the accumulation type before any narrowing by the caller.  The
// product and a following conversion to fp16 can otherwise be selected as one mixed-precision
// FMA that rounds once (fp16 storage), which the GEMM epilogue -- an fp32 product, then fp16 --
// would not match at rounding midpoints; the empty asm keeps the fp32 value.
template <typename A> __device__ __forceinline__ A act_bwd_value(int kind, A x, A dy) {
#pragma clang fp contract(off)
    A r = act_grad(kind, x) * dy;
    asm volatile("" : "+v"(r));
    return r;
}

}  // namespace ctattn
