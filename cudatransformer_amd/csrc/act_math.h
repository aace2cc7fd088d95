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

// tanh in fp32 from two textbook identities instead of the library tanhf, whose argument
// reduction and branches left the GELU and tanh kernels compute-bound (6.3 M GELUs took 12 us,
// six times their memory time): the Maclaurin series
//   tanh x = x - x^3/3 + 2x^5/15 - 17x^7/315 + 62x^9/2835 - 1382x^11/155925 + 21844x^13/6081075
// (coefficients 2^2n (2^2n - 1) B_2n / (2n)!, B the Bernoulli numbers) below |x| = 0.3, and
//   tanh|x| = 1 - 2 / (1 + e^(2|x|))
// above, e^(2|x|) on v_exp_f32 and the reciprocal on v_rcp_f32.  Emulated in float32 with
// correctly rounded exp2 and reciprocal against float64 tanh over [-12, 12]: at most 2.8 ulp,
// just above |x| = 0.3, where the subtraction cancels one to two bits; 0.6 ulp in the series
// range, 1.2 ulp above |x| = 1.  Large |x| give e = inf, 1 - 2 / inf = 1; NaN stays NaN.
__device__ __forceinline__ float act_tanh(float x) {
#pragma clang fp contract(off)
    const float a = fabsf(x);
    const float x2 = x * x;
    float p = fmaf(21844.f / 6081075.f, x2, -1382.f / 155925.f);
    p = fmaf(p, x2, 62.f / 2835.f);
    p = fmaf(p, x2, -17.f / 315.f);
    p = fmaf(p, x2, 2.f / 15.f);
    p = fmaf(p, x2, -1.f / 3.f);
    const float s = fmaf(x * x2, p, x);
    const float e = __builtin_amdgcn_exp2f(2.f * 1.44269504088896341f * a);
    const float t = fmaf(-2.f, __builtin_amdgcn_rcpf(1.f + e), 1.f);
    return a < 0.3f ? s : __builtin_copysignf(t, x);
}
__device__ __forceinline__ double act_tanh(double x) { return tanh(x); }

// Contraction into fused multiply-adds is off in both functions, so each call site (the
// elementwise kernels, every GEMM epilogue instantiation) evaluates them as written and the
// fused and separate paths agree bit for bit.
template <typename A> __device__ __forceinline__ A act_fwd(int kind, A x) {
#pragma clang fp contract(off)
    switch (kind) {
        case CTATTN_ACT_RELU: return x > A(0) ? x : A(0);
        case CTATTN_ACT_GELU: return A(0.5) * x * (A(1) + act_tanh(A(kGeluC) * (x + A(kGeluA) * x * x * x)));
        case CTATTN_ACT_SIGMOID: return A(1) / (A(1) + acc_exp(-x));
        default: return act_tanh(x);
    }
}

template <typename A> __device__ __forceinline__ A act_grad(int kind, A x) {
#pragma clang fp contract(off)
    switch (kind) {
        case CTATTN_ACT_RELU: return x > A(0) ? A(1) : A(0);
        case CTATTN_ACT_GELU: {
            const A t = act_tanh(A(kGeluC) * (x + A(kGeluA) * x * x * x));
            return A(0.5) * (A(1) + t) + A(0.5) * x * (A(1) - t * t) * A(kGeluC) * (A(1) + A(3) * A(kGeluA) * x * x);
        }
        case CTATTN_ACT_SIGMOID: {
            const A s = A(1) / (A(1) + acc_exp(-x));
            return s * (A(1) - s);
        }
        default: {
            const A t = act_tanh(x);
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
