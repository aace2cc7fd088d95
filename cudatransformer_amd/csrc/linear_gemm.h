// Internal launch interface of the plain row-major GEMMs (linear_gemm.hip): the linear layers'
// products and the Tensor matmul.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ctattn {

// C[m][n] (+)= sum_k A(m, k) B(k, n) (+ bias[n]), all row-major:
//   a_kc: A(m, k) = a[m * lda + k]   else  A(m, k) = a[k * lda + m]
//   b_kc: B(k, n) = b[n * ldb + k]   else  B(k, n) = b[k * ldb + n]
//   C(m, n) = c[m * ldc + n]; beta: add into C; bias: per column n, or null.
struct LinGemm {
    int dtype;  // 0 fp32 (the only storage type these kernels take)
    bool a_kc, b_kc;
    int64_t M, N, K;
    const void *a;
    int64_t lda;
    const void *b;
    int64_t ldb;
    void *c;
    int64_t ldc;
    const void *bias;
    bool beta;
};

// Whether the product is in these kernels' domain: fp32, K a multiple of 16, 16-byte aligned
// operands and pitches, M/N-contiguous extents a multiple of 4, 32-bit tile offsets.
bool lin_gemm_supported(const LinGemm &g);

// Bytes of split-K partials the product's launch plan uses when workspace is allowed (0: the
// plan does not split K across workgroups, or the shape is not supported).  Depends on the
// dtype, layout and sizes only: the pointers may be null.
int64_t lin_gemm_workspace_bytes(const LinGemm &g);

// Launches the product.  ws / ws_bytes: workspace for split-K partials (may be null / 0: the
// plan then keeps K inside the workgroup).  Deterministic: fixed summation order, no atomics.
hipError_t launch_lin_gemm(const LinGemm &g, void *ws, int64_t ws_bytes, hipStream_t stream);

}  // namespace ctattn
