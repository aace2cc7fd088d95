// hipBLASLt GEMM for the plain row-major products of the linear layers (blaslt_gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ctattn {

// Column-major C (m x n, ld ldc) = op(A) op(B) + beta C [+ bias per row of C], op = transpose
// when trans_*; dtype 0 fp32, 1 bf16, 2 fp16 (fp32 compute).  Enqueues on `stream` and
// returns true, or returns false without enqueuing anything when hipBLASLt cannot run the
// problem (the caller then uses its own kernel).
bool blaslt_gemm(int dtype, bool trans_a, bool trans_b, int64_t m, int64_t n, int64_t k, const void *A, int64_t lda,
                 const void *B, int64_t ldb, void *C, int64_t ldc, float beta, const void *bias, hipStream_t stream);

}  // namespace ctattn
