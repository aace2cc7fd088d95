// MFMA helpers for gfx950 (CDNA4).
//
// v_mfma_f32_32x32x2f32, D[32x32] += A[32x2] * B[2x32], one wave64.  Operand/result lane
// layout (lane l, col = l & 31, half = l >> 5):
//   A[i][kk] is supplied by lane (i + 32 * kk)        -> lane (col=i, half=kk)
//   B[kk][j] is supplied by lane (j + 32 * kk)        -> lane (col=j, half=kk)
//   D[i][j]  lives in lane (j + 32 * ((i / 4) % 2)), register (i % 4) + 4 * (i / 8)
// i.e. register r of lane (col, half) holds row  i = 8 * (r / 4) + 4 * half + (r % 4),
// column j = col.  The helpers below name that mapping so kernels never hard-code it.
#pragma once

#include "attn_common.h"

namespace ctattn {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ floatx16 mfma32x32x2(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row index (within the 32-row tile) held by accumulator register r of a lane in `half`.
__host__ __device__ constexpr int acc_row(int r, int half) { return 8 * (r / 4) + 4 * half + (r % 4); }

// Contraction index fed by k-step s from lane half `half` when four consecutive k-steps
// read one 16-byte vector: steps 4m..4m+3 cover indices 8m + 4*half + 0..3.
__host__ __device__ constexpr int kstep_index(int s, int half) { return 8 * (s / 4) + 4 * half + (s % 4); }

__device__ __forceinline__ floatx16 zero16() {
    floatx16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace ctattn
