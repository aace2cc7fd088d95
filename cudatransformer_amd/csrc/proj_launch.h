// Internal launch interface of the projection GEMMs (proj_gemm.hip) used by the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ctattn {

constexpr int kViewLinear = 0;     // element (i, j) at i * ld + j
constexpr int kViewHeadSplit = 1;  // [B, H, T, d] seen as [B*T, H*d]

// A separable 2-D view of memory: element (i, j) at p + row_off(i) + col_off(j).
struct MatView {
    const void *p;
    int64_t ld;  // linear views: row pitch in elements
    int32_t kind, T, H, d;  // head-split views: sequence length, heads, head dim
};

inline MatView linear_view(const void *p, int64_t ld) { return MatView{p, ld, kViewLinear, 0, 0, 0}; }
inline MatView head_view(const void *p, int64_t T, int64_t H, int64_t d) {
    return MatView{p, 0, kViewHeadSplit, int32_t(T), int32_t(H), int32_t(d)};
}

constexpr int kMaxSeg = 3;    // K segments summed into one output (dX = dQ Wq + dK Wk + dV Wv)
constexpr int kMaxBatch = 3;  // independent products per launch (Q, K, V)

// One output of a launch: out [+]= sum_seg A_seg B_seg (+ bias).
struct GemmBatch {
    MatView a[kMaxSeg];  // A(m, k) views; all segments share kind / ld / shape
    MatView b[kMaxSeg];  // B(k, n) views
    int32_t nseg;
    void *out;
    const void *bias;  // per column n, or null
};

struct GemmParams {
    int32_t M, N, K;  // K per segment
    int32_t beta;     // 1: add into out
    int32_t splits;   // K splits; > 1 -> partial tiles in ws, then an ordered reduction
    MatView outv;     // view of every batch's out (pointer taken from the batch)
    float *ws;        // splits * M * N floats per batch when splits > 1
    GemmBatch batch[kMaxBatch];
};

int gemm_tile_count(int64_t M, int64_t N);
int gemm_k_steps(int64_t K);

// dtype: 0 fp32, 1 bf16, 2 fp16 (MFMA GEMM, fp32 arithmetic), 3 fp64 (fp64 GEMM; splits must
// be 1).  a_kc / b_kc: operand is K-contiguous in memory (A stored [m][k], B stored [n][k]); else
// A is stored [k][m], B [k][n].  vec4: every extent, pitch and head dim is a multiple of 4
// and every base pointer is 4-element aligned.
hipError_t launch_proj_gemm(int dtype, const GemmParams &prm, int nbatch, bool a_kc, bool b_kc,
                            bool vec4, hipStream_t stream);

// out[c] += sum_r g(r, c), deterministic; ws holds colsum_workspace_bytes(dtype, R, C) bytes.
int64_t colsum_workspace_bytes(int dtype, int64_t R, int64_t C);
hipError_t launch_colsum_add(int dtype, const MatView &g, int R, int C, void *out, void *ws,
                             hipStream_t stream);

// params -= lr * grads, elementwise.
hipError_t launch_sgd(int dtype, void *params, const void *grads, double lr, int64_t n, hipStream_t stream);

}  // namespace ctattn
