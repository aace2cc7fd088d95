// Internal launch interface of the split-K-in-workgroup MFMA GEMMs (linear_gemm.hip): the
// linear layers' products, the attention layer's projections and the Tensor matmul.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ctattn {

// A separable 2-D view of memory: element (i, j) at base + row_off(i) + col_off(j) elements.
//   linear (heads == 0):  row_off(i) = i * ld,  col_off(j) = j
//   head-split [B, H, T, d] seen as a [B*T, H*d] matrix (heads != 0):
//     row_off(r) = (r / T) * H*T*d + (r % T) * d,  col_off(c) = (c / d) * T*d + c % d
struct LinView {
    int64_t ld;
    int32_t heads, T, d;
};
inline LinView lin_linear(int64_t ld) { return LinView{ld, 0, 0, 0}; }
inline LinView lin_heads(int64_t T, int64_t H, int64_t d) {
    return LinView{0, int32_t(H), int32_t(T), int32_t(d)};
}

constexpr int kLinMaxBatch = 3;  // independent products per launch (Q, K, V)
constexpr int kLinMaxSeg = 3;    // K segments summed into one output (dX = dQ Wq + dK Wk + dV Wv)

// out_z(m, n) [+]= sum over segments s of sum_k A_zs(m, k) B_zs(k, n) (+ bias_z[n]), z < nbatch:
//   a_kc: A(m, k) = element (m, k) of the view av;  else A(m, k) = element (k, m)
//   b_kc: B(k, n) = element (n, k) of bv;            else B(k, n) = element (k, n)
//   out(m, n) = element (m, n) of cv;  K is per segment; beta: add into out.
struct LinGemm {
    int dtype;  // 0 fp32, 1 bf16, 2 fp16 storage (fp32 accumulation)
    bool a_kc, b_kc;
    int64_t M, N, K;
    int nbatch, nseg;
    LinView av, bv, cv;
    const void *a[kLinMaxBatch][kLinMaxSeg];
    const void *b[kLinMaxBatch][kLinMaxSeg];
    void *c[kLinMaxBatch];
    const void *bias[kLinMaxBatch];  // per column n, storage type, or null
    // Weight gradients (A M/N-contiguous, A = dY^T): db[m] += sum_k A(m, k), the bias
    // gradient, accumulated in storage type; null for none.  Ignored for K-contiguous A.
    void *db[kLinMaxBatch];
    bool beta;
    // An elementwise activation (act_kind: enum ctattn_activation) fused into the epilogue of
    // a K-contiguous-A product without beta, aux[z] in out's view (0: none):
    //   act_mode 1: out = the pre-activation p (bias included), aux[z] = act(p);
    //   act_mode 2: out = act'(aux[z]) * product, aux[z] holding the pre-activation.
    // Each value is rounded to storage type where the separate kernels would round it, so the
    // results equal a product followed by the activation kernel.
    int act_mode, act_kind;
    void *aux[kLinMaxBatch];
};

// One row-major product: C[m][n] (+)= sum_k A(m, k) B(k, n) (+ bias[n]) with
//   a_kc: A(m, k) = a[m * lda + k]   else  A(m, k) = a[k * lda + m]
//   b_kc: B(k, n) = b[n * ldb + k]   else  B(k, n) = b[k * ldb + n]
//   C(m, n) = c[m * ldc + n].
LinGemm lin_plain(int dtype, bool a_kc, bool b_kc, int64_t M, int64_t N, int64_t K, const void *a, int64_t lda,
                  const void *b, int64_t ldb, void *c, int64_t ldc, const void *bias, bool beta);

// Whether the product is in these kernels' domain: fp32 / bf16 / fp16; K a multiple of the
// 64-byte K chunk (16 fp32 or 32 16-bit elements) and, for head-split operands, chunks and
// 4- (fp32) or 8-element (16-bit) column groups inside one head; 16-byte aligned operands and
// pitches; M/N-contiguous extents a multiple of 4 (fp32) or 8 (16-bit); 32-bit lane offsets.
bool lin_gemm_supported(const LinGemm &g);

// Bytes of split-K partials the product's launch plan uses when workspace is allowed (0: the
// plan does not split K across workgroups, or the shape is not supported).  Depends on the
// dtype, layout, views and sizes only: the pointers may be null.
int64_t lin_gemm_workspace_bytes(const LinGemm &g);

// Launches the product.  ws / ws_bytes: workspace for split-K partials (may be null / 0: the
// plan then keeps K inside the workgroup).  Deterministic: fixed summation order, no atomics.
hipError_t launch_lin_gemm(const LinGemm &g, void *ws, int64_t ws_bytes, hipStream_t stream);

}  // namespace ctattn
