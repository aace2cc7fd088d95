/*
 * ctattn -- C-ABI of the MI355X (gfx950) flash-attention kernels.
 *
 * This is the whole boundary between host code and the HIP kernels: plain pointers and
 * sizes, no C++ or framework types.  The C++ FlashAttentionLayer<DType> of this project
 * (cudatransformer_amd/csrc/host/FlashAttentionLayer.h) is its caller; any other host
 * (ctypes, cgo, JNI) can bind the same symbols.
 *
 * Conventions shared by every entry point
 *   - q, k, v, o, dout, dq, dk, dv are DEVICE pointers to contiguous row-major
 *     [B, H, T, d] tensors of the element type `dtype`; lse is a DEVICE pointer to a
 *     contiguous [B, H, T] tensor holding LSE_i = m_i + ln(l_i) (natural log), fp64 for
 *     dtype CTATTN_F64 and fp32 for every other dtype.
 *   - the score scale is 1/sqrt(d); causal != 0 masks key j > query i.  causal == 0 is
 *     the reference's behaviour (it has no mask).
 *   - keys past T do not take part in the softmax (no zero padding).
 *   - calls are asynchronous on `stream` (a hipStream_t; NULL = the default stream).
 *     Borrowed pointers must stay valid until the stream has finished with them.
 *   - return 0 on success, otherwise a hipError_t value; ctattn_last_error() then gives a
 *     message (per calling thread).  Argument errors are detected before any launch and
 *     return hipErrorInvalidValue (1); unsupported head dims return
 *     hipErrorNotSupported (801).
 *   - supported: dtype f32, bf16 or f16 (storage; arithmetic accumulates in fp32) or f64
 *     (arithmetic in fp64, the reference's ComputeType<double>), 1 <= d <= 256, T >= 0,
 *     B, H >= 0.  d in {32, 64, 128} runs on the MFMA kernels (fp32 on f32 MFMA, bf16 and
 *     f16 on 16-bit MFMA with fp32 accumulation, f64 on f64 MFMA).  Every other d <= 128
 *     runs on the MFMA kernels of the next width (32, 64 or 128) over zero-padded copies of
 *     the tensors, still scaled by 1/sqrt(d) (zero columns add nothing to a score; the
 *     padded columns of the outputs are dropped): the backward keeps the copies in its
 *     workspace, the forward takes them from a stream-ordered memory pool the library owns
 *     per device (hipMallocFromPoolAsync / hipFreeAsync on `stream`).  d above 128 runs on
 *     the generic kernels.  Tensors must be element-aligned; the MFMA kernels at d in
 *     {32, 64, 128} also need 16-byte-aligned q, k, v, o, lse (and dout, dq, dk, dv,
 *     workspace in the backward); calls whose pointers are not take the generic kernels
 *     (same results, slower).
 */
#ifndef CTATTN_H
#define CTATTN_H

#include <stdint.h>

/* Only the functions below are exported from libctattn.so (it is built with hidden
 * visibility), so two builds of the library can share a process without interposing. */
#define CTATTN_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* Storage types.  The attention, projection and layer entry points take the four floating
 * types; the tensor operations at the end of this header take all of them (bool is one byte
 * holding 0 or 1). */
enum ctattn_dtype {
    CTATTN_F32 = 0,
    CTATTN_BF16 = 1,
    CTATTN_F16 = 2,
    CTATTN_F64 = 3,
    CTATTN_I32 = 4,
    CTATTN_I64 = 5,
    CTATTN_I16 = 6,
    CTATTN_I8 = 7,
    CTATTN_BOOL = 8
};

/* Kernel selection policy (process-wide).
 *   AUTO           MFMA kernels where they apply (fastest).  The fp32 MFMA backward adds
 *                  dQ contributions of different key blocks with fp32 atomics, so an fp32
 *                  dQ may differ between runs in the last bits; dK, dV, O and LSE do not,
 *                  and the bf16 MFMA backward uses no atomics (bitwise reproducible).
 *   GENERIC        the generic kernels only, at every head dim (used to cross-check the
 *                  paths); the linear layers' fp32 GEMMs (ctattn_linear_*,
 *                  ctattn_tensor_matmul) then run on the projection GEMM family instead of
 *                  the split-K-in-workgroup linear GEMMs.
 *   DETERMINISTIC  MFMA kernels without atomics, bitwise-reproducible gradients.  The fp32
 *                  backward at d in {64, 128}, given a workspace that holds its dS tiles
 *                  (ctattn_bwd_workspace_bytes_max), stores dS from the key-major kernel
 *                  and computes dQ = dS K query-major (each element summed by one lane in a
 *                  fixed order).  Otherwise it stores dQ partials per 128-key block and sums
 *                  them in a fixed order while T <= 1024 (workspace: ceil(T/128) * B*H*T*d
 *                  fp32 more than AUTO, at most 8 dQ planes); for longer T it computes dK /
 *                  dV in a key-major kernel and dQ in a query-major one that recomputes S and
 *                  dP, with the same workspace as AUTO.  bf16 / fp16 / fp64: the same kernels
 *                  as AUTO, which use no atomics. */
enum ctattn_policy {
    CTATTN_POLICY_AUTO = 0,
    CTATTN_POLICY_GENERIC = 1,
    CTATTN_POLICY_DETERMINISTIC = 2
};

/*
 * Forward: O = softmax(Q K^T / sqrt(d)) V and LSE.
 * Replaces the flashAttention<DType> launch of FlashAttentionLayer::computeAttention
 * (reference FlashAttentionLayer.cu:73-79; kernel flash_attention.cu:57-169).  The
 * reference writes (maxScores, denominators) as two [B,H,T] DType buffers
 * (flash_attention.cu:164-167); this boundary writes the single LSE instead (fp32, or fp64
 * for f64).  lse may be NULL when the caller does not keep state for a backward.
 */
CTATTN_API int ctattn_fwd(int dtype, const void *q, const void *k, const void *v, void *o, void *lse,
               int64_t B, int64_t H, int64_t T, int64_t d, int causal, void *stream);

/*
 * Bytes of device workspace ctattn_fwd_ws needs (>= 0), or -1 on invalid arguments: 0 unless
 * the head dim runs padded (see the conventions above), then four [B,H,T,dp] copies (q, k,
 * v, o).  ctattn_fwd takes that memory from a stream-ordered pool the library owns (up to
 * 1 GiB of it stays cached per device); ctattn_fwd_ws takes it from the caller instead.
 */
CTATTN_API int64_t ctattn_fwd_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t T, int64_t d);

/*
 * ctattn_fwd with a caller workspace of at least ctattn_fwd_workspace_bytes bytes (16-byte
 * aligned; may be NULL when that is 0): the same kernels and results, and no memory
 * allocated by the library.  Replaces the same launch as ctattn_fwd
 * (FlashAttentionLayer.cu:73-79); the C++ layer and the Python wrapper call this one.
 */
CTATTN_API int ctattn_fwd_ws(int dtype, const void *q, const void *k, const void *v, void *o, void *lse,
                             void *workspace, int64_t workspace_bytes, int64_t B, int64_t H, int64_t T,
                             int64_t d, int causal, void *stream);

/*
 * Bytes of device workspace ctattn_bwd needs for this problem (>= 0), or -1 on invalid
 * arguments.  Replaces nothing in the reference: its backward zero-fills and atomically
 * accumulates straight into dq/dk/dv (FlashAttentionLayer.cu:103-106, flash_attention.cu:317-321).
 * A head dim that runs padded to width dp (see the conventions above) also needs room for
 * the eight padded copies (q, k, v, o, dout, dq, dk, dv: 8 * B*H*T*dp elements).
 * The size is linear in B*H*T, as the reference's backward memory is (it never holds a
 * T x T object): the dS tiles below are included only while the bytes they add take at most
 * twice the bytes of q, k and v together (bf16 / fp16 causal: T <= 12 d).
 */
CTATTN_API int64_t ctattn_bwd_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t T, int64_t d,
                                   int causal);

/*
 * The workspace of ctattn_bwd's fastest path (>= ctattn_bwd_workspace_bytes), or -1 on
 * invalid arguments.  No counterpart in the reference.  bf16 / fp16 at d = 128 (also padded
 * onto it): the dS tiles -- the dK/dV kernel stores the bf16 dS it computes and the dQ kernel
 * multiplies it by K instead of recomputing S and dP, 2 bytes per (row, key) pair of the mask
 * rounded to 32 x 32 tiles (causal B*H*T^2 bytes, B1 H32 T8192: 2.2 GB; 2-7 % faster
 * backward).  fp32 at d in {64, 128} under DETERMINISTIC, and at d = 128 with at least 1024
 * key blocks of 64 (ceil(T/64)*B*H) under AUTO: the fp32 dS tiles, 16 KiB per 64 x 64 tile of
 * the mask (causal about 2*B*H*T^2 bytes; B8 H12 T1024: 214 MB), from which dQ is computed
 * without atomics (DETERMINISTIC 5-46 % faster than without them, AUTO at d = 128 1-3 %).
 * Above 4 GiB of dS they are left out and this equals ctattn_bwd_workspace_bytes.
 */
CTATTN_API int64_t ctattn_bwd_workspace_bytes_max(int dtype, int64_t B, int64_t H, int64_t T, int64_t d,
                                                  int causal);

/*
 * Backward: dQ, dK, dV given Q, K, V, the forward's O and LSE, and dO.
 * Replaces the flashAttentionBackward<DType> launch of FlashAttentionLayer::computeBackward
 * (reference FlashAttentionLayer.cu:129-140; kernel flash_attention.cu:226-326).
 * dq, dk, dv are fully overwritten (no pre-zeroing needed).  workspace should hold
 * ctattn_bwd_workspace_bytes(...) bytes, queried under the same policy, or any size up to
 * ctattn_bwd_workspace_bytes_max(...); a smaller one works down to the size without the
 * dS tiles (the error message names the minimum).  With a workspace that holds the dS tiles
 * dQ = dS K reads them back; else bf16 / fp16 dQ recomputes S and dP (the same results up to
 * bf16 rounding of dS) and fp32 takes the policy's other dQ scheme.
 * Reproducibility depends on the policy (see enum ctattn_policy).
 */
CTATTN_API int ctattn_bwd(int dtype, const void *q, const void *k, const void *v, const void *o,
               const void *dout, const void *lse, void *dq, void *dk, void *dv,
               void *workspace, int64_t workspace_bytes, int64_t B, int64_t H, int64_t T,
               int64_t d, int causal, void *stream);

/* Size of the static device scratch buffer ctattn_bwd_noalloc works in (bytes, per GPU). */
#define CTATTN_NOALLOC_SCRATCH_BYTES (32LL << 20)

/*
 * Backward that allocates nothing: ctattn_bwd with its workspace taken from a static device
 * array of CTATTN_NOALLOC_SCRATCH_BYTES (32 MiB) that the library holds on each GPU it runs
 * on until the process ends.  No counterpart in the reference; it is for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  It calls no hipMalloc / hipFree and no allocating library routine.
 *   - same arguments, kernels and results as ctattn_bwd under the current policy, minus the
 *     workspace; it uses the smallest workspace ctattn_bwd accepts (the dS tiles only when
 *     they fit too), and problems that need more than the scratch size are
 *     rejected with hipErrorInvalidValue before any GPU work (AUTO needs 4 bytes per row
 *     B*H*T for fp32, 8 for bf16 / fp16 / fp64: up to 8 Mi or 4 Mi rows).
 *   - the scratch of the stream's device is found once per device (hipGetSymbolAddress) and
 *     shared by every call on that GPU: calls that overlap on one GPU (two streams, two host
 *     threads) race on it and must be serialised by the caller.  The kernels write every
 *     scratch byte they read, so leftover contents from an earlier call do not matter.
 */
CTATTN_API int ctattn_bwd_noalloc(int dtype, const void *q, const void *k, const void *v, const void *o,
                                  const void *dout, const void *lse, void *dq, void *dk, void *dv,
                                  int64_t B, int64_t H, int64_t T, int64_t d, int causal, void *stream);

/* Message describing the last failure of a ctattn_* call on this thread ("" if none). */
CTATTN_API const char *ctattn_last_error(void);

/* Set / get the process-wide kernel selection policy (enum ctattn_policy).  Returns the
 * previous policy, or -1 for an unknown value.  Not synchronised with calls in flight on
 * other threads: set it before issuing work. */
CTATTN_API int ctattn_set_policy(int policy);
CTATTN_API int ctattn_get_policy(void);

/* Library version, major * 10000 + minor * 100 + patch. */
CTATTN_API int ctattn_version(void);

/* ---- Attention-layer projections (the producer and consumer of the [B, H, T, d] layout) ----
 *
 * x, dx, y, dy: [B, T, E] row-major.  q, k, v, dq, dk, dv, c (the attention output), dc:
 * [B, H, T, d].  wq, wk, wv: [H*d][E] (row j holds the weights of output feature j, as the
 * reference's kernels index them, attention_qkv_kernels.cu:92; its getter's [E, H*d] shape
 * is only a label).  wo: [E][H*d].  bq, bk, bv: [H*d]; bo: [E].  Same dtype codes as above;
 * all arithmetic accumulates in fp32.  E >= 1, H >= 1, d >= 1 (any values; multiples of 4
 * take the vectorised loads), B*T, E and H*d below 2^31.  Asynchronous on `stream`.
 */

/*
 * q/k/v = x W^T + b, written straight into [B, H, T, d].  Bias pointers may be NULL (no bias).
 * Replaces the getQKVmatrices launch of QKVProjectionLayer::computeQKV
 * (QKVProjectionLayer.cu:82-87; kernel attention_qkv_kernels.cu:51-122).
 */
CTATTN_API int ctattn_qkv_proj_fwd(int dtype, const void *x, const void *wq, const void *wk,
                                   const void *wv, const void *bq, const void *bk, const void *bv,
                                   void *q, void *k, void *v, int64_t B, int64_t T, int64_t E,
                                   int64_t H, int64_t d, void *stream);

/* Workspace bytes ctattn_qkv_proj_bwd needs (>= 0), or -1 on invalid arguments. */
CTATTN_API int64_t ctattn_qkv_proj_bwd_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t E,
                                                       int64_t H, int64_t d);

/*
 * Backward of the QKV projection:
 *   dwq/dwk/dwv += dq/dk/dv^T x   (accumulated into the existing gradient, like the
 *                                  reference's atomicAdd into weightsQueryGrad etc.)
 *   dbq/dbk/dbv += column sums of dq/dk/dv over all B*T rows
 *   dx = dq wq + dk wk + dv wv     (overwritten)
 * Pass NULL for all three dw (or all three db, or dx) to skip that part; the workspace is
 * only needed for dw / db.  Replaces the qkvBackwardWB and qkvBackward launches of
 * QKVProjectionLayer::computeBackward (QKVProjectionLayer.cu:124-137; kernels
 * attention_qkv_kernels.cu:171-364).  Unlike the reference's bias gradient, which sums only
 * the first row of each 32-row tile (attention_qkv_kernels.cu:233-237), every row counts.
 * Deterministic: no atomics.
 */
CTATTN_API int ctattn_qkv_proj_bwd(int dtype, const void *x, const void *dq, const void *dk,
                                   const void *dv, const void *wq, const void *wk, const void *wv,
                                   void *dwq, void *dwk, void *dwv, void *dbq, void *dbk, void *dbv,
                                   void *dx, void *workspace, int64_t workspace_bytes, int64_t B,
                                   int64_t T, int64_t E, int64_t H, int64_t d, void *stream);

/*
 * y = c wo^T + bo, reading the attention output c in [B, H, T, d]; bo may be NULL.
 * Replaces the attentionProj launch of OutputProjectionLayer::forward
 * (OutputProjectionLayer.cu:60-63; kernel attention_proj_kernels.cu:48-98).
 */
CTATTN_API int ctattn_out_proj_fwd(int dtype, const void *c, const void *wo, const void *bo, void *y,
                                   int64_t B, int64_t T, int64_t E, int64_t H, int64_t d,
                                   void *stream);

/* Workspace bytes ctattn_out_proj_bwd needs (>= 0), or -1 on invalid arguments. */
CTATTN_API int64_t ctattn_out_proj_bwd_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t E,
                                                       int64_t H, int64_t d);

/*
 * Backward of the output projection:
 *   dwo += dy^T c,  dbo += column sums of dy,  dc = dy wo  (dc in [B, H, T, d], overwritten).
 * dwo, dbo or dc may be NULL to skip; the workspace is only needed for dwo / dbo.  Replaces
 * the projBackwardWB and projBackward launches of OutputProjectionLayer::backward
 * (OutputProjectionLayer.cu:83-94; kernels attention_proj_kernels.cu:142-288), with every
 * row in the bias gradient (the reference's sums one row per 32-row tile,
 * attention_proj_kernels.cu:188,194-196).  Deterministic.
 */
CTATTN_API int ctattn_out_proj_bwd(int dtype, const void *c, const void *dy, const void *wo,
                                   void *dwo, void *dbo, void *dc, void *workspace,
                                   int64_t workspace_bytes, int64_t B, int64_t T, int64_t E,
                                   int64_t H, int64_t d, void *stream);

/*
 * params[i] -= lr * grads[i] for i < n.  Replaces runSgdUpdate / sgdUpdateKernel
 * (headers.cu:249-275), which every layer's sgdUpdate calls (AttentionLayer.cu:326-333).
 */
CTATTN_API int ctattn_sgd_update(int dtype, void *params, const void *grads, double lr, int64_t n,
                                 void *stream);

/* ---- Layers around the attention path that a NanoGPT training step needs ----
 *
 * Activations are row-major [rows, features]; ids / targets are int32 device arrays.  Same
 * dtype codes as above: fp32, bf16, fp16 or fp64 storage.  Arithmetic is fp64 for fp64
 * storage and fp32 otherwise, and the "statistic" buffers below (LayerNorm row statistics,
 * losses, Adam moments) hold that type: fp64 for CTATTN_F64, fp32 for every other dtype.
 * Asynchronous on `stream`, 0 or a hipError_t value.
 */

/*
 * Linear layer: y[m][n] = sum_k x[m][k] w[n][k] + b[n] (w is [N][K], b [N] or NULL), on the
 * MFMA GEMMs.  Replaces the linearForward launch of LinearLayer::forward (LinearLayer.cu:55;
 * kernel linear_kernels.cu:36) and of UnEmbedding::forward (Embedding.cu:346).
 */
CTATTN_API int ctattn_linear_fwd(int dtype, const void *x, const void *w, const void *b, void *y,
                                 int64_t M, int64_t N, int64_t K, void *stream);

/* Workspace bytes ctattn_linear_bwd needs (>= 0), or -1 on invalid arguments. */
CTATTN_API int64_t ctattn_linear_bwd_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t K);

/*
 * Backward of the linear layer: dw += dy^T x, db += column sums of dy, dx = dy w
 * (overwritten).  dw, db or dx may be NULL to skip; the workspace is only needed for dw / db.
 * Replaces the linearBackwardWB and linearBackward launches of LinearLayer::backward
 * (LinearLayer.cu:83,95; kernels linear_kernels.cu:115,199) and UnEmbedding::backward
 * (Embedding.cu:378,390).  Deterministic.
 */
CTATTN_API int ctattn_linear_bwd(int dtype, const void *x, const void *w, const void *dy, void *dx,
                                 void *dw, void *db, void *workspace, int64_t workspace_bytes,
                                 int64_t M, int64_t N, int64_t K, void *stream);

/*
 * A linear layer followed by an activation, in one GEMM launch where the MFMA GEMMs take the
 * shape (else the two steps): pre = x w^T + b as ctattn_linear_fwd, y = act(pre) as
 * ctattn_activation_fwd; both written, results equal to those two calls.  No counterpart in
 * the reference, which runs the two kernels (LinearLayer.cu:55 then ActivationLayer.cu:55-64);
 * for the MLP of a transformer block, whose backward needs pre.
 */
CTATTN_API int ctattn_linear_act_fwd(int dtype, int act, const void *x, const void *w, const void *b,
                                     void *pre, void *y, int64_t M, int64_t N, int64_t K, void *stream);

/*
 * Backward of an activation followed by a linear layer: with x [M][K] the linear layer's input
 * (= act(pre)), dw += dy^T x and db += column sums of dy as ctattn_linear_bwd, and
 * dpre[m][k] = act'(pre[m][k]) * sum_n dy[m][n] w[n][k] -- the linear layer's dX and the
 * activation's backward in one GEMM epilogue where the MFMA GEMMs take the shape.  Results equal
 * ctattn_linear_bwd followed by ctattn_activation_bwd; dw / db may be NULL; the workspace is
 * only needed for dw / db (ctattn_linear_bwd_workspace_bytes).  No counterpart in the
 * reference (LinearLayer.cu:83,95 then ActivationLayer.cu:83-92).
 */
CTATTN_API int ctattn_linear_act_bwd(int dtype, int act, const void *x, const void *w, const void *dy,
                                     const void *pre, void *dpre, void *dw, void *db, void *workspace,
                                     int64_t workspace_bytes, int64_t M, int64_t N, int64_t K, void *stream);

/*
 * LayerNorm over the last dimension of x [N][D]: y = (x - mean) * rstd * gamma + beta, with
 * the row statistics written to mean / rstd (statistic type, [N]).  Replaces the
 * layerNormForwardKernel launch of LayerNormLayer::forward (LayerNorm.cu:119; kernel
 * layer_norm_kernels.cu).
 */
CTATTN_API int ctattn_layernorm_fwd(int dtype, const void *x, const void *gamma, const void *beta,
                                    void *y, void *mean, void *rstd, int64_t N, int64_t D,
                                    double eps, void *stream);

/* Workspace bytes ctattn_layernorm_bwd needs for the gamma / beta gradients. */
CTATTN_API int64_t ctattn_layernorm_bwd_workspace_bytes(int dtype, int64_t N, int64_t D);

/*
 * Backward of LayerNorm from the forward's mean / rstd: dx (overwritten), dgamma +=
 * sum_rows dy * xhat, dbeta += sum_rows dy (either may be NULL; deterministic, no atomics).
 * Replaces the layerNormBackwardKernel launch of LayerNormLayer::backward (LayerNorm.cu:143).
 */
CTATTN_API int ctattn_layernorm_bwd(int dtype, const void *x, const void *gamma, const void *dy,
                                    const void *mean, const void *rstd, void *dx, void *dgamma,
                                    void *dbeta, void *workspace, int64_t workspace_bytes,
                                    int64_t N, int64_t D, void *stream);

/* Activation kinds (the reference's ActivationType: ReLU, GELU (tanh form), Sigmoid, Tanh). */
enum ctattn_activation { CTATTN_ACT_RELU = 0, CTATTN_ACT_GELU = 1, CTATTN_ACT_SIGMOID = 2, CTATTN_ACT_TANH = 3 };

/*
 * y = act(x), elementwise over n values (y may be x).  Replaces the four forward launches of
 * ActivationLayer::forward (ActivationLayer.cu:55-64; kernels relu_kernels.cu:26,
 * gelu_kernels.cu:31, sigmoid_kernels.cu:26, tanh_kernels.cu:27).
 */
CTATTN_API int ctattn_activation_fwd(int dtype, int kind, const void *x, void *y, int64_t n,
                                     void *stream);

/*
 * dx = act'(x) * dy, elementwise (dx overwritten; it may be dy).  Replaces the backward launches of
 * ActivationLayer::backward (ActivationLayer.cu:83-92; kernels relu_kernels.cu:62,
 * gelu_kernels.cu:79, sigmoid_kernels.cu:63, tanh_kernels.cu:62).
 */
CTATTN_API int ctattn_activation_bwd(int dtype, int kind, const void *x, const void *dy, void *dx,
                                     int64_t n, void *stream);

/*
 * out[b][t][:] = tok[ids[b][t]][:] + pos[t][:] for ids [B][T] (int32), tok [vocab][E],
 * pos [max_len][E], T <= max_len; an id outside [0, vocab) contributes a zero row.  Either
 * table may be NULL (not both) to look up only the other.
 * Replaces the tokenEmbeddingForwardKernel and positionEmbeddingForwardKernel launches
 * (Embedding.cu:49,200; kernels embedding_kernels.cu:26,64), indexing positions by t (the
 * reference's position kernel uses the flattened row b * T + t).
 */
CTATTN_API int ctattn_embedding_fwd(int dtype, const int32_t *ids, const void *tok, const void *pos,
                                    void *out, int64_t B, int64_t T, int64_t E, int64_t vocab,
                                    int64_t max_len, void *stream);

/*
 * dtok[ids[b][t]][:] += dout[b][t][:] (atomic adds in the storage type: hardware fp32 / fp64
 * atomics, a compare-and-swap per pair of 16-bit values, so bf16 / fp16 need an even E and a
 * 4-byte aligned dtok), dpos[t][:] += sum_b dout[b][t][:] (deterministic); dtok or dpos may
 * be NULL.  Replaces the tokenEmbeddingBackwardKernel and positionEmbeddingBackwardKernel
 * launches (Embedding.cu:82,234; kernels embedding_kernels.cu:98,135).
 */
CTATTN_API int ctattn_embedding_bwd(int dtype, const int32_t *ids, const void *dout, void *dtok,
                                    void *dpos, int64_t B, int64_t T, int64_t E, int64_t vocab,
                                    void *stream);

/*
 * p = softmax(z / temperature) over the last dimension of z [N][V].  Replaces the
 * softmaxKernel launch of Softmax::forward (SoftmaxLoss.cu:42; kernel loss_kernels.cu:29).
 */
CTATTN_API int ctattn_softmax_fwd(int dtype, const void *z, void *p, int64_t N, int64_t V,
                                  double temperature, void *stream);

/*
 * dz = p * (dp - sum_c p dp) / temperature from the forward's output p.  Replaces the
 * softmaxBackwardKernel launch of Softmax::backward (SoftmaxLoss.cu:69; kernel
 * loss_kernels.cu:87), which recomputes p from z.
 */
CTATTN_API int ctattn_softmax_bwd(int dtype, const void *p, const void *dp, void *dz, int64_t N,
                                  int64_t V, double temperature, void *stream);

/*
 * Cross-entropy on probabilities: loss[r] = -log(p[r][target[r]]) / N (statistic type, [N];
 * 0 for a target outside [0, V)), so sum(loss) is the mean loss.  Replaces the
 * crossEntropyLossKernel launch of CrossEntropyLoss::forward (SoftmaxLoss.cu:177; kernel
 * loss_kernels.cu:150), with an output of N rows (the reference allocates shape[0]).
 */
CTATTN_API int ctattn_cross_entropy_fwd(int dtype, const void *p, const int32_t *target, void *loss,
                                        int64_t N, int64_t V, void *stream);

/*
 * dp[r][c] = -1 / (p[r][c] N) at c == target[r], 0 elsewhere.  Replaces the
 * crossEntropyLossBackwardKernel launch of CrossEntropyLoss::backward (SoftmaxLoss.cu:205;
 * kernel loss_kernels.cu:191).
 */
CTATTN_API int ctattn_cross_entropy_bwd(int dtype, const void *p, const int32_t *target, void *dp,
                                        int64_t N, int64_t V, void *stream);

/*
 * The two backward passes above composed: dz = (p - onehot(target)) / (N * temperature), the
 * gradient of the mean cross-entropy of softmax(z / temperature) without the division by p.
 * No counterpart in the reference, which chains CrossEntropyLoss::backward and
 * Softmax::backward (NanoGPT.cu backward); used by NanoGPT training steps.
 */
CTATTN_API int ctattn_softmax_cross_entropy_bwd(int dtype, const void *p, const int32_t *target,
                                                void *dz, int64_t N, int64_t V, double temperature,
                                                void *stream);

/*
 * Mean squared error per row of x, target [N][D]: loss[r] = sum_c (x - target)^2 / D
 * (statistic type, [N]).  Replaces the mseLossKernel launch of MSELoss::forward
 * (SoftmaxLoss.cu:239; kernel loss_kernels.cu:233), with an output of N rows (the reference
 * allocates shape[0]).
 */
CTATTN_API int ctattn_mse_loss_fwd(int dtype, const void *x, const void *target, void *loss,
                                   int64_t N, int64_t D, void *stream);

/*
 * dx = 2 (x - target) / D, elementwise (dx overwritten).  Replaces the mseLossBackwardKernel
 * launch of MSELoss::backward (SoftmaxLoss.cu:267; kernel loss_kernels.cu:267).
 */
CTATTN_API int ctattn_mse_loss_bwd(int dtype, const void *x, const void *target, void *dx,
                                   int64_t N, int64_t D, void *stream);

/*
 * One Adam or AdamW step on n parameters with moments m, v in the statistic type (step >= 1,
 * the 1-based count of this update), c1 = 1 / (1 - b1^step), c2 = 1 / (1 - b2^step):
 *   decoupled = 0 (Adam):  g = grad + weight_decay * param,
 *                          param -= lr * c1 m / (sqrt(c2 v) + eps);
 *   decoupled = 1 (AdamW): g = grad,
 *                          param = param (1 - lr weight_decay) - lr * c1 m / (sqrt(c2 v) + eps);
 * after m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g^2 (m, v keep the uncorrected moments).
 * Replaces the adamUpdateKernel launch of AdamOptimizer::step (AdamOptimizer.cu:90; kernel
 * adam_kernels.cu:25) and the adamWUpdateKernel launch of AdamWOptimizer::step
 * (AdamOptimizer.cu:195).  The reference advances its step counter twice per update and
 * stores the bias-corrected moments back; here the caller passes the step and the moments
 * stay uncorrected.
 */
CTATTN_API int ctattn_adam_update(int dtype, void *param, const void *grad, void *m, void *v,
                                  int64_t n, double lr, double beta1, double beta2, double eps,
                                  double weight_decay, int64_t step, int decoupled, void *stream);

/*
 * ctattn_adam_update over `count` tensors of one dtype in one launch per 32 tensors: tensor i has n[i]
 * elements at param[i], grad[i], m[i], v[i] (host arrays of device pointers; the tables are
 * copied into the launch, so they may be freed on return).  Same arithmetic as
 * ctattn_adam_update.  No counterpart in the reference, whose AdamOptimizer::step launches one
 * adamUpdateKernel per tensor (AdamOptimizer.cu:90); used by the optimizer classes here.
 */
CTATTN_API int ctattn_adam_update_multi(int dtype, int count, void *const *param,
                                        const void *const *grad, void *const *m, void *const *v,
                                        const int64_t *n, double lr, double beta1, double beta2,
                                        double eps, double weight_decay, int64_t step,
                                        int decoupled, void *stream);

/*
 * Zeroes `count` device buffers (bytes[i] bytes at ptr[i], 4-byte aligned; host tables) in one
 * launch per 32 buffers.  No counterpart in the reference (each layer's zeroGrad issues its
 * own cudaMemset, e.g. LinearLayer.cu zeroGrad); used by NanoGPT::zeroGrad here.
 */
CTATTN_API int ctattn_zero_multi(int count, void *const *ptr, const int64_t *bytes, void *stream);

/* ---- Tensor operations behind the Python Tensor classes ----
 *
 * Contiguous row-major device tensors of any ctattn_dtype.  Arithmetic runs in fp32 for
 * bf16 / fp16 storage, fp64 for fp64 and int64 for the integer and bool types, rounded once
 * to the storage type; integer division and remainder by zero give 0.  Asynchronous on
 * `stream`, 0 or a hipError_t value.
 */

/* Element-wise operations: the arithmetic ones write the operand dtype, the comparisons
 * (EQ .. GE) write bool.  MOD is the integer remainder (truncated) and 0 for floating types,
 * as the reference's binaryOpKernel has it (tensor_kernels.cu:245). */
enum ctattn_tensor_op {
    CTATTN_OP_ADD = 0, CTATTN_OP_SUB = 1, CTATTN_OP_MUL = 2, CTATTN_OP_DIV = 3, CTATTN_OP_MOD = 4,
    CTATTN_OP_EQ = 5, CTATTN_OP_NE = 6, CTATTN_OP_LT = 7, CTATTN_OP_LE = 8, CTATTN_OP_GT = 9,
    CTATTN_OP_GE = 10
};
/* Unary maps (the reference's UnaryOp, tensor_kernels.cu:159-190; NEG / NOT of bool are the
 * logical not). */
enum ctattn_unary_op {
    CTATTN_UN_NEG = 0, CTATTN_UN_NOT = 1, CTATTN_UN_INV = 2, CTATTN_UN_EXP = 3, CTATTN_UN_LOG = 4,
    CTATTN_UN_SQR = 5, CTATTN_UN_SQRT = 6, CTATTN_UN_ABS = 7
};
/* Reductions (the reference's ReductionOp, tensor_kernels.cu:537-543). */
enum ctattn_reduce_op {
    CTATTN_RED_SUM = 0, CTATTN_RED_MEAN = 1, CTATTN_RED_MAX = 2, CTATTN_RED_MIN = 3,
    CTATTN_RED_NORM_L1 = 4, CTATTN_RED_NORM_L2 = 5
};

/* dst = src converted element by element (round to nearest even for floating targets,
 * truncation toward zero and wrap-around for integer targets, x != 0 for bool).  Replaces
 * Tensor::to<NewDType> (Tensor.cu:267; castKernel). */
CTATTN_API int ctattn_tensor_cast(int src_dtype, const void *src, int dst_dtype, void *dst, int64_t n,
                                  void *stream);

/* out = a op b with numpy broadcasting of shapes a_shape [a_ndim] and b_shape [b_ndim]
 * (ndim <= 8, aligned at the last dimension); out has the broadcast shape.  Replaces
 * Tensor::binary / Tensor::predicate (Tensor.cu:650-740; binaryOpKernel,
 * binaryPredicateOpKernel). */
CTATTN_API int ctattn_tensor_binary(int dtype, int op, const void *a, int a_ndim, const int64_t *a_shape,
                                    const void *b, int b_ndim, const int64_t *b_shape, void *out,
                                    void *stream);

/* out[i] = a[i] op s (scalar_left = 0) or s op a[i] (scalar_left = 1), s converted to the
 * storage type first.  Replaces the scalar Tensor::binary / predicate (Tensor.cu:742-790). */
CTATTN_API int ctattn_tensor_scalar(int dtype, int op, const void *a, double scalar, int scalar_left,
                                    void *out, int64_t n, void *stream);

/* out = op(a), element-wise.  Replaces Tensor::unary (Tensor.cu:624-637; unaryOpKernel). */
CTATTN_API int ctattn_tensor_unary(int dtype, int op, const void *a, void *out, int64_t n, void *stream);

/* Workspace bytes ctattn_tensor_reduce needs, or -1 on invalid arguments. */
CTATTN_API int64_t ctattn_tensor_reduce_workspace_bytes(int dtype, int64_t outer, int64_t R, int64_t inner);

/* a viewed as [outer][R][inner] reduced over R into out [outer][inner] (R >= 1; outer <= 65535
 * when inner > 1).  Deterministic: a fixed order per output.  Replaces Tensor::reduce
 * (Tensor.cu:807-870; reduceKernel) for one axis or all of them. */
CTATTN_API int ctattn_tensor_reduce(int dtype, int op, const void *a, int64_t outer, int64_t R, int64_t inner,
                                    void *out, void *workspace, int64_t workspace_bytes, void *stream);

/* out = a with its axes permuted: out axis k is input axis perm[k].  Replaces
 * Tensor::transpose (Tensor.cu:577-616; transposeKernel). */
CTATTN_API int ctattn_tensor_permute(int dtype, const void *a, int ndim, const int64_t *shape,
                                     const int32_t *perm, void *out, void *stream);

/* Kronecker product of two tensors of equal rank: out shape a_shape[k] * b_shape[k].
 * Replaces Tensor::kron (Tensor.cu:877-905; kronKernel). */
CTATTN_API int ctattn_tensor_kron(int dtype, const void *a, const void *b, int ndim, const int64_t *a_shape,
                                  const int64_t *b_shape, void *out, void *stream);

/* c[z] = a[z] (M x K) times b[z] (K x N), z < batch, with one b for every z when batch_b == 1.
 * Floating types run on the projection GEMMs, integer and bool types on a per-output kernel.
 * Replaces Tensor::matmul (Tensor.cu:912-950; matmulKernel). */
CTATTN_API int ctattn_tensor_matmul(int dtype, const void *a, const void *b, void *c, int64_t batch,
                                    int64_t batch_b, int64_t M, int64_t K, int64_t N, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* CTATTN_H */
