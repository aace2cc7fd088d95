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
 *     contiguous fp32 [B, H, T] tensor holding LSE_i = m_i + ln(l_i) (natural log).
 *   - the score scale is 1/sqrt(d); causal != 0 masks key j > query i.  causal == 0 is
 *     the reference's behaviour (it has no mask).
 *   - keys past T do not take part in the softmax (no zero padding).
 *   - calls are asynchronous on `stream` (a hipStream_t; NULL = the default stream).
 *     Borrowed pointers must stay valid until the stream has finished with them.
 *   - return 0 on success, otherwise a hipError_t value; ctattn_last_error() then gives a
 *     message (per calling thread).  Argument errors are detected before any launch and
 *     return hipErrorInvalidValue (1); unsupported head dims return
 *     hipErrorNotSupported (801).
 *   - supported: dtype f32 or bf16 (storage; all arithmetic accumulates in fp32),
 *     1 <= d <= 256, T >= 0, B, H >= 0.  d in {32, 64, 128} run on the MFMA
 *     kernels; other d on a generic kernel.
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

enum ctattn_dtype { CTATTN_F32 = 0, CTATTN_BF16 = 1 };

/* Kernel selection policy (process-wide).
 *   AUTO           MFMA kernels where they apply (fastest).  The MFMA backward adds dQ
 *                  contributions of different key blocks with fp32 atomics, so dQ may
 *                  differ between runs in the last bits; dK, dV, O and LSE do not.
 *   GENERIC        the generic kernels only (used to cross-check the two paths).
 *   DETERMINISTIC  MFMA kernels, with dQ summed over key blocks in a fixed order through a
 *                  workspace buffer: bitwise-reproducible gradients, larger workspace. */
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
 * (flash_attention.cu:164-167); this boundary writes the single fp32 LSE instead.
 * lse may be NULL when the caller does not keep state for a backward.
 */
CTATTN_API int ctattn_fwd(int dtype, const void *q, const void *k, const void *v, void *o, float *lse,
               int64_t B, int64_t H, int64_t T, int64_t d, int causal, void *stream);

/*
 * Bytes of device workspace ctattn_bwd needs for this problem (>= 0), or -1 on invalid
 * arguments.  Replaces nothing in the reference: its backward zero-fills and atomically
 * accumulates straight into dq/dk/dv (FlashAttentionLayer.cu:103-106, flash_attention.cu:317-321).
 */
CTATTN_API int64_t ctattn_bwd_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t T, int64_t d,
                                   int causal);

/*
 * Backward: dQ, dK, dV given Q, K, V, the forward's O and LSE, and dO.
 * Replaces the flashAttentionBackward<DType> launch of FlashAttentionLayer::computeBackward
 * (reference FlashAttentionLayer.cu:129-140; kernel flash_attention.cu:226-326).
 * dq, dk, dv are fully overwritten (no pre-zeroing needed).  workspace must hold at least
 * ctattn_bwd_workspace_bytes(...) bytes, queried under the same policy.  Reproducibility
 * depends on the policy (see enum ctattn_policy).
 */
CTATTN_API int ctattn_bwd(int dtype, const void *q, const void *k, const void *v, const void *o,
               const void *dout, const float *lse, void *dq, void *dk, void *dv,
               void *workspace, int64_t workspace_bytes, int64_t B, int64_t H, int64_t T,
               int64_t d, int causal, void *stream);

/* Message describing the last failure of a ctattn_* call on this thread ("" if none). */
CTATTN_API const char *ctattn_last_error(void);

/* Set / get the process-wide kernel selection policy (enum ctattn_policy).  Returns the
 * previous policy, or -1 for an unknown value.  Not synchronised with calls in flight on
 * other threads: set it before issuing work. */
CTATTN_API int ctattn_set_policy(int policy);
CTATTN_API int ctattn_get_policy(void);

/* Library version, major * 10000 + minor * 100 + patch. */
CTATTN_API int ctattn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CTATTN_H */
