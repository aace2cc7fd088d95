// Internal launcher interface between the C-ABI layer (ctattn_capi.hip) and the kernel
// translation units.  Every launcher validates nothing (the C-ABI layer already did),
// enqueues on `stream` and returns hipGetLastError() of its launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ctattn {

struct AttnShape {
    int64_t B, H, T, d;
    bool causal;
    // Head dim whose 1 / sqrt scales the scores: d itself, unless the tensors are copies
    // zero-padded from a smaller head dim (scale_d), whose scale the kernels must keep.
    int64_t scale_d = 0;
    int64_t bh() const { return B * H; }
    int64_t rows() const { return B * H * T; }
    int64_t scale_dim() const { return scale_d > 0 ? scale_d : d; }
};

// A launch may hold at most 2^32 - 1 work-items (gridDim.x * blockDim.x) and 2^31 - 1
// workgroups.  Fixed-shape kernels check their grid with grid_fits and refuse larger
// problems; grid-stride kernels (generic attention, preprocess, reductions) cap their grid
// with stride_grid and loop.
inline bool grid_fits(int64_t blocks, int threads) {
    return blocks >= 0 && blocks <= 0x7FFFFFFFll && blocks * threads <= 0xFFFFFFFFll;
}
inline unsigned stride_grid(int64_t blocks, int threads) {
    const int64_t cap = (int64_t(1) << 30) / threads;  // 2^30 work-items: fills the chip many times over
    return unsigned(blocks < 1 ? 1 : (blocks < cap ? blocks : cap));
}

// ---- generic kernels: any 1 <= d <= 256; dtype 0 fp32, 1 bf16, 2 fp16, 3 fp64.  lse and
// delta are fp64 for dtype 3 and fp32 otherwise. ----
hipError_t launch_generic_fwd(int dtype, const void *q, const void *k, const void *v, void *o,
                              void *lse, const AttnShape &s, hipStream_t stream);
hipError_t launch_generic_bwd(int dtype, const void *q, const void *k, const void *v,
                              const void *o, const void *dout, const void *lse, void *dq,
                              void *dk, void *dv, void *delta, const AttnShape &s,
                              hipStream_t stream);

// ---- shared backward preprocess: delta[row] = sum_c dO[row][c] * O[row][c] ----
hipError_t launch_bwd_preprocess(int dtype, const void *o, const void *dout, void *delta,
                                 const AttnShape &s, hipStream_t stream);

// ---- MFMA kernels (fp32, bf16 and fp16: d in {32, 64, 128}) ----
bool mfma_fwd_supported(int dtype, int64_t d);
bool mfma_bwd_supported(int dtype, int64_t d);
hipError_t launch_mfma_fwd(int dtype, const void *q, const void *k, const void *v, void *o,
                           float *lse, const AttnShape &s, hipStream_t stream);
// bf16 forward on bf16 MFMA (d in {32, 64, 128}); called by launch_mfma_fwd for dtype 1.
hipError_t launch_bf16_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                           const AttnShape &s, hipStream_t stream);
// bf16 backward on bf16 MFMA (d in {32, 64, 128}); called by launch_mfma_bwd for dtype 1.
// Scratch: -LSE log2(e) per row, [B, H, T] fp32 (256-byte aligned size), then at d = 128,
// with_ds, the bf16 dS tiles (bf16_ds_bytes: causal about B H T^2 bytes, at most 4 GiB, 0
// beyond).  Given a scratch of extra_bytes, the launch stores and reuses dS when it fits and
// recomputes S and dP in the dQ kernel otherwise.
int64_t bf16_ds_bytes(const AttnShape &s);
int64_t bf16_bwd_workspace_bytes(const AttnShape &s, bool deterministic, bool with_ds);
// fp16 forward / backward: the bf16 kernels instantiated for IEEE fp16 (fp16 MFMA), same
// workspace as bf16.
hipError_t launch_f16_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                          const AttnShape &s, hipStream_t stream);
hipError_t launch_f16_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
                          const float *lse, float *delta, void *dq, void *dk, void *dv, void *extra,
                          int64_t extra_bytes, const AttnShape &s, hipStream_t stream);
hipError_t launch_bf16_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
                           const float *lse, float *delta, void *dq, void *dk, void *dv, void *extra,
                           int64_t extra_bytes, bool deterministic, const AttnShape &s, hipStream_t stream);
// fp32 dS tiles (d in {64, 128}): 16 KB per pair of 64-row query and 64-key blocks of the mask,
// at most 4 GiB (0 beyond).  Given that much scratch, the fp32 backward stores dS from its
// key-major kernel and computes dQ query-major from it, without atomics: under DETERMINISTIC,
// and under AUTO at d = 128 on grids of at least 1024 key blocks (f32_ds_wanted).
int64_t f32_ds_bytes(const AttnShape &s);
bool f32_ds_wanted(const AttnShape &s, bool deterministic);
// Scratch of launch_mfma_bwd beyond delta; with_ds = false gives the smallest that works (the
// bf16 / fp16 / fp32 dS tiles left out).
int64_t mfma_bwd_workspace_bytes(int dtype, const AttnShape &s, bool deterministic, bool with_ds = true);
// ---- fp64 kernels on fp64 MFMA (attn_f64_mfma.hip), d in {32, 64, 128}; lse and delta fp64.
// The backward runs its own preprocess into `delta` ([B, H, T] fp64) and needs no other
// scratch; dq, dk, dv are written, not accumulated. ----
bool f64_mfma_supported(int64_t d);
hipError_t launch_f64_fwd(const void *q, const void *k, const void *v, void *o, void *lse, const AttnShape &s,
                          hipStream_t stream);
hipError_t launch_f64_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
                          const void *lse, void *delta, void *dq, void *dk, void *dv, const AttnShape &s,
                          hipStream_t stream);
// Compute units of the device that owns `stream` (the current device for the null stream),
// cached per device; 0 if it cannot be queried.
int device_cus(hipStream_t stream);
// fp32 backward main kernel with 128-key workgroups (attn_bwd_k128.hip), d in {32, 64, 128}:
// dK and dV, plus dQ accumulated into dq with atomics (Atomic: dq pre-zeroed), stored as
// per-128-key-block partials in dq_part (Partial: plane kb holds key block kb's share), or
// not at all (None).  delta must already hold rowsum(dO * O).  split: every key block's query
// rows are shared by two workgroups, each adding its dK / dV share to dk / dv (pre-zeroed)
// with one atomic add per element -- two addends, so the sum is the same in either order.
enum class K128Dq { Atomic, Partial, None };
hipError_t launch_bwd_f32_k128(const float *q, const float *k, const float *v, const float *dout,
                               const float *lse, const float *delta, float *dq, float *dq_part, float *dk, float *dv,
                               K128Dq mode, bool split, const AttnShape &s, hipStream_t stream);
// Whether the fp32 backward's key-major grid is short enough (no more workgroups than the chip
// holds at once: two per CU at d <= 64, one at d = 128) to split every key block's rows in two.
bool bwd_f32_use_split(const AttnShape &s, bool k64, hipStream_t stream);
// fp32 dQ, query-major and atomic-free (attn_bwd_dq_f32.hip), d in {32, 64, 128}: dq is
// written, not accumulated; delta must already hold rowsum(dO * O).
hipError_t launch_bwd_dq_f32(const float *q, const float *k, const float *v, const float *dout, const float *lse,
                             const float *delta, float *dq, const AttnShape &s, hipStream_t stream);
// Row copies for head dims without an MFMA kernel of their own (attn_pad.hip): pad copies
// each of `count` (<= kMaxRowCopies) [rows][d] tensors in[i] into a [rows][dp] buffer out[i]
// with columns d .. dp - 1 zero, unpad copies the d leading columns of each [rows][dp] buffer
// in[i] into the [rows][d] tensor out[i]; elem_bytes is the storage element size (2, 4, 8).
// One bandwidth-bound launch on `stream` per call.
constexpr int kMaxRowCopies = 5;
hipError_t launch_pad_rows(int elem_bytes, const void *const *in, void *const *out, int count, int64_t rows, int d,
                           int dp, hipStream_t stream);
hipError_t launch_unpad_rows(int elem_bytes, const void *const *in, void *const *out, int count, int64_t rows,
                             int d, int dp, hipStream_t stream);
// Runs the whole MFMA backward: its own preprocess (delta = rowsum(dO * O) into `delta`,
// fp32 [B, H, T]) and the main kernel(s).  `extra` points at mfma_bwd_workspace_bytes()
// bytes of scratch (256-byte aligned).  `deterministic` (fp32): no atomics -- dQ from
// per-key-block partials summed in a fixed order (up to 8 blocks of 128 keys) or from the
// query-major kernel, dK / dV from the 128-key kernel (bitwise reproducible).
hipError_t launch_mfma_bwd(int dtype, const void *q, const void *k, const void *v,
                           const void *o, const void *dout, const float *lse, float *delta,
                           void *dq, void *dk, void *dv, void *extra, int64_t extra_bytes,
                           bool deterministic, const AttnShape &s, hipStream_t stream);

}  // namespace ctattn
