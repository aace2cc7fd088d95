// Kernels and C-ABI entry points of the layers around the attention path that a NanoGPT
// training step needs (declared in include/ctattn.h): LayerNorm, the elementwise
// activations, token + position embeddings, softmax with temperature, cross-entropy on
// probabilities, mean squared error, and the Adam update.  The linear layers run on the
// projection GEMM family (proj_capi.hip).
//
// These replace the reference's per-layer kernels (layer_norm_kernels.cu, relu_/gelu_/
// sigmoid_/tanh_kernels.cu, embedding_kernels.cu, loss_kernels.cu, adam_kernels.cu) with
// the same math, with these deliberate differences:
//   * LayerNorm keeps its row statistics in buffers the caller owns and sums the gamma /
//     beta gradients deterministically (two-stage column sums, no atomics; the reference
//     atomically adds every row, layer_norm_kernels.cu backward);
//   * one wave per row (64 lanes) for the row-wise kernels instead of one thread per row
//     (loss_kernels.cu: softmaxKernel walks a whole row in one thread);
//   * ids / targets outside [0, vocab) read nothing: an embedding row of zeros and a zero
//     loss (the reference checks targets, loss_kernels.cu, but not embedding ids);
//   * the position embedding is indexed by the position t of each row, not by the flattened
//     b * T + t (out of bounds for B > 1 in embedding_kernels.cu);
//   * Adam / AdamW are the textbook updates, the step counter advanced once per step by the
//     caller (the reference increments it twice per step, AdamOptimizer.cu:75,95, and stores
//     the bias-corrected moments back, adam_kernels.cu adamUpdateKernel).
// Storage is fp32, bf16, fp16 or fp64.  Arithmetic is in the storage type's accumulation
// type (the reference's ComputeType, headers.cu:47-48): fp64 for fp64 storage, fp32
// otherwise; row statistics, losses and Adam moments are kept in that type too.
#include "act_math.h"
#include "attn_common.h"
#include "capi_util.h"
#include "ctattn.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace ctattn {
namespace {

template <typename T> __device__ __forceinline__ acc_t<T> ld(const T *p, int64_t i) { return to_acc(p[i]); }
// Stores round the fp32 (fp64) value to the storage type as computed: for fp16 the empty asm
// keeps the backend from folding the last multiply or add and the conversion into one
// mixed-precision FMA, which rounds once and would make the result depend on which kernel
// computed it (the fused LayerNorm / activation paths must equal the separate ones).
template <typename T> __device__ __forceinline__ void st(T *p, int64_t i, acc_t<T> x) {
    if constexpr (std::is_same_v<T, f16_t>) asm volatile("" : "+v"(x));
    p[i] = from_acc<T>(x);
}

// ---------------------------------------------------------------------------------------
// LayerNorm over the last dimension (layer_norm_kernels.cu): y = (x - mean) rstd g + b.
// One wave per row.
// ---------------------------------------------------------------------------------------
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void layernorm_fwd_kernel(const T *__restrict__ x, const T *__restrict__ g,
                                                           const T *__restrict__ b, T *__restrict__ y,
                                                           A *__restrict__ mean_out, A *__restrict__ rstd_out,
                                                           int64_t N, int D, A eps) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= N) return;
    const T *xr = x + row * D;
    A s = 0;
    for (int c = lane; c < D; c += kWave) s += ld(xr, c);
    const A mean = wave_sum(s) / A(D);
    A v = 0;
    for (int c = lane; c < D; c += kWave) {
        const A dx = ld(xr, c) - mean;
        v += dx * dx;
    }
    const A rstd = A(1) / acc_sqrt(wave_sum(v) / A(D) + eps);
    T *yr = y + row * D;
    for (int c = lane; c < D; c += kWave) st(yr, c, (ld(xr, c) - mean) * rstd * ld(g, c) + ld(b, c));
    if (lane == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
}

// dx = rstd (dxhat - mean(dxhat) - xhat mean(dxhat xhat)), dxhat = dy g.  One wave per row.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void layernorm_bwd_dx_kernel(const T *__restrict__ x, const T *__restrict__ g,
                                                              const T *__restrict__ dy, const A *__restrict__ mean,
                                                              const A *__restrict__ rstd, T *__restrict__ dx,
                                                              int64_t N, int D) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= N) return;
    const T *xr = x + row * D;
    const T *dyr = dy + row * D;
    const A mu = mean[row], rs = rstd[row];
    A s1 = 0, s2 = 0;
    for (int c = lane; c < D; c += kWave) {
        const A xh = (ld(xr, c) - mu) * rs;
        const A dxh = ld(dyr, c) * ld(g, c);
        s1 += dxh;
        s2 += dxh * xh;
    }
    const A m1 = wave_sum(s1) / A(D), m2 = wave_sum(s2) / A(D);
    T *dxr = dx + row * D;
    for (int c = lane; c < D; c += kWave) {
        const A xh = (ld(xr, c) - mu) * rs;
        st(dxr, c, rs * (ld(dyr, c) * ld(g, c) - m1 - xh * m2));
    }
}

constexpr int kLnRowsPerChunk = 32;

// Stage 1 of the gamma / beta gradients: part[chunk][c] = sum over the chunk's rows of
// dy * xhat (first D values) and dy (next D values).  256 threads = 64 columns x 4 row lanes
// (8 rows each), combined in LDS in a fixed order.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void layernorm_bwd_part_kernel(const T *__restrict__ x, const T *__restrict__ dy,
                                                                const A *__restrict__ mean,
                                                                const A *__restrict__ rstd,
                                                                A *__restrict__ part, int64_t N, int D) {
    __shared__ A red[2][4][64];
    const int cl = threadIdx.x & 63, rl = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl;
    const int64_t chunk = blockIdx.y;
    const int64_t r0 = chunk * kLnRowsPerChunk;
    A sg = 0, sb = 0;
    if (c < D) {
#pragma unroll
        for (int i = 0; i < kLnRowsPerChunk / 4; ++i) {
            const int64_t r = r0 + rl + 4 * i;
            if (r < N) {
                const A d = ld(dy, r * D + c);
                sg += d * (ld(x, r * D + c) - mean[r]) * rstd[r];
                sb += d;
            }
        }
    }
    red[0][rl][cl] = sg;
    red[1][rl][cl] = sb;
    __syncthreads();
    if (rl == 0 && c < D) {
        part[chunk * 2 * D + c] = ((red[0][0][cl] + red[0][1][cl]) + red[0][2][cl]) + red[0][3][cl];
        part[chunk * 2 * D + D + c] = ((red[1][0][cl] + red[1][1][cl]) + red[1][2][cl]) + red[1][3][cl];
    }
}

// dx and the stage-1 gamma / beta partial sums of one 32-row chunk in one pass over x and dy
// (D <= 64 CPL): wave w takes rows w, w + 4, ..., w + 28 of the chunk -- the rows lane w of the
// stage-1 kernel sums -- computing each row's dx as layernorm_bwd_dx_kernel does and keeping
// the partial sums of its columns c = lane + 64 j in registers in the same row order; the four
// waves' sums are combined in LDS in the stage-1 kernel's order, so both paths give the same
// bits.  The loads of RB rows are issued before any of them is used.
template <typename T, int CPL, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void layernorm_bwd_fused_kernel(const T *__restrict__ x, const T *__restrict__ g,
                                                                 const T *__restrict__ dy, const A *__restrict__ mean,
                                                                 const A *__restrict__ rstd, T *__restrict__ dx,
                                                                 A *__restrict__ part, int64_t N, int D) {
    constexpr int RB = CPL <= 6 ? 8 : CPL <= 8 ? 4 : 2;  // rows loaded ahead
    __shared__ A red[2][4][64 * CPL];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int64_t r0 = int64_t(blockIdx.x) * kLnRowsPerChunk;
    A sg[CPL], sb[CPL], gv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        sg[j] = sb[j] = A(0);
        gv[j] = lane + 64 * j < D ? ld(g, lane + 64 * j) : A(0);
    }
#pragma unroll
    for (int i0 = 0; i0 < kLnRowsPerChunk / 4; i0 += RB) {
        A xv[RB][CPL], dv[RB][CPL];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int64_t r = r0 + w + 4 * (i0 + i);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                const bool in = r < N && c < D;
                xv[i][j] = in ? ld(x, r * D + c) : A(0);
                dv[i][j] = in ? ld(dy, r * D + c) : A(0);
            }
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int64_t r = r0 + w + 4 * (i0 + i);
            if (r >= N) break;  // wave-uniform
            const A mu = mean[r], rs = rstd[r];
            A s1 = 0, s2 = 0;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if (lane + 64 * j >= D) continue;
                sg[j] += dv[i][j] * (xv[i][j] - mu) * rs;
                sb[j] += dv[i][j];
                const A xh = (xv[i][j] - mu) * rs;
                const A dxh = dv[i][j] * gv[j];
                s1 += dxh;
                s2 += dxh * xh;
            }
            const A m1 = wave_sum(s1) / A(D), m2 = wave_sum(s2) / A(D);
            T *dxr = dx + r * D;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                if (c >= D) continue;
                const A xh = (xv[i][j] - mu) * rs;
                st(dxr, c, rs * (dv[i][j] * gv[j] - m1 - xh * m2));
            }
        }
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        red[0][w][lane + 64 * j] = sg[j];
        red[1][w][lane + 64 * j] = sb[j];
    }
    __syncthreads();
    A *pc = part + int64_t(blockIdx.x) * 2 * D;
    for (int c = threadIdx.x; c < D; c += 256) {
        pc[c] = ((red[0][0][c] + red[0][1][c]) + red[0][2][c]) + red[0][3][c];
        pc[D + c] = ((red[1][0][c] + red[1][1][c]) + red[1][2][c]) + red[1][3][c];
    }
}

// Stage 2: dgamma[c] += sum_chunk part[chunk][c], dbeta likewise.  16 columns x 16 lanes per
// block; lane l takes chunks l, l+16, ... in increasing order, then lane 0 adds the 16 lane
// sums in order.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void layernorm_bwd_reduce_kernel(const A *__restrict__ part, T *__restrict__ dg,
                                                                  T *__restrict__ db, int64_t chunks, int D) {
    __shared__ A red[2][16][17];
    const int cl = threadIdx.x & 15, rl = threadIdx.x >> 4;
    const int c = blockIdx.x * 16 + cl;
    A sg = 0, sb = 0;
    if (c < D) {
        for (int64_t k = rl; k < chunks; k += 16) {
            sg += part[k * 2 * D + c];
            sb += part[k * 2 * D + D + c];
        }
    }
    red[0][rl][cl] = sg;
    red[1][rl][cl] = sb;
    __syncthreads();
    if (rl != 0 || c >= D) return;
    sg = 0;
    sb = 0;
#pragma unroll
    for (int l = 0; l < 16; ++l) {
        sg += red[0][l][cl];
        sb += red[1][l][cl];
    }
    if (dg != nullptr) st(dg, c, ld(dg, c) + sg);
    if (db != nullptr) st(db, c, ld(db, c) + sb);
}

// ---------------------------------------------------------------------------------------
// Activations (relu_/gelu_/sigmoid_/tanh_kernels.cu), elementwise.
// ---------------------------------------------------------------------------------------
// act_fwd / act_grad: act_math.h (shared with the GEMM epilogues that fuse them).

// Elementwise with each element read before it is written: y may alias x, dx may alias dy.
template <typename T>
__global__ __launch_bounds__(256) void act_fwd_kernel(int kind, const T *x, T *y, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
        st(y, i, act_fwd(kind, ld(x, i)));
}

template <typename T>
__global__ __launch_bounds__(256) void act_bwd_kernel(int kind, const T *x, const T *dy, T *dx, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
        st(dx, i, act_bwd_value(kind, ld(x, i), ld(dy, i)));
}

// ---------------------------------------------------------------------------------------
// Token + position embedding (embedding_kernels.cu).
// ---------------------------------------------------------------------------------------
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void embedding_fwd_kernel(const int32_t *__restrict__ ids, const T *__restrict__ tok,
                                                           const T *__restrict__ pos, T *__restrict__ out, int64_t rows,
                                                           int T_, int E, int64_t vocab) {
    const int64_t n = rows * E;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t r = i / E;
        const int e = int(i - r * E);
        const int t = int(r % T_);
        A v = pos != nullptr ? ld(pos, int64_t(t) * E + e) : A(0);
        if (tok != nullptr) {
            const int64_t id = ids[r];
            if (id >= 0 && id < vocab) v += ld(tok, id * E + e);
        }
        st(out, i, v);
    }
}

// Atomic adds into the token-gradient table: hardware float / double atomics; a pair of
// 16-bit values (one aligned 32-bit word) by compare-and-swap, each half rounded to nearest
// even after its add.
__device__ __forceinline__ void atomic_add(float *p, float x) { unsafeAtomicAdd(p, x); }
__device__ __forceinline__ void atomic_add(double *p, double x) { unsafeAtomicAdd(p, x); }
template <typename H> __device__ __forceinline__ void atomic_add_pair(H *p, float lo, float hi) {
    uint32_t *w = reinterpret_cast<uint32_t *>(p);
    uint32_t old = *w, assumed;
    do {
        assumed = old;
        const uint16_t nlo = from_f32<H>(to_f32(H{uint16_t(assumed & 0xffffu)}) + lo).bits;
        const uint16_t nhi = from_f32<H>(to_f32(H{uint16_t(assumed >> 16)}) + hi).bits;
        old = atomicCAS(w, assumed, uint32_t(nlo) | (uint32_t(nhi) << 16));
    } while (old != assumed);
}

// dtok[ids[r]][e] += dout[r][e].  fp32 / fp64: one element per thread.  16-bit: one pair of
// columns (e, e + 1) per thread; E is even and the table 4-byte aligned (checked on the host),
// so each pair is one aligned word inside the table.
template <typename T>
__global__ __launch_bounds__(256) void embedding_bwd_tok_kernel(const int32_t *__restrict__ ids,
                                                               const T *__restrict__ dout, T *__restrict__ dtok,
                                                               int64_t rows, int E, int64_t vocab) {
    if constexpr (sizeof(T) >= 4) {
        const int64_t n = rows * E;
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
            const int64_t r = i / E;
            const int64_t id = ids[r];
            if (id >= 0 && id < vocab) atomic_add(dtok + id * E + (i - r * E), dout[i]);
        }
    } else {
        const int half = E / 2;
        const int64_t n = rows * half;
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
            const int64_t r = i / half;
            const int e = 2 * int(i - r * half);
            const int64_t id = ids[r];
            if (id >= 0 && id < vocab)
                atomic_add_pair(dtok + id * E + e, to_f32(dout[r * E + e]), to_f32(dout[r * E + e + 1]));
        }
    }
}

// dpos[t][e] += sum_b dout[b][t][e]: one thread per (t, e), fixed order over b.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void embedding_bwd_pos_kernel(const T *__restrict__ dout, T *__restrict__ dpos,
                                                               int64_t B, int T_, int E) {
    const int64_t n = int64_t(T_) * E;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        A s = 0;
        for (int64_t b = 0; b < B; ++b) s += ld(dout, b * n + i);
        st(dpos, i, ld(dpos, i) + s);
    }
}

// ---------------------------------------------------------------------------------------
// Softmax with temperature, cross-entropy, mean squared error (loss_kernels.cu).  One wave
// per row for the row reductions.
// ---------------------------------------------------------------------------------------
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void softmax_fwd_kernel(const T *__restrict__ z, T *__restrict__ p, int64_t N, int V,
                                                         A inv_temp) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= N) return;
    const T *zr = z + row * V;
    A m = -INFINITY;
    for (int c = lane; c < V; c += kWave) m = fmax(m, ld(zr, c));
    m = wave_max(m);
    A s = 0;
    for (int c = lane; c < V; c += kWave) s += acc_exp((ld(zr, c) - m) * inv_temp);
    const A inv_s = A(1) / wave_sum(s);
    T *pr = p + row * V;
    for (int c = lane; c < V; c += kWave) st(pr, c, acc_exp((ld(zr, c) - m) * inv_temp) * inv_s);
}

// dz = p (dp - sum_c p dp) / temperature (softmaxBackwardKernel's formula, from p).
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void softmax_bwd_kernel(const T *__restrict__ p, const T *__restrict__ dp,
                                                         T *__restrict__ dz, int64_t N, int V, A inv_temp) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= N) return;
    const T *pr = p + row * V;
    const T *dpr = dp + row * V;
    A s = 0;
    for (int c = lane; c < V; c += kWave) s += ld(pr, c) * ld(dpr, c);
    s = wave_sum(s);
    T *dzr = dz + row * V;
    for (int c = lane; c < V; c += kWave) st(dzr, c, ld(pr, c) * (ld(dpr, c) - s) * inv_temp);
}

// loss[r] = -log(p[r][target[r]]) / N (0 for a target outside [0, V)).  One thread per row.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void xent_fwd_kernel(const T *__restrict__ p, const int32_t *__restrict__ tgt,
                                                      A *__restrict__ loss, int64_t N, int V) {
    const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= N) return;
    const int t = tgt[r];
    loss[r] = (t >= 0 && t < V) ? -acc_log(ld(p, r * V + t)) / A(N) : A(0);
}

// dp[r][c] = -1 / (p N) at the target, 0 elsewhere (crossEntropyLossBackwardKernel).
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void xent_bwd_kernel(const T *__restrict__ p, const int32_t *__restrict__ tgt,
                                                      T *__restrict__ dp, int64_t N, int V) {
    const int64_t n = N * V;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t r = i / V;
        const int c = int(i - r * V);
        st(dp, i, c == tgt[r] ? A(-1) / (ld(p, i) * A(N)) : A(0));
    }
}

// The two above composed with the softmax backward: dz = (p - onehot(target)) / (N T), the
// same gradient without dividing by p.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void softmax_xent_bwd_kernel(const T *__restrict__ p, const int32_t *__restrict__ tgt,
                                                              T *__restrict__ dz, int64_t N, int V, A scale) {
    const int64_t n = N * V;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t r = i / V;
        const int c = int(i - r * V);
        const int t = tgt[r];
        const A onehot = c == t ? A(1) : A(0);
        st(dz, i, (t >= 0 && t < V) ? (ld(p, i) - onehot) * scale : A(0));
    }
}

// loss[r] = sum_c (x[r][c] - y[r][c])^2 / D (mseLossKernel, loss_kernels.cu).  One wave per row.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void mse_fwd_kernel(const T *__restrict__ x, const T *__restrict__ y,
                                                     A *__restrict__ loss, int64_t N, int D) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= N) return;
    A s = 0;
    for (int c = lane; c < D; c += kWave) {
        const A d = ld(x, row * D + c) - ld(y, row * D + c);
        s += d * d;
    }
    s = wave_sum(s);
    if (lane == 0) loss[row] = s / A(D);
}

// dx = 2 (x - y) / D (mseLossBackwardKernel).
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void mse_bwd_kernel(const T *__restrict__ x, const T *__restrict__ y,
                                                     T *__restrict__ dx, int64_t n, int D) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
        st(dx, i, A(2) * (ld(x, i) - ld(y, i)) / A(D));
}

// ---------------------------------------------------------------------------------------
// Adam / AdamW (adam_kernels.cu:25 adamUpdateKernel, adamWUpdateKernel), textbook
// bias-corrected form.  Adam folds the weight decay into the gradient (g + decay p, as
// adamUpdateKernel does); AdamW decays the parameter itself, p (1 - lr decay) - lr update
// (adamWUpdateKernel).  m and v keep the uncorrected moments (the reference stores the
// bias-corrected ones back, so its correction compounds from step to step), in the
// accumulation type.
// ---------------------------------------------------------------------------------------
template <typename A> struct AdamHyper {
    A lr, b1, b2, eps, decay, c1, c2;
    int decoupled;
};

typedef float adam_f4 __attribute__((ext_vector_type(4)));

// One element's update from its loaded values: p (parameter), gr (gradient), mo / vo (moments);
// returns the new parameter and writes the new moments.
template <typename A>
__device__ __forceinline__ A adam_math(A p, A gr, A mo, A vo, A &mi, A &vi, const AdamHyper<A> &h) {
    const A g = h.decoupled ? gr : gr + h.decay * p;
    mi = h.b1 * mo + (A(1) - h.b1) * g;
    vi = h.b2 * vo + (A(1) - h.b2) * g * g;
    const A upd = h.lr * (mi * h.c1) / (acc_sqrt(vi * h.c2) + h.eps);
    return h.decoupled ? p * (A(1) - h.lr * h.decay) - upd : p - upd;
}

template <typename T, typename A>
__device__ __forceinline__ void adam_elem(T *param, const T *grad, A *m, A *v, int64_t i, const AdamHyper<A> &h) {
    A mi, vi;
    const A pn = adam_math(ld(param, i), ld(grad, i), m[i], v[i], mi, vi, h);
    m[i] = mi;
    v[i] = vi;
    st(param, i, pn);
}

template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void adam_kernel(T *__restrict__ param, const T *__restrict__ grad,
                                                  A *__restrict__ m, A *__restrict__ v, int64_t n, AdamHyper<A> h) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
        adam_elem(param, grad, m, v, i, h);
}

// Multi-tensor launches: up to kMultiMax tensors per launch, described in the kernel
// arguments (no device-side table).  Each workgroup takes one kMultiChunk-element chunk of one
// tensor; chunk_begin[i] is the first chunk of tensor i (chunk_begin[count] = total).
constexpr int kMultiMax = 32;
constexpr int kMultiChunk = 4096;  // elements per workgroup: 256 threads x 16

struct AdamMulti {
    void *param[kMultiMax];
    const void *grad[kMultiMax];
    void *m[kMultiMax];
    void *v[kMultiMax];
    int64_t n[kMultiMax];
    int32_t chunk_begin[kMultiMax + 1];
    int32_t count;
};

struct ZeroMulti {
    void *p[kMultiMax];
    int64_t bytes[kMultiMax];
    int32_t chunk_begin[kMultiMax + 1];  // chunks of kMultiChunk * 4 bytes
    int32_t count;
};

// Tensor owning chunk `b` (a uniform linear scan over at most kMultiMax entries).
__device__ __forceinline__ int multi_owner(const int32_t *chunk_begin, int count, int b) {
    int t = 0;
    while (t + 1 < count && chunk_begin[t + 1] <= b) ++t;
    return t;
}

template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void adam_multi_kernel(AdamMulti a, AdamHyper<A> h) {
    const int t = multi_owner(a.chunk_begin, a.count, int(blockIdx.x));
    const int64_t base = int64_t(blockIdx.x - a.chunk_begin[t]) * kMultiChunk;
    const int64_t end = min(a.n[t], base + kMultiChunk);
    T *__restrict__ param = static_cast<T *>(a.param[t]);
    const T *__restrict__ grad = static_cast<const T *>(a.grad[t]);
    A *__restrict__ m = static_cast<A *>(a.m[t]);
    A *__restrict__ v = static_cast<A *>(a.v[t]);
    if constexpr (std::is_same_v<T, float>) {
        // fp32 tensors with 16-byte aligned bases (chunks are 4096 elements): four consecutive
        // elements per thread in 16-byte accesses, the gradient (read once, never written)
        // non-temporal; the same per-element arithmetic as adam_elem.
        if (((uintptr_t(param) | uintptr_t(grad) | uintptr_t(m) | uintptr_t(v)) & 15) == 0) {
            const int64_t n4 = (end - base) / 4;
            for (int64_t q = threadIdx.x; q < n4; q += blockDim.x) {
                const int64_t i = base + 4 * q;
                const adam_f4 p4 = *reinterpret_cast<const adam_f4 *>(param + i);
                const adam_f4 g4 = __builtin_nontemporal_load(reinterpret_cast<const adam_f4 *>(grad + i));
                const adam_f4 m4 = *reinterpret_cast<const adam_f4 *>(m + i);
                const adam_f4 v4 = *reinterpret_cast<const adam_f4 *>(v + i);
                adam_f4 pn, mn, vn;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float me, ve;
                    pn[e] = adam_math(p4[e], g4[e], m4[e], v4[e], me, ve, h);
                    mn[e] = me;
                    vn[e] = ve;
                }
                *reinterpret_cast<adam_f4 *>(m + i) = mn;
                *reinterpret_cast<adam_f4 *>(v + i) = vn;
                *reinterpret_cast<adam_f4 *>(param + i) = pn;
            }
            for (int64_t i = base + 4 * n4 + threadIdx.x; i < end; i += blockDim.x) adam_elem(param, grad, m, v, i, h);
            return;
        }
    }
    for (int64_t i = base + threadIdx.x; i < end; i += blockDim.x) adam_elem(param, grad, m, v, i, h);
}

// Zeroes whole 4-byte words; a byte tail (sizes not a multiple of 4) is cleared bytewise.
__global__ __launch_bounds__(256) void zero_multi_kernel(ZeroMulti z) {
    const int t = multi_owner(z.chunk_begin, z.count, int(blockIdx.x));
    const int64_t words = z.bytes[t] / 4;
    const int64_t base = int64_t(blockIdx.x - z.chunk_begin[t]) * kMultiChunk;
    const int64_t end = min(words, base + kMultiChunk);
    uint32_t *w = static_cast<uint32_t *>(z.p[t]);
    for (int64_t i = base + threadIdx.x; i < end; i += blockDim.x) w[i] = 0u;
    if (blockIdx.x == z.chunk_begin[t] && threadIdx.x < (z.bytes[t] & 3))
        static_cast<unsigned char *>(z.p[t])[words * 4 + threadIdx.x] = 0;
}

unsigned grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return unsigned(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

unsigned rows_grid(int64_t rows) { return unsigned((rows + 3) / 4); }  // 4 waves (rows) per block

}  // namespace
}  // namespace ctattn

namespace {

using ctattn::acc_t;
using ctattn::bf16_t;
using ctattn::f16_t;
using ctattn::capi::align_up;
using ctattn::capi::fail;
using ctattn::capi::finish;
using ctattn::capi::ok;

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

int check_dtype(const char *fn, int dtype) {
    if (dtype >= CTATTN_F32 && dtype <= CTATTN_F64) return 0;
    return fail(hipErrorInvalidValue, "%s: unknown dtype %d (0 = f32, 1 = bf16, 2 = f16, 3 = f64)", fn, dtype);
}

// Bytes of one row statistic / loss / Adam moment: fp64 for fp64 storage, fp32 otherwise.
int64_t stat_bytes(int dtype) { return dtype == CTATTN_F64 ? 8 : 4; }

int check_rows(const char *fn, int64_t N, int64_t D, const char *dname) {
    if (N < 0 || D < 1)
        return fail(hipErrorInvalidValue, "%s: need rows >= 0 and %s >= 1 (got %lld, %lld)", fn, dname, (long long)N,
                    (long long)D);
    if (D > 2147483647 || N > 2147483647) return fail(hipErrorInvalidValue, "%s: sizes too large", fn);
    return 0;
}

// Calls f with a null pointer of the storage type of `dtype` (checked beforehand).
template <typename F>
hipError_t by_dtype(int dtype, F f) {
    switch (dtype) {
        case CTATTN_F32: return f(static_cast<float *>(nullptr));
        case CTATTN_BF16: return f(static_cast<bf16_t *>(nullptr));
        case CTATTN_F16: return f(static_cast<f16_t *>(nullptr));
        default: return f(static_cast<double *>(nullptr));
    }
}

template <typename T> ctattn::AdamHyper<acc_t<T>> adam_hyper(double lr, double b1, double b2, double eps, double decay,
                                                              int64_t step, int decoupled) {
    using A = acc_t<T>;
    ctattn::AdamHyper<A> h;
    h.lr = A(lr);
    h.b1 = A(b1);
    h.b2 = A(b2);
    h.eps = A(eps);
    h.decay = A(decay);
    h.c1 = A(1.0 / (1.0 - pow(b1, double(step))));
    h.c2 = A(1.0 / (1.0 - pow(b2, double(step))));
    h.decoupled = decoupled ? 1 : 0;
    return h;
}

int check_adam(const char *fn, int64_t step, double beta1, double beta2, double eps) {
    if (step < 1 || !(beta1 >= 0.0 && beta1 < 1.0) || !(beta2 >= 0.0 && beta2 < 1.0) || !(eps > 0.0))
        return fail(hipErrorInvalidValue, "%s: need step >= 1, 0 <= beta < 1, eps > 0", fn);
    return 0;
}

}  // namespace

extern "C" {

int ctattn_layernorm_fwd(int dtype, const void *x, const void *gamma, const void *beta, void *y, void *mean,
                         void *rstd, int64_t N, int64_t D, double eps, void *stream) {
    const char *fn = "ctattn_layernorm_fwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, D, "D")) return rc;
    if (N == 0) return ok();
    if (!x || !gamma || !beta || !y || !mean || !rstd) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    if (!(eps >= 0.0)) return fail(hipErrorInvalidValue, "%s: eps must be >= 0", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using A = acc_t<T>;
        hipLaunchKernelGGL(ctattn::layernorm_fwd_kernel<T>, dim3(ctattn::rows_grid(N)), dim3(256), 0, st,
                           static_cast<const T *>(x), static_cast<const T *>(gamma), static_cast<const T *>(beta),
                           static_cast<T *>(y), static_cast<A *>(mean), static_cast<A *>(rstd), N, int(D), A(eps));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int64_t ctattn_layernorm_bwd_workspace_bytes(int dtype, int64_t N, int64_t D) {
    if (check_dtype("ctattn_layernorm_bwd_workspace_bytes", dtype) ||
        check_rows("ctattn_layernorm_bwd_workspace_bytes", N, D, "D"))
        return -1;
    ok();
    const int64_t chunks = (N + ctattn::kLnRowsPerChunk - 1) / ctattn::kLnRowsPerChunk;
    return align_up(chunks * 2 * D * stat_bytes(dtype));
}

int ctattn_layernorm_bwd(int dtype, const void *x, const void *gamma, const void *dy, const void *mean,
                         const void *rstd, void *dx, void *dgamma, void *dbeta, void *workspace,
                         int64_t workspace_bytes, int64_t N, int64_t D, void *stream) {
    const char *fn = "ctattn_layernorm_bwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, D, "D")) return rc;
    if (N == 0) return ok();
    if (!x || !dy || !mean || !rstd) return fail(hipErrorInvalidValue, "%s: null x/dy/mean/rstd pointer", fn);
    if (dx && !gamma) return fail(hipErrorInvalidValue, "%s: dx needs gamma", fn);
    const int64_t chunks = (N + ctattn::kLnRowsPerChunk - 1) / ctattn::kLnRowsPerChunk;
    if (chunks > 65535) return fail(hipErrorInvalidValue, "%s: N = %lld rows exceed the gradient reduction's limit", fn, (long long)N);
    const int64_t need = ctattn_layernorm_bwd_workspace_bytes(dtype, N, D);
    if ((dgamma || dbeta) && (workspace == nullptr || workspace_bytes < need))
        return fail(hipErrorInvalidValue, "%s: workspace of %lld bytes given, %lld needed", fn,
                    (long long)workspace_bytes, (long long)need);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using A = acc_t<T>;
        const T *xt = static_cast<const T *>(x);
        const T *dyt = static_cast<const T *>(dy);
        const A *mu = static_cast<const A *>(mean);
        const A *rs = static_cast<const A *>(rstd);
        A *part = static_cast<A *>(workspace);
        // dx and the partial sums together while the columns fit a lane's registers.
        auto fused = [&](auto cpl) {
            constexpr int CPL = decltype(cpl)::value;
            hipLaunchKernelGGL((ctattn::layernorm_bwd_fused_kernel<T, CPL>), dim3(unsigned(chunks)), dim3(256), 0, st,
                               xt, static_cast<const T *>(gamma), dyt, mu, rs, static_cast<T *>(dx), part, N, int(D));
        };
        const bool both = dx && (dgamma || dbeta) && D <= 1024;
        if (both) {
            if (D <= 128) fused(std::integral_constant<int, 2>{});
            else if (D <= 256) fused(std::integral_constant<int, 4>{});
            else if (D <= 384) fused(std::integral_constant<int, 6>{});
            else if (D <= 512) fused(std::integral_constant<int, 8>{});
            else fused(std::integral_constant<int, 16>{});
        } else if (dx) {
            hipLaunchKernelGGL(ctattn::layernorm_bwd_dx_kernel<T>, dim3(ctattn::rows_grid(N)), dim3(256), 0, st, xt,
                               static_cast<const T *>(gamma), dyt, mu, rs, static_cast<T *>(dx), N, int(D));
        }
        if (dgamma || dbeta) {
            if (!both)
                hipLaunchKernelGGL(ctattn::layernorm_bwd_part_kernel<T>, dim3(unsigned((D + 63) / 64), unsigned(chunks)),
                                   dim3(256), 0, st, xt, dyt, mu, rs, part, N, int(D));
            hipLaunchKernelGGL(ctattn::layernorm_bwd_reduce_kernel<T>, dim3(unsigned((D + 15) / 16)), dim3(256), 0,
                               st, static_cast<const A *>(part), static_cast<T *>(dgamma), static_cast<T *>(dbeta),
                               chunks, int(D));
        }
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_activation_fwd(int dtype, int kind, const void *x, void *y, int64_t n, void *stream) {
    const char *fn = "ctattn_activation_fwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (kind < CTATTN_ACT_RELU || kind > CTATTN_ACT_TANH)
        return fail(hipErrorInvalidValue, "%s: unknown activation %d", fn, kind);
    if (n < 0) return fail(hipErrorInvalidValue, "%s: negative size", fn);
    if (n == 0) return ok();
    if (!x || !y) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::act_fwd_kernel<T>, dim3(ctattn::grid_for(n)), dim3(256), 0, st, kind,
                           static_cast<const T *>(x), static_cast<T *>(y), n);
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_activation_bwd(int dtype, int kind, const void *x, const void *dy, void *dx, int64_t n, void *stream) {
    const char *fn = "ctattn_activation_bwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (kind < CTATTN_ACT_RELU || kind > CTATTN_ACT_TANH)
        return fail(hipErrorInvalidValue, "%s: unknown activation %d", fn, kind);
    if (n < 0) return fail(hipErrorInvalidValue, "%s: negative size", fn);
    if (n == 0) return ok();
    if (!x || !dy || !dx) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::act_bwd_kernel<T>, dim3(ctattn::grid_for(n)), dim3(256), 0, st, kind,
                           static_cast<const T *>(x), static_cast<const T *>(dy), static_cast<T *>(dx), n);
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_embedding_fwd(int dtype, const int32_t *ids, const void *tok, const void *pos, void *out, int64_t B,
                         int64_t T, int64_t E, int64_t vocab, int64_t max_len, void *stream) {
    const char *fn = "ctattn_embedding_fwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (B < 0 || T < 0 || E < 1 || vocab < 1 || max_len < 1 || T > max_len || E > 2147483647 || T > 2147483647)
        return fail(hipErrorInvalidValue, "%s: invalid sizes B=%lld T=%lld E=%lld vocab=%lld max_len=%lld", fn,
                    (long long)B, (long long)T, (long long)E, (long long)vocab, (long long)max_len);
    if (B * T == 0) return ok();
    if (!ids || !out || (!tok && !pos)) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T_ = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::embedding_fwd_kernel<T_>, dim3(ctattn::grid_for(B * T * E)), dim3(256), 0, st, ids,
                           static_cast<const T_ *>(tok), static_cast<const T_ *>(pos), static_cast<T_ *>(out), B * T,
                           int(T), int(E), vocab);
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_embedding_bwd(int dtype, const int32_t *ids, const void *dout, void *dtok, void *dpos, int64_t B,
                         int64_t T, int64_t E, int64_t vocab, void *stream) {
    const char *fn = "ctattn_embedding_bwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (B < 0 || T < 0 || E < 1 || vocab < 1 || E > 2147483647 || T > 2147483647)
        return fail(hipErrorInvalidValue, "%s: invalid sizes", fn);
    const bool narrow = dtype == CTATTN_BF16 || dtype == CTATTN_F16;
    if (dtok && narrow && ((E & 1) != 0 || (uintptr_t(dtok) & 3) != 0))
        return fail(hipErrorInvalidValue,
                    "%s: 16-bit token gradients need an even embedding width and a 4-byte aligned table", fn);
    if (B * T == 0) return ok();
    if (!ids || !dout) return fail(hipErrorInvalidValue, "%s: null ids/dout pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T_ = std::remove_pointer_t<decltype(tag)>;
        const T_ *g = static_cast<const T_ *>(dout);
        if (dtok) {
            const int64_t work = narrow ? B * T * (E / 2) : B * T * E;
            hipLaunchKernelGGL(ctattn::embedding_bwd_tok_kernel<T_>, dim3(ctattn::grid_for(work)), dim3(256), 0, st,
                               ids, g, static_cast<T_ *>(dtok), B * T, int(E), vocab);
        }
        if (dpos)
            hipLaunchKernelGGL(ctattn::embedding_bwd_pos_kernel<T_>, dim3(ctattn::grid_for(T * E)), dim3(256), 0, st,
                               g, static_cast<T_ *>(dpos), B, int(T), int(E));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_softmax_fwd(int dtype, const void *z, void *p, int64_t N, int64_t V, double temperature, void *stream) {
    const char *fn = "ctattn_softmax_fwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, V, "V")) return rc;
    if (!(temperature > 0.0)) return fail(hipErrorInvalidValue, "%s: temperature must be > 0", fn);
    if (N == 0) return ok();
    if (!z || !p) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using A = acc_t<T>;
        hipLaunchKernelGGL(ctattn::softmax_fwd_kernel<T>, dim3(ctattn::rows_grid(N)), dim3(256), 0, st,
                           static_cast<const T *>(z), static_cast<T *>(p), N, int(V), A(1) / A(temperature));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_softmax_bwd(int dtype, const void *p, const void *dp, void *dz, int64_t N, int64_t V, double temperature,
                       void *stream) {
    const char *fn = "ctattn_softmax_bwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, V, "V")) return rc;
    if (!(temperature > 0.0)) return fail(hipErrorInvalidValue, "%s: temperature must be > 0", fn);
    if (N == 0) return ok();
    if (!p || !dp || !dz) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using A = acc_t<T>;
        hipLaunchKernelGGL(ctattn::softmax_bwd_kernel<T>, dim3(ctattn::rows_grid(N)), dim3(256), 0, st,
                           static_cast<const T *>(p), static_cast<const T *>(dp), static_cast<T *>(dz), N, int(V),
                           A(1) / A(temperature));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_cross_entropy_fwd(int dtype, const void *p, const int32_t *target, void *loss, int64_t N, int64_t V,
                             void *stream) {
    const char *fn = "ctattn_cross_entropy_fwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, V, "V")) return rc;
    if (N == 0) return ok();
    if (!p || !target || !loss) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::xent_fwd_kernel<T>, dim3(unsigned((N + 255) / 256)), dim3(256), 0, st,
                           static_cast<const T *>(p), target, static_cast<acc_t<T> *>(loss), N, int(V));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_cross_entropy_bwd(int dtype, const void *p, const int32_t *target, void *dp, int64_t N, int64_t V,
                             void *stream) {
    const char *fn = "ctattn_cross_entropy_bwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, V, "V")) return rc;
    if (N == 0) return ok();
    if (!p || !target || !dp) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::xent_bwd_kernel<T>, dim3(ctattn::grid_for(N * V)), dim3(256), 0, st,
                           static_cast<const T *>(p), target, static_cast<T *>(dp), N, int(V));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_softmax_cross_entropy_bwd(int dtype, const void *p, const int32_t *target, void *dz, int64_t N, int64_t V,
                                     double temperature, void *stream) {
    const char *fn = "ctattn_softmax_cross_entropy_bwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, V, "V")) return rc;
    if (!(temperature > 0.0)) return fail(hipErrorInvalidValue, "%s: temperature must be > 0", fn);
    if (N == 0) return ok();
    if (!p || !target || !dz) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using A = acc_t<T>;
        hipLaunchKernelGGL(ctattn::softmax_xent_bwd_kernel<T>, dim3(ctattn::grid_for(N * V)), dim3(256), 0, st,
                           static_cast<const T *>(p), target, static_cast<T *>(dz), N, int(V),
                           A(1) / (A(N) * A(temperature)));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_mse_loss_fwd(int dtype, const void *x, const void *target, void *loss, int64_t N, int64_t D,
                        void *stream) {
    const char *fn = "ctattn_mse_loss_fwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, D, "D")) return rc;
    if (N == 0) return ok();
    if (!x || !target || !loss) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::mse_fwd_kernel<T>, dim3(ctattn::rows_grid(N)), dim3(256), 0, st,
                           static_cast<const T *>(x), static_cast<const T *>(target), static_cast<acc_t<T> *>(loss), N,
                           int(D));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_mse_loss_bwd(int dtype, const void *x, const void *target, void *dx, int64_t N, int64_t D, void *stream) {
    const char *fn = "ctattn_mse_loss_bwd";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_rows(fn, N, D, "D")) return rc;
    if (N == 0) return ok();
    if (!x || !target || !dx) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::mse_bwd_kernel<T>, dim3(ctattn::grid_for(N * D)), dim3(256), 0, st,
                           static_cast<const T *>(x), static_cast<const T *>(target), static_cast<T *>(dx), N * D,
                           int(D));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_adam_update(int dtype, void *param, const void *grad, void *m, void *v, int64_t n, double lr, double beta1,
                       double beta2, double eps, double weight_decay, int64_t step, int decoupled, void *stream) {
    const char *fn = "ctattn_adam_update";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_adam(fn, step, beta1, beta2, eps)) return rc;
    if (n < 0) return fail(hipErrorInvalidValue, "%s: negative size", fn);
    if (n == 0) return ok();
    if (!param || !grad || !m || !v) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using A = acc_t<T>;
        hipLaunchKernelGGL(ctattn::adam_kernel<T>, dim3(ctattn::grid_for(n)), dim3(256), 0, st,
                           static_cast<T *>(param), static_cast<const T *>(grad), static_cast<A *>(m),
                           static_cast<A *>(v), n, adam_hyper<T>(lr, beta1, beta2, eps, weight_decay, step, decoupled));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_adam_update_multi(int dtype, int count, void *const *param, const void *const *grad, void *const *m,
                             void *const *v, const int64_t *n, double lr, double beta1, double beta2, double eps,
                             double weight_decay, int64_t step, int decoupled, void *stream) {
    const char *fn = "ctattn_adam_update_multi";
    if (int rc = check_dtype(fn, dtype)) return rc;
    if (int rc = check_adam(fn, step, beta1, beta2, eps)) return rc;
    if (count < 0) return fail(hipErrorInvalidValue, "%s: negative count", fn);
    if (count == 0) return ok();
    if (!param || !grad || !m || !v || !n) return fail(hipErrorInvalidValue, "%s: null table", fn);
    for (int i = 0; i < count; ++i) {
        if (n[i] < 0) return fail(hipErrorInvalidValue, "%s: tensor %d has a negative size", fn, i);
        if (n[i] > 0 && (!param[i] || !grad[i] || !m[i] || !v[i]))
            return fail(hipErrorInvalidValue, "%s: null pointer for tensor %d", fn, i);
        if ((n[i] + ctattn::kMultiChunk - 1) / ctattn::kMultiChunk > (int64_t(1) << 30))
            return fail(hipErrorInvalidValue, "%s: tensor %d too large", fn, i);
    }
    hipStream_t st = as_stream(stream);
    for (int first = 0; first < count; first += ctattn::kMultiMax) {
        ctattn::AdamMulti a{};
        int64_t chunks = 0;
        for (int i = first; i < count && a.count < ctattn::kMultiMax; ++i) {
            if (n[i] == 0) continue;
            const int k = a.count++;
            a.param[k] = param[i];
            a.grad[k] = grad[i];
            a.m[k] = m[i];
            a.v[k] = v[i];
            a.n[k] = n[i];
            a.chunk_begin[k] = int32_t(chunks);
            chunks += (n[i] + ctattn::kMultiChunk - 1) / ctattn::kMultiChunk;
            if (chunks > (int64_t(1) << 30)) return fail(hipErrorInvalidValue, "%s: too many elements per launch", fn);
        }
        if (a.count == 0) continue;
        a.chunk_begin[a.count] = int32_t(chunks);
        const hipError_t e = by_dtype(dtype, [&](auto *tag) {
            using T = std::remove_pointer_t<decltype(tag)>;
            hipLaunchKernelGGL(ctattn::adam_multi_kernel<T>, dim3(unsigned(chunks)), dim3(256), 0, st, a,
                               adam_hyper<T>(lr, beta1, beta2, eps, weight_decay, step, decoupled));
            return hipGetLastError();
        });
        if (e != hipSuccess) return finish(fn, e, st);
    }
    return finish(fn, hipSuccess, st);
}

int ctattn_zero_multi(int count, void *const *ptr, const int64_t *bytes, void *stream) {
    const char *fn = "ctattn_zero_multi";
    if (count < 0) return fail(hipErrorInvalidValue, "%s: negative count", fn);
    if (count == 0) return ok();
    if (!ptr || !bytes) return fail(hipErrorInvalidValue, "%s: null table", fn);
    for (int i = 0; i < count; ++i) {
        if (bytes[i] < 0) return fail(hipErrorInvalidValue, "%s: buffer %d has a negative size", fn, i);
        if (bytes[i] > 0 && !ptr[i]) return fail(hipErrorInvalidValue, "%s: null pointer for buffer %d", fn, i);
        if (bytes[i] > 0 && (uintptr_t(ptr[i]) & 3) != 0)
            return fail(hipErrorInvalidValue, "%s: buffer %d is not 4-byte aligned", fn, i);
    }
    hipStream_t st = as_stream(stream);
    for (int first = 0; first < count; first += ctattn::kMultiMax) {
        ctattn::ZeroMulti z{};
        int64_t chunks = 0;
        for (int i = first; i < count && z.count < ctattn::kMultiMax; ++i) {
            if (bytes[i] == 0) continue;
            const int k = z.count++;
            z.p[k] = ptr[i];
            z.bytes[k] = bytes[i];
            z.chunk_begin[k] = int32_t(chunks);
            chunks += std::max<int64_t>(1, (bytes[i] / 4 + ctattn::kMultiChunk - 1) / ctattn::kMultiChunk);
            if (chunks > (int64_t(1) << 30)) return fail(hipErrorInvalidValue, "%s: too many bytes per launch", fn);
        }
        if (z.count == 0) continue;
        z.chunk_begin[z.count] = int32_t(chunks);
        hipLaunchKernelGGL(ctattn::zero_multi_kernel, dim3(unsigned(chunks)), dim3(256), 0, st, z);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return finish(fn, e, st);
    }
    return finish(fn, hipSuccess, st);
}

}  // extern "C"
