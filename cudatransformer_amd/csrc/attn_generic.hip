// Generic attention kernels: any head dim 1 <= d <= 256, fp32, bf16, fp16 or fp64 storage,
// causal or not.  One wave64 per query row (forward, dQ) or per key row (dK/dV); scalar FMAs
// in the storage type's accumulation type (fp64 for fp64 storage, the reference's
// ComputeType; fp32 otherwise), with LSE and delta in that type.
//
// These serve head dims and dtypes the MFMA kernels do not cover (fp16, fp64) and are the
// GPU-side cross-check of those kernels.  The math is the reference's
// (flash_attention.cu:97-161 forward online softmax; :269-299 delta, P and dS), with the
// causal mask, no padded keys, and the correct dK/dV.  Deterministic: no atomics.
#include "attn_common.h"
#include "attn_launch.h"

#include <math.h>

#include <type_traits>

namespace ctattn {
namespace {

constexpr int kMaxD = 256;
constexpr int kSlots = kMaxD / kWave;  // d elements per lane

template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(kWave) void generic_fwd_kernel(const T *__restrict__ q,
                                                           const T *__restrict__ k,
                                                           const T *__restrict__ v,
                                                           T *__restrict__ o,
                                                           A *__restrict__ lse,
                                                           int64_t rows, int64_t seq, int d, int causal) {
    __shared__ A qs[kMaxD];
    __shared__ A ps[kWave];
    const int lane = threadIdx.x;
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        __syncthreads();  // the previous row's reads of qs / ps are done
        const int64_t bh = row / seq;
        const int64_t i = row - bh * seq;
        const int64_t base = bh * seq * d;
        const A sqrt_d = acc_sqrt(A(d));

        for (int c = lane; c < d; c += kWave) qs[c] = to_acc(q[base + i * d + c]);
        __syncthreads();

        const int64_t nkeys = causal ? i + 1 : seq;
        A m = -INFINITY, l = 0;
        A acc[kSlots] = {0, 0, 0, 0};
        for (int64_t j0 = 0; j0 < nkeys; j0 += kWave) {
            const int64_t j = j0 + lane;
            A s = -INFINITY;
            if (j < nkeys) {
                A dot = 0;
                const T *kr = k + base + j * d;
                for (int c = 0; c < d; ++c) dot += qs[c] * to_acc(kr[c]);
                s = dot / sqrt_d;  // division by sqrt(d), flash_attention.cu:116
            }
            const A mnew = fmax(m, wave_max(s));  // finite: key j0 is always valid
            const A rescale = (m == -INFINITY) ? A(0) : acc_exp(m - mnew);
            const A p = (j < nkeys) ? acc_exp(s - mnew) : A(0);
            l = l * rescale + wave_sum(p);
            ps[lane] = p;
            __syncthreads();
            const int cnt = int(nkeys - j0 < kWave ? nkeys - j0 : kWave);
#pragma unroll
            for (int r = 0; r < kSlots; ++r) {
                const int c = lane + r * kWave;
                if (c < d) {
                    A a = acc[r] * rescale;
                    for (int jj = 0; jj < cnt; ++jj) a += ps[jj] * to_acc(v[base + (j0 + jj) * d + c]);
                    acc[r] = a;
                }
            }
            __syncthreads();
            m = mnew;
        }
        const A inv_l = A(1) / l;
#pragma unroll
        for (int r = 0; r < kSlots; ++r) {
            const int c = lane + r * kWave;
            if (c < d) o[base + i * d + c] = from_acc<T>(acc[r] * inv_l);
        }
        if (lse != nullptr && lane == 0) lse[row] = m + acc_log(l);
    }
}

// delta[row] = sum_c dO[row][c] * O[row][c]   (flash_attention.cu:269-273), one wave per row.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(const T *__restrict__ o,
                                                            const T *__restrict__ dout,
                                                            A *__restrict__ delta,
                                                            int64_t rows, int d) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wpb = blockDim.x / kWave;
    for (int64_t row = int64_t(blockIdx.x) * wpb + threadIdx.x / kWave; row < rows; row += int64_t(gridDim.x) * wpb) {
        A s = 0;
        for (int c = lane; c < d; c += kWave) s += to_acc(o[row * d + c]) * to_acc(dout[row * d + c]);
        s = wave_sum(s);
        if (lane == 0) delta[row] = s;
    }
}

// dQ_i = sum_j dS_ij K_j / sqrt(d), one wave per query row (flash_attention.cu:297-311).
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(kWave) void generic_bwd_dq_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const A *__restrict__ lse, const A *__restrict__ delta,
    T *__restrict__ dq, int64_t rows, int64_t seq, int d, int causal) {
    __shared__ A qs[kMaxD];
    __shared__ A dos[kMaxD];
    __shared__ A dss[kWave];
    const int lane = threadIdx.x;
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        __syncthreads();  // the previous row's reads of qs / dos / dss are done
        const int64_t bh = row / seq;
        const int64_t i = row - bh * seq;
        const int64_t base = bh * seq * d;
        const A sqrt_d = acc_sqrt(A(d));
        for (int c = lane; c < d; c += kWave) {
            qs[c] = to_acc(q[base + i * d + c]);
            dos[c] = to_acc(dout[base + i * d + c]);
        }
        __syncthreads();
        const A lse_i = lse[row];
        const A delta_i = delta[row];
        const int64_t nkeys = causal ? i + 1 : seq;
        A acc[kSlots] = {0, 0, 0, 0};
        for (int64_t j0 = 0; j0 < nkeys; j0 += kWave) {
            const int64_t j = j0 + lane;
            A ds = 0;
            if (j < nkeys) {
                A sdot = 0, pdot = 0;
                const T *kr = k + base + j * d;
                const T *vr = v + base + j * d;
                for (int c = 0; c < d; ++c) {
                    sdot += qs[c] * to_acc(kr[c]);
                    pdot += dos[c] * to_acc(vr[c]);
                }
                const A p = acc_exp(sdot / sqrt_d - lse_i);
                ds = p * (pdot - delta_i);
            }
            dss[lane] = ds;
            __syncthreads();
            const int cnt = int(nkeys - j0 < kWave ? nkeys - j0 : kWave);
#pragma unroll
            for (int r = 0; r < kSlots; ++r) {
                const int c = lane + r * kWave;
                if (c < d) {
                    A a = acc[r];
                    for (int jj = 0; jj < cnt; ++jj) a += dss[jj] * to_acc(k[base + (j0 + jj) * d + c]);
                    acc[r] = a;
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int r = 0; r < kSlots; ++r) {
            const int c = lane + r * kWave;
            if (c < d) dq[base + i * d + c] = from_acc<T>(acc[r] / sqrt_d);
        }
    }
}

// dK_j = sum_i dS_ij Q_i / sqrt(d), dV_j = sum_i P_ij dO_i; one wave per key row.
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(kWave) void generic_bwd_dkdv_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const A *__restrict__ lse, const A *__restrict__ delta,
    T *__restrict__ dk, T *__restrict__ dv, int64_t rows, int64_t seq, int d, int causal) {
    __shared__ A ks[kMaxD];
    __shared__ A vs[kMaxD];
    __shared__ A ps[kWave];
    __shared__ A dss[kWave];
    const int lane = threadIdx.x;
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        __syncthreads();  // the previous row's reads of ks / vs / ps / dss are done
        const int64_t bh = row / seq;
        const int64_t j = row - bh * seq;
        const int64_t base = bh * seq * d;
        const A sqrt_d = acc_sqrt(A(d));
        for (int c = lane; c < d; c += kWave) {
            ks[c] = to_acc(k[base + j * d + c]);
            vs[c] = to_acc(v[base + j * d + c]);
        }
        __syncthreads();
        A acck[kSlots] = {0, 0, 0, 0};
        A accv[kSlots] = {0, 0, 0, 0};
        for (int64_t i0 = causal ? j : 0; i0 < seq; i0 += kWave) {
            const int64_t i = i0 + lane;
            A p = 0, ds = 0;
            if (i < seq) {
                A sdot = 0, pdot = 0;
                const T *qr = q + base + i * d;
                const T *dor = dout + base + i * d;
                for (int c = 0; c < d; ++c) {
                    sdot += to_acc(qr[c]) * ks[c];
                    pdot += to_acc(dor[c]) * vs[c];
                }
                p = acc_exp(sdot / sqrt_d - lse[bh * seq + i]);
                ds = p * (pdot - delta[bh * seq + i]);
            }
            ps[lane] = p;
            dss[lane] = ds;
            __syncthreads();
            const int cnt = int(seq - i0 < kWave ? seq - i0 : kWave);
#pragma unroll
            for (int r = 0; r < kSlots; ++r) {
                const int c = lane + r * kWave;
                if (c < d) {
                    A ak = acck[r], av = accv[r];
                    for (int ii = 0; ii < cnt; ++ii) {
                        ak += dss[ii] * to_acc(q[base + (i0 + ii) * d + c]);
                        av += ps[ii] * to_acc(dout[base + (i0 + ii) * d + c]);
                    }
                    acck[r] = ak;
                    accv[r] = av;
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int r = 0; r < kSlots; ++r) {
            const int c = lane + r * kWave;
            if (c < d) {
                dk[base + j * d + c] = from_acc<T>(acck[r] / sqrt_d);
                dv[base + j * d + c] = from_acc<T>(accv[r]);
            }
        }
    }
}

template <typename T>
hipError_t generic_fwd_t(const void *q, const void *k, const void *v, void *o, void *lse,
                         const AttnShape &s, hipStream_t stream) {
    hipLaunchKernelGGL(generic_fwd_kernel<T>, dim3(stride_grid(s.rows(), kWave)), dim3(kWave), 0, stream,
                       static_cast<const T *>(q), static_cast<const T *>(k),
                       static_cast<const T *>(v), static_cast<T *>(o), static_cast<acc_t<T> *>(lse), s.rows(),
                       s.T, int(s.d), int(s.causal));
    return hipGetLastError();
}

template <typename T>
hipError_t preprocess_t(const void *o, const void *dout, void *delta, const AttnShape &s,
                        hipStream_t stream) {
    const int64_t rows = s.rows();
    hipLaunchKernelGGL(bwd_preprocess_kernel<T>, dim3(stride_grid((rows + 3) / 4, 256)), dim3(256), 0, stream,
                       static_cast<const T *>(o), static_cast<const T *>(dout),
                       static_cast<acc_t<T> *>(delta), rows, int(s.d));
    return hipGetLastError();
}

template <typename T>
hipError_t generic_bwd_t(const void *q, const void *k, const void *v, const void *o,
                         const void *dout, const void *lse, void *dq, void *dk, void *dv,
                         void *delta, const AttnShape &s, hipStream_t stream) {
    using A = acc_t<T>;
    hipError_t e = preprocess_t<T>(o, dout, delta, s, stream);
    if (e != hipSuccess) return e;
    const dim3 grid(stride_grid(s.rows(), kWave));
    hipLaunchKernelGGL(generic_bwd_dq_kernel<T>, grid, dim3(kWave), 0, stream,
                       static_cast<const T *>(q), static_cast<const T *>(k),
                       static_cast<const T *>(v), static_cast<const T *>(dout), static_cast<const A *>(lse),
                       static_cast<const A *>(delta), static_cast<T *>(dq), s.rows(), s.T, int(s.d), int(s.causal));
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(generic_bwd_dkdv_kernel<T>, grid, dim3(kWave), 0, stream,
                       static_cast<const T *>(q), static_cast<const T *>(k),
                       static_cast<const T *>(v), static_cast<const T *>(dout), static_cast<const A *>(lse),
                       static_cast<const A *>(delta), static_cast<T *>(dk), static_cast<T *>(dv), s.rows(),
                       s.T, int(s.d), int(s.causal));
    return hipGetLastError();
}

// dtype codes: 0 fp32, 1 bf16, 2 fp16, 3 fp64.
template <typename F>
hipError_t by_dtype(int dtype, F &&f) {
    switch (dtype) {
        case 0: return f(static_cast<float *>(nullptr));
        case 1: return f(static_cast<bf16_t *>(nullptr));
        case 2: return f(static_cast<f16_t *>(nullptr));
        default: return f(static_cast<double *>(nullptr));
    }
}

}  // namespace

hipError_t launch_generic_fwd(int dtype, const void *q, const void *k, const void *v, void *o,
                              void *lse, const AttnShape &s, hipStream_t stream) {
    return by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        return generic_fwd_t<T>(q, k, v, o, lse, s, stream);
    });
}

hipError_t launch_bwd_preprocess(int dtype, const void *o, const void *dout, void *delta,
                                 const AttnShape &s, hipStream_t stream) {
    return by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        return preprocess_t<T>(o, dout, delta, s, stream);
    });
}

hipError_t launch_generic_bwd(int dtype, const void *q, const void *k, const void *v,
                              const void *o, const void *dout, const void *lse, void *dq,
                              void *dk, void *dv, void *delta, const AttnShape &s,
                              hipStream_t stream) {
    return by_dtype(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        return generic_bwd_t<T>(q, k, v, o, dout, lse, dq, dk, dv, delta, s, stream);
    });
}

}  // namespace ctattn
