// Generic attention kernels: any head dim 1 <= d <= 256, fp32 or bf16 storage, causal or
// not.  One wave64 per query row (forward, dQ) or per key row (dK/dV); scalar fp32 FMAs.
//
// These are the fallback for head dims the MFMA kernels do not cover and the GPU-side
// cross-check of those kernels.  The math is the reference's
// (flash_attention.cu:97-161 forward online softmax; :269-299 delta, P and dS), with the
// causal mask, no padded keys, and the correct dK/dV.  Deterministic: no atomics.
#include "attn_common.h"
#include "attn_launch.h"

#include <math.h>

namespace ctattn {
namespace {

constexpr int kMaxD = 256;
constexpr int kSlots = kMaxD / kWave;  // d elements per lane

template <typename T>
__global__ __launch_bounds__(kWave) void generic_fwd_kernel(const T *__restrict__ q,
                                                           const T *__restrict__ k,
                                                           const T *__restrict__ v,
                                                           T *__restrict__ o,
                                                           float *__restrict__ lse,
                                                           int64_t seq, int d, int causal) {
    __shared__ float qs[kMaxD];
    __shared__ float ps[kWave];
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t bh = row / seq;
    const int64_t i = row - bh * seq;
    const int64_t base = bh * seq * d;
    const float sqrt_d = sqrtf(float(d));

    for (int c = lane; c < d; c += kWave) qs[c] = to_f32(q[base + i * d + c]);
    __syncthreads();

    const int64_t nkeys = causal ? i + 1 : seq;
    float m = -INFINITY, l = 0.f;
    float acc[kSlots] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t j0 = 0; j0 < nkeys; j0 += kWave) {
        const int64_t j = j0 + lane;
        float s = -INFINITY;
        if (j < nkeys) {
            float dot = 0.f;
            const T *kr = k + base + j * d;
            for (int c = 0; c < d; ++c) dot += qs[c] * to_f32(kr[c]);
            s = dot / sqrt_d;  // division by sqrt(d), flash_attention.cu:116
        }
        const float mnew = fmaxf(m, wave_max(s));  // finite: key j0 is always valid
        const float rescale = (m == -INFINITY) ? 0.f : expf(m - mnew);
        const float p = (j < nkeys) ? expf(s - mnew) : 0.f;
        l = l * rescale + wave_sum(p);
        ps[lane] = p;
        __syncthreads();
        const int cnt = int(nkeys - j0 < kWave ? nkeys - j0 : kWave);
#pragma unroll
        for (int r = 0; r < kSlots; ++r) {
            const int c = lane + r * kWave;
            if (c < d) {
                float a = acc[r] * rescale;
                for (int jj = 0; jj < cnt; ++jj) a += ps[jj] * to_f32(v[base + (j0 + jj) * d + c]);
                acc[r] = a;
            }
        }
        __syncthreads();
        m = mnew;
    }
    const float inv_l = 1.f / l;
#pragma unroll
    for (int r = 0; r < kSlots; ++r) {
        const int c = lane + r * kWave;
        if (c < d) o[base + i * d + c] = from_f32<T>(acc[r] * inv_l);
    }
    if (lse != nullptr && lane == 0) lse[row] = m + logf(l);
}

// delta[row] = sum_c dO[row][c] * O[row][c]   (flash_attention.cu:269-273), one wave per row.
template <typename T>
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(const T *__restrict__ o,
                                                            const T *__restrict__ dout,
                                                            float *__restrict__ delta,
                                                            int64_t rows, int d) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    float s = 0.f;
    for (int c = lane; c < d; c += kWave) s += to_f32(o[row * d + c]) * to_f32(dout[row * d + c]);
    s = wave_sum(s);
    if (lane == 0) delta[row] = s;
}

// dQ_i = sum_j dS_ij K_j / sqrt(d), one wave per query row (flash_attention.cu:297-311).
template <typename T>
__global__ __launch_bounds__(kWave) void generic_bwd_dq_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    T *__restrict__ dq, int64_t seq, int d, int causal) {
    __shared__ float qs[kMaxD];
    __shared__ float dos[kMaxD];
    __shared__ float dss[kWave];
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t bh = row / seq;
    const int64_t i = row - bh * seq;
    const int64_t base = bh * seq * d;
    const float sqrt_d = sqrtf(float(d));
    for (int c = lane; c < d; c += kWave) {
        qs[c] = to_f32(q[base + i * d + c]);
        dos[c] = to_f32(dout[base + i * d + c]);
    }
    __syncthreads();
    const float lse_i = lse[row];
    const float delta_i = delta[row];
    const int64_t nkeys = causal ? i + 1 : seq;
    float acc[kSlots] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t j0 = 0; j0 < nkeys; j0 += kWave) {
        const int64_t j = j0 + lane;
        float ds = 0.f;
        if (j < nkeys) {
            float sdot = 0.f, pdot = 0.f;
            const T *kr = k + base + j * d;
            const T *vr = v + base + j * d;
            for (int c = 0; c < d; ++c) {
                sdot += qs[c] * to_f32(kr[c]);
                pdot += dos[c] * to_f32(vr[c]);
            }
            const float p = expf(sdot / sqrt_d - lse_i);
            ds = p * (pdot - delta_i);
        }
        dss[lane] = ds;
        __syncthreads();
        const int cnt = int(nkeys - j0 < kWave ? nkeys - j0 : kWave);
#pragma unroll
        for (int r = 0; r < kSlots; ++r) {
            const int c = lane + r * kWave;
            if (c < d) {
                float a = acc[r];
                for (int jj = 0; jj < cnt; ++jj) a += dss[jj] * to_f32(k[base + (j0 + jj) * d + c]);
                acc[r] = a;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < kSlots; ++r) {
        const int c = lane + r * kWave;
        if (c < d) dq[base + i * d + c] = from_f32<T>(acc[r] / sqrt_d);
    }
}

// dK_j = sum_i dS_ij Q_i / sqrt(d), dV_j = sum_i P_ij dO_i; one wave per key row.
template <typename T>
__global__ __launch_bounds__(kWave) void generic_bwd_dkdv_kernel(
    const T *__restrict__ q, const T *__restrict__ k, const T *__restrict__ v,
    const T *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    T *__restrict__ dk, T *__restrict__ dv, int64_t seq, int d, int causal) {
    __shared__ float ks[kMaxD];
    __shared__ float vs[kMaxD];
    __shared__ float ps[kWave];
    __shared__ float dss[kWave];
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t bh = row / seq;
    const int64_t j = row - bh * seq;
    const int64_t base = bh * seq * d;
    const float sqrt_d = sqrtf(float(d));
    for (int c = lane; c < d; c += kWave) {
        ks[c] = to_f32(k[base + j * d + c]);
        vs[c] = to_f32(v[base + j * d + c]);
    }
    __syncthreads();
    float acck[kSlots] = {0.f, 0.f, 0.f, 0.f};
    float accv[kSlots] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t i0 = causal ? j : 0; i0 < seq; i0 += kWave) {
        const int64_t i = i0 + lane;
        float p = 0.f, ds = 0.f;
        if (i < seq) {
            float sdot = 0.f, pdot = 0.f;
            const T *qr = q + base + i * d;
            const T *dor = dout + base + i * d;
            for (int c = 0; c < d; ++c) {
                sdot += to_f32(qr[c]) * ks[c];
                pdot += to_f32(dor[c]) * vs[c];
            }
            p = expf(sdot / sqrt_d - lse[bh * seq + i]);
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
                float ak = acck[r], av = accv[r];
                for (int ii = 0; ii < cnt; ++ii) {
                    ak += dss[ii] * to_f32(q[base + (i0 + ii) * d + c]);
                    av += ps[ii] * to_f32(dout[base + (i0 + ii) * d + c]);
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
            dk[base + j * d + c] = from_f32<T>(acck[r] / sqrt_d);
            dv[base + j * d + c] = from_f32<T>(accv[r]);
        }
    }
}

template <typename T>
hipError_t generic_fwd_t(const void *q, const void *k, const void *v, void *o, float *lse,
                         const AttnShape &s, hipStream_t stream) {
    hipLaunchKernelGGL(generic_fwd_kernel<T>, dim3(unsigned(s.rows())), dim3(kWave), 0, stream,
                       static_cast<const T *>(q), static_cast<const T *>(k),
                       static_cast<const T *>(v), static_cast<T *>(o), lse, s.T, int(s.d),
                       int(s.causal));
    return hipGetLastError();
}

template <typename T>
hipError_t preprocess_t(const void *o, const void *dout, float *delta, const AttnShape &s,
                        hipStream_t stream) {
    const int64_t rows = s.rows();
    const unsigned blocks = unsigned((rows + 3) / 4);
    hipLaunchKernelGGL(bwd_preprocess_kernel<T>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const T *>(o), static_cast<const T *>(dout), delta, rows,
                       int(s.d));
    return hipGetLastError();
}

template <typename T>
hipError_t generic_bwd_t(const void *q, const void *k, const void *v, const void *o,
                         const void *dout, const float *lse, void *dq, void *dk, void *dv,
                         float *delta, const AttnShape &s, hipStream_t stream) {
    hipError_t e = preprocess_t<T>(o, dout, delta, s, stream);
    if (e != hipSuccess) return e;
    const dim3 grid(unsigned(s.rows()));
    hipLaunchKernelGGL(generic_bwd_dq_kernel<T>, grid, dim3(kWave), 0, stream,
                       static_cast<const T *>(q), static_cast<const T *>(k),
                       static_cast<const T *>(v), static_cast<const T *>(dout), lse, delta,
                       static_cast<T *>(dq), s.T, int(s.d), int(s.causal));
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(generic_bwd_dkdv_kernel<T>, grid, dim3(kWave), 0, stream,
                       static_cast<const T *>(q), static_cast<const T *>(k),
                       static_cast<const T *>(v), static_cast<const T *>(dout), lse, delta,
                       static_cast<T *>(dk), static_cast<T *>(dv), s.T, int(s.d),
                       int(s.causal));
    return hipGetLastError();
}

}  // namespace

hipError_t launch_generic_fwd(int dtype, const void *q, const void *k, const void *v, void *o,
                              float *lse, const AttnShape &s, hipStream_t stream) {
    return dtype == 0 ? generic_fwd_t<float>(q, k, v, o, lse, s, stream)
                      : generic_fwd_t<bf16_t>(q, k, v, o, lse, s, stream);
}

hipError_t launch_bwd_preprocess(int dtype, const void *o, const void *dout, float *delta,
                                 const AttnShape &s, hipStream_t stream) {
    return dtype == 0 ? preprocess_t<float>(o, dout, delta, s, stream)
                      : preprocess_t<bf16_t>(o, dout, delta, s, stream);
}

hipError_t launch_generic_bwd(int dtype, const void *q, const void *k, const void *v,
                              const void *o, const void *dout, const float *lse, void *dq,
                              void *dk, void *dv, float *delta, const AttnShape &s,
                              hipStream_t stream) {
    return dtype == 0
               ? generic_bwd_t<float>(q, k, v, o, dout, lse, dq, dk, dv, delta, s, stream)
               : generic_bwd_t<bf16_t>(q, k, v, o, dout, lse, dq, dk, dv, delta, s, stream);
}

}  // namespace ctattn
