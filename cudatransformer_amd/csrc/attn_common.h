// Device-side helpers shared by the attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace ctattn {

constexpr int kWave = 64;

// bf16 is carried as its raw 16-bit pattern; arithmetic is fp32.
struct bf16_t {
    uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(uint32_t(x.bits) << 16); }

// Round-to-nearest-even fp32 -> bf16 (NaN stays a quiet NaN).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return bf16_t{uint16_t((u >> 16) | 0x40)};
    u += 0x7fffu + ((u >> 16) & 1u);
    return bf16_t{uint16_t(u >> 16)};
}

// IEEE binary16, carried as its raw 16-bit pattern; arithmetic is fp32 (hardware conversion,
// round to nearest even).
struct f16_t {
    uint16_t bits;
};
__device__ __forceinline__ float to_f32(f16_t x) { return float(__builtin_bit_cast(_Float16, x.bits)); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return f32_to_bf16(x); }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) {
    return f16_t{__builtin_bit_cast(uint16_t, _Float16(x))};
}

// Accumulation type of a storage type: fp64 for double, fp32 for everything narrower (the
// reference's ComputeType, headers.cu:47-48).
template <typename T> struct AccOf {
    using type = float;
};
template <> struct AccOf<double> {
    using type = double;
};
template <typename T> using acc_t = typename AccOf<T>::type;

__device__ __forceinline__ float to_acc(float x) { return x; }
__device__ __forceinline__ float to_acc(bf16_t x) { return to_f32(x); }
__device__ __forceinline__ float to_acc(f16_t x) { return to_f32(x); }
__device__ __forceinline__ double to_acc(double x) { return x; }
template <typename T> __device__ __forceinline__ T from_acc(acc_t<T> x) { return from_f32<T>(x); }
template <> __device__ __forceinline__ double from_acc<double>(double x) { return x; }

__device__ __forceinline__ float acc_exp(float x) { return expf(x); }
__device__ __forceinline__ double acc_exp(double x) { return exp(x); }
__device__ __forceinline__ float acc_log(float x) { return logf(x); }
__device__ __forceinline__ double acc_log(double x) { return log(x); }
__device__ __forceinline__ float acc_sqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ double acc_sqrt(double x) { return sqrt(x); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}
__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
    return x;
}
__device__ __forceinline__ double wave_max(double x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x = fmax(x, __shfl_xor(x, off, kWave));
    return x;
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64).
template <int width> __device__ __forceinline__ float group_sum(float x) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace ctattn
