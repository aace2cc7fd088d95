// Tensor operations behind the Python Tensor classes (declared in include/ctattn.h): dtype
// casts, elementwise arithmetic and comparisons with numpy-style broadcasting, unary maps,
// reductions, axis permutation, the Kronecker product and batched matrix products.
//
// They replace the reference's Tensor<DType> methods and their kernels: to<>()
// (Tensor.cu:267, castKernel), transpose (Tensor.cu:577-616, transposeKernel), unary
// (Tensor.cu:624-637, unaryOpKernel), binary / predicate with broadcasting (Tensor.cu:650-802,
// binaryOpKernel, binaryPredicateOpKernel, the scalar variants), reduce (Tensor.cu:807-870,
// reduceKernel), kron (Tensor.cu:877-905, kronKernel) and matmul (Tensor.cu:912-950,
// matmulKernel).  Same results, with these deliberate differences:
//   * arithmetic runs in fp32 for bf16 / fp16 storage, fp64 for fp64 and int64 for the
//     integer and bool types (the reference computes in the storage type for + - * / and
//     sums reductions in it), then rounds once to the storage type;
//   * integer division and remainder by zero give 0 (undefined in the reference);
//   * reductions are two-stage and deterministic (a fixed order per output) instead of one
//     thread walking every reduced element;
//   * fp32 / bf16 / fp16 products run on the MFMA GEMMs of linear_gemm.hip (16-bit storage on
//     the 16-bit MFMA), fp64 and shapes outside that family's domain on the projection GEMM
//     family, instead of one thread per output.
// Storage codes: ctattn_dtype plus CTATTN_I32 .. CTATTN_BOOL.  bool is one byte, 0 or 1.
#include "attn_common.h"
#include "capi_util.h"
#include "ctattn.h"
#include "linear_gemm.h"
#include "proj_launch.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace ctattn {
namespace {

constexpr int kMaxDims = 8;

// Arithmetic type of a storage type.
template <typename T> struct CalcOf { using type = int64_t; };
template <> struct CalcOf<float> { using type = float; };
template <> struct CalcOf<bf16_t> { using type = float; };
template <> struct CalcOf<f16_t> { using type = float; };
template <> struct CalcOf<double> { using type = double; };
template <typename T> using calc_t = typename CalcOf<T>::type;

template <typename T> __device__ __forceinline__ calc_t<T> ldv(const T *p, int64_t i) {
    if constexpr (std::is_same_v<T, bf16_t> || std::is_same_v<T, f16_t>) return to_f32(p[i]);
    else if constexpr (std::is_same_v<T, bool>) return p[i] ? 1 : 0;
    else return calc_t<T>(p[i]);
}

// fp64 -> fp32 rounded to odd: exact values unchanged, inexact ones truncated toward zero with
// the last mantissa bit set.  Rounding that to bf16 / fp16 (fewer than 23 mantissa bits) is
// the correctly rounded fp64 -> bf16 / fp16 conversion (no double rounding).
__device__ __forceinline__ float f32_round_odd(double d) {
    float f = float(d);
    if (double(f) != d && d == d) {
        if (fabs(double(f)) > fabs(d)) f = __uint_as_float(__float_as_uint(f) - 1u);  // toward zero
        f = __uint_as_float(__float_as_uint(f) | 1u);
    }
    return f;
}

// Integer from a float value: truncation toward zero, NaN -> 0, saturated to int64.
__device__ __forceinline__ int64_t to_i64(double x) {
    if (!(x == x)) return 0;
    if (x >= 9223372036854775807.0) return INT64_MAX;
    if (x <= -9223372036854775808.0) return INT64_MIN;
    return int64_t(x);
}

// Stores a value of any arithmetic type into storage type T.
template <typename T, typename V> __device__ __forceinline__ void stv(T *p, int64_t i, V x) {
    if constexpr (std::is_same_v<T, bool>) {
        p[i] = x != V(0);
    } else if constexpr (std::is_same_v<T, float>) {
        p[i] = float(x);
    } else if constexpr (std::is_same_v<T, double>) {
        p[i] = double(x);
    } else if constexpr (std::is_same_v<T, bf16_t> || std::is_same_v<T, f16_t>) {
        if constexpr (std::is_same_v<V, float>) p[i] = from_f32<T>(x);
        else p[i] = from_f32<T>(f32_round_odd(double(x)));
    } else {  // integer storage: wraps modulo 2^bits
        if constexpr (std::is_floating_point_v<V>) p[i] = T(to_i64(double(x)));
        else p[i] = T(x);
    }
}

// The scalar operand of a tensor-scalar operation, converted to the storage type first as
// the reference does (static_cast<DType>(b), cuda_transformer.cu:79-98).
template <typename T> __device__ __forceinline__ calc_t<T> scalar_as(double s) {
    T t[1];
    stv(t, 0, s);
    return ldv(t, 0);
}

// ---- elementwise ------------------------------------------------------------------------

template <typename S, typename D> __device__ __forceinline__ void cast_one(const S *src, D *dst, int64_t i) {
    if constexpr (std::is_same_v<S, D>) dst[i] = src[i];
    else if constexpr (std::is_same_v<S, bool>) stv(dst, i, int64_t(src[i] ? 1 : 0));
    else if constexpr (std::is_same_v<S, bf16_t> || std::is_same_v<S, f16_t>) stv(dst, i, to_f32(src[i]));
    else stv(dst, i, src[i]);  // fp32, fp64 and integers convert from their own value
}

// Four consecutive elements of T in one aligned load / store.
template <typename T> struct alignas(4 * sizeof(T)) Quad {
    T e[4];
};

// One aligned load of a streamed input, marked non-temporal (`nt`: evict-first in L2): the
// elementwise, cast and transpose kernels read every input element exactly once, so keeping
// it in the caches only displaces other data.  a + b on two 256 MiB fp32 tensors: 5989 ->
// 6811 GB/s in a probe (non-temporal stores as well: 6527; stores stay ordinary).  The row
// reductions keep ordinary loads: same-process A/B, the hint there was 0-2 % slower.
template <typename Q> __device__ __forceinline__ Q load_stream(const Q *p) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    if constexpr (sizeof(Q) == 4) {
        return __builtin_bit_cast(Q, __builtin_nontemporal_load(reinterpret_cast<const unsigned *>(p)));
    } else if constexpr (sizeof(Q) == 8) {
        return __builtin_bit_cast(Q, __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p)));
    } else if constexpr (sizeof(Q) == 16) {
        return __builtin_bit_cast(Q, __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p)));
    } else if constexpr (sizeof(Q) == 32) {
        struct Pair {
            u32x4 lo, hi;
        };
        const u32x4 *v = reinterpret_cast<const u32x4 *>(p);
        return __builtin_bit_cast(Q, Pair{__builtin_nontemporal_load(v), __builtin_nontemporal_load(v + 1)});
    } else {
        return *p;
    }
}

// VEC4: n % 4 == 0 and both pointers aligned to four elements (checked on the host), so each
// thread moves one Quad per step.
template <typename S, typename D, bool VEC4>
__global__ __launch_bounds__(256) void cast_kernel(const S *__restrict__ src, D *__restrict__ dst, int64_t n) {
    if constexpr (VEC4) {
        const Quad<S> *s4 = reinterpret_cast<const Quad<S> *>(src);
        Quad<D> *d4 = reinterpret_cast<Quad<D> *>(dst);
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n / 4;
             i += int64_t(gridDim.x) * blockDim.x) {
            const Quad<S> x = load_stream(s4 + i);
            Quad<D> y;
#pragma unroll
            for (int e = 0; e < 4; ++e) cast_one(x.e, y.e, e);
            d4[i] = y;
        }
    } else {
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
            cast_one(src, dst, i);
    }
}

template <typename C> __device__ __forceinline__ C arith(int op, C a, C b) {
    switch (op) {
        case CTATTN_OP_ADD: return a + b;
        case CTATTN_OP_SUB: return a - b;
        case CTATTN_OP_MUL: return a * b;
        case CTATTN_OP_DIV:
            if constexpr (std::is_integral_v<C>) {
                if (b == 0) return 0;
                if (b == -1) return C(uint64_t(0) - uint64_t(a));
            }
            return a / b;
        default:  // CTATTN_OP_MOD: integers only; 0 for floating types (tensor_kernels.cu:245)
            if constexpr (std::is_integral_v<C>) {
                if (b == 0 || b == -1) return 0;
                return a % b;
            } else {
                return C(0);
            }
    }
}

template <typename C> __device__ __forceinline__ bool compare(int op, C a, C b) {
    switch (op) {
        case CTATTN_OP_EQ: return a == b;
        case CTATTN_OP_NE: return a != b;
        case CTATTN_OP_LT: return a < b;
        case CTATTN_OP_LE: return a <= b;
        case CTATTN_OP_GT: return a > b;
        default: return a >= b;  // CTATTN_OP_GE
    }
}

// Broadcast geometry: the output shape and each operand's element strides (0 along a
// broadcast dimension), innermost dimension last.
struct Bcast {
    int64_t shape[kMaxDims];
    int64_t sa[kMaxDims];
    int64_t sb[kMaxDims];
    int32_t ndim;
    int32_t plain;  // both operands have the output's shape: offsets are the index itself
};

__device__ __forceinline__ void bcast_offsets(const Bcast &g, int64_t i, int64_t &oa, int64_t &ob) {
    if (g.plain) {
        oa = ob = i;
        return;
    }
    oa = ob = 0;
    for (int k = g.ndim - 1; k >= 0; --k) {
        const int64_t c = i % g.shape[k];
        i /= g.shape[k];
        oa += c * g.sa[k];
        ob += c * g.sb[k];
    }
}

// CMP: a comparison writing bool; otherwise arithmetic writing T (bool included).
template <typename T, bool CMP, typename O = std::conditional_t<CMP, bool, T>>
__global__ __launch_bounds__(256) void binary_kernel(int op, const T *__restrict__ a, const T *__restrict__ b,
                                                    O *__restrict__ out, Bcast g, int64_t n, int vec4) {
    if (vec4) {  // same shapes, n % 4 == 0, every pointer aligned to four elements
        const Quad<T> *a4 = reinterpret_cast<const Quad<T> *>(a), *b4 = reinterpret_cast<const Quad<T> *>(b);
        Quad<O> *o4 = reinterpret_cast<Quad<O> *>(out);
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n / 4;
             i += int64_t(gridDim.x) * blockDim.x) {
            const Quad<T> x = load_stream(a4 + i), y = load_stream(b4 + i);
            Quad<O> z;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (CMP) z.e[e] = compare(op, ldv(x.e, e), ldv(y.e, e));
                else stv(z.e, e, arith(op, ldv(x.e, e), ldv(y.e, e)));
            }
            o4[i] = z;
        }
        return;
    }
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        int64_t oa, ob;
        bcast_offsets(g, i, oa, ob);
        const calc_t<T> x = ldv(a, oa), y = ldv(b, ob);
        if constexpr (CMP) out[i] = compare(op, x, y);
        else stv(out, i, arith(op, x, y));
    }
}

// a op s (scalar_left = 0) or s op a (scalar_left = 1).
template <typename T, bool CMP, typename O = std::conditional_t<CMP, bool, T>>
__global__ __launch_bounds__(256) void scalar_kernel(int op, const T *__restrict__ a, double s, int scalar_left,
                                                    O *__restrict__ out, int64_t n) {
    const calc_t<T> y = scalar_as<T>(s);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const calc_t<T> x = ldv(a, i);
        const calc_t<T> l = scalar_left ? y : x, r = scalar_left ? x : y;
        if constexpr (CMP) out[i] = compare(op, l, r);
        else stv(out, i, arith(op, l, r));
    }
}

template <typename T>
__global__ __launch_bounds__(256) void unary_kernel(int op, const T *__restrict__ a, T *__restrict__ out, int64_t n) {
    using C = calc_t<T>;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const C x = ldv(a, i);
        if constexpr (std::is_same_v<T, bool>) {  // NEG and NOT are logical not (tensor_kernels.cu:176)
            out[i] = (op == CTATTN_UN_ABS || op == CTATTN_UN_SQR) ? x != 0 : x == 0;
            continue;
        }
        switch (op) {
            case CTATTN_UN_NEG:
                if constexpr (std::is_integral_v<C>) stv(out, i, C(uint64_t(0) - uint64_t(x)));
                else stv(out, i, -x);
                break;
            case CTATTN_UN_NOT:
                if constexpr (std::is_integral_v<C>) stv(out, i, ~x);
                else stv(out, i, C(x == C(0)));
                break;
            case CTATTN_UN_INV:
                if constexpr (std::is_integral_v<C>) stv(out, i, x == 0 ? C(0) : C(1) / x);
                else stv(out, i, C(1) / x);
                break;
            case CTATTN_UN_EXP:
                if constexpr (std::is_integral_v<C>) stv(out, i, exp(double(x)));
                else stv(out, i, acc_exp(x));
                break;
            case CTATTN_UN_LOG:
                if constexpr (std::is_integral_v<C>) stv(out, i, log(double(x)));
                else stv(out, i, acc_log(x));
                break;
            case CTATTN_UN_SQR: stv(out, i, C(x * x)); break;
            case CTATTN_UN_SQRT:
                if constexpr (std::is_integral_v<C>) stv(out, i, sqrt(double(x)));
                else stv(out, i, acc_sqrt(x));
                break;
            default: stv(out, i, x < C(0) ? C(C(0) - x) : x); break;  // CTATTN_UN_ABS
        }
    }
}

// ---- reductions: [outer][R][inner] -> [outer][inner] ----------------------------------------

template <typename C> __device__ __forceinline__ C red_init(int op) {
    if (op == CTATTN_RED_MAX) {
        if constexpr (std::is_integral_v<C>) return INT64_MIN;
        else return C(-INFINITY);
    }
    if (op == CTATTN_RED_MIN) {
        if constexpr (std::is_integral_v<C>) return INT64_MAX;
        else return C(INFINITY);
    }
    return C(0);
}
// One element folded into a partial result.
template <typename C> __device__ __forceinline__ C red_elem(int op, C acc, C x) {
    switch (op) {
        case CTATTN_RED_MAX: return x > acc ? x : acc;
        case CTATTN_RED_MIN: return x < acc ? x : acc;
        case CTATTN_RED_NORM_L1: return acc + (x < C(0) ? C(C(0) - x) : x);
        case CTATTN_RED_NORM_L2: return acc + x * x;
        default: return acc + x;  // SUM, MEAN
    }
}
// Two partial results combined.
template <typename C> __device__ __forceinline__ C red_join(int op, C a, C b) {
    if (op == CTATTN_RED_MAX) return b > a ? b : a;
    if (op == CTATTN_RED_MIN) return b < a ? b : a;
    return a + b;
}
template <typename C> __device__ __forceinline__ C red_final(int op, C acc, int64_t R) {
    if (op == CTATTN_RED_MEAN) return acc / C(R);
    if (op == CTATTN_RED_NORM_L2) {
        if constexpr (std::is_integral_v<C>) return C(sqrt(double(acc)));
        else return acc_sqrt(acc);
    }
    return acc;
}

template <typename C> __device__ __forceinline__ C wave_join(int op, C x) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x = red_join(op, x, C(__shfl_xor(x, off, kWave)));
    return x;
}

// inner == 1, stage 1: workgroup (o, s) folds elements [s*chunk, (s+1)*chunk) of row o; the
// four wave results are joined in wave order.
// VEC: 16-byte loads (the row base and the chunk bounds are multiples of 16 bytes, checked on
// the host); each thread folds its vector's elements in order.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void reduce_rows_kernel(int op, const T *__restrict__ a, int64_t R, int64_t chunk,
                                                         calc_t<T> *__restrict__ part, int S) {
    using C = calc_t<T>;
    __shared__ C waves[4];
    const int64_t o = blockIdx.x, s = blockIdx.y;
    const int64_t r0 = s * chunk, r1 = min(R, r0 + chunk);
    // Four independent partial results per thread keep four loads in flight; they are joined
    // in a fixed order.
    const T *row = a + o * R;
    C acc0 = red_init<C>(op), acc1 = acc0, acc2 = acc0, acc3 = acc0;
    if constexpr (VEC) {
        constexpr int V = 16 / int(sizeof(T));
        struct alignas(16) Vec {
            T e[V];
        };
        const Vec *vrow = reinterpret_cast<const Vec *>(row);
        const int64_t v0 = r0 / V, v1 = r1 / V;
        auto fold = [&](C acc, const Vec &x) {
#pragma unroll
            for (int e = 0; e < V; ++e) acc = red_elem(op, acc, ldv(x.e, e));
            return acc;
        };
        int64_t v = v0 + threadIdx.x;
        for (; v + 3 * int64_t(blockDim.x) < v1; v += 4 * int64_t(blockDim.x)) {
            const Vec x0 = vrow[v], x1 = vrow[v + blockDim.x], x2 = vrow[v + 2 * blockDim.x],
                      x3 = vrow[v + 3 * blockDim.x];
            acc0 = fold(acc0, x0);
            acc1 = fold(acc1, x1);
            acc2 = fold(acc2, x2);
            acc3 = fold(acc3, x3);
        }
        for (; v < v1; v += blockDim.x) acc0 = fold(acc0, vrow[v]);
    } else {
        int64_t r = r0 + threadIdx.x;
        for (; r + 3 * int64_t(blockDim.x) < r1; r += 4 * int64_t(blockDim.x)) {
            const C x0 = ldv(row, r), x1 = ldv(row, r + blockDim.x), x2 = ldv(row, r + 2 * blockDim.x),
                    x3 = ldv(row, r + 3 * blockDim.x);
            acc0 = red_elem(op, acc0, x0);
            acc1 = red_elem(op, acc1, x1);
            acc2 = red_elem(op, acc2, x2);
            acc3 = red_elem(op, acc3, x3);
        }
        for (; r < r1; r += blockDim.x) acc0 = red_elem(op, acc0, ldv(row, r));
    }
    C acc = red_join(op, red_join(op, acc0, acc1), red_join(op, acc2, acc3));
    acc = wave_join(op, acc);
    if ((threadIdx.x & (kWave - 1)) == 0) waves[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
        part[o * S + s] = red_join(op, red_join(op, waves[0], waves[1]), red_join(op, waves[2], waves[3]));
}

// inner > 1, stage 1: thread (o, s, i) folds rows [s*chunk, (s+1)*chunk) of column i.
template <typename T>
__global__ __launch_bounds__(256) void reduce_cols_kernel(int op, const T *__restrict__ a, int64_t R, int64_t inner,
                                                         int64_t chunk, calc_t<T> *__restrict__ part) {
    using C = calc_t<T>;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= inner) return;
    const int64_t o = blockIdx.y, s = blockIdx.z, S = gridDim.z;
    const int64_t r0 = s * chunk, r1 = min(R, r0 + chunk);
    C acc = red_init<C>(op);
    for (int64_t r = r0; r < r1; ++r) acc = red_elem(op, acc, ldv(a, (o * R + r) * inner + i));
    part[(o * S + s) * inner + i] = acc;
}

// Stage 2: output (o, i) joins its S partials part[(o*S + s)*inner + i] in order of s.
template <typename T>
__global__ __launch_bounds__(256) void reduce_final_kernel(int op, const calc_t<T> *__restrict__ part, int64_t outer,
                                                          int64_t inner, int S, int64_t R, T *__restrict__ out) {
    using C = calc_t<T>;
    const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (j >= outer * inner) return;
    const int64_t o = j / inner, i = j - o * inner;
    C acc = part[(o * S) * inner + i];
    for (int s = 1; s < S; ++s) acc = red_join(op, acc, part[(o * S + s) * inner + i]);
    stv(out, j, red_final(op, acc, R));
}

// Stage 2 for few outputs: one workgroup per output; thread t joins partials t, t + 256, ...
// in order, then the 256 results meet in a fixed order (waves, then the four wave results).
template <typename T>
__global__ __launch_bounds__(256) void reduce_final_wide_kernel(int op, const calc_t<T> *__restrict__ part,
                                                               int64_t inner, int S, int64_t R,
                                                               T *__restrict__ out) {
    using C = calc_t<T>;
    __shared__ C waves[4];
    const int64_t j = blockIdx.x;
    const int64_t o = j / inner, i = j - o * inner;
    C acc = red_init<C>(op);
    for (int s = threadIdx.x; s < S; s += blockDim.x) acc = red_join(op, acc, part[(o * S + s) * inner + i]);
    acc = wave_join(op, acc);
    if ((threadIdx.x & (kWave - 1)) == 0) waves[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
        stv(out, j, red_final(op, red_join(op, red_join(op, waves[0], waves[1]), red_join(op, waves[2], waves[3])), R));
}

// ---- permutation, Kronecker product, integer matmul ---------------------------------------

struct Perm {
    int64_t out_shape[kMaxDims];
    int64_t in_stride[kMaxDims];  // input stride of the input axis that output axis k takes
    int32_t ndim;
};

template <typename W>
__global__ __launch_bounds__(256) void permute_kernel(const W *__restrict__ a, W *__restrict__ out, Perm g, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        int64_t rem = i, off = 0;
        for (int k = g.ndim - 1; k >= 0; --k) {
            const int64_t c = rem % g.out_shape[k];
            rem /= g.out_shape[k];
            off += c * g.in_stride[k];
        }
        out[i] = a[off];
    }
}

// out[z][c][r] = in[z][r][c] (the last two axes swapped) through a 64 x 64 LDS tile: reads and
// writes both coalesced.  Grid (ceil(C / 64), ceil(R / 64), Z), 256 threads.
template <typename W>
__global__ __launch_bounds__(256) void transpose2d_kernel(const W *__restrict__ a, W *__restrict__ out, int64_t R,
                                                         int64_t C) {
    __shared__ W tile[64][65];
    const int64_t z = blockIdx.z;
    const int64_t c0 = int64_t(blockIdx.x) * 64, r0 = int64_t(blockIdx.y) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const W *src = a + z * R * C;
    W *dst = out + z * R * C;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int64_t r = r0 + ty + 4 * i, c = c0 + tx;
        if (r < R && c < C) tile[ty + 4 * i][tx] = load_stream(src + r * C + c);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int64_t c = c0 + ty + 4 * i, r = r0 + tx;
        if (r < R && c < C) dst[c * R + r] = tile[tx][ty + 4 * i];
    }
}

struct Kron {
    int64_t a_shape[kMaxDims], b_shape[kMaxDims];
    int32_t ndim;
};

template <typename T>
__global__ __launch_bounds__(256) void kron_kernel(const T *__restrict__ a, const T *__restrict__ b, T *__restrict__ out,
                                                  Kron g, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        int64_t rem = i, oa = 0, ob = 0, sa = 1, sb = 1;
        for (int k = g.ndim - 1; k >= 0; --k) {
            const int64_t extent = g.a_shape[k] * g.b_shape[k];
            const int64_t c = rem % extent;
            rem /= extent;
            oa += (c / g.b_shape[k]) * sa;
            ob += (c % g.b_shape[k]) * sb;
            sa *= g.a_shape[k];
            sb *= g.b_shape[k];
        }
        stv(out, i, ldv(a, oa) * ldv(b, ob));
    }
}

// C[z] = A[z] B[z or 0] for the integer and bool types (and any type when K == 0): one thread
// per output, sums in the arithmetic type.
template <typename T>
__global__ __launch_bounds__(256) void matmul_int_kernel(const T *__restrict__ a, const T *__restrict__ b,
                                                        T *__restrict__ c, int64_t batch, int64_t batch_b, int64_t M,
                                                        int64_t K, int64_t N) {
    const int64_t n = batch * M * N;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t z = i / (M * N), mn = i - z * M * N, m = mn / N, col = mn - m * N;
        const T *ar = a + (z * M + m) * K;
        const T *bc = b + (batch_b == 1 ? 0 : z) * K * N + col;
        calc_t<T> s = 0;
        for (int64_t k = 0; k < K; ++k) s += ldv(ar, k) * ldv(bc, k * N);
        stv(c, i, s);
    }
}

unsigned grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return unsigned(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace
}  // namespace ctattn

namespace {

using ctattn::bf16_t;
using ctattn::calc_t;
using ctattn::f16_t;
using ctattn::capi::align_up;
using ctattn::capi::fail;
using ctattn::capi::finish;
using ctattn::capi::ok;

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

bool known(int dtype) { return dtype >= CTATTN_F32 && dtype <= CTATTN_BOOL; }
int64_t elem_size(int dtype) {
    switch (dtype) {
        case CTATTN_F64:
        case CTATTN_I64: return 8;
        case CTATTN_F32:
        case CTATTN_I32: return 4;
        case CTATTN_BF16:
        case CTATTN_F16:
        case CTATTN_I16: return 2;
        default: return 1;
    }
}
int64_t calc_size(int dtype) {
    return (dtype == CTATTN_F32 || dtype == CTATTN_BF16 || dtype == CTATTN_F16) ? 4 : 8;
}

// Calls f with a null pointer of the storage type of `dtype` (checked beforehand).
template <typename F>
hipError_t by_type(int dtype, F &&f) {
    switch (dtype) {
        case CTATTN_F32: return f(static_cast<float *>(nullptr));
        case CTATTN_BF16: return f(static_cast<bf16_t *>(nullptr));
        case CTATTN_F16: return f(static_cast<f16_t *>(nullptr));
        case CTATTN_F64: return f(static_cast<double *>(nullptr));
        case CTATTN_I32: return f(static_cast<int32_t *>(nullptr));
        case CTATTN_I64: return f(static_cast<int64_t *>(nullptr));
        case CTATTN_I16: return f(static_cast<int16_t *>(nullptr));
        case CTATTN_I8: return f(static_cast<int8_t *>(nullptr));
        default: return f(static_cast<bool *>(nullptr));
    }
}

int check_dims(const char *fn, int ndim, const int64_t *shape) {
    if (ndim < 0 || ndim > ctattn::kMaxDims) return fail(hipErrorInvalidValue, "%s: ndim must be 0..8", fn);
    for (int k = 0; k < ndim; ++k)
        if (shape == nullptr || shape[k] < 0) return fail(hipErrorInvalidValue, "%s: invalid shape", fn);
    return 0;
}

int64_t numel(int ndim, const int64_t *shape) {
    int64_t n = 1;
    for (int k = 0; k < ndim; ++k) n *= shape[k];
    return n;
}

// Reduction split: S stage-1 partials per output, chosen to give the GPU about 1024
// workgroups (rows) or 256K threads (columns) without chunks shorter than 1024 / 64 elements.
int reduce_splits(int64_t outer, int64_t R, int64_t inner) {
    int64_t s;
    if (inner == 1) s = std::min<int64_t>((1024 + outer - 1) / outer, (R + 1023) / 1024);
    else s = std::min<int64_t>((262144 + outer * inner - 1) / (outer * inner), (R + 63) / 64);
    return int(std::max<int64_t>(1, std::min<int64_t>(s, 65535)));
}

}  // namespace

extern "C" {

int ctattn_tensor_cast(int src_dtype, const void *src, int dst_dtype, void *dst, int64_t n, void *stream) {
    const char *fn = "ctattn_tensor_cast";
    if (!known(src_dtype) || !known(dst_dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype", fn);
    if (n < 0) return fail(hipErrorInvalidValue, "%s: negative size", fn);
    if (n == 0) return ok();
    if (!src || !dst) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_type(src_dtype, [&](auto *stag) {
        using S = std::remove_pointer_t<decltype(stag)>;
        return by_type(dst_dtype, [&](auto *dtag) {
            using D = std::remove_pointer_t<decltype(dtag)>;
            const bool v4 = n % 4 == 0 && uintptr_t(src) % (4 * sizeof(S)) == 0 && uintptr_t(dst) % (4 * sizeof(D)) == 0;
            if (v4)
                hipLaunchKernelGGL((ctattn::cast_kernel<S, D, true>), dim3(ctattn::grid_for(n / 4)), dim3(256), 0, st,
                                   static_cast<const S *>(src), static_cast<D *>(dst), n);
            else
                hipLaunchKernelGGL((ctattn::cast_kernel<S, D, false>), dim3(ctattn::grid_for(n)), dim3(256), 0, st,
                                   static_cast<const S *>(src), static_cast<D *>(dst), n);
            return hipGetLastError();
        });
    });
    return finish(fn, e, st);
}

int ctattn_tensor_binary(int dtype, int op, const void *a, int a_ndim, const int64_t *a_shape, const void *b,
                         int b_ndim, const int64_t *b_shape, void *out, void *stream) {
    const char *fn = "ctattn_tensor_binary";
    if (!known(dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype %d", fn, dtype);
    if (op < CTATTN_OP_ADD || op > CTATTN_OP_GE) return fail(hipErrorInvalidValue, "%s: unknown op %d", fn, op);
    if (int rc = check_dims(fn, a_ndim, a_shape)) return rc;
    if (int rc = check_dims(fn, b_ndim, b_shape)) return rc;
    ctattn::Bcast g{};
    g.ndim = std::max(a_ndim, b_ndim);
    g.plain = a_ndim == b_ndim;
    int64_t stride_a = 1, stride_b = 1;
    for (int k = g.ndim - 1; k >= 0; --k) {
        const int ka = k - (g.ndim - a_ndim), kb = k - (g.ndim - b_ndim);
        const int64_t da = ka >= 0 ? a_shape[ka] : 1, db = kb >= 0 ? b_shape[kb] : 1;
        if (da != db && da != 1 && db != 1)
            return fail(hipErrorInvalidValue, "%s: shapes do not broadcast (dimension %d: %lld vs %lld)", fn, k,
                        (long long)da, (long long)db);
        g.shape[k] = da == 1 ? db : da;  // a 1 stretches to the other extent, 0 included
        if (da != db) g.plain = 0;
        g.sa[k] = da == 1 ? 0 : stride_a;
        g.sb[k] = db == 1 ? 0 : stride_b;
        stride_a *= da;
        stride_b *= db;
    }
    const int64_t n = numel(g.ndim, g.shape);
    if (n == 0) return ok();
    if (!a || !b || !out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_type(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        const uintptr_t al = 4 * sizeof(T), ol = op >= CTATTN_OP_EQ ? 4 : al;
        const int v4 = g.plain && n % 4 == 0 && uintptr_t(a) % al == 0 && uintptr_t(b) % al == 0 &&
                       uintptr_t(out) % ol == 0;
        const dim3 grid(ctattn::grid_for(v4 ? n / 4 : n));
        if (op >= CTATTN_OP_EQ)
            hipLaunchKernelGGL((ctattn::binary_kernel<T, true>), grid, dim3(256), 0, st, op, static_cast<const T *>(a),
                               static_cast<const T *>(b), static_cast<bool *>(out), g, n, v4);
        else
            hipLaunchKernelGGL((ctattn::binary_kernel<T, false>), grid, dim3(256), 0, st, op, static_cast<const T *>(a),
                               static_cast<const T *>(b), static_cast<T *>(out), g, n, v4);
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_tensor_scalar(int dtype, int op, const void *a, double scalar, int scalar_left, void *out, int64_t n,
                         void *stream) {
    const char *fn = "ctattn_tensor_scalar";
    if (!known(dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype %d", fn, dtype);
    if (op < CTATTN_OP_ADD || op > CTATTN_OP_GE) return fail(hipErrorInvalidValue, "%s: unknown op %d", fn, op);
    if (n < 0) return fail(hipErrorInvalidValue, "%s: negative size", fn);
    if (n == 0) return ok();
    if (!a || !out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_type(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        if (op >= CTATTN_OP_EQ)
            hipLaunchKernelGGL((ctattn::scalar_kernel<T, true>), dim3(ctattn::grid_for(n)), dim3(256), 0, st, op,
                               static_cast<const T *>(a), scalar, scalar_left ? 1 : 0, static_cast<bool *>(out), n);
        else
            hipLaunchKernelGGL((ctattn::scalar_kernel<T, false>), dim3(ctattn::grid_for(n)), dim3(256), 0, st, op,
                               static_cast<const T *>(a), scalar, scalar_left ? 1 : 0, static_cast<T *>(out), n);
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_tensor_unary(int dtype, int op, const void *a, void *out, int64_t n, void *stream) {
    const char *fn = "ctattn_tensor_unary";
    if (!known(dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype %d", fn, dtype);
    if (op < CTATTN_UN_NEG || op > CTATTN_UN_ABS) return fail(hipErrorInvalidValue, "%s: unknown op %d", fn, op);
    if (n < 0) return fail(hipErrorInvalidValue, "%s: negative size", fn);
    if (n == 0) return ok();
    if (!a || !out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_type(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::unary_kernel<T>, dim3(ctattn::grid_for(n)), dim3(256), 0, st, op,
                           static_cast<const T *>(a), static_cast<T *>(out), n);
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int64_t ctattn_tensor_reduce_workspace_bytes(int dtype, int64_t outer, int64_t R, int64_t inner) {
    if (!known(dtype) || outer < 0 || R < 1 || inner < 0) {
        fail(hipErrorInvalidValue, "ctattn_tensor_reduce_workspace_bytes: invalid arguments");
        return -1;
    }
    ok();
    return align_up(int64_t(reduce_splits(std::max<int64_t>(outer, 1), R, std::max<int64_t>(inner, 1))) *
                    std::max<int64_t>(outer, 1) * std::max<int64_t>(inner, 1) * calc_size(dtype));
}

int ctattn_tensor_reduce(int dtype, int op, const void *a, int64_t outer, int64_t R, int64_t inner, void *out,
                         void *workspace, int64_t workspace_bytes, void *stream) {
    const char *fn = "ctattn_tensor_reduce";
    if (!known(dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype %d", fn, dtype);
    if (op < CTATTN_RED_SUM || op > CTATTN_RED_NORM_L2) return fail(hipErrorInvalidValue, "%s: unknown op %d", fn, op);
    if (outer < 0 || inner < 0) return fail(hipErrorInvalidValue, "%s: negative size", fn);
    if (R < 1) return fail(hipErrorInvalidValue, "%s: the reduced extent must be >= 1", fn);
    if (outer == 0 || inner == 0) return ok();
    if (outer > 2147483647 || (inner > 1 && outer > 65535))
        return fail(hipErrorInvalidValue, "%s: too many outputs along the leading dimensions", fn);
    if (!a || !out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    const int64_t need = ctattn_tensor_reduce_workspace_bytes(dtype, outer, R, inner);
    if (workspace == nullptr || workspace_bytes < need)
        return fail(hipErrorInvalidValue, "%s: workspace of %lld bytes given, %lld needed", fn,
                    (long long)workspace_bytes, (long long)need);
    const int S = reduce_splits(outer, R, inner);
    int64_t chunk = (R + S - 1) / S;
    // 16-byte loads along contiguous rows when the rows and chunks stay 16-byte aligned.
    const int64_t vw = 16 / elem_size(dtype);
    const bool vec = inner == 1 && uintptr_t(a) % 16 == 0 && R % vw == 0;
    if (vec) chunk = (chunk + vw - 1) / vw * vw;
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_type(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using C = calc_t<T>;
        C *part = static_cast<C *>(workspace);
        if (inner == 1 && vec)
            hipLaunchKernelGGL((ctattn::reduce_rows_kernel<T, true>), dim3(unsigned(outer), unsigned(S)), dim3(256), 0,
                               st, op, static_cast<const T *>(a), R, chunk, part, S);
        else if (inner == 1)
            hipLaunchKernelGGL((ctattn::reduce_rows_kernel<T, false>), dim3(unsigned(outer), unsigned(S)), dim3(256),
                               0, st, op, static_cast<const T *>(a), R, chunk, part, S);
        else
            hipLaunchKernelGGL(ctattn::reduce_cols_kernel<T>,
                               dim3(unsigned((inner + 255) / 256), unsigned(outer), unsigned(S)), dim3(256), 0, st, op,
                               static_cast<const T *>(a), R, inner, chunk, part);
        hipError_t le = hipGetLastError();
        if (le != hipSuccess) return le;
        if (outer * inner <= 4096 && S >= 64)
            hipLaunchKernelGGL(ctattn::reduce_final_wide_kernel<T>, dim3(unsigned(outer * inner)), dim3(256), 0, st,
                               op, static_cast<const C *>(part), inner, S, R, static_cast<T *>(out));
        else
            hipLaunchKernelGGL(ctattn::reduce_final_kernel<T>, dim3(unsigned((outer * inner + 255) / 256)), dim3(256),
                               0, st, op, static_cast<const C *>(part), outer, inner, S, R, static_cast<T *>(out));
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_tensor_permute(int dtype, const void *a, int ndim, const int64_t *shape, const int32_t *perm, void *out,
                          void *stream) {
    const char *fn = "ctattn_tensor_permute";
    if (!known(dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype %d", fn, dtype);
    if (int rc = check_dims(fn, ndim, shape)) return rc;
    if (ndim > 0 && perm == nullptr) return fail(hipErrorInvalidValue, "%s: null perm", fn);
    bool seen[ctattn::kMaxDims] = {};
    for (int k = 0; k < ndim; ++k) {
        if (perm[k] < 0 || perm[k] >= ndim || seen[perm[k]])
            return fail(hipErrorInvalidValue, "%s: perm is not a permutation of 0..%d", fn, ndim - 1);
        seen[perm[k]] = true;
    }
    ctattn::Perm g{};
    g.ndim = ndim;
    int64_t in_stride[ctattn::kMaxDims];
    int64_t s = 1;
    for (int k = ndim - 1; k >= 0; --k) {
        in_stride[k] = s;
        s *= shape[k];
    }
    for (int k = 0; k < ndim; ++k) {
        g.out_shape[k] = shape[perm[k]];
        g.in_stride[k] = in_stride[perm[k]];
    }
    const int64_t n = numel(ndim, shape);
    if (n == 0) return ok();
    if (!a || !out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    // The last two axes swapped, the others in place: batched tiled transpose.
    bool swap_last = ndim >= 2 && perm[ndim - 1] == ndim - 2 && perm[ndim - 2] == ndim - 1;
    for (int k = 0; k + 2 < ndim && swap_last; ++k) swap_last = perm[k] == k;
    if (swap_last) {
        const int64_t R = shape[ndim - 2], C = shape[ndim - 1], Z = n / (R * C);
        if (Z <= 65535 && (R + 63) / 64 <= 65535) {
            const dim3 g2(unsigned((C + 63) / 64), unsigned((R + 63) / 64), unsigned(Z));
            switch (elem_size(dtype)) {
                case 8:
                    hipLaunchKernelGGL(ctattn::transpose2d_kernel<uint64_t>, g2, dim3(256), 0, st,
                                       static_cast<const uint64_t *>(a), static_cast<uint64_t *>(out), R, C);
                    break;
                case 4:
                    hipLaunchKernelGGL(ctattn::transpose2d_kernel<uint32_t>, g2, dim3(256), 0, st,
                                       static_cast<const uint32_t *>(a), static_cast<uint32_t *>(out), R, C);
                    break;
                case 2:
                    hipLaunchKernelGGL(ctattn::transpose2d_kernel<uint16_t>, g2, dim3(256), 0, st,
                                       static_cast<const uint16_t *>(a), static_cast<uint16_t *>(out), R, C);
                    break;
                default:
                    hipLaunchKernelGGL(ctattn::transpose2d_kernel<uint8_t>, g2, dim3(256), 0, st,
                                       static_cast<const uint8_t *>(a), static_cast<uint8_t *>(out), R, C);
            }
            return finish(fn, hipGetLastError(), st);
        }
    }
    const dim3 grid(ctattn::grid_for(n));
    switch (elem_size(dtype)) {
        case 8:
            hipLaunchKernelGGL(ctattn::permute_kernel<uint64_t>, grid, dim3(256), 0, st,
                               static_cast<const uint64_t *>(a), static_cast<uint64_t *>(out), g, n);
            break;
        case 4:
            hipLaunchKernelGGL(ctattn::permute_kernel<uint32_t>, grid, dim3(256), 0, st,
                               static_cast<const uint32_t *>(a), static_cast<uint32_t *>(out), g, n);
            break;
        case 2:
            hipLaunchKernelGGL(ctattn::permute_kernel<uint16_t>, grid, dim3(256), 0, st,
                               static_cast<const uint16_t *>(a), static_cast<uint16_t *>(out), g, n);
            break;
        default:
            hipLaunchKernelGGL(ctattn::permute_kernel<uint8_t>, grid, dim3(256), 0, st, static_cast<const uint8_t *>(a),
                               static_cast<uint8_t *>(out), g, n);
    }
    return finish(fn, hipGetLastError(), st);
}

int ctattn_tensor_kron(int dtype, const void *a, const void *b, int ndim, const int64_t *a_shape,
                       const int64_t *b_shape, void *out, void *stream) {
    const char *fn = "ctattn_tensor_kron";
    if (!known(dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype %d", fn, dtype);
    if (int rc = check_dims(fn, ndim, a_shape)) return rc;
    if (int rc = check_dims(fn, ndim, b_shape)) return rc;
    ctattn::Kron g{};
    g.ndim = ndim;
    int64_t n = 1;
    for (int k = 0; k < ndim; ++k) {
        g.a_shape[k] = a_shape[k];
        g.b_shape[k] = b_shape[k];
        n *= a_shape[k] * b_shape[k];
    }
    if (n == 0) return ok();
    if (!a || !b || !out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    const hipError_t e = by_type(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(ctattn::kron_kernel<T>, dim3(ctattn::grid_for(n)), dim3(256), 0, st,
                           static_cast<const T *>(a), static_cast<const T *>(b), static_cast<T *>(out), g, n);
        return hipGetLastError();
    });
    return finish(fn, e, st);
}

int ctattn_tensor_matmul(int dtype, const void *a, const void *b, void *c, int64_t batch, int64_t batch_b, int64_t M,
                         int64_t K, int64_t N, void *stream) {
    const char *fn = "ctattn_tensor_matmul";
    if (!known(dtype)) return fail(hipErrorInvalidValue, "%s: unknown dtype %d", fn, dtype);
    if (batch < 0 || M < 0 || K < 0 || N < 0 || (batch_b != 1 && batch_b != batch))
        return fail(hipErrorInvalidValue, "%s: need sizes >= 0 and batch_b == 1 or batch", fn);
    if (batch * M * N == 0) return ok();
    if (!c || (K > 0 && (!a || !b))) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    if (dtype > CTATTN_F64 || K == 0) {
        const hipError_t e = by_type(dtype, [&](auto *tag) {
            using T = std::remove_pointer_t<decltype(tag)>;
            hipLaunchKernelGGL(ctattn::matmul_int_kernel<T>, dim3(ctattn::grid_for(batch * M * N)), dim3(256), 0, st,
                               static_cast<const T *>(a), static_cast<const T *>(b), static_cast<T *>(c), batch,
                               batch_b, M, K, N);
            return hipGetLastError();
        });
        return finish(fn, e, st);
    }
    // fp32 / bf16 / fp16 on the plain GEMMs of linear_gemm.hip (A [M][K] K-contiguous, B stored
    // [K][N]): one launch when the batches stack (one B), one per batch for up to 16 batches.
    const int64_t rows = batch_b == 1 ? batch * M : M;
    if ((dtype == CTATTN_F32 || dtype == CTATTN_BF16 || dtype == CTATTN_F16) &&
        ctattn_get_policy() != CTATTN_POLICY_GENERIC && (batch_b == 1 || batch <= 16)) {
        const int ld = dtype == CTATTN_F32 ? 0 : dtype == CTATTN_BF16 ? 1 : 2;
        const int64_t es1 = elem_size(dtype);
        const int64_t calls = batch_b == 1 ? 1 : batch;
        auto product = [&](int64_t z) {
            return ctattn::lin_plain(ld, true, false, rows, N, K, static_cast<const char *>(a) + z * M * K * es1, K,
                                     static_cast<const char *>(b) + z * K * N * es1, N,
                                     static_cast<char *>(c) + z * M * N * es1, N, nullptr, false);
        };
        bool all = true;
        for (int64_t z = 0; z < calls && all; ++z) all = ctattn::lin_gemm_supported(product(z));
        for (int64_t z = 0; z < calls && all; ++z) {
            const hipError_t e = ctattn::launch_lin_gemm(product(z), nullptr, 0, st);
            if (e != hipSuccess) return finish(fn, e, st);
        }
        if (all) return finish(fn, hipSuccess, st);
    }
    // The projection GEMMs: A [M][K] K-contiguous, B stored [K][N].  With one B the batches
    // stack into one product of batch * M rows.
    if (rows > 2147483647 || N > 2147483647 || K > 2147483647)
        return fail(hipErrorInvalidValue, "%s: sizes must be below 2^31", fn);
    const int64_t es = elem_size(dtype);
    const bool v4 = rows % 4 == 0 && N % 4 == 0 && K % 4 == 0 &&
                    uintptr_t(a) % uintptr_t(4 * es) == 0 && uintptr_t(b) % uintptr_t(4 * es) == 0 &&
                    uintptr_t(c) % uintptr_t(4 * es) == 0;
    const int64_t launches = batch_b == 1 ? 1 : batch;
    for (int64_t z0 = 0; z0 < launches; z0 += ctattn::kMaxBatch) {
        ctattn::GemmParams p{};
        p.M = int32_t(rows);
        p.N = int32_t(N);
        p.K = int32_t(K);
        p.beta = 0;
        p.splits = 1;
        p.outv = ctattn::linear_view(nullptr, N);
        p.ws = nullptr;
        const int nb = int(std::min<int64_t>(ctattn::kMaxBatch, launches - z0));
        for (int j = 0; j < nb; ++j) {
            const int64_t z = z0 + j;
            ctattn::GemmBatch &bt = p.batch[j];
            bt.nseg = 1;
            bt.a[0] = ctattn::linear_view(static_cast<const char *>(a) + z * M * K * es, K);
            bt.b[0] = ctattn::linear_view(static_cast<const char *>(b) + z * K * N * es, N);
            bt.out = static_cast<char *>(c) + z * M * N * es;
            bt.bias = nullptr;
        }
        const hipError_t e = ctattn::launch_proj_gemm(dtype, p, nb, true, false, v4, st);
        if (e != hipSuccess) return finish(fn, e, st);
    }
    return finish(fn, hipSuccess, st);
}

}  // extern "C"
