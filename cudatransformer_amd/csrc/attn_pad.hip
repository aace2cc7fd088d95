// Row copies between [rows][d] tensors and [rows][dp] buffers (dp >= d) whose columns d ..
// dp - 1 are zero.  They let head dims without an MFMA kernel of their own (d <= 128, not 32,
// 64 or 128) run on the MFMA kernels of the next width: a zero column adds nothing to a
// score, and the padded columns of O, dQ, dK and dV come out zero and are not copied back.
// Plain bandwidth-bound passes, all tensors of one call in one launch (blockIdx.y picks the
// tensor).  Rows move in 16-byte chunks when d * element size is a multiple of 16 and every
// pointer is 16-byte aligned (dp * element size always is: dp in {32, 64, 128}), element by
// element otherwise; the all-zero bit pattern is 0.0 in every floating format.
#include "attn_launch.h"

#include <stdint.h>

namespace ctattn {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct RowCopies {
    const void *in[kMaxRowCopies];
    void *out[kMaxRowCopies];
};

// PAD: out[r][c] = c < d ? in[r][c] : 0 over the dp columns of every row; else out[r][c] =
// in[r][c] over the d leading columns of every dp-wide row.  Columns count units of E.
template <typename E, bool PAD>
__global__ __launch_bounds__(256) void row_copy_kernel(RowCopies job, int64_t rows, int d, int dp) {
    const E *__restrict__ in = static_cast<const E *>(job.in[blockIdx.y]);
    E *__restrict__ out = static_cast<E *>(job.out[blockIdx.y]);
    const int w = PAD ? dp : d;  // columns written per row
    const int64_t n = rows * w;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t r = i / w;
        const int c = int(i - r * w);
        if (PAD) {
            E x;
            if (c < d) x = in[r * d + c];
            else x = E{};
            out[i] = x;
        } else {
            out[i] = in[r * dp + c];
        }
    }
}

template <typename E, bool PAD>
hipError_t launch_copy(const RowCopies &job, int count, int64_t rows, int d, int dp, hipStream_t stream) {
    const int64_t n = rows * (PAD ? dp : d);
    if (n == 0 || count == 0) return hipSuccess;
    const unsigned grid = stride_grid((n + 255) / 256, 256);
    hipLaunchKernelGGL((row_copy_kernel<E, PAD>), dim3(grid, unsigned(count)), dim3(256), 0, stream, job, rows, d, dp);
    return hipGetLastError();
}

template <bool PAD>
hipError_t row_copies(int elem_bytes, const void *const *in, void *const *out, int count, int64_t rows, int d,
                      int dp, hipStream_t stream) {
    if (count < 0 || count > kMaxRowCopies || d < 1 || dp < d) return hipErrorInvalidValue;
    RowCopies job{};
    bool vec = (int64_t(d) * elem_bytes) % 16 == 0 && (int64_t(dp) * elem_bytes) % 16 == 0;
    for (int i = 0; i < count; ++i) {
        job.in[i] = in[i];
        job.out[i] = out[i];
        vec = vec && reinterpret_cast<uintptr_t>(in[i]) % 16 == 0 && reinterpret_cast<uintptr_t>(out[i]) % 16 == 0;
    }
    if (vec) return launch_copy<u32x4, PAD>(job, count, rows, d * elem_bytes / 16, dp * elem_bytes / 16, stream);
    switch (elem_bytes) {
        case 2: return launch_copy<uint16_t, PAD>(job, count, rows, d, dp, stream);
        case 4: return launch_copy<uint32_t, PAD>(job, count, rows, d, dp, stream);
        case 8: return launch_copy<uint64_t, PAD>(job, count, rows, d, dp, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_pad_rows(int elem_bytes, const void *const *in, void *const *out, int count, int64_t rows, int d,
                           int dp, hipStream_t stream) {
    return row_copies<true>(elem_bytes, in, out, count, rows, d, dp, stream);
}

hipError_t launch_unpad_rows(int elem_bytes, const void *const *in, void *const *out, int count, int64_t rows,
                             int d, int dp, hipStream_t stream) {
    return row_copies<false>(elem_bytes, in, out, count, rows, d, dp, stream);
}

}  // namespace ctattn
