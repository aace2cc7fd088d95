// fp32 dQ on fp32 MFMA, query-major and atomic-free (gfx950): the dQ half of the
// deterministic fp32 backward.
//
// Replaces the dQ accumulation of the reference's flashAttentionBackward<float>
// (flash_attention.cu:226-326: dQ_i += sum_j dS_ij K_j / sqrt(d) by atomicAdd, :311, :317)
// with a kernel that owns its rows: every dQ element is summed by one lane in a fixed key
// order and written once, so the result is bitwise reproducible and needs no workspace
// beyond delta.  dK and dV come from the 128-key kernel run without its dQ part
// (attn_bwd_k128.hip); the scores S and dP are computed by both kernels.
//
// Work decomposition: one workgroup = 4 waves = 128 query rows of one (batch, head); wave w
// owns rows 32 w .. 32 w + 31 for the whole key loop, which walks 32-key blocks (causal: up to
// the workgroup's last row).  K and V blocks go global -> LDS directly (padded rows, stride
// d + 4 floats), double-buffered with one barrier per block.  Per wave and block, on
// v_mfma_f32_32x32x2f32, everything is transposed so that each lane holds ONE query row:
//   S^T  = K Q^T       (A = K rows from LDS, B = Q^T scaled by log2(e)/sqrt(d) in registers)
//   dP^T = V dO^T      (A = V rows from LDS, B = dO^T in registers)
//   P^T  = exp2(S^T - LSE log2(e)),  dS^T = P^T (dP^T - delta)      (per-lane row terms)
//   dQ^T += K^T dS^T   (A = K columns from LDS, B = the dS^T accumulator registers as they
//                       are: register s holds key kstep_index(s, half), the k-step-s index)
// and dQ = (dQ^T)^T / sqrt(d) is stored row by row at the end.
#include "attn_launch.h"
#include "attn_mfma_common.h"

#include <math.h>

namespace ctattn {
namespace {

template <int D>
struct DqF32Cfg {
    static constexpr int NW = 4;
    static constexpr int BM = 32 * NW;  // query rows per workgroup
    static constexpr int BN = 32;       // keys per block
    static constexpr int DT = D / 32;   // 32-wide d tiles of dQ^T
    static constexpr int KS = D + 4;    // LDS row stride (floats): one pad chunk
    static constexpr int C4 = D / 4;    // 16-byte chunks of data per row
    static constexpr int C4P = C4 + 1;  // ... per LDS row
    static constexpr int TILE = BN * KS;
    static constexpr int CHUNKS = BN * C4P;
    static constexpr int INSTR = (CHUNKS + NW * kWave - 1) / (NW * kWave);  // loads per lane per tile
    static_assert(D == 32 || D == 64 || D == 128, "d in {32, 64, 128}");
};

#define CTATTN_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// Registers: d = 128 keeps Q^T, dO^T and dQ^T (64 each) and runs one wave per SIMD.
template <int D> struct DqF32Occupancy { static constexpr int waves = D <= 64 ? 2 : 1; };

// One 32-key block for one wave.  MASK: the block crosses the wave's diagonal or the
// sequence end (keys > row or >= T get P = 0).
template <int D, bool MASK>
__device__ __forceinline__ void dq_f32_block(floatx16 (&dq_acc)[D / 32], const float (&qreg)[D / 2],
                                             const float (&doreg)[D / 2], const float *k_lds, const float *v_lds,
                                             float nl2, float dl, int j0, int row, int T, int causal, int col,
                                             int half) {
    using C = DqF32Cfg<D>;
    floatx16 s = zero16(), dp = zero16();
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
        const floatx4 kv = *reinterpret_cast<const floatx4 *>(k_lds + col * C::KS + 8 * m + 4 * half);
        const floatx4 vv = *reinterpret_cast<const floatx4 *>(v_lds + col * C::KS + 8 * m + 4 * half);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            s = mfma32x32x2(kv[t], qreg[4 * m + t], s);
            dp = mfma32x32x2(vv[t], doreg[4 * m + t], dp);
        }
    }
    // lane = query row; register r = key j0 + acc_row(r, half)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(s[r] + nl2);
        if (MASK) {
            const int key = j0 + acc_row(r, half);
            p = (key >= T || (causal && key > row)) ? 0.f : p;
        }
        dp[r] = p * (dp[r] - dl);
    }
    // dQ^T += K^T dS^T over the block's 32 keys
#pragma unroll
    for (int st = 0; st < 16; ++st) {
        const int kl = kstep_index(st, half);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) dq_acc[dt] = mfma32x32x2(k_lds[kl * C::KS + dt * 32 + col], dp[st], dq_acc[dt]);
    }
}

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DqF32Occupancy<D>::waves,
                                                                     DqF32Occupancy<D>::waves))) void bwd_dq_f32_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    float *__restrict__ dq, int T, int BH, int causal, float qscale, float inv_sqrt_d) {
    using C = DqF32Cfg<D>;
    __shared__ __attribute__((aligned(16))) float k_lds[2][C::TILE];
    __shared__ __attribute__((aligned(16))) float v_lds[2][C::TILE];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int nqb = (T + C::BM - 1) / C::BM;
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int qb = causal ? (nqb - 1 - id / BH) : id / BH;  // causal: longest first
    const int64_t base = int64_t(bh) * T * D;
    const int64_t rbase = int64_t(bh) * T;
    const int r0 = qb * C::BM;
    const int wave_first_row = r0 + 32 * wave;
    const int wave_last_row = wave_first_row + 31;
    const int row = wave_first_row + col;

    // Q^T (scaled by log2(e)/sqrt(d)) and dO^T as B operands: lane (col = row, half) holds
    // element kstep_index(s, half) of its row.
    float qreg[D / 2], doreg[D / 2];
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
        floatx4 xq = {0.f, 0.f, 0.f, 0.f}, xd = {0.f, 0.f, 0.f, 0.f};
        if (row < T) {
            xq = *reinterpret_cast<const floatx4 *>(q + base + int64_t(row) * D + 8 * m + 4 * half);
            xd = *reinterpret_cast<const floatx4 *>(dout + base + int64_t(row) * D + 8 * m + 4 * half);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            qreg[4 * m + t] = xq[t] * qscale;
            doreg[4 * m + t] = xd[t];
        }
    }
    const float nl2 = row < T ? -lse[rbase + row] * kLog2e : 0.f;
    const float dl = row < T ? delta[rbase + row] : 0.f;

    floatx16 dq_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) dq_acc[dt] = zero16();

    const int kend = causal ? min(T, r0 + C::BM) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;

    // Global -> LDS for one block: lane writes LDS chunk P = (wave * INSTR + i) * 64 + lane of
    // the padded tile, i.e. row P / C4P, chunk P % C4P; the pad chunk re-reads chunk 0 of the
    // row and is never used.  Rows past T re-read row T - 1 (their P is 0).
    auto issue = [&](int j0, int buf) {
#pragma unroll
        for (int i = 0; i < C::INSTR; ++i) {
            const int P = (wave * C::INSTR + i) * kWave + lane;
            if (C::CHUNKS % (C::NW * kWave) == 0 || P < C::CHUNKS) {
                const int r = P / C::C4P;
                const int c = P - r * C::C4P;
                const int64_t goff = base + int64_t(min(j0 + r, T - 1)) * D + 4 * (c < C::C4 ? c : 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(k + goff),
                                                 CTATTN_LDS(&k_lds[buf][(wave * C::INSTR + i) * 4 * kWave]), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(v + goff),
                                                 CTATTN_LDS(&v_lds[buf][(wave * C::INSTR + i) * 4 * kWave]), 16, 0, 0);
            }
        }
    };

    issue(0, 0);
    for (int kb = 0; kb < nkb; ++kb) {
        const int j0 = kb * C::BN;
        const int buf = kb & 1;
        // This lane's loads into `buf` have landed; after the barrier every lane's have, and
        // every wave is done reading buf ^ 1.
        __builtin_amdgcn_s_waitcnt(0xF70);
        __syncthreads();
        if (kb + 1 < nkb) issue(j0 + C::BN, buf ^ 1);
        if (causal && j0 > wave_last_row) continue;  // keys wholly above this wave's rows
        const bool masked = (j0 + C::BN > T) || (causal && j0 + C::BN - 1 > wave_first_row);
        if (masked)
            dq_f32_block<D, true>(dq_acc, qreg, doreg, k_lds[buf], v_lds[buf], nl2, dl, j0, row, T, causal, col,
                                  half);
        else
            dq_f32_block<D, false>(dq_acc, qreg, doreg, k_lds[buf], v_lds[buf], nl2, dl, j0, row, T, causal, col,
                                   half);
    }

    // dq_acc[dt]: lane (col = row, half), register r -> column 32 dt + acc_row(r, half).
    if (row < T) {
        float *dqr = dq + base + int64_t(row) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                floatx4 x;
#pragma unroll
                for (int t = 0; t < 4; ++t) x[t] = dq_acc[dt][4 * g + t] * inv_sqrt_d;
                *reinterpret_cast<floatx4 *>(dqr + dt * 32 + 8 * g + 4 * half) = x;
            }
        }
    }
}

template <int D>
hipError_t launch_dq(const float *q, const float *k, const float *v, const float *dout, const float *lse,
                     const float *delta, float *dq, const AttnShape &s, hipStream_t stream) {
    using C = DqF32Cfg<D>;
    const int64_t blocks = ((s.T + C::BM - 1) / C::BM) * s.bh();
    if (!grid_fits(blocks, C::NW * kWave) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const float qscale = kLog2e / sqrtf(float(s.scale_dim()));
    const float inv_sqrt_d = 1.f / sqrtf(float(s.scale_dim()));
    hipLaunchKernelGGL((bwd_dq_f32_kernel<D>), dim3(unsigned(blocks)), dim3(C::NW * kWave), 0, stream, q, k, v, dout,
                       lse, delta, dq, int(s.T), int(s.bh()), int(s.causal), qscale, inv_sqrt_d);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bwd_dq_f32(const float *q, const float *k, const float *v, const float *dout, const float *lse,
                             const float *delta, float *dq, const AttnShape &s, hipStream_t stream) {
    switch (s.d) {
        case 32: return launch_dq<32>(q, k, v, dout, lse, delta, dq, s, stream);
        case 64: return launch_dq<64>(q, k, v, dout, lse, delta, dq, s, stream);
        case 128: return launch_dq<128>(q, k, v, dout, lse, delta, dq, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
