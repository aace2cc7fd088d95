// fp32 flash-attention backward on fp32 MFMA, 128-key workgroups (gfx950).
//
// The 128-key variant of the backward main kernel (attn_bwd_mfma.hip holds the 64-key one,
// the preprocess / reduction kernels and the choice between the two).  Same math and
// reference mapping: P = exp(S - LSE) (flash_attention.cu:297-298), dS = P (dP - delta)
// (:299), dQ = dS K / sqrt(d) (:311), dK = dS^T Q / sqrt(d), dV = P^T dO.
//
// Work decomposition
//   * one workgroup = 4 waves owns BN = 128 keys of one (batch, head); wave w owns keys
//     32w .. 32w+31 and accumulates dK^T and dV^T for them in registers for the whole
//     kernel -- dK / dV are written exactly once, no atomics.
//   * the workgroup walks query blocks of BM = 32 rows (causal: only rows >= its first
//     key).  Q, dO, LSE and delta of the block are staged global -> registers -> LDS; the
//     next block's loads are issued before this block's MFMAs.
//   * per wave and query block, with v_mfma_f32_32x32x2f32: S = Q K^T, dP = dO V^T (each
//     lane holds one key and 16 rows), P and dS elementwise, then dV^T += dO^T P and
//     dK^T += Q^T dS with P / dS as the B operands.
//   * dQ: each wave writes its dS tile to LDS, then every wave computes a quarter of the
//     32 x d block of dQ = dS K over the workgroup's 128 keys with v_mfma_f32_16x16x4f32,
//     added with fp32 atomics (Atomic) or stored as a per-128-key-block partial (Partial).
//     Without dQ (None) the kernel produces dK and dV only, for the deterministic backward
//     whose dQ comes from the query-major kernel of attn_bwd_dq_f32.hip.
//   Against the 64-key kernel it issues half the dQ atomics (one set per 128 keys) but
//   leaves more waves idle on the causal diagonal; it is the faster one without a mask and
//   at d = 32.
#include "attn_launch.h"
#include "attn_mfma_common.h"

#include <math.h>

namespace ctattn {
namespace {



__device__ __forceinline__ floatx4 mfma16x16x4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int D>
struct BwdK128Cfg {
    static constexpr int NW = 4;              // waves per workgroup
    static constexpr int BN = 32 * NW;        // keys per workgroup
    static constexpr int BM = 32;             // query rows per iteration
    static constexpr int KS = D + 4;          // LDS row stride (floats) for K, Q, dO
    static constexpr int SS = BN + 4;         // LDS row stride for dS
    static constexpr int DT = D / 32;         // 32-wide d tiles of dK^T / dV^T
    static constexpr int F4_ROW = D / 4;
    static constexpr int QF4 = BM * F4_ROW / (NW * kWave);  // float4 per thread per Q block
    static constexpr int KF4 = BN * F4_ROW / (NW * kWave);  // float4 per thread for the K block
    // dQ of one 32-row block is (2 x D/16) 16x16 tiles; each wave takes a quarter: for
    // d >= 64 both row tiles of a D/4-column slice, for d = 32 one tile
    // (row tile wave >> 1, column tile wave & 1).
    static constexpr int DQ_RT = D >= 64 ? 2 : 1;   // 16-row tiles per wave
    static constexpr int DQ_COLS = D >= 64 ? D / NW : 16;  // dQ columns per wave
    static constexpr int DQ_CT = DQ_COLS / 16;      // 16-wide column tiles per wave
    static_assert(D == 32 || D == 64 || D == 128, "MFMA backward supports d in {32, 64, 128}");
    static_assert(DQ_RT * DQ_CT * NW == 2 * (D / 16), "dQ tiles split over the waves");
    static_assert(QF4 >= 1 && KF4 >= 1, "block load split");
};

// S, dP, P, dS and the dV^T / dK^T updates of one wave for one query block, then (WRITE_DS)
// dS -> LDS.  MASK selects the diagonal / sequence-end variant (per-element causal and bounds
// checks); the unmasked variant carries none.
template <int D, bool MASK, bool WRITE_DS>
__device__ __forceinline__ void bwd_k128_wave_block(floatx16 (&dk_acc)[D / 32], floatx16 (&dv_acc)[D / 32],
                                               const float (&vT)[D / 2], const float *q_lds,
                                               const float *do_lds, const float *k_lds,
                                               const float *lse_lds, const float *dl_lds,
                                               float *ds_lds, int r0, int key, int T, int causal,
                                               float kscale, int wave, int col, int half) {
    using C = BwdK128Cfg<D>;
    floatx16 s = zero16(), dp = zero16();
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
        const floatx4 qa = *reinterpret_cast<const floatx4 *>(&q_lds[col * C::KS + 8 * m + 4 * half]);
        const floatx4 da = *reinterpret_cast<const floatx4 *>(&do_lds[col * C::KS + 8 * m + 4 * half]);
        const floatx4 kb4 = *reinterpret_cast<const floatx4 *>(&k_lds[(32 * wave + col) * C::KS + 8 * m + 4 * half]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            s = mfma32x32x2(qa[t], kb4[t], s);
            dp = mfma32x32x2(da[t], vT[4 * m + t], dp);
        }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const floatx4 l4 = *reinterpret_cast<const floatx4 *>(&lse_lds[8 * g + 4 * half]);
        const floatx4 d4 = *reinterpret_cast<const floatx4 *>(&dl_lds[8 * g + 4 * half]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int r = 4 * g + t;
            float p = fast_exp2(fmaf(s[r], kscale, -l4[t]));
            if (MASK) {
                const int row = r0 + acc_row(r, half);
                p = (row >= T || key >= T || (causal && key > row)) ? 0.f : p;
            }
            s[r] = p;
            dp[r] = p * (dp[r] - d4[t]);
        }
    }
    // dV^T += dO^T P,  dK^T += Q^T dS   (contraction over this block's 32 rows)
#pragma unroll
    for (int st = 0; st < 16; ++st) {
        const int rl = kstep_index(st, half);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
            const float a_do = do_lds[rl * C::KS + dt * 32 + col];
            const float a_q = q_lds[rl * C::KS + dt * 32 + col];
            dv_acc[dt] = mfma32x32x2(a_do, s[st], dv_acc[dt]);
            dk_acc[dt] = mfma32x32x2(a_q, dp[st], dk_acc[dt]);
        }
    }
    if constexpr (WRITE_DS) {
#pragma unroll
        for (int r = 0; r < 16; ++r) ds_lds[acc_row(r, half) * C::SS + 32 * wave + col] = dp[r];
    }
}

// Waves per SIMD the kernel is compiled for: two for d <= 64 (<= 256 VGPRs); d = 128 needs
// more registers than that and runs one wave per SIMD.
template <int D> struct BwdK128Occupancy { static constexpr int waves = D <= 64 ? 2 : 1; };

template <int D, K128Dq MODE, bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BwdK128Occupancy<D>::waves,
                                                                     BwdK128Occupancy<D>::waves))) void bwd_f32_k128_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, float *__restrict__ dq, float *__restrict__ dq_part,
    float *__restrict__ dk, float *__restrict__ dv, int T, int BH, int causal, float kscale, float inv_sqrt_d) {
    using C = BwdK128Cfg<D>;
    constexpr int split = SPLIT ? 1 : 0;
    __shared__ __attribute__((aligned(16))) float k_lds[C::BN * C::KS];
    __shared__ __attribute__((aligned(16))) float q_lds[C::BM * C::KS];
    __shared__ __attribute__((aligned(16))) float do_lds[C::BM * C::KS];
    __shared__ __attribute__((aligned(16))) float ds_lds[C::BM * C::SS];
    __shared__ __attribute__((aligned(16))) float lse_lds[C::BM];  // log2 units
    __shared__ __attribute__((aligned(16))) float dl_lds[C::BM];   // delta

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int c16 = lane & 15;
    const int quad = lane >> 4;

    // split: key block kb's query blocks are shared by workgroups (kb, part 0) and (kb, part 1).
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int kb = (id / BH) >> split;  // causal: key block 0 has the most query blocks -> launched first
    const int part = (id / BH) & split;
    const int k0 = kb * C::BN;
    const int64_t base = int64_t(bh) * T * D;
    const int64_t rbase = int64_t(bh) * T;
    const int kw0 = k0 + 32 * wave;
    const int key = kw0 + col;  // key owned by this lane in S / dP / dK^T / dV^T

    // K block -> LDS (B operand of dQ = dS K).
#pragma unroll
    for (int i = 0; i < C::KF4; ++i) {
        const int f = tid + i * C::NW * kWave;
        const int r = f / C::F4_ROW;
        const int c4 = f - r * C::F4_ROW;
        floatx4 x = {0.f, 0.f, 0.f, 0.f};
        if (k0 + r < T) x = *reinterpret_cast<const floatx4 *>(k + base + int64_t(k0 + r) * D + 4 * c4);
        *reinterpret_cast<floatx4 *>(&k_lds[r * C::KS + 4 * c4]) = x;
    }
    // V^T as the B operand of dP = dO V^T, held in registers for the whole kernel:
    // lane (col = key, half) holds V[key][kstep_index(s, half)].  K^T, the B operand of
    // S = Q K^T, is read from the K block in LDS with the same mapping.
    float vT[D / 2];
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
        floatx4 vx = {0.f, 0.f, 0.f, 0.f};
        if (key < T) vx = *reinterpret_cast<const floatx4 *>(v + base + int64_t(key) * D + 8 * m + 4 * half);
#pragma unroll
        for (int t = 0; t < 4; ++t) vT[4 * m + t] = vx[t];
    }

    floatx16 dk_acc[C::DT], dv_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
        dk_acc[dt] = zero16();
        dv_acc[dt] = zero16();
    }

    const int nqb_all = (T + C::BM - 1) / C::BM;
    const int qb_first = causal ? k0 / C::BM : 0;
    const int qb_mid = qb_first + (nqb_all - qb_first + 1) / 2;
    const int qb_begin = split && part ? qb_mid : qb_first;
    const int nqb = split && !part ? qb_mid : nqb_all;  // end of this workgroup's query blocks

    floatx4 qpre[C::QF4], dopre[C::QF4];
    float lpre = 0.f, dpre = 0.f;
    auto load_qblock = [&](int r0) {
#pragma unroll
        for (int i = 0; i < C::QF4; ++i) {
            const int f = tid + i * C::NW * kWave;
            const int r = f / C::F4_ROW;
            const int c4 = f - r * C::F4_ROW;
            const int row = r0 + r;
            floatx4 qx = {0.f, 0.f, 0.f, 0.f}, dx = {0.f, 0.f, 0.f, 0.f};
            if (row < T) {
                qx = *reinterpret_cast<const floatx4 *>(q + base + int64_t(row) * D + 4 * c4);
                dx = *reinterpret_cast<const floatx4 *>(dout + base + int64_t(row) * D + 4 * c4);
            }
            qpre[i] = qx;
            dopre[i] = dx;
        }
        if (tid < C::BM) {
            const int row = r0 + tid;
            lpre = row < T ? lse[rbase + row] * kLog2e : 0.f;
            dpre = row < T ? delta[rbase + row] : 0.f;
        }
    };
    auto store_qblock = [&]() {
#pragma unroll
        for (int i = 0; i < C::QF4; ++i) {
            const int f = tid + i * C::NW * kWave;
            const int r = f / C::F4_ROW;
            const int c4 = f - r * C::F4_ROW;
            *reinterpret_cast<floatx4 *>(&q_lds[r * C::KS + 4 * c4]) = qpre[i];
            *reinterpret_cast<floatx4 *>(&do_lds[r * C::KS + 4 * c4]) = dopre[i];
        }
        if (tid < C::BM) {
            lse_lds[tid] = lpre;
            dl_lds[tid] = dpre;
        }
    };

    if (qb_begin < nqb) load_qblock(qb_begin * C::BM);
    for (int qb = qb_begin; qb < nqb; ++qb) {
        const int r0 = qb * C::BM;
        // q/do/lse/delta of the previous block were last read before the previous dQ-phase
        // barrier, so they can be overwritten without another barrier; ds_lds is only
        // rewritten after the barrier below, which every wave reaches after its dQ phase.
        store_qblock();
        __syncthreads();
        if (qb + 1 < nqb) load_qblock(r0 + C::BM);

        const bool wave_active = kw0 < T && (!causal || kw0 <= r0 + C::BM - 1);
        if (wave_active) {
            const bool masked = (r0 + C::BM > T) || (kw0 + 32 > T) || (causal && kw0 + 31 > r0);
            constexpr bool WDS = MODE != K128Dq::None;
            if (masked)
                bwd_k128_wave_block<D, true, WDS>(dk_acc, dv_acc, vT, q_lds, do_lds, k_lds, lse_lds, dl_lds,
                                                  ds_lds, r0, key, T, causal, kscale, wave, col, half);
            else
                bwd_k128_wave_block<D, false, WDS>(dk_acc, dv_acc, vT, q_lds, do_lds, k_lds, lse_lds, dl_lds,
                                                   ds_lds, r0, key, T, causal, kscale, wave, col, half);
        }
        // dS of every wave visible; every wave is done reading this block's Q / dO / LSE /
        // delta before the next iteration overwrites them.
        __syncthreads();
        if constexpr (MODE == K128Dq::None) continue;

        // dQ[r0 .. r0+31][wave * DQ_COLS ..] = sum over the workgroup's active keys of dS K.
        const int rt0 = D >= 64 ? 0 : (wave >> 1);                 // first 16-row tile
        const int dq_col0 = D >= 64 ? wave * C::DQ_COLS : (wave & 1) * 16;  // first column
        floatx4 dq_acc[C::DQ_RT][C::DQ_CT];
#pragma unroll
        for (int rt = 0; rt < C::DQ_RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < C::DQ_CT; ++ct) dq_acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w2 = 0; w2 < C::NW; ++w2) {
            const int kw2 = k0 + 32 * w2;
            if (!(kw2 < T && (!causal || kw2 <= r0 + C::BM - 1))) continue;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                const int kl = 32 * w2 + 16 * sb + 4 * quad;  // local key of step t: kl + t
                floatx4 a[C::DQ_RT];
#pragma unroll
                for (int rt = 0; rt < C::DQ_RT; ++rt)
                    a[rt] = *reinterpret_cast<const floatx4 *>(&ds_lds[((rt0 + rt) * 16 + c16) * C::SS + kl]);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
#pragma unroll
                    for (int ct = 0; ct < C::DQ_CT; ++ct) {
                        const float b = k_lds[(kl + t) * C::KS + dq_col0 + ct * 16 + c16];
#pragma unroll
                        for (int rt = 0; rt < C::DQ_RT; ++rt) dq_acc[rt][ct] = mfma16x16x4(a[rt][t], b, dq_acc[rt][ct]);
                    }
                }
            }
        }
#pragma unroll
        for (int rt = 0; rt < C::DQ_RT; ++rt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = r0 + (rt0 + rt) * 16 + 4 * quad + r;
                if (row >= T) continue;
#pragma unroll
                for (int ct = 0; ct < C::DQ_CT; ++ct) {
                    const int c = dq_col0 + ct * 16 + c16;
                    const float val = dq_acc[rt][ct][r] * inv_sqrt_d;
                    if constexpr (MODE == K128Dq::Atomic) {
                        unsafeAtomicAdd(dq + base + int64_t(row) * D + c, val);
                    } else {
                        dq_part[(int64_t(kb) * BH * T + rbase + row) * D + c] = val;
                    }
                }
            }
        }
    }

    // dK = (Q^T dS)^T / sqrt(d), dV = (dO^T P)^T; lane (key, half) holds d = dt*32 + acc_row(r, half).
    if constexpr (SPLIT) {
        // Two workgroups add to each element (two addends: the same sum in either order).  The
        // lane-per-key layout would scatter every atomic instruction over 64 rows, so each
        // tensor goes through LDS (k_lds, [key][KS], free after the loop) and is added with
        // lanes along d.
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            __syncthreads();  // every wave is done with k_lds (the loop, or the previous tensor)
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    floatx4 x;
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        x[t] = which == 0 ? dk_acc[dt][4 * g + t] * inv_sqrt_d : dv_acc[dt][4 * g + t];
                    *reinterpret_cast<floatx4 *>(&k_lds[(32 * wave + col) * C::KS + dt * 32 + 8 * g + 4 * half]) = x;
                }
            __syncthreads();
            float *dst = (which == 0 ? dk : dv) + base + int64_t(k0) * D;
            for (int e = tid; e < C::BN * D; e += C::NW * kWave) {
                const int kr = e / D, c = e - (e / D) * D;
                if (k0 + kr < T) unsafeAtomicAdd(dst + int64_t(kr) * D + c, k_lds[kr * C::KS + c]);
            }
        }
        return;
    }
    if (key < T) {
        float *dkr = dk + base + int64_t(key) * D;
        float *dvr = dv + base + int64_t(key) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                floatx4 xk, xv;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    xk[t] = dk_acc[dt][4 * g + t] * inv_sqrt_d;
                    xv[t] = dv_acc[dt][4 * g + t];
                }
                *reinterpret_cast<floatx4 *>(dkr + dt * 32 + 8 * g + 4 * half) = xk;
                *reinterpret_cast<floatx4 *>(dvr + dt * 32 + 8 * g + 4 * half) = xv;
            }
        }
    }
}

template <int D, K128Dq MODE>
void launch_k128_mode(dim3 grid, const float *q, const float *k, const float *v, const float *dout, const float *lse,
                      const float *delta, float *dq, float *dq_part, float *dk, float *dv, const AttnShape &s,
                      float kscale, float inv_sqrt_d, int split, hipStream_t stream) {
    if (split)
        hipLaunchKernelGGL((bwd_f32_k128_kernel<D, MODE, true>), grid, dim3(BwdK128Cfg<D>::NW * kWave), 0, stream, q,
                           k, v, dout, lse, delta, dq, dq_part, dk, dv, int(s.T), int(s.bh()), int(s.causal), kscale,
                           inv_sqrt_d);
    else
        hipLaunchKernelGGL((bwd_f32_k128_kernel<D, MODE, false>), grid, dim3(BwdK128Cfg<D>::NW * kWave), 0, stream, q,
                           k, v, dout, lse, delta, dq, dq_part, dk, dv, int(s.T), int(s.bh()), int(s.causal), kscale,
                           inv_sqrt_d);
}

template <int D>
hipError_t launch_k128(const float *q, const float *k, const float *v, const float *dout, const float *lse,
                       const float *delta, float *dq, float *dq_part, float *dk, float *dv, K128Dq mode,
                       bool split, const AttnShape &s, hipStream_t stream) {
    using C = BwdK128Cfg<D>;
    const int64_t blocks = ((s.T + C::BN - 1) / C::BN) * s.bh() * (split ? 2 : 1);
    if (!grid_fits(blocks, C::NW * kWave) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const float kscale = kLog2e / sqrtf(float(s.scale_dim()));
    const float inv_sqrt_d = 1.f / sqrtf(float(s.scale_dim()));
    const dim3 grid{unsigned(blocks)};
    switch (mode) {
        case K128Dq::Atomic:
            launch_k128_mode<D, K128Dq::Atomic>(grid, q, k, v, dout, lse, delta, dq, dq_part, dk, dv, s, kscale,
                                                inv_sqrt_d, int(split), stream);
            break;
        case K128Dq::Partial:
            launch_k128_mode<D, K128Dq::Partial>(grid, q, k, v, dout, lse, delta, dq, dq_part, dk, dv, s, kscale,
                                                 inv_sqrt_d, int(split), stream);
            break;
        case K128Dq::None:
            launch_k128_mode<D, K128Dq::None>(grid, q, k, v, dout, lse, delta, dq, dq_part, dk, dv, s, kscale,
                                              inv_sqrt_d, int(split), stream);
            break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bwd_f32_k128(const float *q, const float *k, const float *v, const float *dout,
                               const float *lse, const float *delta, float *dq, float *dq_part, float *dk, float *dv,
                               K128Dq mode, bool split, const AttnShape &s, hipStream_t stream) {
    switch (s.d) {
        case 32: return launch_k128<32>(q, k, v, dout, lse, delta, dq, dq_part, dk, dv, mode, split, s, stream);
        case 64: return launch_k128<64>(q, k, v, dout, lse, delta, dq, dq_part, dk, dv, mode, split, s, stream);
        case 128: return launch_k128<128>(q, k, v, dout, lse, delta, dq, dq_part, dk, dv, mode, split, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
