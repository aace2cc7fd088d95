// bf16 flash-attention backward on bf16 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulate.
//
// Same math as the fp32 backward (attn_bwd_mfma.hip) and the reference's
// flashAttentionBackward (flash_attention.cu:226-326, with correct dK / dV): P and dS are
// computed in fp32 and rounded to bf16 only as MFMA operands; dK, dV, dQ accumulate in fp32
// and are rounded to bf16 once.
//
// Decomposition: a workgroup of 4 waves owns 128 keys (wave w: 32 keys) and keeps dK^T,
// dV^T in registers; it walks 32-row query blocks from the LAST block down to its diagonal,
// so the key-block workgroups of one (batch, head) add into the same dQ rows at the same
// time (those lines stay in L2).  Per wave and query block (lane l: col = l & 31, half =
// l >> 5; 32x32x16 bf16 operands take 8 consecutive k from lane (i, k/8)):
//   S = Q K^T, dP = dO V^T   A = Q / dO rows from LDS, B = K / V rows in registers
//   P = exp2(S c - LSE log2 e), dS = P (dP - delta)        (lane = one key, 16 rows)
//   dV^T += dO^T P, dK^T += Q^T dS   B = P / dS straight from the accumulator (registers
//                                    8s..8s+7 = rows 16s + 8(e/4) + 4 half + e%4), A = dO^T /
//                                    Q^T rows, staged TRANSPOSED in LDS next to Q / dO
//   dQ = dS K                        dS -> LDS ([row][key]); A = dS rows, B = K^T rows
//                                    (staged once); fp32 atomics into the dq accumulator or a
//                                    per-key-block partial buffer (deterministic policy).
#include "attn_launch.h"
#include "attn_mfma_common.h"

#include <math.h>

namespace ctattn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx16 mfma_bf16(bf16x8 a, bf16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <int D>
struct BwdBf16Cfg {
    static constexpr int NW = 4;
    static constexpr int BN = 32 * NW;  // keys per workgroup
    static constexpr int BM = 32;       // query rows per iteration
    static constexpr int QS = D + 8;    // row stride (bf16) of Q / dO in LDS
    static constexpr int TS = BM + 4;   // row stride of Q^T / dO^T (conflict-free 8-byte reads)
    static constexpr int KS = BN + 8;   // row stride of K^T and of dS
    static constexpr int DT = D / 32;
    static constexpr int PATCHES = (BM / 4) * (D / 8);  // 4-row x 8-d patches per block (per tensor)
    static_assert(D % 32 == 0 && 2 * PATCHES <= NW * kWave, "tile shape");
};

// Gathers A-operand element e of a transposed row: rows r0..r0+3 and r0+8..r0+11.
__device__ __forceinline__ bf16x8 load_split8(const __bf16 *p) {
    const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(p);
    const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(p + 8);
    bf16x8 a;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        a[e] = lo[e];
        a[4 + e] = hi[e];
    }
    return a;
}

template <int D, bool MASK>
__device__ __forceinline__ void bwd_bf16_wave_block(
    floatx16 (&dk_acc)[D / 32], floatx16 (&dv_acc)[D / 32], const bf16x8 (&kB)[D / 16],
    const bf16x8 (&vB)[D / 16], const __bf16 *q_lds, const __bf16 *do_lds, const __bf16 *qt_lds,
    const __bf16 *dot_lds, const float *lse_lds, const float *dl_lds, __bf16 *ds_lds, int r0, int key,
    int T, int causal, float c, int wave, int col, int half) {
    using C = BwdBf16Cfg<D>;
    floatx16 s = zero16(), dp = zero16();
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        const bf16x8 qa = *reinterpret_cast<const bf16x8 *>(q_lds + col * C::QS + 16 * st + 8 * half);
        const bf16x8 da = *reinterpret_cast<const bf16x8 *>(do_lds + col * C::QS + 16 * st + 8 * half);
        s = mfma_bf16(qa, kB[st], s);
        dp = mfma_bf16(da, vB[st], dp);
    }
    bf16x8 pb[2], dsb[2];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const floatx4 l4 = *reinterpret_cast<const floatx4 *>(&lse_lds[8 * g + 4 * half]);
        const floatx4 d4 = *reinterpret_cast<const floatx4 *>(&dl_lds[8 * g + 4 * half]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int r = 4 * g + t;
            float p = fast_exp2(fmaf(s[r], c, -l4[t]));
            if (MASK) {
                const int row = r0 + acc_row(r, half);
                p = (row >= T || key >= T || (causal && key > row)) ? 0.f : p;
            }
            const float ds = p * (dp[r] - d4[t]);
            pb[r / 8][r % 8] = (__bf16)p;
            dsb[r / 8][r % 8] = (__bf16)ds;
            ds_lds[acc_row(r, half) * C::KS + 32 * wave + col] = (__bf16)ds;
        }
    }
    // dV^T += dO^T P, dK^T += Q^T dS over this block's 32 rows (2 k-steps of 16 rows).
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int rr = 16 * ks + 4 * half;  // rows rr..rr+3 and rr+8..rr+11
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
            const bf16x8 a_do = load_split8(dot_lds + (dt * 32 + col) * C::TS + rr);
            const bf16x8 a_q = load_split8(qt_lds + (dt * 32 + col) * C::TS + rr);
            dv_acc[dt] = mfma_bf16(a_do, pb[ks], dv_acc[dt]);
            dk_acc[dt] = mfma_bf16(a_q, dsb[ks], dk_acc[dt]);
        }
    }
}

// d = 64 fits 256 registers (2 waves per SIMD); d = 128 needs more than 256 and runs one
// wave per SIMD with up to 512.
template <int D> struct BwdBf16Occupancy { static constexpr int waves = D <= 64 ? 2 : 1; };

template <int D, bool PARTIAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BwdBf16Occupancy<D>::waves,
                                                                      BwdBf16Occupancy<D>::waves))) void bwd_bf16_mfma_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const uint16_t *__restrict__ dout, const float *__restrict__ lse, const float *__restrict__ delta,
    float *__restrict__ dq_acc, uint16_t *__restrict__ dk, uint16_t *__restrict__ dv, int T, int BH,
    int causal, float c, float inv_sqrt_d) {
    using C = BwdBf16Cfg<D>;
    __shared__ __attribute__((aligned(16))) __bf16 q_lds[C::BM * C::QS];
    __shared__ __attribute__((aligned(16))) __bf16 do_lds[C::BM * C::QS];
    __shared__ __attribute__((aligned(16))) __bf16 qt_lds[D * C::TS];
    __shared__ __attribute__((aligned(16))) __bf16 dot_lds[D * C::TS];
    __shared__ __attribute__((aligned(16))) __bf16 kt_lds[D * C::KS];
    __shared__ __attribute__((aligned(16))) __bf16 ds_lds[C::BM * C::KS];
    __shared__ __attribute__((aligned(16))) float lse_lds[C::BM];
    __shared__ __attribute__((aligned(16))) float dl_lds[C::BM];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int id = blockIdx.x;
    const int bh = id % BH;
    const int kb = id / BH;
    const int k0 = kb * C::BN;
    const int64_t base = int64_t(bh) * T * D;
    const int64_t rbase = int64_t(bh) * T;
    const int kw0 = k0 + 32 * wave;
    const int key = kw0 + col;

    // K / V rows of this lane's key as B operands (8 consecutive d per step); K^T -> LDS.
    bf16x8 kB[D / 16], vB[D / 16];
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        u16x8 kx = {0, 0, 0, 0, 0, 0, 0, 0}, vx = {0, 0, 0, 0, 0, 0, 0, 0};
        if (key < T) {
            kx = *reinterpret_cast<const u16x8 *>(k + base + int64_t(key) * D + 16 * st + 8 * half);
            vx = *reinterpret_cast<const u16x8 *>(v + base + int64_t(key) * D + 16 * st + 8 * half);
        }
        kB[st] = __builtin_bit_cast(bf16x8, kx);
        vB[st] = __builtin_bit_cast(bf16x8, vx);
#pragma unroll
        for (int e = 0; e < 8; ++e) kt_lds[(16 * st + 8 * half + e) * C::KS + 32 * wave + col] = kB[st][e];
    }

    floatx16 dk_acc[C::DT], dv_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
        dk_acc[dt] = zero16();
        dv_acc[dt] = zero16();
    }

    const int nqb = (T + C::BM - 1) / C::BM;
    const int qb_first = causal ? k0 / C::BM : 0;

    // Staging: threads [0, PATCHES) take Q, [PATCHES, 2*PATCHES) take dO; each holds a
    // 4-row x 8-d patch and writes it row-major (4 x 16 B) and transposed (8 x 8 B).
    const bool stager = tid < 2 * C::PATCHES;
    const bool is_do = tid >= C::PATCHES;
    const int pt = is_do ? tid - C::PATCHES : tid;
    const int prg = pt % (C::BM / 4);  // rows 4*prg .. 4*prg+3
    const int pdg = pt / (C::BM / 4);  // d 8*pdg .. 8*pdg+7
    const uint16_t *src = is_do ? dout : q;
    __bf16 *dst = is_do ? do_lds : q_lds;
    __bf16 *dstT = is_do ? dot_lds : qt_lds;
    u16x8 pre[4];
    float lpre = 0.f, dpre = 0.f;
    auto load_qblock = [&](int r0) {
        if (stager) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = r0 + 4 * prg + i;
                u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
                if (row < T) x = *reinterpret_cast<const u16x8 *>(src + base + int64_t(row) * D + 8 * pdg);
                pre[i] = x;
            }
        }
        if (tid < C::BM) {
            const int row = r0 + tid;
            lpre = row < T ? lse[rbase + row] * kLog2e : 0.f;
            dpre = row < T ? delta[rbase + row] : 0.f;
        }
    };
    auto store_qblock = [&]() {
        if (stager) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<u16x8 *>(dst + (4 * prg + i) * C::QS + 8 * pdg) = pre[i];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const u16x4 t = {pre[0][e], pre[1][e], pre[2][e], pre[3][e]};
                *reinterpret_cast<u16x4 *>(dstT + (8 * pdg + e) * C::TS + 4 * prg) = t;
            }
        }
        if (tid < C::BM) {
            lse_lds[tid] = lpre;
            dl_lds[tid] = dpre;
        }
    };

    if (qb_first < nqb) load_qblock((nqb - 1) * C::BM);
    for (int qb = nqb - 1; qb >= qb_first; --qb) {
        const int r0 = qb * C::BM;
        // Q / dO / LSE / delta of the previous block were last read before the previous
        // dQ-phase barrier; ds_lds is rewritten only after the barrier below.
        store_qblock();
        __syncthreads();
        if (qb - 1 >= qb_first) load_qblock(r0 - C::BM);

        const bool wave_active = kw0 < T && (!causal || kw0 <= r0 + C::BM - 1);
        if (wave_active) {
            const bool masked = (r0 + C::BM > T) || (kw0 + 32 > T) || (causal && kw0 + 31 > r0);
            if (masked)
                bwd_bf16_wave_block<D, true>(dk_acc, dv_acc, kB, vB, q_lds, do_lds, qt_lds, dot_lds, lse_lds,
                                             dl_lds, ds_lds, r0, key, T, causal, c, wave, col, half);
            else
                bwd_bf16_wave_block<D, false>(dk_acc, dv_acc, kB, vB, q_lds, do_lds, qt_lds, dot_lds, lse_lds,
                                              dl_lds, ds_lds, r0, key, T, causal, c, wave, col, half);
        }
        __syncthreads();  // dS of every wave visible

        // dQ[r0..r0+31][32*wave .. 32*wave+31] over the workgroup's active keys; waves past
        // d / 32 have no columns (d = 64: waves 2, 3 skip this phase; d = 32: waves 1-3).
        if (wave >= C::DT) continue;
        floatx16 dq = zero16();
#pragma unroll
        for (int w2 = 0; w2 < C::NW; ++w2) {
            const int kw2 = k0 + 32 * w2;
            if (!(kw2 < T && (!causal || kw2 <= r0 + C::BM - 1))) continue;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int kl = 32 * w2 + 16 * ks + 8 * half;
                const bf16x8 a = *reinterpret_cast<const bf16x8 *>(ds_lds + col * C::KS + kl);
                const bf16x8 b = *reinterpret_cast<const bf16x8 *>(kt_lds + (32 * wave + col) * C::KS + kl);
                dq = mfma_bf16(a, b, dq);
            }
        }
        // dq tile: lane (col = d - 32*wave, half), register r -> row acc_row(r, half) =
        // row0 + acc_row(r, 0), with the offset acc_row(r, 0) * D a compile-time constant.
        const int row0 = r0 + 4 * half;
        float *p0 = dq_acc + (PARTIAL ? int64_t(kb) * BH * T * D : 0) + (rbase + row0) * D + 32 * wave + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int dr = acc_row(r, 0);
            if (row0 + dr >= T) continue;
            const float val = dq[r] * inv_sqrt_d;
            if constexpr (PARTIAL) {
                p0[dr * D] = val;
            } else {
                unsafeAtomicAdd(p0 + dr * D, val);
            }
        }
    }

    if (key < T) {
        uint16_t *dkr = dk + base + int64_t(key) * D;
        uint16_t *dvr = dv + base + int64_t(key) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                u16x4 xk, xv;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    xk[t] = f32_to_bf16(dk_acc[dt][4 * g + t] * inv_sqrt_d).bits;
                    xv[t] = f32_to_bf16(dv_acc[dt][4 * g + t]).bits;
                }
                *reinterpret_cast<u16x4 *>(dkr + dt * 32 + 8 * g + 4 * half) = xk;
                *reinterpret_cast<u16x4 *>(dvr + dt * 32 + 8 * g + 4 * half) = xv;
            }
        }
    }
}

// delta[row] = sum_c dO[row][c] O[row][c] from bf16 (flash_attention.cu:269-273); zeroes the
// fp32 dq accumulator row when ZERO.  One wave per row.
template <bool ZERO>
__global__ __launch_bounds__(256) void bwd_preprocess_bf16_kernel(const uint16_t *__restrict__ o,
                                                                 const uint16_t *__restrict__ dout,
                                                                 float *__restrict__ delta,
                                                                 float *__restrict__ dq_acc, int64_t rows,
                                                                 int d) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    float s = 0.f;
    for (int cc = lane; cc < d; cc += kWave) {
        s += to_f32(bf16_t{o[row * d + cc]}) * to_f32(bf16_t{dout[row * d + cc]});
        if (ZERO) dq_acc[row * d + cc] = 0.f;
    }
    s = wave_sum(s);
    if (lane == 0) delta[row] = s;
}

// dq (bf16) = fp32 accumulator, rounded to nearest even.  4 elements per thread.
__global__ __launch_bounds__(256) void dq_to_bf16_kernel(const float *__restrict__ acc,
                                                        uint16_t *__restrict__ dq, int64_t n4) {
    const int64_t f = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (f >= n4) return;
    const floatx4 x = *reinterpret_cast<const floatx4 *>(acc + 4 * f);
    u16x4 y;
#pragma unroll
    for (int t = 0; t < 4; ++t) y[t] = f32_to_bf16(x[t]).bits;
    *reinterpret_cast<u16x4 *>(dq + 4 * f) = y;
}

// dq (bf16) = sum over key blocks kb <= last(row) of the partials, in increasing kb order.
template <int D>
__global__ __launch_bounds__(256) void dq_reduce_bf16_kernel(const float *__restrict__ part,
                                                            uint16_t *__restrict__ dq, int T, int BH,
                                                            int causal, int nkb, int bn) {
    const int64_t f = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t total = int64_t(BH) * T * (D / 4);
    if (f >= total) return;
    const int64_t row_g = f / (D / 4);
    const int row = int(row_g % T);
    const int last = causal ? row / bn : nkb - 1;
    const int64_t plane = int64_t(BH) * T * D;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb <= last; ++kb) acc += *reinterpret_cast<const floatx4 *>(part + kb * plane + 4 * f);
    u16x4 y;
#pragma unroll
    for (int t = 0; t < 4; ++t) y[t] = f32_to_bf16(acc[t]).bits;
    *reinterpret_cast<u16x4 *>(dq + 4 * f) = y;
}

template <int D>
hipError_t bwd_bf16(const void *q, const void *k, const void *v, const void *o, const void *dout,
                    const float *lse, float *delta, void *dq, void *dk, void *dv, float *acc,
                    bool deterministic, const AttnShape &s, hipStream_t stream) {
    using C = BwdBf16Cfg<D>;
    const int64_t nkb = (s.T + C::BN - 1) / C::BN;
    const int64_t blocks = nkb * s.bh();
    if (blocks > 2147483647 || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const int64_t rows = s.rows();
    auto u16 = [](const void *p) { return static_cast<const uint16_t *>(p); };
    if (deterministic)
        hipLaunchKernelGGL(bwd_preprocess_bf16_kernel<false>, dim3(unsigned((rows + 3) / 4)), dim3(256), 0,
                           stream, u16(o), u16(dout), delta, acc, rows, D);
    else
        hipLaunchKernelGGL(bwd_preprocess_bf16_kernel<true>, dim3(unsigned((rows + 3) / 4)), dim3(256), 0,
                           stream, u16(o), u16(dout), delta, acc, rows, D);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const float c = kLog2e / sqrtf(float(D));
    const float inv_sqrt_d = 1.f / sqrtf(float(D));
    if (deterministic)
        hipLaunchKernelGGL((bwd_bf16_mfma_kernel<D, true>), dim3(unsigned(blocks)), dim3(C::NW * kWave), 0,
                           stream, u16(q), u16(k), u16(v), u16(dout), lse, delta, acc,
                           static_cast<uint16_t *>(dk), static_cast<uint16_t *>(dv), int(s.T), int(s.bh()),
                           int(s.causal), c, inv_sqrt_d);
    else
        hipLaunchKernelGGL((bwd_bf16_mfma_kernel<D, false>), dim3(unsigned(blocks)), dim3(C::NW * kWave), 0,
                           stream, u16(q), u16(k), u16(v), u16(dout), lse, delta, acc,
                           static_cast<uint16_t *>(dk), static_cast<uint16_t *>(dv), int(s.T), int(s.bh()),
                           int(s.causal), c, inv_sqrt_d);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t n4 = rows * (D / 4);
    if (deterministic)
        hipLaunchKernelGGL(dq_reduce_bf16_kernel<D>, dim3(unsigned((n4 + 255) / 256)), dim3(256), 0, stream, acc,
                           static_cast<uint16_t *>(dq), int(s.T), int(s.bh()), int(s.causal), int(nkb), C::BN);
    else
        hipLaunchKernelGGL(dq_to_bf16_kernel, dim3(unsigned((n4 + 255) / 256)), dim3(256), 0, stream, acc,
                           static_cast<uint16_t *>(dq), n4);
    return hipGetLastError();
}

}  // namespace

int64_t bf16_bwd_workspace_bytes(const AttnShape &s, bool deterministic) {
    const int64_t plane = s.rows() * s.d * int64_t(sizeof(float));
    const int64_t nkb = (s.T + 127) / 128;
    return deterministic ? nkb * plane : plane;
}

hipError_t launch_bf16_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
                           const float *lse, float *delta, void *dq, void *dk, void *dv, void *extra,
                           bool deterministic, const AttnShape &s, hipStream_t stream) {
    float *acc = static_cast<float *>(extra);
    switch (s.d) {
        case 32: return bwd_bf16<32>(q, k, v, o, dout, lse, delta, dq, dk, dv, acc, deterministic, s, stream);
        case 64: return bwd_bf16<64>(q, k, v, o, dout, lse, delta, dq, dk, dv, acc, deterministic, s, stream);
        case 128: return bwd_bf16<128>(q, k, v, o, dout, lse, delta, dq, dk, dv, acc, deterministic, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
