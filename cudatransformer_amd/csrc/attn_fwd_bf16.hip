// bf16 flash-attention forward on bf16 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulate.
//
// Same result as the fp32 forward and as the reference's flashAttention<__nv_bfloat16>
// (flash_attention.cu:57-169) except that scores and sums accumulate in fp32 (the reference
// accumulates the dot products in bf16, flash_attention.cu:112-116).  O is rounded to bf16
// (nearest even) once at the end; LSE is fp32.
//
// Decomposition as in the fp32 kernel (attn_fwd_mfma.hip): a workgroup of 4 waves owns 128
// query rows, a wave 32 rows; keys stream through LDS in 64-key blocks; scores are computed
// transposed, S^T = K Q^T, so each lane holds one query row.  MFMA operand layout of
// 32x32x16 bf16 (lane l, col = l & 31, half = l >> 5): A[i][k] comes from lane
// (i, k / 8) element k % 8, B[k][j] from lane (j, k / 8) element k % 8, D as for 32x32x2.
//   * S^T: A = 8 consecutive d of one key row (one ds_read_b128), B = 8 consecutive d of
//     this lane's query row, in registers for the whole kernel.
//   * O^T += V^T P^T: B = P^T straight from the S^T accumulator -- step s of a 32-key tile
//     takes accumulator registers 8s..8s+7 converted to bf16, i.e. keys
//     16s + 8*(e/4) + 4*half + e%4 -- and A = V^T rows for those keys.  V is therefore
//     staged TRANSPOSED in LDS ([d][key]), so one operand is two 8-byte LDS reads.
//   * the score scale log2(e)/sqrt(d) is applied in fp32 inside exp2's argument (an fma),
//     not folded into bf16 Q.
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
struct FwdBf16Cfg {
    static constexpr int NW = 4;
    static constexpr int BM = 32 * NW;   // query rows per workgroup
    static constexpr int BN = 64;        // keys per block
    static constexpr int KT = BN / 32;   // 32-key tiles per block
    static constexpr int DT = D / 32;    // 32-wide d tiles of O^T
    static constexpr int KS = D + 8;     // K row stride (bf16): 16-byte pad, conflict-free b128 reads
    static constexpr int VS = BN + 4;    // V^T row stride (bf16): 8-byte pad, conflict-free b64 reads
    static constexpr int K_CHUNKS = BN * D / 8 / (NW * kWave);  // 16-byte K chunks per thread
    static constexpr int V_PATCHES = (BN / 4) * (D / 8);        // 4-key x 8-d patches per block
    static_assert(D % 32 == 0 && K_CHUNKS >= 1 && V_PATCHES <= NW * kWave, "tile shape");
};

constexpr float kRescaleThresholdBf16 = 8.0f;

template <int D>
struct FwdBf16State {
    floatx16 oacc[D / 32];
    float m_run;  // running max of S * log2(e)/sqrt(d), identical in both halves
    float l_run;
};

template <int D, bool MASK>
__device__ __forceinline__ void fwd_bf16_block(FwdBf16State<D> &st, const bf16x8 (&qb)[D / 16],
                                               const __bf16 *k_lds, const __bf16 *vt_lds, int j0,
                                               int row, int wave_last_row, int T, int causal,
                                               float c, int col, int half) {
    using C = FwdBf16Cfg<D>;
    bool active[C::KT];
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        const int t0 = j0 + kt * 32;
        active[kt] = !MASK || (t0 < T && (!causal || t0 <= wave_last_row));
    }
    floatx16 sacc[C::KT];
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        sacc[kt] = zero16();
        if (!active[kt]) continue;
        const __bf16 *krow = k_lds + (kt * 32 + col) * C::KS + 8 * half;
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
            const bf16x8 a = *reinterpret_cast<const bf16x8 *>(krow + 16 * s);
            sacc[kt] = mfma_bf16(a, qb[s], sacc[kt]);
        }
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        if (!active[kt]) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float s = sacc[kt][r];
            if (MASK) {
                const int key = j0 + kt * 32 + acc_row(r, half);
                s = (key >= T || (causal && key > row)) ? -INFINITY : s;
                sacc[kt][r] = s;
            }
            mloc = fmaxf(mloc, s);
        }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave)) * c;  // c > 0: max(S) * c = max(S * c)
    if (__any(mloc > st.m_run + kRescaleThresholdBf16)) {
        const float m_new = fmaxf(st.m_run, mloc);
        const float resc = fast_exp2(st.m_run - m_new);
        st.m_run = m_new;
        st.l_run *= resc;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) st.oacc[dt] *= resc;
    }
    // P^T = exp2(S c - m), rounded to bf16 as the B operand; the denominator sums the same
    // fp32 values.
    bf16x8 pb[C::KT][2];
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        if (!active[kt]) continue;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float p = fast_exp2(fmaf(sacc[kt][8 * s + e], c, -st.m_run));
                psum += p;
                pb[kt][s][e] = (__bf16)p;
            }
        }
    }
    st.l_run += psum;
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        if (!active[kt]) continue;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int k0 = kt * 32 + 16 * s + 4 * half;  // keys k0..k0+3 and k0+8..k0+11
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt) {
                const __bf16 *vrow = vt_lds + (dt * 32 + col) * C::VS;
                const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(vrow + k0);
                const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(vrow + k0 + 8);
                bf16x8 a;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[e] = lo[e];
                    a[4 + e] = hi[e];
                }
                st.oacc[dt] = mfma_bf16(a, pb[kt][s], st.oacc[dt]);
            }
        }
    }
}

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_bf16_mfma_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    uint16_t *__restrict__ o, float *__restrict__ lse, int T, int BH, int causal, float c) {
    using C = FwdBf16Cfg<D>;
    __shared__ __attribute__((aligned(16))) __bf16 k_lds[C::BN * C::KS];
    __shared__ __attribute__((aligned(16))) __bf16 vt_lds[D * C::VS];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int nqb = (T + C::BM - 1) / C::BM;
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int qblk = causal ? (nqb - 1 - id / BH) : id / BH;
    const int64_t base = int64_t(bh) * T * D;
    const int q0 = qblk * C::BM;
    const int row = q0 + wave * 32 + col;
    const int wave_first_row = q0 + wave * 32;
    const int wave_last_row = wave_first_row + 31;

    // Q^T as the B operand: lane (row, half) holds Q[row][16s + 8*half .. +7].
    bf16x8 qb[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
        u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
        if (row < T) x = *reinterpret_cast<const u16x8 *>(q + base + int64_t(row) * D + 16 * s + 8 * half);
        qb[s] = __builtin_bit_cast(bf16x8, x);
    }

    FwdBf16State<D> st;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) st.oacc[dt] = zero16();
    st.m_run = -INFINITY;
    st.l_run = 0.f;

    const int kend = causal ? min(T, q0 + C::BM) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;

    // Staging registers: K as 16-byte row chunks; V as a 4-key x 8-d patch per thread.
    u16x8 kpre[C::K_CHUNKS];
    u16x8 vpre[4];
    const bool v_owner = tid < C::V_PATCHES;
    const int vkg = tid % (C::BN / 4);  // keys 4*vkg .. 4*vkg+3
    const int vdg = tid / (C::BN / 4);  // d 8*vdg .. 8*vdg+7
    auto load_block = [&](int j0) {
#pragma unroll
        for (int i = 0; i < C::K_CHUNKS; ++i) {
            const int f = tid + i * C::NW * kWave;
            const int r = f / (D / 8);
            const int c8 = f - r * (D / 8);
            u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
            if (j0 + r < T) x = *reinterpret_cast<const u16x8 *>(k + base + int64_t(j0 + r) * D + 8 * c8);
            kpre[i] = x;
        }
        if (v_owner) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = j0 + 4 * vkg + i;
                u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
                if (key < T) x = *reinterpret_cast<const u16x8 *>(v + base + int64_t(key) * D + 8 * vdg);
                vpre[i] = x;
            }
        }
    };
    auto store_block = [&]() {
#pragma unroll
        for (int i = 0; i < C::K_CHUNKS; ++i) {
            const int f = tid + i * C::NW * kWave;
            const int r = f / (D / 8);
            const int c8 = f - r * (D / 8);
            *reinterpret_cast<u16x8 *>(k_lds + r * C::KS + 8 * c8) = kpre[i];
        }
        if (v_owner) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const u16x4 t = {vpre[0][e], vpre[1][e], vpre[2][e], vpre[3][e]};
                *reinterpret_cast<u16x4 *>(vt_lds + (8 * vdg + e) * C::VS + 4 * vkg) = t;
            }
        }
    };

    load_block(0);
    for (int kb = 0; kb < nkb; ++kb) {
        const int j0 = kb * C::BN;
        __syncthreads();
        store_block();
        __syncthreads();
        if (kb + 1 < nkb) load_block(j0 + C::BN);
        const bool masked = (j0 + C::BN > T) || (causal && j0 + C::BN - 1 > wave_first_row);
        if (masked) {
            if (!causal || j0 <= wave_last_row)
                fwd_bf16_block<D, true>(st, qb, k_lds, vt_lds, j0, row, wave_last_row, T, causal, c, col,
                                        half);
        } else {
            fwd_bf16_block<D, false>(st, qb, k_lds, vt_lds, j0, row, wave_last_row, T, causal, c, col, half);
        }
    }

    const float l_tot = st.l_run + __shfl_xor(st.l_run, 32, kWave);
    const float inv_l = 1.f / l_tot;
    if (row < T) {
        uint16_t *orow = o + base + int64_t(row) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                u16x4 x;
#pragma unroll
                for (int t = 0; t < 4; ++t) x[t] = f32_to_bf16(st.oacc[dt][4 * g + t] * inv_l).bits;
                *reinterpret_cast<u16x4 *>(orow + dt * 32 + 8 * g + 4 * half) = x;
            }
        }
        if (lse != nullptr && half == 0) lse[int64_t(bh) * T + row] = (st.m_run + __log2f(l_tot)) * kLn2;
    }
}

template <int D>
hipError_t fwd_bf16(const void *q, const void *k, const void *v, void *o, float *lse, const AttnShape &s,
                    hipStream_t stream) {
    using C = FwdBf16Cfg<D>;
    const int64_t nqb = (s.T + C::BM - 1) / C::BM;
    const int64_t blocks = nqb * s.bh();
    if (blocks > 2147483647 || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const float c = kLog2e / sqrtf(float(D));
    hipLaunchKernelGGL(fwd_bf16_mfma_kernel<D>, dim3(unsigned(blocks)), dim3(C::NW * kWave), 0, stream,
                       static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                       static_cast<const uint16_t *>(v), static_cast<uint16_t *>(o), lse, int(s.T),
                       int(s.bh()), int(s.causal), c);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bf16_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                           const AttnShape &s, hipStream_t stream) {
    switch (s.d) {
        case 32: return fwd_bf16<32>(q, k, v, o, lse, s, stream);
        case 64: return fwd_bf16<64>(q, k, v, o, lse, s, stream);
        case 128: return fwd_bf16<128>(q, k, v, o, lse, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
