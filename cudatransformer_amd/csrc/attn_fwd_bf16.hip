// bf16 / fp16 flash-attention forward on 16-bit MFMA (v_mfma_f32_32x32x16_bf16 / _f16), fp32
// accumulate.  The fp16 instantiation (F16Fmt) is the same code with the fp16 MFMA and fp16
// rounding of P and O.
//
// Same result as the fp32 forward and as the reference's flashAttention<__nv_bfloat16>
// (flash_attention.cu:57-169) except that scores and sums accumulate in fp32 (the reference
// accumulates the dot products in bf16, flash_attention.cu:112-116).  O is rounded to bf16
// (nearest even) once at the end; LSE is fp32.
//
// Decomposition: a workgroup of 4 waves owns 128 query rows (wave w: 32 rows for the whole
// key loop); K and V stream through LDS in 64-key blocks, loaded global -> LDS directly into
// swizzled row-major tiles (attn_bf16_tiles.h), double-buffered with one barrier per block.
// Scores are computed transposed, S^T = K Q^T (A = K rows from LDS, B = this lane's Q row in
// registers for the whole kernel), so each lane holds one query row and the online-softmax
// statistics need one lane ^ 32 exchange.  After exponentiation the accumulator registers
// 8 s .. 8 s + 7 are the B operand of O^T += V^T P^T for keys 16 s + 8 (e / 4) + 4 half +
// e % 4, and A = V^T comes from the row-major V tile through ds_read_b64_tr_b16 in that key
// order.  The score scale log2(e)/sqrt(d) is applied in fp32 inside exp2's argument (an fma),
// not folded into bf16 Q; O and l are rescaled lazily, only when the row max grows by more
// than 2^8.
#include "attn_bf16_tiles.h"
#include "attn_launch.h"

#include <math.h>

namespace ctattn {
namespace {

using namespace bf16tile;

template <int D>
struct FwdBf16Cfg {
    static constexpr int NW = 4;
    static constexpr int BM = 32 * NW;   // query rows per workgroup
    static constexpr int BN = 64;        // keys per block
    static constexpr int KT = BN / 32;   // 32-key tiles per block
    static constexpr int DT = D / 32;    // 32-wide d tiles of O^T
    static constexpr int KSTEPS = D / 16;
    static constexpr int ROW = 2 * D;             // bytes per tile row
    static constexpr int KB = BN * ROW;           // bytes of a K (or V) block tile
    static constexpr int LDS_BYTES = 4 * KB;      // buffer b: K at 2 b KB, V at 2 b KB + KB
    static_assert(KB + BN * ROW <= 65536, "immediate offsets");
};

constexpr float kRescaleThresholdBf16 = 8.0f;

template <int D>
struct FwdBf16State {
    floatx16 oacc[D / 32];  // O^T: lane (row, half), register r of tile dt -> d = 32 dt + acc_row(r, half)
    float m_run;            // running max of S * log2(e)/sqrt(d), identical in both halves
    float l_run;            // this half's share of the running denominator
};

// One 64-key block for one wave.  ak: row_base of the block's K tile for key `col` (V at
// + KB); vc0 / vc1: col_base of the V tile.  MASK selects the diagonal / sequence-end variant.
template <int D, bool MASK, typename F>
__device__ __forceinline__ void fwd_bf16_block(FwdBf16State<D> &st, const typename F::vec (&qb)[D / 16], uint32_t ak,
                                               uint32_t vc0, uint32_t vc1, int j0, int row, int wave_last_row,
                                               int T, int causal, float c, int half) {
    using C = FwdBf16Cfg<D>;
    using V = typename F::vec;
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
        const uint32_t a = ak + uint32_t(32 * kt * C::ROW);
        V ka[2];
        ka[0] = lds_b128<V>(a);
#pragma unroll
        for (int s = 0; s < C::KSTEPS; ++s) {
            if (s + 1 < C::KSTEPS) ka[(s + 1) & 1] = lds_b128<V>(a ^ uint32_t((s + 1) << 5));
            read_fence();
            sacc[kt] = F::mfma(ka[s & 1], qb[s], sacc[kt]);
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
    V pb[C::KT][2];
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
                pb[kt][s][e] = (typename F::elem)p;
            }
        }
    }
    st.l_run += psum;
    // O^T += V^T P^T: k-step kk of key tile kt covers tile rows 16 (2 kt + kk) + ...
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        if (!active[kt]) continue;
        constexpr int NS = 2 * C::DT;
        V va[2];
        va[0] = read_col<D, V>(vc0, vc1, 2 * kt, 0);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (i + 1 < NS) va[(i + 1) & 1] = read_col<D, V>(vc0, vc1, 2 * kt + (i + 1) / C::DT, (i + 1) % C::DT);
            read_fence();
            st.oacc[i % C::DT] = F::mfma(va[i & 1], pb[kt][i / C::DT], st.oacc[i % C::DT]);
        }
    }
}

template <int D, typename F>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_bf16_mfma_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    uint16_t *__restrict__ o, float *__restrict__ lse, int T, int BH, int causal, float c) {
    using C = FwdBf16Cfg<D>;
    using V = typename F::vec;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
    const uint32_t L = lds_addr(smem);

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int nqb = (T + C::BM - 1) / C::BM;
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int qblk = causal ? (nqb - 1 - id / BH) : id / BH;  // causal: longest first
    const int64_t base = int64_t(bh) * T * D;
    const int q0 = qblk * C::BM;
    const int row = q0 + wave * 32 + col;
    const int wave_first_row = q0 + wave * 32;
    const int wave_last_row = wave_first_row + 31;

    // Q^T as the B operand: lane (row, half) holds Q[row][16s + 8*half .. +7].
    V qb[C::KSTEPS];
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) {
        u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
        if (row < T) x = *reinterpret_cast<const u16x8 *>(q + base + int64_t(row) * D + 16 * s + 8 * half);
        qb[s] = __builtin_bit_cast(V, x);
    }

    FwdBf16State<D> st;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) st.oacc[dt] = zero16();
    st.m_run = -INFINITY;
    st.l_run = 0.f;

    const uint32_t rk = uint32_t(Tile<D>::off(col, half));
    const uint32_t cv0 = col_base<D>(0, 0, 0, lane), cv1 = col_base<D>(0, 0, 1, lane);

    const int kend = causal ? min(T, q0 + C::BM) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;
    auto issue = [&](int j0, int buf) {
        load_tile<D, C::BN, C::NW>(smem + 2 * buf * C::KB, k + base, j0, T, wave, lane);
        load_tile<D, C::BN, C::NW>(smem + 2 * buf * C::KB + C::KB, v + base, j0, T, wave, lane);
    };

    issue(0, 0);
    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        // This wave's loads of `buf` have landed (vmcnt = 0); after the barrier every wave's
        // have, and every wave is done reading buf ^ 1.
        __builtin_amdgcn_s_waitcnt(0xF70);
        __syncthreads();
        if (kb + 1 < nkb) issue((kb + 1) * C::BN, buf ^ 1);
        const int j0 = kb * C::BN;
        const uint32_t kt = L + uint32_t(2 * buf * C::KB);
        const bool masked = (j0 + C::BN > T) || (causal && j0 + C::BN - 1 > wave_first_row);
        if (masked) {
            if (!causal || j0 <= wave_last_row)
                fwd_bf16_block<D, true, F>(st, qb, kt + rk, kt + C::KB + cv0, kt + C::KB + cv1, j0, row,
                                        wave_last_row, T, causal, c, half);
        } else {
            fwd_bf16_block<D, false, F>(st, qb, kt + rk, kt + C::KB + cv0, kt + C::KB + cv1, j0, row, wave_last_row,
                                     T, causal, c, half);
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
                for (int t = 0; t < 4; ++t) x[t] = F::bits(st.oacc[dt][4 * g + t] * inv_l);
                *reinterpret_cast<u16x4 *>(orow + dt * 32 + 8 * g + 4 * half) = x;
            }
        }
        if (lse != nullptr && half == 0) lse[int64_t(bh) * T + row] = (st.m_run + __log2f(l_tot)) * kLn2;
    }
}

template <int D, typename F>
hipError_t fwd_bf16(const void *q, const void *k, const void *v, void *o, float *lse, const AttnShape &s,
                    hipStream_t stream) {
    using C = FwdBf16Cfg<D>;
    const int64_t nqb = (s.T + C::BM - 1) / C::BM;
    const int64_t blocks = nqb * s.bh();
    if (!grid_fits(blocks, C::NW * kWave) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const float c = kLog2e / sqrtf(float(D));
    hipLaunchKernelGGL((fwd_bf16_mfma_kernel<D, F>), dim3(unsigned(blocks)), dim3(C::NW * kWave), 0, stream,
                       static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                       static_cast<const uint16_t *>(v), static_cast<uint16_t *>(o), lse, int(s.T),
                       int(s.bh()), int(s.causal), c);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bf16_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                           const AttnShape &s, hipStream_t stream) {
    switch (s.d) {
        case 32: return fwd_bf16<32, Bf16Fmt>(q, k, v, o, lse, s, stream);
        case 64: return fwd_bf16<64, Bf16Fmt>(q, k, v, o, lse, s, stream);
        case 128: return fwd_bf16<128, Bf16Fmt>(q, k, v, o, lse, s, stream);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_f16_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                          const AttnShape &s, hipStream_t stream) {
    switch (s.d) {
        case 32: return fwd_bf16<32, F16Fmt>(q, k, v, o, lse, s, stream);
        case 64: return fwd_bf16<64, F16Fmt>(q, k, v, o, lse, s, stream);
        case 128: return fwd_bf16<128, F16Fmt>(q, k, v, o, lse, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
