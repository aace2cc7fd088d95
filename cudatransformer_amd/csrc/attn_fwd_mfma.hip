// fp32 flash-attention forward on fp32 MFMA (v_mfma_f32_32x32x2f32), gfx950.
//
// Replaces the reference forward kernel flashAttention<float> (flash_attention.cu:57-169):
// same result (O = softmax(Q K^T / sqrt(d)) V per (batch, head)), plus a causal mask and
// no zero-padded keys; it saves LSE = m + ln(l) instead of (m, l).
//
// Work decomposition
//   * one workgroup = 4 waves = BM = 128 query rows of one (batch, head); each wave owns
//     32 rows and keeps them for the whole key loop.  A causal grid (d <= 64) too short to
//     fill the chip twice over instead runs split workgroups: 64 rows, the key range halved
//     between two wave pairs, merged through LDS (fwd_split).
//   * the key loop walks BN-key blocks.  K and V blocks go straight from global memory to
//     LDS (global_load_lds_dwordx4, no staging registers), double-buffered: the next
//     block's loads are in flight during the current block's MFMAs, one barrier per block.
//     Rows are padded by one 16-byte chunk (stride d + 4 floats), which keeps the K
//     (ds_read_b128, one key row per lane) and V (ds_read_b32, one d column per lane)
//     operand reads free of bank conflicts and their addresses affine.
//   * scores are computed transposed, S^T = K Q^T (A = K from LDS, B = Q^T held in
//     registers for the whole kernel, pre-scaled by log2(e)/sqrt(d)).  In the resulting
//     accumulator each lane holds ONE query row (its column) and 16 keys per 32-key tile,
//     so the online-softmax row statistics need a single cross-lane exchange (lane ^ 32)
//     and, after exponentiation, the accumulator registers ARE the B operand of
//     O^T += V^T P^T without any data movement.
//   * the running max/denominator are kept in log2 units; exp is v_exp_f32.  O and l are
//     rescaled lazily: only when the row max grows by more than 2^8.
//   * each block runs one of two wave-uniform variants: the unmasked one (no per-element
//     checks) for blocks wholly below the wave's diagonal and inside the sequence, the
//     masked one otherwise.  Key tiles wholly above a wave's diagonal are skipped (no
//     MFMA); causal workgroups are ordered longest-first so the tail of the grid is short.
#include "attn_launch.h"
#include "attn_mfma_common.h"

#include <math.h>

#include <atomic>

namespace ctattn {
namespace {

template <int D, int BN>
struct FwdCfg {
    static constexpr int NW = 4;               // waves per workgroup
    static constexpr int BM = 32 * NW;         // query rows per workgroup
    static constexpr int KT = BN / 32;         // 32-key tiles per block
    static constexpr int DT = D / 32;          // 32-wide d tiles of O^T
    static constexpr int KS = D + 4;           // LDS row stride (floats): one pad chunk
    static constexpr int C4 = D / 4;           // 16-byte chunks of data per row
    static constexpr int C4P = C4 + 1;         // ... per LDS row
    static constexpr int TILE = BN * KS;       // floats per padded K (or V) tile
    static constexpr int CHUNKS = BN * C4P;    // 16-byte chunks per padded tile
    static constexpr int INSTR = (CHUNKS + NW * kWave - 1) / (NW * kWave);  // loads per lane per tile
    static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");
};

#define CTATTN_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// Lazy online-softmax rescaling: the running row max m (log2 units) is only raised when a
// block's max exceeds it by more than this, so most blocks skip rescaling O and l.  Scores
// are then exponentiated against a max that may be stale by up to 2^8 -- no overflow risk in
// fp32 -- and O / l and LSE = m + log2(l) use the same m, so the result is unchanged.
constexpr float kRescaleThreshold = 8.0f;

// Per-wave state of the forward key loop.
template <int D>
struct FwdState {
    floatx16 oacc[D / 32];  // O^T accumulators: lane (col=row, half) holds d = dt*32 + acc_row(r, half)
    float m_run;            // running row max (log2 units), identical in both halves
    float l_run;            // this half's share of the running denominator
};

// One BN-key block for one wave.  MASK selects the diagonal / sequence-end variant: it skips
// key tiles wholly above the wave's diagonal and masks keys > row or >= T; the unmasked
// variant carries no per-element checks.
template <int D, int BN, bool MASK>
__device__ __forceinline__ void fwd_block(FwdState<D> &st, const float (&qreg)[D / 2],
                                          const float *k_lds, const float *v_lds, int j0,
                                          int row, int wave_first_row, int wave_last_row,
                                          int T, int causal, int col, int half) {
    using C = FwdCfg<D, BN>;
    bool active[C::KT];
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        const int t0 = j0 + kt * 32;
        active[kt] = !MASK || (t0 < T && (!causal || t0 <= wave_last_row));
    }

    // S^T = K Q^T for each active 32-key tile.
    floatx16 sacc[C::KT];
    if constexpr (!MASK) {
        // Every tile active: the K reads (one ds_read_b128 per 4 MFMAs) go through a ring and
        // are issued two reads ahead of their MFMAs (sched_barrier keeps that order), so the
        // LDS latency hides behind the 8 MFMAs in between.
        constexpr int NL = C::KT * (D / 8);
        auto kread = [&](int i) __attribute__((always_inline)) {
            return *reinterpret_cast<const floatx4 *>(k_lds + ((i / (D / 8)) * 32 + col) * C::KS + 8 * (i % (D / 8)) +
                                                      4 * half);
        };
        floatx4 ring[3];
        ring[0] = kread(0);
        if (NL > 1) ring[1] = kread(1);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            if (i + 2 < NL) ring[(i + 2) % 3] = kread(i + 2);
            __builtin_amdgcn_sched_barrier(0);
            const int kt = i / (D / 8), m = i % (D / 8);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                sacc[kt] = mfma32x32x2(ring[i % 3][t], qreg[4 * m + t], (m == 0 && t == 0) ? zero16() : sacc[kt]);
        }
    } else {
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
            sacc[kt] = zero16();
            if (!active[kt]) continue;
            const int key = kt * 32 + col;
#pragma unroll
            for (int m = 0; m < D / 8; ++m) {
                const floatx4 kv = *reinterpret_cast<const floatx4 *>(k_lds + key * C::KS + 8 * m + 4 * half);
#pragma unroll
                for (int t = 0; t < 4; ++t) sacc[kt] = mfma32x32x2(kv[t], qreg[4 * m + t], sacc[kt]);
            }
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
    (void)wave_first_row;
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
    // Raise the running max only when it grew by more than the threshold somewhere.
    if (__any(mloc > st.m_run + kRescaleThreshold)) {
        const float m_new = fmaxf(st.m_run, mloc);
        const float resc = fast_exp2(st.m_run - m_new);  // 0 on the first block (m_run = -inf)
        st.m_run = m_new;
        st.l_run *= resc;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) st.oacc[dt] *= resc;
    }
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt) {
        if (!active[kt]) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = fast_exp2(sacc[kt][r] - st.m_run);
            sacc[kt][r] = p;
            psum += p;
        }
    }
    st.l_run += psum;

    // O^T += V^T P^T: the exponentiated S^T registers are the B operand.
    if constexpr (!MASK) {
        // One ds_read_b32 of V per MFMA, through a ring of 8 issued 6 MFMAs ahead.
        constexpr int NV = C::KT * C::DT * 16;
        constexpr int R = 8, AHEAD = 6;
        auto vread = [&](int i) __attribute__((always_inline)) {
            const int kt = i / (C::DT * 16), dt = (i / 16) % C::DT, s2 = i % 16;
            return v_lds[(kt * 32 + kstep_index(s2, half)) * C::KS + dt * 32 + col];
        };
        float ring[R];
#pragma unroll
        for (int i = 0; i < AHEAD && i < NV; ++i) ring[i % R] = vread(i);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (i + AHEAD < NV) ring[(i + AHEAD) % R] = vread(i + AHEAD);
            __builtin_amdgcn_sched_barrier(0);
            const int kt = i / (C::DT * 16), dt = (i / 16) % C::DT, s2 = i % 16;
            st.oacc[dt] = mfma32x32x2(ring[i % R], sacc[kt][s2], st.oacc[dt]);
        }
    } else {
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
            if (!active[kt]) continue;
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
                for (int s = 0; s < 16; ++s) {
                    const float a = v_lds[(kt * 32 + kstep_index(s, half)) * C::KS + dt * 32 + col];
                    st.oacc[dt] = mfma32x32x2(a, sacc[kt][s], st.oacc[dt]);
                }
            }
        }
    }
}

// Q^T as the B operand: lane (col = row, half) holds Q[row][kstep_index(s, half)], scaled.
template <int D>
__device__ __forceinline__ void load_qT(float (&qreg)[D / 2], const float *q, int64_t base, int row, int T,
                                        float qscale, int half) {
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
        floatx4 x = {0.f, 0.f, 0.f, 0.f};
        if (row < T) x = *reinterpret_cast<const floatx4 *>(q + base + int64_t(row) * D + 8 * m + 4 * half);
#pragma unroll
        for (int t = 0; t < 4; ++t) qreg[4 * m + t] = x[t] * qscale;
    }
}

// O row = O^T accumulators / l, LSE = (m + log2 l) ln 2 (l summed over the lane pair).
template <int D>
__device__ __forceinline__ void store_rows(const FwdState<D> &st, float *o, float *lse, int64_t base, int bh,
                                           int row, int T, int half) {
    const float l_tot = st.l_run + __shfl_xor(st.l_run, 32, kWave);
    const float inv_l = 1.f / l_tot;
    if (row < T) {
        float *orow = o + base + int64_t(row) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                floatx4 x;
#pragma unroll
                for (int t = 0; t < 4; ++t) x[t] = st.oacc[dt][4 * g + t] * inv_l;
                *reinterpret_cast<floatx4 *>(orow + dt * 32 + 8 * g + 4 * half) = x;
            }
        }
        if (lse != nullptr && half == 0) lse[int64_t(bh) * T + row] = (st.m_run + __log2f(l_tot)) * kLn2;
    }
}

// A whole 128-row query block: wave w owns rows q0 + 32 w .., the key loop walks BN-key blocks
// up to the block's last row (causal) or T.
template <int D, int BN>
__device__ __forceinline__ void fwd_whole(float *k_lds, float *v_lds,
                                          const float *__restrict__ q, const float *__restrict__ k,
                                          const float *__restrict__ v, float *__restrict__ o,
                                          float *__restrict__ lse, int T, int bh, int qb, int causal, float qscale,
                                          int wave, int lane) {
    using C = FwdCfg<D, BN>;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int64_t base = int64_t(bh) * T * D;
    const int q0 = qb * C::BM;
    const int row = q0 + wave * 32 + col;  // query row owned by this lane
    const int wave_first_row = q0 + wave * 32;
    const int wave_last_row = wave_first_row + 31;

    float qreg[D / 2];
    load_qT<D>(qreg, q, base, row, T, qscale, half);

    FwdState<D> st;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) st.oacc[dt] = zero16();
    st.m_run = -INFINITY;
    st.l_run = 0.f;

    const int kend = causal ? min(T, q0 + C::BM) : T;
    const int nkb = (kend + BN - 1) / BN;

    // Global -> LDS for one block: lane writes LDS chunk P = (wave * INSTR + i) * 64 + lane of
    // the padded tile, i.e. row P / C4P, chunk P % C4P; the pad chunk (C4) re-reads chunk 0
    // of the row and is never used.  Rows past T re-read row T - 1 (masked).
    auto issue = [&](int j0, int buf) {
#pragma unroll
        for (int i = 0; i < C::INSTR; ++i) {
            const int P = (wave * C::INSTR + i) * kWave + lane;
            if (C::CHUNKS % (C::NW * kWave) == 0 || P < C::CHUNKS) {
                const int r = P / C::C4P;
                const int c = P - r * C::C4P;
                const int64_t goff = base + int64_t(min(j0 + r, T - 1)) * D + 4 * (c < C::C4 ? c : 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(k + goff),
                                                 CTATTN_LDS(k_lds + buf * C::TILE + (wave * C::INSTR + i) * 4 * kWave), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(v + goff),
                                                 CTATTN_LDS(v_lds + buf * C::TILE + (wave * C::INSTR + i) * 4 * kWave), 16, 0, 0);
            }
        }
    };

    issue(0, 0);
    for (int kb = 0; kb < nkb; ++kb) {
        const int j0 = kb * BN;
        const int buf = kb & 1;
        // This lane's loads into `buf` have landed (vmcnt = 0); the barrier then makes every
        // lane's loads visible and guarantees every wave is done reading buf ^ 1.
        __builtin_amdgcn_s_waitcnt(0xF70);
        __syncthreads();
        if (kb + 1 < nkb) issue(j0 + BN, buf ^ 1);

        // Wave-uniform: does this block touch the diagonal or the sequence end for this wave?
        const bool masked = (j0 + BN > T) || (causal && j0 + BN - 1 > wave_first_row);
        if (masked) {
            if (!causal || j0 <= wave_last_row)
                fwd_block<D, BN, true>(st, qreg, k_lds + buf * C::TILE, v_lds + buf * C::TILE, j0, row, wave_first_row,
                                       wave_last_row, T, causal, col, half);
        } else {
            fwd_block<D, BN, false>(st, qreg, k_lds + buf * C::TILE, v_lds + buf * C::TILE, j0, row, wave_first_row,
                                    wave_last_row, T, causal, col, half);
        }
    }
    store_rows<D>(st, o, lse, base, bh, row, T, half);
}

// A split workgroup (causal only): 64 query rows R0 .. R0 + 63, its key range [0, R0 + 64)
// cut in two halves of 32-key blocks.  Waves 2 h and 2 h + 1 (rows R0 .. R0 + 31 and
// R0 + 32 .. R0 + 63) walk half h with their own double-buffered tiles (the first / second
// 32 rows of each BN = 64 tile buffer), then half 1 hands its O^T, m and l to half 0 through
// LDS and half 0 merges and stores.  Each 128-row query block of a short causal grid becomes
// two such workgroups, each with about a quarter of its key work, so the longest block no
// longer sets the kernel's length.
template <int D>
__device__ __forceinline__ void fwd_split(float *k_lds, float *v_lds,
                                          const float *__restrict__ q, const float *__restrict__ k,
                                          const float *__restrict__ v, float *__restrict__ o,
                                          float *__restrict__ lse, int T, int bh, int R0, float qscale, int wave,
                                          int lane) {
    using C = FwdCfg<D, 32>;
    constexpr int GW = 2;                                      // waves per half
    constexpr int INSTR = (C::CHUNKS + GW * kWave - 1) / (GW * kWave);  // loads per lane per tile
    const int rs = wave & 1, h = wave >> 1;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int64_t base = int64_t(bh) * T * D;
    const int wave_first_row = R0 + 32 * rs;
    const int wave_last_row = wave_first_row + 31;
    const int row = wave_first_row + col;

    float qreg[D / 2];
    load_qT<D>(qreg, q, base, row, T, qscale, half);

    FwdState<D> st;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) st.oacc[dt] = zero16();
    st.m_run = -INFINITY;
    st.l_run = 0.f;

    const int nk = (min(T, R0 + 64) + 31) / 32;  // 32-key blocks of the workgroup
    const int n0 = (nk + 1) / 2;                  // half 0: [0, n0), half 1: [n0, nk)
    const int kb0 = h ? n0 : 0, kb1 = h ? nk : n0;
    float *kt0 = k_lds + h * C::TILE, *kt1 = k_lds + 2 * C::TILE + h * C::TILE;
    float *vt0 = v_lds + h * C::TILE, *vt1 = v_lds + 2 * C::TILE + h * C::TILE;

    auto issue = [&](int kb, int buf) {
        float *kt = buf ? kt1 : kt0;
        float *vt = buf ? vt1 : vt0;
        const int j0 = kb * 32;
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int P = (rs * INSTR + i) * kWave + lane;
            if (C::CHUNKS % (GW * kWave) == 0 || P < C::CHUNKS) {
                const int r = P / C::C4P;
                const int c = P - r * C::C4P;
                const int64_t goff = base + int64_t(min(j0 + r, T - 1)) * D + 4 * (c < C::C4 ? c : 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(k + goff),
                                                 CTATTN_LDS(kt + (rs * INSTR + i) * 4 * kWave), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(v + goff),
                                                 CTATTN_LDS(vt + (rs * INSTR + i) * 4 * kWave), 16, 0, 0);
            }
        }
    };

    if (kb0 < kb1) issue(kb0, 0);
    for (int it = 0; it < n0; ++it) {  // half 1 has n0 or n0 - 1 blocks: every wave meets n0 barriers
        const int kb = kb0 + it;
        const int buf = it & 1;
        __builtin_amdgcn_s_waitcnt(0xF70);
        __syncthreads();
        if (kb + 1 < kb1) issue(kb + 1, buf ^ 1);
        if (kb < kb1) {
            const int j0 = kb * 32;
            const float *kt = buf ? kt1 : kt0;
            const float *vt = buf ? vt1 : vt0;
            const bool masked = (j0 + 32 > T) || (j0 + 31 > wave_first_row);
            if (masked) {
                if (j0 <= wave_last_row)
                    fwd_block<D, 32, true>(st, qreg, kt, vt, j0, row, wave_first_row, wave_last_row, T, 1, col,
                                           half);
            } else {
                fwd_block<D, 32, false>(st, qreg, kt, vt, j0, row, wave_first_row, wave_last_row, T, 1, col, half);
            }
        }
    }

    // Merge: half 1's lane (row, half) state lands at mb[(rs * NR + i) * 64 + lane]; both
    // halves' O^T / l are relative to their own running max m (log2 units), so
    //   m = max(m0, m1), O = O0 2^(m0 - m) + O1 2^(m1 - m), l likewise.
    // Half 0 always holds key 0 of its rows, so m0 is finite; an empty half 1 has m1 = -inf,
    // weight 0.
    constexpr int NR = C::DT * 16 + 2;
    float *mb = k_lds;
    __syncthreads();  // every wave is done with the tiles
    if (h == 1) {
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) mb[(rs * NR + dt * 16 + r) * kWave + lane] = st.oacc[dt][r];
        mb[(rs * NR + NR - 2) * kWave + lane] = st.m_run;
        mb[(rs * NR + NR - 1) * kWave + lane] = st.l_run;
    }
    __syncthreads();
    if (h == 0) {
        const float m1 = mb[(rs * NR + NR - 2) * kWave + lane];
        const float l1 = mb[(rs * NR + NR - 1) * kWave + lane];
        const float m = fmaxf(st.m_run, m1);
        const float a0 = fast_exp2(st.m_run - m), a1 = fast_exp2(m1 - m);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st.oacc[dt][r] = st.oacc[dt][r] * a0 + mb[(rs * NR + dt * 16 + r) * kWave + lane] * a1;
        st.l_run = st.l_run * a0 + l1 * a1;
        st.m_run = m;
        store_rows<D>(st, o, lse, base, bh, row, T, half);
    }
}

template <int D, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_f32_mfma_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v, float *__restrict__ o,
    float *__restrict__ lse, int T, int BH, int causal, float qscale, int split) {
    using C = FwdCfg<D, BN>;
    __shared__ __attribute__((aligned(16))) float k_lds[2][C::TILE];
    __shared__ __attribute__((aligned(16))) float v_lds[2][C::TILE];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int id = blockIdx.x;
    const int bh = id % BH;
    if constexpr (BN == 64) {
        if (split) {  // causal, 64-row split workgroups, longest first
            const int rb = (T + 63) / 64 - 1 - id / BH;
            fwd_split<D>(&k_lds[0][0], &v_lds[0][0], q, k, v, o, lse, T, bh, 64 * rb, qscale, wave, lane);
            return;
        }
    }
    const int nqb = (T + C::BM - 1) / C::BM;
    const int qb = causal ? (nqb - 1 - id / BH) : id / BH;  // causal: longest first
    fwd_whole<D, BN>(&k_lds[0][0], &v_lds[0][0], q, k, v, o, lse, T, bh, qb, causal, qscale, wave, lane);
}

// Split workgroups pay for themselves when the causal grid of whole 128-row blocks has no more
// workgroups than the chip has slots (two per CU): then the longest blocks are the whole
// kernel, and cutting every block into two 64-row workgroups with halved key ranges shortens
// them four times over.  Measured (B x H x T, d = 64): 1x4x2048 83.6 -> 50.7 us, 2x16x1024
// 76.7 -> 61.7, 8x12x512 55.6 -> 47.9; at 768 and more whole blocks splitting is within
// +-3 % (8x12x1024 133.4 / 132.1, 1x12x8192 859.5 / 877.4, 32x12x1024 479.4 / 494.2), so
// those keep whole blocks.
bool fwd_use_split(const AttnShape &s, hipStream_t stream) {
    const int cus = device_cus(stream);
    return cus > 0 && (s.T + 127) / 128 * s.bh() <= int64_t(2) * cus;
}

template <int D, int BN>
hipError_t fwd_f32(const float *q, const float *k, const float *v, float *o, float *lse,
                   const AttnShape &s, hipStream_t stream) {
    using C = FwdCfg<D, BN>;
    const int64_t nqb = (s.T + C::BM - 1) / C::BM;
    const int64_t blocks = nqb * s.bh();
    if (!grid_fits(blocks, C::NW * kWave) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const float qscale = kLog2e / sqrtf(float(s.scale_dim()));
    const int split = BN == 64 && s.causal && fwd_use_split(s, stream);
    const int64_t grid = split ? (s.T + 63) / 64 * s.bh() : blocks;
    if (!grid_fits(grid, C::NW * kWave)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((fwd_f32_mfma_kernel<D, BN>), dim3(unsigned(grid)), dim3(C::NW * kWave), 0, stream, q, k, v,
                       o, lse, int(s.T), int(s.bh()), int(s.causal), qscale, split);
    return hipGetLastError();
}

}  // namespace

int device_cus(hipStream_t stream) {
    static std::atomic<int> cus_of[64];
    int dev = 0;
    if ((stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev)) != hipSuccess || dev < 0 || dev >= 64)
        return 0;
    int cus = cus_of[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return 0;
        cus_of[dev].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

bool mfma_fwd_supported(int dtype, int64_t d) {
    (void)dtype;  // the fp32, bf16 and fp16 kernels all cover d in {32, 64, 128}
    return d == 32 || d == 64 || d == 128;
}

hipError_t launch_mfma_fwd(int dtype, const void *q, const void *k, const void *v, void *o,
                           float *lse, const AttnShape &s, hipStream_t stream) {
    if (dtype == 1) return launch_bf16_fwd(q, k, v, o, lse, s, stream);
    if (dtype == 2) return launch_f16_fwd(q, k, v, o, lse, s, stream);
    const float *qf = static_cast<const float *>(q);
    const float *kf = static_cast<const float *>(k);
    const float *vf = static_cast<const float *>(v);
    float *of = static_cast<float *>(o);
    switch (s.d) {
        case 32: return fwd_f32<32, 64>(qf, kf, vf, of, lse, s, stream);
        case 64: return fwd_f32<64, 64>(qf, kf, vf, of, lse, s, stream);
        case 128: return fwd_f32<128, 32>(qf, kf, vf, of, lse, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
