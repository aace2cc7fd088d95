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

#include <type_traits>

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
// Bound on a lane's share of one block's P in the ping-pong kernel (2^8, the same bound on
// every P as kRescaleThresholdBf16 gives).
constexpr float kPsumLimit = 256.0f;

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
    if (MASK) {
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
            if (!active[kt]) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = j0 + kt * 32 + acc_row(r, half);
                if (key >= T || (causal && key > row)) sacc[kt][r] = -INFINITY;
            }
        }
    }
    // P^T = exp2(S c - m), rounded to bf16 as the B operand; the denominator sums the same
    // fp32 values.  First against the running max without the block's max: if every lane's
    // share of the block's P stays <= 2^8, so does every P, i.e. the block max is within the
    // lazy-rescale threshold of m and the max-based rule would not rescale either.  Otherwise
    // (the max grew by more, or m is still -inf and the sums are inf / NaN) the block max is
    // taken, the rule applied as before and P recomputed: the same values either way, one
    // max per score saved on every block where the max holds.
    V pb[C::KT][2];
    float psum = 0.f;
    auto exp_block = [&]() __attribute__((always_inline)) {
        psum = 0.f;
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
    };
    exp_block();
    if (__any(!(psum <= kPsumLimit))) {
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
            if (!active[kt]) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, sacc[kt][r]);
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
        exp_block();
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

template <int D, typename F, bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_bf16_mfma_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    uint16_t *__restrict__ o, float *__restrict__ lse, int T, int BH, int causal, float c) {
    using C = FwdBf16Cfg<D>;
    using V = typename F::vec;
    // SPLIT (causal): 64 query rows per workgroup; waves 2 h and 2 h + 1 (rows q0 .. q0 + 31
    // and q0 + 32 .. q0 + 63) walk half h of the key blocks with their own tiles, and half 1's
    // O / m / l are merged into half 0's through LDS at the end.
    constexpr int GW = SPLIT ? 2 : C::NW;    // waves that load one half's tiles
    constexpr int RB = SPLIT ? 64 : C::BM;   // query rows per workgroup
    __shared__ __attribute__((aligned(1024))) char smem_all[(SPLIT ? 2 : 1) * C::LDS_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int hk = SPLIT ? wave >> 1 : 0;      // key half
    const int wl = SPLIT ? (wave & 1) : wave;  // row slot
    const int col = lane & 31;
    const int half = lane >> 5;
    char *smem = smem_all + (SPLIT ? hk * C::LDS_BYTES : 0);
    const uint32_t L = lds_addr(smem);

    const int nqb = (T + RB - 1) / RB;
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int qblk = causal ? (nqb - 1 - id / BH) : id / BH;  // causal: longest first
    const int64_t base = int64_t(bh) * T * D;
    const int q0 = qblk * RB;
    const int row = q0 + wl * 32 + col;
    const int wave_first_row = q0 + wl * 32;
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

    const int kend = causal ? min(T, q0 + RB) : T;
    const int nkb_all = (kend + C::BN - 1) / C::BN;
    // This wave's key blocks: [kb_lo, kb_hi); every wave meets `iters` barriers.
    const int n0 = (nkb_all + 1) / 2;
    const int kb_lo = SPLIT && hk ? n0 : 0;
    const int kb_hi = SPLIT && !hk ? n0 : nkb_all;
    const int iters = SPLIT ? n0 : nkb_all;
    auto issue = [&](int j0, int buf) {
        load_tile<D, C::BN, GW>(smem + 2 * buf * C::KB, k + base, j0, T, wl, lane);
        load_tile<D, C::BN, GW>(smem + 2 * buf * C::KB + C::KB, v + base, j0, T, wl, lane);
    };

    if (kb_lo < kb_hi) issue(kb_lo * C::BN, 0);
    for (int it = 0; it < iters; ++it) {
        const int kb = kb_lo + it;
        const int buf = it & 1;
        // This wave's loads of `buf` have landed (vmcnt = 0); after the barrier every wave's
        // have, and every wave is done reading buf ^ 1.
        __builtin_amdgcn_s_waitcnt(0xF70);
        __syncthreads();
        if (kb + 1 < kb_hi) issue((kb + 1) * C::BN, buf ^ 1);
        if (kb >= kb_hi) continue;
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

    if constexpr (SPLIT) {
        // Half 1's lane state at mb[(wl NR + i) 64 + lane]; half 0's wave wl merges it:
        // m = max(m0, m1) (log2 units, times c), O = O0 2^(m0 - m) + O1 2^(m1 - m), l likewise.
        // Half 0 holds key 0 of its rows, so m0 is finite; an empty half 1 has m1 = -inf.
        constexpr int NR = C::DT * 16 + 2;
        static_assert(2 * NR * kWave * 4 <= 2 * C::LDS_BYTES, "merge buffer");
        float *mb = reinterpret_cast<float *>(smem_all);
        __syncthreads();  // every wave is done with the tiles
        if (hk == 1) {
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) mb[(wl * NR + dt * 16 + r) * kWave + lane] = st.oacc[dt][r];
            mb[(wl * NR + NR - 2) * kWave + lane] = st.m_run;
            mb[(wl * NR + NR - 1) * kWave + lane] = st.l_run;
        }
        __syncthreads();
        if (hk == 1) return;
        const float m1 = mb[(wl * NR + NR - 2) * kWave + lane];
        const float l1 = mb[(wl * NR + NR - 1) * kWave + lane];
        const float m = fmaxf(st.m_run, m1);
        const float a0 = fast_exp2(st.m_run - m), a1 = fast_exp2(m1 - m);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st.oacc[dt][r] = st.oacc[dt][r] * a0 + mb[(wl * NR + dt * 16 + r) * kWave + lane] * a1;
        st.l_run = st.l_run * a0 + l1 * a1;
        st.m_run = m;
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

// ---- Ping-pong forward: 8 waves, two groups offset by one phase ----
//
// The softmax of a 64-key block (max, exp2, sum, bf16 rounding: ~1000 VALU cycles per wave)
// costs about as much as the block's MFMAs (32 x 32 cycles), and two independent waves on a
// SIMD drift into running both phases at the same time.  Here a workgroup holds 8 waves, two
// per SIMD (waves w and w + 4 share one): group A (waves 0-3) and group B (waves 4-7)
// alternate between an MFMA phase M(j) -- S_j = K_j Q^T and O += V_{j-1} P_{j-1} -- and a
// VALU phase V(j) -- the online softmax of S_j into P_j -- with group B one phase behind
// group A: between two workgroup barriers (one per iteration; SPLIT: one per phase) group A
// runs M(j + 1), V(j + 1) and group B V(j), M(j + 1), so one wave of each SIMD runs MFMAs
// while the other runs VALU work (s_setprio raises the MFMA phase's issue priority).  Each
// wave owns 32 query rows (256 per workgroup).
//
// K and V blocks are double-buffered (block j in buffer j & 1).  The loads of K_{j+1} and V_j
// are issued at the start of the iteration in which A runs M(j) and awaited (vmcnt) before
// its closing barrier; they go through load_tile_dma, and the barrier (lds_barrier) does not
// drain them, so no LDS read ever waits for a prefetch.
// Short causal grids take the split kernel when they have at most this many whole
// workgroups per CU (two per CU made B1 H32 T4096 and B2 H16 T4096 slower, 136 -> 160 us).
constexpr int kPpSplitWorkgroupsPerCu = 1;
template <int D>
struct FwdPpCfg {
    static constexpr int NW = 8;          // waves: group A = 0-3, group B = 4-7
    static constexpr int BM = 32 * NW;    // query rows per workgroup
    static constexpr int BN = 64;         // keys per block
    static constexpr int KT = BN / 32;
    static constexpr int DT = D / 32;
    static constexpr int KSTEPS = D / 16;
    static constexpr int ROW = 2 * D;
    static constexpr int KB = BN * ROW;   // bytes of one K or V tile
    static constexpr int LDS_BYTES = 4 * KB;  // K0, K1, V0, V1
};

template <int D, typename F, bool SPLIT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_bf16_pp_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    uint16_t *__restrict__ o, float *__restrict__ lse, int T, int BH, int causal, float c) {
    using C = FwdPpCfg<D>;
    using V = typename F::vec;
    // SPLIT (causal): the workgroup owns 128 query rows; both groups hold the same rows
    // (waves w and w + 4 the same 32), group A walks the first half of the key blocks and
    // group B the second, each with its own tiles, and B's O / m / l are merged into A's at
    // the end.
    constexpr int GW = SPLIT ? 4 : C::NW;    // waves that load one group's tiles
    constexpr int RB = SPLIT ? 128 : C::BM;  // query rows per workgroup
    __shared__ __attribute__((aligned(1024))) char smem_all[(SPLIT ? 2 : 1) * C::LDS_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    // Wave-uniform: every branch on the wave index is a scalar branch.
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int group = wave >> 2;
    const int wl = SPLIT ? (wave & 3) : wave;  // row slot of the wave
    const int col = lane & 31;
    const int half = lane >> 5;
    char *smem = smem_all + (SPLIT ? group * C::LDS_BYTES : 0);

    const int nqb = (T + RB - 1) / RB;
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int qblk = causal ? (nqb - 1 - id / BH) : id / BH;  // causal: longest first
    const int64_t base = int64_t(bh) * T * D;
    const int q0 = qblk * RB;
    const int row = q0 + wl * 32 + col;
    const int wave_first_row = q0 + wl * 32;
    const int wave_last_row = wave_first_row + 31;

    V qb[C::KSTEPS];
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) {
        u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
        if (row < T) x = *reinterpret_cast<const u16x8 *>(q + base + int64_t(row) * D + 16 * s + 8 * half);
        qb[s] = __builtin_bit_cast(V, x);
    }

    floatx16 oacc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) oacc[dt] = zero16();
    float m_run = -INFINITY, l_run = 0.f;
    floatx16 sacc[C::KT];
    V pb[C::KT][2];

    const uint32_t rk = uint32_t(Tile<D>::off(col, half));
    const uint32_t cv0 = col_base<D>(0, 0, 0, lane), cv1 = col_base<D>(0, 0, 1, lane);
    // Register r of a lane in `half` holds key j0 + 32 kt + acc_row(r, 0) + 4 half: masks
    // compare that uniform part against per-lane bounds shifted by 4 half.
    const int row_lim = causal ? row - 4 * half : 0x7fffffff;  // masked: key_u > row_lim
    const int t_lim = T - 4 * half;                            // masked: key_u >= t_lim

    const int kend = causal ? min(T, q0 + RB) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;
    // This group's key blocks: global block kb_lo + j for local j in [0, len); every wave runs
    // local iterations 0 .. jlast (the last one only finishes O).
    const int n0 = (nkb + 1) / 2;
    const int kb_lo = SPLIT && group ? n0 : 0;
    const int len = SPLIT ? (group ? nkb - n0 : n0) : nkb;
    const int jlast = SPLIT ? n0 : nkb;
    // Blocks this wave has keys in: the causal diagonal ends it early.
    const int wave_nkb = causal ? min(nkb, min(wave_last_row, T - 1) / C::BN + 1) : nkb;

    auto ktile = [&](int j) __attribute__((always_inline)) { return smem + (j & 1) * C::KB; };
    auto vtile = [&](int j) __attribute__((always_inline)) { return smem + (2 + (j & 1)) * C::KB; };
    // Key tiles of block j this wave computes: inside the sequence and, causal, not wholly
    // above its diagonal.
    auto tile_active = [&](int j, int kt) __attribute__((always_inline)) {
        const int t0 = (kb_lo + j) * C::BN + kt * 32;
        return t0 < T && (!causal || t0 <= wave_last_row);
    };
    // Batch j: K_{j+1} and V_j, each wave its share.
    auto issue = [&](int j) __attribute__((always_inline)) {
        const int jk = kb_lo + j + 1, jv = kb_lo + j;  // global key blocks of K_{j+1} and V_j
        if (j + 1 < len)
            load_tile_dma<D, C::BN, GW>(ktile(j + 1), k + base + int64_t(jk) * C::BN * D, T - jk * C::BN,
                                        SPLIT ? wl : wave, lane);
        if (j < len)
            load_tile_dma<D, C::BN, GW>(vtile(j), v + base + int64_t(jv) * C::BN * D, T - jv * C::BN,
                                        SPLIT ? wl : wave, lane);
    };

    // M(j): O += V_{j-1} P_{j-1} (16 MFMAs at d = 128), then S_j = K_j Q^T (16), as one
    // sequence whose operands come through a ring of kRing registers, read kRing - 1 MFMAs
    // ahead so the LDS latency hides behind the MFMAs in between.  Key tiles above a wave's
    // diagonal are computed anyway (their P is zero, their S is never read): the sequence has
    // no branches.
    constexpr int kRing = 4;
    constexpr int NPV = C::KT * 2 * C::DT;
    constexpr int NSC = C::KT * C::KSTEPS;
    auto mphase_t = [&](auto has_pv, auto has_s, int j) __attribute__((always_inline)) {
        constexpr bool PV = decltype(has_pv)::value, SC = decltype(has_s)::value;
        constexpr int FIRST = PV ? 0 : NPV, LAST = SC ? NPV + NSC : NPV;
        const char *vt_ = vtile(j - 1);
        const char *kt_ = ktile(j);
        auto operand = [&](int i) __attribute__((always_inline)) -> V {
            if (i < NPV) {
                const int kt = i / (2 * C::DT), ii = i % (2 * C::DT);
                return tile_col<D, V>(vt_, cv0, cv1, 2 * kt + ii / C::DT, ii % C::DT);
            }
            const int kt = (i - NPV) / C::KSTEPS, st = (i - NPV) % C::KSTEPS;
            return tile_b128<V>(kt_, (rk + uint32_t(32 * kt * C::ROW)) ^ uint32_t(st << 5));
        };
        V ring[kRing];
#pragma unroll
        for (int i = FIRST; i < FIRST + kRing - 1 && i < LAST; ++i) ring[i % kRing] = operand(i);
#pragma unroll
        for (int i = FIRST; i < LAST; ++i) {
            if (i + kRing - 1 < LAST) ring[(i + kRing - 1) % kRing] = operand(i + kRing - 1);
            read_fence();
            if (i < NPV) {
                const int kt = i / (2 * C::DT), ii = i % (2 * C::DT);
                oacc[ii % C::DT] = F::mfma(ring[i % kRing], pb[kt][ii / C::DT], oacc[ii % C::DT]);
            } else {
                const int kt = (i - NPV) / C::KSTEPS, st = (i - NPV) % C::KSTEPS;
                sacc[kt] = F::mfma(ring[i % kRing], qb[st], st == 0 ? zero16() : sacc[kt]);
            }
        }
    };
    // V(j): online softmax of S_j into P_j (bf16), running max / denominator.  MASK: the
    // block crosses the wave's diagonal or the sequence end (masked scores become -inf).
    // P is computed against the running max without a block max first: if every lane's share
    // of the block's P stays <= 2^8 (so every P does), that P stands -- the same bound the
    // lazy rescale keeps.  Otherwise (the max grew by more, or m_run is still -inf and the
    // sums are inf / NaN) the wave takes the block max, rescales O and l and recomputes P.
    // That is one max per score saved on every block where the max holds.
    auto exp_block = [&](auto mask, int j, float &psum) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask)::value;
        psum = 0.f;
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
            if (MASK && !tile_active(j, kt)) {  // P = 0: the next M phase multiplies it anyway
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                    for (int e = 0; e < 8; ++e) pb[kt][s2][e] = (typename F::elem)0.f;
                continue;
            }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float p = fast_exp2(fmaf(sacc[kt][8 * s2 + e], c, -m_run));
                    psum += p;
                    pb[kt][s2][e] = (typename F::elem)p;
                }
            }
        }
    };
    auto softmax = [&](auto mask, int j) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask)::value;
        if constexpr (MASK) {
            const int j0 = (kb_lo + j) * C::BN;
#pragma unroll
            for (int kt = 0; kt < C::KT; ++kt) {
                if (!tile_active(j, kt)) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key_u = j0 + kt * 32 + acc_row(r, 0);
                    if (key_u >= t_lim || key_u > row_lim) sacc[kt][r] = -INFINITY;
                }
            }
        }
        float psum;
        exp_block(mask, j, psum);
        if (__any(!(psum <= kPsumLimit))) {
            float mloc = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < C::KT; ++kt) {
                if (MASK && !tile_active(j, kt)) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, sacc[kt][r]);
            }
            mloc = max_xor32(mloc) * c;  // c > 0: max(S) * c = max(S * c)
            // Every row has a valid key in the first block, so m_new is finite from there on.
            const float m_new = fmaxf(m_run, mloc);
            const float resc = fast_exp2(m_run - m_new);
            m_run = m_new;
            l_run *= resc;
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt) oacc[dt] *= resc;
            exp_block(mask, j, psum);
        }
        l_run += psum;
    };
    // Block j needs the masked softmax when it crosses the sequence end or, causal, the
    // wave's diagonal; both conditions hold from some block on: masked(j) <=> j >= jm.
    const int jm_t = T / C::BN;
    const int jm_g = causal ? min(jm_t, max(0, (wave_first_row - 62 + C::BN - 1) / C::BN)) : jm_t;
    // Local forms of the first masked block and of this wave's block count.
    const int jm = SPLIT ? min(len, max(0, jm_g - kb_lo)) : jm_g;
    const int wnkb = SPLIT ? min(len, max(0, wave_nkb - kb_lo)) : wave_nkb;

    // One iteration = both phases of block j for this wave, and one workgroup barrier: group A
    // runs M(j), V(j), barrier; group B runs M(j), barrier, V(j).  Between two barriers group A
    // runs M(j + 1) then V(j + 1) while group B runs V(j) then M(j + 1), so each SIMD's two
    // waves meet MFMA phase against softmax phase without a barrier between the phases (a
    // second barrier per iteration, at the phase change, cost ~250 cycles of its ~3 500).
    // Group A issues batch j at the start of M(j) and awaits it at the end of V(j); group B
    // issues batch j + 1 at the start of V(j) and awaits batch j at the end of M(j); the
    // barrier then publishes batch j, which M(j + 1) reads.  No load overwrites a tile a wave
    // may still read: batch j + 1 (K_{j+2}, V_{j+1}) replaces K_j and V_{j-1}, which M(j)
    // read before the barrier.  PV / SC / SM: what this wave computes (the O update of block
    // j - 1, the scores of block j, their softmax: none, unmasked or masked); every wave runs
    // every iteration up to nkb.
    // SPLIT keeps a barrier at every phase change (group B then waits one phase before its
    // first M): with one per iteration its short grids ran ~3 % slower.
    constexpr bool ONE_BARRIER = !SPLIT;
    auto iter = [&](auto pv, auto sc, auto sm, int j) __attribute__((always_inline)) {
        constexpr int SM = decltype(sm)::value;
        if (group == 0) issue(j);
        __builtin_amdgcn_s_setprio(1);
        mphase_t(pv, sc, j);
        __builtin_amdgcn_s_setprio(0);
        if (group == 1) wait_loads();
        if (!ONE_BARRIER || group == 1) lds_barrier();
        if (group == 1) issue(j + 1);
        if constexpr (SM == 1) softmax(std::false_type{}, j);
        if constexpr (SM == 2) softmax(std::true_type{}, j);
        if (group == 0) wait_loads();
        if (!ONE_BARRIER || group == 0) lds_barrier();
    };
    using Y = std::true_type;
    using N = std::false_type;
    using NoSm = std::integral_constant<int, 0>;
    using Plain = std::integral_constant<int, 1>;
    using Masked = std::integral_constant<int, 2>;

    // K_0 before the first phase; batch 0 (K_1, V_0) lands during the first iteration.
    if (len > 0)
        load_tile_dma<D, C::BN, GW>(ktile(0), k + base + int64_t(kb_lo) * C::BN * D, T - kb_lo * C::BN,
                                    SPLIT ? wl : wave, lane);
    wait_loads();
    lds_barrier();
    if (group == 1) {
        issue(0);
        if (!ONE_BARRIER) lds_barrier();  // group B one phase behind group A
    }
    int j = 0;
    if (wnkb > 0) {  // always, unless SPLIT and none of the wave's keys is in its group's half
        if (jm > 0) iter(N{}, Y{}, Plain{}, 0);
        else iter(N{}, Y{}, Masked{}, 0);
        j = 1;
        for (; j < min(jm, wnkb); ++j) iter(Y{}, Y{}, Plain{}, j);
        for (; j < wnkb; ++j) iter(Y{}, Y{}, Masked{}, j);
        iter(Y{}, N{}, NoSm{}, j);  // j == wnkb: the last O update
        ++j;
    }
    for (; j <= jlast; ++j) iter(N{}, N{}, NoSm{}, j);  // keys past this wave's diagonal
    if (!ONE_BARRIER && group == 0) lds_barrier();  // matches group B's extra barrier

    if constexpr (SPLIT) {
        // Group B's lane state lands at mb[(wl NR + i) 64 + lane]; group A's wave wl merges it:
        // m = max(mA, mB) (log2 units, times c), O = OA 2^(mA - m) + OB 2^(mB - m), l likewise.
        // Group A holds key 0 of every row, so mA is finite; a wave of B without keys keeps
        // m = -inf, weight 0.
        constexpr int NR = C::DT * 16 + 2;
        static_assert(4 * NR * kWave * 4 <= 2 * C::LDS_BYTES, "merge buffer");
        float *mb = reinterpret_cast<float *>(smem_all);
        lds_barrier();  // every wave is done with the tiles
        if (group == 1) {
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) mb[(wl * NR + dt * 16 + r) * kWave + lane] = oacc[dt][r];
            mb[(wl * NR + NR - 2) * kWave + lane] = m_run;
            mb[(wl * NR + NR - 1) * kWave + lane] = l_run;
        }
        lds_barrier();
        if (group == 1) return;
        const float m1 = mb[(wl * NR + NR - 2) * kWave + lane];
        const float l1 = mb[(wl * NR + NR - 1) * kWave + lane];
        const float m = fmaxf(m_run, m1);
        const float a0 = fast_exp2(m_run - m), a1 = fast_exp2(m1 - m);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                oacc[dt][r] = oacc[dt][r] * a0 + mb[(wl * NR + dt * 16 + r) * kWave + lane] * a1;
        l_run = l_run * a0 + l1 * a1;
        m_run = m;
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv_l = 1.f / l_tot;
    if (row < T) {
        uint16_t *orow = o + base + int64_t(row) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                u16x4 x;
#pragma unroll
                for (int t = 0; t < 4; ++t) x[t] = F::bits(oacc[dt][4 * g + t] * inv_l);
                *reinterpret_cast<u16x4 *>(orow + dt * 32 + 8 * g + 4 * half) = x;
            }
        }
        if (lse != nullptr && half == 0) lse[int64_t(bh) * T + row] = (m_run + __log2f(l_tot)) * kLn2;
    }
}

template <int D, typename F>
hipError_t fwd_bf16_pp(const void *q, const void *k, const void *v, void *o, float *lse, const AttnShape &s,
                       hipStream_t stream) {
    using C = FwdPpCfg<D>;
    const int64_t nqb = (s.T + C::BM - 1) / C::BM;
    const int64_t blocks = nqb * s.bh();
    if (!grid_fits(blocks, C::NW * kWave) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const float c = kLog2e / sqrtf(float(s.scale_dim()));
    // A causal grid of no more whole workgroups than CUs (one each) runs as long as its longest
    // query block: then 128-row workgroups with the key range halved between the groups.
    const int cus = device_cus(stream);
    const bool split = s.causal && cus > 0 && blocks <= kPpSplitWorkgroupsPerCu * int64_t(cus);
    const int64_t grid = split ? (s.T + 127) / 128 * s.bh() : blocks;
    if (!grid_fits(grid, C::NW * kWave)) return hipErrorInvalidValue;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(unsigned(grid)), dim3(C::NW * kWave), 0, stream,
                           static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                           static_cast<const uint16_t *>(v), static_cast<uint16_t *>(o), lse, int(s.T), int(s.bh()),
                           int(s.causal), c);
    };
    if (split) launch(fwd_bf16_pp_kernel<D, F, true>);
    else launch(fwd_bf16_pp_kernel<D, F, false>);
    return hipGetLastError();
}

template <int D, typename F>
hipError_t fwd_bf16(const void *q, const void *k, const void *v, void *o, float *lse, const AttnShape &s,
                    hipStream_t stream) {
    using C = FwdBf16Cfg<D>;
    const int64_t nqb = (s.T + C::BM - 1) / C::BM;
    const int64_t blocks = nqb * s.bh();
    if (!grid_fits(blocks, C::NW * kWave) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    const float c = kLog2e / sqrtf(float(s.scale_dim()));
    // A causal grid of no more whole workgroups than the chip holds at once (two per CU) runs
    // as long as its longest query block: then 64-row workgroups with halved key ranges.
    const int cus = device_cus(stream);
    const bool split = s.causal && cus > 0 && blocks <= 2 * int64_t(cus);
    const int64_t grid = split ? (s.T + 63) / 64 * s.bh() : blocks;
    if (!grid_fits(grid, C::NW * kWave)) return hipErrorInvalidValue;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(unsigned(grid)), dim3(C::NW * kWave), 0, stream,
                           static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                           static_cast<const uint16_t *>(v), static_cast<uint16_t *>(o), lse, int(s.T), int(s.bh()),
                           int(s.causal), c);
    };
    if (split) launch(fwd_bf16_mfma_kernel<D, F, true>);
    else launch(fwd_bf16_mfma_kernel<D, F, false>);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bf16_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                           const AttnShape &s, hipStream_t stream) {
    switch (s.d) {
        case 32: return fwd_bf16<32, Bf16Fmt>(q, k, v, o, lse, s, stream);
        case 64: return fwd_bf16<64, Bf16Fmt>(q, k, v, o, lse, s, stream);
        case 128: return fwd_bf16_pp<128, Bf16Fmt>(q, k, v, o, lse, s, stream);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_f16_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                          const AttnShape &s, hipStream_t stream) {
    switch (s.d) {
        case 32: return fwd_bf16<32, F16Fmt>(q, k, v, o, lse, s, stream);
        case 64: return fwd_bf16<64, F16Fmt>(q, k, v, o, lse, s, stream);
        case 128: return fwd_bf16_pp<128, F16Fmt>(q, k, v, o, lse, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
