// fp32 flash-attention backward on fp32 MFMA (gfx950).
//
// Replaces the reference backward kernel flashAttentionBackward<float>
// (flash_attention.cu:226-326) with the same per-element math -- P = exp(S - LSE)
// (:297-298), dS = P (dP - delta) (:299), dQ = dS K / sqrt(d) (:311) -- but correct dK and
// dV (dK = dS^T Q / sqrt(d), dV = P^T dO; the reference's :312-313 sum the wrong index),
// a causal mask, no zero-padded keys, and no atomics on dK / dV.
//
// Work decomposition ("key-block major")
//   * one workgroup = 4 waves owns BN = 64 keys of one (batch, head) and walks query blocks
//     of BM = 64 rows (causal: only rows >= its first key).  The waves form 2 key slices x
//     2 row slices: wave (ks, rs) handles keys 32ks..32ks+31 against rows 32rs..32rs+31 of
//     each query block and accumulates dK^T and dV^T of its keys in registers; the two row
//     slices' partial sums are added through LDS once at the end, so dK / dV are written
//     exactly once, without atomics.  With 64-key blocks the causal diagonal leaves one
//     wave in four idle for one block per workgroup, and there are twice as many, half as
//     long workgroups as with 128-key blocks, which balances the causal grid.
//   * Q, dO, LSE and delta of a query block go straight from global memory to LDS
//     (global_load_lds into rows padded by one 16-byte chunk, no staging registers); the
//     next block's loads are issued once every wave is past the block's S/dP/dV/dK phase
//     and land during the dQ phase.
//   * per wave and query block, with v_mfma_f32_32x32x2f32:
//       S  = Q K^T      (A = Q rows from LDS, B = K^T from the LDS K block)
//       dP = dO V^T     (A = dO rows from LDS, B = V^T held in registers)
//     In these accumulators each lane holds ONE key (its column) and 16 query rows, so
//       P  = exp2(S log2(e)/sqrt(d) - LSE log2(e)),  dS = P (dP - delta)
//     are elementwise, and P / dS are directly the B operands of
//       dV^T += dO^T P  and  dK^T += Q^T dS     (A = dO / Q columns from LDS).
//   * dQ needs dS with rows on lanes: each wave writes its dS tile to LDS, then every wave
//     computes a 32-row x (d/2)-column tile of dQ = dS K over the block's 64 keys (d = 32:
//     two waves, 32 x 32 each) and adds it with fp32 atomics into dq (pre-zeroed by the
//     preprocess kernel), one iteration later (see flush_dq).
//   * dS mode (DS, d >= 64, when the workspace holds every 64 x 64 dS tile of the mask): no
//     dQ work and no atomics here.  Each wave copies a quarter of the block's dS from LDS to
//     the workspace instead, in the order of the A operands of dQ = dS K, and
//     bwd_f32_dq_ds_kernel then computes dQ query-major from those tiles, each element summed
//     by one lane in key-block order: deterministic, and the atomics' write traffic (about
//     ten times the dQ bytes) becomes one pass of dS stores and loads.
//
// Which kernels run: this 64-key kernel for causal masks with atomic dQ and d >= 64 (where
// its balance and smaller diagonal win); the 128-key kernel of attn_bwd_k128.hip, with half
// the dQ atomics, without a mask and at d = 32.  The deterministic policy takes no atomics:
// up to 8 key blocks of 128 the 128-key kernel stores per-key-block dQ partials that the
// reduction kernel here sums in a fixed order; beyond that it computes dK / dV only and the
// query-major kernel of attn_bwd_dq_f32.hip computes dQ, each element summed by one lane in a
// fixed order (two fewer planes of traffic per key block, two more matmuls).
#include "attn_launch.h"
#include "attn_mfma_common.h"

#include <math.h>

#include <algorithm>

namespace ctattn {
namespace {

// dQ of the fp32 backward: fp32 atomics (AUTO); per-128-key-block partials summed in a fixed
// order (DETERMINISTIC, up to kMaxPartialBlocks key blocks); the query-major dQ kernel
// (DETERMINISTIC, longer sequences).
enum class DqMode { Atomic, Partial, Separate };

template <int D>
struct BwdCfg {
    static constexpr int NW = 4;              // waves per workgroup
    static constexpr int BN = 64;             // keys per workgroup
    static constexpr int BM = 64;             // query rows per iteration
    static constexpr int KS = D + 4;          // LDS row stride (floats) of K, Q and dO
    static constexpr int SS = BN + 4;         // LDS row stride of dS
    static constexpr int DT = D / 32;         // 32-wide d tiles of dK^T / dV^T
    static constexpr int C4 = D / 4;          // 16-byte chunks per row of data
    static constexpr int C4P = C4 + 1;        // ... per LDS row, including the pad chunk
    static constexpr int TILE = BM * KS;      // floats per padded Q (or dO) block
    static constexpr int CHUNKS = BM * C4P;   // 16-byte chunks per padded block
    static constexpr int INSTR = (CHUNKS + NW * kWave - 1) / (NW * kWave);  // direct loads per lane per tensor
    static constexpr int KF4 = BN * C4 / (NW * kWave);    // float4 per thread for the K block
    // dQ of a 64 x D block: d >= 64 -> every wave a 32 x D/2 tile (row slice wave >> 1,
    // column half wave & 1); d = 32 -> waves 0, 1 a 32 x 32 tile each.
    static constexpr int DQ_WAVES = D >= 64 ? 4 : 2;
    static constexpr int DQ_COLS = D >= 64 ? D / 2 : 32;
    static constexpr int DQ_T = DQ_COLS / 32;  // 32x32 dQ tiles per wave
    static_assert(D == 32 || D == 64 || D == 128, "MFMA backward supports d in {32, 64, 128}");
    static_assert(KF4 * NW * kWave == BN * C4, "block load split");
};

#define CTATTN_LDS(p) ((__attribute__((address_space(3))) void *)(p))

// dS tiles of the dS mode: one 64 x 64 tile (16 KB) per (query block, key block) pair of 64,
// causal: key block <= query block, packed per head in row-major (triangle) order.  A tile is
// four 32 x 32 sub-tiles, sub-tile (row slice rs, key slice ks) at 1024 (2 rs + ks); in a
// sub-tile, float4 m (m = 0..3) of lane (col, half) holds dS[row 32 rs + col][key 32 ks + 8 m
// + 4 half + t], t = 0..3, at floats 4 (64 m + lane) .. + 3: the A operands of four MFMA steps
// of dQ = dS K, so one 16-byte store per lane writes (and one load reads) 1 KB contiguously.
constexpr int kDsTileFloats = 64 * 64;
__host__ __device__ inline int64_t f32_ds_tiles_per_head(int64_t T, bool causal) {
    const int64_t n = (T + 63) / 64;
    return causal ? n * (n + 1) / 2 : n * n;
}
__device__ inline int64_t f32_ds_tile(int bh, int qb, int kb, int nqb, int causal, int64_t tph) {
    const int64_t t = causal ? int64_t(qb) * (qb + 1) / 2 + kb : int64_t(qb) * nqb + kb;
    return (int64_t(bh) * tph + t) * kDsTileFloats;
}

// Waves per SIMD the kernel is compiled for: two for d <= 64 (<= 256 VGPRs); d = 128 needs
// more registers than that and runs one wave per SIMD.
template <int D> struct BwdF32Occupancy { static constexpr int waves = D <= 64 ? 2 : 1; };

// S, dP, P, dS and the dV^T / dK^T updates of wave (ks, rs) for one query block, then its
// dS tile -> LDS.  rb = 32 rs is the wave's first row in the block, r0w its global index.
// MASK selects the diagonal / sequence-end variant (per-element causal and bounds checks).
template <int D, bool MASK>
__device__ __forceinline__ void bwd_wave_block(floatx16 (&dk_acc)[D / 32], floatx16 (&dv_acc)[D / 32],
                                               const float (&vT)[D / 2], const float *q_lds,
                                               const float *do_lds, const float *k_lds,
                                               const float *lse_lds, const float *dl_lds,
                                               float *ds_lds, int rb, int r0w, int kb_local, int key,
                                               int T, int causal, float kscale, int col, int half) {
    using C = BwdCfg<D>;
    floatx16 s = zero16(), dp = zero16();
    const int qrow = rb + col;  // A-operand row of this lane
    // Q, dO and K reads (three ds_read_b128 per 8 MFMAs) double-buffered: group m + 1 is
    // issued before the MFMAs of group m.
    {
        floatx4 qa[2], da[2], kb4[2];
        auto rd = [&](int m, int b) __attribute__((always_inline)) {
            qa[b] = *reinterpret_cast<const floatx4 *>(&q_lds[qrow * C::KS + 8 * m + 4 * half]);
            da[b] = *reinterpret_cast<const floatx4 *>(&do_lds[qrow * C::KS + 8 * m + 4 * half]);
            kb4[b] = *reinterpret_cast<const floatx4 *>(&k_lds[(kb_local + col) * C::KS + 8 * m + 4 * half]);
        };
        rd(0, 0);
#pragma unroll
        for (int m = 0; m < D / 8; ++m) {
            if (m + 1 < D / 8) rd(m + 1, (m + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            const int b = m & 1;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s = mfma32x32x2(qa[b][t], kb4[b][t], s);
                dp = mfma32x32x2(da[b][t], vT[4 * m + t], dp);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const floatx4 l4 = *reinterpret_cast<const floatx4 *>(&lse_lds[rb + 8 * g + 4 * half]);
        const floatx4 d4 = *reinterpret_cast<const floatx4 *>(&dl_lds[rb + 8 * g + 4 * half]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int r = 4 * g + t;
            float p = fast_exp2(fmaf(s[r], kscale, l4[t] * -kLog2e));
            if (MASK) {
                const int row = r0w + acc_row(r, half);
                p = (row >= T || key >= T || (causal && key > row)) ? 0.f : p;
            }
            s[r] = p;
            dp[r] = p * (dp[r] - d4[t]);
        }
    }
    // dV^T += dO^T P,  dK^T += Q^T dS   (contraction over the wave's 32 rows).  One
    // ds_read_b32 per MFMA, through a ring of 8 issued 6 reads ahead of their MFMAs.
    {
        constexpr int NR = 16 * C::DT * 2;
        constexpr int R = 8, AHEAD = 6;
        auto rd = [&](int i) __attribute__((always_inline)) {
            const int st = i / (2 * C::DT), dt = (i / 2) % C::DT;
            const int off = (rb + kstep_index(st, half)) * C::KS + dt * 32 + col;
            return (i & 1) ? q_lds[off] : do_lds[off];
        };
        float ring[R];
#pragma unroll
        for (int i = 0; i < AHEAD; ++i) ring[i % R] = rd(i);
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            if (i + AHEAD < NR) ring[(i + AHEAD) % R] = rd(i + AHEAD);
            __builtin_amdgcn_sched_barrier(0);
            const int st = i / (2 * C::DT), dt = (i / 2) % C::DT;
            if (i & 1) dk_acc[dt] = mfma32x32x2(ring[i % R], dp[st], dk_acc[dt]);
            else dv_acc[dt] = mfma32x32x2(ring[i % R], s[st], dv_acc[dt]);
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) ds_lds[(rb + acc_row(r, half)) * C::SS + kb_local + col] = dp[r];
}

template <int D, bool SPLIT, bool DS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BwdF32Occupancy<D>::waves,
                                                                     BwdF32Occupancy<D>::waves))) void bwd_f32_mfma_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ delta, float *__restrict__ dq, float *__restrict__ dk,
    float *__restrict__ dv, float *__restrict__ ds_ws, int T, int BH, int causal, float kscale,
    float inv_sqrt_d) {
    using C = BwdCfg<D>;
    constexpr int split = SPLIT ? 1 : 0;
    __shared__ __attribute__((aligned(16))) float qdo_lds[2 * C::TILE];  // Q then dO, [BM][KS] each
    float *q_lds = qdo_lds;
    float *do_lds = qdo_lds + C::TILE;
    __shared__ __attribute__((aligned(16))) float k_lds[C::BN * C::KS];
    __shared__ __attribute__((aligned(16))) float ds_lds[C::BM * C::SS];
    __shared__ __attribute__((aligned(16))) float lse_lds[C::BM];  // natural-log LSE
    __shared__ __attribute__((aligned(16))) float dl_lds[C::BM];   // delta

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int ks = wave & 1, rs = wave >> 1;

    // split: key block kb's query blocks are shared by workgroups (kb, part 0) and (kb, part 1).
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int kb = (id / BH) >> split;  // causal: key block 0 has the most query blocks -> launched first
    const int part = (id / BH) & split;
    const int k0 = kb * C::BN;
    const int64_t base = int64_t(bh) * T * D;
    const int64_t rbase = int64_t(bh) * T;
    const int kw0 = k0 + 32 * ks;
    const int key = kw0 + col;  // key owned by this lane in S / dP / dK^T / dV^T

    // K block -> LDS (B operand of S = Q K^T and of dQ = dS K), rows past T zero.
#pragma unroll
    for (int i = 0; i < C::KF4; ++i) {
        const int f = tid + i * C::NW * kWave;
        const int r = f / C::C4;
        const int c4 = f - r * C::C4;
        floatx4 x = {0.f, 0.f, 0.f, 0.f};
        if (k0 + r < T) x = *reinterpret_cast<const floatx4 *>(k + base + int64_t(k0 + r) * D + 4 * c4);
        *reinterpret_cast<floatx4 *>(&k_lds[r * C::KS + 4 * c4]) = x;
    }
    // V^T as the B operand of dP = dO V^T, held in registers for the whole kernel:
    // lane (col = key, half) holds V[key][kstep_index(s, half)].
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

    const int nqb = (T + C::BM - 1) / C::BM;
    const int qb_first = causal ? k0 / C::BM : 0;
    const int qb_mid = qb_first + (nqb - qb_first + 1) / 2;
    const int qb_begin = split && part ? qb_mid : qb_first;
    const int qb_end = split && !part ? qb_mid : nqb;

    // Global -> LDS for one query block: lane writes LDS chunk P = (wave * INSTR + i) * 64 +
    // lane of the padded block, i.e. row P / C4P, chunk P % C4P; the pad chunk (C4) re-reads
    // chunk 0 of the row and is never used.  Rows past T re-read row T - 1 (their P is
    // masked to 0).  Waves 0 / 1 also fetch the block's LSE / delta (one dword per lane).
    auto issue = [&](int r0) {
#pragma unroll
        for (int i = 0; i < C::INSTR; ++i) {
            const int P = (wave * C::INSTR + i) * kWave + lane;
            if (C::CHUNKS % (C::NW * kWave) == 0 || P < C::CHUNKS) {
                const int r = P / C::C4P;
                const int c = P - r * C::C4P;
                const int64_t goff = base + int64_t(min(r0 + r, T - 1)) * D + 4 * (c < C::C4 ? c : 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(q + goff),
                                                 CTATTN_LDS(&q_lds[(wave * C::INSTR + i) * 4 * kWave]), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(dout + goff),
                                                 CTATTN_LDS(&do_lds[(wave * C::INSTR + i) * 4 * kWave]), 16, 0, 0);
            }
        }
        if (wave < 2) {
            const float *src = wave == 0 ? lse : delta;
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(src + rbase + min(r0 + lane, T - 1)),
                                             CTATTN_LDS(wave == 0 ? lse_lds : dl_lds), 4, 0, 0);
        }
    };

    // dQ tile of this wave: rows 32 * qrs .. of the block, columns dq_col0 ..
    const bool dq_wave = wave < C::DQ_WAVES;
    const int qrs = D >= 64 ? (wave >> 1) : wave;
    const int dq_col0 = D >= 64 ? (wave & 1) * C::DQ_COLS : 0;

    // A block's dQ tile is added to global memory one iteration late, right after the next
    // block's first barrier: the wait for the next block's loads at the top of each
    // iteration (vmcnt counts both) then finds those atomics long completed instead of
    // stalling on atomics issued just before it.
    floatx16 dq_pend[C::DQ_T];
    int pend_rq0 = -1;  // first row of the pending tile, -1 if none
    auto flush_dq = [&]() {
        // Lane (col, half), register r: row pend_rq0 + acc_row(r, half), column dq_col0 + 32 j + col.
        const int row0 = pend_rq0 + 4 * half;
        float *p0 = dq + base + int64_t(row0) * D + dq_col0 + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int dr = acc_row(r, 0);  // row offset from row0, a compile-time constant
            if (row0 + dr >= T) continue;
#pragma unroll
            for (int j = 0; j < C::DQ_T; ++j) unsafeAtomicAdd(p0 + dr * D + 32 * j, dq_pend[j][r] * inv_sqrt_d);
        }
    };

    // DS: this wave's quarter of the previous block's dS (row slice wave >> 1, key slice
    // wave & 1), read from LDS before the barrier that lets the next block overwrite it and
    // stored after that barrier, so the loop-top wait never waits on fresh stores.
    const int64_t ds_tph = f32_ds_tiles_per_head(T, causal != 0);
    floatx4 ds_pend[4];
    float *ds_dst = nullptr;  // the pending sub-tile's place in the workspace, null if none
    auto flush_ds = [&]() {
#pragma unroll
        for (int m = 0; m < 4; ++m) *reinterpret_cast<floatx4 *>(ds_dst + (m * kWave + lane) * 4) = ds_pend[m];
    };

    if (qb_begin < qb_end) issue(qb_begin * C::BM);
    for (int qb = qb_begin; qb < qb_end; ++qb) {
        const int r0 = qb * C::BM;
        // The block's loads have landed (vmcnt = 0) and, after the barrier, every wave's are
        // visible; every wave is also done reading the previous block's dS (DS: its LDS reads
        // of that dS have returned, lgkmcnt = 0).
        __builtin_amdgcn_s_waitcnt(DS ? 0x070 : 0xF70);
        __syncthreads();
        if constexpr (DS) {
            if (ds_dst != nullptr) flush_ds();
        } else {
            if (pend_rq0 >= 0) flush_dq();
        }

        const int r0w = r0 + 32 * rs;
        const bool wave_active = kw0 < T && r0w < T && (!causal || kw0 <= r0w + 31);
        if (wave_active) {
            const bool masked = (r0w + 32 > T) || (kw0 + 32 > T) || (causal && kw0 + 31 > r0w);
            if (masked)
                bwd_wave_block<D, true>(dk_acc, dv_acc, vT, q_lds, do_lds, k_lds, lse_lds, dl_lds, ds_lds,
                                        32 * rs, r0w, 32 * ks, key, T, causal, kscale, col, half);
            else
                bwd_wave_block<D, false>(dk_acc, dv_acc, vT, q_lds, do_lds, k_lds, lse_lds, dl_lds, ds_lds,
                                         32 * rs, r0w, 32 * ks, key, T, causal, kscale, col, half);
        }
        __syncthreads();  // dS of every wave visible; Q / dO / LSE / delta no longer read
        if (qb + 1 < qb_end) issue(r0 + C::BM);

        if constexpr (DS) {
            const int srs = wave >> 1, sks = wave & 1;
            const int rq0 = r0 + 32 * srs, kw2 = k0 + 32 * sks;
            ds_dst = nullptr;
            if (kw2 < T && rq0 < T && (!causal || kw2 <= rq0 + 31)) {
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    ds_pend[m] = *reinterpret_cast<const floatx4 *>(
                        &ds_lds[(32 * srs + col) * C::SS + 32 * sks + 8 * m + 4 * half]);
                ds_dst = ds_ws + f32_ds_tile(bh, qb, kb, nqb, causal, ds_tph) + (2 * srs + sks) * 1024;
            }
        } else if (dq_wave) {
            // dQ[r0 + 32 qrs .. +31][dq_col0 ..] = sum over the block's active keys of dS K.
#pragma unroll
            for (int j = 0; j < C::DQ_T; ++j) dq_pend[j] = zero16();
            const int rq0 = r0 + 32 * qrs;
#pragma unroll
            for (int ks2 = 0; ks2 < 2; ++ks2) {
                const int kw2 = k0 + 32 * ks2;
                if (!(kw2 < T && rq0 < T && (!causal || kw2 <= rq0 + 31))) continue;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int kl = 32 * ks2 + 8 * m + 4 * half;  // local key of step t: kl + t
                    const floatx4 a = *reinterpret_cast<const floatx4 *>(&ds_lds[(32 * qrs + col) * C::SS + kl]);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
#pragma unroll
                        for (int j = 0; j < C::DQ_T; ++j)
                            dq_pend[j] = mfma32x32x2(a[t], k_lds[(kl + t) * C::KS + dq_col0 + 32 * j + col], dq_pend[j]);
                    }
                }
            }
            pend_rq0 = rq0;
        }
    }
    if constexpr (DS) {
        if (ds_dst != nullptr) flush_ds();
    } else {
        if (pend_rq0 >= 0) flush_dq();
    }

    // dK^T / dV^T of the two row slices: rs = 1 hands its sums to rs = 0 through LDS (the Q /
    // dO blocks are free: no load is in flight after the last block, and every wave has
    // passed the last block's second barrier).  Lane (key, half) holds d = dt*32 + acc_row(r, half).
    float *red = qdo_lds;  // 2 (ks) x DT x 2 (dk, dv) x 16 x 64 floats
    static_assert(2 * C::DT * 2 * 16 * kWave <= 2 * C::TILE, "reduction buffer");
    __syncthreads();
    if (rs == 1) {
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                red[(((ks * C::DT + dt) * 2 + 0) * 16 + r) * kWave + lane] = dk_acc[dt][r];
                red[(((ks * C::DT + dt) * 2 + 1) * 16 + r) * kWave + lane] = dv_acc[dt][r];
            }
    }
    __syncthreads();
    // Lane (key, half), register r of tile dt: the final dK (g = 0) or dV (g = 1) value of
    // d = dt * 32 + 8 * (r / 4) + 4 * half + r % 4, row-slice sums included.
    auto final_val = [&](int which, int dt, int r) __attribute__((always_inline)) {
        const float other = red[(((ks * C::DT + dt) * 2 + which) * 16 + r) * kWave + lane];
        return which == 0 ? (dk_acc[dt][r] + other) * inv_sqrt_d : dv_acc[dt][r] + other;
    };
    if constexpr (SPLIT) {
        // Two workgroups add to each element (two addends: the same sum in either order).  The
        // lane-per-key layout would scatter every atomic instruction over 64 rows, so each
        // tensor goes through LDS (k_lds, [key][KS]) and is added with lanes along d.
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            if (rs == 0) {
#pragma unroll
                for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        floatx4 x;
#pragma unroll
                        for (int t = 0; t < 4; ++t) x[t] = final_val(which, dt, 4 * g + t);
                        *reinterpret_cast<floatx4 *>(&k_lds[(32 * ks + col) * C::KS + dt * 32 + 8 * g + 4 * half]) = x;
                    }
            }
            __syncthreads();
            float *dst = (which == 0 ? dk : dv) + base + int64_t(k0) * D;
            for (int e = tid; e < C::BN * D; e += C::NW * kWave) {
                const int kr = e / D, c = e - (e / D) * D;
                if (k0 + kr < T) unsafeAtomicAdd(dst + int64_t(kr) * D + c, k_lds[kr * C::KS + c]);
            }
            __syncthreads();
        }
        return;
    }
    if (rs == 0 && key < T) {
        float *dkr = dk + base + int64_t(key) * D;
        float *dvr = dv + base + int64_t(key) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                floatx4 xk, xv;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    xk[t] = final_val(0, dt, 4 * g + t);
                    xv[t] = final_val(1, dt, 4 * g + t);
                }
                *reinterpret_cast<floatx4 *>(dkr + dt * 32 + 8 * g + 4 * half) = xk;
                *reinterpret_cast<floatx4 *>(dvr + dt * 32 + 8 * g + 4 * half) = xv;
            }
        }
    }
}

// delta[row] = sum_c dO[row][c] * O[row][c] (flash_attention.cu:269-273); also zeroes the
// dq row when dQ is accumulated with atomics, and the dk / dv rows when the key blocks are
// split (dk_zero / dv_zero non-null).  D / 4 lanes per row, one 16-byte load of O and
// of dO (and one 16-byte store of zeros) each.
template <int D, bool ZERO_DQ>
__global__ __launch_bounds__(256) void bwd_preprocess_f32_kernel(const float *__restrict__ o,
                                                                const float *__restrict__ dout,
                                                                float *__restrict__ delta,
                                                                float *__restrict__ dq,
                                                                float *__restrict__ dk_zero,
                                                                float *__restrict__ dv_zero,
                                                                int64_t rows) {
    constexpr int LPR = D / 4;  // lanes per row
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    // Grid-stride; the block size and the stride are multiples of LPR, so the LPR lanes of a
    // row enter and leave the loop together (group_sum stays inside the group).
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t / LPR < rows; t += stride) {
        const int64_t row = t / LPR;
        const int c4 = int(t % LPR);
        float s = 0.f;
        if (row < rows) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(o + row * D + 4 * c4);
            const floatx4 b = *reinterpret_cast<const floatx4 *>(dout + row * D + 4 * c4);
            s = (a[0] * b[0] + a[1] * b[1]) + (a[2] * b[2] + a[3] * b[3]);
            if (ZERO_DQ) *reinterpret_cast<floatx4 *>(dq + row * D + 4 * c4) = floatx4{0.f, 0.f, 0.f, 0.f};
            if (dk_zero != nullptr) {  // split key blocks: dK / dV are sums of atomic adds
                *reinterpret_cast<floatx4 *>(dk_zero + row * D + 4 * c4) = floatx4{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<floatx4 *>(dv_zero + row * D + 4 * c4) = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
        s = group_sum<LPR>(s);
        if (row < rows && c4 == 0) delta[row] = s;
    }
}

// dq[bh][row][:] = sum over key blocks kb <= (causal ? row / BN : nkb - 1) of dq_part[kb][bh][row][:],
// summed in increasing kb order (deterministic).  One thread per float4.
template <int D>
__global__ __launch_bounds__(256) void dq_reduce_kernel(const float *__restrict__ dq_part,
                                                       float *__restrict__ dq, int T, int BH,
                                                       int causal, int nkb, int bn) {
    const int64_t total = int64_t(BH) * T * (D / 4);
    const int64_t plane = int64_t(BH) * T * D;
    for (int64_t f = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; f < total; f += int64_t(gridDim.x) * blockDim.x) {
        const int64_t row_g = f / (D / 4);  // bh * T + row
        const int row = int(row_g % T);
        const int last = causal ? row / bn : nkb - 1;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int kb = 0; kb <= last; ++kb)
            acc += *reinterpret_cast<const floatx4 *>(dq_part + kb * plane + 4 * f);
        *reinterpret_cast<floatx4 *>(dq + 4 * f) = acc;
    }
}

// dQ = dS K / sqrt(d) from the dS tiles of the dS mode (d >= 64), query-major: a workgroup
// owns 64 rows of one head and walks its key blocks (causal: up to the diagonal); causal
// workgroups run longest first.  Four waves:
//   KH = 1 (d = 128): row slice w >> 1, column half w & 1, every key block in order;
//   KH = 2 (d = 64):  row slice w >> 1, all d columns, key blocks of parity w & 1 (its own
//     double-buffered K tiles), so the longest workgroup takes half as many steps and each
//     dS sub-tile is loaded once; the odd half hands its sums to the even half through LDS
//     at the end.
// Each dQ element is thus summed in a fixed order and stored once.  K blocks go global ->
// LDS directly (padded rows; rows past T re-read row T - 1, whose dS is 0); dS goes global ->
// registers a step ahead, one 16-byte load per lane per four MFMA steps.
template <int D, int KH>
__global__ __launch_bounds__(256) void bwd_f32_dq_ds_kernel(const float *__restrict__ k,
                                                           const float *__restrict__ ds_ws,
                                                           float *__restrict__ dq, int T, int BH, int causal,
                                                           float inv_sqrt_d) {
    using C = BwdCfg<D>;
    static_assert(KH == 1 || KH == 2, "key halves");
    constexpr int DT = KH == 1 ? D / 64 : D / 32;  // 32-wide dQ tiles per wave
    constexpr int LW = C::NW / KH;                 // waves loading one K tile
    constexpr int KI = (C::CHUNKS + LW * kWave - 1) / (LW * kWave);  // its loads per lane
    __shared__ __attribute__((aligned(16))) float k_lds[KH][2][C::TILE];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int qrs = wave >> 1;
    const int kh = KH == 2 ? (wave & 1) : 0;
    const int lw = KH == 2 ? qrs : wave;  // index among the waves loading this K tile
    const int dq_col0 = KH == 1 ? (wave & 1) * (D / 2) : 0;

    const int id = blockIdx.x;
    const int bh = id % BH;
    const int nqb = (T + C::BM - 1) / C::BM;
    const int qb = causal ? nqb - 1 - id / BH : id / BH;
    const int rq0 = qb * C::BM + 32 * qrs;  // first row of this wave's tile
    const int nkb = causal ? qb + 1 : nqb;
    const int nit = (nkb + KH - 1) / KH;
    const int64_t base = int64_t(bh) * T * D;
    const int64_t tph = f32_ds_tiles_per_head(T, causal != 0);

    // Key block kb -> k_lds[kh][buf]: lane writes chunk P = (lw * KI + i) * 64 + lane of the
    // padded block (row P / C4P, chunk P % C4P; the pad chunk re-reads chunk 0).
    auto issue_k = [&](int kb, int buf) {
        const int j0 = kb * C::BN;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int P = (lw * KI + i) * kWave + lane;
            if (C::CHUNKS % (LW * kWave) == 0 || P < C::CHUNKS) {
                const int r = P / C::C4P;
                const int c = P - r * C::C4P;
                const int64_t goff = base + int64_t(min(j0 + r, T - 1)) * D + 4 * (c < C::C4 ? c : 0);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(k + goff),
                                                 CTATTN_LDS(&k_lds[kh][buf][(lw * KI + i) * 4 * kWave]), 16, 0, 0);
            }
        }
    };
    // Sub-tile (qrs, ks2) of key block kb holds dS only where the key-major kernel stored it.
    auto active = [&](int kb, int ks2) {
        const int kw2 = kb * C::BN + 32 * ks2;
        return kb < nkb && kw2 < T && rq0 < T && (!causal || kw2 <= rq0 + 31);
    };
    auto load_ds = [&](int kb, floatx4 (&a)[2][4]) {
        const float *t = ds_ws + f32_ds_tile(bh, qb, kb, nqb, causal, tph) + 2 * qrs * 1024;
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ++ks2) {
            if (!active(kb, ks2)) continue;
#pragma unroll
            for (int m = 0; m < 4; ++m)
                a[ks2][m] = *reinterpret_cast<const floatx4 *>(t + ks2 * 1024 + (m * kWave + lane) * 4);
        }
    };

    floatx16 acc[DT];
#pragma unroll
    for (int j = 0; j < DT; ++j) acc[j] = zero16();
    // Step it: this wave's key block kb = KH it + kh.  Wait for its K and dS, prefetch the
    // next, then the MFMAs.
    auto step = [&](int it, floatx4 (&cur)[2][4], floatx4 (&nxt)[2][4]) __attribute__((always_inline)) {
        const int buf = it & 1;
        const int kb = KH * it + kh;
        __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt = 0: this block's K (to LDS) and dS (to registers)
        __syncthreads();                    // every lane's K visible; every wave done with buf ^ 1
        if (kb + KH < nkb) {
            issue_k(kb + KH, buf ^ 1);
            load_ds(kb + KH, nxt);
        }
        const float *kt = k_lds[kh][buf];
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ++ks2) {
            if (!active(kb, ks2)) continue;
            // MFMA i = (4 m + t) DT + j: A = dS of key 32 ks2 + 8 m + 4 half + t, B = K of that
            // key, column dq_col0 + 32 j + col.  The B reads (one ds_read_b32 each) go through
            // a ring of 8 issued 6 MFMAs ahead, so no MFMA waits on its own read.
            constexpr int NV = 16 * DT, R = 8, AHEAD = 6;
            auto bread = [&](int i) __attribute__((always_inline)) {
                const int st = i / DT, j = i % DT;
                return kt[(32 * ks2 + 8 * (st / 4) + 4 * half + st % 4) * C::KS + dq_col0 + 32 * j + col];
            };
            float ring[R];
#pragma unroll
            for (int i = 0; i < AHEAD; ++i) ring[i % R] = bread(i);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                if (i + AHEAD < NV) ring[(i + AHEAD) % R] = bread(i + AHEAD);
                __builtin_amdgcn_sched_barrier(0);
                const int st = i / DT, j = i % DT;
                acc[j] = mfma32x32x2(cur[ks2][st / 4][st % 4], ring[i % R], acc[j]);
            }
        }
    };
    floatx4 a0[2][4], a1[2][4];
    if (kh < nkb) {
        issue_k(kh, 0);
        load_ds(kh, a0);
    }
    for (int it = 0; it < nit; it += 2) {
        step(it, a0, a1);
        if (it + 1 < nit) step(it + 1, a1, a0);
    }
    if constexpr (KH == 2) {
        // The odd key half's sums -> LDS (the K tiles are free once every wave is past its
        // last step), added by the even half in that order.
        float *red = &k_lds[0][0][0];  // [qrs][DT][16][64]
        static_assert(2 * DT * 16 * kWave <= KH * 2 * C::TILE, "reduction buffer");
        __syncthreads();
        if (kh == 1) {
#pragma unroll
            for (int j = 0; j < DT; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) red[((qrs * DT + j) * 16 + r) * kWave + lane] = acc[j][r];
        }
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int j = 0; j < DT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][r] += red[((qrs * DT + j) * 16 + r) * kWave + lane];
    }
    if (rq0 >= T) return;
    // Lane (col, half), register r of tile j: row rq0 + acc_row(r, half), column dq_col0 + 32 j + col.
    float *p0 = dq + base + int64_t(rq0) * D + dq_col0 + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int dr = acc_row(r, half);
        if (rq0 + dr >= T) continue;
#pragma unroll
        for (int j = 0; j < DT; ++j) p0[dr * D + 32 * j] = acc[j][r] * inv_sqrt_d;
    }
}

// Key-block size of the deterministic dQ partials: they come from the 128-key kernel.  The
// partials cost one [B, H, T, d] fp32 plane per key block, so they are used only up to
// kMaxPartialBlocks key blocks (workspace <= 8 planes, linear in B*H*T); longer sequences
// take the query-major dQ kernel instead.
constexpr int kPartialBN = 128;
constexpr int kMaxPartialBlocks = 8;

bool use_k64_kernel(const AttnShape &s, DqMode mode) {
    return s.causal && s.d >= 64 && mode == DqMode::Atomic;
}

// ds: the dS tiles' workspace (d >= 64, f32_ds_bytes of it), or null.  With it the 64-key
// kernel runs in dS mode (any mask, either policy: no atomics on dQ) and the query-major
// bwd_f32_dq_ds_kernel computes dQ.
template <int D>
hipError_t bwd_f32(const float *q, const float *k, const float *v, const float *o,
                   const float *dout, const float *lse, float *delta, float *dq, float *dk,
                   float *dv, float *dq_part, float *ds, DqMode mode, const AttnShape &s, hipStream_t stream) {
    const int64_t rows = s.rows();
    if (s.T > 2147483647 / D) return hipErrorInvalidValue;
    const unsigned pre_blocks = stride_grid((rows * (D / 4) + 255) / 256, 256);
    const bool ds_mode = D >= 64 && ds != nullptr;
    const bool k64 = D >= 64 && (ds_mode || use_k64_kernel(s, mode));
    const bool split = bwd_f32_use_split(s, k64, stream);
    float *dk_zero = split ? dk : nullptr, *dv_zero = split ? dv : nullptr;
    if (mode == DqMode::Atomic && !ds_mode) {
        hipLaunchKernelGGL((bwd_preprocess_f32_kernel<D, true>), dim3(pre_blocks), dim3(256), 0, stream,
                           o, dout, delta, dq, dk_zero, dv_zero, rows);
    } else {
        hipLaunchKernelGGL((bwd_preprocess_f32_kernel<D, false>), dim3(pre_blocks), dim3(256), 0, stream,
                           o, dout, delta, dq, dk_zero, dv_zero, rows);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if constexpr (D >= 64) {
      if (k64) {
        using C = BwdCfg<D>;
        const int64_t blocks = ((s.T + C::BN - 1) / C::BN) * s.bh() * (split ? 2 : 1);
        if (!grid_fits(blocks, C::NW * kWave)) return hipErrorInvalidValue;
        const float kscale = kLog2e / sqrtf(float(s.scale_dim()));
        const float inv_sqrt_d = 1.f / sqrtf(float(s.scale_dim()));
        auto kern = split ? (ds_mode ? bwd_f32_mfma_kernel<D, true, true> : bwd_f32_mfma_kernel<D, true, false>)
                          : (ds_mode ? bwd_f32_mfma_kernel<D, false, true> : bwd_f32_mfma_kernel<D, false, false>);
        hipLaunchKernelGGL(kern, dim3(unsigned(blocks)), dim3(C::NW * kWave), 0, stream, q, k, v, dout, lse, delta,
                           dq, dk, dv, ds, int(s.T), int(s.bh()), int(s.causal), kscale, inv_sqrt_d);
        e = hipGetLastError();
        if (e != hipSuccess || !ds_mode) return e;
        const int64_t qblocks = (s.T + C::BM - 1) / C::BM * s.bh();
        if (!grid_fits(qblocks, C::NW * kWave)) return hipErrorInvalidValue;
        hipLaunchKernelGGL((bwd_f32_dq_ds_kernel<D, D == 64 ? 2 : 1>), dim3(unsigned(qblocks)), dim3(C::NW * kWave), 0,
                           stream, k, ds,
                           dq, int(s.T), int(s.bh()), int(s.causal), inv_sqrt_d);
        return hipGetLastError();
      }
    }
    const K128Dq k128 = mode == DqMode::Atomic ? K128Dq::Atomic : mode == DqMode::Partial ? K128Dq::Partial : K128Dq::None;
    e = launch_bwd_f32_k128(q, k, v, dout, lse, delta, dq, dq_part, dk, dv, k128, split, s, stream);
    if (e != hipSuccess || mode == DqMode::Atomic) return e;
    if (mode == DqMode::Separate) return launch_bwd_dq_f32(q, k, v, dout, lse, delta, dq, s, stream);
    const int64_t nkb = (s.T + kPartialBN - 1) / kPartialBN;
    const int64_t n4 = rows * (D / 4);
    hipLaunchKernelGGL(dq_reduce_kernel<D>, dim3(stride_grid((n4 + 255) / 256, 256)), dim3(256), 0, stream,
                       dq_part, dq, int(s.T), int(s.bh()), int(s.causal), int(nkb), kPartialBN);
    return hipGetLastError();
}

}  // namespace

// A key-major grid with no more workgroups than the chip holds at once (two per CU at
// d <= 64, one at d = 128) runs as long as its longest key block -- key block 0 with every
// query row when causal -- while most CUs idle: then each key block's rows are split between
// two workgroups.  For the 64-key kernel that pays only when the halved walk is long enough
// to outweigh the dK / dV atomics the split adds: with 16 or more query blocks of 64 up to a
// full chip, with 4 to 15 only while the grid fills at most half of it, with fewer never.
// Same-process A/B, d = 64 (split / not, us): B16 H6 T256 56.1 / 44.7, B16 H6 T128 28.0 /
// 21.0, B4 H12 T512 75.1 / 72.0 (grids of 0.4-0.75 of the chip, short walks: not split);
// B8 H6 T256 29.9 / 32.3, B4 H6 T256 22.3 / 30.8, B2 H12 T512 45.4 / 54.7, B2 H16 T1024 129.7
// / 143.8 (split); d = 128: B8 H6 T256 61.9 / 60.7, B4 H8 T512 97.2 / 107.4.
bool bwd_f32_use_split(const AttnShape &s, bool k64, hipStream_t stream) {
    const int64_t bn = k64 ? 64 : 128;
    const int per_cu = s.d <= 64 ? 2 : 1;
    const int cus = device_cus(stream);
    if (cus <= 0) return false;
    const int64_t blocks = (s.T + bn - 1) / bn * s.bh();
    const int64_t slots = int64_t(per_cu) * cus;
    if (!k64) return blocks <= slots;
    const int64_t nqb = (s.T + 63) / 64;
    return nqb >= 16 ? blocks <= slots : nqb >= 4 && 2 * blocks <= slots;
}

namespace {

// The deterministic fp32 dQ scheme for this problem: partials while they stay small.
DqMode deterministic_mode(const AttnShape &s) {
    return (s.T + kPartialBN - 1) / kPartialBN <= kMaxPartialBlocks ? DqMode::Partial : DqMode::Separate;
}

// The fp32 dS tiles take the workspace only up to this size.
constexpr int64_t kF32DsMaxBytes = int64_t(4) << 30;

}  // namespace

int64_t f32_ds_bytes(const AttnShape &s) {
    if ((s.d != 64 && s.d != 128) || s.T > 32768) return 0;
    const int64_t per_head = f32_ds_tiles_per_head(s.T, s.causal) * kDsTileFloats * int64_t(sizeof(float));
    if (per_head > kF32DsMaxBytes || s.bh() > kF32DsMaxBytes / per_head) return 0;
    return s.bh() * per_head;
}

// Whether the fp32 backward takes the dS path when its scratch holds the tiles.  DETERMINISTIC:
// always -- same-process A/B against the dQ partials / query-major kernel, 0.54-0.95 of their
// time (B8 H12 T1024 d64 causal 337 against 355 us, B4 H12 T4096 d64 2241 against 2889).
// AUTO: only at d = 128 with at least 1024 key blocks of 64 in the grid, where it beat the
// atomic kernel (0.974-0.989: B8 H12 T1024, B4 H16 T2048, causal and full); at d = 64 the
// separate dQ pass costs more than the atomics it removes (+3 to +8 % on the same grids), and
// short grids pay its launch and tail (+3 to +27 %).
bool f32_ds_wanted(const AttnShape &s, bool deterministic) {
    if (f32_ds_bytes(s) == 0) return false;
    return deterministic || (s.d == 128 && (s.T + 63) / 64 * s.bh() >= 1024);
}

bool mfma_bwd_supported(int dtype, int64_t d) {
    (void)dtype;  // the fp32, bf16 and fp16 kernels all cover d in {32, 64, 128}
    return d == 32 || d == 64 || d == 128;
}

int64_t mfma_bwd_workspace_bytes(int dtype, const AttnShape &s, bool deterministic, bool with_ds) {
    if (dtype == 1 || dtype == 2) return bf16_bwd_workspace_bytes(s, deterministic, with_ds);
    // fp32: the deterministic partials (<= 8 dQ planes) or nothing beyond delta; with_ds, room
    // for the dS tiles where the policy takes them (f32_ds_wanted), which then use the scratch.
    int64_t b = 0;
    if (deterministic && deterministic_mode(s) == DqMode::Partial)
        b = (s.T + kPartialBN - 1) / kPartialBN * s.rows() * s.d * int64_t(sizeof(float));
    return with_ds && f32_ds_wanted(s, deterministic) ? std::max(b, f32_ds_bytes(s)) : b;
}

hipError_t launch_mfma_bwd(int dtype, const void *q, const void *k, const void *v,
                           const void *o, const void *dout, const float *lse, float *delta,
                           void *dq, void *dk, void *dv, void *extra, int64_t extra_bytes,
                           bool deterministic, const AttnShape &s, hipStream_t stream) {
    if (dtype == 1)
        return launch_bf16_bwd(q, k, v, o, dout, lse, delta, dq, dk, dv, extra, extra_bytes, deterministic, s,
                               stream);
    if (dtype == 2) return launch_f16_bwd(q, k, v, o, dout, lse, delta, dq, dk, dv, extra, extra_bytes, s, stream);
    const DqMode mode = deterministic ? deterministic_mode(s) : DqMode::Atomic;
    auto f = [](const void *p) { return static_cast<const float *>(p); };
    auto g = [](void *p) { return static_cast<float *>(p); };
    const int64_t dsb = f32_ds_bytes(s);
    float *ds = f32_ds_wanted(s, deterministic) && extra != nullptr && extra_bytes >= dsb ? g(extra) : nullptr;
    switch (s.d) {
        case 32:
            return bwd_f32<32>(f(q), f(k), f(v), f(o), f(dout), lse, delta, g(dq), g(dk), g(dv), g(extra), nullptr,
                               mode, s, stream);
        case 64:
            return bwd_f32<64>(f(q), f(k), f(v), f(o), f(dout), lse, delta, g(dq), g(dk), g(dv), g(extra), ds, mode,
                               s, stream);
        case 128:
            return bwd_f32<128>(f(q), f(k), f(v), f(o), f(dout), lse, delta, g(dq), g(dk), g(dv), g(extra), ds, mode,
                                s, stream);
        default:
            return hipErrorNotSupported;
    }
}

}  // namespace ctattn
