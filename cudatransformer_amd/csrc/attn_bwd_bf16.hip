// bf16 / fp16 flash-attention backward on 16-bit MFMA (v_mfma_f32_32x32x16_bf16 / _f16), fp32
// accumulate; the fp16 instantiation (F16Fmt) is the same code with the fp16 MFMA and fp16
// rounding.
//
// Same math as the fp32 backward (attn_bwd_mfma.hip) and the reference's
// flashAttentionBackward (flash_attention.cu:226-326, with correct dK / dV): P and dS are
// computed in fp32 and rounded to bf16 only as MFMA operands; dK, dV, dQ accumulate in fp32
// and are rounded to bf16 once.
//
// Two kernels, no atomics.  fp32 global atomics run at ~1.35 TB/s on MI355X, and the fused
// key-major design's dQ atomics (T^2/2 * d / 128 per head, 4.3 GB at B1 H32 T8192 d128)
// bound it at ~3 ms; recomputing S and dP in a second, query-major kernel costs 2 of the
// backward's 5 matmuls again but runs at MFMA speed and is deterministic by construction.
//   * bwd_bf16_dkdv_kernel (key-major): a workgroup of 8 waves owns 128 keys (4 key slices
//     of 32 x 2 row slices), keeps dK^T and dV^T in registers and walks 64-row query blocks
//     (causal: from its diagonal on), row slice rs taking rows 32 rs .. 32 rs + 31 of each;
//     the two row slices' sums meet in LDS at the end.  S = Q K^T, dP = dO V^T (lane = one
//     key, registers = rows), then
//     P = exp2(S c + nl2), dS = P (dP - delta) elementwise (the dP accumulator starts from
//     -delta), and dV^T += dO^T P,
//     dK^T += Q^T dS with P / dS straight from the accumulator as B operands.
//   * bwd_bf16_dq_kernel (query-major): a workgroup of 4 waves owns 128 query rows (wave w:
//     32), keeps dQ in registers and walks 32-key blocks (causal: up to its diagonal).
//     S^T = K Q^T, dP^T = V dO^T (lane = one row), P^T, dS^T elementwise, and
//     dQ += dS K with dS straight from the accumulator as the A operand.
// A 32x32x16 operand takes 8 consecutive contraction indices from lane (i, k / 8); an S /
// dP accumulator holds rows 16 s + 8 (e / 4) + 4 half + e % 4 in registers 8 s + e, so the
// contractions over rows (dV, dK) and keys (dQ) run in that permuted order, and their other
// operand (dO^T, Q^T, K^T) is read column-wise from the same row-major LDS tile with
// ds_read_b64_tr_b16 (two reads of 4 rows each).
//
// LDS tiles are row-major, D bf16 per row, loaded global -> LDS directly
// (global_load_lds_dwordx4), with the 16-byte chunk index XOR-swizzled by the row
// (Tile<D>::swz) so that both the row reads (16 lanes, 16 rows, one chunk) and the
// transposed reads (32 lanes, 4 rows x 4 chunks) hit 64 distinct banks.
#include "attn_bf16_tiles.h"
#include "attn_launch.h"

#include <math.h>

#include <type_traits>

namespace ctattn {
namespace {

using namespace bf16tile;

// ---------------------------------------------------------------------------------------
// dS tiles (d = 128): the dK/dV kernel stores the bf16 dS it computes, and the dQ kernel
// reads it back instead of recomputing S and dP.
// ---------------------------------------------------------------------------------------
// One 32-row x 32-key tile of dS, 2 KiB, laid out as the LDS tile Tile<32> of a [key][32]
// matrix whose columns hold the tile's query rows in the accumulator order: column
// 16 kk + 8 h + e is row 16 kk + 8 (e / 4) + 4 h + e % 4 (e < 8).
// Copied byte for byte into LDS, its transposed reads (read_col<32>) are the A operands of
// dQ += dS K, in the key order read_col gives the K operands.  Tiles of a (batch, head) are
// packed by (row tile rt, key tile kt): rt (rt + 1) / 2 + kt with kt <= rt when causal,
// rt * NT + kt otherwise (NT = ceil(T / 32)).
constexpr int kDsTileElems = 32 * 32;

__device__ __host__ inline int64_t ds_tiles_per_head(int64_t T, bool causal) {
    const int64_t nt = (T + 31) / 32;
    return causal ? nt * (nt + 1) / 2 : nt * nt;
}
__device__ __forceinline__ int64_t ds_tile_index(int bh, int rt, int kt, int T, int causal) {
    const int64_t nt = (T + 31) / 32;
    return int64_t(bh) * ds_tiles_per_head(T, causal != 0) +
           (causal ? int64_t(rt) * (rt + 1) / 2 + kt : int64_t(rt) * nt + kt);
}
// Query row of DsTile column c.
__device__ __forceinline__ int ds_col_row(int c) {
    const int e = c & 7;
    return (c & 16) + 8 * (e >> 2) + ((c >> 1) & 4) + (e & 3);
}

// ---------------------------------------------------------------------------------------
// dK / dV (key-major)
// ---------------------------------------------------------------------------------------
template <int D>
struct KvCfg {
    static constexpr int NW = 8;       // waves: 4 key slices (ks = wave & 3) x 2 row slices (rs = wave >> 2)
    static constexpr int BN = 128;     // keys per workgroup; key slice ks: 32 ks .. 32 ks + 31
    static constexpr int BM = 64;      // query rows per iteration; row slice rs: 32 rs .. 32 rs + 31
    static constexpr int DT = D / 32;
    static constexpr int KSTEPS = D / 16;
    static constexpr int ROW = 2 * D;            // bytes per tile row
    static constexpr int KV_BYTES = BN * ROW;    // K (or V) tile
    static constexpr int Q_BYTES = BM * ROW;     // Q (or dO) tile
    // LDS map: per buffer b, Q and dO at Q_OFF + b * 2 * Q_BYTES (+ Q_BYTES); then K, V; then
    // per buffer b, nl2 and delta (BM floats each) at S_OFF + b * 2 * BM * 4.  Every offset
    // added to a per-lane address is an immediate (< 64 KiB).
    static constexpr int Q_OFF = 0;
    static constexpr int K_OFF = 4 * Q_BYTES;
    static constexpr int V_OFF = K_OFF + KV_BYTES;
    static constexpr int S_OFF = V_OFF + KV_BYTES;
    static constexpr int LDS_BYTES = S_OFF + 4 * BM * 4;
    static_assert(Q_BYTES + 16 * ROW < 65536 && KV_BYTES < 65536, "immediate offsets");
    // The row slices' dK^T / dV^T partial sums meet in LDS at the end.
    static_assert(4 * DT * 2 * 16 * kWave * 4 <= LDS_BYTES, "reduction buffer");
};

// One 32-row x 32-key wave tile: S, dP, P, dS and the dV^T / dK^T updates.
//   aq   : row_base of this wave's first Q row in the block's Q tile (dO at + Q_BYTES)
//   ak   : row_base of this wave's first key in the K tile (V at + KV_BYTES)
//   ac0/1: col_base of the wave's Q rows (dO at + Q_BYTES)
//   anl  : address of nl2[32 rs + 4 half] of the block (delta at + BM * 4)
//   dsw  : when DS, where the tile's dS goes (a 32 x 32 DsTile, rows = keys)
template <int D, bool MASK, bool DS, typename F>
__device__ __forceinline__ void kv_block(floatx16 (&dk_acc)[D / 32], floatx16 (&dv_acc)[D / 32], uint32_t aq,
                                         uint32_t ak, uint32_t ac0, uint32_t ac1, uint32_t anl, int r0w,
                                         int key, int T, int causal, float c, int half, uint16_t *dsw) {
    using C = KvCfg<D>;
    using V = typename F::vec;
    // dP starts from -delta of the rows (register r: row acc_row(r, half)), so the
    // accumulator ends as dP - delta and dS = P * acc.
    floatx16 s = zero16(), dp;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const floatx4 d4 = lds_f4(anl + C::BM * 4 + 32 * g);
#pragma unroll
        for (int t = 0; t < 4; ++t) dp[4 * g + t] = d4[t];
    }
    {
        V qa[2], ka[2], da[2], va[2];
        qa[0] = lds_b128<V>(aq);
        ka[0] = lds_b128<V>(ak);
        da[0] = lds_b128<V>(aq + C::Q_BYTES);
        va[0] = lds_b128<V>(ak + C::KV_BYTES);
#pragma unroll
        for (int st = 0; st < C::KSTEPS; ++st) {
            const int cur = st & 1, nxt = cur ^ 1;
            if (st + 1 < C::KSTEPS) {
                const uint32_t xq = aq ^ uint32_t((st + 1) << 5), xk = ak ^ uint32_t((st + 1) << 5);
                qa[nxt] = lds_b128<V>(xq);
                ka[nxt] = lds_b128<V>(xk);
                da[nxt] = lds_b128<V>(xq + C::Q_BYTES);
                va[nxt] = lds_b128<V>(xk + C::KV_BYTES);
            }
            read_fence();
            s = F::mfma(qa[cur], ka[cur], s);
            dp = F::mfma(da[cur], va[cur], dp);
        }
    }
    // lane = key; register r = row r0w + acc_row(r, half)
    V pb[2], dsb[2];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const floatx4 n4 = lds_f4(anl + 32 * g);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int r = 4 * g + t;
            float p = fast_exp2(fmaf(s[r], c, n4[t]));
            if (MASK) {
                const int row = r0w + acc_row(r, half);
                p = (row >= T || key >= T || (causal && key > row)) ? 0.f : p;
            }
            pb[r / 8][r % 8] = (typename F::elem)p;
            dsb[r / 8][r % 8] = (typename F::elem)(p * dp[r]);
        }
    }
    if (DS) {
        // The tile's dS for the dQ kernel: lane (key, half) holds, in dsb[kk], the 8 rows of
        // logical chunk 2 kk + half of the key's DsTile row.
        const int key_l = __lane_id() & 31;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            u16x8 *dst = reinterpret_cast<u16x8 *>(reinterpret_cast<char *>(dsw) + Tile<32>::off(key_l, 2 * kk + half));
            *dst = __builtin_bit_cast(u16x8, dsb[kk]);
        }
    }
    // dV^T += dO^T P, dK^T += Q^T dS over the tile's 32 rows (two k-steps of 16).
    {
        constexpr int NS = 2 * C::DT;
        V ao[2], aqT[2];
        ao[0] = read_col<D, V>(ac0 + C::Q_BYTES, ac1 + C::Q_BYTES, 0, 0);
        aqT[0] = read_col<D, V>(ac0, ac1, 0, 0);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int cur = i & 1, nxt = cur ^ 1;
            if (i + 1 < NS) {
                const int kk = (i + 1) / C::DT, dt = (i + 1) % C::DT;
                ao[nxt] = read_col<D, V>(ac0 + C::Q_BYTES, ac1 + C::Q_BYTES, kk, dt);
                aqT[nxt] = read_col<D, V>(ac0, ac1, kk, dt);
            }
            read_fence();
            const int kk = i / C::DT, dt = i % C::DT;
            dv_acc[dt] = F::mfma(ao[cur], pb[kk], dv_acc[dt]);
            dk_acc[dt] = F::mfma(aqT[cur], dsb[kk], dk_acc[dt]);
        }
    }
}

template <int D, bool DS, typename F>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_bf16_dkdv_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const uint16_t *__restrict__ dout, const float *__restrict__ nl2, const float *__restrict__ delta,
    uint16_t *__restrict__ dk, uint16_t *__restrict__ dv, uint16_t *__restrict__ ds, int T, int BH, int causal,
    float c, float inv_sqrt_d) {
    using C = KvCfg<D>;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
    const uint32_t L = lds_addr(smem);

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int ks = wave & 3, rs = wave >> 2;

    const int id = blockIdx.x;
    const int bh = id % BH;
    const int kb = id / BH;  // causal: key block 0 has the most query blocks -> launched first
    const int k0 = kb * C::BN;
    const int64_t base = int64_t(bh) * T * D;
    const int64_t rbase = int64_t(bh) * T;
    const int kw0 = k0 + 32 * ks;
    const int key = kw0 + col;

    // Tile loads go through load_tile_dma / load_dword_dma, which the compiler does not see:
    // it would otherwise make the block's first LDS read wait for the next block's prefetch.
    // The loop waits for each block's loads itself, before the barrier that publishes them.
    load_tile_dma<D, C::BN, C::NW>(smem + C::K_OFF, k + base + int64_t(k0) * D, T - k0, wave, lane);
    load_tile_dma<D, C::BN, C::NW>(smem + C::V_OFF, v + base + int64_t(k0) * D, T - k0, wave, lane);
    floatx16 dk_acc[C::DT], dv_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
        dk_acc[dt] = zero16();
        dv_acc[dt] = zero16();
    }

    // Per-lane parts of the operand addresses (the swizzle depends on the row mod 16 only, so
    // the slice offsets 32 rs / 32 ks rows keep the pattern).
    const uint32_t rq = uint32_t(Tile<D>::off(32 * rs + col, half));
    const uint32_t ak = row_base<D>(L + C::K_OFF, 32 * ks + col, half);
    const uint32_t cq0 = col_base<D>(0, 32 * rs, 0, lane), cq1 = col_base<D>(0, 32 * rs, 1, lane);
    const uint32_t rnl = uint32_t(4 * (32 * rs + 4 * half));

    const int nqb = (T + C::BM - 1) / C::BM;
    const int qb_first = causal ? k0 / C::BM : 0;
    auto issue = [&](int r0, int buf) {
        char *qt = smem + C::Q_OFF + buf * 2 * C::Q_BYTES;
        load_tile_dma<D, C::BM, C::NW>(qt, q + base + int64_t(r0) * D, T - r0, wave, lane);
        load_tile_dma<D, C::BM, C::NW>(qt + C::Q_BYTES, dout + base + int64_t(r0) * D, T - r0, wave, lane);
        if (wave >= C::NW - 2) {  // nl2 / delta of the block's rows, one dword per lane
            const bool is_nl = wave == C::NW - 2;
            load_dword_dma((is_nl ? nl2 : delta) + rbase + min(r0 + lane, T - 1),
                           lds_addr(smem + C::S_OFF + buf * 2 * C::BM * 4 + (is_nl ? 0 : C::BM * 4)));
        }
    };

    if (qb_first < nqb) issue(qb_first * C::BM, 0);
    bool stored = false;  // DS: this wave stored a dS tile (two stores) after its last loads
    for (int qb = qb_first; qb < nqb; ++qb) {
        const int buf = (qb - qb_first) & 1;
        // This wave's loads of `buf` have landed; after the barrier every wave's have, and
        // every wave is done reading buf ^ 1.  The dS stores of the previous block, issued
        // after those loads, may stay in flight (vmcnt counts in issue order): nothing in this
        // kernel reads them.
        if (DS) {
            if (stored) __builtin_amdgcn_s_waitcnt(0xF72);  // vmcnt(2)
            else __builtin_amdgcn_s_waitcnt(0xF70);
            lds_barrier();
        } else {
            __builtin_amdgcn_s_waitcnt(0xF70);
            __syncthreads();
        }
        if (qb + 1 < nqb) issue((qb + 1) * C::BM, buf ^ 1);
        const int r0w = qb * C::BM + 32 * rs;
        const bool active = kw0 < T && r0w < T && (!causal || kw0 <= r0w + 31);
        stored = DS && active;
        if (!active) continue;
        const uint32_t qt = L + C::Q_OFF + uint32_t(buf * 2 * C::Q_BYTES);
        const uint32_t anl = L + C::S_OFF + uint32_t(buf * 2 * C::BM * 4) + rnl;
        const bool masked = (r0w + 32 > T) || (kw0 + 32 > T) || (causal && kw0 + 31 > r0w);
        uint16_t *dsw = DS ? ds + ds_tile_index(bh, r0w / 32, kw0 / 32, T, causal) * kDsTileElems : nullptr;
        if (masked)
            kv_block<D, true, DS, F>(dk_acc, dv_acc, qt + rq, ak, qt + cq0, qt + cq1, anl, r0w, key, T, causal, c,
                                     half, dsw);
        else
            kv_block<D, false, DS, F>(dk_acc, dv_acc, qt + rq, ak, qt + cq0, qt + cq1, anl, r0w, key, T, causal, c,
                                      half, dsw);
    }

    // Row slice 1 hands its dK^T / dV^T sums to row slice 0 through LDS (no load is in flight
    // and, after the barrier, no wave reads a tile any more).  Lane (key, half), register r
    // of tile dt holds d = 32 dt + acc_row(r, half).
    float *red = reinterpret_cast<float *>(smem);
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
    if (rs == 0 && key < T) {
        uint16_t *dkr = dk + base + int64_t(key) * D;
        uint16_t *dvr = dv + base + int64_t(key) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                u16x4 xk, xv;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int r = 4 * g + t;
                    const float sk = dk_acc[dt][r] + red[(((ks * C::DT + dt) * 2 + 0) * 16 + r) * kWave + lane];
                    const float sv = dv_acc[dt][r] + red[(((ks * C::DT + dt) * 2 + 1) * 16 + r) * kWave + lane];
                    xk[t] = F::bits(sk * inv_sqrt_d);
                    xv[t] = F::bits(sv);
                }
                *reinterpret_cast<u16x4 *>(dkr + dt * 32 + 8 * g + 4 * half) = xk;
                *reinterpret_cast<u16x4 *>(dvr + dt * 32 + 8 * g + 4 * half) = xv;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// dQ (query-major)
// ---------------------------------------------------------------------------------------
template <int D>
struct QCfg {
    static constexpr int NW = 4;
    static constexpr int BM = 32 * NW;  // query rows per workgroup
    static constexpr int BN = 32;       // keys per iteration
    static constexpr int DT = D / 32;
    static constexpr int KSTEPS = D / 16;
    static constexpr int KB = BN * 2 * D;       // bytes of a K (or V) tile
    static constexpr int LDS_BYTES = 4 * KB;    // buffer b: K at 2 b KB, V at 2 b KB + KB
};

// One 32-key block for one wave (32 rows): S^T, dP^T, P^T, dS^T and the dQ update.
//   ak   : row_base of the block's K tile for key `col` (V at + KB)
//   ac0/1: col_base of the K tile
template <int D, bool MASK, typename F>
__device__ __forceinline__ void dq_block(floatx16 (&dq_acc)[D / 32], const typename F::vec (&qB)[D / 16],
                                         const typename F::vec (&doB)[D / 16], uint32_t ak, uint32_t ac0,
                                         uint32_t ac1, float nlr, const floatx16 &ndl, int j0, int row, int T,
                                         int causal, float c, int half) {
    using C = QCfg<D>;
    using V = typename F::vec;
    // dP^T starts from -delta of the lane's row, so the accumulator ends as dP^T - delta.
    floatx16 s = zero16(), dp = ndl;
    {
        V ka[2], va[2];
        ka[0] = lds_b128<V>(ak);
        va[0] = lds_b128<V>(ak + C::KB);
#pragma unroll
        for (int st = 0; st < C::KSTEPS; ++st) {
            const int cur = st & 1, nxt = cur ^ 1;
            if (st + 1 < C::KSTEPS) {
                const uint32_t x = ak ^ uint32_t((st + 1) << 5);
                ka[nxt] = lds_b128<V>(x);
                va[nxt] = lds_b128<V>(x + C::KB);
            }
            read_fence();
            s = F::mfma(ka[cur], qB[st], s);
            dp = F::mfma(va[cur], doB[st], dp);
        }
    }
    // lane = query row; register r = key j0 + acc_row(r, half)
    V dsb[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], c, nlr));
        if (MASK) {
            const int key = j0 + acc_row(r, half);
            p = (key >= T || row >= T || (causal && key > row)) ? 0.f : p;
        }
        dsb[r / 8][r % 8] = (typename F::elem)(p * dp[r]);
    }
    // dQ += dS K over the block's 32 keys (two k-steps of 16).
    {
        constexpr int NS = 2 * C::DT;
        V kt[2];
        kt[0] = read_col<D, V>(ac0, ac1, 0, 0);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int cur = i & 1, nxt = cur ^ 1;
            if (i + 1 < NS) kt[nxt] = read_col<D, V>(ac0, ac1, (i + 1) / C::DT, (i + 1) % C::DT);
            read_fence();
            dq_acc[i % C::DT] = F::mfma(dsb[i / C::DT], kt[cur], dq_acc[i % C::DT]);
        }
    }
}

template <int D, typename F>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_bf16_dq_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const uint16_t *__restrict__ dout, const float *__restrict__ nl2, const float *__restrict__ delta,
    uint16_t *__restrict__ dq, int T, int BH, int causal, float c, float inv_sqrt_d) {
    using C = QCfg<D>;
    using V = typename F::vec;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
    const uint32_t L = lds_addr(smem);

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform
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

    // Q^T and dO^T as B operands: lane (row, half) holds Q[row][16 st + 8 half ..].
    V qB[C::KSTEPS], doB[C::KSTEPS];
#pragma unroll
    for (int st = 0; st < C::KSTEPS; ++st) {
        u16x8 xq = {0, 0, 0, 0, 0, 0, 0, 0}, xd = {0, 0, 0, 0, 0, 0, 0, 0};
        if (row < T) {
            xq = *reinterpret_cast<const u16x8 *>(q + base + int64_t(row) * D + 16 * st + 8 * half);
            xd = *reinterpret_cast<const u16x8 *>(dout + base + int64_t(row) * D + 16 * st + 8 * half);
        }
        qB[st] = __builtin_bit_cast(V, xq);
        doB[st] = __builtin_bit_cast(V, xd);
    }
    const float nlr = row < T ? nl2[rbase + row] : 0.f;
    const float ndr = row < T ? delta[rbase + row] : 0.f;  // -delta
    floatx16 ndl;
#pragma unroll
    for (int r = 0; r < 16; ++r) ndl[r] = ndr;
    floatx16 dq_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) dq_acc[dt] = zero16();

    const uint32_t rk = uint32_t(Tile<D>::off(col, half));
    const uint32_t ck0 = col_base<D>(0, 0, 0, lane), ck1 = col_base<D>(0, 0, 1, lane);

    const int kend = causal ? min(T, r0 + C::BM) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;
    // K / V blocks through load_tile_dma (invisible to the compiler, so the block's LDS reads do
    // not wait for the next block's prefetch); the loop awaits each block before its barrier.
    auto issue = [&](int j0, int buf) {
        load_tile_dma<D, C::BN, C::NW>(smem + 2 * buf * C::KB, k + base + int64_t(j0) * D, T - j0, wave, lane);
        load_tile_dma<D, C::BN, C::NW>(smem + 2 * buf * C::KB + C::KB, v + base + int64_t(j0) * D, T - j0, wave, lane);
    };

    // Block kb: wait for its loads (this wave's, then everyone's through the barrier, which
    // also ends every wave's reads of the other buffer) and prefetch the next; returns the
    // block's K tile address.
    auto step = [&](int kb) __attribute__((always_inline)) {
        const int buf = kb & 1;
        __builtin_amdgcn_s_waitcnt(0xF70);
        __syncthreads();
        if (kb + 1 < nkb) issue((kb + 1) * C::BN, buf ^ 1);
        return L + uint32_t(2 * buf * C::KB);
    };
    // Three loops without branches inside, so dq_acc keeps its registers across blocks (one
    // loop over both variants made the compiler copy all 64 accumulator registers per block):
    // [0, jm) unmasked, [jm, wave_nkb) masked (the wave's diagonal or the sequence end),
    // [wave_nkb, nkb) keys wholly above the wave's rows (barriers and loads only).
    const int jm = min(min(nkb, T / C::BN), causal ? (wave_first_row + 1) / C::BN : nkb);
    const int wave_nkb = causal ? min(nkb, wave_last_row / C::BN + 1) : nkb;
    issue(0, 0);
    int kb = 0;
    for (; kb < jm; ++kb) {
        const uint32_t kt = step(kb);
        dq_block<D, false, F>(dq_acc, qB, doB, kt + rk, kt + ck0, kt + ck1, nlr, ndl, kb * C::BN, row, T, causal, c,
                           half);
    }
    for (; kb < wave_nkb; ++kb) {
        const uint32_t kt = step(kb);
        dq_block<D, true, F>(dq_acc, qB, doB, kt + rk, kt + ck0, kt + ck1, nlr, ndl, kb * C::BN, row, T, causal, c,
                          half);
    }
    for (; kb < nkb; ++kb) step(kb);

    // dq_acc[dt]: lane (col, half), register r -> row wave_first_row + acc_row(r, half),
    // column 32 dt + col.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int rr = wave_first_row + acc_row(r, half);
        if (rr >= T) continue;
        uint16_t *p = dq + base + int64_t(rr) * D + col;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) p[32 * dt] = F::bits(dq_acc[dt][r] * inv_sqrt_d);
    }
}

// ---------------------------------------------------------------------------------------
// dQ from stored dS (d = 128)
// ---------------------------------------------------------------------------------------
// dQ = dS K / sqrt(d) from the dS tiles the dK/dV kernel stored: no recompute of S or dP.  A
// workgroup of 8 waves owns 256 query rows (wave w: row tile r0 / 32 + w) and walks 64-key
// blocks: the block's K rows (a Tile<D>) and each wave's two dS tiles go global -> LDS
// directly, three blocks in flight; dS^T columns (read_col<32>) are the A operands, K^T columns
// (read_col<D>) the B operands, both in the same key order.  Bound by the dS stream from HBM.
template <int D>
struct DqDsCfg {
    static constexpr int NW = 8;
    static constexpr int BM = 32 * NW;        // query rows per workgroup
    static constexpr int BN = 64;             // keys per iteration: key tiles 2 kb, 2 kb + 1
    static constexpr int DT = D / 32;
    static constexpr int ROW = 2 * D;
    static constexpr int D8 = D / 8;          // 16-byte chunks per row
    static constexpr int KB = BN * ROW;       // K tile
    static constexpr int SB = NW * 2 * 2048;  // the waves' dS tiles
    static constexpr int BUF = KB + SB;
    static constexpr int STAGES = 3;          // blocks kb + 1 and kb + 2 load during block kb
    static constexpr int LDS_BYTES = STAGES * BUF;
};

// 2 KiB global -> LDS (one wave): lane l moves bytes 16 l and 1024 + 16 l.  Non-temporal
// (`nt`): each dS tile is read once, and streaming it through L2 as evict-first keeps the K
// blocks, which every query block re-reads, resident there.  Same-process A/B of the dQ pass
// (outputs bitwise equal): B1 H32 T8192 causal 459 -> 426 us, B1 H64 T4096 251 -> 219, B1 H64
// T2048 67.0 -> 60.3.
__device__ __forceinline__ void dma_2k(const uint16_t *src, uint32_t dst, int lane) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const char *g = reinterpret_cast<const char *>(src) + h * 1024 + 16 * lane;
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g),
                     "s"(__builtin_amdgcn_readfirstlane(dst + uint32_t(h * 1024)))
                     : "memory", "m0");
    }
}

template <int D, typename F>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_bf16_dq_ds_kernel(
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ ds, uint16_t *__restrict__ dq, int T, int BH,
    int causal, float inv_sqrt_d) {
    using C = DqDsCfg<D>;
    using V = typename F::vec;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
    const uint32_t L = lds_addr(smem);

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int col = lane & 31;
    const int half = lane >> 5;

    const int nqb = (T + C::BM - 1) / C::BM;
    const int id = blockIdx.x;
    const int bh = id % BH;
    const int qb = causal ? (nqb - 1 - id / BH) : id / BH;  // causal: longest first
    const int64_t base = int64_t(bh) * T * D;
    const int r0 = qb * C::BM;
    const int nt = (T + 31) / 32;
    const int rt = r0 / 32 + wave;  // this wave's row tile
    // Key tiles [0, wave_nkt) of this wave (none when its rows are past T).
    const int wave_nkt = rt >= nt ? 0 : causal ? rt + 1 : nt;
    const int kend = causal ? min(T, r0 + C::BM) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;

    floatx16 dq_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) dq_acc[dt] = zero16();
    const uint32_t ck0 = col_base<D>(0, 0, 0, lane), ck1 = col_base<D>(0, 0, 1, lane);
    const uint32_t cs0 = col_base<32>(0, 0, 0, lane), cs1 = col_base<32>(0, 0, 1, lane);

    auto issue = [&](int kb, int buf) {
        char *b = smem + buf * C::BUF;
        load_tile_dma<D, C::BN, C::NW>(b, k + base + int64_t(kb) * C::BN * D, T - kb * C::BN, wave, lane);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int kt = 2 * kb + tt;
            if (kt < wave_nkt)
                dma_2k(ds + ds_tile_index(bh, rt, kt, T, causal) * kDsTileElems,
                       lds_addr(b + C::KB + (wave * 2 + tt) * 2048), lane);
        }
    };
    // Loads this wave issues for block kb: the K tile's share (load_tile_dma: 2 per wave) and
    // two per live dS tile.  The wait before block kb lets block kb + 1's stay in flight
    // (vmcnt counts in issue order).
    auto wave_loads = [&](int kb) {
        return kb >= nkb ? 0 : 2 + 2 * (int(2 * kb < wave_nkt) + int(2 * kb + 1 < wave_nkt));
    };
    static_assert(C::BN * C::D8 / (C::NW * kWave) == 2, "K tile loads per wave");
    if (nkb > 0) issue(0, 0);
    if (nkb > 1) issue(1, 1);
    int buf = 0;
    for (int kb = 0; kb < nkb; ++kb) {
        switch (wave_loads(kb + 1)) {
            case 0: __builtin_amdgcn_s_waitcnt(0xF70); break;
            case 2: __builtin_amdgcn_s_waitcnt(0xF72); break;
            case 4: __builtin_amdgcn_s_waitcnt(0xF74); break;
            default: __builtin_amdgcn_s_waitcnt(0xF76); break;
        }
        lds_barrier();
        if (kb + 2 < nkb) issue(kb + 2, buf == 0 ? 2 : buf - 1);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            if (2 * kb + tt >= wave_nkt) continue;
            const uint32_t ka = L + uint32_t(buf * C::BUF + tt * 32 * C::ROW);
            const uint32_t sa = L + uint32_t(buf * C::BUF + C::KB + (wave * 2 + tt) * 2048);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const V a = read_col<32, V>(sa + cs0, sa + cs1, kk, 0);
#pragma unroll
                for (int dt = 0; dt < C::DT; ++dt)
                    dq_acc[dt] = F::mfma(a, read_col<D, V>(ka + ck0, ka + ck1, kk, dt), dq_acc[dt]);
            }
        }
        buf = buf == 2 ? 0 : buf + 1;
    }

    // dq_acc[dt]: lane (col, half), register r -> dS column acc_row(r, half) of the tile, i.e.
    // query row 32 rt + ds_col_row(acc_row(r, half)); d = 32 dt + col.
    if (wave_nkt == 0) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = 32 * rt + ds_col_row(acc_row(r, half));
        if (row >= T) continue;
        uint16_t *p = dq + base + int64_t(row) * D + col;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) p[32 * dt] = F::bits(dq_acc[dt][r] * inv_sqrt_d);
    }
}

// delta[row] = -sum_c dO[row][c] O[row][c] from bf16 (the negated delta of
// flash_attention.cu:269-273: the dP accumulators of both kernels start from it) and
// nl2[row] = -LSE[row] * log2(e), the per-row term of P = exp2(S log2(e)/sqrt(d) + nl2).
// D / 8 lanes per row, one 16-byte load of O and of dO each.
template <int D, typename F>
__global__ __launch_bounds__(256) void bwd_preprocess_bf16_kernel(const uint16_t *__restrict__ o,
                                                                 const uint16_t *__restrict__ dout,
                                                                 const float *__restrict__ lse,
                                                                 float *__restrict__ delta,
                                                                 float *__restrict__ nl2, int64_t rows) {
    constexpr int LPR = D / 8;  // lanes per row
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    // Grid-stride; the block size and the stride are multiples of LPR, so the LPR lanes of a
    // row enter and leave the loop together (group_sum stays inside the group).
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t / LPR < rows; t += stride) {
        const int64_t row = t / LPR;
        const int c8 = int(t % LPR);
        float s = 0.f;
        if (row < rows) {
            const u16x8 a = *reinterpret_cast<const u16x8 *>(o + row * D + 8 * c8);
            const u16x8 b = *reinterpret_cast<const u16x8 *>(dout + row * D + 8 * c8);
#pragma unroll
            for (int e = 0; e < 8; ++e) s += F::widen(a[e]) * F::widen(b[e]);
        }
        s = group_sum<LPR>(s);
        if (row < rows && c8 == 0) {
            delta[row] = -s;
            nl2[row] = -lse[row] * kLog2e;
        }
    }
}

template <int D, typename F>
hipError_t bwd_bf16(const void *q, const void *k, const void *v, const void *o, const void *dout,
                    const float *lse, float *delta, void *dq, void *dk, void *dv, float *nl2, uint16_t *ds,
                    const AttnShape &s, hipStream_t stream) {
    using KC = KvCfg<D>;
    using QC = QCfg<D>;
    const int64_t kv_blocks = ((s.T + KC::BN - 1) / KC::BN) * s.bh();
    const int64_t q_blocks = ((s.T + QC::BM - 1) / QC::BM) * s.bh();
    if (!grid_fits(kv_blocks, KC::NW * kWave) || !grid_fits(q_blocks, QC::NW * kWave) || s.T > 2147483647 / D)
        return hipErrorInvalidValue;
    const int64_t rows = s.rows();
    auto u16 = [](const void *p) { return static_cast<const uint16_t *>(p); };
    const int64_t pre_threads = rows * (D / 8);
    hipLaunchKernelGGL((bwd_preprocess_bf16_kernel<D, F>), dim3(stride_grid((pre_threads + 255) / 256, 256)), dim3(256), 0, stream,
                       u16(o), u16(dout), lse, delta, nl2, rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const float c = kLog2e / sqrtf(float(s.scale_dim()));
    const float inv_sqrt_d = 1.f / sqrtf(float(s.scale_dim()));
    if constexpr (D == 128) {
        if (ds != nullptr) {
            // dS through the workspace: the dK/dV kernel stores it, the dQ kernel multiplies it by K.
            hipLaunchKernelGGL((bwd_bf16_dkdv_kernel<D, true, F>), dim3(unsigned(kv_blocks)), dim3(KC::NW * kWave), 0,
                               stream, u16(q), u16(k), u16(v), u16(dout), nl2, delta, static_cast<uint16_t *>(dk),
                               static_cast<uint16_t *>(dv), ds, int(s.T), int(s.bh()), int(s.causal), c, inv_sqrt_d);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            using DC = DqDsCfg<D>;
            const int64_t dq_blocks = ((s.T + DC::BM - 1) / DC::BM) * s.bh();
            hipLaunchKernelGGL((bwd_bf16_dq_ds_kernel<D, F>), dim3(unsigned(dq_blocks)), dim3(DC::NW * kWave), 0, stream,
                               u16(k), ds, static_cast<uint16_t *>(dq), int(s.T), int(s.bh()), int(s.causal), inv_sqrt_d);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((bwd_bf16_dkdv_kernel<D, false, F>), dim3(unsigned(kv_blocks)), dim3(KC::NW * kWave), 0,
                       stream, u16(q), u16(k), u16(v), u16(dout), nl2, delta, static_cast<uint16_t *>(dk),
                       static_cast<uint16_t *>(dv), nullptr, int(s.T), int(s.bh()), int(s.causal), c, inv_sqrt_d);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_bf16_dq_kernel<D, F>), dim3(unsigned(q_blocks)), dim3(QC::NW * kWave), 0, stream, u16(q),
                       u16(k), u16(v), u16(dout), nl2, delta, static_cast<uint16_t *>(dq), int(s.T), int(s.bh()),
                       int(s.causal), c, inv_sqrt_d);
    return hipGetLastError();
}

}  // namespace

namespace {
// The dS tiles take the workspace only up to this size; longer problems recompute S and dP in
// the dQ kernel instead (their workspace stays linear in rows).
constexpr int64_t kDsMaxBytes = int64_t(4) << 30;
int64_t nl2_bytes(const AttnShape &s) { return (s.rows() * int64_t(sizeof(float)) + 255) / 256 * 256; }
}  // namespace

int64_t bf16_ds_bytes(const AttnShape &s) {
    // T > 65536 needs more than 4 GiB of tiles even for one causal head (and the product
    // below could overflow for the longest sequences), so it never takes the dS path.
    if (s.d != 128 || s.T > 65536) return 0;
    const int64_t b = s.bh() * ds_tiles_per_head(s.T, s.causal) * kDsTileElems * int64_t(sizeof(uint16_t));
    return b <= kDsMaxBytes ? b : 0;
}

int64_t bf16_bwd_workspace_bytes(const AttnShape &s, bool deterministic, bool with_ds) {
    (void)deterministic;  // both paths are deterministic: no atomics, fixed summation order
    return nl2_bytes(s) + (with_ds ? bf16_ds_bytes(s) : 0);
}

hipError_t launch_bf16_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
                           const float *lse, float *delta, void *dq, void *dk, void *dv, void *extra,
                           int64_t extra_bytes, bool deterministic, const AttnShape &s, hipStream_t stream) {
    (void)deterministic;
    float *nl2 = static_cast<float *>(extra);
    const int64_t dsb = bf16_ds_bytes(s);
    uint16_t *ds = dsb > 0 && extra_bytes >= nl2_bytes(s) + dsb
                       ? reinterpret_cast<uint16_t *>(static_cast<char *>(extra) + nl2_bytes(s))
                       : nullptr;
    switch (s.d) {
        case 32: return bwd_bf16<32, Bf16Fmt>(q, k, v, o, dout, lse, delta, dq, dk, dv, nl2, nullptr, s, stream);
        case 64: return bwd_bf16<64, Bf16Fmt>(q, k, v, o, dout, lse, delta, dq, dk, dv, nl2, nullptr, s, stream);
        case 128: return bwd_bf16<128, Bf16Fmt>(q, k, v, o, dout, lse, delta, dq, dk, dv, nl2, ds, s, stream);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_f16_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
                          const float *lse, float *delta, void *dq, void *dk, void *dv, void *extra,
                          int64_t extra_bytes, const AttnShape &s, hipStream_t stream) {
    float *nl2 = static_cast<float *>(extra);
    const int64_t dsb = bf16_ds_bytes(s);
    uint16_t *ds = dsb > 0 && extra_bytes >= nl2_bytes(s) + dsb
                       ? reinterpret_cast<uint16_t *>(static_cast<char *>(extra) + nl2_bytes(s))
                       : nullptr;
    switch (s.d) {
        case 32: return bwd_bf16<32, F16Fmt>(q, k, v, o, dout, lse, delta, dq, dk, dv, nl2, nullptr, s, stream);
        case 64: return bwd_bf16<64, F16Fmt>(q, k, v, o, dout, lse, delta, dq, dk, dv, nl2, nullptr, s, stream);
        case 128: return bwd_bf16<128, F16Fmt>(q, k, v, o, dout, lse, delta, dq, dk, dv, nl2, ds, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
