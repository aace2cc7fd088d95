// fp64 flash attention on v_mfma_f64_16x16x4f64 (the reference's Double classes compute in
// double, ComputeType<double>, headers.cu:47-48): forward, and a two-kernel atomic-free
// backward (dK / dV key-major, dQ query-major), all arithmetic in fp64, LSE and delta fp64.
// Same results as the generic fp64 kernels to rounding; d in {32, 64, 128}.
//
// 16x16x4 operand layout (lane l, c = l % 16, g = l / 16), measured on gfx950:
//   A[i][k] comes from lane (i, k): A row i = c, k = g;  B[k][j] from lane (j, k): col j = c;
//   accumulator register r of lane l holds D[i = 4 r + g][j = c].
// With the contraction order "k-step s covers index 4 s + g", accumulator register s of a
// tile is directly the operand a lane supplies in k-step s, so P / dS never move between
// lanes:
//   forward      S^T = K Q^T (keys x queries), O^T += V^T P^T
//   dK / dV      S = Q K^T (queries x keys),   dV^T += dO^T P,  dK^T += Q^T dS
//   dQ           S^T = K Q^T,                 dQ += dS K      (A = dS from S^T registers)
// Operand tiles come from LDS rows padded to D + 4 doubles (16 rows x 4 lane groups of one
// operand read fall in distinct bank pairs, the 2-cycle minimum of a 64 x 8-byte read).
// Global -> register -> LDS staging, double-buffered, one barrier per block.
#include "attn_common.h"
#include "attn_launch.h"

#include <math.h>

namespace ctattn {
namespace {

typedef double doublex4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ doublex4 mfma_f64(double a, double b, doublex4 c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ doublex4 zero4() { return doublex4{0.0, 0.0, 0.0, 0.0}; }

constexpr double kLog2eD = 1.4426950408889634073599;
constexpr double kLn2D = 0.6931471805599453094172;
constexpr double kRescaleF64 = 8.0;  // lazy rescale threshold (log2 units), as the fp32 kernel

// Copies `rows` rows of a [T][D] matrix (rows past T re-read row T - 1) into a padded LDS
// tile through registers: thread t owns the 16-byte pairs t, t + 256, ... of the tile.
template <int D, int ROWS>
struct Stage {
    static constexpr int PAIRS = ROWS * D / 2;
    static constexpr int PER = (PAIRS + 255) / 256;
    double2 reg[PER];
    __device__ __forceinline__ void load(const double *src, int r0, int T, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int p = tid + 256 * i;
            if (PAIRS % 256 == 0 || p < PAIRS) {
                const int r = p / (D / 2), c = 2 * (p % (D / 2));
                reg[i] = *reinterpret_cast<const double2 *>(src + int64_t(min(r0 + r, T - 1)) * D + c);
            }
        }
    }
    __device__ __forceinline__ void store(double *tile, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int p = tid + 256 * i;
            if (PAIRS % 256 == 0 || p < PAIRS) {
                const int r = p / (D / 2), c = 2 * (p % (D / 2));
                *reinterpret_cast<double2 *>(tile + r * (D + 4) + c) = reg[i];
            }
        }
    }
};

// ---------------------------------------------------------------------------------------
// Forward: a workgroup of 4 waves owns 4 * 16 * QT query rows (wave w: QT tiles of 16),
// K / V stream through LDS in BN-key blocks.
// ---------------------------------------------------------------------------------------
template <int D>
struct F64Fwd {
    // Measured per d (B8 H12 T1024 causal): d = 64 runs best with 2 query tiles and 32-key
    // blocks at 2 waves / SIMD; d = 32 with 1 tile and 16-key blocks at 4 waves / SIMD
    // (187 vs 231 us); d = 128 is bounded by registers to 1 tile and 16 keys.
    static constexpr int QT = D == 64 ? 2 : 1;   // 16-query tiles per wave
    static constexpr int BM = 64 * QT;           // query rows per workgroup
    static constexpr int BN = D == 64 ? 32 : 16;
    static constexpr int WAVES = D == 32 ? 4 : 2;  // waves per SIMD
    static constexpr int KT = BN / 16;
    static constexpr int DT = D / 16;
    static constexpr int KS = D / 4;             // k-steps over d
    static constexpr int LD = D + 4;             // padded LDS row (doubles)
    static constexpr int TILE = BN * LD;
};

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(F64Fwd<D>::WAVES, F64Fwd<D>::WAVES))) void fwd_f64_mfma_kernel(
    const double *__restrict__ q, const double *__restrict__ k, const double *__restrict__ v, double *__restrict__ o,
    double *__restrict__ lse, int T, int BH, int causal, double c) {
    using C = F64Fwd<D>;
    __shared__ __attribute__((aligned(16))) double smem[4 * C::TILE];  // buffer b: K at 2 b TILE, V at 2 b TILE + TILE
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cl = lane & 15, g = lane >> 4;
    const int nqb = (T + C::BM - 1) / C::BM;
    const int bh = blockIdx.x % BH;
    const int qblk = causal ? (nqb - 1 - int(blockIdx.x) / BH) : int(blockIdx.x) / BH;  // causal: longest first
    const int64_t base = int64_t(bh) * T * D;
    const int q0 = qblk * C::BM;
    const int wq0 = q0 + wave * 16 * C::QT;  // first query row of this wave
    const int wq1 = wq0 + 16 * C::QT - 1;

    // Q^T as B operand: lane (c, g) supplies Q[query][4 s + g] in k-step s.
    double qreg[C::QT][C::KS];
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
        const int row = min(wq0 + qt * 16 + cl, T - 1);
#pragma unroll
        for (int s = 0; s < C::KS; ++s) qreg[qt][s] = q[base + int64_t(row) * D + 4 * s + g];
    }
    doublex4 oacc[C::DT][C::QT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt) oacc[dt][qt] = zero4();
    double m_run[C::QT], l_run[C::QT];
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
        m_run[qt] = -INFINITY;
        l_run[qt] = 0.0;
    }

    const int kend = causal ? min(T, q0 + C::BM) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;
    Stage<D, C::BN> sk, sv;
    sk.load(k + base, 0, T, tid);
    sv.load(v + base, 0, T, tid);
    sk.store(smem, tid);
    sv.store(smem + C::TILE, tid);
    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        __syncthreads();  // buffer `buf` is written; every wave is done with buf ^ 1
        if (kb + 1 < nkb) {
            sk.load(k + base, (kb + 1) * C::BN, T, tid);
            sv.load(v + base, (kb + 1) * C::BN, T, tid);
        }
        const int j0 = kb * C::BN;
        const double *kt_lds = smem + 2 * buf * C::TILE;
        const double *vt_lds = kt_lds + C::TILE;
        if (!causal || j0 <= wq1) {
            // S^T = K Q^T per 16-key tile and query tile.
            doublex4 sacc[C::KT][C::QT];
            bool act[C::KT];
#pragma unroll
            for (int kt = 0; kt < C::KT; ++kt) {
                act[kt] = j0 + 16 * kt < T && (!causal || j0 + 16 * kt <= wq1);
#pragma unroll
                for (int qt = 0; qt < C::QT; ++qt) sacc[kt][qt] = zero4();
                if (!act[kt]) continue;
#pragma unroll
                for (int s = 0; s < C::KS; ++s) {
                    const double a = kt_lds[(16 * kt + cl) * C::LD + 4 * s + g];
#pragma unroll
                    for (int qt = 0; qt < C::QT; ++qt) sacc[kt][qt] = mfma_f64(a, qreg[qt][s], sacc[kt][qt]);
                }
            }
            // Masks and the online softmax: lane (c, g) register r = key j0 + 16 kt + 4 r + g
            // of query wq0 + 16 qt + c.
#pragma unroll
            for (int qt = 0; qt < C::QT; ++qt) {
                const int row = wq0 + 16 * qt + cl;
                double mloc = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < C::KT; ++kt) {
                    if (!act[kt]) continue;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = j0 + 16 * kt + 4 * r + g;
                        double s = sacc[kt][qt][r];
                        s = (key >= T || (causal && key > row)) ? -INFINITY : s;
                        sacc[kt][qt][r] = s;
                        mloc = fmax(mloc, s);
                    }
                }
                mloc = fmax(mloc, __shfl_xor(mloc, 16, 64));
                mloc = fmax(mloc, __shfl_xor(mloc, 32, 64)) * c;
                if (__any(mloc > m_run[qt] + kRescaleF64)) {
                    const double m_new = fmax(m_run[qt], mloc);
                    const double resc = m_run[qt] == -INFINITY ? 0.0 : exp2(m_run[qt] - m_new);
                    m_run[qt] = m_new;
                    l_run[qt] *= resc;
#pragma unroll
                    for (int dt = 0; dt < C::DT; ++dt) oacc[dt][qt] *= resc;
                }
                double psum = 0.0;
#pragma unroll
                for (int kt = 0; kt < C::KT; ++kt) {
                    if (!act[kt]) continue;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const double s = sacc[kt][qt][r];
                        const double p = s == -INFINITY ? 0.0 : exp2(fma(s, c, -m_run[qt]));
                        sacc[kt][qt][r] = p;
                        psum += p;
                    }
                }
                l_run[qt] += psum;
            }
            // O^T += V^T P^T: k-step s of key tile kt covers keys 16 kt + 4 s + g.
#pragma unroll
            for (int kt = 0; kt < C::KT; ++kt) {
                if (!act[kt]) continue;
#pragma unroll
                for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const double a = vt_lds[(16 * kt + 4 * s + g) * C::LD + 16 * dt + cl];
#pragma unroll
                        for (int qt = 0; qt < C::QT; ++qt) oacc[dt][qt] = mfma_f64(a, sacc[kt][qt][s], oacc[dt][qt]);
                    }
            }
        }
        if (kb + 1 < nkb) {
            sk.store(smem + 2 * (buf ^ 1) * C::TILE, tid);
            sv.store(smem + 2 * (buf ^ 1) * C::TILE + C::TILE, tid);
        }
    }
    // O^T register r of lane (c, g): d = 16 dt + 4 r + g of query wq0 + 16 qt + c.
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
        double lt = l_run[qt] + __shfl_xor(l_run[qt], 16, 64);
        lt += __shfl_xor(lt, 32, 64);
        const int row = wq0 + 16 * qt + cl;
        if (row < T) {
            const double inv = 1.0 / lt;
            double *orow = o + base + int64_t(row) * D;
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) orow[16 * dt + 4 * r + g] = oacc[dt][qt][r] * inv;
            if (lse != nullptr && g == 0) lse[int64_t(bh) * T + row] = (m_run[qt] + log2(lt)) * kLn2D;
        }
    }
}

// Waves per SIMD of the backward kernels: d = 128 tiles take > 80 KiB of LDS (one workgroup
// per CU); at d = 32 the dQ kernel fits four workgroups in registers and LDS, the dK / dV
// kernel three (four would spill); at d = 64 the dQ kernel with 16-key blocks fits three
// (1.005 against 1.077 ms for the c3d backward), while the dK / dV kernel stays at two (at
// three it spills 50 registers).
template <int D, bool KV>
struct F64BwdWaves {
    static constexpr int value = D == 128 ? 1 : D == 32 ? (KV ? 3 : 4) : (KV ? 2 : 3);
};

// ---------------------------------------------------------------------------------------
// Backward dK / dV (key-major): a workgroup of 4 waves owns 64 keys (wave w: keys 16 w ..),
// keeps K and V of its keys as B operands in registers and walks 32-query blocks.
// ---------------------------------------------------------------------------------------
template <int D>
struct F64Kv {
    static constexpr int BN = 64;  // keys per workgroup
    static constexpr int BM = 32;  // queries per block
    static constexpr int QT = BM / 16;
    static constexpr int DT = D / 16;
    static constexpr int KS = D / 4;
    static constexpr int LD = D + 4;
    static constexpr int TILE = BM * LD;  // Q (or dO) tile
};

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(F64BwdWaves<D, true>::value, F64BwdWaves<D, true>::value))) void bwd_f64_dkdv_kernel(
    const double *__restrict__ q, const double *__restrict__ k, const double *__restrict__ v,
    const double *__restrict__ dout, const double *__restrict__ lse, const double *__restrict__ delta,
    double *__restrict__ dk, double *__restrict__ dv, int T, int BH, int causal, double c, double inv_sqrt_d) {
    using C = F64Kv<D>;
    __shared__ __attribute__((aligned(16))) double smem[4 * C::TILE + 4 * C::BM];  // buffer b: Q, dO tiles; then nl2 / delta
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cl = lane & 15, g = lane >> 4;
    const int bh = blockIdx.x % BH;
    const int k0 = (int(blockIdx.x) / BH) * C::BN;  // causal: key block 0 (most queries) first
    const int64_t base = int64_t(bh) * T * D;
    const int64_t rbase = int64_t(bh) * T;
    const int wk0 = k0 + 16 * wave;
    const int key = wk0 + cl;

    // K^T and V^T as B operands: lane (c, g) supplies K[key][4 s + g] in k-step s.
    double kreg[C::KS], vreg[C::KS];
    {
        const int kr = min(key, T - 1);
#pragma unroll
        for (int s = 0; s < C::KS; ++s) {
            kreg[s] = k[base + int64_t(kr) * D + 4 * s + g];
            vreg[s] = v[base + int64_t(kr) * D + 4 * s + g];
        }
    }
    doublex4 dk_acc[C::DT], dv_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
        dk_acc[dt] = zero4();
        dv_acc[dt] = zero4();
    }

    const int nqb = (T + C::BM - 1) / C::BM;
    const int qb_first = causal ? k0 / C::BM : 0;
    double *stat = smem + 4 * C::TILE;  // [buf][2][BM]: nl2 then delta
    Stage<D, C::BM> sq, sd;
    auto load_stats = [&](int r0, int buf) {
        if (tid < 2 * C::BM) {
            const int i = tid % C::BM, r = min(r0 + i, T - 1);
            stat[buf * 2 * C::BM + tid] = tid < C::BM ? -lse[rbase + r] * kLog2eD : delta[rbase + r];
        }
    };
    if (qb_first < nqb) {
        sq.load(q + base, qb_first * C::BM, T, tid);
        sd.load(dout + base, qb_first * C::BM, T, tid);
        sq.store(smem, tid);
        sd.store(smem + C::TILE, tid);
        load_stats(qb_first * C::BM, 0);
    }
    for (int qb = qb_first; qb < nqb; ++qb) {
        const int buf = (qb - qb_first) & 1;
        __syncthreads();
        if (qb + 1 < nqb) {
            sq.load(q + base, (qb + 1) * C::BM, T, tid);
            sd.load(dout + base, (qb + 1) * C::BM, T, tid);
        }
        const int r0 = qb * C::BM;
        const double *qt_lds = smem + 2 * buf * C::TILE;
        const double *dt_lds = qt_lds + C::TILE;
        const double *nl2 = stat + buf * 2 * C::BM;
        const double *dl = nl2 + C::BM;
        if (wk0 < T && (!causal || wk0 <= r0 + C::BM - 1)) {
#pragma unroll
            for (int qt = 0; qt < C::QT; ++qt) {
                const int rq0 = r0 + 16 * qt;
                if (rq0 >= T || (causal && wk0 > rq0 + 15)) continue;
                // S = Q K^T and dP = dO V^T: lane (c, g) register r = query rq0 + 4 r + g, key `key`.
                doublex4 s4 = zero4(), dp4 = zero4();
#pragma unroll
                for (int s = 0; s < C::KS; ++s) {
                    const double aq = qt_lds[(16 * qt + cl) * C::LD + 4 * s + g];
                    const double ad = dt_lds[(16 * qt + cl) * C::LD + 4 * s + g];
                    s4 = mfma_f64(aq, kreg[s], s4);
                    dp4 = mfma_f64(ad, vreg[s], dp4);
                }
                double p[4], ds[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int qi = 16 * qt + 4 * r + g, row = r0 + qi;
                    const bool ok = row < T && key < T && (!causal || key <= row);
                    p[r] = ok ? exp2(fma(s4[r], c, nl2[qi])) : 0.0;
                    ds[r] = p[r] * (dp4[r] - dl[qi]);
                }
                // dV^T += dO^T P, dK^T += Q^T dS: k-step s covers queries rq0 + 4 s + g.
#pragma unroll
                for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const int qi = 16 * qt + 4 * s + g;
                        const double ado = dt_lds[qi * C::LD + 16 * dt + cl];
                        const double aq = qt_lds[qi * C::LD + 16 * dt + cl];
                        dv_acc[dt] = mfma_f64(ado, p[s], dv_acc[dt]);
                        dk_acc[dt] = mfma_f64(aq, ds[s], dk_acc[dt]);
                    }
            }
        }
        if (qb + 1 < nqb) {
            sq.store(smem + 2 * (buf ^ 1) * C::TILE, tid);
            sd.store(smem + 2 * (buf ^ 1) * C::TILE + C::TILE, tid);
            load_stats((qb + 1) * C::BM, buf ^ 1);
        }
    }
    // dK^T / dV^T register r of lane (c, g): d = 16 dt + 4 r + g of key `key`.
    if (key < T) {
        double *dkr = dk + base + int64_t(key) * D;
        double *dvr = dv + base + int64_t(key) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                dkr[16 * dt + 4 * r + g] = dk_acc[dt][r] * inv_sqrt_d;
                dvr[16 * dt + 4 * r + g] = dv_acc[dt][r];
            }
    }
}

// ---------------------------------------------------------------------------------------
// Backward dQ (query-major): a workgroup of 4 waves owns 64 queries (wave w: 16), keeps Q and
// dO of its queries as B operands and walks 32-key blocks.
// ---------------------------------------------------------------------------------------
template <int D>
struct F64Dq {
    static constexpr int BM = 64;
    static constexpr int BN = D == 64 ? 16 : 32;  // d = 64: 16-key blocks, 3 waves / SIMD
    static constexpr int KT = BN / 16;
    static constexpr int DT = D / 16;
    static constexpr int KS = D / 4;
    static constexpr int LD = D + 4;
    static constexpr int TILE = BN * LD;
};

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(F64BwdWaves<D, false>::value, F64BwdWaves<D, false>::value))) void bwd_f64_dq_kernel(
    const double *__restrict__ q, const double *__restrict__ k, const double *__restrict__ v,
    const double *__restrict__ dout, const double *__restrict__ lse, const double *__restrict__ delta,
    double *__restrict__ dq, int T, int BH, int causal, double c, double inv_sqrt_d) {
    using C = F64Dq<D>;
    __shared__ __attribute__((aligned(16))) double smem[4 * C::TILE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cl = lane & 15, g = lane >> 4;
    const int nqb = (T + C::BM - 1) / C::BM;
    const int bh = blockIdx.x % BH;
    const int qblk = causal ? (nqb - 1 - int(blockIdx.x) / BH) : int(blockIdx.x) / BH;
    const int64_t base = int64_t(bh) * T * D;
    const int64_t rbase = int64_t(bh) * T;
    const int q0 = qblk * C::BM;
    const int wq0 = q0 + 16 * wave;
    const int row = wq0 + cl;
    const int rr = min(row, T - 1);

    double qreg[C::KS], dreg[C::KS];
#pragma unroll
    for (int s = 0; s < C::KS; ++s) {
        qreg[s] = q[base + int64_t(rr) * D + 4 * s + g];
        dreg[s] = dout[base + int64_t(rr) * D + 4 * s + g];
    }
    const double nl2 = -lse[rbase + rr] * kLog2eD;
    const double dl = delta[rbase + rr];
    doublex4 dq_acc[C::DT];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) dq_acc[dt] = zero4();

    const int kend = causal ? min(T, q0 + C::BM) : T;
    const int nkb = (kend + C::BN - 1) / C::BN;
    Stage<D, C::BN> sk, sv;
    sk.load(k + base, 0, T, tid);
    sv.load(v + base, 0, T, tid);
    sk.store(smem, tid);
    sv.store(smem + C::TILE, tid);
    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        __syncthreads();
        if (kb + 1 < nkb) {
            sk.load(k + base, (kb + 1) * C::BN, T, tid);
            sv.load(v + base, (kb + 1) * C::BN, T, tid);
        }
        const int j0 = kb * C::BN;
        const double *kt_lds = smem + 2 * buf * C::TILE;
        const double *vt_lds = kt_lds + C::TILE;
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
            const int tk0 = j0 + 16 * kt;
            if (tk0 >= T || (causal && tk0 > wq0 + 15)) continue;
            // S^T = K Q^T, dP^T = V dO^T: lane (c, g) register r = key tk0 + 4 r + g, query `row`.
            doublex4 s4 = zero4(), dp4 = zero4();
#pragma unroll
            for (int s = 0; s < C::KS; ++s) {
                const double ak = kt_lds[(16 * kt + cl) * C::LD + 4 * s + g];
                const double av = vt_lds[(16 * kt + cl) * C::LD + 4 * s + g];
                s4 = mfma_f64(ak, qreg[s], s4);
                dp4 = mfma_f64(av, dreg[s], dp4);
            }
            double ds[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = tk0 + 4 * r + g;
                const bool ok = key < T && row < T && (!causal || key <= row);
                const double p = ok ? exp2(fma(s4[r], c, nl2)) : 0.0;
                ds[r] = p * (dp4[r] - dl);
            }
            // dQ += dS K: A = dS[query c][key tk0 + 4 s + g] is register s; B = K rows.
#pragma unroll
            for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const double bk = kt_lds[(16 * kt + 4 * s + g) * C::LD + 16 * dt + cl];
                    dq_acc[dt] = mfma_f64(ds[s], bk, dq_acc[dt]);
                }
        }
        if (kb + 1 < nkb) {
            sk.store(smem + 2 * (buf ^ 1) * C::TILE, tid);
            sv.store(smem + 2 * (buf ^ 1) * C::TILE + C::TILE, tid);
        }
    }
    // dQ register r of lane (c, g): query wq0 + 4 r + g, d = 16 dt + c.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qr = wq0 + 4 * r + g;
        if (qr >= T) continue;
        double *p = dq + base + int64_t(qr) * D;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) p[16 * dt + cl] = dq_acc[dt][r] * inv_sqrt_d;
    }
}

template <int D>
hipError_t fwd_f64(const void *q, const void *k, const void *v, void *o, void *lse, const AttnShape &s,
                   hipStream_t stream) {
    using C = F64Fwd<D>;
    const int64_t blocks = ((s.T + C::BM - 1) / C::BM) * s.bh();
    if (!grid_fits(blocks, 256) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fwd_f64_mfma_kernel<D>, dim3(unsigned(blocks)), dim3(256), 0, stream,
                       static_cast<const double *>(q), static_cast<const double *>(k),
                       static_cast<const double *>(v), static_cast<double *>(o), static_cast<double *>(lse),
                       int(s.T), int(s.bh()), int(s.causal), kLog2eD / sqrt(double(s.scale_dim())));
    return hipGetLastError();
}

template <int D>
hipError_t bwd_f64(const void *q, const void *k, const void *v, const void *o, const void *dout, const void *lse,
                   void *delta, void *dq, void *dk, void *dv, const AttnShape &s, hipStream_t stream) {
    const int64_t kv_blocks = ((s.T + F64Kv<D>::BN - 1) / F64Kv<D>::BN) * s.bh();
    const int64_t q_blocks = ((s.T + F64Dq<D>::BM - 1) / F64Dq<D>::BM) * s.bh();
    if (!grid_fits(kv_blocks, 256) || !grid_fits(q_blocks, 256) || s.T > 2147483647 / D) return hipErrorInvalidValue;
    hipError_t e = launch_bwd_preprocess(3, o, dout, delta, s, stream);  // delta = rowsum(dO * O), fp64
    if (e != hipSuccess) return e;
    const double c = kLog2eD / sqrt(double(s.scale_dim())), inv_sqrt_d = 1.0 / sqrt(double(s.scale_dim()));
    auto cd = [](const void *p) { return static_cast<const double *>(p); };
    hipLaunchKernelGGL(bwd_f64_dkdv_kernel<D>, dim3(unsigned(kv_blocks)), dim3(256), 0, stream, cd(q), cd(k), cd(v),
                       cd(dout), cd(lse), cd(delta), static_cast<double *>(dk), static_cast<double *>(dv), int(s.T),
                       int(s.bh()), int(s.causal), c, inv_sqrt_d);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(bwd_f64_dq_kernel<D>, dim3(unsigned(q_blocks)), dim3(256), 0, stream, cd(q), cd(k), cd(v),
                       cd(dout), cd(lse), cd(delta), static_cast<double *>(dq), int(s.T), int(s.bh()),
                       int(s.causal), c, inv_sqrt_d);
    return hipGetLastError();
}

}  // namespace

bool f64_mfma_supported(int64_t d) { return d == 32 || d == 64 || d == 128; }

hipError_t launch_f64_fwd(const void *q, const void *k, const void *v, void *o, void *lse, const AttnShape &s,
                          hipStream_t stream) {
    switch (s.d) {
        case 32: return fwd_f64<32>(q, k, v, o, lse, s, stream);
        case 64: return fwd_f64<64>(q, k, v, o, lse, s, stream);
        case 128: return fwd_f64<128>(q, k, v, o, lse, s, stream);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_f64_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
                          const void *lse, void *delta, void *dq, void *dk, void *dv, const AttnShape &s,
                          hipStream_t stream) {
    switch (s.d) {
        case 32: return bwd_f64<32>(q, k, v, o, dout, lse, delta, dq, dk, dv, s, stream);
        case 64: return bwd_f64<64>(q, k, v, o, dout, lse, delta, dq, dk, dv, s, stream);
        case 128: return bwd_f64<128>(q, k, v, o, dout, lse, delta, dq, dk, dv, s, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ctattn
