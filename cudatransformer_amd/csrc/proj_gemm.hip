// MFMA GEMMs of the attention layer's projections (fp32 MFMA v_mfma_f32_32x32x2f32, gfx950).
//
// Replaces the reference's shared-memory-tiled scalar projection kernels
// (attention_qkv_kernels.cu:51-364: getQKVmatrices, qkvBackwardWB, qkvBackward;
// attention_proj_kernels.cu:48-290: attentionProj, projBackwardWB, projBackward).  All six
// products are one kernel family:
//
//     out(m, n) [+]= sum_k A(m, k) B(k, n)   (+ bias(n))
//
// where every operand is a separable 2-D view of memory, element (i, j) at
// base + row_off(i) + col_off(j), with either plain row-major offsets (i * ld, j) or the
// head-split offsets of a [B, H, T, d] tensor seen as a [B*T, H*d] matrix:
//     row_off(r) = ((r / T) * H * T + r % T) * d,   col_off(c) = (c / d) * T * d + c % d.
// So the QKV projection writes Q/K/V in attention layout and the output projection reads the
// attention output in place: no transpose kernels, no extra HBM passes.
//
// Tiling: a workgroup (4 waves, 2 x 2) computes a BM x BN tile of out, BM, BN in {64, 128},
// each wave a (BM/2) x (BN/2) block of 32x32 MFMA tiles, over K in steps of BK.  The tile
// configurations are 128 x 128 x 16, 128 x 64 x 32, 64 x 128 x 32 and 64 x 64 x 64: each
// gives a wave 32 MFMAs (2048 cycles) per K step, so smaller tiles wait on their global
// loads as rarely as the large one.  choose_tile() picks one by a makespan model (rounds of
// 256 workgroups x tile area / measured tile efficiency): the 4096 x 384 products of a d384
// model run 64 x 64, 4096 x 1536 runs 64 x 128, the E = 1024 layer 128 x 128.  Operand tiles are staged global ->
// registers -> LDS (double-buffered, one barrier per step; the next step's global loads are
// in flight during this step's MFMAs).  A K-contiguous operand is stored [row][k] in LDS
// and read as float4 along k; an M/N-contiguous one is stored [k][row] and read per element
// -- each lane (i, h) feeds MFMA (s, t) with k = 8s + 4h + t for both operands, which is a
// valid pairing of the 32x32x2 instruction's two k slots.  Storage may be fp32 or bf16; bf16
// is widened to fp32 on its way into LDS, arithmetic is fp32 throughout.
//
// Weight gradients (K = B*T, small M x N) split K over several workgroups; the partial
// tiles go to a workspace and a second kernel adds them in a fixed order (deterministic,
// no atomics).  Bias gradients are column sums, also two-stage and deterministic.
#include "proj_launch.h"

#include <type_traits>

#include "attn_common.h"
#include "attn_mfma_common.h"

namespace ctattn {
namespace {

constexpr int kThreads = 256;
constexpr int kFillWorkgroups = 256;  // one per CU

template <typename T> __device__ __forceinline__ float load_f(const T *p);
template <> __device__ __forceinline__ float load_f<float>(const float *p) { return *p; }
template <> __device__ __forceinline__ float load_f<uint16_t>(const uint16_t *p) {
    return __uint_as_float(uint32_t(*p) << 16);
}
template <typename T> __device__ __forceinline__ floatx4 load4_f(const T *p);
template <> __device__ __forceinline__ floatx4 load4_f<float>(const float *p) {
    return *reinterpret_cast<const floatx4 *>(p);
}
template <> __device__ __forceinline__ floatx4 load4_f<uint16_t>(const uint16_t *p) {
    typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
    const u16x4 u = *reinterpret_cast<const u16x4 *>(p);
    return floatx4{__uint_as_float(uint32_t(u[0]) << 16), __uint_as_float(uint32_t(u[1]) << 16),
                   __uint_as_float(uint32_t(u[2]) << 16), __uint_as_float(uint32_t(u[3]) << 16)};
}
template <> __device__ __forceinline__ float load_f<f16_t>(const f16_t *p) { return to_f32(*p); }
template <> __device__ __forceinline__ floatx4 load4_f<f16_t>(const f16_t *p) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 u = *reinterpret_cast<const h4 *>(p);
    return floatx4{float(u[0]), float(u[1]), float(u[2]), float(u[3])};
}
template <typename T> __device__ __forceinline__ void store_f(T *p, float x);
template <> __device__ __forceinline__ void store_f<float>(float *p, float x) { *p = x; }
template <> __device__ __forceinline__ void store_f<uint16_t>(uint16_t *p, float x) { *p = f32_to_bf16(x).bits; }
template <> __device__ __forceinline__ void store_f<f16_t>(f16_t *p, float x) { *p = from_f32<f16_t>(x); }

// Loads / stores in the accumulation type: fp64 for fp64 storage, fp32 otherwise.
template <typename T> __device__ __forceinline__ acc_t<T> load_a(const T *p) { return load_f<T>(p); }
template <> __device__ __forceinline__ double load_a<double>(const double *p) { return *p; }
template <typename T> __device__ __forceinline__ void store_a(T *p, acc_t<T> x) { store_f<T>(p, x); }
template <> __device__ __forceinline__ void store_a<double>(double *p, double x) { *p = x; }

// Indices are < 2^31 (checked on the host), so the divisions are 32-bit.
__device__ __forceinline__ int64_t view_row_off(const MatView &v, int i) {
    if (v.kind == kViewLinear) return int64_t(i) * v.ld;
    return (int64_t(i / v.T) * v.H * v.T + i % v.T) * v.d;
}
__device__ __forceinline__ int64_t view_col_off(const MatView &v, int j) {
    if (v.kind == kViewLinear) return j;
    return int64_t(j / v.d) * v.T * v.d + j % v.d;
}

// Loads one operand tile (rows = the operand's M or N index, k = its K index) into registers.
// KC: the operand is K-contiguous in memory (storage rows = tile rows, storage cols = k);
// otherwise storage rows = k and storage cols = tile rows.  VEC elements per load.  The
// tile-row part of each address (with its integer divisions for head-split views) is fixed
// for the whole K loop and computed once in init().
template <typename T, bool KC, int VEC, int ROWS, int BK>
struct TileLoader {
    static constexpr int LOADS = ROWS * BK / VEC / kThreads;  // per thread
    static_assert(LOADS >= 1 && LOADS * VEC * kThreads == ROWS * BK, "tile does not split over the workgroup");
    floatx4 reg[LOADS];
    int64_t rpart[LOADS];  // offset of this load's tile row; -1 when the row is out of range

    __device__ __forceinline__ static void coords(int tid, int i, int &r, int &kk) {
        const int e = (tid + i * kThreads) * VEC;  // element index in the tile, storage-row-major
        if (KC) {  // storage [row][k]: BK k per row
            r = e / BK;
            kk = e % BK;
        } else {  // storage [k][row]: ROWS rows per k
            kk = e / ROWS;
            r = e % ROWS;
        }
    }

    __device__ __forceinline__ void init(const MatView &v, int row0, int nrows, int tid) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            int r, kk;
            coords(tid, i, r, kk);
            rpart[i] = row0 + r < nrows ? (KC ? view_row_off(v, row0 + r) : view_col_off(v, row0 + r)) : -1;
        }
    }

    // Fast path (VEC = 4, K a multiple of BK, every K step inside one head of a head-split
    // K-contiguous view and inside one sequence of a head-split M/N-contiguous one): each
    // lane's vector sits at a fixed byte offset from the tile origin, which moves by a
    // uniform amount per K step, so a load needs no address arithmetic, bounds test or zero
    // fill.  Rows past the matrix are clamped to its last row (vector); their results are
    // never stored.  Offsets are 32-bit; the host checks that they fit.
    uint32_t loff[LOADS];

    __device__ __forceinline__ void init_fast(const MatView &v, int row0, int nrows, int tid) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            int r, kk;
            coords(tid, i, r, kk);
            const int rc = min(row0 + r, nrows - (KC ? 1 : VEC));
            // KC: storage row = tile row, column = k; else storage row = k, column = tile row.
            const int64_t e = KC ? view_row_off(v, rc) - view_row_off(v, row0) + kk
                                 : view_col_off(v, rc) - view_col_off(v, row0) +
                                       int64_t(kk) * (v.kind == kViewLinear ? v.ld : int64_t(v.d));
            loff[i] = uint32_t(e * int64_t(sizeof(T)));
        }
    }

    // The tile origin, element (row0, k0), of the operand in the fast path, kept as a cursor
    // that advances one K step at a time with uniform adds instead of recomputing the view's
    // divisions: within a period (one head of a K-contiguous head-split view, one sequence
    // of an M/N-contiguous one) the k part grows by BK * unit, crossing a period boundary
    // adds `jump` once, and a new K segment restarts at k = 0.
    struct Cursor {
        int64_t row_part;  // elements: the (row0) part of the origin
        int64_t k_part;    // elements: the (k0) part
        int64_t unit, jump;
        int kin, period;   // k0 within the current period; period 0 = none (row-major view)

        __device__ __forceinline__ void init(const MatView &v, int row0, int k0) {
            row_part = KC ? view_row_off(v, row0) : view_col_off(v, row0);
            k_part = KC ? view_col_off(v, k0) : view_row_off(v, k0);
            if (v.kind == kViewLinear) {
                unit = KC ? 1 : v.ld;
                jump = 0;
                period = 0;
                kin = 0;
            } else {
                unit = KC ? 1 : v.d;
                period = KC ? v.d : v.T;
                jump = KC ? int64_t(v.T) * v.d - v.d : (int64_t(v.H) - 1) * v.T * v.d;
                kin = k0 % period;
            }
        }
        __device__ __forceinline__ void step() {
            k_part += BK * unit;
            if (period != 0) {
                kin += BK;
                if (kin == period) {
                    kin = 0;
                    k_part += jump;
                }
            }
        }
        __device__ __forceinline__ void restart() {
            k_part = 0;
            kin = 0;
        }
        __device__ __forceinline__ const T *origin(const void *base) const {
            return static_cast<const T *>(base) + row_part + k_part;
        }
    };

    __device__ __forceinline__ void load_fast(const T *org) {
        const char *o = reinterpret_cast<const char *>(org);
#pragma unroll
        for (int i = 0; i < LOADS; ++i) reg[i] = load4_f<T>(reinterpret_cast<const T *>(o + loff[i]));
    }

    // VEC = 4: KC -> 4 consecutive k of one row; !KC -> 4 consecutive rows of one k.  Callers
    // guarantee every extent is a multiple of 4, so a vector is wholly in or out of range.
    __device__ __forceinline__ void load(const MatView &v, int k0, int kend, int tid) {
        const T *base = static_cast<const T *>(v.p);
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            int r, kk;
            coords(tid, i, r, kk);
            floatx4 x = {0.f, 0.f, 0.f, 0.f};
            if (rpart[i] >= 0 && k0 + kk < kend) {
                const int64_t off = rpart[i] + (KC ? view_col_off(v, k0 + kk) : view_row_off(v, k0 + kk));
                if (VEC == 4) x = load4_f<T>(base + off);
                else x[0] = load_f<T>(base + off);
            }
            reg[i] = x;
        }
    }

    // LDS layouts: KC -> [row][KS] with KS = BK + 4 (float4-aligned; the 16 lanes of a
    // float4 read hit 16 distinct 4-bank groups for BK = 16, 32, 64); !KC -> [k][MS] with
    // MS = ROWS + 4.
    static constexpr int KS = BK + 4;
    static constexpr int MS = ROWS + 4;
    static constexpr int LDS_FLOATS = KC ? ROWS * KS : BK * MS;

    __device__ __forceinline__ void store(float *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int e = (tid + i * kThreads) * VEC;
            if (KC) {
                const int r = e / BK, kk = e % BK;
                if (VEC == 4) *reinterpret_cast<floatx4 *>(lds + r * KS + kk) = reg[i];
                else lds[r * KS + kk] = reg[i][0];
            } else {
                const int kk = e / ROWS, r = e % ROWS;
                if (VEC == 4) *reinterpret_cast<floatx4 *>(lds + kk * MS + r) = reg[i];
                else lds[kk * MS + r] = reg[i][0];
            }
        }
    }

    // Operand values of lane (row rl, half h) for the four MFMAs of k-group s: k = 8s + 4h + t.
    __device__ __forceinline__ static floatx4 fetch(const float *lds, int rl, int s, int h) {
        if (KC) return *reinterpret_cast<const floatx4 *>(lds + rl * KS + 8 * s + 4 * h);
        floatx4 x;
#pragma unroll
        for (int t = 0; t < 4; ++t) x[t] = lds[(8 * s + 4 * h + t) * MS + rl];
        return x;
    }
};

template <typename T, bool A_KC, bool B_KC, int VEC, int BM, int BN, int BK, bool FAST>
__global__ __launch_bounds__(kThreads) void proj_gemm_kernel(GemmParams prm) {
    static_assert(!FAST || VEC == 4, "the fast path uses vector loads");
    using LA = TileLoader<T, A_KC, VEC, BM, BK>;
    using LB = TileLoader<T, B_KC, VEC, BN, BK>;
    constexpr int TM = BM / 64, TN = BN / 64;  // 32x32 MFMA tiles per wave along M and N
    constexpr int WM = BM / 2, WN = BN / 2;    // the wave's block of out
    __shared__ __attribute__((aligned(16))) float a_lds[2][LA::LDS_FLOATS];
    __shared__ __attribute__((aligned(16))) float b_lds[2][LB::LDS_FLOATS];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int wm = wave & 1, wn = wave >> 1;

    const int m0 = blockIdx.x * BM;
    const int n0 = blockIdx.y * BN;
    const int batch = blockIdx.z / prm.splits;
    const int split = blockIdx.z % prm.splits;
    const GemmBatch &bt = prm.batch[batch];

    // Flat list of K steps over the segments: step st -> segment st / nks, k0 = (st % nks) * BK.
    const int nks = (prm.K + BK - 1) / BK;
    const int total = bt.nseg * nks;
    const int per = (total + prm.splits - 1) / prm.splits;
    const int st_begin = split * per;
    const int st_end = min(total, st_begin + per);

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = zero16();

    // Every segment's views share their kind and shape (only the base pointer differs), so
    // the row parts computed from segment 0 hold for all of them.
    LA la;
    LB lb;
    if constexpr (FAST) {
        la.init_fast(bt.a[0], m0, prm.M, tid);
        lb.init_fast(bt.b[0], n0, prm.N, tid);
    } else {
        la.init(bt.a[0], m0, prm.M, tid);
        lb.init(bt.b[0], n0, prm.N, tid);
    }
    // Fast path: cursors at step st_begin; load_step is called for st_begin, st_begin + 1, ...
    // in order and advances them.
    typename LA::Cursor ca{};
    typename LB::Cursor cb{};
    int cur_seg = 0, cur_k0 = 0;
    if constexpr (FAST) {
        cur_seg = st_begin / nks;
        cur_k0 = (st_begin % nks) * BK;
        ca.init(bt.a[0], m0, cur_k0);
        cb.init(bt.b[0], n0, cur_k0);
    }
    auto load_step = [&](int st) {
        if constexpr (FAST) {
            la.load_fast(ca.origin(bt.a[cur_seg].p));
            lb.load_fast(cb.origin(bt.b[cur_seg].p));
            cur_k0 += BK;
            if (cur_k0 == prm.K) {
                cur_k0 = 0;
                ++cur_seg;
                ca.restart();
                cb.restart();
            } else {
                ca.step();
                cb.step();
            }
        } else {
            const int seg = st / nks;
            const int k0 = (st % nks) * BK;
            la.load(bt.a[seg], k0, prm.K, tid);
            lb.load(bt.b[seg], k0, prm.K, tid);
        }
    };

    if (st_begin < st_end) load_step(st_begin);
    for (int st = st_begin; st < st_end; ++st) {
        const int buf = (st - st_begin) & 1;
        la.store(a_lds[buf], tid);
        lb.store(b_lds[buf], tid);
        // One barrier per step: buffer `buf` was last read two steps ago, before the previous
        // step's barrier, so the stores above cannot race with readers.
        __syncthreads();
        if (st + 1 < st_end) load_step(st + 1);
#pragma unroll
        for (int s = 0; s < BK / 8; ++s) {
            floatx4 a4[TM], b4[TN];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) a4[tm] = LA::fetch(a_lds[buf], wm * WM + tm * 32 + col, s, half);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) b4[tn] = LB::fetch(b_lds[buf], wn * WN + tn * 32 + col, s, half);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn)
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[tm][t], b4[tn][t], acc[tm][tn], 0, 0, 0);
        }
    }

    // Epilogue.  acc[tm][tn]: lane (col, half), register r holds out row acc_row(r, half),
    // column col of the 32x32 tile.  The MFMA's A operand is the row index here (A = rows of
    // out), B the column: D[i][j] = sum_k A[i][k] B[k][j].
    if (prm.splits > 1) {
        float *ws = prm.ws + int64_t(blockIdx.z) * prm.M * prm.N;
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int n = n0 + wn * WN + tn * 32 + col;
                if (n >= prm.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * WM + tm * 32 + acc_row(r, half);
                    if (m < prm.M) ws[int64_t(m) * prm.N + n] = acc[tm][tn][r];
                }
            }
        return;
    }
    T *out = static_cast<T *>(bt.out);
    const T *bias = static_cast<const T *>(bt.bias);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const int n = n0 + wn * WN + tn * 32 + col;
        if (n >= prm.N) continue;
        const float bn = bias != nullptr ? load_f<T>(bias + n) : 0.f;
        const int64_t coff = view_col_off(prm.outv, n);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * WM + tm * 32 + acc_row(r, half);
                if (m >= prm.M) continue;
                T *p = out + view_row_off(prm.outv, m) + coff;
                float x = acc[tm][tn][r] + bn;
                if (prm.beta) x += load_f<T>(p);
                store_f<T>(p, x);
            }
        }
    }
}

// out(m, n) [+]= sum_s ws[batch][s][m][n], s in increasing order.
template <typename T>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams prm) {
    const int64_t mn = int64_t(prm.M) * prm.N;
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int batch = blockIdx.y;
    if (idx >= mn) return;
    const int m = int(idx / prm.N), n = int(idx % prm.N);
    const float *ws = prm.ws + int64_t(batch) * prm.splits * mn + idx;
    float x = 0.f;
    for (int s = 0; s < prm.splits; ++s) x += ws[int64_t(s) * mn];
    const GemmBatch &bt = prm.batch[batch];
    T *p = static_cast<T *>(bt.out) + view_row_off(prm.outv, m) + view_col_off(prm.outv, n);
    if (bt.bias != nullptr) x += load_f<T>(static_cast<const T *>(bt.bias) + n);
    if (prm.beta) x += load_f<T>(p);
    store_f<T>(p, x);
}

// Column sums, stage 1: part[rb][c] = sum of rows rb*kColRows .. +kColRows-1 of column c.
// 256 threads = 64 columns x 4 row lanes, each lane 8 rows; the lanes combine in LDS in a
// fixed order.  32-row blocks give 768 workgroups for a 4096 x 384 gradient.  Partial sums
// are in the accumulation type (fp64 for fp64 storage).
constexpr int kColRows = 32;
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void colsum_partial_kernel(MatView g, int R, int C, A *part) {
    __shared__ A red[4][64];
    const int cl = threadIdx.x & 63, rl = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl;
    const int r0 = blockIdx.y * kColRows;
    const T *base = static_cast<const T *>(g.p);
    A s = 0;
    if (c < C) {
        const int64_t coff = view_col_off(g, c);
        const int r1 = min(R, r0 + kColRows);
#pragma unroll
        for (int i = 0; i < kColRows / 4; ++i) {
            const int r = r0 + rl + 4 * i;
            if (r < r1) s += load_a<T>(base + view_row_off(g, r) + coff);
        }
    }
    red[rl][cl] = s;
    __syncthreads();
    if (rl == 0 && c < C) part[int64_t(blockIdx.y) * C + c] = ((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl];
}

// Stage 2: out[c] += sum over row blocks of part[rb][c].  16 columns x 16 lanes per block;
// lane l sums row blocks l, l+16, ... in increasing order, then lane 0 adds the 16 lane sums
// in order (fixed order: deterministic).
template <typename T, typename A = acc_t<T>>
__global__ __launch_bounds__(256) void colsum_final_kernel(const A *part, int nrb, int C, T *out) {
    __shared__ A red[16][17];
    const int cl = threadIdx.x & 15, rl = threadIdx.x >> 4;
    const int c = blockIdx.x * 16 + cl;
    A s = 0;
    if (c < C)
        for (int rb = rl; rb < nrb; rb += 16) s += part[int64_t(rb) * C + c];
    red[rl][cl] = s;
    __syncthreads();
    if (rl == 0 && c < C) {
        A t = 0;
#pragma unroll
        for (int l = 0; l < 16; ++l) t += red[l][cl];
        store_a<T>(out + c, load_a<T>(out + c) + t);
    }
}

// params[i] -= lr * grads[i]  (headers.cu:249-275: sgdUpdateKernel / runSgdUpdate).
template <typename T>
__global__ __launch_bounds__(256) void sgd_kernel(T *params, const T *grads, acc_t<T> lr, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    store_a<T>(params + i, load_a<T>(params + i) - lr * load_a<T>(grads + i));
}

// fp64 GEMM for fp64 storage (the reference's Double classes): the same products and views as
// proj_gemm_kernel, on fp64 FMAs (no K split).  64 x 64 output tile per 256-thread workgroup,
// 4 x 4 outputs per thread, K steps of 16 staged in LDS.
constexpr int kF64Tile = 64, kF64K = 16;
__global__ __launch_bounds__(256) void gemm_f64_kernel(GemmParams prm, int a_kc, int b_kc) {
    __shared__ double as[kF64K][kF64Tile + 1];
    __shared__ double bs[kF64K][kF64Tile + 1];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m0 = blockIdx.x * kF64Tile, n0 = blockIdx.y * kF64Tile;
    const GemmBatch &bt = prm.batch[blockIdx.z];
    double acc[4][4] = {};
    for (int seg = 0; seg < bt.nseg; ++seg) {
        const MatView &va = bt.a[seg], &vb = bt.b[seg];
        const double *pa = static_cast<const double *>(va.p), *pb = static_cast<const double *>(vb.p);
        for (int k0 = 0; k0 < prm.K; k0 += kF64K) {
            // Element e of the 64 x 16 tile: row e % 64, k e / 64.
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const int e = threadIdx.x + 256 * l;
                const int r = e % kF64Tile, kk = e / kF64Tile;
                const int m = m0 + r, n = n0 + r, k = k0 + kk;
                double a = 0.0, b = 0.0;
                if (m < prm.M && k < prm.K)
                    a = pa[a_kc ? view_row_off(va, m) + view_col_off(va, k) : view_row_off(va, k) + view_col_off(va, m)];
                if (n < prm.N && k < prm.K)
                    b = pb[b_kc ? view_row_off(vb, n) + view_col_off(vb, k) : view_row_off(vb, k) + view_col_off(vb, n)];
                as[kk][r] = a;
                bs[kk][r] = b;
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < kF64K; ++kk) {
                double a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = as[kk][ty * 4 + i];
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = bs[kk][tx * 4 + j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
            }
            __syncthreads();
        }
    }
    double *out = static_cast<double *>(bt.out);
    const double *bias = static_cast<const double *>(bt.bias);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= prm.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n >= prm.N) continue;
            double *p = out + view_row_off(prm.outv, m) + view_col_off(prm.outv, n);
            double x = acc[i][j] + (bias != nullptr ? bias[n] : 0.0);
            if (prm.beta) x += *p;
            *p = x;
        }
    }
}

// Whether a view can take the fast load path as a K-contiguous (kc) or M/N-contiguous
// operand of a tile with at most 128 rows: the lane offsets must be affine in the K step
// (a head-split view needs every K step inside one head, kc: d % BK == 0, or inside one
// sequence, T % BK == 0) and the largest one must fit 31 bits.
bool fast_view_ok(const MatView &v, bool kc, int bk, int elem_bytes) {
    int64_t max_elems;
    if (v.kind == kViewLinear) {
        max_elems = kc ? 127 * v.ld + bk : int64_t(bk) * v.ld + 128;
    } else {
        if (kc ? v.d % bk != 0 : v.T % bk != 0) return false;
        const int64_t htd = int64_t(v.H) * v.T * v.d;
        // 128 consecutive rows (b, t) span at most 127 / T + 2 batch slices; 128 columns
        // (h, dd) at most 127 / d + 2 heads.
        max_elems = kc ? (127 / v.T + 2) * htd + bk : (127 / v.d + 2) * int64_t(v.T) * v.d + int64_t(bk) * v.d;
    }
    return max_elems * elem_bytes < (int64_t(1) << 31);
}

// The fast load path applies when loads are vectors, K is a multiple of the K step (no K
// tail) and every operand view qualifies.
bool fast_path_ok(const GemmParams &prm, int nbatch, bool vec4, int bk, bool a_kc, bool b_kc, int elem_bytes) {
    if (!vec4 || prm.K % bk != 0) return false;
    for (int z = 0; z < nbatch; ++z)
        for (int sg = 0; sg < prm.batch[z].nseg; ++sg)
            if (!fast_view_ok(prm.batch[z].a[sg], a_kc, bk, elem_bytes) ||
                !fast_view_ok(prm.batch[z].b[sg], b_kc, bk, elem_bytes))
                return false;
    return true;
}

template <typename T, bool A_KC, bool B_KC, int BM, int BN>
void launch_tile(const GemmParams &prm, int nbatch, bool vec4, hipStream_t stream) {
    constexpr int BK = 16 * (128 / BM) * (128 / BN);  // 32 MFMAs per wave per K step
    const dim3 grid(unsigned((prm.M + BM - 1) / BM), unsigned((prm.N + BN - 1) / BN), unsigned(nbatch * prm.splits));
    if (fast_path_ok(prm, nbatch, vec4, BK, A_KC, B_KC, int(sizeof(T)))) {
        hipLaunchKernelGGL((proj_gemm_kernel<T, A_KC, B_KC, 4, BM, BN, BK, true>), grid, dim3(kThreads), 0, stream, prm);
        return;
    }
    if (vec4)
        hipLaunchKernelGGL((proj_gemm_kernel<T, A_KC, B_KC, 4, BM, BN, BK, false>), grid, dim3(kThreads), 0, stream, prm);
    else
        hipLaunchKernelGGL((proj_gemm_kernel<T, A_KC, B_KC, 1, BM, BN, BK, false>), grid, dim3(kThreads), 0, stream, prm);
}

// Workgroups of a BM x BN tiling of the launch.
int64_t tile_workgroups(const GemmParams &prm, int nbatch, int bm, int bn) {
    return int64_t((prm.M + bm - 1) / bm) * ((prm.N + bn - 1) / bn) * nbatch * prm.splits;
}

// Tile choice by a makespan model: the CUs take workgroups in rounds of kFillWorkgroups, a
// round costs the tile's area over its relative MFMA efficiency (measured on MI355X at
// 8192 x 1024 x 1024: 64 x 128 and 128 x 64 tiles run at 0.963 and 0.955 of 128 x 128, 64 x 64
// at 0.915).  Ties keep the larger tile.  Returns 0: 128 x 128, 1: 64 x 128, 2: 128 x 64,
// 3: 64 x 64.  At the 4096 x {384, 1152, 1536} products this picks within 8% of the fastest
// tile measured, where "largest tile that fills the CUs" lost up to 27%.
int choose_tile(const GemmParams &prm, int nbatch) {
    struct Cand {
        int bm, bn;
        double eff;
    };
    static constexpr Cand cands[4] = {{128, 128, 1.0}, {64, 128, 0.963}, {128, 64, 0.955}, {64, 64, 0.915}};
    int best = 0;
    double best_cost = 0.0;
    for (int c = 0; c < 4; ++c) {
        const int64_t rounds = (tile_workgroups(prm, nbatch, cands[c].bm, cands[c].bn) + kFillWorkgroups - 1) /
                               kFillWorkgroups;
        const double cost = double(rounds) * cands[c].bm * cands[c].bn / cands[c].eff;
        if (c == 0 || cost < best_cost * 0.999) {
            best = c;
            best_cost = cost;
        }
    }
    return best;
}

template <typename T, bool A_KC, bool B_KC>
hipError_t launch_gemm_t(const GemmParams &prm, int nbatch, bool vec4, hipStream_t stream) {
    switch (choose_tile(prm, nbatch)) {
        case 0: launch_tile<T, A_KC, B_KC, 128, 128>(prm, nbatch, vec4, stream); break;
        case 1: launch_tile<T, A_KC, B_KC, 64, 128>(prm, nbatch, vec4, stream); break;
        case 2: launch_tile<T, A_KC, B_KC, 128, 64>(prm, nbatch, vec4, stream); break;
        default: launch_tile<T, A_KC, B_KC, 64, 64>(prm, nbatch, vec4, stream); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || prm.splits == 1) return e;
    const int64_t mn = int64_t(prm.M) * prm.N;
    hipLaunchKernelGGL(splitk_reduce_kernel<T>, dim3(unsigned((mn + 255) / 256), unsigned(nbatch)), dim3(256), 0,
                       stream, prm);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_gemm_dt(const GemmParams &prm, int nbatch, bool a_kc, bool b_kc, bool vec4,
                          hipStream_t stream) {
    if (a_kc && b_kc) return launch_gemm_t<T, true, true>(prm, nbatch, vec4, stream);
    if (a_kc && !b_kc) return launch_gemm_t<T, true, false>(prm, nbatch, vec4, stream);
    if (!a_kc && !b_kc) return launch_gemm_t<T, false, false>(prm, nbatch, vec4, stream);
    return launch_gemm_t<T, false, true>(prm, nbatch, vec4, stream);
}

}  // namespace

int gemm_tile_count(int64_t M, int64_t N) { return int(((M + 127) / 128) * ((N + 127) / 128)); }
int gemm_k_steps(int64_t K) { return int((K + 15) / 16); }

// Storage type of a dtype code: 0 fp32, 1 bf16 (raw 16-bit), 2 fp16, 3 fp64.
template <typename F>
hipError_t by_storage(int dtype, F &&f) {
    switch (dtype) {
        case 0: return f(static_cast<float *>(nullptr));
        case 1: return f(static_cast<uint16_t *>(nullptr));
        case 2: return f(static_cast<f16_t *>(nullptr));
        default: return f(static_cast<double *>(nullptr));
    }
}

hipError_t launch_proj_gemm(int dtype, const GemmParams &prm, int nbatch, bool a_kc, bool b_kc,
                            bool vec4, hipStream_t stream) {
    if (prm.M <= 0 || prm.N <= 0 || nbatch <= 0) return hipSuccess;
    if (dtype == 3) {
        if (prm.splits != 1) return hipErrorInvalidValue;  // the fp64 GEMM does not split K
        if ((prm.N + kF64Tile - 1) / kF64Tile > 65535) return hipErrorInvalidValue;  // grid.y limit
        const dim3 grid(unsigned((prm.M + kF64Tile - 1) / kF64Tile), unsigned((prm.N + kF64Tile - 1) / kF64Tile),
                        unsigned(nbatch));
        hipLaunchKernelGGL(gemm_f64_kernel, grid, dim3(256), 0, stream, prm, int(a_kc), int(b_kc));
        return hipGetLastError();
    }
    return by_storage(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        if constexpr (std::is_same_v<T, double>) return hipErrorInvalidValue;
        else return launch_gemm_dt<T>(prm, nbatch, a_kc, b_kc, vec4, stream);
    });
}

int64_t colsum_workspace_bytes(int dtype, int64_t R, int64_t C) {
    return ((R + kColRows - 1) / kColRows) * C * (dtype == 3 ? 8 : 4);
}

hipError_t launch_colsum_add(int dtype, const MatView &g, int R, int C, void *out, void *ws,
                             hipStream_t stream) {
    if (R <= 0 || C <= 0) return hipSuccess;
    const int nrb = (R + kColRows - 1) / kColRows;
    if (nrb > 65535) return hipErrorInvalidValue;  // grid.y limit: at most 2^21 - 32 rows
    const dim3 grid1(unsigned((C + 63) / 64), unsigned(nrb));
    const dim3 grid2(unsigned((C + 15) / 16));
    return by_storage(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        using A = acc_t<T>;
        hipLaunchKernelGGL(colsum_partial_kernel<T>, grid1, dim3(256), 0, stream, g, R, C, static_cast<A *>(ws));
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(colsum_final_kernel<T>, grid2, dim3(256), 0, stream, static_cast<const A *>(ws), nrb, C,
                           static_cast<T *>(out));
        return hipGetLastError();
    });
}

hipError_t launch_sgd(int dtype, void *params, const void *grads, double lr, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const dim3 grid(unsigned((n + 255) / 256));
    return by_storage(dtype, [&](auto *tag) {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL(sgd_kernel<T>, grid, dim3(256), 0, stream, static_cast<T *>(params),
                           static_cast<const T *>(grads), acc_t<T>(lr), n);
        return hipGetLastError();
    });
}

}  // namespace ctattn
