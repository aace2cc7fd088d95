// Plain row-major fp32 GEMMs on v_mfma_f32_32x32x2f32 (gfx950): the linear layers' three
// products and the Tensor matmul.
//
// Replaces the reference's tiled linear kernels (linear_kernels.cu:36-241: the forward
// y = x W^T + b, the input gradient dX = dY W and the weight gradient dW += dY^T X, launched
// from LinearLayer.cu:52-63,81-102 and from the un-embedding, Embedding.cu:344-397) and the
// Tensor matmul (Tensor.cu:912-950).
//
// The products of a small transformer are skinny: 4096 x 384 outputs with K = 1536, or
// 1536 x 384 weight gradients with K = 4096.  A classic 2-D tiling gives such an output only
// a few hundred workgroups for the 1024 SIMDs of the chip, so most SIMDs run one or two
// waves with a long K loop and nothing to hide latency behind.  These kernels split K inside
// the workgroup instead:
//
//   * a workgroup of NW waves owns one (32 TM) x (32 TN) tile of C; every wave accumulates
//     the WHOLE tile over its own share of K -- the KW-deep K chunks w, w + NW, w + 2 NW, ...
//     of the workgroup's K range -- so the tile count times NW fills the SIMDs evenly;
//   * each wave streams its chunks global -> LDS directly (global_load_lds_dwordx4, 16 bytes
//     per lane, no staging registers) through a private S-slot ring: the wave waits only for
//     its own loads (s_waitcnt vmcnt) and no barrier runs in the main loop;
//   * at the end the NW partial tiles meet in LDS and are added in wave order (fixed order:
//     bitwise reproducible), bias and the old C (beta) are added, and the tile is stored with
//     coalesced 16-byte stores;
//   * when even that leaves SIMDs idle (weight gradients: small C, long K), K is also split
//     across workgroups; their partial tiles go to a caller workspace and a second kernel adds
//     them in split order (still deterministic, no atomics).
//
// Operand tiles in LDS.  The MFMA takes A[i][kk] from lane (i, kk) and B[kk][j] from lane
// (j, kk); a lane reads four contraction indices k = 8 s + 4 h + t (t = 0..3) at once and
// feeds them to four consecutive MFMAs (h = lane / 32), for both operands, so the pairing of
// A and B indices is consistent.
//   * K-contiguous operand (A stored [m][k], B stored [n][k]): LDS [row][KW] -- one
//     ds_read_b128 per lane gives four MFMAs' operands.  16-byte chunk c of row r sits at
//     physical chunk c ^ swz(r), so the 16 lanes that one LDS cycle serves (16 rows, one
//     chunk) hit 16 distinct bank groups.
//   * M/N-contiguous operand (A stored [k][m], B stored [k][n]): LDS [k][rows] -- one
//     ds_read_b32 per lane per MFMA, lanes 0-31 on k-row kk and lanes 32-63 on kk + 4.  Those
//     two k-rows are kept on different halves of the 64 banks: by swapping row positions
//     (tiles 32 or 96 wide, whose rows alternate halves) or by flipping chunk bit 3 (64 or 128
//     wide).
// The direct-to-LDS load writes 64 consecutive 16-byte chunks per instruction; the swizzle
// is applied by choosing which global chunk each lane fetches.  Rows / columns past the
// matrix edge re-read the last valid one; their results are never stored.
#include "linear_gemm.h"

#include <algorithm>
#include <type_traits>

#include "attn_mfma_common.h"

namespace ctattn {
namespace lin {

typedef __attribute__((address_space(3))) const floatx4 lds_cf4;
typedef __attribute__((address_space(3))) const float lds_cf;
typedef __attribute__((address_space(3))) float lds_f;

__device__ __forceinline__ floatx4 ld4(uint32_t addr) { return *(lds_cf4 *)(uintptr_t)addr; }
__device__ __forceinline__ float ld1(uint32_t addr) { return *(lds_cf *)(uintptr_t)addr; }
__device__ __forceinline__ void st1(uint32_t addr, float x) { *(lds_f *)(uintptr_t)addr = x; }

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return uint32_t(uintptr_t((__attribute__((address_space(3))) const char *)p));
}

// 16 bytes per lane, global -> LDS: lane l's bytes at sbase + voff land at LDS byte address
// dst + 16 l.  sbase and dst are wave-uniform (SGPRs; dst through m0).  The compiler does not
// see this load, so it never makes LDS reads wait for it; the kernel waits itself (wait_vm).
__device__ __forceinline__ void dma16(const char *sbase, uint32_t voff, uint32_t dst) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
                 "s"(__builtin_amdgcn_readfirstlane(dst))
                 : "memory", "m0");
}

// Wait until at most N of the wave's vector-memory loads are outstanding.  The "memory"
// clobber keeps the LDS reads of the stage that this wait publishes below it.
template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// K-contiguous operand: R rows x KW k per stage, LDS [r][KW], chunk c of row r at physical
// chunk c ^ swz(r).  Rows are 4 KW bytes: for KW = 32 (8 chunks) the 16 rows of one LDS cycle
// cover bank groups 8 (r & 1) + (c ^ ((r >> 1) & 7)); for KW = 16 (4 chunks) 4 (r & 3) +
// (c ^ ((r >> 2) & 3)): distinct either way.
template <int R, int KW>
struct OpKC {
    static constexpr int CH = KW / 4;
    static constexpr int BYTES = R * KW * 4;
    static constexpr int NL = BYTES / 1024;  // load instructions per stage
    static_assert(KW == 16 || KW == 32, "K chunk of 16 or 32 fp32");
    static_assert(BYTES % 1024 == 0, "a stage is whole 1 KiB load instructions");
    __host__ __device__ static constexpr int swz(int r) { return CH == 8 ? (r >> 1) & 7 : (r >> 2) & 3; }
    // Byte offset of load instruction i's lane from the stage origin (row 0, chunk 0); rows at
    // or past `rows_left` re-read row rows_left - 1.
    __device__ static uint32_t voff(int i, int lane, int64_t ld_bytes, int rows_left) {
        const int P = 64 * i + lane;
        const int r = P / CH;
        const int lc = (P % CH) ^ swz(r);
        return uint32_t(int64_t(min(r, rows_left - 1)) * ld_bytes + 16 * lc);
    }
    // Per-lane read offsets: offs[s] for k-group s (k = 8 s .. 8 s + 7) of 32-row tile 0.
    struct Lane {
        uint32_t offs[KW / 8];
        __device__ void init(int col, int h) {
#pragma unroll
            for (int s = 0; s < KW / 8; ++s) offs[s] = uint32_t(col * KW * 4 + ((((2 * s) | h) ^ swz(col)) << 4));
        }
        __device__ floatx4 read(uint32_t base, int tt, int s) const { return ld4(base + tt * 32 * KW * 4 + offs[s]); }
    };
};

// M/N-contiguous operand: KW k-rows x R columns per stage, LDS [k][R] (row pitch 4 R bytes).
template <int R, int KW>
struct OpMN {
    static constexpr int CHR = R / 4;
    static constexpr int BYTES = R * KW * 4;
    static constexpr int NL = BYTES / 1024;
    static constexpr bool ODD = (R / 32) % 2 == 1;  // rows alternate bank halves
    static_assert(R % 32 == 0 && R <= 128, "tile width 32, 64, 96 or 128");
    static_assert(BYTES % 1024 == 0, "a stage is whole 1 KiB load instructions");
    // k-row kk sits at row position kk ^ ((kk >> 2) & 1) (ODD); chunk c of k-row kk at
    // physical chunk c ^ (8 ((kk >> 2) & 1)) (!ODD).  Both maps are involutions.
    __host__ __device__ static constexpr int rowpos(int kk) { return ODD ? kk ^ ((kk >> 2) & 1) : kk; }
    __host__ __device__ static constexpr int chunk(int kk, int c) { return ODD ? c : c ^ (((kk >> 2) & 1) << 3); }
    // Columns at or past `cols_left` (a multiple of 4) re-read the last valid chunk.
    __device__ static uint32_t voff(int i, int lane, int64_t ld_bytes, int cols_left) {
        const int P = 64 * i + lane;
        const int kk = rowpos(P / CHR);
        const int lc = chunk(kk, P % CHR);
        return uint32_t(int64_t(kk) * ld_bytes + 4 * min(4 * lc, cols_left - 4));
    }
    // Element (kk = 8 s + 4 h + t, column 32 tt + col) at
    //   ODD:  rowpos(kk) * 4R + 4 (32 tt + col), rowpos(kk) = 8 s + 4 h + (t ^ h);
    //   !ODD: kk * 4R + 16 (8 (tt ^ h) + col / 4) + 4 (col % 4).
    struct Lane {
        uint32_t offt[4];  // per t, tile 0
        int h;
        __device__ void init(int col, int hh) {
            h = hh;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                offt[t] = uint32_t((ODD ? 4 * h + (t ^ h) : 4 * h + t) * 4 * R + 4 * col + (ODD ? 0 : 128 * h));
        }
        __device__ floatx4 read(uint32_t base, int tt, int s) const {
            // !ODD: 128 (tt ^ h) = 128 h + 128 tt - 256 h (tt & 1); the 128 h is in offt.
            const uint32_t tile = ODD ? uint32_t(128 * tt) : uint32_t(128 * tt) - ((tt & 1) ? uint32_t(256 * h) : 0u);
            floatx4 x;
#pragma unroll
            for (int t = 0; t < 4; ++t) x[t] = ld1(base + s * 8 * 4 * R + tile + offt[t]);
            return x;
        }
    };
};

struct Args {
    const char *a, *b;
    float *c;
    const float *bias;
    float *ws;             // split-K partials: splits x M x N floats
    int64_t lda_b, ldb_b;  // operand pitches in bytes
    int64_t ldc;           // elements
    int32_t M, N;
    int32_t tiles_m, tiles_n;
    int32_t splits;
    int32_t chunks;  // K / KW
    int32_t cps;     // chunks per split
    int32_t beta;
    int32_t vec_out;  // C takes 16-byte stores (N % 4 == 0, ldc % 4 == 0, c aligned)
};

template <bool A_KC, bool B_KC, int TM, int TN, int NW, int KW, int S>
struct Cfg {
    static constexpr int BM = 32 * TM, BN = 32 * TN;
    using OA = std::conditional_t<A_KC, OpKC<BM, KW>, OpMN<BM, KW>>;
    using OB = std::conditional_t<B_KC, OpKC<BN, KW>, OpMN<BN, KW>>;
    static constexpr int STAGE = OA::BYTES + OB::BYTES;
    static constexpr int L = OA::NL + OB::NL;  // load instructions per stage
    static constexpr int PIPE = NW * S * STAGE;
    static constexpr int RED = NW * BM * BN * 4;
    static constexpr int LDS = PIPE > RED ? PIPE : RED;
    static_assert(S >= 2 && (S - 1) * L < 64, "outstanding loads must fit vmcnt");
    static_assert(LDS <= 160 * 1024, "LDS of one workgroup");
};

template <int L, int S>
__device__ __forceinline__ void wait_tail(int r) {
    // r stages issued after the one needed (0 <= r <= S - 2).
    if (S > 3 && r >= 2) {
        wait_vm<(S > 3 ? 2 * L : 0)>();
    } else if (S > 2 && r == 1) {
        wait_vm<(S > 2 ? L : 0)>();
    } else {
        wait_vm<0>();
    }
}

template <bool A_KC, bool B_KC, int TM, int TN, int NW, int KW, int S>
__global__ __launch_bounds__(NW * 64) void lin_f32_kernel(Args p) {
    using C = Cfg<A_KC, B_KC, TM, TN, NW, KW, S>;
    using OA = typename C::OA;
    using OB = typename C::OB;
    constexpr int BM = C::BM, BN = C::BN;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int col = lane & 31, h = lane >> 5;

    // Workgroup b runs on XCD b % 8.  XCD x takes the contiguous work items [x q, x q + q), so
    // the workgroups of one XCD share A row blocks (consecutive items: same tile row) in its L2.
    const int nblk = int(gridDim.x), blk = int(blockIdx.x);
    const int q = nblk >> 3;
    const int work = blk < 8 * q ? (blk & 7) * q + (blk >> 3) : blk;
    const int ntiles = p.tiles_m * p.tiles_n;
    const int split = work / ntiles;
    const int tile = work - split * ntiles;
    const int ti = tile / p.tiles_n;
    const int m0 = ti * BM, n0 = (tile - ti * p.tiles_n) * BN;

    // This wave's K chunks: c_first, c_first + NW, ... below c_end.
    const int c_begin = split * p.cps;
    const int c_end = min(p.chunks, c_begin + p.cps);
    const int c_first = c_begin + wave;
    const int nst = c_first < c_end ? (c_end - c_first + NW - 1) / NW : 0;

    const char *ga = p.a + (A_KC ? int64_t(m0) * p.lda_b + int64_t(c_first) * KW * 4
                                 : int64_t(c_first) * KW * p.lda_b + int64_t(m0) * 4);
    const char *gb = p.b + (B_KC ? int64_t(n0) * p.ldb_b + int64_t(c_first) * KW * 4
                                 : int64_t(c_first) * KW * p.ldb_b + int64_t(n0) * 4);
    const int64_t da = A_KC ? int64_t(NW) * KW * 4 : int64_t(NW) * KW * p.lda_b;
    const int64_t db = B_KC ? int64_t(NW) * KW * 4 : int64_t(NW) * KW * p.ldb_b;

    uint32_t va[OA::NL], vb[OB::NL];
#pragma unroll
    for (int i = 0; i < OA::NL; ++i) va[i] = OA::voff(i, lane, p.lda_b, p.M - m0);
#pragma unroll
    for (int i = 0; i < OB::NL; ++i) vb[i] = OB::voff(i, lane, p.ldb_b, p.N - n0);
    typename OA::Lane ra;
    typename OB::Lane rb;
    ra.init(col, h);
    rb.init(col, h);

    const uint32_t wbase = lds_addr(smem) + uint32_t(wave * S * C::STAGE);

    auto issue = [&](int slot) {
        const uint32_t sa = wbase + uint32_t(slot * C::STAGE);
        // The slot's previous contents were read by the last stage's MFMAs: those reads have
        // returned (their results were consumed), this makes it explicit.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < OA::NL; ++i) dma16(ga, va[i], sa + uint32_t(1024 * i));
#pragma unroll
        for (int i = 0; i < OB::NL; ++i) dma16(gb, vb[i], sa + uint32_t(OA::BYTES + 1024 * i));
        ga += da;
        gb += db;
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = zero16();

    const int pro = min(S - 1, nst);
    for (int j = 0; j < pro; ++j) issue(j);
    int slot = 0, islot = S - 1;
    for (int j = 0; j < nst; ++j) {
        if (j + S - 1 < nst) {
            issue(islot);
            wait_vm<(S - 1) * C::L>();
        } else {
            wait_tail<C::L, S>(nst - 1 - j);
        }
        const uint32_t sa = wbase + uint32_t(slot * C::STAGE);
        const uint32_t sb = sa + uint32_t(OA::BYTES);
#pragma unroll
        for (int s = 0; s < KW / 8; ++s) {
            floatx4 av[TM], bv[TN];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) av[tm] = ra.read(sa, tm, s);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) bv[tn] = rb.read(sb, tn, s);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn)
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[tm][t], bv[tn][t], acc[tm][tn], 0, 0, 0);
        }
        slot = slot + 1 == S ? 0 : slot + 1;
        islot = islot + 1 == S ? 0 : islot + 1;
    }

    // Partial tiles -> LDS [wave][BM][BN]; register r of lane (col, h) holds row
    // acc_row(r, h) of column col of each 32 x 32 tile.
    __syncthreads();
    const uint32_t red = lds_addr(smem);
    const uint32_t mine = red + uint32_t(wave * BM * BN * 4);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st1(mine + uint32_t(((32 * tm + acc_row(r, h)) * BN + 32 * tn + col) * 4), acc[tm][tn][r]);
    __syncthreads();

    // Sum the partials in wave order and store, 4 columns per thread.
    constexpr int Q = BM * BN / 4;
    for (int qi = int(threadIdx.x); qi < Q; qi += NW * 64) {
        const int m = qi / (BN / 4);
        const int n = (qi - m * (BN / 4)) * 4;
        const int gm = m0 + m, gn = n0 + n;
        if (gm >= p.M || gn >= p.N) continue;
        floatx4 x = ld4(red + uint32_t((m * BN + n) * 4));
#pragma unroll
        for (int w = 1; w < NW; ++w) x += ld4(red + uint32_t(((w * BM + m) * BN + n) * 4));
        if (p.splits > 1) {
            float *dst = p.ws + (int64_t(split) * p.M + gm) * p.N + gn;
            if (p.N % 4 == 0) {
                *reinterpret_cast<floatx4 *>(dst) = x;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gn + e < p.N) dst[e] = x[e];
            }
            continue;
        }
        float *dst = p.c + int64_t(gm) * p.ldc + gn;
        if (p.vec_out) {
            if (p.bias != nullptr) x += *reinterpret_cast<const floatx4 *>(p.bias + gn);
            if (p.beta) x += *reinterpret_cast<const floatx4 *>(dst);
            *reinterpret_cast<floatx4 *>(dst) = x;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (gn + e >= p.N) break;
                float y = x[e];
                if (p.bias != nullptr) y += p.bias[gn + e];
                if (p.beta) y += dst[e];
                dst[e] = y;
            }
        }
    }
}

// C(m, n) [+]= sum over splits z = 0, 1, ... of ws[z][m][n] (+ bias[n]), 4 columns per thread
// when N % 4 == 0 (vec), else one.
__global__ __launch_bounds__(256) void lin_splitk_reduce_kernel(const float *ws, int splits, int M, int N, float *c,
                                                                int64_t ldc, const float *bias, int beta, int vec) {
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int64_t mn = int64_t(M) * N;
    const int w = vec ? 4 : 1;
    if (idx * w >= mn) return;
    const int64_t e0 = idx * w;
    const int m = int(e0 / N), n = int(e0 - int64_t(m) * N);
    float *dst = c + int64_t(m) * ldc + n;
    if (vec) {
        floatx4 x = *reinterpret_cast<const floatx4 *>(ws + e0);
        for (int z = 1; z < splits; ++z) x += *reinterpret_cast<const floatx4 *>(ws + z * mn + e0);
        if (bias != nullptr) x += *reinterpret_cast<const floatx4 *>(bias + n);
        if (beta) x += *reinterpret_cast<const floatx4 *>(dst);
        *reinterpret_cast<floatx4 *>(dst) = x;
    } else {
        float x = ws[e0];
        for (int z = 1; z < splits; ++z) x += ws[z * mn + e0];
        if (bias != nullptr) x += bias[n];
        if (beta) x += *dst;
        *dst = x;
    }
}

// ---- host side ----

struct Plan {
    int cfg;     // index into the configuration table of the layout
    int splits;  // K splits across workgroups
};

// One launchable configuration.
struct CfgInfo {
    int tm, tn, nw, kw, s;
    int lds;
    hipError_t (*launch)(const Args &, int nblk, hipStream_t);
};

template <bool A_KC, bool B_KC, int TM, int TN, int NW, int KW, int S>
hipError_t launch_cfg(const Args &a, int nblk, hipStream_t stream) {
    hipLaunchKernelGGL((lin_f32_kernel<A_KC, B_KC, TM, TN, NW, KW, S>), dim3(unsigned(nblk)), dim3(NW * 64), 0,
                       stream, a);
    return hipGetLastError();
}

template <bool A_KC, bool B_KC, int TM, int TN, int NW, int KW, int S>
constexpr CfgInfo cfg_info() {
    return CfgInfo{TM, TN, NW, KW, S, Cfg<A_KC, B_KC, TM, TN, NW, KW, S>::LDS,
                   &launch_cfg<A_KC, B_KC, TM, TN, NW, KW, S>};
}

// Builds the kernel arguments of a product for a configuration and split count; returns the
// workgroup count.
inline int make_args(const LinGemm &g, const CfgInfo &c, int splits, void *ws, Args &a) {
    const int bm = 32 * c.tm, bn = 32 * c.tn;
    a.a = static_cast<const char *>(g.a);
    a.b = static_cast<const char *>(g.b);
    a.c = static_cast<float *>(g.c);
    a.bias = static_cast<const float *>(g.bias);
    a.ws = static_cast<float *>(ws);
    a.lda_b = g.lda * 4;
    a.ldb_b = g.ldb * 4;
    a.ldc = g.ldc;
    a.M = int32_t(g.M);
    a.N = int32_t(g.N);
    a.tiles_m = int32_t((g.M + bm - 1) / bm);
    a.tiles_n = int32_t((g.N + bn - 1) / bn);
    a.chunks = int32_t(g.K / c.kw);
    a.cps = (a.chunks + splits - 1) / splits;
    a.splits = (a.chunks + a.cps - 1) / a.cps;  // no empty split
    a.beta = g.beta ? 1 : 0;
    a.vec_out = g.N % 4 == 0 && g.ldc % 4 == 0 && uintptr_t(g.c) % 16 == 0 &&
                (g.bias == nullptr || uintptr_t(g.bias) % 16 == 0);
    return a.tiles_m * a.tiles_n * a.splits;
}

inline hipError_t run(const LinGemm &g, const CfgInfo &c, int splits, void *ws, int64_t ws_bytes,
                      hipStream_t stream) {
    Args a{};
    const int nblk = make_args(g, c, splits, ws, a);
    // Split-K partials: a.splits x M x N floats, which the workspace must hold.
    if (a.splits > 1 && (ws == nullptr || ws_bytes < int64_t(a.splits) * g.M * g.N * 4)) return hipErrorInvalidValue;
    hipError_t e = c.launch(a, nblk, stream);
    if (e != hipSuccess || a.splits == 1) return e;
    const int vec = g.N % 4 == 0 && g.ldc % 4 == 0 && uintptr_t(g.c) % 16 == 0 &&
                    (g.bias == nullptr || uintptr_t(g.bias) % 16 == 0);
    const int64_t items = vec ? g.M * g.N / 4 : g.M * g.N;
    hipLaunchKernelGGL(lin_splitk_reduce_kernel, dim3(unsigned((items + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const float *>(ws), a.splits, a.M, a.N, static_cast<float *>(g.c), g.ldc,
                       static_cast<const float *>(g.bias), a.beta, vec);
    return hipGetLastError();
}

inline int64_t splits_bytes(const LinGemm &g, int splits) { return splits > 1 ? int64_t(splits) * g.M * g.N * 4 : 0; }

}  // namespace lin
}  // namespace ctattn

namespace ctattn {
namespace {

using lin::CfgInfo;
using lin::cfg_info;

// The launchable configurations, per operand layout (tile 32 TM x 32 TN, NW waves, K chunks of
// KW, S-stage ring).  The choice among them (plan below) was fitted to a forced-configuration
// sweep of 132 configurations per layout over the products of a d384 / d1024 transformer and
// a 4096^3 matmul.
const CfgInfo kFwd[] = {cfg_info<true, true, 2, 1, 4, 16, 2>(), cfg_info<true, true, 2, 1, 1, 16, 2>(),
                        cfg_info<true, true, 2, 1, 1, 16, 3>()};
const CfgInfo kDx[] = {cfg_info<true, false, 2, 1, 4, 16, 2>(), cfg_info<true, false, 2, 1, 1, 16, 2>(),
                       cfg_info<true, false, 2, 1, 1, 16, 3>()};
const CfgInfo kDw[] = {cfg_info<false, false, 1, 1, 4, 16, 2>(), cfg_info<false, false, 2, 2, 8, 16, 2>()};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Chooses a configuration and a K split count.  allow_split: the caller has workspace for
// split-K partials.
//   * Both operands M/N-contiguous (weight gradients: small output, K = rows): 64 x 64 tiles
//     of 8 waves when there are at least 256 of them, else 32 x 32 tiles of 4 waves with K
//     split across workgroups up to 2048 workgroups, each wave keeping >= 12 K chunks.
//   * Otherwise 64 x 32 tiles: 4 waves (K split inside the workgroup) while there are fewer
//     than 3072 tiles, else one wave per tile (3 stages once K reaches 1024).
lin::Plan plan(const LinGemm &g, bool allow_split, const CfgInfo **cfg) {
    const int64_t chunks = g.K / 16;
    if (!g.a_kc) {
        if (cdiv(g.M, 64) * cdiv(g.N, 64) >= 256) {
            *cfg = &kDw[1];
            return lin::Plan{1, 1};
        }
        const int64_t tiles = cdiv(g.M, 32) * cdiv(g.N, 32);
        int64_t sp = std::min<int64_t>(cdiv(2048, tiles), chunks / 48);
        sp = allow_split ? std::max<int64_t>(1, std::min<int64_t>(sp, 16)) : 1;
        *cfg = &kDw[0];
        return lin::Plan{0, int(sp)};
    }
    const CfgInfo *tab = g.b_kc ? kFwd : kDx;
    const int64_t tiles = cdiv(g.M, 64) * cdiv(g.N, 32);
    const int i = tiles < 3072 ? 0 : chunks >= 64 ? 2 : 1;
    *cfg = &tab[i];
    return lin::Plan{i, 1};
}

}  // namespace

namespace {

// The shape / pitch part of lin_gemm_supported (pointers are not looked at).
bool shape_ok(const LinGemm &g) {
    if (g.dtype != 0 || (!g.a_kc && g.b_kc)) return false;
    if (g.M < 1 || g.N < 1 || g.K < 16 || g.K % 16 != 0) return false;
    if (g.M > 2147483647 || g.N > 2147483647 || g.K > 2147483647) return false;
    // 16-byte operand rows for the direct-to-LDS loads.
    if (g.lda % 4 != 0 || g.ldb % 4 != 0) return false;
    // An M/N-contiguous operand is read in whole 16-byte chunks of its M / N extent.
    if ((!g.a_kc && g.M % 4 != 0) || (!g.b_kc && g.N % 4 != 0)) return false;
    // Lane offsets within a stage are 32-bit: at most 128 rows (or 16 k-rows) of one pitch.
    if (g.lda > (int64_t(1) << 22) || g.ldb > (int64_t(1) << 22)) return false;
    if (g.ldc < g.N) return false;
    // Launch size: workgroups x threads below 2^32.
    const CfgInfo *c = nullptr;
    const lin::Plan pl = plan(g, true, &c);
    const int64_t wg = cdiv(g.M, 32 * c->tm) * cdiv(g.N, 32 * c->tn) * pl.splits;
    return wg * c->nw * 64 < (int64_t(1) << 32);
}

}  // namespace

bool lin_gemm_supported(const LinGemm &g) {
    if (!shape_ok(g) || !g.a || !g.b || !g.c) return false;
    return uintptr_t(g.a) % 16 == 0 && uintptr_t(g.b) % 16 == 0;
}

int64_t lin_gemm_workspace_bytes(const LinGemm &g) {
    if (!shape_ok(g)) return 0;
    const CfgInfo *c = nullptr;
    const lin::Plan pl = plan(g, true, &c);
    // The launch trims empty splits, never adds any: splits x M x N floats is an upper bound.
    return pl.splits > 1 ? lin::splits_bytes(g, pl.splits) : 0;
}

hipError_t launch_lin_gemm(const LinGemm &g, void *ws, int64_t ws_bytes, hipStream_t stream) {
    if (!lin_gemm_supported(g)) return hipErrorInvalidValue;
    const CfgInfo *c = nullptr;
    lin::Plan pl = plan(g, true, &c);
    if (pl.splits > 1 && (ws == nullptr || ws_bytes < lin::splits_bytes(g, pl.splits))) pl = plan(g, false, &c);
    return lin::run(g, *c, pl.splits, ws, ws_bytes, stream);
}

}  // namespace ctattn
