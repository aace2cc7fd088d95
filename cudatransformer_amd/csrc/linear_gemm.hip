// Split-K-in-workgroup MFMA GEMMs (gfx950): the linear layers' three products, the attention
// layer's projections and the Tensor matmul, fp32 on v_mfma_f32_32x32x2f32 and bf16 / fp16 on
// v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulation.
//
// Replaces the reference's tiled linear kernels (linear_kernels.cu:36-241: the forward
// y = x W^T + b, the input gradient dX = dY W and the weight gradient dW += dY^T X, launched
// from LinearLayer.cu:52-63,81-102 and from the un-embedding, Embedding.cu:344-397), its
// projection kernels (attention_qkv_kernels.cu:51-364, attention_proj_kernels.cu:48-290) and
// the Tensor matmul (Tensor.cu:912-950).
//
// Every operand is a separable 2-D view of memory (element (i, j) at row_off(i) + col_off(j)):
// row-major, or the head-split view of a [B, H, T, d] tensor as a [B*T, H*d] matrix, so the
// projections read and write the attention layout in place.  A launch computes up to three
// independent products (Q, K, V) and sums up to three K segments into one output
// (dX = dQ Wq + dK Wk + dV Wv).
//
// The products of a small transformer are skinny: 4096 x 384 outputs with K = 1536, or
// 1536 x 384 weight gradients with K = 4096.  A classic 2-D tiling gives such an output only
// a few hundred workgroups for the 1024 SIMDs of the chip, so most SIMDs run one or two
// waves with a long K loop and nothing to hide latency behind.  These kernels split K inside
// the workgroup instead:
//
//   * a workgroup of NW waves owns one (32 TM) x (32 TN) tile of C; every wave accumulates
//     the WHOLE tile over its own share of K -- the 64-byte K chunks w, w + NW, w + 2 NW, ...
//     of the workgroup's K range (16 fp32 or 32 16-bit elements) -- so the tile count times
//     NW fills the SIMDs evenly;
//   * each wave streams its chunks global -> LDS directly (global_load_lds_dwordx4, 16 bytes
//     per lane, no staging registers) through a private S-slot ring: the wave waits only for
//     its own loads (s_waitcnt vmcnt) and no barrier runs in the main loop;
//   * at the end the NW partial tiles meet in LDS and are added in wave order (fixed order:
//     bitwise reproducible), bias and the old C (beta) are added, and the tile is stored with
//     coalesced vector stores;
//   * when even that leaves SIMDs idle (weight gradients: small C, long K), K is also split
//     across workgroups; their partial tiles go to a caller workspace and a second kernel adds
//     them in split order (still deterministic, no atomics);
//   * a weight gradient can also produce its bias gradient db[m] += sum_k A(m, k) (A = dY: the
//     column sums of dY): every wave adds up the A operand values it already reads for its
//     MFMAs, the workgroups of the first tile column store the sums (fixed order).
//
// Operand tiles in LDS.  The fp32 MFMA takes A[i][kk] from lane (i, kk) and B[kk][j] from lane
// (j, kk); a lane reads four contraction indices k = 8 s + 4 h + t (t = 0..3) at once and
// feeds them to four consecutive MFMAs (h = lane / 32).  The 16-bit MFMA takes eight
// consecutive k = 16 s + 8 h + 0..7 from one lane per instruction.  Either way a lane's
// operand for step s is 16 bytes, and A and B pair the same indices.
//   * K-contiguous operand (A stored [m][k], B stored [n][k]): LDS [row][64 bytes] -- one
//     ds_read_b128 per lane per step.  16-byte chunk c of row r sits at physical chunk
//     c ^ swz(r), so the 16 lanes that one LDS cycle serves (16 rows, one chunk) hit 16
//     distinct bank groups.
//   * M/N-contiguous operand (A stored [k][m], B stored [k][n]), fp32: LDS [16 k][rows] -- one
//     ds_read_b32 per lane per MFMA, lanes 0-31 on k-row kk and lanes 32-63 on kk + 4.  Those
//     two k-rows are kept on different halves of the 64 banks: by swapping row positions
//     (tiles 32 or 96 wide, whose rows alternate halves) or by flipping chunk bit 3 (64 or 128
//     wide).
//     A 64-wide fp32 operand of two 32-wide MFMA tiles instead interleaves them: row i of
//     tile t is column 2 i + t of the 64, so one ds_read_b64 per lane gives both tiles'
//     operands at one k (the partial-tile epilogue undoes the interleave).
//   * M/N-contiguous operand, 16-bit: LDS [32 k][rows] -- two ds_read_b64_tr_b16 per lane per
//     step (each: a 16-lane group reads 4 k-rows x 16 columns and lane l receives column l's
//     four values).  The 64-byte segment index of a k-row is XOR-swizzled by the row so the 32
//     lanes of one LDS cycle (4 k-rows x 32 columns) cover the 64 banks once.
// The direct-to-LDS load writes 64 consecutive 16-byte chunks per instruction; the swizzle
// is applied by choosing which global chunk each lane fetches.  Rows / columns past the
// matrix edge re-read the last valid one; their results are never stored.
#include "linear_gemm.h"

#include <algorithm>
#include <type_traits>

#include "act_math.h"
#include "attn_common.h"
#include "attn_mfma_common.h"

namespace ctattn {
namespace lin {

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) const floatx4 lds_cf4;
typedef __attribute__((address_space(3))) const float lds_cf;
typedef __attribute__((address_space(3))) float lds_f;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ floatx4 ld4(uint32_t addr) { return *(lds_cf4 *)(uintptr_t)addr; }
__device__ __forceinline__ float ld1(uint32_t addr) { return *(lds_cf *)(uintptr_t)addr; }
__device__ __forceinline__ void st1(uint32_t addr, float x) { *(lds_f *)(uintptr_t)addr = x; }
__device__ __forceinline__ i16x4 ldtr(uint32_t addr) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(uintptr_t)addr);
}

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

// ---- element formats ----

struct F32Fmt {
    static constexpr int EB = 4;    // bytes per element
    static constexpr int KWE = 16;  // elements per 64-byte K chunk
    static constexpr bool WIDE = true;
    __device__ static float load(const char *p) { return *reinterpret_cast<const float *>(p); }
    __device__ static floatx4 load4(const char *p) { return *reinterpret_cast<const floatx4 *>(p); }
    __device__ static void store(char *p, float x) { *reinterpret_cast<float *>(p) = x; }
    __device__ static void store4(char *p, floatx4 x) { *reinterpret_cast<floatx4 *>(p) = x; }
    // The value a store and a load back give (the storage type's rounding).
    __device__ static float round(float x) { return x; }
    // Sum of the 16-byte MFMA operand (4 fp32 values).
    __device__ static float sum(floatx4 v) { return (v[0] + v[1]) + (v[2] + v[3]); }
};
template <bool BF>
struct H16Fmt {
    static constexpr int EB = 2;
    static constexpr int KWE = 32;
    static constexpr bool WIDE = false;
    __device__ static float widen(uint16_t b) {
        return BF ? __uint_as_float(uint32_t(b) << 16) : float(__builtin_bit_cast(_Float16, b));
    }
    __device__ static uint16_t narrow(float x) {
        return BF ? f32_to_bf16(x).bits : __builtin_bit_cast(uint16_t, _Float16(x));
    }
    __device__ static floatx16 mfma(floatx4 a, floatx4 b, floatx16 c) {
        if constexpr (BF)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                           c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                          0, 0, 0);
    }
    __device__ static float load(const char *p) { return widen(*reinterpret_cast<const uint16_t *>(p)); }
    __device__ static float round(float x) { return widen(narrow(x)); }
    __device__ static floatx4 load4(const char *p) {
        const u16x4 u = *reinterpret_cast<const u16x4 *>(p);
        return floatx4{widen(u[0]), widen(u[1]), widen(u[2]), widen(u[3])};
    }
    __device__ static void store(char *p, float x) { *reinterpret_cast<uint16_t *>(p) = narrow(x); }
    __device__ static void store4(char *p, floatx4 x) {
        *reinterpret_cast<u16x4 *>(p) = u16x4{narrow(x[0]), narrow(x[1]), narrow(x[2]), narrow(x[3])};
    }
    // Sum of the 16-byte MFMA operand (8 16-bit values).
    __device__ static float sum(floatx4 v) {
        const i16x8 u = __builtin_bit_cast(i16x8, v);
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += widen(uint16_t(u[e]));
        return s;
    }
};
using BF16Fmt = H16Fmt<true>;
using F16Fmt = H16Fmt<false>;

// ---- views ----

// Division by a run-time divisor D >= 1 of indices 0 <= i < 2^31 as a multiply and a shift
// (Granlund & Montgomery, "Division by invariant integers using multiplication", 1994, the
// unsigned case): with l = ceil(log2 D) and m = floor(2^32 (2^l - D) / D) + 1,
// i / D = (mulhi(i, m) + i) >> l exactly for every 32-bit i; mulhi(i, m) < i keeps the sum
// below 2^32 for i < 2^31.
struct FastDiv {
    uint32_t mul, shift;
};
inline FastDiv make_fastdiv(uint32_t D) {
    if (D == 0) return FastDiv{0, 0};  // no index to divide (an empty view)
    uint32_t l = 0;
    while (l < 32 && (uint64_t(1) << l) < D) ++l;
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - D)) / D + 1;
    return FastDiv{uint32_t(m), l};
}
__device__ __forceinline__ int fastdiv(int i, FastDiv f) {
    return int((__umulhi(uint32_t(i), f.mul) + uint32_t(i)) >> f.shift);
}

// A LinView on the device, in bytes.  Indices are below 2^31 (checked on the host).  The
// head-split offsets divide by T and d through FastDiv: the store loops of a tile compute
// one row and one column offset per 4 elements.
struct DView {
    int64_t ld_b;    // linear: row pitch
    int64_t bstr_b;  // head-split: one batch, H*T*d elements
    int64_t hstr_b;  // head-split: one head, T*d elements
    int32_t heads, T, d, eb;
    FastDiv tdiv, ddiv;  // head-split: i / T, j / d
};
__device__ __forceinline__ int64_t rowoff(const DView &v, int i) {
    if (v.heads == 0) return int64_t(i) * v.ld_b;
    const int b = fastdiv(i, v.tdiv);
    return int64_t(b) * v.bstr_b + int64_t(i - b * v.T) * (v.d * v.eb);
}
__device__ __forceinline__ int64_t coloff(const DView &v, int j) {
    if (v.heads == 0) return int64_t(j) * v.eb;
    const int h = fastdiv(j, v.ddiv);
    return int64_t(h) * v.hstr_b + int64_t(j - h * v.d) * v.eb;
}
// Byte distance between consecutive rows inside one K chunk of an M/N-contiguous operand (a
// chunk never crosses a batch of a head-split view: T is a multiple of the chunk).
__device__ __forceinline__ int64_t krow_b(const DView &v) { return v.heads == 0 ? v.ld_b : int64_t(v.d) * v.eb; }

// ---- operand tiles ----

// K-contiguous operand: R rows x 64 bytes per stage, LDS [r][64 B], chunk c of row r at
// physical chunk c ^ swz(r): the 16 rows of one LDS cycle cover bank groups
// 4 (r & 3) + (c ^ ((r >> 2) & 3)), all distinct.
template <int R>
struct OpKC {
    static constexpr int CH = 4;  // 16-byte chunks per row
    static constexpr int BYTES = R * 64;
    static constexpr int NL = BYTES / 1024;  // load instructions per stage
    static_assert(BYTES % 1024 == 0, "a stage is whole 1 KiB load instructions");
    __host__ __device__ static constexpr int swz(int r) { return (r >> 2) & 3; }
    // Lane offset of load instruction i from the stage origin (row 0, chunk 0 of the tile);
    // rows at or past `rows` re-read row rows - 1.
    __device__ static uint32_t voff(int i, int lane, const DView &v, int r0, int rows) {
        const int P = 64 * i + lane;
        const int r = P / CH;
        const int lc = (P % CH) ^ swz(r);
        return uint32_t(rowoff(v, r0 + min(r, rows - 1)) - rowoff(v, r0) + 16 * lc);
    }
    // Read of step s (16 bytes: k-group s of lane half h) of 32-row tile tt.
    struct Lane {
        uint32_t offs[2];
        __device__ void init(int lane) {
            const int col = lane & 31, h = lane >> 5;
#pragma unroll
            for (int s = 0; s < 2; ++s) offs[s] = uint32_t(col * 64 + ((((2 * s) | h) ^ swz(col)) << 4));
        }
        __device__ floatx4 read(uint32_t base, int tt, int s) const { return ld4(base + tt * 32 * 64 + offs[s]); }
    };
    // Index (row of A / column of B) of MFMA row i of 32-wide tile t.
    __host__ __device__ static constexpr int idx(int t, int i) { return 32 * t + i; }
};

// K-contiguous operand two 64-byte K chunks deep: R rows x 128 bytes per stage, LDS
// [r][128 B], chunk c of row r at physical chunk c ^ swz(r): the 16 lanes of one LDS cycle of
// a step's read (16 consecutive rows, one chunk) cover bank groups 8 (r & 1) + (c ^ swz(r)),
// all distinct.
template <int R>
struct OpKC2 {
    static constexpr int CH = 8;
    static constexpr int BYTES = R * 128;
    static constexpr int NL = BYTES / 1024;
    static_assert(BYTES % 1024 == 0, "a stage is whole 1 KiB load instructions");
    __host__ __device__ static constexpr int swz(int r) { return (r >> 1) & 7; }
    __device__ static uint32_t voff(int i, int lane, const DView &v, int r0, int rows) {
        const int P = 64 * i + lane;
        const int r = P / CH;
        const int lc = (P % CH) ^ swz(r);
        return uint32_t(rowoff(v, r0 + min(r, rows - 1)) - rowoff(v, r0) + 16 * lc);
    }
    // Read of step s (0..3: 16 bytes, k-group s of lane half h) of 32-row tile tt.
    struct Lane {
        uint32_t offs[4];
        __device__ void init(int lane) {
            const int col = lane & 31, h = lane >> 5;
#pragma unroll
            for (int s = 0; s < 4; ++s) offs[s] = uint32_t(col * 128 + ((((2 * s) | h) ^ swz(col)) << 4));
        }
        __device__ floatx4 read(uint32_t base, int tt, int s) const { return ld4(base + tt * 32 * 128 + offs[s]); }
    };
    __host__ __device__ static constexpr int idx(int t, int i) { return 32 * t + i; }
};

// M/N-contiguous fp32 operand: 16 k-rows x R columns per stage, LDS [k][R] (row pitch 4 R).
template <int R>
struct OpMN32 {
    static constexpr int CHR = R / 4;  // 16-byte chunks per k-row
    static constexpr int BYTES = R * 64;
    static constexpr int NL = BYTES / 1024;
    static constexpr bool ODD = (R / 32) % 2 == 1;  // rows alternate bank halves
    static_assert(R % 32 == 0 && R <= 128, "tile width 32, 64, 96 or 128");
    // k-row kk sits at row position kk ^ ((kk >> 2) & 1) (ODD); chunk c of k-row kk at
    // physical chunk c ^ (8 ((kk >> 2) & 1)) (!ODD).  Both maps are involutions.
    __host__ __device__ static constexpr int rowpos(int kk) { return ODD ? kk ^ ((kk >> 2) & 1) : kk; }
    __host__ __device__ static constexpr int chunk(int kk, int c) { return ODD ? c : c ^ (((kk >> 2) & 1) << 3); }
    // Columns at or past `cols` (a multiple of 4) re-read the last valid chunk.
    __device__ static uint32_t voff(int i, int lane, const DView &v, int c0, int cols) {
        const int P = 64 * i + lane;
        const int kk = rowpos(P / CHR);
        const int lc = chunk(kk, P % CHR);
        return uint32_t(int64_t(kk) * krow_b(v) + coloff(v, c0 + min(4 * lc, cols - 4)) - coloff(v, c0));
    }
    // Element (kk = 8 s + 4 h + t, column 32 tt + col) at
    //   ODD:  rowpos(kk) * 4R + 4 (32 tt + col), rowpos(kk) = 8 s + 4 h + (t ^ h);
    //   !ODD: kk * 4R + 16 (8 (tt ^ h) + col / 4) + 4 (col % 4).
    struct Lane {
        uint32_t offt[4];  // per t, tile 0
        int h;
        __device__ void init(int lane) {
            const int col = lane & 31;
            h = lane >> 5;
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
    __host__ __device__ static constexpr int idx(int t, int i) { return 32 * t + i; }
};

// M/N-contiguous fp32 operand of two interleaved 32-wide tiles: 16 k-rows x 64 columns per
// stage, LDS [k][64] (row pitch 256 bytes, no swizzle), MFMA row i of tile t at column 2 i + t.
// Lane (col, h) reads columns 2 col, 2 col + 1 of k-row 8 s + 4 h + t with one ds_read_b64:
// each half-wave reads one whole 256-byte k-row, the 64 banks once.
struct OpMN32P {
    static constexpr int R = 64;
    static constexpr int CHR = 16;  // 16-byte chunks per k-row
    static constexpr int BYTES = R * 64;
    static constexpr int NL = BYTES / 1024;
    __device__ static uint32_t voff(int i, int lane, const DView &v, int c0, int cols) {
        const int P = 64 * i + lane;
        const int kk = P / CHR, lc = P % CHR;
        return uint32_t(int64_t(kk) * krow_b(v) + coloff(v, c0 + min(4 * lc, cols - 4)) - coloff(v, c0));
    }
    struct Lane {
        uint32_t off;
        __device__ void init(int lane) { off = uint32_t((4 * (lane >> 5)) * 4 * R + 8 * (lane & 31)); }
    };
    __host__ __device__ static constexpr int idx(int t, int i) { return 2 * i + t; }
};

// M/N-contiguous 16-bit operand: KR k-rows (32 or 64) x R columns per stage, LDS [k][R] (row
// pitch 2 R), the 64-byte segment sg of k-row kr at physical segment sg ^ gsw(kr).
template <int R, int KR = 32>
struct OpMN16 {
    static constexpr int BYTES = R * 2 * KR;
    static constexpr int NL = BYTES / 1024;
    static constexpr int PITCH = 2 * R;
    static constexpr int SEGS = R / 32;
    static_assert(R == 32 || R == 64 || R == 128, "tile width 32, 64 or 128");
    static_assert(KR == 32 || KR == 64, "one or two 32-row K chunks");
    __host__ __device__ static constexpr int gsw(int kr) {
        return SEGS == 4 ? (kr & 3) : SEGS == 2 ? ((kr >> 1) & 1) : 0;
    }
    // Columns at or past `cols` (a multiple of 8) re-read the last valid chunk.
    __device__ static uint32_t voff(int i, int lane, const DView &v, int c0, int cols) {
        const int P = 64 * i + lane;
        const int kr = P / (R / 8);
        const int lc = (P % (R / 8)) ^ (gsw(kr) << 2);
        return uint32_t(int64_t(kr) * krow_b(v) + coloff(v, c0 + min(8 * lc, cols - 8)) - coloff(v, c0));
    }
    // Step s (< KR / 16), lane (16-lane group g, sl = lane % 16): rows 16 s + 8 (g >> 1) + sl / 4 (+ 4 for
    // the second read), columns 32 tt + 16 (g & 1) + 4 (sl % 4) .. + 3; the lane receives its
    // column's 4 + 4 values, k = 16 s + 8 h + 0..7 in order.  gsw of those rows is the same
    // for every s and both reads.
    struct Lane {
        uint32_t off;
        int gs;
        __device__ void init(int lane) {
            const int g = lane >> 4, sl = lane & 15;
            const int row = 8 * (g >> 1) + (sl >> 2);
            gs = gsw(row);
            off = uint32_t(row * PITCH + 32 * (g & 1) + 8 * (sl & 3));
        }
        __device__ floatx4 read(uint32_t base, int tt, int s) const {
            const uint32_t a = base + off + uint32_t((tt ^ gs) * 64 + 16 * s * PITCH);
            const i16x4 lo = ldtr(a), hi = ldtr(a + 4 * PITCH);
            const i16x8 x = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            return __builtin_bit_cast(floatx4, x);
        }
    };
    __host__ __device__ static constexpr int idx(int t, int i) { return 32 * t + i; }
};

typedef __attribute__((address_space(3))) const floatx2 lds_cf2;

// Operands of step s of every 32-wide tile of an operand (NT tiles).
template <typename Op, int NT>
__device__ __forceinline__ void read_all(const typename Op::Lane &l, uint32_t base, int s, floatx4 (&out)[NT]) {
    if constexpr (std::is_same_v<Op, OpMN32P>) {
        static_assert(NT == 2, "the interleaved operand holds two tiles");
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const floatx2 x = *(lds_cf2 *)(uintptr_t)(base + l.off + uint32_t((8 * s + t) * 4 * Op::R));
            out[0][t] = x[0];
            out[1][t] = x[1];
        }
    } else {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) out[tt] = l.read(base, tt, s);
    }
}

struct Args {
    const char *a[kLinMaxBatch][kLinMaxSeg];
    const char *b[kLinMaxBatch][kLinMaxSeg];
    char *c[kLinMaxBatch];
    const char *bias[kLinMaxBatch];
    char *db[kLinMaxBatch];  // bias gradients (M-contiguous A only), or null
    float *ws;  // split-K partials: [batch][split][M][N] fp32, then [batch][split][M] of db
    DView av, bv, cv;
    int32_t M, N;
    int32_t tiles_m, tiles_n;
    int32_t splits, nbatch;
    int32_t chunks;      // K chunks over all segments
    int32_t seg_chunks;  // K chunks per segment
    int32_t cps;         // chunks per split
    int32_t beta;
    int32_t vec_out;  // C takes 4-column vector stores
    int32_t act_mode, act_kind;  // fused activation (LinGemm::act_mode), aux in C's view
    char *aux[kLinMaxBatch];
};

template <typename F, bool A_KC, bool B_KC, int TM, int TN, int NW, int S>
struct Cfg {
    static constexpr int BM = 32 * TM, BN = 32 * TN;
    // An fp32 M/N-contiguous operand two tiles wide reads both tiles at once (OpMN32P).
    template <bool KC, int NT>
    using Op = std::conditional_t<KC, OpKC<32 * NT>,
                                  std::conditional_t<!F::WIDE, OpMN16<32 * NT>,
                                                     std::conditional_t<NT == 2, OpMN32P, OpMN32<32 * NT>>>>;
    using OA = Op<A_KC, TM>;
    using OB = Op<B_KC, TN>;
    static constexpr int STAGE = OA::BYTES + OB::BYTES;
    static constexpr int L = OA::NL + OB::NL;  // load instructions per stage
    static constexpr int PIPE = NW * S * STAGE;
    static constexpr int RED = NW * BM * BN * 4;
    static constexpr int DBR = A_KC ? 0 : NW * 2 * BM * 4;  // per-wave, per-lane-half bias sums
    static constexpr int LDS = PIPE > RED + DBR ? PIPE : RED + DBR;
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

// Wave-uniform base of segment `seg` (seg < 3): a select, not an indexed register array.
__device__ __forceinline__ const char *pick(const char *const (&arr)[kLinMaxSeg], int seg) {
    return seg == 0 ? arr[0] : seg == 1 ? arr[1] : arr[2];
}

// GEN: some operand or the output is a head-split view, or K has several segments, so every K
// chunk's origin is computed from the views; otherwise (row-major matrices, one segment) the
// stage pointers just advance by a fixed stride per chunk.
template <typename F, bool A_KC, bool B_KC, int TM, int TN, int NW, int S, bool GEN>
__global__ __launch_bounds__(NW * 64) void lin_kernel(Args p) {
    using C = Cfg<F, A_KC, B_KC, TM, TN, NW, S>;
    using OA = typename C::OA;
    using OB = typename C::OB;
    constexpr int BM = C::BM, BN = C::BN;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS];

    // Without GEN every view is linear: heads = 0 as a constant folds the head-split arithmetic
    // (divisions by T and d) out of the origins, lane offsets and stores.
    DView view_a = p.av, view_b = p.bv, view_c = p.cv;
    if constexpr (!GEN) view_a.heads = view_b.heads = view_c.heads = 0;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int h = lane >> 5, col = lane & 31;

    // Workgroup b runs on XCD b % 8.  XCD x takes the contiguous work items [x q, x q + q), so
    // the workgroups of one XCD share A row blocks (consecutive items: same tile row) in its L2.
    const int nblk = int(gridDim.x), blk = int(blockIdx.x);
    const int q = nblk >> 3;
    const int work = blk < 8 * q ? (blk & 7) * q + (blk >> 3) : blk;
    const int ntiles = p.tiles_m * p.tiles_n;
    const int per_batch = ntiles * p.splits;
    const int z = work / per_batch;
    const int rem = work - z * per_batch;
    const int split = rem / ntiles;
    const int tile = rem - split * ntiles;
    const int ti = tile / p.tiles_n;
    const int m0 = ti * BM, n0 = (tile - ti * p.tiles_n) * BN;

    // This wave's K chunks: c_first, c_first + NW, ... below c_end.
    const int c_begin = split * p.cps;
    const int c_end = min(p.chunks, c_begin + p.cps);
    const int c_first = c_begin + wave;
    const int nst = c_first < c_end ? (c_end - c_first + NW - 1) / NW : 0;

    // Tile origins (the M / N offset of the tile; the K offset is added per chunk).
    const char *a_seg[kLinMaxSeg], *b_seg[kLinMaxSeg];
    const int64_t a_t = A_KC ? rowoff(view_a, m0) : coloff(view_a, m0);
    const int64_t b_t = B_KC ? rowoff(view_b, n0) : coloff(view_b, n0);
#pragma unroll
    for (int s = 0; s < kLinMaxSeg; ++s) {
        a_seg[s] = p.a[z][s] + a_t;
        b_seg[s] = p.b[z][s] + b_t;
    }

    uint32_t va[OA::NL], vb[OB::NL];
#pragma unroll
    for (int i = 0; i < OA::NL; ++i) va[i] = OA::voff(i, lane, view_a, m0, p.M - m0);
#pragma unroll
    for (int i = 0; i < OB::NL; ++i) vb[i] = OB::voff(i, lane, view_b, n0, p.N - n0);
    typename OA::Lane ra;
    typename OB::Lane rb;
    ra.init(lane);
    rb.init(lane);

    const uint32_t wbase = lds_addr(smem) + uint32_t(wave * S * C::STAGE);

    // Row-major operands: chunk c's origin is base + c * (64 bytes along a K-contiguous row,
    // or KWE rows of an M/N-contiguous operand), issued in order.
    const int64_t da = A_KC ? 64 : int64_t(F::KWE) * view_a.ld_b;
    const int64_t db = B_KC ? 64 : int64_t(F::KWE) * view_b.ld_b;
    const char *ga_next = a_seg[0] + int64_t(c_first) * da;
    const char *gb_next = b_seg[0] + int64_t(c_first) * db;

    auto issue = [&](int slot, int j) {
        const char *ga, *gb;
        if constexpr (GEN) {
            const int c = c_first + j * NW;
            const int seg = p.seg_chunks == p.chunks ? 0 : c / p.seg_chunks;
            const int kk = (c - seg * p.seg_chunks) * F::KWE;
            ga = pick(a_seg, seg) + (A_KC ? coloff(view_a, kk) : rowoff(view_a, kk));
            gb = pick(b_seg, seg) + (B_KC ? coloff(view_b, kk) : rowoff(view_b, kk));
        } else {
            (void)j;
            ga = ga_next;
            gb = gb_next;
            ga_next += NW * da;
            gb_next += NW * db;
        }
        const uint32_t sa = wbase + uint32_t(slot * C::STAGE);
        // The slot's previous contents were read by the last stage's MFMAs: those reads have
        // returned (their results were consumed), this makes it explicit.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < OA::NL; ++i) dma16(ga, va[i], sa + uint32_t(1024 * i));
#pragma unroll
        for (int i = 0; i < OB::NL; ++i) dma16(gb, vb[i], sa + uint32_t(OA::BYTES + 1024 * i));
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = zero16();
    // Bias gradient of an M-contiguous A: the workgroups of the first tile column sum A.
    const bool want_db = !A_KC && p.db[z] != nullptr && n0 == 0;
    float dsum[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) dsum[i] = 0.f;

    const int pro = min(S - 1, nst);
    for (int j = 0; j < pro; ++j) issue(j, j);
    int slot = 0, islot = S - 1;
    for (int j = 0; j < nst; ++j) {
        if (j + S - 1 < nst) {
            issue(islot, j + S - 1);
            wait_vm<(S - 1) * C::L>();
        } else {
            wait_tail<C::L, S>(nst - 1 - j);
        }
        const uint32_t sa = wbase + uint32_t(slot * C::STAGE);
        const uint32_t sb = sa + uint32_t(OA::BYTES);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            floatx4 av[TM], bv[TN];
            read_all<OA>(ra, sa, s, av);
            read_all<OB>(rb, sb, s, bv);
            if (!A_KC && want_db) {
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) dsum[tm] += F::sum(av[tm]);
            }
            if constexpr (F::WIDE) {
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                        for (int tn = 0; tn < TN; ++tn)
                            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[tm][t], bv[tn][t], acc[tm][tn], 0, 0, 0);
            } else {
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = F::mfma(av[tm], bv[tn], acc[tm][tn]);
            }
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
                st1(mine + uint32_t((OA::idx(tm, acc_row(r, h)) * BN + OB::idx(tn, col)) * 4), acc[tm][tn][r]);
    if (!A_KC && want_db) {
        // Lane (col, h) holds the sum over its k of A row 32 tm + col: LDS [wave][h][BM].
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
            st1(red + uint32_t(C::RED + ((wave * 2 + h) * BM + OA::idx(tm, col)) * 4), dsum[tm]);
    }
    __syncthreads();
    if (!A_KC && want_db && int(threadIdx.x) < BM && m0 + int(threadIdx.x) < p.M) {
        // Sum in wave order, then lane-half order; one thread per row.
        const int m = int(threadIdx.x);
        float x = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) x += ld1(red + uint32_t(C::RED + ((w * 2 + hh) * BM + m) * 4));
        if (p.splits > 1) {
            p.ws[int64_t(p.nbatch) * p.splits * p.M * p.N + (int64_t(z) * p.splits + split) * p.M + m0 + m] = x;
        } else {
            char *dst = p.db[z] + int64_t(m0 + m) * F::EB;
            F::store(dst, F::load(dst) + x);
        }
    }

    // Sum the partials in wave order and store, 4 columns per thread.
    constexpr int Q = BM * BN / 4;
    char *const cz = p.c[z];
    const char *const bz = p.bias[z];
    for (int qi = int(threadIdx.x); qi < Q; qi += NW * 64) {
        const int m = qi / (BN / 4);
        const int n = (qi - m * (BN / 4)) * 4;
        const int gm = m0 + m, gn = n0 + n;
        if (gm >= p.M || gn >= p.N) continue;
        floatx4 x = ld4(red + uint32_t((m * BN + n) * 4));
#pragma unroll
        for (int w = 1; w < NW; ++w) x += ld4(red + uint32_t(((w * BM + m) * BN + n) * 4));
        if (p.splits > 1) {
            float *dst = p.ws + ((int64_t(z) * p.splits + split) * p.M + gm) * p.N + gn;
            if (p.N % 4 == 0) {
                *reinterpret_cast<floatx4 *>(dst) = x;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gn + e < p.N) dst[e] = x[e];
            }
            continue;
        }
        if (p.vec_out) {
            const int64_t off = rowoff(view_c, gm) + coloff(view_c, gn);
            char *dst = cz + off;
            if (bz != nullptr) x += F::load4(bz + int64_t(gn) * F::EB);
            if (p.beta) x += F::load4(dst);
            if (p.act_mode == 1) {
                floatx4 y;
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = act_fwd(p.act_kind, F::round(x[e]));
                F::store4(p.aux[z] + off, y);
            } else if (p.act_mode == 2) {
                const floatx4 pre = F::load4(p.aux[z] + off);
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = act_bwd_value(p.act_kind, pre[e], F::round(x[e]));
            }
            F::store4(dst, x);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (gn + e >= p.N) break;
                const int64_t off = rowoff(view_c, gm) + coloff(view_c, gn + e);
                char *de = cz + off;
                float y = x[e];
                if (bz != nullptr) y += F::load(bz + int64_t(gn + e) * F::EB);
                if (p.beta) y += F::load(de);
                if (p.act_mode == 1) F::store(p.aux[z] + off, act_fwd(p.act_kind, F::round(y)));
                else if (p.act_mode == 2) y = act_bwd_value(p.act_kind, F::load(p.aux[z] + off), F::round(y));
                F::store(de, y);
            }
        }
    }
}

// C_z(m, n) [+]= sum over splits s = 0, 1, ... of ws[z][s][m][n] (+ bias_z[n]), 4 columns per
// thread when vec (N % 4 == 0, aligned C), else one.
template <typename F>
__global__ __launch_bounds__(256) void lin_splitk_reduce_kernel(Args p, int64_t items_per_batch, int vec) {
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int z = int(blockIdx.y);
    const int w = vec ? 4 : 1;
    const int64_t mn = int64_t(p.M) * p.N;
    const int64_t e0 = idx * w;
    const int m = int(e0 / p.N), n = int(e0 - int64_t(m) * p.N);
    const float *src = p.ws + int64_t(z) * p.splits * mn + e0;
    const char *bz = p.bias[z];
    if (p.db[z] != nullptr && idx < p.M) {
        // Bias gradient: db[idx] += its split partials, in split order.
        const float *dsrc = p.ws + int64_t(p.nbatch) * p.splits * mn + int64_t(z) * p.splits * p.M + idx;
        float x = dsrc[0];
        for (int s = 1; s < p.splits; ++s) x += dsrc[int64_t(s) * p.M];
        char *dst = p.db[z] + idx * F::EB;
        F::store(dst, F::load(dst) + x);
    }
    if (idx >= items_per_batch) return;
    char *dst = p.c[z] + rowoff(p.cv, m) + coloff(p.cv, n);
    if (vec) {
        floatx4 x = *reinterpret_cast<const floatx4 *>(src);
        for (int s = 1; s < p.splits; ++s) x += *reinterpret_cast<const floatx4 *>(src + s * mn);
        if (bz != nullptr) x += F::load4(bz + int64_t(n) * F::EB);
        if (p.beta) x += F::load4(dst);
        F::store4(dst, x);
    } else {
        float x = src[0];
        for (int s = 1; s < p.splits; ++s) x += src[s * mn];
        if (bz != nullptr) x += F::load(bz + int64_t(n) * F::EB);
        if (p.beta) x += F::load(dst);
        F::store(dst, x);
    }
}

// ---- shared-tile products (16-bit storage; fp32 forwards) ----
//
// The kernels above give every wave its own tile, so each wave streams its own A and B rows
// from L2: a one-wave 128 x 64 tile stages 12 KB per 32-deep K chunk for 0.5 MFLOP, which at
// the 16-bit MFMA rate needs several times the L2 bandwidth a CU gets.  Here WM x WN waves
// share one (32 TM WM) x (32 TN WN) tile: each K stage (KS 64-byte chunks of every
// K-contiguous row, or KS 32-row chunks of an M/N-contiguous operand) goes global -> LDS once
// per workgroup, the direct loads split across the waves, through an S-slot ring with one
// barrier per stage, and wave (wm, wn) multiplies A rows wm by B columns wn.  Operands in any
// layout and view (a K-contiguous head-split stage inside one head, an M/N-contiguous one
// inside one batch), K segments and K splits across workgroups as lin_kernel, the bias
// gradient of an M-contiguous A summed by the first tile column.  fp32 (four k-steps of
// v_mfma_f32_32x32x2f32 per 16-byte operand) takes K-contiguous operands only.  GEN: some
// view is head-split or K has several segments.
template <typename F, bool A_KC, bool B_KC, int WM, int WN, int TM, int TN, int S, int KS>
struct ShCfg {
    static_assert(!F::WIDE || (A_KC && B_KC), "fp32: K-contiguous operands only");
    static constexpr int NW = WM * WN;
    static constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
    template <bool KC, int R>
    using Op = std::conditional_t<KC, std::conditional_t<KS == 1, OpKC<R>, OpKC2<R>>, OpMN16<R, 32 * KS>>;
    using OA = Op<A_KC, BM>;
    using OB = Op<B_KC, BN>;
    static constexpr int STAGE = OA::BYTES + OB::BYTES;
    static constexpr int LA = OA::NL / NW, LB = OB::NL / NW;  // load instructions per wave per stage
    static constexpr int L = LA + LB;
    static_assert(OA::NL % NW == 0 && OB::NL % NW == 0, "a stage's loads split evenly over the waves");
    static constexpr int PIPE = S * STAGE;
    static constexpr int EPI = 32 * TM * BN * 4;     // one wave row of the tile, fp32, for the stores
    static constexpr int DBB = A_KC ? 0 : 2 * BM * 4;  // bias-gradient sums per lane half
    static constexpr int LDS = PIPE > EPI + DBB ? PIPE : EPI + DBB;
    static_assert(LDS <= 160 * 1024, "LDS of one workgroup");
    static_assert(S >= 2 && (S - 1) * L < 64, "outstanding loads must fit vmcnt");
};

template <typename F, bool A_KC, bool B_KC, int WM, int WN, int TM, int TN, int S, int KS, bool GEN>
__global__ __launch_bounds__(WM * WN * 64) void lin_shared_kernel(Args p) {
    using C = ShCfg<F, A_KC, B_KC, WM, WN, TM, TN, S, KS>;
    using OA = typename C::OA;
    using OB = typename C::OB;
    constexpr int BM = C::BM, BN = C::BN, NW = C::NW;
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS];
    DView view_a = p.av, view_b = p.bv, view_c = p.cv;
    if constexpr (!GEN) view_a.heads = view_b.heads = view_c.heads = 0;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int wm = wave / WN, wn = wave - (wave / WN) * WN;
    const int h = lane >> 5, col = lane & 31;

    // XCD-aware order, as lin_kernel: XCD x runs the contiguous work items [x q, x q + q).
    const int nblk = int(gridDim.x), blk = int(blockIdx.x);
    const int q = nblk >> 3;
    const int work = blk < 8 * q ? (blk & 7) * q + (blk >> 3) : blk;
    const int ntiles = p.tiles_m * p.tiles_n;
    const int per_batch = ntiles * p.splits;
    const int z = work / per_batch;
    const int rem = work - z * per_batch;
    const int split = rem / ntiles;
    const int tile = rem - split * ntiles;
    const int ti = tile / p.tiles_n;
    const int m0 = ti * BM, n0 = (tile - ti * p.tiles_n) * BN;
    // This workgroup's stages (KS K chunks each; cps is a multiple of KS).
    const int st0 = split * (p.cps / KS);
    const int nst = min(p.chunks / KS - st0, p.cps / KS);
    const int sst = p.seg_chunks / KS;  // stages per segment

    const int64_t a_t = A_KC ? rowoff(view_a, m0) : coloff(view_a, m0);
    const int64_t b_t = B_KC ? rowoff(view_b, n0) : coloff(view_b, n0);
    uint32_t va[C::LA], vb[C::LB];
#pragma unroll
    for (int u = 0; u < C::LA; ++u) va[u] = OA::voff(wave + NW * u, lane, view_a, m0, p.M - m0);
#pragma unroll
    for (int u = 0; u < C::LB; ++u) vb[u] = OB::voff(wave + NW * u, lane, view_b, n0, p.N - n0);
    typename OA::Lane ra;
    typename OB::Lane rb;
    ra.init(lane);
    rb.init(lane);
    const uint32_t base = lds_addr(smem);

    auto issue = [&](int slot, int c) {
        const uint32_t sa = base + uint32_t(slot * C::STAGE);
        int seg = 0, cs = c;
        if constexpr (GEN) {
            seg = c / sst;
            cs = c - seg * sst;
        }
        // Stage cs of segment seg: K [kk, kk + KS KWE), inside one head / one batch.
        const int kk = cs * KS * F::KWE;
        const char *gac = pick(p.a[z], seg) + a_t + (A_KC ? coloff(view_a, kk) : rowoff(view_a, kk));
        const char *gbc = pick(p.b[z], seg) + b_t + (B_KC ? coloff(view_b, kk) : rowoff(view_b, kk));
#pragma unroll
        for (int u = 0; u < C::LA; ++u) dma16(gac, va[u], sa + uint32_t(1024 * (wave + NW * u)));
#pragma unroll
        for (int u = 0; u < C::LB; ++u) dma16(gbc, vb[u], sa + uint32_t(OA::BYTES + 1024 * (wave + NW * u)));
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = zero16();
    // Bias gradient of an M-contiguous A: the first tile column's waves of column 0 sum A.
    const bool want_db = !A_KC && p.db[z] != nullptr && n0 == 0;
    const bool sum_a = want_db && wn == 0;
    float dsum[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) dsum[i] = 0.f;

    const int pro = min(S - 1, nst);
    for (int j = 0; j < pro; ++j) issue(j, st0 + j);
    int slot = 0, islot = S - 1;
    for (int j = 0; j < nst; ++j) {
        // This wave's loads of stage j have landed once at most the later stages' are in
        // flight; after the barrier every wave's have, and every wave is done with the slot
        // the next issue refills (read in the previous iteration).
        wait_tail<C::L, S>(min(S - 2, nst - 1 - j));
        __syncthreads();
        if (j + S - 1 < nst) issue(islot, st0 + j + S - 1);
        const uint32_t sa = base + uint32_t(slot * C::STAGE);
        const uint32_t sb = sa + uint32_t(OA::BYTES);
        if constexpr (!F::WIDE && A_KC) {
            // 16-bit products with a K-contiguous A (forwards, dX): step s + 1's operands are
            // read before step s's MFMAs, and the scheduling fence keeps the compiler from
            // hoisting every step's reads to the top of the stage, so each step's MFMAs wait
            // only for reads issued a whole step earlier.
            floatx4 av[2][TM], bv[2][TN];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) av[0][tm] = ra.read(sa, TM * wm + tm, 0);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) bv[0][tn] = rb.read(sb, TN * wn + tn, 0);
#pragma unroll
            for (int s = 0; s < 2 * KS; ++s) {
                const int cur = s & 1;
                if (s + 1 < 2 * KS) {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm) av[cur ^ 1][tm] = ra.read(sa, TM * wm + tm, s + 1);
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) bv[cur ^ 1][tn] = rb.read(sb, TN * wn + tn, s + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = F::mfma(av[cur][tm], bv[cur][tn], acc[tm][tn]);
            }
        } else {
            // fp32 and the 16-bit weight gradients: the compiler schedules the stage's reads
            // (the same fence measured neutral in fp32 and 2-3.5 % slower on the transposed
            // M/N-contiguous reads).
#pragma unroll
            for (int s = 0; s < 2 * KS; ++s) {
                floatx4 av[TM], bv[TN];
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) av[tm] = ra.read(sa, TM * wm + tm, s);
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) bv[tn] = rb.read(sb, TN * wn + tn, s);
                if (!A_KC && sum_a) {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm) dsum[tm] += F::sum(av[tm]);
                }
                if constexpr (F::WIDE) {
                    // fp32: the 16-byte operand is four k-steps of v_mfma_f32_32x32x2f32.
#pragma unroll
                    for (int t = 0; t < 4; ++t)
#pragma unroll
                        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                            for (int tn = 0; tn < TN; ++tn)
                                acc[tm][tn] =
                                    __builtin_amdgcn_mfma_f32_32x32x2f32(av[tm][t], bv[tn][t], acc[tm][tn], 0, 0, 0);
                } else {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                        for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = F::mfma(av[tm], bv[tn], acc[tm][tn]);
                }
            }
        }
        slot = slot + 1 == S ? 0 : slot + 1;
        islot = islot + 1 == S ? 0 : islot + 1;
    }

    const uint32_t ebuf = base;
    if (!A_KC && want_db) {
        // Lane (col, h) holds the sum over its k of A row 32 (TM wm + tm) + col: LDS [h][BM]
        // past the store buffer; one thread per row adds the halves in order.
        const uint32_t dbuf = base + uint32_t(C::EPI);
        __syncthreads();  // the ring is no longer read
        if (sum_a) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) st1(dbuf + uint32_t((h * BM + 32 * (TM * wm + tm) + col) * 4), dsum[tm]);
        }
        __syncthreads();
        const int m = int(threadIdx.x);
        if (m < BM && m0 + m < p.M) {
            const float x = ld1(dbuf + uint32_t(m * 4)) + ld1(dbuf + uint32_t((BM + m) * 4));
            if (p.splits > 1) {
                p.ws[int64_t(p.nbatch) * p.splits * p.M * p.N + (int64_t(z) * p.splits + split) * p.M + m0 + m] = x;
            } else {
                char *dst = p.db[z] + int64_t(m0 + m) * F::EB;
                F::store(dst, F::load(dst) + x);
            }
        }
    }

    // Stores, one wave row of the tile (32 TM rows x BN columns) at a time through LDS:
    // register r of lane (col, h) holds row acc_row(r, h) of column col of each 32 x 32 tile.
    char *const cz = p.c[z];
    const char *const bz = p.bias[z];
    constexpr int Q = 32 * TM * BN / 4;
#pragma unroll 1
    for (int pm = 0; pm < WM; ++pm) {
        __syncthreads();  // the ring (or the previous pass) is no longer read
        if (wm == pm) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        st1(ebuf + uint32_t(((32 * tm + acc_row(r, h)) * BN + 32 * (TN * wn + tn) + col) * 4),
                            acc[tm][tn][r]);
        }
        __syncthreads();
        for (int qi = int(threadIdx.x); qi < Q; qi += NW * 64) {
            const int m = qi / (BN / 4);
            const int n = (qi - m * (BN / 4)) * 4;
            const int gm = m0 + pm * 32 * TM + m, gn = n0 + n;
            if (gm >= p.M || gn >= p.N) continue;
            floatx4 x = ld4(ebuf + uint32_t((m * BN + n) * 4));
            if (p.splits > 1) {
                float *dst = p.ws + ((int64_t(z) * p.splits + split) * p.M + gm) * p.N + gn;
                if (p.N % 4 == 0) {
                    *reinterpret_cast<floatx4 *>(dst) = x;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (gn + e < p.N) dst[e] = x[e];
                }
                continue;
            }
            if (p.vec_out) {
                const int64_t off = rowoff(view_c, gm) + coloff(view_c, gn);
                char *dst = cz + off;
                if (bz != nullptr) x += F::load4(bz + int64_t(gn) * F::EB);
                if (p.beta) x += F::load4(dst);
                if (p.act_mode == 1) {
                    floatx4 y;
#pragma unroll
                    for (int e = 0; e < 4; ++e) y[e] = act_fwd(p.act_kind, F::round(x[e]));
                    F::store4(p.aux[z] + off, y);
                } else if (p.act_mode == 2) {
                    const floatx4 pre = F::load4(p.aux[z] + off);
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = act_bwd_value(p.act_kind, pre[e], F::round(x[e]));
                }
                F::store4(dst, x);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (gn + e >= p.N) break;
                    const int64_t off = rowoff(view_c, gm) + coloff(view_c, gn + e);
                    char *de = cz + off;
                    float y = x[e];
                    if (bz != nullptr) y += F::load(bz + int64_t(gn + e) * F::EB);
                    if (p.beta) y += F::load(de);
                    if (p.act_mode == 1) F::store(p.aux[z] + off, act_fwd(p.act_kind, F::round(y)));
                    else if (p.act_mode == 2) y = act_bwd_value(p.act_kind, F::load(p.aux[z] + off), F::round(y));
                    F::store(de, y);
                }
            }
        }
    }
}

// ---- host side ----

struct Plan {
    int cfg;     // index into the configuration table of the layout
    int splits;  // K splits across workgroups
};

// One launchable configuration.
struct CfgInfo {
    int tm, tn, nw, s;
    hipError_t (*launch)(const Args &, int nblk, hipStream_t);      // row-major, one segment
    hipError_t (*launch_gen)(const Args &, int nblk, hipStream_t);  // any views / segments
};

template <typename F, bool A_KC, bool B_KC, int TM, int TN, int NW, int S, bool GEN>
hipError_t launch_cfg(const Args &a, int nblk, hipStream_t stream) {
    hipLaunchKernelGGL((lin_kernel<F, A_KC, B_KC, TM, TN, NW, S, GEN>), dim3(unsigned(nblk)), dim3(NW * 64), 0,
                       stream, a);
    return hipGetLastError();
}

template <typename F, bool A_KC, bool B_KC, int TM, int TN, int NW, int S>
constexpr CfgInfo cfg_info() {
    return CfgInfo{TM, TN, NW, S, &launch_cfg<F, A_KC, B_KC, TM, TN, NW, S, false>,
                   &launch_cfg<F, A_KC, B_KC, TM, TN, NW, S, true>};
}

inline int elem_bytes(int dtype) { return dtype == 0 ? 4 : 2; }
inline int chunk_elems(int dtype) { return 64 / elem_bytes(dtype); }

inline DView dview(const LinView &v, int eb) {
    DView d{};
    d.heads = v.heads;
    d.T = v.T;
    d.d = v.d;
    d.eb = eb;
    d.ld_b = v.ld * eb;
    d.hstr_b = int64_t(v.T) * v.d * eb;
    d.bstr_b = int64_t(v.heads) * v.T * v.d * eb;
    if (v.heads != 0) {
        d.tdiv = make_fastdiv(uint32_t(v.T));
        d.ddiv = make_fastdiv(uint32_t(v.d));
    }
    return d;
}

inline int64_t splits_bytes(const LinGemm &g, int splits) {
    return splits > 1 ? int64_t(splits) * g.nbatch * (g.M * g.N + g.M) * 4 : 0;
}

// Builds the kernel arguments of a product for a configuration and split count; returns the
// workgroup count.
inline int make_args(const LinGemm &g, const CfgInfo &c, int splits, void *ws, Args &a) {
    const int eb = elem_bytes(g.dtype);
    const int bm = 32 * c.tm, bn = 32 * c.tn;
    for (int z = 0; z < kLinMaxBatch; ++z) {
        const int zz = z < g.nbatch ? z : 0;
        for (int s = 0; s < kLinMaxSeg; ++s) {
            const int ss = s < g.nseg ? s : 0;
            a.a[z][s] = static_cast<const char *>(g.a[zz][ss]);
            a.b[z][s] = static_cast<const char *>(g.b[zz][ss]);
        }
        a.c[z] = static_cast<char *>(g.c[zz]);
        a.bias[z] = static_cast<const char *>(g.bias[zz]);
        a.db[z] = g.a_kc || z >= g.nbatch ? nullptr : static_cast<char *>(g.db[z]);
        a.aux[z] = static_cast<char *>(g.aux[zz]);
    }
    a.act_mode = g.act_mode;
    a.act_kind = g.act_kind;
    a.ws = static_cast<float *>(ws);
    a.av = dview(g.av, eb);
    a.bv = dview(g.bv, eb);
    a.cv = dview(g.cv, eb);
    a.M = int32_t(g.M);
    a.N = int32_t(g.N);
    a.tiles_m = int32_t((g.M + bm - 1) / bm);
    a.tiles_n = int32_t((g.N + bn - 1) / bn);
    a.nbatch = g.nbatch;
    a.seg_chunks = int32_t(g.K / chunk_elems(g.dtype));
    a.chunks = a.seg_chunks * g.nseg;
    a.cps = (a.chunks + splits - 1) / splits;
    a.splits = (a.chunks + a.cps - 1) / a.cps;  // no empty split
    a.beta = g.beta ? 1 : 0;
    bool vec = g.N % 4 == 0;
    for (int z = 0; z < g.nbatch; ++z)
        vec = vec && uintptr_t(g.c[z]) % (4 * eb) == 0 && (g.bias[z] == nullptr || uintptr_t(g.bias[z]) % (4 * eb) == 0) &&
              (g.act_mode == 0 || uintptr_t(g.aux[z]) % (4 * eb) == 0);
    if (g.cv.heads == 0) vec = vec && g.cv.ld % 4 == 0;
    a.vec_out = vec ? 1 : 0;
    return a.tiles_m * a.tiles_n * a.splits * g.nbatch;
}

// Some view is head-split or K has several segments (the kernels' GEN variant).
inline bool lin_gen(const LinGemm &g) {
    return g.nseg > 1 || g.av.heads != 0 || g.bv.heads != 0 || g.cv.heads != 0;
}

// The split-K reduction: C (and the bias gradients) from the partials of a.splits splits.
template <typename F>
hipError_t launch_reduce(const LinGemm &g, const Args &a, hipStream_t stream) {
    const int64_t items = a.vec_out ? g.M * g.N / 4 : g.M * g.N;
    const int64_t threads = std::max<int64_t>(items, g.M);  // bias gradients: one thread per row
    hipLaunchKernelGGL(lin_splitk_reduce_kernel<F>, dim3(unsigned((threads + 255) / 256), unsigned(g.nbatch)),
                       dim3(256), 0, stream, a, items, a.vec_out);
    return hipGetLastError();
}

template <typename F>
hipError_t run(const LinGemm &g, const CfgInfo &c, int splits, void *ws, int64_t ws_bytes, hipStream_t stream) {
    Args a{};
    const int nblk = make_args(g, c, splits, ws, a);
    if (a.splits > 1 && (ws == nullptr || ws_bytes < splits_bytes(g, a.splits))) return hipErrorInvalidValue;
    if (a.splits > 1 && g.act_mode != 0) return hipErrorInvalidValue;  // the epilogue applies it
    hipError_t e = (lin_gen(g) ? c.launch_gen : c.launch)(a, nblk, stream);
    if (e != hipSuccess || a.splits == 1) return e;
    return launch_reduce<F>(g, a, stream);
}

// Launch of the shared-tile kernel: WM x WN waves on a (32 TM WM) x (32 TN WN) tile, an S-slot
// ring of KS-chunk stages, K split across up to `splits` workgroups (ws: the partials).  The
// product must be one shared_plan (below) takes with KS.
template <typename F, bool A_KC, bool B_KC, int WM, int WN, int TM, int TN, int S, int KS>
hipError_t run_shared(const LinGemm &g, int splits, void *ws, int64_t ws_bytes, hipStream_t stream) {
    Args a{};
    const CfgInfo c{TM * WM, TN * WN, WM * WN, S, nullptr, nullptr};
    make_args(g, c, splits, ws, a);
    if (a.seg_chunks % KS != 0) return hipErrorInvalidValue;
    a.cps = (a.cps + KS - 1) / KS * KS;  // whole stages per split
    a.splits = (a.chunks + a.cps - 1) / a.cps;
    if (a.splits > 1 && (ws == nullptr || ws_bytes < splits_bytes(g, a.splits) || g.act_mode != 0))
        return hipErrorInvalidValue;
    const int nblk = a.tiles_m * a.tiles_n * a.splits * g.nbatch;
    if (lin_gen(g))
        hipLaunchKernelGGL((lin_shared_kernel<F, A_KC, B_KC, WM, WN, TM, TN, S, KS, true>), dim3(unsigned(nblk)),
                           dim3(WM * WN * 64), 0, stream, a);
    else
        hipLaunchKernelGGL((lin_shared_kernel<F, A_KC, B_KC, WM, WN, TM, TN, S, KS, false>), dim3(unsigned(nblk)),
                           dim3(WM * WN * 64), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splits == 1) return e;
    return launch_reduce<F>(g, a, stream);
}

// The shared-tile plan of a supported product: ks 0 (not taken), or the stage depth in K
// chunks (1 or 2) and the K split count.
struct SharedPlan {
    int ks, splits;
};

// Whether a view holds whole stages of `rows` K elements: a K-contiguous head-split stage
// inside one head, an M/N-contiguous one inside one batch.
inline bool stage_in_view(const LinView &v, bool kc, int rows) {
    return v.heads == 0 || (kc ? v.d % rows == 0 : v.T % rows == 0);
}

// fp32 forward products (both operands K-contiguous) with at least 768 tiles of 128 x 64 take
// it as 4 x 1 waves of 32 x 64, one 64-byte chunk (16 elements) per stage: in a sweep of the
// configurations, 8192 x 3072 x 1024 ran 400 against lin_kernel's 440 us, 4096^3 1029 against
// 1120, 4096 x 1536 x 384 45.7 against 52.1; with fewer tiles (4096 x 1152 x 384: 576) or
// short N and long K lin_kernel's split-K-in-workgroup tiles stayed ahead.
// 16-bit products take the shared-tile kernel, with two-chunk stages where every segment is an
// even number of chunks and the views hold whole stages:
//   * K-contiguous A (forward, dX): with at least 256 128 x 128 tiles, K never split (smaller
//     grids keep lin_kernel's smaller tiles and more workgroups);
//   * weight gradients (M/N-contiguous A): with at least 64 tiles, K split across
//     floor(512 / tiles) workgroups (two workgroups per CU fill the chip once; a split keeps
//     >= 8 stages, at most 16 splits) when the caller has workspace, else unsplit from 256
//     tiles.  Fitted to sweeps of 384..4096-wide products: e.g. dW of 3072 x 1024 over 8192
//     rows (192 tiles, 2 splits) 81 us against lin_kernel's 88, 4096^3 164 against 312.
inline SharedPlan shared_plan(const LinGemm &g, bool allow_split) {
    if (g.dtype == 0) {
        // fp32: both operands K-contiguous and at least 768 128 x 64 tiles, one-chunk stages.
        const int64_t t64 = ((g.M + 127) / 128) * ((g.N + 63) / 64) * g.nbatch;
        const bool ok = g.a_kc && g.b_kc && g.bv.heads == 0 && t64 >= 768 && t64 < (int64_t(1) << 24);
        return ok ? SharedPlan{1, 1} : SharedPlan{0, 1};
    }
    const int64_t tiles = ((g.M + 127) / 128) * ((g.N + 127) / 128) * g.nbatch;
    if (tiles >= (int64_t(1) << 24)) return SharedPlan{0, 1};
    const int64_t seg_chunks = g.K / 32;
    const bool two = seg_chunks % 2 == 0 && stage_in_view(g.av, g.a_kc, 64) && stage_in_view(g.bv, g.b_kc, 64);
    const int ks = two ? 2 : 1;
    if (g.a_kc) return tiles >= 256 ? SharedPlan{ks, 1} : SharedPlan{0, 1};
    if (tiles < 64) return SharedPlan{0, 1};
    const int64_t stages = seg_chunks * g.nseg / ks;
    const int64_t sp = allow_split ? std::min<int64_t>(std::min<int64_t>(512 / tiles, stages / 8), 16) : 1;
    if (sp >= 2) return SharedPlan{ks, int(sp)};
    return tiles >= 256 ? SharedPlan{ks, 1} : SharedPlan{0, 1};
}

// The shared-tile launch of a plan: 16-bit, 128 x 128 tiles of 2 x 2 waves; fp32, 128 x 64 tiles
// of 4 x 1 waves; 2 stages.
template <typename F, bool A_KC, bool B_KC>
hipError_t run_shared_ks(const LinGemm &g, const SharedPlan &sp, void *ws, int64_t ws_bytes, hipStream_t stream) {
    return sp.ks == 2 ? run_shared<F, A_KC, B_KC, 2, 2, 2, 2, 2, 2>(g, sp.splits, ws, ws_bytes, stream)
                      : run_shared<F, A_KC, B_KC, 2, 2, 2, 2, 2, 1>(g, sp.splits, ws, ws_bytes, stream);
}
template <typename F>
hipError_t run_shared_plan(const LinGemm &g, const SharedPlan &sp, void *ws, int64_t ws_bytes, hipStream_t stream) {
    if constexpr (F::WIDE) {
        return run_shared<F, true, true, 4, 1, 1, 2, 2, 1>(g, sp.splits, ws, ws_bytes, stream);
    } else {
        if (!g.a_kc) return run_shared_ks<F, false, false>(g, sp, ws, ws_bytes, stream);
        return g.b_kc ? run_shared_ks<F, true, true>(g, sp, ws, ws_bytes, stream)
                      : run_shared_ks<F, true, false>(g, sp, ws, ws_bytes, stream);
    }
}

}  // namespace lin

namespace {

using lin::BF16Fmt;
using lin::CfgInfo;
using lin::cfg_info;
using lin::F16Fmt;
using lin::F32Fmt;

// The launchable configurations per operand layout (tile 32 TM x 32 TN, NW waves, S-stage
// ring).  The choice among them (plan below) was fitted to forced-configuration sweeps over the
// products of a d384 and a d1024 transformer and a 4096^3 matmul: 132 fp32 configurations per
// layout, 82 bf16 ones.
template <typename F>
struct Tables {
    static constexpr CfgInfo fwd[] = {cfg_info<F, true, true, 2, 1, 4, 2>(), cfg_info<F, true, true, 2, 1, 1, 2>(),
                                      cfg_info<F, true, true, 2, 1, 1, 3>()};
    // An M/N-contiguous B is read through the two-tile interleaved operand (32 x 64 tiles).
    static constexpr CfgInfo dx[] = {cfg_info<F, true, false, 1, 2, 4, 2>(), cfg_info<F, true, false, 1, 2, 1, 2>(),
                                     cfg_info<F, true, false, 1, 2, 1, 3>()};
    static constexpr CfgInfo dw[] = {cfg_info<F, false, false, 1, 2, 4, 2>(), cfg_info<F, false, false, 2, 2, 8, 2>(),
                                     cfg_info<F, false, false, 1, 2, 8, 2>()};
};
// 16-bit storage: the MFMA does 16x the work per operand byte, so the tiles are larger (the
// 64 x 32 tiles of fp32 leave the 16-bit kernels bound by L2 and LDS bandwidth).
template <typename F>
struct Tables16 {
    static constexpr CfgInfo fwd[] = {cfg_info<F, true, true, 4, 2, 1, 3>(), cfg_info<F, true, true, 2, 2, 4, 2>()};
    static constexpr CfgInfo dx[] = {cfg_info<F, true, false, 2, 4, 1, 2>(), cfg_info<F, true, false, 2, 2, 4, 2>()};
    static constexpr CfgInfo dw[] = {cfg_info<F, false, false, 2, 2, 2, 2>()};
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Chooses a configuration (index into the layout's table) and a K split count.
// allow_split: the caller has workspace for split-K partials.
// fp32:
//   * Both operands M/N-contiguous (weight gradients: small output, K = rows): 64 x 64 tiles
//     of 8 waves when there are at least 256 of them; else 32 x 64 tiles, of 8 waves with K
//     split across workgroups up to 256 workgroups below 256 tiles, of 4 waves up to 1280
//     workgroups otherwise, each wave keeping >= 8 K chunks.
//   * Otherwise 64 x 32 (forward) or 32 x 64 (dX) tiles: 4 waves (K split inside the
//     workgroup) while there are fewer than 3072 tiles, else one wave per tile (3 stages once
//     K reaches 64 chunks, else 2).
// bf16 / fp16:
//   * weight gradients: 64 x 64 tiles of 2 waves, K split across workgroups below 512 tiles
//     (up to 1024 workgroups, each wave keeping >= 12 K chunks);
//   * the shared-tile kernel where shared_plan takes the product (chosen before this plan);
//   * otherwise, with at least 1024 64 x 64 tiles and 24 K chunks: one wave per 128 x 64
//     (forward) or 64 x 128 (dX) tile; else 64 x 64 tiles of 4 waves.
lin::Plan plan(const LinGemm &g, bool allow_split) {
    const int64_t chunks = g.K / lin::chunk_elems(g.dtype) * g.nseg;
    if (g.dtype != 0) {
        const int64_t t64 = cdiv(g.M, 64) * cdiv(g.N, 64) * g.nbatch;
        if (g.a_kc) return lin::Plan{t64 >= 1024 && chunks >= 24 ? 0 : 1, 1};
        if (t64 >= 512 || !allow_split) return lin::Plan{0, 1};
        const int64_t sp = std::min<int64_t>(cdiv(1024, t64), chunks / 24);
        return lin::Plan{0, int(std::max<int64_t>(1, std::min<int64_t>(sp, 16)))};
    }
    if (!g.a_kc) {
        if (cdiv(g.M, 64) * cdiv(g.N, 64) * g.nbatch >= 256) return lin::Plan{1, 1};
        const int64_t tiles = cdiv(g.M, 64) * cdiv(g.N, 32) * g.nbatch;
        const bool few = tiles < 256;
        int64_t sp = few ? std::min<int64_t>(256 / tiles, chunks / 64) : std::min<int64_t>(1280 / tiles, chunks / 32);
        sp = allow_split ? std::max<int64_t>(1, std::min<int64_t>(sp, 16)) : 1;
        return lin::Plan{few ? 2 : 0, int(sp)};
    }
    const int64_t tiles = cdiv(g.M, 64) * cdiv(g.N, 32) * g.nbatch;
    return lin::Plan{tiles < 3072 ? 0 : chunks >= 64 ? 2 : 1, 1};
}

template <typename Tb>
const CfgInfo &cfg_of(const LinGemm &g, const lin::Plan &pl) {
    if (!g.a_kc) return Tb::dw[pl.cfg];
    return g.b_kc ? Tb::fwd[pl.cfg] : Tb::dx[pl.cfg];
}
const CfgInfo &cfg_for(const LinGemm &g, const lin::Plan &pl) {
    return g.dtype == 0   ? cfg_of<Tables<F32Fmt>>(g, pl)
           : g.dtype == 1 ? cfg_of<Tables16<BF16Fmt>>(g, pl)
                          : cfg_of<Tables16<F16Fmt>>(g, pl);
}

// A view the kernels can address: 16-byte aligned row pitch and 32-bit lane offsets within a
// tile (linear); or head-split with every 64-byte K chunk inside one head (K-contiguous), or
// every 16-byte column chunk inside one head and every stage of k-rows inside one batch
// (M/N-contiguous).
bool view_ok(const LinView &v, bool kc, int dtype) {
    const int eb = lin::elem_bytes(dtype), kwe = lin::chunk_elems(dtype), ce = 16 / eb;
    if (v.heads == 0) return v.ld >= 0 && v.ld % ce == 0 && v.ld * eb <= (int64_t(1) << 24);
    if (v.heads < 1 || v.T < 1 || v.d < 1) return false;
    if (int64_t(v.heads) * v.T * v.d * eb >= (int64_t(1) << 30)) return false;  // tile offsets stay 32-bit
    return kc ? v.d % kwe == 0 : v.d % ce == 0 && v.T % kwe == 0;
}

// The shape / pitch part of lin_gemm_supported (pointers are not looked at).
bool shape_ok(const LinGemm &g) {
    if (g.dtype < 0 || g.dtype > 2 || (!g.a_kc && g.b_kc)) return false;
    // A fused activation: forward / dX layouts (never split), output not accumulated.
    if (g.act_mode != 0 && (g.act_mode > 2 || !g.a_kc || g.beta || g.act_kind < CTATTN_ACT_RELU ||
                            g.act_kind > CTATTN_ACT_TANH))
        return false;
    if (g.nbatch < 1 || g.nbatch > kLinMaxBatch || g.nseg < 1 || g.nseg > kLinMaxSeg) return false;
    const int kwe = lin::chunk_elems(g.dtype), ce = 16 / lin::elem_bytes(g.dtype);
    if (g.M < 1 || g.N < 1 || g.K < kwe || g.K % kwe != 0) return false;
    if (g.M > 2147483647 || g.N > 2147483647 || g.K * g.nseg > 2147483647) return false;
    // An M/N-contiguous operand is read in whole 16-byte chunks of its M / N extent.
    if ((!g.a_kc && g.M % ce != 0) || (!g.b_kc && g.N % ce != 0)) return false;
    if (!view_ok(g.av, g.a_kc, g.dtype) || !view_ok(g.bv, g.b_kc, g.dtype)) return false;
    // The output: a linear pitch of at least N, or head-split with 4-column groups in one head.
    if (g.cv.heads == 0 ? g.cv.ld < g.N : (g.cv.d % 4 != 0 || g.cv.T < 1)) return false;
    // Launch size: workgroups x threads below 2^32.
    const lin::Plan pl = plan(g, true);
    const CfgInfo &c = cfg_for(g, pl);
    const int64_t wg = cdiv(g.M, 32 * c.tm) * cdiv(g.N, 32 * c.tn) * pl.splits * g.nbatch;
    return wg * c.nw * 64 < (int64_t(1) << 32);
}

}  // namespace

LinGemm lin_plain(int dtype, bool a_kc, bool b_kc, int64_t M, int64_t N, int64_t K, const void *a, int64_t lda,
                  const void *b, int64_t ldb, void *c, int64_t ldc, const void *bias, bool beta) {
    LinGemm g{};
    g.dtype = dtype;
    g.a_kc = a_kc;
    g.b_kc = b_kc;
    g.M = M;
    g.N = N;
    g.K = K;
    g.nbatch = 1;
    g.nseg = 1;
    g.av = lin_linear(lda);
    g.bv = lin_linear(ldb);
    g.cv = lin_linear(ldc);
    g.a[0][0] = a;
    g.b[0][0] = b;
    g.c[0] = c;
    g.bias[0] = bias;
    g.beta = beta;
    return g;
}

bool lin_gemm_supported(const LinGemm &g) {
    if (!shape_ok(g)) return false;
    for (int z = 0; z < g.nbatch; ++z) {
        if (g.c[z] == nullptr || (g.act_mode != 0 && g.aux[z] == nullptr)) return false;
        for (int s = 0; s < g.nseg; ++s)
            if (g.a[z][s] == nullptr || g.b[z][s] == nullptr || uintptr_t(g.a[z][s]) % 16 != 0 ||
                uintptr_t(g.b[z][s]) % 16 != 0)
                return false;
    }
    return true;
}

int64_t lin_gemm_workspace_bytes(const LinGemm &g) {
    if (!shape_ok(g)) return 0;
    // The launch trims empty splits, never adds any: this is an upper bound.
    const lin::SharedPlan sp = lin::shared_plan(g, true);
    return lin::splits_bytes(g, sp.ks != 0 ? sp.splits : plan(g, true).splits);
}

hipError_t launch_lin_gemm(const LinGemm &g, void *ws, int64_t ws_bytes, hipStream_t stream) {
    if (!lin_gemm_supported(g)) return hipErrorInvalidValue;
    lin::SharedPlan sp = lin::shared_plan(g, true);
    if (sp.splits > 1 && (ws == nullptr || ws_bytes < lin::splits_bytes(g, sp.splits))) sp = lin::shared_plan(g, false);
    if (sp.ks != 0)
        return g.dtype == 0   ? lin::run_shared_plan<F32Fmt>(g, sp, ws, ws_bytes, stream)
               : g.dtype == 1 ? lin::run_shared_plan<BF16Fmt>(g, sp, ws, ws_bytes, stream)
                              : lin::run_shared_plan<F16Fmt>(g, sp, ws, ws_bytes, stream);
    lin::Plan pl = plan(g, true);
    if (pl.splits > 1 && (ws == nullptr || ws_bytes < lin::splits_bytes(g, pl.splits))) pl = plan(g, false);
    const CfgInfo &c = cfg_for(g, pl);
    switch (g.dtype) {
        case 0: return lin::run<F32Fmt>(g, c, pl.splits, ws, ws_bytes, stream);
        case 1: return lin::run<BF16Fmt>(g, c, pl.splits, ws, ws_bytes, stream);
        default: return lin::run<F16Fmt>(g, c, pl.splits, ws, ws_bytes, stream);
    }
}

}  // namespace ctattn
