// bf16 LDS tile machinery shared by the bf16 attention kernels (gfx950): swizzled row-major
// tiles loaded global -> LDS directly, row and transposed (ds_read_b64_tr_b16) MFMA operand
// reads by explicit LDS byte address, and the bf16 / fp16 32x32x16 MFMA formats.
//
// 32x32x16 operand layout (lane l, col = l & 31, half = l >> 5): A[i][k] comes from lane
// (i, k / 8) element k % 8, B[k][j] from lane (j, k / 8) element k % 8; accumulator register r
// of lane (j, half) holds row acc_row(r, half) of column j.
#pragma once

#include "attn_mfma_common.h"

#include <stdint.h>

namespace ctattn {
namespace bf16tile {

#define CTATTN_LDS(p) ((__attribute__((address_space(3))) void *)(p))

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// The two 16-bit formats of these kernels.  bf16 and IEEE fp16 share the tiles, the
// operand layout (32x32x16, 8 elements per lane) and every address; they differ in the MFMA
// instruction and in the rounding of fp32 values to 16 bits (nearest even for both).
struct Bf16Fmt {
    using vec = bf16x8;
    using elem = __bf16;
    __device__ static floatx16 mfma(vec a, vec b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static uint16_t bits(float x) { return f32_to_bf16(x).bits; }
    __device__ static float widen(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
};
struct F16Fmt {
    using vec = f16x8;
    using elem = _Float16;
    __device__ static floatx16 mfma(vec a, vec b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    __device__ static uint16_t bits(float x) { return __builtin_bit_cast(uint16_t, _Float16(x)); }
    __device__ static float widen(uint16_t b) { return float(__builtin_bit_cast(_Float16, b)); }
};

// Row-major bf16 tile with D elements (D / 8 16-byte chunks) per row.  Logical chunk c of
// row r sits at physical chunk c ^ swz(r).  The LDS has 64 four-byte banks (256 bytes per
// bank row); swz makes
//   * a row read (lanes 0-15: rows r0..r0+15, one chunk) and
//   * a transposed read (lanes 0-31: rows R..R+3, R % 4 == 0, chunks C..C+3, C % 4 == 0)
// touch each bank once.
template <int D>
struct Tile {
    static_assert(D == 32 || D == 64 || D == 128, "bf16 MFMA kernels support d in {32, 64, 128}");
    static constexpr int CH = D / 8;         // 16-byte chunks per row
    static constexpr int ROW_BYTES = 2 * D;  // bytes per row
    __device__ static constexpr int swz(int r) {
        return D == 128 ? 4 * (r & 3) + ((r >> 2) & 3)
             : D == 64  ? 4 * ((r >> 1) & 1) + ((r >> 2) & 3)
                        : (r >> 2) & 3;
    }
    __device__ static int off(int r, int chunk) { return r * ROW_BYTES + ((chunk ^ swz(r)) << 4); }
};

// Loads rows r0 .. r0 + ROWS - 1 of one (batch, head)'s [T][D] tensor into a swizzled tile:
// lane writes the 16-byte LDS chunk P = (wave * NL + i) * 64 + lane, i.e. row P / CH,
// physical chunk P % CH, which holds logical chunk (P % CH) ^ swz(row).  Rows past T re-read
// row T - 1 (their results are masked).  Every wave calls this; waves past the tile skip.
template <int D, int ROWS, int NW>
__device__ __forceinline__ void load_tile(char *tile, const uint16_t *src, int r0, int T, int wave, int lane) {
    using L = Tile<D>;
    constexpr int TOTAL = ROWS * L::CH;
    constexpr int NL = (TOTAL + NW * kWave - 1) / (NW * kWave);
    static_assert(TOTAL % kWave == 0, "tile size");
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int P = (wave * NL + i) * kWave + lane;
        if (TOTAL % (NW * kWave) == 0 || (wave * NL + i) * kWave < TOTAL) {
            const int r = P / L::CH;
            const int lc = (P % L::CH) ^ L::swz(r);
            const uint16_t *g = src + int64_t(min(r0 + r, T - 1)) * D + 8 * lc;
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(g),
                                             CTATTN_LDS(tile + (wave * NL + i) * kWave * 16), 16, 0, 0);
        }
    }
}

// The same load with a wave-uniform block base (src + r0 * D, in SGPRs) and a 32-bit per-lane
// offset, so the load uses saddr + voffset addressing and keeps no 64-bit address per lane;
// rows at or past `rows` (the rows left in the sequence, uniform) re-read row rows - 1.
template <int D, int ROWS, int NW>
__device__ __forceinline__ void load_tile_u(char *tile, const uint16_t *block, int rows, int wave, int lane) {
    using L = Tile<D>;
    constexpr int TOTAL = ROWS * L::CH;
    constexpr int NL = (TOTAL + NW * kWave - 1) / (NW * kWave);
    static_assert(TOTAL % kWave == 0, "tile size");
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int P = (wave * NL + i) * kWave + lane;
        if (TOTAL % (NW * kWave) == 0 || (wave * NL + i) * kWave < TOTAL) {
            const int r = P / L::CH;
            const int lc = (P % L::CH) ^ L::swz(r);
            const uint32_t e = uint32_t(min(r, rows - 1) * D + 8 * lc);
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(block + e),
                                             CTATTN_LDS(tile + (wave * NL + i) * kWave * 16), 16, 0, 0);
        }
    }
}

// The same load issued through inline asm.  The compiler does not see these loads, so it
// never makes an LDS read wait (s_waitcnt vmcnt) for them -- it would for every read it cannot
// prove disjoint from an in-flight load, which exposes a prefetch's whole latency at the next
// read of the other buffer.  The kernel itself waits (wait_loads) before the barrier that
// publishes the tile.  The LDS destination of a wave's load goes to m0 (a lane's 16 bytes land
// at m0 + 16 lane); it is wave-uniform.
template <int D, int ROWS, int NW>
__device__ __forceinline__ void load_tile_dma(const char *tile, const uint16_t *block, int rows, int wave, int lane) {
    using L = Tile<D>;
    constexpr int TOTAL = ROWS * L::CH;
    constexpr int NL = (TOTAL + NW * kWave - 1) / (NW * kWave);
    static_assert(TOTAL % kWave == 0, "tile size");
    const uint32_t tile_lds = uint32_t(uintptr_t((__attribute__((address_space(3))) const char *)tile));
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int P = (wave * NL + i) * kWave + lane;
        if (TOTAL % (NW * kWave) == 0 || (wave * NL + i) * kWave < TOTAL) {
            const int r = P / L::CH;
            const int lc = (P % L::CH) ^ L::swz(r);
            const uint16_t *g = block + uint32_t(min(r, rows - 1) * D + 8 * lc);
            // m0 takes an SGPR: the destination is wave-uniform, readfirstlane makes that explicit.
            const uint32_t dst = __builtin_amdgcn_readfirstlane(tile_lds + uint32_t((wave * NL + i) * kWave * 16));
            asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(dst)
                         : "memory", "m0");
        }
    }
}

// One dword per lane, global -> LDS, through inline asm like load_tile_dma: lane l's value
// lands at LDS byte address `dst` + 4 l (`dst` wave-uniform).
__device__ __forceinline__ void load_dword_dma(const void *g, uint32_t dst) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(dst))
                 : "memory", "m0");
}

// LDS reads by byte address (LDS addresses are 32-bit).
typedef __attribute__((address_space(3))) const u16x8 lds_u16x8;
typedef __attribute__((address_space(3))) const floatx4 lds_floatx4;

template <typename V> __device__ __forceinline__ V lds_b128(uint32_t addr) {
    return __builtin_bit_cast(V, *(lds_u16x8 *)(uintptr_t)(addr));
}
__device__ __forceinline__ floatx4 lds_f4(uint32_t addr) { return *(lds_floatx4 *)(uintptr_t)(addr); }

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return uint32_t(uintptr_t((__attribute__((address_space(3))) const char *)p));
}

// Operand reads.  Tiles start on 1 KiB boundaries and a row's chunk field occupies address
// bits 4 .. 4 + log2(D / 8) - 1, so with row_base(r) = tile + Tile::off(r, half):
//   * row read, step st (elements 16 st + 8 half .. + 7 of row r):  row_base ^ (st << 5),
//     because (2 st + half) ^ swz = (2 st) ^ (half ^ swz);
//   * column read, d-tile dt (column 32 dt + col), k-step kk: rows 16 kk + 4 half + e and
//     16 kk + 8 + 4 half + (e - 4) -- the row order of accumulator registers 8 kk .. 8 kk + 7
//     -- from two ds_read_b64_tr_b16 at (col_base[hi] ^ (dt << 6)) + 16 kk * ROW, hi = 0, 1.
//     In each 16-lane group, lane s addresses 4 elements of row R + s / 4 at column
//     cb + 4 (s % 4) and lane l receives column cb + l of rows R .. R + 3; the swizzle of those
//     rows does not depend on kk and flips only the chunk bits that dt sets (bits 6, 7).
template <int D>
__device__ __forceinline__ uint32_t row_base(uint32_t tile, int r, int half) {
    return tile + uint32_t(Tile<D>::off(r, half));
}
template <int D>
__device__ __forceinline__ uint32_t col_base(uint32_t tile, int r0, int hi, int lane) {
    const int s = lane & 15;
    const int half = lane >> 5;
    const int chunk = 2 * ((lane >> 4) & 1) + ((s & 3) >> 1);
    return tile + uint32_t(Tile<D>::off(r0 + 4 * half + (s >> 2) + 8 * hi, chunk) + 8 * (s & 1));
}
template <int D, typename V>
__device__ __forceinline__ V read_col(uint32_t cb0, uint32_t cb1, int kk, int dt) {
    const uint32_t off = uint32_t(16 * kk * 2 * D);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(uintptr_t)((cb0 ^ uint32_t(dt << 6)) + off));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(uintptr_t)((cb1 ^ uint32_t(dt << 6)) + off));
    const i16x8 x = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(V, x);
}

// Operand reads through pointers into a __shared__ tile (`off` is the byte offset from the
// tile's start, as row_base / col_base compute it for tile = 0).  Keeping the pointer's
// provenance, instead of a raw LDS address, lets the compiler see which tile an access
// touches: reads of one buffer then do not wait (s_waitcnt vmcnt) for global -> LDS loads
// still in flight into another, provided the buffers are distinct __shared__ arrays.
template <typename V> __device__ __forceinline__ V tile_b128(const char *tile, uint32_t off) {
    return __builtin_bit_cast(V, *(__attribute__((address_space(3))) const u16x8 *)(tile + off));
}
template <int D, typename V>
__device__ __forceinline__ V tile_col(const char *tile, uint32_t cb0, uint32_t cb1, int kk, int dt) {
    const uint32_t off = uint32_t(16 * kk * 2 * D);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(tile + ((cb0 ^ uint32_t(dt << 6)) + off)));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(tile + ((cb1 ^ uint32_t(dt << 6)) + off)));
    const i16x8 x = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(V, x);
}

// Workgroup barrier that leaves global -> LDS loads in flight (__syncthreads first waits for
// every outstanding memory operation of the wave, prefetches included).  The wave's own LDS
// reads and writes are complete when it arrives; the "memory" clobber keeps the compiler from
// moving memory accesses across it.  Loads whose data the next phase reads must be awaited
// (s_waitcnt vmcnt) before it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0xF70); }  // vmcnt(0)

// max(x, x of lane ^ 32) in one v_permlane32_swap: the swap leaves the partner's value in one
// of the two results and the lane's own in the other.
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Scheduling fence between a step's operand reads and the previous step's MFMAs: nothing
// crosses it, so step st + 1's reads are issued before step st's MFMAs and about two steps'
// operands are live at once (the MFMAs of step st wait only for step st's reads).
__device__ __forceinline__ void read_fence() { __builtin_amdgcn_sched_barrier(0); }

}  // namespace bf16tile
}  // namespace ctattn
