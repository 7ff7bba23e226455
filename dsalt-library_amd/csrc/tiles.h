// LDS tiles of 64 rows x D 16-bit elements (rows are tokens: keys or queries), filled
// with direct global->LDS loads (global_load_lds_dwordx4, gfx950) and read back as
// v_mfma_f32_32x32x16 operands.
//
// The direct loads are issued through inline asm and completed with explicit
// s_waitcnt vmcnt(N) + s_barrier (tile_barrier): when the compiler sees an LDS DMA it
// must assume every later LDS read may alias it and every workgroup fence must drain
// it, so it emits s_waitcnt vmcnt(0) before each tile read and each __syncthreads -
// which would wait for the tiles being prefetched as well and serialise the ring. Rows are unpadded; the 16-byte chunks of each row are
// XOR-swizzled so that the two read patterns are bank-conflict free:
//   swz_row  : chunk ^ (row & 7)          row-major operand reads (16 B per lane, 8
//                                         consecutive rows, same logical chunk)
//   swz_tr   : chunk ^ ((row & 3) << 1)   transposing reads (ds_read_b64_tr_b16: 4
//                                         consecutive rows x 2 chunks x 2 halves)
#pragma once

#include "common.h"

namespace dsalt {

typedef short shortx4 __attribute__((ext_vector_type(4)));

enum { kSwzRow = 0, kSwzTr = 1 };

template <int SWZ>
__device__ __forceinline__ int tile_swz(int row) {
    return SWZ == kSwzRow ? (row & 7) : ((row & 3) << 1);
}

template <int D>
struct Tile64 {
    static constexpr int CPR = D / 8;                    // 16-byte chunks per row
    static constexpr int ROWB = D * 2;                   // bytes per row
    static constexpr int BYTES = 64 * ROWB;              // bytes per tile
    static constexpr int LOADS_PER_WAVE = 64 * CPR / 256;  // 64-lane load instructions per wave
};

// Byte address in LDS of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}

// global_load_lds_dwordx4: lane i's 16 bytes at `src` land at LDS byte m0 + 16 * i.
// `lds` must be wave-uniform (it is moved into m0).
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

// This wave's share of the direct loads of one tile (4 waves cover the tile): LPW load
// instructions, counted by vmcnt. Physical chunk slot g holds logical chunk
// (g % CPR) ^ swz(row) of row g / CPR; `row_src(row)` returns the byte address of that
// row's element 0 in global memory (always a valid address: callers clamp out-of-range
// rows onto a real row and mask them later). `tile_lds` = lds_addr(tile), wave-uniform.
template <int D, int SWZ, typename RowSrc>
__device__ __forceinline__ void tile_load_async(uint32_t tile_lds, int wave, int lane, RowSrc row_src) {
    constexpr int CPR = Tile64<D>::CPR, LPW = Tile64<D>::LOADS_PER_WAVE;
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
        const int slot0 = (wave * LPW + u) * 64;
        const int g = slot0 + lane;
        const int row = g / CPR;
        const int c = (g % CPR) ^ tile_swz<SWZ>(row);
        dma16(row_src(row) + c * 16, __builtin_amdgcn_readfirstlane(tile_lds + slot0 * 16));
    }
}

// Wait until at most N of this wave's vector-memory operations are outstanding (they
// complete in issue order), i.e. until every direct load issued before the last N has
// landed in LDS, drain this wave's LDS operations, then synchronise the workgroup: after
// it every wave may read what every wave's completed loads wrote, and every wave's
// earlier LDS reads are done (their buffers may be refilled).
template <int N>
__device__ __forceinline__ void tile_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Row-major operand read: 16 bytes = logical chunk c of `row` (8 consecutive elements).
template <int D>
__device__ __forceinline__ uint4 tile_read_row16(const char *tile, int row, int c) {
    return *reinterpret_cast<const uint4 *>(tile + row * Tile64<D>::ROWB + ((c ^ tile_swz<kSwzRow>(row)) << 4));
}

// Transposed operand for a k-step over 16 tile rows starting at `row0` and head-dim
// column block `col0` (32 columns): lane l receives, in order, rows
// row0 + (l/32)*4 + {0..3} and row0 + 8 + (l/32)*4 + {0..3} of column col0 + l%32 -
// the row order of the packed P / dS registers of the MFMA accumulator layout.
// ds_read_b64_tr_b16 gives lane l element l%4 of the 8-byte chunks addressed by lanes
// 16*(l/16) + 4e + (l%16)/4, e = 0..3; each lane therefore addresses row
// row0 + (l/32)*4 + ((l%16)/4) and the 4 columns col0 + 16*((l/16)%2) + 4*(l%4).
template <int D>
__device__ __forceinline__ uint4 tile_read_tr(const char *tile, int row0, int col0, int lane) {
    const int row = row0 + ((lane >> 5) << 2) + ((lane >> 2) & 3);
    const int col = col0 + (((lane >> 4) & 1) << 4) + ((lane & 3) << 2);
    const int c = col >> 3, half = (col >> 2) & 1;
    const char *a = tile + row * Tile64<D>::ROWB + ((c ^ tile_swz<kSwzTr>(row)) << 4) + (half << 3);
    const shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) shortx4 *)a);
    // row + 8 has the same swizzle ((row & 3) unchanged)
    const shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) shortx4 *)(a + 8 * Tile64<D>::ROWB));
    const uint2 l2 = bitcast<uint2>(lo), h2 = bitcast<uint2>(hi);
    return make_uint4(l2.x, l2.y, h2.x, h2.y);
}

}  // namespace dsalt
