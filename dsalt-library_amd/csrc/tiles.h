// LDS tiles of ROWS (64 or 32) rows x D 16-bit elements (rows are tokens: keys or queries), filled
// with direct global->LDS loads (buffer_load_dwordx4 ... lds) and read back as
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

template <int D, int ROWS = 64, int NW = 4>
struct TileN {
    static constexpr int CPR = D / 8;                              // 16-byte chunks per row
    static constexpr int ROWB = D * 2;                             // bytes per row
    static constexpr int BYTES = ROWS * ROWB;                      // bytes per tile
    static constexpr int LOADS_PER_WAVE = ROWS * CPR / (64 * NW);  // load instructions per wave
    static_assert(ROWS * CPR % (64 * NW) == 0, "NW waves x 64 lanes must cover the tile's 16-byte chunks");
};
template <int D>
using Tile64 = TileN<D, 64>;

// Byte address in LDS of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource (V#) over `bytes` bytes at `base`: loads at byte offsets >= bytes
// (including offsets that wrapped below 0) are out of range and return zeros instead of
// faulting. Word 3 is the gfx9 default (32-bit dwords, no swizzle, no stride).
__device__ __forceinline__ i32x4 buffer_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    i32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
    r.z = __builtin_amdgcn_readfirstlane((int)bytes);
    r.w = 0x00020000;
    return r;
}

// A descriptor re-read as wave-uniform, for callers whose loops the compiler cannot
// prove uniform: it may otherwise hold the descriptor in vector registers, which the "s"
// operand of the direct loads below does not accept.
__device__ __forceinline__ i32x4 uniform_rsrc(i32x4 r) {
    r.x = __builtin_amdgcn_readfirstlane(r.x);
    r.y = __builtin_amdgcn_readfirstlane(r.y);
    r.z = __builtin_amdgcn_readfirstlane(r.z);
    r.w = __builtin_amdgcn_readfirstlane(r.w);
    return r;
}

// buffer_load_dwordx4 ... lds: lane i's 16 bytes at byte offset voff of the buffer land
// at LDS byte m0 + 16 * i. `lds` must be wave-uniform (it is moved into m0).
__device__ __forceinline__ void dma16(uint32_t voff, i32x4 rsrc, uint32_t lds) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}

// This wave's share of the direct loads of one tile (NW waves cover the tile): LPW load
// instructions per tile, counted by vmcnt. Physical chunk slot g holds logical chunk
// (g % CPR) ^ swz(row) of tile row g / CPR. The per-lane parts (tile row, byte offset of
// the row and chunk for a given row stride) are computed once; a band tile then costs
// one add per load, a gathered tile one multiply-add.
template <int D, int SWZ, int ROWS = 64, int NW = 4>
struct TileLanes {
    static constexpr int CPR = D / 8, LPW = TileN<D, ROWS, NW>::LOADS_PER_WAVE;
    int row[LPW];
    uint32_t chunk_off[LPW];  // byte offset of the lane's chunk inside its row
    uint32_t lane_off[LPW];   // row * stride + chunk_off
    __device__ __forceinline__ TileLanes(int wave, int lane, uint32_t stride) {
#pragma unroll
        for (int u = 0; u < LPW; ++u) {
            const int g = (wave * LPW + u) * 64 + lane;
            row[u] = g / CPR;
            chunk_off[u] = (uint32_t)(((g % CPR) ^ tile_swz<SWZ>(row[u])) << 4);
            uint32_t m = (uint32_t)row[u] * stride;
            asm volatile("" : "+v"(m));  // no v_mad_u64_u32 (it would hold chunk_off as a pair)
            lane_off[u] = m + chunk_off[u];
        }
    }
    __device__ __forceinline__ static uint32_t lds_slot(uint32_t tile_lds, int wave, int u) {
        return __builtin_amdgcn_readfirstlane(tile_lds + (wave * LPW + u) * 64 * 16);
    }
    // Rows row0 .. row0+ROWS-1 (row0 * stride = base_off, may wrap below 0) into the tile at
    // LDS byte tile_lds (wave-uniform).
    __device__ __forceinline__ void load_band(uint32_t tile_lds, int wave, i32x4 rsrc, uint32_t base_off) const {
#pragma unroll
        for (int u = 0; u < LPW; ++u) dma16(base_off + lane_off[u], rsrc, lds_slot(tile_lds, wave, u));
    }
    // When the rows of consecutive loads of a lane are 8 apart (D = 64), every load has
    // the swizzle of the first, so later offsets are lane_off[0] plus a uniform step:
    // one register per tile side instead of LPW.
    static constexpr int ROWSTEP = 64 / CPR;
    __device__ __forceinline__ void load_band(uint32_t tile_lds, int wave, i32x4 rsrc, uint32_t base_off,
                                              uint32_t stride) const {
#pragma unroll
        for (int u = 0; u < LPW; ++u) {
            if constexpr (ROWSTEP % 8 == 0) {
                // opaque uniform sum: otherwise lane_off[0] + step is hoisted out of the
                // tile loop into a register of its own
                uint32_t b = base_off + (uint32_t)(u * ROWSTEP) * stride;
                asm volatile("" : "+s"(b));
                dma16(b + lane_off[0], rsrc, lds_slot(tile_lds, wave, u));
            }
            else
                dma16(base_off + lane_off[u], rsrc, lds_slot(tile_lds, wave, u));
        }
    }
    // Tile row r from buffer row rows[r], with the lane's tile row and chunk recomputed
    // from the lane id (mbcnt) instead of held in registers across a tile loop.
    __device__ __forceinline__ static void load_gather_lean(uint32_t tile_lds, int wave, i32x4 rsrc, uint32_t stride,
                                                            const int *rows) {
        int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        asm volatile("" : "+v"(lane));  // opaque: nothing derived from it is hoisted out of the loop
#pragma unroll
        for (int u = 0; u < LPW; ++u) {
            const int g = (wave * LPW + u) * 64 + lane;
            const int r = g / CPR;
            const uint32_t chunk = (uint32_t)(((g % CPR) ^ tile_swz<SWZ>(r)) << 4);
            uint32_t off = (uint32_t)rows[r] * stride;
            asm volatile("" : "+v"(off));
            dma16(off + chunk, rsrc, lds_slot(tile_lds, wave, u));
        }
    }
    // Tile row r from buffer row rows[r].
    __device__ __forceinline__ void load_gather(uint32_t tile_lds, int wave, i32x4 rsrc, uint32_t stride,
                                                const int *rows) const {
#pragma unroll
        for (int u = 0; u < LPW; ++u) {
            // 32-bit multiply, then add: left to itself the compiler fuses these into
            // v_mad_u64_u32, which holds chunk_off as a 64-bit register pair
            uint32_t off = (uint32_t)rows[row[u]] * stride;
            asm volatile("" : "+v"(off));
            dma16(off + chunk_off[u], rsrc, lds_slot(tile_lds, wave, u));
        }
    }
};

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
// The tile is conflict-free for this pattern with the kSwzTr swizzle; a kSwzRow tile
// (read both ways) serves it with 2-way bank conflicts.
template <int D, int SWZ = kSwzTr>
__device__ __forceinline__ uint4 tile_read_tr(const char *tile, int row0, int col0, int lane) {
    const int row = row0 + ((lane >> 5) << 2) + ((lane >> 2) & 3);
    const int col = col0 + (((lane >> 4) & 1) << 4) + ((lane & 3) << 2);
    const int c = col >> 3, half = (col >> 2) & 1;
    const char *a = tile + row * Tile64<D>::ROWB + ((c ^ tile_swz<SWZ>(row)) << 4) + (half << 3);
    const shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) shortx4 *)a);
    // row + 8 has the same swizzle (row & 7 and row & 3 unchanged)
    const shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) shortx4 *)(a + 8 * Tile64<D>::ROWB));
    const uint2 l2 = bitcast<uint2>(lo), h2 = bitcast<uint2>(hi);
    return make_uint4(l2.x, l2.y, h2.x, h2.y);
}

constexpr uint32_t kNegInfBits = 0xff800000u;

// Bit (rb*16 + r) of a lane's 32-bit tile mask stands for accumulator element
// sacc[rb][r], i.e. tile row rb*32 + acc_row_const(r) + hh*4. The row offset
// rb*32 + acc_row_const(r) increases with the bit index, so the elements whose offset
// is <= a form a prefix of the bits.
__device__ __forceinline__ uint32_t rows_le(int a) {
    const int n = min(max(4 * (a >> 3) + min((a & 7) + 1, 4), 0), 32);  // 0 for a < 0
    return (uint32_t)((1ull << n) - 1ull);
}

// x if bit j of `mask` is set, else -inf. With j a compile-time constant this is
// v_bfe_i32 + v_bfi_b32: no compare into a lane-mask SGPR (and no hazard wait after it).
__device__ __forceinline__ float keep_if(uint32_t mask, int j, float x) {
    const uint32_t m = (uint32_t)((int32_t)(mask << (31 - j)) >> 31);
    return __uint_as_float((m & __float_as_uint(x)) | (~m & kNegInfBits));
}

}  // namespace dsalt
