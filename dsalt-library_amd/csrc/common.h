// Device-side building blocks shared by the gfx950 DSALT kernels: MFMA wrappers for
// bf16/fp16, wave64 reductions, the packed-sequence block lookup and launch constants.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <limits.h>

namespace dsalt {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From &x) {
    static_assert(sizeof(To) == sizeof(From), "bitcast size mismatch");
    return __builtin_bit_cast(To, x);
}

// 16-bit element types. Storage is always raw uint16_t; `vec8` is the MFMA operand of
// v_mfma_f32_32x32x16_{bf16,f16}: 8 consecutive K-elements of one M row (A) or one N
// column (B) per lane, lane l covering row/column l%32 and K-elements (l/32)*8..+7.
struct BF16 {
    typedef bf16x8 vec8;
    static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    // Round-to-nearest-even pack of two fp32 values (v_cvt_pk_bf16_f32).
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        bf16x2 v = {(__bf16)lo, (__bf16)hi};
        return bitcast<uint32_t>(v);
    }
    static __device__ __forceinline__ float to_f32(uint16_t x) {
        return __uint_as_float(((uint32_t)x) << 16);
    }
    // the low / high element of a packed pair
    static __device__ __forceinline__ float lo_f32(uint32_t x) { return __uint_as_float(x << 16); }
    static __device__ __forceinline__ float hi_f32(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
    // x rounded to the nearest bf16 (ties to even), returned as fp32
    static __device__ __forceinline__ float round(float x) { return (float)(__bf16)x; }
    // acc + lo + hi of a packed pair, in fp32 (v_dot2c_f32_bf16 against (1, 1))
    static __device__ __forceinline__ float add_pair(uint32_t x, float acc) {
        const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(x), one, acc, false);
    }
};

struct F16 {
    typedef f16x8 vec8;
    static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        f16x2 v = {(_Float16)lo, (_Float16)hi};
        return bitcast<uint32_t>(v);
    }
    static __device__ __forceinline__ float to_f32(uint16_t x) {
        return (float)bitcast<_Float16>(x);
    }
    static __device__ __forceinline__ float lo_f32(uint32_t x) { return to_f32((uint16_t)x); }
    static __device__ __forceinline__ float hi_f32(uint32_t x) { return to_f32((uint16_t)(x >> 16)); }
    // x rounded to the nearest fp16 (ties to even), returned as fp32
    static __device__ __forceinline__ float round(float x) { return (float)(_Float16)x; }
    // acc + lo + hi of a packed pair, in fp32 (v_dot2c_f32_f16 against (1, 1))
    static __device__ __forceinline__ float add_pair(uint32_t x, float acc) {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(bitcast<f16x2>(x), one, acc, false);
    }
};

// Row index (within a 32-row MFMA block) of accumulator register r of a lane in half
// `hh` (= lane / 32): the 32x32 accumulator holds, for column lane%32, the rows
// (r/4)*8 + hh*4 + r%4. acc_row_const() is the part that does not depend on the lane.
__device__ __forceinline__ constexpr int acc_row_const(int r) { return (r >> 2) * 8 + (r & 3); }

// ---- wave64 reductions (all lanes receive the result) ----------------------------
__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ int wave_sum(int x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}
__device__ __forceinline__ float wave_sumf(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    return x;
}

// Combine the two 32-lane halves of a wave (lanes l and l^32 hold the same query
// column in the 32x32 MFMA layout): v_permlane32_swap returns both halves, so one
// swap plus one VALU op gives the pair maximum / sum in every lane.
__device__ __forceinline__ float half_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max(a, b, c) as one v_maximum3_f32 (gfx950). IEEE maximum propagates NaN and needs
// no quieted inputs; through fmaxf (maxNum) the compiler quiets MFMA results with an
// extra v_max_f32 x, x per operand before combining them.
__device__ __forceinline__ float max3f(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Bounds of sequence s as the kernels use them: cu_seqlens entries clamped to [0, T] and
// the end to at least the start. For every packing with 0 <= cu[0] <= ... <= cu[S] <= T
// this is (cu[s], cu[s+1]); for any other content of cu_seqlens it still keeps every row
// a kernel reads or writes inside the T rows of its tensors.
__device__ __forceinline__ void seq_bounds(const int32_t *__restrict__ cu, int s, int total_len, int &c0, int &c1) {
    c0 = min(max(cu[s], 0), total_len);
    c1 = max(min(cu[s + 1], total_len), c0);
}

// Workgroup ids over the query (or key) blocks of a packed batch. Sequence s (start
// cu[s], length L_s) owns the ceil(L_s / bm) consecutive ids starting at
// first(s) = floor(cu[s] / bm) + s. first() is strictly increasing and the ranges are
// disjoint; the largest id is at most ceil(T / bm) + S - 2, so a grid of
// block_upper_bound(T, S, bm) ids covers every block, and the ids in the gaps between
// ranges map to no block (false). The lookup is one coalesced load of 64 cu_seqlens
// entries and a ballot per 64 sequences - no prefix sum and no host-side block map,
// so launches need no device-to-host synchronisation. Every lane returns the same
// (wave-uniform) answer, with the sequence's start and length.
__device__ __forceinline__ bool find_block(const int32_t *__restrict__ cu, int num_seqs, int total_len,
                                           int target, int bm, int lane, int &seq, int &blk, int &seq_start,
                                           int &seq_len) {
    int cand = -1, cand_first = 0, cand_start = 0, cand_end = 0;
    for (int base = 0; base < num_seqs; base += 64) {
        const int s = base + lane;
        int c0 = 0, c1 = 0, first = INT_MAX;
        if (s < num_seqs) {
            seq_bounds(cu, s, total_len, c0, c1);
            first = c0 / bm + s;
        }
        const unsigned long long m = __ballot(first <= target);  // a prefix of the lanes
        if (m == 0) break;
        const int last = 63 - __clzll((long long)m);
        cand = base + last;
        cand_first = __builtin_amdgcn_readlane(first, last);
        cand_start = __builtin_amdgcn_readlane(c0, last);
        cand_end = __builtin_amdgcn_readlane(c1, last);
        if (last < 63) break;
    }
    if (cand < 0) return false;
    const int len = cand_end - cand_start;
    if (target - cand_first >= (len + bm - 1) / bm) return false;
    seq = cand;
    blk = target - cand_first;
    seq_start = cand_start;
    seq_len = len;
    return true;
}
__device__ __forceinline__ bool find_block(const int32_t *__restrict__ cu, int num_seqs, int total_len,
                                           int target, int bm, int lane, int &seq, int &blk) {
    int start, len;
    return find_block(cu, num_seqs, total_len, target, bm, lane, seq, blk, start, len);
}

// Wave-uniform reductions over all 64 lanes without LDS: DPP quad/row permutations
// reduce each row of 16 lanes, then the four row results are read as scalars.
template <typename Op>
__device__ __forceinline__ int wave_reduce_dpp(int x, Op op) {
    x = op(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    x = op(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    x = op(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false));  // row_half_mirror
    x = op(x, __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false));  // row_mirror
    const int r0 = __builtin_amdgcn_readlane(x, 0), r1 = __builtin_amdgcn_readlane(x, 16);
    const int r2 = __builtin_amdgcn_readlane(x, 32), r3 = __builtin_amdgcn_readlane(x, 48);
    return op(op(r0, r1), op(r2, r3));
}
struct MinOp {
    __device__ __forceinline__ int operator()(int a, int b) const { return min(a, b); }
};
struct MaxOp {
    __device__ __forceinline__ int operator()(int a, int b) const { return max(a, b); }
};
__device__ __forceinline__ int wave_min_u(int x) { return wave_reduce_dpp(x, MinOp()); }
__device__ __forceinline__ int wave_max_u(int x) { return wave_reduce_dpp(x, MaxOp()); }

// Window modes of the kernels. kSoft and kSoftWide have the same SOFT semantics and
// differ only in how the forward applies the window edge: kSoft starts the scores of
// each query from a short row of edge biases (at most ceil(win_edge) = 4 edge keys);
// kSoftWide computes the bias on every band element below the core (wider edges). The
// backward instantiates kHard and kSoft only.
enum { kHard = 0, kSoft = 1, kSoftWide = 2 };

// Key ranges of query offset i (all inclusive, relative to its sequence) given its
// window value wv:
//   lo     first band key           HARD: max(0, i - w + 1), w = max(1, trunc(wv)), NaN -> 1
//                                   SOFT: max(0, i - floor(w~)); i + 1 (empty) if w~ < 0 / NaN
//   corelo first zero-bias key      HARD: lo; SOFT: i - floor(w~ - win_edge) (fp32 difference),
//                                   i + 1 when that difference is negative
//   pmax   largest admissible landmark position (-1: none)
//                                   HARD: p <= i - w            (dsalt_triton_attn.py:133-135)
//                                   SOFT: p <= i and (float)p < (float)i - w~ (dsalt_triton_train.py:183-185)
// The SOFT band 0 <= i-j <= w~ (dsalt_triton_train.py:147-150) is j >= i - floor(w~) for
// integer j, and the core test d <= w~ - win_edge (:154) is j >= i - floor(w~ - win_edge).
template <int MODE>
__device__ __forceinline__ void query_ranges(int i, float wv, float win_edge, int &lo, int &corelo,
                                             int &pmax) {
    if (MODE == kHard) {
        const int wi = (wv >= 1.f) ? (int)fminf(wv, 1073741824.f) : 1;
        lo = max(0, i - wi + 1);
        corelo = lo;
        pmax = lo - 1;
    } else {
        lo = (wv >= 0.f) ? max(0, i - (int)floorf(fminf(wv, 1073741824.f))) : i + 1;
        const float wce = wv - win_edge;
        corelo = (wce >= 0.f) ? i - (int)floorf(fminf(wce, 1073741824.f)) : i + 1;
        corelo = max(corelo, lo);
        const float t = (float)i - wv;  // p admissible <=> p <= ceil(t) - 1 (and p <= i)
        pmax = (t == t) ? (int)fminf(fmaxf(ceilf(fminf(t, 1073741824.f)) - 1.f, -1.f), (float)i) : -1;
    }
}

// Soft window edge of key distance d for continuous window w~: returns
// log2(sigmoid(z)) with z = (w~ - d) / tau (the logit bias log sigmoid(z) in log2 units,
// dsalt_triton_train.py:152-155) and, through `one_minus_sig`, 1 - sigmoid(z), which is
// tau * d(log sigmoid(z))/d w~ (dsalt_triton_train.py:370-373).
__device__ __forceinline__ float soft_edge_log2(float wc, float d, float inv_tau, float &one_minus_sig) {
    const float z = (wc - d) * inv_tau;
    const float e = __builtin_amdgcn_exp2f(-z * kLog2e);  // exp(-z)
    const float onep = 1.f + e;
    one_minus_sig = e / onep;
    return -__builtin_amdgcn_logf(onep);
}

// Workgroup index remap for the 8 XCDs of MI355X. Consecutive hardware workgroup ids
// are dispatched round-robin over the XCDs; remapping them so that each XCD receives a
// contiguous range of logical ids keeps neighbouring query/key blocks (which share
// K/V rows) on the same XCD and therefore in the same L2. `grid` must be a multiple of 8.
__device__ __forceinline__ int xcd_remap(int bid, int grid) {
    const int per = grid >> 3;
    return (bid & 7) * per + (bid >> 3);
}

// (head, rank) of hardware workgroup `bid` in a grid of n_heads x n_rank items (grid a
// multiple of 8). When n_heads is a multiple of 8, XCD x = bid % 8 owns the heads
// [x * n_heads / 8, (x + 1) * n_heads / 8) (their K/V rows stay in one L2) and receives
// its items rank-major, the heads interleaved: rank 0 of every head first. Otherwise XCD
// x owns a contiguous range of head-major items. `head` may be >= n_heads for padding.
// K/V head of query head `head` when `rep` consecutive query heads share one K/V head
// (grouped-query attention); a uniform branch, no division without grouping.
__device__ __forceinline__ int kv_head(int head, int rep) { return rep == 1 ? head : head / rep; }

__device__ __forceinline__ void head_rank(int bid, int grid, int n_heads, int n_rank, int &head, int &rank) {
    if ((n_heads & 7) == 0) {
        const int hpx = n_heads >> 3, j = bid >> 3;
        head = (bid & 7) * hpx + j % hpx;
        rank = j / hpx;
    } else {
        const int logical = xcd_remap(bid, grid);
        head = logical / n_rank;
        rank = logical - head * n_rank;
    }
}

struct AddOp {
    __device__ __forceinline__ int operator()(int a, int b) const { return a + b; }
};
__device__ __forceinline__ int wave_sum_u(int x) { return wave_reduce_dpp(x, AddOp()); }

// Block of rank `rank` (0 <= rank < n_rank) when the blocks of all sequences are taken
// in decreasing block index, ties in increasing sequence order: the late blocks of the
// sequences, whose key ranges are the longest, are dispatched first and the short
// first blocks of every sequence last, which shortens the tail of a launch. Ranks past
// the number of blocks map to no block (false). Level b (block index b) holds the
// sequences with more than b blocks; C(b) = sum_s max(0, nblk_s - b) ranks lie at levels
// >= b, so the level of `rank` is the largest b with C(b) > rank (binary search over
// DPP wave sums) and its sequence is the (rank - C(b+1))-th of that level. One lane per
// sequence: more than 64 sequences use find_block over reversed ids instead.
__device__ __forceinline__ bool find_block_desc(const int32_t *__restrict__ cu, int num_seqs, int total_len,
                                                int rank, int n_rank, int bm, int lane, int &seq, int &blk,
                                                int &seq_start, int &seq_len) {
    if (num_seqs > 64)
        return find_block(cu, num_seqs, total_len, n_rank - 1 - rank, bm, lane, seq, blk, seq_start, seq_len);
    int c0 = 0, c1 = 0, nblk = 0;
    if (lane < num_seqs) {
        seq_bounds(cu, lane, total_len, c0, c1);
        nblk = (c1 - c0 + bm - 1) / bm;
    }
    if (rank >= wave_sum_u(nblk)) return false;
    int lo = 0, hi = wave_max_u(nblk);  // C(lo) > rank >= C(hi) = 0
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (wave_sum_u(max(nblk - mid, 0)) > rank) lo = mid;
        else hi = mid;
    }
    const int j = rank - wave_sum_u(max(nblk - lo - 1, 0));
    const unsigned long long level = __ballot(nblk > lo);
    const int before = __builtin_amdgcn_mbcnt_hi((uint32_t)(level >> 32),
                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)level, 0u));
    const int s = __builtin_ctzll(__ballot(((level >> lane) & 1ull) && before == j));
    seq = s;
    blk = lo;
    seq_start = __builtin_amdgcn_readlane(c0, s);
    seq_len = __builtin_amdgcn_readlane(c1, s) - seq_start;
    return true;
}

}  // namespace dsalt
