// DSALT sparse-attention backward for gfx950 (HARD and SOFT semantics), deterministic
// and atomic-free.
//
// Reference semantics: _train_bwd_preprocess / _train_bwd_kernel / _train_bwd_dkdv_kernel
// (dsalt/kernels/dsalt_triton_train.py:220-481) and _dsalt_bwd_preprocess /
// _dsalt_bwd_kernel (dsalt/kernels/dsalt_triton_bwd.py:17-216):
//   P = exp(logit - LSE), dP = dO . V^T, Delta_i = sum_d O_i dO_i, dS = P (dP - Delta)
//   dQ = scale * dS K, dK = scale * dS^T Q, dV = P^T dO
//   d_bias[h,s,slot] = sum_i dS[i, slot]                                   (:325-327)
//   d_w~[i] = sum_h sum_{edge keys j} dS[i, j] (1 - sigmoid(z_ij)) / tau_win  (:370-373, :748)
// The reference adds landmark dK/dV, d_bias and d_w~ with atomics; here every output
// element is produced by exactly one thread, in a fixed order.
//
// Kernels, launched in this order on one stream:
//   dq      query-parallel, kDqW waves x 32 queries per workgroup, the forward's tiling
//           (band tiles of kDqBN keys, then gathered landmark tiles); S^T, dP^T and dQ^T
//           on MFMA. Computes
//           Delta = rowsum(O * dO) for its queries and writes dQ, the per-head soft-edge
//           d_w~, the per-query records of the key-parallel passes and (head 0) the
//           block's smallest band start, which bounds the query scan of `kv` (workspace).
//   lmk_kv  key-parallel over landmark slots: one workgroup per (head, 64 slots, chunk of
//           512 queries of one sequence); 4 waves = 2 slot groups x 2 query sub-blocks scan
//           the chunk's queries in 64-query LDS tiles. Writes landmark dK/dV and d_bias
//           partials per chunk (workspace).
//   kv      key-parallel band dK/dV, kv_waves(D) waves x 32 keys per workgroup, scanning
//           kv_qt(D)-query LDS tiles from the key block to the last dq query block whose
//           band reaches it; keys that are landmark positions start from their landmark
//           dK/dV (the lmk_kv chunk partials summed in chunk order in the prologue); its
//           head-0 workgroups reduce d_w~ over heads, and H x S workgroups appended to its
//           grid sum the d_bias partials of each (head, sequence).
// Every MFMA is v_mfma_f32_32x32x16 with operands in the layouts of the forward kernel:
// a lane owns one column (query or key) of each 32x32 block and 16 rows of it.
#include "common.h"
#include "launch.h"
#include "tiles.h"

#include <algorithm>
#include <type_traits>

namespace dsalt {
namespace {

// band kv workgroups: waves (32 keys each), queries per tile and LDS ring depth; at
// D = 128 one 32-query sub-block per tile would need more than 256 VGPRs
constexpr int kv_waves(int d) { return d == 64 ? 2 : 4; }
constexpr int kv_bm(int d) { return 32 * kv_waves(d); }  // keys per band kv workgroup
constexpr int kv_qt(int d) { return d == 64 ? 32 : 64; }
constexpr int kv_stages(int) { return 4; }
constexpr int kTN = 64;     // queries per lmk_kv tile
constexpr int kDqW = 2;     // waves per dq workgroup
constexpr int kDqBM = 64;   // queries per dq workgroup (32 per wave)
constexpr int kDqBN = 32;   // keys per dq tile
constexpr int kDqStages = 3;  // dq LDS ring depth
constexpr int kLC = 512;  // queries per lmk_kv chunk (chunks are numbered like query blocks)

enum { kCoreTile = 0, kEdgeTile = 1, kLmkTile = 2 };  // tile kinds of the dq loop phases

// Per-(head, query) record written by dq and streamed by kv next to the Q / dO tiles,
// field-major ([H][field][T]) so that one field of a 64-query tile is one 256-byte
// direct load (two fields of a 32-query tile share one). Integer fields are encoded so that an all-zero record (what an
// out-of-range load returns) admits no key: lo and corelo as INT_MAX - x, pmax as x + 1.
enum {
    kRecLse2 = 0,    // -LSE / scale: minus the LSE in raw q.k units (float; -inf * sign(scale)
                     // for empty rows), the initial value of an S accumulator
    kRecDelta = 1,   // -rowsum(O * dO) (float), the initial value of a dP accumulator
    kRecLo = 2,      // INT_MAX - first band key
    kRecClo = 3,     // INT_MAX - first zero-bias band key (SOFT core start)
    kRecPmax = 4,    // largest admissible landmark position + 1
    kRecWc = 5,      // window w~ (float)
    kRecGLo = 6,     // INT_MAX - min lo over the query's 32-query group
    kRecGClo = 7,    // INT_MAX - max corelo over the query's 32-query group
    kRecFields = 8
};

struct BwdParams {
    const uint16_t *q, *k, *v, *dout;
    const void *o;  // forward output: fp32 if o_f32, else the compute dtype
    const float *lse, *w;
    const int64_t *lmk_pos;
    const float *lmk_bias;
    const int32_t *cu;
    void *dq, *dk, *dv;  // gradient outputs: fp32 if grad_f32, else the compute dtype
    float *d_bias, *d_w;
    float *ws_qrec;          // per-query records [H][kRecFields][T], written by bwd_dq_kernel
    int *ws_minlo;           // [n_dqblk]: smallest band start of each dq query block
    float *ws_dwh;           // [T*H] or null
    float *ws_ldk, *ws_ldv;  // landmark dK/dV partials [H][n_lchunk][k_pad][D] or null
    float *ws_ldb;           // landmark d_bias partials [H][n_lchunk][k_pad] or null
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, do_st, do_sh, lse_st, lse_sh, w_st;
    int64_t lp_sh, lp_ss, lp_sk, lb_sh, lb_ss, lb_sk;
    int64_t dq_st, dq_sh, dk_st, dk_sh, dv_st, dv_sh;
    int total_len, num_seqs, n_heads, k_lmk, k_pad, n_qblk, grid_q, n_dqblk, grid_dq, n_lgrp, n_lchunk, grad_f32, o_f32;
    int kv_rep;  // query heads per K/V head
    float scale, scale_log2, inv_tau, win_edge;
    float inv_c2;  // 1 / scale_log2: log2-unit bias -> raw q.k units
};

__device__ __forceinline__ uint4 ld16(const uint16_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// A operand of a k-step over 16 tokens from a transposed tile row: 4 tokens at `at` and
// 4 at `at + 8` (the token order of the packed P/dS registers, see the forward kernel).
template <typename vec8>
__device__ __forceinline__ vec8 ld_tr_operand(const uint16_t *at) {
    const uint2 a = *reinterpret_cast<const uint2 *>(at);
    const uint2 b = *reinterpret_cast<const uint2 *>(at + 8);
    return bitcast<vec8>(make_uint4(a.x, a.y, b.x, b.y));
}

// Store D/32 transposed 32x32 accumulator blocks (lane = row token, registers = head-dim
// (r/4)*8 + hh*4 + r%4) times `mul` as one row of a gradient tensor: fp32 when `f32`,
// else the 16-bit compute dtype.
template <typename DT, int ND>
__device__ __forceinline__ void store_row(void *base, int64_t off, bool f32, const f32x16 (&acc)[ND],
                                          float mul, int hh) {
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int dd = d * 32 + g * 8 + hh * 4;
            if (f32) {
                *reinterpret_cast<float4 *>(static_cast<float *>(base) + off + dd) =
                    make_float4(acc[d][g * 4] * mul, acc[d][g * 4 + 1] * mul, acc[d][g * 4 + 2] * mul,
                                acc[d][g * 4 + 3] * mul);
            } else {
                uint2 val;
                val.x = DT::pack2(acc[d][g * 4 + 0] * mul, acc[d][g * 4 + 1] * mul);
                val.y = DT::pack2(acc[d][g * 4 + 2] * mul, acc[d][g * 4 + 3] * mul);
                *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(base) + off + dd) = val;
            }
        }
}

template <typename DT>
__device__ __forceinline__ void pack_block(const f32x16 &x, uint32_t (&pk)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) pk[j] = DT::pack2(x[2 * j], x[2 * j + 1]);
}

// ==================================================================================
// dq: query-parallel dQ (band + landmarks) and per-head soft-edge d_w~
// ==================================================================================
// The forward's structure: one workgroup = kDqW waves x 32 queries of one (sequence,
// head); K and V tiles of kDqBN keys stream through a kDqStages-deep LDS ring by direct
// global->LDS loads (band tiles from the diagonal down, then the gathered landmark
// tiles). Small workgroups and tiles keep the LDS ring (24 KB at D = 64) and the
// registers small enough for 3 workgroups per SIMD set at D = 64. Per tile a wave
// computes S^T = K.Q^T and dP^T = V.dO^T (lane = query column), P = 2^(S c + bias - lse2)
// on admitted pairs, dS = P (dP - Delta), and dQ^T += K^T.dS^T with K read transposed.
template <typename DT, int D, int MODE, bool EFAST>
__global__ void __launch_bounds__(64 * kDqW, D == 64 ? 3 : 2) bwd_dq_kernel(const BwdParams p) {
    typedef typename DT::vec8 vec8;
    constexpr int NW = kDqW, BM = kDqBM, NT = 64 * NW;
    constexpr int BN = kDqBN, NRB = BN / 32;
    constexpr int KS = D / 16, ND = D / 32;
    typedef TileN<D, BN, NW> Tile;
    constexpr int TB = Tile::BYTES;
    constexpr int NSTAGE = kDqStages;
    constexpr int LPT = 2 * Tile::LOADS_PER_WAVE;

    __shared__ __align__(1024) char s_tiles[NSTAGE][2][TB];  // [stage][K, V], both row-swizzled
    __shared__ int s_red[NW][2];
    __shared__ int s_ltmin[DSALT_MAX_K_LMK / BN];
    // SOFT edge factors ec[j] = exp((kEdgeMid - cst_j) / tau) of the element slots j
    __shared__ __align__(16) float s_ec[16 * NRB];
    extern __shared__ int s_dyn[];
    int *s_lpos = s_dyn;                                          // INT_MAX: empty slot
    float *s_lbias = reinterpret_cast<float *>(s_dyn + p.k_pad);  // log2 units
    int *s_lrow = s_dyn + 2 * p.k_pad;
    // SOFT edge tiles (EFAST, chosen by dq_edge_fast on the host): exp(-z) of an edge key
    // factors as E ec[j], both factors in the fp32 range while (win_edge + 1 + 16 NRB) / tau
    // < 80 (edge keys have 0 <= z < (win_edge + 1) / tau); otherwise each element takes
    // its own exp. One path per instantiation keeps the kernel within its scalar registers.
    constexpr float kEdgeMid = 16.f * NRB - 2.5f;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    // the forward's dispatch order: XCDs own whole heads, and blocks arrive rank-major over
    // the heads in decreasing block index (the long late blocks of every sequence first,
    // the short first blocks last, in the last dispatch round)
    int head, rank;
    head_rank(blockIdx.x, p.grid_dq, p.n_heads, p.n_dqblk, head, rank);
    if (head >= p.n_heads) return;
    int seq, blk, seq_start, seq_len;
    if (!find_block_desc(p.cu, p.num_seqs, p.total_len, rank, p.n_dqblk, BM, lane, seq, blk, seq_start, seq_len)) return;
    const int target = seq_start / BM + seq + blk;  // the block's find_block id (ws_minlo index)
    const int wq0 = blk * BM + wave * 32;
    const int i = wq0 + ql;
    const bool qvalid = i < seq_len;
    const int64_t tok_i = (int64_t)seq_start + i;
    const int ghi = min(blk * BM + BM - 1, seq_len - 1);

    // ---- tile staging (band tiles from the diagonal down, then landmark tiles) ---------
    const uint32_t kst = (uint32_t)p.k_st * 2u, vst = (uint32_t)p.v_st * 2u;
    const i32x4 krs = buffer_rsrc(p.k + (int64_t)seq_start * p.k_st + (int64_t)kv_head(head, p.kv_rep) * p.k_sh, (uint32_t)seq_len * kst);
    const i32x4 vrs = buffer_rsrc(p.v + (int64_t)seq_start * p.v_st + (int64_t)kv_head(head, p.kv_rep) * p.v_sh, (uint32_t)seq_len * vst);
    const TileLanes<D, kSwzRow, BN, NW> klanes(wave, lane, kst);
    const TileLanes<D, kSwzRow, BN, NW> vlanes(wave, lane, vst);
    const uint32_t tiles_lds = lds_addr(&s_tiles[0][0][0]);
    auto band_key0 = [&](int t) { return ghi - (BN - 1) - t * BN; };
    auto stage_of = [](int t) { return t % NSTAGE; };  // t >= 0, wave-uniform
    auto issue_band = [&](int t) {
        const int key0 = band_key0(t);
        const uint32_t kl = tiles_lds + stage_of(t) * (2 * TB);
        klanes.load_band(kl, wave, krs, (uint32_t)key0 * kst);  // wraps when key0 < 0
        vlanes.load_band(kl + TB, wave, vrs, (uint32_t)key0 * vst);
    };
#pragma unroll
    for (int t = 0; t < NSTAGE - 1; ++t) issue_band(t);

    // ---- this lane's query: Q and dO as B operands, LSE, Delta, ranges ------------------
    vec8 qv[KS], dov[KS];
    {
        const uint16_t *qp = p.q + tok_i * p.q_st + (int64_t)head * p.q_sh + hh * 8;
        const uint16_t *dp = p.dout + tok_i * p.do_st + (int64_t)head * p.do_sh + hh * 8;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            uint4 a = make_uint4(0, 0, 0, 0), b = a;
            if (qvalid) {
                a = ld16(qp + s * 16);
                b = ld16(dp + s * 16);
            }
            qv[s] = bitcast<vec8>(a);
            dov[s] = bitcast<vec8>(b);
        }
    }
    const float lsev = qvalid ? p.lse[tok_i * p.lse_st + (int64_t)head * p.lse_sh] : -INFINITY;
    const float lse2 = (lsev == -INFINITY) ? INFINITY : lsev * kLog2e;  // +inf: every P is 0
    // Delta_i = sum_d O_i dO_i with O as stored (fp32 when the forward wrote fp32) and dO
    // in the compute dtype (dsalt_triton_train.py:673-674): this lane holds the dims
    // s*16 + hh*8 .. +7 of dO (its B operand), the other half-wave the rest
    float delta;
    {
        float acc = 0.f;
        if (qvalid) {
            const int64_t ooff = tok_i * p.o_st + (int64_t)head * p.o_sh + hh * 8;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const uint4 d8 = bitcast<uint4>(dov[s]);
                const uint16_t *de = reinterpret_cast<const uint16_t *>(&d8);
                float of[8];
                if (p.o_f32) {
                    const float *op = static_cast<const float *>(p.o) + ooff + s * 16;
                    const float4 x = *reinterpret_cast<const float4 *>(op);
                    const float4 y = *reinterpret_cast<const float4 *>(op + 4);
                    of[0] = x.x; of[1] = x.y; of[2] = x.z; of[3] = x.w;
                    of[4] = y.x; of[5] = y.y; of[6] = y.z; of[7] = y.w;
                } else {
                    const uint4 o8 = ld16(static_cast<const uint16_t *>(p.o) + ooff + s * 16);
                    const uint16_t *oe = reinterpret_cast<const uint16_t *>(&o8);
#pragma unroll
                    for (int x = 0; x < 8; ++x) of[x] = DT::to_f32(oe[x]);
                }
#pragma unroll
                for (int x = 0; x < 8; ++x) acc = fmaf(of[x], DT::to_f32(de[x]), acc);
            }
        }
        delta = half_sum(acc);
    }
    const float wc = qvalid ? p.w[tok_i * p.w_st] : 0.f;
    int lo, corelo, pmax;
    query_ranges<MODE>(i, wc, p.win_edge, lo, corelo, pmax);
    const int wlo = wave_min_u(qvalid ? lo : INT_MAX);
    const int wclo = wave_max_u(qvalid ? corelo : INT_MIN);
    // per-query records for the key-parallel passes (field-major [H][field][T]; the wave
    // is the query's 32-query group) and, from head 0, the block's smallest band start
    if (qvalid && hh == 0) {
        float *rec = p.ws_qrec + (size_t)head * kRecFields * p.total_len + tok_i;
        const size_t T = (size_t)p.total_len;
        rec[kRecLse2 * T] = -lse2 * p.inv_c2;  // (S + this) * scale_log2 = S scale_log2 - lse2
        rec[kRecDelta * T] = -delta;
        reinterpret_cast<int *>(rec)[kRecLo * T] = INT_MAX - lo;
        reinterpret_cast<int *>(rec)[kRecClo * T] = INT_MAX - corelo;
        reinterpret_cast<int *>(rec)[kRecPmax * T] = pmax + 1;
        rec[kRecWc * T] = wc;
        reinterpret_cast<int *>(rec)[kRecGLo * T] = INT_MAX - wlo;
        reinterpret_cast<int *>(rec)[kRecGClo * T] = INT_MAX - wclo;
    }
    const int wpmax = wave_max_u(qvalid ? pmax : -1);
    const int whi = min(wq0 + 31, seq_len - 1);

    for (int s = tid; s < p.k_pad; s += NT) {  // wave-uniform: k_pad is a multiple of 64
        int pos = INT_MAX;
        float b = 0.f;
        if (s < p.k_lmk) {
            const int64_t pp = p.lmk_pos[head * p.lp_sh + seq * p.lp_ss + s * p.lp_sk];
            if (pp >= 0 && pp < seq_len) {
                pos = (int)pp;
                if (p.lmk_bias) b = p.lmk_bias[head * p.lb_sh + seq * p.lb_ss + s * p.lb_sk] * kLog2e;
            }
        }
        s_lpos[s] = pos;
        s_lbias[s] = b;
        s_lrow[s] = pos == INT_MAX ? 0 : pos;
        // smallest position of each landmark tile (a wave holds 64 consecutive slots)
        if (BN == 64) {
            const int tmin = wave_min_u(pos);
            if (lane == 0) s_ltmin[s >> 6] = tmin;
        } else {
            const int tlo = wave_min_u(hh == 0 ? pos : INT_MAX);
            const int thi = wave_min_u(hh == 1 ? pos : INT_MAX);
            if (lane == 0) {
                s_ltmin[s >> 5] = tlo;
                s_ltmin[(s >> 5) + 1] = thi;
            }
        }
    }
    if (lane == 0) {
        s_red[wave][0] = wlo;
        s_red[wave][1] = wpmax;
    }
    if (MODE == kSoft && EFAST && tid < 16 * NRB)
        s_ec[tid] = fast_exp2((kEdgeMid - (float)((tid >> 4) * 32 + acc_row_const(tid & 15))) * p.inv_tau * kLog2e);
    __syncthreads();
    int glo = s_red[0][0], gpmax = s_red[0][1];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        glo = min(glo, s_red[w][0]);
        gpmax = max(gpmax, s_red[w][1]);
    }
    if (head == 0 && tid == 0) p.ws_minlo[target] = glo;  // bounds the query scan of the kv pass
    const int n_lt = p.k_pad / BN;
    const uint64_t lmask = __ballot(lane < n_lt && s_ltmin[lane < n_lt ? lane : 0] <= gpmax);
    const int nb = max((ghi - glo) / BN + 1, NSTAGE - 1);
    const int nt = nb + __popcll(lmask);
    auto lmk_tile = [&](int t) {
        uint64_t m = lmask;
        for (int j = nb; j < t; ++j) m &= m - 1;
        return (int)__builtin_ctzll(m);
    };
    auto issue_tile = [&](int t) {
        if (t < nb) {
            issue_band(t);
        } else {
            const int *lrow = s_lrow + lmk_tile(t) * BN;
            const uint32_t kl = tiles_lds + stage_of(t) * (2 * TB);
            klanes.load_gather(kl, wave, krs, kst, lrow);
            vlanes.load_gather(kl + TB, wave, vrs, vst, lrow);
        }
    };

    f32x16 dqacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dqacc[d][r] = 0.f;
    float dw = 0.f;
    const float c = p.scale_log2;

    // dS = P (dP - Delta) from shifted logits x = logit - lse2 (log2 units incl. biases,
    // -inf where not admitted), then dQ^T += K^T . dS^T with K of stage `stage` read
    // transposed
    auto dq_mfma = [&](const uint32_t (&pk)[NRB][8], int stage) {
        const char *ktile = s_tiles[stage][0];
#pragma unroll
        for (int kk = 0; kk < 2 * NRB; ++kk) {
            const int rb = kk >> 1, g = kk & 1;
            const vec8 b = bitcast<vec8>(
                make_uint4(pk[rb][g * 4 + 0], pk[rb][g * 4 + 1], pk[rb][g * 4 + 2], pk[rb][g * 4 + 3]));
#pragma unroll
            for (int d = 0; d < ND; ++d) {
                const vec8 a = bitcast<vec8>(tile_read_tr<D, kSwzRow>(ktile, kk * 16, d * 32, lane));
                dqacc[d] = DT::mfma(a, b, dqacc[d]);
            }
        }
    };
    auto ds_dq = [&](f32x16 (&x)[NRB], const f32x16 (&pacc)[NRB], int stage) {
        uint32_t pk[NRB][8];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p0 = fast_exp2(x[rb][2 * j]), p1 = fast_exp2(x[rb][2 * j + 1]);
                pk[rb][j] = DT::pack2(p0 * (pacc[rb][2 * j] - delta), p1 * (pacc[rb][2 * j + 1] - delta));
            }
        dq_mfma(pk, stage);
    };

    // Band tile t holds keys tb = ghi - BN + 1 - BN t ..: the bounds cst <= A and cst >= B of
    // the tile below are A0 + BN t and B0 + BN t; nA0 / nB0 are the bit counts of rows_le
    // at t = 0.
    const int A0 = i - ghi + BN - 1 - hh * 4, B0 = lo - ghi + BN - 1 - hh * 4;
    const int nA0 = 4 * (A0 >> 3) + min((A0 & 7) + 1, 4);
    const int nB0 = 4 * ((B0 - 1) >> 3) + min(((B0 - 1) & 7) + 1, 4);

    // ---- tile loop, in phases of one tile kind: band tiles inside every row's core
    // (keep mask only), SOFT band tiles that reach below a row's core start (a suffix of
    // the band tiles; edge bias and d_w~), landmark tiles (bias, admission). A tile's
    // work is one basic block: S^T/dP^T of the lower 32 keys (MFMA), then the masks, P
    // and dS of that half (VALU) under the S^T/dP^T MFMAs of the upper half, then the
    // upper half's VALU work under the dQ^T MFMAs of the lower half.
    auto tile = [&](int t, auto kind) {
        constexpr int KIND = decltype(kind)::value;
        if (t + NSTAGE - 1 < nt) issue_tile(t + NSTAGE - 1);
        const int stage = stage_of(t);
        const int tb = KIND != kLmkTile ? band_key0(t) : 0;
        const int lt = KIND == kLmkTile ? lmk_tile(t) : 0;
        const bool active = KIND != kLmkTile ? ((tb <= whi) && (tb + BN - 1 >= wlo)) : (s_ltmin[lt] <= wpmax);
        if (active) {
            // S^T = K . Q^T and dP^T = V . dO^T (BN keys x 32 queries)
            f32x16 sacc[NRB], pacc[NRB];
            const char *ktile = s_tiles[stage][0];
            const char *vtile = s_tiles[stage][1];
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb) {
                f32x16 a0, a1;
#pragma unroll
                for (int r = 0; r < 16; ++r) a0[r] = a1[r] = 0.f;
#pragma unroll
                for (int s = 0; s < KS; ++s) {
                    const vec8 ka = bitcast<vec8>(tile_read_row16<D>(ktile, rb * 32 + ql, 2 * s + hh));
                    const vec8 va = bitcast<vec8>(tile_read_row16<D>(vtile, rb * 32 + ql, 2 * s + hh));
                    a0 = DT::mfma(ka, qv[s], a0);
                    a1 = DT::mfma(va, dov[s], a1);
                }
                sacc[rb] = a0;
                pacc[rb] = a1;
            }
            // logits minus lse2 in log2 units with biases, -inf where not admitted
            f32x16 x[NRB];
            if constexpr (KIND == kLmkTile) {
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int slot = lt * BN + rb * 32 + g * 8 + hh * 4;
                        const int4 pos = *reinterpret_cast<const int4 *>(&s_lpos[slot]);
                        const float4 bia = *reinterpret_cast<const float4 *>(&s_lbias[slot]);
                        const int pp[4] = {pos.x, pos.y, pos.z, pos.w};
                        const float bb[4] = {bia.x, bia.y, bia.z, bia.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = g * 4 + e;
                            x[rb][r] = (pp[e] <= pmax) ? fmaf(sacc[rb][r], c, bb[e] - lse2) : -INFINITY;
                        }
                    }
            } else {
                // element (rb, r) is key tb + rb*32 + acc_row_const(r) + hh*4 =: tb + hh*4 + cst
                const int A = i - tb - hh * 4;   // key <= i  <=> cst <= A
                const int B = lo - tb - hh * 4;  // key >= lo <=> cst >= B
                if constexpr (MODE == kSoft && KIND == kEdgeTile) {
                    // edge bias, P, dS and the d_w~ term fused per element: dS (1 - sigma) on
                    // edge keys (cst < Bc; such keys also satisfy cst <= A)
                    const int Bc = corelo - tb - hh * 4;
                    uint32_t pk[NRB][8];
                    if constexpr (EFAST) {
                        // sigma(z) = 1 / (1 + u), u = exp(-z) = E ec[j] (E per lane and tile,
                        // ec[j] per element slot, both in range on edge keys); the edge bias
                        // enters P as the factor sigma (P = 2^(S c - lse2) sigma), and
                        // 1 - sigma = 0 exactly where u = 0 (core keys, masked elements)
                        const float E = fast_exp2(((float)A - wc - kEdgeMid) * p.inv_tau * kLog2e);
#pragma unroll
                        for (int rb = 0; rb < NRB; ++rb) {
                            float ec[16];
#pragma unroll
                            for (int g = 0; g < 4; ++g) {
                                const float4 e4 = *reinterpret_cast<const float4 *>(&s_ec[rb * 16 + g * 4]);
                                ec[4 * g] = e4.x;
                                ec[4 * g + 1] = e4.y;
                                ec[4 * g + 2] = e4.z;
                                ec[4 * g + 3] = e4.w;
                            }
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                float ds2[2];
#pragma unroll
                                for (int h2 = 0; h2 < 2; ++h2) {
                                    const int r = 2 * j + h2;
                                    const int cst = rb * 32 + acc_row_const(r);
                                    const bool ok = (cst <= A) & (cst >= B);
                                    const float u = ((cst < Bc) & (cst >= B)) ? E * ec[r] : 0.f;
                                    const float sig = __builtin_amdgcn_rcpf(1.f + u);
                                    const float pr = fast_exp2(ok ? fmaf(sacc[rb][r], c, -lse2) : -INFINITY) * sig;
                                    const float dsv = pr * (pacc[rb][r] - delta);
                                    dw = fmaf(dsv, 1.f - sig, dw);
                                    ds2[h2] = dsv;
                                }
                                pk[rb][j] = DT::pack2(ds2[0], ds2[1]);
                            }
                        }
                    } else {
                        // every factor formed per element (exp(-z) may overflow off the edge)
#pragma unroll
                        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                float ds2[2];
#pragma unroll
                                for (int h2 = 0; h2 < 2; ++h2) {
                                    const int r = 2 * j + h2;
                                    const int cst = rb * 32 + acc_row_const(r);
                                    const bool ok = (cst <= A) & (cst >= B);
                                    const bool is_edge = (cst < Bc) & ok;
                                    const float z = ((float)wc - (float)(A - cst)) * p.inv_tau;
                                    const float e = fast_exp2(is_edge ? -z * kLog2e : 0.f);  // exp(-z)
                                    const float onep = 1.f + e;
                                    const float edge = is_edge ? -fast_log2(onep) : 0.f;  // log2 sigmoid(z)
                                    const float y = fmaf(sacc[rb][r], c, edge);
                                    const float pr = ok ? fast_exp2(y - lse2) : 0.f;
                                    const float dsv = pr * (pacc[rb][r] - delta);
                                    dw += is_edge ? dsv * (e * __builtin_amdgcn_rcpf(onep)) : 0.f;
                                    ds2[h2] = dsv;
                                }
                                pk[rb][j] = DT::pack2(ds2[0], ds2[1]);
                            }
                    }
                    dq_mfma(pk, stage);
                } else {
                    uint32_t keep;
                    if constexpr (NRB == 1) {
                        // rows_le(A0 + BN t) keeps the low clamp(nA0 + 16 t, 0, 16) bits (BN t
                        // is a multiple of 8): the band is the bit field [nB, nA)
                        const int nA = min(max(nA0 + 16 * t, 0), 16);
                        const int nB = min(max(nB0 + 16 * t, 0), 16);
                        keep = ((1u << (nA - nB)) - 1u) << nB;
                    } else {
                        keep = rows_le(A) & ~rows_le(B - 1);
                    }
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) x[rb][r] = keep_if(keep, rb * 16 + r, fmaf(sacc[rb][r], c, -lse2));
                }
            }
            if constexpr (KIND != kEdgeTile) ds_dq(x, pacc, stage);
            if constexpr (KIND != kEdgeTile && NRB == 2) {
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // K/V reads, lower half
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // S^T/dP^T MFMAs, lower half
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // K/V reads, upper half
#pragma unroll
                for (int m = 0; m < 8; ++m) {  // upper-half MFMAs under lower-half VALU
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x402, 12, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // K^T reads
#pragma unroll
                for (int m = 0; m < 8; ++m) {  // dQ^T MFMAs under upper-half VALU
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x402, 10, 0);
                }
            }
        }
        // tile t+1 must have landed; tiles t+2 .. t+NSTAGE-1 may stay in flight
        if (t + NSTAGE - 1 < nt) tile_barrier<(NSTAGE - 2) * LPT>();
        else tile_barrier<0>();
    };
    // band tiles inside every row's core: tile t holds keys ghi-BN+1-BN*t .. ghi-BN*t,
    // all >= wclo for t <= (ghi-BN+1-wclo)/BN
    const int n_core =
        MODE == kSoft ? min(nb, (ghi - (BN - 1) - wclo >= 0) ? (ghi - (BN - 1) - wclo) / BN + 1 : 0) : nb;

    tile_barrier<(NSTAGE - 2) * LPT>();  // tile 0 landed (later ones may be in flight)
    int t = 0;
    for (; t < n_core; ++t) tile(t, std::integral_constant<int, kCoreTile>());
    if constexpr (MODE == kSoft)
        for (; t < nb; ++t) tile(t, std::integral_constant<int, kEdgeTile>());
    for (; t < nt; ++t) tile(t, std::integral_constant<int, kLmkTile>());

    if (qvalid) store_row<DT, ND>(p.dq, tok_i * p.dq_st + (int64_t)head * p.dq_sh, p.grad_f32, dqacc, p.scale, hh);
    if (MODE == kSoft && p.ws_dwh) {
        const float dwt = half_sum(dw) * p.inv_tau;
        if (hh == 0 && qvalid) p.ws_dwh[tok_i * p.n_heads + head] = dwt;
    }
}

// ==================================================================================
// kv (LMK = false): key-parallel band dK/dV;  lmk_kv (LMK = true): landmark dK/dV + d_bias
// ==================================================================================
// A wave owns 32 keys (band: consecutive keys; LMK: 32 landmark slots) held in registers
// as B operands, and streams tiles of Q, dO and the per-query records through an LDS ring
// (direct global->LDS loads, one barrier per tile): band workgroups are kv_waves(D)
// waves with kv_qt(D)-query tiles on a kv_stages(D)-deep ring (2 waves, 32 queries, 4
// stages = 36 KB at D = 64: registers, not LDS, limit it to 4 workgroups per CU),
// lmk_kv workgroups 4 waves with 64-query tiles on a 2-stage ring (37 KB; 4 stages, 74 KB,
// halved the workgroups per CU and measured 1.5 us slower at c3). Per 32-query
// sub-block: S = Q.K^T and dP = dO.V^T (lane = key column, registers = query rows),
// P = 2^(S c + bias - lse2) on admitted pairs, dS = P (dP - Delta), then dV^T += dO^T.P
// and dK^T += Q^T.dS with Q and dO read transposed.
template <typename DT, int D, int MODE, bool LMK, bool EFAST>
__global__ void __launch_bounds__(LMK ? 256 : 64 * kv_waves(D), D == 64 ? 2 : 1) bwd_kv_kernel(const BwdParams p) {
    typedef typename DT::vec8 vec8;
    constexpr int NW = LMK ? 4 : kv_waves(D), NT = 64 * NW;  // waves, threads
    constexpr int kBM = kv_bm(D);                            // keys per band workgroup
    constexpr int QT = LMK ? kTN : kv_qt(D);                 // queries per tile
    constexpr int NSB = QT / 32;                       // 32-query sub-blocks per tile
    constexpr int KS = D / 16, ND = D / 32;
    typedef TileN<D, QT, NW> Tile;
    constexpr int TB = Tile::BYTES;
    constexpr int NSTAGE = LMK ? 2 : kv_stages(D);
    constexpr int RB = QT * 4;                         // bytes of one record field per tile
    constexpr int FPI = 64 / QT;                       // record fields per 64-lane load
    constexpr int RLW = kRecFields / (FPI * NW);       // record loads per wave per tile
    constexpr int LPT = 2 * Tile::LOADS_PER_WAVE + RLW;  // Q, dO and record loads per wave
    static_assert(kRecFields % (FPI * NW) == 0, "record fields split evenly over the waves");

    __shared__ __align__(1024) char s_tiles[NSTAGE][2][TB];  // [stage][Q, dO], row-swizzled
    __shared__ __align__(16) char s_rec[NSTAGE][kRecFields][RB];
    __shared__ int s_misc[8];
    // band pass: one landmark slot's summed dK and dV rows, handed from the whole wave to
    // the key's two lanes
    __shared__ __align__(16) float s_lx[LMK ? 1 : NW][LMK ? 4 : 2 * D];
    // SOFT edge (EFAST): per wave, the query factors R_q of the current sub-block
    // (the D = 64 band loop double-buffers it: row t & 1 holds tile t's factors)
    __shared__ __align__(16) float s_rq[EFAST ? NW : 1][EFAST ? 2 : 1][EFAST ? 32 : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;

    if (!LMK && (int)blockIdx.x >= p.grid_q) {
        // the landmark-bias gradient of (head, sequence) blockIdx.x - grid_q: the lmk_kv
        // chunk partials summed in chunk order (zero for an empty sequence)
        const int id = blockIdx.x - p.grid_q;
        const int h = id / p.num_seqs, sq = id - h * p.num_seqs;
        int st0, en0;
        seq_bounds(p.cu, sq, p.total_len, st0, en0);
        const int len = en0 - st0;
        const int n_ch = (len + kLC - 1) / kLC;
        const size_t base = (size_t)h * p.n_lchunk + st0 / kLC + sq;  // the sequence's first chunk row
        for (int sl = threadIdx.x; sl < p.k_lmk; sl += NT) {
            float acc = 0.f;
            for (int ch = 0; ch < n_ch; ++ch) acc += p.ws_ldb[(base + ch) * p.k_pad + sl];
            p.d_bias[((size_t)h * p.num_seqs + sq) * p.k_lmk + sl] = acc;
        }
        return;
    }
    int head, seq, seq_start, seq_len, kblk = 0, q_begin, q_end, slot = 0, sbw = 0, kw = 0, lcid = 0;
    int key = INT_MAX;  // this lane's key position in the sequence (INT_MAX: none)
    float kbias2 = 0.f;
    if (!LMK) {
        // XCDs own whole heads; key blocks arrive rank-major over the heads, farthest from
        // the sequence end first (they are attended by the most queries): the short last
        // blocks of every sequence fill the last dispatch round
        int rank, bdesc;
        head_rank(blockIdx.x, p.grid_q, p.n_heads, p.n_qblk, head, rank);
        if (head >= p.n_heads) return;
        if (!find_block_desc(p.cu, p.num_seqs, p.total_len, rank, p.n_qblk, kBM, lane, seq, bdesc, seq_start, seq_len)) return;
        kblk = (seq_len + kBM - 1) / kBM - 1 - bdesc;
    } else {
        // workgroup = (head, 64-slot group, query chunk); chunk ids follow find_block
        const int per_head = p.n_lgrp * p.n_lchunk;
        head = blockIdx.x / per_head;
        const int rem = blockIdx.x - head * per_head;
        const int gp = rem / p.n_lchunk;
        lcid = rem - gp * p.n_lchunk;
        int lchunk;
        if (!find_block(p.cu, p.num_seqs, p.total_len, lcid, kLC, lane, seq, lchunk, seq_start, seq_len)) return;
        sbw = wave & 1;
        slot = gp * 64 + (wave >> 1) * 32 + ql;
        q_begin = lchunk * kLC;  // refined below
        q_end = min(seq_len, (lchunk + 1) * kLC);
    }

    if (!LMK) {
        const int kb = kblk * kBM;
        kw = kb + wave * 32;
        if (kw + ql < seq_len) key = kw + ql;
        // last dq query block (kDqBM queries; block ids of the sequence start at
        // seq_start / kDqBM + seq) whose smallest band start reaches this key block
        const int dqbase = seq_start / kDqBM + seq;
        const int nbs = (seq_len + kDqBM - 1) / kDqBM;
        const int own = (kb + kBM - 1) / kDqBM;  // dq block of the key block's last key
        int last = own;
        for (int b = own + 1 + tid; b < nbs; b += NT)
            if (p.ws_minlo[dqbase + b] <= kb + kBM - 1) last = max(last, b);
        last = wave_max_u(last);
        if (lane == 0) s_misc[wave] = last;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; ++w) last = max(last, s_misc[w]);
        last = __builtin_amdgcn_readfirstlane(last);  // wave-uniform: it bounds the tile loops
        q_begin = kb;
        q_end = min(seq_len, (last + 1) * kDqBM);
    } else {
        if (slot < p.k_lmk) {
            const int64_t pp = p.lmk_pos[head * p.lp_sh + seq * p.lp_ss + slot * p.lp_sk];
            if (pp >= 0 && pp < seq_len) {
                key = (int)pp;
                if (p.lmk_bias) kbias2 = p.lmk_bias[head * p.lb_sh + seq * p.lb_ss + slot * p.lb_sk] * kLog2e;
            }
        }
        // queries admitting a landmark p satisfy q > p: start at the first 64-query tile
        // of the chunk that holds a query after the smallest position
        const int mn = wave_min_u(key);
        if (lane == 0) s_misc[wave] = mn;
        __syncthreads();
        const int gmin = __builtin_amdgcn_readfirstlane(min(min(s_misc[0], s_misc[1]), min(s_misc[2], s_misc[3])));
        if (gmin == INT_MAX || gmin >= q_end) q_begin = q_end;
        else if (gmin > q_begin) q_begin += (gmin - q_begin) / QT * QT;
    }
    const bool kvalid = key != INT_MAX;
    const int wkmin = LMK ? wave_min_u(key) : kw;
    const int wkmax = LMK ? wave_max_u(kvalid ? key : -1) : min(kw + 31, seq_len - 1);
    // SOFT edge factors (EFAST): exp(-z) = exp((q - key - w~_q) / tau) splits as R_q L_key
    // with L_key = exp((wkmin - key) / tau); on an edge pair of this wave both factors stay
    // in the fp32 range while (win_edge + 33) / tau < 80 (kv_edge_fast)
    const float kit = p.inv_tau * kLog2e;
    const float lkey = EFAST ? fast_exp2((float)(wkmin - (kvalid ? key : wkmin + 31)) * kit) : 0.f;

    // this lane's key row as the B operand of S = Q K^T and dP = dO V^T
    vec8 kreg[KS], vreg[KS];
    {
        const int64_t tok = (int64_t)seq_start + (kvalid ? key : 0);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            uint4 a = make_uint4(0, 0, 0, 0), b = a;
            if (kvalid) {
                a = ld16(p.k + tok * p.k_st + (int64_t)kv_head(head, p.kv_rep) * p.k_sh + s * 16 + hh * 8);
                b = ld16(p.v + tok * p.v_st + (int64_t)kv_head(head, p.kv_rep) * p.v_sh + s * 16 + hh * 8);
            }
            kreg[s] = bitcast<vec8>(a);
            vreg[s] = bitcast<vec8>(b);
        }
    }

    // ---- tile staging: Q, dO and 8 record fields of 64 queries per tile ----------------
    const uint32_t qst = (uint32_t)p.q_st * 2u, dst = (uint32_t)p.do_st * 2u;
    const i32x4 qrs = buffer_rsrc(p.q + (int64_t)seq_start * p.q_st + (int64_t)head * p.q_sh, (uint32_t)seq_len * qst);
    const i32x4 drs = buffer_rsrc(p.dout + (int64_t)seq_start * p.do_st + (int64_t)head * p.do_sh,
                                  (uint32_t)seq_len * dst);
    // records of this head: field f of query q at byte (f * T + seq_start + q) * 4; queries
    // at or past seq_len get an out-of-range offset (zeros: admit nothing)
    const i32x4 rrs = buffer_rsrc(p.ws_qrec + (size_t)head * kRecFields * p.total_len,
                                  (uint32_t)(kRecFields * p.total_len * 4));
    const TileLanes<D, kSwzRow, QT, NW> qlanes(wave, lane, qst);
    const TileLanes<D, kSwzRow, QT, NW> dlanes(wave, lane, dst);
    const uint32_t tiles_lds = lds_addr(&s_tiles[0][0][0]);
    const uint32_t rec_lds = lds_addr(&s_rec[0][0][0]);
    const int ntile = (q_end > q_begin) ? (q_end - q_begin + QT - 1) / QT : 0;
    auto stage_of = [](int t) { return t % NSTAGE; };  // t >= 0, wave-uniform
    auto issue_tile = [&](int t) {
        const int q0 = q_begin + t * QT;
        const int st = stage_of(t);
        const uint32_t tl = tiles_lds + st * (2 * TB);
        qlanes.load_band(tl, wave, uniform_rsrc(qrs), (uint32_t)q0 * qst);
        dlanes.load_band(tl + TB, wave, uniform_rsrc(drs), (uint32_t)q0 * dst);
        // one load covers FPI consecutive fields (lane l: field f0 + l / QT, query l % QT),
        // which are consecutive in LDS
        const int q = q0 + lane % QT;
#pragma unroll
        for (int u = 0; u < RLW; ++u) {
            const int f0 = (wave * RLW + u) * FPI;
            const int f = f0 + lane / QT;
            const uint32_t off = (q < seq_len) ? (uint32_t)(((size_t)f * p.total_len + seq_start + q) * 4) : 0xFFFFFF00u;
            asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(off), "s"(uniform_rsrc(rrs)),
                         "{m0}"(__builtin_amdgcn_readfirstlane(rec_lds + (st * kRecFields + f0) * RB))
                         : "memory");
        }
    };
    auto rec_i = [&](int st, int f, int q) -> const int * { return reinterpret_cast<const int *>(&s_rec[st][f][q * 4]); };
    auto rec_f = [&](int st, int f, int q) -> const float * { return reinterpret_cast<const float *>(&s_rec[st][f][q * 4]); };

    f32x16 dk[ND], dv[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[d][r] = dv[d][r] = 0.f;
    float dbias = 0.f;
    const float c = p.scale_log2;
    const int nkey = INT_MAX - (kvalid ? key : INT_MAX / 2);  // lo(q) <= key <=> rec lo >= nkey

#pragma unroll
    for (int t = 0; t < NSTAGE - 1; ++t)
        if (t < ntile) issue_tile(t);
    if (!LMK && p.ws_ldk) {
        // Keys that are landmark positions start from their landmark dK/dV: the slot's
        // lmk_kv partials summed over the sequence's query chunks in chunk order. The whole
        // wave sums each such slot (lane j: DV consecutive floats of the dK row for j < 32,
        // of the dV row for j >= 32; one load per chunk, all chunks in flight together) and
        // hands the sums to the key's two lanes through LDS. These loads go out after the
        // ring's first tiles, so that their latency overlaps the tiles'; they are consumed
        // here, before the first counted wait, and the compiler's wait for them (for every
        // load before them, the ring's included) leaves nothing of them in flight at that
        // wait.
        constexpr int DV = D / 32;  // floats per lane of one slot's dK + dV rows
        typedef float fvec __attribute__((ext_vector_type(DV)));
        const int c_first = seq_start / kLC + seq;
        const int n_ch = (seq_len + kLC - 1) / kLC;
        const float *src0 = (lane < 32 ? p.ws_ldk : p.ws_ldv) + (lane & 31) * DV;
        float *xch = s_lx[wave];
        for (int s0 = 0; s0 < p.k_lmk; s0 += 64) {
            int pos = -1;
            if (s0 + lane < p.k_lmk) {
                const int64_t pp = p.lmk_pos[head * p.lp_sh + seq * p.lp_ss + (s0 + lane) * p.lp_sk];
                if (pp >= kw && pp < min(kw + 32, seq_len)) pos = (int)pp;
            }
            unsigned long long m = __ballot(pos >= 0);
            while (m) {
                const int b = __ffsll((long long)m) - 1;
                m &= m - 1;
                const int pb = __shfl(pos, b);
                const size_t row0 = ((size_t)head * p.n_lchunk + c_first) * p.k_pad + s0 + b;
                const size_t cstride = (size_t)p.k_pad * D;  // floats between chunk rows of a slot
                fvec acc = *reinterpret_cast<const fvec *>(src0 + row0 * D);
                int ch = 1;
                for (; ch + 4 <= n_ch; ch += 4) {
                    fvec x[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        x[u] = *reinterpret_cast<const fvec *>(src0 + row0 * D + (size_t)(ch + u) * cstride);
#pragma unroll
                    for (int u = 0; u < 4; ++u) acc += x[u];
                }
                for (; ch < n_ch; ++ch) acc += *reinterpret_cast<const fvec *>(src0 + row0 * D + (size_t)ch * cstride);
                *reinterpret_cast<fvec *>(xch + (lane < 32 ? 0 : D) + (lane & 31) * DV) = acc;
                __builtin_amdgcn_wave_barrier();  // a wave's LDS operations run in order
                if (key == pb) {
#pragma unroll
                    for (int d = 0; d < ND; ++d)
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int dd = d * 32 + g * 8 + hh * 4;
                            const float4 a = *reinterpret_cast<const float4 *>(xch + dd);
                            const float4 b4 = *reinterpret_cast<const float4 *>(xch + D + dd);
                            dk[d][g * 4 + 0] += a.x; dk[d][g * 4 + 1] += a.y;
                            dk[d][g * 4 + 2] += a.z; dk[d][g * 4 + 3] += a.w;
                            dv[d][g * 4 + 0] += b4.x; dv[d][g * 4 + 1] += b4.y;
                            dv[d][g * 4 + 2] += b4.z; dv[d][g * 4 + 3] += b4.w;
                        }
                }
                __builtin_amdgcn_wave_barrier();  // read before the next slot's write
            }
        }
    }
    if (ntile >= NSTAGE - 1) tile_barrier<(NSTAGE - 2) * LPT>();
    else tile_barrier<0>();

    // dV^T += dO^T . P ; dK^T += Q^T . dS   (k-steps over the 32 queries of sub-block sb)
    auto kv_mfma = [&](const char *qtile, const char *dtile, int sb, const uint32_t (&pkp)[8],
                       const uint32_t (&pks)[8]) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const vec8 bp = bitcast<vec8>(make_uint4(pkp[g * 4], pkp[g * 4 + 1], pkp[g * 4 + 2], pkp[g * 4 + 3]));
            const vec8 bs = bitcast<vec8>(make_uint4(pks[g * 4], pks[g * 4 + 1], pks[g * 4 + 2], pks[g * 4 + 3]));
#pragma unroll
            for (int d = 0; d < ND; ++d) {
                dv[d] = DT::mfma(bitcast<vec8>(tile_read_tr<D, kSwzRow>(dtile, sb * 32 + g * 16, d * 32, lane)), bp, dv[d]);
                dk[d] = DT::mfma(bitcast<vec8>(tile_read_tr<D, kSwzRow>(qtile, sb * 32 + g * 16, d * 32, lane)), bs, dk[d]);
            }
        }
    };
    // S and dP (32 queries x 32 keys) of sub-block sb: lane = key column, registers = query rows
    auto sdp_mfma = [&](const char *qtile, const char *dtile, int sb, f32x16 &sacc, f32x16 &pacc) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const vec8 qa = bitcast<vec8>(tile_read_row16<D>(qtile, sb * 32 + ql, 2 * s + hh));
            const vec8 da = bitcast<vec8>(tile_read_row16<D>(dtile, sb * 32 + ql, 2 * s + hh));
            sacc = DT::mfma(qa, kreg[s], sacc);
            pacc = DT::mfma(da, vreg[s], pacc);
        }
    };

    if constexpr (!LMK && NSB == 1) {
        // Band, one 32-query sub-block per tile (D = 64), software-pipelined: step t runs the
        // S/dP MFMAs of tile t+1 under the masks, P and dS (VALU) of tile t, then dV/dK +=
        // of tile t. Every tile of the scan is computed: a tile without admitted pairs gives
        // P = dS = 0. The band masks (q >= key, lo(q) <= key) are branch-free. SOFT edge
        // biases (key < corelo(q)) are added in place per element, or (EFAST) enter P as a
        // factor in the steps from the first tile with an edge pair on; the query factors
        // R_q of tile t+1 go to this wave's LDS row (t+1) & 1 during step t.
        static_assert(NSTAGE >= 3, "the pipelined band loop keeps two tiles ahead of the MFMAs");
        // (summary fields read as wave-uniform values: they steer the loops)
        auto tile_live = [&](int st, int qsb) {
            const int gmin_lo = INT_MAX - __builtin_amdgcn_readfirstlane(*rec_i(st, kRecGLo, 0));
            return !((qsb >= q_end) || (qsb + 31 < kw) || (gmin_lo > wkmax));
        };
        // EFAST: R_q = exp((q - w~_q - wkmin) / tau) of tile tt's queries, one per lane, into
        // row tt & 1 (a NaN window - no band, no edge pair - gets 0, so u is never NaN)
        auto put_rq = [&](int tt) {
            if constexpr (MODE == kSoft && EFAST) {
                const float wq = *rec_f(stage_of(tt), kRecWc, ql);
                const float rq = fast_exp2(((float)(q_begin + tt * QT + ql - wkmin) - wq) * kit);
                if (hh == 0) s_rq[wave][tt & 1][ql] = (rq == rq) ? rq : 0.f;
            }
        };
        // P and dS of the tile in stage st (first query qsb) from its accumulators: sc = S - L
        // (raw units, L the query's LSE / scale) and pc = dP - Delta, both started from the
        // records. DIAG: the tile may hold pairs with q < key (the causal test is needed).
        auto p_ds1 = [&](int st, int qsb, bool live, f32x16 &sc, const f32x16 &pc, int row, auto with_edge,
                         auto diag, uint32_t (&pkp)[8], uint32_t (&pks)[8]) {
            constexpr bool WE = decltype(with_edge)::value;
            constexpr bool DIAG = decltype(diag)::value;
            const int Cj = (kvalid ? key : INT_MAX / 2) - qsb - hh * 4;  // q >= key <=> cst >= Cj
            // lo(q) <= key <=> rec lo >= nkey; records hold INT_MAX - lo >= 0 (0 when out of
            // range), so one unsigned compare against ~0 admits nothing
            const uint32_t nk = (kvalid & live) ? (uint32_t)nkey : 0xFFFFFFFFu;
            if constexpr (MODE == kSoft && !EFAST) {
                const int gmax_clo = INT_MAX - *rec_i(st, kRecGClo, 0);
                if (live && gmax_clo > wkmin) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int qi = g * 8 + hh * 4;
                        const int4 c4 = *reinterpret_cast<const int4 *>(rec_i(st, kRecClo, qi));
                        const float4 w4 = *reinterpret_cast<const float4 *>(rec_f(st, kRecWc, qi));
                        const int ca[4] = {c4.x, c4.y, c4.z, c4.w};
                        const float wa[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = g * 4 + e;
                            float oms;
                            const float eb = soft_edge_log2(wa[e], (float)(acc_row_const(r) - Cj), p.inv_tau, oms);
                            sc[r] += (nkey > ca[e]) ? eb * p.inv_c2 : 0.f;  // key < corelo(q), raw-score units
                        }
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int qi = g * 8 + hh * 4;
                const int4 o4 = *reinterpret_cast<const int4 *>(rec_i(st, kRecLo, qi));
                const uint32_t oa[4] = {(uint32_t)o4.x, (uint32_t)o4.y, (uint32_t)o4.z, (uint32_t)o4.w};
                int ca[4] = {0, 0, 0, 0};
                float ra[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (WE) {
                    const int4 c4 = *reinterpret_cast<const int4 *>(rec_i(st, kRecClo, qi));
                    const float4 r4 = *reinterpret_cast<const float4 *>(&s_rq[wave][row][qi]);
                    ca[0] = c4.x; ca[1] = c4.y; ca[2] = c4.z; ca[3] = c4.w;
                    ra[0] = r4.x; ra[1] = r4.y; ra[2] = r4.z; ra[3] = r4.w;
                }
                float pr4[4], ds4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = g * 4 + e;
                    bool ok = oa[e] >= nk;
                    if constexpr (DIAG) ok = ok & (acc_row_const(r) >= Cj);
                    // masked before the exp (exp2(-inf) = 0): a select, never a branch
                    float pr = fast_exp2(ok ? sc[r] * c : -INFINITY);
                    if constexpr (WE) {
                        // u in [0, inf] (R_q >= 0, L_key > 0): sigma = 0 where it overflows,
                        // which only masked pairs (P = 0) reach
                        const float u = (nkey > ca[e]) ? ra[e] * lkey : 0.f;
                        pr *= __builtin_amdgcn_rcpf(1.f + u);
                    }
                    pr4[e] = pr;
                    ds4[e] = pr * pc[r];
                }
                pkp[g * 2] = DT::pack2(pr4[0], pr4[1]);
                pkp[g * 2 + 1] = DT::pack2(pr4[2], pr4[3]);
                pks[g * 2] = DT::pack2(ds4[0], ds4[1]);
                pks[g * 2 + 1] = DT::pack2(ds4[2], ds4[3]);
            }
        };
        // 32 x 32 accumulators of the tile in stage st started from record field f of its
        // queries, plus the products of tile half `half` (0: Q, 1: dO) with the lane's key
        // row `kr` (kreg or vreg): lane = key column, registers = query rows
        auto rec_mfma = [&](int st, int f, int half, const vec8 (&kr)[KS], f32x16 &acc) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 v = *reinterpret_cast<const float4 *>(rec_f(st, f, g * 8 + hh * 4));
                acc[4 * g] = v.x;
                acc[4 * g + 1] = v.y;
                acc[4 * g + 2] = v.z;
                acc[4 * g + 3] = v.w;
            }
#pragma unroll
            for (int s = 0; s < KS; ++s)
                acc = DT::mfma(bitcast<vec8>(tile_read_row16<D>(s_tiles[st][half], ql, 2 * s + hh)), kr[s], acc);
        };
        // step t: dP - Delta of tile t and S - L of tile t+1 (MFMA) under P and dS of tile t
        // (VALU), then dV/dK += of tile t
        auto pstep = [&](int t, auto we, auto diag, f32x16 &sc, f32x16 &sn) {
            constexpr bool WE = decltype(we)::value;
            if (t + NSTAGE - 1 < ntile) issue_tile(t + NSTAGE - 1);
            const int st = stage_of(t);
            const int qsb = q_begin + t * QT;
            const bool live = tile_live(st, qsb);
            uint32_t pkp[8], pks[8];
            f32x16 pc;
            rec_mfma(st, kRecDelta, 1, vreg, pc);
            // S of tile t+1 (landed; past the last tile a stale stage, ignored)
            rec_mfma(stage_of(t + 1), kRecLse2, 0, kreg, sn);
            p_ds1(st, qsb, live, sc, pc, t & 1, we, diag, pkp, pks);
            if constexpr (!(MODE == kSoft && !EFAST)) {
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // dP initial values, dO operands
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // dP MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // S initial values, Q operands
                    __builtin_amdgcn_sched_group_barrier(0x402, WE ? 10 : 6, 0);  // VALU (P)
                }
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // S MFMA
                    __builtin_amdgcn_sched_group_barrier(0x402, WE ? 20 : 12, 0);  // VALU
                }
            }
            put_rq(t + 1);
            kv_mfma(s_tiles[st][0], s_tiles[st][1], 0, pkp, pks);
            // tile t+2 must have landed (the next step's S); tiles t+3 .. t+NSTAGE-1 may
            // stay in flight
            if (t + NSTAGE - 1 < ntile) tile_barrier<(NSTAGE - 3) * LPT>();
            else tile_barrier<0>();
        };
        // tiles 0 and 1 landed (tile 2 may be in flight)
        if (ntile >= NSTAGE - 1) tile_barrier<(NSTAGE - 3) * LPT>();
        else tile_barrier<0>();
        f32x16 sA, sB;
        rec_mfma(0, kRecLse2, 0, kreg, sA);
        put_rq(0);
        using yes = std::true_type;
        using no = std::false_type;
        // Steps 0 and 1 are the only ones with pairs q < key (tile t holds queries
        // kb + 32 t .., wave w keys kb + 32 w ..); after them the next tile's S is in sA
        // again. Then steps two at a time with the two S accumulators swapping roles; a loop
        // that ends after an odd step leaves the next tile's S in sB and moves it to sA.
        int t = 0;
        if constexpr (MODE == kSoft && EFAST) {
            // tile t has landed at the start of step t: its summary says whether it holds an
            // edge pair; the edge phase starts at the first such tile
            auto has_edge = [&](int tt) {
                const int st = stage_of(tt);
                const int gmax_clo = INT_MAX - __builtin_amdgcn_readfirstlane(*rec_i(st, kRecGClo, 0));
                return tile_live(st, q_begin + tt * QT) && (gmax_clo > wkmin);
            };
            bool edge_on = false;
            if (t < ntile) {
                edge_on = has_edge(t);
                if (edge_on) pstep(t, yes(), yes(), sA, sB);
                else pstep(t, no(), yes(), sA, sB);
                ++t;
            }
            if (t < ntile) {
                edge_on = edge_on || has_edge(t);
                if (edge_on) pstep(t, yes(), yes(), sB, sA);
                else pstep(t, no(), yes(), sB, sA);
                ++t;
            }
            if (!edge_on) {
                while (t < ntile && !has_edge(t)) {
                    pstep(t, no(), no(), sA, sB);
                    if (++t >= ntile || has_edge(t)) {
                        sA = sB;
                        break;
                    }
                    pstep(t, no(), no(), sB, sA);
                    ++t;
                }
            }
            while (t < ntile) {
                pstep(t, yes(), no(), sA, sB);
                if (++t >= ntile) break;
                pstep(t, yes(), no(), sB, sA);
                ++t;
            }
        } else {
            if (t < ntile) pstep(t++, no(), yes(), sA, sB);
            if (t < ntile) pstep(t++, no(), yes(), sB, sA);
            while (t < ntile) {
                pstep(t, no(), no(), sA, sB);
                if (++t >= ntile) break;
                pstep(t, no(), no(), sB, sA);
                ++t;
            }
        }
    } else if (!LMK) {
        // Band: one basic block per tile of NSB 32-query sub-blocks (two at D = 128: the
        // masks, P and dS of sub-block 0 (VALU) run under the S/dP MFMAs of sub-block 1,
        // and sub-block 1's VALU work under the dV/dK MFMAs of sub-block 0). The band masks
        // (q >= key, lo(q) <= key) are branch-free; a sub-block without admitted pairs is
        // fully masked, a tile without any is skipped. SOFT edge biases (key < corelo(q))
        // are added in place by a wave-uniform branch, or (EFAST) enter P as a factor in the
        // tiles from the first one with an edge pair on (a second copy of the tile loop).
        auto band_tile = [&](int t, auto edge_phase) {
            constexpr bool EP = decltype(edge_phase)::value;
            if (t + NSTAGE - 1 < ntile) issue_tile(t + NSTAGE - 1);
            const int st = stage_of(t);
            const char *qtile = s_tiles[st][0];
            const char *dtile = s_tiles[st][1];
            const int q0 = q_begin + t * QT;
            bool live[NSB], edge[NSB], any = false;
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb) {
                const int qsb = q0 + sb * 32;
                const int gmin_lo = INT_MAX - *rec_i(st, kRecGLo, sb * 32);
                const int gmax_clo = INT_MAX - *rec_i(st, kRecGClo, sb * 32);
                live[sb] = !((qsb >= q_end) || (qsb + 31 < kw) || (gmin_lo > wkmax));
                edge[sb] = (MODE == kSoft) && live[sb] && (gmax_clo > wkmin);
                any |= live[sb];
            }
            if (any) {
                f32x16 sacc[NSB], pacc[NSB];
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb) sdp_mfma(qtile, dtile, sb, sacc[sb], pacc[sb]);
                if (MODE == kSoft && !EFAST) {
#pragma unroll
                    for (int sb = 0; sb < NSB; ++sb) {
                        if (!edge[sb]) continue;
                        const int qsb = q0 + sb * 32;
                        const int Cj = (kvalid ? key : INT_MAX / 2) - qsb - hh * 4;
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int qi = sb * 32 + g * 8 + hh * 4;
                            const int4 c4 = *reinterpret_cast<const int4 *>(rec_i(st, kRecClo, qi));
                            const float4 w4 = *reinterpret_cast<const float4 *>(rec_f(st, kRecWc, qi));
                            const int ca[4] = {c4.x, c4.y, c4.z, c4.w};
                            const float wa[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int r = g * 4 + e;
                                float oms;
                                const float eb = soft_edge_log2(wa[e], (float)(acc_row_const(r) - Cj), p.inv_tau, oms);
                                // raw-score units: the logit is sacc * c + eb
                                sacc[sb][r] += (nkey > ca[e]) ? eb * p.inv_c2 : 0.f;  // key < corelo(q)
                            }
                        }
                    }
                }
                uint32_t pkp[NSB][8], pks[NSB][8];
                // P and dS of sub-block sb; with_edge (EFAST): the SOFT edge enters P as the
                // factor sigma(z) = 1 / (1 + u), u = exp(-z) = R_q L_key, on edge pairs
                // (key < corelo(q)); u = 0 elsewhere, so that sigma = 1 exactly
                auto p_ds = [&](int sb, auto with_edge) {
                    constexpr bool WE = decltype(with_edge)::value;
                    const int qsb = q0 + sb * 32;
                    const int Cj = (kvalid ? key : INT_MAX / 2) - qsb - hh * 4;  // q >= key <=> cst >= Cj
                    const bool kv_ok = kvalid & live[sb];
                    if constexpr (WE) {
                        // R_q = exp((q - w~_q - wkmin) / tau) of the sub-block's 32 queries, one per
                        // lane, through this wave's LDS row (LDS operations of a wave run in order)
                        const float wq = *rec_f(st, kRecWc, sb * 32 + ql);
                        const float rq = fast_exp2(((float)(qsb + ql - wkmin) - wq) * kit);
                        // a NaN window (no band, no edge pair) gets 0: u is never NaN
                        if (hh == 0) s_rq[wave][0][ql] = (rq == rq) ? rq : 0.f;
                        __builtin_amdgcn_wave_barrier();
                    }
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int qi = sb * 32 + g * 8 + hh * 4;
                        float4 l4 = *reinterpret_cast<const float4 *>(rec_f(st, kRecLse2, qi));
                        float4 d4 = *reinterpret_cast<const float4 *>(rec_f(st, kRecDelta, qi));
                        int4 o4 = *reinterpret_cast<const int4 *>(rec_i(st, kRecLo, qi));
                        // whole 16-byte reads, taken unconditionally (otherwise the compiler
                        // splits them and sinks the parts into per-element branches)
                        asm volatile("" : "+v"(l4.x), "+v"(l4.y), "+v"(l4.z), "+v"(l4.w), "+v"(d4.x), "+v"(d4.y),
                                     "+v"(d4.z), "+v"(d4.w), "+v"(o4.x), "+v"(o4.y), "+v"(o4.z), "+v"(o4.w));
                        const float la[4] = {l4.x, l4.y, l4.z, l4.w};
                        const float da[4] = {d4.x, d4.y, d4.z, d4.w};
                        const int oa[4] = {o4.x, o4.y, o4.z, o4.w};
                        int ca[4] = {0, 0, 0, 0};
                        float ra[4] = {0.f, 0.f, 0.f, 0.f};
                        if constexpr (WE) {
                            const int4 c4 = *reinterpret_cast<const int4 *>(rec_i(st, kRecClo, qi));
                            const float4 r4 = *reinterpret_cast<const float4 *>(&s_rq[wave][0][g * 8 + hh * 4]);
                            ca[0] = c4.x; ca[1] = c4.y; ca[2] = c4.z; ca[3] = c4.w;
                            ra[0] = r4.x; ra[1] = r4.y; ra[2] = r4.z; ra[3] = r4.w;
                        }
                        float pr4[4], ds4[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = g * 4 + e;
                            const bool ok = (acc_row_const(r) >= Cj) & (oa[e] >= nkey) & kv_ok;
                            // masked before the exp (exp2(-inf) = 0): a select, never a branch
                            float pr = fast_exp2(ok ? (sacc[sb][r] + la[e]) * c : -INFINITY);
                            if constexpr (WE) {
                                // u in [0, inf] (R_q >= 0, L_key > 0): sigma = 0 where it
                                // overflows, which only masked pairs (P = 0) reach
                                const float u = (nkey > ca[e]) ? ra[e] * lkey : 0.f;
                                pr *= __builtin_amdgcn_rcpf(1.f + u);
                            }
                            pr4[e] = pr;
                            ds4[e] = pr * (pacc[sb][r] + da[e]);
                        }
                        pkp[sb][g * 2] = DT::pack2(pr4[0], pr4[1]);
                        pkp[sb][g * 2 + 1] = DT::pack2(pr4[2], pr4[3]);
                        pks[sb][g * 2] = DT::pack2(ds4[0], ds4[1]);
                        pks[sb][g * 2 + 1] = DT::pack2(ds4[2], ds4[3]);
                    }
                    if constexpr (WE) __builtin_amdgcn_wave_barrier();  // R row read before the next write
                };
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb) p_ds(sb, std::integral_constant<bool, EP>());
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb) kv_mfma(qtile, dtile, sb, pkp[sb], pks[sb]);
            }
            // tile t+1 must have landed; tiles t+2 .. t+NSTAGE-1 may stay in flight
            if (t + NSTAGE - 1 < ntile) tile_barrier<(NSTAGE - 2) * LPT>();
            else tile_barrier<0>();
        };
        int t = 0;
        if constexpr (MODE == kSoft && EFAST) {
            // tile t has landed here: its sub-block summaries say whether it holds an edge pair
            auto has_edge = [&](int tt) {
                const int st = stage_of(tt);
                bool e = false;
#pragma unroll
                for (int sb = 0; sb < NSB; ++sb) {
                    const int qsb = q_begin + tt * QT + sb * 32;
                    const int gmin_lo = INT_MAX - *rec_i(st, kRecGLo, sb * 32);
                    const int gmax_clo = INT_MAX - *rec_i(st, kRecGClo, sb * 32);
                    e |= !((qsb >= q_end) || (qsb + 31 < kw) || (gmin_lo > wkmax)) && (gmax_clo > wkmin);
                }
                return e;
            };
            for (; t < ntile && !has_edge(t); ++t) band_tile(t, std::false_type());
            for (; t < ntile; ++t) band_tile(t, std::true_type());
        } else {
            for (; t < ntile; ++t) band_tile(t, std::false_type());
        }
    } else {
    for (int t = 0; t < ntile; ++t) {
            if (t + NSTAGE - 1 < ntile) issue_tile(t + NSTAGE - 1);
            const int st = stage_of(t);
            const char *qtile = s_tiles[st][0];
            const char *dtile = s_tiles[st][1];
    #pragma unroll
            for (int sbi = 0; sbi < (LMK ? 1 : 2); ++sbi) {
                const int sb = LMK ? sbw : sbi;
                const int qsb = q_begin + t * QT + sb * 32;  // first query of the sub-block
                // group summaries of the sub-block (wave-uniform LDS reads)
                const int gmin_lo = INT_MAX - *rec_i(st, kRecGLo, sb * 32);
                const int gmax_clo = INT_MAX - *rec_i(st, kRecGClo, sb * 32);
                bool skip = qsb >= q_end;
                if (!LMK) skip = skip || (qsb + 31 < kw) || (gmin_lo > wkmax);
                else skip = skip || (gmax_clo <= wkmin);  // pmax < corelo
                if (skip) continue;
    
                // S and dP (32 queries x 32 keys): lane = key column, registers = query rows
                f32x16 sacc, pacc;
    #pragma unroll
                for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
    #pragma unroll
                for (int s = 0; s < KS; ++s) {
                    const vec8 qa = bitcast<vec8>(tile_read_row16<D>(qtile, sb * 32 + ql, 2 * s + hh));
                    const vec8 da = bitcast<vec8>(tile_read_row16<D>(dtile, sb * 32 + ql, 2 * s + hh));
                    sacc = DT::mfma(qa, kreg[s], sacc);
                    pacc = DT::mfma(da, vreg[s], pacc);
                }
                // register r holds query q = qsb + hh*4 + acc_row_const(r) of the lane's key
                const int Cj = (kvalid ? key : INT_MAX / 2) - qsb - hh * 4;  // q >= key <=> cst >= Cj
                const bool need_hi = LMK || (qsb < wkmax);
                const bool need_lo = LMK || (gmax_clo > wkmin);
                const bool need_edge = (MODE == kSoft) && !LMK && need_lo;
                uint32_t pkp[8], pks[8], plo[8], slo[8];
    #pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int qi = sb * 32 + g * 8 + hh * 4;
                    const float4 l4 = *reinterpret_cast<const float4 *>(rec_f(st, kRecLse2, qi));
                    const float4 d4 = *reinterpret_cast<const float4 *>(rec_f(st, kRecDelta, qi));
                    const int4 o4 = *reinterpret_cast<const int4 *>(rec_i(st, LMK ? kRecPmax : kRecLo, qi));
                    const float la[4] = {l4.x, l4.y, l4.z, l4.w};
                    const float da[4] = {d4.x, d4.y, d4.z, d4.w};
                    const int oa[4] = {o4.x, o4.y, o4.z, o4.w};
                    int ca[4] = {0, 0, 0, 0};
                    float wa[4] = {0.f, 0.f, 0.f, 0.f};
                    if (need_edge) {
                        const int4 c4 = *reinterpret_cast<const int4 *>(rec_i(st, kRecClo, qi));
                        const float4 w4 = *reinterpret_cast<const float4 *>(rec_f(st, kRecWc, qi));
                        ca[0] = c4.x; ca[1] = c4.y; ca[2] = c4.z; ca[3] = c4.w;
                        wa[0] = w4.x; wa[1] = w4.y; wa[2] = w4.z; wa[3] = w4.w;
                    }
                    float pr4[4], ds4[4];
    #pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = g * 4 + e;
                        const int cst = acc_row_const(r);
                        float pr;
                        if (LMK) {
                            // landmark admitted: key <= pmax(q) <=> key < rec pmax (key = INT_MAX when empty)
                            pr = (key < oa[e]) ? fast_exp2(fmaf(sacc[r] + la[e], c, kbias2)) : 0.f;
                        } else {
                            const bool ok = (!need_hi | (cst >= Cj)) & (!need_lo | (oa[e] >= nkey)) & kvalid;
                            float x = (sacc[r] + la[e]) * c;
                            if (MODE == kSoft && need_edge) {
                                float oms;
                                const float edge = soft_edge_log2(wa[e], (float)(cst - Cj), p.inv_tau, oms);
                                x += (nkey > ca[e]) ? edge : 0.f;  // key < corelo(q)
                            }
                            pr = ok ? fast_exp2(x) : 0.f;
                        }
                        const float ds = pr * (pacc[r] + da[e]);
                        if (LMK) dbias += ds;
                        pr4[e] = pr;
                        ds4[e] = ds;
                    }
                    pkp[g * 2] = DT::pack2(pr4[0], pr4[1]);
                    pkp[g * 2 + 1] = DT::pack2(pr4[2], pr4[3]);
                    pks[g * 2] = DT::pack2(ds4[0], ds4[1]);
                    pks[g * 2 + 1] = DT::pack2(ds4[2], ds4[3]);
                    // rounding remainders x - 16bit(x) (exact in fp32), rounded in turn
                    plo[g * 2] = DT::pack2(pr4[0] - DT::lo_f32(pkp[g * 2]), pr4[1] - DT::hi_f32(pkp[g * 2]));
                    plo[g * 2 + 1] = DT::pack2(pr4[2] - DT::lo_f32(pkp[g * 2 + 1]), pr4[3] - DT::hi_f32(pkp[g * 2 + 1]));
                    slo[g * 2] = DT::pack2(ds4[0] - DT::lo_f32(pks[g * 2]), ds4[1] - DT::hi_f32(pks[g * 2]));
                    slo[g * 2 + 1] = DT::pack2(ds4[2] - DT::lo_f32(pks[g * 2 + 1]), ds4[3] - DT::hi_f32(pks[g * 2 + 1]));
                }
                // dV^T += dO^T . P ; dK^T += Q^T . dS   (k-steps over the 32 queries). A
                // landmark key sums over every query of its sequence, so P and dS enter as
                // 16-bit high part + 16-bit remainder (relative error ~2^-17 instead of
                // ~2^-9 of a single rounding); the operand read is shared by both MFMAs.
    #pragma unroll
                for (int g = 0; g < 2; ++g) {
                    const vec8 bp = bitcast<vec8>(make_uint4(pkp[g * 4], pkp[g * 4 + 1], pkp[g * 4 + 2], pkp[g * 4 + 3]));
                    const vec8 bs = bitcast<vec8>(make_uint4(pks[g * 4], pks[g * 4 + 1], pks[g * 4 + 2], pks[g * 4 + 3]));
                    const vec8 bpl = bitcast<vec8>(make_uint4(plo[g * 4], plo[g * 4 + 1], plo[g * 4 + 2], plo[g * 4 + 3]));
                    const vec8 bsl = bitcast<vec8>(make_uint4(slo[g * 4], slo[g * 4 + 1], slo[g * 4 + 2], slo[g * 4 + 3]));
    #pragma unroll
                    for (int d = 0; d < ND; ++d) {
                        const vec8 ad = bitcast<vec8>(tile_read_tr<D, kSwzRow>(dtile, sb * 32 + g * 16, d * 32, lane));
                        const vec8 aq = bitcast<vec8>(tile_read_tr<D, kSwzRow>(qtile, sb * 32 + g * 16, d * 32, lane));
                        dv[d] = DT::mfma(ad, bp, dv[d]);
                        dk[d] = DT::mfma(aq, bs, dk[d]);
                        dv[d] = DT::mfma(ad, bpl, dv[d]);
                        dk[d] = DT::mfma(aq, bsl, dk[d]);
                    }
                }
            }
            // tile t+1 must have landed; tiles t+2 .. t+NSTAGE-1 may stay in flight
            if (t + NSTAGE - 1 < ntile) tile_barrier<(NSTAGE - 2) * LPT>();
            else tile_barrier<0>();
        }
    
    }

    if (!LMK) {
        if (kvalid) {
            const int64_t tok = (int64_t)seq_start + key;
            store_row<DT, ND>(p.dk, tok * p.dk_st + (int64_t)head * p.dk_sh, p.grad_f32, dk, p.scale, hh);
            store_row<DT, ND>(p.dv, tok * p.dv_st + (int64_t)head * p.dv_sh, p.grad_f32, dv, 1.f, hh);
        }
        if (MODE == kSoft && p.d_w && p.ws_dwh && head == 0 && tid < kBM) {
            const int tq = kblk * kBM + tid;
            if (tq < seq_len) {
                const int64_t tok = (int64_t)seq_start + tq;
                float acc = 0.f;
                for (int h = 0; h < p.n_heads; ++h) acc += p.ws_dwh[tok * p.n_heads + h];
                p.d_w[tok] = acc;
            }
        }
    } else {
        // combine the two query sub-blocks of each slot group (waves 2g+1 into 2g), fixed
        // order, through LDS (the tile ring is idle after the last barrier)
        float *red = reinterpret_cast<float *>(&s_tiles[0][0][0]);
        constexpr int PER_LANE = ND * 16 + 1;  // dK (then dV) of a lane, and its d_bias term
        static_assert(!LMK || 2 * 64 * PER_LANE * 4 <= sizeof(s_tiles), "reduction scratch");
        const int g = wave >> 1;
        float *mine = red + (size_t)(g * 64 + lane) * PER_LANE;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            f32x16 (&acc)[ND] = half ? dv : dk;
            if (sbw == 1) {
#pragma unroll
                for (int d = 0; d < ND; ++d)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mine[d * 16 + r] = acc[d][r];
                if (half == 0) mine[ND * 16] = dbias;
            }
            __syncthreads();
            if (sbw == 0) {
#pragma unroll
                for (int d = 0; d < ND; ++d)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[d][r] += mine[d * 16 + r];
                if (half == 0) dbias += mine[ND * 16];
            }
            __syncthreads();
        }
        if (sbw == 0) {
            const float db = half_sum(dbias);
            const size_t row = ((size_t)head * p.n_lchunk + lcid) * p.k_pad + slot;
            float *gk = p.ws_ldk + row * D;
            float *gv = p.ws_ldv + row * D;
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) {
                    const int dd = d * 32 + gg * 8 + hh * 4;
                    *reinterpret_cast<float4 *>(gk + dd) =
                        make_float4(dk[d][gg * 4], dk[d][gg * 4 + 1], dk[d][gg * 4 + 2], dk[d][gg * 4 + 3]);
                    *reinterpret_cast<float4 *>(gv + dd) =
                        make_float4(dv[d][gg * 4], dv[d][gg * 4 + 1], dv[d][gg * 4 + 2], dv[d][gg * 4 + 3]);
                }
            if (hh == 0) p.ws_ldb[row] = db;
        }
    }
}

struct WsLayout {
    size_t qrec, minlo, dwh, ldk, ldv, ldb, total;
};

WsLayout ws_layout(int T, int S, int H, int D, int k) {
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    WsLayout L;
    size_t off = 0;
    L.qrec = off;
    off += al((size_t)H * kRecFields * T * 4);
    L.minlo = off;
    off += al((size_t)block_upper_bound(T, S, kDqBM) * 4);
    L.dwh = off;
    off += al((size_t)T * H * 4);
    const size_t kp = (size_t)((k + 63) / 64 * 64);
    const size_t nch = (size_t)block_upper_bound(T, S, kLC);
    L.ldk = off;
    off += al((size_t)H * nch * kp * D * 4);
    L.ldv = off;
    off += al((size_t)H * nch * kp * D * 4);
    L.ldb = off;
    off += al((size_t)H * nch * kp * 4);
    L.total = off;
    return L;
}

// Whether the SOFT dq / band dK-dV kernels take their factored edge paths (see the kernels).
inline bool dq_edge_fast(const BwdParams &p) { return (p.win_edge + 1.f + 16.f * (kDqBN / 32)) * p.inv_tau < 80.f; }
inline bool kv_edge_fast(const BwdParams &p) { return (p.win_edge + 33.f) * p.inv_tau < 80.f; }

template <typename DT, int D, int MODE>
hipError_t launch_typed(const BwdParams &p, hipStream_t stream) {
    // dq writes the per-query records that the key-parallel passes stream
    const size_t dyn = (size_t)p.k_pad * (2 * sizeof(int) + sizeof(float));
    bool efast = false;
    if constexpr (MODE == kSoft) efast = dq_edge_fast(p);
    if (efast)  // instantiated for SOFT only
        hipLaunchKernelGGL((bwd_dq_kernel<DT, D, MODE, MODE == kSoft>), dim3(p.grid_dq), dim3(64 * kDqW), dyn, stream, p);
    else
        hipLaunchKernelGGL((bwd_dq_kernel<DT, D, MODE, false>), dim3(p.grid_dq), dim3(64 * kDqW), dyn, stream, p);
    if (p.k_lmk > 0)
        hipLaunchKernelGGL((bwd_kv_kernel<DT, D, MODE, true, false>), dim3(p.n_heads * p.n_lgrp * p.n_lchunk), dim3(256),
                           0, stream, p);
    // the band pass also sums the landmark partials: each landmark key's dK/dV in its
    // prologue, d_bias in H x S workgroups appended to its grid
    const int grid_kv = p.grid_q + ((p.k_lmk > 0 && p.d_bias) ? p.n_heads * p.num_seqs : 0);
    // the factored edge path of the band dK/dV kernel exists at D = 64 only (at D = 128 its
    // second tile loop does not fit the scalar registers)
    constexpr bool kKvFast = MODE == kSoft && D == 64;
    bool kv_fast = false;
    if constexpr (kKvFast) kv_fast = kv_edge_fast(p);
    if (kv_fast)
        hipLaunchKernelGGL((bwd_kv_kernel<DT, D, MODE, false, kKvFast>), dim3(grid_kv), dim3(64 * kv_waves(D)), 0,
                           stream, p);
    else
        hipLaunchKernelGGL((bwd_kv_kernel<DT, D, MODE, false, false>), dim3(grid_kv), dim3(64 * kv_waves(D)), 0,
                           stream, p);
    return hipGetLastError();
}

template <typename DT>
hipError_t launch_dt(const BwdParams &p, int head_dim, int mode, hipStream_t stream) {
    if (head_dim == 64)
        return mode == DSALT_MODE_HARD ? launch_typed<DT, 64, kHard>(p, stream)
                                       : launch_typed<DT, 64, kSoft>(p, stream);
    return mode == DSALT_MODE_HARD ? launch_typed<DT, 128, kHard>(p, stream)
                                   : launch_typed<DT, 128, kSoft>(p, stream);
}

}  // namespace

int64_t bwd_workspace_bytes(int total_len, int num_seqs, int n_heads, int head_dim, int k_lmk) {
    const int64_t sparse = (int64_t)ws_layout(total_len, num_seqs, n_heads, head_dim, k_lmk).total;
    // one sequence without landmark slots may also be a dense-mode call
    if (num_seqs == 1 && k_lmk == 0) return std::max(sparse, dense_bwd_workspace_bytes(total_len, n_heads));
    return sparse;
}

hipError_t launch_bwd(const dsalt_bwd_args &a, hipStream_t stream) {
    if (a.mode == DSALT_MODE_DENSE) return launch_dense_bwd(a, stream);
    if (a.total_len == 0) {
        return hipSuccess;
    }
    const WsLayout L = ws_layout(a.total_len, a.num_seqs, a.n_heads, a.head_dim, a.k_lmk);
    char *ws = static_cast<char *>(a.workspace);
    BwdParams p;
    p.q = static_cast<const uint16_t *>(a.q);
    p.k = static_cast<const uint16_t *>(a.k);
    p.v = static_cast<const uint16_t *>(a.v);
    p.o = a.out;
    p.o_f32 = a.out_dtype == DSALT_DTYPE_F32;
    p.dout = static_cast<const uint16_t *>(a.dout);
    p.lse = a.lse;
    p.w = a.w;
    p.lmk_pos = a.lmk_pos;
    p.lmk_bias = a.lmk_bias;
    p.cu = a.cu_seqlens;
    p.dq = a.dq;
    p.dk = a.dk;
    p.dv = a.dv;
    p.grad_f32 = a.grad_dtype == DSALT_DTYPE_F32;
    p.d_bias = a.d_lmk_bias;
    p.d_w = (a.mode == DSALT_MODE_SOFT) ? a.d_w : nullptr;
    p.ws_qrec = reinterpret_cast<float *>(ws + L.qrec);
    p.ws_minlo = reinterpret_cast<int *>(ws + L.minlo);
    p.ws_dwh = p.d_w ? reinterpret_cast<float *>(ws + L.dwh) : nullptr;
    p.ws_ldk = a.k_lmk > 0 ? reinterpret_cast<float *>(ws + L.ldk) : nullptr;
    p.ws_ldv = a.k_lmk > 0 ? reinterpret_cast<float *>(ws + L.ldv) : nullptr;
    p.ws_ldb = a.k_lmk > 0 ? reinterpret_cast<float *>(ws + L.ldb) : nullptr;
    p.q_st = a.q_stride_t; p.q_sh = a.q_stride_h;
    p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
    p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
    p.o_st = a.out_stride_t; p.o_sh = a.out_stride_h;
    p.do_st = a.dout_stride_t; p.do_sh = a.dout_stride_h;
    p.lse_st = a.lse_stride_t; p.lse_sh = a.lse_stride_h;
    p.w_st = a.w_stride;
    p.lp_sh = a.lmk_pos_stride_h; p.lp_ss = a.lmk_pos_stride_s; p.lp_sk = a.lmk_pos_stride_k;
    p.lb_sh = a.lmk_bias_stride_h; p.lb_ss = a.lmk_bias_stride_s; p.lb_sk = a.lmk_bias_stride_k;
    p.dq_st = a.dq_stride_t; p.dq_sh = a.dq_stride_h;
    p.dk_st = a.dk_stride_t; p.dk_sh = a.dk_stride_h;
    p.dv_st = a.dv_stride_t; p.dv_sh = a.dv_stride_h;
    p.total_len = a.total_len;
    p.num_seqs = a.num_seqs;
    p.n_heads = a.n_heads;
    p.kv_rep = a.n_kv_heads > 0 ? a.n_heads / a.n_kv_heads : 1;
    p.k_lmk = a.k_lmk;
    p.k_pad = (a.k_lmk + 63) / 64 * 64;
    p.n_lgrp = p.k_pad / 64;
    p.n_lchunk = block_upper_bound(a.total_len, a.num_seqs, kLC);
    p.n_qblk = block_upper_bound(a.total_len, a.num_seqs, kv_bm(a.head_dim));
    p.grid_q = (int)(((int64_t)p.n_qblk * a.n_heads + 7) / 8 * 8);
    p.n_dqblk = block_upper_bound(a.total_len, a.num_seqs, kDqBM);
    p.grid_dq = (int)(((int64_t)p.n_dqblk * a.n_heads + 7) / 8 * 8);
    p.scale = a.scale;
    p.scale_log2 = a.scale * kLog2e;
    p.inv_c2 = 1.f / p.scale_log2;
    p.inv_tau = 1.f / a.tau_win;
    p.win_edge = a.win_edge;
    if (a.dtype == DSALT_DTYPE_BF16) return launch_dt<BF16>(p, a.head_dim, a.mode, stream);
    return launch_dt<F16>(p, a.head_dim, a.mode, stream);
}

}  // namespace dsalt
