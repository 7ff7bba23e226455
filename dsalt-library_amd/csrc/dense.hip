// Dense batched DSALT attention for gfx950: the soft-tail variant that the reference
// module runs for unpacked [1, T, d] input (no cu_seqlens), forward and backward.
//
// Reference semantics: DSALTAttention._batched / _diff_logbias / _soft_window_logbias /
// _soft_landmark_logbias (dsalt/modules/dsalt_attention.py:286-329, :371-438). For query
// i and key j <= i of one sequence (d = i - j) and head h:
//   window    bw = 0 when d <= w~_i - win_edge (fp32 compare), else
//                  log(max(sigmoid((w~_i - d) / tau), 1e-20))
//   landmark  bl = lmk_bias[h, j] when d >= max(1, floor(w~_i)), else -inf
//             (lmk_bias is -inf for the keys that are not landmarks of head h)
//   logit     = scale q.k + max(bw, bl), softmax over every j <= i.
// Backward: dS = P (dP - Delta) is the gradient of a logit and of its bias; the window
// term passes dS (1 - sigmoid) / tau to w~_i where it is the larger bias and the sigmoid
// is above the clamp, the landmark term passes dS to lmk_bias[h, j] where it is the
// larger one, and equal biases share dS in halves (torch.maximum's gradient).
//
// Kernels (one launch each, in this order for the backward):
//   dense_fwd_kernel   query-parallel, 64 queries per workgroup, 32-key tiles from the
//                      diagonal down to key 0, split over wave groups (4 at D = 64, 2 at
//                      D = 128; a group is 2 waves x 32 queries walking every NG-th tile
//                      on its own double-buffered direct-load LDS ring); S^T = K.Q^T and
//                      O^T += V^T.P^T on MFMA, online softmax per group, the groups'
//                      (max, sum, O) merged through LDS at the end.
//   dense_prep_kernel  Delta = rowsum(O dO) per (head, query) and the per-query window
//                      record (w~, first core key, last landmark key).
//   dense_dq_kernel    query-parallel: P, dP^T = V.dO^T, dS, dQ^T += K^T.dS^T and the
//                      per-head window gradient of each query (the forward's group split,
//                      partial sums merged in group order).
//   dense_kv_kernel    key-parallel, 64 keys per workgroup: S = Q.K^T, dP = dO.V^T, dS,
//                      dV^T += dO^T.P, dK^T += Q^T.dS and the landmark-bias gradient of
//                      each key, over the query tiles at or after the key block, the tiles
//                      split over wave groups as above.
//   dense_dw_kernel    d_w~[i] = sum over heads of the window gradients.
// Every output element is written by one thread: the results are deterministic.
#include "common.h"
#include "launch.h"
#include "tiles.h"

#include <type_traits>

namespace dsalt {
namespace {

constexpr int kDB = 64;        // queries (or keys) per workgroup
constexpr int kDN = 32;        // keys (or queries) per tile
constexpr float kLog2Clamp = -66.43856189774724f;  // log2(1e-20): the reference's sigmoid clamp
constexpr float kEdgeMidD = 13.5f;                 // centre of acc_row_const's range [0, 27]

// record fields per query (workspace, [kDRec][T])
enum { kRecW = 0, kRecCore = 1, kRecPmax = 2, kDRec = 3 };

struct DenseParams {
    const uint16_t *q, *k, *v, *dout;
    const void *o;     // forward output (backward input): fp32 if o_f32, else the compute dtype
    void *out;         // forward output
    float *lse;        // [T, H] natural log
    const float *w;    // [T] continuous windows
    const float *lb;   // [H, T] natural-log landmark bias, or null
    void *dq, *dk, *dv;
    float *d_lb;       // [H, T] or null
    float *d_w;        // [T] or null
    float *ws_delta;   // [H][T]
    float *ws_rec;     // [kDRec][T] (w~ as float, first core key and last landmark key as int)
    float *ws_dwh;     // [T][H]
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, do_st, do_sh, lse_st, lse_sh, w_st;
    int64_t lb_sh, lb_st;
    int64_t dq_st, dq_sh, dk_st, dk_sh, dv_st, dv_sh;
    int T, H, n_blk, grid, out_f32, o_f32, grad_f32;
    int kv_rep;      // query heads per K/V head
    float c;         // scale * log2(e): raw q.k -> log2-unit logit
    float inv_c;     // 1 / c
    float scale;
    float inv_tau, win_edge;
    int edge_fast;   // the window tail from per-tile factors (13.5 / tau < 40)
};

// First key of the zero-bias core (d <= w~ - win_edge, i.e. j >= i - floor(w~ - win_edge))
// and last admissible landmark key (d >= max(1, floor(w~)), i.e. j <= i - wd); keys
// beyond the sequence or NaN windows admit nothing.
__device__ __forceinline__ void dense_ranges(int i, float wv, float win_edge, int &corelo, int &pmax) {
    const float wce = wv - win_edge;
    corelo = (wce >= 0.f) ? i - (int)floorf(fminf(wce, 1073741824.f)) : i + 1;
    pmax = (wv == wv) ? i - max(1, (int)floorf(fminf(fmaxf(wv, 1.f), 1073741824.f))) : -1;
}

// Window bias of one element in log2 units and its w~ derivative factor (1 - sigmoid):
// e = exp((d - w~) / tau) = exp(-z); log2 sigmoid(z) = -log2(1 + e), clamped at
// log2(1e-20) where the reference's clamp cuts the gradient.
__device__ __forceinline__ float window_bias2(float e, bool core, float &oms, bool &clamped) {
    const float onep = 1.f + e;
    const float l = -fast_log2(onep);
    clamped = !(l > kLog2Clamp);  // also true for e = inf
    oms = clamped ? 0.f : e * __builtin_amdgcn_rcpf(onep);
    if (core) {
        oms = 0.f;
        clamped = false;
        return 0.f;
    }
    return clamped ? kLog2Clamp : l;
}

// ==================================================================================
// forward
// ==================================================================================
// Key tiles of a workgroup are split over kFwdGroups(D) wave groups: group g (waves 2g,
// 2g+1, the workgroup's 64 queries) walks tiles t = g, g + NG, ... on its own double-
// buffered ring, keeping its own running max, sum and O; the groups step together (one
// workgroup barrier per step) and their states are merged through LDS at the end, in
// group order. A workgroup's serial tile chain is NG times shorter.
constexpr int dense_fwd_groups(int D) { return D == 64 ? 4 : 2; }

template <typename DT, int D>
__global__ void __launch_bounds__(128 * dense_fwd_groups(D), 1) dense_fwd_kernel(const DenseParams p) {
    typedef typename DT::vec8 vec8;
    constexpr int NG = dense_fwd_groups(D);
    constexpr int BM = kDB, BN = kDN;
    constexpr int KS = D / 16, ND = D / 32;
    typedef TileN<D, BN, 2> Tile;
    constexpr int TB = Tile::BYTES;
    constexpr int MERGE = ND * 16 + 2;  // floats per lane of a group state: O, max, sum
    static_assert((NG - 1) * 2 * 64 * MERGE * 4 <= NG * 2 * 2 * TB, "merge buffer fits in the tile rings");

    __shared__ __align__(1024) char s_tiles[NG][2][2][TB];  // [group][slot][K, V]
    __shared__ __align__(16) float s_lb[NG][2][BN];          // landmark bias of the slot's keys (log2 units)

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 1, wi = wave & 1;
    const int ql = lane & 31, hh = lane >> 5;
    int head, rank;
    head_rank(blockIdx.x, p.grid, p.H, p.n_blk, head, rank);
    if (head >= p.H) return;
    const int blk = p.n_blk - 1 - rank;  // long blocks first
    const int wq0 = blk * BM + wi * 32;
    const int i = wq0 + ql;
    const bool qvalid = i < p.T;
    const int ghi = min(blk * BM + BM - 1, p.T - 1);
    const int nt = ghi / BN + 1;             // tiles reaching key 0
    const int nit = (nt + NG - 1) / NG;      // steps of the workgroup

    const uint32_t kst = (uint32_t)p.k_st * 2u, vst = (uint32_t)p.v_st * 2u;
    const int kvh = kv_head(head, p.kv_rep);
    const i32x4 krs = buffer_rsrc(p.k + (int64_t)kvh * p.k_sh, (uint32_t)p.T * kst);
    const i32x4 vrs = buffer_rsrc(p.v + (int64_t)kvh * p.v_sh, (uint32_t)p.T * vst);
    const TileLanes<D, kSwzRow, BN, 2> klanes(wi, lane, kst);
    const TileLanes<D, kSwzTr, BN, 2> vlanes(wi, lane, vst);
    const uint32_t tiles_lds = lds_addr(&s_tiles[grp][0][0][0]);
    auto key0 = [&](int t) { return ghi - (BN - 1) - t * BN; };
    auto issue = [&](int it) {  // the group's tile of step it into slot it % 2 (keys below 0 read zeros)
        const int t = grp + NG * it;
        const uint32_t base = tiles_lds + (it & 1) * (2 * TB);
        klanes.load_band(base, wi, krs, (uint32_t)key0(t) * kst);
        vlanes.load_band(base + TB, wi, vrs, (uint32_t)key0(t) * vst);
    };
    // landmark bias of tile t's keys, staged through registers by the group's first wave
    auto lb_load = [&](int t) -> float {
        const int j = key0(t) + ql;
        if (!p.lb || wi != 0 || hh != 0 || j < 0 || j >= p.T) return -INFINITY;
        return p.lb[(int64_t)head * p.lb_sh + (int64_t)j * p.lb_st] * kLog2e;
    };

    vec8 qv[KS];
    {
        const int tq = qvalid ? i : p.T - 1;
        const uint16_t *qp = p.q + (int64_t)tq * p.q_st + (int64_t)head * p.q_sh + hh * 8;
#pragma unroll
        for (int s = 0; s < KS; ++s) qv[s] = bitcast<vec8>(*reinterpret_cast<const uint4 *>(qp + s * 16));
    }
    const float wv = qvalid ? p.w[(int64_t)i * p.w_st] : 0.f;
    int corelo, pmax;
    dense_ranges(i, wv, p.win_edge, corelo, pmax);
    const float c = p.c;
    // window-tail factors: exp((d - w~)/tau) = E * ec[r] (see window_bias2)
    float ec[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ec[r] = fast_exp2((kEdgeMidD - (float)acc_row_const(r)) * p.inv_tau * kLog2e);

    const bool act0 = grp < nt;
    if (act0) issue(0);
    float lbr = act0 ? lb_load(grp) : -INFINITY;

    f32x16 oacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[d][r] = 0.f;
    float m2 = -INFINITY, mu = 0.f, thr = -INFINITY;
    float lsum0 = 0.f, lsum1 = 0.f;

    for (int it = 0; it < nit; ++it) {
        const int t = grp + NG * it;
        const bool act = t < nt;               // group-uniform
        const int slot = it & 1;
        if (wi == 0 && hh == 0) s_lb[grp][slot][ql] = lbr;
        tile_barrier<0>();  // the step's tiles landed for every group; everyone left step it-1
        if (t + NG < nt) {
            issue(it + 1);
            lbr = lb_load(t + NG);
        }
        if (!act) continue;
        const char *ktile = s_tiles[grp][slot][0];
        const char *vtile = s_tiles[grp][slot][1];
        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            s = DT::mfma(bitcast<vec8>(tile_read_row16<D>(ktile, ql, 2 * ks + hh)), qv[ks], s);

        // biases: element r is key tb + hh*4 + acc_row_const(r), distance d = A - cst
        const int tb = key0(t);
        const int A = i - tb - hh * 4;
        const int Bc = corelo - tb - hh * 4;  // core: cst >= Bc
        const int Pm = pmax - tb - hh * 4;    // landmark admitted: cst <= Pm
        const int Bz = -tb - hh * 4;          // key >= 0: cst >= Bz
        const float E = fast_exp2(((float)A - wv - kEdgeMidD) * p.inv_tau * kLog2e);
        float lbv[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 l4 = *reinterpret_cast<const float4 *>(&s_lb[grp][slot][g * 8 + hh * 4]);
            lbv[4 * g] = l4.x; lbv[4 * g + 1] = l4.y; lbv[4 * g + 2] = l4.z; lbv[4 * g + 3] = l4.w;
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int cst = acc_row_const(r);
            const float e = p.edge_fast ? E * ec[r] : fast_exp2(((float)(A - cst) - wv) * p.inv_tau * kLog2e);
            float oms;
            bool clamped;
            const float bw = window_bias2(e, cst >= Bc, oms, clamped);
            const float bl = cst <= Pm ? lbv[r] : -INFINITY;
            const bool keep = cst <= A && cst >= Bz && qvalid;
            const float x = keep ? s[r] + fmaxf(bw, bl) * p.inv_c : -INFINITY;
            s[r] = x;
            tmax = fmaxf(tmax, x);
        }
        tmax = half_max(tmax);
        const bool raise = tmax > thr;
        if (__builtin_amdgcn_ballot_w64(raise)) {
            const float tm2 = tmax * c;
            const float alpha = raise ? fast_exp2(m2 - tm2) : 1.f;
            lsum0 *= alpha;
            lsum1 *= alpha;
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[d][r] *= alpha;
            m2 = raise ? tm2 : m2;
            mu = (m2 == -INFINITY) ? 0.f : m2;
            thr = raise ? tmax + 8.f * p.inv_c : thr;
        }
        // the row sums take the fp32 P (the LSE then matches the fp32 softmax the
        // backward recomputes); O accumulates the 16-bit P the MFMA consumes
        uint32_t pk[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float e0 = fast_exp2(fmaf(s[2 * j], c, -mu)), e1 = fast_exp2(fmaf(s[2 * j + 1], c, -mu));
            pk[j] = DT::pack2(e0, e1);
            if (j & 1) lsum1 += e0 + e1;
            else lsum0 += e0 + e1;
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const vec8 b = bitcast<vec8>(make_uint4(pk[kk * 4], pk[kk * 4 + 1], pk[kk * 4 + 2], pk[kk * 4 + 3]));
#pragma unroll
            for (int d = 0; d < ND; ++d)
                oacc[d] = DT::mfma(bitcast<vec8>(tile_read_tr<D>(vtile, kk * 16, d * 32, lane)), b, oacc[d]);
        }
    }
    tile_barrier<0>();  // every group is done with its ring: the rings become the merge buffer

    // merge: groups 1..NG-1 publish (O, max, sum) per lane, group 0 folds them in group
    // order (the max of the maxima, each state rescaled to it)
    float *mbuf = reinterpret_cast<float *>(&s_tiles[0][0][0][0]);
    auto mslot = [&](int g, int e) { return mbuf + ((((g - 1) * 2 + wi) * MERGE + e) * 64 + lane); };
    float lsum = lsum0 + lsum1;
    if (grp > 0) {
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) *mslot(grp, d * 16 + r) = oacc[d][r];
        *mslot(grp, ND * 16) = m2;
        *mslot(grp, ND * 16 + 1) = lsum;
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int g = 1; g < NG; ++g) {
        const float mg = *mslot(g, ND * 16), lg = *mslot(g, ND * 16 + 1);
        const float mn = fmaxf(m2, mg);
        const float a0 = (m2 == -INFINITY) ? 0.f : fast_exp2(m2 - mn);
        const float ag = (mg == -INFINITY) ? 0.f : fast_exp2(mg - mn);
        lsum = lsum * a0 + lg * ag;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[d][r] = oacc[d][r] * a0 + *mslot(g, d * 16 + r) * ag;
        m2 = mn;
    }

    const float ltot = half_sum(lsum);
    const bool nonempty = ltot > 1e-9f;
    const float inv = nonempty ? 1.f / ltot : 0.f;
    if (qvalid) {
        const int64_t ooff = (int64_t)i * p.o_st + (int64_t)head * p.o_sh;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dd = d * 32 + g * 8 + hh * 4;
                const float o0 = oacc[d][g * 4] * inv, o1 = oacc[d][g * 4 + 1] * inv;
                const float o2 = oacc[d][g * 4 + 2] * inv, o3 = oacc[d][g * 4 + 3] * inv;
                if (p.out_f32) {
                    *reinterpret_cast<float4 *>(static_cast<float *>(p.out) + ooff + dd) = make_float4(o0, o1, o2, o3);
                } else {
                    uint2 val;
                    val.x = DT::pack2(o0, o1);
                    val.y = DT::pack2(o2, o3);
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p.out) + ooff + dd) = val;
                }
            }
        if (hh == 0)
            p.lse[(int64_t)i * p.lse_st + (int64_t)head * p.lse_sh] = nonempty ? (m2 + fast_log2(ltot)) * kLn2 : -INFINITY;
    }
}

// ==================================================================================
// backward
// ==================================================================================
// Delta = rowsum(O dO) per (head, query) into ws_delta [H][T]; head 0 threads also
// write the query's window record.
template <typename DT>
__global__ void __launch_bounds__(256) dense_prep_kernel(const DenseParams p, int D) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (query, head)
    if (e >= (int64_t)p.T * p.H) return;
    const int i = (int)(e / p.H), h = (int)(e % p.H);
    const uint16_t *dp = p.dout + (int64_t)i * p.do_st + (int64_t)h * p.do_sh;
    float acc = 0.f;
    if (p.o_f32) {
        const float *op = static_cast<const float *>(p.o) + (int64_t)i * p.o_st + (int64_t)h * p.o_sh;
        for (int d = 0; d < D; d += 8) {
            const uint4 u = *reinterpret_cast<const uint4 *>(dp + d);
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
            const float4 a = *reinterpret_cast<const float4 *>(op + d);
            const float4 b = *reinterpret_cast<const float4 *>(op + d + 4);
            const float o8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = fmaf(o8[2 * j], DT::lo_f32(w4[j]), acc);
                acc = fmaf(o8[2 * j + 1], DT::hi_f32(w4[j]), acc);
            }
        }
    } else {
        const uint16_t *op = static_cast<const uint16_t *>(p.o) + (int64_t)i * p.o_st + (int64_t)h * p.o_sh;
        for (int d = 0; d < D; d += 8) {
            const uint4 u = *reinterpret_cast<const uint4 *>(dp + d);
            const uint4 o = *reinterpret_cast<const uint4 *>(op + d);
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w}, o4[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = fmaf(DT::lo_f32(o4[j]), DT::lo_f32(w4[j]), acc);
                acc = fmaf(DT::hi_f32(o4[j]), DT::hi_f32(w4[j]), acc);
            }
        }
    }
    p.ws_delta[(int64_t)h * p.T + i] = acc;
    if (h == 0) {
        const float wv = p.w[(int64_t)i * p.w_st];
        int corelo, pmax;
        dense_ranges(i, wv, p.win_edge, corelo, pmax);
        p.ws_rec[(int64_t)kRecW * p.T + i] = wv;
        p.ws_rec[(int64_t)kRecCore * p.T + i] = __int_as_float(corelo);
        p.ws_rec[(int64_t)kRecPmax * p.T + i] = __int_as_float(pmax);
    }
}

// Share of an element's bias gradient that goes to the window term and to the landmark
// term: the larger bias takes all of it, equal biases half each (torch.maximum).
__device__ __forceinline__ void bias_shares(float bw, float bl, float &sw, float &sl) {
    sw = bw > bl ? 1.f : (bw == bl ? 0.5f : 0.f);
    sl = bl > bw ? 1.f : (bw == bl ? 0.5f : 0.f);
}

// Query-parallel dQ and the per-head window gradient, the forward's tiling and its
// key-tile split over dense_bwd_groups(D) wave groups (partial dQ and window gradients
// summed through LDS in group order at the end).
constexpr int dense_bwd_groups(int D) { return D == 64 ? 4 : 2; }

template <typename DT, int D>
__global__ void __launch_bounds__(128 * dense_bwd_groups(D), 1) dense_dq_kernel(const DenseParams p) {
    typedef typename DT::vec8 vec8;
    constexpr int NG = dense_bwd_groups(D);
    constexpr int BM = kDB, BN = kDN;
    constexpr int KS = D / 16, ND = D / 32;
    typedef TileN<D, BN, 2> Tile;
    constexpr int TB = Tile::BYTES;
    constexpr int MERGE = ND * 16 + 1;  // floats per lane of a group's partial: dQ, window gradient
    static_assert((NG - 1) * 2 * 64 * MERGE * 4 <= NG * 2 * 2 * TB, "merge buffer fits in the tile rings");

    __shared__ __align__(1024) char s_tiles[NG][2][2][TB];  // [group][slot][K, V], both row-swizzled
    __shared__ __align__(16) float s_lb[NG][2][BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 1, wi = wave & 1;
    const int ql = lane & 31, hh = lane >> 5;
    int head, rank;
    head_rank(blockIdx.x, p.grid, p.H, p.n_blk, head, rank);
    if (head >= p.H) return;
    const int blk = p.n_blk - 1 - rank;
    const int wq0 = blk * BM + wi * 32;
    const int i = wq0 + ql;
    const bool qvalid = i < p.T;
    const int ghi = min(blk * BM + BM - 1, p.T - 1);
    const int nt = ghi / BN + 1;
    const int nit = (nt + NG - 1) / NG;

    const uint32_t kst = (uint32_t)p.k_st * 2u, vst = (uint32_t)p.v_st * 2u;
    const i32x4 krs = buffer_rsrc(p.k + (int64_t)kv_head(head, p.kv_rep) * p.k_sh, (uint32_t)p.T * kst);
    const i32x4 vrs = buffer_rsrc(p.v + (int64_t)kv_head(head, p.kv_rep) * p.v_sh, (uint32_t)p.T * vst);
    const TileLanes<D, kSwzRow, BN, 2> klanes(wi, lane, kst);
    const TileLanes<D, kSwzRow, BN, 2> vlanes(wi, lane, vst);
    const uint32_t tiles_lds = lds_addr(&s_tiles[grp][0][0][0]);
    auto key0 = [&](int t) { return ghi - (BN - 1) - t * BN; };
    auto issue = [&](int it) {  // the group's tile of step it into slot it % 2
        const int t = grp + NG * it;
        const uint32_t base = tiles_lds + (it & 1) * (2 * TB);
        klanes.load_band(base, wi, krs, (uint32_t)key0(t) * kst);
        vlanes.load_band(base + TB, wi, vrs, (uint32_t)key0(t) * vst);
    };
    auto lb_load = [&](int t) -> float {
        const int j = key0(t) + ql;
        if (!p.lb || wi != 0 || hh != 0 || j < 0 || j >= p.T) return -INFINITY;
        return p.lb[(int64_t)head * p.lb_sh + (int64_t)j * p.lb_st] * kLog2e;
    };

    const int tq = qvalid ? i : p.T - 1;
    vec8 qv[KS], dov[KS];
    {
        const uint16_t *qp = p.q + (int64_t)tq * p.q_st + (int64_t)head * p.q_sh + hh * 8;
        const uint16_t *dp = p.dout + (int64_t)tq * p.do_st + (int64_t)head * p.do_sh + hh * 8;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            qv[s] = bitcast<vec8>(*reinterpret_cast<const uint4 *>(qp + s * 16));
            dov[s] = bitcast<vec8>(*reinterpret_cast<const uint4 *>(dp + s * 16));
        }
    }
    const float lse2 = p.lse[(int64_t)tq * p.lse_st + (int64_t)head * p.lse_sh] * kLog2e;
    const float delta = p.ws_delta[(int64_t)head * p.T + tq];
    const float wv = qvalid ? p.w[(int64_t)i * p.w_st] : 0.f;
    int corelo, pmax;
    dense_ranges(i, wv, p.win_edge, corelo, pmax);
    const float c = p.c;
    float ec[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ec[r] = fast_exp2((kEdgeMidD - (float)acc_row_const(r)) * p.inv_tau * kLog2e);
    const bool live = qvalid && lse2 < INFINITY && lse2 > -INFINITY;

    if (grp < nt) issue(0);
    float lbr = grp < nt ? lb_load(grp) : -INFINITY;
    f32x16 dq[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[d][r] = 0.f;
    float dwl = 0.f;

    for (int it = 0; it < nit; ++it) {
        const int t = grp + NG * it;
        const int slot = it & 1;
        if (wi == 0 && hh == 0) s_lb[grp][slot][ql] = lbr;
        tile_barrier<0>();  // the step's tiles landed for every group; everyone left step it-1
        if (t + NG < nt) {
            issue(it + 1);
            lbr = lb_load(t + NG);
        }
        if (t >= nt) continue;  // group-uniform
        const char *ktile = s_tiles[grp][slot][0];
        const char *vtile = s_tiles[grp][slot][1];
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = 0.f;
            dp[r] = 0.f;
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s = DT::mfma(bitcast<vec8>(tile_read_row16<D>(ktile, ql, 2 * ks + hh)), qv[ks], s);
            dp = DT::mfma(bitcast<vec8>(tile_read_row16<D>(vtile, ql, 2 * ks + hh)), dov[ks], dp);
        }
        const int tb = key0(t);
        const int A = i - tb - hh * 4;
        const int Bc = corelo - tb - hh * 4;
        const int Pm = pmax - tb - hh * 4;
        const int Bz = -tb - hh * 4;
        const float E = fast_exp2(((float)A - wv - kEdgeMidD) * p.inv_tau * kLog2e);
        float lbv[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 l4 = *reinterpret_cast<const float4 *>(&s_lb[grp][slot][g * 8 + hh * 4]);
            lbv[4 * g] = l4.x; lbv[4 * g + 1] = l4.y; lbv[4 * g + 2] = l4.z; lbv[4 * g + 3] = l4.w;
        }
        uint32_t pk[8];
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            float ds2[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int rr = r + u, cst = acc_row_const(rr);
                const float e = p.edge_fast ? E * ec[rr] : fast_exp2(((float)(A - cst) - wv) * p.inv_tau * kLog2e);
                float oms;
                bool clamped;
                const float bw = window_bias2(e, cst >= Bc, oms, clamped);
                const float bl = cst <= Pm ? lbv[rr] : -INFINITY;
                const bool keep = cst <= A && cst >= Bz && live;
                const float pr = keep ? fast_exp2(fmaf(s[rr], c, fmaxf(bw, bl) - lse2)) : 0.f;
                const float dsv = pr * (dp[rr] - delta);
                float sw, sl;
                bias_shares(bw, bl, sw, sl);
                dwl = fmaf(dsv * sw, oms, dwl);
                ds2[u] = dsv;
            }
            pk[r >> 1] = DT::pack2(ds2[0], ds2[1]);
        }
        // dQ^T += K^T . dS^T (K read transposed from the row-swizzled tile)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const vec8 b = bitcast<vec8>(make_uint4(pk[kk * 4], pk[kk * 4 + 1], pk[kk * 4 + 2], pk[kk * 4 + 3]));
#pragma unroll
            for (int d = 0; d < ND; ++d)
                dq[d] = DT::mfma(bitcast<vec8>(tile_read_tr<D, kSwzRow>(ktile, kk * 16, d * 32, lane)), b, dq[d]);
        }
    }
    tile_barrier<0>();  // every group is done with its ring: the rings become the merge buffer
    {
        float *mbuf = reinterpret_cast<float *>(&s_tiles[0][0][0][0]);
        auto mslot = [&](int g, int e) { return mbuf + ((((g - 1) * 2 + wi) * MERGE + e) * 64 + lane); };
        if (grp > 0) {
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) *mslot(grp, d * 16 + r) = dq[d][r];
            *mslot(grp, ND * 16) = dwl;
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int g = 1; g < NG; ++g) {
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) dq[d][r] += *mslot(g, d * 16 + r);
            dwl += *mslot(g, ND * 16);
        }
    }
    const float dw = half_sum(dwl) * p.inv_tau;
    if (qvalid) {
        const int64_t off = (int64_t)i * p.dq_st + (int64_t)head * p.dq_sh;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dd = d * 32 + g * 8 + hh * 4;
                const float a0 = dq[d][g * 4] * p.scale, a1 = dq[d][g * 4 + 1] * p.scale;
                const float a2 = dq[d][g * 4 + 2] * p.scale, a3 = dq[d][g * 4 + 3] * p.scale;
                if (p.grad_f32) {
                    *reinterpret_cast<float4 *>(static_cast<float *>(p.dq) + off + dd) = make_float4(a0, a1, a2, a3);
                } else {
                    uint2 val;
                    val.x = DT::pack2(a0, a1);
                    val.y = DT::pack2(a2, a3);
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p.dq) + off + dd) = val;
                }
            }
        if (hh == 0) p.ws_dwh[(int64_t)i * p.H + head] = dw;
    }
}

// Key-parallel dK, dV and the landmark-bias gradient: a wave owns 32 keys (lane = key
// column of S = Q.K^T), and scans the 32-query tiles at or after its workgroup's keys,
// split over dense_bwd_groups(D) wave groups as in dense_dq_kernel (partial dK, dV and
// bias gradients summed through LDS in group order).
template <typename DT, int D>
__global__ void __launch_bounds__(128 * dense_bwd_groups(D), 1) dense_kv_kernel(const DenseParams p) {
    typedef typename DT::vec8 vec8;
    constexpr int NG = dense_bwd_groups(D);
    constexpr int BK = kDB, QN = kDN;
    constexpr int KS = D / 16, ND = D / 32;
    typedef TileN<D, QN, 2> Tile;
    constexpr int TB = Tile::BYTES;
    constexpr int MERGE = ND * 16 + 1;  // floats per lane and merge round: dK (+ bias gradient), then dV
    static_assert((NG - 1) * 2 * 64 * MERGE * 4 <= NG * 2 * 2 * TB, "merge buffer fits in the tile rings");

    __shared__ __align__(1024) char s_tiles[NG][2][2][TB];   // [group][slot][Q, dO], both row-swizzled
    __shared__ __align__(16) float s_qf[NG][2][5][QN];        // per-query lse2, delta, w~, core, pmax

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 1, wi = wave & 1;
    const int kl = lane & 31, hh = lane >> 5;
    int head, rank;
    head_rank(blockIdx.x, p.grid, p.H, p.n_blk, head, rank);
    if (head >= p.H) return;
    const int kblk = rank;                 // early keys see the most queries: launched first
    const int k0 = kblk * BK;
    const int j = k0 + wi * 32 + kl;       // this lane's key
    const bool kvalid = j < p.T;
    const int nu = (p.T - k0 + QN - 1) / QN;  // query tiles from k0 to T - 1
    const int nit = (nu + NG - 1) / NG;

    const uint32_t qst = (uint32_t)p.q_st * 2u, dst = (uint32_t)p.do_st * 2u;
    const i32x4 qrs = buffer_rsrc(p.q + (int64_t)head * p.q_sh, (uint32_t)p.T * qst);
    const i32x4 drs = buffer_rsrc(p.dout + (int64_t)head * p.do_sh, (uint32_t)p.T * dst);
    const TileLanes<D, kSwzRow, QN, 2> qlanes(wi, lane, qst);
    const TileLanes<D, kSwzRow, QN, 2> dlanes(wi, lane, dst);
    const uint32_t tiles_lds = lds_addr(&s_tiles[grp][0][0][0]);
    auto qtile0 = [&](int u) { return k0 + u * QN; };
    auto issue = [&](int it) {  // the group's query tile of step it into slot it % 2
        const int u = grp + NG * it;
        const uint32_t base = tiles_lds + (it & 1) * (2 * TB);
        qlanes.load_band(base, wi, qrs, (uint32_t)qtile0(u) * qst);  // rows past T read zeros
        dlanes.load_band(base + TB, wi, drs, (uint32_t)qtile0(u) * dst);
    };
    // per-query fields of tile u (the group's first wave, lanes 0..31), staged through registers
    auto qf_load = [&](int u, float (&f)[5]) {
        const int iq = qtile0(u) + kl;
        const bool ok = wi == 0 && hh == 0 && iq < p.T;
        const int ii = ok ? iq : 0;
        f[0] = ok ? p.lse[(int64_t)ii * p.lse_st + (int64_t)head * p.lse_sh] * kLog2e : INFINITY;
        f[1] = ok ? p.ws_delta[(int64_t)head * p.T + ii] : 0.f;
        f[2] = ok ? p.ws_rec[(int64_t)kRecW * p.T + ii] : 0.f;
        f[3] = ok ? p.ws_rec[(int64_t)kRecCore * p.T + ii] : __int_as_float(INT_MAX);
        f[4] = ok ? p.ws_rec[(int64_t)kRecPmax * p.T + ii] : __int_as_float(-1);
    };

    const int tj = kvalid ? j : p.T - 1;
    vec8 kv[KS], vv[KS];
    {
        const uint16_t *kp = p.k + (int64_t)tj * p.k_st + (int64_t)kv_head(head, p.kv_rep) * p.k_sh + hh * 8;
        const uint16_t *vp = p.v + (int64_t)tj * p.v_st + (int64_t)kv_head(head, p.kv_rep) * p.v_sh + hh * 8;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            kv[s] = bitcast<vec8>(*reinterpret_cast<const uint4 *>(kp + s * 16));
            vv[s] = bitcast<vec8>(*reinterpret_cast<const uint4 *>(vp + s * 16));
        }
    }
    const float lbj = (p.lb && kvalid) ? p.lb[(int64_t)head * p.lb_sh + (int64_t)j * p.lb_st] * kLog2e : -INFINITY;
    const float c = p.c;

    if (grp < nu) issue(0);
    float qf[5];
    qf_load(grp, qf);  // fields of a tile past the sequence read as "no query"
    f32x16 dk[ND], dv[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dk[d][r] = 0.f;
            dv[d][r] = 0.f;
        }
    float dlb = 0.f;

    for (int it = 0; it < nit; ++it) {
        const int u = grp + NG * it;
        const int slot = it & 1;
        if (wi == 0 && hh == 0) {
#pragma unroll
            for (int f = 0; f < 5; ++f) s_qf[grp][slot][f][kl] = qf[f];
        }
        tile_barrier<0>();  // the step's tiles landed for every group; everyone left step it-1
        if (u + NG < nu) {
            issue(it + 1);
            qf_load(u + NG, qf);
        }
        if (u >= nu) continue;  // group-uniform
        const char *qtile = s_tiles[grp][slot][0];
        const char *dtile = s_tiles[grp][slot][1];
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = 0.f;
            dp[r] = 0.f;
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            s = DT::mfma(bitcast<vec8>(tile_read_row16<D>(qtile, kl, 2 * ks + hh)), kv[ks], s);
            dp = DT::mfma(bitcast<vec8>(tile_read_row16<D>(dtile, kl, 2 * ks + hh)), vv[ks], dp);
        }
        // element r is query q0 + hh*4 + acc_row_const(r) of this tile, key j
        const int q0 = qtile0(u);
        uint32_t pkp[8], pks[8];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float fv[5][4];
#pragma unroll
            for (int f = 0; f < 5; ++f) {
                const float4 v4 = *reinterpret_cast<const float4 *>(&s_qf[grp][slot][f][g * 8 + hh * 4]);
                fv[f][0] = v4.x; fv[f][1] = v4.y; fv[f][2] = v4.z; fv[f][3] = v4.w;
            }
            float pr[4], dsv[4];
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                const int rr = g * 4 + e4;
                const int iq = q0 + hh * 4 + acc_row_const(rr);
                const int dd = iq - j;
                const float wq = fv[2][e4];
                const float e = fast_exp2(((float)dd - wq) * p.inv_tau * kLog2e);
                float oms;
                bool clamped;
                const float bw = window_bias2(e, j >= __float_as_int(fv[3][e4]), oms, clamped);
                const float bl = j <= __float_as_int(fv[4][e4]) ? lbj : -INFINITY;
                const bool keep = dd >= 0 && iq < p.T && kvalid && fv[0][e4] < INFINITY;
                pr[e4] = keep ? fast_exp2(fmaf(s[rr], c, fmaxf(bw, bl) - fv[0][e4])) : 0.f;
                dsv[e4] = pr[e4] * (dp[rr] - fv[1][e4]);
                float sw, sl;
                bias_shares(bw, bl, sw, sl);
                dlb = fmaf(dsv[e4], sl, dlb);
            }
            pkp[2 * g] = DT::pack2(pr[0], pr[1]);
            pkp[2 * g + 1] = DT::pack2(pr[2], pr[3]);
            pks[2 * g] = DT::pack2(dsv[0], dsv[1]);
            pks[2 * g + 1] = DT::pack2(dsv[2], dsv[3]);
        }
        // dV^T += dO^T . P and dK^T += Q^T . dS (the query tiles read transposed)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const vec8 bp = bitcast<vec8>(make_uint4(pkp[kk * 4], pkp[kk * 4 + 1], pkp[kk * 4 + 2], pkp[kk * 4 + 3]));
            const vec8 bs = bitcast<vec8>(make_uint4(pks[kk * 4], pks[kk * 4 + 1], pks[kk * 4 + 2], pks[kk * 4 + 3]));
#pragma unroll
            for (int d = 0; d < ND; ++d) {
                dv[d] = DT::mfma(bitcast<vec8>(tile_read_tr<D, kSwzRow>(dtile, kk * 16, d * 32, lane)), bp, dv[d]);
                dk[d] = DT::mfma(bitcast<vec8>(tile_read_tr<D, kSwzRow>(qtile, kk * 16, d * 32, lane)), bs, dk[d]);
            }
        }
    }
    tile_barrier<0>();  // every group is done with its ring: the rings become the merge buffer
    {
        float *mbuf = reinterpret_cast<float *>(&s_tiles[0][0][0][0]);
        auto mslot = [&](int g, int e) { return mbuf + ((((g - 1) * 2 + wi) * MERGE + e) * 64 + lane); };
        // round 1: dK and the bias gradient
        if (grp > 0) {
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) *mslot(grp, d * 16 + r) = dk[d][r];
            *mslot(grp, ND * 16) = dlb;
        }
        __syncthreads();
        if (grp == 0) {
#pragma unroll
            for (int g = 1; g < NG; ++g) {
#pragma unroll
                for (int d = 0; d < ND; ++d)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dk[d][r] += *mslot(g, d * 16 + r);
                dlb += *mslot(g, ND * 16);
            }
        }
        __syncthreads();
        // round 2: dV
        if (grp > 0) {
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) *mslot(grp, d * 16 + r) = dv[d][r];
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int g = 1; g < NG; ++g)
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) dv[d][r] += *mslot(g, d * 16 + r);
    }
    const float dl = half_sum(dlb);  // dS is the gradient of a natural-log logit, hence of its bias
    if (kvalid) {
        const int64_t ok = (int64_t)j * p.dk_st + (int64_t)head * p.dk_sh;
        const int64_t ov = (int64_t)j * p.dv_st + (int64_t)head * p.dv_sh;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dd = d * 32 + g * 8 + hh * 4;
                const float k0_ = dk[d][g * 4] * p.scale, k1 = dk[d][g * 4 + 1] * p.scale;
                const float k2 = dk[d][g * 4 + 2] * p.scale, k3 = dk[d][g * 4 + 3] * p.scale;
                const float v0 = dv[d][g * 4], v1 = dv[d][g * 4 + 1], v2 = dv[d][g * 4 + 2], v3 = dv[d][g * 4 + 3];
                if (p.grad_f32) {
                    *reinterpret_cast<float4 *>(static_cast<float *>(p.dk) + ok + dd) = make_float4(k0_, k1, k2, k3);
                    *reinterpret_cast<float4 *>(static_cast<float *>(p.dv) + ov + dd) = make_float4(v0, v1, v2, v3);
                } else {
                    uint2 a, b;
                    a.x = DT::pack2(k0_, k1);
                    a.y = DT::pack2(k2, k3);
                    b.x = DT::pack2(v0, v1);
                    b.y = DT::pack2(v2, v3);
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p.dk) + ok + dd) = a;
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p.dv) + ov + dd) = b;
                }
            }
        if (hh == 0 && p.d_lb) p.d_lb[(int64_t)head * p.T + j] = dl;
    }
}

__global__ void __launch_bounds__(256) dense_dw_kernel(const DenseParams p) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= p.T) return;
    float acc = 0.f;
    for (int h = 0; h < p.H; ++h) acc += p.ws_dwh[(int64_t)i * p.H + h];
    p.d_w[i] = acc;
}

DenseParams dense_params(int T, int H, int D) {
    DenseParams p{};
    p.T = T;
    p.H = H;
    p.n_blk = (T + kDB - 1) / kDB;
    const int64_t blocks = (int64_t)p.n_blk * H;
    p.grid = (int)((blocks + 7) / 8 * 8);
    (void)D;
    return p;
}

void set_common(DenseParams &p, float scale, float tau_win, float win_edge) {
    p.scale = scale;
    p.c = scale * kLog2e;
    p.inv_c = 1.f / p.c;
    p.inv_tau = 1.f / tau_win;
    p.win_edge = win_edge;
    // The factored tail e = E * ec[r] needs E = exp((A - w~ - 13.5) / tau) finite wherever
    // the true e = exp((d - w~) / tau) is below the clamp (e <= e^46; beyond it the bias is
    // log 1e-20 either way): E <= e^46 / min ec = e^(46 + 13.5 / tau) < e^88 needs
    // 13.5 / tau < 42; with a margin, tau > 0.3375. Smaller tau takes one exp per element.
    p.edge_fast = kEdgeMidD * p.inv_tau < 40.f;
}

template <typename DT>
hipError_t dense_fwd_dt(const DenseParams &p, int D, hipStream_t stream) {
    if (D == 64) hipLaunchKernelGGL((dense_fwd_kernel<DT, 64>), dim3(p.grid), dim3(128 * dense_fwd_groups(64)), 0, stream, p);
    else hipLaunchKernelGGL((dense_fwd_kernel<DT, 128>), dim3(p.grid), dim3(128 * dense_fwd_groups(128)), 0, stream, p);
    return hipGetLastError();
}

template <typename DT>
hipError_t dense_bwd_dt(const DenseParams &p, int D, hipStream_t stream) {
    const int64_t n = (int64_t)p.T * p.H;
    hipLaunchKernelGGL((dense_prep_kernel<DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p, D);
    if (D == 64) {
        hipLaunchKernelGGL((dense_dq_kernel<DT, 64>), dim3(p.grid), dim3(128 * dense_bwd_groups(64)), 0, stream, p);
        hipLaunchKernelGGL((dense_kv_kernel<DT, 64>), dim3(p.grid), dim3(128 * dense_bwd_groups(64)), 0, stream, p);
    } else {
        hipLaunchKernelGGL((dense_dq_kernel<DT, 128>), dim3(p.grid), dim3(128 * dense_bwd_groups(128)), 0, stream, p);
        hipLaunchKernelGGL((dense_kv_kernel<DT, 128>), dim3(p.grid), dim3(128 * dense_bwd_groups(128)), 0, stream, p);
    }
    if (p.d_w) hipLaunchKernelGGL(dense_dw_kernel, dim3((p.T + 255) / 256), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dense_fwd(const dsalt_fwd_args &a, hipStream_t stream) {
    if (a.total_len == 0) return hipSuccess;
    DenseParams p = dense_params(a.total_len, a.n_heads, a.head_dim);
    p.kv_rep = a.n_kv_heads > 0 ? a.n_heads / a.n_kv_heads : 1;
    p.q = static_cast<const uint16_t *>(a.q);
    p.k = static_cast<const uint16_t *>(a.k);
    p.v = static_cast<const uint16_t *>(a.v);
    p.out = a.out;
    p.out_f32 = a.out_dtype == DSALT_DTYPE_F32;
    p.lse = a.lse;
    p.w = a.w;
    p.lb = a.lmk_bias;
    p.q_st = a.q_stride_t; p.q_sh = a.q_stride_h;
    p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
    p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
    p.o_st = a.out_stride_t; p.o_sh = a.out_stride_h;
    p.lse_st = a.lse_stride_t; p.lse_sh = a.lse_stride_h;
    p.w_st = a.w_stride;
    p.lb_sh = a.lmk_bias_stride_h; p.lb_st = a.lmk_bias_stride_k;
    set_common(p, a.scale, a.tau_win, a.win_edge);
    return a.dtype == DSALT_DTYPE_BF16 ? dense_fwd_dt<BF16>(p, a.head_dim, stream)
                                       : dense_fwd_dt<F16>(p, a.head_dim, stream);
}

int64_t dense_bwd_workspace_bytes(int total_len, int n_heads) {
    auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
    return al((int64_t)n_heads * total_len * 4) + al((int64_t)kDRec * total_len * 4) +
           al((int64_t)n_heads * total_len * 4);
}

hipError_t launch_dense_bwd(const dsalt_bwd_args &a, hipStream_t stream) {
    if (a.total_len == 0) return hipSuccess;
    DenseParams p = dense_params(a.total_len, a.n_heads, a.head_dim);
    p.kv_rep = a.n_kv_heads > 0 ? a.n_heads / a.n_kv_heads : 1;
    p.q = static_cast<const uint16_t *>(a.q);
    p.k = static_cast<const uint16_t *>(a.k);
    p.v = static_cast<const uint16_t *>(a.v);
    p.dout = static_cast<const uint16_t *>(a.dout);
    p.o = a.out;
    p.o_f32 = a.out_dtype == DSALT_DTYPE_F32;
    p.lse = const_cast<float *>(a.lse);  // read only in the backward
    p.w = a.w;
    p.lb = a.lmk_bias;
    p.dq = a.dq;
    p.dk = a.dk;
    p.dv = a.dv;
    p.grad_f32 = a.grad_dtype == DSALT_DTYPE_F32;
    p.d_lb = a.d_lmk_bias;
    p.d_w = a.d_w;
    char *ws = static_cast<char *>(a.workspace);
    auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
    p.ws_delta = reinterpret_cast<float *>(ws);
    ws += al((int64_t)a.n_heads * a.total_len * 4);
    p.ws_rec = reinterpret_cast<float *>(ws);
    ws += al((int64_t)kDRec * a.total_len * 4);
    p.ws_dwh = reinterpret_cast<float *>(ws);
    p.q_st = a.q_stride_t; p.q_sh = a.q_stride_h;
    p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
    p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
    p.o_st = a.out_stride_t; p.o_sh = a.out_stride_h;
    p.do_st = a.dout_stride_t; p.do_sh = a.dout_stride_h;
    p.lse_st = a.lse_stride_t; p.lse_sh = a.lse_stride_h;
    p.w_st = a.w_stride;
    p.lb_sh = a.lmk_bias_stride_h; p.lb_st = a.lmk_bias_stride_k;
    p.dq_st = a.dq_stride_t; p.dq_sh = a.dq_stride_h;
    p.dk_st = a.dk_stride_t; p.dk_sh = a.dk_stride_h;
    p.dv_st = a.dv_stride_t; p.dv_sh = a.dv_stride_h;
    set_common(p, a.scale, a.tau_win, a.win_edge);
    return a.dtype == DSALT_DTYPE_BF16 ? dense_bwd_dt<BF16>(p, a.head_dim, stream)
                                       : dense_bwd_dt<F16>(p, a.head_dim, stream);
}

}  // namespace dsalt
