// Fused DSALT sparse-attention forward for gfx950 (HARD and SOFT semantics).
//
// Reference semantics: _dsalt_fwd_kernel (dsalt/kernels/dsalt_triton_attn.py:27-169) and
// _train_fwd_kernel (dsalt/kernels/dsalt_triton_train.py:74-214); the landmark K/V
// gather of _build_landmark_kv (dsalt/kernels/selectors.py:137-159) is done in-kernel.
//
// Design (one workgroup = fwd_waves(D) waves of 32 consecutive queries each, of one
// (sequence, head)):
//  * Each wave owns 32 queries and computes S^T = K . Q^T with v_mfma_f32_32x32x16, so
//    a lane holds ONE query (column lane%32) and 16 keys per 32-key block: the row max
//    is an in-register max plus one v_permlane32_swap between the two lane halves, and
//    P^T converts in place into the B operand of O^T += V^T . P^T (no data movement).
//  * K and V tiles (BN = 32 keys: 4 KB each at D = 64, 8 KB at D = 128) go global ->
//    LDS with direct loads (buffer_load_dwordx4 ... lds, no register staging) into two
//    rings of R slots, one for K and one for V: K runs R tiles ahead of the S = K Q^T
//    MFMAs, V R-1 tiles ahead of the P V MFMAs. At D = 64 (R = 2: 16 KB of tiles, 128
//    VGPRs) that fits 8 HARD workgroups per CU, i.e. a whole 2048-token x 16-head batch
//    of 4 sequences in one dispatch round; 2 workgroups at D = 128. K is read
//    row-major, V with the transposing
//    ds_read_b64_tr_b16 (the PV operand needs keys along K); both tiles are XOR-swizzled
//    so that either read pattern is bank-conflict free (tiles.h).
//  * The workgroup streams the union of its waves' key ranges
//    [min_i(i - w_i + 1), max_i i]. Each tile iteration is branch-free: the band mask
//    (keys outside [lo_i, i], which also covers tiles outside a wave's range) is applied
//    to every tile, so that the softmax VALU work of tile t and the S = K Q^T MFMAs of
//    tile t+1 form one basic block, as do the O += P V MFMAs of tile t and the mask and
//    row max of tile t+1; sched_group_barrier interleaves MFMA and VALU inside each.
//  * Landmark K/V rows are gathered straight from K/V into the same tile buffers after
//    the band, with per-slot admission (p <= p_max(i)) and per-slot logit bias applied
//    in place by a rare (wave-uniform) branch, as is the SOFT edge bias of band tiles
//    that reach below a row's core.
//  * Online softmax in base 2 with a stale maximum: the running max is only raised (and
//    O rescaled) when a tile exceeds it by more than 2^8, which keeps P <= 256.
//  * The workgroup -> (head, sequence, block) map is computed in-kernel from cu_seqlens
//    (no host-side block map): each XCD owns whole heads, and blocks arrive in
//    decreasing block index so that the long late blocks start first.
#include "common.h"
#include "launch.h"
#include "tiles.h"

#include <atomic>
#include <type_traits>

namespace dsalt {
namespace {

constexpr float kStaleMax = 8.0f;  // allowed growth of the row max before a rescale (log2)
// SOFT: win_edge <= kEdgeTab runs kSoft, whose score accumulators start from a per-query
// row of kEtabLen initial values. The row holds ceil(win_edge) <= kEdgeTab edge keys,
// which is every edge while w~ - win_edge is exact in fp32 (w~ < 2^25). Wider edges run
// kSoftWide (edge bias computed on every band element below the core).
constexpr int kEdgeTab = 4;
constexpr int kEtabLen = kEdgeTab + 8;  // entries per query row: keys lo - 4 .. lo + kEdgeTab + 3
// row of query q (of the workgroup) at q * kEtabLen + q / 8: with kEtabLen = 12 the 32
// rows of a wave then start in 32 different banks
__host__ __device__ constexpr int etab_row(int q) { return q * kEtabLen + (q >> 3); }
static_assert(kEdgeTab == 4, "edge table rows are laid out for 4 edge keys");
// Band mask table: acc_row_const(r) <= 27 for the 16 accumulator elements of a lane, so
// rows d = 0 (nothing masked) .. 28 (everything masked) cover every clamped bound.
constexpr int kMaskRows = 29;
constexpr int kMaskStride = 20;

struct FwdParams {
    const uint16_t *q, *k, *v;
    void *o;  // [T,H,D]: fp32 if out_f32, else the compute dtype
    float *lse;
    const float *w;
    const int64_t *lmk_pos;
    const float *lmk_bias;
    const int32_t *cu;
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lse_st, lse_sh, w_st;
    int64_t lp_sh, lp_ss, lp_sk, lb_sh, lb_ss, lb_sk;
    int total_len, num_seqs, n_heads, k_lmk, k_pad, n_qblk, grid, out_f32;
    int prio_span;    // > 0: wave priority by dispatch order over the first prio_span workgroups
    int kv_rep;       // query heads per K/V head
    const float *rope_cos, *rope_sin;  // non-null: rotate Q on load (RoPE tables [rope_rows][D])
    int64_t rope_st;
    int rope_rows;
    int rope_half;    // the tables' second half equals the first: read D/2 columns
    uint32_t q_sign;  // 0x80008000 when scale < 0 (Q is negated on load and |scale| used)
    float c;          // |scale| * log2(e): raw q.k -> log2-unit logit
    float inv_c;      // 1 / c: log2-unit (or natural, times log2 e) bias -> raw units
    float inv_tau, win_edge;
};

template <typename DT, int D, int MODE>
__global__ void __launch_bounds__(64 * fwd_waves(D), fwd_waves_per_simd(D, MODE == kSoftWide)) fwd_kernel(const FwdParams p) {
    typedef typename DT::vec8 vec8;
    constexpr int NW = fwd_waves(D);        // waves per workgroup
    constexpr int BM = 32 * NW;             // queries per workgroup
    constexpr int NT = 64 * NW;             // threads per workgroup
    constexpr int BN = fwd_bn(D);           // keys per tile
    constexpr int NRB = BN / 32;            // 32-key row blocks of S^T per tile
    constexpr int KS = D / 16;              // MFMA k-steps over the head dim
    constexpr int ND = D / 32;              // 32-row blocks of O^T
    typedef TileN<D, BN, NW> Tile;
    constexpr int TB = Tile::BYTES;
    constexpr int R = fwd_ring(D);                     // depth of the K ring and of the V ring
    constexpr int LPT = 2 * Tile::LOADS_PER_WAVE;      // load instructions per tile per wave
    constexpr int NC = BM / BN;                        // band tiles reaching past a wave's first query
    static_assert(NC >= 1 && NC <= 4, "causal peel covers at most four tiles");
    static_assert(R <= NC, "the tiles issued before the set-up are peel band tiles");
    // The first attempt keeps the exponent offset mu where the diagonal tiles (which hold
    // every query's own key) put it and takes no row max after them: P = 2^(S c - mu) may
    // then exceed the usual 2^8, which needs the 16-bit type to have the exponent range of
    // fp32: bf16. (The wide-edge SOFT kernel, whose edge factors fill the registers, keeps
    // the single attempt.)
    constexpr bool kTryFast = std::is_same<DT, BF16>::value && MODE != kSoftWide;

    __shared__ __align__(1024) char s_tiles[2][R][TB];  // [K, V][slot]
    __shared__ int s_red[NW][2];
    __shared__ int s_ltmin[DSALT_MAX_K_LMK / BN];  // smallest position in each landmark tile
    // Band mask rows: row d holds, per accumulator element r of a 32-key row block, -inf
    // when the element's row offset acc_row_const(r) is below d, else 0 (rows padded to
    // 80 bytes so that lanes reading different rows spread over the banks).
    __shared__ __align__(16) float s_mtab[MODE == kSoft ? 1 : kMaskRows][kMaskStride];
    // kSoft: per query, the initial scores of keys lo - 4 .. lo + kEdgeTab + 3 (-inf below
    // the band, the edge biases, 0 in the core)
    __shared__ float s_etab[MODE == kSoft ? etab_row(BM) : 1];
    extern __shared__ int s_dyn[];
    int *s_lpos = s_dyn;                                          // INT_MAX: empty slot
    float *s_lbias = reinterpret_cast<float *>(s_dyn + p.k_pad);  // raw-unit bias
    int *s_lrow = s_dyn + 2 * p.k_pad;                            // row to load (0 if empty)

    // `wave` through readfirstlane: the compiler then knows it is wave-uniform, so every
    // per-wave decision below is a scalar branch (no exec masking, no register merges).
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;

    // ---- workgroup -> (head, sequence, query block) -----------------------------------
    // Blocks are dispatched in decreasing block index: late blocks have the widest key
    // ranges, and starting them first shortens the tail of the launch.
    int head, rank;
    head_rank(blockIdx.x, p.grid, p.n_heads, p.n_qblk, head, rank);
    if (head >= p.n_heads) return;
    int seq, blk, seq_start, seq_len;
    if (!find_block_desc(p.cu, p.num_seqs, p.total_len, rank, p.n_qblk, BM, lane, seq, blk, seq_start, seq_len)) return;
    const int wq0 = blk * BM + wave * 32;      // first query of this wave
    const int i = wq0 + ql;                    // query offset inside the sequence
    const bool qvalid = i < seq_len;
    const int64_t tok_i = (int64_t)seq_start + i;
    const int ghi = min(blk * BM + BM - 1, seq_len - 1);  // last query of the workgroup

    // ---- tile staging: direct global -> LDS loads ----------------------------------------
    // Tile order: the NC band tiles of the diagonal (t < NC; band tile b holds keys
    // ghi-BN+1-BN*b .. ghi-BN*b, so they are known before the windows are read and their
    // loads overlap the setup), then the landmark tiles, then the remaining band tiles
    // from the diagonal down. A wave whose own band ends before the workgroup's has its
    // idle tiles last and only takes part in the loads and barriers for them. K/V rows are
    // read through buffer resources whose range is this (sequence, head): rows below the
    // sequence start (wrapped offsets) read as zeros, empty landmark slots load row 0; the
    // masks give all of them probability 0.
    const uint32_t kst = (uint32_t)p.k_st * 2u, vst = (uint32_t)p.v_st * 2u;  // row strides (bytes)
    const i32x4 krs = buffer_rsrc(p.k + (int64_t)seq_start * p.k_st + (int64_t)kv_head(head, p.kv_rep) * p.k_sh, (uint32_t)seq_len * kst);
    const i32x4 vrs = buffer_rsrc(p.v + (int64_t)seq_start * p.v_st + (int64_t)kv_head(head, p.kv_rep) * p.v_sh, (uint32_t)seq_len * vst);
    const TileLanes<D, kSwzRow, BN, NW> klanes(wave, lane, kst);
    const TileLanes<D, kSwzTr, BN, NW> vlanes(wave, lane, vst);
    const uint32_t tiles_lds = lds_addr(&s_tiles[0][0][0]);
    auto band_key0 = [&](int b) { return ghi - (BN - 1) - b * BN; };
    auto slot_of = [](int t) { return t % R; };  // ring slot of tile t >= 0, wave-uniform
    auto k_lds = [&](int t) { return tiles_lds + slot_of(t) * TB; };
    auto v_lds = [&](int t) { return tiles_lds + (R + slot_of(t)) * TB; };
    // ---- global loads of the setup, issued before the first tile loads: loads complete
    // in issue order, so waiting for these does not wait for the tiles ----------------
    // Invalid lanes load a clamped valid row (their results are never stored), so no
    // load sits in a divergent branch (which would make the compiler wait on it early).
    vec8 qv[KS];
    {
        const int64_t tq = qvalid ? tok_i : (int64_t)seq_start + seq_len - 1;
        const uint16_t *qp = p.q + tq * p.q_st + (int64_t)head * p.q_sh + hh * 8;
#pragma unroll
        for (int s = 0; s < KS; ++s) qv[s] = bitcast<vec8>(*reinterpret_cast<const uint4 *>(qp + s * 16));
    }
    const float wraw = p.w[(qvalid ? tok_i : (int64_t)seq_start + seq_len - 1) * p.w_st];
    // landmark slots s = tid + NT j (k_pad <= DSALT_MAX_K_LMK)
    constexpr int LMK_PER_THREAD = DSALT_MAX_K_LMK / NT;
    int64_t lpp[LMK_PER_THREAD];
    float lbb[LMK_PER_THREAD];
#pragma unroll
    for (int j = 0; j < LMK_PER_THREAD; ++j) {
        lpp[j] = -1;
        lbb[j] = 0.f;
        if (NT * j < p.k_lmk) {  // wave-uniform
            const int s = min(tid + NT * j, p.k_lmk - 1);
            lpp[j] = p.lmk_pos[head * p.lp_sh + seq * p.lp_ss + s * p.lp_sk];
            if (p.lmk_bias) lbb[j] = p.lmk_bias[head * p.lb_sh + seq * p.lb_ss + s * p.lb_sk];
        }
    }
    // the first band tiles (K of tiles 0 .. R-1, V of tiles 0 .. R-2, in tile order,
    // K before V) through the compiler builtin, so that the waits for the loads above
    // count them (in-loop refills use inline asm, see tiles.h)
    {
        const __amdgpu_buffer_rsrc_t kbr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(p.k + (int64_t)seq_start * p.k_st + (int64_t)kv_head(head, p.kv_rep) * p.k_sh), (short)0, (int)((uint32_t)seq_len * kst), 0x00020000);
        const __amdgpu_buffer_rsrc_t vbr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(p.v + (int64_t)seq_start * p.v_st + (int64_t)kv_head(head, p.kv_rep) * p.v_sh), (short)0, (int)((uint32_t)seq_len * vst), 0x00020000);
#pragma unroll
        for (int t = 0; t < R; ++t) {
            const uint32_t key0 = (uint32_t)band_key0(t);  // wraps below the sequence start: reads zeros
#pragma unroll
            for (int u = 0; u < Tile::LOADS_PER_WAVE; ++u) {
                const int slot0 = (wave * Tile::LOADS_PER_WAVE + u) * 64;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    kbr, (__attribute__((address_space(3))) void *)(s_tiles[0][t] + slot0 * 16), 16,
                    (int)(key0 * kst + klanes.lane_off[u]), 0, 0, 0);
            }
            if (t < R - 1) {
#pragma unroll
                for (int u = 0; u < Tile::LOADS_PER_WAVE; ++u) {
                    const int slot0 = (wave * Tile::LOADS_PER_WAVE + u) * 64;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        vbr, (__attribute__((address_space(3))) void *)(s_tiles[1][t] + slot0 * 16), 16,
                        (int)(key0 * vst + vlanes.lane_off[u]), 0, 0, 0);
                }
            }
        }
    }

    // ---- Q (B operand: query column ql, head-dim chunk hh*8 of every 16) ---------------
    // With RoPE tables, Q is rotated here exactly as dsalt_rope does it: the lane holds
    // both halves of every rotated pair (chunk s and s + KS/2 are head dims c and c + D/2),
    // cos/sin of the query's position are rounded to the element type, products and
    // difference / sum in fp32 without contraction, the fp32 result rounded to the
    // element type.
    if (p.rope_cos) {
        const int pos = qvalid ? i : seq_len - 1;
        const bool in_table = pos < p.rope_rows;
        const float *cr = p.rope_cos + (int64_t)(in_table ? pos : 0) * p.rope_st + hh * 8;
        const float *sr = p.rope_sin + (int64_t)(in_table ? pos : 0) * p.rope_st + hh * 8;
        // the lane's 8 columns of each half as two 16-byte loads per table and half
        auto ld8 = [&](const float *t, float (&x)[8]) {
            const float4 u = *reinterpret_cast<const float4 *>(t), v4 = *reinterpret_cast<const float4 *>(t + 4);
            x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w; x[4] = v4.x; x[5] = v4.y; x[6] = v4.z; x[7] = v4.w;
        };
#pragma unroll
        for (int s = 0; s < KS / 2; ++s) {
            const int s2 = s + KS / 2;
            float c0[8], c1[8], s0[8], s1[8];
            ld8(cr + s * 16, c0);
            ld8(sr + s * 16, s0);
            if (p.rope_half) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    c1[e] = c0[e];
                    s1[e] = s0[e];
                }
            } else {
                ld8(cr + s * 16 + D / 2, c1);
                ld8(sr + s * 16 + D / 2, s1);
            }
            uint4 ra = bitcast<uint4>(qv[s]), rb = bitcast<uint4>(qv[s2]);
            const uint32_t wa[4] = {ra.x, ra.y, ra.z, ra.w}, wb[4] = {rb.x, rb.y, rb.z, rb.w};
            uint32_t oa[4], ob[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float lo[2], hi[2];
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    const int c = 2 * e + h2;
                    const float a = h2 ? DT::hi_f32(wa[e]) : DT::lo_f32(wa[e]);
                    const float b = h2 ? DT::hi_f32(wb[e]) : DT::lo_f32(wb[e]);
                    const float cc0 = in_table ? DT::round(c0[c]) : NAN, cc1 = in_table ? DT::round(c1[c]) : NAN;
                    const float ss0 = in_table ? DT::round(s0[c]) : NAN, ss1 = in_table ? DT::round(s1[c]) : NAN;
                    lo[h2] = __fsub_rn(__fmul_rn(a, cc0), __fmul_rn(b, ss0));
                    hi[h2] = __fadd_rn(__fmul_rn(b, cc1), __fmul_rn(a, ss1));
                    // rounded to fp32 first: no fp16 fma_mix folding of the sum and the conversion
                    asm volatile("" : "+v"(lo[h2]), "+v"(hi[h2]));
                }
                oa[e] = DT::pack2(lo[0], lo[1]);
                ob[e] = DT::pack2(hi[0], hi[1]);
            }
            qv[s] = bitcast<vec8>(make_uint4(oa[0], oa[1], oa[2], oa[3]));
            qv[s2] = bitcast<vec8>(make_uint4(ob[0], ob[1], ob[2], ob[3]));
        }
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        uint4 raw = bitcast<uint4>(qv[s]);
        raw.x ^= p.q_sign; raw.y ^= p.q_sign; raw.z ^= p.q_sign; raw.w ^= p.q_sign;
        qv[s] = bitcast<vec8>(raw);
    }

    // ---- per-query key ranges -----------------------------------------------------------
    // lo: first band key; corelo: first key of the zero-bias core; pmax: largest
    // admissible landmark position (-1: none). All inclusive, relative to the sequence.
    const float wv = qvalid ? wraw : 0.f;
    int lo, corelo, pmax;
    query_ranges<MODE>(i, wv, p.win_edge, lo, corelo, pmax);
    const int wlo = wave_min_u(qvalid ? lo : INT_MAX);
    const int wclo = MODE == kSoftWide ? wave_max_u(qvalid ? corelo : INT_MIN) : INT_MIN;
    const int wpmax = wave_max_u(qvalid ? pmax : -1);

    // ---- landmark slots -> LDS (invalid / out-of-sequence slots become INT_MAX) --------
    // k_pad is a multiple of 64: slot block j of wave w (64 slots from s = 64 (NW j + w))
    // is landmark tile s / 64 when BN = 64, tiles s / 32 and s / 32 + 1 when BN = 32.
#pragma unroll
    for (int j = 0; j < LMK_PER_THREAD; ++j) {
        const int s = tid + NT * j;
        if (NT * j < p.k_pad) {  // wave-uniform (k_pad is a multiple of 64)
            if (s < p.k_pad) {
                const bool ok = s < p.k_lmk && lpp[j] >= 0 && lpp[j] < seq_len;
                const int pos = ok ? (int)lpp[j] : INT_MAX;
                s_lpos[s] = pos;
                s_lbias[s] = ok ? lbb[j] * (kLog2e * p.inv_c) : 0.f;
                s_lrow[s] = ok ? pos : 0;
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
        }
    }
    if (lane == 0) {
        s_red[wave][0] = wlo;
        s_red[wave][1] = wpmax;
    }
    if constexpr (MODE != kSoft) {
        for (int e = tid; e < kMaskRows * 16; e += NT) {
            const int d = e >> 4, r = e & 15;
            s_mtab[d][r] = acc_row_const(r) < d ? -INFINITY : 0.f;
        }
    } else {
        // the query's row: entry x + 4 holds the initial score of key lo + x, x = -4 ..
        // kEdgeTab + 3: -inf below the band, the edge bias log2 sigmoid((w~ - d) / tau)
        // for lo <= key < corelo (dsalt_triton_train.py:151-155), 0 in the core. The lane
        // pair splits the row.
        constexpr int EH = kEtabLen / 2;
        float *erow = s_etab + etab_row(wave * 32 + ql);
        const int ne = corelo - lo;
#pragma unroll
        for (int e = 0; e < EH; ++e) {
            const int x = hh * EH + e - 4;
            float oms;
            const float edge = soft_edge_log2(wv, (float)(i - lo - x), p.inv_tau, oms) * p.inv_c;
            erow[hh * EH + e] = x < 0 ? -INFINITY : (x < ne ? edge : 0.f);
        }
    }
    // LDS writes visible to the workgroup; the tile loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    int glo = s_red[0][0], gpmax = s_red[0][1];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        glo = min(glo, s_red[w][0]);
        gpmax = max(gpmax, s_red[w][1]);
    }
    // landmark tiles holding at least one position admissible for the workgroup
    const int n_lt = p.k_pad / BN;
    const uint64_t lmask = __ballot(lane < n_lt && s_ltmin[lane < n_lt ? lane : 0] <= gpmax);
    const int nl = __popcll(lmask);
    // band tiles of the workgroup (at least the NC of the peel; extra ones are inactive)
    const int nb = max((ghi - glo) / BN + 1, NC);
    const int nt = nb + nl;
    // tile t: band tile t for t < NC, landmark tile for NC <= t < NC + nl, band tile t - nl after
    auto is_lmk = [&](int t) { return t >= NC && t < NC + nl; };
    auto band_of = [&](int t) { return t < NC ? t : t - nl; };
    auto lmk_tile = [&](int t) {  // landmark tile of iteration t: the (t-NC)-th set bit
        uint64_t m = lmask;
        for (int j = NC; j < t; ++j) m &= m - 1;
        return (int)__builtin_ctzll(m);
    };
    // the band tiles with work for this wave: 0 .. nbw-1; its steps: t < t_end
    const int nbw = wlo <= ghi ? (ghi - wlo) / BN + 1 : 0;
    const int t_end = NC + nl + max(nbw - NC, 0);
    // band tile 0 (keys from ghi - BN + 1) reaches this wave's last query
    const bool live0 = ghi - (BN - 1) <= min(wq0 + 31, seq_len - 1);
    // K or V rows of tile t into their ring slot
    auto issue_k = [&](int t) {
        if (is_lmk(t)) klanes.load_gather_lean(k_lds(t), wave, krs, kst, s_lrow + lmk_tile(t) * BN);
        else klanes.load_band(k_lds(t), wave, krs, (uint32_t)band_key0(band_of(t)) * kst, kst);  // wraps when key0 < 0
    };
    auto issue_v = [&](int t) {
        if (is_lmk(t)) vlanes.load_gather_lean(v_lds(t), wave, vrs, vst, s_lrow + lmk_tile(t) * BN);
        else vlanes.load_band(v_lds(t), wave, vrs, (uint32_t)band_key0(band_of(t)) * vst, vst);
    };

    // S^T (BN keys x 32 queries) = K . Q^T, raw q.k, of tile t from the K tile in ring
    // slot `slot`. The accumulator starts from the band mask's lower edge: element (rb, r)
    // is key tb + 32 rb + acc_row_const(r) + 4 hh, below lo exactly when
    // acc_row_const(r) < lo - tb - 32 rb - 4 hh = mb + BN b - 32 rb (b the band index), so
    // its initial value is mask row clamp(mb + BN b - 32 rb, 0, 28): -inf there (the MFMA
    // keeps it -inf), 0 elsewhere. No VALU touches the elements; landmark tiles start from
    // row 0 (zeros). kSoft instead reads the initial values from the query's edge row,
    // four consecutive keys (elements 4g .. 4g + 3) at a time: the entries of keys
    // x .. x + 3 relative to lo with x clamped to [-4, kEdgeTab] (one v_med3 and two
    // ds_read2 per group; all four entries are -inf below the clamp and 0 above it;
    // landmark tiles clamp to the top, 0): the band's lower edge and the SOFT edge bias
    // together.
    int mb = lo - ghi + BN - 1 - hh * 4;
    auto qk_tile = [&](int t, int slot, f32x16 (&sacc)[NRB]) {
        const char *ktile = s_tiles[0][slot];
        const bool band = !is_lmk(t);
        const int b = band_of(t);
        // kSoft: the edge row from the lane id, per tile (opaque: not held across the loop)
        int el = 0;
        if constexpr (MODE == kSoft) {
            el = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
            asm volatile("" : "+v"(el));
        }
        const float *erow = s_etab + etab_row(wave * 32 + (el & 31)) + 4;
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            f32x16 acc;
            if constexpr (MODE == kSoft) {
                const int x0 = band ? -(mb + BN * b - 32 * rb) : (1 << 20);  // key - lo of row offset 0
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int y = min(max(x0, -4 - 8 * g), kEdgeTab - 8 * g);
                    const float *e4 = erow + 8 * g + y;
                    acc[4 * g + 0] = e4[0];
                    acc[4 * g + 1] = e4[1];
                    acc[4 * g + 2] = e4[2];
                    acc[4 * g + 3] = e4[3];
                }
            } else {
                const int d = band ? min(max(mb + BN * b - 32 * rb, 0), kMaskRows - 1) : 0;
                const float4 *mrow = reinterpret_cast<const float4 *>(&s_mtab[d][0]);
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 m4 = mrow[g];
                    acc[4 * g + 0] = m4.x;
                    acc[4 * g + 1] = m4.y;
                    acc[4 * g + 2] = m4.z;
                    acc[4 * g + 3] = m4.w;
                }
            }
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const vec8 a = bitcast<vec8>(tile_read_row16<D>(ktile, rb * 32 + ql, 2 * s + hh));
                acc = DT::mfma(a, qv[s], acc);
            }
            sacc[rb] = acc;
        }
    };

    const float c = p.c;
    f32x16 oacc[ND];
    float m2, mu, thr;     // running max (log2 units, stale by at most kStaleMax), exponent offset, raise threshold (raw)
    float lsum0, lsum1;    // row sums of the rounded P
    // kSoftWide edge factors: for element slot j (tile row offset cst_j), exp(-z) of the edge
    // logit z = (w~ - d) / tau splits as E * ec[j] with E = exp((A - w~ - mid) / tau) per
    // lane and tile and ec[j] = exp((mid - cst_j) / tau) fixed. Every factor stays in the
    // fp32 range while (win_edge + 1 + 16 NRB) / tau < 80 (edge keys have
    // 0 <= z < (win_edge + 1) / tau); otherwise each element takes its own exp.
    constexpr float kEdgeMid = 16.f * NRB - 2.5f;
    const bool edge_fast = MODE == kSoftWide && (p.win_edge + 1.f + 16.f * NRB) * p.inv_tau < 80.f;
    float ec[MODE == kSoftWide ? 16 * NRB : 1];
    if constexpr (MODE == kSoftWide) {
#pragma unroll
        for (int j = 0; j < 16 * NRB; ++j)
            ec[j] = fast_exp2((kEdgeMid - (float)((j >> 4) * 32 + acc_row_const(j & 15))) * p.inv_tau * kLog2e);
    }

    // P = 2^(S c - mu) of one tile: the 16-bit P^T operand, and
    // the row sums of the same rounded P in fp32 (one v_dot2 per pair), so that O is
    // normalised by exactly the weights its P V products used. Masked scores are -inf
    // and give 0.
    auto exp_pack = [&](const f32x16 (&sacc)[NRB], uint32_t (&pk)[NRB][8]) {
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float e0 = fast_exp2(fmaf(sacc[rb][2 * j], c, -mu));
                const float e1 = fast_exp2(fmaf(sacc[rb][2 * j + 1], c, -mu));
                pk[rb][j] = DT::pack2(e0, e1);
                if (j & 1) lsum1 = DT::add_pair(pk[rb][j], lsum1);
                else lsum0 = DT::add_pair(pk[rb][j], lsum0);
            }
    };
    // O^T (D x 32 queries) += V^T . P^T ; k-step kk covers tile keys kk*16..+15
    auto pv = [&](const uint32_t (&pk)[NRB][8], int slot) {
        const char *vtile = s_tiles[1][slot];
#pragma unroll
        for (int kk = 0; kk < 2 * NRB; ++kk) {
            const int rb = kk >> 1, g = kk & 1;
            const vec8 b = bitcast<vec8>(
                make_uint4(pk[rb][g * 4 + 0], pk[rb][g * 4 + 1], pk[rb][g * 4 + 2], pk[rb][g * 4 + 3]));
#pragma unroll
            for (int d = 0; d < ND; ++d) {
                const vec8 a = bitcast<vec8>(tile_read_tr<D>(vtile, kk * 16, d * 32, lane));
                oacc[d] = DT::mfma(a, b, oacc[d]);
            }
        }
    };
    // Per-element adjustments that only some tiles need, applied in place to the scores
    // of tile t: landmark admission (p <= p_max(i)) and bias, and (kSoftWide) the SOFT
    // edge bias of band tiles that reach below a row's core.
    auto adjust = [&](int t, f32x16 (&sacc)[NRB]) {
        if (is_lmk(t)) {
            const int lt = lmk_tile(t);
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
                        sacc[rb][r] = (pp[e] <= pmax) ? sacc[rb][r] + bb[e] : -INFINITY;
                    }
                }
        } else if (MODE == kSoftWide && band_key0(band_of(t)) < wclo) {
            const int tb = band_key0(band_of(t));
            const int A = i - tb - hh * 4;
            const int Bc = corelo - tb - hh * 4;  // key >= corelo <=> cst >= Bc
            if (edge_fast) {
                // log2 sigmoid(z) = -log2(1 + E ec[j]): one v_log per element
                const float E = fast_exp2(((float)A - wv - kEdgeMid) * p.inv_tau * kLog2e);
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int cst = rb * 32 + acc_row_const(r);
                        const float edge = -__builtin_amdgcn_logf(fmaf(E, ec[rb * 16 + r], 1.f));
                        sacc[rb][r] += (cst < Bc) ? edge * p.inv_c : 0.f;
                    }
            } else {
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int cst = rb * 32 + acc_row_const(r);
                        float oms;
                        const float edge = soft_edge_log2(wv, (float)(A - cst), p.inv_tau, oms);
                        sacc[rb][r] += (cst < Bc) ? edge * p.inv_c : 0.f;
                    }
            }
        }
    };
    // Causal edge of band tile t < NC (keys after the lane's query), applied in place by
    // VALU; later band tiles lie below every query of the workgroup. Element (rb, r) is key
    // tb + hh*4 + cst with cst = rb*32 + acc_row_const(r), kept iff cst <= A0 + BN t; nA0 is
    // the bit count of rows_le at t = 0.
    int A0 = i - ghi + BN - 1 - hh * 4;
    int nA0 = 4 * (A0 >> 3) + min((A0 & 7) + 1, 4);
    auto causal_keep = [&](int t, f32x16 (&sacc)[NRB]) {
        uint32_t keep;
        if constexpr (NRB == 1) {
            // rows_le(A0 + BN t) keeps the low clamp(nA0 + 16 t, 0, 16) bits
            const int nA = min(max(nA0 + 16 * t, 0), 16);
            keep = (uint32_t)((1ull << nA) - 1ull);
        } else {
            keep = rows_le(A0 + BN * t);
        }
        // opaque: the per-element masks are formed here, at each use (the two attempts
        // would otherwise share them and hold them across the first attempt's loop)
        asm volatile("" : "+v"(keep));
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[rb][r] = keep_if(keep, rb * 16 + r, sacc[rb][r]);
    };
    // The tile's row max (raw units, -inf if empty), used by the second attempt only.
    auto tile_max = [&](const f32x16 (&sacc)[NRB]) -> float {
        // v_max3 trees, two chains per row block
        float tm[2 * NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            tm[2 * rb] = max3f(sacc[rb][0], sacc[rb][1], sacc[rb][2]);
            tm[2 * rb + 1] = max3f(sacc[rb][3], sacc[rb][4], sacc[rb][5]);
        }
#pragma unroll
        for (int r = 6; r < 16; r += 2)
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb) {
                float &x = tm[2 * rb + (NRB == 1 ? ((r >> 1) & 1) : 0)];
                x = max3f(x, sacc[rb][r], sacc[rb][r + 1]);
            }
        float mx = max3f(tm[0], tm[1], tm[1]);
        if constexpr (NRB == 2) mx = max3f(mx, tm[2], tm[3]);
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        return max3f(__uint_as_float(sw[0]), __uint_as_float(sw[1]), __uint_as_float(sw[1]));
    };
    // Second attempt: raise the running max when the tile max exceeds it by more than
    // kStaleMax (wave-uniform branch, rare after the first tile): O and l are rescaled to it.
    auto rescale = [&](bool more, float tmax) {
        const bool raise = tmax > thr;
        if (__builtin_amdgcn_ballot_w64(raise) && more) {
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
            thr = raise ? tmax + kStaleMax * p.inv_c : thr;
        }
    };

    // ---- software-pipelined tile loop ----------------------------------------------------
    // Step t: issue K of tile t+R and V of tile t+R-1; part A: P of tile t (VALU)
    // interleaved with S of tile t+1 (MFMA); part B: O += P V of tile t (MFMA) interleaved
    // with the adjustments (and, in the second attempt, the row max) of tile t+1; then a
    // wait until K of tile t+2 and V of tile t+1 have landed. K of tile t+R takes the slot
    // of K of tile t, last read by step t-1; V of tile t+R-1 takes the slot of V of tile
    // t-1, also last read by step t-1; every wave finished those reads before the barrier
    // that ended step t-1. With R = 2 the loads issued in step t itself must land by its
    // end (wait for all); with R = 3 the needed ones were issued a step earlier and the
    // newest LPT loads may stay in flight. A wave computes steps t < t_end (its last one
    // computes S of a tile it does not use) and then only issues its share of the
    // remaining tiles' loads and waits at their barriers (drain).
    constexpr int NQK = KS * NRB, NPV = 2 * ND * NRB;
    constexpr int VALU_A = (NRB * 56 - 16 + NQK - 1) / NQK + 2;
    constexpr int VALU_B = 2;
    using causal_edge = std::true_type;
    using no_causal_edge = std::false_type;
    // `causal`: tile t+1 has a causal edge (t + 1 < NC); `live`: tile t has work for the wave
    auto step = [&](auto fast, auto causal, int t, bool live, f32x16 (&cur)[NRB], f32x16 (&nxt)[NRB]) {
        if (t + R < nt) issue_k(t + R);
        if (t + R - 1 < nt) issue_v(t + R - 1);
        uint32_t pk[NRB][8];
        qk_tile(t + 1, slot_of(t + 1), nxt);
        if (live) {
            exp_pack(cur, pk);
            __builtin_amdgcn_sched_group_barrier(0x100, NQK + 4 * NRB, 0);  // mask rows, K operand reads
            __builtin_amdgcn_sched_group_barrier(0x402, 16, 0);   // VALU / transcendental
#pragma unroll
            for (int m = 0; m < NQK; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
                __builtin_amdgcn_sched_group_barrier(0x402, VALU_A, 0);  // VALU / transcendental
            }
            // keep P and the row sums in part A (otherwise they sink past the branch below)
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
                for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(pk[rb][j]));
            asm volatile("" : "+v"(lsum0), "+v"(lsum1));
        }
        const bool more = t + 1 < t_end;
        if (more) adjust(t + 1, nxt);
        if (live) pv(pk, slot_of(t));
        if constexpr (decltype(fast)::value && !decltype(causal)::value) {
            // first attempt after the peel: the offset stays where the peel left it
        } else {
            if constexpr (decltype(causal)::value) causal_keep(t + 1, nxt);
            const float tmax = tile_max(nxt);
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * NPV, 1);  // V operand reads
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 1);        // VALU
#pragma unroll
            for (int m = 0; m < NPV; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);       // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, VALU_B, 1);  // VALU
            }
            rescale(more, tmax);
        }
        if (t + R < nt) tile_barrier<(R - 2) * LPT>();
        else tile_barrier<0>();
    };
    // One pass over the tiles: the peel (tiles 0 .. NC-1 with their causal edge), the
    // pipelined loop over the wave's steps, the drain. oacc / l / m2 start at zero / -inf.
    auto attempt = [&](auto fast) {
        // opaque per attempt: values derived from these for the peel tiles are recomputed
        // in each attempt instead of being held across the first one
        asm volatile("" : "+v"(mb), "+v"(A0), "+v"(nA0));
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[d][r] = 0.f;
        m2 = -INFINITY;
        mu = 0.f;
        thr = -INFINITY;
        lsum0 = 0.f;
        lsum1 = 0.f;
        f32x16 sA[NRB], sB[NRB];
        tile_barrier<(R - 2) * LPT>();  // K of tiles 0, 1 and V of tile 0 landed
        if (live0) {
            qk_tile(0, slot_of(0), sA);
            adjust(0, sA);
            causal_keep(0, sA);
            // the first tile's max: O and l are still zero, so nothing is rescaled
            const float tmax = tile_max(sA);
            const bool raise = tmax > thr;
            m2 = raise ? tmax * c : m2;
            mu = (m2 == -INFINITY) ? 0.f : m2;
            thr = raise ? tmax + kStaleMax * p.inv_c : thr;
        }
        // step 0 refills the slot of K of tile 0: every wave must have read it first
        tile_barrier<(R - 2) * LPT>();
        // steps 0 .. NC-2 mask the causal edge of tiles 1 .. NC-1 (nt >= NC >= R)
        if constexpr (NC > 1) step(fast, causal_edge(), 0, live0, sA, sB);
        if constexpr (NC > 2) step(fast, causal_edge(), 1, true, sB, sA);
        if constexpr (NC > 3) step(fast, causal_edge(), 2, true, sA, sB);
        constexpr int T0 = NC - 1;  // first step without a causal edge
        int t = T0;
        for (; t < t_end; t += 2) {
            if constexpr (T0 % 2 == 0) {
                step(fast, no_causal_edge(), t, true, sA, sB);
                if (t + 1 < t_end) step(fast, no_causal_edge(), t + 1, true, sB, sA);
            } else {
                step(fast, no_causal_edge(), t, true, sB, sA);
                if (t + 1 < t_end) step(fast, no_causal_edge(), t + 1, true, sA, sB);
            }
        }
        for (t = max(t_end, T0); t < nt; ++t) {
            if (t + R < nt) issue_k(t + R);
            if (t + R - 1 < nt) issue_v(t + R - 1);
            if (t + R < nt) tile_barrier<(R - 2) * LPT>();
            else tile_barrier<0>();
        }
    };

    // Wave priority by dispatch order (grids of at most two dispatch rounds): the
    // workgroups of a round start together, but the later-dispatched ones get their
    // set-up loads served last and start their tile loops up to ~5 us later (c2), so the
    // loop issues the later quarters of the round first (s_setprio 1 .. 3; workgroups of a
    // second round 3).
    if (p.prio_span > 0) {
        const int pq = __builtin_amdgcn_readfirstlane(
            (int)blockIdx.x < p.prio_span ? (int)(((int64_t)blockIdx.x * 4) / p.prio_span) : 3);
        if (pq == 1) __builtin_amdgcn_s_setprio(1);
        else if (pq == 2) __builtin_amdgcn_s_setprio(2);
        else if (pq >= 3) __builtin_amdgcn_s_setprio(3);
    }
    // First attempt with the offset fixed after the diagonal tiles (bf16). It stands when
    // every valid row total lies in [2^-60, 2^60]: then no P exceeded 2^60 (nothing
    // overflowed) and every P that underflowed weighs less than 2^-66 of its row. Otherwise
    // (logits far above the diagonal tiles' maximum, rows without keys there, NaN) the
    // workgroup runs the tiles again with the running max.
    bool redo = true;
    if constexpr (kTryFast) {
        attempt(std::true_type());
        const float lt = half_sum(lsum0 + lsum1);
        const bool bad = qvalid && !(lt >= 0x1p-60f && lt <= 0x1p60f);
        const int wave_bad = __builtin_amdgcn_ballot_w64(bad) != 0;  // every lane votes
        if (lane == 0) s_red[wave][0] = wave_bad;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        int any = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) any |= s_red[w][0];
        redo = __builtin_amdgcn_readfirstlane(any) != 0;
        if (redo) {
            // the ring is idle (every wave passed the last tile barrier): reload its first tiles
#pragma unroll
            for (int tt = 0; tt < R; ++tt) {
                klanes.load_band(k_lds(tt), wave, krs, (uint32_t)band_key0(tt) * kst, kst);
                if (tt < R - 1) vlanes.load_band(v_lds(tt), wave, vrs, (uint32_t)band_key0(tt) * vst, vst);
            }
        }
    }
#ifndef DSALT_NO_SLOW
    if (redo) attempt(std::false_type());
#endif

    // ---- epilogue: O = acc / l, LSE = (mu + log2 l) * ln 2 --------------------------------
    const float ltot = half_sum(lsum0 + lsum1);
    const bool nonempty = ltot > 0x1p-100f;
    const float inv = nonempty ? 1.f / ltot : 0.f;
    // the query of this lane again from the lane id (opaque, so that i and its token
    // offset are not kept in registers across the tile loop)
    int lq = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) & 31;
    asm volatile("" : "+v"(lq));
    const int ie = wq0 + lq;
    const int64_t tok_e = (int64_t)seq_start + ie;
    if (ie < seq_len) {
        const int64_t ooff = tok_e * p.o_st + (int64_t)head * p.o_sh;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dd = d * 32 + g * 8 + hh * 4;
                const float o0 = oacc[d][g * 4 + 0] * inv, o1 = oacc[d][g * 4 + 1] * inv;
                const float o2 = oacc[d][g * 4 + 2] * inv, o3 = oacc[d][g * 4 + 3] * inv;
                if (p.out_f32) {
                    *reinterpret_cast<float4 *>(static_cast<float *>(p.o) + ooff + dd) = make_float4(o0, o1, o2, o3);
                } else {
                    uint2 val;
                    val.x = DT::pack2(o0, o1);
                    val.y = DT::pack2(o2, o3);
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p.o) + ooff + dd) = val;
                }
            }
        if (hh == 0)
            p.lse[tok_e * p.lse_st + (int64_t)head * p.lse_sh] =
                nonempty ? (mu + fast_log2(ltot)) * kLn2 : -INFINITY;
    }
}

// Workgroups of fwd_kernel<DT, D, MODE> resident on the whole device at once (one dispatch
// round) for `dyn` bytes of dynamic LDS, or 0 when HIP cannot say. Queried once per
// (device, landmark padding) and cached: a forward launch then makes no HIP queries
// besides hipGetDevice. Concurrent first calls store the same value.
template <typename DT, int D, int MODE>
int64_t dispatch_round(int dev, size_t dyn) {
    constexpr int kDevs = 64, kPads = DSALT_MAX_K_LMK / kFwdBN + 1;
    static std::atomic<int64_t> cache[kDevs][kPads];  // 0: not queried yet; -1: unknown
    const int pad = (int)(dyn / (kFwdBN * (2 * sizeof(int) + sizeof(float))));
    if (dev < 0 || dev >= kDevs || pad >= kPads) return 0;
    int64_t r = cache[dev][pad].load(std::memory_order_relaxed);
    if (r == 0) {
        int n_cu = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fwd_kernel<DT, D, MODE>, 64 * fwd_waves(D), dyn) ==
                hipSuccess &&
            n_cu > 0 && per_cu > 0)
            r = (int64_t)n_cu * per_cu;
        else
            r = -1;
        (void)hipGetLastError();  // a failed query must not be reported as a launch error
        cache[dev][pad].store(r, std::memory_order_relaxed);
    }
    return r > 0 ? r : 0;
}

template <typename DT, int D, int MODE>
hipError_t launch_typed(FwdParams p, size_t dyn, hipStream_t stream) {
    // the wave-priority span: the first dispatch round, for grids of at most two rounds
    int dev = -1;
    const int64_t round = hipGetDevice(&dev) == hipSuccess ? dispatch_round<DT, D, MODE>(dev, dyn) : 0;
    (void)hipGetLastError();
    p.prio_span = (round > 0 && p.grid <= 2 * round) ? (int)(p.grid < round ? p.grid : round) : 0;
    hipLaunchKernelGGL((fwd_kernel<DT, D, MODE>), dim3(p.grid), dim3(64 * fwd_waves(D)), dyn, stream, p);
    return hipGetLastError();
}

template <typename DT>
hipError_t launch_dt(const FwdParams &p, int head_dim, int mode, size_t dyn, hipStream_t stream) {
    // SOFT edges of at most kEdgeTab keys per query start the scores from the edge rows
    const bool wide = mode == DSALT_MODE_SOFT && !(p.win_edge <= (float)kEdgeTab);
    if (head_dim == 64) {
        if (mode == DSALT_MODE_HARD) return launch_typed<DT, 64, kHard>(p, dyn, stream);
        return wide ? launch_typed<DT, 64, kSoftWide>(p, dyn, stream) : launch_typed<DT, 64, kSoft>(p, dyn, stream);
    }
    if (mode == DSALT_MODE_HARD) return launch_typed<DT, 128, kHard>(p, dyn, stream);
    return wide ? launch_typed<DT, 128, kSoftWide>(p, dyn, stream) : launch_typed<DT, 128, kSoft>(p, dyn, stream);
}

}  // namespace

hipError_t launch_fwd(const dsalt_fwd_args &a, hipStream_t stream) {
    if (a.mode == DSALT_MODE_DENSE) return launch_dense_fwd(a, stream);
    if (a.total_len == 0) return hipSuccess;
    FwdParams p;
    p.q = static_cast<const uint16_t *>(a.q);
    p.k = static_cast<const uint16_t *>(a.k);
    p.v = static_cast<const uint16_t *>(a.v);
    p.o = a.out;
    p.out_f32 = a.out_dtype == DSALT_DTYPE_F32;
    p.lse = a.lse;
    p.w = a.w;
    p.lmk_pos = a.lmk_pos;
    p.lmk_bias = a.lmk_bias;
    p.cu = a.cu_seqlens;
    p.q_st = a.q_stride_t; p.q_sh = a.q_stride_h;
    p.k_st = a.k_stride_t; p.k_sh = a.k_stride_h;
    p.v_st = a.v_stride_t; p.v_sh = a.v_stride_h;
    p.o_st = a.out_stride_t; p.o_sh = a.out_stride_h;
    p.lse_st = a.lse_stride_t; p.lse_sh = a.lse_stride_h;
    p.w_st = a.w_stride;
    p.lp_sh = a.lmk_pos_stride_h; p.lp_ss = a.lmk_pos_stride_s; p.lp_sk = a.lmk_pos_stride_k;
    p.lb_sh = a.lmk_bias_stride_h; p.lb_ss = a.lmk_bias_stride_s; p.lb_sk = a.lmk_bias_stride_k;
    p.total_len = a.total_len;
    p.num_seqs = a.num_seqs;
    p.n_heads = a.n_heads;
    p.kv_rep = a.n_kv_heads > 0 ? a.n_heads / a.n_kv_heads : 1;
    p.rope_cos = a.rope_cos;
    p.rope_sin = a.rope_sin;
    p.rope_st = a.rope_stride;
    p.rope_rows = a.rope_rows;
    p.rope_half = a.rope_half;
    p.k_lmk = a.k_lmk;
    p.k_pad = (a.k_lmk + kFwdBN - 1) / kFwdBN * kFwdBN;
    p.n_qblk = block_upper_bound(a.total_len, a.num_seqs, fwd_bm(a.head_dim));
    const int64_t blocks = (int64_t)p.n_qblk * a.n_heads;
    p.grid = (int)((blocks + 7) / 8 * 8);
    p.prio_span = 0;  // set per kernel in launch_typed
    p.q_sign = a.scale < 0.f ? 0x80008000u : 0u;
    p.c = fabsf(a.scale) * kLog2e;
    p.inv_c = 1.f / p.c;
    p.inv_tau = 1.f / a.tau_win;
    p.win_edge = a.win_edge;
    const size_t dyn = (size_t)p.k_pad * (2 * sizeof(int) + sizeof(float));
    if (a.dtype == DSALT_DTYPE_BF16) return launch_dt<BF16>(p, a.head_dim, a.mode, dyn, stream);
    return launch_dt<F16>(p, a.head_dim, a.mode, dyn, stream);
}

}  // namespace dsalt
