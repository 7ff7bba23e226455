// Landmark top-k selection and window quantisation for gfx950.
//
// Reference semantics: _compute_landmark_indices (dsalt/kernels/selectors.py:75-134):
// covered tokens (offset < trunc(w)) get score -inf, each (head, sequence) takes
// torch.topk(min(k, L), sorted=False) and non-finite picks become -1. The window
// quantisation is DSALTAttention._window_sizes(floor=True) / the floor+clamp of
// _train_selectors (dsalt/modules/dsalt_attention.py:277-284, :471).
//
// Design: a 1024-thread workgroup selects the top k_eff of n items (select_block):
//  * Each score becomes a 32-bit key whose unsigned order is the score order
//    (NaN > +inf > finite > ..., -0 folded onto +0); covered tokens and -inf get key 0,
//    which marks "not a candidate". Keys are cached in LDS for n <= 16384.
//  * If more than k_eff candidates exist, an MSB-first radix select over key - min_key
//    (8-bit digits starting at the top bit of the candidates' key range, so that the
//    first LDS histogram is not concentrated on a few exponent values) finds the exact
//    k_eff-th key `thr` and how many keys equal to it are still needed. Each pass is one
//    barrier: the histograms rotate over three LDS buffers (a pass counts into one and
//    clears the next pass's, which the waves finished reading two barriers earlier) and
//    every wave scans the 256 bins itself (one ds_read_b128 and a DPP scan), so no
//    second barrier broadcasts the boundary bin. A pass whose boundary bin holds exactly
//    the keys still needed ends the search: the selection is then every key at or above
//    that bin's lower bound.
//  * A final ordered pass emits the selected items in ascending order: each thread owns
//    a contiguous run of items, and one workgroup scan of (keys > thr, keys == thr) gives
//    every thread its first output slot. Keys == thr are taken in item order (ties: lower
//    item wins). Final selections skip NaN/+inf picks (they occupy their slot but are not
//    emitted; every slot after the last emitted one is -1).
// The selection is the top k_eff under the total order (key descending, position
// ascending). Short sequences (L <= kSplitMin) take one workgroup per (head, sequence)
// over the scores. Longer ones, when the caller passes a workspace, first take one
// workgroup per 2048-position chunk (select_chunk_kernel: the chunk's own top k_eff,
// non-finite picks included, written as (key, position) candidates in position order):
// the global top k_eff is contained in the union of the chunks' (an item ranked above
// another globally is ranked above it in its chunk too). select_kernel then selects
// from the candidates, concatenated in chunk order (hence in position order).
// Fully deterministic; integer-exact with respect to the fp32 scores.
//
// Scores formed in the launch (dsalt_select_hybrid): instead of reading fp32 scores, each
// workgroup takes the norms pass's per-token norms and per-block partial sums, derives
// the mean / std of x's norms and of its head group's value norms with the score kernels'
// own arithmetic (hybrid.h: one wave each, the same fixed order), and forms every score
// as standardize_kernel would - the same bits, without the stats and standardise launches.
//
// Window quantisation can ride along (w_out): the windows are then the continuous w~,
// a token is covered when its offset o satisfies o + 1 <= q(w~) with q(w) = max(1,
// floor(w)) (NaN kept, so never covered) - exactly the test on the quantised windows,
// since q is idempotent - and the workgroups of head 0 write q(w~) for the tokens they
// read, which saves the quantisation its own launch.
#include "common.h"
#include "hybrid.h"
#include "launch.h"

namespace dsalt {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelCache = 16384;               // keys cached in LDS (64 KB)
constexpr uint32_t kKeyPosInf = 0xFF800000u;   // key of +inf; finite keys are below it
constexpr int kSelChunk = 2048;                // positions per chunk of a long sequence
constexpr int kSplitMin = 4096;                // longer sequences are selected chunk-wise
constexpr int kMergeCap = 8192;                // candidate slots a final selection may gather
static_assert(2 * kMergeCap <= kSelCache, "candidate keys and positions share the key cache");

// Candidate slots per chunk: the chunk's top k, or a superset of at most k + min(k, 128)
// items when the first radix pass already bounds one (see select_block's `cap`).
__host__ __device__ inline int chunk_slots(int k) { return k + (k < 128 ? k : 128); }

// Whether a sequence of length L is selected chunk-wise (when a workspace is given): its
// chunks' candidate slots must fit the final workgroup's LDS.
__host__ __device__ inline bool split_sequence(int L, int k) {
    const int nch = (L + kSelChunk - 1) / kSelChunk;
    return L > kSplitMin && (int64_t)nch * chunk_slots(k) <= kMergeCap;
}

struct SelParams {
    const float *scores;
    int64_t sc_st, sc_sh;
    const float *w;
    int64_t w_st;
    const int32_t *cu;
    int64_t *out;
    float *w_out;  // non-null: w holds w~; q(w~) is written here and used for the covered test
    const void *w_logit;  // non-null: w~ is formed from these window-gate logits instead of read
    int64_t w_logit_st;
    int w_logit_dt;
    float n_min, span;    // w~ = n_min + sigmoid(logit) * span
    // hybrid scores (non-null xn): norms [T] / [T, n_kv], fp64 partials [nblk][1 + n_kv][2]
    const float *xn, *vn;
    const double *part;
    const float *alpha;
    int nblk, n_kv, rep, total_len;
    int num_seqs, n_heads, k;
    // chunked selection of long sequences (null ws_key: one workgroup per (head, sequence))
    uint32_t *ws_key;  // [H][n_chunk_ub][chunk_slots(k)] candidate keys, 0 in unused slots
    int32_t *ws_pos;   // [H][n_chunk_ub][chunk_slots(k)] candidate positions in the sequence
    int n_chunk_ub;
};

// Order-preserving 32-bit key of an fp32 score (unsigned order = score order).
__device__ __forceinline__ uint32_t order_key(float s) {
    if (s != s) return 0xFFFFFFFFu;       // NaN ranks above everything (torch.topk)
    if (s == -INFINITY) return 0u;        // never a finite pick: treated as not selectable
    uint32_t u = __float_as_uint(s);
    if (u == 0x80000000u) u = 0u;         // -0 == +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP (rows of 16 by row_shr,
// then row_bcast15 / row_bcast31 across rows); no LDS traffic.
__device__ __forceinline__ int wave_incl_scan_dpp(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
    return x;
}

// Workgroup-wide exclusive prefix sums of two counters (thread order = tid order). One
// barrier: s_w must not be written again by the caller afterwards.
__device__ __forceinline__ void block_excl_scan2(int a, int b, int lane, int wave, int (*s_w)[2], int &ea,
                                                 int &eb, int &ta, int &tb) {
    const int ia = wave_incl_scan_dpp(a), ib = wave_incl_scan_dpp(b);
    if (lane == 63) {
        s_w[wave][0] = ia;
        s_w[wave][1] = ib;
    }
    __syncthreads();
    int oa = 0, ob = 0;
    ta = 0;
    tb = 0;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) {
        const int xa = s_w[w][0], xb = s_w[w][1];
        if (w < wave) {
            oa += xa;
            ob += xb;
        }
        ta += xa;
        tb += xb;
    }
    ea = oa + ia - a;
    eb = ob + ib - b;
}

// max(1, floor(w)), NaN kept: DSALTAttention._window_sizes(floor=True)
__device__ __forceinline__ float quantize_window(float x) { return (x != x) ? x : fmaxf(floorf(x), 1.f); }

// The module's continuous window of token `tok` from its 16-bit gate logit, in torch's
// operation order and roundings: sigmoid(x) = 1 / (1 + exp(-x)) in fp32 (expf, IEEE
// division), rounded to the logit's dtype; times span, rounded; plus n_min, rounded
// (dsalt_attention.py:270-276 of the reference: n_min + sigmoid(win_gate(x)) * (n_max - n_min)).
template <typename R>
__device__ __forceinline__ float gate_window(float x, float n_min, float span, R rnd) {
    const float sg = rnd(1.f / (1.f + expf(-x)));
    const float t = rnd(__fmul_rn(sg, span));
    return rnd(__fadd_rn(n_min, t));
}
__device__ __forceinline__ float window_of(const float *w, int64_t w_st, const void *logit, int64_t l_st, int l_dt,
                                           float n_min, float span, int64_t tok) {
    if (!logit) return w[tok * w_st];
    if (l_dt == DSALT_DTYPE_BF16) {
        const float x = BF16::to_f32(static_cast<const uint16_t *>(logit)[tok * l_st]);
        return gate_window(x, n_min, span, [](float v) { return BF16::round(v); });
    }
    const float x = F16::to_f32(static_cast<const uint16_t *>(logit)[tok * l_st]);
    return gate_window(x, n_min, span, [](float v) { return F16::round(v); });
}

struct SelShared {
    uint32_t keys[kSelCache];
    __align__(16) int hist[3][256];  // radix pass p counts into hist[p % 3], clears hist[(p + 1) % 3]
    int w[kSelWaves][2];
    int cnt[kSelWaves];  // written once: its readers need no trailing barrier
    uint32_t mm[kSelWaves][2];
    float st[4];  // hybrid scores: mean / std of x's norms, then of the head group's value norms
};

// The standardisation of one workgroup's head (hybrid scores): waves 0 and 1 derive the
// two (mean, std) pairs, shared through LDS. Every thread of the workgroup calls it.
struct HybridStats {
    float mx, sx, mv, sv, alpha;
    int g;
};
__device__ __forceinline__ HybridStats hybrid_stats(const SelParams &p, SelShared &sh, int head) {
    HybridStats h{};
    if (!p.xn) return h;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    h.g = head / p.rep;
    if (wave < 2) {
        float m, sd;
        hybrid_stat(p.part, p.nblk, 1 + p.n_kv, wave == 0 ? 0 : 1 + h.g, (double)p.total_len, lane, m, sd);
        if (lane == 0) {
            sh.st[2 * wave] = m;
            sh.st[2 * wave + 1] = sd;
        }
    }
    __syncthreads();
    h.mx = sh.st[0];
    h.sx = sh.st[1];
    h.mv = sh.st[2];
    h.sv = sh.st[3];
    h.alpha = p.alpha[head];
    return h;
}

// The top k_eff of items 0 .. n-1 of key key_of(j, first) (0: not a candidate; `first`
// is true on the first of possibly several calls per item), emitted as emit(slot, j, key)
// in ascending item order. The key pass and the histogram passes stride
// over items (j = tid + 1024 i: coalesced loads, conflict-free LDS); for the emission
// thread t owns the contiguous items [t*C, t*C + C) (C = ceil(n / 1024)), which keeps
// the output in item order with one workgroup scan. `all` emits NaN/+inf picks too (for
// candidates); otherwise they only count towards k_eff. cap >= k_eff: a set of at most
// cap items that contains the top k_eff may be emitted instead (every candidate when there
// are at most cap, else the keys at or above a radix bin that already bounds such a set);
// cap = k_eff gives exactly the top k_eff. Returns the number of slots emitted. Every
// thread of the workgroup calls it; `sh` is the workgroup's LDS.
template <class KeyFn, class EmitFn>
__device__ __forceinline__ int select_block(SelShared &sh, int n, int k_eff, int cap, bool all, KeyFn key_of,
                                            EmitFn emit) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool cached = n <= kSelCache;
    const int C = (max(n, 0) + kSelThreads - 1) / kSelThreads;
    const int j0 = tid * C, j1 = min(j0 + C, max(n, 0));
    auto key_at = [&](int j) -> uint32_t { return cached ? sh.keys[j] : key_of(j, false); };

    // pass 0: keys, candidate count and the candidates' key range
    int cnt = 0;
    uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
    for (int j = tid; j < n; j += kSelThreads) {
        const uint32_t key = key_of(j, true);
        if (cached) sh.keys[j] = key;
        if (key != 0u) {
            ++cnt;
            kmin = min(kmin, key);
            kmax = max(kmax, key);
        }
    }
    kmin = (uint32_t)wave_min_u((int)(kmin ^ 0x80000000u)) ^ 0x80000000u;  // unsigned via sign flip
    kmax = (uint32_t)wave_max_u((int)(kmax ^ 0x80000000u)) ^ 0x80000000u;
    if (lane == 0) {
        sh.mm[wave][0] = kmin;
        sh.mm[wave][1] = kmax;
    }
    // candidate count and key range: per-wave values, one barrier (which also publishes
    // the cleared histogram of the first pass); cnt and mm are never rewritten
    cnt = wave_sum_u(cnt);
    if (lane == 0) sh.cnt[wave] = cnt;
    if (tid < 256) sh.hist[0][tid] = 0;
    __syncthreads();
    int ncand = 0;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) {
        ncand += sh.cnt[w];
        kmin = min(kmin, sh.mm[w][0]);
        kmax = max(kmax, sh.mm[w][1]);
    }

    uint32_t thr = 0u;  // select key > thr, plus the first need_eq keys == thr
    int need_eq = 0;
    if (k_eff > 0 && ncand > cap) {
        // MSB-first radix select on rel = key - kmin, 8-bit digits from the top set bit of
        // the candidates' range (the first digit is spread over the whole histogram).
        // hist[0] was cleared before the barrier above; pass p clears hist[(p + 1) % 3] for
        // the next pass: that buffer was counted in pass p - 2 and read by every wave
        // before it counted pass p - 1, i.e. before the barrier that ended pass p - 1.
        const uint32_t range = kmax - kmin;
        const int nbits = range ? 32 - __clz((int)range) : 0;
        uint32_t prefix = 0u, pmask = 0u;
        int remaining = k_eff;
        for (int pass = 0, shift = max(nbits - 8, 0);; ++pass, shift = max(shift - 8, 0)) {
            int *hist = sh.hist[pass % 3];
            if (tid < 256) sh.hist[(pass + 1) % 3][tid] = 0;
            for (int j = tid; j < n; j += kSelThreads) {
                const uint32_t key = key_at(j);
                const uint32_t rel = key - kmin;
                if (key != 0u && (rel & pmask) == prefix) atomicAdd(&hist[(rel >> shift) & 255u], 1);
            }
            __syncthreads();
            // every wave finds the boundary digit: lane l holds digits 255-4l .. 252-4l
            // (descending); exactly one lane's range reaches the remaining count
            const int4 h4 = *reinterpret_cast<const int4 *>(&hist[252 - 4 * lane]);
            const int c0 = h4.w, c1 = h4.z, c2 = h4.y, c3 = h4.x;
            const int sum4 = c0 + c1 + c2 + c3;
            const int incl = wave_incl_scan_dpp(sum4);
            int cum = incl - sum4, d, cd;
            if (cum + c0 >= remaining) {
                d = 255 - 4 * lane;
                cd = c0;
            } else if ((cum += c0) + c1 >= remaining) {
                d = 254 - 4 * lane;
                cd = c1;
            } else if ((cum += c1) + c2 >= remaining) {
                d = 253 - 4 * lane;
                cd = c2;
            } else {
                cum += c2;
                d = 252 - 4 * lane;
                cd = c3;
            }
            const int src = __builtin_ctzll(__ballot(incl - sum4 < remaining && incl >= remaining));
            d = __builtin_amdgcn_readlane(d, src);
            cum = __builtin_amdgcn_readlane(cum, src);  // keys in the prefix with a larger digit
            cd = __builtin_amdgcn_readlane(cd, src);    // keys in the prefix with digit d
            prefix |= (uint32_t)d << shift;
            pmask |= 0xFFu << shift;
            remaining -= cum;
            // the keys with rel >= prefix (the bin and everything above it) number at most
            // `cap`: they are the selection (cap = k_eff: every key of the bin is needed)
            // or a superset of it (cap > k_eff, for candidates), whatever the lower digits
            // are - the passes for them are skipped
            if (k_eff - remaining + cd <= cap) {
                thr = kmin + prefix - 1u;  // kmin >= 1: thr >= 0 and key 0 is never taken
                need_eq = 0;
                break;
            }
            if (shift == 0) {
                thr = kmin + prefix;
                need_eq = remaining;
                break;
            }
        }
    }

    // ordered emission: emitted slots before this thread = emitted keys > thr before it
    // plus the equal keys selected before it (equal keys are selected in item order)
    if (k_eff <= 0) return 0;
    const bool eq_ok = all || thr < kKeyPosInf;  // equal keys emitted (not NaN / +inf finals)
    auto is_gt = [&](uint32_t key) { return key > thr && (all || key < kKeyPosInf); };
    int n_gt = 0, n_eq = 0;
    for (int j = j0; j < j1; ++j) {
        const uint32_t key = key_at(j);
        n_gt += is_gt(key);
        n_eq += (need_eq > 0) && (key == thr);
    }
    int gt_before, eq_before, gt_tot, eq_tot;
    block_excl_scan2(n_gt, n_eq, lane, wave, sh.w, gt_before, eq_before, gt_tot, eq_tot);
    int slot = gt_before + (eq_ok ? min(eq_before, need_eq) : 0);
    int eq_rank = eq_before;
    for (int j = j0; j < j1; ++j) {
        const uint32_t key = key_at(j);
        bool take = is_gt(key);
        if ((need_eq > 0) && (key == thr)) {
            take = eq_ok && eq_rank < need_eq;
            ++eq_rank;
        }
        if (take) {
            emit(slot, j, key);
            ++slot;
        }
    }
    return gt_tot + (eq_ok ? min(eq_tot, need_eq) : 0);
}

// Key of token `tok` at offset `pos` of its sequence for `head`: 0 when covered
// (pos < trunc(w), i.e. pos + 1 <= w for the integer pos + 1; with w_out the test is on
// q(w~) and, on the first visit by a head-0 workgroup, q(w~) is stored).
__device__ __forceinline__ uint32_t cand_key(const SelParams &p, const HybridStats &hs, int head, int pos,
                                             int64_t tok, bool first) {
    float wv = window_of(p.w, p.w_st, p.w_logit, p.w_logit_st, p.w_logit_dt, p.n_min, p.span, tok);
    float sc;
    if (p.xn)
        sc = hybrid_mix(hybrid_z(p.xn[tok], hs.mx, hs.sx), hybrid_z(p.vn[tok * p.n_kv + hs.g], hs.mv, hs.sv),
                        hs.alpha);
    else
        sc = p.scores[tok * p.sc_st + (int64_t)head * p.sc_sh];
    const uint32_t key = order_key(sc);
    if (p.w_out) {
        wv = quantize_window(wv);
        if (first && head == 0) p.w_out[tok] = wv;
    }
    return ((float)(pos + 1) <= wv) ? 0u : key;
}

// Chunks of long sequences (L > kSplitMin): one workgroup per (head, chunk id of
// find_block over kSelChunk-position chunks); a superset of the chunk's top k (at most
// chunk_slots(k) items, NaN/+inf picks included) to the workspace as (key, position)
// candidates in position order, the remaining slots with key 0.
__global__ void __launch_bounds__(kSelThreads) select_chunk_kernel(const SelParams p) {
    __shared__ SelShared sh;
    const int lane = threadIdx.x & 63;
    const int head = blockIdx.x / p.n_chunk_ub;
    const int cid = blockIdx.x - head * p.n_chunk_ub;
    int seq, chunk, start, L;
    if (!find_block(p.cu, p.num_seqs, p.total_len, cid, kSelChunk, lane, seq, chunk, start, L)) return;
    if (!split_sequence(L, p.k)) return;  // selected from the scores by select_kernel
    const int c0 = chunk * kSelChunk;
    const int n = min(kSelChunk, L - c0);
    const int k_eff = min(min(p.k, L), n);
    const int cs = chunk_slots(p.k);
    uint32_t *ck = p.ws_key + ((int64_t)head * p.n_chunk_ub + cid) * cs;
    int32_t *cp = p.ws_pos + ((int64_t)head * p.n_chunk_ub + cid) * cs;
    const HybridStats hs = hybrid_stats(p, sh, head);
    auto key_of = [&](int j, bool first) -> uint32_t {
        const int pos = c0 + j;
        const int64_t tok = (int64_t)start + pos;
        return cand_key(p, hs, head, pos, tok, first);
    };
    auto emit = [&](int slot, int j, uint32_t key) {
        if (slot < cs) {
            ck[slot] = key;
            cp[slot] = c0 + j;
        }
    };
    const int total = min(select_block(sh, n, k_eff, max(k_eff, cs), true, key_of, emit), cs);
    for (int sl = total + (int)threadIdx.x; sl < cs; sl += kSelThreads) ck[sl] = 0u;
}

// One workgroup per (head, sequence): the final selection, from the scores or (long
// sequences with a workspace) from the chunks' candidates.
__global__ void __launch_bounds__(kSelThreads) select_kernel(const SelParams p) {
    __shared__ SelShared sh;
    const int tid = threadIdx.x;
    const int head = blockIdx.x / p.num_seqs;
    const int seq = blockIdx.x - head * p.num_seqs;
    int start, end;
    seq_bounds(p.cu, seq, p.total_len, start, end);
    const int L = end - start;
    int64_t *out = p.out + ((int64_t)head * p.num_seqs + seq) * p.k;
    const int k_eff = min(p.k, L);
    int total;
    if (p.ws_key && split_sequence(L, p.k)) {
        // the chunks' candidate slots, concatenated in chunk order (the candidates in
        // position order, unused slots key 0): keys cached by select_block in
        // sh.keys[0, n), positions in s_pos = sh.keys[kMergeCap, 2 kMergeCap)
        const int cs = chunk_slots(p.k);
        const int n = (L + kSelChunk - 1) / kSelChunk * cs;
        const uint32_t *gk = p.ws_key + ((int64_t)head * p.n_chunk_ub + start / kSelChunk + seq) * cs;
        const int32_t *gp = p.ws_pos + ((int64_t)head * p.n_chunk_ub + start / kSelChunk + seq) * cs;
        int32_t *s_pos = reinterpret_cast<int32_t *>(sh.keys + kMergeCap);
        auto key_of = [&](int j, bool) -> uint32_t {  // pass 0 only (n <= kMergeCap: cached)
            s_pos[j] = gp[j];
            return gk[j];
        };
        auto emit = [&](int slot, int j, uint32_t) {
            if (slot < p.k) out[slot] = s_pos[j];
        };
        total = select_block(sh, n, k_eff, k_eff, false, key_of, emit);
    } else {
        const HybridStats hs = hybrid_stats(p, sh, head);
        auto key_of = [&](int j, bool first) -> uint32_t {
            return cand_key(p, hs, head, j, (int64_t)start + j, first);
        };
        auto emit = [&](int slot, int j, uint32_t) {
            if (slot < p.k) out[slot] = j;
        };
        total = select_block(sh, L, k_eff, k_eff, false, key_of, emit);
    }
    for (int s2 = total + tid; s2 < p.k; s2 += kSelThreads) out[s2] = -1;
}

__global__ void quantize_kernel(const float *__restrict__ w, int64_t w_st, int64_t n, float *__restrict__ wq,
                                int32_t *__restrict__ wi, const void *logit, int64_t l_st, int l_dt, float n_min,
                                float span) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const float x = window_of(w, w_st, logit, l_st, l_dt, n_min, span, idx);
    const float f = floorf(x);
    if (wq) wq[idx] = quantize_window(x);
    if (wi) wi[idx] = (x >= 1.f) ? (int32_t)fminf(f, 1073741824.f) : 1;
}

}  // namespace

// Workspace of the chunk-wise selection: per (head, chunk id) chunk_slots(k) candidate
// keys and as many positions.
int64_t select_workspace_bytes(int total_len, int num_seqs, int n_heads, int k) {
    if (total_len <= kSplitMin || k == 0) return 0;
    auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
    const int64_t n = (int64_t)n_heads * block_upper_bound(total_len, num_seqs, kSelChunk);
    return 2 * al(n * chunk_slots(k) * 4);
}

hipError_t launch_select(const dsalt_select_args &a, hipStream_t stream, const HybridSrc *hy) {
    if (a.k_lmk == 0) {  // nothing to select; the windows are still quantised
        if (!a.w_out || a.total_len == 0) return hipSuccess;
        const int64_t blocks = ((int64_t)a.total_len + 255) / 256;
        hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a.w, a.w_stride,
                           (int64_t)a.total_len, a.w_out, (int32_t *)nullptr, a.w_logit, a.w_logit_stride,
                           (int)a.w_logit_dtype, a.n_min, a.n_max - a.n_min);
        return hipGetLastError();
    }
    SelParams p;
    p.scores = a.scores;
    p.sc_st = a.scores_stride_t;
    p.sc_sh = a.scores_stride_h;
    p.w = a.w;
    p.w_st = a.w_stride;
    p.cu = a.cu_seqlens;
    p.out = a.lmk_pos;
    p.w_out = a.w_out;
    p.w_logit = a.w_logit;
    p.w_logit_st = a.w_logit_stride;
    p.w_logit_dt = a.w_logit_dtype;
    p.n_min = a.n_min;
    p.span = a.n_max - a.n_min;
    p.xn = hy ? hy->xn : nullptr;
    p.vn = hy ? hy->vn : nullptr;
    p.part = hy ? hy->part : nullptr;
    p.alpha = hy ? hy->alpha : nullptr;
    p.nblk = hy ? hy->nblk : 0;
    p.n_kv = hy ? hy->n_kv : 1;
    p.rep = hy ? hy->n_heads / hy->n_kv : 1;
    p.total_len = a.total_len;
    p.num_seqs = a.num_seqs;
    p.n_heads = a.n_heads;
    p.k = a.k_lmk;
    p.ws_key = nullptr;
    p.ws_pos = nullptr;
    p.n_chunk_ub = block_upper_bound(a.total_len, a.num_seqs, kSelChunk);
    const int64_t need = select_workspace_bytes(a.total_len, a.num_seqs, a.n_heads, a.k_lmk);
    if (a.workspace && need > 0 && (a.max_seqlen <= 0 || a.max_seqlen > kSplitMin)) {
        const int64_t n = (int64_t)a.n_heads * p.n_chunk_ub;
        char *ws = static_cast<char *>(a.workspace);
        p.ws_key = reinterpret_cast<uint32_t *>(ws);
        p.ws_pos = reinterpret_cast<int32_t *>(ws + need / 2);
        hipLaunchKernelGGL(select_chunk_kernel, dim3((unsigned)n), dim3(kSelThreads), 0, stream, p);
    }
    hipLaunchKernelGGL(select_kernel, dim3(a.num_seqs * a.n_heads), dim3(kSelThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_quantize(const float *w_cont, int64_t n, float *w_out, int32_t *w_int,
                           hipStream_t stream) {
    if (n == 0 || (!w_out && !w_int)) return hipSuccess;
    const int threads = 256;
    const int64_t blocks = (n + threads - 1) / threads;
    hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)blocks), dim3(threads), 0, stream, w_cont, (int64_t)1, n,
                       w_out, w_int, (const void *)nullptr, (int64_t)0, 0, 0.f, 0.f);
    return hipGetLastError();
}

}  // namespace dsalt
