// Landmark top-k selection and window quantisation for gfx950.
//
// Reference semantics: _compute_landmark_indices (dsalt/kernels/selectors.py:75-134):
// covered tokens (offset < trunc(w)) get score -inf, each (head, sequence) takes
// torch.topk(min(k, L), sorted=False) and non-finite picks become -1. The window
// quantisation is DSALTAttention._window_sizes(floor=True) / the floor+clamp of
// _train_selectors (dsalt/modules/dsalt_attention.py:277-284, :471).
//
// Design: one 1024-thread workgroup per (head, sequence).
//  * Each score becomes a 32-bit key whose unsigned order is the score order
//    (NaN > +inf > finite > ..., -0 folded onto +0); covered tokens and -inf get key 0,
//    which marks "not a candidate". Keys are cached in LDS for L <= 16384.
//  * If more than k_eff candidates exist, an MSB-first radix select over key - min_key
//    (8-bit digits starting at the top bit of the candidates' key range, so that the
//    first LDS histogram is not concentrated on a few exponent values; one wave scans
//    the 256 bins) finds the exact k_eff-th key `thr` and how many keys equal to it are
//    still needed. A pass whose boundary bin holds exactly the keys still needed ends the
//    search: the selection is then every key at or above that bin's lower bound.
//  * A final ordered pass emits the selected positions in ascending order: each thread
//    owns a contiguous run of positions, and one workgroup scan of (finite keys > thr,
//    keys == thr) gives every thread its first output slot. Keys == thr are taken by
//    position (ties: lower position wins). NaN/+inf picks occupy their slot but are not
//    emitted; every slot after the last emitted one is -1.
// Fully deterministic; integer-exact with respect to the fp32 scores.
#include "common.h"
#include "launch.h"

namespace dsalt {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelCache = 16384;               // keys cached in LDS (64 KB)
constexpr uint32_t kKeyPosInf = 0xFF800000u;   // key of +inf; finite keys are below it

struct SelParams {
    const float *scores;
    int64_t sc_st, sc_sh;
    const float *w;
    int64_t w_st;
    const int32_t *cu;
    int64_t *out;
    int num_seqs, n_heads, k;
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

// One workgroup of 1024 threads per (head, sequence). The key pass and the histogram
// passes stride over positions (j = tid + 1024 i: coalesced loads, conflict-free LDS);
// for the emission thread t owns the contiguous positions [t*C, t*C + C)
// (C = ceil(L / 1024)), which keeps the output in position order with one workgroup scan.
__global__ void __launch_bounds__(kSelThreads) select_kernel(const SelParams p) {
    __shared__ uint32_t s_keys[kSelCache];
    __shared__ int s_hist[2][256];  // double-buffered: pass n clears the buffer of pass n + 1
    __shared__ int s_w[kSelWaves][2];
    __shared__ int s_cnt[kSelWaves];  // written once: its readers need no trailing barrier
    __shared__ uint32_t s_mm[kSelWaves][2];
    __shared__ int s_bc[3];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int head = blockIdx.x / p.num_seqs;
    const int seq = blockIdx.x - head * p.num_seqs;
    const int start = p.cu[seq];
    const int L = p.cu[seq + 1] - start;
    int64_t *out = p.out + ((int64_t)head * p.num_seqs + seq) * p.k;
    const int k_eff = min(p.k, max(L, 0));
    const bool cached = L <= kSelCache;
    const int C = (max(L, 0) + kSelThreads - 1) / kSelThreads;
    const int j0 = tid * C, j1 = min(j0 + C, max(L, 0));

    auto make_key = [&](int j) -> uint32_t {
        const int64_t tok = (int64_t)start + j;
        const float wj = p.w[tok * p.w_st];
        // covered <=> j < trunc(w_j) <=> j + 1 <= w_j   (j >= 0 integer)
        if ((float)(j + 1) <= wj) return 0u;
        return order_key(p.scores[tok * p.sc_st + (int64_t)head * p.sc_sh]);
    };
    auto key_at = [&](int j) -> uint32_t { return cached ? s_keys[j] : make_key(j); };

    // pass 0: keys, candidate count and the candidates' key range
    int cnt = 0;
    uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
    for (int j = tid; j < L; j += kSelThreads) {
        const uint32_t key = make_key(j);
        if (cached) s_keys[j] = key;
        if (key != 0u) {
            ++cnt;
            kmin = min(kmin, key);
            kmax = max(kmax, key);
        }
    }
    kmin = (uint32_t)wave_min_u((int)(kmin ^ 0x80000000u)) ^ 0x80000000u;  // unsigned via sign flip
    kmax = (uint32_t)wave_max_u((int)(kmax ^ 0x80000000u)) ^ 0x80000000u;
    if (lane == 0) {
        s_mm[wave][0] = kmin;
        s_mm[wave][1] = kmax;
    }
    // candidate count and key range: per-wave values, one barrier (which also publishes
    // the cleared histogram of the first pass); s_cnt and s_mm are never rewritten
    cnt = wave_sum_u(cnt);
    if (lane == 0) s_cnt[wave] = cnt;
    if (tid < 256) s_hist[0][tid] = 0;
    __syncthreads();
    int ncand = 0;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) {
        ncand += s_cnt[w];
        kmin = min(kmin, s_mm[w][0]);
        kmax = max(kmax, s_mm[w][1]);
    }

    uint32_t thr = 0u;  // select key > thr, plus the first need_eq keys == thr
    int need_eq = 0;
    if (k_eff > 0 && ncand > k_eff) {
        // MSB-first radix select on rel = key - kmin, 8-bit digits from the top set bit of
        // the candidates' range (the first digit is spread over the whole histogram)
        const uint32_t range = kmax - kmin;
        const int nbits = range ? 32 - __clz((int)range) : 0;
        uint32_t prefix = 0u, pmask = 0u;
        int remaining = k_eff, buf = 0;
        for (int shift = max(nbits - 8, 0);; shift = max(shift - 8, 0)) {
            // s_hist[buf] is zero here (cleared before the previous barrier)
            int *hist = s_hist[buf];
            for (int j = tid; j < L; j += kSelThreads) {
                const uint32_t key = key_at(j);
                const uint32_t rel = key - kmin;
                if (key != 0u && (rel & pmask) == prefix) atomicAdd(&hist[(rel >> shift) & 255u], 1);
            }
            __syncthreads();
            if (wave == 1) s_hist[buf ^ 1][lane * 4 + 0] = s_hist[buf ^ 1][lane * 4 + 1] =
                s_hist[buf ^ 1][lane * 4 + 2] = s_hist[buf ^ 1][lane * 4 + 3] = 0;  // next pass
            if (wave == 0) {
                // lane covers digits 255-4*lane .. 252-4*lane (descending)
                const int c0 = hist[255 - 4 * lane], c1 = hist[254 - 4 * lane];
                const int c2 = hist[253 - 4 * lane], c3 = hist[252 - 4 * lane];
                const int sum4 = c0 + c1 + c2 + c3;
                const int incl = wave_incl_scan_dpp(sum4);
                const int excl = incl - sum4;
                if (excl < remaining && incl >= remaining) {
                    int cum = excl, d, cd;
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
                    s_bc[0] = d;
                    s_bc[1] = cum;  // keys in the prefix with a larger digit
                    s_bc[2] = cd;   // keys in the prefix with digit d
                }
            }
            __syncthreads();
            prefix |= (uint32_t)s_bc[0] << shift;
            pmask |= 0xFFu << shift;
            remaining -= s_bc[1];
            // every key of the chosen bin is needed: the selection is exactly the keys
            // with rel >= prefix (the bin and everything above it), whatever the lower
            // digits are - the passes for them are skipped
            const bool whole_bin = s_bc[2] == remaining;
            buf ^= 1;
            // no barrier here: s_bc is rewritten only after the next pass's histogram
            // barrier, which every thread reaches after this read
            if (whole_bin) {
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

    // ordered emission: emitted slots before this thread = finite keys > thr before it plus
    // the equal keys selected before it (equal keys are selected in position order)
    if (k_eff > 0) {
        int n_gt = 0, n_eq = 0;
        for (int j = j0; j < j1; ++j) {
            const uint32_t key = key_at(j);
            n_gt += (key > thr) && (key < kKeyPosInf);
            n_eq += (need_eq > 0) && (key == thr);
        }
        int gt_before, eq_before, gt_tot, eq_tot;
        block_excl_scan2(n_gt, n_eq, lane, wave, s_w, gt_before, eq_before, gt_tot, eq_tot);
        const bool thr_finite = thr < kKeyPosInf;
        int slot = gt_before + (thr_finite ? min(eq_before, need_eq) : 0);
        int eq_rank = eq_before;
        for (int j = j0; j < j1; ++j) {
            const uint32_t key = key_at(j);
            bool emit = (key > thr) && (key < kKeyPosInf);
            if ((need_eq > 0) && (key == thr)) {
                emit = thr_finite && eq_rank < need_eq;
                ++eq_rank;
            }
            if (emit) {
                if (slot < p.k) out[slot] = j;
                ++slot;
            }
        }
        const int total = gt_tot + (thr_finite ? min(eq_tot, need_eq) : 0);
        for (int s2 = total + tid; s2 < p.k; s2 += kSelThreads) out[s2] = -1;
    } else {
        for (int s2 = tid; s2 < p.k; s2 += kSelThreads) out[s2] = -1;
    }
}

__global__ void quantize_kernel(const float *__restrict__ w, int64_t n, float *__restrict__ wq,
                                int32_t *__restrict__ wi) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const float x = w[idx];
    const float f = floorf(x);
    if (wq) wq[idx] = (x != x) ? x : fmaxf(f, 1.f);
    if (wi) wi[idx] = (x >= 1.f) ? (int32_t)fminf(f, 1073741824.f) : 1;
}

}  // namespace

hipError_t launch_select(const dsalt_select_args &a, hipStream_t stream) {
    if (a.k_lmk == 0) return hipSuccess;
    SelParams p;
    p.scores = a.scores;
    p.sc_st = a.scores_stride_t;
    p.sc_sh = a.scores_stride_h;
    p.w = a.w;
    p.w_st = a.w_stride;
    p.cu = a.cu_seqlens;
    p.out = a.lmk_pos;
    p.num_seqs = a.num_seqs;
    p.n_heads = a.n_heads;
    p.k = a.k_lmk;
    hipLaunchKernelGGL(select_kernel, dim3(a.num_seqs * a.n_heads), dim3(kSelThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_quantize(const float *w_cont, int64_t n, float *w_out, int32_t *w_int,
                           hipStream_t stream) {
    if (n == 0 || (!w_out && !w_int)) return hipSuccess;
    const int threads = 256;
    const int64_t blocks = (n + threads - 1) / threads;
    hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)blocks), dim3(threads), 0, stream, w_cont, n, w_out,
                       w_int);
    return hipGetLastError();
}

}  // namespace dsalt
