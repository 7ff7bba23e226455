// Landmark top-k selection and window quantisation for gfx950.
//
// Reference semantics: _compute_landmark_indices (dsalt/kernels/selectors.py:75-134):
// covered tokens (offset < trunc(w)) get score -inf, each (head, sequence) takes
// torch.topk(min(k, L), sorted=False) and non-finite picks become -1. The window
// quantisation is DSALTAttention._window_sizes(floor=True) / the floor+clamp of
// _train_selectors (dsalt/modules/dsalt_attention.py:277-284, :471).
//
// Design: one 256-thread workgroup per (head, sequence).
//  * Each score becomes a 32-bit key whose unsigned order is the score order
//    (NaN > +inf > finite > ..., -0 folded onto +0); covered tokens and -inf get key 0,
//    which marks "not a candidate". Keys are cached in LDS for L <= 16384.
//  * If more than k_eff candidates exist, an MSB-first radix select (4 passes of 8-bit
//    digits; LDS histogram, one wave scans the 256 bins) finds the exact k_eff-th key
//    `thr` and how many keys equal to it are still needed.
//  * A final ordered pass emits the selected positions in ascending order with two
//    workgroup prefix scans per 256-token chunk: keys > thr, plus the first `need_eq`
//    keys == thr by position (ties: lower position wins). NaN/+inf picks occupy their
//    slot but are not emitted; every slot after the last emitted one is -1.
// Fully deterministic; integer-exact with respect to the fp32 scores.
#include "common.h"
#include "launch.h"

namespace dsalt {
namespace {

constexpr int kSelThreads = 256;
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

__device__ __forceinline__ uint32_t order_key(float s) {
    if (s != s) return 0xFFFFFFFFu;       // NaN ranks above everything (torch.topk)
    if (s == -INFINITY) return 0u;        // never a finite pick: treated as not selectable
    uint32_t u = __float_as_uint(s);
    if (u == 0x80000000u) u = 0u;         // -0 == +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum over the 256 threads of the workgroup; `total` gets the sum.
__device__ __forceinline__ int block_excl_scan(int x, int lane, int wave, int *s_tot, int &total) {
    const int incl = wave_incl_scan(x, lane);
    if (lane == 63) s_tot[wave] = incl;
    __syncthreads();
    const int w0 = s_tot[0], w1 = s_tot[1], w2 = s_tot[2], w3 = s_tot[3];
    const int off = (wave > 0 ? w0 : 0) + (wave > 1 ? w1 : 0) + (wave > 2 ? w2 : 0);
    total = w0 + w1 + w2 + w3;
    __syncthreads();
    return off + incl - x;
}

__global__ void __launch_bounds__(kSelThreads) select_kernel(const SelParams p) {
    __shared__ uint32_t s_keys[kSelCache];
    __shared__ int s_hist[256];
    __shared__ int s_tot[4];
    __shared__ int s_bc[2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int head = blockIdx.x / p.num_seqs;
    const int seq = blockIdx.x - head * p.num_seqs;
    const int start = p.cu[seq];
    const int L = p.cu[seq + 1] - start;
    int64_t *out = p.out + ((int64_t)head * p.num_seqs + seq) * p.k;
    const int k_eff = min(p.k, max(L, 0));
    const bool cached = L <= kSelCache;

    auto make_key = [&](int j) -> uint32_t {
        const int64_t tok = (int64_t)start + j;
        const float wj = p.w[tok * p.w_st];
        // covered <=> j < trunc(w_j) <=> j + 1 <= w_j   (j >= 0 integer)
        if ((float)(j + 1) <= wj) return 0u;
        return order_key(p.scores[tok * p.sc_st + (int64_t)head * p.sc_sh]);
    };
    auto key_at = [&](int j) -> uint32_t { return cached ? s_keys[j] : make_key(j); };

    // pass 0: keys and candidate count
    int cnt = 0;
    for (int j = tid; j < L; j += kSelThreads) {
        const uint32_t key = make_key(j);
        if (cached) s_keys[j] = key;
        cnt += key != 0u;
    }
    int ncand;
    (void)block_excl_scan(cnt, lane, wave, s_tot, ncand);

    uint32_t thr = 0u;  // select key > thr, plus the first need_eq keys == thr
    int need_eq = 0;
    if (k_eff > 0 && ncand > k_eff) {
        uint32_t prefix = 0u, pmask = 0u;
        int remaining = k_eff;
        for (int shift = 24; shift >= 0; shift -= 8) {
            s_hist[tid] = 0;
            __syncthreads();
            for (int j = tid; j < L; j += kSelThreads) {
                const uint32_t key = key_at(j);
                if (key != 0u && (key & pmask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255u], 1);
            }
            __syncthreads();
            if (wave == 0) {
                // lane covers digits 255-4*lane .. 252-4*lane (descending)
                const int c0 = s_hist[255 - 4 * lane], c1 = s_hist[254 - 4 * lane];
                const int c2 = s_hist[253 - 4 * lane], c3 = s_hist[252 - 4 * lane];
                const int sum4 = c0 + c1 + c2 + c3;
                const int incl = wave_incl_scan(sum4, lane);
                const int excl = incl - sum4;
                if (excl < remaining && incl >= remaining) {
                    int cum = excl, d;
                    if (cum + c0 >= remaining) {
                        d = 255 - 4 * lane;
                    } else if ((cum += c0) + c1 >= remaining) {
                        d = 254 - 4 * lane;
                    } else if ((cum += c1) + c2 >= remaining) {
                        d = 253 - 4 * lane;
                    } else {
                        cum += c2;
                        d = 252 - 4 * lane;
                    }
                    s_bc[0] = d;
                    s_bc[1] = cum;  // keys in the prefix with a larger digit
                }
            }
            __syncthreads();
            prefix |= (uint32_t)s_bc[0] << shift;
            pmask |= 0xFFu << shift;
            remaining -= s_bc[1];
            __syncthreads();
        }
        thr = prefix;
        need_eq = remaining;
    }

    // ordered emission
    int run_eq = 0, run_out = 0;
    if (k_eff > 0) {
        for (int base = 0; base < L; base += kSelThreads) {
            const int j = base + tid;
            const uint32_t key = j < L ? key_at(j) : 0u;
            const int is_gt = key > thr;
            const int is_eq = (need_eq > 0) && (key == thr);
            int eq_tot, out_tot;
            const int eq_rank = run_eq + block_excl_scan(is_eq, lane, wave, s_tot, eq_tot);
            const bool sel = is_gt || (is_eq && eq_rank < need_eq);
            const int emit = sel && key < kKeyPosInf;
            const int slot = run_out + block_excl_scan(emit, lane, wave, s_tot, out_tot);
            if (emit && slot < p.k) out[slot] = j;
            run_eq += eq_tot;
            run_out += out_tot;
        }
    }
    for (int s = run_out + tid; s < p.k; s += kSelThreads) out[s] = -1;
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
