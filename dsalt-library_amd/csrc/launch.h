// Internal interface between the C-ABI layer (api.hip) and the kernel translation
// units. Arguments arrive here already validated.
#pragma once

#include <hip/hip_runtime.h>
#include "../../include/dsalt_hip.h"

namespace dsalt {

// Forward: one workgroup of fwd_waves(D) waves owns fwd_bm(D) = 32 * fwd_waves(D)
// consecutive queries of one (sequence, head); each wave owns 32 of them. Key tiles
// hold fwd_bn(D) = 32 keys; K and V tiles each sit on an fwd_ring(D)-deep LDS ring
// (2 + 2 tiles = 16 KB at D = 64, 32 KB at D = 128). The HARD kernel runs
// fwd_waves_per_simd(D, false) waves per SIMD: at D = 64 that is 4 (128 VGPRs, 8
// workgroups per CU), and so does the SOFT kernel whose scores start from per-query edge
// rows; the wide-edge SOFT kernel (win_edge > 4, edge bias computed per element) keeps 3
// (its edge factors need more registers). At D = 128 all run 2 (about 210-230 VGPRs, 4 workgroups per CU, which the 35 KB of
// LDS per workgroup also allows; 4-wave workgroups with a 3-deep ring ran the same
// residency with twice the queries per key union: c4 167.7 against 158.4 us). The
// kernel also supports 64-key tiles, 4-wave workgroups and 3-deep rings. Landmark slots
// are padded to a multiple of kFwdBN = 64, which every tile size divides. kFwdBM is the
// smallest block size (size checks).
constexpr int kFwdBN = 64;
constexpr int fwd_bn(int) { return 32; }
constexpr int fwd_waves(int) { return 2; }
constexpr int fwd_bm(int head_dim) { return 32 * fwd_waves(head_dim); }
constexpr int kFwdBM = 64;
constexpr int fwd_waves_per_simd(int head_dim, bool wide_edge) { return head_dim == 64 ? (wide_edge ? 3 : 4) : 2; }
constexpr int fwd_ring(int) { return 2; }  // K / V ring depth

hipError_t launch_fwd(const dsalt_fwd_args &a, hipStream_t stream);
hipError_t launch_bwd(const dsalt_bwd_args &a, hipStream_t stream);
// Selection scores formed on the fly from the norms pass's outputs (scores workspace):
// per-token norms, per-block fp64 partial sums, and the per-head balance alpha.
struct HybridSrc {
    const float *xn, *vn;
    const double *part;
    const float *alpha;
    int nblk, n_kv, n_heads, total_len;
};
hipError_t launch_select(const dsalt_select_args &a, hipStream_t stream, const HybridSrc *hy = nullptr);
hipError_t launch_norms_for_select(const dsalt_scores_args &a, HybridSrc &src, hipStream_t stream);
int64_t select_workspace_bytes(int total_len, int num_seqs, int n_heads, int k);
hipError_t launch_rope(const dsalt_rope_args &a, hipStream_t stream);
hipError_t launch_scores(const dsalt_scores_args &a, hipStream_t stream);
int64_t scores_workspace_bytes(int total_len, int n_kv);
int scores_max_kv();
hipError_t launch_quantize(const float *w_cont, int64_t n, float *w_out, int32_t *w_int,
                           hipStream_t stream);
hipError_t launch_swiglu(const void *gate, const void *up, void *out, int64_t n, int dtype, hipStream_t stream);
hipError_t launch_add_rms_norm(const void *x, const void *h, void *x_out, void *y, const void *weight, int64_t rows,
                               int d, float eps, int dtype, hipStream_t stream);
int rms_norm_max_dim();

// Number of query blocks of `bm` tokens over a packed batch, as an upper bound that is
// computable without reading cu_seqlens: sum_s ceil(L_s/bm) <= ceil(T/bm) + S.
inline int block_upper_bound(int total_len, int num_seqs, int bm) {
    return (total_len + bm - 1) / bm + num_seqs;
}

int64_t bwd_workspace_bytes(int total_len, int num_seqs, int n_heads, int head_dim, int k_lmk);

// Dense batched mode (dense.hip): one sequence, every causal key, the [H, T] landmark
// bias table.
hipError_t launch_dense_fwd(const dsalt_fwd_args &a, hipStream_t stream);
hipError_t launch_dense_bwd(const dsalt_bwd_args &a, hipStream_t stream);
int64_t dense_bwd_workspace_bytes(int total_len, int n_heads);

}  // namespace dsalt
