// Rotary position embedding of q and k in one pass (the module's RoPE, §8 row f3).
//
// Reference: apply_rotary_emb (dsalt/kernels/window_utils.py:73-88), called by
// DSALTAttention._packed (dsalt/modules/dsalt_attention.py:570-585) with
// cos/sin = rope_cos/rope_sin[pos] cast to q's dtype, pos the token's offset inside
// its sequence. Half-split convention, per head, for j < D/2:
//   out[j]       = q[j] c[j]             - q[j + D/2] s[j]
//   out[j + D/2] = q[j + D/2] c[j + D/2] + q[j] s[j + D/2]
// The reference compiles it (torch.compile): products and sum in fp32, one rounding of
// the result to the tensor dtype. Here the same, with FMA contraction off. The
// transposed mode is the backward: g -> dq with
//   dq[j]       = g[j] c[j]             + g[j + D/2] s[j + D/2]
//   dq[j + D/2] = g[j + D/2] c[j + D/2] - g[j] s[j]
// Positions come from cu_seqlens in-kernel (no per-token cos/sin copies); with
// per-token tables (the module's rope_cs argument) row t is token t.
#include "common.h"
#include "launch.h"
#include "rotary.h"

namespace dsalt {
namespace {

struct RopeParams {
    const void *in[2];
    void *out[2];
    int64_t in_st[2], in_sh[2], out_st[2], out_sh[2];
    int heads[2];
    const float *cos, *sin;
    int64_t cs_st;
    const int32_t *cu;  // NULL: row t of the tables is token t
    int T, D, S, transpose, rows;
};

// One thread per (token, head, VW consecutive j < D/2) of q then k: both elements of
// each rotated pair. Reads and writes of a pair happen in the same thread, so out may
// alias in. VW = 8 moves 16-byte (16-bit types) or 32-byte (fp32) vectors per half.
template <typename DT, int VW>
__global__ void __launch_bounds__(256) rope_kernel(const RopeParams p) {
    const int half = p.D >> 1;
    const int nj = half / VW;  // vectors per half-row
    const int64_t per_tok = (int64_t)(p.heads[0] + p.heads[1]) * nj;
    const int64_t n = (int64_t)p.T * per_tok;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(idx / per_tok);
        int r = (int)(idx - (int64_t)t * per_tok);
        const int which = r >= p.heads[0] * nj;  // 0: q, 1: k
        if (which) r -= p.heads[0] * nj;
        const int h = r / nj, j0 = (r - h * nj) * VW;
        const int pos = p.cu ? seq_offset(p.cu, p.S, p.T, t) : t;
        const bool in_table = pos >= 0 && pos < p.rows;  // no table row (past it, or a token before cu[0]): NaN outputs
        const float *cr = p.cos + (int64_t)(in_table ? pos : 0) * p.cs_st;
        const float *sr = p.sin + (int64_t)(in_table ? pos : 0) * p.cs_st;
        const int64_t ib = (int64_t)t * p.in_st[which] + (int64_t)h * p.in_sh[which];
        const int64_t ob = (int64_t)t * p.out_st[which] + (int64_t)h * p.out_sh[which];
        rotate_vec<DT, VW>(p.in[which], ib, p.out[which], ob, cr, sr, half, j0, in_table, p.transpose != 0);
    }
}

}  // namespace

hipError_t launch_rope(const dsalt_rope_args &a, hipStream_t stream) {
    if (a.total_len == 0) return hipSuccess;
    RopeParams p;
    p.in[0] = a.q;
    p.in[1] = a.k;
    p.out[0] = a.q_out;
    p.out[1] = a.k_out;
    p.in_st[0] = a.q_stride_t;
    p.in_sh[0] = a.q_stride_h;
    p.in_st[1] = a.k_stride_t;
    p.in_sh[1] = a.k_stride_h;
    p.out_st[0] = a.q_out_stride_t;
    p.out_sh[0] = a.q_out_stride_h;
    p.out_st[1] = a.k_out_stride_t;
    p.out_sh[1] = a.k_out_stride_h;
    p.heads[0] = a.n_q_heads;
    p.heads[1] = a.n_k_heads;
    p.cos = a.cos;
    p.sin = a.sin;
    p.cs_st = a.cos_sin_stride;
    p.cu = a.cu_seqlens;
    p.T = a.total_len;
    p.D = a.head_dim;
    p.S = a.num_seqs;
    p.transpose = a.transpose;
    p.rows = a.table_rows;
    // 8 pairs per thread when every half-row vector is 16-byte aligned (16-bit types)
    const int half = a.head_dim / 2;
    auto al16 = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
    const bool vec = a.dtype == DSALT_DTYPE_BF16 && half % 8 == 0 && al16(a.q) && al16(a.k) && al16(a.q_out) &&
                     al16(a.k_out) && a.q_stride_t % 8 == 0 && a.q_stride_h % 8 == 0 && a.k_stride_t % 8 == 0 &&
                     a.k_stride_h % 8 == 0 && a.q_out_stride_t % 8 == 0 && a.q_out_stride_h % 8 == 0 &&
                     a.k_out_stride_t % 8 == 0 && a.k_out_stride_h % 8 == 0;
    const int64_t n = (int64_t)a.total_len * (a.n_q_heads + a.n_k_heads) * (vec ? half / 8 : half);
    const int grid = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    if (vec) hipLaunchKernelGGL((rope_kernel<BF16, 8>), dim3(grid), dim3(256), 0, stream, p);
    else if (a.dtype == DSALT_DTYPE_BF16) hipLaunchKernelGGL((rope_kernel<BF16, 1>), dim3(grid), dim3(256), 0, stream, p);
    else if (a.dtype == DSALT_DTYPE_F16) hipLaunchKernelGGL((rope_kernel<F16, 1>), dim3(grid), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((rope_kernel<F32, 1>), dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace dsalt
