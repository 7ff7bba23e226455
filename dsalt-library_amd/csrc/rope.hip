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

template <typename DT>
struct Elem;
template <>
struct Elem<BF16> {
    static __device__ __forceinline__ float ld(const void *p, int64_t i) {
        return __uint_as_float((uint32_t)static_cast<const uint16_t *>(p)[i] << 16);
    }
    static __device__ __forceinline__ float round(float x) {
        uint32_t u = __float_as_uint(x);
        if ((u & 0x7fffffffu) > 0x7f800000u) return x;
        u += 0x7fffu + ((u >> 16) & 1u);
        return __uint_as_float(u & 0xffff0000u);
    }
    static __device__ __forceinline__ void st(void *p, int64_t i, float x) {
        static_cast<uint16_t *>(p)[i] = (uint16_t)(__float_as_uint(round(x)) >> 16);
    }
};
template <>
struct Elem<F16> {
    static __device__ __forceinline__ float ld(const void *p, int64_t i) {
        return (float)static_cast<const _Float16 *>(p)[i];
    }
    static __device__ __forceinline__ float round(float x) { return (float)(_Float16)x; }
    static __device__ __forceinline__ void st(void *p, int64_t i, float x) { static_cast<_Float16 *>(p)[i] = (_Float16)x; }
};
struct F32 {};
template <>
struct Elem<F32> {
    static __device__ __forceinline__ float ld(const void *p, int64_t i) { return static_cast<const float *>(p)[i]; }
    static __device__ __forceinline__ float round(float x) { return x; }
    static __device__ __forceinline__ void st(void *p, int64_t i, float x) { static_cast<float *>(p)[i] = x; }
};

// One thread per (token, head, j < D/2) of q then k: both elements of the rotated pair.
// Reads and writes of a pair happen in the same thread, so out may alias in.
template <typename DT>
__global__ void __launch_bounds__(256) rope_kernel(const RopeParams p) {
#pragma clang fp contract(off)
    typedef Elem<DT> E;
    const int half = p.D >> 1;
    const int64_t per_tok = (int64_t)(p.heads[0] + p.heads[1]) * half;
    const int64_t n = (int64_t)p.T * per_tok;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int t = (int)(idx / per_tok);
        int r = (int)(idx - (int64_t)t * per_tok);
        const int which = r >= p.heads[0] * half;  // 0: q, 1: k
        if (which) r -= p.heads[0] * half;
        const int h = r / half, j = r - h * half;
        int pos = t;
        if (p.cu) {  // offset inside the sequence: binary search over cu_seqlens
            int lo = 0, hi = p.S;  // cu[lo] <= t < cu[hi]
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (p.cu[mid] <= t) lo = mid;
                else hi = mid;
            }
            pos = t - p.cu[lo];
        }
        float c0 = NAN, c1 = NAN, s0 = NAN, s1 = NAN;  // a row past the table: NaN outputs
        if (pos < p.rows) {
            const float *cr = p.cos + (int64_t)pos * p.cs_st, *sr = p.sin + (int64_t)pos * p.cs_st;
            c0 = E::round(cr[j]);
            c1 = E::round(cr[j + half]);
            s0 = E::round(sr[j]);
            s1 = E::round(sr[j + half]);
        }
        const int64_t ib = (int64_t)t * p.in_st[which] + (int64_t)h * p.in_sh[which];
        const float a = E::ld(p.in[which], ib + j), b = E::ld(p.in[which], ib + j + half);
        float o0, o1;
        if (!p.transpose) {
            o0 = a * c0 - b * s0;
            o1 = b * c1 + a * s1;
        } else {
            o0 = a * c0 + b * s1;
            o1 = b * c1 - a * s0;
        }
        const int64_t ob = (int64_t)t * p.out_st[which] + (int64_t)h * p.out_sh[which];
        E::st(p.out[which], ob + j, o0);
        E::st(p.out[which], ob + j + half, o1);
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
    const int64_t n = (int64_t)a.total_len * (a.n_q_heads + a.n_k_heads) * (a.head_dim / 2);
    const int grid = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    if (a.dtype == DSALT_DTYPE_BF16) hipLaunchKernelGGL(rope_kernel<BF16>, dim3(grid), dim3(256), 0, stream, p);
    else if (a.dtype == DSALT_DTYPE_F16) hipLaunchKernelGGL(rope_kernel<F16>, dim3(grid), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(rope_kernel<F32>, dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace dsalt
