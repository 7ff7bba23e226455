// Hybrid landmark scores from the value projection (fused selector front-end).
//
// Reference: hybrid_scores_per_head (dsalt/kernels/landmark_tokens_ker.py:19-61):
//   s[t, h] = alpha[h] * z(||x_t W_V,g(h)||) + (1 - alpha[h]) * z(||x_t||)
// where z standardises over all T packed tokens (mean, unbiased std clamped at 1e-6) and
// g(h) is the kv group of query head h. The reference forms x W_V^T with a GEMM; the
// attention module has that product already (its pre-RoPE value projection v), so this
// path takes v and reads each of x and v once.
//
// Three kernels, deterministic (no atomics, fixed reduction orders):
//  1. norms_kernel: one wave per token, 16 tokens per workgroup. ||x_t|| and ||v_t,g||
//     in fp32, each rounded to its input's dtype (what .norm() returns for a 16-bit
//     tensor, before .float()) unless norms_f32 is set (autocast runs .norm() in fp32
//     and returns it unrounded), written to the
//     workspace, plus the workgroup's fp64 partial sums of each quantity and its square.
//  2. stats_kernel (one workgroup): the partials summed in a fixed order (lanes stride
//     the blocks, then a fixed shuffle tree), the mean and the unbiased std in fp64,
//     rounded to fp32, the std clamped at 1e-6 with NaN kept.
//  3. standardize_kernel: z_x, z_v and the scores, elementwise, with the reference's
//     fp32 operation order (no FMA contraction).
// With k given, norms_kernel also applies RoPE to the token's k row (dsalt_rope's
// arithmetic, rotary.h): the module's k rotation rides on the pass that reads x and v
// anyway instead of taking a launch of its own. With gate_w given (16-bit x), it also
// forms the window gate's logit x_t . w + b (win_gate, dsalt_attention.py:270-276) from
// the x chunks it loads: fp32 products and sums in a fixed order, the bias added, one
// rounding to x's dtype; this replaces the module's GEMV and its bias copy.
#include "common.h"
#include "launch.h"
#include "hybrid.h"
#include "rotary.h"

namespace dsalt {
namespace {

constexpr int kNormTokens = 16;    // tokens (= waves) per workgroup of norms_kernel
constexpr int kStdTokens = 64;     // tokens per workgroup of standardize_kernel
constexpr int kMaxKvScores = 128;  // largest n_kv_heads (LDS of norms_kernel)

struct ScoreParams {
    const void *x, *v;
    const float *alpha;
    float *scores, *z_x, *z_v;
    float *xn, *vn;   // workspace: [T], [T, n_kv]
    double *part;     // workspace: [nblk][1 + n_kv][2]
    float *stats;     // workspace: [1 + n_kv][2] (mean, std)
    int64_t x_st, v_st, v_sh, s_st, s_sh, zv_st, zv_sh;
    int T, d, n_kv, D, H, nblk, norms_f32;
    // optional RoPE of k: null k, or k / k_out [T, n_kv, D] in v's dtype
    const void *k;
    void *k_out;
    int64_t k_st, k_sh, ko_st, ko_sh, cs_st;
    const float *cos, *sin;
    const int32_t *cu;
    int rows, S;
    // optional window-gate logit: x_t . gate_w + gate_b[0], rounded to x's dtype
    const void *gate_w, *gate_b;
    void *gate_out;
};

// Element loads and the dtype rounding of a norm, per storage type.
struct LdBF16 {
    static constexpr int E = 8;  // elements per 16 bytes
    static __device__ __forceinline__ float sumsq16(const void *p) { return sumsq(*reinterpret_cast<const uint4 *>(p)); }
    static __device__ __forceinline__ float sumsq(const uint4 u) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xffff0000u);
            s += a * a;
            s += b * b;
        }
        return s;
    }
    // round to nearest even bf16 (NaN kept)
    static __device__ __forceinline__ float round(float x) {
        uint32_t u = __float_as_uint(x);
        if ((u & 0x7fffffffu) > 0x7f800000u) return x;
        u += 0x7fffu + ((u >> 16) & 1u);
        return __uint_as_float(u & 0xffff0000u);
    }
    // acc + the 8 products of a chunk with the gate weights, in element order (each
    // product of two 16-bit values is exact in fp32)
    static __device__ __forceinline__ float dot(const uint4 x, const uint4 g, float acc) {
        const uint32_t a[4] = {x.x, x.y, x.z, x.w}, b[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = fmaf(__uint_as_float(a[i] << 16), __uint_as_float(b[i] << 16), acc);
            acc = fmaf(__uint_as_float(a[i] & 0xffff0000u), __uint_as_float(b[i] & 0xffff0000u), acc);
        }
        return acc;
    }
    static __device__ __forceinline__ float ld1(const void *p) {
        return __uint_as_float((uint32_t)*static_cast<const uint16_t *>(p) << 16);
    }
    static __device__ __forceinline__ void st1(void *p, float rounded) {
        *static_cast<uint16_t *>(p) = (uint16_t)(__float_as_uint(rounded) >> 16);
    }
};
struct LdF16 {
    static constexpr int E = 8;
    static __device__ __forceinline__ float sumsq16(const void *p) { return sumsq(*reinterpret_cast<const uint4 *>(p)); }
    static __device__ __forceinline__ float sumsq(const uint4 u) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = F16::lo_f32(w[i]), b = F16::hi_f32(w[i]);
            s += a * a;
            s += b * b;
        }
        return s;
    }
    static __device__ __forceinline__ float round(float x) { return (float)(_Float16)x; }
    static __device__ __forceinline__ float dot(const uint4 x, const uint4 g, float acc) {
        const uint32_t a[4] = {x.x, x.y, x.z, x.w}, b[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = fmaf(F16::lo_f32(a[i]), F16::lo_f32(b[i]), acc);
            acc = fmaf(F16::hi_f32(a[i]), F16::hi_f32(b[i]), acc);
        }
        return acc;
    }
    static __device__ __forceinline__ float ld1(const void *p) { return (float)*static_cast<const _Float16 *>(p); }
    static __device__ __forceinline__ void st1(void *p, float rounded) { *static_cast<_Float16 *>(p) = (_Float16)rounded; }
};
struct LdF32 {
    static constexpr int E = 4;
    static __device__ __forceinline__ float sumsq16(const void *p) {
        const float4 f = *reinterpret_cast<const float4 *>(p);
        float s = f.x * f.x;
        s += f.y * f.y;
        s += f.z * f.z;
        s += f.w * f.w;
        return s;
    }
    static __device__ __forceinline__ float round(float x) { return x; }
};

// Element tag (rotary.h) of each load type.
template <typename L> struct ElemOf;
template <> struct ElemOf<LdBF16> { typedef BF16 T; };
template <> struct ElemOf<LdF16> { typedef F16 T; };
template <> struct ElemOf<LdF32> { typedef F32 T; };

// Sum over the `width` lanes of each aligned lane group (width a power of two <= 64);
// every lane of the group receives it.
__device__ __forceinline__ float group_sum(float x, int width) {
    for (int o = 1; o < width; o <<= 1) x += __shfl_xor(x, o);
    return x;
}

template <typename LX, typename LV>
__global__ void __launch_bounds__(64 * kNormTokens) norms_kernel(const ScoreParams p) {
    constexpr int EX = LX::E, EV = LV::E;
    constexpr int BX = EX == 8 ? 2 : 4, BV = EV == 8 ? 2 : 4;  // bytes per element
    __shared__ float s_n[kNormTokens][1 + kMaxKvScores];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * kNormTokens;
    const int G = p.D / EV;         // lanes per v row
    const int rows_per = 64 / G;    // v rows per load instruction
    const int j = wave, t = t0 + wave;
    if (t < p.T) {  // wave-uniform
        // ||x_t||: lanes stride the row in 16-byte chunks
        const char *xr = static_cast<const char *>(p.x) + (int64_t)t * p.x_st * BX;
        float sx = 0.f;
        if constexpr (EX == 8) {
            if (p.gate_w) {
                // the window gate's logit from the same chunks: each lane sums its chunks'
                // products in order, then the lanes' sums are added by a fixed butterfly
                const char *gw = static_cast<const char *>(p.gate_w);
                float gd = 0.f;
                for (int c = lane * EX; c < p.d; c += 64 * EX) {
                    const uint4 xv = *reinterpret_cast<const uint4 *>(xr + (int64_t)c * BX);
                    sx += LX::sumsq(xv);
                    gd = LX::dot(xv, *reinterpret_cast<const uint4 *>(gw + (int64_t)c * BX), gd);
                }
                gd = group_sum(gd, 64);
                if (lane == 0) {
                    float logit = p.gate_b ? gd + LX::ld1(p.gate_b) : gd;
                    // rounded to fp32 first: no mixed-precision fold of the sum and the conversion
                    asm volatile("" : "+v"(logit));
                    LX::st1(static_cast<char *>(p.gate_out) + (int64_t)t * BX, LX::round(logit));
                }
            } else {
                for (int c = lane * EX; c < p.d; c += 64 * EX) sx += LX::sumsq16(xr + (int64_t)c * BX);
            }
        } else {
            for (int c = lane * EX; c < p.d; c += 64 * EX) sx += LX::sumsq16(xr + (int64_t)c * BX);
        }
        sx = group_sum(sx, 64);
        const float xn = p.norms_f32 ? sqrtf(sx) : LX::round(sqrtf(sx));
        if (lane == 0) {
            p.xn[t] = xn;
            s_n[j][0] = xn;
        }
        // ||v_t,g||: G lanes per row, rows_per rows per step
        const char *vr = static_cast<const char *>(p.v) + (int64_t)t * p.v_st * BV;
        for (int g0 = 0; g0 < p.n_kv; g0 += rows_per) {
            const int g = g0 + lane / G;
            float sv = 0.f;
            if (g < p.n_kv) sv = LV::sumsq16(vr + ((int64_t)g * p.v_sh + (lane % G) * EV) * BV);
            sv = group_sum(sv, G);
            const float vn = p.norms_f32 ? sqrtf(sv) : LV::round(sqrtf(sv));
            if (g < p.n_kv && lane % G == 0) {
                p.vn[(int64_t)t * p.n_kv + g] = vn;
                s_n[j][1 + g] = vn;
            }
        }
        if (p.k) {
            // RoPE of the token's k row: lane r takes pair vector r (16 bytes of each half)
            constexpr int VW = EV;
            const int half = p.D >> 1, nj = half / VW;
            const int pos = p.cu ? seq_offset(p.cu, p.S, p.T, t) : t;
            const bool in_table = pos >= 0 && pos < p.rows;
            const float *cr = p.cos + (int64_t)(in_table ? pos : 0) * p.cs_st;
            const float *sr = p.sin + (int64_t)(in_table ? pos : 0) * p.cs_st;
            for (int r = lane; r < p.n_kv * nj; r += 64) {
                const int h = r / nj, j0 = (r - h * nj) * VW;
                rotate_vec<typename ElemOf<LV>::T, VW>(p.k, (int64_t)t * p.k_st + (int64_t)h * p.k_sh, p.k_out,
                                                       (int64_t)t * p.ko_st + (int64_t)h * p.ko_sh, cr, sr, half, j0,
                                                       in_table, false);
            }
        }
    }
    __syncthreads();
    // fp64 partial sums of this block's tokens, in token order
    const int nt = min(kNormTokens, p.T - t0);
    for (int q = threadIdx.x; q <= p.n_kv; q += blockDim.x) {
        double s = 0.0, s2 = 0.0;
        for (int j = 0; j < nt; ++j) {
            const double a = s_n[j][q];
            s += a;
            s2 += a * a;
        }
        double *o = p.part + ((int64_t)blockIdx.x * (1 + p.n_kv) + q) * 2;
        o[0] = s;
        o[1] = s2;
    }
}

__global__ void __launch_bounds__(1024) stats_kernel(const ScoreParams p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int q = wave; q <= p.n_kv; q += 16) {  // wave-uniform
        float mean, sd;
        hybrid_stat(p.part, p.nblk, 1 + p.n_kv, q, (double)p.T, lane, mean, sd);
        if (lane == 0) {
            p.stats[2 * q] = mean;
            p.stats[2 * q + 1] = sd;
        }
    }
}

__global__ void __launch_bounds__(256) standardize_kernel(const ScoreParams p) {
#pragma clang fp contract(off)
    __shared__ float s_mean[1 + kMaxKvScores], s_std[1 + kMaxKvScores];
    for (int q = threadIdx.x; q <= p.n_kv; q += blockDim.x) {
        s_mean[q] = p.stats[2 * q];
        s_std[q] = p.stats[2 * q + 1];
    }
    __syncthreads();
    const int rep = p.H / p.n_kv;
    const int t0 = blockIdx.x * kStdTokens;
    const int nt = min(kStdTokens, p.T - t0);
    for (int e = threadIdx.x; e < nt * p.H; e += blockDim.x) {
        const int t = t0 + e / p.H, h = e % p.H, g = h / rep;
        const float zx = hybrid_z(p.xn[t], s_mean[0], s_std[0]);
        const float zv = hybrid_z(p.vn[(int64_t)t * p.n_kv + g], s_mean[1 + g], s_std[1 + g]);
        p.scores[(int64_t)t * p.s_st + (int64_t)h * p.s_sh] = hybrid_mix(zx, zv, p.alpha[h]);
        if (p.z_v) p.z_v[(int64_t)t * p.zv_st + (int64_t)h * p.zv_sh] = zv;
        if (p.z_x && h == 0) p.z_x[t] = zx;
    }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

template <typename LX>
void launch_norms_x(int v_dtype, const ScoreParams &p, hipStream_t stream) {
    if (v_dtype == DSALT_DTYPE_BF16)
        hipLaunchKernelGGL((norms_kernel<LX, LdBF16>), dim3(p.nblk), dim3(64 * kNormTokens), 0, stream, p);
    else if (v_dtype == DSALT_DTYPE_F16)
        hipLaunchKernelGGL((norms_kernel<LX, LdF16>), dim3(p.nblk), dim3(64 * kNormTokens), 0, stream, p);
    else
        hipLaunchKernelGGL((norms_kernel<LX, LdF32>), dim3(p.nblk), dim3(64 * kNormTokens), 0, stream, p);
}

void launch_norms(int x_dtype, int v_dtype, const ScoreParams &p, hipStream_t stream) {
    if (x_dtype == DSALT_DTYPE_BF16) launch_norms_x<LdBF16>(v_dtype, p, stream);
    else if (x_dtype == DSALT_DTYPE_F16) launch_norms_x<LdF16>(v_dtype, p, stream);
    else launch_norms_x<LdF32>(v_dtype, p, stream);
}

}  // namespace

int64_t scores_workspace_bytes(int total_len, int n_kv) {
    const int nblk = (total_len + kNormTokens - 1) / kNormTokens;
    return (int64_t)(align256((size_t)total_len * 4) + align256((size_t)total_len * n_kv * 4) +
                     align256((size_t)nblk * (1 + n_kv) * 2 * 8) + align256((size_t)(1 + n_kv) * 2 * 4));
}

int scores_max_kv() { return kMaxKvScores; }

namespace {

ScoreParams make_params(const dsalt_scores_args &a) {
    ScoreParams p;
    p.x = a.x;
    p.v = a.v;
    p.alpha = a.alpha;
    p.scores = a.scores;
    p.z_x = a.z_x;
    p.z_v = a.z_v;
    p.T = a.total_len;
    p.d = a.d_model;
    p.n_kv = a.n_kv_heads;
    p.D = a.head_dim;
    p.H = a.n_heads;
    p.nblk = (a.total_len + kNormTokens - 1) / kNormTokens;
    p.norms_f32 = a.norms_f32 != 0;
    char *ws = static_cast<char *>(a.workspace);
    p.xn = reinterpret_cast<float *>(ws);
    ws += align256((size_t)p.T * 4);
    p.vn = reinterpret_cast<float *>(ws);
    ws += align256((size_t)p.T * p.n_kv * 4);
    p.part = reinterpret_cast<double *>(ws);
    ws += align256((size_t)p.nblk * (1 + p.n_kv) * 2 * 8);
    p.stats = reinterpret_cast<float *>(ws);
    p.x_st = a.x_stride_t;
    p.v_st = a.v_stride_t;
    p.v_sh = a.v_stride_h;
    p.s_st = a.scores_stride_t;
    p.s_sh = a.scores_stride_h;
    p.zv_st = a.z_v_stride_t;
    p.zv_sh = a.z_v_stride_h;
    p.k = a.k;
    p.k_out = a.k_out;
    p.k_st = a.k_stride_t;
    p.k_sh = a.k_stride_h;
    p.ko_st = a.k_out_stride_t;
    p.ko_sh = a.k_out_stride_h;
    p.cos = a.rope_cos;
    p.sin = a.rope_sin;
    p.cs_st = a.rope_stride;
    p.cu = a.cu_seqlens;
    p.rows = a.rope_rows;
    p.S = a.num_seqs;
    p.gate_w = a.gate_w;
    p.gate_b = a.gate_b;
    p.gate_out = a.gate_out;
    return p;
}

}  // namespace

hipError_t launch_scores(const dsalt_scores_args &a, hipStream_t stream) {
    if (a.total_len == 0) return hipSuccess;
    const ScoreParams p = make_params(a);
    launch_norms(a.x_dtype, a.v_dtype, p, stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(stats_kernel, dim3(1), dim3(1024), 0, stream, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(standardize_kernel, dim3((p.T + kStdTokens - 1) / kStdTokens), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_norms_for_select(const dsalt_scores_args &a, HybridSrc &src, hipStream_t stream) {
    const ScoreParams p = make_params(a);
    src.xn = p.xn;
    src.vn = p.vn;
    src.part = p.part;
    src.alpha = a.alpha;
    src.nblk = p.nblk;
    src.n_kv = p.n_kv;
    src.n_heads = p.H;
    src.total_len = p.T;
    if (a.total_len == 0) return hipSuccess;
    launch_norms(a.x_dtype, a.v_dtype, p, stream);
    return hipGetLastError();
}

}  // namespace dsalt
