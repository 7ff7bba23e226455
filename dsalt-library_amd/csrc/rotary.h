// Rotary position embedding helpers shared by the RoPE kernel (rope.hip) and the score
// pass that rotates k alongside the selector norms (scores.hip).
//
// Reference: apply_rotary_emb (dsalt/kernels/window_utils.py:73-88), half-split, per
// head, for j < D/2 with cos/sin rows rounded to the tensor dtype:
//   out[j]       = x[j] c[j]             - x[j + D/2] s[j]
//   out[j + D/2] = x[j + D/2] c[j + D/2] + x[j] s[j + D/2]
// products and sum in fp32 without FMA contraction, one rounding of the result. The
// transposed rotation (the backward) swaps the signs: g -> dx with
//   dx[j]       = g[j] c[j]             + g[j + D/2] s[j + D/2]
//   dx[j + D/2] = g[j + D/2] c[j + D/2] - g[j] s[j]
#pragma once

#include "common.h"

namespace dsalt {

struct F32 {};  // element tag of fp32 tensors

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
    template <int VW>
    static __device__ __forceinline__ void ldv(const void *p, int64_t i, float *x) {
        if constexpr (VW == 8) {
            const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + i);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = __uint_as_float(w[e] << 16);
                x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int e = 0; e < VW; ++e) x[e] = ld(p, i + e);
        }
    }
    template <int VW>
    static __device__ __forceinline__ void stv(void *p, int64_t i, const float *x) {
        if constexpr (VW == 8) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = (__float_as_uint(round(x[2 * e])) >> 16) | (__float_as_uint(round(x[2 * e + 1])) & 0xffff0000u);
            *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p) + i) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int e = 0; e < VW; ++e) st(p, i + e, x[e]);
        }
    }
};
template <>
struct Elem<F16> {
    static __device__ __forceinline__ float ld(const void *p, int64_t i) {
        return (float)static_cast<const _Float16 *>(p)[i];
    }
    static __device__ __forceinline__ float round(float x) { return (float)(_Float16)x; }
    static __device__ __forceinline__ void st(void *p, int64_t i, float x) { static_cast<_Float16 *>(p)[i] = (_Float16)x; }
    template <int VW>
    static __device__ __forceinline__ void ldv(const void *p, int64_t i, float *x) {
        if constexpr (VW == 8) {  // one 16-byte load
            const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const _Float16 *>(p) + i);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = F16::lo_f32(w[e]);
                x[2 * e + 1] = F16::hi_f32(w[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < VW; ++e) x[e] = ld(p, i + e);
        }
    }
    template <int VW>
    static __device__ __forceinline__ void stv(void *p, int64_t i, const float *x) {
        if constexpr (VW == 8) {  // one 16-byte store
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = F16::pack2(x[2 * e], x[2 * e + 1]);
            *reinterpret_cast<uint4 *>(static_cast<_Float16 *>(p) + i) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int e = 0; e < VW; ++e) st(p, i + e, x[e]);
        }
    }
};
template <>
struct Elem<F32> {
    static __device__ __forceinline__ float ld(const void *p, int64_t i) { return static_cast<const float *>(p)[i]; }
    static __device__ __forceinline__ float round(float x) { return x; }
    static __device__ __forceinline__ void st(void *p, int64_t i, float x) { static_cast<float *>(p)[i] = x; }
    template <int VW>
    static __device__ __forceinline__ void ldv(const void *p, int64_t i, float *x) {
        if constexpr (VW == 4) {  // one 16-byte load
            const float4 v = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
            x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        } else {
#pragma unroll
            for (int e = 0; e < VW; ++e) x[e] = ld(p, i + e);
        }
    }
    template <int VW>
    static __device__ __forceinline__ void stv(void *p, int64_t i, const float *x) {
        if constexpr (VW == 4) {  // one 16-byte store
            *reinterpret_cast<float4 *>(static_cast<float *>(p) + i) = make_float4(x[0], x[1], x[2], x[3]);
        } else {
#pragma unroll
            for (int e = 0; e < VW; ++e) st(p, i + e, x[e]);
        }
    }
};

template <int VW>
__device__ __forceinline__ void ldv_f32(const float *p, float *x) {
#pragma unroll
    for (int e = 0; e < VW; ++e) x[e] = p[e];
}


// Offset of token t inside its sequence (binary search over cu_seqlens[0 .. S], its
// entries clamped to [0, T] as seq_bounds clamps them). Negative for a token before the
// first sequence.
__device__ __forceinline__ int seq_offset(const int32_t *cu, int S, int T, int t) {
    auto at = [&](int s) { return min(max(cu[s], 0), T); };
    int lo = 0, hi = S;  // cu[lo] <= t < cu[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (at(mid) <= t) lo = mid;
        else hi = mid;
    }
    return t - at(lo);
}

// Rotate the VW pairs (j0 + e, j0 + e + half) of one head row: reads in[ib + ...], writes
// out[ob + ...] (out may alias in: each pair is read before it is written), tables row
// cr / sr (fp32, rounded to DT here; NaN when !in_table).
// The products and the sum are __fmul_rn / __fsub_rn / __fadd_rn (never contracted into
// an FMA), and each fp32 result is made opaque before its conversion to the 16-bit type:
// otherwise the backend may fold the sum and the conversion into one mixed-precision
// v_fma_mix{lo,hi}_f16, which rounds the exact sum once instead of to fp32 first.
template <typename DT, int VW>
__device__ __forceinline__ void rotate_vec(const void *in, int64_t ib, void *out, int64_t ob, const float *cr,
                                           const float *sr, int half, int j0, bool in_table, bool transpose) {
    typedef Elem<DT> E;
    float a[VW], b[VW], c0[VW], c1[VW], s0[VW], s1[VW], o0[VW], o1[VW];
    E::template ldv<VW>(in, ib + j0, a);
    E::template ldv<VW>(in, ib + j0 + half, b);
    ldv_f32<VW>(cr + j0, c0);
    ldv_f32<VW>(cr + j0 + half, c1);
    ldv_f32<VW>(sr + j0, s0);
    ldv_f32<VW>(sr + j0 + half, s1);
#pragma unroll
    for (int e = 0; e < VW; ++e) {
        const float cc0 = in_table ? E::round(c0[e]) : NAN, cc1 = in_table ? E::round(c1[e]) : NAN;
        const float ss0 = in_table ? E::round(s0[e]) : NAN, ss1 = in_table ? E::round(s1[e]) : NAN;
        if (!transpose) {
            o0[e] = __fsub_rn(__fmul_rn(a[e], cc0), __fmul_rn(b[e], ss0));
            o1[e] = __fadd_rn(__fmul_rn(b[e], cc1), __fmul_rn(a[e], ss1));
        } else {
            o0[e] = __fadd_rn(__fmul_rn(a[e], cc0), __fmul_rn(b[e], ss1));
            o1[e] = __fsub_rn(__fmul_rn(b[e], cc1), __fmul_rn(a[e], ss0));
        }
        asm volatile("" : "+v"(o0[e]), "+v"(o1[e]));
    }
    E::template stv<VW>(out, ob + j0, o0);
    E::template stv<VW>(out, ob + j0 + half, o1);
}

}  // namespace dsalt
