// Gated SwiGLU product of the LM's feed-forward blocks, in one pass.
//
// Reference: SwiGLUFFN.forward (dsalt/modules/dsalt_transformer.py:20-21):
//   F.silu(gate_proj(x)) * up_proj(x)
// which torch runs as two elementwise passes: silu(g) = g / (1 + exp(-g)) in fp32, rounded
// to the tensor dtype, then the product with u in fp32, rounded again. This kernel reads
// g and u once and writes the product once, with the same two roundings (bit for bit
// torch's result): 3 bytes moved per 5 of the two passes.
//
// The pass is VALU-bound, not HBM-bound: expf and the IEEE division take ~25 instructions
// per element, and a wave64 instruction occupies a 16-lane SIMD for 4 cycles. The 16-bit
// roundings therefore use the hardware round-to-nearest-even conversions
// (v_cvt_pk_bf16_f32, v_cvt_f16_f32: one instruction per pair or value) rather than
// integer arithmetic. This file is built with hipcc's default contraction: under
// -ffp-contract=fast the backend fuses the range reduction inside expf into one fma and
// exp's last bit no longer matches torch's build.
#include "common.h"
#include "launch.h"
#include "rotary.h"  // the F32 element tag

#include <algorithm>
#include <type_traits>

namespace dsalt {
namespace {

// silu(g) rounded to the tensor dtype, as fp32. The fp32 quotient is made opaque before the
// conversion: otherwise the backend may fold the last step of the division and the
// conversion into one mixed-precision instruction that rounds the exact value once
// instead of to fp32 first.
template <typename DT>
__device__ __forceinline__ float silu_rounded(float g) {
    float s = g / (1.f + expf(-g));
    asm volatile("" : "+v"(s));
    if constexpr (std::is_same<DT, F32>::value)
        return s;
    else
        return DT::round(s);
}

// The fp32 product, opaque for the same reason, before its rounding by the caller's pack.
__device__ __forceinline__ float product(float s, float u) {
    float r = s * u;
    asm volatile("" : "+v"(r));
    return r;
}

// One 32-bit word of a 16-bit tensor: two elements, lo and hi.
template <typename DT>
__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g, uint32_t u) {
    const float r0 = product(silu_rounded<DT>(DT::lo_f32(g)), DT::lo_f32(u));
    const float r1 = product(silu_rounded<DT>(DT::hi_f32(g)), DT::hi_f32(u));
    return DT::pack2(r0, r1);
}

// One 16-byte word: 8 elements of a 16-bit tensor, 4 of an fp32 one.
template <typename DT>
__device__ __forceinline__ uint4 swiglu_word(uint4 g, uint4 u) {
    if constexpr (std::is_same<DT, F32>::value) {
        float4 a = bitcast<float4>(g), b = bitcast<float4>(u), r;
        r.x = product(silu_rounded<F32>(a.x), b.x);
        r.y = product(silu_rounded<F32>(a.y), b.y);
        r.z = product(silu_rounded<F32>(a.z), b.z);
        r.w = product(silu_rounded<F32>(a.w), b.w);
        return bitcast<uint4>(r);
    } else {
        return make_uint4(swiglu_pair<DT>(g.x, u.x), swiglu_pair<DT>(g.y, u.y), swiglu_pair<DT>(g.z, u.z),
                          swiglu_pair<DT>(g.w, u.w));
    }
}

// n16: 16-byte words of each tensor; grid-stride over them, two words in flight per
// iteration (the loads of both issued before either's arithmetic).
template <typename DT>
__global__ void __launch_bounds__(256) swiglu_kernel(const uint4 *__restrict__ g, const uint4 *__restrict__ u,
                                                     uint4 *__restrict__ o, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + stride < n16; i += 2 * stride) {
        const uint4 g0 = g[i], u0 = u[i], g1 = g[i + stride], u1 = u[i + stride];
        o[i] = swiglu_word<DT>(g0, u0);
        o[i + stride] = swiglu_word<DT>(g1, u1);
    }
    if (i < n16) o[i] = swiglu_word<DT>(g[i], u[i]);
}

}  // namespace

hipError_t launch_swiglu(const void *gate, const void *up, void *out, int64_t n, int dtype, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const int per = dtype == DSALT_DTYPE_F32 ? 4 : 8;  // elements per 16-byte word
    const int64_t n16 = n / per;
    const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, 8192);
    const uint4 *g = static_cast<const uint4 *>(gate), *u = static_cast<const uint4 *>(up);
    uint4 *o = static_cast<uint4 *>(out);
    if (dtype == DSALT_DTYPE_BF16)
        hipLaunchKernelGGL(swiglu_kernel<BF16>, dim3((unsigned)blocks), dim3(256), 0, stream, g, u, o, n16);
    else if (dtype == DSALT_DTYPE_F16)
        hipLaunchKernelGGL(swiglu_kernel<F16>, dim3((unsigned)blocks), dim3(256), 0, stream, g, u, o, n16);
    else
        hipLaunchKernelGGL(swiglu_kernel<F32>, dim3((unsigned)blocks), dim3(256), 0, stream, g, u, o, n16);
    return hipGetLastError();
}

}  // namespace dsalt
