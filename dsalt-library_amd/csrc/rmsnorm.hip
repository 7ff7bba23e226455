// Residual add and RMSNorm of the LM's pre-norm blocks, in one pass.
//
// Reference: x = x + x_attn and x = x + x_ffn of DSALTTransformerBlock.forward
// (dsalt/modules/dsalt_transformer.py:81-84), each followed by the next RMSENorm
// (dsalt/kernels/RMSENorm.py:21-23: F.rms_norm with a per-channel weight), and the LM's
// final norm (dsalt/model/dsalt_lm.py:273). torch runs the add and the norm as two
// passes; here one wave takes one row of d elements:
//   x_out = x + h           each sum in fp32, rounded to the dtype (torch's add, exactly)
//   rstd  = rsqrt(sum(x_out^2) / d + eps)   fp32, this pass's fixed order of adds
//   y     = (x_out * rstd) * w              fp32, rounded to the dtype
// The operation order of y and the rsqrt are torch's (measured on this GPU: 38 of 16.8 M
// bf16 outputs differ at d = 1024, from rows whose fp32 sum of squares rounds
// differently). Bytes per row: x and h read, x_out and y written (4 passes of 16 bits
// per element against 6 for the add and the norm apart).
#include "common.h"
#include "launch.h"

#include <type_traits>

namespace dsalt {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row
constexpr int kMaxChunks = 8;     // 16-byte chunks per lane: d <= 64 * 8 * 8 = 4096

struct RmsParams {
    const uint4 *x, *h, *w;
    uint4 *x_out, *y;
    int64_t rows;
    int nch;  // 16-byte chunks per row
    float d, eps;
};

// fp32 value made opaque: a sum or product is rounded to fp32 before its 16-bit
// conversion (no mixed-precision fold that would round the exact value once).
__device__ __forceinline__ float opaque(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// NCH: 16-byte chunks per lane (d <= 512 NCH). Every load of the row (x, h and the
// weight chunks) is issued before any arithmetic; the arithmetic order is that of one
// chunk after the other.
template <typename DT, bool ADD, int NCH>
__global__ void __launch_bounds__(64 * kRowsPerBlock) add_rms_norm_kernel(const RmsParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // wave-uniform
    const int64_t base = row * p.nch;
    // chunk c of the lane holds elements (64 c + lane) * 8 .. + 7 (coalesced per chunk)
    uint4 s[NCH], hv[NCH], wv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int ch = c * 64 + lane;
        if (ch < p.nch) {
            s[c] = p.x[base + ch];
            if constexpr (ADD) hv[c] = p.h[base + ch];
            wv[c] = p.w[ch];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int ch = c * 64 + lane;
        if (ch < p.nch) {
            uint4 v = s[c];
            if constexpr (ADD) {
                const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = DT::pack2(opaque(DT::lo_f32(a[e]) + DT::lo_f32(b[e])),
                                     opaque(DT::hi_f32(a[e]) + DT::hi_f32(b[e])));
                v = make_uint4(o[0], o[1], o[2], o[3]);
                p.x_out[base + ch] = v;
            }
            s[c] = v;
            const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = DT::lo_f32(a[e]), hi = DT::hi_f32(a[e]);
                ss = fmaf(lo, lo, ss);
                ss = fmaf(hi, hi, ss);
            }
        }
    }
    ss = wave_sumf(ss);
    const float rstd = rsqrtf(ss / p.d + p.eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int ch = c * 64 + lane;
        if (ch < p.nch) {
            const uint4 v = s[c];
            const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = DT::pack2(opaque((DT::lo_f32(a[e]) * rstd) * DT::lo_f32(b[e])),
                                 opaque((DT::hi_f32(a[e]) * rstd) * DT::hi_f32(b[e])));
            p.y[base + ch] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

template <typename DT, bool ADD>
void launch_add(const RmsParams &p, const dim3 grid, const dim3 block, hipStream_t stream) {
    if (p.nch <= 64)
        hipLaunchKernelGGL((add_rms_norm_kernel<DT, ADD, 1>), grid, block, 0, stream, p);
    else if (p.nch <= 128)
        hipLaunchKernelGGL((add_rms_norm_kernel<DT, ADD, 2>), grid, block, 0, stream, p);
    else if (p.nch <= 256)
        hipLaunchKernelGGL((add_rms_norm_kernel<DT, ADD, 4>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((add_rms_norm_kernel<DT, ADD, kMaxChunks>), grid, block, 0, stream, p);
}

template <typename DT>
void launch_dt(const RmsParams &p, bool add, hipStream_t stream) {
    const dim3 grid((unsigned)((p.rows + kRowsPerBlock - 1) / kRowsPerBlock)), block(64 * kRowsPerBlock);
    if (add) launch_add<DT, true>(p, grid, block, stream);
    else launch_add<DT, false>(p, grid, block, stream);
}

}  // namespace

int rms_norm_max_dim() { return 64 * 8 * kMaxChunks; }

hipError_t launch_add_rms_norm(const void *x, const void *h, void *x_out, void *y, const void *weight, int64_t rows,
                               int d, float eps, int dtype, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    RmsParams p;
    p.x = static_cast<const uint4 *>(x);
    p.h = static_cast<const uint4 *>(h);
    p.w = static_cast<const uint4 *>(weight);
    p.x_out = static_cast<uint4 *>(x_out);
    p.y = static_cast<uint4 *>(y);
    p.rows = rows;
    p.nch = d / 8;
    p.d = (float)d;
    p.eps = eps;
    if (dtype == DSALT_DTYPE_BF16) launch_dt<BF16>(p, h != nullptr, stream);
    else launch_dt<F16>(p, h != nullptr, stream);
    return hipGetLastError();
}

}  // namespace dsalt
