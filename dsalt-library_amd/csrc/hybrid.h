// Arithmetic of the hybrid landmark score shared by the score kernels (scores.hip) and the
// selection that forms the scores on the fly from the norms pass (select.hip), so that
// both give the same bits.
//
// Reference: hybrid_scores_per_head (dsalt/kernels/landmark_tokens_ker.py:45-61):
//   z = (norm - mean) / std.clamp(min=1e-6) over all T packed tokens (unbiased std),
//   score = alpha * z_v + (1 - alpha) * z_x, in fp32.
#pragma once

#include "common.h"

namespace dsalt {

// Mean and unbiased std (clamped at 1e-6, NaN kept) of quantity q from the norms pass's
// fp64 partial sums part[b][nq][2] (sum, sum of squares) over b < nblk blocks and T tokens.
// One wave, fixed order: lane l adds blocks l, l + 64, ..., then a shuffle tree; products
// and differences rounded separately (no FMA). The result is valid in every lane. The
// partials are loaded kStatBatch blocks per lane at a time, ahead of their adds (the
// order of the adds is unchanged), so that the loads' latencies overlap.
constexpr int kStatBatch = 8;
__device__ __forceinline__ void hybrid_stat(const double *part, int nblk, int nq, int q, double T, int lane,
                                            float &mean, float &sd) {
    double s = 0.0, s2 = 0.0;
    for (int b0 = lane; b0 < nblk; b0 += 64 * kStatBatch) {
        double a[kStatBatch], a2[kStatBatch];
#pragma unroll
        for (int u = 0; u < kStatBatch; ++u) {
            const int b = min(b0 + 64 * u, nblk - 1);  // past the end: a valid block, not added
            const double *o = part + ((int64_t)b * nq + q) * 2;
            a[u] = o[0];
            a2[u] = o[1];
        }
#pragma unroll
        for (int u = 0; u < kStatBatch; ++u)
            if (b0 + 64 * u < nblk) {
                s = __dadd_rn(s, a[u]);
                s2 = __dadd_rn(s2, a2[u]);
            }
    }
    for (int off = 1; off < 64; off <<= 1) {
        s = __dadd_rn(s, __shfl_xor(s, off));
        s2 = __dadd_rn(s2, __shfl_xor(s2, off));
    }
    const double mn = __ddiv_rn(s, T);
    // unbiased variance; T = 1 gives 0/0 = NaN, as torch.std does
    const double var = __ddiv_rn(fmax(__dsub_rn(s2, __dmul_rn(s, mn)), 0.0), __dsub_rn(T, 1.0));
    const float f = (float)__dsqrt_rn(var);
    mean = (float)mn;
    sd = (f != f) ? f : fmaxf(f, 1e-6f);  // clamp(min=1e-6) keeps NaN
}

// z = (n - mean) / sd in fp32, correctly rounded at each step.
__device__ __forceinline__ float hybrid_z(float n, float mean, float sd) { return __fdiv_rn(__fsub_rn(n, mean), sd); }

// alpha * z_v + (1 - alpha) * z_x in the reference's fp32 operation order, never contracted.
__device__ __forceinline__ float hybrid_mix(float zx, float zv, float alpha) {
    return __fadd_rn(__fmul_rn(alpha, zv), __fmul_rn(__fsub_rn(1.0f, alpha), zx));
}

}  // namespace dsalt
