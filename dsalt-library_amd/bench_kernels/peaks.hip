// Peak probes for bench.py (not part of the DSALT C ABI): what one MI355X sustains of its
// published dense bf16 MFMA rate and of its HBM read rate, with kernels that do nothing
// else. Built by build.py into libdsalt_peaks.so next to the product library.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Four independent chains of v_mfma_f32_32x32x16_bf16 per wave (the MFMA pipe never waits
// on a result), `iters` rounds; one float per thread keeps the chains alive.
__global__ void __launch_bounds__(256) mfma_loop_kernel(float *out, int iters) {
    const float t = (float)(threadIdx.x & 63) * 1e-3f;
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(t + e);
        b[e] = (__bf16)(t - e);
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Grid-stride read of `n16` 16-byte words: every word read once, one float per thread out.
__global__ void __launch_bounds__(256) read_kernel(const uint4 *src, int64_t n16, float *out) {
    uint32_t acc = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = (float)acc;
}

extern "C" {

// Milliseconds of one launch of `blocks` x 256 threads running `iters` rounds of four MFMAs
// per wave (after one warm-up launch), or a negative value on error. FLOPs =
// blocks * 4 waves * iters * 4 * 32 * 32 * 16 * 2.
float dsalt_bench_mfma(int blocks, int iters) {
    float *out = nullptr;
    if (blocks < 1 || iters < 1 || hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) return -1.f;
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    hipLaunchKernelGGL(mfma_loop_kernel, dim3(blocks), dim3(256), 0, 0, out, iters);
    (void)hipEventRecord(e0, 0);
    hipLaunchKernelGGL(mfma_loop_kernel, dim3(blocks), dim3(256), 0, 0, out, iters);
    (void)hipEventRecord(e1, 0);
    float ms = -1.f;
    if (hipEventSynchronize(e1) == hipSuccess) (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipFree(out);
    return ms;
}

// Milliseconds of one read of `bytes` (a multiple of 16, 16-byte aligned) at `src` by
// `blocks` x 256 threads (after one warm-up launch), or a negative value on error.
float dsalt_bench_read(const void *src, int64_t bytes, int blocks) {
    float *out = nullptr;
    if (blocks < 1 || bytes < 16 || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16 ||
        hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess)
        return -1.f;
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    const uint4 *p = static_cast<const uint4 *>(src);
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, 0, p, bytes / 16, out);
    (void)hipEventRecord(e0, 0);
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, 0, p, bytes / 16, out);
    (void)hipEventRecord(e1, 0);
    float ms = -1.f;
    if (hipEventSynchronize(e1) == hipSuccess) (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipFree(out);
    return ms;
}

}  // extern "C"
