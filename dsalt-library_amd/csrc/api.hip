// extern "C" entry points of libdsalt_hip.so: host-side argument validation, error
// reporting and dispatch to the kernel launchers. Declared in include/dsalt_hip.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <initializer_list>
#include <mutex>

#include "launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Shared checks of a packed [T, H, D] 16-bit tensor read/written with 16-byte
// (or `vec_elems`-element) vector accesses along D.
int check_tensor(const char *name, const void *p, int64_t st, int64_t sh, int vec_elems) {
    if (!p) return fail(DSALT_ERR_INVALID, "%s is NULL", name);
    if (!aligned(p, vec_elems * 2))
        return fail(DSALT_ERR_INVALID, "%s must be %d-byte aligned", name, vec_elems * 2);
    if (st < 0 || sh < 0 || st % vec_elems || sh % vec_elems)
        return fail(DSALT_ERR_INVALID, "%s strides (t=%lld, h=%lld) must be non-negative multiples of %d",
                    name, (long long)st, (long long)sh, vec_elems);
    return DSALT_OK;
}

int check_common(int mode, int dtype, int T, int S, int H, int D, int k, const int32_t *cu,
                 const float *w, const int64_t *lmk_pos) {
    if (mode != DSALT_MODE_HARD && mode != DSALT_MODE_SOFT && mode != DSALT_MODE_DENSE)
        return fail(DSALT_ERR_INVALID, "mode must be DSALT_MODE_HARD, DSALT_MODE_SOFT or DSALT_MODE_DENSE (got %d)",
                    mode);
    if (dtype != DSALT_DTYPE_BF16 && dtype != DSALT_DTYPE_F16)
        return fail(DSALT_ERR_INVALID, "dtype must be DSALT_DTYPE_BF16 or DSALT_DTYPE_F16 (got %d)", dtype);
    if (T < 0) return fail(DSALT_ERR_INVALID, "total_len must be >= 0 (got %d)", T);
    if (S < 1) return fail(DSALT_ERR_INVALID, "num_seqs must be >= 1 (got %d)", S);
    if (H < 1) return fail(DSALT_ERR_INVALID, "n_heads must be >= 1 (got %d)", H);
    if (D != 64 && D != 128)
        return fail(DSALT_ERR_UNSUPPORTED, "head_dim must be 64 or 128 (got %d)", D);
    if (k < 0 || k > DSALT_MAX_K_LMK)
        return fail(DSALT_ERR_UNSUPPORTED, "k_lmk must be in [0, %d] (got %d)", DSALT_MAX_K_LMK, k);
    if (mode == DSALT_MODE_DENSE) {
        if (S != 1) return fail(DSALT_ERR_INVALID, "DSALT_MODE_DENSE takes one sequence (num_seqs = %d)", S);
        if (k != 0)
            return fail(DSALT_ERR_INVALID, "DSALT_MODE_DENSE takes its landmarks as an [H, T] bias table (k_lmk = %d)", k);
    } else if (!cu) {
        return fail(DSALT_ERR_INVALID, "cu_seqlens is NULL");
    }
    if (!w) return fail(DSALT_ERR_INVALID, "w (window sizes) is NULL");
    if (k > 0 && !lmk_pos) return fail(DSALT_ERR_INVALID, "lmk_pos is NULL while k_lmk = %d", k);
    const int64_t blocks = (int64_t)dsalt::block_upper_bound(T, S, dsalt::kFwdBM) * H;
    if (blocks > (int64_t)INT32_MAX / 2)
        return fail(DSALT_ERR_UNSUPPORTED, "problem too large: %lld query blocks", (long long)blocks);
    return DSALT_OK;
}

int check_kv_heads(int n_heads, int n_kv) {
    if (n_kv < 0 || (n_kv > 0 && n_heads % n_kv != 0))
        return fail(DSALT_ERR_INVALID, "n_kv_heads must be 0 or divide n_heads = %d (got %d)", n_heads, n_kv);
    return DSALT_OK;
}

int check_mode_scalars(int mode, float scale, float tau_win, float win_edge) {
    if (mode != DSALT_MODE_HARD && !(tau_win > 0.f))
        return fail(DSALT_ERR_INVALID, "tau_win must be > 0 (got %g)", (double)tau_win);
    if (mode == DSALT_MODE_DENSE && !(fabsf(win_edge) < INFINITY))
        return fail(DSALT_ERR_INVALID, "win_edge must be finite (got %g)", (double)win_edge);
    if (!(scale == scale)) return fail(DSALT_ERR_INVALID, "scale is NaN");
    if (scale == 0.f || !(fabsf(scale) < INFINITY))
        return fail(DSALT_ERR_UNSUPPORTED, "scale must be finite and non-zero (got %g)", (double)scale);
    if (mode == DSALT_MODE_DENSE && !(scale > 0.f))
        return fail(DSALT_ERR_UNSUPPORTED, "DSALT_MODE_DENSE needs scale > 0 (got %g)", (double)scale);
    return DSALT_OK;
}

// Rows of one sequence are addressed through buffer resources with 32-bit byte
// offsets (row index x row stride): every such operand must span < 4 GiB over total_len
// rows plus kSpanMargin, so that the rows of a tile that starts up to kSpanMargin rows
// below the buffer (their offsets wrap to above 4 GiB - kSpanMargin x stride) fall out
// of range and read zeros. `row_bytes` lists each operand's row stride in bytes.
constexpr int64_t kSpanMargin = 64;
int check_span32(int total_len, std::initializer_list<int64_t> row_bytes) {
    int64_t widest = 0;
    for (int64_t b : row_bytes) widest = b > widest ? b : widest;
    if (((int64_t)total_len + kSpanMargin) * widest >= ((int64_t)1 << 32))
        return fail(DSALT_ERR_UNSUPPORTED,
                    "a sequence's rows must span < 4 GiB (total_len %d x row stride %lld B)", total_len,
                    (long long)widest);
    return DSALT_OK;
}

// Scratch of dsalt_bwd_noalloc: one static array per GPU (each device holds its own copy
// at its own address from the moment the library's code is loaded on it). In host code
// `scratch` names a host-side stand-in, not device memory: its device address is looked
// up once per device with hipGetSymbolAddress (that device current) and only that
// address is ever handed to kernels.
__device__ __align__(256) char scratch[DSALT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 256;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device id, null until looked up

int scratch_address(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(DSALT_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(DSALT_ERR_UNSUPPORTED, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(DSALT_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DSALT_OK;
}

}  // namespace

extern "C" {

int dsalt_abi_version(void) { return DSALT_ABI_VERSION; }
const char *dsalt_last_error(void) { return g_err; }
size_t dsalt_fwd_args_size(void) { return sizeof(dsalt_fwd_args); }
size_t dsalt_bwd_args_size(void) { return sizeof(dsalt_bwd_args); }
size_t dsalt_select_args_size(void) { return sizeof(dsalt_select_args); }
size_t dsalt_scores_args_size(void) { return sizeof(dsalt_scores_args); }
size_t dsalt_rope_args_size(void) { return sizeof(dsalt_rope_args); }

int dsalt_fwd_check(const dsalt_fwd_args *a) {
    if (!a) return fail(DSALT_ERR_INVALID, "args is NULL");
    int rc = check_common(a->mode, a->dtype, a->total_len, a->num_seqs, a->n_heads, a->head_dim,
                          a->k_lmk, a->cu_seqlens, a->w, a->lmk_pos);
    if (rc) return rc;
    if ((rc = check_tensor("q", a->q, a->q_stride_t, a->q_stride_h, 8))) return rc;
    if ((rc = check_tensor("k", a->k, a->k_stride_t, a->k_stride_h, 8))) return rc;
    if ((rc = check_tensor("v", a->v, a->v_stride_t, a->v_stride_h, 8))) return rc;
    if (a->out_dtype != a->dtype && a->out_dtype != DSALT_DTYPE_F32)
        return fail(DSALT_ERR_INVALID, "out_dtype must equal dtype or be DSALT_DTYPE_F32 (got %d)", a->out_dtype);
    {  // rows are written 4 elements at a time; check_tensor counts 16-bit elements
        const int64_t m = a->out_dtype == DSALT_DTYPE_F32 ? 2 : 1;
        if ((rc = check_tensor("out", a->out, a->out_stride_t * m, a->out_stride_h * m, (int)(4 * m)))) return rc;
    }
    if (!a->lse) return fail(DSALT_ERR_INVALID, "lse is NULL");
    if ((rc = check_mode_scalars(a->mode, a->scale, a->tau_win, a->win_edge))) return rc;
    if ((rc = check_kv_heads(a->n_heads, a->n_kv_heads))) return rc;
    if (a->rope_cos || a->rope_sin) {
        if (!a->rope_cos || !a->rope_sin) return fail(DSALT_ERR_INVALID, "rope_cos and rope_sin must both be set");
        if (a->mode == DSALT_MODE_DENSE)
            return fail(DSALT_ERR_UNSUPPORTED, "the RoPE of Q on load is not available in DSALT_MODE_DENSE");
        if (a->rope_rows < 1 || a->rope_stride < a->head_dim || !aligned(a->rope_cos, 16) || !aligned(a->rope_sin, 16) ||
            a->rope_stride % 4)
            return fail(DSALT_ERR_INVALID,
                        "RoPE tables need rope_rows >= 1, rope_stride >= head_dim and a multiple of 4, 16-byte "
                        "alignment (rows %d, stride %lld)", a->rope_rows, (long long)a->rope_stride);
    }
    return check_span32(a->total_len, {2 * a->q_stride_t, 2 * a->k_stride_t, 2 * a->v_stride_t});
}

int dsalt_fwd(const dsalt_fwd_args *a, void *stream) {
    int rc = dsalt_fwd_check(a);
    if (rc) return rc;
    hipError_t e = dsalt::launch_fwd(*a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(DSALT_ERR_LAUNCH, "dsalt_fwd launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

namespace {

// hybrid: the scores are formed in the launch (dsalt_select_hybrid), so none are read
int check_select(const dsalt_select_args *a, bool hybrid) {
    if (!a) return fail(DSALT_ERR_INVALID, "args is NULL");
    if (a->total_len < 0) return fail(DSALT_ERR_INVALID, "total_len must be >= 0");
    if (a->num_seqs < 1) return fail(DSALT_ERR_INVALID, "num_seqs must be >= 1");
    if (a->n_heads < 1) return fail(DSALT_ERR_INVALID, "n_heads must be >= 1");
    if (a->k_lmk < 0 || a->k_lmk > DSALT_MAX_K_LMK)
        return fail(DSALT_ERR_UNSUPPORTED, "k_lmk must be in [0, %d] (got %d)", DSALT_MAX_K_LMK, a->k_lmk);
    if ((!a->scores && !hybrid) || (!a->w && !a->w_logit) || !a->cu_seqlens || (!a->lmk_pos && a->k_lmk > 0))
        return fail(DSALT_ERR_INVALID, "scores, w (or w_logit), cu_seqlens and lmk_pos must be non-NULL");
    if (a->w_logit) {
        if (!a->w_out) return fail(DSALT_ERR_INVALID, "w_logit needs w_out (the quantised windows are returned there)");
        if (a->w_logit_dtype != DSALT_DTYPE_BF16 && a->w_logit_dtype != DSALT_DTYPE_F16)
            return fail(DSALT_ERR_UNSUPPORTED, "w_logit_dtype must be DSALT_DTYPE_BF16 or _F16 (got %d)",
                        a->w_logit_dtype);
        if (!(a->n_min == a->n_min) || !(a->n_max == a->n_max))
            return fail(DSALT_ERR_INVALID, "n_min and n_max must not be NaN");
    }
    if ((int64_t)a->num_seqs * a->n_heads > (int64_t)INT32_MAX)
        return fail(DSALT_ERR_UNSUPPORTED, "too many (head, sequence) pairs");
    if (a->max_seqlen < 0) return fail(DSALT_ERR_INVALID, "max_seqlen must be >= 0 (0: unknown)");
    if (a->workspace) {
        const int64_t need = dsalt::select_workspace_bytes(a->total_len, a->num_seqs, a->n_heads, a->k_lmk);
        if (a->workspace_bytes < need || !aligned(a->workspace, 16))
            return fail(DSALT_ERR_INVALID, "select workspace needs %lld bytes, 16-byte aligned (got %lld)",
                        (long long)need, (long long)a->workspace_bytes);
    }
    return DSALT_OK;
}

}  // namespace

int dsalt_select_check(const dsalt_select_args *a) { return check_select(a, false); }

int64_t dsalt_select_workspace_size(int32_t total_len, int32_t num_seqs, int32_t n_heads, int32_t k_lmk) {
    if (total_len < 0 || num_seqs < 1 || n_heads < 1 || k_lmk < 0 || k_lmk > DSALT_MAX_K_LMK) return -1;
    return dsalt::select_workspace_bytes(total_len, num_seqs, n_heads, k_lmk);
}

int dsalt_select_landmarks(const dsalt_select_args *a, void *stream) {
    int rc = dsalt_select_check(a);
    if (rc) return rc;
    hipError_t e = dsalt::launch_select(*a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return fail(DSALT_ERR_LAUNCH, "dsalt_select_landmarks launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int64_t dsalt_scores_workspace_size(int32_t total_len, int32_t n_kv_heads) {
    if (total_len < 0 || n_kv_heads < 1) return -1;
    return dsalt::scores_workspace_bytes(total_len, n_kv_heads);
}

namespace {

// hybrid: dsalt_select_hybrid, which writes no scores (scores, z_x and z_v must be NULL)
int check_scores(const dsalt_scores_args *a, bool hybrid) {
    if (!a) return fail(DSALT_ERR_INVALID, "args is NULL");
    if (a->total_len < 0) return fail(DSALT_ERR_INVALID, "total_len must be >= 0");
    if (a->d_model < 1 || a->head_dim < 1 || a->n_heads < 1 || a->n_kv_heads < 1)
        return fail(DSALT_ERR_INVALID, "d_model, head_dim, n_heads and n_kv_heads must be >= 1");
    if (a->n_heads % a->n_kv_heads)
        return fail(DSALT_ERR_INVALID, "n_kv_heads (%d) must divide n_heads (%d)", a->n_kv_heads, a->n_heads);
    if (a->n_kv_heads > dsalt::scores_max_kv())
        return fail(DSALT_ERR_UNSUPPORTED, "n_kv_heads must be <= %d (got %d)", dsalt::scores_max_kv(), a->n_kv_heads);
    for (int dt : {a->x_dtype, a->v_dtype})
        if (dt != DSALT_DTYPE_BF16 && dt != DSALT_DTYPE_F16 && dt != DSALT_DTYPE_F32)
            return fail(DSALT_ERR_INVALID, "x_dtype and v_dtype must be DSALT_DTYPE_BF16, _F16 or _F32 (got %d, %d)",
                        a->x_dtype, a->v_dtype);
    const int ex = a->x_dtype == DSALT_DTYPE_F32 ? 4 : 8;  // elements per 16-byte load
    const int ev = a->v_dtype == DSALT_DTYPE_F32 ? 4 : 8;
    if (a->d_model % ex || a->head_dim % ev)
        return fail(DSALT_ERR_UNSUPPORTED, "d_model (%d) and head_dim (%d) must be multiples of %d and %d",
                    a->d_model, a->head_dim, ex, ev);
    const int g = a->head_dim / ev;
    if (g > 64 || (g & (g - 1)))
        return fail(DSALT_ERR_UNSUPPORTED, "head_dim / %d must be a power of two <= 64 (head_dim %d)", ev, a->head_dim);
    if (hybrid && (a->scores || a->z_x || a->z_v))
        return fail(DSALT_ERR_INVALID, "dsalt_select_hybrid writes no scores: scores, z_x and z_v must be NULL");
    if (hybrid && !a->alpha) return fail(DSALT_ERR_INVALID, "alpha must be non-NULL");
    if (!a->gate_w && (a->gate_b || a->gate_out))
        return fail(DSALT_ERR_INVALID, "gate_b and gate_out need gate_w");
    if (a->gate_w && a->x_dtype == DSALT_DTYPE_F32)
        return fail(DSALT_ERR_UNSUPPORTED, "the window-gate logit needs 16-bit x (x_dtype BF16 or F16)");
    if (a->total_len == 0) return DSALT_OK;
    if (!a->x || !a->v || !a->alpha || (!a->scores && !hybrid))
        return fail(DSALT_ERR_INVALID, "x, v, alpha and scores must be non-NULL");
    if (!aligned(a->x, 16) || !aligned(a->v, 16)) return fail(DSALT_ERR_INVALID, "x and v must be 16-byte aligned");
    if (a->x_stride_t < a->d_model || a->x_stride_t % ex)
        return fail(DSALT_ERR_INVALID, "x row stride (%lld) must be >= d_model and a multiple of %d",
                    (long long)a->x_stride_t, ex);
    if (a->v_stride_t < 0 || a->v_stride_h < 0 || a->v_stride_t % ev || a->v_stride_h % ev)
        return fail(DSALT_ERR_INVALID, "v strides (t=%lld, h=%lld) must be non-negative multiples of %d",
                    (long long)a->v_stride_t, (long long)a->v_stride_h, ev);
    if (a->scores_stride_t < 0 || a->scores_stride_h < 0 || (a->z_v && (a->z_v_stride_t < 0 || a->z_v_stride_h < 0)))
        return fail(DSALT_ERR_INVALID, "output strides must be non-negative");
    const int64_t need = dsalt::scores_workspace_bytes(a->total_len, a->n_kv_heads);
    if (!a->workspace) return fail(DSALT_ERR_INVALID, "workspace is NULL (%lld bytes needed)", (long long)need);
    if (a->workspace_bytes < need)
        return fail(DSALT_ERR_INVALID, "workspace too small: %lld < %lld bytes", (long long)a->workspace_bytes,
                    (long long)need);
    if (!aligned(a->workspace, 256)) return fail(DSALT_ERR_INVALID, "workspace must be 256-byte aligned");
    if (a->k) {  // RoPE of k riding along: dsalt_rope's rules for k alone
        if (!a->k_out || !a->rope_cos || !a->rope_sin)
            return fail(DSALT_ERR_INVALID, "k needs k_out, rope_cos and rope_sin");
        if (a->head_dim % 2) return fail(DSALT_ERR_INVALID, "head_dim must be even for RoPE (got %d)", a->head_dim);
        if (a->rope_rows < 1 || a->rope_stride < a->head_dim)
            return fail(DSALT_ERR_INVALID, "rope tables need >= 1 row of >= head_dim entries");
        if (a->cu_seqlens && a->num_seqs < 1) return fail(DSALT_ERR_INVALID, "num_seqs must be >= 1 with cu_seqlens");
        const int ev = a->v_dtype == DSALT_DTYPE_F32 ? 4 : 8;
        if (!aligned(a->k, 16) || !aligned(a->k_out, 16) || a->k_stride_t % ev || a->k_stride_h % ev ||
            a->k_out_stride_t % ev || a->k_out_stride_h % ev || (a->head_dim / 2) % ev)
            return fail(DSALT_ERR_INVALID, "k / k_out must be 16-byte aligned with strides and head_dim / 2 multiples of %d",
                        ev);
        if (!aligned(a->rope_cos, 16) || !aligned(a->rope_sin, 16) || a->rope_stride % 4)
            return fail(DSALT_ERR_INVALID, "rope tables must be 16-byte aligned with a row stride multiple of 4");
    }
    if (a->gate_w) {
        if (!a->gate_out) return fail(DSALT_ERR_INVALID, "gate_w needs gate_out");
        if (!aligned(a->gate_w, 16) || !aligned(a->gate_out, 2) || !aligned(a->gate_b, 2))
            return fail(DSALT_ERR_INVALID, "gate_w must be 16-byte aligned, gate_b and gate_out 2-byte aligned");
    }
    return DSALT_OK;
}

}  // namespace

int dsalt_scores_check(const dsalt_scores_args *a) { return check_scores(a, false); }

int dsalt_hybrid_scores(const dsalt_scores_args *a, void *stream) {
    int rc = dsalt_scores_check(a);
    if (rc) return rc;
    hipError_t e = dsalt::launch_scores(*a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return fail(DSALT_ERR_LAUNCH, "dsalt_hybrid_scores launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int dsalt_select_hybrid(const dsalt_scores_args *sa, const dsalt_select_args *a, void *stream) {
    int rc = check_scores(sa, true);
    if (rc) return rc;
    if ((rc = check_select(a, true))) return rc;
    if (sa->total_len != a->total_len || sa->n_heads != a->n_heads)
        return fail(DSALT_ERR_INVALID, "score and selection arguments disagree: total_len %d / %d, n_heads %d / %d",
                    sa->total_len, a->total_len, sa->n_heads, a->n_heads);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    dsalt::HybridSrc src;
    hipError_t e = dsalt::launch_norms_for_select(*sa, src, st);
    if (e == hipSuccess) e = dsalt::launch_select(*a, st, &src);
    if (e != hipSuccess) return fail(DSALT_ERR_LAUNCH, "dsalt_select_hybrid launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int dsalt_swiglu(const void *gate, const void *up, void *out, int64_t n, int32_t dtype, void *stream) {
    if (n < 0) return fail(DSALT_ERR_INVALID, "n must be >= 0 (got %lld)", (long long)n);
    if (dtype != DSALT_DTYPE_BF16 && dtype != DSALT_DTYPE_F16 && dtype != DSALT_DTYPE_F32)
        return fail(DSALT_ERR_INVALID, "dtype must be DSALT_DTYPE_BF16, _F16 or _F32 (got %d)", dtype);
    const int per = dtype == DSALT_DTYPE_F32 ? 4 : 8;  // elements per 16-byte access
    if (n % per) return fail(DSALT_ERR_UNSUPPORTED, "n must be a multiple of %d (got %lld)", per, (long long)n);
    if (n == 0) return DSALT_OK;
    if (!gate || !up || !out) return fail(DSALT_ERR_INVALID, "gate, up and out must be non-NULL");
    if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(out, 16))
        return fail(DSALT_ERR_INVALID, "gate, up and out must be 16-byte aligned");
    hipError_t e = dsalt::launch_swiglu(gate, up, out, n, dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(DSALT_ERR_LAUNCH, "dsalt_swiglu launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int dsalt_add_rms_norm(const void *x, const void *h, void *x_out, void *y, const void *weight, int64_t rows,
                       int32_t d, float eps, int32_t dtype, void *stream) {
    if (rows < 0) return fail(DSALT_ERR_INVALID, "rows must be >= 0 (got %lld)", (long long)rows);
    if (dtype != DSALT_DTYPE_BF16 && dtype != DSALT_DTYPE_F16)
        return fail(DSALT_ERR_INVALID, "dtype must be DSALT_DTYPE_BF16 or _F16 (got %d)", dtype);
    if (d < 8 || d % 8 || d > dsalt::rms_norm_max_dim())
        return fail(DSALT_ERR_UNSUPPORTED, "d must be a multiple of 8 in [8, %d] (got %d)", dsalt::rms_norm_max_dim(), d);
    if (!(eps >= 0.f)) return fail(DSALT_ERR_INVALID, "eps must be >= 0");
    if (h && !x_out) return fail(DSALT_ERR_INVALID, "h needs x_out");
    if (rows == 0) return DSALT_OK;
    if (!x || !y || !weight) return fail(DSALT_ERR_INVALID, "x, y and weight must be non-NULL");
    if (!aligned(x, 16) || !aligned(h, 16) || !aligned(x_out, 16) || !aligned(y, 16) || !aligned(weight, 16))
        return fail(DSALT_ERR_INVALID, "x, h, x_out, y and weight must be 16-byte aligned");
    if (y == x || y == h || (h && y == x_out))
        return fail(DSALT_ERR_INVALID, "y must not alias x, h or x_out");
    hipError_t e = dsalt::launch_add_rms_norm(x, h, h ? x_out : nullptr, y, weight, rows, d, eps, dtype,
                                              static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(DSALT_ERR_LAUNCH, "dsalt_add_rms_norm launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int dsalt_rope_check(const dsalt_rope_args *a) {
    if (!a) return fail(DSALT_ERR_INVALID, "args is NULL");
    if (a->total_len < 0 || a->n_q_heads < 0 || a->n_k_heads < 0)
        return fail(DSALT_ERR_INVALID, "total_len and head counts must be >= 0");
    if (a->head_dim < 2 || a->head_dim % 2) return fail(DSALT_ERR_INVALID, "head_dim must be even and >= 2");
    if (a->dtype != DSALT_DTYPE_BF16 && a->dtype != DSALT_DTYPE_F16 && a->dtype != DSALT_DTYPE_F32)
        return fail(DSALT_ERR_INVALID, "dtype must be DSALT_DTYPE_BF16, _F16 or _F32 (got %d)", a->dtype);
    if (a->transpose != 0 && a->transpose != 1) return fail(DSALT_ERR_INVALID, "transpose must be 0 or 1");
    if (a->total_len == 0) return DSALT_OK;
    if ((a->n_q_heads && (!a->q || !a->q_out)) || (a->n_k_heads && (!a->k || !a->k_out)) || !a->cos || !a->sin)
        return fail(DSALT_ERR_INVALID, "q, k, their outputs, cos and sin must be non-NULL");
    if (a->cos_sin_stride < a->head_dim) return fail(DSALT_ERR_INVALID, "cos_sin_stride must be >= head_dim");
    if (a->table_rows < 1) return fail(DSALT_ERR_INVALID, "table_rows must be >= 1");
    if (!a->cu_seqlens && a->table_rows < a->total_len)
        return fail(DSALT_ERR_INVALID, "per-token tables need total_len (%d) rows (got %d)", a->total_len, a->table_rows);
    if (a->cu_seqlens && a->num_seqs < 1) return fail(DSALT_ERR_INVALID, "num_seqs must be >= 1 with cu_seqlens");
    for (int64_t st : {a->q_stride_t, a->q_stride_h, a->k_stride_t, a->k_stride_h, a->q_out_stride_t,
                       a->q_out_stride_h, a->k_out_stride_t, a->k_out_stride_h})
        if (st < 0) return fail(DSALT_ERR_INVALID, "strides must be non-negative");
    return DSALT_OK;
}

int dsalt_rope(const dsalt_rope_args *a, void *stream) {
    int rc = dsalt_rope_check(a);
    if (rc) return rc;
    hipError_t e = dsalt::launch_rope(*a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(DSALT_ERR_LAUNCH, "dsalt_rope launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int dsalt_quantize_windows(const float *w_cont, int64_t n, float *w_out, int32_t *w_int_out,
                           void *stream) {
    if (n < 0) return fail(DSALT_ERR_INVALID, "n must be >= 0");
    if (n > 0 && !w_cont) return fail(DSALT_ERR_INVALID, "w_cont is NULL");
    hipError_t e = dsalt::launch_quantize(w_cont, n, w_out, w_int_out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return fail(DSALT_ERR_LAUNCH, "dsalt_quantize_windows launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int64_t dsalt_bwd_workspace_size(int32_t total_len, int32_t num_seqs, int32_t n_heads,
                                 int32_t head_dim, int32_t k_lmk) {
    if (total_len < 0 || num_seqs < 1 || n_heads < 1 || k_lmk < 0) return -1;
    return dsalt::bwd_workspace_bytes(total_len, num_seqs, n_heads, head_dim, k_lmk);
}

int dsalt_bwd_check(const dsalt_bwd_args *a) {
    if (!a) return fail(DSALT_ERR_INVALID, "args is NULL");
    int rc = check_common(a->mode, a->dtype, a->total_len, a->num_seqs, a->n_heads, a->head_dim,
                          a->k_lmk, a->cu_seqlens, a->w, a->lmk_pos);
    if (rc) return rc;
    if ((rc = check_tensor("q", a->q, a->q_stride_t, a->q_stride_h, 8))) return rc;
    if ((rc = check_tensor("k", a->k, a->k_stride_t, a->k_stride_h, 8))) return rc;
    if ((rc = check_tensor("v", a->v, a->v_stride_t, a->v_stride_h, 8))) return rc;
    if (a->out_dtype != a->dtype && a->out_dtype != DSALT_DTYPE_F32)
        return fail(DSALT_ERR_INVALID, "out_dtype must equal dtype or be DSALT_DTYPE_F32 (got %d)", a->out_dtype);
    {  // O rows are read 8 elements at a time (16 bytes in 16-bit types, 32 in fp32)
        const int64_t m = a->out_dtype == DSALT_DTYPE_F32 ? 2 : 1;
        if ((rc = check_tensor("out", a->out, a->out_stride_t * m, a->out_stride_h * m, 8))) return rc;
    }
    if ((rc = check_tensor("dout", a->dout, a->dout_stride_t, a->dout_stride_h, 8))) return rc;
    if (a->grad_dtype != a->dtype && a->grad_dtype != DSALT_DTYPE_F32)
        return fail(DSALT_ERR_INVALID, "grad_dtype must equal dtype or be DSALT_DTYPE_F32 (got %d)", a->grad_dtype);
    // gradient rows are written 4 elements at a time (8 bytes in 16-bit types, 16 in fp32)
    const int gv = a->grad_dtype == DSALT_DTYPE_F32 ? 8 : 4;  // check_tensor counts 16-bit elements
    const int64_t gm = a->grad_dtype == DSALT_DTYPE_F32 ? 2 : 1;
    if ((rc = check_tensor("dq", a->dq, a->dq_stride_t * gm, a->dq_stride_h * gm, gv))) return rc;
    if ((rc = check_tensor("dk", a->dk, a->dk_stride_t * gm, a->dk_stride_h * gm, gv))) return rc;
    if ((rc = check_tensor("dv", a->dv, a->dv_stride_t * gm, a->dv_stride_h * gm, gv))) return rc;
    if (!a->lse) return fail(DSALT_ERR_INVALID, "lse is NULL");
    if ((rc = check_mode_scalars(a->mode, a->scale, a->tau_win, a->win_edge))) return rc;
    if ((rc = check_kv_heads(a->n_heads, a->n_kv_heads))) return rc;
    const int64_t need = a->mode == DSALT_MODE_DENSE
                             ? dsalt::dense_bwd_workspace_bytes(a->total_len, a->n_heads)
                             : dsalt::bwd_workspace_bytes(a->total_len, a->num_seqs, a->n_heads, a->head_dim,
                                                          a->k_lmk);
    if (need > 0) {
        if (!a->workspace) return fail(DSALT_ERR_INVALID, "workspace is NULL (%lld bytes needed)", (long long)need);
        if (a->workspace_bytes < need)
            return fail(DSALT_ERR_INVALID, "workspace too small: %lld < %lld bytes",
                        (long long)a->workspace_bytes, (long long)need);
        if (!aligned(a->workspace, 256)) return fail(DSALT_ERR_INVALID, "workspace must be 256-byte aligned");
    }
    const int64_t ob = a->out_dtype == DSALT_DTYPE_F32 ? 4 : 2;
    return check_span32(a->total_len, {2 * a->q_stride_t, 2 * a->k_stride_t, 2 * a->v_stride_t,
                                       2 * a->dout_stride_t, ob * a->out_stride_t});
}

int dsalt_bwd(const dsalt_bwd_args *a, void *stream) {
    int rc = dsalt_bwd_check(a);
    if (rc) return rc;
    hipError_t e = dsalt::launch_bwd(*a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(DSALT_ERR_LAUNCH, "dsalt_bwd launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

int dsalt_bwd_noalloc(const dsalt_bwd_args *a, void *stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "args is NULL");
    const int64_t need = dsalt_bwd_workspace_size(a->total_len, a->num_seqs, a->n_heads, a->head_dim, a->k_lmk);
    if (need < 0) return fail(DSALT_ERR_INVALID, "invalid sizes (total_len, num_seqs, n_heads, k_lmk)");
    if (need > DSALT_NOALLOC_SCRATCH_BYTES)
        return fail(DSALT_ERR_UNSUPPORTED,
                    "dsalt_bwd_noalloc: this call needs %lld bytes of scratch, above the static %lld "
                    "(use dsalt_bwd with a caller workspace)",
                    (long long)need, (long long)DSALT_NOALLOC_SCRATCH_BYTES);
    void *scratch_ptr = nullptr;
    int rc = scratch_address(&scratch_ptr);
    if (rc) return rc;
    dsalt_bwd_args b = *a;
    b.workspace = scratch_ptr;
    b.workspace_bytes = DSALT_NOALLOC_SCRATCH_BYTES;
    if ((rc = dsalt_bwd_check(&b))) return rc;
    hipError_t e = dsalt::launch_bwd(b, static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return fail(DSALT_ERR_LAUNCH, "dsalt_bwd_noalloc launch failed: %s", hipGetErrorString(e));
    return DSALT_OK;
}

}  // extern "C"
