"""ctypes binding of libdsalt_hip.so (the gfx950 HIP kernels behind the DSALT API).

The structures below mirror include/dsalt_hip.h field by field; ``check_abi()``
compares their sizes with the library's own ``sizeof``. Every call runs on the
current torch stream of the tensors' device and never synchronises. There is no
fallback: a missing library or a non-GPU tensor raises ``DsaltError``.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p

import torch

# the in-tree build; DSALT_HIP_LIB names another copy of the library
LIB_PATH = os.environ.get("DSALT_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                           "libdsalt_hip.so")

DSALT_OK = 0
MODE_HARD = 0
MODE_SOFT = 1
MODE_DENSE = 2
DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2
MAX_K_LMK = 1024
ABI_VERSION = 3

_DTYPES = {torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}


class DsaltError(RuntimeError):
    """Raised for invalid arguments, a missing library or a failed launch."""


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("mode", c_int32), ("dtype", c_int32), ("total_len", c_int32), ("num_seqs", c_int32),
        ("n_heads", c_int32), ("head_dim", c_int32), ("k_lmk", c_int32), ("out_dtype", c_int32),
        ("q", c_void_p), ("q_stride_t", c_int64), ("q_stride_h", c_int64),
        ("k", c_void_p), ("k_stride_t", c_int64), ("k_stride_h", c_int64),
        ("v", c_void_p), ("v_stride_t", c_int64), ("v_stride_h", c_int64),
        ("out", c_void_p), ("out_stride_t", c_int64), ("out_stride_h", c_int64),
        ("lse", c_void_p), ("lse_stride_t", c_int64), ("lse_stride_h", c_int64),
        ("w", c_void_p), ("w_stride", c_int64),
        ("lmk_pos", c_void_p), ("lmk_pos_stride_h", c_int64), ("lmk_pos_stride_s", c_int64),
        ("lmk_pos_stride_k", c_int64),
        ("lmk_bias", c_void_p), ("lmk_bias_stride_h", c_int64), ("lmk_bias_stride_s", c_int64),
        ("lmk_bias_stride_k", c_int64),
        ("cu_seqlens", c_void_p),
        ("scale", c_float), ("tau_win", c_float), ("win_edge", c_float), ("n_kv_heads", c_int32),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p), ("rope_stride", c_int64), ("rope_rows", c_int32),
        ("rope_half", c_int32),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("mode", c_int32), ("dtype", c_int32), ("total_len", c_int32), ("num_seqs", c_int32),
        ("n_heads", c_int32), ("head_dim", c_int32), ("k_lmk", c_int32), ("grad_dtype", c_int32),
        ("out_dtype", c_int32), ("n_kv_heads", c_int32),
        ("q", c_void_p), ("q_stride_t", c_int64), ("q_stride_h", c_int64),
        ("k", c_void_p), ("k_stride_t", c_int64), ("k_stride_h", c_int64),
        ("v", c_void_p), ("v_stride_t", c_int64), ("v_stride_h", c_int64),
        ("out", c_void_p), ("out_stride_t", c_int64), ("out_stride_h", c_int64),
        ("lse", c_void_p), ("lse_stride_t", c_int64), ("lse_stride_h", c_int64),
        ("dout", c_void_p), ("dout_stride_t", c_int64), ("dout_stride_h", c_int64),
        ("w", c_void_p), ("w_stride", c_int64),
        ("lmk_pos", c_void_p), ("lmk_pos_stride_h", c_int64), ("lmk_pos_stride_s", c_int64),
        ("lmk_pos_stride_k", c_int64),
        ("lmk_bias", c_void_p), ("lmk_bias_stride_h", c_int64), ("lmk_bias_stride_s", c_int64),
        ("lmk_bias_stride_k", c_int64),
        ("cu_seqlens", c_void_p),
        ("dq", c_void_p), ("dq_stride_t", c_int64), ("dq_stride_h", c_int64),
        ("dk", c_void_p), ("dk_stride_t", c_int64), ("dk_stride_h", c_int64),
        ("dv", c_void_p), ("dv_stride_t", c_int64), ("dv_stride_h", c_int64),
        ("d_lmk_bias", c_void_p), ("d_w", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_int64),
        ("scale", c_float), ("tau_win", c_float), ("win_edge", c_float), ("reserved1", c_float),
    ]


class SelectArgs(ctypes.Structure):
    _fields_ = [
        ("total_len", c_int32), ("num_seqs", c_int32), ("n_heads", c_int32), ("k_lmk", c_int32),
        ("scores", c_void_p), ("scores_stride_t", c_int64), ("scores_stride_h", c_int64),
        ("w", c_void_p), ("w_stride", c_int64),
        ("cu_seqlens", c_void_p),
        ("lmk_pos", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_int64),
        ("max_seqlen", c_int32),
        ("w_out", c_void_p),
        ("w_logit", c_void_p), ("w_logit_stride", c_int64), ("w_logit_dtype", c_int32),
        ("n_min", c_float), ("n_max", c_float),
    ]


class ScoresArgs(ctypes.Structure):
    _fields_ = [
        ("total_len", c_int32), ("d_model", c_int32), ("n_kv_heads", c_int32), ("head_dim", c_int32),
        ("n_heads", c_int32), ("x_dtype", c_int32), ("v_dtype", c_int32), ("norms_f32", c_int32),
        ("x", c_void_p), ("x_stride_t", c_int64),
        ("v", c_void_p), ("v_stride_t", c_int64), ("v_stride_h", c_int64),
        ("alpha", c_void_p),
        ("scores", c_void_p), ("scores_stride_t", c_int64), ("scores_stride_h", c_int64),
        ("z_x", c_void_p),
        ("z_v", c_void_p), ("z_v_stride_t", c_int64), ("z_v_stride_h", c_int64),
        ("workspace", c_void_p), ("workspace_bytes", c_int64),
        ("k", c_void_p), ("k_stride_t", c_int64), ("k_stride_h", c_int64),
        ("k_out", c_void_p), ("k_out_stride_t", c_int64), ("k_out_stride_h", c_int64),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p), ("rope_stride", c_int64),
        ("rope_rows", c_int32), ("num_seqs", c_int32),
        ("cu_seqlens", c_void_p),
        ("gate_w", c_void_p), ("gate_b", c_void_p), ("gate_out", c_void_p),
    ]


class RopeArgs(ctypes.Structure):
    _fields_ = [
        ("total_len", c_int32), ("num_seqs", c_int32), ("n_q_heads", c_int32), ("n_k_heads", c_int32),
        ("head_dim", c_int32), ("dtype", c_int32), ("transpose", c_int32), ("table_rows", c_int32),
        ("q", c_void_p), ("q_stride_t", c_int64), ("q_stride_h", c_int64),
        ("k", c_void_p), ("k_stride_t", c_int64), ("k_stride_h", c_int64),
        ("q_out", c_void_p), ("q_out_stride_t", c_int64), ("q_out_stride_h", c_int64),
        ("k_out", c_void_p), ("k_out_stride_t", c_int64), ("k_out_stride_h", c_int64),
        ("cos", c_void_p), ("sin", c_void_p), ("cos_sin_stride", c_int64),
        ("cu_seqlens", c_void_p),
    ]


EXPORTED_SYMBOLS = (
    "dsalt_fwd", "dsalt_fwd_check", "dsalt_bwd", "dsalt_bwd_check", "dsalt_bwd_workspace_size",
    "dsalt_select_landmarks", "dsalt_select_check", "dsalt_quantize_windows",
    "dsalt_abi_version", "dsalt_last_error", "dsalt_fwd_args_size", "dsalt_bwd_args_size",
    "dsalt_select_args_size", "dsalt_hybrid_scores", "dsalt_scores_check", "dsalt_scores_workspace_size",
    "dsalt_scores_args_size", "dsalt_rope", "dsalt_rope_check", "dsalt_rope_args_size",
    "dsalt_bwd_noalloc", "dsalt_select_workspace_size", "dsalt_select_hybrid", "dsalt_swiglu",
    "dsalt_add_rms_norm",
)
NOALLOC_SCRATCH_BYTES = 76 << 20  # DSALT_NOALLOC_SCRATCH_BYTES
SELECT_SPLIT_MIN = 4096  # longer sequences can be selected chunk-wise

_lib = None


def lib() -> ctypes.CDLL:
    """Load libdsalt_hip.so once; raise DsaltError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise DsaltError(
            f"{LIB_PATH} is missing: build it with `python dsalt-library_amd/build.py` "
            "(the DSALT path has no non-HIP fallback)")
    h = ctypes.CDLL(LIB_PATH)
    for name, argtypes in (
        ("dsalt_fwd", [ctypes.POINTER(FwdArgs), c_void_p]),
        ("dsalt_fwd_check", [ctypes.POINTER(FwdArgs)]),
        ("dsalt_bwd", [ctypes.POINTER(BwdArgs), c_void_p]),
        ("dsalt_bwd_check", [ctypes.POINTER(BwdArgs)]),
        ("dsalt_bwd_noalloc", [ctypes.POINTER(BwdArgs), c_void_p]),
        ("dsalt_select_landmarks", [ctypes.POINTER(SelectArgs), c_void_p]),
        ("dsalt_select_check", [ctypes.POINTER(SelectArgs)]),
        ("dsalt_hybrid_scores", [ctypes.POINTER(ScoresArgs), c_void_p]),
        ("dsalt_scores_check", [ctypes.POINTER(ScoresArgs)]),
        ("dsalt_select_hybrid", [ctypes.POINTER(ScoresArgs), ctypes.POINTER(SelectArgs), c_void_p]),
        ("dsalt_rope", [ctypes.POINTER(RopeArgs), c_void_p]),
        ("dsalt_rope_check", [ctypes.POINTER(RopeArgs)]),
        ("dsalt_quantize_windows", [c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
        ("dsalt_swiglu", [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
        ("dsalt_add_rms_norm", [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_float, c_int32,
                                c_void_p]),
    ):
        fn = getattr(h, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    h.dsalt_bwd_workspace_size.argtypes = [c_int32] * 5
    h.dsalt_bwd_workspace_size.restype = c_int64
    h.dsalt_scores_workspace_size.argtypes = [c_int32] * 2
    h.dsalt_scores_workspace_size.restype = c_int64
    h.dsalt_select_workspace_size.argtypes = [c_int32] * 4
    h.dsalt_select_workspace_size.restype = c_int64
    h.dsalt_abi_version.restype = ctypes.c_int
    h.dsalt_last_error.restype = ctypes.c_char_p
    for n in ("dsalt_fwd_args_size", "dsalt_bwd_args_size", "dsalt_select_args_size", "dsalt_scores_args_size",
              "dsalt_rope_args_size"):
        getattr(h, n).restype = c_size_t
    _lib = h
    check_abi()
    return h


def check_abi() -> None:
    h = lib()
    if h.dsalt_abi_version() != ABI_VERSION:
        raise DsaltError(f"ABI version mismatch: library {h.dsalt_abi_version()} vs binding {ABI_VERSION}")
    for struct, fn in ((FwdArgs, h.dsalt_fwd_args_size), (BwdArgs, h.dsalt_bwd_args_size),
                       (SelectArgs, h.dsalt_select_args_size), (ScoresArgs, h.dsalt_scores_args_size),
                       (RopeArgs, h.dsalt_rope_args_size)):
        if ctypes.sizeof(struct) != fn():
            raise DsaltError(f"{struct.__name__} layout mismatch: {ctypes.sizeof(struct)} vs {fn()} bytes")


def _raise(rc: int, what: str) -> None:
    if rc != DSALT_OK:
        msg = lib().dsalt_last_error().decode(errors="replace")
        raise DsaltError(f"{what} failed (code {rc}): {msg}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise DsaltError(
                f"the DSALT HIP path needs tensors on a ROCm GPU, got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise DsaltError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise DsaltError("no tensor given")
    return dev


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def compute_dtype(dtype: torch.dtype) -> torch.dtype:
    """bf16/fp16 compute as is; anything else computes in fp16, as the reference's
    kernels do (dsalt/kernels/dsalt_triton_attn.py:266)."""
    return dtype if dtype in _DTYPES else torch.float16


def as_kernel_operand(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """[T,H,D] operand with unit stride on D, 16-byte aligned rows (copy only if needed)."""
    if t.dtype != dtype:
        t = t.to(dtype)
    ok = (t.dim() == 3 and t.stride(2) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0
          and t.data_ptr() % 16 == 0)
    return t if ok else t.contiguous()


_ROPE_TABLES = {}


def rope_tables(cos: torch.Tensor, sin: torch.Tensor):
    """(cos, sin) as contiguous fp32 tables and whether every row repeats its first half in
    its second (tables built as cat(freqs, freqs): the kernel then reads half of each row).
    Cached per source storage and version, so a module's tables are converted and checked
    once, not on every forward (the check synchronises)."""
    key = (cos.data_ptr(), sin.data_ptr(), tuple(cos.shape), cos.dtype, cos._version, sin._version)
    hit = _ROPE_TABLES.get(key)
    if hit is None:
        c32, s32 = cos.to(torch.float32).contiguous(), sin.to(torch.float32).contiguous()
        h = c32.shape[-1] // 2
        half = c32.dim() == 2 and bool(torch.equal(c32[:, :h], c32[:, h:])) and bool(torch.equal(s32[:, :h], s32[:, h:]))
        if len(_ROPE_TABLES) > 64:
            _ROPE_TABLES.clear()
        hit = _ROPE_TABLES[key] = (c32, s32, half, (cos, sin))  # the sources stay alive with the key
    return hit[0], hit[1], hit[2]


def kv_heads(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> int:
    """Number of K/V heads of q [T, H, D], k / v [T, n_kv, D] (n_kv divides H: query head h
    reads K/V head h // (H // n_kv)); validates the shapes and dtypes."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise DsaltError(f"q/k/v must be [T, H, D], got {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    T, H, D = q.shape
    n_kv = k.shape[1]
    if k.shape != v.shape or k.shape[0] != T or k.shape[2] != D or n_kv < 1 or H % n_kv:
        raise DsaltError(f"k/v must be [T, n_kv, D] with n_kv dividing H = {H}: q {tuple(q.shape)}, "
                         f"k {tuple(k.shape)}, v {tuple(v.shape)}")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise DsaltError(f"q/k/v must share a bf16/fp16 dtype, got {q.dtype} {k.dtype} {v.dtype}")
    return n_kv


def group_sum(g: torch.Tensor, n_kv: int) -> torch.Tensor:
    """Per-query-head gradients [T, H, D] summed over each group of H // n_kv heads ->
    [T, n_kv, D] (the gradient of a K/V head that several query heads share)."""
    T, H, D = g.shape
    return g if n_kv == H else g.view(T, n_kv, H // n_kv, D).sum(2)


def _f32_vec(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.float32 else t.float()


def _cu_i32(cu: torch.Tensor) -> torch.Tensor:
    if cu.dtype != torch.int32 or not cu.is_contiguous():
        cu = cu.to(torch.int32).contiguous()
    return cu


def fwd(mode: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, w: torch.Tensor,
        lmk_pos: torch.Tensor | None, lmk_bias: torch.Tensor | None, cu_seqlens: torch.Tensor,
        scale: float, tau_win: float = 1.0, win_edge: float = 4.0,
        out: torch.Tensor | None = None, lse: torch.Tensor | None = None,
        out_dtype: torch.dtype | None = None, rope: tuple | None = None):
    """Sparse-attention forward. q/k/v must already be kernel operands (see
    ``as_kernel_operand``). ``rope = (cos, sin)`` (fp32 tables [rows, D], rows = positions
    inside a sequence) rotates the un-rotated q on load; k must be rotated already.
    Returns (out [T,H,D] in ``out_dtype`` (q.dtype or float32, default q.dtype, or the
    dtype of a given ``out``), lse [T,H] fp32)."""
    launcher = FwdLauncher(mode, q, k, v, w, lmk_pos, lmk_bias, cu_seqlens, scale, tau_win, win_edge,
                           out, lse, out_dtype, rope)
    launcher()
    return launcher.out, launcher.lse


class FwdLauncher:
    """A forward launch with its argument block built once; calling it re-launches on
    the current stream with the same buffers (used for repeated timing and replay)."""

    def __init__(self, mode: int, q, k, v, w, lmk_pos, lmk_bias, cu_seqlens, scale: float,
                 tau_win: float = 1.0, win_edge: float = 4.0, out=None, lse=None, out_dtype=None, rope=None):
        self.args, self._keep, self.out, self.lse, self.device = _fwd_args(
            mode, q, k, v, w, lmk_pos, lmk_bias, cu_seqlens, scale, tau_win, win_edge, out, lse, out_dtype, rope)
        self._fn = lib().dsalt_fwd
        self._ref = ctypes.byref(self.args)

    def __call__(self) -> None:
        _raise(self._fn(self._ref, stream_handle(self.device)), "dsalt_fwd")


def _fwd_args(mode, q, k, v, w, lmk_pos, lmk_bias, cu_seqlens, scale, tau_win, win_edge, out, lse, out_dtype,
              rope=None):
    dev = require_gpu(q, k, v, w, cu_seqlens)
    T, H, D = q.shape
    n_kv = kv_heads(q, k, v)
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise DsaltError(f"q/k/v must share a bf16/fp16 dtype, got {q.dtype} {k.dtype} {v.dtype}")
    cu = _cu_i32(cu_seqlens)
    S = cu.shape[0] - 1
    w = _f32_vec(w)
    if w.dim() != 1 or w.shape[0] != T:
        raise DsaltError(f"w must be [T={T}], got {tuple(w.shape)}")
    kl = 0
    if lmk_pos is not None:
        if lmk_pos.dim() != 3 or lmk_pos.shape[0] != H or lmk_pos.shape[1] != S:
            raise DsaltError(f"landmark positions must be [H={H}, S={S}, k], got {tuple(lmk_pos.shape)}")
        if lmk_pos.dtype != torch.int64:
            lmk_pos = lmk_pos.long()
        kl = lmk_pos.shape[2]
        if lmk_bias is not None:
            if lmk_bias.shape != lmk_pos.shape:
                raise DsaltError(f"landmark bias shape {tuple(lmk_bias.shape)} != {tuple(lmk_pos.shape)}")
            lmk_bias = _f32_vec(lmk_bias)
    odt = out.dtype if out is not None else (q.dtype if out_dtype is None else out_dtype)
    if odt not in (q.dtype, torch.float32):
        raise DsaltError(f"out dtype must be {q.dtype} or torch.float32, got {odt}")
    if out is None:
        out = torch.empty((T, H, D), device=dev, dtype=odt)
    if lse is None:
        # [T, H] view of head-major storage: a workgroup (one head, consecutive tokens)
        # then writes its LSE values contiguously
        lse = torch.empty((H, T), device=dev, dtype=torch.float32).t()
    a = FwdArgs()
    a.mode, a.dtype, a.total_len, a.num_seqs = mode, _DTYPES[q.dtype], T, S
    a.n_heads, a.head_dim, a.k_lmk, a.n_kv_heads = H, D, kl, n_kv
    a.out_dtype = DTYPE_F32 if odt == torch.float32 else _DTYPES[q.dtype]
    a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.lse, a.lse_stride_t, a.lse_stride_h = lse.data_ptr(), lse.stride(0), lse.stride(1)
    a.w, a.w_stride = w.data_ptr(), w.stride(0)
    if kl > 0:
        a.lmk_pos = lmk_pos.data_ptr()
        a.lmk_pos_stride_h, a.lmk_pos_stride_s, a.lmk_pos_stride_k = lmk_pos.stride()
        if lmk_bias is not None:
            a.lmk_bias = lmk_bias.data_ptr()
            a.lmk_bias_stride_h, a.lmk_bias_stride_s, a.lmk_bias_stride_k = lmk_bias.stride()
    a.cu_seqlens = cu.data_ptr()
    a.scale, a.tau_win, a.win_edge = float(scale), float(tau_win), float(win_edge)
    cos = sin = None
    if rope is not None:
        require_gpu(*rope)
        cos, sin, half = rope_tables(*rope)
        if cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] != D:
            raise DsaltError(f"RoPE tables must be [rows, {D}] (got {tuple(cos.shape)}, {tuple(sin.shape)})")
        a.rope_cos, a.rope_sin, a.rope_stride, a.rope_rows = cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0]
        a.rope_half = int(half)
    keep = (q, k, v, w, lmk_pos, lmk_bias, cu, out, lse, cos, sin)  # converted tensors must outlive the args
    return a, keep, out, lse, dev


def bwd_workspace_size(T: int, S: int, H: int, D: int, k: int) -> int:
    n = lib().dsalt_bwd_workspace_size(T, S, H, D, k)
    if n < 0:
        raise DsaltError("invalid sizes for dsalt_bwd_workspace_size")
    return int(n)


def bwd(mode: int, q, k, v, out, lse, dout, w, lmk_pos, lmk_bias, cu_seqlens, scale: float,
        tau_win: float = 1.0, win_edge: float = 4.0, need_dw: bool = False,
        grad_dtype: torch.dtype | None = None):
    """Sparse-attention backward. Returns (dq, dk, dv, d_lmk_bias [H,S,k] fp32 or None,
    d_w [T] fp32 or None); dq/dk/dv are [T, H, D] per query head in ``grad_dtype`` (q.dtype
    or torch.float32, default q.dtype): with grouped K/V heads ``group_sum`` gives the K/V
    gradients."""
    launcher = BwdLauncher(mode, q, k, v, out, lse, dout, w, lmk_pos, lmk_bias, cu_seqlens, scale,
                           tau_win, win_edge, need_dw, grad_dtype)
    launcher()
    return launcher.results


class BwdLauncher:
    """A backward launch with its argument block, outputs and workspace built once;
    calling it re-launches on the current stream with the same buffers."""

    def __init__(self, mode: int, q, k, v, out, lse, dout, w, lmk_pos, lmk_bias, cu_seqlens, scale: float,
                 tau_win: float = 1.0, win_edge: float = 4.0, need_dw: bool = False,
                 grad_dtype: torch.dtype | None = None):
        self.args, self._keep, self.results, self.device = _bwd_args(
            mode, q, k, v, out, lse, dout, w, lmk_pos, lmk_bias, cu_seqlens, scale, tau_win, win_edge,
            need_dw, grad_dtype)
        self._fn = lib().dsalt_bwd
        self._ref = ctypes.byref(self.args)

    def __call__(self) -> None:
        _raise(self._fn(self._ref, stream_handle(self.device)), "dsalt_bwd")


def _bwd_args(mode, q, k, v, out, lse, dout, w, lmk_pos, lmk_bias, cu_seqlens, scale, tau_win, win_edge,
              need_dw, grad_dtype):
    dev = require_gpu(q, k, v, out, lse, dout, w, cu_seqlens)
    if q.dim() != 3:
        raise DsaltError(f"q must be [T, H, D], got {tuple(q.shape)}")
    T, H, D = q.shape
    n_kv = kv_heads(q, k, v)
    for name, t in (("out", out), ("dout", dout)):
        if tuple(t.shape) != (T, H, D):
            raise DsaltError(f"{name} shape {tuple(t.shape)} != q shape {(T, H, D)}")
    if k.dtype != q.dtype or v.dtype != q.dtype or q.dtype not in _DTYPES:
        raise DsaltError(f"q/k/v must share a bf16/fp16 dtype, got {q.dtype} {k.dtype} {v.dtype}")
    if tuple(lse.shape) != (T, H) or lse.dtype != torch.float32:
        raise DsaltError(f"lse must be float32 [T={T}, H={H}], got {lse.dtype} {tuple(lse.shape)}")
    cu = _cu_i32(cu_seqlens)
    S = cu.shape[0] - 1
    w = _f32_vec(w)
    if w.dim() != 1 or w.shape[0] != T:
        raise DsaltError(f"w must be [T={T}], got {tuple(w.shape)}")
    dout = as_kernel_operand(dout, q.dtype)
    kl = 0 if lmk_pos is None else lmk_pos.shape[-1]
    if lmk_pos is not None:
        if lmk_pos.dim() != 3 or lmk_pos.shape[0] != H or lmk_pos.shape[1] != S:
            raise DsaltError(f"landmark positions must be [H={H}, S={S}, k], got {tuple(lmk_pos.shape)}")
        if lmk_pos.dtype != torch.int64:
            lmk_pos = lmk_pos.long()
    if lmk_bias is not None:
        if lmk_pos is None or lmk_bias.shape != lmk_pos.shape:
            raise DsaltError(f"landmark bias shape {tuple(lmk_bias.shape)} does not match the positions")
        lmk_bias = _f32_vec(lmk_bias)
    gdt = q.dtype if grad_dtype is None else grad_dtype
    if gdt not in (q.dtype, torch.float32):
        raise DsaltError(f"grad_dtype must be {q.dtype} or torch.float32, got {gdt}")
    dq = torch.empty(q.shape, device=dev, dtype=gdt)
    dk = torch.empty(q.shape, device=dev, dtype=gdt)
    dv = torch.empty(q.shape, device=dev, dtype=gdt)
    d_bias = torch.empty((H, S, kl), device=dev, dtype=torch.float32) if kl > 0 else None
    d_w = torch.empty((T,), device=dev, dtype=torch.float32) if need_dw else None
    ws_bytes = bwd_workspace_size(T, S, H, D, kl)
    ws = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    a = BwdArgs()
    a.mode, a.dtype, a.total_len, a.num_seqs = mode, _DTYPES[q.dtype], T, S
    a.n_heads, a.head_dim, a.k_lmk, a.n_kv_heads = H, D, kl, n_kv
    a.grad_dtype = DTYPE_F32 if gdt == torch.float32 else _DTYPES[q.dtype]
    if out.dtype not in (q.dtype, torch.float32):
        raise DsaltError(f"saved output must be {q.dtype} or torch.float32, got {out.dtype}")
    a.out_dtype = DTYPE_F32 if out.dtype == torch.float32 else _DTYPES[q.dtype]
    a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.lse, a.lse_stride_t, a.lse_stride_h = lse.data_ptr(), lse.stride(0), lse.stride(1)
    a.dout, a.dout_stride_t, a.dout_stride_h = dout.data_ptr(), dout.stride(0), dout.stride(1)
    a.w, a.w_stride = w.data_ptr(), w.stride(0)
    if kl > 0:
        a.lmk_pos = lmk_pos.data_ptr()
        a.lmk_pos_stride_h, a.lmk_pos_stride_s, a.lmk_pos_stride_k = lmk_pos.stride()
        if lmk_bias is not None:
            a.lmk_bias = lmk_bias.data_ptr()
            a.lmk_bias_stride_h, a.lmk_bias_stride_s, a.lmk_bias_stride_k = lmk_bias.stride()
        a.d_lmk_bias = d_bias.data_ptr()
    a.cu_seqlens = cu.data_ptr()
    a.dq, a.dq_stride_t, a.dq_stride_h = dq.data_ptr(), dq.stride(0), dq.stride(1)
    a.dk, a.dk_stride_t, a.dk_stride_h = dk.data_ptr(), dk.stride(0), dk.stride(1)
    a.dv, a.dv_stride_t, a.dv_stride_h = dv.data_ptr(), dv.stride(0), dv.stride(1)
    a.d_w = _ptr(d_w)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
    a.scale, a.tau_win, a.win_edge = float(scale), float(tau_win), float(win_edge)
    keep = (q, k, v, out, lse, dout, w, lmk_pos, lmk_bias, cu, ws)  # must outlive the args
    return a, keep, (dq, dk, dv, d_bias, d_w), dev


def _dense_common(q, k, v, w_cont, lmk_bias):
    """Shape and dtype checks shared by the dense-mode forward and backward."""
    T, H, D = q.shape if q.dim() == 3 else (0, 0, 0)
    n_kv = kv_heads(q, k, v)
    w = _f32_vec(w_cont)
    if w.dim() != 1 or w.shape[0] != T:
        raise DsaltError(f"w_cont must be [T={T}], got {tuple(w.shape)}")
    if lmk_bias is not None:
        if tuple(lmk_bias.shape) != (H, T):
            raise DsaltError(f"dense landmark bias must be [H={H}, T={T}], got {tuple(lmk_bias.shape)}")
        lmk_bias = _f32_vec(lmk_bias)
    return T, H, D, n_kv, w, lmk_bias


def dense_fwd(q, k, v, w_cont, lmk_bias, scale: float, tau_win: float = 1.0, win_edge: float = 4.0,
              out_dtype: torch.dtype | None = None):
    """Dense batched forward of one sequence (DSALT_MODE_DENSE): q/k/v [T, H, D] kernel
    operands, w_cont [T], lmk_bias [H, T] fp32 (-inf off the landmarks) or None. Returns
    (out [T, H, D] in ``out_dtype`` (default q.dtype), lse [T, H] fp32)."""
    launcher = DenseFwdLauncher(q, k, v, w_cont, lmk_bias, scale, tau_win, win_edge, out_dtype)
    launcher()
    return launcher.out, launcher.lse


class DenseFwdLauncher:
    """A dense-mode forward with its argument block built once (re-launchable)."""

    def __init__(self, q, k, v, w_cont, lmk_bias, scale: float, tau_win: float = 1.0, win_edge: float = 4.0,
                 out_dtype: torch.dtype | None = None):
        self.device = require_gpu(q, k, v, w_cont, lmk_bias)
        T, H, D, n_kv, w, lb = _dense_common(q, k, v, w_cont, lmk_bias)
        odt = q.dtype if out_dtype is None else out_dtype
        if odt not in (q.dtype, torch.float32):
            raise DsaltError(f"out dtype must be {q.dtype} or torch.float32, got {odt}")
        self.out = torch.empty((T, H, D), device=self.device, dtype=odt)
        self.lse = torch.empty((H, T), device=self.device, dtype=torch.float32).t()
        a = FwdArgs()
        a.mode, a.dtype, a.total_len, a.num_seqs = MODE_DENSE, _DTYPES[q.dtype], T, 1
        a.n_heads, a.head_dim, a.k_lmk, a.n_kv_heads = H, D, 0, n_kv
        a.out_dtype = DTYPE_F32 if odt == torch.float32 else _DTYPES[q.dtype]
        a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
        a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
        a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
        a.out, a.out_stride_t, a.out_stride_h = self.out.data_ptr(), self.out.stride(0), self.out.stride(1)
        a.lse, a.lse_stride_t, a.lse_stride_h = self.lse.data_ptr(), self.lse.stride(0), self.lse.stride(1)
        a.w, a.w_stride = w.data_ptr(), w.stride(0)
        if lb is not None:
            a.lmk_bias = lb.data_ptr()
            a.lmk_bias_stride_h, a.lmk_bias_stride_k = lb.stride(0), lb.stride(1)
        a.scale, a.tau_win, a.win_edge = float(scale), float(tau_win), float(win_edge)
        self.args = a
        self._keep = (q, k, v, w, lb)
        self._fn = lib().dsalt_fwd
        self._ref = ctypes.byref(self.args)

    def __call__(self) -> None:
        _raise(self._fn(self._ref, stream_handle(self.device)), "dsalt_fwd (dense)")


def dense_bwd(q, k, v, out, lse, dout, w_cont, lmk_bias, scale: float, tau_win: float = 1.0,
              win_edge: float = 4.0, need_dw: bool = True, grad_dtype: torch.dtype | None = None):
    """Dense-mode backward. Returns (dq, dk, dv in ``grad_dtype`` (default q.dtype),
    d_lmk_bias [H, T] fp32 or None (when lmk_bias is None), d_w [T] fp32 or None)."""
    launcher = DenseBwdLauncher(q, k, v, out, lse, dout, w_cont, lmk_bias, scale, tau_win, win_edge,
                                need_dw, grad_dtype)
    launcher()
    return launcher.results


class DenseBwdLauncher:
    """A dense-mode backward with its argument block, outputs and workspace built once."""

    def __init__(self, q, k, v, out, lse, dout, w_cont, lmk_bias, scale: float, tau_win: float = 1.0,
                 win_edge: float = 4.0, need_dw: bool = True, grad_dtype: torch.dtype | None = None):
        self.device = require_gpu(q, k, v, out, lse, dout, w_cont, lmk_bias)
        T, H, D, n_kv, w, lb = _dense_common(q, k, v, w_cont, lmk_bias)
        if tuple(out.shape) != (T, H, D) or tuple(dout.shape) != (T, H, D):
            raise DsaltError(f"out/dout must be [{T}, {H}, {D}], got {tuple(out.shape)} {tuple(dout.shape)}")
        if out.dtype not in (q.dtype, torch.float32):
            raise DsaltError(f"saved output must be {q.dtype} or torch.float32, got {out.dtype}")
        if tuple(lse.shape) != (T, H) or lse.dtype != torch.float32:
            raise DsaltError(f"lse must be float32 [T={T}, H={H}], got {lse.dtype} {tuple(lse.shape)}")
        dout = as_kernel_operand(dout, q.dtype)
        gdt = q.dtype if grad_dtype is None else grad_dtype
        if gdt not in (q.dtype, torch.float32):
            raise DsaltError(f"grad_dtype must be {q.dtype} or torch.float32, got {gdt}")
        dev = self.device
        dq = torch.empty(q.shape, device=dev, dtype=gdt)
        dk = torch.empty(q.shape, device=dev, dtype=gdt)
        dv = torch.empty(q.shape, device=dev, dtype=gdt)
        d_lb = torch.empty((H, T), device=dev, dtype=torch.float32) if lb is not None else None
        d_w = torch.empty((T,), device=dev, dtype=torch.float32) if need_dw else None
        ws_bytes = bwd_workspace_size(T, 1, H, D, 0)
        ws = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
        a = BwdArgs()
        a.mode, a.dtype, a.total_len, a.num_seqs = MODE_DENSE, _DTYPES[q.dtype], T, 1
        a.n_heads, a.head_dim, a.k_lmk, a.n_kv_heads = H, D, 0, n_kv
        a.grad_dtype = DTYPE_F32 if gdt == torch.float32 else _DTYPES[q.dtype]
        a.out_dtype = DTYPE_F32 if out.dtype == torch.float32 else _DTYPES[q.dtype]
        a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
        a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
        a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
        a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
        a.lse, a.lse_stride_t, a.lse_stride_h = lse.data_ptr(), lse.stride(0), lse.stride(1)
        a.dout, a.dout_stride_t, a.dout_stride_h = dout.data_ptr(), dout.stride(0), dout.stride(1)
        a.w, a.w_stride = w.data_ptr(), w.stride(0)
        if lb is not None:
            a.lmk_bias = lb.data_ptr()
            a.lmk_bias_stride_h, a.lmk_bias_stride_k = lb.stride(0), lb.stride(1)
            a.d_lmk_bias = d_lb.data_ptr()
        a.dq, a.dq_stride_t, a.dq_stride_h = dq.data_ptr(), dq.stride(0), dq.stride(1)
        a.dk, a.dk_stride_t, a.dk_stride_h = dk.data_ptr(), dk.stride(0), dk.stride(1)
        a.dv, a.dv_stride_t, a.dv_stride_h = dv.data_ptr(), dv.stride(0), dv.stride(1)
        a.d_w = _ptr(d_w)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
        a.scale, a.tau_win, a.win_edge = float(scale), float(tau_win), float(win_edge)
        self.args = a
        self._keep = (q, k, v, out, lse, dout, w, lb, ws)
        self.results = (dq, dk, dv, d_lb, d_w)
        self._fn = lib().dsalt_bwd
        self._ref = ctypes.byref(self.args)

    def __call__(self) -> None:
        _raise(self._fn(self._ref, stream_handle(self.device)), "dsalt_bwd (dense)")


def _select_args(scores, w, cu, k_lmk, out, chunked, max_seqlen=None, w_out=None, gate=None, shape=None):
    """The argument block of one selection and the tensors it points into. scores: fp32
    [T, H], or None with shape = (T, H) (dsalt_select_hybrid forms the scores). chunked:
    pass the workspace, so that long sequences are selected chunk-wise; max_seqlen (a
    bound on the sequence lengths, None: unknown) lets the library skip the chunk stage
    when no sequence is long; w_out (fp32 [T], contiguous): w is the continuous w~ and
    the kernel also writes the quantised windows there; gate = (logits [T], n_min, n_max):
    the windows are formed from the window gate's logits in the launch (w unused)."""
    if scores is not None and scores.dtype != torch.float32:
        raise DsaltError(f"scores must be float32, got {scores.dtype}")
    T, H = scores.shape if scores is not None else shape
    S = cu.shape[0] - 1
    a = SelectArgs()
    a.total_len, a.num_seqs, a.n_heads, a.k_lmk = T, S, H, k_lmk
    if scores is not None:
        a.scores, a.scores_stride_t, a.scores_stride_h = scores.data_ptr(), scores.stride(0), scores.stride(1)
    if w is not None:
        a.w, a.w_stride = w.data_ptr(), w.stride(0)
    if gate is not None:
        logit, n_min, n_max = gate
        if logit.dtype not in (torch.bfloat16, torch.float16) or logit.dim() != 1 or logit.shape[0] != T:
            raise DsaltError(f"window-gate logits must be a [T] bf16 or fp16 vector (got {logit.dtype}, "
                             f"{tuple(logit.shape)})")
        a.w_logit, a.w_logit_stride, a.w_logit_dtype = logit.data_ptr(), logit.stride(0), _SCORE_DTYPES[logit.dtype]
        a.n_min, a.n_max = float(n_min), float(n_max)
    a.cu_seqlens = cu.data_ptr()
    a.lmk_pos = out.data_ptr()
    a.max_seqlen = 0 if max_seqlen is None else min(int(max_seqlen), 2**31 - 1)
    if w_out is not None:
        if w_out.dtype != torch.float32 or w_out.numel() != T or (T > 1 and w_out.stride(0) != 1):
            raise DsaltError("w_out must be a contiguous float32 tensor of total_len entries")
        a.w_out = w_out.data_ptr()
    ws = None
    if chunked and (max_seqlen is None or max_seqlen > SELECT_SPLIT_MIN):
        ws_bytes = lib().dsalt_select_workspace_size(T, S, H, k_lmk)
        if ws_bytes < 0:
            raise DsaltError(f"dsalt_select_workspace_size: invalid shape (T={T}, S={S}, H={H}, k={k_lmk})")
        if ws_bytes > 0:
            ws = torch.empty(ws_bytes, device=out.device, dtype=torch.uint8)
            a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
    return a, (scores, w, cu, out, ws, w_out, gate)


def select_landmarks(scores: torch.Tensor, w: torch.Tensor, cu_seqlens: torch.Tensor,
                     k_lmk: int, chunked: bool = True, max_seqlen: int | None = None) -> torch.Tensor:
    """Top-k landmark positions [H, S, k] int64 (ascending, -1 padded) from fp32 scores [T, H].
    chunked=False selects every sequence with one workgroup per (head, sequence);
    max_seqlen: a bound on the sequence lengths when the caller knows one (None: unknown)."""
    dev = require_gpu(scores, w, cu_seqlens)
    cu = _cu_i32(cu_seqlens)
    w = _f32_vec(w)
    out = torch.empty((scores.shape[1], cu.shape[0] - 1, k_lmk), device=dev, dtype=torch.int64)
    if k_lmk == 0:
        return out
    a, _keep = _select_args(scores, w, cu, k_lmk, out, chunked, max_seqlen)
    _raise(lib().dsalt_select_landmarks(ctypes.byref(a), stream_handle(dev)), "dsalt_select_landmarks")
    return out


def select_landmarks_quantize(scores: torch.Tensor, w_cont: torch.Tensor | None, cu_seqlens: torch.Tensor,
                              k_lmk: int, chunked: bool = True, max_seqlen: int | None = None, gate=None):
    """The window quantisation and the landmark selection in one launch: returns (w [T]
    fp32 = max(1, floor(w~)), NaN kept; landmark positions [H, S, k] as select_landmarks
    returns them for that w). ``gate = (logits [T], n_min, n_max)`` forms w~ = n_min +
    sigmoid(logits) * (n_max - n_min) in the launch, with torch's roundings in the logits'
    16-bit dtype (``w_cont`` is then unused and may be None)."""
    dev = require_gpu(scores, cu_seqlens, w_cont if gate is None else gate[0])
    cu = _cu_i32(cu_seqlens)
    w_cont, gate = _window_source(w_cont, gate)
    out = torch.empty((scores.shape[1], cu.shape[0] - 1, k_lmk), device=dev, dtype=torch.int64)
    w_out = torch.empty(scores.shape[0], device=dev, dtype=torch.float32)
    a, _keep = _select_args(scores, w_cont, cu, k_lmk, out, chunked, max_seqlen, w_out, gate)
    _raise(lib().dsalt_select_landmarks(ctypes.byref(a), stream_handle(dev)), "dsalt_select_landmarks")
    return w_out, out


def _window_source(w_cont, gate):
    """(w_cont as an fp32 vector or None, gate with [T] logits or None)."""
    if gate is None:
        return _f32_vec(w_cont), None
    logit = gate[0]
    if logit.dim() == 2 and logit.shape[1] == 1:
        logit = logit[:, 0]
    return None, (logit, gate[1], gate[2])


def select_hybrid(x: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, n_heads: int,
                  w_cont: torch.Tensor | None, cu_seqlens: torch.Tensor, k_lmk: int, chunked: bool = True,
                  max_seqlen: int | None = None, gate=None, norms_f32: bool | None = None, rope_k=None,
                  gate_linear=None):
    """hybrid_scores followed by select_landmarks_quantize in two launches
    (dsalt_select_hybrid): the selection forms each score from the norms pass's outputs
    instead of reading a [T, H] score tensor, with the same bits. Arguments as for those
    two calls; returns (w [T] fp32 quantised windows, landmark positions [H, S, k],
    rotated k or None when rope_k is None). ``gate_linear = (weight, bias, n_min, n_max)``
    (the window gate's [1, d] weight and [1] bias or None, in x's 16-bit dtype) forms the
    gate's logits in the norms pass (dsalt_scores_args.gate_w) instead of taking them
    from ``gate``; the windows then come from those logits as with ``gate``."""
    f = SelectHybridLauncher(x, v, alpha, n_heads, w_cont, cu_seqlens, k_lmk, chunked, max_seqlen, gate, norms_f32,
                             rope_k, gate_linear)
    f()
    return f.w_out, f.out, f.k_out


def gate_linear_supported(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> bool:
    """Whether the norms pass can form win_gate(x) = x @ weight.T + bias for these operands:
    16-bit x on the GPU, weight [1, d] (or [d]) and bias [1] (or None) in x's dtype on x's
    device, weight contiguous and 16-byte aligned."""
    if x.dtype not in (torch.bfloat16, torch.float16) or x.dim() != 2 or x.device.type != "cuda":
        return False
    w = weight.reshape(-1) if weight.dim() == 2 and weight.shape[0] == 1 else weight
    if (w.dim() != 1 or w.shape[0] != x.shape[1] or w.dtype != x.dtype or w.device != x.device or w.stride(0) != 1
            or w.data_ptr() % 16):
        return False
    return bias is None or (bias.dtype == x.dtype and bias.numel() == 1 and bias.device == x.device)


class SelectHybridLauncher:
    """select_hybrid with its argument blocks, outputs and workspaces built once: each call
    launches the norms pass and the selection on the current stream (for timing loops
    and graph capture); `w_out`, `out` and `k_out` (None without rope_k) hold the result."""

    def __init__(self, x: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, n_heads: int,
                 w_cont: torch.Tensor | None, cu_seqlens: torch.Tensor, k_lmk: int, chunked: bool = True,
                 max_seqlen: int | None = None, gate=None, norms_f32: bool | None = None, rope_k=None,
                 gate_linear=None):
        if norms_f32 is None:
            norms_f32 = autocast_norms()
        if gate_linear is not None and (gate is not None or w_cont is not None):
            raise DsaltError("gate_linear replaces gate and w_cont: pass neither with it")
        self.device = require_gpu(x, v, alpha, cu_seqlens,
                                  gate_linear[0] if gate_linear is not None else w_cont if gate is None else gate[0])
        x, v, alpha = _score_operands(x, v, alpha, n_heads)
        cu = _cu_i32(cu_seqlens)
        T = x.shape[0]
        self.logit = None  # the window gate's logits [T] when gate_linear forms them
        keep_g = None
        if gate_linear is not None:
            weight, bias, n_min, n_max = gate_linear
            if not gate_linear_supported(x, weight, bias):
                raise DsaltError(f"gate_linear needs 16-bit x with a contiguous, 16-byte aligned [1, d] weight and a "
                                 f"[1] bias (or None) of x's dtype (x {x.dtype}, weight {weight.dtype} "
                                 f"{tuple(weight.shape)})")
            self.logit = torch.empty(T, device=self.device, dtype=x.dtype)
            gate = (self.logit, n_min, n_max)
            keep_g = (weight, bias)
        w_cont, gate = _window_source(w_cont, gate)
        ws = torch.empty((scores_workspace_size(T, v.shape[1]),), device=self.device, dtype=torch.uint8)
        self._sa = scores_args(x, v, alpha, n_heads, None, None, None, ws, norms_f32)
        if keep_g is not None:
            self._sa.gate_w = keep_g[0].data_ptr()
            self._sa.gate_b = _ptr(keep_g[1])
            self._sa.gate_out = self.logit.data_ptr()
        self.k_out, keep_k = _rope_k_args(self._sa, v, rope_k)
        self.out = torch.empty((n_heads, cu.shape[0] - 1, k_lmk), device=self.device, dtype=torch.int64)
        self.w_out = torch.empty(T, device=self.device, dtype=torch.float32)
        self._a, keep_s = _select_args(None, w_cont, cu, k_lmk, self.out, chunked, max_seqlen, self.w_out, gate,
                                       shape=(T, n_heads))
        self._keep = (x, v, alpha, cu, ws, keep_k, keep_s, keep_g)
        self._refs = (ctypes.byref(self._sa), ctypes.byref(self._a))
        self._fn = lib().dsalt_select_hybrid

    def __call__(self) -> None:
        _raise(self._fn(*self._refs, stream_handle(self.device)), "dsalt_select_hybrid")


_SCORE_DTYPES = {torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16, torch.float32: DTYPE_F32}


def autocast_norms() -> bool:
    """True when torch's GPU autocast is on: .norm() then runs in fp32 and returns its
    result unrounded, whatever the 16-bit input dtype."""
    try:
        return bool(torch.is_autocast_enabled("cuda"))
    except TypeError:  # torch < 2.4 takes no device type
        return bool(torch.is_autocast_enabled())


def scores_args(x: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, n_heads: int,
                scores: torch.Tensor | None, z_x: torch.Tensor | None, z_v: torch.Tensor | None,
                ws: torch.Tensor | None, norms_f32: bool = False) -> ScoresArgs:
    """Argument block of dsalt_hybrid_scores (x [T, d], v [T, n_kv, D], alpha [H] fp32)."""
    T, d = x.shape
    _, n_kv, D = v.shape
    a = ScoresArgs()
    a.total_len, a.d_model, a.n_kv_heads, a.head_dim, a.n_heads = T, d, n_kv, D, n_heads
    a.norms_f32 = int(bool(norms_f32))
    a.x_dtype = _SCORE_DTYPES.get(x.dtype, -1)
    a.v_dtype = _SCORE_DTYPES.get(v.dtype, -1)
    a.x, a.x_stride_t = x.data_ptr(), x.stride(0)
    a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.alpha = alpha.data_ptr()
    if scores is not None:
        a.scores, a.scores_stride_t, a.scores_stride_h = scores.data_ptr(), scores.stride(0), scores.stride(1)
    a.z_x = _ptr(z_x)
    if z_v is not None:
        a.z_v, a.z_v_stride_t, a.z_v_stride_h = z_v.data_ptr(), z_v.stride(0), z_v.stride(1)
    if ws is not None:
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    return a


def scores_workspace_size(T: int, n_kv: int) -> int:
    n = lib().dsalt_scores_workspace_size(T, n_kv)
    if n < 0:
        raise DsaltError("invalid sizes for dsalt_scores_workspace_size")
    return n


SCORES_MAX_KV = 128  # largest n_kv_heads of dsalt_hybrid_scores


def scores_supported(x: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether dsalt_hybrid_scores takes x [T, d] and v [T, n_kv, D] (dtype and shape rules
    of dsalt_scores_check): bf16 / fp16 / fp32, d and D multiples of one 16-byte load,
    D / (elements per load) a power of two <= 64, n_kv <= 128."""
    if x.dtype not in _SCORE_DTYPES or v.dtype not in _SCORE_DTYPES or x.dim() != 2 or v.dim() != 3:
        return False
    ex = 4 if x.dtype == torch.float32 else 8
    ev = 4 if v.dtype == torch.float32 else 8
    d, n_kv, D = x.shape[1], v.shape[1], v.shape[2]
    g = D // ev
    if not (d % ex == 0 and D % ev == 0 and 0 < g <= 64 and (g & (g - 1)) == 0 and 1 <= n_kv <= SCORES_MAX_KV):
        return False
    # operands as hybrid_scores passes them (a strided last dim is made contiguous there)
    xs = x.stride(0) if x.stride(1) == 1 else d
    vt, vh = (v.stride(0), v.stride(1)) if v.stride(2) == 1 else (n_kv * D, D)
    aligned = (x.stride(1) != 1 or x.data_ptr() % 16 == 0) and (v.stride(2) != 1 or v.data_ptr() % 16 == 0)
    return aligned and xs >= d and xs % ex == 0 and vt >= 0 and vh >= 0 and vt % ev == 0 and vh % ev == 0


def hybrid_scores(x: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, n_heads: int,
                  norms_f32: bool | None = None, rope_k=None):
    """``(scores [T, H], z_x [T], z_v [T, H])`` fp32 of the hybrid landmark score from the
    hidden states x [T, d] and their value projection v = x W_V^T [T, n_kv, D]
    (pre-RoPE), without the GEMM; no gradient (the selection is detached).
    ``norms_f32`` (default: whether autocast is on) keeps the norms of 16-bit inputs in
    fp32 instead of rounding them to the input dtype. ``rope_k = (k, cos, sin,
    cu_seqlens)`` also rotates k [T, n_kv, D] (v's dtype) in the same pass, exactly as
    ``rope`` rotates k alone, and returns the rotated k as a fourth value."""
    if norms_f32 is None:
        norms_f32 = autocast_norms()
    dev = require_gpu(x, v, alpha)
    x, v, alpha = _score_operands(x, v, alpha, n_heads)
    T = x.shape[0]
    scores = torch.empty((T, n_heads), device=dev, dtype=torch.float32)
    z_x = torch.empty((T,), device=dev, dtype=torch.float32)
    z_v = torch.empty((T, n_heads), device=dev, dtype=torch.float32)
    ws = torch.empty((scores_workspace_size(T, v.shape[1]),), device=dev, dtype=torch.uint8)
    a = scores_args(x, v, alpha, n_heads, scores, z_x, z_v, ws, norms_f32)
    k_out, keep = _rope_k_args(a, v, rope_k)
    _raise(lib().dsalt_hybrid_scores(ctypes.byref(a), stream_handle(dev)), "dsalt_hybrid_scores")
    del keep
    if rope_k is not None:
        return scores, z_x, z_v, k_out
    return scores, z_x, z_v


def _score_operands(x, v, alpha, n_heads):
    """x [T, d] and v [T, n_kv, D] with unit inner strides, alpha as a contiguous fp32 [H]."""
    if x.dim() != 2 or v.dim() != 3 or v.shape[0] != x.shape[0]:
        raise DsaltError(f"x must be [T, d] and v [T, n_kv, D] with the same T (got {tuple(x.shape)}, "
                         f"{tuple(v.shape)})")
    if x.dtype not in _SCORE_DTYPES or v.dtype not in _SCORE_DTYPES:
        raise DsaltError(f"x and v must be bf16, fp16 or fp32 (got {x.dtype}, {v.dtype})")
    x = x if x.stride(1) == 1 else x.contiguous()
    v = v if v.stride(2) == 1 else v.contiguous()
    alpha = alpha.detach().to(torch.float32).contiguous()
    if alpha.shape != (n_heads,):
        raise DsaltError(f"alpha must be [{n_heads}] (got {tuple(alpha.shape)})")
    return x, v, alpha


def _rope_k_args(a: ScoresArgs, v: torch.Tensor, rope_k):
    """Fill the k-rotation fields of a score argument block from rope_k = (k, cos, sin,
    cu_seqlens) or leave them empty (rope_k None); returns (k_out or None, tensors to keep
    alive until the launch)."""
    if rope_k is None:
        return None, None
    k, cos, sin, cu = rope_k
    if k.dtype != v.dtype or k.shape != v.shape:
        raise DsaltError(f"k must match v's shape and dtype (got {tuple(k.shape)} {k.dtype}, "
                         f"{tuple(v.shape)} {v.dtype})")
    k = k if k.stride(2) == 1 else k.contiguous()
    k_out = torch.empty_like(k)
    cos = cos.to(torch.float32).contiguous()
    sin = sin.to(torch.float32).contiguous()
    cu = _cu_i32(cu) if cu is not None else None
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.k_out, a.k_out_stride_t, a.k_out_stride_h = k_out.data_ptr(), k_out.stride(0), k_out.stride(1)
    a.rope_cos, a.rope_sin, a.rope_stride, a.rope_rows = cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0]
    a.cu_seqlens = _ptr(cu)
    a.num_seqs = cu.shape[0] - 1 if cu is not None else 1
    return k_out, (k, cos, sin, cu)


def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         cu_seqlens: torch.Tensor | None = None, transpose: bool = False,
         q_out: torch.Tensor | None = None, k_out: torch.Tensor | None = None):
    """Rotary embedding of q [T, Hq, D] and k [T, Hk, D] (half-split) with fp32 tables
    cos/sin [rows, D]: rows are positions inside the sequence when cu_seqlens is given,
    tokens otherwise. ``transpose`` applies the backward rotation. Either of q and k may be
    None (only the other is rotated). Returns (q_out, k_out)."""
    if q is None and k is None:
        raise DsaltError("rope needs q or k")
    ref = q if q is not None else k
    dev = require_gpu(ref, k, cos, sin, cu_seqlens)
    q_only, k_only = k is None, q is None
    q = ref if q is None else q
    k = ref if k is None else k
    if q.dtype != k.dtype or q.dtype not in _SCORE_DTYPES:
        raise DsaltError(f"q and k must share a dtype of bf16, fp16 or fp32 (got {q.dtype}, {k.dtype})")
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise DsaltError(f"q and k must be [T, H, D] with the same T and D (got {tuple(q.shape)}, {tuple(k.shape)})")
    q = q if q.stride(2) == 1 else q.contiguous()
    k = k if k.stride(2) == 1 else k.contiguous()
    cos = cos.to(torch.float32).contiguous()
    sin = sin.to(torch.float32).contiguous()
    if cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] != q.shape[2]:
        raise DsaltError(f"cos and sin must be [rows, {q.shape[2]}] (got {tuple(cos.shape)}, {tuple(sin.shape)})")
    q_out = (torch.empty_like(q) if q_out is None else q_out) if not k_only else q
    k_out = (torch.empty_like(k) if k_out is None else k_out) if not q_only else k
    cu = _cu_i32(cu_seqlens) if cu_seqlens is not None else None
    a = RopeArgs()
    a.total_len, a.head_dim = q.shape[0], q.shape[2]
    a.n_q_heads = 0 if k_only else q.shape[1]
    a.n_k_heads = 0 if q_only else k.shape[1]
    a.num_seqs = cu.shape[0] - 1 if cu is not None else 1
    a.dtype, a.transpose, a.table_rows = _SCORE_DTYPES[q.dtype], int(bool(transpose)), cos.shape[0]
    a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1)
    a.q_out, a.q_out_stride_t, a.q_out_stride_h = q_out.data_ptr(), q_out.stride(0), q_out.stride(1)
    a.k_out, a.k_out_stride_t, a.k_out_stride_h = k_out.data_ptr(), k_out.stride(0), k_out.stride(1)
    a.cos, a.sin, a.cos_sin_stride = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    a.cu_seqlens = _ptr(cu)
    _raise(lib().dsalt_rope(ctypes.byref(a), stream_handle(dev)), "dsalt_rope")
    return (None if k_only else q_out), (None if q_only else k_out)


class ScoresLauncher:
    """hybrid_scores with its argument block, outputs and workspace built once: each call
    launches the two score kernels on the current stream (for timing loops and graph
    capture); `scores`, `z_x`, `z_v` hold the result."""

    def __init__(self, x: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, n_heads: int,
                 norms_f32: bool = False):
        self.device = require_gpu(x, v, alpha)
        self._keep = (x, v, alpha.detach().to(torch.float32).contiguous())
        T = x.shape[0]
        self.scores = torch.empty((T, n_heads), device=self.device, dtype=torch.float32)
        self.z_x = torch.empty((T,), device=self.device, dtype=torch.float32)
        self.z_v = torch.empty((T, n_heads), device=self.device, dtype=torch.float32)
        self._ws = torch.empty((scores_workspace_size(T, v.shape[1]),), device=self.device, dtype=torch.uint8)
        self._args = scores_args(x, v, self._keep[2], n_heads, self.scores, self.z_x, self.z_v, self._ws, norms_f32)
        _raise(lib().dsalt_scores_check(ctypes.byref(self._args)), "dsalt_scores_check")

    def __call__(self) -> None:
        _raise(lib().dsalt_hybrid_scores(ctypes.byref(self._args), stream_handle(self.device)), "dsalt_hybrid_scores")


class SelectLauncher:
    """select_landmarks with its argument block built once: each call launches the
    selection kernel on the current stream (for timing loops); `out` holds the result."""

    def __init__(self, scores: torch.Tensor, w: torch.Tensor, cu_seqlens: torch.Tensor, k_lmk: int,
                 chunked: bool = True, max_seqlen: int | None = None, quantize: bool = False):
        self.device = require_gpu(scores, w, cu_seqlens)
        cu = _cu_i32(cu_seqlens)
        self.out = torch.empty((scores.shape[1], cu.shape[0] - 1, k_lmk), device=self.device, dtype=torch.int64)
        w = _f32_vec(w)
        # quantize: w is w~ and the launch also writes the quantised windows to self.w_out
        self.w_out = torch.empty(w.shape[0], device=self.device, dtype=torch.float32) if quantize else None
        self._args, self._keep = _select_args(scores, w, cu, k_lmk, self.out, chunked, max_seqlen, self.w_out)
        self._ref = ctypes.byref(self._args)
        self._fn = lib().dsalt_select_landmarks

    def __call__(self) -> None:
        _raise(self._fn(self._ref, stream_handle(self.device)), "dsalt_select_landmarks")


class QuantizeLauncher:
    """quantize_windows with the buffers allocated once (for timing loops)."""

    def __init__(self, w_cont: torch.Tensor):
        self.device = require_gpu(w_cont)
        self._w = _f32_vec(w_cont).contiguous()
        self.out = torch.empty_like(self._w)
        self._fn = lib().dsalt_quantize_windows

    def __call__(self) -> None:
        _raise(self._fn(self._w.data_ptr(), self._w.numel(), self.out.data_ptr(), None, stream_handle(self.device)),
               "dsalt_quantize_windows")


def quantize_windows(w_cont: torch.Tensor, want_int: bool = False):
    """w = max(1, floor(w~)) as float32 (NaN stays NaN); optionally also as int32."""
    dev = require_gpu(w_cont)
    w_cont = _f32_vec(w_cont).contiguous()
    n = w_cont.numel()
    wq = torch.empty_like(w_cont)
    wi = torch.empty(w_cont.shape, device=dev, dtype=torch.int32) if want_int else None
    _raise(lib().dsalt_quantize_windows(w_cont.data_ptr(), n, wq.data_ptr(), _ptr(wi), stream_handle(dev)),
           "dsalt_quantize_windows")
    return (wq, wi) if want_int else wq


def swiglu_supported(gate: torch.Tensor, up: torch.Tensor) -> bool:
    """Whether dsalt_swiglu takes these operands: GPU tensors of one shape and dtype (bf16,
    fp16 or fp32), contiguous and 16-byte aligned, with a multiple of 8 (4 for fp32)
    elements."""
    if gate.device.type != "cuda" or up.device != gate.device or gate.dtype not in _SCORE_DTYPES:
        return False
    if up.dtype != gate.dtype or up.shape != gate.shape or not (gate.is_contiguous() and up.is_contiguous()):
        return False
    per = 4 if gate.dtype == torch.float32 else 8
    return gate.numel() % per == 0 and gate.data_ptr() % 16 == 0 and up.data_ptr() % 16 == 0


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``F.silu(gate) * up`` in one HIP pass, bit for bit torch's two ops (no autograd)."""
    dev = require_gpu(gate, up)
    if not swiglu_supported(gate, up):
        raise DsaltError(f"dsalt_swiglu needs contiguous, 16-byte aligned gate and up of one shape and "
                         f"dtype with a multiple of 8 (4 for fp32) elements (got {tuple(gate.shape)} "
                         f"{gate.dtype}, {tuple(up.shape)} {up.dtype})")
    out = torch.empty_like(gate)
    _raise(lib().dsalt_swiglu(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
                              _SCORE_DTYPES[gate.dtype], stream_handle(dev)), "dsalt_swiglu")
    return out


RMS_NORM_MAX_DIM = 4096  # largest row length of dsalt_add_rms_norm


def add_rms_norm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether dsalt_add_rms_norm takes rows of x [..., d] with this weight [d]: a GPU
    tensor in bf16 or fp16, contiguous and 16-byte aligned, d a multiple of 8 up to 4096,
    the weight of the same dtype, contiguous and aligned."""
    if x.device.type != "cuda" or x.dtype not in (torch.bfloat16, torch.float16) or x.dim() < 1:
        return False
    d = x.shape[-1]
    if not (8 <= d <= RMS_NORM_MAX_DIM and d % 8 == 0 and x.is_contiguous() and x.data_ptr() % 16 == 0):
        return False
    return (weight.device == x.device and weight.dtype == x.dtype and weight.shape == (d,) and weight.is_contiguous()
            and weight.data_ptr() % 16 == 0)


def add_rms_norm(x: torch.Tensor, h: torch.Tensor | None, weight: torch.Tensor, eps: float):
    """``x_out = x + h`` (torch's add, bit for bit) and ``y = F.rms_norm(x_out, (d,), weight,
    eps)`` in one HIP pass over the rows (no autograd); h = None normalises x alone.
    Returns (x_out, y), x_out None without h. y can differ from F.rms_norm in an output's
    last bit (the sum of squares runs in another order)."""
    dev = require_gpu(x, weight, h)
    if not add_rms_norm_supported(x, weight) or (h is not None and (h.shape != x.shape or h.dtype != x.dtype or
                                                                    not h.is_contiguous() or h.data_ptr() % 16)):
        raise DsaltError(f"dsalt_add_rms_norm needs contiguous, 16-byte aligned bf16/fp16 rows of d = 8k <= "
                         f"{RMS_NORM_MAX_DIM} with a weight [d] of the same dtype (got x {tuple(x.shape)} {x.dtype}, "
                         f"weight {tuple(weight.shape)} {weight.dtype})")
    d = x.shape[-1]
    x_out = torch.empty_like(x) if h is not None else None
    y = torch.empty_like(x)
    _raise(lib().dsalt_add_rms_norm(x.data_ptr(), _ptr(h), _ptr(x_out), y.data_ptr(), weight.data_ptr(),
                                    x.numel() // d, d, float(eps), _SCORE_DTYPES[x.dtype], stream_handle(dev)),
           "dsalt_add_rms_norm")
    return x_out, y
