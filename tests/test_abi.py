"""The C-ABI library: it loads, exports every function include/dsalt_hip.h declares, its
argument structs match the ctypes mirror, and host-side validation rejects bad
arguments. No device memory is touched (validation reads no device data). CPU only."""
import ctypes
import os
import re

import pytest

import dsalt._hip as hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsalt_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(dsalt_\w+)\s*\(", text, re.M)))


def test_library_built_and_loads():
    assert os.path.exists(hip.LIB_PATH), "run dsalt-library_amd/build.py"
    hip.lib()
    hip.check_abi()


def test_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 13
    lib = ctypes.CDLL(hip.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(hip.EXPORTED_SYMBOLS) <= set(names)


def test_struct_sizes():
    lib = hip.lib()
    assert ctypes.sizeof(hip.FwdArgs) == lib.dsalt_fwd_args_size()
    assert ctypes.sizeof(hip.BwdArgs) == lib.dsalt_bwd_args_size()
    assert ctypes.sizeof(hip.SelectArgs) == lib.dsalt_select_args_size()
    assert ctypes.sizeof(hip.ScoresArgs) == lib.dsalt_scores_args_size()


def _fake_fwd(**kw):
    a = hip.FwdArgs()
    a.mode, a.dtype, a.total_len, a.num_seqs, a.n_heads, a.head_dim, a.k_lmk = 0, 0, 256, 2, 4, 64, 16
    base = 0x10000000
    for i, name in enumerate(("q", "k", "v", "out", "lse", "w", "lmk_pos", "cu_seqlens")):
        setattr(a, name, base + i * 0x100000)
    a.q_stride_t = a.k_stride_t = a.v_stride_t = a.out_stride_t = 4 * 64
    a.q_stride_h = a.k_stride_h = a.v_stride_h = a.out_stride_h = 64
    a.lse_stride_t, a.lse_stride_h, a.w_stride = 4, 1, 1
    a.lmk_pos_stride_h, a.lmk_pos_stride_s, a.lmk_pos_stride_k = 32, 16, 1
    a.scale, a.tau_win, a.win_edge = 0.125, 1.0, 4.0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _check(a):
    lib = hip.lib()
    rc = lib.dsalt_fwd_check(ctypes.byref(a))
    return rc, lib.dsalt_last_error().decode()


def test_fwd_check_accepts_valid_args():
    assert _check(_fake_fwd()) == (0, "") or _check(_fake_fwd())[0] == 0


@pytest.mark.parametrize("field,value,code,needle", [
    ("head_dim", 96, 2, "head_dim"),
    ("mode", 7, 1, "mode"),
    ("dtype", 5, 1, "dtype"),
    ("k_lmk", 5000, 2, "k_lmk"),
    ("num_seqs", 0, 1, "num_seqs"),
    ("q", None, 1, "q is NULL"),
    ("lmk_pos", None, 1, "lmk_pos"),
    ("q", 0x10000008, 1, "aligned"),
    ("k_stride_t", 250, 1, "strides"),
    ("tau_win", 0.0, 1, "tau_win"),
    ("scale", 0.0, 2, "scale"),
    ("scale", float("inf"), 2, "scale"),
    ("k_stride_t", 1 << 30, 2, "4 GiB"),
    ("n_kv_heads", 3, 1, "n_kv_heads"),
    ("n_kv_heads", -1, 1, "n_kv_heads"),
])
def test_fwd_check_rejects(field, value, code, needle):
    kw = {field: value}
    if field == "tau_win":
        kw["mode"] = 1
    rc, msg = _check(_fake_fwd(**kw))
    assert rc == code and needle in msg, (rc, msg)


def test_bwd_workspace_and_check():
    lib = hip.lib()
    assert lib.dsalt_bwd_workspace_size(1024, 2, 8, 64, 16) >= 0
    assert lib.dsalt_bwd_workspace_size(-1, 2, 8, 64, 16) == -1
    a = hip.BwdArgs()
    a.mode, a.dtype, a.total_len, a.num_seqs, a.n_heads, a.head_dim = 0, 0, 128, 1, 2, 128
    assert lib.dsalt_bwd_check(ctypes.byref(a)) != 0


def _fake_bwd(**kw):
    a = hip.BwdArgs()
    a.mode, a.dtype, a.total_len, a.num_seqs, a.n_heads, a.head_dim, a.k_lmk = 0, 0, 256, 2, 4, 64, 16
    base = 0x10000000
    names = ("q", "k", "v", "out", "lse", "dout", "w", "lmk_pos", "cu_seqlens", "dq", "dk", "dv", "workspace")
    for i, name in enumerate(names):
        setattr(a, name, base + i * 0x1000000)
    for t in ("q", "k", "v", "out", "dout", "dq", "dk", "dv"):
        setattr(a, t + "_stride_t", 4 * 64)
        setattr(a, t + "_stride_h", 64)
    a.lse_stride_t, a.lse_stride_h, a.w_stride = 4, 1, 1
    a.lmk_pos_stride_h, a.lmk_pos_stride_s, a.lmk_pos_stride_k = 32, 16, 1
    a.workspace_bytes = 1 << 30
    a.scale, a.tau_win, a.win_edge = 0.125, 1.0, 4.0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("value", [0.0, float("inf"), float("nan")])
def test_bwd_check_rejects_bad_scale(value):
    lib = hip.lib()
    assert lib.dsalt_bwd_check(ctypes.byref(_fake_bwd())) == 0, lib.dsalt_last_error().decode()
    rc = lib.dsalt_bwd_check(ctypes.byref(_fake_bwd(scale=value)))
    assert rc != 0 and "scale" in lib.dsalt_last_error().decode()


def test_select_check():
    lib = hip.lib()
    a = hip.SelectArgs()
    a.total_len, a.num_seqs, a.n_heads, a.k_lmk = 100, 1, 2, 2000
    a.scores, a.w, a.cu_seqlens, a.lmk_pos = 0x1000, 0x2000, 0x3000, 0x4000
    assert lib.dsalt_select_check(ctypes.byref(a)) == 2
    a.k_lmk = 16
    assert lib.dsalt_select_check(ctypes.byref(a)) == 0


def test_select_workspace_size_and_check():
    """The chunk-wise selection's workspace: none below 4097 tokens; with one, the size
    per (head, chunk id) is k + min(k, 128) candidate keys and as many positions; too
    small or misaligned workspaces are rejected."""
    lib = hip.lib()
    assert lib.dsalt_select_workspace_size(4096, 1, 16, 128) == 0
    assert lib.dsalt_select_workspace_size(16384, 1, 16, 0) == 0
    assert lib.dsalt_select_workspace_size(-1, 1, 16, 128) < 0
    need = lib.dsalt_select_workspace_size(16384, 1, 16, 128)
    n = 16 * (16384 // 2048 + 1)  # heads x chunk ids (ceil(T / 2048) + S)
    al = lambda b: -(-b // 256) * 256
    assert need == 2 * al(n * (128 + 128) * 4)
    a = hip.SelectArgs()
    a.total_len, a.num_seqs, a.n_heads, a.k_lmk = 16384, 1, 16, 128
    a.scores, a.w, a.cu_seqlens, a.lmk_pos = 0x1000, 0x2000, 0x3000, 0x4000
    a.workspace, a.workspace_bytes = 0x10000, need
    assert lib.dsalt_select_check(ctypes.byref(a)) == 0, lib.dsalt_last_error().decode()
    a.workspace_bytes = need - 1
    assert lib.dsalt_select_check(ctypes.byref(a)) != 0 and "workspace" in lib.dsalt_last_error().decode()
    a.workspace, a.workspace_bytes = 0x10008, need
    assert lib.dsalt_select_check(ctypes.byref(a)) != 0
    a.workspace, a.max_seqlen = 0x10000, -1
    assert lib.dsalt_select_check(ctypes.byref(a)) != 0 and "max_seqlen" in lib.dsalt_last_error().decode()


def test_cpu_tensors_raise():
    import torch
    q = torch.zeros(8, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(hip.DsaltError, match="ROCm GPU"):
        hip.fwd(0, q, q, q, torch.ones(8), None, None, torch.tensor([0, 8], dtype=torch.int32), 0.125)


def test_tuned_config_matches_kernel_constants():
    # the reported tiles are the ones csrc/launch.h and csrc/bwd.hip compile in
    from dsalt.kernels import autotune_blocks, get_tuned_config
    here = os.path.dirname(os.path.abspath(__file__))
    launch = open(os.path.join(here, "..", "dsalt-library_amd", "csrc", "launch.h")).read()
    bwd = open(os.path.join(here, "..", "dsalt-library_amd", "csrc", "bwd.hip")).read()

    def const_fn(src, name):  # constexpr int name(int d) { return d == 64 ? A : B; }
        m = re.search(r"constexpr int %s\(int[^)]*\) \{ return (?:\w+ == 64 \? (\d+) : (\d+)|(\d+)); \}" % name, src)
        assert m, name
        return (int(m.group(1)), int(m.group(2))) if m.group(1) else (int(m.group(3)),) * 2

    waves, bn, stages, kv_qt = (const_fn(launch, "fwd_waves"), const_fn(launch, "fwd_bn"),
                                const_fn(launch, "fwd_ring"), const_fn(bwd, "kv_qt"))
    for i, d in enumerate((64, 128)):
        cfg = get_tuned_config(d)
        assert cfg == autotune_blocks(d)
        assert cfg["num_warps"] == waves[i] and cfg["BLOCK_M"] == 32 * waves[i]
        assert cfg["BLOCK_N"] == bn[i] and cfg["num_stages"] == stages[i] and cfg["BLOCK_N_BWD"] == kv_qt[i]
    with pytest.raises(ValueError):
        get_tuned_config(96)


def _scores_args(**kw):
    a = hip.ScoresArgs()
    a.total_len, a.d_model, a.n_kv_heads, a.head_dim, a.n_heads = 100, 512, 4, 64, 8
    a.x_dtype = a.v_dtype = hip.DTYPE_BF16
    a.x, a.x_stride_t = 0x10000, 512
    a.v, a.v_stride_t, a.v_stride_h = 0x20000, 256, 64
    a.alpha, a.scores, a.scores_stride_t, a.scores_stride_h = 0x30000, 0x40000, 8, 1
    a.workspace = 0x50000
    for k, v in kw.items():
        setattr(a, k, v)
    if "workspace_bytes" not in kw:
        a.workspace_bytes = hip.lib().dsalt_scores_workspace_size(a.total_len, a.n_kv_heads)
    return a


def test_scores_workspace_size():
    lib = hip.lib()
    assert lib.dsalt_scores_workspace_size(-1, 4) == -1
    assert lib.dsalt_scores_workspace_size(10, 0) == -1
    small, big = lib.dsalt_scores_workspace_size(100, 4), lib.dsalt_scores_workspace_size(10000, 16)
    assert 0 < small < big and small % 256 == 0


@pytest.mark.parametrize("field,value,code,needle", [
    ("n_kv_heads", 3, 1, "divide"),                 # 3 does not divide 8
    ("x_dtype", 7, 1, "x_dtype"),
    ("v_dtype", -1, 1, "v_dtype"),
    ("head_dim", 96, 2, "power of two"),           # 96 / 8 = 12 chunks
    ("d_model", 100, 2, "multiples"),
    ("x", 0x10008, 1, "aligned"),
    ("x_stride_t", 256, 1, "row stride"),           # < d_model
    ("v_stride_h", 60, 1, "v strides"),
    ("workspace", 0, 1, "workspace is NULL"),
    ("workspace_bytes", 16, 1, "too small"),
    ("workspace", 0x50010, 1, "256-byte"),
    ("alpha", 0, 1, "non-NULL"),
])
def test_scores_check_rejects(field, value, code, needle):
    lib = hip.lib()
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args())) == 0
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(**{field: value}))) == code
    assert needle in lib.dsalt_last_error().decode()


def test_scores_check_fp32_and_gqa():
    lib = hip.lib()
    # fp32: 4 elements per 16-byte load, head_dim 64 -> 16 lanes per row
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(x_dtype=hip.DTYPE_F32, v_dtype=hip.DTYPE_F32))) == 0
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(v_dtype=hip.DTYPE_F32, head_dim=512))) == 2
    # autocast: fp32 x with bf16 v
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(x_dtype=hip.DTYPE_F32))) == 0
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(n_kv_heads=8, v_stride_t=512))) == 0
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(n_kv_heads=1, v_stride_t=64))) == 0
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(n_kv_heads=256, n_heads=256))) == 2


def test_scores_check_gate_fields():
    """The window-gate logit of the norms pass: 16-bit x only, weights 16-byte aligned, an
    output with every gate, and neither bias nor output without weights."""
    lib = hip.lib()
    gate = dict(gate_w=0x60000, gate_b=0x70000, gate_out=0x80000)
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(**gate))) == 0
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(**dict(gate, gate_b=0)))) == 0  # no bias
    assert lib.dsalt_scores_check(ctypes.byref(_scores_args(**dict(gate, x_dtype=hip.DTYPE_F16)))) == 0
    for kw, code, needle in ((dict(gate, x_dtype=hip.DTYPE_F32), 2, "16-bit x"),
                             (dict(gate, gate_out=0), 1, "gate_out"),
                             (dict(gate, gate_w=0x60008), 1, "16-byte aligned"),
                             (dict(gate, gate_out=0x80001), 1, "2-byte aligned"),
                             (dict(gate_b=0x70000), 1, "need gate_w"),
                             (dict(gate_out=0x80000), 1, "need gate_w"),
                             (dict(gate, x_dtype=hip.DTYPE_F32, total_len=0), 2, "16-bit x")):
        assert lib.dsalt_scores_check(ctypes.byref(_scores_args(**kw))) == code, kw
        assert needle in lib.dsalt_last_error().decode()


def test_rope_check():
    lib = hip.lib()
    a = hip.RopeArgs()
    a.total_len, a.num_seqs, a.n_q_heads, a.n_k_heads, a.head_dim = 100, 2, 4, 2, 64
    a.dtype, a.transpose, a.table_rows = hip.DTYPE_BF16, 0, 80
    a.q = a.k = a.q_out = a.k_out = 0x10000
    a.cos, a.sin, a.cos_sin_stride, a.cu_seqlens = 0x20000, 0x30000, 64, 0x40000
    assert lib.dsalt_rope_check(ctypes.byref(a)) == 0
    assert ctypes.sizeof(hip.RopeArgs) == lib.dsalt_rope_args_size()
    for field, value, needle in (("head_dim", 63, "even"), ("dtype", 9, "dtype"), ("transpose", 2, "transpose"),
                                 ("cos_sin_stride", 32, "cos_sin_stride"), ("table_rows", 0, "table_rows"),
                                 ("cos", 0, "non-NULL")):
        old = getattr(a, field)
        setattr(a, field, value)
        assert lib.dsalt_rope_check(ctypes.byref(a)) == 1
        assert needle in lib.dsalt_last_error().decode()
        setattr(a, field, old)
    a.cu_seqlens = None  # per-token tables need total_len rows
    assert lib.dsalt_rope_check(ctypes.byref(a)) == 1
    a.table_rows = 100
    assert lib.dsalt_rope_check(ctypes.byref(a)) == 0


def test_exports_are_none_without_the_library():
    # the reference leaves its kernel entry points None when its kernels cannot load
    # (dsalt/kernels/__init__.py:23-35); the same holds here when libdsalt_hip.so is absent
    import subprocess
    import sys

    code = ("import dsalt, dsalt.kernels as k\n"
            "assert not k._HIP_OK\n"
            "assert k.dsalt_triton_attention is None and k.dsalt_triton_backward is None\n"
            "assert k.autotune_blocks is None and k.get_tuned_config is None\n"
            "assert dsalt.dsalt_triton_attention is None\n"
            "print('ok')\n")
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "dsalt-library_amd")
    env = dict(os.environ, PYTHONPATH=pkg, DSALT_HIP_LIB="/nonexistent/libdsalt_hip.so")
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert res.returncode == 0 and res.stdout.strip() == "ok", res.stderr


def test_dense_mode_checks():
    # DSALT_MODE_DENSE: one sequence, landmarks as a table (k_lmk = 0), positive scale;
    # cu_seqlens may be NULL; grouped K/V heads accepted when they divide n_heads
    ok = _fake_fwd(mode=hip.MODE_DENSE, num_seqs=1, k_lmk=0, lmk_pos=None, cu_seqlens=None)
    assert _check(ok)[0] == 0, _check(ok)
    assert _check(_fake_fwd(mode=hip.MODE_DENSE, num_seqs=1, k_lmk=0, lmk_pos=None, n_kv_heads=2))[0] == 0
    for kw, needle in ((dict(num_seqs=2), "one sequence"), (dict(num_seqs=1, k_lmk=4), "table"),
                       (dict(num_seqs=1, k_lmk=0, lmk_pos=None, scale=-0.125), "scale > 0")):
        rc, msg = _check(_fake_fwd(mode=hip.MODE_DENSE, **kw))
        assert rc != 0 and needle in msg, (kw, rc, msg)


def test_select_hybrid_rejects_before_launching():
    """dsalt_select_hybrid validates both argument blocks and their agreement on the host
    and returns before any launch when they are wrong."""
    lib = hip.lib()
    sel = hip.SelectArgs()
    sel.total_len, sel.num_seqs, sel.n_heads, sel.k_lmk = 100, 1, 8, 16
    sel.w, sel.cu_seqlens, sel.lmk_pos = 0x2000, 0x3000, 0x4000  # scores NULL: formed in the launch
    fn = lib.dsalt_select_hybrid
    assert fn(ctypes.byref(_scores_args()), ctypes.byref(sel), None) == 1
    assert "writes no scores" in lib.dsalt_last_error().decode()
    assert fn(ctypes.byref(_scores_args(scores=0, alpha=0)), ctypes.byref(sel), None) == 1
    assert "alpha" in lib.dsalt_last_error().decode()
    sel.n_heads = 4
    assert fn(ctypes.byref(_scores_args(scores=0)), ctypes.byref(sel), None) == 1
    assert "disagree" in lib.dsalt_last_error().decode()
    sel.n_heads, sel.w = 8, 0
    assert fn(ctypes.byref(_scores_args(scores=0)), ctypes.byref(sel), None) == 1
    assert "w_logit" in lib.dsalt_last_error().decode()
    # the plain selection still needs its scores
    sel.w = 0x2000
    assert lib.dsalt_select_check(ctypes.byref(sel)) == 1


def test_noalloc_scratch_size_matches_header():
    text = open(HEADER).read()
    m = re.search(r"#define DSALT_NOALLOC_SCRATCH_BYTES \(\(int64_t\)(\d+) << (\d+)\)", text)
    assert m and hip.NOALLOC_SCRATCH_BYTES == int(m.group(1)) << int(m.group(2))


def test_peak_probe_library_is_built_apart_from_the_abi():
    """bench.py's peak probes live in their own library: built next to the product, not
    exported by libdsalt_hip.so."""
    path = os.path.join(os.path.dirname(hip.LIB_PATH), "libdsalt_peaks.so")
    assert os.path.exists(path), "run dsalt-library_amd/build.py"
    peaks = ctypes.CDLL(path)
    assert hasattr(peaks, "dsalt_bench_mfma") and hasattr(peaks, "dsalt_bench_read")
    assert not hasattr(ctypes.CDLL(hip.LIB_PATH), "dsalt_bench_mfma")


def test_swiglu_rejects_before_launching():
    lib = hip.lib()
    fn = lib.dsalt_swiglu
    assert fn(0x1000, 0x2000, 0x3000, -1, hip.DTYPE_BF16, None) == 1
    assert fn(0x1000, 0x2000, 0x3000, 64, 9, None) == 1
    assert fn(0x1000, 0x2000, 0x3000, 12, hip.DTYPE_BF16, None) == 2  # not a multiple of 8
    assert fn(0x1000, 0x2000, 0x3000, 6, hip.DTYPE_F32, None) == 2    # not a multiple of 4
    assert fn(0x1008, 0x2000, 0x3000, 64, hip.DTYPE_BF16, None) == 1  # misaligned
    assert "aligned" in lib.dsalt_last_error().decode()
    assert fn(0, 0x2000, 0x3000, 64, hip.DTYPE_BF16, None) == 1
    assert fn(0, 0, 0, 0, hip.DTYPE_BF16, None) == 0  # nothing to do


def test_add_rms_norm_rejects_before_launching():
    lib = hip.lib()
    fn = lib.dsalt_add_rms_norm
    x, h, xo, y, w = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    bf = hip.DTYPE_BF16
    for args, code, needle in (((x, h, xo, y, w, -1, 1024, 1e-6, bf), 1, "rows"),
                               ((x, h, xo, y, w, 4, 1024, 1e-6, hip.DTYPE_F32), 1, "dtype"),
                               ((x, h, xo, y, w, 4, 12, 1e-6, bf), 2, "multiple of 8"),
                               ((x, h, xo, y, w, 4, 8192, 1e-6, bf), 2, "4096"),
                               ((x, h, xo, y, w, 4, 1024, -1.0, bf), 1, "eps"),
                               ((x, h, 0, y, w, 4, 1024, 1e-6, bf), 1, "x_out"),
                               ((x, h, xo, 0, w, 4, 1024, 1e-6, bf), 1, "non-NULL"),
                               ((x + 8, h, xo, y, w, 4, 1024, 1e-6, bf), 1, "aligned"),
                               ((x, h, xo, x, w, 4, 1024, 1e-6, bf), 1, "alias"),
                               ((x, h, xo, xo, w, 4, 1024, 1e-6, bf), 1, "alias")):
        assert fn(*args, None) == code, args
        assert needle in lib.dsalt_last_error().decode(), (args, lib.dsalt_last_error())
    assert fn(0, 0, 0, 0, 0, 0, 1024, 1e-6, bf, None) == 0  # no rows: nothing to do


def test_gate_linear_supported_rejects_cpu_operands():
    """The window gate's operands must all live on the GPU with x: a CPU weight or bias (or
    x) is refused before any pointer reaches the library."""
    import torch
    x = torch.zeros(4, 16, dtype=torch.bfloat16)
    w = torch.zeros(1, 16, dtype=torch.bfloat16)
    b = torch.zeros(1, dtype=torch.bfloat16)
    assert not hip.gate_linear_supported(x, w, b)  # CPU x
    assert not hip.gate_linear_supported(x, w, None)
