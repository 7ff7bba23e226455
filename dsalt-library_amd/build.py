"""Build libdsalt_hip.so (gfx950 only) from csrc/ with hipcc, in-tree.

Usage: python dsalt-library_amd/build.py [--jobs N]
The library lands in dsalt-library_amd/dsalt/libdsalt_hip.so, next to the Python
package that loads it. Objects are compiled in parallel into _build/ and linked once.
bench_kernels/peaks.hip (bench.py's peak probes, not part of the DSALT ABI) becomes
libdsalt_peaks.so beside it.
"""
from __future__ import annotations

import argparse
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "dsalt", "libdsalt_hip.so")
PEAKS_SRC = os.path.join(HERE, "bench_kernels", "peaks.hip")
PEAKS_OUT = os.path.join(HERE, "dsalt", "libdsalt_peaks.so")
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast", "-Wall", "-Wno-unused-result",
    "-mllvm", "-amdgpu-mfma-vgpr-form",  # MFMA C/D in VGPRs: no accvgpr copies for softmax
    "-Rpass-analysis=kernel-resource-usage",  # per-kernel register / scratch report (checked below)
]

# Sources whose results must equal torch's elementwise kernels bit for bit are built with
# hipcc's default contraction (fused only where the source or the device library marks an
# operation contractible). -ffp-contract=fast lets the backend fuse any multiply-add, among
# them the range reduction inside the device library's expf (x*log2e - round(x*log2e)
# becomes one fma), which changes exp's last bit against torch's build.
TORCH_ROUNDING_SOURCES = {"swiglu.hip", "rmsnorm.hip"}


def flags_for(src: str) -> list[str]:
    if os.path.basename(src) in TORCH_ROUNDING_SOURCES:
        return [f for f in HIPCC_FLAGS if f != "-ffp-contract=fast"]
    return HIPCC_FLAGS

_REMARK = re.compile(r"remark:\s+(Function Name|TotalSGPRs|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                     r"Dynamic Stack|Occupancy \[waves/SIMD\]|SGPRs Spill|VGPRs Spill|"
                     r"LDS Size \[bytes/block\]): (\S+)")


def resource_report(stderr: str) -> list[dict]:
    """Per-kernel resource figures from the compiler's kernel-resource-usage remarks."""
    kernels: list[dict] = []
    for line in stderr.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            kernels.append({"name": val})
        elif kernels:
            kernels[-1][key] = val
    return kernels


def spill_violations(kernels: list[dict]) -> list[str]:
    """Kernels that spill registers or use scratch memory. The tile rings wait on
    hand-counted vector-memory counters (s_waitcnt vmcnt(N)); a compiler-inserted
    scratch access would be counted too and silently break them, so none is allowed."""
    bad = []
    for k in kernels:
        why = [f"{f}={k[f]}" for f in ("SGPRs Spill", "VGPRs Spill", "ScratchSize [bytes/lane]")
               if k.get(f, "0") != "0"]
        if k.get("Dynamic Stack", "False") != "False":
            why.append("dynamic stack")
        if why:
            bad.append(f"{k['name']}: {', '.join(why)}")
    return bad


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (expected ROCm at /opt/rocm)")
    return path


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def compile_one(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *flags_for(src), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    kernels = resource_report(res.stderr)
    bad = spill_violations(kernels)
    if bad:
        raise RuntimeError(f"{os.path.basename(src)}: register spills / scratch use are not allowed:\n  "
                           + "\n  ".join(bad))
    with open(obj + ".resources.txt", "w") as f:
        for k in kernels:
            f.write(" ".join(f"{a}={b}" for a, b in k.items()) + "\n")
    warn = "\n".join(l for l in res.stderr.splitlines()
                     if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l and l.strip()
                     and not re.match(r"^\s*\d*\s*\|", l) and "remark" not in l)
    if warn:
        print(warn, file=sys.stderr)
    return obj


def link(objs: list[str], out: str) -> None:
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources() + [PEAKS_SRC]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2) // 2))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    link(objs[:-1], OUT)
    link(objs[-1:], PEAKS_OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    print(build(args.jobs))
