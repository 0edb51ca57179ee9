"""Build libek_hip.so (the gfx950 decode kernels) in-tree with hipcc.

    python -m enginekernel_amd.build [--verbose]

Each .hip source compiles to an object under enginekernel_amd/_build/ (in
parallel), then one shared library is linked next to this file. The library
links libamdhip64.so.7; when torch is imported first, the runtime torch
already loaded (same soname) is the one it binds to, so kernels launched
through the C ABI share torch's streams and graph captures.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libek_hip.so")
SOURCES = ["ek_abi.hip", "ek_norm.hip", "ek_gemv.hip", "ek_attn.hip", "ek_prefill.hip", "ek_spec.hip", "ek_step.hip"]
# head dims of the persistent decode-step kernel; ek_step_inst.hip is compiled once per head dim
STEP_HEAD_DIMS = [32, 64, 128]
# row bounds of the batch decode-step kernel; ek_bstep_inst.hip is compiled once per bound
BSTEP_ROWS = [2, 4, 8]
# (prologue, epilogue) pairs of the GEMV family; ek_gemv_inst.hip is compiled
# once per pair (must match EK_GEMV_PAIRS in csrc/ek_gemv_impl.h)
GEMV_PAIRS = [(0, 0), (0, 1), (0, 2), (0, 3), (1, 0), (1, 2), (2, 0), (2, 2),
              (3, 0), (3, 2), (3, 3), (4, 0)]
ARCH = os.environ.get("EK_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
# Packed FP32 ops are disabled for every device pass; -O3 would otherwise
# emit them from plain float code.
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include"), "-I", CSRC,
         "-Wno-unused-result"]


def _units():
    """(source, object name, extra flags) for every translation unit."""
    out = [(s, os.path.splitext(s)[0], []) for s in SOURCES]
    for pro, epi in GEMV_PAIRS:
        out.append(("ek_gemv_inst.hip", f"ek_gemv_inst_{pro}_{epi}",
                    [f"-DEK_PRO={pro}", f"-DEK_EPI={epi}"]))
    for d in STEP_HEAD_DIMS:
        out.append(("ek_step_inst.hip", f"ek_step_inst_{d}", [f"-DEK_STEP_D={d}"]))
    for mb in BSTEP_ROWS:
        out.append(("ek_bstep_inst.hip", f"ek_bstep_inst_{mb}", [f"-DEK_BSTEP_MB={mb}"]))
    return out


def _compile(unit, verbose: bool) -> str:
    src, name, extra = unit
    obj = os.path.join(BUILD, name + ".o")
    cmd = [HIPCC, *FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {name}:\n{err}")
    if verbose and err.strip():
        print(err)
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 and link libek_hip.so. Returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    units = _units()
    jobs = max(1, min(len(units), len(os.sched_getaffinity(0)), 16))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda u: _compile(u, verbose), units))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
