"""Build libinsitu_hip.so in-tree for gfx950 with hipcc (no JIT cache, no torch extension).

    python -m insitu_amd.build [--stamps]

Each .hip file compiles to an object in parallel, then one shared library is
linked next to this file so it travels with the source tree. --stamps also links
libinsitu_hip_stamps.so, the decode step kernel with its phase stamps compiled in
(timing studies: python -m insitu_amd.phases).
"""

from __future__ import annotations

import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libinsitu_hip.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("INSITU_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Keep the compiler from forming packed-FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-function",
]


# Sources built more than once, each time with other defines: the chunked attend with
# 512-token chunks (namespace insitu::c512) beside its default 1,024-token build.
VARIANTS = {"attend_chunked.hip": [("c512", ["-DINSITU_CHUNK_TPT=1"])]}


def _compile(job) -> str:
    src, tag, defs = job
    obj = os.path.join(BUILD, os.path.basename(src) + (f".{tag}" if tag else "") + ".o")
    cmd = [HIPCC, *FLAGS, *defs, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = [(src, "", []) for src in srcs]
    jobs += [(os.path.join(CSRC, name), tag, defs) for name, vs in VARIANTS.items() for tag, defs in vs]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        objs = list(ex.map(_compile, jobs))
    tmp = OUT + ".tmp"
    # rocBLAS runs the host half's plain fp16 GEMMs (host_half.hip)
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lrocblas"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


STAMPS_OUT = os.path.join(HERE, "libinsitu_hip_stamps.so")


def build_stamps(verbose: bool = False) -> str:
    """libinsitu_hip_stamps.so: the library with the decode step kernel's phase stamps
    compiled in (attend_step.hip with INSITU_STEP_STAMPS), for insitu_amd.phases only.
    It reuses build()'s other objects, so build() runs first."""
    if not os.path.exists(OUT):
        build(verbose)
    obj = _compile((os.path.join(CSRC, "attend_step.hip"), "stamps", ["-DINSITU_STEP_STAMPS"]))
    others = [o for o in sorted(glob.glob(os.path.join(BUILD, "*.o")))
              if not os.path.basename(o).startswith("attend_step.hip")]
    tmp = STAMPS_OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, obj, *others, "-lrocblas"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, STAMPS_OUT)
    if verbose:
        print(f"built {STAMPS_OUT}")
    return STAMPS_OUT


if __name__ == "__main__":
    build(verbose=True)
    if "--stamps" in sys.argv:
        build_stamps(verbose=True)
    sys.exit(0)
