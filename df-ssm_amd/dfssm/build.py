"""Build libdfssm_hip.so (gfx950) in-tree with hipcc.

Every .hip file under csrc/ is compiled in parallel to csrc/../_build/*.o and linked into
dfssm/libdfssm_hip.so. Flags:
  --offload-arch=gfx950          MI355X only
  -ffp-contract=off              the kernels spell out every fused multiply-add they want
  -target-feature -packed-fp32-ops  no packed fp32 VALU instructions
  -target-feature -fma-mix-insts    no v_fma_mix*: the compiler otherwise folds
                                 fptrunc(fmul_f32(a, b)) into one fma_mix rounding the exact product
                                 straight to fp16, which differs from fp32-then-fp16 on ties
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)                       # df-ssm_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libdfssm_hip.so")
# profiling variant: the one-launch layer with per-phase wall-clock stamps (-DDFSSM_TIMELINE)
LIB_TIMELINE = os.path.join(PKG, "libdfssm_hip_timeline.so")
TIMELINE_SRCS = ("fused.hip",)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else "hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Xclang", "-target-feature", "-Xclang", "-fma-mix-insts",
         "-I" + os.path.join(REPO, "include"), "-I" + CSRC]


def _compile(src: str, timeline: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", "_tl.o" if timeline else ".o"))
    cmd = [HIPCC] + FLAGS + (["-DDFSSM_TIMELINE"] if timeline else []) + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every kernel source and link the shared library; returns its path."""
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError("hipcc not found")
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    tl_srcs = [p for p in srcs if os.path.basename(p) in TIMELINE_SRCS]
    jobs = [(p, False) for p in srcs] + [(p, True) for p in tl_srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        built = list(ex.map(lambda j: _compile(*j), jobs))
    objs = built[:len(srcs)]
    tl_objs = [o for p, o in zip(srcs, objs) if p not in tl_srcs] + built[len(srcs):]
    for out, parts in ((LIB, objs), (LIB_TIMELINE, tl_objs)):
        tmp = out + ".tmp"
        r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + parts + ["-o", tmp],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr}")
        os.replace(tmp, out)
        if verbose:
            print(f"built {out}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
