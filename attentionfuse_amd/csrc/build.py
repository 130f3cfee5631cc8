"""Build libattnfuse_hip.so for gfx950 with hipcc, in-tree, in parallel.

Usage: python -m attentionfuse_amd.csrc.build [--jobs N] [--quick]

Every HIP source is compiled with -Xclang -target-feature -Xclang
-packed-fp32-ops (packed fp32 VALU instructions are kept out of the code
objects) and linked into attentionfuse_amd/libattnfuse_hip.so.  All but the
units in DEFAULT_FORM_UNITS keep MFMA accumulators in VGPRs.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
ROOT = PKG.parent
OUT = PKG / "libattnfuse_hip.so"
BUILD = ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

BASE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{HERE}", "-Wno-unused-result",
]
# keep MFMA accumulators in VGPRs: VALU work on them (the softmax rescale)
# then needs no AGPR<->VGPR copies around the loop
FLAGS = BASE_FLAGS + ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
# units built with the compiler's default MFMA register form
DEFAULT_FORM_UNITS = {"fwd_d256_alt", "bwd_d256_alt"}

# (object name, source, extra defines)
UNITS = [
    ("api", "api.hip", []),
    ("decode", "decode_inst.hip", []),
    ("decode_noalloc", "decode_noalloc.hip", []),
    ("bs_split", "bs_split.hip", []),
    ("bwd", "bwd.hip", []),
    ("fwd_f32", "fwd_f32.hip", []),
    ("bwd_f32", "bwd_f32.hip", []),
    ("fwd_d256_alt", "fwd_d256_alt.hip", []),
    ("bwd_d256_alt", "bwd_d256_alt.hip", []),
] + [
    (f"{kind}_{dt}_d{d}", f"{kind}_inst.hip", [f"-DAF_DT={code}", f"-DAF_D={d}"])
    for kind in ("fwd", "bwd")
    for dt, code in (("f16", 0), ("bf16", 1)) for d in (32, 64, 128)
] + [
    # head dim 256: one wave per SIMD, accumulators past 256 registers in AGPRs
    (f"{kind}_{dt}_d256", f"{kind}_inst.hip", [f"-DAF_DT={code}", "-DAF_D=256"])
    for kind in ("fwd", "bwd") for dt, code in (("f16", 0), ("bf16", 1))
]


def _compile(unit) -> tuple:
    name, src, defs = unit
    obj = BUILD / f"{name}.o"
    flags = BASE_FLAGS if name in DEFAULT_FORM_UNITS else FLAGS
    cmd = [HIPCC, *flags, *defs, "-c", str(HERE / src), "-o", str(obj)]
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines()
                     if "packed-fp32-ops" not in l)
    return name, r.returncode, errs, time.time() - t0, obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(len(UNITS), os.cpu_count() or 4)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for name, rc, errs, dt, obj in ex.map(_compile, UNITS):
            if rc != 0:
                raise RuntimeError(f"hipcc failed for {name}:\n{errs}")
            if verbose:
                print(f"  [{dt:5.1f}s] {name}", flush=True)
            objs.append(str(obj))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs,
           "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}", flush=True)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    build(a.jobs)
    sys.exit(0)
