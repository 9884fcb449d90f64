"""Build libpairformer_hip.so in-tree with hipcc for gfx950.

Run as ``python tt-boltz_amd/build.py`` or through ``__graft_entry__.build()``.
The library is written next to this file and loaded from there by ``_lib.py``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(HERE, "_build")

SOURCES = ["api.cpp", "trimul.hip", "triatt.hip", "transition.hip", "single.hip", "fast8.hip", "msa.hip", "diffusion.hip",
           "measure.hip"]

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}",
    # packed fp32 VALU ops are disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


#: library variants: file name -> extra defines.  The default library uses IEEE fp16
#: MFMA operands; the _bf16 variant uses bf16 operands (same kernels, same ABI).
VARIANTS = {
    "libpairformer_hip.so": [],
    "libpairformer_hip_bf16.so": ["-DPF_OPERAND_BF16"],
}


def _compile(job) -> str:
    src, defines, objdir = job
    obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, *defines, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src} {defines}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> list:
    jobs, outs = [], []
    for lib, defines in VARIANTS.items():
        objdir = os.path.join(OBJDIR, os.path.splitext(lib)[0])
        os.makedirs(objdir, exist_ok=True)
        jobs.append([(src, defines, objdir) for src in SOURCES])
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = [list(ex.map(_compile, j)) for j in jobs]
    for (lib, _), o in zip(VARIANTS.items(), objs):
        path = os.path.join(HERE, lib)
        tmp = path + ".tmp"
        r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *o, "-o", tmp],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed for {lib}:\n{r.stderr}")
        os.replace(tmp, path)
        outs.append(path)
        if verbose:
            print(f"built {path}")
    return outs


if __name__ == "__main__":
    build()
    sys.exit(0)
