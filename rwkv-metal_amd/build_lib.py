"""Build librwkvq_hip.so (gfx950) from rwkv-metal_amd/csrc with hipcc.

Every translation unit is compiled in parallel; the per-bit-width GEMV/GEMM
units are compiled once per bit width (-DRQ_BITS=n) so that no single unit
carries all template instantiations.  The library lands next to the Python
package (rwkv-metal_amd/rwkvq/librwkvq_hip.so), in-tree, so that it travels
with the repository snapshot to the GPU box.

Usage: python rwkv-metal_amd/build_lib.py [-j N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "rwkvq", "librwkvq_hip.so")
BITS = (2, 3, 4, 5, 6, 8)

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    # never let the backend form packed-fp32 (v_pk_*_f32) instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _units():
    units = [("rq_quant.hip", [], "rq_quant.o"), ("rq_sb6.hip", [], "rq_sb6.o"),
             ("rq_lora.hip", [], "rq_lora.o"),
             ("rq_abi.cpp", ["-x", "hip"], "rq_abi.o")]
    for b in BITS:
        # MFMA results straight into VGPRs: the GEMV consumes every MFMA
        # result with VALU fmas, so accumulator registers only add copies
        units.append(("rq_qmv.hip", [f"-DRQ_BITS={b}", "-mllvm", "-amdgpu-mfma-vgpr-form=1"],
                      f"rq_qmv_b{b}.o"))
        units.append(("rq_qmm.hip", [f"-DRQ_BITS={b}"], f"rq_qmm_b{b}.o"))
    return units


def _compile(src, extra, obj, objdir=OBJ):
    cmd = [HIPCC, *FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", os.path.join(objdir, obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src} {extra}:\n{err}")
    return obj


def build(jobs: int | None = None, verbose: bool = False, defines=(), out: str = LIB,
          objdir: str = OBJ) -> str:
    """Compile and link.  `defines` (e.g. ["-DRQ_QMV_NS=6"]) override the
    kernels' compile-time tuning constants; `out`/`objdir` redirect the
    products (used to build side-by-side variants)."""
    os.makedirs(objdir, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    units = [(src, [*extra, *defines], obj, objdir) for src, extra, obj in _units()]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, *u) for u in units]
        for f in cf.as_completed(futs):
            obj = f.result()
            if verbose:
                print(f"  compiled {obj}", flush=True)
    objs = [os.path.join(objdir, u[2]) for u in units]
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", flush=True)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-D", action="append", default=[], help="extra -D define")
    ap.add_argument("-o", default=LIB)
    ap.add_argument("--objdir", default=OBJ)
    a = ap.parse_args()
    build(a.j, verbose=True, defines=[f"-D{d}" for d in a.D], out=a.o, objdir=a.objdir)
    sys.exit(0)
