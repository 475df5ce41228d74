"""Build the HIP library ``vxg_amd/libvxt_hip.so`` for gfx950 with hipcc,
and beside it ``libvxt_hip_blas.so``, the hipBLASLt plugin that only the
pinned library GEMM path opens.

Run ``python -m vxg_amd.build`` (or ``__graft_entry__.build()``).  hipcc
cross-compiles for gfx950 without a GPU present.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libvxt_hip.so")
SOURCES = ["vxt_hip.hip", "gemv.hip", "gemv_q8.hip", "gemv_q8p.hip", "gemv_q40.hip", "gemv_cb4.hip", "gemv_g64.hip", "gemm_panel.hip", "gemm_fused.hip", "gemm_tile.hip", "gemm_dense.hip", "gemm_dense3.hip",
           "blas_plugin.cpp", "dequant.hip", "greedy.hip", "probe.hip", "ffn.hip", "attn.hip", "archive.cpp"]
LIBS = ["-ldl"]

# The pinned comparison path's dense phase on hipBLASLt (gemm_blas.cpp), a
# library of its own that libvxt_hip.so opens on first use (blas_plugin.cpp).
BLAS_LIB = os.path.join(HERE, "libvxt_hip_blas.so")
BLAS_SOURCES = ["gemm_blas.cpp"]
BLAS_LIBS = ["-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops off: the compiler must not form v_pk_{add,mul,fma}_f32.
_NOISE = "is not a recognized feature for this target"
OBJ_DIR = os.path.join(HERE, "_build")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-I" + os.path.join(ROOT, "include"),
]


# Per-source flags: MFMA results in VGPRs where the VALU scales each fresh
# fragment right after its MFMAs (in AGPRs every element needs a
# v_accvgpr_read first): the persistent Q8 GEMV (gemv_q8p.hip) and the fused
# Q8 GEMM (gemm_fused.hip; Q8 M = 128 graph-timed 102 -> 114 and 106 -> 119
# TFLOP/s on the same box, the g64 instantiations unchanged).
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
FILE_FLAGS = {"gemv_q8p.hip": _VGPR_MFMA, "gemm_fused.hip": _VGPR_MFMA}


def _compile(src: str, obj: str, verbose: bool) -> None:
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if _NOISE not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)} ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def _link(objs: list[str], libs: list[str], out: str, verbose: bool) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, *libs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {os.path.basename(out)} failed ({r.returncode}):\n{r.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source to an object in parallel, then link the library
    and the hipBLASLt plugin."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OBJ_DIR, exist_ok=True)
    names = SOURCES + BLAS_SOURCES
    srcs = [os.path.join(CSRC, s) for s in names]
    objs = [os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o") for s in names]
    jobs = jobs or min(len(srcs), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], verbose), zip(srcs, objs)))
    _link(objs[:len(SOURCES)], LIBS, LIB, verbose)
    _link(objs[len(SOURCES):], BLAS_LIBS, BLAS_LIB, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
