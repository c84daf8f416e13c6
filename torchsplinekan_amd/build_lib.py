"""Builds libkan_hip.so (the gfx950 kernels and their C-ABI) in-tree.

Usage: ``python -m torchsplinekan_amd.build_lib`` or ``build_library()``.
The library is compiled with hipcc for gfx950 only, from the sources in
``csrc/``, into the package directory, so that it travels with the source
tree and is found by :mod:`torchsplinekan_amd._lib` without any install step.
"""

import hashlib
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libkan_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["kan_capi.hip", "kan_basis.hip", "kan_gemm.hip", "kan_edge.hip", "kan_edge_mfma.hip",
           "kan_edge_mfma64.hip", "kan_refit.hip", "kan_stream.hip", "kan_reg.hip"]
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-FP32 instructions are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Per-source additions.  The edge-statistic kernels read every MFMA result
# with VALU instructions (abs-sums, sign tests); MFMAs that write VGPRs
# instead of accumulation registers save a copy per value and registers.
SOURCE_FLAGS = {
    "kan_edge_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "kan_edge_mfma64.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def source_hash() -> str:
    """SHA-256 over every source, header and flag the library is built from
    (csrc/*, include/kan_hip.h when present, the flag lists); compiled into
    the library and checked by the loader."""
    h = hashlib.sha256()
    paths = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                   if f.endswith((".hip", ".h")))
    header = os.path.join(os.path.dirname(PKG_DIR), "include", "kan_hip.h")
    if os.path.exists(header):
        paths.append(header)
    for path in paths:
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    h.update(repr((ARCH, COMMON_FLAGS, sorted(SOURCE_FLAGS.items()))).encode())
    return h.hexdigest()


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "unknown target feature" not in l and "packed-fp32-ops" not in l
                    and l.strip() not in ("", "1 warning generated.", "2 warnings generated."))
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_library(verbose: bool = False) -> str:
    """Compiles every source for gfx950 and links libkan_hip.so; returns its path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = []
    cmds = []
    digest = source_hash()
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        extra = [f'-DKAN_SOURCE_HASH="{digest}"'] if src == "kan_capi.hip" else []
        cmds.append([hipcc, *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), *extra, "-c",
                     os.path.join(CSRC, src), "-o", obj])
    workers = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for out in ex.map(_run, cmds):
            if verbose and out:
                print(out)
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build_library(verbose=True)
