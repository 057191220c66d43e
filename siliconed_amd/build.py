"""Builds the gfx950 library libsiliconed_q8.so in-tree with hipcc.

Each .hip source is compiled to an object in parallel, then linked. The flags every HIP object
gets: --offload-arch=gfx950 only, -O3, and packed-fp32 instructions disabled for the device code
(`-Xclang -target-feature -Xclang -packed-fp32-ops`; the host pass warns that it does not know the
feature, which is harmless).
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libsiliconed_q8.so")
# (source, object name, extra defines): the FAST kernel set is one source compiled per weight type
# and layout, so the sets compile in parallel.
SOURCES = [
    ("sq8_gemm.hip", "sq8_gemm", []),
    ("sq8_gemm_general.hip", "sq8_gemm_general", []),
    ("sq8_gemm_inst.hip", "sq8_gemm_i8_kn", ["-DSQ8_WT=0", "-DSQ8_WL=0"]),
    ("sq8_gemm_inst.hip", "sq8_gemm_i8_nk", ["-DSQ8_WT=0", "-DSQ8_WL=1"]),
    ("sq8_gemm_inst.hip", "sq8_gemm_f8_kn", ["-DSQ8_WT=1", "-DSQ8_WL=0"]),
    ("sq8_gemm_inst.hip", "sq8_gemm_f8_nk", ["-DSQ8_WT=1", "-DSQ8_WL=1"]),
    ("sq8_wdirect_inst.hip", "sq8_wdirect_i8_nk", ["-DSQ8_WT=0", "-DSQ8_WL=1"]),
    ("sq8_wdirect_inst.hip", "sq8_wdirect_i8_packed", ["-DSQ8_WT=0", "-DSQ8_WL=2"]),
    ("sq8_wdirect_inst.hip", "sq8_wdirect_f8_nk", ["-DSQ8_WT=1", "-DSQ8_WL=1"]),
    ("sq8_wdirect_inst.hip", "sq8_wdirect_f8_packed", ["-DSQ8_WT=1", "-DSQ8_WL=2"]),
    ("sq8_aux.hip", "sq8_aux", []),
    ("sq8_block.hip", "sq8_block", []),
    ("sq8_convrot.hip", "sq8_convrot", []),
    ("sq8_w8a8.hip", "sq8_w8a8", []),
    ("sq8_i8_inst.hip", "sq8_i8_inst", []),
    ("sq8_blocks.hip", "sq8_blocks", []),
    ("sq8_api.hip", "sq8_api", []),
]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Every product and sum rounded on its own, as the reference's kernels (`fp contract(off)`): HIP
    # contracts a·b + c into one FMA by default, and its __fmul_rn / __fadd_rn are plain operators.
    # Where a fused multiply-add is meant, the code says __builtin_fmaf.
    "-ffp-contract=off",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def _compile(item) -> str:
    src, name, defines = item
    obj = os.path.join(OBJ, name + ".o")
    cmd = [HIPCC, *FLAGS, *defines, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def _stale(item) -> bool:
    """True when the object is missing or older than its source or any header it may include."""
    src, name, _ = item
    obj = os.path.join(OBJ, name + ".o")
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [os.path.join(CSRC, src)] + [os.path.join(d, f) for d in (CSRC, os.path.join(ROOT, "include"))
                                         for f in os.listdir(d) if f.endswith(".h")]
    return any(os.path.getmtime(d) > t for d in deps)


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compiles the sources and links the library; returns its path. Always recompiles every source,
    unless `incremental` (then only those whose object is older than the source or a header)."""
    os.makedirs(OBJ, exist_ok=True)
    todo = [it for it in SOURCES if _stale(it)] if incremental else SOURCES
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(len(todo), 1)) as pool:
        list(pool.map(_compile, todo))
    objs = [os.path.join(OBJ, name + ".o") for _, name, _ in SOURCES]
    tmp = LIB + ".tmp"
    # rocBLAS: the bf16-weight product's plain GEMM.
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-lrocblas", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv[1:])
