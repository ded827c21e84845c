"""Build libkai_gdn_hip.so (gfx950) and the C harnesses, in-tree.

    python -m orionsbelt_amd.build          # library + harness binaries

Outputs:
    orionsbelt_amd/lib/libkai_gdn_hip.so    the C-ABI library
    orionsbelt_amd/bin/test_kai_gdn         kai test harness (C), links the library
    orionsbelt_amd/bin/bench_kai_gdn        kai bench harness (C), links the library
    orionsbelt_amd/bin/gdn_e2e_decode       hybrid decode benchmark (C), the reference e2e
                                            program's interface

Every HIP translation unit is compiled with
`-Xclang -target-feature -Xclang -packed-fp32-ops` (no packed fp32 ops are
emitted).  The host pass of hipcc warns that it does not know the feature;
that warning is expected.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
BINDIR = os.path.join(PKG, "bin")
OBJDIR = os.path.join(PKG, "csrc", "_build")
INCLUDE = os.path.join(REPO, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CC = os.environ.get("CC", "gcc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

SOURCES = ["gdn_stream.hip", "gdn_decode.hip", "gdn_prefill.hip", "gdn_layer.hip", "gdn_state.hip", "gdn_model.hip", "gdn_prefill_model.hip", "gdn_hybrid.hip", "gdn_probe.hip", "kai_shim.hip"]
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", f"-I{INCLUDE}",
]
LIB_NAME = "libkai_gdn_hip.so"
# Per-file code generation options.  The prefill keeps its MFMA accumulators
# in ordinary VGPRs: its state tiles are rescaled and converted by VALU every
# chunk, and accumulators in AGPRs would cost a move each way.
EXTRA_FLAGS = {"gdn_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build_library(verbose: bool = False) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(OBJDIR, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src),
                     "-o", obj])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for out in ex.map(_run, cmds):
            if verbose and out.strip():
                print(out)
    lib = os.path.join(LIBDIR, LIB_NAME)
    tmp = lib + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", tmp])
    os.replace(tmp, lib)
    return lib


def build_harness() -> None:
    os.makedirs(BINDIR, exist_ok=True)
    common = ["-O2", "-std=c11", "-Wall", "-Wextra", f"-I{INCLUDE}", f"-I{ROCM}/include",
              "-D__HIP_PLATFORM_AMD__"]
    link = [f"-L{LIBDIR}", "-lkai_gdn_hip", "-Wl,-rpath,$ORIGIN/../lib",
            f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-lm"]
    for name in ("test_kai_gdn", "bench_kai_gdn", "gdn_e2e_decode"):
        _run([CC, *common, os.path.join(PKG, "harness", f"{name}.c"),
              "-o", os.path.join(BINDIR, name), *link])


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_harness()


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", os.path.join(LIBDIR, LIB_NAME))
