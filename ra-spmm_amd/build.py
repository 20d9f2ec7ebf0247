"""Build the MI355X (gfx950) extension in-tree.

Outputs (next to the Python package, so they travel with the source tree):
  ra-spmm_amd/ra_spmm/libra_spmm_hip.so   C ABI (include/ra_spmm.h): HIP kernels + host code
  ra-spmm_amd/ra_spmm/_C.<abi>.so          thin torch binding (the `ra_spmm` names)

Usage: python ra-spmm_amd/build.py [--jobs N] [--no-binding]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT_DIR = PKG_ROOT / "ra_spmm"
OBJ_DIR = PKG_ROOT / "_build"
ARCH = os.environ.get("RA_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 VALU instructions are kept out of all device code (some of their
# forms gave silent wrong results on this GPU pool); -ffp-contract=off is per
# file where host arithmetic must match the Python router bit for bit.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
SOURCES = {
    "common.cpp": [],
    "router.cpp": ["-ffp-contract=off"],
    "diagnostics.cpp": ["-ffp-contract=off"],
    "tile_build.cpp": [],
    "csr_kernels.hip": [],
    "tile_kernels.hip": [],
    "tile_build_gpu.hip": [],
    "zo_build_gpu.hip": [],
    "zo_noalloc.hip": [],
    "tile_f32_route.hip": [],
}
LIB_NAME = "libra_spmm_hip.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature; drop that noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_library(jobs: int) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    cmds = []
    objs = []
    for src, extra in SOURCES.items():
        obj = OBJ_DIR / (src.replace(".", "_") + ".o")
        lang = (["-x", "hip"] if src.endswith(".hip")
                else ["-x", "c++", "-D__HIP_PLATFORM_AMD__=1", "-I/opt/rocm/include"])
        cmds.append([HIPCC] + HIP_FLAGS + extra + lang + ["-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    lib = OUT_DIR / LIB_NAME
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(lib)]
         + [str(o) for o in objs] + ["-lpthread", f"-Wl,-soname,{LIB_NAME}"])
    return lib


def build_vendor() -> Path:
    """The rocSPARSE comparator (csrc/vendor_spmm.cpp): a measurement tool
    for bench.py, kept out of the product library."""
    out = OUT_DIR / "libra_vendor_spmm.so"
    _run([HIPCC, "-O2", "-fPIC", "-shared", "-std=c++17", "-x", "c++", "-D__HIP_PLATFORM_AMD__=1",
          "-I/opt/rocm/include", str(CSRC / "vendor_spmm.cpp"), "-o", str(out),
          "-L/opt/rocm/lib", "-lrocsparse", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"])
    return out


def build_probe() -> Path:
    """The gather probe (csrc/gather_probe.hip): a measurement tool for
    bench.py, kept out of the product library."""
    out = OUT_DIR / "libra_gather_probe.so"
    _run([HIPCC] + HIP_FLAGS + ["-shared", "-x", "hip", str(CSRC / "gather_probe.hip"), "-o", str(out)])
    return out


def build_binding() -> Path:
    import torch  # noqa: F401  (headers and libraries of the running torch)
    from torch.utils import cpp_extension

    torch_lib = Path(cpp_extension.library_paths()[0])
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = OUT_DIR / f"_C{suffix}"
    incs = []
    for p in cpp_extension.include_paths():
        incs += ["-I", p]
    py_inc = sysconfig.get_paths()["include"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = (["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-D__HIP_PLATFORM_AMD__=1",
            "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_C",
            "-DTORCH_API_INCLUDE_EXTENSION_H"]
           + incs + ["-I", py_inc, "-I", "/opt/rocm/include", str(CSRC / "torch_binding.cpp"),
                     "-o", str(out), "-L", str(OUT_DIR), "-lra_spmm_hip", "-L", str(torch_lib),
                     "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-L/opt/rocm/lib", "-lamdhip64",
                     "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"])
    _run(cmd)
    return out


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--no-binding", action="store_true")
    args = ap.parse_args(argv)
    lib = build_library(args.jobs)
    print(f"built {lib}")
    print(f"built {build_vendor()}")
    print(f"built {build_probe()}")
    if not args.no_binding:
        print(f"built {build_binding()}")


if __name__ == "__main__":
    main()
