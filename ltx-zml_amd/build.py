"""Build the MI355X block library in-tree.

1. Each kernel source csrc/k_*.hip -> a gfx950 code object (hipcc --genco).
2. The code objects are embedded with .incbin into the host library, which
   loads them at ltx_init() with hipModuleLoadData.
3. Host runtime (csrc/host/*.cpp, plain C++ over the HIP runtime API; and
   csrc/host/*.hip, host code with a device array of its own, by hipcc) + the
   embedded objects -> libltx_amd.so next to this file.
4. csrc/tools/mfma_ceiling.hip -> mfma_ceiling next to this file (the
   practical MFMA-rate ceiling that the benchmark's roofline is read against).

Usage: python ltx-zml_amd/build.py [-v]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libltx_amd.so"
CEILING = PKG / "mfma_ceiling"
INCLUDE = PKG.parent / "include"
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
KERNELS = ["k_gemm", "k_gemm_s4", "k_attn", "k_norm", "k_f32", "k_core"]
HOST = ["ltx_runtime", "ltx_forward", "ltx_weights", "ltx_rope", "ltx_loader", "ltx_core", "sha256"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "--genco",
    # packed-FP32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_HIP = ["ltx_noalloc"]
HIP_HOST_FLAGS = [
    "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", "-D__HIP_PLATFORM_AMD__",
             f"-I{ROCM / 'include'}", f"-I{INCLUDE}", "-pthread"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout[-4000:] + r.stderr[-8000:])
        raise RuntimeError(f"build step failed: {cmd[0]} {cmd[-1]}")


def build(verbose: bool = False) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    hipcc = str(ROCM / "bin" / "hipcc")
    jobs = []
    for k in KERNELS:
        jobs.append([hipcc, *HIPCC_FLAGS, f"-I{CSRC}", str(CSRC / f"{k}.hip"), "-o", str(BUILD / f"{k}.hsaco")])
    asm = BUILD / "ltx_codeobjects.S"
    lines = [".section .rodata"]
    for k in KERNELS:
        lines += [f".global ltx_co_{k}", ".balign 4096", f"ltx_co_{k}:", f'.incbin "{BUILD / (k + ".hsaco")}"',
                  ".byte 0"]
    lines += ['.section .note.GNU-stack,"",@progbits', ""]
    asm.write_text("\n".join(lines))
    objs = []
    for h in HOST:
        o = BUILD / f"{h}.o"
        jobs.append(["g++", *CXX_FLAGS, "-c", str(CSRC / "host" / f"{h}.cpp"), "-o", str(o)])
        objs.append(o)
    # host objects with device globals of their own (hipcc: registered with
    # the HIP runtime when the library loads)
    for h in HOST_HIP:
        o = BUILD / f"{h}.o"
        jobs.append([hipcc, *HIP_HOST_FLAGS, f"-I{CSRC}", f"-I{INCLUDE}", "-c", str(CSRC / "host" / f"{h}.hip"),
                     "-o", str(o)])
        objs.append(o)
    jobs.append([hipcc, *HIP_HOST_FLAGS, str(CSRC / "tools" / "mfma_ceiling.hip"), "-o", str(CEILING)])
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    _run(["g++", "-c", str(asm), "-o", str(BUILD / "ltx_codeobjects.o")], verbose)
    tmp = LIB.with_suffix(".so.tmp")
    _run(["g++", "-shared", "-o", str(tmp), *map(str, objs), str(BUILD / "ltx_codeobjects.o"),
          f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-pthread"], verbose)
    shutil.move(str(tmp), str(LIB))
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
