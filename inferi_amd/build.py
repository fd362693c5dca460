"""Builds the inferi_hip product library in-tree.

Two artefacts, both written next to this file:
  inferi_kernels.hsaco  gfx950 code object of csrc/kernels.hip
                        (hipcc --genco --offload-arch=gfx950), loaded at run
                        time with hipModuleLoad;
  libinferi_hip.so      host library with the C ABI of include/inferi_hip.h
                        (csrc/host.cpp and csrc/gguf.cpp, C++17, links
                        libamdhip64).

Every HIP compile carries ``-Xclang -target-feature -Xclang -packed-fp32-ops``
so the compiler never emits packed FP32 instructions.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HSACO = os.path.join(HERE, "inferi_kernels.hsaco")
LIB = os.path.join(HERE, "libinferi_hip.so")

HIP_FLAGS = [
    "--genco",
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


def build_kernels(out: str = HSACO) -> str:
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = out + ".tmp"
    _run([hipcc, *HIP_FLAGS, os.path.join(CSRC, "kernels.hip"), "-o", tmp])
    os.replace(tmp, out)
    return out


def build_host(out: str = LIB) -> str:
    cxx = shutil.which("g++") or "g++"
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = out + ".tmp"
    obj_dir = os.path.join(ROOT, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    # the fixed scratch of ifr_matmul_quant_noalloc: a device array, so this
    # one file is compiled by hipcc (for gfx950) and linked into the library
    noalloc_o = os.path.join(obj_dir, "noalloc.o")
    _run([hipcc, "-c", "-fPIC", "--offload-arch=gfx950", "-O2", "-std=c++17", "-fvisibility=hidden",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          os.path.join(CSRC, "noalloc.hip"), "-o", noalloc_o])
    _run([cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-result",
          "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
          os.path.join(CSRC, "host.cpp"), os.path.join(CSRC, "gguf.cpp"), noalloc_o,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", tmp])
    os.replace(tmp, out)
    return out


ASAN_LIB = os.path.join(ROOT, "_build", "libinferi_hip_asan.so")


def asan_runtime() -> str:
    """Path of the compiler's AddressSanitizer runtime (to preload into an
    uninstrumented interpreter)."""
    cxx = shutil.which("g++") or "g++"
    r = subprocess.run([cxx, "-print-file-name=libasan.so"], stdout=subprocess.PIPE, text=True, check=True)
    return r.stdout.strip()


def build_host_asan(out: str = ASAN_LIB) -> str:
    """The host library (C ABI, GGUF reader, launches) built by g++ with
    AddressSanitizer for CPU-side checks; the device code is the ordinary
    code object.  Load it with IFR_LIB=<out> and the runtime preloaded."""
    cxx = shutil.which("g++") or "g++"
    obj_dir = os.path.join(ROOT, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    noalloc_o = os.path.join(obj_dir, "noalloc.o")
    if not os.path.exists(noalloc_o):
        build_host()
    _run([cxx, "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer", "-std=c++17", "-shared", "-fPIC",
          "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
          os.path.join(CSRC, "host.cpp"), os.path.join(CSRC, "gguf.cpp"), noalloc_o,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", out])
    return out


def build() -> None:
    build_kernels()
    build_host()


if __name__ == "__main__":
    build()
    print(HSACO)
    print(LIB)
