"""Build recipe for librtq.so (the C-ABI library) and the CPU oracle.

1. ``rtq_kernels.hip`` -> gfx950 code object (``hipcc --genco``), into ``rust_trainer_amd/_build/``;
2. ``rtq_runtime.cpp`` + ``rtq_gguf.cpp`` + ``rtq_model.cpp`` -> ``rust_trainer_amd/librtq.so`` (g++ against the HIP runtime), with the
   code object embedded (``.incbin``) and loaded at run time with ``hipModuleLoadData``, plus
   ``rtq_noalloc.hip`` compiled by hipcc (its device array is registered with the HIP runtime);
3. ``oracle/`` -> ``oracle/liboracle.so`` (test infrastructure, plain gcc).

Everything is built in-tree so the shared objects travel with the repository snapshot.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",          # fusions are written explicitly (fmaf); dequant rounds like the reference
    "-munsafe-fp-atomics",        # hardware f32 atomic add for split reductions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",  # MFMA results in VGPRs: the epilogues read them with VALU
]


def _run(cmd: list[str], cwd: str | None = None) -> None:
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


def build_kernels() -> str:
    os.makedirs(BUILD, exist_ok=True)
    out = os.path.join(BUILD, "rtq_kernels.hsaco")
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, "--genco", "--no-gpu-bundle-output", "-I", CSRC,
          os.path.join(CSRC, "rtq_kernels.hip"), "-o", tmp])
    os.replace(tmp, out)
    return out


def build_noalloc() -> str:
    """rtq_noalloc.hip (host + gfx950 device code: the no-allocation entry point's scratch array)
    -> an object linked into librtq.so"""
    os.makedirs(BUILD, exist_ok=True)
    out = os.path.join(BUILD, "rtq_noalloc.o")
    tmp = out + ".tmp.o"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, "-fPIC", "-c", "-I", os.path.join(ROOT, "include"),
          "-I", CSRC, os.path.join(CSRC, "rtq_noalloc.hip"), "-o", tmp])
    os.replace(tmp, out)
    return out


def build_runtime(hsaco: str, noalloc_obj: str) -> str:
    out = os.path.join(PKG, "librtq.so")
    tmp = out + ".tmp"
    cxx = shutil.which("g++") or "g++"
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter", "-Wno-attributes",
          "-D__HIP_PLATFORM_AMD__", f'-DRTQ_HSACO_PATH="{hsaco}"',
          "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"), "-I", CSRC,
          os.path.join(CSRC, "rtq_runtime.cpp"), os.path.join(CSRC, "rtq_gguf.cpp"),
          os.path.join(CSRC, "rtq_model.cpp"), noalloc_obj, "-o", tmp,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"])
    os.replace(tmp, out)
    return out


def build_oracle() -> None:
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])


def build() -> None:
    hsaco = build_kernels()
    build_runtime(hsaco, build_noalloc())
    build_oracle()


if __name__ == "__main__":
    build()
    sys.exit(0)
