"""Build the gfx950 code object and the C-ABI library ``libhayai_hip.so`` in-tree.

Steps (all offline, no GPU needed):
  1. hipcc --genco: every kernel source (one translation unit, csrc/kernels/all.hip) into
     one gfx950 code object, with -ffp-contract=off and packed FP32 disabled.
  2. An assembler stub .incbin's that code object into the library, so the engine loads it
     with hipModuleLoadData and the .so is the only file a deployment needs (the engine
     also accepts a code-object file via HAYAI_HIP_CODE_OBJECT, loaded with hipModuleLoad).
  3. g++ builds the host runtime (csrc/runtime/*.cpp) against the HIP runtime.

Run ``python -m hayai_amd.build`` or call :func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libhayai_hip.so")
CODE_OBJECT = os.path.join(BUILD, "hayai_kernels_gfx950.hsaco")
ARCH = "gfx950"

KERNEL_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "--genco",
    "-ffp-contract=off",
    # packed FP32 (v_pk_*_f32) stays off on this platform
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # kernel-argument preload: the first 16 dwords of a kernel's scalar parameters arrive in
    # SGPRs (kernels taking a struct by value keep the scalar load)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def rocm_path() -> str:
    return os.environ.get("ROCM_PATH", "/opt/rocm")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out:
        print(out)


def build_kernels(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = os.path.join(rocm_path(), "bin", "hipcc")
    src = os.path.join(CSRC, "kernels", "all.hip")
    tmp = CODE_OBJECT + ".tmp"
    _run([hipcc, *KERNEL_FLAGS, "-o", tmp, src], verbose)
    os.replace(tmp, CODE_OBJECT)
    return CODE_OBJECT


def build_runtime(verbose: bool = False) -> list[str]:
    """Compile the host runtime objects (independent of the code object)."""
    os.makedirs(BUILD, exist_ok=True)
    cxx = os.environ.get("CXX", "g++")
    objs = []
    for name in ("engine.cpp", "capi.cpp", "streamer.cpp", "gguf.cpp"):
        src = os.path.join(CSRC, "runtime", name)
        obj = os.path.join(BUILD, name.replace(".cpp", ".o"))
        _run([cxx, "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
              "-D__HIP_PLATFORM_AMD__", f"-I{rocm_path()}/include", f"-I{ROOT}/include", "-c", src, "-o", obj],
             verbose)
        objs.append(obj)
    return objs


def build_noalloc(verbose: bool = False) -> str:
    """The one host+device translation unit (runtime/noalloc.hip: the no-allocation entry
    point's file-scope scratch array and its address lookup), compiled by hipcc for gfx950."""
    os.makedirs(BUILD, exist_ok=True)
    hipcc = os.path.join(rocm_path(), "bin", "hipcc")
    src = os.path.join(CSRC, "runtime", "noalloc.hip")
    obj = os.path.join(BUILD, "noalloc.o")
    _run([hipcc, f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-Wall",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          f"-I{ROOT}/include", "-c", src, "-o", obj], verbose)
    return obj


def link(objs: list[str], verbose: bool = False) -> str:
    blob_s = os.path.join(BUILD, "blob.S")
    with open(blob_s, "w") as f:
        f.write(
            "\t.section .rodata\n"
            "\t.global hh_kernels_blob\n\t.type hh_kernels_blob, @object\n\t.balign 4096\n"
            "hh_kernels_blob:\n"
            f"\t.incbin \"{CODE_OBJECT}\"\n"
            "\t.global hh_kernels_blob_end\nhh_kernels_blob_end:\n\t.byte 0\n"
            "\t.section .note.GNU-stack,\"\",@progbits\n")
    blob_o = os.path.join(BUILD, "blob.o")
    _run(["gcc", "-c", blob_s, "-o", blob_o], verbose)
    tmp = LIB + ".tmp"
    _run(["g++", "-shared", "-o", tmp, *objs, blob_o, f"-L{rocm_path()}/lib", "-lamdhip64",
          f"-Wl,-rpath,{rocm_path()}/lib", "-Wl,--no-undefined"], verbose)
    os.replace(tmp, LIB)
    return LIB


def build(verbose: bool = False) -> str:
    """Compile everything; always rebuilds (this is the "does it build" check)."""
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=3) as ex:
        fk = ex.submit(build_kernels, verbose)
        fr = ex.submit(build_runtime, verbose)
        fn = ex.submit(build_noalloc, verbose)
        fk.result()
        objs = fr.result() + [fn.result()]
    lib = link(objs, verbose)
    if verbose:
        print(f"built {lib} in {time.time() - t0:.1f}s", flush=True)
    return lib


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
