"""Build the native CKL backend in-tree: libckl_hip.so (host compiler pipeline, HIP executor,
C ABI), ckl_kernels_gfx950.hsaco (hand-written gfx950 kernel library) and the ckl-opt
command-line pass driver (linked against libckl_hip.so).

Usage: python build.py [--jobs N]. Outputs go to python/ckl/_lib/.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "python" / "ckl" / "_lib"
BUILD = ROOT / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("CKL_OFFLOAD_ARCH", "gfx950")

HOST_SOURCES = [
    "core/ir.cpp", "core/planner.cpp", "core/analysis.cpp", "core/verify.cpp", "core/fusion.cpp", "core/compiler.cpp",
    "runtime/runtime.cpp", "runtime/chains.cpp", "runtime/codegen.cpp", "runtime/kernarg.cpp", "capi.cpp",
]
KERNEL_SOURCES = ["kernels/library.hip"]
# Host sources with device code of their own (the static scratch arena), built by hipcc into
# objects of libckl_hip.so.
HIP_HOST_SOURCES = ["runtime/scratch.hip"]
# Packed FP32 instructions are disabled for all device code built here.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def run(command: list[str]) -> None:
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode:
        sys.stderr.write(" ".join(command) + "\n" + result.stdout + result.stderr)
        raise SystemExit(f"build step failed: {command[0]}")


def compile_host(source: str) -> Path:
    obj = BUILD / (source.replace("/", "_") + ".o")
    src = CSRC / source
    deps = [src, *CSRC.glob("**/*.h"), ROOT.parent / "include" / "ckl_hip.h"]
    if obj.exists() and obj.stat().st_mtime >= max(p.stat().st_mtime for p in deps):
        return obj
    run(["g++", "-std=c++17", "-O2", "-g", "-fPIC", "-Wall", "-Wno-unused-function",
         "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", "-c", str(src), "-o", str(obj)])
    return obj


def compile_hip_host(source: str) -> Path:
    obj = BUILD / (source.replace("/", "_") + ".o")
    src = CSRC / source
    deps = [src, *CSRC.glob("**/*.h"), ROOT.parent / "include" / "ckl_hip.h"]
    if obj.exists() and obj.stat().st_mtime >= max(p.stat().st_mtime for p in deps):
        return obj
    run([str(ROCM / "bin" / "hipcc"), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", *DEVICE_FLAGS,
         "-c", str(src), "-o", str(obj)])
    return obj


def build(jobs: int = 8) -> None:
    BUILD.mkdir(exist_ok=True)
    OUT.mkdir(parents=True, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        kernels = pool.submit(build_kernels)
        hip_objects = [pool.submit(compile_hip_host, s) for s in HIP_HOST_SOURCES]
        objects = list(pool.map(compile_host, HOST_SOURCES)) + [f.result() for f in hip_objects]
        kernels.result()
    library = OUT / "libckl_hip.so"
    tmp = library.with_suffix(".so.tmp")
    run(["g++", "-shared", "-o", str(tmp), *map(str, objects), f"-L{ROCM / 'lib'}",
         f"-Wl,-rpath,{ROCM / 'lib'}", "-lamdhip64", "-lhiprtc", "-ldl", "-pthread"])
    os.replace(tmp, library)
    build_tool(library)


def build_tool(library: Path) -> None:
    """ckl-opt beside the library it links (found at run time through an $ORIGIN rpath)."""
    tool = OUT / "ckl-opt"
    tmp = tool.with_suffix(".tmp")
    run(["g++", "-std=c++17", "-O2", "-Wall", str(CSRC / "tools" / "ckl_opt.cpp"), "-o", str(tmp),
         f"-L{OUT}", "-l:" + library.name, "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, tool)


def build_kernels() -> None:
    output = OUT / f"ckl_kernels_{ARCH}.hsaco"
    tmp = output.with_suffix(".hsaco.tmp")
    sources = [str(CSRC / s) for s in KERNEL_SOURCES]
    run([str(ROCM / "bin" / "hipcc"), "--genco", "--no-gpu-bundle-output", f"--offload-arch={ARCH}", "-O3", "-std=c++17",
         *DEVICE_FLAGS, "-o", str(tmp), *sources])
    os.replace(tmp, output)


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=8)
    parser.add_argument("--clean", action="store_true")
    args = parser.parse_args()
    if args.clean:
        clean()
    build(args.jobs)
    print(f"built {OUT}")
