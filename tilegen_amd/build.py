"""Build everything native, in-tree: ``python -m tilegen_amd.build``.

1. ``tilegen_amd/_lib/libtgrt.so`` (the runtime, include/tgrt.h) with the host
   C++ compiler against the ROCm HIP runtime and hipRTC;
2. ``libtg_vendor.so``, the rocSPARSE comparison (when rocSPARSE is installed),
   and ``tilegen_bench``, the native host harness (TGM1 matrix + variant library);
3. the test oracle (``oracle/Makefile``: the C restatement, and the
   reference's own ref.cpp where its sources are present);
4. the hipRTC code objects and C launchers of every named schedule
   (``schedules.TUNED`` and ``TEST_SCHEDULES``) into the kernel cache, so GPU
   runs load prebuilt variants instead of compiling.  hipRTC needs no GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time
from typing import List, Optional

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _run(cmd: List[str], cwd: Optional[str] = None) -> None:
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("command failed (%d): %s\n%s%s" % (res.returncode, " ".join(cmd),
                                                              res.stdout, res.stderr))


def build_runtime() -> str:
    out_dir = os.path.join(PKG, "_lib")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libtgrt.so")
    tmp = out + ".tmp%d" % os.getpid()
    cxx = os.environ.get("CXX") or shutil.which("g++") or "c++"
    _run([cxx, "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(REPO, "include"), "-I", os.path.join(ROCM, "include"),
          os.path.join(PKG, "csrc", "tgrt.cpp"), "-o", tmp, "-Wl,-soname,libtgrt.so",
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-lhiprtc",
          "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, out)
    return out


def build_vendor() -> Optional[str]:
    """libtg_vendor.so (rocSPARSE comparison); skipped when rocSPARSE is absent."""
    if not os.path.exists(os.path.join(ROCM, "include", "rocsparse", "rocsparse.h")):
        return None
    out = os.path.join(PKG, "_lib", "libtg_vendor.so")
    tmp = out + ".tmp%d" % os.getpid()
    cxx = os.environ.get("CXX") or shutil.which("g++") or "c++"
    _run([cxx, "-std=c++17", "-O2", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
          "-Wno-deprecated-declarations", "-I", os.path.join(ROCM, "include"),
          os.path.join(PKG, "csrc", "vendor.cpp"), "-o", tmp, "-L", os.path.join(ROCM, "lib"),
          "-lrocsparse", "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, out)
    return out


def build_harness() -> str:
    """tilegen_bench, the native host harness (csrc/bench_main.cpp)."""
    lib_dir = os.path.join(PKG, "_lib")
    out = os.path.join(lib_dir, "tilegen_bench")
    tmp = out + ".tmp%d" % os.getpid()
    cxx = os.environ.get("CXX") or shutil.which("g++") or "c++"
    _run([cxx, "-std=c++17", "-O2", "-Wall", "-I", os.path.join(REPO, "include"),
          os.path.join(PKG, "csrc", "bench_main.cpp"), "-o", tmp, "-L", lib_dir, "-ltgrt",
          "-ldl", "-Wl,-rpath," + lib_dir])
    os.replace(tmp, out)
    return out


def build_oracle(force: bool = False) -> None:
    _run(["make", "-s"] + (["-B"] if force else []) + ["-C", os.path.join(REPO, "oracle")])


def warm_cache(verbose: bool = False) -> int:
    """Compile every named schedule for every kernel it applies to, and the
    one-pass-skipped variants the pass ablation times."""
    from . import runtime
    runtime._LIB = None  # pick up a freshly built library
    from .ablation import DEFAULT_CASES
    from .codegen import Config, generate
    from .dsl import standard_kernels
    from .matrices import baseline_case
    from .passes import PASS_NAMES
    from .schedules import (HYBRID_TEST_SCHEDULES, MERGE_TEST_SCHEDULES, ODD_BLOCK_SCHEDULES,
                            TEST_KERNELS, TEST_SCHEDULES, TUNED)
    from .verify import compile_generated

    kernels = standard_kernels()
    todo = []
    for case_id, cfg in TUNED.items():
        todo.append((baseline_case(case_id).kernel, cfg, ()))
    for name in TEST_KERNELS:
        for cfg in TEST_SCHEDULES + ODD_BLOCK_SCHEDULES:
            todo.append((name, cfg, ()))
        todo.append((name, Config(tile_size=32, threads_per_row=4, unroll=2, vector_width=1,
                                  block_size=256, inject_bug=True), ()))
    for name in ("spmv", "fused_spmv_axpy"):
        for cfg in MERGE_TEST_SCHEDULES + HYBRID_TEST_SCHEDULES:
            todo.append((name, cfg, ()))
    for name, cases in DEFAULT_CASES.items():
        for case_id in cases:
            todo += [(name, TUNED[case_id], skip) for skip in [()] + [(p,) for p in PASS_NAMES]]
    workdir = os.path.join(REPO, "build", "generated")
    n, seen = 0, set()
    for name, cfg, skip in todo:
        gen = generate(kernels[name], cfg, "hip", outdir=workdir, skip_passes=skip)
        if gen.filename in seen:
            continue
        seen.add(gen.filename)
        if skip:
            full = generate(kernels[name], cfg, "hip", write=False)
            if gen.abi_args != full.abi_args:
                continue  # the ablation reports these as invalid and never runs them
        compile_generated(gen, "hip", workdir)
        n += 1
        if verbose:
            print("[build] %s %s %s" % (name, cfg.short(), " ".join(skip)))
    return n


def build_all(verbose: bool = True, force: bool = False) -> None:
    """Build everything; ``force`` also recompiles the oracle and every cached
    kernel variant instead of reusing up-to-date outputs."""
    t0 = time.time()
    path = build_runtime()
    if verbose:
        print("[build] runtime %s (%.1fs)" % (path, time.time() - t0))
    build_vendor()
    build_harness()
    build_oracle(force)
    if force:
        from .verify import cache_dir
        shutil.rmtree(cache_dir(), ignore_errors=True)
    if verbose:
        print("[build] oracle (%.1fs)" % (time.time() - t0))
    n = warm_cache()
    if verbose:
        print("[build] %d HIP variants cached (%.1fs)" % (n, time.time() - t0))


if __name__ == "__main__":
    build_all(verbose=True, force="--force" in sys.argv[1:])
    sys.exit(0)
