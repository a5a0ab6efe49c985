"""Builds libmigemm.so (the HIP kernels + C ABI) in-tree for gfx950 with hipcc.

The library is compiled from my_pytchon_opencl_lib_amd/csrc/*.hip into
my_pytchon_opencl_lib_amd/libmigemm.so. Every call recompiles.
"""
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libmigemm.so")
SOURCES = ["gemm_direct_256.hip", "gemm_direct_128x256.hip", "gemm_direct_128.hip",
           "gemm_direct_64.hip", "gemm_mfma.hip", "api.hip", "gemm_direct.hip", "gemm_small.hip",
           "gemm_skinny.hip", "aux_kernels.hip", "runtime.hip", "gemm_panel.hip",
           "gemm_tiny.hip"]
ARCH = "gfx950"


def hipcc_path():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libmigemm")


def hip_flags():
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Packed fp32 instructions are kept out of every kernel.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
        # gemm_direct.h declares M0 clobbered by its inline-assembly loads into LDS (the
        # compiler warns about any reserved register there); tests/test_codegen.py checks
        # that nothing else in the generated code uses M0.
        "-Wno-inline-asm",
    ]


def build(verbose=False, jobs=8):
    """Compile each source to an object in parallel, then link the shared library."""
    hipcc = hipcc_path()
    objdir = os.path.join(PKG_DIR, "_build")
    os.makedirs(objdir, exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [hipcc, *hip_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        # compiler output goes to a file: a pipe nobody drains until every job has started
        # can fill and stall the compiler
        log = open(obj + ".log", "w+b")
        procs.append((src, subprocess.Popen(cmd, stdout=log, stderr=subprocess.STDOUT), log))
        while len([p for _, p, _ in procs if p.poll() is None]) >= jobs:
            next(p for _, p, _ in procs if p.poll() is None).wait()
    failed = []
    for src, p, log in procs:
        p.wait()
        log.seek(0)
        out = log.read()
        log.close()
        text = "\n".join(l for l in out.decode(errors="replace").splitlines()
                         if "packed-fp32-ops" not in l)
        if text.strip() and (verbose or p.returncode != 0):
            print(text, file=sys.stderr)
        if p.returncode != 0:
            failed.append(src)
    if failed:
        raise RuntimeError(f"hipcc failed for {failed}")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
