"""Sanitizer builds for the CPU suite (tests/test_sanitizers.py), all under tests/_bin/san
(git-ignored), rebuilt when a source is newer:
  * oracle_san       the CPU oracle (oracle/oracle.c) with tests/oracle_san.c, gcc,
                     AddressSanitizer + UndefinedBehaviorSanitizer;
  * libmigemm.so     the library with its host code instrumented the same way (ROCm clang,
                     -Xarch_host before every sanitizer flag; the gfx950 device code is the
                     ordinary build, never run here);
  * c_abi_check      tests/c_abi_check.c built with ROCm clang and the same sanitizers,
                     linked against that library (one sanitizer runtime per process).
Only argument-validation and runtime-service paths run: there is no GPU here.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "_bin", "san")
CLANG = "/opt/rocm/llvm/bin/clang"
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}

sys.path.insert(0, ROOT)


def _newer(target, sources):
    return not os.path.exists(target) or os.path.getmtime(target) < max(
        os.path.getmtime(s) for s in sources)


def oracle_driver():
    os.makedirs(OUT, exist_ok=True)
    exe = os.path.join(OUT, "oracle_san")
    srcs = [os.path.join(ROOT, "oracle", "oracle.c"), os.path.join(HERE, "oracle_san.c")]
    if _newer(exe, srcs):
        subprocess.run(["gcc", "-std=c11", "-O1", "-g", "-fno-omit-frame-pointer",
                        "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-ffp-contract=off", "-fopenmp", *srcs, "-o", exe, "-lm"], check=True)
    return exe


def library():
    """libmigemm.so with sanitized host code, compiled in parallel like build_native."""
    from my_pytchon_opencl_lib_amd import build_native as bn
    os.makedirs(OUT, exist_ok=True)
    lib = os.path.join(OUT, "libmigemm.so")
    srcs = [os.path.join(bn.CSRC, s) for s in bn.SOURCES]
    deps = srcs + [os.path.join(bn.CSRC, f) for f in os.listdir(bn.CSRC) if f.endswith(".h")] + \
        [os.path.join(ROOT, "include", "migemm.h")]
    if not _newer(lib, deps):
        return lib
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
           "-Xarch_host", "-g"]
    procs, objs = [], []
    for src in srcs:
        obj = os.path.join(OUT, os.path.basename(src).replace(".hip", ".o"))
        objs.append(obj)
        cmd = [bn.hipcc_path(), *bn.hip_flags(), *san, "-c", src, "-o", obj]
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT)))
        while sum(p.poll() is None for _, p in procs) >= 8:
            next(p for _, p in procs if p.poll() is None).wait()
    for src, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            raise RuntimeError(f"sanitized build of {src} failed:\n{out.decode()[-3000:]}")
    subprocess.run([bn.hipcc_path(), f"--offload-arch={bn.ARCH}", "-shared", "-fPIC",
                    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                    *objs, "-o", lib], check=True)
    return lib


def c_caller():
    lib = library()
    exe = os.path.join(OUT, "c_abi_check")
    srcs = [os.path.join(HERE, "c_abi_check.c"), os.path.join(ROOT, "include", "migemm.h"), lib]
    if _newer(exe, srcs):
        subprocess.run([CLANG, "-std=c99", "-O1", "-g", "-fno-omit-frame-pointer", "-pthread",
                        "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-I", os.path.join(ROOT, "include"), srcs[0], "-L", OUT, "-lmigemm",
                        "-Wl,-rpath," + OUT, "-o", exe], check=True)
    return exe


def run(exe, *args, timeout=300):
    env = dict(os.environ, **SAN_ENV)
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout, env=env)
