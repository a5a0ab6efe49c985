"""Builds tests/c_abi_check.c, a plain C99 caller of libmigemm (no torch, no Python), into
tests/_bin/c_abi_check (git-ignored). __graft_entry__.build() builds it with the library;
the tests rebuild it when the source or the header is newer."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "c_abi_check.c")
HEADER = os.path.join(ROOT, "include", "migemm.h")
PKG = os.path.join(ROOT, "my_pytchon_opencl_lib_amd")
BIN = os.path.join(HERE, "_bin", "c_abi_check")


def build():
    os.makedirs(os.path.dirname(BIN), exist_ok=True)
    # rpath relative to the binary, so the tree can move (the GPU box copies it elsewhere)
    subprocess.run(["gcc", "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic", "-pthread",
                    "-I", os.path.join(ROOT, "include"), SRC, "-L", PKG, "-lmigemm",
                    "-Wl,-rpath,$ORIGIN/../../my_pytchon_opencl_lib_amd", "-o", BIN],
                   check=True)
    return BIN


def binary():
    if (not os.path.exists(BIN) or
            os.path.getmtime(BIN) < max(os.path.getmtime(SRC), os.path.getmtime(HEADER))):
        build()
    return BIN


def run(mode, timeout=120):
    return subprocess.run([binary(), mode], capture_output=True, text=True, timeout=timeout)
