"""Checks on the generated gfx950 code of the direct-to-LDS GEMM kernels (CPU only: hipcc
cross-compiles the device code to assembly text).

gemm_direct_kernel (gemm_direct.h) and gemm_panel_kernel (gemm_panel.hip) issue
global_load_lds_dwordx4 / global_load_lds_dword through inline assembly that sets M0 itself
and declares it clobbered. M0 is a register the compiler
reserves, so the kernels may only be correct if no compiler-generated code relies on M0
across those statements. This test pins that: in the device assembly, M0 is written only by
`s_mov_b32 m0, s<n>` immediately followed by one of those loads, and nothing reads it
otherwise."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "my_pytchon_opencl_lib_amd", "csrc")
# the translation units that instantiate gemm_direct_kernel (one per tile shape) and the
# panel kernel (every operand layout, one or two operand pairs)
SRCS = [os.path.join(CSRC, f"gemm_direct_{t}.hip") for t in ("256", "128x256", "128", "64")] + \
    [os.path.join(CSRC, "gemm_panel.hip")]


def _hipcc():
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_m0_only_feeds_the_lds_loads(tmp_path):
    procs = []
    for src in SRCS:
        out = tmp_path / (os.path.basename(src) + ".s")
        procs.append((src, out, subprocess.Popen(
            [_hipcc(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
             "-Xclang", "-packed-fp32-ops", "-Wno-inline-asm", "--cuda-device-only", "-S", src,
             "-o", str(out)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    for src, out, p in procs:
        log, _ = p.communicate()
        assert p.returncode == 0, log.decode(errors="replace")[-2000:]
        lines = [l.split(";")[0].strip() for l in out.read_text().splitlines()]
        code = [l for l in lines if l and not l.startswith(".") and not l.endswith(":")]
        loads = 0
        for i, l in enumerate(code):
            if not re.search(r"\bm0\b", l):
                continue
            assert re.fullmatch(r"s_mov_b32 m0, s\d+", l), f"{src}: unexpected use of M0: {l!r}"
            assert re.match(r"global_load_lds_dword(x4)? ", code[i + 1]), \
                f"{src}: M0 written without a following LDS load: {l!r} then {code[i + 1]!r}"
            loads += 1
        assert loads > 0, f"{src}: no global_load_lds_dword(x4) found"
        n_lds = sum(1 for l in code if re.match(r"global_load_lds_dword(x4)? ", l))
        assert n_lds == loads, (src, n_lds, loads)
