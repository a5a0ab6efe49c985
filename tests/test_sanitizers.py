"""The CPU sanitizer leg: AddressSanitizer and UndefinedBehaviorSanitizer over the code that
runs on the host (builds in tests/sanitize.py).
  * the CPU oracle, every function over edge-case shapes with exactly sized buffers
    (tests/oracle_san.c);
  * the library's host code -- argument validation of every entry point, the runtime
    services' checks, the thread-local error state, the plan record -- driven by the plain C
    caller tests/c_abi_check.c (mode validate, several POSIX threads) against a build of
    libmigemm.so whose host code is instrumented.
A sanitizer report fails the run (halt_on_error, no recovery)."""
import os
import shutil

import pytest

import sanitize

REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer",
           "SUMMARY: UndefinedBehaviorSanitizer")


def clean(r):
    text = r.stdout + r.stderr
    return r.returncode == 0 and not any(s in text for s in REPORTS), text[-4000:]


def test_oracle_under_asan_ubsan():
    exe = sanitize.oracle_driver()
    ok, text = clean(sanitize.run(exe))
    assert ok, text
    assert "oracle_san: ok" in text


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_library_host_code_under_asan_ubsan():
    exe = sanitize.c_caller()
    ok, text = clean(sanitize.run(exe, "validate"))
    assert ok, text
    assert "c_abi_check validate: ok" in text
