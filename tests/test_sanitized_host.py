"""The library's host code (argument validation, tile tables and rules, workspace sizes, error
reporting) under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

`make -C skinny-mlx_amd/csrc san` builds the same sources with the host half instrumented
(`-Xarch_host -fsanitize=address,undefined`, every report fatal); device code is compiled as usual
and never runs here. A child process loads that build through SKINNY_HIP_LIB with the sanitizer
runtime preloaded and runs the ABI tests, which call every entry point's validation and every
host query. Any report ends the child with an error and fails this test.
"""

import glob
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "skinny-mlx_amd", "csrc")
SAN_LIB = os.path.join(ROOT, "_build", "san", "libskinny_hip_san.so")


def _asan_runtime():
    found = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def test_host_code_clean_under_asan_and_ubsan():
    if shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc") or _asan_runtime() is None:
        pytest.skip("hipcc or the sanitizer runtime is not installed")
    jobs = str(min(8, os.cpu_count() or 4))
    subprocess.run(["make", "-s", "-j", jobs, "-C", CSRC, "san"], check=True, stdout=subprocess.DEVNULL)
    syms = subprocess.run(["nm", "-D", SAN_LIB], check=True, capture_output=True, text=True).stdout
    assert "__asan_report_load" in syms and "__ubsan_handle_" in syms, "the build is not instrumented"
    env = dict(os.environ)
    env.update({
        "SKINNY_HIP_LIB": SAN_LIB,
        "LD_PRELOAD": _asan_runtime(),
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0:exitcode=86",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1:exitcode=87",
        "HIP_VISIBLE_DEVICES": "",  # host code only: no device is touched
    })
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu",
                           os.path.join(ROOT, "tests", "test_abi.py")],
                          cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = proc.stdout + proc.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert proc.returncode == 0, out[-4000:]
    assert " passed" in out
