"""The host-side code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

Builds the host-only sanitized C ABI and the sanitized oracle (their Makefiles' sanitizer
targets) and runs tests/sanitize_driver.py in a child process with clang's sanitizer runtime
preloaded: an invalid access, a leak-free misuse of the heap or any undefined behaviour aborts
the child, which fails this test with the report."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


@pytest.mark.skipif(_runtime() is None, reason="clang's AddressSanitizer runtime is not installed")
def test_host_code_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-j6", "-C", os.path.join(ROOT, "vllm_webgpu_amd", "csrc"), "san"],
                   check=True)
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "_san/liboracle.so"], check=True)
    env = dict(os.environ, LD_PRELOAD=_runtime(),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    p = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "sanitize_driver.py")], env=env,
                       capture_output=True, text=True, timeout=600)
    out = p.stdout + p.stderr
    assert p.returncode == 0, out[-4000:]
    assert "C ABI host paths: ok" in out and "oracle:" in out, out[-2000:]
