"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer.

The reference's CI runs its tests with the race detector (go test -race,
.github/workflows/ci.yml:44-45).  Here the library's host code -- the
safetensors parser that reads untrusted archive headers, the ABI's argument
checks -- is built with -fsanitize=address,undefined (build.py,
build_sanitized: _build/asan/libsrq_asan.so) and the CPU archive and ABI
tests run against it in a child process with the sanitizer runtime
preloaded.  Any sanitizer report ends the child with an error."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN_LIB = os.path.join(ROOT, "sr_go_tranformer_amd", "_build", "asan", "libsrq_asan.so")


def _runtime():
    found = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def test_archive_and_abi_tests_under_sanitizers():
    rt = _runtime()
    if not os.path.exists(ASAN_LIB) or rt is None:
        pytest.skip("the host-sanitized library is not built (sr_go_tranformer_amd/build.py build_sanitized)")
    env = dict(os.environ)
    env.update(LD_PRELOAD=rt, SRQ_LIB=ASAN_LIB, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        "tests/test_archive_cpu.py", "tests/test_abi_cpu.py"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in out
