"""The library's host code (GGUF parser, residency map, planner, the C ABI's
argument checks) under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C mobile-moe.zig_amd sanitize` builds lib/libmmhip_san.so: the .cpp
files instrumented (hipcc -Xarch_host -fsanitize=address / undefined), the
device code as in the normal build. A child Python process with the ASan
runtime preloaded and MMHIP_LIBRARY pointing at that build runs the host test
files (GGUF round trips and error files, the bounded GGUF fuzz, the planner,
the ABI export and type checks); any invalid read or write, or undefined
behaviour, aborts it. No device is touched."""
import glob
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mobile-moe.zig_amd")
ASAN_RT = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
HOST_TESTS = ["test_gguf.py", "test_gguf_fuzz.py", "test_planner.py", "test_abi_exports.py", "test_zig_abi_types.py"]


@pytest.mark.skipif(not ASAN_RT or shutil.which("make") is None, reason="no ASan runtime or make in this image")
def test_host_code_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", PKG, "-j8", "sanitize"], check=True)
    env = dict(os.environ)
    env.update(LD_PRELOAD=ASAN_RT[-1], ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               MMHIP_LIBRARY=os.path.join(PKG, "lib", "libmmhip_san.so"))
    cmd = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu"] + \
          [os.path.join(ROOT, "tests", t) for t in HOST_TESTS]
    r = subprocess.run(cmd, env=env, cwd=ROOT, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert " passed" in r.stdout and "error" not in r.stdout.splitlines()[-1].lower(), tail
