"""The C-ABI boundary: every function include/mmhip.h declares is exported by
the built libmmhip.so, the header is valid C, and the Zig binding
(mobile-moe.zig_amd/zig/hip_backend.zig) declares exactly those functions.
No device is touched."""
import os
import re
import shutil
import subprocess

import pytest

import mmhip as mm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mmhip.h")
ZIG = os.path.join(ROOT, "mobile-moe.zig_amd", "zig", "hip_backend.zig")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mmhip_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_expected_surface():
    fns = header_functions()
    for name in ("mmhip_init", "mmhip_destroy", "mmhip_last_error", "mmhip_mat_vec_mul", "mmhip_batch_mat_mul",
                 "mmhip_dequantize", "mmhip_gemv_batched_dev", "mmhip_qmm_dev", "mmhip_moe_ffn",
                 "mmhip_moe_ffn_dev", "mmhip_plan_layer"):
        assert name in fns
    assert len(fns) >= 35


def test_library_exports_every_declared_function():
    lib = mm.load_library()
    missing = [f for f in header_functions() if not hasattr(lib, f)]
    assert not missing, f"declared but not exported: {missing}"


@pytest.mark.skipif(shutil.which("nm") is None, reason="nm not available")
def test_no_undeclared_exports():
    out = subprocess.run(["nm", "-D", "--defined-only", mm.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(mmhip_[a-z0-9_]+)$", out, flags=re.M))
    assert exported == set(header_functions())


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_header_is_plain_c(tmp_path):
    c = tmp_path / "t.c"
    c.write_text('#include "mmhip.h"\nint main(void) { return mmhip_version() == 0; }\n')
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.dirname(HEADER), str(c)],
                   check=True)


def test_zig_binding_matches_header():
    zig = open(ZIG).read()
    externs = sorted(set(re.findall(r"^extern fn (mmhip_[a-z0-9_]+)\(", zig, flags=re.M)))
    assert externs == header_functions()
