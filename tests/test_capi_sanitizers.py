"""C-ABI host validation under AddressSanitizer + UndefinedBehaviorSanitizer.

Builds ``tests/asan/capi_validation.cpp`` against an ASan/UBSan build of the
entry points' host code (``make asan`` in the package directory: capi.hip's
host side instrumented, the kernels' objects as shipped) and runs it on the
CPU. The driver calls every entry point in ``include/pallas_flash_amd.h``
with NULL and invalid argument blocks, the workspace-size queries on valid
shapes and the tuning round trip; no call reaches a kernel launch, so no GPU
is needed. The reference has no C layer; the refusal rules the driver checks
follow its Python validation (flash_attention.py:527-545, fused_rope.py:
165-169, paged.py:129-149) plus this library's own workspace and 32-bit
range rules.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import PKG_DIR

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CLANGXX = "/opt/rocm/llvm/bin/clang++"


@pytest.mark.skipif(not (os.path.exists(HIPCC) and os.path.exists(CLANGXX) and shutil.which("make")),
                    reason="needs hipcc, ROCm's clang++ and make")
def test_capi_validation_under_asan_ubsan():
    build = subprocess.run(["make", "-s", "-j8", "asan"], cwd=PKG_DIR, capture_output=True, text=True,
                           timeout=900)
    assert build.returncode == 0, build.stderr[-4000:]
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:halt_on_error=1:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    # no device is needed or wanted: every call is refused before a launch
    env["HIP_VISIBLE_DEVICES"] = ""
    run = subprocess.run([os.path.join(PKG_DIR, "_build", "asan", "capi_validation")], env=env,
                         capture_output=True, text=True, timeout=120)
    out = run.stdout + run.stderr
    assert run.returncode == 0, out[-4000:]
    assert "OK: 0 failed expectations" in run.stdout
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
