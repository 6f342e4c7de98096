"""The host side of libqr_attn under the sanitizers, on the CPU.

``make -C qauntrunner_amd/csrc asan`` rebuilds the host translation units (C ABI argument
checks, page accounting, the hand-written .qw JSON parser, the threaded file reader) with
AddressSanitizer + UndefinedBehaviorSanitizer, ``tsan`` with ThreadSanitizer; each links them
with the ordinary device objects and runs the host-only tests (tests/test_abi.py,
tests/test_model_store.py, tests/test_model_fuzz.py) against that library with the sanitizer
runtime preloaded.  Any report aborts the run (halt_on_error / -fno-sanitize-recover).
"""
import os
import shutil
import subprocess

import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qauntrunner_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not (shutil.which("make") and os.path.exists(HIPCC)), reason="needs make and hipcc")
@pytest.mark.parametrize("target", ["asan", "tsan"])
def test_host_library_under_sanitizer(target):
    r = subprocess.run(["make", "-s", "-j8", "-C", CSRC, target], capture_output=True, text=True, timeout=1200)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert " passed" in out and "failed" not in out, out[-3000:]
