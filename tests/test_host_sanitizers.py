"""The C ABI's host-side code under AddressSanitizer and UBSan (CPU only).

tests/sanitize/build.sh compiles the library's sources for the host alone
(no device code) with both sanitizers on the host code, and links
tests/sanitize/host_abi_check.c: argument validation of the entry points,
workspace layouts over the configs' shapes and beyond (every region
aligned, in bounds and in order), refused shapes with their messages, and
the reference-compatible host entry points' argument and index checks.  On
a host without a GPU, calls that pass validation stop at their first HIP
call, so those error paths run as well.  A sanitizer report ends the
program with a non-zero status."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SCRIPT = os.path.join(HERE, "sanitize", "build.sh")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not (os.path.exists(SCRIPT) and os.path.exists(HIPCC)),
                    reason="needs hipcc and tests/sanitize")
def test_host_abi_under_asan_and_ubsan(tmp_path):
    r = subprocess.run(["bash", SCRIPT, str(tmp_path)], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([str(tmp_path / "host_abi_check")], capture_output=True, text=True,
                       timeout=300, env=env)
    assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
    assert "host ABI checks passed" in r.stdout
