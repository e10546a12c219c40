"""AddressSanitizer + UndefinedBehaviorSanitizer run of the C ABI's host code and of the oracle's
C expert MLP (tests/sanitize: capi.cpp built for the host with both sanitizers, linked with the
built library; every call stops before a launch, so no GPU is needed)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_abi_and_oracle_under_asan_ubsan(tmp_path):
    if not os.path.exists(os.path.join(ROOT, "kandiga_amd", "libkandiga_amd.so")):
        pytest.skip("library not built")
    if not shutil.which("/opt/rocm/bin/hipcc") and not shutil.which("hipcc"):
        pytest.skip("no hipcc")
    out = str(tmp_path / "san")
    b = subprocess.run(["make", "-C", os.path.join(HERE, "sanitize"), f"OUT={out}"], capture_output=True, text=True,
                       timeout=600)
    assert b.returncode == 0, b.stdout[-3000:] + b.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([os.path.join(out, "abi_check")], capture_output=True, text=True, timeout=300, env=env)
    report = r.stdout + r.stderr
    assert r.returncode == 0 and "OK" in r.stdout, report[-4000:]
    assert "ERROR: AddressSanitizer" not in report and "runtime error" not in report, report[-4000:]
