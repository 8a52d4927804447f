"""The CPU oracle and the host-side layout code under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/sanitize/: gcc/g++ builds of host code
only, run as programs)."""
import os
import shutil
import subprocess

import pytest

SAN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


def _sanitizers_available(tmp_path):
    src = tmp_path / "t.c"
    src.write_text("int main(void) { return 0; }\n")
    r = subprocess.run(["gcc", "-fsanitize=address,undefined", "-o", str(tmp_path / "t"), str(src)],
                       capture_output=True, text=True)
    return r.returncode == 0


def test_sanitized_oracle_and_host_logic(tmp_path):
    if shutil.which("make") is None or shutil.which("gcc") is None or not _sanitizers_available(tmp_path):
        pytest.skip("gcc with AddressSanitizer/UndefinedBehaviorSanitizer is not available")
    r = subprocess.run(["make", "-s", "-C", SAN_DIR, "run"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, (r.stdout[-4000:], r.stderr[-4000:])
    assert "no sanitizer finding" in r.stdout
